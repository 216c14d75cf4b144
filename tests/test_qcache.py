"""The qcache sidecar reader on the CPU (no device calls): FNV-1a against
its published test vectors, a file written from the documented layout opens
in read mode, and every inconsistency (magic, stale fingerprint, entry count,
name length, payload beyond the end, truncated table) leaves write mode."""
import ctypes
import os
import struct

import pytest

import qcache_format as qf
import s2pamd


@pytest.fixture(scope="module")
def lib():
    return s2pamd.load()


def test_fnv1a_published_vectors():
    # FNV-1a 64 test vectors (Fowler / Noll / Vo reference page)
    assert qf.fnv1a(b"") == 0xCBF29CE484222325
    assert qf.fnv1a(b"a") == 0xAF63DC4C8601EC8C
    assert qf.fnv1a(b"foobar") == 0x85944171F73967E8


def model_dir(tmp_path):
    d = tmp_path / "model"
    d.mkdir()
    (d / "model-00001-of-00002.safetensors").write_bytes(b"x" * 100)
    (d / "model-00002-of-00002.safetensors").write_bytes(b"y" * 37)
    (d / "config.json").write_text("{}")
    os.utime(d / "model-00001-of-00002.safetensors", (1_700_000_000, 1_700_000_000))
    return d


ENTRIES = [("layers.0.attention.wqkv", 2, 32, 64, 32, bytes(range(256)) * 4, b"\x01\x3c" * 64),
           ("layers.0.feed_forward.w2", 1, 16, 128, 0, bytes(16 * 128), b"\x00\x00\x80\x3f" * 16)]


def open_reading(lib, d, mode=2):
    qc = ctypes.c_void_p()
    s2pamd.check(lib.s2p_qcache_open(str(d).encode(), mode, ctypes.byref(qc)), "qcache open")
    try:
        return None if not qc.value else lib.s2p_qcache_reading(qc)
    finally:
        if qc.value:
            lib.s2p_qcache_free(qc)


def test_reader_accepts_layout(lib, tmp_path):
    d = model_dir(tmp_path)
    (d / "s2p_qcache.bin").write_bytes(qf.file_bytes(qf.fingerprint(d), ENTRIES))
    assert open_reading(lib, d) == 1


@pytest.mark.parametrize("case", ["magic", "stale", "count0", "count_big", "name0",
                                  "payload_past_end", "truncated_table"])
def test_reader_rejects(lib, tmp_path, case):
    d = model_dir(tmp_path)
    fp = qf.fingerprint(d)
    b = bytearray(qf.file_bytes(fp if case != "stale" else fp ^ 1, ENTRIES))
    if case == "magic":
        b[5] = 2
    elif case == "count0":
        b[16:20] = struct.pack("<I", 0)
    elif case == "count_big":
        b[16:20] = struct.pack("<I", 513)
    elif case == "name0":
        b[24:28] = struct.pack("<I", 0)
    elif case == "payload_past_end":
        b[24 + 32:24 + 40] = struct.pack("<Q", len(b))  # q_len of entry 0
    elif case == "truncated_table":
        b = b[:24 + 40]
    (d / "s2p_qcache.bin").write_bytes(bytes(b))
    assert open_reading(lib, d) == 0


def test_fingerprint_follows_files(lib, tmp_path):
    d = model_dir(tmp_path)
    (d / "s2p_qcache.bin").write_bytes(qf.file_bytes(qf.fingerprint(d), ENTRIES))
    os.utime(d / "model-00002-of-00002.safetensors", (1_700_000_500, 1_700_000_500))
    assert open_reading(lib, d) == 0  # mtime changed: stale


def test_disabled_and_unquantised(lib, tmp_path, monkeypatch):
    d = model_dir(tmp_path)
    assert open_reading(lib, d, mode=0) is None  # bf16 mode: no cache
    monkeypatch.setenv("S2P_QCACHE", "0")
    assert open_reading(lib, d) is None
    monkeypatch.delenv("S2P_QCACHE")
    empty = tmp_path / "empty"
    empty.mkdir()
    assert open_reading(lib, empty) is None  # no *.safetensors: no cache
