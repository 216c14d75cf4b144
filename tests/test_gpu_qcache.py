"""The qcache sidecar through device tensors: a write-mode cache snapshots
three quantised linears (per-channel INT8, packed INT4-g32, INT4 in an int8
container), the file it writes equals the documented layout byte for byte,
and a read-mode cache of that file restores every tensor bit for bit with
the quantisation flags set."""
import ctypes
import os

import numpy as np
import pytest
import torch

import qcache_format as qf
import s2pamd
from gpu_util import S, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return s2pamd.load()


def tensor_of(t, arr):
    t.data, t.bytes, t.on_device, t.ndim = arr.data_ptr(), arr.numel() * arr.element_size(), 1, 1
    t.shape[0] = arr.numel()


def make_linears(seed):
    r = np.random.default_rng(seed)
    specs = []  # (name, kind, N, K, group, codes np, scales np)
    specs.append(("layers.3.attention.wo", 1, 48, 256, 0,
                  r.integers(-127, 128, (48, 256), dtype=np.int8),
                  r.random(48, dtype=np.float32)))
    specs.append(("layers.3.feed_forward.w13", 2, 64, 512, 32,
                  r.integers(0, 256, (64, 256), dtype=np.uint8),
                  r.random(64 * 16).astype(np.float16)))
    specs.append(("layers.3.feed_forward.w2", 3, 32, 128, 64,
                  r.integers(-8, 8, (32, 128), dtype=np.int8),
                  r.random(32 * 2).astype(np.float16)))
    keep, lins = [], []
    for name, kind, N, K, g, q, s in specs:
        lin = s2pamd.Linear()
        lin.in_features, lin.out_features = K, N
        lin.int8_ready, lin.q_group, lin.q_packed = 1, g, 1 if kind == 2 else 0
        qd, sd = to_dev(q), to_dev(s)
        keep += [qd, sd]
        tensor_of(lin.w_pack if kind == 2 else lin.w_int8, qd)
        tensor_of(lin.w_iscale, sd)
        lins.append(lin)
    return specs, lins, keep


def test_qcache_round_trip(lib, tmp_path):
    d = tmp_path / "model"
    d.mkdir()
    (d / "model.safetensors").write_bytes(b"z" * 64)
    specs, lins, keep = make_linears(3)
    qc = ctypes.c_void_p()
    s2pamd.check(lib.s2p_qcache_open(str(d).encode(), 2, ctypes.byref(qc)), "open")
    assert qc.value and lib.s2p_qcache_reading(qc) == 0
    for (name, *_), lin in zip(specs, lins):
        s2pamd.check(lib.s2p_qcache_put_linear(qc, name.encode(), ctypes.byref(lin), S()), name)
    s2pamd.check(lib.s2p_qcache_finish(qc, S()), "finish (write)")
    lib.s2p_qcache_free(qc)
    got = (d / "s2p_qcache.bin").read_bytes()
    want = qf.file_bytes(qf.fingerprint(d), [(n, k, N, K, g, q.tobytes(), s.tobytes())
                                             for n, k, N, K, g, q, s in specs])
    assert got == want, f"file differs from the layout ({len(got)} vs {len(want)} bytes)"
    assert not os.path.exists(str(d / "s2p_qcache.bin") + ".tmp")

    qc = ctypes.c_void_p()
    s2pamd.check(lib.s2p_qcache_open(str(d).encode(), 2, ctypes.byref(qc)), "reopen")
    assert lib.s2p_qcache_reading(qc) == 1
    try:
        for name, kind, N, K, g, q, s in specs:
            lin = s2pamd.Linear()
            assert lib.s2p_qcache_try_load(qc, name.encode(), K, N, ctypes.byref(lin), S()) == 1
            torch.cuda.synchronize()
            qt = lin.w_pack if kind == 2 else lin.w_int8
            from gpu_util import d2h
            assert np.array_equal(d2h(qt.data, q.nbytes, np.uint8), q.view(np.uint8).ravel())
            assert np.array_equal(d2h(lin.w_iscale.data, s.nbytes, np.uint8),
                                  s.view(np.uint8).ravel())
            assert (lin.int8_ready, lin.q_group, lin.q_packed) == (1, g, int(kind == 2))
            lib.s2p_tensor_free(ctypes.byref(qt))
            lib.s2p_tensor_free(ctypes.byref(lin.w_iscale))
        lin = s2pamd.Linear()
        assert lib.s2p_qcache_try_load(qc, b"not.there", 8, 8, ctypes.byref(lin), S()) == 0
        assert lib.s2p_qcache_try_load(qc, specs[0][0].encode(), 8, 8, ctypes.byref(lin), S()) == 0
        s2pamd.check(lib.s2p_qcache_finish(qc, S()), "finish (read)")
    finally:
        lib.s2p_qcache_free(qc)
    del keep


def test_qcache_file_shrinking_under_a_reader_is_a_miss(lib, tmp_path):
    """The reader keeps the file open and reads payloads on demand: when the
    file is cut short after the cache opened, a lookup whose payload is gone
    is a miss (no crash), and the linear passed in is left untouched."""
    d = tmp_path / "model"
    d.mkdir()
    (d / "model.safetensors").write_bytes(b"w" * 32)
    specs, _, keep = make_linears(5)
    path = d / "s2p_qcache.bin"
    path.write_bytes(qf.file_bytes(qf.fingerprint(d), [(n, k, N, K, g, q.tobytes(), s.tobytes())
                                                       for n, k, N, K, g, q, s in specs]))
    qc = ctypes.c_void_p()
    s2pamd.check(lib.s2p_qcache_open(str(d).encode(), 2, ctypes.byref(qc)), "open")
    try:
        assert lib.s2p_qcache_reading(qc) == 1
        name, kind, N, K, g, q, s = specs[-1]
        os.truncate(path, os.path.getsize(path) - 16)   # the last scales lose their tail
        lin = s2pamd.Linear()
        lin.in_features, lin.out_features = 7, 9
        assert lib.s2p_qcache_try_load(qc, name.encode(), K, N, ctypes.byref(lin), S()) == 0
        assert (lin.in_features, lin.out_features, lin.int8_ready) == (7, 9, 0)
        # an entry whose payload is still complete is served
        name0, kind0, N0, K0, *_ = specs[0]
        lin0 = s2pamd.Linear()
        assert lib.s2p_qcache_try_load(qc, name0.encode(), K0, N0, ctypes.byref(lin0), S()) == 1
        s2pamd.check(lib.s2p_qcache_finish(qc, S()), "finish (read)")
        lib.s2p_tensor_free(ctypes.byref(lin0.w_int8))
        lib.s2p_tensor_free(ctypes.byref(lin0.w_iscale))
    finally:
        lib.s2p_qcache_free(qc)
    del keep
