"""The qcache sidecar layout written out independently (test
infrastructure): FNV-1a 64, the staleness fingerprint and the file writer,
restated from the documented format of the reference's
src/sched/qcache.c:1-16 (header) and :69-107 (fingerprint).  The library's
reader and writer are checked against these bytes."""
import os
import struct

FNV_BASIS = 0xCBF29CE484222325
FNV_PRIME = 0x100000001B3
MAGIC = b"S2PQC\x01\x00\x00"


def fnv1a(data, h=FNV_BASIS):
    for b in data:
        h = ((h ^ b) * FNV_PRIME) & 0xFFFFFFFFFFFFFFFF
    return h


def config_string(mode=2, int4=0, group="32", mse=1, packed=1, all_=0):
    return f"v1|mode={mode}|int4={int4}|g={group}|mse={mse}|pk={packed}|all={all_}"


def fingerprint(model_dir, mode=2):
    h = fnv1a(config_string(mode).encode())
    names = sorted(n for n in os.listdir(model_dir)
                   if len(n) > 12 and n.endswith(".safetensors"))
    for n in names:
        st = os.stat(os.path.join(model_dir, n))
        h = fnv1a(n.encode(), h)
        h = fnv1a(struct.pack("<q", st.st_size), h)
        h = fnv1a(struct.pack("<q", int(st.st_mtime)), h)
    return h


def file_bytes(fp, entries):
    """entries: (name, kind, N, K, group, codes bytes, scales bytes)"""
    table = 24 + sum(56 + len(e[0].encode()) for e in entries)
    off, offs = table, []
    for e in entries:
        q_off = (off + 255) & ~255
        off = q_off + len(e[5])
        s_off = (off + 255) & ~255
        off = s_off + len(e[6])
        offs.append((q_off, s_off))
    out = bytearray(MAGIC + struct.pack("<QII", fp, len(entries), 0))
    for e, (q_off, s_off) in zip(entries, offs):
        name = e[0].encode()
        out += struct.pack("<IIiiiIQQQQ", len(name), e[1], e[2], e[3], e[4], 0,
                           q_off, len(e[5]), s_off, len(e[6]))
        out += name
    for e, (q_off, s_off) in zip(entries, offs):
        out += b"\x00" * (q_off - len(out)) + e[5]
        out += b"\x00" * (s_off - len(out)) + e[6]
    return bytes(out)
