"""INT8 / INT4 KV cache on the GPU through the C ABI (s2pk_kv_append8,
s2pk_kv_append8_ptrs, s2pk_attention8, s2pk_attention8_decode) against the
oracle restatement of kernels.cu:510-946: quantised payloads and f16 scales
bit-exact; the single-pass attention bit-exact (same arithmetic order); the
split decode within 5e-3 of the single pass and 1e-2 of binary64 per row and
head (L2), its splits merged in another order."""
import ctypes

import numpy as np
import pytest
import torch

import pyoracle as po
import s2pamd
from gpu_util import P, S, bf16_bits, empty, to_dev, to_host
from test_oracle_kv8 import HD, KVH, caches

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return s2pamd.load()


def dev_caches(host):
    return [[to_dev(a.copy()) for a in group] for group in host]


def ptr_array(ts):
    return to_dev(np.array([t.data_ptr() for t in ts], np.int64))


@pytest.mark.parametrize("bw", [8, 4])
def test_append8_bit_exact(lib, bw):
    r = np.random.default_rng(10 + bw)
    max_seq, rows, pos0 = 64, 5, 17
    k = bf16_bits(r.standard_normal((rows, KVH * HD)).astype(np.float32))
    v = bf16_bits(r.standard_normal((rows, KVH * HD)).astype(np.float32) * 3)
    k[1, :32] = 0  # a zero group
    host = caches(1, max_seq, bw)
    dkc, dvc, dks, dvs = dev_caches(host)
    s2pamd.hip_check(lib.s2pk_kv_append8(P(to_dev(k)), P(to_dev(v)), P(dkc[0]), P(dvc[0]),
                                         P(dks[0]), P(dvs[0]), rows, KVH, HD, pos0, max_seq, bw,
                                         S()), "append8")
    po.kv_append8(k, v, *host, rows, KVH, pos0, None, max_seq, bw)
    for d, h in zip((dkc[0], dvc[0], dks[0], dvs[0]), (host[0][0], host[1][0], host[2][0],
                                                       host[3][0])):
        assert np.array_equal(to_host(d, h.dtype).reshape(h.shape), h)
    # ptrs form: rows to their own caches and slots
    n = 3
    host = caches(n, max_seq, bw)
    devs = dev_caches(host)
    slots = np.array([0, 63, 9], np.int32)
    k3 = np.ascontiguousarray(k[:n])
    v3 = np.ascontiguousarray(v[:n])
    s2pamd.hip_check(lib.s2pk_kv_append8_ptrs(P(to_dev(k3)), P(to_dev(v3)), P(ptr_array(devs[0])),
                                              P(ptr_array(devs[1])), P(ptr_array(devs[2])),
                                              P(ptr_array(devs[3])), n, KVH, HD,
                                              P(to_dev(slots)), max_seq, bw, S()), "append8 ptrs")
    po.kv_append8(k3, v3, *host, n, KVH, 0, slots, max_seq, bw)
    for g in range(4):
        for i in range(n):
            h = host[g][i]
            assert np.array_equal(to_host(devs[g][i], h.dtype).reshape(h.shape), h), (g, i)


def fill(r, n, max_seq, bw, lens):
    """n caches quantised from N(0,1) K/V at slots [0, lens[i])."""
    host = caches(n, max_seq, bw)
    for i in range(n):
        kv = bf16_bits(r.standard_normal((lens[i], KVH * HD)).astype(np.float32))
        vv = bf16_bits(r.standard_normal((lens[i], KVH * HD)).astype(np.float32))
        po.kv_append8(kv, vv, [host[0][i]], [host[1][i]], [host[2][i]], [host[3][i]], lens[i],
                      KVH, 0, None, max_seq, bw)
    return host


@pytest.mark.parametrize("bw", [8, 4])
def test_attention8_bit_exact(lib, bw):
    r = np.random.default_rng(20 + bw)
    max_seq, rows, pos0, qh = 512, 5, 300, 32
    host = fill(r, 1, max_seq, bw, [pos0 + rows])
    devs = dev_caches(host)
    q = bf16_bits(r.standard_normal((rows, qh * HD)).astype(np.float32))
    out = empty((rows, qh * HD))
    s2pamd.hip_check(lib.s2pk_attention8(P(to_dev(q)), P(devs[0][0]), P(devs[1][0]),
                                         P(devs[2][0]), P(devs[3][0]), P(out), rows, qh, KVH, HD,
                                         pos0, max_seq, bw, S()), "attention8")
    want = po.attention8(q, host[0][0], host[1][0], host[2][0], host[3][0], rows, qh, KVH, pos0,
                         max_seq, bw)
    got = to_host(out, np.uint16)
    assert np.array_equal(got, want), f"{int((got != want).sum())} of {got.size} differ"


@pytest.mark.parametrize("bw", [8, 4])
def test_attention8_decode(lib, bw):
    r = np.random.default_rng(30 + bw)
    max_seq, qh = 1664, 32
    pos = np.array([100, 700, 1500, 0], np.int32)
    n = len(pos)
    host = fill(r, n, max_seq, bw, [int(p) + 1 for p in pos])
    devs = dev_caches(host)
    q = bf16_bits(r.standard_normal((n, qh * HD)).astype(np.float32))
    max_len = int(pos.max()) + 1
    part = torch.empty(lib.s2pk_attention_part_floats(n, qh, max_len), dtype=torch.float32,
                       device="cuda")
    out = empty((n, qh * HD))
    s2pamd.hip_check(lib.s2pk_attention8_decode(P(to_dev(q)), P(ptr_array(devs[0])),
                                                P(ptr_array(devs[1])), P(ptr_array(devs[2])),
                                                P(ptr_array(devs[3])), P(out), n, qh, KVH, HD,
                                                P(to_dev(pos)), max_seq, max_len, P(part), bw,
                                                S()), "attention8 decode")
    got = po.bf16_to_f32(to_host(out, np.uint16)).reshape(n, qh, HD)
    truth = po.attention8_f64(q, *host, n, qh, KVH, pos, max_seq, bw).reshape(n, qh, HD)
    for i in range(n):
        single = po.bf16_to_f32(po.attention8(np.ascontiguousarray(q[i:i + 1]), host[0][i],
                                              host[1][i], host[2][i], host[3][i], 1, qh, KVH,
                                              int(pos[i]), max_seq, bw)).reshape(qh, HD)
        e1 = np.linalg.norm(got[i] - single, axis=1) / np.linalg.norm(single, axis=1)
        e2 = np.linalg.norm(got[i] - truth[i], axis=1) / np.linalg.norm(truth[i], axis=1)
        assert e1.max() < 5e-3, (i, e1.max())
        assert e2.max() < 1e-2, (i, e2.max())


def test_kv8_argument_errors(lib):
    bad = lib.s2pk_attention8(None, None, None, None, None, None, 1, 32, 8, 64, 0, 16, 8, S())
    assert bad != 0
    assert lib.s2pk_kv_append8(None, None, None, None, None, None, 1, 8, 128, 0, 16, 5, S()) != 0
    assert lib.s2pk_kv_append8(None, None, None, None, None, None, 0, 8, 128, 0, 16, 8, S()) == 0
