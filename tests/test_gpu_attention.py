"""Attention kernels vs the oracle: binary64 ground truth within 1e-2 (the
GPU kernel uses MFMA with bf16 probabilities; the oracle restates the
reference's fp32 order, or_attention / or_attention_split)."""
import numpy as np
import pytest

import pyoracle as po
import s2pamd
from gpu_util import P, S, assert_close_rel, bf16_bits, bf16_vals, empty, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return s2pamd.load()


def cache(seed, max_seq):
    r = np.random.default_rng(seed)
    kc = bf16_bits(r.standard_normal((8, max_seq, 128)).astype(np.float32))
    vc = bf16_bits(r.standard_normal((8, max_seq, 128)).astype(np.float32))
    return kc, vc


@pytest.mark.parametrize("rows,pos,max_seq", [(5, 512, 1024), (1, 0, 64), (37, 100, 256),
                                              (5, 2043, 2048), (8, 4000, 4096)])
def test_attention_contig(lib, rows, pos, max_seq):
    kc, vc = cache(rows + pos, max_seq)
    q = bf16_bits(np.random.default_rng(pos).standard_normal((rows, 4096)).astype(np.float32))
    out = empty((rows, 4096))
    s2pamd.hip_check(lib.s2pk_attention(P(to_dev(q)), P(to_dev(kc)), P(to_dev(vc)), P(out), rows,
                                        32, 8, 128, pos, max_seq, S()))
    got = bf16_vals(to_host(out, np.uint16))
    exact = po.attention_f64(q, kc, vc, rows, 32, 8, 128, pos, max_seq)
    assert np.max(np.abs(got - exact)) < 2e-2, np.max(np.abs(got - exact))
    ref = bf16_vals(po.attention(q, kc, vc, rows, 32, 8, 128, pos, max_seq))
    assert np.max(np.abs(got - ref)) < 2e-2


def test_attention_decode_ptrs(lib):
    rows, max_seq = 6, 2048
    caches = [cache(50 + r, max_seq) for r in range(rows)]
    pos = np.array([0, 1, 63, 64, 1000, 2047], np.int32)
    q = bf16_bits(np.random.default_rng(9).standard_normal((rows, 4096)).astype(np.float32))
    dk = [to_dev(c[0]) for c in caches]
    dv = [to_dev(c[1]) for c in caches]
    pk = to_dev(np.array([t.data_ptr() for t in dk], np.int64))
    pv = to_dev(np.array([t.data_ptr() for t in dv], np.int64))
    max_len = int(pos.max()) + 1
    nf = lib.s2pk_attention_part_floats(rows, 32, max_len)
    part = empty((nf,), dtype=__import__("torch").float32)
    for fn in ("decode", "ptrs"):
        out = empty((rows, 4096))
        if fn == "decode":
            s2pamd.hip_check(lib.s2pk_attention_decode(P(to_dev(q)), P(pk), P(pv), P(out), rows,
                                                       32, 8, 128, P(to_dev(pos)), max_seq,
                                                       max_len, P(part), S()))
        else:
            s2pamd.hip_check(lib.s2pk_attention_ptrs(P(to_dev(q)), P(pk), P(pv), P(out), rows, 32,
                                                     8, 128, P(to_dev(pos)), max_seq, S()))
        got = bf16_vals(to_host(out, np.uint16))
        for r in range(rows):
            exact = po.attention_f64(q[r:r + 1], caches[r][0], caches[r][1], 1, 32, 8, 128,
                                     int(pos[r]), max_seq)
            assert np.max(np.abs(got[r] - exact[0])) < 2e-2, (fn, r)


def test_attention_single_key_returns_v(lib):
    max_seq = 32
    kc, vc = cache(3, max_seq)
    q = bf16_bits(np.random.default_rng(4).standard_normal((1, 4096)).astype(np.float32))
    out = empty((1, 4096))
    s2pamd.hip_check(lib.s2pk_attention(P(to_dev(q)), P(to_dev(kc)), P(to_dev(vc)), P(out), 1,
                                        32, 8, 128, 0, max_seq, S()))
    got = to_host(out, np.uint16).reshape(32, 128)
    assert np.array_equal(got, np.repeat(vc[:, 0, :], 4, axis=0))
