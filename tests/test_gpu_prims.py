"""Transformer primitives (kernels.h / slowar_kernels.h launchers) vs the CPU
oracle: bit-exact (same rounding points, same reduction trees, the rule's
1/sqrt and binary64 pow/cos/sin rounded once)."""
import ctypes

import numpy as np
import pytest
import torch

import pyoracle as po
import s2pamd
from gpu_util import P, S, bf16_bits, empty, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return s2pamd.load()


def rnd(seed, shape, sd=1.0):
    return bf16_bits(np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * sd)


def test_rms_norm(lib):
    rows, width = 5, 2560
    x, w = rnd(1, (rows, width), 3.0), rnd(2, (width,), 0.1)
    w = bf16_bits(1 + po.bf16_to_f32(w))
    y = empty((rows, width))
    s2pamd.hip_check(lib.s2pk_rms_norm(P(to_dev(x)), P(to_dev(w)), P(y), rows, width, 1e-6, S()))
    assert np.array_equal(to_host(y, np.uint16), po.rms_norm(x, w, rows, width))


def test_qk_norm(lib):
    rows, heads = 5, 32
    x, w = rnd(3, (rows, heads * 128)), bf16_bits(1 + 0.05 * np.arange(128, dtype=np.float32) / 128)
    t = to_dev(x)
    s2pamd.hip_check(lib.s2pk_qk_norm(P(t), P(to_dev(w)), rows, heads, 128, 1e-6, S()))
    assert np.array_equal(to_host(t, np.uint16), po.qk_norm(x, w, rows, heads))


@pytest.mark.parametrize("pos0", [0, 7, 2048, 8191])
def test_rope(lib, pos0):
    rows = 5
    q, k = rnd(4, (rows, 32 * 128)), rnd(5, (rows, 8 * 128))
    tq, tk = to_dev(q), to_dev(k)
    s2pamd.hip_check(lib.s2pk_rope(P(tq), P(tk), rows, 32, 8, 128, pos0, 1e6, S()))
    assert np.array_equal(to_host(tq, np.uint16), po.rope(q, rows, 32, 128, pos0=pos0))
    assert np.array_equal(to_host(tk, np.uint16), po.rope(k, rows, 8, 128, pos0=pos0))
    pos = np.array([3, 100, 4097, 2050, 0], np.int32)
    tq, tk = to_dev(q), to_dev(k)
    s2pamd.hip_check(lib.s2pk_rope_pos(P(tq), P(tk), rows, 32, 8, 128, P(to_dev(pos)), 1e6, S()))
    assert np.array_equal(to_host(tq, np.uint16), po.rope(q, rows, 32, 128, pos=pos))


def test_kv_append_and_ptrs(lib):
    rows, max_seq = 5, 64
    k, v = rnd(6, (rows, 1024)), rnd(7, (rows, 1024))
    kc = np.zeros((8, max_seq, 128), np.uint16)
    vc = np.zeros((8, max_seq, 128), np.uint16)
    tkc, tvc = to_dev(kc), to_dev(vc)
    s2pamd.hip_check(lib.s2pk_kv_append(P(to_dev(k)), P(to_dev(v)), P(tkc), P(tvc), rows, 8, 128,
                                        17, max_seq, S()))
    po.lib().or_kv_append(po.ptr(k), po.ptr(v), po.ptr(kc), po.ptr(vc), rows, 8, 128, 17, None,
                          max_seq)
    assert np.array_equal(to_host(tkc, np.uint16), kc) and np.array_equal(to_host(tvc, np.uint16), vc)
    # per-row caches and positions
    caches_k = [to_dev(np.zeros((8, max_seq, 128), np.uint16)) for _ in range(rows)]
    caches_v = [to_dev(np.zeros((8, max_seq, 128), np.uint16)) for _ in range(rows)]
    pk = to_dev(np.array([t.data_ptr() for t in caches_k], np.int64))
    pv = to_dev(np.array([t.data_ptr() for t in caches_v], np.int64))
    pos = np.array([0, 5, 63, 9, 1], np.int32)
    s2pamd.hip_check(lib.s2pk_kv_append_ptrs(P(to_dev(k)), P(to_dev(v)), P(pk), P(pv), rows, 8,
                                             128, P(to_dev(pos)), max_seq, S()))
    for r in range(rows):
        hk = to_host(caches_k[r], np.uint16)
        assert np.array_equal(hk[:, pos[r], :], k[r].reshape(8, 128))
        assert np.count_nonzero(hk) == np.count_nonzero(k[r])


def test_qkv_split_silu_add(lib):
    rows = 5
    qkv = rnd(8, (rows, 6144))
    q, k, v = empty((rows, 4096)), empty((rows, 1024)), empty((rows, 1024))
    s2pamd.hip_check(lib.s2pk_qkv_split(P(to_dev(qkv)), P(q), P(k), P(v), rows, 4096, 1024, S()))
    assert np.array_equal(to_host(q, np.uint16), qkv[:, :4096])
    assert np.array_equal(to_host(v, np.uint16), qkv[:, 5120:])
    gu = rnd(9, (rows, 2 * 9728), 4.0)
    h = empty((rows, 9728))
    s2pamd.hip_check(lib.s2pk_silu_mul(P(to_dev(gu)), P(h), rows, 9728, S()))
    assert np.array_equal(to_host(h, np.uint16), po.silu_mul(gu, rows, 9728))
    y, x = rnd(10, (rows, 2560), 30.0), rnd(11, (rows, 2560))
    ty = to_dev(y)
    s2pamd.hip_check(lib.s2pk_add(P(ty), P(to_dev(x)), rows * 2560, S()))
    assert np.array_equal(to_host(ty, np.uint16), po.add(y, x))


def test_rows_zero_is_success(lib):
    assert lib.s2pk_rms_norm(None, None, None, 0, 2560, 1e-6, S()) == 0
    assert lib.s2pk_attention(None, None, None, None, 0, 32, 8, 128, 0, 16, S()) == 0


def test_f2bf_matches_rule(lib):
    """The hardware float -> bf16 conversion the kernels use equals the
    rule's rounding (or_f2bf: nearest even, NaN quieted with its payload's
    top bits) on random bit patterns and the edge cases: ties, carries into
    the exponent, overflow to inf, infinities, NaN payloads, subnormals."""
    r = np.random.default_rng(77)
    bits = r.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    edge = []
    for sign in (0, 0x80000000):
        for e in (0x00000000, 0x00800000, 0x3F800000, 0x7F000000, 0x7F800000):
            for m in (0, 1, 0x7FFF, 0x8000, 0x8001, 0x18000, 0x10000, 0x7FFFFF, 0x7F8000,
                      0x400000, 0x400001, 0x3FFFFF):
                edge.append(sign | e | m)
    bits = np.concatenate([bits, np.array(edge, np.uint32)])
    x = bits.view(np.float32)
    out = empty((x.size,))
    s2pamd.hip_check(lib.s2p_test_f2bf(P(to_dev(x)), P(out), x.size, S()))
    got = to_host(out, np.uint16)
    want = po.f32_to_bf16(x)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(bits[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]


@pytest.mark.parametrize("vocab,off", [(155776, 0), (4097, 0), (4097, 3), (1, 0)])
def test_sample_prepare_widens_exactly(lib, vocab, off):
    """s2pk_sample_prepare (kernels.h:65-66): f32 scratch = the bf16 logits,
    exactly, on aligned and misaligned buffers and ragged lengths; nothing
    past vocab is written."""
    r = np.random.default_rng(vocab + off)
    x = bf16_bits(r.standard_normal(vocab + 8).astype(np.float32) * 4.0)
    x[:4] = bf16_bits(np.array([np.inf, -np.inf, 0.0, -0.0], np.float32))[: min(4, vocab + 8)]
    tx = to_dev(x)
    out = torch.full((vocab + 16,), 7.0, dtype=torch.float32, device="cuda")
    xp = tx.data_ptr() + 2 * off
    yp = out.data_ptr() + 4 * off
    s2pamd.hip_check(lib.s2pk_sample_prepare(ctypes.c_void_p(xp), ctypes.c_void_p(yp), vocab, S()))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = po.bf16_to_f32(x[off:off + vocab])
    assert np.array_equal(got[off:off + vocab].view(np.uint32), want.view(np.uint32))
    assert np.all(got[:off] == 7.0) and np.all(got[off + vocab:] == 7.0)
    assert lib.s2pk_sample_prepare(None, None, 0, S()) == 0
