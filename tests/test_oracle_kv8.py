"""CPU oracle of the INT8 / INT4 KV cache (kernels.cu:510-946), pinned by
closed forms and bounds of the quantiser and by binary64 attention over the
dequantised cache.  Oracle only; the GPU parity is tests/test_gpu_kv8.py."""
import numpy as np
import pytest

import pyoracle as po

HD, KVH = 128, 8


def caches(n, max_seq, bw):
    el = HD if bw == 8 else HD // 2
    kc = [np.zeros((KVH, max_seq, el), np.int8) for _ in range(n)]
    vc = [np.zeros((KVH, max_seq, el), np.int8) for _ in range(n)]
    ks = [np.zeros((KVH, max_seq, 4), np.uint16) for _ in range(n)]
    vs = [np.zeros((KVH, max_seq, 4), np.uint16) for _ in range(n)]
    return kc, vc, ks, vs


def decode(pay, bw):
    """payload [..., el] -> int values [..., 128] (bw 4: two's complement nibbles)"""
    if bw == 8:
        return pay.astype(np.int32)
    b = pay.view(np.uint8).astype(np.int32)
    lo, hi = b & 0xF, b >> 4
    out = np.empty(pay.shape[:-1] + (HD,), np.int32)
    out[..., 0::2] = np.where(lo >= 8, lo - 16, lo)
    out[..., 1::2] = np.where(hi >= 8, hi - 16, hi)
    return out


@pytest.mark.parametrize("bw", [8, 4])
def test_quant_closed_form(bw):
    """Groups whose absmax is QMAX * 2^-e and whose values are integer
    multiples of 2^-e: the scale is exactly 2^-e and the values come back as
    the integers."""
    qmax = 127 if bw == 8 else 7
    r = np.random.default_rng(1)
    rows = 3
    ints = r.integers(-qmax, qmax + 1, (rows, KVH, HD))
    ints[..., ::32] = qmax * np.where(r.random((rows, KVH, 4)) < 0.5, -1, 1)
    e = 6
    x = po.f32_to_bf16((ints * 2.0 ** -e).astype(np.float32)).reshape(rows, KVH * HD)
    kc, vc, ks, vs = caches(1, 16, bw)
    po.kv_append8(x, x, kc, vc, ks, vs, rows, KVH, 5, None, 16, bw)
    got = decode(kc[0][:, 5:5 + rows], bw)
    assert np.array_equal(got, ints.transpose(1, 0, 2))
    assert np.array_equal(decode(vc[0][:, 5:5 + rows], bw), got)
    assert np.all(ks[0][:, 5:5 + rows] == np.float16(2.0 ** -e).view(np.uint16))
    # untouched slots stay zero
    assert not kc[0][:, :5].any() and not kc[0][:, 5 + rows:].any()


@pytest.mark.parametrize("bw", [8, 4])
def test_quant_bounds(bw):
    """Random rows: |q| <= QMAX, the group absmax lands on +-QMAX (or one
    below, the f16 scale rounding), and every dequantised value is within
    half a scale step (plus the f16 scale's rounding) of the input; a zero
    group has scale 0 and values 0."""
    qmax = 127 if bw == 8 else 7
    r = np.random.default_rng(2)
    rows = 4
    xf = r.standard_normal((rows, KVH * HD)).astype(np.float32)
    xf[0, :32] = 0.0
    x = po.f32_to_bf16(xf)
    xv = po.bf16_to_f32(x).reshape(rows, KVH, 4, 32)
    kc, vc, ks, vs = caches(2, 8, bw)
    slots = np.array([7, 0, 3, 6], np.int32)
    # ptrs form: row r -> cache r % 2
    kcp = [kc[i % 2] for i in range(rows)]
    vcp = [vc[i % 2] for i in range(rows)]
    ksp = [ks[i % 2] for i in range(rows)]
    vsp = [vs[i % 2] for i in range(rows)]
    po.kv_append8(x, x, kcp, vcp, ksp, vsp, rows, KVH, 0, slots, 8, bw)
    for i in range(rows):
        q = decode(kcp[i][:, slots[i]], bw).reshape(KVH, 4, 32)
        s = ksp[i][:, slots[i]].view(np.float16).astype(np.float64)
        assert np.all(np.abs(q) <= qmax)
        amax = np.abs(xv[i]).max(axis=2)
        qm = np.abs(q).max(axis=2)
        nz = amax > 0
        assert np.all(qm[nz] >= qmax - 1)
        deq = q * s[..., None]
        step = s[..., None] * (0.5 + qmax * 2.0 ** -10)
        assert np.all(np.abs(deq - xv[i]) <= step + 1e-12)
    assert np.all(ksp[0][0, slots[0], 0] == 0) and not kcp[0][0, slots[0], :32 if bw == 8 else 16].any()


@pytest.mark.parametrize("bw", [8, 4])
def test_attention8_vs_binary64(bw):
    """or_attention8 (reference order, fp32) against binary64 attention over
    the same dequantised cache, rows at pos0.. with causal visibility."""
    r = np.random.default_rng(3)
    max_seq, pos0, rows, qh = 400, 260, 5, 32
    kc, vc, ks, vs = caches(1, max_seq, bw)
    n = pos0 + rows
    kv = po.f32_to_bf16(r.standard_normal((n, KVH * HD)).astype(np.float32))
    vv = po.f32_to_bf16(r.standard_normal((n, KVH * HD)).astype(np.float32))
    po.kv_append8(kv, vv, kc, vc, ks, vs, n, KVH, 0, None, max_seq, bw)
    q = po.f32_to_bf16(r.standard_normal((rows, qh * HD)).astype(np.float32))
    got = po.bf16_to_f32(po.attention8(q, kc[0], vc[0], ks[0], vs[0], rows, qh, KVH, pos0,
                                       max_seq, bw)).reshape(rows, qh, HD)
    want = po.attention8_f64(q, kc * rows, vc * rows, ks * rows, vs * rows, rows, qh, KVH,
                             np.arange(pos0, pos0 + rows), max_seq, bw).reshape(rows, qh, HD)
    err = np.linalg.norm(got - want, axis=2) / np.linalg.norm(want, axis=2)
    assert err.max() < 1e-2, err.max()
    # a key moved to another slot: every row's output changes (indexing)
    kc2 = [kc[0].copy()]
    kc2[0][:, [10, 11]] = kc2[0][:, [11, 10]]
    got2 = po.bf16_to_f32(po.attention8(q, kc2[0], vc[0], ks[0], vs[0], rows, qh, KVH, pos0,
                                        max_seq, bw)).reshape(rows, qh, HD)
    assert np.any(got2 != got)


def test_attention8_single_slot_returns_v():
    """One visible slot: the output is that slot's dequantised V, rounded."""
    r = np.random.default_rng(4)
    kc, vc, ks, vs = caches(1, 4, 8)
    kv = po.f32_to_bf16(r.standard_normal((1, KVH * HD)).astype(np.float32))
    vv = po.f32_to_bf16(r.standard_normal((1, KVH * HD)).astype(np.float32))
    po.kv_append8(kv, vv, kc, vc, ks, vs, 1, KVH, 0, None, 4, 8)
    q = po.f32_to_bf16(r.standard_normal((1, 32 * HD)).astype(np.float32))
    got = po.attention8(q, kc[0], vc[0], ks[0], vs[0], 1, 32, KVH, 0, 4, 8).reshape(32, HD)
    deq = (vc[0][:, 0].astype(np.float32).reshape(KVH, 4, 32) *
           vs[0][:, 0].view(np.float16).astype(np.float32)[..., None]).reshape(KVH, HD)
    want = po.f32_to_bf16(np.repeat(deq, 4, axis=0))
    assert np.array_equal(got, want)
