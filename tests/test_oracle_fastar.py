"""Pins of the oracle's fast-AR frame (or_fastar_frame, restating
src/fastar/fastar.cu:726-789) and VQ-embedding sum (or_vq_embed_add,
fastar.cu:104-127).  The reference ships no fast-AR fixture (its parity
fixtures are not in the repository), so the frame is pinned by what the
mathematics fixes:

* KV caching is a recomputation shortcut: step cb's output must equal the
  last row of an uncached causal forward over the whole sequence
  [hidden, emb[sem], emb[c1], ..] at positions 0..cb (pins the prime pass,
  the positions, the cache slots and the step inputs);
* with the attention and FFN outputs zeroed (wo and w2 scales 0) every layer
  is the identity, so code k is argmax(head(norm(emb[code k-1]))) whatever
  the hidden (pins the embedding table, the semantic seed, the clamp, the
  final norm and the head);
* the argmax is brute force (numpy, lowest index on ties).
The VQ sum is checked against a float64 sum, which equals the f32 sum of
ten bf16 values exactly when no rounding occurs (small-integer tables), and
on a case where one rounding of the whole sum differs from rounding after
every add."""
import numpy as np
import pytest

import pyoracle as po

DIM, FFN, CB = 2560, 9728, 4096


def _int8_linear(r, N, K, keep, zero=False):
    w = r.integers(-127, 128, (N, K), dtype=np.int8)
    s = np.full(N, 0.0 if zero else 1.0 / (np.sqrt(K) * 73.9), np.float32)
    keep.append((w, s))
    return po.make_linear(w, s, N, K, 0)


def _bf16(a):
    return po.f32_to_bf16(np.ascontiguousarray(a, np.float32))


@pytest.fixture(scope="module")
def weights():
    return _make(np.random.default_rng(8), zero=False)


def _make(r, zero):
    keep = []
    layers = []
    for _ in range(4):
        an = _bf16(1 + 0.02 * r.standard_normal(DIM))
        fn = _bf16(1 + 0.02 * r.standard_normal(DIM))
        keep += [an, fn]
        layers.append(po.OrLayerW(_int8_linear(r, 6144, DIM, keep),
                                  _int8_linear(r, DIM, 4096, keep, zero),
                                  _int8_linear(r, 2 * FFN, DIM, keep),
                                  _int8_linear(r, DIM, FFN, keep, zero),
                                  po.ptr(an), po.ptr(fn), None, None))
    norm = _bf16(1 + 0.02 * r.standard_normal(DIM))
    head = _int8_linear(r, CB, DIM, keep)
    emb = _bf16(r.standard_normal((CB, DIM)))
    keep += [norm, emb]
    faw = po.OrFaW((po.OrLayerW * 4)(*layers), po.ptr(norm), head, po.ptr(emb))
    return faw, keep, layers, norm, head, emb


def _hidden(seed):
    r = np.random.default_rng(seed)
    return _bf16(r.standard_normal(DIM)).reshape(DIM)


def _argmax(bits):
    v = po.bf16_to_f32(bits).astype(np.float64)
    return int(np.flatnonzero(v == v.max())[0])


def test_frame_equals_uncached_causal_forward(weights):
    faw, keep, layers, norm, head, emb = weights
    hidden = _hidden(1)
    sem = 1234
    codes, logits = po.fastar_frame(faw, hidden, sem)
    prev = [sem] + [int(c) for c in codes]
    for cb in (1, 4, 9):
        n = cb + 1
        x = np.empty((n, DIM), np.uint16)
        x[0] = hidden
        for j in range(1, n):
            x[j] = emb[prev[j - 1]]
        kc = np.zeros((8, 11, 128), np.uint16)
        vc = np.zeros((8, 11, 128), np.uint16)
        for lw in layers:
            kc[:] = 0
            vc[:] = 0
            po.layer(lw, x, n, kc, vc, 11, 0, np.arange(n))
        lg = po.linear_fwd(head, po.rms_norm(x[-1:], norm, 1, DIM), 1)[0]
        assert np.array_equal(lg, logits[cb - 1]), f"step {cb}"
        assert _argmax(lg) == codes[cb - 1]


def test_frame_with_identity_layers_is_an_embedding_chain():
    faw, keep, layers, norm, head, emb = _make(np.random.default_rng(2), zero=True)
    for sem, hid_seed in ((-9, 3), (99999, 4)):
        codes, logits = po.fastar_frame(faw, _hidden(hid_seed), sem)
        c = min(max(sem, 0), CB - 1)
        for k in range(9):
            # the hidden enters only through the attention, zeroed here
            lg = po.linear_fwd(head, po.rms_norm(emb[c][None], norm, 1, DIM), 1)[0]
            assert np.array_equal(lg, logits[k]), f"sem {sem} step {k + 1}"
            c = _argmax(lg)
            assert codes[k] == c


def test_vq_embed_add_exact_sum():
    r = np.random.default_rng(6)
    T = 3
    codes = r.integers(0, CB, (10, T)).astype(np.int32)
    codes[2, 0], codes[7, 2] = -1, CB + 5
    cl = np.clip(codes, 0, CB - 1)
    # small integers in the rows the codes select (elsewhere zero): every
    # partial sum is exact in f32 and bf16
    cbe = np.zeros((10 * CB, DIM), np.uint16)
    for k in range(10):
        cbe[k * CB + cl[k]] = _bf16(r.integers(-8, 9, (T, DIM)))
    rows = _bf16(r.integers(-4, 5, (T, DIM)))
    out = rows.copy()
    po.vq_embed_add(cbe, codes, out)
    want = po.bf16_to_f32(rows).astype(np.float64)
    for k in range(10):
        want = want + po.bf16_to_f32(cbe[k * CB + cl[k]]).astype(np.float64)
    assert np.array_equal(po.bf16_to_f32(out).astype(np.float64), want)
    # one rounding of the f32 sum: 1 + 3 * 2^-9 rounds to 1 + 2^-7 in bf16
    # (8 significant bits), while rounding after every add would keep 1
    cbe[:] = 0
    cbe[cl[0, 0], 0] = _bf16([1.0])[0]
    for k in (1, 2, 3):
        cbe[k * CB + cl[k, 0], 0] = _bf16([2.0 ** -9])[0]
    one = _bf16(np.zeros((T, DIM)))
    po.vq_embed_add(cbe, codes, one)
    assert po.bf16_to_f32(one)[0, 0] == np.float32(1.0 + 2.0 ** -7)
