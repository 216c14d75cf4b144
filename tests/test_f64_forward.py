"""Pins the binary64 ground-truth layer (tests/f64_forward.py) against the
reference-order oracle layer (or_layer) on small shapes: both restate
slowar.c:156-260, one exactly, one with the reference's bf16 rounding
points, so they must agree to bf16-level error.  A convention slip in either
(rope pairing, GQA head map, norm axis, gate/up order, tree visibility)
gives O(1) differences."""
import numpy as np
import pytest

import f64_forward as f64
import pyoracle as po


def rand_int4(r, N, K, w_rms):
    w = r.integers(0, 256, (N, K // 2), dtype=np.uint8)
    s = (np.abs(r.standard_normal((N, K // 32))) * w_rms / 4.61).astype(np.float16).view(np.uint16)
    return w, s


def rand_int8(r, N, K, w_rms):
    w = r.integers(-128, 128, (N, K), dtype=np.int8)
    s = (np.abs(r.standard_normal(N)) * w_rms / 73.9).astype(np.float32)
    return w, s


@pytest.mark.parametrize("int4,parent,L", [(True, [-1, 0, 1, 2, 3], 37),
                                           (False, [-1, 0, 0, 1, 2, 2, 5], 20)])
def test_f64_layer_matches_oracle_layer(int4, parent, L):
    r = np.random.default_rng(3 if int4 else 4)
    dim, ffn, ctx = 256, 512, 64
    R = len(parent)
    shapes = {"wqkv": (6144, dim), "wo": (dim, 4096), "gate_up": (2 * ffn, dim), "w2": (dim, ffn)}
    raw, lins, W = {}, [], {}
    for name, (N, K) in shapes.items():
        w, s = (rand_int4 if int4 else rand_int8)(r, N, K, 1 / np.sqrt(K))
        raw[name] = (w, s)
        lins.append(po.make_linear(w, s, N, K, 32 if int4 else 0))
        W[name] = f64.dequant(w, s, N, K)
    norms = [po.f32_to_bf16(1 + 0.02 * r.standard_normal(n)) for n in (dim, dim, 128, 128)]
    for key, nb in zip(("attn_norm", "ffn_norm", "q_norm", "k_norm"), norms):
        W[key] = f64.bf(nb)
    lw = po.OrLayerW(*lins, *(po.ptr(n) for n in norms))
    kv = po.f32_to_bf16(r.standard_normal((16, ctx, 128)))
    x = po.f32_to_bf16(r.standard_normal((R, dim)))
    depth, vis = [0] * R, np.zeros(R, np.uint64)
    for i in range(R):
        if i:
            depth[i] = depth[parent[i]] + 1
        m, j = 0, i
        while j >= 0:
            m |= 1 << j
            j = parent[j]
        vis[i] = m
    pos = np.array([L + d for d in depth], np.int32)
    chain = all(parent[i] == i - 1 for i in range(1, R))
    xo = x.copy()
    kc, vc = np.ascontiguousarray(kv[:8]), np.ascontiguousarray(kv[8:])
    po.layer(lw, xo, R, kc, vc, ctx, L, pos, None if chain else vis)
    want = f64.forward([W], np.ones(dim), np.eye(dim), x, kv[None], L, parent)
    # forward() ends with an rms norm; compare the normalised states
    got = f64.rms(f64.bf(xo), np.ones(dim))
    err = np.abs(got - want)
    assert np.sqrt(np.mean(err ** 2)) < 1e-2, np.sqrt(np.mean(err ** 2))
    assert err.max() < 5e-2, err.max()
    # a perturbed convention fails: swapping gate and up
    W2 = dict(W)
    W2["gate_up"] = np.concatenate([W["gate_up"][ffn:], W["gate_up"][:ffn]])
    bad = f64.forward([W2], np.ones(dim), np.eye(dim), x, kv[None], L, parent)
    assert np.sqrt(np.mean((got - bad) ** 2)) > 0.1
