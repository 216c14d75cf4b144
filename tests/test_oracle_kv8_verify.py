"""CPU oracle of the verify path over the INT8 / INT4 KV cache: the attention
with tree visibility (or_attention8_vis) and the layer (or_layer8).

Pins: with chain visibility the masked attention equals the causal
reference-order kernel bit for bit; with a tree it matches binary64
attention over a cache compacted to the row's visible slots; or_layer8
appends exactly the quantisation of what the bf16-cache layer appends (same
qkv, qk-norm and RoPE), and its output tracks the bf16-cache layer to the
quantisation error.  Oracle only; the GPU parity is
tests/test_gpu_verify_kv8.py."""
import numpy as np
import pytest

import pyoracle as po
from test_f64_forward import rand_int4
from test_oracle_kv8 import HD, KVH, caches, decode

TREE = [-1, 0, 0, 1, 1, 2, 5, 3]


def masks(parent):
    R = len(parent)
    depth, vis = [0] * R, np.zeros(R, np.uint64)
    for i in range(R):
        if i:
            depth[i] = depth[parent[i]] + 1
        m, j = 0, i
        while j >= 0:
            m |= 1 << j
            j = parent[j]
        vis[i] = m
    return np.array(depth), vis


def filled(r, n, max_seq, bw):
    kc, vc, ks, vs = caches(1, max_seq, bw)
    kv = po.f32_to_bf16(r.standard_normal((n, KVH * HD)).astype(np.float32))
    vv = po.f32_to_bf16(r.standard_normal((n, KVH * HD)).astype(np.float32))
    po.kv_append8(kv, vv, kc, vc, ks, vs, n, KVH, 0, None, max_seq, bw)
    return kc[0], vc[0], ks[0], vs[0]


@pytest.mark.parametrize("bw", [8, 4])
def test_vis_chain_equals_causal(bw):
    r = np.random.default_rng(11)
    max_seq, L, R = 300, 250, 5
    kc, vc, ks, vs = filled(r, L + R, max_seq, bw)
    q = po.f32_to_bf16(r.standard_normal((R, 32 * HD)).astype(np.float32))
    _, vis = masks([-1, 0, 1, 2, 3])
    a = po.attention8_vis(q, kc, vc, ks, vs, R, 32, KVH, L, vis, max_seq, bw)
    b = po.attention8(q, kc, vc, ks, vs, R, 32, KVH, L, max_seq, bw)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("bw", [8, 4])
def test_vis_tree_vs_binary64_compacted(bw):
    """Row r sees [0, L) and its ancestors' slots: binary64 attention over a
    per-row cache holding exactly those slots, in order, agrees; changing an
    invisible slot changes nothing, a visible one changes the row."""
    r = np.random.default_rng(12)
    max_seq, L = 300, 140
    R = len(TREE)
    depth, vis = masks(TREE)
    kc, vc, ks, vs = filled(r, L + R, max_seq, bw)
    q = po.f32_to_bf16(r.standard_normal((R, 32 * HD)).astype(np.float32))
    got = po.bf16_to_f32(po.attention8_vis(q, kc, vc, ks, vs, R, 32, KVH, L, vis, max_seq, bw))
    cks, cvs, ckss, cvss = [], [], [], []
    for i in range(R):
        sl = list(range(L)) + [L + b for b in range(R) if (int(vis[i]) >> b) & 1]
        for src, dst in ((kc, cks), (vc, cvs), (ks, ckss), (vs, cvss)):
            c = np.zeros_like(src)
            c[:, :len(sl)] = src[:, sl]
            dst.append(c)
    want = po.attention8_f64(q, cks, cvs, ckss, cvss, R, 32, KVH, L + depth, max_seq, bw)
    g, w = got.reshape(R, 32, HD), want.reshape(R, 32, HD)
    err = np.linalg.norm(g - w, axis=2) / np.linalg.norm(w, axis=2)
    assert err.max() < 1e-2, err.max()
    # node 4's slot is invisible to row 2 (sibling subtree) and visible to row 4
    kc2 = kc.copy()
    kc2[:, L + 4] = np.roll(kc2[:, L + 4], 7, axis=1)
    got2 = po.bf16_to_f32(po.attention8_vis(q, kc2, vc, ks, vs, R, 32, KVH, L, vis, max_seq, bw))
    assert np.array_equal(got2[2], got[2])
    assert not np.array_equal(got2[4], got[4])


@pytest.mark.parametrize("bw,parent", [(8, [-1, 0, 1, 2, 3]), (4, TREE)])
def test_layer8_tracks_bf16_layer(bw, parent):
    r = np.random.default_rng(13)
    dim, ffn, ctx, L = 256, 512, 96, 60
    R = len(parent)
    shapes = {"wqkv": (6144, dim), "wo": (dim, 4096), "gate_up": (2 * ffn, dim), "w2": (dim, ffn)}
    lins, keep = [], []  # make_linear holds pointers: keep the arrays alive
    for name, (N, K) in shapes.items():
        w, s = rand_int4(r, N, K, 1 / np.sqrt(K))
        keep.append((w, s))
        lins.append(po.make_linear(w, s, N, K, 32))
    norms = [po.f32_to_bf16(1 + 0.02 * r.standard_normal(n)) for n in (dim, dim, 128, 128)]
    lw = po.OrLayerW(*lins, *(po.ptr(n) for n in norms))
    # prefix: quantised cache, and its dequantised values (bf16) for the bf16 layer
    kc8, vc8, ks8, vs8 = filled(r, L, ctx, bw)
    deq_k = decode(kc8, bw) * ks8.view(np.float16).astype(np.float32).repeat(32, axis=2)
    deq_v = decode(vc8, bw) * vs8.view(np.float16).astype(np.float32).repeat(32, axis=2)
    kc = po.f32_to_bf16(deq_k.astype(np.float32)).reshape(KVH, ctx, HD)
    vc = po.f32_to_bf16(deq_v.astype(np.float32)).reshape(KVH, ctx, HD)
    depth, vis = masks(parent)
    chain = all(parent[i] == i - 1 for i in range(1, R))
    pos = (L + depth).astype(np.int32)
    x = po.f32_to_bf16(r.standard_normal((R, dim)).astype(np.float32))
    x8, xb = x.copy(), x.copy()
    kc8_0, vc8_0, ks8_0, vs8_0 = kc8.copy(), vc8.copy(), ks8.copy(), vs8.copy()
    po.layer8(lw, x8, R, kc8, vc8, ks8, vs8, ctx, L, pos, None if chain else vis, bw)
    po.layer(lw, xb, R, kc, vc, ctx, L, pos, None if chain else vis)
    # the appended slots are the quantisation of the bf16 layer's appended K / V
    ek, ev, eks, evs = caches(1, ctx, bw)
    kb = np.ascontiguousarray(kc[:, L:L + R].transpose(1, 0, 2)).reshape(R, KVH * HD)
    vb = np.ascontiguousarray(vc[:, L:L + R].transpose(1, 0, 2)).reshape(R, KVH * HD)
    po.kv_append8(kb, vb, ek, ev, eks, evs, R, KVH, L, None, ctx, bw)
    assert np.array_equal(kc8[:, L:L + R], ek[0][:, L:L + R])
    assert np.array_equal(vc8[:, L:L + R], ev[0][:, L:L + R])
    assert np.array_equal(ks8[:, L:L + R], eks[0][:, L:L + R])
    assert np.array_equal(vs8[:, L:L + R], evs[0][:, L:L + R])
    # outputs differ only by the quantisation of the new slots (and bf16 rounding)
    a, b = po.bf16_to_f32(x8), po.bf16_to_f32(xb)
    rel = np.sqrt(np.mean((a - b) ** 2) / np.mean(b ** 2))
    assert rel < (2e-2 if bw == 8 else 6e-2), rel
    assert not np.array_equal(a, b)
    # append=False over the appended cache reproduces the forward exactly;
    # over the cache before the append it does not (the new slots are read)
    for kc_, vc_, ks_, vs_, same in ((kc8, vc8, ks8, vs8, True),
                                     (kc8_0, vc8_0, ks8_0, vs8_0, False)):
        x2 = x.copy()
        po.layer8(lw, x2, R, kc_.copy(), vc_.copy(), ks_.copy(), vs_.copy(), ctx, L, pos,
                  None if chain else vis, bw, append=False)
        assert np.array_equal(x2, x8) == same
