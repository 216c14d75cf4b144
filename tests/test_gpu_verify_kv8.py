"""Verify forward over INT8 / INT4 session caches (backbone kv_bits 8 / 4):
the reference's quantised-cache serving mode (model.c:201-215, kernels.cu:
510-946) inside the verify plan, vs the oracle's layer composition over the
same quantised caches (or_layer8), and the tree commit of quantised slots.

Logits: within 1e-2 relative per row (L2 and max norm), as the bf16-cache
path, of the oracle's forward over the cache contents the GPU produced (a
code that rounds the other way, from a last-bit difference upstream, moves
the result by a whole quantisation step: the appended codes are checked on
their own).  The appended K / V: the dequantised rows within one
quantisation step plus 2e-2 of the oracle's (a code can round the other way
where the GEMV rounding of an element differs) and within 2e-2 (INT4: 6e-2)
in rms; every
other slot untouched.  Commit: the moved
payload rows and scales equal the accepted nodes' rows bit for bit."""
import ctypes

import numpy as np
import pytest

import pyoracle as po
import s2pamd
from gpu_util import (P, S, assert_close_norm, bf16_bits, bf16_vals, d2h,
                      empty, to_dev, to_host)
from test_gpu_verify import TREE16, host_layer, host_linear, make_backbone, plan
from test_oracle_kv8 import decode

pytestmark = pytest.mark.gpu

HD, KVH = 128, 8


@pytest.fixture(scope="module")
def lib():
    return s2pamd.load()


def layout(n_layers, ctx, bw):
    """A session cache as held here: the code tensor kv [layers][16][ctx][el]
    followed by the scale tensor kvs [layers][16][ctx][4] f16 in one buffer
    (the reference's two tensors of s2p_session, slowar_internal.h:177-179);
    returns (el, code bytes per layer, offset of kvs, total bytes)."""
    el = HD if bw == 8 else HD // 2
    pay = 16 * ctx * el
    return el, pay, n_layers * pay, n_layers * (pay + 16 * ctx * 8)


def new_kv8(lib, bb, n_layers, ctx, L, bw, seed):
    """A session cache whose slots [0, L) hold quantised N(0,1) rows (the
    oracle's append), the rest zero; returns (device tensor, host bytes,
    device address of its scale tensor)."""
    el, pay, soff, total = layout(n_layers, ctx, bw)
    assert lib.s2p_backbone_kv_bytes(bb) == soff
    assert lib.s2p_backbone_kv_scale_bytes(bb) == total - soff
    host = np.zeros(total, np.uint8)
    r = np.random.default_rng(seed)
    for l in range(n_layers):
        kc, vc, ks, vs = planes(host, l, ctx, bw, n_layers)
        k = po.f32_to_bf16(r.standard_normal((L, KVH * HD)).astype(np.float32))
        v = po.f32_to_bf16(r.standard_normal((L, KVH * HD)).astype(np.float32))
        kcc, vcc = [np.ascontiguousarray(kc)], [np.ascontiguousarray(vc)]
        kss, vss = [np.ascontiguousarray(ks)], [np.ascontiguousarray(vs)]
        po.kv_append8(k, v, kcc, vcc, kss, vss, L, KVH, 0, None, ctx, bw)
        kc[...], vc[...], ks[...], vs[...] = kcc[0], vcc[0], kss[0], vss[0]
    dev = to_dev(host)
    return dev, host, dev.data_ptr() + soff


def planes(buf, l, ctx, bw, n_layers):
    """Views (kc, vc, ks, vs) of layer l of a session cache held as bytes."""
    el, pay, soff, total = layout(n_layers, ctx, bw)
    p = buf[l * pay:(l + 1) * pay].view(np.int8).reshape(16, ctx, el)
    sb = 16 * ctx * 8
    s = buf[soff + l * sb:soff + (l + 1) * sb].view(np.uint16).reshape(16, ctx, 4)
    return p[:8], p[8:], s[:8], s[8:]


def oracle_forward8(lib, bb, n_layers, x, host, ctx, L, parent, bw, append=True):
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
    pos = np.array([L + d for d in depth], np.int32)
    x = np.array(x, np.uint16, copy=True)
    host = host.copy()
    for l in range(n_layers):
        lw, keep = host_layer(lib, bb, l)
        kc, vc, ks, vs = [np.ascontiguousarray(a) for a in planes(host, l, ctx, bw, n_layers)]
        po.layer8(lw, x, R, kc, vc, ks, vs, ctx, L, pos, vis, bw, append)
        dst = planes(host, l, ctx, bw, n_layers)
        for d, a in zip(dst, (kc, vc, ks, vs)):
            d[...] = a
    fnorm = d2h(lib.s2p_backbone_final_norm(bb), 2560 * 2, np.uint16)
    xn = po.rms_norm(x, fnorm, R, 2560)
    head, keep = host_linear(lib.s2p_backbone_head(bb).contents)
    return po.linear_fwd(head, xn, R), host


def step(ks):
    """the quantisation step (the group scale) of every element"""
    return ks.view(np.float16).astype(np.float64).repeat(32, axis=-1)


def check_appended(got, want, st, what, bw):
    """Dequantised appended rows: every element within two quantisation steps
    plus 2e-2 relative of the oracle's, and the rms difference within 2e-2
    (INT4, whose steps are 18x larger: 6e-2) of the rows' rms.  Two steps:
    the K / V being quantised come out of the GEMVs in another rounding order
    (the persistent kernel applies the RMSNorm's inverse RMS after the dot
    product; the layer path sums in its own order from layer 1 on), and an
    element that moved by a bf16 unit next to a rounding boundary of the code
    moves its code by one step, and its group scale (the group maximum) moves too:
    measured up to 2.0 steps for both forwards on a 6-row plan."""
    err = np.abs(got - want)
    bad = err > 2.01 * st + 2e-2 * np.abs(want)
    assert not np.any(bad), (f"{what}: beyond two steps at {np.argwhere(bad)[:4].tolist()}: "
                             f"got {got[bad][:4]}, want {want[bad][:4]}, step {st[bad][:4]}")
    rel = np.sqrt(np.mean(err ** 2) / np.mean(want ** 2))
    assert rel <= (2e-2 if bw == 8 else 6e-2), f"{what}: rms difference {rel:.3g}"


def deq(kc, ks, bw):
    return decode(kc, bw) * ks.view(np.float16).astype(np.float64).repeat(32, axis=-1)


@pytest.mark.parametrize("bw,parent,lens,ctx", [(8, [-1, 0, 1, 2, 3], [300], 384),
                                                # INT8 / INT4 plans of <= 6 rows run on the
                                                # persistent kernel: 17 splits, a 6-node tree,
                                                # two segments
                                                (8, [-1, 0, 1, 2, 3], [2043], 2304),
                                                (8, [-1, 0, 0, 1, 1, 2], [301], 640),
                                                (8, [-1, 0, 1], [500, 777], 1024),
                                                (4, [-1, 0, 1, 2, 3], [2043], 2304),
                                                (4, [-1, 0, 0, 1, 1, 2], [301], 640),
                                                (4, [-1, 0, 1, 2, 3], [129], 384),
                                                (8, TREE16, [130, 301], 384),
                                                # 8 segments over a 4608-slot span: the
                                                # one-round split sizing gives 160-slot
                                                # splits (not a multiple of 128)
                                                (4, TREE16, [4500, 4321, 4402, 4570], 4608)])
def test_verify_forward_kv8_vs_oracle(lib, bw, parent, lens, ctx):
    n_layers = 2
    R, n = len(parent), len(lens)
    bb = make_backbone(lib, n_layers, s2pamd.WQ_INT4, s2pamd.S2P_HEAD_SLICE, n * R, n, ctx,
                       321 + bw, kv_bits=bw)
    try:
        kvs, hosts, scs = zip(*[new_kv8(lib, bb, n_layers, ctx, lens[s], bw, 40 + s)
                                for s in range(n)])
        plan(lib, bb, parent, list(kvs), lens, list(scs))
        mk = lib.s2p_backbone_mk_status(bb)
        print(f"kv{bw}: {n} sessions x {R} rows, lens {lens}, "
              f"{'persistent kernel' if mk == 1 else 'layer path'}", flush=True)
        assert mk == (1 if n * R <= 6 else 0)
        x = bf16_bits(np.random.default_rng(9).standard_normal((n * R, 2560)).astype(np.float32))
        logits = empty((n * R, s2pamd.S2P_HEAD_SLICE))
        s2pamd.check(lib.s2p_verify_forward(bb, P(to_dev(x)), P(logits), S()), "forward")
        got = bf16_vals(to_host(logits, np.uint16))
        assert lib.s2p_backbone_mk_status(bb) == mk, "a flag wait timed out"
        for s in range(n):
            rows = slice(s * R, (s + 1) * R)
            _, ref = oracle_forward8(lib, bb, n_layers, x[rows], hosts[s], ctx, lens[s],
                                     parent, bw)
            dev = to_host(kvs[s], np.uint8)
            # the forward on the cache contents the GPU produced
            want, _ = oracle_forward8(lib, bb, n_layers, x[rows], dev, ctx, lens[s], parent, bw,
                                      append=False)
            assert_close_norm(got[rows], bf16_vals(want), rel=1e-2, what=f"session {s} logits")
            L = lens[s]
            for l in range(n_layers):
                gp, rp = planes(dev, l, ctx, bw, n_layers), planes(ref, l, ctx, bw, n_layers)
                for a, b in zip(gp, rp):  # prefix and free slots untouched
                    assert np.array_equal(a[:, :L], b[:, :L])
                    assert np.array_equal(a[:, L + R:], b[:, L + R:])
                for c, sc in ((0, 2), (1, 3)):
                    check_appended(deq(gp[c][:, L:L + R], gp[sc][:, L:L + R], bw),
                                   deq(rp[c][:, L:L + R], rp[sc][:, L:L + R], bw),
                                   np.maximum(step(gp[sc][:, L:L + R]), step(rp[sc][:, L:L + R])),
                                   f"layer {l} appended {'KV'[c]}", bw)
    finally:
        lib.s2p_backbone_free(bb)


@pytest.mark.parametrize("bw", [8, 4])
def test_kv_commit8_moves_accepted_nodes(lib, bw):
    """Tree commit over quantised caches: after a forward, accepted path
    (2, 5, 10, 15) of TREE16 moves to slots L+1..L+4 of every layer and plane,
    payload and scales, and nothing else changes."""
    n_layers, ctx, L = 2, 256, 77
    R = len(TREE16)
    bb = make_backbone(lib, n_layers, s2pamd.WQ_INT4, s2pamd.S2P_HEAD_SLICE, R, 1, ctx, 55,
                       kv_bits=bw)
    try:
        kv, _, sc = new_kv8(lib, bb, n_layers, ctx, L, bw, 7)
        plan(lib, bb, TREE16, [kv], [L], [sc])
        x = bf16_bits(np.random.default_rng(3).standard_normal((R, 2560)).astype(np.float32))
        logits = empty((R, s2pamd.S2P_HEAD_SLICE))
        s2pamd.check(lib.s2p_verify_forward(bb, P(to_dev(x)), P(logits), S()), "forward")
        before = to_host(kv, np.uint8).copy()
        path = np.zeros(R, np.int32)
        path[:4] = [2, 5, 10, 15]
        nacc = np.array([4], np.int32)
        s2pamd.check(lib.s2p_verify_kv_commit(bb, P(to_dev(path)), P(to_dev(nacc)), S()),
                     "commit")
        after = to_host(kv, np.uint8)
        for l in range(n_layers):
            b, a = planes(before, l, ctx, bw, n_layers), planes(after, l, ctx, bw, n_layers)
            for pb, pa in zip(b, a):
                want = pb.copy()
                for d, node in enumerate([2, 5, 10, 15], start=1):
                    want[:, L + d] = pb[:, L + node]
                assert np.array_equal(pa, want)
                assert np.any(pa[:, L + 1:L + 5] != pb[:, L + 1:L + 5])
    finally:
        lib.s2p_backbone_free(bb)


def test_kv_bits_rejected(lib):
    o = s2pamd.BackboneOpts(1, s2pamd.WQ_INT4, s2pamd.WQ_INT4, s2pamd.S2P_HEAD_SLICE, 8, 1, 64, 6)
    bb = ctypes.c_void_p()
    assert lib.s2p_backbone_create_random(ctypes.byref(o), 1, S(), ctypes.byref(bb)) != 0
