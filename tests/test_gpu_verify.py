"""Verify forward (s2p_verify_plan + s2p_verify_forward) vs the oracle's
layer composition (run_layer restated, slowar.c:156-260), and properties of
the full-size 36-layer step.

Logits tolerance (north star): within 1e-2 relative of the oracle's
reference-order forward on the same weights, caches and inputs, per row in
the L2 and the max norm.  Two bf16 rounding orders of the same stack can only
agree as well as each agrees with exact arithmetic, so a row on which the
reference order itself is more than 2e-2 away from the binary64 forward
(tests/f64_forward.py) gets half of that distance as its tolerance.  Over
all rows the GPU must also be no less accurate than the reference order:
rms error against binary64 at most 1.25x the oracle's."""
import ctypes

import numpy as np
import pytest
import torch

import pyoracle as po
import s2pamd
import f64_forward as f64
import gpu_util
from gpu_util import P, S, assert_close_norm, assert_close_rel, bf16_bits, bf16_vals, d2h, empty, to_dev, to_host

pytestmark = pytest.mark.gpu

TREE16 = [-1, 0, 0, 1, 1, 2, 2, 3, 3, 4, 5, 6, 6, 7, 8, 10, 11]


@pytest.fixture(scope="module")
def lib():
    return s2pamd.load()


def make_backbone(lib, n_layers, quant, head_rows, max_rows, max_sessions, ctx, seed, kv_bits=0):
    o = s2pamd.BackboneOpts(n_layers, quant, quant, head_rows, max_rows, max_sessions, ctx, kv_bits)
    bb = ctypes.c_void_p()
    s2pamd.check(lib.s2p_backbone_create_random(ctypes.byref(o), seed, S(), ctypes.byref(bb)),
                 "backbone")
    return bb


def host_linear(lin):
    if lin.q_packed:
        w = d2h(lin.w_pack.data, lin.w_pack.bytes, np.uint8)
        s = d2h(lin.w_iscale.data, lin.w_iscale.bytes, np.uint16)
        keep = (w, s)
        return po.make_linear(w, s, lin.out_features, lin.in_features, 32), keep
    w = d2h(lin.w_int8.data, lin.w_int8.bytes, np.int8)
    s = d2h(lin.w_iscale.data, lin.w_iscale.bytes, np.float32)
    return po.make_linear(w, s, lin.out_features, lin.in_features, 0), (w, s)


def host_layer(lib, bb, l):
    L = lib.s2p_backbone_layer(bb, l).contents
    keep = []
    lins = []
    for name in ("wqkv", "wo", "gate_up", "w2"):
        li, k = host_linear(getattr(L, name))
        lins.append(li)
        keep.append(k)
    norms = [d2h(getattr(L, n).data, getattr(L, n).bytes, np.uint16)
             for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm")]
    keep.append(norms)
    lw = po.OrLayerW(lins[0], lins[1], lins[2], lins[3], *(po.ptr(n) for n in norms))
    return lw, keep


def new_kv(lib, bb, seed):
    nbytes = lib.s2p_backbone_kv_bytes(bb)
    kv = torch.empty(nbytes // 2, dtype=torch.int16, device="cuda")
    s2pamd.hip_check(lib.s2p_synth_bf16_normal(P(kv), kv.numel(), 0.0, 1.0, seed, S()))
    return kv


def plan(lib, bb, parent, kvs, lens, scales=None):
    """kvs: device tensors (the caches' codes for INT8 / INT4); scales: the
    device addresses of the INT8 / INT4 caches' scale tensors, or None"""
    n = len(kvs)
    par = np.asarray(parent, np.int32)
    kvp = (ctypes.c_void_p * n)(*[t.data_ptr() for t in kvs])
    ln = np.asarray(lens, np.int32)
    scp = (ctypes.c_void_p * n)(*scales) if scales is not None else None
    vb = s2pamd.VerifyBatch(n, len(parent), par.ctypes.data, ctypes.addressof(kvp), ln.ctypes.data,
                            ctypes.addressof(scp) if scp is not None else None)
    s2pamd.check(lib.s2p_verify_plan(bb, ctypes.byref(vb), S()), "plan")


def oracle_forward(lib, bb, n_layers, x, kv_host, ctx, L, parent, head_rows):
    """Oracle forward of one session (rows = len(parent)) on host copies."""
    R = len(parent)
    depth = [0] * R
    vis = np.zeros(R, np.uint64)
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
    kv = kv_host.reshape(n_layers, 16, ctx, 128)
    chain = all(parent[i] == i - 1 for i in range(1, R))
    for l in range(n_layers):
        lw, keep = host_layer(lib, bb, l)
        kc = np.ascontiguousarray(kv[l, :8])
        vc = np.ascontiguousarray(kv[l, 8:])
        po.layer(lw, x, R, kc, vc, ctx, L, pos, None if chain else vis)
        kv[l, :8] = kc
        kv[l, 8:] = vc
    fnorm = d2h(lib.s2p_backbone_final_norm(bb), 2560 * 2, np.uint16)
    xn = po.rms_norm(x, fnorm, R, 2560)
    head, keep = host_linear(lib.s2p_backbone_head(bb).contents)
    return po.linear_fwd(head, xn, R), kv


def f64_weights(lib, bb, n_layers):
    layers = []
    for l in range(n_layers):
        L = lib.s2p_backbone_layer(bb, l).contents
        W = {}
        for name in ("wqkv", "wo", "gate_up", "w2"):
            lin = getattr(L, name)
            _, (w, s) = host_linear(lin)
            W[name] = f64.dequant(w, s, lin.out_features, lin.in_features)
        for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm"):
            t = getattr(L, n)
            W[n] = f64.bf(d2h(t.data, t.bytes, np.uint16))
        layers.append(W)
    fnorm = f64.bf(d2h(lib.s2p_backbone_final_norm(bb), 2560 * 2, np.uint16))
    hl = lib.s2p_backbone_head(bb).contents
    _, (w, s) = host_linear(hl)
    return layers, fnorm, f64.dequant(w, s, hl.out_features, hl.in_features)


LOGITS_REL = 1e-2  # logits within 1e-2 of the reference
LOGITS_CAP = 2e-2  # hard cap for a named exception row (see check_logits)


def check_logits(got, want_bits, truth, what, rms=True, allow_exceptions=False):
    """Per-row tolerance against the oracle and (rms=True) the accuracy
    criterion over these rows; callers pooling several sessions pass
    rms=False and apply check_rms to all rows at once.

    The bar is 1e-2 L2-relative per row against the reference order.  Only a
    caller that passes allow_exceptions=True (and names why in its docstring)
    may let a row exceed it, and then only when the GPU row is at least as
    close to binary64 as the reference order is (the distance is then the
    reference order's own rounding error), and never beyond LOGITS_CAP.
    Every call is recorded (gpu_util.LOGITS_RECORD) and summarised at the end
    of the pytest run: the largest gpu-oracle distance and the exception rows
    used."""
    want = bf16_vals(want_bits)
    tn = np.linalg.norm(truth, axis=1)
    rows = [f"{r}: gpu {np.linalg.norm(got[r] - truth[r]) / tn[r]:.2e} "
            f"oracle {np.linalg.norm(want[r] - truth[r]) / tn[r]:.2e} "
            f"gpu-oracle {np.linalg.norm(got[r] - want[r]) / tn[r]:.2e}" for r in range(len(got))]
    print(what, "per-row L2 rel err vs binary64:\n  " + "\n  ".join(rows))
    e_ref = np.linalg.norm(want - truth, axis=1) / tn
    e_gpu = np.linalg.norm(got - truth, axis=1) / tn
    d = np.linalg.norm(got - want, axis=1) / np.maximum(np.linalg.norm(want, axis=1), 1e-30)
    exc = (d > LOGITS_REL) & (e_gpu <= e_ref)
    if not allow_exceptions:
        exc[:] = False
    tol = np.where(exc, LOGITS_CAP, LOGITS_REL)
    for r in np.nonzero(exc)[0]:
        print(f"{what}: EXCEPTION row {r}: gpu-oracle {d[r]:.3e} > {LOGITS_REL:g}, gpu vs "
              f"binary64 {e_gpu[r]:.3e} <= oracle vs binary64 {e_ref[r]:.3e}")
    print(f"{what}: largest per-row tolerance applied {tol.max():g} "
          f"(largest gpu-oracle {d.max():.3e}, {int(exc.sum())} exception rows)")
    gpu_util.LOGITS_RECORD.append((what, float(d.max()), int(exc.sum()), len(d)))
    assert_close_norm(got, want, rel=tol, what=what)
    if rms:
        check_rms(got, want, truth, what)


def check_rms(got, want, truth, what):
    """Over all rows the GPU is no less accurate than the reference order:
    rms error against binary64 at most 1.25x the oracle's."""
    e_gpu = np.sqrt(np.mean((got - truth) ** 2))
    e_ref = np.sqrt(np.mean((want - truth) ** 2))
    assert e_gpu <= 1.25 * e_ref, f"{what}: GPU rms err {e_gpu:.4g} vs oracle {e_ref:.4g}"


@pytest.mark.parametrize("quant,n_layers,L", [(s2pamd.WQ_INT4, 2, 100), (s2pamd.WQ_INT8, 1, 512)])
def test_verify_chain_vs_oracle(lib, quant, n_layers, L):
    """Config 1/2 shapes: K=4 chain (M=5) over one session's cache."""
    ctx = 640
    bb = make_backbone(lib, n_layers, quant, s2pamd.S2P_HEAD_SLICE, 16, 2, ctx, 1234)
    try:
        parent = [-1, 0, 1, 2, 3]
        R = len(parent)
        kv = new_kv(lib, bb, 77)
        kv_host = to_host(kv, np.uint16).copy()
        plan(lib, bb, parent, [kv], [L])
        x = bf16_bits(np.random.default_rng(5).standard_normal((R, 2560)).astype(np.float32))
        logits = empty((R, s2pamd.S2P_HEAD_SLICE))
        s2pamd.check(lib.s2p_verify_forward(bb, P(to_dev(x)), P(logits), S()), "forward")
        got = bf16_vals(to_host(logits, np.uint16))
        want, kv_ref = oracle_forward(lib, bb, n_layers, x, kv_host, ctx, L, parent,
                                      s2pamd.S2P_HEAD_SLICE)
        W, fn, head = f64_weights(lib, bb, n_layers)
        truth = f64.forward(W, fn, head, x, kv_host.reshape(n_layers, 16, ctx, 128), L, parent)
        check_logits(got, want, truth, "chain logits")
        # the verify rows' K/V landed in slots L..L+R-1; everything else untouched
        kv_dev = to_host(kv, np.uint16).reshape(n_layers, 16, ctx, 128)
        kv_ref = kv_ref.reshape(n_layers, 16, ctx, 128)
        assert np.array_equal(kv_dev[:, :, :L], kv_ref[:, :, :L])
        assert np.array_equal(kv_dev[:, :, L + R:], kv_ref[:, :, L + R:])
        assert_close_rel(bf16_vals(kv_dev[:, :, L:L + R]), bf16_vals(kv_ref[:, :, L:L + R]),
                         rel=2e-2, floor_frac=2e-2, what="appended K/V")
    finally:
        lib.s2p_backbone_free(bb)


TREE32 = [-1] + [int(p) for p in np.random.default_rng(32).integers(0, np.arange(1, 32))]


@pytest.mark.parametrize("tree", [TREE16, TREE32], ids=["17-node", "32-node"])
def test_verify_tree_two_sessions_vs_oracle(lib, tree):
    """Config 5 shape on 2 layers: a 16-node tree + root (and the largest
    tree of the per-session attention kernel, 32 nodes), two sessions with
    different prefix lengths, tree visibility masks; the rows' K/V appended
    to their slots and nothing else touched."""
    ctx, n_layers = 512, 2
    R = len(tree)
    bb = make_backbone(lib, n_layers, s2pamd.WQ_INT4, s2pamd.S2P_HEAD_SLICE, 2 * R, 2, ctx, 99)
    try:
        kvs = [new_kv(lib, bb, 5), new_kv(lib, bb, 6)]
        hosts = [to_host(k, np.uint16).copy() for k in kvs]
        lens = [130, 301]
        plan(lib, bb, tree, kvs, lens)
        x = bf16_bits(np.random.default_rng(8).standard_normal((2 * R, 2560)).astype(np.float32))
        logits = empty((2 * R, s2pamd.S2P_HEAD_SLICE))
        s2pamd.check(lib.s2p_verify_forward(bb, P(to_dev(x)), P(logits), S()), "forward")
        got = bf16_vals(to_host(logits, np.uint16))
        W, fn, head = f64_weights(lib, bb, n_layers)
        for s in range(2):
            want, kv_ref = oracle_forward(lib, bb, n_layers, x[s * R:(s + 1) * R], hosts[s], ctx,
                                          lens[s], tree, s2pamd.S2P_HEAD_SLICE)
            truth = f64.forward(W, fn, head, x[s * R:(s + 1) * R],
                                hosts[s].reshape(n_layers, 16, ctx, 128), lens[s], tree)
            check_logits(got[s * R:(s + 1) * R], want, truth, f"{R}-row tree session {s}")
            L = lens[s]
            kv_dev = to_host(kvs[s], np.uint16).reshape(n_layers, 16, ctx, 128)
            kv_ref = kv_ref.reshape(n_layers, 16, ctx, 128)
            assert np.array_equal(kv_dev[:, :, :L], kv_ref[:, :, :L])
            assert np.array_equal(kv_dev[:, :, L + R:], kv_ref[:, :, L + R:])
            assert_close_rel(bf16_vals(kv_dev[:, :, L:L + R]), bf16_vals(kv_ref[:, :, L:L + R]),
                             rel=2e-2, floor_frac=2e-2, what=f"session {s} appended K/V")
    finally:
        lib.s2p_backbone_free(bb)


def test_verify_full_size_step_properties(lib):
    """Config 3: 36L INT4-g32, full 155,776-row head, K=4, ctx 2048.
    Deterministic, finite, graph replay == eager, acceptance sane."""
    ctx = 2304
    side = torch.cuda.Stream()  # graphs cannot be captured on the legacy default stream
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        _full_size_body(lib, ctx)
    torch.cuda.synchronize()


def _full_size_body(lib, ctx):
    bb = make_backbone(lib, 36, s2pamd.WQ_INT4, s2pamd.S2P_VOCAB, 16, 1, ctx, 7)
    try:
        kv = new_kv(lib, bb, 11)
        parent = [-1, 0, 1, 2, 3]
        R = 5
        plan(lib, bb, parent, [kv], [2048])
        x = to_dev(bf16_bits(np.random.default_rng(1).standard_normal((R, 2560)).astype(np.float32)))
        l1 = empty((R, s2pamd.S2P_VOCAB))
        l2 = empty((R, s2pamd.S2P_VOCAB))
        s2pamd.check(lib.s2p_verify_forward(bb, P(x), P(l1), S()))
        s2pamd.check(lib.s2p_verify_forward(bb, P(x), P(l2), S()))
        a, b = to_host(l1, np.uint16), to_host(l2, np.uint16)
        assert np.array_equal(a, b), "forward is not deterministic"
        v = bf16_vals(a)
        assert np.all(np.isfinite(v)) and v.std() > 0.1
        # full step through the graph path, twice, equals the eager path
        drf = to_dev(bf16_bits(bf16_vals(a) + np.random.default_rng(3).standard_normal(
            a.shape).astype(np.float32) * 0.5))
        st = po.state(temperature=0.8, top_p=0.8, seed=0, entropy=0)
        states = [st]
        outs = []
        for use_graph in (0, 1, 1):
            d_states = to_dev(np.frombuffer(bytes(st), np.uint8).copy())
            d_ptrs = to_dev(np.array([d_states.data_ptr()], np.int64))
            tok = np.zeros(R, np.int64)
            sd = po.copy_state(st)
            dv = to_host(drf, np.uint16)
            for i in range(1, R):
                tok[i] = po.sample(sd, dv[i - 1])[0]
            work = torch.empty(lib.s2p_verify_accept_work_bytes(1, R), dtype=torch.uint8,
                               device="cuda")
            path = torch.zeros(R, dtype=torch.int32, device="cuda")
            nacc = torch.zeros(1, dtype=torch.int32, device="cuda")
            emit = torch.zeros(R + 1, dtype=torch.int64, device="cuda")
            nemit = torch.zeros(1, dtype=torch.int32, device="cuda")
            logits = empty((R, s2pamd.S2P_VOCAB))
            io = s2pamd.StepIO(x.data_ptr(), logits.data_ptr(), drf.data_ptr(), s2pamd.S2P_VOCAB,
                               to_dev(np.array(parent, np.int32)).data_ptr(),
                               to_dev(tok).data_ptr(), d_ptrs.data_ptr(), path.data_ptr(),
                               nacc.data_ptr(), emit.data_ptr(), nemit.data_ptr(),
                               work.data_ptr())
            keep = (d_states, d_ptrs, work, path, nacc, emit, nemit, logits)
            s2pamd.check(lib.s2p_verify_step(bb, ctypes.byref(io), use_graph, S()), "step")
            lg = to_host(logits, np.uint16)
            assert np.array_equal(lg, a)
            n = int(to_host(nemit)[0])
            outs.append((int(to_host(nacc)[0]), list(to_host(emit)[:n])))
            # host rule on the same logits
            st_ref = po.copy_state(st)
            p_ref, e_ref = po.accept_tree(st_ref, lg, to_host(drf, np.uint16), parent, tok)
            assert outs[-1] == (len(p_ref), list(e_ref))
            del keep
        assert outs[0] == outs[1] == outs[2]
        assert states
        # the plan ran on the persistent kernel and no flag wait timed out
        assert lib.s2p_backbone_mk_status(bb) == 1
    finally:
        lib.s2p_backbone_free(bb)


@pytest.mark.parametrize("quant,L", [(s2pamd.WQ_INT8, 512), (s2pamd.WQ_INT4, 300)])
def test_verify_stages_one_layer(lib, quant, L):
    """Stage-by-stage parity of one fused layer: each stage is checked against
    the oracle applied to the GPU's own input of that stage."""
    ctx = 640
    bb = make_backbone(lib, 1, quant, s2pamd.S2P_HEAD_SLICE, 16, 1, ctx, 4321)
    try:
        parent = [-1, 0, 1, 2, 3]
        R = 5
        kv = new_kv(lib, bb, 12)
        kv0 = to_host(kv, np.uint16).copy().reshape(1, 16, ctx, 128)
        plan(lib, bb, parent, [kv], [L])
        x_in = bf16_bits(np.random.default_rng(2).standard_normal((R, 2560)).astype(np.float32))
        logits = empty((R, s2pamd.S2P_HEAD_SLICE))
        s2pamd.check(lib.s2p_verify_forward(bb, P(to_dev(x_in)), P(logits), S()))
        ptrs = [ctypes.c_void_p() for _ in range(5)]
        dbg = lib.s2p_backbone_debug_ptrs
        dbg.restype = None
        dbg.argtypes = [ctypes.c_void_p] + [ctypes.c_void_p] * 5
        dbg(bb, *[ctypes.byref(p) for p in ptrs])
        g_x = d2h(ptrs[0].value, R * 2560 * 2, np.uint16).reshape(R, 2560)
        g_qkv = d2h(ptrs[1].value, R * 6144 * 2, np.uint16).reshape(R, 6144)
        g_q = d2h(ptrs[2].value, R * 4096 * 2, np.uint16).reshape(R, 4096)
        g_attn = d2h(ptrs[3].value, R * 4096 * 2, np.uint16).reshape(R, 4096)
        g_h = d2h(ptrs[4].value, R * 9728 * 2, np.uint16).reshape(R, 9728)
        g_kv = to_host(kv, np.uint16).reshape(1, 16, ctx, 128)
        lw, keep = host_layer(lib, bb, 0)
        norms = keep[-1]  # attn_norm, ffn_norm, q_norm, k_norm
        # (a) RMSNorm + qkv GEMV
        xn = po.rms_norm(x_in, norms[0], R, 2560)
        assert_close_rel(bf16_vals(g_qkv), bf16_vals(po.linear_fwd(lw.wqkv, xn, R)), what="qkv")
        # (b) qk-norm + RoPE of the GPU's qkv: bit-exact
        q = np.ascontiguousarray(g_qkv[:, :4096])
        k = np.ascontiguousarray(g_qkv[:, 4096:5120])
        v = np.ascontiguousarray(g_qkv[:, 5120:])
        pos = np.arange(L, L + R, dtype=np.int32)
        q_ref = po.rope(po.qk_norm(q, norms[2], R, 32), R, 32, 128, pos=pos)
        k_ref = po.rope(po.qk_norm(k, norms[3], R, 8), R, 8, 128, pos=pos)
        assert np.array_equal(g_q, q_ref), f"q differs in {np.count_nonzero(g_q != q_ref)} elems"
        assert np.array_equal(g_kv[0, :8, L:L + R].transpose(1, 0, 2).reshape(R, 1024), k_ref)
        assert np.array_equal(g_kv[0, 8:, L:L + R].transpose(1, 0, 2).reshape(R, 1024), v)
        assert np.array_equal(g_kv[0, :, :L], kv0[0, :, :L]), "prefix KV modified"
        # (c) attention on the GPU's q and cache
        exact = po.attention_f64(g_q, np.ascontiguousarray(g_kv[0, :8]),
                                 np.ascontiguousarray(g_kv[0, 8:]), R, 32, 8, 128, L, ctx)
        assert np.max(np.abs(bf16_vals(g_attn) - exact)) < 2e-2, "attention"
        # (d) wo + residual, ffn norm + gate_up with the fused SwiGLU epilogue.
        # The persistent kernel (INT4 plans) rounds x * w to bf16 and applies
        # the inverse RMS to the f32 dot product, where the reference rounds
        # x * inv * w: per row within 1e-2 of the oracle (L2, max norm 2e-2)
        # and, against binary64 on the same weights and attention output, no
        # less accurate than the oracle's order (rms error <= 1.25x)
        x_mid = po.add(x_in, po.linear_fwd(lw.wo, g_attn, R))
        xn2 = po.rms_norm(x_mid, norms[1], R, 2560)
        h_ref = po.silu_mul(po.linear_fwd(lw.gate_up, xn2, R), R, 9728)
        if quant == s2pamd.WQ_INT8:
            assert_close_rel(bf16_vals(g_h), bf16_vals(h_ref), what="gate_up + SwiGLU")
        else:
            L0 = lib.s2p_backbone_layer(bb, 0).contents
            Wd = {}
            for name in ("wo", "gate_up"):
                lin = getattr(L0, name)
                _, (w, sc) = host_linear(lin)
                Wd[name] = f64.dequant(w, sc, lin.out_features, lin.in_features)
            xm64 = f64.bf(x_in) + f64.bf(g_attn) @ Wd["wo"].T
            gu64 = f64.rms(xm64, f64.bf(norms[1])) @ Wd["gate_up"].T
            g64, u64 = gu64[:, :9728], gu64[:, 9728:]
            h64 = g64 / (1 + np.exp(-g64)) * u64
            got, want = bf16_vals(g_h).astype(np.float64), bf16_vals(h_ref).astype(np.float64)
            assert_close_norm(got, want, rel=1e-2, what="gate_up + SwiGLU")
            e_gpu = np.sqrt(np.mean((got - h64) ** 2))
            e_ref = np.sqrt(np.mean((want - h64) ** 2))
            print(f"gate_up + SwiGLU rms err vs binary64: gpu {e_gpu:.4g} oracle {e_ref:.4g}")
            assert e_gpu <= 1.25 * e_ref, (e_gpu, e_ref)
        # (e) w2 + residual on the GPU's SwiGLU output
        x_out = po.add(x_mid, po.linear_fwd(lw.w2, g_h, R))
        assert_close_rel(bf16_vals(g_x), bf16_vals(x_out), what="layer output")
    finally:
        lib.s2p_backbone_free(bb)


def test_verify_plan_device_tree(lib):
    """s2p_verify_plan_device on a 17-row tree plan (per-session tree
    attention segments): lengths advanced on the device give the same logits,
    bit for bit, as a host plan at those lengths."""
    ctx, n_layers = 512, 1
    R = len(TREE16)
    bb = make_backbone(lib, n_layers, s2pamd.WQ_INT4, s2pamd.S2P_HEAD_SLICE, 2 * R, 2, ctx, 7)
    try:
        kvs = [new_kv(lib, bb, 11), new_kv(lib, bb, 12)]
        base = [to_host(k, np.uint16).copy() for k in kvs]
        x = bf16_bits(np.random.default_rng(3).standard_normal((2 * R, 2560)).astype(np.float32))
        xd = to_dev(x)
        new_lens = [140, 333]
        # device-advanced plan: planned at shorter lengths (same 512-slot span bucket)
        plan(lib, bb, TREE16, kvs, [100, 300])
        lend = to_dev(np.asarray(new_lens, np.int32))
        ovf = to_dev(np.zeros(1, np.int32))
        s2pamd.check(lib.s2p_verify_plan_device(bb, P(lend), P(ovf), S()), "plan device")
        la = empty((2 * R, s2pamd.S2P_HEAD_SLICE))
        s2pamd.check(lib.s2p_verify_forward(bb, P(xd), P(la), S()), "forward a")
        got_a = to_host(la, np.uint16)
        assert int(to_host(ovf, np.int32)[0]) == 0
        # host plan at the new lengths on fresh copies of the same caches
        for k, h in zip(kvs, base):
            k.copy_(torch.from_numpy(h.view(np.int16)).to(k.device))
        plan(lib, bb, TREE16, kvs, new_lens)
        lb = empty((2 * R, s2pamd.S2P_HEAD_SLICE))
        s2pamd.check(lib.s2p_verify_forward(bb, P(xd), P(lb), S()), "forward b")
        got_b = to_host(lb, np.uint16)
        assert np.array_equal(got_a, got_b)
    finally:
        lib.s2p_backbone_free(bb)
