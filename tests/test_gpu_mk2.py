"""Persistent verify kernel (csrc/mk2.hip, one launch per forward; plans of
at most 6 rows over bf16 caches with INT4-g32 weights) against the oracle's
layer composition and binary64, with the same logits tolerance as the
layer-by-layer path (tests/test_gpu_verify.py: check_logits), and against
the layer-by-layer path itself.  The kernel's own split of the attention
(128-position splits merged by the last one) and its tree masks are
exercised by long prefixes and a 6-node tree; the full 155,776-row head by
a short stack.  No flag wait may time out (s2p_backbone_mk_status)."""
import numpy as np
import pytest
import torch

import f64_forward as f64
import s2pamd
import pyoracle as po
from gpu_util import P, S, assert_close_rel, bf16_bits, bf16_vals, d2h, empty, to_dev, to_host
from test_gpu_verify import (check_logits, check_rms, f64_weights, host_layer, host_linear, make_backbone,
                             new_kv, oracle_forward, plan)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return s2pamd.load()


def _forward(lib, bb, x, R, head_rows):
    logits = empty((R, head_rows))
    s2pamd.check(lib.s2p_verify_forward(bb, P(to_dev(x)), P(logits), S()), "forward")
    return to_host(logits, np.uint16)


@pytest.mark.parametrize("parent,n_layers,L,ctx", [
    ([-1, 0, 1, 2, 3], 2, 200, 512),          # chain, one 128-position split + the new rows
    ([-1, 0, 1, 2, 3], 1, 2043, 2304),        # chain across 17 splits (merge by the last)
    ([-1, 0, 0, 1, 1, 2], 2, 301, 640),        # 6-node tree, masks over the new slots
])
def test_mk2_vs_oracle(lib, parent, n_layers, L, ctx):
    R = len(parent)
    bb = make_backbone(lib, n_layers, s2pamd.WQ_INT4, s2pamd.S2P_HEAD_SLICE, 8, 1, ctx, 4321)
    try:
        kv = new_kv(lib, bb, 19)
        kv_host = to_host(kv, np.uint16).copy()
        plan(lib, bb, parent, [kv], [L])
        assert lib.s2p_backbone_mk_status(bb) == 1, "plan did not run on the persistent kernel"
        x = bf16_bits(np.random.default_rng(L).standard_normal((R, 2560)).astype(np.float32))
        got = bf16_vals(_forward(lib, bb, x, R, s2pamd.S2P_HEAD_SLICE))
        assert lib.s2p_backbone_mk_status(bb) == 1, "a flag wait timed out"
        want, kv_ref = oracle_forward(lib, bb, n_layers, x, kv_host, ctx, L, parent,
                                      s2pamd.S2P_HEAD_SLICE)
        W, fn, head = f64_weights(lib, bb, n_layers)
        truth = f64.forward(W, fn, head, x, kv_host.reshape(n_layers, 16, ctx, 128), L, parent)
        check_logits(got, want, truth, f"mk2 logits L={L}")
        kv_dev = to_host(kv, np.uint16).reshape(n_layers, 16, ctx, 128)
        kv_ref = kv_ref.reshape(n_layers, 16, ctx, 128)
        assert np.array_equal(kv_dev[:, :, :L], kv_ref[:, :, :L])
        assert np.array_equal(kv_dev[:, :, L + R:], kv_ref[:, :, L + R:])
        assert_close_rel(bf16_vals(kv_dev[:, :, L:L + R]), bf16_vals(kv_ref[:, :, L:L + R]),
                         rel=2e-2, floor_frac=2e-2, what="mk2 appended K/V")
    finally:
        lib.s2p_backbone_free(bb)


def test_mk2_two_sessions_vs_layer_path(lib):
    """Two sessions x 3 rows (two attention segments, different prefixes):
    the persistent kernel and the layer path agree within the logits bar;
    the persistent forward is deterministic."""
    ctx, n_layers, parent = 1024, 2, [-1, 0, 1]
    R = 2 * len(parent)
    bb = make_backbone(lib, n_layers, s2pamd.WQ_INT4, s2pamd.S2P_HEAD_SLICE, 8, 2, ctx, 77)
    try:
        kvs = [new_kv(lib, bb, 3), new_kv(lib, bb, 4)]
        hosts = [to_host(k, np.uint16).copy() for k in kvs]
        x = bf16_bits(np.random.default_rng(2).standard_normal((R, 2560)).astype(np.float32))
        out = {}
        for mode in (0, 1):
            lib.s2p_backbone_set_mk(bb, mode)
            for k, h in zip(kvs, hosts):
                k.copy_(torch.from_numpy(h.view(np.int16)).to(k.device))
            plan(lib, bb, parent, kvs, [500, 777])
            assert lib.s2p_backbone_mk_status(bb) == mode
            out[mode] = _forward(lib, bb, x, R, s2pamd.S2P_HEAD_SLICE)
            assert lib.s2p_backbone_mk_status(bb) == mode
        a, b = bf16_vals(out[1]), bf16_vals(out[0])
        rel = np.linalg.norm(a - b, axis=1) / np.linalg.norm(b, axis=1)
        print("mk2 vs layer path, per-row L2 rel:", rel)
        assert np.all(rel < 1e-2), rel
        for _ in range(2):
            assert np.array_equal(_forward(lib, bb, x, R, s2pamd.S2P_HEAD_SLICE), out[1])
    finally:
        lib.s2p_backbone_set_mk(bb, 1)
        lib.s2p_backbone_free(bb)


def test_mk2_full_head_vs_oracle(lib):
    """The 155,776-row head (39 tiles per workgroup, streamed through the
    ring) on a 1-layer stack, against the oracle."""
    ctx, n_layers, parent, L = 512, 1, [-1, 0, 1, 2, 3], 64
    R = len(parent)
    bb = make_backbone(lib, n_layers, s2pamd.WQ_INT4, s2pamd.S2P_VOCAB, 8, 1, ctx, 555)
    try:
        kv = new_kv(lib, bb, 23)
        kv_host = to_host(kv, np.uint16).copy()
        plan(lib, bb, parent, [kv], [L])
        assert lib.s2p_backbone_mk_status(bb) == 1
        x = bf16_bits(np.random.default_rng(9).standard_normal((R, 2560)).astype(np.float32))
        got = bf16_vals(_forward(lib, bb, x, R, s2pamd.S2P_VOCAB))
        assert lib.s2p_backbone_mk_status(bb) == 1
        want, _ = oracle_forward(lib, bb, n_layers, x, kv_host, ctx, L, parent, s2pamd.S2P_VOCAB)
        W, fn, head = f64_weights(lib, bb, n_layers)
        truth = f64.forward(W, fn, head, x, kv_host.reshape(n_layers, 16, ctx, 128), L, parent)
        check_logits(got, want, truth, "mk2 full-head logits")
    finally:
        lib.s2p_backbone_free(bb)


def _streamed_references(lib, bb, n_layers, x, kv_host, ctx, L, parent, head_rows):
    """The oracle's reference-order forward and the binary64 forward of one
    session, layer by layer (one layer's weights on the host at a time, so a
    36-layer stack needs ~1 GB instead of ~30): returns (oracle logits bits,
    binary64 logits)."""
    import sys
    import time
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
    chain = all(parent[i] == i - 1 for i in range(1, R))
    xo = np.array(x, np.uint16, copy=True)
    appended = np.zeros((n_layers, 16, R, 128), np.uint16)
    x64 = f64.bf(x)
    kv = kv_host.reshape(n_layers, 16, ctx, 128)
    t0 = time.time()
    for l in range(n_layers):
        lw, keep = host_layer(lib, bb, l)
        kc0 = f64.bf(kv[l, :8])
        vc0 = f64.bf(kv[l, 8:])
        kc = kv[l, :8].copy()  # (a contiguous slice: without the copy the layer
        vc = kv[l, 8:].copy()  # would write into the caller's cache)
        po.layer(lw, xo, R, kc, vc, ctx, L, pos, None if chain else vis)
        appended[l, :8] = kc[:, L:L + R]
        appended[l, 8:] = vc[:, L:L + R]
        W = {}
        (w_qkv, w_o, w_gu, w_2), norms = keep[:4], keep[4]
        Lr = lib.s2p_backbone_layer(bb, l).contents
        for name, (w, sc) in zip(("wqkv", "wo", "gate_up", "w2"), (w_qkv, w_o, w_gu, w_2)):
            lin = getattr(Lr, name)
            W[name] = f64.dequant(w, sc, lin.out_features, lin.in_features)
        for name, n in zip(("attn_norm", "ffn_norm", "q_norm", "k_norm"), norms):
            W[name] = f64.bf(n)
        x64 = f64.layer(W, x64, kc0, vc0, L, list(pos), [int(v) for v in vis])
        del W
        if l % 6 == 5:
            print(f"  references: layer {l + 1}/{n_layers} ({time.time() - t0:.0f} s)", flush=True)
            sys.stdout.flush()
    fnorm = d2h(lib.s2p_backbone_final_norm(bb), 2560 * 2, np.uint16)
    head, (hw, hs) = host_linear(lib.s2p_backbone_head(bb).contents)
    want = po.linear_fwd(head, po.rms_norm(xo, fnorm, R, 2560), R)
    hl = lib.s2p_backbone_head(bb).contents
    truth = f64.rms(x64, f64.bf(fnorm)) @ f64.dequant(hw, hs, hl.out_features, hl.in_features).T
    return want, truth, appended


def check_depth(got, want, truth, what):
    """The accuracy criterion at full depth.  Over 36 random-init layers the
    reference order itself lands 2.8-3.1e-2 (per-row L2) from the binary64
    forward, because every layer rounds its stages to bf16; any other order
    of the same roundings lands as far, on its own side (the layer-by-layer
    path, which rounds at the reference's points, is 2.7-3.1e-2 from it).
    So at this depth the GPU must be per row no less accurate than the
    reference order (error against binary64 at most 1.25x the oracle's) and
    over all rows (check_rms).  A wrong layer offset, flag or plane stride
    moves a row by O(1), far outside this."""
    tn = np.linalg.norm(truth, axis=1)
    e_gpu = np.linalg.norm(got - truth, axis=1) / tn
    e_ref = np.linalg.norm(bf16_vals(want) - truth, axis=1) / tn
    d = np.linalg.norm(got - bf16_vals(want), axis=1) / tn
    for r in range(len(got)):
        print(f"{what} row {r}: gpu vs binary64 {e_gpu[r]:.3e}, oracle vs binary64 "
              f"{e_ref[r]:.3e}, gpu vs oracle {d[r]:.3e}")
    assert np.all(e_gpu <= 1.25 * e_ref), (what, e_gpu, e_ref)
    check_rms(got, bf16_vals(want), truth, what)


@pytest.mark.timeout(400)
def test_mk2_config3_depth_vs_oracle(lib):
    """Config 3 exactly (36 INT4-g32 layers, the full 155,776-row INT4 head,
    K=4 chain, bf16 KV 2048, ctx 2304 as the bench plans it) on the
    persistent kernel and on the layer-by-layer path, each against the
    oracle's 36-layer forward and binary64 (check_depth).  Pins what only
    full depth exercises: every layer's weight block base, flag values and
    KV plane strides.  No flag wait may time out."""
    ctx, n_layers, parent, L = 2304, 36, [-1, 0, 1, 2, 3], 2048
    R = len(parent)
    print("config-3 depth test: building the 36-layer backbone", flush=True)
    bb = make_backbone(lib, n_layers, s2pamd.WQ_INT4, s2pamd.S2P_VOCAB, 8, 1, ctx, 2026)
    try:
        kv = new_kv(lib, bb, 31)
        kv_host = to_host(kv, np.uint16).copy()
        x = bf16_bits(np.random.default_rng(36).standard_normal((R, 2560)).astype(np.float32))
        got, kv_dev = {}, {}
        for mode in (1, 0):
            lib.s2p_backbone_set_mk(bb, mode)
            kv.copy_(torch.from_numpy(kv_host.view(np.int16)).to(kv.device))
            plan(lib, bb, parent, [kv], [L])
            assert lib.s2p_backbone_mk_status(bb) == mode, "plan did not run where expected"
            got[mode] = bf16_vals(_forward(lib, bb, x, R, s2pamd.S2P_VOCAB))
            assert lib.s2p_backbone_mk_status(bb) == mode, "a flag wait timed out"
            kv_dev[mode] = to_host(kv, np.uint16).reshape(n_layers, 16, ctx, 128)
        print("config-3 depth test: GPU forwards done, running the references", flush=True)
        want, truth, appended = _streamed_references(lib, bb, n_layers, x, kv_host, ctx, L,
                                                     parent, s2pamd.S2P_VOCAB)
        d = np.linalg.norm(got[1] - got[0], axis=1) / np.linalg.norm(got[0], axis=1)
        print("mk2 vs layer path, per-row L2 rel:", d)
        check_depth(got[0], want, truth, "layer path, 36 layers + full head")
        check_depth(got[1], want, truth, "mk2, 36 layers + full head")
        # every layer appended its rows at L..L+R-1 (the first two layers,
        # before the orders drift apart, within 2e-2 of the oracle's rows)
        # and touched nothing else
        kv0 = kv_host.reshape(n_layers, 16, ctx, 128)
        bad = []
        for mode in (1, 0):
            new_rows = kv_dev[mode][:, :, L:L + R]
            same = np.all(new_rows == kv0[:, :, L:L + R], axis=(2, 3))
            for l, h in zip(*np.nonzero(same)):
                bad.append(f"{'mk2' if mode else 'layer path'}: layer {l} plane {h} not appended")
            for l in range(2):
                a, w = bf16_vals(new_rows[l]), bf16_vals(appended[l])
                rel = np.linalg.norm(a - w) / np.linalg.norm(w)
                print(f"{'mk2' if mode else 'layer path'} layer {l} appended K/V vs oracle: {rel:.3e}")
                if rel > 2e-2:
                    bad.append(f"{'mk2' if mode else 'layer path'}: layer {l} appended rows {rel:.3e}")
            assert np.array_equal(kv_dev[mode][:, :, :L], kv0[:, :, :L])
            assert np.array_equal(kv_dev[mode][:, :, L + R:], kv0[:, :, L + R:])
        assert not bad, "\n".join(bad[:40])
    finally:
        lib.s2p_backbone_set_mk(bb, 1)
        lib.s2p_backbone_free(bb)


def test_mk2_wait_timeout_is_reported(lib):
    """A flag wait that gives up (forced from the host with a tiny poll
    limit, so every workgroup still drains and exits normally) is reported
    on the product path: the step's acceptance decides nothing (n_acc = -1,
    n_emit = 0, state untouched) and s2p_verify_status reads 1; after the
    word is cleared and the limit restored, the same step is valid again and
    matches the eager forward of a fresh plan."""
    import ctypes
    ctx, n_layers, parent, L = 512, 2, [-1, 0, 1, 2, 3], 200
    R = len(parent)
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        bb = make_backbone(lib, n_layers, s2pamd.WQ_INT4, s2pamd.S2P_HEAD_SLICE, 8, 1, ctx, 99)
        try:
            kv = new_kv(lib, bb, 5)
            plan(lib, bb, parent, [kv], [L])
            assert lib.s2p_backbone_mk_status(bb) == 1
            x_host = bf16_bits(np.random.default_rng(4).standard_normal((R, 2560))
                               .astype(np.float32))
            x = to_dev(x_host)
            ref = _forward(lib, bb, x_host, R, s2pamd.S2P_HEAD_SLICE)
            st = po.state(temperature=0.8, top_p=0.8, seed=3, entropy=0)
            st_bytes = np.frombuffer(bytes(st), np.uint8).copy()
            drf = to_dev(bf16_bits(bf16_vals(ref) + 0.5 * np.random.default_rng(5)
                                   .standard_normal(ref.shape).astype(np.float32)))
            tok = np.zeros(R, np.int64)
            sd = po.copy_state(st)
            dv = to_host(drf, np.uint16)
            for i in range(1, R):
                tok[i] = po.sample(sd, dv[i - 1, :4096], int(dv[i - 1, 4096]))[0]
            d_states = to_dev(st_bytes)
            d_ptrs = to_dev(np.array([d_states.data_ptr()], np.int64))
            work = torch.empty(lib.s2p_verify_accept_work_bytes(1, R), dtype=torch.uint8,
                               device="cuda")
            path = torch.zeros(R, dtype=torch.int32, device="cuda")
            nacc = torch.zeros(1, dtype=torch.int32, device="cuda")
            emit = torch.zeros(R + 1, dtype=torch.int64, device="cuda")
            nemit = torch.zeros(1, dtype=torch.int32, device="cuda")
            status = torch.full((1,), 7, dtype=torch.int32, device="cuda")
            logits = empty((R, s2pamd.S2P_HEAD_SLICE))
            io = s2pamd.StepIO(x.data_ptr(), logits.data_ptr(), drf.data_ptr(),
                               s2pamd.S2P_HEAD_SLICE,
                               to_dev(np.array(parent, np.int32)).data_ptr(),
                               to_dev(tok).data_ptr(), d_ptrs.data_ptr(), path.data_ptr(),
                               nacc.data_ptr(), emit.data_ptr(), nemit.data_ptr(),
                               work.data_ptr())
            # healthy step first: status 0
            s2pamd.check(lib.s2p_verify_status(bb, P(status), 0, S()))
            assert int(to_host(status)[0]) == 0
            # forced timeout: 1 poll per wait
            lib.s2p_backbone_set_mk_spin(bb, 1)
            for use_graph in (0, 1):
                d_states.copy_(torch.from_numpy(st_bytes).to(d_states.device))
                s2pamd.check(lib.s2p_verify_step(bb, ctypes.byref(io), use_graph, S()), "step")
                assert int(to_host(nacc)[0]) == -1, "a timed-out forward was accepted"
                assert int(to_host(nemit)[0]) == 0
                assert np.array_equal(to_host(d_states, np.uint8), st_bytes), "state advanced"
                s2pamd.check(lib.s2p_verify_status(bb, P(status), 0, S()))
                assert int(to_host(status)[0]) == 1
            # recovery: default limit, clear the word, the step is valid again
            lib.s2p_backbone_set_mk_spin(bb, 0)
            s2pamd.check(lib.s2p_verify_status(bb, P(status), 1, S()))
            assert int(to_host(status)[0]) == 1
            d_states.copy_(torch.from_numpy(st_bytes).to(d_states.device))
            s2pamd.check(lib.s2p_verify_step(bb, ctypes.byref(io), 1, S()), "step")
            assert lib.s2p_backbone_mk_status(bb) == 1
            s2pamd.check(lib.s2p_verify_status(bb, P(status), 0, S()))
            assert int(to_host(status)[0]) == 0
            assert int(to_host(nacc)[0]) >= 0
            lg = to_host(logits, np.uint16)
            # the K/V rows the drained launches wrote are rewritten by this one,
            # so its logits equal the first forward's
            assert np.array_equal(lg, ref)
            p_ref, e_ref = po.accept_tree(po.copy_state(st), np.ascontiguousarray(lg[:, :4096]),
                                          np.ascontiguousarray(dv[:, :4096]), parent, tok,
                                          np.ascontiguousarray(lg[:, 4096]),
                                          np.ascontiguousarray(dv[:, 4096]))
            n = int(to_host(nemit)[0])
            assert (int(to_host(nacc)[0]), list(to_host(emit)[:n])) == (len(p_ref), list(e_ref))
        finally:
            lib.s2p_backbone_free(bb)
    torch.cuda.synchronize()
