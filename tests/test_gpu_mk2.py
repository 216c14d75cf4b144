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
from gpu_util import P, S, assert_close_rel, bf16_bits, bf16_vals, empty, to_dev, to_host
from test_gpu_verify import check_logits, f64_weights, make_backbone, new_kv, oracle_forward, plan

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
