"""Persistent verify kernel (one launch per forward) vs the layer-by-layer
kernels: same device code over the same work decomposition, so logits and
the appended K/V must be identical bit for bit; no barrier wait may time
out."""
import numpy as np
import pytest

import s2pamd
from gpu_util import P, S, bf16_bits, empty, to_dev, to_host
from test_gpu_verify import make_backbone, new_kv, plan

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return s2pamd.load()


@pytest.mark.parametrize("quant,n_layers,L", [(s2pamd.WQ_INT4, 2, 100), (s2pamd.WQ_INT8, 1, 512),
                                              (s2pamd.WQ_INT4, 3, 2043)])
def test_mk_matches_layerwise(lib, quant, n_layers, L):
    ctx = 2048 + 64
    bb = make_backbone(lib, n_layers, quant, s2pamd.S2P_HEAD_SLICE, 16, 1, ctx, 321)
    try:
        parent = [-1, 0, 1, 2, 3]
        R = len(parent)
        kv = new_kv(lib, bb, 17)
        kv0 = to_host(kv, np.uint16).copy()
        x = to_dev(bf16_bits(np.random.default_rng(3).standard_normal((R, 2560)).astype(np.float32)))
        out = {}
        # the layer-by-layer GEMVs planned for the persistent kernel's grid
        lib.s2p_gemv_set_slots(lib.s2p_backbone_mk_grid(bb))
        # the layer kernels shaped like the persistent kernel's phases:
        # whole-K GEMVs of 8 waves on its grid, attention blocks of 8 waves
        lib.s2p_gemv_set_v3_nw(8)
        lib.s2p_attn_set_waves(8)
        for mode in (1, 0):
            lib.s2p_backbone_set_mk(bb, mode)
            kv.copy_(__import__("torch").from_numpy(kv0.view(np.int16)).to(kv.device))
            plan(lib, bb, parent, [kv], [L])
            st = lib.s2p_backbone_mk_status(bb)
            assert st == mode, f"plan ran on the {'persistent' if st == 1 else 'layer'} path"
            logits = empty((R, s2pamd.S2P_HEAD_SLICE))
            s2pamd.check(lib.s2p_verify_forward(bb, P(x), P(logits), S()), "forward")
            assert lib.s2p_backbone_mk_status(bb) == mode, "barrier wait timed out"
            out[mode] = (to_host(logits, np.uint16).copy(), to_host(kv, np.uint16).copy())
        assert np.array_equal(out[1][0], out[0][0]), \
            f"logits differ at {np.count_nonzero(out[1][0] != out[0][0])} places"
        assert np.array_equal(out[1][1], out[0][1]), "KV caches differ"
        # and the forward is deterministic on the persistent path
        lib.s2p_backbone_set_mk(bb, 1)
        kv.copy_(__import__("torch").from_numpy(kv0.view(np.int16)).to(kv.device))
        plan(lib, bb, parent, [kv], [L])
        logits = empty((R, s2pamd.S2P_HEAD_SLICE))
        for _ in range(3):
            s2pamd.check(lib.s2p_verify_forward(bb, P(x), P(logits), S()), "forward")
        assert lib.s2p_backbone_mk_status(bb) == 1
        assert np.array_equal(to_host(logits, np.uint16), out[1][0])
    finally:
        lib.s2p_gemv_set_slots(0)
        lib.s2p_gemv_set_v3_nw(0)
        lib.s2p_attn_set_waves(4)
        lib.s2p_backbone_free(bb)
