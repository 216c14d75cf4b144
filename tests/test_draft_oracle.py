"""Draft model (reference src/draft/draft.c) on the CPU: the bf16 GEMM
contract and the draft step of the oracle against binary64 truth and closed
forms, and the safetensors loader's error paths (they fail before any device
work, so no GPU is needed)."""
import ctypes
import os

import numpy as np
import pytest

import draft_util as du
import f64_forward as f64
import pyoracle as po
import s2pamd


def test_gemm_bf16_closed_forms():
    """One-hot weights pick an activation exactly; small-integer operands
    give exact sums."""
    r = np.random.default_rng(1)
    M, N, K = 3, 40, 256
    x = du.bf16_bits(r.standard_normal((M, K)).astype(np.float32))
    w = np.zeros((N, K), np.float32)
    for n in range(N):
        w[n, (n * 7) % K] = 1.0
    y = po.gemm_bf16(x, du.bf16_bits(w), M, N, K)
    assert np.array_equal(y, x[:, [(n * 7) % K for n in range(N)]])
    xi = r.integers(-8, 9, (M, K)).astype(np.float32)
    wi = r.integers(-8, 9, (N, K)).astype(np.float32)
    y = po.bf16_to_f32(po.gemm_bf16(du.bf16_bits(xi), du.bf16_bits(wi), M, N, K))
    want = (xi.astype(np.float64) @ wi.T.astype(np.float64))
    assert np.array_equal(y, po.bf16_to_f32(po.f32_to_bf16(want.astype(np.float32))))


def test_gemm_bf16_vs_f64():
    r = np.random.default_rng(2)
    M, N, K = 4, 300, 2560
    x = du.bf16_bits(r.standard_normal((M, K)).astype(np.float32))
    w = du.bf16_bits(r.standard_normal((N, K)).astype(np.float32))
    y = po.bf16_to_f32(po.gemm_bf16(x, w, M, N, K)).astype(np.float64)
    t = po.gemm_bf16_f64(x, w, M, N, K)
    # fp32 sum then one bf16 rounding: within 2^-8 relative of the exact dot
    # plus the fp32 sum's error (~K * 2^-24 * sum |w x|)
    bound = np.abs(t) * 2.0 ** -8 + K * 2.0 ** -24 * (np.abs(f64.bf(x)) @ np.abs(f64.bf(w)).T)
    assert np.all(np.abs(y - t) <= bound)


@pytest.fixture(scope="module")
def weights():
    return du.make_weights(11)


def test_draft_steps_vs_f64(weights):
    """Four steps from an empty state, then two steps at position 700 over a
    pre-filled cache: the oracle's output stays within 1e-2 (L2, relative)
    of binary64 and its K/V writes land at the step's slot only."""
    w = weights
    arrs = du.oracle_arrays(w)
    d = po.make_draft(arrs)
    W = du.f64_weights(w)
    r = np.random.default_rng(3)
    ctx = 4096
    kc = np.zeros((8, ctx, 128), np.uint16)
    vc = np.zeros((8, ctx, 128), np.uint16)
    k64, v64 = np.zeros((8, ctx, 128)), np.zeros((8, ctx, 128))
    positions = [0, 1, 2, 3, 700, 701]
    for i, pos in enumerate(positions):
        if pos == 700:
            fill = du.bf16_bits(r.standard_normal((2, 8, 700, 128)).astype(np.float32))
            kc[:, 4:700], vc[:, 4:700] = fill[0][:, 4:], fill[1][:, 4:]
            k64[:, 4:700], v64[:, 4:700] = f64.bf(kc[:, 4:700]), f64.bf(vc[:, 4:700])
        h = du.bf16_bits(r.standard_normal(2560).astype(np.float32))
        e = du.bf16_bits(r.standard_normal(2560).astype(np.float32))
        before_k = kc.copy()
        out = po.draft_step(d, kc, vc, ctx, pos, h, e)
        truth = f64.draft_step(W, f64.bf(h), f64.bf(e), k64, v64, pos)
        err = np.linalg.norm(f64.bf(out) - truth) / np.linalg.norm(truth)
        assert err < 1e-2, f"step at {pos}: rel err {err:.3g}"
        changed = np.nonzero(np.any(kc != before_k, axis=(0, 2)))[0]
        assert set(changed.tolist()) <= {pos}
        # the next steps attend over the oracle's own (rounded) K/V, as the
        # GPU does: keep the truth's cache on the same values
        k64[:, pos], v64[:, pos] = f64.bf(kc[:, pos]), f64.bf(vc[:, pos])


def test_draft_loader_errors(tmp_path):
    """Missing file -> S2P_ERR_IO; the first tensor missing, mis-shaped or not
    bf16 -> S2P_ERR_INVALID (checked before any device allocation)."""
    lib = s2pamd.load()
    m = s2pamd.DraftModel()
    assert lib.s2p_draft_load(ctypes.byref(m), str(tmp_path / "none.safetensors").encode()) == -3
    small = {"q_norm": np.ones(128, np.uint16)}
    p = tmp_path / "a.safetensors"
    du.write_safetensors(p, small)
    assert lib.s2p_draft_load(ctypes.byref(m), str(p).encode()) == -1
    bad = {"fuse.weight": np.zeros((4, 4), np.uint16)}
    du.write_safetensors(p, bad)
    assert lib.s2p_draft_load(ctypes.byref(m), str(p).encode()) == -1
    du.write_safetensors(p, bad, dtype="F16", shapes={"fuse.weight": [2560, 5120]})
    assert lib.s2p_draft_load(ctypes.byref(m), str(p).encode()) == -1
    st = s2pamd.DraftState()
    # stepping an unloaded model is rejected
    assert lib.s2p_draft_step(ctypes.byref(m), ctypes.byref(st), None, None, None, None) == -1
