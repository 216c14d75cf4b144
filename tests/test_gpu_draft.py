"""Draft model on the GPU (reference src/draft/draft.c): s2p_gemm_bf16 (the bf16 path of
the GEMV engine) against the oracle and binary64, and s2p_draft_load +
s2p_draft_step against the oracle's draft step and binary64 truth.

Tolerance (north star: 1e-2 relative): the GPU output within max(1e-2, half
the oracle's own distance to binary64) of the oracle in L2 norm, and no less
accurate than 1.25x the oracle's error against binary64."""
import ctypes

import numpy as np
import pytest

import draft_util as du
import f64_forward as f64
import pyoracle as po
import s2pamd
from gpu_util import P, S, assert_close_norm, bf16_vals, empty, h2d_raw, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    lib = s2pamd.load()
    s2pamd.check(lib.s2p_gemm_init(128), "gemm init")
    return lib


@pytest.mark.parametrize("M,N,K", [(1, 2560, 5120), (1, 6144, 2560), (1, 2560, 9728),
                                   (5, 9728, 2560), (16, 2560, 9728), (3, 100, 200)])
def test_gemm_bf16_vs_oracle(lib, M, N, K):
    r = np.random.default_rng(M * 31 + N + K)
    x = du.bf16_bits(r.standard_normal((M, K)).astype(np.float32))
    w = du.bf16_bits(r.standard_normal((N, K)).astype(np.float32) / np.float32(np.sqrt(K)))
    y = empty((M, N))
    s2pamd.check(lib.s2p_gemm_bf16(P(to_dev(x)), P(to_dev(w)), P(y), M, N, K, S()), "gemm_bf16")
    got = bf16_vals(to_host(y, np.uint16)).astype(np.float64)
    want = bf16_vals(po.gemm_bf16(x, w, M, N, K)).astype(np.float64)
    t = po.gemm_bf16_f64(x, w, M, N, K)
    bound = np.abs(t) * 2.0 ** -8 + K * 2.0 ** -23 * (np.abs(f64.bf(x)) @ np.abs(f64.bf(w)).T)
    assert np.all(np.abs(got - t) <= bound), f"max excess {np.max(np.abs(got - t) - bound):.3g}"
    # one bf16 rounding of two fp32 sums in different orders: mostly equal
    assert np.mean(got == want) > 0.9


def test_gemm_bf16_argument_errors(lib):
    assert lib.s2p_gemm_bf16(None, None, None, 1, 1, 1, S()) == -1
    x = empty((1, 128))
    assert lib.s2p_gemm_bf16(P(x), P(x), P(x), 0, 1, 128, S()) == -1


@pytest.fixture(scope="module")
def draft(lib, tmp_path_factory):
    w = du.make_weights(21)
    path = tmp_path_factory.mktemp("draft") / "draft.safetensors"
    du.write_safetensors(path, w)
    m = s2pamd.DraftModel()
    s2pamd.check(lib.s2p_draft_load(ctypes.byref(m), str(path).encode()), "draft load")
    yield m, w
    lib.s2p_draft_free(ctypes.byref(m))


def test_draft_load_places_weights(lib, draft):
    m, w = draft
    for name, field in du.FIELD.items():
        t = getattr(m, field)
        assert t.bytes == w[name].nbytes and t.on_device == 1
    got = s2pamd_d2h(m.wqkv.data, w["wqkv.weight"].nbytes)
    assert np.array_equal(got.reshape(w["wqkv.weight"].shape), w["wqkv.weight"])


def s2pamd_d2h(ptr, nbytes):
    from gpu_util import d2h
    return d2h(ptr, nbytes, np.uint16)


def test_draft_steps_vs_oracle(lib, draft):
    """Four steps from an empty state, then two at position 700 over a
    pre-filled cache; outputs vs the oracle and binary64, and the cache
    (appended K/V) vs the oracle's."""
    m, w = draft
    arrs = du.oracle_arrays(w)
    d = po.make_draft(arrs)
    W = du.f64_weights(w)
    st = s2pamd.DraftState()
    s2pamd.check(lib.s2p_draft_state_init(ctypes.byref(st)), "state init")
    try:
        ctx = 4096
        kc = np.zeros((8, ctx, 128), np.uint16)
        vc = np.zeros((8, ctx, 128), np.uint16)
        h2d_raw(kc, st.kc.data)
        h2d_raw(vc, st.vc.data)
        k64, v64 = np.zeros((8, ctx, 128)), np.zeros((8, ctx, 128))
        r = np.random.default_rng(5)
        out = empty((2560,))
        for pos in [0, 1, 2, 3, 700, 701]:
            if pos == 700:
                fill = du.bf16_bits(r.standard_normal((2, 8, 700, 128)).astype(np.float32))
                kc[:, 4:700], vc[:, 4:700] = fill[0][:, 4:], fill[1][:, 4:]
                h2d_raw(kc, st.kc.data)
                h2d_raw(vc, st.vc.data)
                k64[:, 4:700], v64[:, 4:700] = f64.bf(kc[:, 4:700]), f64.bf(vc[:, 4:700])
                st.pos = 700
            assert st.pos == pos
            h = du.bf16_bits(r.standard_normal(2560).astype(np.float32))
            e = du.bf16_bits(r.standard_normal(2560).astype(np.float32))
            s2pamd.check(lib.s2p_draft_step(ctypes.byref(m), ctypes.byref(st), P(to_dev(h)),
                                            P(to_dev(e)), P(out), S()), f"draft step {pos}")
            got = bf16_vals(to_host(out, np.uint16)).astype(np.float64)
            want_bits = po.draft_step(d, kc, vc, ctx, pos, h, e)
            want = f64.bf(want_bits)
            truth = f64.draft_step(W, f64.bf(h), f64.bf(e), k64, v64, pos)
            e_ref = np.linalg.norm(want - truth) / np.linalg.norm(truth)
            e_gpu = np.linalg.norm(got - truth) / np.linalg.norm(truth)
            print(f"pos {pos}: gpu {e_gpu:.2e} oracle {e_ref:.2e}")
            assert_close_norm(got[None], want[None], rel=1e-2, what=f"draft out {pos}")
            assert e_gpu <= 1.25 * e_ref + 1e-3, f"pos {pos}: gpu {e_gpu:.3g} oracle {e_ref:.3g}"
            # the step's K/V against the oracle's (same bf16 values up to the
            # GPU's own roundings of the wqkv GEMV)
            kd = s2pamd_d2h(st.kc.data, kc.nbytes).reshape(8, ctx, 128)
            assert np.allclose(f64.bf(kd[:, pos]), f64.bf(kc[:, pos]), rtol=3e-2, atol=3e-2)
            # the GPU's next steps read its own K/V; the oracle and truth read
            # the oracle's: keep the three on the oracle's values
            kc[:, pos] = kd[:, pos]
            vc[:, pos] = s2pamd_d2h(st.vc.data, vc.nbytes).reshape(8, ctx, 128)[:, pos]
            k64[:, pos], v64[:, pos] = f64.bf(kc[:, pos]), f64.bf(vc[:, pos])
        assert st.pos == 702
        st.pos = 4096
        assert lib.s2p_draft_step(ctypes.byref(m), ctypes.byref(st), P(out), P(out), P(out),
                                  S()) == -1
    finally:
        lib.s2p_draft_state_free(ctypes.byref(st))


def int4_linear(packed_d, scales_d, N, K):
    lin = s2pamd.Linear()
    lin.in_features, lin.out_features = K, N
    lin.q_packed, lin.q_group = 1, 32
    lin.w_pack.data, lin.w_pack.bytes, lin.w_pack.on_device = packed_d.data_ptr(), N * K // 2, 1
    lin.w_iscale.data, lin.w_iscale.bytes, lin.w_iscale.on_device = (scales_d.data_ptr(),
                                                                     N * K // 16, 1)
    return lin


def test_draft_head_slice(lib):
    """s2p_draft_head: the draft's q logits over the tied-head slice (semantic
    rows 151678.. + EOS 151645) from the full INT4 head read in place, and from
    a 4,097-row slice head; both against binary64 on the gathered rows."""
    N, K, rows = 155776, 2560, 3
    r = np.random.default_rng(41)
    packed = r.integers(0, 256, (N, K // 2), dtype=np.uint8)
    scales = np.abs(r.standard_normal((N, K // 32)) * 0.02).astype(np.float16).view(np.uint16)
    hid = du.bf16_bits(r.standard_normal((rows, K)).astype(np.float32))
    sel = np.r_[151678:151678 + 4096, 151645]
    ps, ss = np.ascontiguousarray(packed[sel]), np.ascontiguousarray(scales[sel])
    want = po.int4p_gemv_f64(hid, ps, ss, rows, 4097, K)
    full_p, full_s = to_dev(packed), to_dev(scales)
    sl_p, sl_s = to_dev(ps), to_dev(ss)
    hd = to_dev(hid)
    for name, lin in (("full", int4_linear(full_p, full_s, N, K)),
                      ("slice", int4_linear(sl_p, sl_s, 4097, K))):
        out = empty((rows, 4097))
        s2pamd.check(lib.s2p_draft_head(ctypes.byref(lin), P(hd), P(out), rows, S()),
                     f"draft head {name}")
        got = bf16_vals(to_host(out, np.uint16))
        assert_close_norm(got, want, rel=1e-2, what=f"draft head ({name})")
    bad = int4_linear(sl_p, sl_s, 4000, K)
    assert lib.s2p_draft_head(ctypes.byref(bad), P(hd), P(out), rows, S()) == -1


def test_draft_step_graph_replay(lib, draft):
    """The step captured into a graph at one position and replayed three
    times (eager work and synchronisation between replays) gives the eager
    step's bits every time."""
    import torch
    m, w = draft
    st = s2pamd.DraftState()
    s2pamd.check(lib.s2p_draft_state_init(ctypes.byref(st)), "state init")
    try:
        r = np.random.default_rng(9)
        kc = du.bf16_bits(r.standard_normal((8, 4096, 128)).astype(np.float32) * 0.5)
        vc = du.bf16_bits(r.standard_normal((8, 4096, 128)).astype(np.float32) * 0.5)
        h = to_dev(du.bf16_bits(r.standard_normal(2560).astype(np.float32)))
        e = to_dev(du.bf16_bits(r.standard_normal(2560).astype(np.float32)))
        pos = 37

        def reset():
            h2d_raw(kc, st.kc.data)
            h2d_raw(vc, st.vc.data)
            st.pos = pos

        reset()
        out_eager = empty((2560,))
        s2pamd.check(lib.s2p_draft_step(ctypes.byref(m), ctypes.byref(st), P(h), P(e),
                                        P(out_eager), S()), "eager step")
        torch.cuda.synchronize()
        want = to_host(out_eager, np.uint16)
        reset()
        out = empty((2560,))
        side = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            s2pamd.check(lib.s2p_draft_step(ctypes.byref(m), ctypes.byref(st), P(h), P(e),
                                            P(out), s2pamd.stream_ptr()), "captured step")
        for i in range(3):
            reset()
            out.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            got = to_host(out, np.uint16)
            assert np.array_equal(got, want), f"replay {i}: {int((got != want).sum())} differ"
    finally:
        lib.s2p_draft_state_free(ctypes.byref(st))
