"""GEMV engine and weight formats on the GPU vs the CPU oracle.

Tolerance (north star: logits within 1e-2 relative, bf16 accumulate to fp32):
every output element within 1e-2 * |exact| + 1e-2 * rms(exact) of the binary64
dot product; quantisers and packing are bit-exact."""
import ctypes

import numpy as np
import pytest
import torch

import pyoracle as po
import s2pamd
from gpu_util import (P, S, assert_close_rel, bf16_bits, bf16_vals, empty, h2d_raw, to_dev,
                      to_host)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    lib = s2pamd.load()
    s2pamd.check(lib.s2p_gemm_init(128), "gemm init")
    return lib


@pytest.fixture(params=[0, 2], ids=["auto", "splitk"])
def engine(request, lib):
    """launcher's engine choice (whole-K workgroups where they fit), then the
    split-K engine forced (per call: s2p_gemv_engine_run)"""
    return request.param


def int4p_gemv(lib, engine, y, x, w, s, M, N, K):
    """the public INT4-g32 GEMV (engine 0) or the same GEMV on the split-K
    engine"""
    if engine == 0:
        return lib.s2p_int4p_gemv(P(y), P(x), P(w), P(s), M, N, K, 32, S())
    return lib.s2p_gemv_engine_run(engine, 0, P(y), P(x), P(w), P(s), M, N, K, S())


def rand_int4(r, N, K):
    packed = r.integers(0, 256, (N, K // 2), dtype=np.uint8)
    scales = np.abs(r.standard_normal((N, K // 32)) * 0.02).astype(np.float16).view(np.uint16)
    return packed, scales


# config 1 first: one INT4-g32 linear 2560 -> 9728 at M = 5
@pytest.mark.parametrize("M,N,K", [(5, 9728, 2560), (1, 6144, 2560), (16, 2560, 4096),
                                   (5, 2560, 9728), (5, 19456, 2560), (3, 4097, 2560),
                                   (7, 100, 512)])
def test_int4p_gemv_vs_oracle(lib, engine, M, N, K):
    r = np.random.default_rng(1000 + M * 7 + N)
    packed, scales = rand_int4(r, N, K)
    x = bf16_bits(r.standard_normal((M, K)).astype(np.float32))
    y = empty((M, N))
    s2pamd.check(int4p_gemv(lib, engine, y, to_dev(x), to_dev(packed), to_dev(scales), M, N, K),
                 "int4p gemv")
    got = bf16_vals(to_host(y, np.uint16))
    exact = po.int4p_gemv_f64(x, packed, scales, M, N, K)
    assert_close_rel(got, exact, what=f"int4p M={M} N={N} K={K}")
    # against the reference-order restatement: at most a few bf16 ulps apart
    ref = bf16_vals(po.int4p_gemv(x, packed, scales, M, N, K))
    assert np.max(np.abs(got - ref) / (np.abs(ref) + 1e-3 * np.abs(ref).max())) < 2e-2


@pytest.mark.parametrize("M,N,K", [(40, 6144, 2560), (68, 2560, 4096), (128, 256, 2560),
                                   (17, 9728, 2560), (96, 4097, 2560), (80, 4097, 2560),
                                   (33, 2560, 9728), (24, 512, 640), (64, 300, 1152),
                                   (70, 1000, 1152)])
def test_int4p_gemm_large_m(lib, M, N, K):
    r = np.random.default_rng(2000 + M)
    packed, scales = rand_int4(r, N, K)
    x = bf16_bits(r.standard_normal((M, K)).astype(np.float32))
    y = empty((M, N))
    s2pamd.check(lib.s2p_int4p_gemm_tc(P(y), P(to_dev(x)), P(to_dev(packed)),
                                       P(to_dev(scales)), M, N, K, 32, S()), "int4p gemm")
    got = bf16_vals(to_host(y, np.uint16))
    assert_close_rel(got, po.int4p_gemv_f64(x, packed, scales, M, N, K), what=f"M={M}")


@pytest.mark.parametrize("M,N,K", [(96, 4097, 2560), (81, 6144, 2560), (88, 2560, 4096)])
def test_int4p_gemm_six_tiles_repeat(lib, M, N, K):
    """k_gemm4 at six column tiles (M = 81..96) with its split-K handoff:
    eight calls on the same inputs give the same bits, within the oracle's
    tolerance"""
    r = np.random.default_rng(5000 + M)
    packed, scales = rand_int4(r, N, K)
    x = bf16_bits(r.standard_normal((M, K)).astype(np.float32))
    xd, wd, sd = to_dev(x), to_dev(packed), to_dev(scales)
    first = None
    for i in range(8):
        y = empty((M, N))
        s2pamd.check(lib.s2p_int4p_gemm_tc(P(y), P(xd), P(wd), P(sd), M, N, K, 32, S()))
        got = to_host(y, np.uint16)
        if first is None:
            first = got
            assert_close_rel(bf16_vals(got), po.int4p_gemv_f64(x, packed, scales, M, N, K),
                             what=f"M={M}")
        else:
            bad = np.argwhere(got != first)
            assert bad.size == 0, f"call {i}: {len(bad)} outputs differ, first at {bad[:4].tolist()}"


def test_int4p_gemv_closed_forms(lib, engine):
    """All weights -8, unit scales: y = -8 * sum(x); single nonzero weight."""
    M, N, K = 4, 64, 2560
    r = np.random.default_rng(3)
    x = bf16_bits(r.standard_normal((M, K)).astype(np.float32))
    xf = bf16_vals(x).astype(np.float64)
    one = np.full((N, K // 32), np.float16(1.0).view(np.uint16), np.uint16)
    packed = np.full((N, K // 2), 0x88, np.uint8)
    y = empty((M, N))
    s2pamd.check(int4p_gemv(lib, engine, y, to_dev(x), to_dev(packed), to_dev(one), M, N, K))
    got = bf16_vals(to_host(y, np.uint16))
    assert_close_rel(got, np.repeat((-8 * xf.sum(1))[:, None], N, 1), what="all -8")
    # a single nonzero weight of +-1 with a power-of-two scale: y = +-x/2,
    # exactly representable, so the GEMV must return it bit for bit
    q = np.zeros((N, K), np.int8)
    for n in range(N):
        q[n, (n * 37) % K] = 1 if n % 2 else -1
    packed = po.int4_pack(q, N, K)
    half = np.full((N, K // 32), np.float16(0.5).view(np.uint16), np.uint16)
    s2pamd.check(int4p_gemv(lib, engine, y, to_dev(x), to_dev(packed), to_dev(half), M, N, K))
    got = bf16_vals(to_host(y, np.uint16))
    want = np.stack([xf[:, (n * 37) % K] * (1 if n % 2 else -1) * 0.5 for n in range(N)], 1)
    # exact up to the output rounding and the fp32 group-bias cancellation
    # (absolute error ~ ulp(1.5 * sum of the group's x), far below 1e-4)
    assert np.all(np.abs(got - want) <= np.abs(want) * 2 ** -8 + 1e-4)


@pytest.mark.parametrize("M,N,K", [(5, 6144, 2560), (5, 2560, 9728), (16, 19456, 2560),
                                   (40, 2560, 4096)])
def test_int8_gemv_vs_oracle(lib, engine, M, N, K):
    r = np.random.default_rng(3000 + M + N)
    q = r.integers(-127, 128, (N, K)).astype(np.int8)
    s = (np.abs(r.standard_normal(N)) * 1e-3).astype(np.float32)
    x = bf16_bits(r.standard_normal((M, K)).astype(np.float32))
    y = empty((M, N))
    lin = s2pamd.Linear()
    lin.in_features, lin.out_features = K, N
    lin.int8_ready, lin.q_group, lin.q_packed = 1, 0, 0
    qd, sd = to_dev(q), to_dev(s)
    lin.w_int8.data, lin.w_iscale.data = qd.data_ptr(), sd.data_ptr()
    if engine != 0:
        s2pamd.check(lib.s2p_gemv_engine_run(engine, 1, P(y), P(to_dev(x)), P(qd), P(sd), M, N, K,
                                             S()))
    elif M <= 16:
        s2pamd.check(lib.s2p_int8_gemv(P(y), P(to_dev(x)), P(qd), P(sd), M, N, K, S()))
    else:
        s2pamd.check(lib.s2p_linear_forward(ctypes_ref(lin), P(to_dev(x)), P(y), M, 2, S()))
    got = bf16_vals(to_host(y, np.uint16))
    assert_close_rel(got, po.int8_gemv_f64(x, q, s, M, N, K), what=f"int8 M={M}")


def ctypes_ref(s):
    return ctypes.byref(s)


def test_quantisers_bit_exact(lib):
    r = np.random.default_rng(5)
    N, K = 96, 2560
    w = bf16_bits(r.standard_normal((N, K)).astype(np.float32) * 0.03)
    wd = to_dev(w)
    q = torch.empty((N, K), dtype=torch.int8, device="cuda")
    sc = empty((N, K // 32))
    s2pamd.check(lib.s2p_intq_quant(P(q), P(sc), P(wd), N, K, 32, 7, 1, S()))
    q_ref, s_ref = po.intq_quant(w, N, K, 32, 7, 1)
    gs = to_host(sc, np.uint16)
    bad = np.flatnonzero(gs.ravel() != s_ref.ravel())
    assert bad.size == 0, (f"{bad.size} group scales differ; first {bad[:4]}: gpu "
                           f"{gs.ravel()[bad[:4]]} oracle {s_ref.ravel()[bad[:4]]}")
    gq = to_host(q)
    bad = np.flatnonzero(gq.ravel() != q_ref.ravel())
    assert bad.size == 0, f"{bad.size} quantised values differ; first {bad[:4]}"
    pk = torch.empty((N, K // 2), dtype=torch.uint8, device="cuda")
    s2pamd.check(lib.s2p_int4_pack(P(pk), P(q), N, K, S()))
    assert np.array_equal(to_host(pk), po.int4_pack(q_ref, N, K))
    deq = empty((N, K))
    s2pamd.check(lib.s2p_int4p_dequant(P(deq), P(pk), P(sc), N, K, 32, S()))
    assert np.array_equal(to_host(deq, np.uint16), po.int4p_dequant(po.int4_pack(q_ref, N, K),
                                                                     s_ref, N, K))
    q8 = torch.empty((N, K), dtype=torch.int8, device="cuda")
    s8 = torch.empty((N,), dtype=torch.float32, device="cuda")
    s2pamd.check(lib.s2p_int8_quant(P(q8), P(s8), P(wd), N, K, S()))
    q8_ref, s8_ref = po.int8_quant(w, N, K)
    assert np.array_equal(to_host(q8), q8_ref)
    assert np.array_equal(to_host(s8), s8_ref)


def test_linear_prepare_site_and_forward(lib):
    """bf16 weights -> INT4-g32 MSE (backbone policy) -> forward at M=5."""
    r = np.random.default_rng(6)
    N, K, M = 512, 2560, 5
    w = bf16_bits(r.standard_normal((N, K)).astype(np.float32) * 0.02)
    # the linear takes ownership of its bf16 weights: allocate them through the library
    t = s2pamd.Tensor()
    shape = (ctypes.c_int64 * 2)(N, K)
    s2pamd.check(lib.s2p_tensor_device_alloc(ctypes_ref(t), 0, 2, shape))
    h2d_raw(w, t.data)
    lin = s2pamd.Linear()
    s2pamd.check(lib.s2p_linear_from_device_bf16(ctypes_ref(lin), t.data, K, N))
    s2pamd.check(lib.s2p_linear_prepare_int8_site(ctypes_ref(lin), 0, S()))
    assert lin.q_packed == 1 and lin.q_group == 32 and lin.w_bf16.data is None
    x = bf16_bits(r.standard_normal((M, K)).astype(np.float32))
    y = empty((M, N))
    s2pamd.check(lib.s2p_linear_forward(ctypes_ref(lin), P(to_dev(x)), P(y), M, 2, S()))
    q_ref, s_ref = po.intq_quant(w, N, K, 32, 7, 1)
    exact = po.int4p_gemv_f64(x, po.int4_pack(q_ref, N, K), s_ref, M, N, K)
    assert_close_rel(bf16_vals(to_host(y, np.uint16)), exact, what="prepared linear")
    lib.s2p_linear_free(ctypes_ref(lin))


@pytest.mark.parametrize("M,blocks,K", [(68, 160, 2560), (40, 160, 2560), (17, 608, 9728)])
def test_g4_rms_inverse_rms(lib, M, blocks, K):
    """k_g4_rms: inv[m] = 1 / sqrt(sum of row m's per-16-column sums of
    squares / K + eps), from the [blocks][128] layout the residual epilogues
    write; against binary64 (the float sums differ only in their order)."""
    r = np.random.default_rng(M + blocks)
    ssq = np.zeros((blocks, 128), np.float32)
    ssq[:, :M] = (r.random((blocks, M)) * 16.0).astype(np.float32)
    ssq[:, 1] = 0.0  # a row of zeros: inv = 1 / sqrt(eps)
    eps = 1e-6
    inv = empty((M,), dtype=torch.float32)
    fn = lib.s2p_g4_rms_launch
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                   ctypes.c_void_p, ctypes.c_void_p]
    s2pamd.hip_check(fn(P(to_dev(ssq)), blocks, M, K, eps, P(inv), S()))
    got = to_host(inv, np.float32).astype(np.float64)
    exact = 1.0 / np.sqrt(ssq[:, :M].astype(np.float64).sum(axis=0) / K + eps)
    assert np.all(np.abs(got - exact) <= 2e-6 * exact), np.max(np.abs(got - exact) / exact)
