"""The allocation-free INT4 GEMM (s2p_int4p_gemm_tc_noalloc) against the
context-scratch entry point it mirrors (s2p_int4p_gemm_tc): same launcher and
kernels, so the same bits, on two calls in a row (the second smaller, on the
scratch the first one left behind), plus the size limit."""
import numpy as np
import pytest

import pyoracle as po
import s2pamd
from gpu_util import P, S, assert_close_rel, bf16_bits, bf16_vals, empty, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    lib = s2pamd.load()
    s2pamd.check(lib.s2p_gemm_init(128), "gemm init")
    return lib


def rand_case(seed, M, N, K):
    r = np.random.default_rng(seed)
    packed = r.integers(0, 256, (N, K // 2), dtype=np.uint8)
    scales = np.abs(r.standard_normal((N, K // 32)) * 0.02).astype(np.float16).view(np.uint16)
    x = bf16_bits(r.standard_normal((M, K)).astype(np.float32))
    return x, packed, scales


@pytest.mark.parametrize("first,second", [((96, 4097, 2560), (24, 2560, 4096)),
                                          ((40, 6144, 2560), (5, 2560, 9728))])
def test_noalloc_matches_context_entry(lib, first, second):
    for i, (M, N, K) in enumerate((first, second)):
        print(f"noalloc call {i}: M={M} N={N} K={K}", flush=True)
        x, packed, scales = rand_case(7000 + 13 * i + M, M, N, K)
        xd, wd, sd = to_dev(x), to_dev(packed), to_dev(scales)
        y0, y1 = empty((M, N)), empty((M, N))
        s2pamd.check(lib.s2p_int4p_gemm_tc(P(y0), P(xd), P(wd), P(sd), M, N, K, 32, S()))
        s2pamd.check(lib.s2p_int4p_gemm_tc_noalloc(P(y1), P(xd), P(wd), P(sd), M, N, K, 32, S()),
                     "noalloc gemm")
        a, b = to_host(y0, np.uint16), to_host(y1, np.uint16)
        assert np.array_equal(a, b), f"call {i}: {int((a != b).sum())} outputs differ"
        assert_close_rel(bf16_vals(b), po.int4p_gemv_f64(x, packed, scales, M, N, K),
                         what=f"noalloc M={M}")


def test_noalloc_rejects_oversize(lib):
    M, N, K = 2, 4096 * 64 + 1, 128
    y = empty((1, 1))
    x = empty((1, 1))
    rc = lib.s2p_int4p_gemm_tc_noalloc(P(y), P(x), P(x), P(x), M, N, K, 32, S())
    assert rc == -1  # S2P_ERR_INVALID
