/* s2pro MI355X — the INT4-g32 GEMM of s2p_int4p_gemm_tc for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).
 *
 * s2p_int4p_gemm_tc runs its split-K paths (k_gemm4's K splits, the split-K
 * GEMV engine) on the process context's scratch: split partials and
 * per-row-block arrival counters that s2p_gemm_init allocates.  This entry
 * point runs the same launcher and kernels on a fixed file-scope device
 * array instead, so it allocates nothing:
 *   - partials: NOALLOC_PART_FLOATS floats (8 MiB); the launcher sizes its
 *     K splits within that capacity (fewer splits when a shape needs more);
 *   - arrival counters: NOALLOC_COUNTERS words, one per 64-row block, so
 *     N <= NOALLOC_COUNTERS * 64;
 *   - every GPU the library runs on holds the array until the process ends.
 * The counters are cleared by a fill kernel on the caller's stream before
 * each call (no memset node); partials need no clearing (every split writes
 * its own before the last arriver reads them).  Calls that overlap on one GPU
 * (two streams, or two host threads) share the array and race: the caller
 * serialises them. */
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "gemv_internal.h"
#include "s2pro/gemm.h"

#define NOALLOC_PART_FLOATS (1u << 21)
#define NOALLOC_COUNTERS 4096u
#define NOALLOC_MAX_DEV 64

static __device__ __align__(256) unsigned char scratch[(size_t)NOALLOC_PART_FLOATS * 4 +
                                                       (size_t)NOALLOC_COUNTERS * 4];

/* the array's device address, per device (each GPU holds its own copy) */
static std::once_flag g_once[NOALLOC_MAX_DEV];
static void* g_ptr[NOALLOC_MAX_DEV];
static hipError_t g_err[NOALLOC_MAX_DEV];

static hipError_t scratch_ptr(unsigned char** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= NOALLOC_MAX_DEV) return hipErrorInvalidDevice;
    std::call_once(g_once[dev], [dev]() {
        void* p = nullptr;
        g_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_ptr[dev] = g_err[dev] == hipSuccess ? p : nullptr;
    });
    if (g_err[dev] != hipSuccess) return g_err[dev];
    *out = (unsigned char*)g_ptr[dev];
    return hipSuccess;
}

__global__ void k_noalloc_zero(unsigned* c, unsigned n) {
    for (unsigned i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        c[i] = 0u;
}

extern "C" s2p_status s2p_int4p_gemm_tc_noalloc(void* y_bf16, const void* x_bf16,
                                                const void* w_pack, const void* scales_f16, int M,
                                                int N, int K, int G, hipStream_t stream) {
    if (!y_bf16 || !x_bf16 || !w_pack || !scales_f16 || M <= 0 || M > GEMV_MAX_M || N <= 0 ||
        K <= 0 || G != 32 || K % 128 != 0)
        return S2P_ERR_INVALID;
    const unsigned nrb = (unsigned)((N + 63) / 64);
    if (nrb > NOALLOC_COUNTERS) {
        fprintf(stderr,
                "[s2pro] s2p_int4p_gemm_tc_noalloc: N = %d exceeds the fixed scratch "
                "(at most %u outputs: %u arrival counters of 64 rows)\n",
                N, NOALLOC_COUNTERS * 64u, NOALLOC_COUNTERS);
        return S2P_ERR_INVALID;
    }
    unsigned char* base = nullptr;
    hipError_t e = scratch_ptr(&base);
    if (e != hipSuccess) {
        fprintf(stderr, "[s2pro] s2p_int4p_gemm_tc_noalloc: scratch address: %s\n",
                hipGetErrorString(e));
        return S2P_ERR_CUDA;
    }
    unsigned* counters = (unsigned*)(base + (size_t)NOALLOC_PART_FLOATS * 4);
    hipLaunchKernelGGL(k_noalloc_zero, dim3((nrb + 255) / 256), dim3(256), 0, stream, counters, nrb);
    e = hipGetLastError();
    if (e != hipSuccess) return S2P_ERR_CUDA;
    GemvArgs a;
    memset(&a, 0, sizeof(a));
    a.w = (const uint8_t*)w_pack;
    a.s = scales_f16;
    a.x = (const uint16_t*)x_bf16;
    a.ldx = K;
    a.y = (uint16_t*)y_bf16;
    a.ldy = N;
    a.M = M;
    a.N = N;
    a.K = K;
    a.wfmt = GEMV_W_INT4;
    a.xmode = GEMV_X_PLAIN;
    a.epi = GEMV_EPI_STORE;
    a.part = (float*)base;
    a.part_cap = NOALLOC_PART_FLOATS;
    a.counters = counters;
    e = s2p_gemv_launch(&a, stream);
    if (e != hipSuccess) {
        fprintf(stderr,
                "[s2pro] s2p_int4p_gemm_tc_noalloc (M=%d, N=%d, K=%d): %s (the split partials "
                "must fit %u floats)\n",
                M, N, K, hipGetErrorString(e), NOALLOC_PART_FLOATS);
        return e == hipErrorInvalidValue ? S2P_ERR_INVALID : S2P_ERR_CUDA;
    }
    return S2P_OK;
}
