/* s2pro MI355X — weight-format kernels: quantisers, nibble packing and
 * dequantisation (reference src/sched/int8_gemv.cu:32-58, 106-114, 135-195,
 * 244-277, 731-744, 752-1001).  Load-time operations; they reproduce the
 * reference's arithmetic (RTN ties-to-even, f16-rounded scale candidates, the
 * MSE clip search with its thread-tree error sum and FMA contraction) so that
 * packed weights are bit-identical to the reference quantiser's output. */
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>

#include "common.h"
#include "s2pro/gemm.h"

/* per-row absmax/levels RTN (int8_gemv.cu:32-58) */
__global__ __launch_bounds__(256) void k_quant(int8_t* __restrict__ q, float* __restrict__ scales,
                                               const uint16_t* __restrict__ w, int K, int levels) {
    __shared__ float red[256];
    const int n = blockIdx.x;
    const uint16_t* row = w + (size_t)n * K;
    float amax = 0.f;
    for (int k = threadIdx.x; k < K; k += 256) amax = fmaxf(amax, fabsf(bf2f(row[k])));
    red[threadIdx.x] = amax;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
        __syncthreads();
    }
    const float scale = red[0] > 0.f ? __fdiv_rn(red[0], (float)levels) : 1.0f;
    const float inv = __fdiv_rn(1.0f, scale);
    if (threadIdx.x == 0) scales[n] = scale;
    for (int k = threadIdx.x; k < K; k += 256) {
        int v = (int)rintf(__fmul_rn(bf2f(row[k]), inv));
        v = v > levels ? levels : (v < -levels ? -levels : v);
        q[(size_t)n * K + k] = (int8_t)v;
    }
}

/* group-wise quantiser, one thread per group; the reference's per-thread
 * strided error sums over min(G,256) threads and their shared-memory tree
 * (int8_gemv.cu:165-186) are evaluated in the same order */
__global__ __launch_bounds__(256) void k_quant_g(int8_t* __restrict__ q,
                                                 uint16_t* __restrict__ scales,
                                                 const uint16_t* __restrict__ w, int64_t n_groups,
                                                 int K, int G, int levels, int mse) {
    const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= n_groups) return;
    const int ng = K / G;
    const int64_t n = gi / ng;
    const int g = (int)(gi - n * ng);
    const uint16_t* wp = w + (size_t)n * K + (size_t)g * G;
    const int T = G < 256 ? G : 256;
    float amax = 0.f;
    for (int k = 0; k < G; k++) amax = fmaxf(amax, fabsf(bf2f(wp[k])));
    const float base = amax > 0.f ? __fdiv_rn(amax, (float)levels) : 1.0f;
    float scale = h2f(f2h(base));
    if (mse && amax > 0.f) {
        float best_err = 3.4e38f, best_s = scale;
        float red[256];
        for (int c = 0; c < 32; c++) {
            const float s = h2f(f2h(__fmul_rn(base, __fsub_rn(1.0f, __fdiv_rn((float)c, 64.0f)))));
            const float inv = __fdiv_rn(1.0f, s);
            for (int t = 0; t < T; t++) {
                float err = 0.f;
                for (int k = t; k < G; k += T) {
                    const float v = bf2f(wp[k]);
                    int qi = (int)rintf(__fmul_rn(v, inv));
                    qi = qi > levels ? levels : (qi < -levels ? -levels : qi);
                    const float d = fmaf(-(float)qi, s, v);
                    err = fmaf(d, d, err);
                }
                red[t] = err;
            }
            for (int r = T / 2; r > 0; r >>= 1)
                for (int t = 0; t < r; t++) red[t] = __fadd_rn(red[t], red[t + r]);
            if (red[0] < best_err) {
                best_err = red[0];
                best_s = s;
            }
        }
        scale = best_s;
    }
    scales[gi] = f2h(scale);
    const float inv = __fdiv_rn(1.0f, scale);
    for (int k = 0; k < G; k++) {
        int v = (int)rintf(__fmul_rn(bf2f(wp[k]), inv));
        v = v > levels ? levels : (v < -levels ? -levels : v);
        q[(size_t)n * K + (size_t)g * G + k] = (int8_t)v;
    }
}

__global__ __launch_bounds__(256) void k_pack_nib(uint8_t* __restrict__ p,
                                                  const int8_t* __restrict__ q, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = (uint8_t)((q[2 * i] & 0xF) | ((q[2 * i + 1] & 0xF) << 4));
}

/* fmt 0: per-channel int8; 1: int8 container group-wise; 2: packed int4 */
__global__ __launch_bounds__(256) void k_dequant(uint16_t* __restrict__ o, const void* __restrict__ w,
                                                 const void* __restrict__ sc, int K, int gshift,
                                                 int fmt) {
    const int n = blockIdx.x;
    for (int k = threadIdx.x; k < K; k += 256) {
        int v;
        float s;
        if (fmt == 2) {
            const uint8_t b = ((const uint8_t*)w)[(size_t)n * (K >> 1) + (k >> 1)];
            v = (k & 1) ? ((int)(int8_t)b >> 4) : ((int)(int8_t)(uint8_t)(b << 4) >> 4);
        } else {
            v = ((const int8_t*)w)[(size_t)n * K + k];
        }
        if (fmt == 0) s = ((const float*)sc)[n];
        else s = h2f(((const uint16_t*)sc)[(size_t)n * (K >> gshift) + (k >> gshift)]);
        o[(size_t)n * K + k] = f2bf(__fmul_rn((float)v, s));
    }
}

static int gshift_of(int G) {
    if (G < 16 || (G & (G - 1)) != 0) return -1;
    int s = 0;
    while ((1 << s) < G) s++;
    return s;
}

static s2p_status launched(const char* what, int N, int K) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "[s2pro] %s launch (N=%d,K=%d): %s\n", what, N, K, hipGetErrorString(e));
        return S2P_ERR_CUDA;
    }
    return S2P_OK;
}

extern "C" s2p_status s2p_int8_quant(void* w_i8, float* scales, const void* w_bf16, int N, int K,
                                     hipStream_t stream) {
    if (!w_i8 || !scales || !w_bf16 || N <= 0 || K <= 0) return S2P_ERR_INVALID;
    hipLaunchKernelGGL(k_quant, dim3(N), dim3(256), 0, stream, (int8_t*)w_i8, scales,
                       (const uint16_t*)w_bf16, K, 127);
    return launched("int8 quant", N, K);
}

extern "C" s2p_status s2p_intq_quant(void* w_i8, void* scales_f16, const void* w_bf16, int N,
                                     int K, int G, int levels, int mse, hipStream_t stream) {
    if (!w_i8 || !scales_f16 || !w_bf16 || N <= 0 || K <= 0 || levels <= 0) return S2P_ERR_INVALID;
    if (gshift_of(G) < 0 || K % G != 0) return S2P_ERR_INVALID;
    const int64_t ng = (int64_t)N * (K / G);
    hipLaunchKernelGGL(k_quant_g, dim3((unsigned)((ng + 255) / 256)), dim3(256), 0, stream,
                       (int8_t*)w_i8, (uint16_t*)scales_f16, (const uint16_t*)w_bf16, ng, K, G,
                       levels, mse);
    return launched("intq quant", N, K);
}

extern "C" s2p_status s2p_int4_pack(void* w_pack, const void* w_i8, int N, int K,
                                    hipStream_t stream) {
    if (!w_pack || !w_i8 || N <= 0 || K <= 0 || (K & 1)) return S2P_ERR_INVALID;
    const int64_t n = (int64_t)N * (K >> 1);
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_pack_nib, dim3((unsigned)blocks), dim3(256), 0, stream,
                       (uint8_t*)w_pack, (const int8_t*)w_i8, n);
    return launched("int4 pack", N, K);
}

extern "C" s2p_status s2p_int8_dequant(void* w_bf16, const void* w_i8, const float* scales, int N,
                                       int K, hipStream_t stream) {
    if (!w_bf16 || !w_i8 || !scales || N <= 0 || K <= 0) return S2P_ERR_INVALID;
    hipLaunchKernelGGL(k_dequant, dim3(N), dim3(256), 0, stream, (uint16_t*)w_bf16, w_i8,
                       (const void*)scales, K, 0, 0);
    return launched("int8 dequant", N, K);
}

extern "C" s2p_status s2p_intq_dequant(void* w_bf16, const void* w_i8, const void* scales_f16,
                                       int N, int K, int G, hipStream_t stream) {
    const int gs = gshift_of(G);
    if (!w_bf16 || !w_i8 || !scales_f16 || N <= 0 || K <= 0 || gs < 0 || K % G != 0)
        return S2P_ERR_INVALID;
    hipLaunchKernelGGL(k_dequant, dim3(N), dim3(256), 0, stream, (uint16_t*)w_bf16, w_i8,
                       scales_f16, K, gs, 1);
    return launched("intq dequant", N, K);
}

extern "C" s2p_status s2p_int4p_dequant(void* w_bf16, const void* w_pack, const void* scales_f16,
                                        int N, int K, int G, hipStream_t stream) {
    const int gs = gshift_of(G);
    if (!w_bf16 || !w_pack || !scales_f16 || N <= 0 || K <= 0 || (K & 1) || gs < 0 || K % G != 0)
        return S2P_ERR_INVALID;
    hipLaunchKernelGGL(k_dequant, dim3(N), dim3(256), 0, stream, (uint16_t*)w_bf16, w_pack,
                       scales_f16, K, gs, 2);
    return launched("int4p dequant", N, K);
}
