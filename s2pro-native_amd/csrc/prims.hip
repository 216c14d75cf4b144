/* s2pro MI355X — transformer primitives on the verify path.
 *
 * Contract launchers of the reference include/s2pro/kernels.h and
 * src/slowar/slowar_kernels.h (rms_norm, qk_norm, rope, rope_pos, kv_append,
 * kv_append_ptrs, qkv_split, silu_mul, add) plus the fused per-layer kernels
 * the verify forward uses (qk-norm + RoPE + KV append in one launch, residual
 * stream init).  Rounding points follow the reference (kernels.cu:4-17):
 *  - RMSNorm / qk-norm: fp32 sum of squares with the reference's reduction
 *    tree, inverse RMS = 1/sqrt(mean + eps) (two correctly rounded ops; the
 *    reference's rsqrtf is approximate), y = bf16((x * inv) * w);
 *  - RoPE: interleaved pairs, inv_freq = 1/powf(base, 2i/d), cos/sin of the
 *    fp32 angle rounded through bf16, butterfly with one rounding per op;
 *    pow/cos/sin are evaluated in binary64 and rounded once to float (the
 *    correctly rounded value);
 *  - silu: 1/(1+exp(-g)) with the rule's exp, two bf16 roundings;
 *  - adds in fp32, one rounding.
 */
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <math.h>
#include <stdint.h>

#include "common.h"
#include "prims_dev.h"
#include "prims_internal.h"
#include "s2pro/kernels.h"
#include "s2pro/s2p_fmath.h"
#include "s2pro/slowar_kernels.h"
#include "s2pro/verify.h"
#include "s2pro/draft.h"

#define PR_THREADS 256
#define PR_MAX_GRID 4096

static inline int pr_blocks(int64_t total, int threads) {
    int64_t b = (total + threads - 1) / threads;
    if (b > PR_MAX_GRID) b = PR_MAX_GRID;
    if (b < 1) b = 1;
    return (int)b;
}

/* --------------------------------------------------------------- rms_norm */

__global__ __launch_bounds__(256) void k_rms_norm(const uint16_t* __restrict__ x,
                                                  const uint16_t* __restrict__ w,
                                                  uint16_t* __restrict__ y, int width,
                                                  float eps) {
    __shared__ float red[256];
    const int row = blockIdx.x;
    const size_t base = (size_t)row * width;
    float s = 0.f;
    for (int i = threadIdx.x; i < width; i += 256) {
        const float v = bf2f(x[base + i]);
        s = fmaf(v, v, s);
    }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if (threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
        __syncthreads();
    }
    const float inv = rsqrt_rule(red[0] / (float)width + eps);
    for (int i = threadIdx.x; i < width; i += 256)
        y[base + i] = f2bf(__fmul_rn(__fmul_rn(bf2f(x[base + i]), inv), bf2f(w[i])));
}

extern "C" hipError_t s2pk_rms_norm(const s2p_bf16* x, const s2p_bf16* w, s2p_bf16* y,
                                    int rows, int width, float eps, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_rms_norm, dim3(rows), dim3(256), 0, st, (const uint16_t*)x,
                       (const uint16_t*)w, (uint16_t*)y, width, eps);
    return hipGetLastError();
}

/* ---------------------------------------------------------------- qk_norm */

/* block = (row, head), 128 threads = one element each (head_dim <= 128) */
__global__ __launch_bounds__(128) void k_qk_norm(uint16_t* __restrict__ qk,
                                                 const uint16_t* __restrict__ w,
                                                 int head_dim, float eps) {
    __shared__ float red[128];
    const size_t base = (size_t)blockIdx.x * head_dim;
    float s = 0.f;
    for (int i = threadIdx.x; i < head_dim; i += 128) {
        const float v = bf2f(qk[base + i]);
        s = fmaf(v, v, s);
    }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int off = 64; off > 0; off >>= 1) {
        if (threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
        __syncthreads();
    }
    const float inv = rsqrt_rule(red[0] / (float)head_dim + eps);
    for (int i = threadIdx.x; i < head_dim; i += 128)
        qk[base + i] = f2bf(__fmul_rn(__fmul_rn(bf2f(qk[base + i]), inv), bf2f(w[i])));
}

extern "C" hipError_t s2pk_qk_norm(s2p_bf16* qk, const s2p_bf16* w, int rows, int heads,
                                   int head_dim, float eps, hipStream_t st) {
    if (rows <= 0 || w == NULL) return hipSuccess;
    if (head_dim > 128) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_qk_norm, dim3(rows * heads), dim3(128), 0, st, (uint16_t*)qk,
                       (const uint16_t*)w, head_dim, eps);
    return hipGetLastError();
}

/* ------------------------------------------------------------------- rope */

__global__ __launch_bounds__(256) void k_rope(uint16_t* __restrict__ x, int rows, int heads,
                                              int head_dim, int pos0,
                                              const int32_t* __restrict__ pos_arr,
                                              float base) {
    const int pairs = head_dim / 2;
    const int64_t total = (int64_t)rows * heads * pairs;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int r = (int)(idx / ((int64_t)heads * pairs));
        const int rem = (int)(idx % ((int64_t)heads * pairs));
        const int h = rem / pairs, i = rem % pairs;
        const int p = pos_arr ? pos_arr[r] : pos0 + r;
        float c, s;
        rope_cs(p, i, head_dim, base, &c, &s);
        const size_t o = ((size_t)r * heads + h) * head_dim + 2 * i;
        const float x0 = bf2f(x[o]), x1 = bf2f(x[o + 1]);
        x[o] = f2bf(__fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s)));
        x[o + 1] = f2bf(__fadd_rn(__fmul_rn(x1, c), __fmul_rn(x0, s)));
    }
}

static hipError_t rope_launch(s2p_bf16* q, s2p_bf16* k, int rows, int qh, int kvh, int hd,
                              int pos0, const int32_t* pos, float base, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    const int64_t tq = (int64_t)rows * qh * (hd / 2);
    hipLaunchKernelGGL(k_rope, dim3(pr_blocks(tq, PR_THREADS)), dim3(PR_THREADS), 0, st,
                       (uint16_t*)q, rows, qh, hd, pos0, pos, base);
    const int64_t tk = (int64_t)rows * kvh * (hd / 2);
    hipLaunchKernelGGL(k_rope, dim3(pr_blocks(tk, PR_THREADS)), dim3(PR_THREADS), 0, st,
                       (uint16_t*)k, rows, kvh, hd, pos0, pos, base);
    return hipGetLastError();
}

extern "C" hipError_t s2pk_rope(s2p_bf16* q, s2p_bf16* k, int rows, int q_heads, int kv_heads,
                                int head_dim, int pos, float rope_base, hipStream_t st) {
    return rope_launch(q, k, rows, q_heads, kv_heads, head_dim, pos, NULL, rope_base, st);
}

extern "C" hipError_t s2pk_rope_pos(s2p_bf16* q, s2p_bf16* k, int rows, int q_heads,
                                    int kv_heads, int head_dim, const int32_t* pos,
                                    float rope_base, hipStream_t st) {
    return rope_launch(q, k, rows, q_heads, kv_heads, head_dim, 0, pos, rope_base, st);
}

/* -------------------------------------------------------------- kv append */

__global__ __launch_bounds__(256) void k_kv_append(const uint16_t* __restrict__ k,
                                                   const uint16_t* __restrict__ v,
                                                   uint16_t* kc0, uint16_t* vc0,
                                                   uint16_t* const* kcs, uint16_t* const* vcs,
                                                   int rows, int kv_heads, int head_dim,
                                                   int pos0, const int32_t* pos_arr,
                                                   int max_seq) {
    /* one thread per 8 elements (16 bytes) */
    const int per_row = kv_heads * head_dim / 8;
    const int64_t total = (int64_t)rows * per_row;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int r = (int)(idx / per_row);
        const int e = (int)(idx % per_row) * 8;
        const int h = e / head_dim, d = e % head_dim;
        const int p = pos_arr ? pos_arr[r] : pos0 + r;
        if (p < 0 || p >= max_seq) continue; /* out-of-range position: nothing written */
        uint16_t* kc = kcs ? kcs[r] : kc0;
        uint16_t* vc = vcs ? vcs[r] : vc0;
        const size_t src = (size_t)r * kv_heads * head_dim + e;
        const size_t dst = ((size_t)h * max_seq + p) * head_dim + d;
        *(s2p_u32x4*)(kc + dst) = *(const s2p_u32x4*)(k + src);
        *(s2p_u32x4*)(vc + dst) = *(const s2p_u32x4*)(v + src);
    }
}

extern "C" hipError_t s2pk_kv_append(const s2p_bf16* k, const s2p_bf16* v, s2p_bf16* k_cache,
                                     s2p_bf16* v_cache, int rows, int kv_heads, int head_dim,
                                     int pos, int max_seq, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (head_dim % 8) return hipErrorInvalidValue;
    const int64_t total = (int64_t)rows * kv_heads * head_dim / 8;
    hipLaunchKernelGGL(k_kv_append, dim3(pr_blocks(total, PR_THREADS)), dim3(PR_THREADS), 0, st,
                       (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)k_cache,
                       (uint16_t*)v_cache, (uint16_t* const*)NULL, (uint16_t* const*)NULL, rows,
                       kv_heads, head_dim, pos, (const int32_t*)NULL, max_seq);
    return hipGetLastError();
}

extern "C" hipError_t s2pk_kv_append_ptrs(const s2p_bf16* k, const s2p_bf16* v,
                                          s2p_bf16* const* k_caches, s2p_bf16* const* v_caches,
                                          int rows, int kv_heads, int head_dim,
                                          const int32_t* pos, int max_seq, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (head_dim % 8) return hipErrorInvalidValue;
    const int64_t total = (int64_t)rows * kv_heads * head_dim / 8;
    hipLaunchKernelGGL(k_kv_append, dim3(pr_blocks(total, PR_THREADS)), dim3(PR_THREADS), 0, st,
                       (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)NULL, (uint16_t*)NULL,
                       (uint16_t* const*)k_caches, (uint16_t* const*)v_caches, rows, kv_heads,
                       head_dim, 0, pos, max_seq);
    return hipGetLastError();
}

/* -------------------------------------------------------------- qkv split */

__global__ __launch_bounds__(256) void k_qkv_split(const uint16_t* __restrict__ qkv,
                                                   uint16_t* __restrict__ q,
                                                   uint16_t* __restrict__ k,
                                                   uint16_t* __restrict__ v, int64_t total,
                                                   int qw, int kvw) {
    const int w = qw + 2 * kvw;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = idx / w;
        const int c = (int)(idx % w);
        const uint16_t val = qkv[idx];
        if (c < qw) q[r * qw + c] = val;
        else if (c < qw + kvw) k[r * kvw + (c - qw)] = val;
        else v[r * kvw + (c - qw - kvw)] = val;
    }
}

extern "C" hipError_t s2pk_qkv_split(const s2p_bf16* qkv, s2p_bf16* q, s2p_bf16* k,
                                     s2p_bf16* v, int rows, int q_width, int kv_width,
                                     hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    const int64_t total = (int64_t)rows * (q_width + 2 * kv_width);
    hipLaunchKernelGGL(k_qkv_split, dim3(pr_blocks(total, PR_THREADS)), dim3(PR_THREADS), 0, st,
                       (const uint16_t*)qkv, (uint16_t*)q, (uint16_t*)k, (uint16_t*)v, total,
                       q_width, kv_width);
    return hipGetLastError();
}

/* ------------------------------------------------------------- silu / add */

__global__ __launch_bounds__(256) void k_silu_mul(const uint16_t* __restrict__ gu,
                                                  uint16_t* __restrict__ h, int64_t total,
                                                  int ffn) {
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = idx / ffn;
        const int c = (int)(idx % ffn);
        const float g = bf2f(gu[(size_t)r * 2 * ffn + c]);
        const float u = bf2f(gu[(size_t)r * 2 * ffn + ffn + c]);
        const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, s2p_expf(-g)));
        const float sil = bf2f(f2bf(__fmul_rn(g, sig)));
        h[idx] = f2bf(__fmul_rn(sil, u));
    }
}

extern "C" hipError_t s2pk_silu_mul(const s2p_bf16* gu, s2p_bf16* h, int rows, int ffn,
                                    hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    const int64_t total = (int64_t)rows * ffn;
    hipLaunchKernelGGL(k_silu_mul, dim3(pr_blocks(total, PR_THREADS)), dim3(PR_THREADS), 0, st,
                       (const uint16_t*)gu, (uint16_t*)h, total, ffn);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_add(uint16_t* __restrict__ y,
                                             const uint16_t* __restrict__ x, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        y[i] = f2bf(__fadd_rn(bf2f(y[i]), bf2f(x[i])));
}

extern "C" hipError_t s2pk_add(s2p_bf16* y, const s2p_bf16* x, int64_t n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_add, dim3(pr_blocks(n, PR_THREADS)), dim3(PR_THREADS), 0, st,
                       (uint16_t*)y, (const uint16_t*)x, n);
    return hipGetLastError();
}

/* logits bf16 [vocab] -> f32 scratch [vocab] (exact widening): the device
 * staging step of the reference sampler contract (kernels.cu:1300-1322).
 * Eight logits per thread: one 16-byte load, two 16-byte stores, when both
 * pointers are 16-byte aligned; element by element otherwise. */
__global__ __launch_bounds__(256) void k_widen(const uint16_t* __restrict__ x,
                                               float* __restrict__ y, int64_t n, int vec) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vec) {
        const int64_t n8 = n >> 3;
        for (int64_t j = i; j < n8; j += stride) {
            const s2p_u32x4 v = *(const s2p_u32x4*)(x + j * 8);
            s2p_f32x4 lo = {bf2f_lo(v.x), bf2f_hi(v.x), bf2f_lo(v.y), bf2f_hi(v.y)};
            s2p_f32x4 hi = {bf2f_lo(v.z), bf2f_hi(v.z), bf2f_lo(v.w), bf2f_hi(v.w)};
            *(s2p_f32x4*)(y + j * 8) = lo;
            *(s2p_f32x4*)(y + j * 8 + 4) = hi;
        }
        i += n8 * 8;
        for (; i < n; i += stride) y[i] = bf2f(x[i]);
        return;
    }
    for (; i < n; i += stride) y[i] = bf2f(x[i]);
}

extern "C" hipError_t s2pk_sample_prepare(const s2p_bf16* logits, float* scratch, int vocab,
                                          hipStream_t st) {
    if (vocab <= 0) return hipSuccess;
    const int vec = ((((uintptr_t)logits) | ((uintptr_t)scratch)) & 15) == 0;
    const int64_t work = vec ? ((int64_t)vocab + 7) / 8 : vocab;
    hipLaunchKernelGGL(k_widen, dim3(pr_blocks(work, PR_THREADS)), dim3(PR_THREADS), 0, st,
                       (const uint16_t*)logits, scratch, (int64_t)vocab, vec);
    return hipGetLastError();
}

/* ----------------------------------------------- fused verify-layer kernels */

/* One wave per (row, head), heads 0..q_heads-1 are query heads, then the
 * kv heads.  Per-head RMSNorm (reference tree order: lane i holds elements
 * i and i+64, exactly the first level of the 128-thread tree), RoPE at the
 * row's position, query -> q_out, key/value -> the row's cache slot.
 * Cache planes of layer l of a session: base + l * layer_stride, k head h at
 * plane h, v head h at plane kv_heads + h, each [max_seq][128]. */
__global__ __launch_bounds__(64) void k_qkrope_append(const uint16_t* __restrict__ qkv,
                                                      uint16_t* __restrict__ q_out,
                                                      const uint16_t* __restrict__ qn_w,
                                                      const uint16_t* __restrict__ kn_w,
                                                      S2pRowPlan plan, int layer, float eps,
                                                      float base) {
    qkrope_item(qkv, q_out, qn_w, kn_w, plan, layer, eps, base, blockIdx.x, blockIdx.y,
                threadIdx.x);
}

/* the same with (cos, sin) from the plan's RoPE table (bit-identical: the
 * table holds rope_cs of the rows' positions), four (row, head) items a
 * block */
__global__ __launch_bounds__(256) void k_qkrope_append_tab(const uint16_t* qkv,
                                                           uint16_t* __restrict__ q_out,
                                                           const uint16_t* __restrict__ qn_w,
                                                           const uint16_t* __restrict__ kn_w,
                                                           S2pRowPlan plan, int layer, float eps,
                                                           const float* __restrict__ rope_tab,
                                                           S2pQkvParts parts) {
    qkrope_item_t<true>(qkv, q_out, qn_w, kn_w, plan, layer, eps, 0.f, blockIdx.x,
                        blockIdx.y * 4 + (threadIdx.x >> 6), threadIdx.x & 63, rope_tab, parts);
}

extern "C" hipError_t s2p_qkrope_append_tab_launch(const void* qkv, void* q_out, const void* qn_w,
                                                   const void* kn_w, const S2pRowPlan* plan,
                                                   int rows, int layer, float eps,
                                                   const float* rope_tab, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (!rope_tab) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_qkrope_append_tab, dim3(rows, 10), dim3(256), 0, st,
                       (const uint16_t*)qkv, (uint16_t*)q_out, (const uint16_t*)qn_w,
                       (const uint16_t*)kn_w, *plan, layer, eps, rope_tab,
                       S2pQkvParts{nullptr, 0, 0, 0});
    return hipGetLastError();
}

extern "C" hipError_t s2p_qkrope_append_tab_parts_launch(void* qkv, const S2pQkvParts* parts,
                                                         void* q_out, const void* qn_w,
                                                         const void* kn_w, const S2pRowPlan* plan,
                                                         int rows, int layer, float eps,
                                                         const float* rope_tab, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (!rope_tab || !parts || (parts->splits > 0 && (!parts->part || parts->M < rows)))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_qkrope_append_tab, dim3(rows, 10), dim3(256), 0, st,
                       (const uint16_t*)qkv, (uint16_t*)q_out, (const uint16_t*)qn_w,
                       (const uint16_t*)kn_w, *plan, layer, eps, rope_tab, *parts);
    return hipGetLastError();
}

extern "C" hipError_t s2p_qkrope_append_launch(const void* qkv, void* q_out, const void* qn_w,
                                               const void* kn_w, const S2pRowPlan* plan,
                                               int rows, int layer, float eps, float base,
                                               hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_qkrope_append, dim3(rows, 40), dim3(64), 0, st, (const uint16_t*)qkv,
                       (uint16_t*)q_out, (const uint16_t*)qn_w, (const uint16_t*)kn_w, *plan,
                       layer, eps, base);
    return hipGetLastError();
}

/* Residual stream init: x = x_in and per-16-column sums of squares of x
 * (layout [N/16][GEMV_MAX_M]) for the first RMSNorm. */
__global__ __launch_bounds__(64) void k_resid_init(const uint16_t* __restrict__ xin,
                                                   uint16_t* __restrict__ x,
                                                   float* __restrict__ ssq, int width) {
    resid_init_item(xin, x, ssq, width, blockIdx.x, blockIdx.y, threadIdx.x);
}

extern "C" hipError_t s2p_resid_init_launch(const void* xin, void* x, float* ssq, int rows,
                                            int width, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (width % 64) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_resid_init, dim3(width / 64, rows), dim3(64), 0, st,
                       (const uint16_t*)xin, (uint16_t*)x, ssq, width);
    return hipGetLastError();
}

/* RoPE table of a verify plan: (cos, sin) of every row's position and pair,
 * the rule's values (rope_cs), computed once per plan. */
__global__ __launch_bounds__(64) void k_rope_tab(S2pRowPlan plan, float base,
                                                 float* __restrict__ tab) {
    rope_tab_item(plan, base, tab, blockIdx.x, threadIdx.x);
}

extern "C" hipError_t s2p_rope_tab_launch(const S2pRowPlan* plan, int rows, float base,
                                          float* tab, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope_tab, dim3((unsigned)rows), dim3(64), 0, st, *plan, base, tab);
    return hipGetLastError();
}

/* Embedding gather, out[r] = table[ids[r]] (reference kernels.h:58-60): one
 * 64-lane block per (row, 8-column group of 64 lanes), 16-byte copies. */
__global__ __launch_bounds__(64) void k_embed(const uint16_t* __restrict__ table,
                                              const int64_t* __restrict__ ids,
                                              uint16_t* __restrict__ out, int dim) {
    const int r = blockIdx.y, c = (blockIdx.x * 64 + threadIdx.x) * 8;
    if (c >= dim) return;
    const s2p_u32x4 v = *(const s2p_u32x4*)(table + (size_t)ids[r] * dim + c);
    *(s2p_u32x4*)(out + (size_t)r * dim + c) = v;
}

extern "C" hipError_t s2pk_embed(const s2p_bf16* table, const int64_t* ids, s2p_bf16* out,
                                 int rows, int dim, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (!table || !ids || !out || dim <= 0 || dim % 8) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_embed, dim3((unsigned)((dim / 8 + 63) / 64), (unsigned)rows), dim3(64), 0,
                       st, (const uint16_t*)table, ids, (uint16_t*)out, dim);
    return hipGetLastError();
}

/* argmax of each row (reference kernels.h:68-70, kernels.cu:1326-1357): the
 * largest value, the lowest index among equal values; NaN never wins.  One
 * 256-thread block per row: each lane keeps its best (value, index) over a
 * strided walk, then a wave reduction and one across the four waves. */
S2P_DEV bool am_better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

__global__ __launch_bounds__(256) void k_argmax(const uint16_t* __restrict__ logits,
                                                int32_t* __restrict__ ids, int vocab) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int r = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint16_t* row = logits + (size_t)r * vocab;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = t; i < vocab; i += 256) {
        const float v = bf2f(row[i]);
        if (am_better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (am_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < 4; w++)
            if (am_better(sv[w], si[w], bv, bi)) {
                bv = sv[w];
                bi = si[w];
            }
        ids[r] = bi == 0x7FFFFFFF ? 0 : bi; /* an all-NaN row: index 0 */
    }
}

extern "C" hipError_t s2pk_argmax(const s2p_bf16* logits, int32_t* ids, int rows, int vocab,
                                  hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (!logits || !ids || vocab <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_argmax, dim3((unsigned)rows), dim3(256), 0, st, (const uint16_t*)logits,
                       ids, vocab);
    return hipGetLastError();
}

/* Fast-AR step input: x[r] = table[clamp(ids[r], 0, n_ids - 1)] and the
 * sums of squares of its 16-column blocks for the next RMSNorm (the
 * residual-init arithmetic of resid_init_item). */
__global__ __launch_bounds__(64) void k_fa_embed_ssq(const uint16_t* __restrict__ table,
                                                     const int32_t* __restrict__ ids, int n_ids,
                                                     uint16_t* __restrict__ x,
                                                     float* __restrict__ ssq, int width) {
    const int m = blockIdx.y, blk = blockIdx.x, lane = threadIdx.x;
    int id = ids[m];
    id = id < 0 ? 0 : (id >= n_ids ? n_ids - 1 : id);
    const int c = blk * 64 + lane;
    const uint16_t v = table[(size_t)id * width + c];
    coh_st16(x + (size_t)m * width + c, v);
    const float f = bf2f(v);
    const float t = sum_lanes16(f * f);
    if ((lane & 15) == 0) coh_stf(ssq + (size_t)(blk * 4 + (lane >> 4)) * 128 + m, t);
}

extern "C" hipError_t s2p_fa_embed_ssq_launch(const void* table, const int32_t* ids, int n_ids,
                                              void* x, float* ssq, int rows, int width,
                                              hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (width % 64) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_fa_embed_ssq, dim3(width / 64, rows), dim3(64), 0, st,
                       (const uint16_t*)table, ids, n_ids, (uint16_t*)x, ssq, width);
    return hipGetLastError();
}

/* The 10-codebook VQ embedding of frame t added onto rows[t] (reference
 * fastar.h:46-52): codes [10][T] codebook-major, clamped to 0..4095; the ten
 * rows of table [10 * 4096][dim] summed in f32 in codebook order, rounded to
 * bf16 once, then added to the row with one bf16 rounding. */
__global__ __launch_bounds__(256) void k_vq_embed_add(const uint16_t* __restrict__ table,
                                                      const int32_t* __restrict__ codes, int T,
                                                      uint16_t* __restrict__ rows, int dim) {
    const int t = blockIdx.x;
    int idx[10];
#pragma unroll
    for (int cb = 0; cb < 10; cb++) {
        int c = codes[(size_t)cb * T + t];
        c = c < 0 ? 0 : (c > 4095 ? 4095 : c);
        idx[cb] = cb * 4096 + c;
    }
    for (int d = threadIdx.x; d < dim; d += 256) {
        float acc = 0.f;
#pragma unroll
        for (int cb = 0; cb < 10; cb++) acc += bf2f(table[(size_t)idx[cb] * dim + d]);
        uint16_t* y = rows + (size_t)t * dim + d;
        *y = f2bf(__fadd_rn(bf2f(*y), bf2f(f2bf(acc))));
    }
}

extern "C" hipError_t s2p_fa_vq_embed_add_launch(const void* table, const int32_t* codes, int T,
                                                 void* rows, int dim, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_vq_embed_add, dim3((unsigned)T), dim3(256), 0, st, (const uint16_t*)table,
                       codes, T, (uint16_t*)rows, dim);
    return hipGetLastError();
}

/* Draft step prologue (one block): the one-row attention plan of the step at
 * position pos over the draft's KV (the backbone's [16][max_seq][128]
 * layout, one layer), its RoPE row, and zeros for the residual row x (the
 * fuse GEMV adds onto it, producing the row's sums of squares) and the
 * attention's split counters. */
__global__ __launch_bounds__(256) void k_draft_prologue(S2pRowPlan plan, S2pAttnSeg* seg,
                                                        void* kv, int pos,
                                                        const int32_t* __restrict__ pos_dev,
                                                        int pos_max, float base,
                                                        float* __restrict__ tab,
                                                        uint16_t* __restrict__ x, int nx,
                                                        unsigned* __restrict__ ctr, int nctr) {
    const int t = threadIdx.x;
    if (pos_dev) {
        /* position pos_dev[0] + pos, kept inside [0, pos_max) so the append
         * never leaves the cache */
        pos += *pos_dev;
        pos = pos < 0 ? 0 : (pos >= pos_max ? pos_max - 1 : pos);
    }
    if (t == 0) {
        *(int32_t*)plan.pos = pos;
        *(int32_t*)plan.slot = pos;
        *(int32_t*)plan.sess = 0;
        *(uint64_t*)plan.vis = 1ull; /* the row sees its own slot */
        *(void**)plan.kv = kv;
        S2pAttnSeg g;
        g.sess = 0;
        g.L = pos;
        g.row0 = 0;
        g.nrows = 1;
        g.span = pos + 1;
        g.first = 0;
        g.kv = kv;
        *seg = g;
    }
    for (int i = t; i < nx; i += 256) x[i] = 0;
    for (int i = t; i < nctr; i += 256) ctr[i] = 0u;
    __syncthreads();
    if (t < 64) rope_tab_item(plan, base, tab, 0, t);
}

extern "C" hipError_t s2p_draft_prologue_launch(const S2pRowPlan* plan, S2pAttnSeg* seg, void* kv,
                                               int pos, const int32_t* pos_dev, int pos_max,
                                               float base, float* tab, void* x, int nx,
                                               unsigned* ctr, int nctr, hipStream_t st) {
    hipLaunchKernelGGL(k_draft_prologue, dim3(1), dim3(256), 0, st, *plan, seg, kv, pos, pos_dev,
                       pos_max, base, tab, (uint16_t*)x, nx, ctr, nctr);
    return hipGetLastError();
}

/* Tree commit: session s, layer l, plane h (16 = 8 K + 8 V heads).  Accepted
 * node path[d-1] (index >= d) moves to slot L + d in increasing d, so no
 * source is overwritten before it is read. */
__global__ __launch_bounds__(64) void k_kv_commit(S2pRowPlan plan, const int32_t* __restrict__ path,
                                                  const int32_t* __restrict__ n_acc, int R) {
    const int s = blockIdx.x, layer = blockIdx.y, plane = blockIdx.z, lane = threadIdx.x;
    int n = n_acc[s];
    n = n < 0 ? 0 : (n > R - 1 ? R - 1 : n);
    const int L = plan.slot[s * R];
    uint16_t* base = (uint16_t*)plan.kv[s] + (size_t)layer * plan.layer_stride +
                     (size_t)plane * plan.max_seq * 128;
    for (int d = 1; d <= n; d++) {
        const int node = path[(size_t)s * R + d - 1];
        if (node == d || node < d || node >= R) continue; /* chain slot, or invalid */
        const uint32_t* src = (const uint32_t*)(base + (size_t)(L + node) * 128);
        uint32_t* dst = (uint32_t*)(base + (size_t)(L + d) * 128);
        dst[lane] = src[lane];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

extern "C" hipError_t s2p_kv_commit_launch(const S2pRowPlan* plan, const int32_t* path,
                                           const int32_t* n_acc, int n_sess, int R, int n_layers,
                                           hipStream_t st) {
    if (n_sess <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_kv_commit, dim3(n_sess, n_layers, 16), dim3(64), 0, st, *plan, path,
                       n_acc, R);
    return hipGetLastError();
}

/* Test hook: the device float -> bf16 conversion every kernel uses, over n
 * values (pinned against the rule by a GPU test). */
__global__ void k_f2bf(const float* __restrict__ in, uint16_t* __restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f2bf(in[i]);
}

/* Test hook: sizes of the internal launch descriptors that tests build
 * through ctypes (0 S2pRowPlan, 1 S2pAttnSeg, then the public structs the
 * Python binding mirrors), so that a stale mirror fails
 * on the CPU instead of handing a kernel a misread descriptor. */
extern "C" size_t s2p_test_desc_bytes(int which) {
    switch (which) {
        case 0: return sizeof(S2pRowPlan);
        case 1: return sizeof(S2pAttnSeg);
        case 2: return sizeof(s2p_backbone_opts);
        case 3: return sizeof(s2p_verify_batch);
        case 4: return sizeof(s2p_verify_step_io);
        case 5: return sizeof(s2p_tensor);
        case 6: return sizeof(s2p_linear);
        case 7: return sizeof(s2p_slow_layer);
        case 8: return sizeof(s2p_draft_model);
        case 9: return sizeof(s2p_draft_state);
        default: return 0;
    }
}

extern "C" hipError_t s2p_test_f2bf(const float* in, uint16_t* out, int64_t n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_f2bf, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, in, out, n);
    return hipGetLastError();
}

/* ---- the chain condition of speculative frames ----
 * prep: for every drafted node (session s, node i >= 1; b = s (R - 1) + i - 1)
 * the final-normed hidden of its parent's row and the node's semantic code
 * (vocab id - the semantic base, 0 for EOS and anything outside the 4,096
 * codes), the fast-AR's inputs; one block per node */
__global__ __launch_bounds__(64) void k_chain_prep(const int32_t* __restrict__ parent,
                                                   const int64_t* __restrict__ tok,
                                                   const uint16_t* __restrict__ hidden,
                                                   uint16_t* __restrict__ par_hidden,
                                                   int32_t* __restrict__ sem, int R, int dim) {
    const int b = blockIdx.x, s = b / (R - 1), i = b - s * (R - 1) + 1;
    const int src = s * R + parent[i];
    for (int c = threadIdx.x * 8; c < dim; c += 64 * 8)
        *(s2p_u32x4*)(par_hidden + (size_t)b * dim + c) = *(const s2p_u32x4*)(hidden + (size_t)src * dim + c);
    if (threadIdx.x == 0) {
        const int64_t t = tok[(size_t)s * R + i] - S2P_TOK_SEMANTIC_START;
        sem[b] = (t >= 0 && t < 4096) ? (int32_t)t : 0;
    }
}

/* check: chain_ok[row] = 1 for roots and EOS nodes, else whether the node's
 * nine fast-AR codes (stage [9][B]) equal the drafted ones; the codes to
 * codes_out [row][9] (zeros for roots) */
__global__ __launch_bounds__(64) void k_chain_check(const int32_t* __restrict__ stage,
                                                    const int32_t* __restrict__ draft_codes,
                                                    const int64_t* __restrict__ tok,
                                                    uint8_t* __restrict__ chain_ok,
                                                    int32_t* __restrict__ codes_out, int n_sess,
                                                    int R) {
    const int row = blockIdx.x * 64 + threadIdx.x;
    if (row >= n_sess * R) return;
    const int s = row / R, i = row - s * R, B = n_sess * (R - 1);
    if (i == 0) {
        chain_ok[row] = 1;
        for (int c = 0; c < 9; c++) codes_out[(size_t)row * 9 + c] = 0;
        return;
    }
    const int b = s * (R - 1) + i - 1;
    bool same = true;
    for (int c = 0; c < 9; c++) {
        const int32_t v = stage[(size_t)c * B + b];
        codes_out[(size_t)row * 9 + c] = v;
        same = same && v == draft_codes[(size_t)row * 9 + c];
    }
    chain_ok[row] = (same || tok[row] == S2P_TOK_EOS) ? 1 : 0;
}

extern "C" hipError_t s2p_chain_prep_launch(const int32_t* parent, const int64_t* tok, const void* hidden,
                                            void* par_hidden, int32_t* sem, int n_sess, int R, int dim,
                                            hipStream_t st) {
    if (n_sess < 1 || R < 2 || dim % 8) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_chain_prep, dim3((unsigned)(n_sess * (R - 1))), dim3(64), 0, st, parent, tok,
                       (const uint16_t*)hidden, (uint16_t*)par_hidden, sem, R, dim);
    return hipGetLastError();
}

extern "C" hipError_t s2p_chain_check_launch(const int32_t* stage, const int32_t* draft_codes,
                                             const int64_t* tok, uint8_t* chain_ok, int32_t* codes_out,
                                             int n_sess, int R, hipStream_t st) {
    if (n_sess < 1 || R < 2) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_chain_check, dim3((unsigned)((n_sess * R + 63) / 64)), dim3(64), 0, st, stage,
                       draft_codes, tok, chain_ok, codes_out, n_sess, R);
    return hipGetLastError();
}

/* The persistent forward's error word (word == NULL: a forward with no
 * bounded waits, reported as 0) copied out, and cleared when asked: one
 * thread, so it is capturable and needs no memset node. */
__global__ void k_word_status(int* __restrict__ word, int32_t* __restrict__ out, int clear) {
    const int v = word ? *(volatile int*)word : 0;
    *out = v;
    if (clear && v) *(volatile int*)word = 0;
}

extern "C" hipError_t s2p_word_status_launch(int* word, int32_t* out, int clear, hipStream_t st) {
    if (!out) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_word_status, dim3(1), dim3(1), 0, st, word, out, clear);
    return hipGetLastError();
}
