/* s2pro MI355X — INT8 / INT4 KV cache: quantise-on-append and attention
 * over the quantised cache (reference kernels.cu:510-946, launchers
 * slowar_kernels.h:84-120).
 *
 * Cache layout (the reference's, so sessions and prefix caches are
 * interchangeable): payload [kv_heads][max_seq][bw == 8 ? 128 : 64] bytes,
 * scales f16 [kv_heads][max_seq][4], one per 32-element group.
 *
 * Append: one workgroup per (row, kv head), thread d = element d; the group
 * absmax is a max over the 32 lanes of a half wave (exact in any order); the
 * scale is f16(absmax / QMAX) and the values rint(x / scale) clamped to
 * +-QMAX, with IEEE division, as the reference (kernels.cu:541-579).
 *
 * Attention: one workgroup of 128 threads per (row, query head) and 128-slot
 * tiles, in the reference's arithmetic order (kernels.cu:614-722), so the
 * result equals the oracle restatement bit for bit: per slot the score is
 * sum_g fma(pp_g, ks_g) of in-order group dots; the tile max and sum follow
 * the 128-lane trees (the sum's first level through LDS, the rest as the
 * shuffle-down tree); V enters as (p * vs_g) * v.  Exponentials are the
 * rule's s2p_expf.  The decode variant gives each 128-slot tile its own
 * workgroup (a split), writes the (m, l, O) partial and merges the splits
 * with the bf16 path's combine.
 *
 * bw 4 decodes both nibbles as the two's complement the append writes (the
 * reference's decode expression sign-extends only the high nibble). */
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "common.h"
#include "s2pro/s2p_fmath.h"
#include "s2pro/slowar_kernels.h"

#define KV8_HD 128
#define KV8_TILE 128

static __device__ __forceinline__ float kv8_val(const int8_t* row, int e, int bw) {
    if (bw == 8) return (float)row[e];
    const uint8_t b = (uint8_t)row[e >> 1];
    const int nib = (e & 1) ? (b >> 4) : (b & 0xF);
    return (float)(nib >= 8 ? nib - 16 : nib);
}

/* max over the 32 lanes of a half wave (the lanes of one 32-element group) */
static __device__ __forceinline__ float max32(float v) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

template <int BW>
__global__ __launch_bounds__(KV8_HD) void k_kv_append8(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int8_t* kc0, int8_t* vc0,
    uint16_t* ks0, uint16_t* vs0, int8_t* const* kcs, int8_t* const* vcs, uint16_t* const* kss,
    uint16_t* const* vss, int kv_heads, int pos0, const int32_t* pos_arr, int max_seq) {
#pragma clang fp contract(off)
    constexpr int QMAX = BW == 8 ? 127 : 7;
    constexpr int EL = BW == 8 ? KV8_HD : KV8_HD / 2;
    const int r = blockIdx.x / kv_heads, h = blockIdx.x % kv_heads;
    const int d = threadIdx.x;
    const int p = pos_arr ? pos_arr[r] : pos0 + r;
    if (p < 0 || p >= max_seq) return; /* never written outside the cache */
    for (int kv = 0; kv < 2; kv++) {
        int8_t* pay = kv ? (vcs ? vcs[r] : vc0) : (kcs ? kcs[r] : kc0);
        uint16_t* sc = kv ? (vss ? vss[r] : vs0) : (kss ? kss[r] : ks0);
        const float x = bf2f((kv ? v : k)[((size_t)r * kv_heads + h) * KV8_HD + d]);
        const float a = max32(fabsf(x));
        const uint16_t hs = f2h(__fdiv_rn(a, (float)QMAX));
        const float s = h2f(hs);
        int q = s > 0.f ? (int)rintf(__fdiv_rn(x, s)) : 0;
        q = max(-QMAX, min(QMAX, q));
        const size_t row = (size_t)h * max_seq + p;
        if (BW == 8) {
            pay[row * EL + d] = (int8_t)q;
        } else {
            const int hi = __shfl_down(q, 1, 64);
            if ((d & 1) == 0) pay[row * EL + (d >> 1)] = (int8_t)((q & 0xF) | ((hi & 0xF) << 4));
        }
        if ((d & 31) == 0) sc[row * 4 + (d >> 5)] = hs;
    }
}

/* Scores, max, exponentials and sum of one 128-slot tile [t0, t0 + 128) of
 * a row attending slots [0, len); sp[] (LDS) gets the tile's p.  Returns the
 * tile's sum (all threads) and updates m (all threads). */
struct Kv8Lds {
    float sq[KV8_HD];
    float sp[KV8_TILE];
    float red[KV8_TILE];
    float bc[2];
};

template <int BW>
static __device__ __forceinline__ float kv8_tile(const int8_t* kb, const uint16_t* ksb, int t0,
                                                 int len, float& m, float& corr, Kv8Lds& L,
                                                 bool split) {
#pragma clang fp contract(off)
    constexpr int EL = BW == 8 ? KV8_HD : KV8_HD / 2;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int j = t0 + t;
    float s = -INFINITY;
    if (j < len) {
        const int8_t* kr = kb + (size_t)j * EL;
        float dsum = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            float pp = 0.f;
#pragma unroll 8
            for (int e = 0; e < 32; e++) pp = fmaf(L.sq[g * 32 + e], kv8_val(kr, g * 32 + e, BW), pp);
            dsum = fmaf(pp, h2f(ksb[(size_t)j * 4 + g]), dsum);
        }
        s = dsum;
    }
    /* tile max: exact in any order */
    float mx = s;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (lane == 0) L.bc[wave] = mx;
    __syncthreads();
    const float tmax = fmaxf(L.bc[0], L.bc[1]);
    const float m_new = split ? tmax : fmaxf(m, tmax);
    corr = (m == -INFINITY) ? 0.f : s2p_expf(m - m_new);
    const float p = (s == -INFINITY) ? 0.f : s2p_expf(s - m_new);
    L.sp[t] = p;
    L.red[t] = p;
    __syncthreads();
    /* the 128-lane tree: red[t] += red[t + 64], then the shuffle-down tree
     * over the first 64 (lane 0 holds the total) */
    float tot = 0.f;
    if (wave == 0) {
        tot = wave_sum_down(L.red[t] + L.red[t + 64]);
        if (lane == 0) L.bc[0] = tot;
    }
    __syncthreads();
    tot = L.bc[0];
    m = m_new;
    return tot;
}

template <int BW>
__global__ __launch_bounds__(KV8_TILE) void k_attention8(
    const uint16_t* __restrict__ q, const int8_t* kc, const int8_t* vc, const uint16_t* ks,
    const uint16_t* vs, uint16_t* out, int q_heads, int kv_heads, int pos0, int max_seq) {
#pragma clang fp contract(off)
    constexpr int EL = BW == 8 ? KV8_HD : KV8_HD / 2;
    __shared__ Kv8Lds L;
    const int row = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    const int len = pos0 + row + 1;
    const int kvh = h / (q_heads / kv_heads);
    const int8_t* kb = kc + (size_t)kvh * max_seq * EL;
    const int8_t* vb = vc + (size_t)kvh * max_seq * EL;
    const uint16_t* ksb = ks + (size_t)kvh * max_seq * 4;
    const uint16_t* vsb = vs + (size_t)kvh * max_seq * 4;
    L.sq[t] = bf2f(q[((size_t)row * q_heads + h) * KV8_HD + t]) * 0.08838834764831845f;
    __syncthreads();
    float m = -INFINITY, l = 0.f, acc = 0.f;
    for (int t0 = 0; t0 < len; t0 += KV8_TILE) {
        float corr;
        const float tsum = kv8_tile<BW>(kb, ksb, t0, len, m, corr, L, false);
        l = fmaf(l, corr, tsum);
        const int lim = min(KV8_TILE, len - t0);
        float a = acc * corr;
        for (int j2 = 0; j2 < lim; j2++) {
            const size_t j = (size_t)(t0 + j2);
            a = fmaf(L.sp[j2] * h2f(vsb[j * 4 + (t >> 5)]), kv8_val(vb + j * EL, t, BW), a);
        }
        acc = a;
        __syncthreads(); /* sp / red are rewritten by the next tile */
    }
    out[((size_t)row * q_heads + h) * KV8_HD + t] = f2bf(__fdiv_rn(acc, l));
}

/* one 128-slot split of a decode row: (m, l, O) partial in the bf16 path's
 * layout (m, l pairs, then the O rows) */
template <int BW>
__global__ __launch_bounds__(KV8_TILE) void k_attention8_split(
    const uint16_t* __restrict__ q, const int8_t* const* kcs, const int8_t* const* vcs,
    const uint16_t* const* kss, const uint16_t* const* vss, int rows, int q_heads, int kv_heads,
    const int32_t* pos, int max_seq, int nsplit, float* part) {
#pragma clang fp contract(off)
    constexpr int EL = BW == 8 ? KV8_HD : KV8_HD / 2;
    __shared__ Kv8Lds L;
    const int row = blockIdx.x, h = blockIdx.y, sp = blockIdx.z, t = threadIdx.x;
    const int p = pos[row];
    const int len = (p >= 0 && p < max_seq) ? p + 1 : 0;
    const size_t pi = ((size_t)row * q_heads + h) * nsplit + sp;
    float* po = part + (size_t)rows * q_heads * nsplit * 2 + pi * KV8_HD;
    const int t0 = sp * KV8_TILE;
    if (t0 >= len) { /* uniform: an empty split */
        po[t] = 0.f;
        if (t == 0) {
            part[pi * 2] = -INFINITY;
            part[pi * 2 + 1] = 0.f;
        }
        return;
    }
    const int kvh = h / (q_heads / kv_heads);
    const int8_t* kb = kcs[row] + (size_t)kvh * max_seq * EL;
    const int8_t* vb = vcs[row] + (size_t)kvh * max_seq * EL;
    const uint16_t* ksb = kss[row] + (size_t)kvh * max_seq * 4;
    const uint16_t* vsb = vss[row] + (size_t)kvh * max_seq * 4;
    L.sq[t] = bf2f(q[((size_t)row * q_heads + h) * KV8_HD + t]) * 0.08838834764831845f;
    __syncthreads();
    float m = -INFINITY, corr;
    const float l = kv8_tile<BW>(kb, ksb, t0, len, m, corr, L, true);
    const int lim = min(KV8_TILE, len - t0);
    float a = 0.f;
    for (int j2 = 0; j2 < lim; j2++) {
        const size_t j = (size_t)(t0 + j2);
        a = fmaf(L.sp[j2] * h2f(vsb[j * 4 + (t >> 5)]), kv8_val(vb + j * EL, t, BW), a);
    }
    po[t] = a;
    if (t == 0) {
        part[pi * 2] = m;
        part[pi * 2 + 1] = l;
    }
}

extern "C" hipError_t s2p_attn_combine_launch(const float* part, uint16_t* out, int rows, int qh,
                                              int nsplit, hipStream_t st);

extern "C" hipError_t s2pk_kv_append8(const s2p_bf16* k, const s2p_bf16* v, int8_t* k_cache,
                                      int8_t* v_cache, void* k_scale, void* v_scale, int rows,
                                      int kv_heads, int head_dim, int pos, int max_seq, int bw,
                                      hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (head_dim != KV8_HD || (bw != 8 && bw != 4) || kv_heads <= 0) return hipErrorInvalidValue;
    const dim3 grid((unsigned)(rows * kv_heads));
    if (bw == 8)
        hipLaunchKernelGGL(k_kv_append8<8>, grid, dim3(KV8_HD), 0, st, (const uint16_t*)k,
                           (const uint16_t*)v, k_cache, v_cache, (uint16_t*)k_scale,
                           (uint16_t*)v_scale, nullptr, nullptr, nullptr, nullptr, kv_heads, pos,
                           nullptr, max_seq);
    else
        hipLaunchKernelGGL(k_kv_append8<4>, grid, dim3(KV8_HD), 0, st, (const uint16_t*)k,
                           (const uint16_t*)v, k_cache, v_cache, (uint16_t*)k_scale,
                           (uint16_t*)v_scale, nullptr, nullptr, nullptr, nullptr, kv_heads, pos,
                           nullptr, max_seq);
    return hipGetLastError();
}

extern "C" hipError_t s2pk_kv_append8_ptrs(const s2p_bf16* k, const s2p_bf16* v,
                                           int8_t* const* k_caches, int8_t* const* v_caches,
                                           void* const* k_scales, void* const* v_scales, int rows,
                                           int kv_heads, int head_dim, const int32_t* pos,
                                           int max_seq, int bw, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (head_dim != KV8_HD || (bw != 8 && bw != 4) || kv_heads <= 0 || !pos)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)(rows * kv_heads));
    if (bw == 8)
        hipLaunchKernelGGL(k_kv_append8<8>, grid, dim3(KV8_HD), 0, st, (const uint16_t*)k,
                           (const uint16_t*)v, nullptr, nullptr, nullptr, nullptr, k_caches,
                           v_caches, (uint16_t* const*)k_scales, (uint16_t* const*)v_scales,
                           kv_heads, 0, pos, max_seq);
    else
        hipLaunchKernelGGL(k_kv_append8<4>, grid, dim3(KV8_HD), 0, st, (const uint16_t*)k,
                           (const uint16_t*)v, nullptr, nullptr, nullptr, nullptr, k_caches,
                           v_caches, (uint16_t* const*)k_scales, (uint16_t* const*)v_scales,
                           kv_heads, 0, pos, max_seq);
    return hipGetLastError();
}

extern "C" hipError_t s2pk_attention8(const s2p_bf16* q, const int8_t* k_cache,
                                      const int8_t* v_cache, const void* k_scale,
                                      const void* v_scale, s2p_bf16* out, int rows, int q_heads,
                                      int kv_heads, int head_dim, int pos, int max_seq, int bw,
                                      hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (head_dim != KV8_HD || (bw != 8 && bw != 4) || kv_heads <= 0 || q_heads % kv_heads ||
        pos < 0 || pos + rows > max_seq)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)rows, (unsigned)q_heads);
    if (bw == 8)
        hipLaunchKernelGGL(k_attention8<8>, grid, dim3(KV8_TILE), 0, st, (const uint16_t*)q,
                           k_cache, v_cache, (const uint16_t*)k_scale, (const uint16_t*)v_scale,
                           (uint16_t*)out, q_heads, kv_heads, pos, max_seq);
    else
        hipLaunchKernelGGL(k_attention8<4>, grid, dim3(KV8_TILE), 0, st, (const uint16_t*)q,
                           k_cache, v_cache, (const uint16_t*)k_scale, (const uint16_t*)v_scale,
                           (uint16_t*)out, q_heads, kv_heads, pos, max_seq);
    return hipGetLastError();
}

extern "C" hipError_t s2pk_attention8_decode(const s2p_bf16* q, const int8_t* const* k_caches,
                                             const int8_t* const* v_caches,
                                             const void* const* k_scales,
                                             const void* const* v_scales, s2p_bf16* out, int rows,
                                             int q_heads, int kv_heads, int head_dim,
                                             const int32_t* pos, int max_seq, int max_len,
                                             float* part, int bw, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (head_dim != KV8_HD || (bw != 8 && bw != 4) || kv_heads <= 0 || q_heads % kv_heads ||
        !part || max_len <= 0 || !pos)
        return hipErrorInvalidValue;
    const int nsplit = (max_len + KV8_TILE - 1) / KV8_TILE;
    const dim3 grid((unsigned)rows, (unsigned)q_heads, (unsigned)nsplit);
    if (bw == 8)
        hipLaunchKernelGGL(k_attention8_split<8>, grid, dim3(KV8_TILE), 0, st, (const uint16_t*)q,
                           k_caches, v_caches, (const uint16_t* const*)k_scales,
                           (const uint16_t* const*)v_scales, rows, q_heads, kv_heads, pos,
                           max_seq, nsplit, part);
    else
        hipLaunchKernelGGL(k_attention8_split<4>, grid, dim3(KV8_TILE), 0, st, (const uint16_t*)q,
                           k_caches, v_caches, (const uint16_t* const*)k_scales,
                           (const uint16_t* const*)v_scales, rows, q_heads, kv_heads, pos,
                           max_seq, nsplit, part);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return s2p_attn_combine_launch(part, (uint16_t*)out, rows, q_heads, nsplit, st);
}

/* ------------------------------------------------------------------------
 * The verify plan over quantised session caches, in the reference session's
 * layout (slowar_internal.h:177-179, 208-225): a session's code tensor
 * kv [layers][16][max_seq][EL] (per layer K heads 0..7, then V heads) and its
 * separate f16 scale tensor kvs [layers][16][max_seq][4].  Rows are planned as for the bf16 cache (S2pRowPlan): row r writes
 * slot plan.slot[r], has RoPE position plan.pos[r] and sees [0, L) plus the
 * node slots of plan.vis[r], whose highest bit is the row's own node. */
#include "attn_dev.h"
#include "gemv_internal.h"
#include "prims_dev.h"


struct Kv8Plane {
    int8_t* pay;    /* [max_seq][EL] */
    uint16_t* sc;   /* [max_seq][4] */
};

template <int BW>
static __device__ __forceinline__ Kv8Plane kv8_plane(const S2pRowPlan& plan, int sess, int layer,
                                                     int plane) {
    constexpr int EL = BW == 8 ? KV8_HD : KV8_HD / 2;
    const size_t pl = (size_t)layer * 16 + plane;
    Kv8Plane p;
    p.pay = (int8_t*)plan.kv[sess] + pl * plan.max_seq * EL;
    p.sc = (uint16_t*)plan.kvs[sess] + pl * plan.max_seq * 4;
    return p;
}

/* quantise element pair (x0 = element lane, x1 = element lane + 64) of one
 * 128-wide row into payload row `pay` and scale row `sc` (kernels.cu:541-579) */
template <int BW>
static __device__ __forceinline__ void kv8_put(float x0, float x1, int8_t* pay, uint16_t* sc,
                                               int lane) {
#pragma clang fp contract(off)
    constexpr int QMAX = BW == 8 ? 127 : 7;
    const float xs[2] = {x0, x1};
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int e = lane + 64 * h;
        const float a = max32(fabsf(xs[h]));
        const uint16_t hs = f2h(__fdiv_rn(a, (float)QMAX));
        const float s = h2f(hs);
        int q = s > 0.f ? (int)rintf(__fdiv_rn(xs[h], s)) : 0;
        q = max(-QMAX, min(QMAX, q));
        if (BW == 8) {
            pay[e] = (int8_t)q;
        } else {
            const int hi = __shfl_down(q, 1, 64);
            if ((e & 1) == 0) pay[e >> 1] = (int8_t)((q & 0xF) | ((hi & 0xF) << 4));
        }
        if ((lane & 31) == 0) sc[e >> 5] = hs;
    }
}

/* qk-norm + RoPE of one (row, head) of the fused qkv output (the rounding
 * points of the bf16 plan's prologue); q heads to q_out, K (rounded to bf16)
 * and V quantised into the row's slot. */
template <int BW>
__global__ __launch_bounds__(64) void k_qkrope_append8(const uint16_t* __restrict__ qkv,
                                                       uint16_t* __restrict__ q_out,
                                                       const uint16_t* __restrict__ qn_w,
                                                       const uint16_t* __restrict__ kn_w,
                                                       S2pRowPlan plan, int layer, float eps,
                                                       const float* __restrict__ rope_tab) {
#pragma clang fp contract(off)
    const int QH = 32, KVH = 8, HD = 128, W = (QH + 2 * KVH) * HD;
    const int row = blockIdx.x, head = blockIdx.y, lane = threadIdx.x;
    const bool is_q = head < QH;
    const int kh = head - QH;
    const uint16_t* src = qkv + (size_t)row * W + (is_q ? head * HD : QH * HD + kh * HD);
    const uint16_t* nw = is_q ? qn_w : kn_w;
    const float v0 = bf2f(src[lane]), v1 = bf2f(src[lane + 64]);
    const float* cs = rope_tab + (size_t)row * 128;
    float o[2];
    qkrope_math(v0, v1, nw[lane], nw[lane + 64], cs[(lane >> 1) * 2], cs[(lane >> 1) * 2 + 1],
                cs[((lane + 64) >> 1) * 2], cs[((lane + 64) >> 1) * 2 + 1], eps, lane, &o[0],
                &o[1]);
    if (is_q) {
        uint16_t* dst = q_out + (size_t)row * QH * HD + head * HD;
        dst[lane] = f2bf(o[0]);
        dst[lane + 64] = f2bf(o[1]);
        return;
    }
    constexpr int EL = BW == 8 ? KV8_HD : KV8_HD / 2;
    const int sess = plan.sess[row];
    const size_t slot = (size_t)plan.slot[row];
    const Kv8Plane kp = kv8_plane<BW>(plan, sess, layer, kh);
    const Kv8Plane vp = kv8_plane<BW>(plan, sess, layer, KVH + kh);
    kv8_put<BW>(bf2f(f2bf(o[0])), bf2f(f2bf(o[1])), kp.pay + slot * EL, kp.sc + slot * 4, lane);
    const uint16_t* vs = qkv + (size_t)row * W + (QH + KVH) * HD + kh * HD;
    kv8_put<BW>(bf2f(vs[lane]), bf2f(vs[lane + 64]), vp.pay + slot * EL, vp.sc + slot * 4, lane);
}

/* Verify-plan attention over quantised caches on the matrix cores: one wave
 * per (segment of <= 8 rows of a session, kv head, position split: splits
 * sized so the grid is one resident round); its 32
 * query vectors (8 rows x the 4 query heads of the kv head) are two 16-row
 * MFMA tiles, as in the bf16 kernel.  Per 32-slot tile:
 *   scores: the int8 (int4) codes are exact in bf16, so each 32-dim group g
 *     is one 16x16x32 MFMA of q against the codes, scaled by the slot's
 *     group scale: s = sum_g ks[slot][g] * (q_g . k_g);
 *   PV: the codes of V (exact in bf16) are the B operand and the group scale
 *     rides in P: the A operand of output dims in group g is p * vs[slot][g],
 *     split hi + lo in bf16 by truncation (16 significant bits).
 * Each split writes the (m, l, O) partial of every (row, head) it serves;
 * s2p_attn_combine_launch merges them.  Arithmetic is fp32 throughout, in an
 * order of its own (tolerance-checked against the reference-order oracle). */
#define A8_TILE 32
#define A8_PS 40 /* P row stride in bf16 (32 slots + 8 pad) */

static __device__ __forceinline__ uint32_t bf_pair(float lo, float hi) {
    /* two values exact in bf16 (the codes, |x| <= 127): their upper halves,
     * packed with one byte permute */
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

template <int BW>
static __device__ __forceinline__ float a8_code(uint32_t word, int k) {
    /* element k (0..3 for BW 8, 0..7 for BW 4) of a little-endian word */
    if (BW == 8) return (float)(int8_t)(word >> (8 * k));
    const int nib = (word >> (4 * k)) & 0xF;
    return (float)(nib >= 8 ? nib - 16 : nib);
}

template <int BW>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void k_attn8_mfma(const uint16_t* __restrict__ q,
                                                   S2pRowPlan plan,
                                                   const S2pAttnSeg* __restrict__ segs,
                                                   int layer, int rows, int nsplit,
                                                   int split_pos, float* __restrict__ part) {
    constexpr int EL = BW == 8 ? KV8_HD : KV8_HD / 2;
    constexpr int QH = 32, KVH = 8;
    __shared__ __attribute__((aligned(16))) uint8_t s_v[A8_TILE * EL];
    /* P of one scale group: [hi / lo][q tile][query][slot] */
    __shared__ __attribute__((aligned(16))) uint16_t s_p[2][2][16][A8_PS];
    __shared__ __attribute__((aligned(16))) uint16_t s_q[32][KV8_HD + 8];
    const int lane = threadIdx.x, qq = lane >> 4, c = lane & 15;
    const S2pAttnSeg sg = segs[blockIdx.x];
    const int kvh = blockIdx.y, sp = blockIdx.z;
    const int span = min(sg.span, plan.max_seq);
    const int p_begin = sp * split_pos;
    const int p_end = min(p_begin + split_pos, span);
    const Kv8Plane kp = kv8_plane<BW>(plan, sg.sess, layer, kvh);
    const Kv8Plane vp = kv8_plane<BW>(plan, sg.sess, layer, KVH + kvh);
    const float scale = 0.08838834764831845f;

    /* visibility of this lane's score rows rl = 4 qt + qq */
    uint64_t vis[2];
    int len[2];
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        const int rl = 4 * qt + qq;
        vis[qt] = rl < sg.nrows ? plan.vis[sg.row0 + rl] : 0ull;
        len[qt] = vis[qt] ? sg.L + 64 - __builtin_clzll(vis[qt]) : 0;
    }
    /* Q operands (A row c of tile qt = query vector 16 qt + c = (row rl, head
     * g)) staged in LDS once and read per use, which keeps registers for
     * two waves per SIMD */
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        const int qv = 16 * qt + c, rl = qv >> 2, g = qv & 3;
#pragma unroll
        for (int ch = 0; ch < 4; ch++)
            *(s2p_u32x4*)&s_q[qv][32 * ch + 8 * qq] =
                rl < sg.nrows ? *(const s2p_u32x4*)(q + (size_t)(sg.row0 + rl) * QH * KV8_HD +
                                                    (4 * kvh + g) * KV8_HD + 32 * ch + 8 * qq)
                              : (s2p_u32x4){0u, 0u, 0u, 0u};
    }
    wave_sync_lds();
    float m[2][4], l[2][4];
    s2p_f32x4 o[2][8];
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
#pragma unroll
        for (int v = 0; v < 4; v++) {
            m[qt][v] = -INFINITY;
            l[qt][v] = 0.f;
        }
#pragma unroll
        for (int dt = 0; dt < 8; dt++) o[qt][dt] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
    }

    /* raw codes and scales of one tile, loaded a tile ahead of their use:
     * V rows (16 B per lane per load; rows past the split read the last
     * row, never used), this lane's K words of slots tb + 16 ps + c (dims
     * 32 ch + 8 qq .. + 8) and those slots' K / V group scales */
    constexpr int NV = A8_TILE * EL / 1024, NKW = BW == 8 ? 2 : 1;
    s2p_u32x4 rv[NV];
    uint32_t rk[2][4][NKW];
    s2p_u32x2 rks[2], rvs[2];
    auto load_tile = [&](int tb) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int off = (i * 64 + lane) * 16, t = off / EL;
            const int pos = min(tb + t, p_end - 1);
            rv[i] = *(const s2p_u32x4*)(vp.pay + (size_t)pos * EL + off % EL);
        }
#pragma unroll
        for (int ps = 0; ps < 2; ps++) {
            const int pos = min(tb + 16 * ps + c, p_end - 1);
            const int8_t* kr0 = kp.pay + (size_t)pos * EL;
#pragma unroll
            for (int ch = 0; ch < 4; ch++) {
                if (BW == 8) {
                    const s2p_u32x2 t = *(const s2p_u32x2*)(kr0 + 32 * ch + 8 * qq);
                    rk[ps][ch][0] = t[0];
                    rk[ps][ch][NKW - 1] = t[1];
                } else {
                    rk[ps][ch][0] = *(const uint32_t*)(kr0 + 16 * ch + 4 * qq);
                }
            }
            rks[ps] = *(const s2p_u32x2*)(kp.sc + (size_t)pos * 4);
            rvs[ps] = *(const s2p_u32x2*)(vp.sc + (size_t)pos * 4);
        }
    };
    if (p_begin < p_end) load_tile(p_begin);

    for (int tb = p_begin; tb < p_end; tb += A8_TILE) {
#pragma unroll
        for (int i = 0; i < NV; i++) *(s2p_u32x4*)(s_v + (i * 64 + lane) * 16) = rv[i];
        /* scores: B column c = slot tb + 16 ps + c; the codes converted as
         * they are used.  lane (qq, c) element v = row 4 qt + qq, head v */
        const s2p_u32x2 ksc[2] = {rks[0], rks[1]}, vsc[2] = {rvs[0], rvs[1]};
        s2p_f32x4 scs[2][2];
#pragma unroll
        for (int ps = 0; ps < 2; ps++) {
            scs[0][ps] = scs[1][ps] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ch = 0; ch < 4; ch++) {
                uint32_t b[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t wd = BW == 8 ? rk[ps][ch][e >> 1] : rk[ps][ch][0];
                    const int k0 = BW == 8 ? 2 * (e & 1) : 2 * e;
                    b[e] = bf_pair(a8_code<BW>(wd, k0), a8_code<BW>(wd, k0 + 1));
                }
                const s2p_u32x4 kb = {b[0], b[1], b[2], b[3]};
                const uint32_t sw = ksc[ps][ch >> 1];
                const float ks = h2f((uint16_t)(ch & 1 ? sw >> 16 : sw & 0xFFFF));
#pragma unroll
                for (int qt = 0; qt < 2; qt++) {
                    const s2p_u32x4 qa = *(const s2p_u32x4*)&s_q[16 * qt + c][32 * ch + 8 * qq];
                    const s2p_f32x4 d = mfma16x16x32(qa, kb, (s2p_f32x4){0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int v = 0; v < 4; v++) scs[qt][ps][v] = fmaf(ks, d[v], scs[qt][ps][v]);
                }
            }
        }
        if (tb + A8_TILE < p_end) load_tile(tb + A8_TILE);
        /* online softmax: p of (row 4 qt + qq, head v) at slots tb + 16 ps + c */
        float pr[2][4][2];
#pragma unroll
        for (int qt = 0; qt < 2; qt++) {
            const s2p_f32x4* sc = scs[qt];
            const int L = sg.L;
            bool vs_ok[2];
#pragma unroll
            for (int ps = 0; ps < 2; ps++) {
                const int j = tb + 16 * ps + c;
                vs_ok[ps] = j < len[qt] && (j < L || ((vis[qt] >> (j - L)) & 1ull));
            }
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float t0 = vs_ok[0] ? sc[0][v] * scale : -INFINITY;
                const float t1 = vs_ok[1] ? sc[1][v] * scale : -INFINITY;
                const float tm = max16(fmaxf(t0, t1));
                const float mn = fmaxf(m[qt][v], tm);
                const float ms = mn == -INFINITY ? 0.f : mn;
                const float corr = __expf(m[qt][v] - ms);
                pr[qt][v][0] = __expf(t0 - ms);
                pr[qt][v][1] = __expf(t1 - ms);
                l[qt][v] = l[qt][v] * corr + pr[qt][v][0] + pr[qt][v][1];
                m[qt][v] = mn;
                /* rescale O only when some running max of the wave moved */
                if (__builtin_amdgcn_ballot_w64(corr != 1.0f)) {
#pragma unroll
                    for (int dt = 0; dt < 8; dt++) o[qt][dt][v] *= corr;
                }
            }
        }
        /* PV one scale group at a time (dims 32 g .. 32 g + 31): A = p * vs[slot][g]
         * through LDS, B = the V codes (column c = dim 16 dt + c, rows = slots
         * 8 qq .. 8 qq + 7) */
#pragma unroll
        for (int g = 0; g < 4; g++) {
#pragma unroll
            for (int ps = 0; ps < 2; ps++) {
                const uint32_t vw = vsc[ps][g >> 1];
                const float vs = h2f((uint16_t)(g & 1 ? vw >> 16 : vw & 0xFFFF));
#pragma unroll
                for (int qt = 0; qt < 2; qt++)
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        /* pv >= 0 = hi + lo, both truncated to bf16: 16
                         * significant bits */
                        const float pv = pr[qt][v][ps] * vs;
                        const uint32_t hb = __float_as_uint(pv) & 0xFFFF0000u;
                        const float lo = pv - __uint_as_float(hb);
                        s_p[0][qt][4 * qq + v][16 * ps + c] = (uint16_t)(hb >> 16);
                        s_p[1][qt][4 * qq + v][16 * ps + c] = (uint16_t)(__float_as_uint(lo) >> 16);
                    }
            }
            wave_sync_lds();
#pragma unroll
            for (int dh = 0; dh < 2; dh++) {
                const int dt = 2 * g + dh, d = 16 * dt + c;
                uint32_t b[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float x[2];
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const uint8_t* row = s_v + (8 * qq + 2 * e + h) * EL;
                        if (BW == 8) {
                            x[h] = (float)(int8_t)row[d];
                        } else {
                            const int nib = (d & 1) ? (row[d >> 1] >> 4) : (row[d >> 1] & 0xF);
                            x[h] = (float)(nib >= 8 ? nib - 16 : nib);
                        }
                    }
                    b[e] = bf_pair(x[0], x[1]);
                }
                const s2p_u32x4 bv = {b[0], b[1], b[2], b[3]};
#pragma unroll
                for (int qt = 0; qt < 2; qt++) {
                    const s2p_u32x4 pa = *(const s2p_u32x4*)&s_p[0][qt][c][8 * qq];
                    const s2p_u32x4 pl = *(const s2p_u32x4*)&s_p[1][qt][c][8 * qq];
                    o[qt][dt] = mfma16x16x32(pl, bv, o[qt][dt]);
                    o[qt][dt] = mfma16x16x32(pa, bv, o[qt][dt]);
                }
            }
            wave_sync_lds(); /* s_p is rewritten by the next group */
        }
    }

    /* partials of the served (row, head) pairs */
    const size_t obase = (size_t)rows * QH * nsplit * 2;
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        const int rl = 4 * qt + qq;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float lt = sum16(l[qt][v]);
            if (rl >= sg.nrows) continue;
            const size_t pi = ((size_t)(sg.row0 + rl) * QH + 4 * kvh + v) * nsplit + sp;
            if (c == 0) {
                part[pi * 2] = m[qt][v];
                part[pi * 2 + 1] = lt;
            }
#pragma unroll
            for (int dt = 0; dt < 8; dt++) part[obase + pi * KV8_HD + 16 * dt + c] = o[qt][dt][v];
        }
    }
}

/* Tree commit over quantised caches: accepted node path[d-1] moves to slot
 * L + d in increasing d (payload row and its four scales), one wave per
 * (session, layer, plane). */
template <int BW>
__global__ __launch_bounds__(64) void k_kv_commit8(S2pRowPlan plan,
                                                   const int32_t* __restrict__ path,
                                                   const int32_t* __restrict__ n_acc, int R) {
    constexpr int EL = BW == 8 ? KV8_HD : KV8_HD / 2;
    const int s = blockIdx.x, layer = blockIdx.y, plane = blockIdx.z, lane = threadIdx.x;
    int n = n_acc[s];
    n = n < 0 ? 0 : (n > R - 1 ? R - 1 : n);
    const int L = plan.slot[s * R];
    const Kv8Plane p = kv8_plane<BW>(plan, s, layer, plane);
    for (int d = 1; d <= n; d++) {
        const int node = path[(size_t)s * R + d - 1];
        if (node == d || node < d || node >= R) continue; /* chain slot, or invalid */
        const int8_t* src = p.pay + (size_t)(L + node) * EL;
        int8_t* dst = p.pay + (size_t)(L + d) * EL;
        if (BW == 8) {
            ((uint16_t*)dst)[lane] = ((const uint16_t*)src)[lane];
        } else {
            dst[lane] = src[lane];
        }
        if (lane < 4) p.sc[(size_t)(L + d) * 4 + lane] = p.sc[(size_t)(L + node) * 4 + lane];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}


extern "C" int64_t s2p_attn8_plan_part_floats(int rows, int max_span) {
    const int64_t nsplit = (max_span + KV8_TILE - 1) / KV8_TILE;
    return (int64_t)rows * 32 * nsplit * (2 + KV8_HD);
}

extern "C" hipError_t s2p_qkrope_append8_launch(const void* qkv, void* q_out, const void* qn_w,
                                                const void* kn_w, const S2pRowPlan* plan,
                                                int rows, int layer, float eps,
                                                const float* rope_tab, int bw, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (bw != 8 && bw != 4) return hipErrorInvalidValue;
    if (bw == 8)
        hipLaunchKernelGGL(k_qkrope_append8<8>, dim3(rows, 40), dim3(64), 0, st,
                           (const uint16_t*)qkv, (uint16_t*)q_out, (const uint16_t*)qn_w,
                           (const uint16_t*)kn_w, *plan, layer, eps, rope_tab);
    else
        hipLaunchKernelGGL(k_qkrope_append8<4>, dim3(rows, 40), dim3(64), 0, st,
                           (const uint16_t*)qkv, (uint16_t*)q_out, (const uint16_t*)qn_w,
                           (const uint16_t*)kn_w, *plan, layer, eps, rope_tab);
    return hipGetLastError();
}

extern "C" hipError_t s2p_attn8_plan_launch(const void* q, void* out, const S2pRowPlan* plan,
                                            const S2pAttnSeg* segs, int n_seg, int rows,
                                            int layer, int max_span, float* part, int bw,
                                            hipStream_t st) {
    if (rows <= 0 || n_seg <= 0) return hipSuccess;
    if ((bw != 8 && bw != 4) || max_span <= 0 || max_span > plan->max_seq)
        return hipErrorInvalidValue;
    /* splits of >= 128 slots (the part scratch is sized for 128), as short
     * as one resident round of waves allows (two per SIMD: 8 per CU) */
    const int cus = s2p_cu_count();
    const int64_t per_split = (int64_t)n_seg * 8;
    int64_t ns_max = (int64_t)cus * 8 / per_split;
    if (ns_max < 1) ns_max = 1;
    int split_pos = (int)((max_span + ns_max - 1) / ns_max);
    split_pos = (split_pos + A8_TILE - 1) / A8_TILE * A8_TILE;
    if (split_pos < KV8_TILE) split_pos = KV8_TILE;
    const int nsplit = (max_span + split_pos - 1) / split_pos;
    const dim3 grid((unsigned)n_seg, 8u, (unsigned)nsplit);
    if (bw == 8)
        hipLaunchKernelGGL(k_attn8_mfma<8>, grid, dim3(64), 0, st, (const uint16_t*)q, *plan,
                           segs, layer, rows, nsplit, split_pos, part);
    else
        hipLaunchKernelGGL(k_attn8_mfma<4>, grid, dim3(64), 0, st, (const uint16_t*)q, *plan,
                           segs, layer, rows, nsplit, split_pos, part);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return s2p_attn_combine_launch(part, (uint16_t*)out, rows, 32, nsplit, st);
}

extern "C" hipError_t s2p_kv_commit8_launch(const S2pRowPlan* plan, const int32_t* path,
                                            const int32_t* n_acc, int n_sess, int R,
                                            int n_layers, int bw, hipStream_t st) {
    if (n_sess <= 0) return hipSuccess;
    if (bw != 8 && bw != 4) return hipErrorInvalidValue;
    if (bw == 8)
        hipLaunchKernelGGL(k_kv_commit8<8>, dim3(n_sess, n_layers, 16), dim3(64), 0, st, *plan,
                           path, n_acc, R);
    else
        hipLaunchKernelGGL(k_kv_commit8<4>, dim3(n_sess, n_layers, 16), dim3(64), 0, st, *plan,
                           path, n_acc, R);
    return hipGetLastError();
}
