/* s2pro MI355X — weight-only INT4 / INT8 GEMV engine for decode / verify M.
 *
 * Replaces the reference's packed-INT4 and per-channel INT8 GEMVs
 * (src/sched/int8_gemv.cu:60-104, 279-324, 836-902, 964-986) and its M > 16
 * dequant + cuBLAS / WMMA paths (gemm.c:444-490, int8_gemv.cu:535-618) with
 * one MI355X kernel:
 *
 *  - Workgroup = 4 waves = 64 output rows x a K range (split-K); grid =
 *    (ceil(N/64), splits).  Wave w owns rows n0..n0+15.
 *  - Each lane issues fully coalesced 16-byte weight loads: lane (q, r)
 *    (q = lane/16, r = lane%16) loads one 32-weight group (INT4) of row r.
 *    A 4x4 transpose across lane quarters (v_permlane32_swap then
 *    v_permlane16_swap) turns four such loads into the A operands of four
 *    v_mfma_f32_16x16x32_bf16, one per group, 16 rows x 32 k each.
 *  - INT4 -> bf16 in registers: nibbles XOR 8 are OR-ed into the top
 *    mantissa bits of bf16 1.0, giving 1.5 + w/16 exactly (a shift and one
 *    v_and_or per two weights); the bias is removed per group with the
 *    activation group sum:  16 * (sum_k (1.5 + w_k/16) x_k - 1.5 sum_k x_k).
 *    The f16 group scale is applied per group in fp32 (as the reference's
 *    acc += s * gs, int8_gemv.cu:312), not folded into bf16 weights.
 *  - INT8 per channel: bytes XOR 0x80 converted with v_cvt_f32_ubyte*, the
 *    128 * sum(x) bias and the row scale are applied once at the end.
 *  - Activations (M <= 128, padded to 16-column MFMA tiles) are staged per
 *    512-k chunk in LDS in the k-slot order the dequantised A operand uses,
 *    with per-group sums; the staging optionally applies the RMSNorm of the
 *    consuming layer (row inverse RMS from partial sums of squares written by
 *    the producing epilogue) or SwiGLU (silu(gate) * up, two bf16 roundings
 *    as kernels.cu:1224-1227).
 *  - Split-K partials go to a device scratch; the last workgroup to finish a
 *    64-row block (arrival counter, self-resetting) sums the partials in
 *    split order (deterministic) and runs the epilogue: bf16 store, or the
 *    residual add y = bf16(y + bf16(acc)) of kernels.cu:1242-1247 with the
 *    per-block sums of squares of the new residual for the next RMSNorm.
 *
 * The arithmetic is fp32 accumulation of exact int x bf16 products; the
 * summation order differs from the reference's lane order (parity is by
 * tolerance, 1e-2 relative, like the reference's own TC path).
 */
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>

#include "common.h"
#include "s2pro/s2p_fmath.h"
#include "s2pro/gemm.h"
#include "gemv_internal.h"

#define GEMV_CHUNK_GROUPS 16          /* 512 k per LDS stage */
#define GEMV_XPAD 8                   /* bf16 elements of row padding */

/* k-slot order of the INT4 A operand inside each 8-weight block: the
 * and/or dequant yields nibble pairs (0,4) (1,5) (2,6) (3,7). */
#define PERM4(e) ((((e) & 1) << 2) | ((e) >> 1))

/* 4x4 transpose of one dword per lane across lane quarters:
 * in: lane quarter q holds d[j] = A[q][j]; out: d[j] = A[j][q]. */
S2P_DEV void xpose4(uint32_t& d0, uint32_t& d1, uint32_t& d2, uint32_t& d3) {
    auto s02 = __builtin_amdgcn_permlane32_swap(d0, d2, false, false);
    d0 = s02[0];
    d2 = s02[1];
    auto s13 = __builtin_amdgcn_permlane32_swap(d1, d3, false, false);
    d1 = s13[0];
    d3 = s13[1];
    auto s01 = __builtin_amdgcn_permlane16_swap(d0, d1, false, false);
    d0 = s01[0];
    d1 = s01[1];
    auto s23 = __builtin_amdgcn_permlane16_swap(d2, d3, false, false);
    d2 = s23[0];
    d3 = s23[1];
}

/* 8 nibbles (two's complement w) -> 8 bf16 holding 1.5 + w/16 exactly (the
 * nibble XOR 8 lands in the top 4 mantissa bits of bf16 1.0), in k-slot order
 * 0,4,1,5,2,6,3,7.  The dot product is then 16 * (raw - 1.5 * sum(x)); the
 * 1.5 bias keeps the cancellation small (|1.5 sum x| ~ 5 |w.x / 16|). */
S2P_DEV s2p_u32x4 deq_int4(uint32_t d) {
    d ^= 0x88888888u;
    s2p_u32x4 a;
    a.x = ((d << 3) & 0x00780078u) | 0x3F803F80u;
    a.y = ((d >> 1) & 0x00780078u) | 0x3F803F80u;
    a.z = ((d >> 5) & 0x00780078u) | 0x3F803F80u;
    a.w = ((d >> 9) & 0x00780078u) | 0x3F803F80u;
    return a;
}

/* 4 int8 (dword) -> 2 bf16x2 holding 128 + w, natural k order */
S2P_DEV s2p_u32x2 deq_int8(uint32_t d) {
    d ^= 0x80808080u;
    const uint32_t f0 = __float_as_uint((float)(d & 0xFFu));
    const uint32_t f1 = __float_as_uint((float)((d >> 8) & 0xFFu));
    const uint32_t f2 = __float_as_uint((float)((d >> 16) & 0xFFu));
    const uint32_t f3 = __float_as_uint((float)(d >> 24));
    s2p_u32x2 r;
    r.x = __builtin_amdgcn_perm(f1, f0, 0x07060302u);
    r.y = __builtin_amdgcn_perm(f3, f2, 0x07060302u);
    return r;
}

/* silu(g) * u with the two bf16 roundings of kernels.cu:1216-1229; exp is
 * the rule's s2p_expf so the value matches the host oracle bit for bit. */
S2P_DEV uint16_t silu_mul_bf16(uint16_t g16, uint16_t u16) {
#pragma clang fp contract(off)
    const float g = bf2f(g16);
    const float u = bf2f(u16);
    const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, s2p_expf(-g)));
    const float sil = bf2f(f2bf(__fmul_rn(g, sig)));
    return f2bf(__fmul_rn(sil, u));
}

struct GemvSmem {
    /* carved from dynamic LDS */
    uint16_t* x;     /* [Mpad][CH*32 + pad] */
    float* xs;       /* [Mpad][CH] group sums */
    uint16_t* sc;    /* [CH][64] f16 scales (INT4) */
    float* inv;      /* [M] inverse RMS (NORM staging) */
    int xstride;
};

template <int WFMT>
__device__ void stage_chunk(const GemvArgs& a, GemvSmem& sm, int g0, int gn, int M,
                            int Mpad, int rb) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    const int chk = gn * 32; /* k elements in this chunk */
    /* activations: one thread per (m, 8-block) */
    const int nblk8 = chk / 8;
    for (int it = tid; it < Mpad * nblk8; it += 256) {
        const int m = it / nblk8, b = it - m * nblk8;
        uint16_t v[8];
        if (m < M) {
            const int k = g0 * 32 + b * 8;
            if (a.xmode == GEMV_X_SILU) {
                const uint16_t* gp = a.x + (size_t)m * a.ldx + k;
                const uint16_t* up = gp + a.K;
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = silu_mul_bf16(gp[e], up[e]);
            } else {
                const s2p_u32x4 raw = *(const s2p_u32x4*)(a.x + (size_t)m * a.ldx + k);
                const uint16_t* rv = (const uint16_t*)&raw;
                if (a.xmode == GEMV_X_NORM) {
                    const float inv = sm.inv[m];
                    const s2p_u32x4 wr = *(const s2p_u32x4*)(a.norm_w + k);
                    const uint16_t* wv = (const uint16_t*)&wr;
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        v[e] = f2bf(__fmul_rn(__fmul_rn(bf2f(rv[e]), inv), bf2f(wv[e])));
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++) v[e] = rv[e];
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = 0;
        }
        uint16_t o[8];
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = WFMT == GEMV_W_INT4 ? v[PERM4(e)] : v[e];
        *(s2p_u32x4*)(sm.x + (size_t)m * sm.xstride + b * 8) = *(const s2p_u32x4*)o;
        /* group sums: the 4 threads of a group are consecutive in `it` when
         * nblk8 % 4 == 0; reduce with shuffles inside aligned quads */
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) s += bf2f(v[e]);
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        if ((b & 3) == 0) sm.xs[m * GEMV_CHUNK_GROUPS + (b >> 2)] = s;
    }
    if (WFMT == GEMV_W_INT4) {
        /* scales: [gn][64 rows]; thread -> (row, group) */
        const int rows0 = rb * 64;
        for (int it = tid; it < 64 * gn; it += 256) {
            const int row = it / gn, g = it - row * gn;
            int n = rows0 + row;
            if (n >= a.N) n = a.N - 1;
            sm.sc[g * 64 + row] =
                ((const uint16_t*)a.s)[(size_t)n * (a.K >> 5) + g0 + g];
        }
    }
}

/* ----------------------------------------------------------------------- */

template <int WFMT, int MT>
__global__ __launch_bounds__(256) void k_gemv_mfma(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int q = lane >> 4, r = lane & 15;
    const int rb = blockIdx.x;
    const int sp = blockIdx.y;
    const int M = a.M;
    const int Mpad = MT * 16;
    const int G_total = a.K >> 5;
    const int g_begin = sp * a.gps;
    const int g_end = min(G_total, g_begin + a.gps);
    const int n0 = rb * 64 + wave * 16;
    const int nrow = min(n0 + r, a.N - 1); /* clamped load row */

    GemvSmem sm;
    sm.xstride = GEMV_CHUNK_GROUPS * 32 + GEMV_XPAD;
    unsigned char* p = smem_raw;
    sm.x = (uint16_t*)p;
    p += (size_t)Mpad * sm.xstride * 2;
    sm.xs = (float*)p;
    p += (size_t)Mpad * GEMV_CHUNK_GROUPS * 4;
    sm.sc = (uint16_t*)p;
    p += GEMV_CHUNK_GROUPS * 64 * 2;
    sm.inv = (float*)p;

    if (a.xmode == GEMV_X_NORM) {
        /* inverse RMS per row from the producer's per-block sums of squares,
         * summed in block order */
        if (threadIdx.x < M) {
            float s = 0.f;
            for (int b = 0; b < a.ssq_in_blocks; b++)
                s += a.ssq_in[(size_t)b * GEMV_MAX_M + threadIdx.x];
            sm.inv[threadIdx.x] = rsqrt_rule(s / (float)a.K + a.norm_eps);
        }
        __syncthreads();
    }

    s2p_f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
    float xs_tot[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) xs_tot[t] = 0.f;

    for (int gc = g_begin; gc < g_end; gc += GEMV_CHUNK_GROUPS) {
        const int gn = min(GEMV_CHUNK_GROUPS, g_end - gc);
        /* weight loads of this chunk first (in flight during the staging) */
        uint32_t wreg[GEMV_CHUNK_GROUPS / 4][8];
        const int nit = gn >> 2;
        if constexpr (WFMT == GEMV_W_INT4) {
            const uint8_t* wrow = a.w + (size_t)nrow * (a.K >> 1) + (size_t)gc * 16;
#pragma unroll
            for (int it = 0; it < GEMV_CHUNK_GROUPS / 4; it++) {
                if (it < nit) {
                    const s2p_u32x4 v = __builtin_nontemporal_load(
                        (const s2p_u32x4*)(wrow + (it * 4 + q) * 16));
                    wreg[it][0] = v.x;
                    wreg[it][1] = v.y;
                    wreg[it][2] = v.z;
                    wreg[it][3] = v.w;
                }
            }
        } else {
            const uint8_t* wrow = a.w + (size_t)nrow * a.K + (size_t)gc * 32;
#pragma unroll
            for (int it = 0; it < GEMV_CHUNK_GROUPS / 4; it++) {
                if (it < nit) {
                    const s2p_u32x4 v0 = __builtin_nontemporal_load(
                        (const s2p_u32x4*)(wrow + it * 128 + q * 32));
                    const s2p_u32x4 v1 = __builtin_nontemporal_load(
                        (const s2p_u32x4*)(wrow + it * 128 + q * 32 + 16));
                    wreg[it][0] = v0.x; wreg[it][1] = v0.y;
                    wreg[it][2] = v0.z; wreg[it][3] = v0.w;
                    wreg[it][4] = v1.x; wreg[it][5] = v1.y;
                    wreg[it][6] = v1.z; wreg[it][7] = v1.w;
                }
            }
        }
        __syncthreads(); /* previous chunk's LDS reads done */
        stage_chunk<WFMT>(a, sm, gc, gn, M, Mpad, rb);
        __syncthreads();

#pragma unroll
        for (int it = 0; it < GEMV_CHUNK_GROUPS / 4; it++) {
            if (it >= nit) break;
            if constexpr (WFMT == GEMV_W_INT4) {
                uint32_t d0 = wreg[it][0], d1 = wreg[it][1], d2 = wreg[it][2], d3 = wreg[it][3];
                xpose4(d0, d1, d2, d3);
                const uint32_t dj[4] = {d0, d1, d2, d3};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int gl = it * 4 + j; /* group within the chunk */
                    const s2p_u32x4 av = deq_int4(dj[j]);
                    /* scales of rows 4q..4q+3 of this wave, group gl */
                    const s2p_u32x2 sw =
                        *(const s2p_u32x2*)(sm.sc + gl * 64 + wave * 16 + q * 4);
                    const float s0 = h2f((uint16_t)(sw.x & 0xFFFFu));
                    const float s1 = h2f((uint16_t)(sw.x >> 16));
                    const float s2 = h2f((uint16_t)(sw.y & 0xFFFFu));
                    const float s3 = h2f((uint16_t)(sw.y >> 16));
#pragma unroll
                    for (int t = 0; t < MT; t++) {
                        const int m = t * 16 + r;
                        const s2p_u32x4 bv =
                            *(const s2p_u32x4*)(sm.x + (size_t)m * sm.xstride + gl * 32 + q * 8);
                        const float xsum = sm.xs[m * GEMV_CHUNK_GROUPS + gl];
                        const s2p_f32x4 raw = mfma16x16x32(av, bv, (s2p_f32x4){0.f, 0.f, 0.f, 0.f});
                        acc[t][0] = fmaf(s0, fmaf(-1.5f, xsum, raw[0]), acc[t][0]);
                        acc[t][1] = fmaf(s1, fmaf(-1.5f, xsum, raw[1]), acc[t][1]);
                        acc[t][2] = fmaf(s2, fmaf(-1.5f, xsum, raw[2]), acc[t][2]);
                        acc[t][3] = fmaf(s3, fmaf(-1.5f, xsum, raw[3]), acc[t][3]);
                    }
                }
            } else {
                uint32_t e0 = wreg[it][0], e1 = wreg[it][2], e2 = wreg[it][4], e3 = wreg[it][6];
                uint32_t o0 = wreg[it][1], o1 = wreg[it][3], o2 = wreg[it][5], o3 = wreg[it][7];
                xpose4(e0, e1, e2, e3);
                xpose4(o0, o1, o2, o3);
                const uint32_t ej[4] = {e0, e1, e2, e3};
                const uint32_t oj[4] = {o0, o1, o2, o3};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int gl = it * 4 + j;
                    const s2p_u32x2 lo = deq_int8(ej[j]);
                    const s2p_u32x2 hi = deq_int8(oj[j]);
                    const s2p_u32x4 av = {lo.x, lo.y, hi.x, hi.y};
#pragma unroll
                    for (int t = 0; t < MT; t++) {
                        const int m = t * 16 + r;
                        const s2p_u32x4 bv =
                            *(const s2p_u32x4*)(sm.x + (size_t)m * sm.xstride + gl * 32 + q * 8);
                        acc[t] = mfma16x16x32(av, bv, acc[t]);
                        if (q == 0) xs_tot[t] += sm.xs[m * GEMV_CHUNK_GROUPS + gl];
                    }
                }
            }
        }
    }

    if (WFMT == GEMV_W_INT4) {
        /* undo the 1/16 of the dequantised weights (exact power of two) */
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[t][i] *= 16.0f;
    } else {
        /* remove the 128 * sum(x) bias; the lanes of quarter 0 carry the
         * column sums, broadcast them to the other quarters */
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const float xsum = __shfl(xs_tot[t], r, 64);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[t][i] = fmaf(-128.0f, xsum, acc[t][i]);
        }
    }

    /* ---- output ---- */
    if (a.splits == 1 && a.epi == GEMV_EPI_STORE) {
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int m = t * 16 + r;
            if (m >= M) continue;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int n = n0 + q * 4 + i;
                if (n >= a.N) continue;
                float v = acc[t][i];
                if (WFMT == GEMV_W_INT8) v *= ((const float*)a.s)[n];
                a.y[(size_t)m * a.ldy + n] = f2bf(v);
            }
        }
        return;
    }

    /* Split-K handoff without cache maintenance.  The 8 XCD L2s are not
     * coherent, and an agent-scope fence would write back / invalidate the
     * whole L2 per workgroup.  Instead every access to the partials and the
     * counter is an agent-scope atomic (device-coherent loads and stores),
     * and each workgroup waits for its partial stores to complete before it
     * signals arrival; the last arrival then reads every split. */
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const int m = t * 16 + r;
        if (m >= M) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = n0 + q * 4 + i;
            if (n >= a.N) continue;
            __hip_atomic_store(&a.part[((size_t)sp * M + m) * a.N + n], acc[t][i],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __shared__ int s_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_fetch_add(&a.counters[rb], 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == (unsigned)(a.splits - 1);
    }
    __syncthreads();
    if (!s_last) return;

    /* last workgroup of this row block: deterministic split-order sum */
    for (int base = 0; base < M * 64; base += 256) {
        const int idx = base + threadIdx.x;
        const int m = idx >> 6;
        const int n = rb * 64 + (idx & 63);
        float ssq = 0.f;
        if (m < M && n < a.N) {
            float s = 0.f;
            for (int k = 0; k < a.splits; k++)
                s += __hip_atomic_load(&a.part[((size_t)k * M + m) * a.N + n],
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (WFMT == GEMV_W_INT8) s *= ((const float*)a.s)[n];
            const uint16_t yb = f2bf(s);
            uint16_t* yp = a.y + (size_t)m * a.ldy + n;
            if (a.epi == GEMV_EPI_RESID) {
                const uint16_t xo = f2bf(__fadd_rn(bf2f(*yp), bf2f(yb)));
                *yp = xo;
                const float xv = bf2f(xo);
                ssq = xv * xv;
            } else {
                *yp = yb;
            }
        }
        if (a.epi == GEMV_EPI_RESID && a.ssq_out) {
            /* one wave = one row m = 64 consecutive columns */
            const float tot = wave_sum_down(ssq);
            if (lane == 0 && m < M) a.ssq_out[(size_t)rb * GEMV_MAX_M + m] = tot;
        }
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(&a.counters[rb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Generic one-wave-per-row GEMV for group sizes other than 32 and the
 * int8-container group-wise format (s2p_intq_gemv); off the verify path.
 * Lane l covers 16-k tiles l*16 + 1024 i; wave tree reduction. */
template <int FMT>
__global__ __launch_bounds__(256) void k_gemv_generic(const uint8_t* __restrict__ w,
                                                      const void* __restrict__ sc,
                                                      const uint16_t* __restrict__ x,
                                                      uint16_t* __restrict__ y, int M,
                                                      int N, int K, int gshift) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;
    for (int m = 0; m < M; m++) {
        float acc = 0.f;
        for (int k0 = lane * 16; k0 < K; k0 += 1024) {
            float s = 0.f;
            for (int j = 0; j < 16; j++) {
                const int k = k0 + j;
                int wv;
                if (FMT == 0) { /* packed int4 */
                    const uint8_t b = w[(size_t)n * (K >> 1) + (k >> 1)];
                    wv = (k & 1) ? ((int)(int8_t)b >> 4) : ((int)(int8_t)(uint8_t)(b << 4) >> 4);
                } else {        /* int8 container */
                    wv = (int)(int8_t)w[(size_t)n * K + k];
                }
                s = fmaf((float)wv, bf2f(x[(size_t)m * K + k]), s);
            }
            const float g = h2f(((const uint16_t*)sc)[(size_t)n * (K >> gshift) + (k0 >> gshift)]);
            acc = fmaf(s, g, acc);
        }
        acc = wave_sum_down(acc);
        if (lane == 0) y[(size_t)m * N + n] = f2bf(acc);
    }
}

/* ------------------------------------------------------------- launchers */

static size_t smem_bytes(int Mpad, int wfmt) {
    const size_t xstride = GEMV_CHUNK_GROUPS * 32 + GEMV_XPAD;
    size_t b = (size_t)Mpad * xstride * 2 + (size_t)Mpad * GEMV_CHUNK_GROUPS * 4;
    b += GEMV_CHUNK_GROUPS * 64 * 2;
    b += GEMV_MAX_M * 4;
    (void)wfmt;
    return b;
}

template <int WFMT, int MT>
static hipError_t launch_mt(const GemvArgs& a, dim3 grid, hipStream_t st) {
    const size_t sb = smem_bytes(MT * 16, WFMT);
    static bool attr_set = false;
    if (!attr_set) {
        (void)hipFuncSetAttribute((const void*)k_gemv_mfma<WFMT, MT>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)sb);
        attr_set = true;
    }
    hipLaunchKernelGGL((k_gemv_mfma<WFMT, MT>), grid, dim3(256), sb, st, a);
    return hipGetLastError();
}

extern "C" hipError_t s2p_gemv_launch(const GemvArgs* ap, hipStream_t st) {
    GemvArgs a = *ap;
    if (a.M <= 0 || a.M > GEMV_MAX_M || a.N <= 0 || a.K <= 0 || (a.K & 127)) return hipErrorInvalidValue;
    if (a.gps <= 0 || (a.gps & 3)) return hipErrorInvalidValue;
    const int G_total = a.K >> 5;
    a.splits = (G_total + a.gps - 1) / a.gps;
    if ((a.splits > 1 || a.epi != GEMV_EPI_STORE) && (!a.part || !a.counters))
        return hipErrorInvalidValue;
    dim3 grid((unsigned)((a.N + 63) / 64), (unsigned)a.splits);
    const int mt = (a.M + 15) / 16;
    if (a.wfmt == GEMV_W_INT4) {
        switch (mt) {
            case 1: return launch_mt<GEMV_W_INT4, 1>(a, grid, st);
            case 2: return launch_mt<GEMV_W_INT4, 2>(a, grid, st);
            case 3: return launch_mt<GEMV_W_INT4, 3>(a, grid, st);
            case 4: return launch_mt<GEMV_W_INT4, 4>(a, grid, st);
            case 5: return launch_mt<GEMV_W_INT4, 5>(a, grid, st);
            case 6: return launch_mt<GEMV_W_INT4, 6>(a, grid, st);
            case 7: return launch_mt<GEMV_W_INT4, 7>(a, grid, st);
            default: return launch_mt<GEMV_W_INT4, 8>(a, grid, st);
        }
    }
    switch (mt) {
        case 1: return launch_mt<GEMV_W_INT8, 1>(a, grid, st);
        case 2: return launch_mt<GEMV_W_INT8, 2>(a, grid, st);
        case 3: return launch_mt<GEMV_W_INT8, 3>(a, grid, st);
        case 4: return launch_mt<GEMV_W_INT8, 4>(a, grid, st);
        case 5: return launch_mt<GEMV_W_INT8, 5>(a, grid, st);
        case 6: return launch_mt<GEMV_W_INT8, 6>(a, grid, st);
        case 7: return launch_mt<GEMV_W_INT8, 7>(a, grid, st);
        default: return launch_mt<GEMV_W_INT8, 8>(a, grid, st);
    }
}

extern "C" hipError_t s2p_gemv_generic_launch(int fmt, const void* w, const void* sc,
                                              const void* x, void* y, int M, int N, int K,
                                              int gshift, hipStream_t st) {
    dim3 grid((unsigned)((N + 3) / 4));
    if (fmt == 0)
        hipLaunchKernelGGL((k_gemv_generic<0>), grid, dim3(256), 0, st, (const uint8_t*)w, sc,
                           (const uint16_t*)x, (uint16_t*)y, M, N, K, gshift);
    else
        hipLaunchKernelGGL((k_gemv_generic<1>), grid, dim3(256), 0, st, (const uint8_t*)w, sc,
                           (const uint16_t*)x, (uint16_t*)y, M, N, K, gshift);
    return hipGetLastError();
}
