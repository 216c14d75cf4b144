/* s2pro MI355X — weight-only INT4 / INT8 GEMV engine for decode / verify M.
 *
 * Replaces the reference's packed-INT4 and per-channel INT8 GEMVs
 * (src/sched/int8_gemv.cu:60-104, 279-324, 836-902, 964-986) and its M > 16
 * dequant + cuBLAS / WMMA paths (gemm.c:444-490, int8_gemv.cu:535-618) with
 * one MI355X kernel.
 *
 * Work decomposition.  The N output rows form 64-row blocks, K forms S
 * splits.  The grid is (P, S): workgroup (p, s) stages the activations of
 * split s in LDS once and then streams the weights of row blocks p, p+P,
 * p+2P, ...; P is sized so the grid is about one resident round of
 * workgroups, so the staging is paid once per workgroup, not once per block.
 * Wave w owns rows 16w..16w+15 of the current block and runs its own weight
 * stream, double buffered (the next chunk's 16-byte loads are in flight
 * while the current chunk is multiplied), with no workgroup barrier between
 * chunks.
 *
 * MFMA mapping (v_mfma_f32_16x16x32_bf16).  Lane (q, r) = (lane / 16,
 * lane % 16) issues coalesced 16-byte loads: INT4 one 32-weight group of row
 * r, INT8 half a group.  A 4 x 4 transpose across lane quarters
 * (v_permlane32_swap, v_permlane16_swap) turns four such loads into the A
 * operands of four MFMAs, 16 rows x 32 k each.  The B operand (16 activation
 * rows x 32 k) comes from LDS; columns beyond M read row M-1 and are dropped.
 *
 * INT4 -> bf16 in registers: nibbles XOR 8 are OR-ed into the top mantissa
 * bits of bf16 1.0, giving 1.5 + w/16 exactly.  Per group the MFMA yields
 * raw_g = 1.5 X_g + (w . x)_g / 16 with X_g the activation group sum; the f16
 * group scale is applied in fp32 (acc += s_g raw_g, as the reference's
 * acc += s * gs, int8_gemv.cu:312) and the bias sum_g s_g X_g is two extra
 * MFMAs per 32 groups per split part on exact bf16 splits of s (hi + lo) and
 * X (hi + mid + lo): result = 16 acc - 24 corr.  The per-group VALU work is
 * then independent of M.
 * INT8 per channel: bytes XOR 0x80 via v_cvt_f32_ubyte*, 128 + w exact in
 * bf16; result = s_n (acc - 128 sum_k x_k).
 *
 * Staging applies the consuming layer's RMSNorm (row inverse RMS from the
 * producer epilogue's per-64-column sums of squares) with the rule's
 * roundings.  Epilogues: bf16 store; residual add y = bf16(y + bf16(acc))
 * (kernels.cu:1242-1247) with sums of squares for the next RMSNorm; or
 * SwiGLU, where a block holds 32 gate rows and the 32 matching up rows and
 * the epilogue writes silu(bf16 g) * bf16 u (kernels.cu:1216-1229).
 *
 * Split-K partials go to a device scratch; the last workgroup to arrive at a
 * row block (self-resetting counter) sums the partials in split order
 * (deterministic) and runs the epilogue.
 */
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "common.h"
#include "s2pro/s2p_fmath.h"
#include "s2pro/gemm.h"
#include "gemv_internal.h"

#define GV_SMAX 32                /* most K splits */
#define GV_XPAD 8                 /* bf16 row padding of the staged x */
#define GV_LDS_BUDGET (40 * 1024) /* staging bytes aimed for: 4 WGs per CU */
#define GV_LDS_MAX (160 * 1024)
#define GV_COUNTERS (1 << 16)     /* arrival counters at GemvArgs.counters */

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
 * 0,4,1,5,2,6,3,7.  The 1.5 bias keeps the cancellation against the bias
 * correction small (|1.5 sum x| ~ 5 |w.x / 16|). */
S2P_DEV s2p_u32x4 deq_int4(uint32_t d, uint32_t mask, uint32_t one) {
    /* mask / one live in VGPRs (gfx9 VOP3 takes no literal), so each pair
     * is one shift and one v_and_or_b32 */
    d ^= 0x88888888u;
    s2p_u32x4 a;
    a.x = ((d << 3) & mask) | one;
    a.y = ((d >> 1) & mask) | one;
    a.z = ((d >> 5) & mask) | one;
    a.w = ((d >> 9) & mask) | one;
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

/* ----------------------------------------------------------------------- */

/* LDS carve-up of one workgroup (dynamic shared memory). */
/* LDS-typed pointers: every access compiles to ds_* (a generic pointer would
 * become flat_*, whose vmcnt accounting waits behind the weight stream) */
#define LDS(T) __attribute__((address_space(3))) T
struct GvLds {
    LDS(uint16_t)* x;   /* [M][xs] staged activations (INT4: PERM4 order) */
    LDS(uint16_t)* X3;  /* [M][3][xg] bf16 hi/mid/lo of the f32 group sums */
    LDS(float)* sc;     /* INT4: [4 waves][16 groups][16 rows] f32 scales */
    LDS(float)* inv;    /* [GEMV_MAX_M] inverse RMS */
    LDS(float)* xtot;   /* [GEMV_MAX_M] INT8: sum of the window's activations */
    LDS(int)* flag;     /* last-arrival broadcast */
    int xs, xg;
};

static __host__ __device__ inline int gv_round32(int v) { return (v + 31) & ~31; }

static __host__ __device__ size_t gv_lds_bytes(int M, int win, int wfmt) {
    const size_t xs = (size_t)win * 32 + GV_XPAD;
    const size_t xg = (size_t)gv_round32(win) + 8;
    size_t b = (size_t)M * xs * 2 + (size_t)M * 3 * xg * 2;
    b = (b + 15) & ~(size_t)15;
    if (wfmt == GEMV_W_INT4) b += 4 * 16 * 16 * 4;
    b += 2 * GEMV_MAX_M * 4 + 16;
    return b;
}

S2P_DEV GvLds gv_carve(LDS(unsigned char)* base, int M, int win, int wfmt) {
    GvLds L;
    L.xs = win * 32 + GV_XPAD;
    L.xg = gv_round32(win) + 8;
    uint32_t off = 0;
    L.x = (LDS(uint16_t)*)(base + off);
    off += (uint32_t)M * L.xs * 2;
    L.X3 = (LDS(uint16_t)*)(base + off);
    off += (uint32_t)M * 3 * L.xg * 2;
    off = (off + 15) & ~15u;
    L.sc = (LDS(float)*)(base + off);
    if (wfmt == GEMV_W_INT4) off += 4 * 16 * 16 * 4;
    L.inv = (LDS(float)*)(base + off);
    off += GEMV_MAX_M * 4;
    L.xtot = (LDS(float)*)(base + off);
    off += GEMV_MAX_M * 4;
    L.flag = (LDS(int)*)(base + off);
    return L;
}

/* output row of local row l (0..63) of row block rb */
S2P_DEV int gv_row(const GemvArgs& a, int rb, int l) {
    if (a.epi == GEMV_EPI_SWIGLU) {
        const int F = a.N >> 1;
        return l < 32 ? rb * 32 + l : F + rb * 32 + (l - 32);
    }
    return rb * 64 + l;
}

/* exact split of an f32 into three bf16 (truncation: each remainder keeps
 * the low bits, so hi + mid + lo == v) */
S2P_DEV void split3(float v, uint16_t& hi, uint16_t& mid, uint16_t& lo) {
    const uint32_t b0 = __float_as_uint(v) & 0xFFFF0000u;
    const float r1 = v - __uint_as_float(b0);
    const uint32_t b1 = __float_as_uint(r1) & 0xFFFF0000u;
    const float r2 = r1 - __uint_as_float(b1);
    hi = (uint16_t)(b0 >> 16);
    mid = (uint16_t)(b1 >> 16);
    lo = (uint16_t)(__float_as_uint(r2) >> 16);
}

/* Stage groups [wg0, wg0 + wn) of every activation row into LDS: thread =
 * one 8-element column block for all rows (loads for 8 rows in flight at
 * once); the 4 threads of a 32-k group are adjacent, so group sums are
 * quad shuffles. */
template <int WFMT>
__device__ void gv_stage(const GemvArgs& a, const GvLds& L, int wg0, int wn) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    const int M = a.M;
    const int nb8 = wn * 4;
    const int wnp = gv_round32(wn);
    /* zero the group sums of the padded tail (read by the correction MFMA) */
    for (int i = tid; i < M * 3 * (wnp - wn); i += 256) {
        const int m = i / (3 * (wnp - wn)), rem = i - m * 3 * (wnp - wn);
        const int p = rem / (wnp - wn), g = wn + rem - p * (wnp - wn);
        L.X3[(m * 3 + p) * L.xg + g] = 0;
    }
    for (int bb = 0; bb < nb8; bb += 256) {
        const int b = bb + tid;
        const bool valid = b < nb8;
        const int k = wg0 * 32 + b * 8;
        s2p_u32x4 wn4 = {0u, 0u, 0u, 0u};
        if (valid && a.xmode == GEMV_X_NORM) wn4 = *(const s2p_u32x4*)(a.norm_w + k);
        for (int m0 = 0; m0 < M; m0 += 4) {
            s2p_u32x4 raw[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                raw[j] = (valid && m0 + j < M)
                             ? *(const s2p_u32x4*)(a.x + (size_t)(m0 + j) * a.ldx + k)
                             : (s2p_u32x4){0u, 0u, 0u, 0u};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int m = m0 + j;
                if (m >= M) break; /* uniform */
                uint32_t v[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w}; /* bf16 pairs */
                if (a.xmode == GEMV_X_NORM) {
                    const float inv = L.inv[m];
                    const uint32_t w4[4] = {wn4.x, wn4.y, wn4.z, wn4.w};
#pragma unroll
                    for (int d = 0; d < 4; d++) {
                        const uint32_t lo = f2bf(__fmul_rn(__fmul_rn(bf2f_lo(v[d]), inv), bf2f_lo(w4[d])));
                        const uint32_t hi = f2bf(__fmul_rn(__fmul_rn(bf2f_hi(v[d]), inv), bf2f_hi(w4[d])));
                        v[d] = lo | (hi << 16);
                    }
                }
                float s = 0.f;
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    s += bf2f_lo(v[d]);
                    s += bf2f_hi(v[d]);
                }
                s2p_u32x4 o;
                if (WFMT == GEMV_W_INT4) { /* k-slot order 0,4,1,5,2,6,3,7 */
                    o.x = (v[0] & 0xFFFFu) | (v[2] << 16);
                    o.y = (v[0] >> 16) | (v[2] & 0xFFFF0000u);
                    o.z = (v[1] & 0xFFFFu) | (v[3] << 16);
                    o.w = (v[1] >> 16) | (v[3] & 0xFFFF0000u);
                } else {
                    o = (s2p_u32x4){v[0], v[1], v[2], v[3]};
                }
                if (valid) *(LDS(s2p_u32x4)*)(L.x + m * L.xs + b * 8) = o;
                s += __shfl_xor(s, 1, 64);
                s += __shfl_xor(s, 2, 64);
                if (valid && (b & 3) == 0) {
                    uint16_t h, md, lo;
                    split3(s, h, md, lo);
                    const int g = b >> 2;
                    L.X3[(m * 3 + 0) * L.xg + g] = h;
                    L.X3[(m * 3 + 1) * L.xg + g] = md;
                    L.X3[(m * 3 + 2) * L.xg + g] = lo;
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    if (WFMT == GEMV_W_INT8) {
        __syncthreads();
        /* window activation total per row, wave per row, fixed order */
        const int lane = tid & 63;
        for (int m = tid >> 6; m < M; m += 4) {
            float s = 0.f;
            for (int g = lane; g < wn; g += 64)
                s += bf2f(L.X3[(m * 3 + 0) * L.xg + g]) +
                     bf2f(L.X3[(m * 3 + 1) * L.xg + g]) +
                     bf2f(L.X3[(m * 3 + 2) * L.xg + g]);
            s = wave_sum_down(s);
            if (lane == 0) L.xtot[m] = s;
        }
    }
}

/* one chunk of a wave's weight stream: INT4 4 loads x 4 groups plus the
 * chunk's 16 group scales (lane (q, r): groups 4q..4q+3 of row r); INT8
 * 2 x (2 loads x 4 groups) */
#define GV_CHG_INT4 16
#define GV_CHG_INT8 8
struct GvBuf {
    uint32_t w[16];
    s2p_u32x2 s;
};

template <int WFMT>
S2P_DEV void gv_load(GvBuf& B, const GemvArgs& a, int nrow, int gabs, int gn, int q) {
    if constexpr (WFMT == GEMV_W_INT4) {
        const uint8_t* wrow = a.w + (size_t)nrow * (a.K >> 1) + (size_t)gabs * 16;
#pragma unroll
        for (int it = 0; it < 4; it++) {
            s2p_u32x4 v = {0u, 0u, 0u, 0u};
            if (it * 4 < gn)
                v = __builtin_nontemporal_load((const s2p_u32x4*)(wrow + (it * 4 + q) * 16));
            B.w[it * 4 + 0] = v.x;
            B.w[it * 4 + 1] = v.y;
            B.w[it * 4 + 2] = v.z;
            B.w[it * 4 + 3] = v.w;
        }
        const uint16_t* srow = (const uint16_t*)a.s + (size_t)nrow * (a.K >> 5) + gabs + 4 * q;
        B.s = 4 * q < gn ? *(const s2p_u32x2*)srow : (s2p_u32x2){0u, 0u};
    } else {
        const uint8_t* wrow = a.w + (size_t)nrow * a.K + (size_t)gabs * 32;
#pragma unroll
        for (int it = 0; it < 2; it++) {
            s2p_u32x4 v0 = {0u, 0u, 0u, 0u}, v1 = {0u, 0u, 0u, 0u};
            if (it * 4 < gn) {
                v0 = __builtin_nontemporal_load((const s2p_u32x4*)(wrow + it * 128 + q * 32));
                v1 = __builtin_nontemporal_load((const s2p_u32x4*)(wrow + it * 128 + q * 32 + 16));
            }
            B.w[it * 8 + 0] = v0.x; B.w[it * 8 + 1] = v0.y;
            B.w[it * 8 + 2] = v0.z; B.w[it * 8 + 3] = v0.w;
            B.w[it * 8 + 4] = v1.x; B.w[it * 8 + 5] = v1.y;
            B.w[it * 8 + 6] = v1.z; B.w[it * 8 + 7] = v1.w;
        }
    }
}

S2P_DEV void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* D = A(16x16) * B(16x16) + C (v_mfma_f32_16x16x16_bf16): lane l supplies A
 * row l % 16 and B column l % 16, k-slots 4 (l / 16) .. +3; D as the x32 form */
S2P_DEV s2p_f32x4 mfma16x16x16(s2p_u32x2 a, s2p_u32x2 b, s2p_f32x4 c) {
    typedef __attribute__((ext_vector_type(4))) short s16x4;
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                      __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}

/* multiply one chunk: cg = chunk's first group within the staged window */
template <int WFMT, int MT>
S2P_DEV void gv_compute(const GvBuf& B, const GvLds& L, int cg, int gn, int M, int wave, int q,
                        int r, s2p_f32x4 (&acc)[MT], s2p_f32x4 (&corr)[MT]) {
    int mrow[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) mrow[t] = min(t * 16 + r, M - 1);
    if constexpr (WFMT == GEMV_W_INT4) {
        /* scales of row r, groups 4q..4q+3: f32 to this wave's LDS slice in
         * [group][row] order, and bf16 hi / lo as the correction's A operand */
        LDS(float)* sc = L.sc + wave * GV_CHG_INT4 * 16;
        uint32_t shi[2], slo[2];
#pragma unroll
        for (int d = 0; d < 2; d++) {
            const uint32_t pair = B.s[d];
            uint32_t hb[2], lb[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const float f = h2f((uint16_t)(e ? pair >> 16 : pair & 0xFFFFu));
                hb[e] = __float_as_uint(f) & 0xFFFF0000u;
                lb[e] = __float_as_uint(f - __uint_as_float(hb[e])) >> 16;
                sc[(4 * q + 2 * d + e) * 16 + r] = f;
            }
            shi[d] = (hb[0] >> 16) | hb[1];
            slo[d] = lb[0] | (lb[1] << 16);
        }
        wave_lds_sync();
        uint32_t kmask = 0x00780078u, kone = 0x3F803F80u;
        asm volatile("" : "+v"(kmask), "+v"(kone));
#pragma unroll
        for (int it = 0; it < GV_CHG_INT4 / 4; it++) {
            if (it * 4 >= gn) break;
            uint32_t d0 = B.w[it * 4 + 0], d1 = B.w[it * 4 + 1];
            uint32_t d2 = B.w[it * 4 + 2], d3 = B.w[it * 4 + 3];
            xpose4(d0, d1, d2, d3);
            const uint32_t dj[4] = {d0, d1, d2, d3};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int g = it * 4 + j;
                const s2p_u32x4 av = deq_int4(dj[j], kmask, kone);
                const s2p_f32x4 s4 = *(const LDS(s2p_f32x4)*)(sc + g * 16 + 4 * q);
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    const s2p_u32x4 bv =
                        *(const LDS(s2p_u32x4)*)(L.x + mrow[t] * L.xs + (cg + g) * 32 + q * 8);
                    const s2p_f32x4 raw = mfma16x16x32(av, bv, (s2p_f32x4){0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[t][i] = fmaf(s4[i], raw[i], acc[t][i]);
                }
            }
            __builtin_amdgcn_sched_barrier(0); /* keep LDS reads from piling up */
        }
        /* bias correction: corr += S (16 rows x 16 groups) . X (16 groups x 16 cols) */
        const s2p_u32x2 ah = {shi[0], shi[1]};
        const s2p_u32x2 al = {slo[0], slo[1]};
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int p = 0; p < 3; p++) {
                const s2p_u32x2 bx = *(const LDS(s2p_u32x2)*)(L.X3 + (mrow[t] * 3 + p) * L.xg +
                                                         cg + 4 * q);
                corr[t] = mfma16x16x16(ah, bx, corr[t]);
                corr[t] = mfma16x16x16(al, bx, corr[t]);
            }
    } else {
#pragma unroll
        for (int it = 0; it < GV_CHG_INT8 / 4; it++) {
            if (it * 4 >= gn) break;
            uint32_t e0 = B.w[it * 8 + 0], e1 = B.w[it * 8 + 2], e2 = B.w[it * 8 + 4],
                     e3 = B.w[it * 8 + 6];
            uint32_t o0 = B.w[it * 8 + 1], o1 = B.w[it * 8 + 3], o2 = B.w[it * 8 + 5],
                     o3 = B.w[it * 8 + 7];
            xpose4(e0, e1, e2, e3);
            xpose4(o0, o1, o2, o3);
            const uint32_t ej[4] = {e0, e1, e2, e3};
            const uint32_t oj[4] = {o0, o1, o2, o3};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int g = it * 4 + j;
                const s2p_u32x2 lo = deq_int8(ej[j]);
                const s2p_u32x2 hi = deq_int8(oj[j]);
                const s2p_u32x4 av = {lo.x, lo.y, hi.x, hi.y};
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    const s2p_u32x4 bv =
                        *(const LDS(s2p_u32x4)*)(L.x + mrow[t] * L.xs + (cg + g) * 32 + q * 8);
                    acc[t] = mfma16x16x32(av, bv, acc[t]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

/* deterministic split-order sum of the partials p[k * stride], k < S, with
 * the loads of 16 splits in flight at a time */
S2P_DEV float gv_sum_splits(const float* p, size_t stride, int S) {
    float s = 0.f;
    for (int k0 = 0; k0 < S; k0 += 16) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; j++)
            v[j] = k0 + j < S ? __hip_atomic_load(p + (size_t)(k0 + j) * stride, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT)
                              : 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++)
            if (k0 + j < S) s += v[j];
    }
    return s;
}

/* last arrival at row block rb: sum the splits and run the epilogue */
template <int WFMT>
__device__ void gv_fixup(const GemvArgs& a, int rb) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x, lane = tid & 63;
    const int M = a.M, S = a.splits;
    const size_t stride = (size_t)M * a.nrb * 64;
    const float* part = a.part;
    if (a.epi == GEMV_EPI_SWIGLU) {
        const int F = a.N >> 1;
        for (int idx = tid; idx < M * 32; idx += 256) {
            const int m = idx >> 5, j = idx & 31;
            const float* p0 = part + ((size_t)m * a.nrb + rb) * 64;
            float g = gv_sum_splits(p0 + j, stride, S);
            float u = gv_sum_splits(p0 + 32 + j, stride, S);
            if (WFMT == GEMV_W_INT8) {
                g *= ((const float*)a.s)[rb * 32 + j];
                u *= ((const float*)a.s)[F + rb * 32 + j];
            }
            if (rb * 32 + j < F)
                a.y[(size_t)m * a.ldy + rb * 32 + j] = silu_mul_bf16(f2bf(g), f2bf(u));
        }
        return;
    }
    for (int base = 0; base < M * 64; base += 256) {
        const int idx = base + tid;
        const int m = idx >> 6, l = idx & 63;
        const int n = rb * 64 + l;
        float ssq = 0.f;
        if (m < M && n < a.N) {
            float s = gv_sum_splits(part + ((size_t)m * a.nrb + rb) * 64 + l, stride, S);
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
            /* one wave = one row m = the block's 64 columns */
            const float tot = wave_sum_down(ssq);
            if (lane == 0 && m < M) a.ssq_out[(size_t)rb * GEMV_MAX_M + m] = tot;
        }
    }
}

/* WIN1: the split's activations fit one LDS window, staged once before the
 * stream; otherwise every (row block, window) segment restages. */
template <int WFMT, int MT, bool WIN1>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(MT == 1 ? 4 : (MT == 2 ? 3 : 2)))) void k_gemv(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    LDS(unsigned char)* smem = (LDS(unsigned char)*)smem_raw;
    constexpr int CHG = WFMT == GEMV_W_INT4 ? GV_CHG_INT4 : GV_CHG_INT8; /* groups per chunk */
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int q = lane >> 4, r = lane & 15;
    const int p = blockIdx.x, P = gridDim.x, sp = blockIdx.y;
    const int M = a.M;
    const int G = a.K >> 5;
    const int gb = sp * a.gps;
    const int ge = min(G, gb + a.gps);
    const int nmine = p < a.nrb ? (a.nrb - p + P - 1) / P : 0;
    if (nmine == 0 || gb >= ge) return; /* uniform over the workgroup */
    const int win = a.win;
    const int nwin = WIN1 ? 1 : (ge - gb + win - 1) / win;
    const int nseg = nmine * nwin;
    const bool handoff = a.splits > 1 || a.epi != GEMV_EPI_STORE;
    const GvLds L = gv_carve(smem, M, win, WFMT);
    const int lrow = wave * 16 + r; /* local row this lane loads */

    if (a.xmode == GEMV_X_NORM) {
        /* inverse RMS per row from the producer's per-block sums of squares:
         * lanes take blocks, fixed-order wave reduction */
        for (int m = wave; m < M; m += 4) {
            float s = 0.f;
            for (int b = lane; b < a.ssq_in_blocks; b += 64) s += a.ssq_in[(size_t)b * GEMV_MAX_M + m];
            s = wave_sum_down(s);
            if (lane == 0) L.inv[m] = rsqrt_rule(s / (float)a.K + a.norm_eps);
        }
    }

    s2p_f32x4 acc[MT], corr[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) {
        acc[t] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
        corr[t] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
    }
    float corr8[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) corr8[t] = 0.f;

    /* position of segment k's chunk c */
    auto seg_rb = [&](int k) { return p + (k / nwin) * P; };
    auto seg_g0 = [&](int k) { return gb + (k % nwin) * win; };
    auto seg_gn = [&](int k) { return min(win, ge - seg_g0(k)); };
    auto load_at = [&](GvBuf& B, int k, int c) {
        const int rb = seg_rb(k);
        const int nrow = min(gv_row(a, rb, lrow), a.N - 1);
        const int g0 = seg_g0(k) + c * CHG;
        const int gn = min(CHG, seg_g0(k) + seg_gn(k) - g0);
        gv_load<WFMT>(B, a, nrow, g0, gn, q);
    };

    GvBuf cur, nxt;
    load_at(cur, 0, 0); /* in flight during the staging */
    if constexpr (WIN1) {
        __syncthreads();
        gv_stage<WFMT>(a, L, gb, ge - gb);
        __syncthreads();
    }
    for (int k = 0; k < nseg; k++) {
        const int rb = seg_rb(k);
        const int w = k % nwin;
        const int g0 = seg_g0(k), gn_w = seg_gn(k);
        const int nch = (gn_w + CHG - 1) / CHG;
        if constexpr (!WIN1) {
            __syncthreads();
            gv_stage<WFMT>(a, L, g0, gn_w);
            __syncthreads();
        }
        const bool last_w = w == nwin - 1;
        for (int c = 0; c < nch; c++) {
            const bool last_c = c == nch - 1;
            const bool has_next = !last_c || k + 1 < nseg;
            const bool defer = last_c && last_w && handoff;
            if (has_next && !defer) {
                if (!last_c)
                    load_at(nxt, k, c + 1);
                else
                    load_at(nxt, k + 1, 0);
            }
            gv_compute<WFMT, MT>(cur, L, c * CHG, min(CHG, gn_w - c * CHG), M, wave, q, r, acc,
                                 corr);
            if (has_next && !defer) cur = nxt;
        }
        if (WFMT == GEMV_W_INT8) {
#pragma unroll
            for (int t = 0; t < MT; t++) corr8[t] += L.xtot[min(t * 16 + r, M - 1)];
        }
        if (!last_w) continue;

        /* ---- row block rb complete ---- */
        float res[MT][4];
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                res[t][i] = WFMT == GEMV_W_INT4 ? 16.0f * acc[t][i] - 24.0f * corr[t][i]
                                                : fmaf(-128.0f, corr8[t], acc[t][i]);
#pragma unroll
        for (int t = 0; t < MT; t++) {
            acc[t] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
            corr[t] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
            corr8[t] = 0.f;
        }
        if (!handoff) {
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const int m = t * 16 + r;
                if (m >= M) continue;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int n = rb * 64 + wave * 16 + q * 4 + i;
                    if (n >= a.N) continue;
                    float v = res[t][i];
                    if (WFMT == GEMV_W_INT8) v *= ((const float*)a.s)[n];
                    a.y[(size_t)m * a.ldy + n] = f2bf(v);
                }
            }
            continue;
        }
        /* Split-K handoff without cache maintenance: the 8 XCD L2s are not
         * coherent and an agent-scope fence would write back / invalidate a
         * whole L2, so the partials are written through to memory (sc1, the
         * encoding of an agent-scope store; one 16-byte store per lane), read
         * back with agent-scope atomic loads, and each workgroup waits for
         * its partial stores to complete before it signals arrival. */
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int m = t * 16 + r;
            if (m >= M) continue;
            float* dst = &a.part[(((size_t)sp * M + m) * a.nrb + rb) * 64 + wave * 16 + q * 4];
            const s2p_f32x4 v4 = {res[t][0], res[t][1], res[t][2], res[t][3]};
            asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(dst), "v"(v4) : "memory");
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) {
            const unsigned prev = __hip_atomic_fetch_add(&a.counters[rb], 1u, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            *L.flag = prev == (unsigned)(a.splits - 1);
        }
        if (k + 1 < nseg) load_at(cur, k + 1, 0); /* the deferred prefetch */
        __syncthreads();
        const bool last = *L.flag != 0;
        if (last) {
            gv_fixup<WFMT>(a, rb);
            if (tid == 0)
                __hip_atomic_store(&a.counters[rb], 0u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads(); /* flag is rewritten at the next block */
    }
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

static int gv_slots(void) {
    static int cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (cache[dev]) return cache[dev];
    int slots = 0;
    const char* e = getenv("S2P_GEMV_TARGET_WG");
    if (e && atoi(e) > 0) slots = atoi(e);
    if (!slots) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        slots = 4 * cus;
    }
    cache[dev] = slots;
    return slots;
}

template <int WFMT, int MT, bool WIN1>
static hipError_t gv_launch_w(const GemvArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    static bool attr_set = false;
    if (!attr_set) {
        (void)hipFuncSetAttribute((const void*)k_gemv<WFMT, MT, WIN1>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, GV_LDS_MAX);
        attr_set = true;
    }
    hipLaunchKernelGGL((k_gemv<WFMT, MT, WIN1>), grid, dim3(256), lds, st, a);
    return hipGetLastError();
}

template <int WFMT, int MT>
static hipError_t gv_launch_mt(const GemvArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    if (a.win >= a.gps) return gv_launch_w<WFMT, MT, true>(a, grid, lds, st);
    return gv_launch_w<WFMT, MT, false>(a, grid, lds, st);
}

extern "C" hipError_t s2p_gemv_launch(const GemvArgs* ap, hipStream_t st) {
    GemvArgs a = *ap;
    if (a.M <= 0 || a.M > GEMV_MAX_M || a.N <= 0 || a.K <= 0 || (a.K & 127))
        return hipErrorInvalidValue;
    if (a.gps < 0 || (a.gps & 3)) return hipErrorInvalidValue;
    if (a.epi == GEMV_EPI_SWIGLU && ((a.N & 1) || ((a.N >> 1) & 31))) return hipErrorInvalidValue;
    if (a.xmode == GEMV_X_NORM && (!a.norm_w || !a.ssq_in || a.ssq_in_blocks <= 0))
        return hipErrorInvalidValue;
    const int G = a.K >> 5;
    a.nrb = a.epi == GEMV_EPI_SWIGLU ? (a.N >> 1) / 32 : (a.N + 63) / 64;
    const int slots = gv_slots();
    const bool autos = a.gps == 0;
    int gps = a.gps;
    if (autos) {
        int S = a.nrb >= slots ? 1 : (slots + a.nrb - 1) / a.nrb;
        int smax = G / 8;
        if (smax < 1) smax = 1;
        if (S > smax) S = smax;
        if (S > GV_SMAX) S = GV_SMAX;
        gps = (((G + S - 1) / S) + 3) & ~3;
    }
    if (gps > G) gps = G;
    a.splits = (G + gps - 1) / gps;
    const bool handoff = a.splits > 1 || a.epi != GEMV_EPI_STORE;
    if (handoff) {
        if (!a.part || !a.counters || a.nrb > GV_COUNTERS) return hipErrorInvalidValue;
        while ((int64_t)a.splits * a.M * a.nrb * 64 > a.part_cap || a.splits > GV_SMAX) {
            if (!autos || a.splits == 1) return hipErrorInvalidValue;
            gps += 4;
            a.splits = (G + gps - 1) / gps;
        }
    }
    /* prefer more splits over LDS windows (restaging per block) */
    while (autos && gps > 4 && gv_lds_bytes(a.M, gps, a.wfmt) > GV_LDS_BUDGET) {
        const int g2 = gps - 4, s2 = (G + g2 - 1) / g2;
        if (s2 > GV_SMAX || (int64_t)s2 * a.M * a.nrb * 64 > a.part_cap || !a.part || !a.counters)
            break;
        gps = g2;
        a.splits = s2;
    }
    a.gps = gps;
    int win = gps;
    while (win > 4 && gv_lds_bytes(a.M, win, a.wfmt) > GV_LDS_BUDGET) win -= 4;
    const size_t lds = gv_lds_bytes(a.M, win, a.wfmt);
    if (lds > GV_LDS_MAX) return hipErrorInvalidValue;
    a.win = win;
    int P = (slots + a.splits - 1) / a.splits;
    if (P > a.nrb) P = a.nrb;
    dim3 grid((unsigned)P, (unsigned)a.splits);
    const int mt = (a.M + 15) / 16;
    if (a.wfmt == GEMV_W_INT4) {
        switch (mt) {
            case 1: return gv_launch_mt<GEMV_W_INT4, 1>(a, grid, lds, st);
            case 2: return gv_launch_mt<GEMV_W_INT4, 2>(a, grid, lds, st);
            case 3: return gv_launch_mt<GEMV_W_INT4, 3>(a, grid, lds, st);
            case 4: return gv_launch_mt<GEMV_W_INT4, 4>(a, grid, lds, st);
            case 5: return gv_launch_mt<GEMV_W_INT4, 5>(a, grid, lds, st);
            case 6: return gv_launch_mt<GEMV_W_INT4, 6>(a, grid, lds, st);
            case 7: return gv_launch_mt<GEMV_W_INT4, 7>(a, grid, lds, st);
            default: return gv_launch_mt<GEMV_W_INT4, 8>(a, grid, lds, st);
        }
    }
    switch (mt) {
        case 1: return gv_launch_mt<GEMV_W_INT8, 1>(a, grid, lds, st);
        case 2: return gv_launch_mt<GEMV_W_INT8, 2>(a, grid, lds, st);
        case 3: return gv_launch_mt<GEMV_W_INT8, 3>(a, grid, lds, st);
        case 4: return gv_launch_mt<GEMV_W_INT8, 4>(a, grid, lds, st);
        case 5: return gv_launch_mt<GEMV_W_INT8, 5>(a, grid, lds, st);
        case 6: return gv_launch_mt<GEMV_W_INT8, 6>(a, grid, lds, st);
        case 7: return gv_launch_mt<GEMV_W_INT8, 7>(a, grid, lds, st);
        default: return gv_launch_mt<GEMV_W_INT8, 8>(a, grid, lds, st);
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
