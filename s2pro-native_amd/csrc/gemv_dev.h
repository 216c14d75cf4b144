/* s2pro MI355X — device code of the INT4 / INT8 GEMV engine (see gemv.hip
 * for the design), shared by the k_gemv kernel and the persistent verify
 * kernel.  Outputs, split-K partials and sums of squares are written
 * through (coh.h); activations are read around the L2 only in the
 * persistent kernel (COH), where their producer ran in the same launch. */
#ifndef S2P_GEMV_DEV_H
#define S2P_GEMV_DEV_H

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "coh.h"
#include "common.h"
#include "gemv_internal.h"
#include "s2pro/s2p_fmath.h"

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

/* LDS writes of a wave visible to all its lanes */
S2P_DEV void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* Activation reads: device-coherent (COH, the persistent kernel, where the
 * producer ran in the same launch) or plain L2-cacheable (layer kernels:
 * the producer was an earlier launch). */
template <bool COH>
S2P_DEV s2p_u32x4 ld_act128(const uint16_t* p) {
    if constexpr (COH) return coh_ld128(p);
    else return *(const s2p_u32x4*)p;
}
template <bool COH>
S2P_DEV float ld_actf(const float* p) {
    if constexpr (COH) return coh_ldf(p);
    else return *p;
}
template <bool COH>
S2P_DEV uint16_t ld_act16(const uint16_t* p) {
    if constexpr (COH) return coh_ld16(p);
    else return *p;
}

/* Transform one activation row m of 8-element column block b (RMSNorm with
 * the rule's roundings when staging a norm), store it in LDS in the
 * A-operand k-slot order, and its 32-k group sums (quad shuffle: the 4
 * blocks of a group are in adjacent lanes). */
template <int WFMT>
S2P_DEV void gv_stage_one(const GemvArgs& a, const GvLds& L, int m, int b, bool valid,
                          s2p_u32x4 raw, s2p_u32x4 wn4) {
#pragma clang fp contract(off)
    uint32_t v[4] = {raw.x, raw.y, raw.z, raw.w}; /* bf16 pairs */
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
    if constexpr (WFMT == GEMV_W_BF16) return; /* no group sums: no bias term */
    s = quad_sum(s);
    if (valid && (b & 3) == 0) {
        uint16_t h, md, lo;
        split3(s, h, md, lo);
        const int g = b >> 2;
        L.X3[(m * 3 + 0) * L.xg + g] = h;
        L.X3[(m * 3 + 1) * L.xg + g] = md;
        L.X3[(m * 3 + 2) * L.xg + g] = lo;
    }
}

/* Stage groups [wg0, wg0 + wn) of every activation row into LDS (and, for a
 * norm with with_inv, the rows' inverse RMS first): thread = one 8-element
 * column block for all rows, loads for 4 rows in flight at once.  NT = 256:
 * the whole (4-wave) workgroup stages a shared window; NT = 64: one wave
 * stages its own window (the inverse RMS is already in L.inv). */
template <int WFMT, bool COH, int NT = 256>
__device__ void gv_stage(const GemvArgs& a, const GvLds& L, int wg0, int wn, bool with_inv) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int tid = NT == 256 ? (int)threadIdx.x : lane, wave = NT == 256 ? tid >> 6 : 0;
    constexpr int NWS = NT / 64; /* waves staging */
    const int M = a.M;
    const int nb8 = wn * 4;
    const int wnp = gv_round32(wn);
    if (NT == 256 && with_inv && a.xmode == GEMV_X_NORM) {
        /* inverse RMS per row from the producer's per-block sums of squares:
         * lanes take blocks, fixed-order wave reduction */
        for (int m = wave; m < M; m += 4) {
            float s = 0.f;
            for (int b = lane; b < a.ssq_in_blocks; b += 64)
                s += ld_actf<COH>(a.ssq_in + (size_t)b * GEMV_MAX_M + m);
            s = wave_sum_down(s);
            if (lane == 0) L.inv[m] = rsqrt_rule(s / (float)a.K + a.norm_eps);
        }
        __syncthreads();
    }
    /* zero the group sums of the padded tail (read by the correction MFMA;
     * fewer than 32 groups per row) */
    for (int row = tid >> 5; row < M * 3; row += NT / 32)
        if ((tid & 31) < wnp - wn) L.X3[row * L.xg + wn + (tid & 31)] = 0;
    for (int bb = 0; bb < nb8; bb += NT) {
        const int b = bb + tid;
        const bool valid = b < nb8;
        const int k = wg0 * 32 + b * 8;
        int m0 = 0;
        s2p_u32x4 wn4 = {0u, 0u, 0u, 0u};
        if (m0 < M && valid && a.xmode == GEMV_X_NORM) wn4 = *(const s2p_u32x4*)(a.norm_w + k);
        for (; m0 < M; m0 += 4) {
            s2p_u32x4 raw[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                raw[j] = (valid && m0 + j < M) ? ld_act128<COH>(a.x + (size_t)(m0 + j) * a.ldx + k)
                                               : (s2p_u32x4){0u, 0u, 0u, 0u};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (m0 + j >= M) break; /* uniform */
                gv_stage_one<WFMT>(a, L, m0 + j, b, valid, raw[j], wn4);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    if (WFMT == GEMV_W_INT8) {
        if constexpr (NT == 256) __syncthreads();
        else wave_lds_sync();
        /* window activation total per row, wave per row, fixed order */
        for (int m = wave; m < M; m += NWS) {
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
#define GV_CHG_BF16 4
static __host__ __device__ constexpr int gv_chg(int wfmt) {
    return wfmt == GEMV_W_INT4 ? GV_CHG_INT4 : (wfmt == GEMV_W_INT8 ? GV_CHG_INT8 : GV_CHG_BF16);
}
struct GvBuf {
    uint32_t w[16];
    s2p_u32x2 s;      /* INT4: f16 scales of row r, groups 4q..4q+3 */
    s2p_u32x2 sa[4];  /* INT4 (whole-K engine): f16 scales of row r, all 16 groups */
};

/* Branch-free: every load is issued (out-of-range groups read a clamped,
 * valid address), so the compiler can keep the next chunk's loads in flight
 * with a partial vmcnt while the current one is multiplied; conditional
 * loads, or selects on the loaded data, make it wait for everything.  The
 * out-of-range data is never used: the multiply stops at gn, and the bias
 * correction pairs those groups' (finite) scales with zero-padded sums. */
template <int WFMT, bool TR = false>
S2P_DEV void gv_load(GvBuf& B, const GemvArgs& a, int nrow, int gabs, int gn, int q) {
    if constexpr (WFMT == GEMV_W_INT4) {
        const uint8_t* wrow = a.w + (size_t)nrow * (a.K >> 1) + (size_t)gabs * 16;
#pragma unroll
        for (int it = 0; it < 4; it++) {
            const bool ok = it * 4 < gn;
            const s2p_u32x4 v = __builtin_nontemporal_load(
                (const s2p_u32x4*)(wrow + (ok ? (it * 4 + q) * 16 : q * 16)));
            B.w[it * 4 + 0] = v.x;
            B.w[it * 4 + 1] = v.y;
            B.w[it * 4 + 2] = v.z;
            B.w[it * 4 + 3] = v.w;
        }
        const bool sok = 4 * q < gn;
        const uint16_t* srow = (const uint16_t*)a.s + (size_t)nrow * (a.K >> 5) + gabs +
                               (sok ? 4 * q : 0);
        B.s = *(const s2p_u32x2*)srow;
        if constexpr (TR) {
            /* every lane of row r takes the row's 16 scales (four lanes read
             * the same bytes: one cache access) */
            const uint16_t* s0 = (const uint16_t*)a.s + (size_t)nrow * (a.K >> 5) + gabs;
#pragma unroll
            for (int d = 0; d < 4; d++) B.sa[d] = *(const s2p_u32x2*)(s0 + (4 * d < gn ? 4 * d : 0));
        }
    } else if constexpr (WFMT == GEMV_W_BF16) {
        /* lane (q, r): k 8q..8q+7 of group it of row r, the A operand as is */
        const uint16_t* wrow = (const uint16_t*)a.w + (size_t)nrow * a.K + (size_t)gabs * 32 + 8 * q;
#pragma unroll
        for (int it = 0; it < GV_CHG_BF16; it++) {
            const s2p_u32x4 v = gld_nt128(wrow + (it < gn ? it * 32 : 0));
            B.w[it * 4 + 0] = v.x;
            B.w[it * 4 + 1] = v.y;
            B.w[it * 4 + 2] = v.z;
            B.w[it * 4 + 3] = v.w;
        }
    } else {
        const uint8_t* wrow = a.w + (size_t)nrow * a.K + (size_t)gabs * 32;
#pragma unroll
        for (int it = 0; it < 2; it++) {
            const bool ok = it * 4 < gn;
            const uint8_t* src = wrow + (ok ? it * 128 + q * 32 : q * 32);
            const s2p_u32x4 v0 = __builtin_nontemporal_load((const s2p_u32x4*)src);
            const s2p_u32x4 v1 = __builtin_nontemporal_load((const s2p_u32x4*)(src + 16));
            B.w[it * 8 + 0] = v0.x; B.w[it * 8 + 1] = v0.y;
            B.w[it * 8 + 2] = v0.z; B.w[it * 8 + 3] = v0.w;
            B.w[it * 8 + 4] = v1.x; B.w[it * 8 + 5] = v1.y;
            B.w[it * 8 + 6] = v1.z; B.w[it * 8 + 7] = v1.w;
        }
    }
}


/* D = A(16x16) * B(16x16) + C (v_mfma_f32_16x16x16_bf16): lane l supplies A
 * row l % 16 and B column l % 16, k-slots 4 (l / 16) .. +3; D as the x32 form */
S2P_DEV s2p_f32x4 mfma16x16x16(s2p_u32x2 a, s2p_u32x2 b, s2p_f32x4 c) {
    typedef __attribute__((ext_vector_type(4))) short s16x4;
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                      __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}

/* multiply one chunk: cg = chunk's first group within the staged window */
/* PIPE (untransposed INT4): a group's MT MFMAs are issued before the
 * previous group's scale FMAs, so one MFMA latency per group is hidden
 * behind the other's work instead of one per column tile exposed (same
 * products, same accumulation order) */
template <int WFMT, int MT, bool TR = false, bool PIPE = false>
S2P_DEV void gv_compute(const GvBuf& B, const GvLds& L, int cg, int gn, int M, int wave, int q,
                        int r, s2p_f32x4 (&acc)[MT], s2p_f32x4 (&corr)[MT]) {
    int mrow[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) mrow[t] = min(t * 16 + r, M - 1);
    if constexpr (WFMT == GEMV_W_INT4 && TR) {
        /* Transposed tile: the staged activations are the A operand (row m)
         * and the dequantised weights of row r the B operand (column n), so
         * lane (q, r) holds D[m = 16t + 4q + i][n = r] and every element of
         * a lane takes the same group scale: one v_fma_mix_f32 per element
         * straight from the loaded f16, no scale staging. */
        static_assert(MT == 1 || !TR, "the transposed tile is one column tile");
        uint32_t kmask = 0x00780078u, kone = 0x3F803F80u;
        asm volatile("" : "+v"(kmask), "+v"(kone));
        /* a block's four activation reads are issued together, ahead of its
         * dequantisation (one LDS latency per 4 groups) */
        const LDS(uint16_t)* xrow = L.x + mrow[0] * L.xs + cg * 32 + q * 8;
#pragma unroll
        for (int it = 0; it < GV_CHG_INT4 / 4; it++) {
            if (it * 4 >= gn) break;
            s2p_u32x4 xa[4];
#pragma unroll
            for (int j = 0; j < 4; j++) xa[j] = *(const LDS(s2p_u32x4)*)(xrow + (it * 4 + j) * 32);
            uint32_t d0 = B.w[it * 4 + 0], d1 = B.w[it * 4 + 1];
            uint32_t d2 = B.w[it * 4 + 2], d3 = B.w[it * 4 + 3];
            xpose4(d0, d1, d2, d3);
            const uint32_t dj[4] = {d0, d1, d2, d3};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int g = it * 4 + j;
                const s2p_u32x4 wv = deq_int4(dj[j], kmask, kone);
                const uint32_t sw = (g & 2) ? B.sa[g >> 2].y : B.sa[g >> 2].x;
                const _Float16 sh = __builtin_bit_cast(
                    _Float16, (uint16_t)((g & 1) ? (sw >> 16) : (sw & 0xFFFFu)));
                const float sf = (float)sh;
                const s2p_f32x4 raw = mfma16x16x32(xa[j], wv, (s2p_f32x4){0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int i = 0; i < 4; i++) acc[0][i] = fmaf(sf, raw[i], acc[0][i]);
            }
            __builtin_amdgcn_sched_barrier(0); /* keep LDS reads from piling up */
        }
        /* bias correction: corr += X (16 cols m x 16 groups) . S (16 groups x
         * 16 rows n), the scales of row r / groups 4q..4q+3 as exact bf16
         * hi + lo (the B operand) */
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
            }
            shi[d] = (hb[0] >> 16) | hb[1];
            slo[d] = lb[0] | (lb[1] << 16);
        }
        const s2p_u32x2 ah = {shi[0], shi[1]};
        const s2p_u32x2 al = {slo[0], slo[1]};
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int p = 0; p < 3; p++) {
                const s2p_u32x2 bx = *(const LDS(s2p_u32x2)*)(L.X3 + (mrow[t] * 3 + p) * L.xg +
                                                         cg + 4 * q);
                corr[t] = mfma16x16x16(bx, ah, corr[t]);
                corr[t] = mfma16x16x16(bx, al, corr[t]);
            }
    } else if constexpr (WFMT == GEMV_W_INT4) {
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
        s2p_f32x4 rp[MT], sp4 = {0.f, 0.f, 0.f, 0.f}; /* PIPE: the pending group */
#pragma unroll
        for (int t = 0; t < MT; t++) rp[t] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
        bool pend = false;
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
                if constexpr (PIPE) {
                    s2p_u32x4 bv[MT];
                    s2p_f32x4 raw[MT];
#pragma unroll
                    for (int t = 0; t < MT; t++)
                        bv[t] = *(const LDS(s2p_u32x4)*)(L.x + mrow[t] * L.xs + (cg + g) * 32 + q * 8);
#pragma unroll
                    for (int t = 0; t < MT; t++)
                        raw[t] = mfma16x16x32(av, bv[t], (s2p_f32x4){0.f, 0.f, 0.f, 0.f});
                    if (pend) {
#pragma unroll
                        for (int t = 0; t < MT; t++)
#pragma unroll
                            for (int i = 0; i < 4; i++) acc[t][i] = fmaf(sp4[i], rp[t][i], acc[t][i]);
                    }
#pragma unroll
                    for (int t = 0; t < MT; t++) rp[t] = raw[t];
                    sp4 = s4;
                    pend = true;
                } else {
#pragma unroll
                    for (int t = 0; t < MT; t++) {
                        const s2p_u32x4 bv =
                            *(const LDS(s2p_u32x4)*)(L.x + mrow[t] * L.xs + (cg + g) * 32 + q * 8);
                        const s2p_f32x4 raw = mfma16x16x32(av, bv, (s2p_f32x4){0.f, 0.f, 0.f, 0.f});
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[t][i] = fmaf(s4[i], raw[i], acc[t][i]);
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0); /* keep LDS reads from piling up */
        }
        if (PIPE && pend) {
#pragma unroll
            for (int t = 0; t < MT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[t][i] = fmaf(sp4[i], rp[t][i], acc[t][i]);
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
    } else if constexpr (WFMT == GEMV_W_BF16) {
#pragma unroll
        for (int g = 0; g < GV_CHG_BF16; g++) {
            if (g >= gn) break;
            const s2p_u32x4 av = {B.w[g * 4 + 0], B.w[g * 4 + 1], B.w[g * 4 + 2], B.w[g * 4 + 3]};
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const s2p_u32x4 bv =
                    *(const LDS(s2p_u32x4)*)(L.x + mrow[t] * L.xs + (cg + g) * 32 + q * 8);
                acc[t] = mfma16x16x32(av, bv, acc[t]);
            }
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

/* last arrival at row block rb: sum the splits in split order and run the
 * epilogue (on 256 threads: thread tid of them).  A thread takes FB groups
 * of four adjacent outputs per round, each split's four partials as one
 * 16-byte agent-scope load (two 8-byte loads), every load of a round in
 * flight before any sum: at 48 rows (FB = 3) a 64-row block takes one round
 * of memory latency, where one output a thread per round took three. */
/* PLAIN: the partials come from an earlier launch (plain 16-byte loads);
 * items base0, base0 + 256 FB, ... of the block go to this thread group
 * (base0 = 0 and step 256 FB: all of them) */
template <int FB, int WFMT = GEMV_W_INT4, bool COH = false, bool PLAIN = false>
__device__ void gv_fixup4(const GemvArgs& a, int rb, uint16_t* Y, int tid, int base0 = 0,
                          int bstep = 256 * FB) {
#pragma clang fp contract(off)
    const int lane = tid & 63;
    const int M = a.M, S = a.splits;
    const size_t stride = (size_t)M * a.nrb * 64;
    const float* part = a.part;
    const bool swiglu = a.epi == GEMV_EPI_SWIGLU;
    /* items: (m, 4 outputs); SWIGLU: 8 gate groups a row (each with its up
     * group 32 later), else 16 groups a row */
    const int per_row = swiglu ? 8 : 16;
    const int items = M * per_row;
    for (int base = base0; base < items; base += bstep) {
        s2p_f32x4 g[FB], u[FB];
        uint16_t yold[FB][4];
#pragma unroll
        for (int j = 0; j < FB; j++) {
            g[j] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
            u[j] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
            const int idx = base + 256 * j + tid;
            const int m = idx / per_row, l4 = (idx % per_row) * 4;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int n = rb * 64 + l4 + e;
                yold[j][e] = !swiglu && idx < items && a.epi == GEMV_EPI_RESID && n < a.N
                                 ? ld_act16<COH>(Y + (size_t)m * a.ldy + n)
                                 : (uint16_t)0;
            }
        }
        /* splits in sets of four, summed in split order */
        auto issue = [&](int k0, s2p_u32x4 (&vg)[FB][4], int off) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < FB; j++) {
                const int idx = base + 256 * j + tid;
                const bool ok = idx < items;
                const int m = idx / per_row, l4 = (idx % per_row) * 4;
                const float* p0 = part + ((size_t)m * a.nrb + rb) * 64 + l4 + off;
#pragma unroll
                for (int k = 0; k < 4; k++)
                    vg[j][k] = !(ok && k0 + k < S) ? (s2p_u32x4){0u, 0u, 0u, 0u}
                               : PLAIN ? *(const s2p_u32x4*)(p0 + (size_t)(k0 + k) * stride)
                                       : coh_ld128(p0 + (size_t)(k0 + k) * stride);
            }
        };
        auto accum = [&](int k0, const s2p_u32x4 (&vg)[FB][4], s2p_f32x4 (&dst)[FB])
            __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < FB; j++)
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    if (k0 + k >= S) break;
                    const s2p_f32x4 f = __builtin_bit_cast(s2p_f32x4, vg[j][k]);
#pragma unroll
                    for (int e = 0; e < 4; e++) dst[j][e] += f[e];
                }
        };
        if (swiglu) {
            /* gate and up partials (32 rows apart), one set at a time */
            for (int k0 = 0; k0 < S; k0 += 4) {
                s2p_u32x4 vg[FB][4], vu[FB][4];
                issue(k0, vg, 0);
                issue(k0, vu, 32);
                accum(k0, vg, g);
                accum(k0, vu, u);
            }
        } else {
            /* the next set's loads in flight while the current one is summed */
            s2p_u32x4 ga[FB][4], gb[FB][4];
            issue(0, ga, 0);
            for (int k0 = 0; k0 < S; k0 += 8) {
                if (k0 + 4 < S) issue(k0 + 4, gb, 0);
                accum(k0, ga, g);
                if (k0 + 4 >= S) break;
                if (k0 + 8 < S) issue(k0 + 8, ga, 0);
                accum(k0 + 4, gb, g);
            }
        }
#pragma unroll
        for (int j = 0; j < FB; j++) {
            const int idx = base + 256 * j + tid;
            const bool ok = idx < items;
            const int m = idx / per_row, l4 = (idx % per_row) * 4;
            float ssq = 0.f;
            /* the item's 4 adjacent outputs: one 8-byte store when all 4
             * exist and the address allows, else one at a time */
            uint16_t ov[4] = {0, 0, 0, 0};
            const int F = a.N >> 1;
            const int n0 = swiglu ? rb * 32 + l4 : rb * 64 + l4;
            const int nlim = swiglu ? F : a.N;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (!ok || n0 + e >= nlim) continue;
                if (swiglu) {
                    float gg = g[j][e], uu = u[j][e];
                    if (WFMT == GEMV_W_INT8) {
                        gg *= ((const float*)a.s)[n0 + e];
                        uu *= ((const float*)a.s)[F + n0 + e];
                    }
                    ov[e] = silu_mul_bf16(f2bf(gg), f2bf(uu));
                    continue;
                }
                float sj = g[j][e];
                if (WFMT == GEMV_W_INT8) sj *= ((const float*)a.s)[n0 + e];
                const uint16_t yb = f2bf(sj);
                if (a.epi == GEMV_EPI_RESID) {
                    const uint16_t xo = f2bf(__fadd_rn(bf2f(yold[j][e]), bf2f(yb)));
                    ov[e] = xo;
                    const float xv = bf2f(xo);
                    ssq += xv * xv;
                } else {
                    ov[e] = yb;
                }
            }
            if (ok) {
                uint16_t* yp = Y + (size_t)m * a.ldy + n0;
                if (n0 + 3 < nlim && ((uintptr_t)yp & 7) == 0) {
                    const uint64_t w = (uint64_t)ov[0] | ((uint64_t)ov[1] << 16) |
                                       ((uint64_t)ov[2] << 32) | ((uint64_t)ov[3] << 48);
                    if (PLAIN) *(uint64_t*)yp = w;
                    else coh_st64(yp, w);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        if (n0 + e >= nlim) break;
                        if (PLAIN) yp[e] = ov[e];
                        else coh_st16(yp + e, ov[e]);
                    }
                }
            }
            if (!swiglu && a.epi == GEMV_EPI_RESID && a.ssq_out) {
                /* a 16-column sum-of-squares block is 4 adjacent lanes (same m:
                 * 16 items a row, rows start at multiples of 16 lanes) */
                ssq += __shfl_xor(ssq, 1, 64);
                ssq += __shfl_xor(ssq, 2, 64);
                if ((lane & 3) == 0 && ok) {
                    float* sp = a.ssq_out + (size_t)(rb * 4 + (l4 >> 4)) * GEMV_MAX_M + m;
                    if (PLAIN) *sp = ssq;
                    else coh_stf(sp, ssq);
                }
            }
        }
    }
}

/* One (row-block stride p of P, K split sp) work unit of the GEMV engine:
 * the body of a k_gemv workgroup, also run by the persistent verify kernel.
 * WIN1: the split's activations fit one LDS window, staged once before the
 * stream; otherwise every (row block, window) segment restages. */
template <int WFMT, int MT, bool WIN1, bool COH>
__device__ void gv_block(const GemvArgs& a, int p, int P, int sp, LDS(unsigned char)* smem,
                         uint16_t* y_override = nullptr, uint64_t* probe = nullptr) {
    /* probe (diagnostics build only): wall clock at the stages of the block */
#ifdef S2P_DIAG
#define GV_PROBE(i)                                                   \
    do {                                                              \
        if (probe && threadIdx.x == 0) probe[i] = wall_clock64();     \
    } while (0)
#else
#define GV_PROBE(i) \
    do {            \
        (void)probe; \
    } while (0)
#endif
    GV_PROBE(0);
    uint16_t* const Y = y_override ? y_override : a.y;
    constexpr int CHG = WFMT == GEMV_W_INT4 ? GV_CHG_INT4 : GV_CHG_INT8; /* groups per chunk */
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int q = lane >> 4, r = lane & 15;
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

    if (!WIN1 && a.xmode == GEMV_X_NORM) {
        /* inverse RMS per row from the producer's per-block sums of squares:
         * lanes take blocks, fixed-order wave reduction */
        for (int m = wave; m < M; m += 4) {
            float s = 0.f;
            for (int b = lane; b < a.ssq_in_blocks; b += 64)
                s += ld_actf<COH>(a.ssq_in + (size_t)b * GEMV_MAX_M + m);
            s = wave_sum_down(s);
            if (lane == 0) L.inv[m] = rsqrt_rule(s / (float)a.K + a.norm_eps);
        }
    }
    GV_PROBE(1);

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
    auto seg_rb = [&](int k) __attribute__((always_inline)) { return p + (k / nwin) * P; };
    auto seg_g0 = [&](int k) { return gb + (k % nwin) * win; };
    auto seg_gn = [&](int k) __attribute__((always_inline)) { return min(win, ge - seg_g0(k)); };
    auto load_at = [&](GvBuf& B, int k, int c) __attribute__((always_inline)) {
        const int rb = seg_rb(k);
        const int nrow = min(gv_row(a, rb, lrow), a.N - 1);
        const int g0 = seg_g0(k) + c * CHG;
        const int gn = min(CHG, seg_g0(k) + seg_gn(k) - g0);
        gv_load<WFMT>(B, a, nrow, g0, gn, q);
    };

    /* ---- end of row block rb: combine, then store or hand off ---- */
    auto finish_rb = [&](int rb) __attribute__((always_inline)) {
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
                    coh_st16(Y + (size_t)m * a.ldy + n, f2bf(v));
                }
            }
            return;
        }
        /* Split-K handoff across the 8 non-coherent XCD L2s: the partials
         * are written through (sc1, the encoding of an agent-scope store; one
         * 16-byte store per lane) and read back with agent-scope atomic
         * loads; each workgroup waits for its partial stores to complete,
         * then signals arrival with an agent-scope acquire-release fetch_add
         * (the memory model's L2 writeback before and invalidate after), so
         * the last arriver's reads are ordered after every split's stores by
         * the model, not only by the completion waits. */
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int m = t * 16 + r;
            if (m >= M) continue;
            float* dst = &a.part[(((size_t)sp * M + m) * a.nrb + rb) * 64 + wave * 16 + q * 4];
            const s2p_f32x4 v4 = {res[t][0], res[t][1], res[t][2], res[t][3]};
            coh_st128(dst, __builtin_bit_cast(s2p_u32x4, v4));
        }
        GV_PROBE(3);
        vm_drain();
        __syncthreads();
        GV_PROBE(4);
        if (tid == 0) {
            /* acquire-release at agent scope: the partials of every split
             * that arrived before are visible to this workgroup's reads */
            const unsigned prev = __hip_atomic_fetch_add(&a.counters[rb], 1u, __ATOMIC_ACQ_REL,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            *L.flag = prev == (unsigned)(a.splits - 1);
        }
        __syncthreads();
        GV_PROBE(5);
        const bool last = *L.flag != 0;
        if (last) {
            gv_fixup4<1, WFMT, COH>(a, rb, Y, threadIdx.x);
            vm_drain();
            GV_PROBE(6);
            if (tid == 0)
                __hip_atomic_store(&a.counters[rb], 0u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads(); /* flag is rewritten at the next block */
    };

    if constexpr (WIN1) {
        /* Flattened (row block, chunk) stream with two named buffers and the
         * next chunk in flight while one is multiplied (no buffer copy for
         * the allocator to coalesce into one register set). */
        const int gn_w = ge - gb;
        const int nch = (gn_w + CHG - 1) / CHG;
        const int T = nseg * nch;
        auto load_t = [&](GvBuf& B, int t) __attribute__((always_inline)) { load_at(B, t / nch, t - (t / nch) * nch); };
        auto step = [&](const GvBuf& B, int t) __attribute__((always_inline)) {
            const int kk = t / nch, cc = t - kk * nch;
            gv_compute<WFMT, MT>(B, L, cc * CHG, min(CHG, gn_w - cc * CHG), M, wave, q, r, acc,
                                 corr);
            if (cc == nch - 1) {
                if (WFMT == GEMV_W_INT8) {
#pragma unroll
                    for (int t2 = 0; t2 < MT; t2++) corr8[t2] += L.xtot[min(t2 * 16 + r, M - 1)];
                }
                finish_rb(seg_rb(kk));
            }
        };
        GvBuf b0, b1;
        load_t(b0, 0); /* the first weight chunk is in flight while staging */
        __syncthreads();
        gv_stage<WFMT, COH>(a, L, gb, gn_w, true);
        __syncthreads();
        GV_PROBE(2);
        /* every path into a step has the same loads outstanding, and no load
         * is issued past the end (the handoff's vmcnt(0) would wait for it) */
        int t = 0;
        for (; t + 2 < T; t += 2) {
            load_t(b1, t + 1);
            step(b0, t);
            load_t(b0, t + 2);
            step(b1, t + 1);
        }
        if (T - t == 2) {
            load_t(b1, t + 1);
            step(b0, t);
            step(b1, t + 1);
        } else {
            step(b0, t);
        }
        return;
    }

    GvBuf cur, nxt;
    load_at(cur, 0, 0);
    for (int k = 0; k < nseg; k++) {
        const int rb = seg_rb(k);
        const int w = k % nwin;
        const int g0 = seg_g0(k), gn_w = seg_gn(k);
        const int nch = (gn_w + CHG - 1) / CHG;
        __syncthreads();
        gv_stage<WFMT, COH>(a, L, g0, gn_w, false);
        __syncthreads();
        const bool last_w = w == nwin - 1;
        for (int c = 0; c < nch; c++) {
            const bool last_c = c == nch - 1;
            const int nk = last_c ? (k + 1 < nseg ? k + 1 : k) : k;
            const int nc = last_c ? (k + 1 < nseg ? 0 : c) : c + 1;
            load_at(nxt, nk, nc);
            gv_compute<WFMT, MT>(cur, L, c * CHG, min(CHG, gn_w - c * CHG), M, wave, q, r, acc,
                                 corr);
            cur = nxt;
        }
        if (WFMT == GEMV_W_INT8) {
#pragma unroll
            for (int t = 0; t < MT; t++) corr8[t] += L.xtot[min(t * 16 + r, M - 1)];
        }
        if (!last_w) continue;
        finish_rb(rb);
    }
}

#undef GV_PROBE

/* ===================================================================== */
/* Whole-K engine (no cross-workgroup handoff).
 *
 * A workgroup of nw = rt * ks waves stays resident and walks tile groups
 * p, p + P, ...: a tile group is rt 16-row tiles (SWIGLU: rt / 2 gate tiles
 * and the matching up tiles), and the ks waves of a tile split K.  The
 * activations are staged in LDS once per workgroup (ks K slices, shared by
 * the rt waves of a slice) and reused by every tile group.  Each wave runs
 * one flattened, double-buffered weight stream over its (tile, K slice)
 * chunks of all its tile groups, so the next group's weights are in flight
 * while a group is reduced: the waves' partial tiles meet in LDS (two
 * buffers, one workgroup barrier per group), are summed in wave order
 * (deterministic) and the epilogue runs.  Nothing but the outputs goes to
 * global memory. */

static __host__ __device__ inline size_t gv3_slice_bytes(int M, int gps, int wfmt) {
    const size_t xs = (size_t)gps * 32 + GV_XPAD;
    const size_t xg = (size_t)gv_round32(gps) + 8;
    size_t b = ((size_t)M * xs * 2 + (size_t)M * 3 * xg * 2 + 15) & ~(size_t)15;
    if (wfmt == GEMV_W_INT8) b += ((size_t)M * 4 + 15) & ~(size_t)15;
    return b;
}
/* slices [ks], INT4 scale staging [nw][16 groups][16 rows] f32, inverse RMS
 * [GEMV_MAX_M], partial tiles [nbuf][nw][MT][64 lanes][4] f32 (two buffers
 * when a workgroup walks more than one tile group) */
static __host__ __device__ inline size_t gv3_lds_bytes(int M, int gps, int wfmt, int ks, int nw,
                                                       int nbuf) {
    const int mt = (M + 15) / 16;
    return (size_t)ks * gv3_slice_bytes(M, gps, wfmt) +
           (wfmt == GEMV_W_INT4 ? (size_t)nw * 1024 : 0) + GEMV_MAX_M * 4 +
           (size_t)nbuf * nw * mt * 1024;
}

/* Loads issued before the weight stream (waits are in issue order, so a
 * load issued after the weights would wait for them too): the producer's
 * sums of squares of row `wave` (blocks lane + 64 i), and rows 0..7 of the
 * wave's first 64 column blocks of its K slice. */
struct Gv3Pre {
    s2p_u32x4 raw[8];
    s2p_u32x4 wn4;
    float ssq[3];
};

template <bool COH>
S2P_DEV void gv3_pre_issue(const GemvArgs& a, Gv3Pre& pre, bool stager, int wave, int lane,
                           int gb, int gn) {
    const int M = a.M;
    const bool norm = a.xmode == GEMV_X_NORM;
    if (norm && wave < M) {
#pragma unroll
        for (int i = 0; i < 3; i++)
            if (lane + 64 * i < a.ssq_in_blocks)
                pre.ssq[i] = ld_actf<COH>(a.ssq_in + (size_t)(lane + 64 * i) * GEMV_MAX_M + wave);
    }
    if (stager && lane < gn * 4) {
        const int k = gb * 32 + lane * 8;
#pragma unroll
        for (int m = 0; m < 8; m++)
            if (m < M) pre.raw[m] = ld_act128<COH>(a.x + (size_t)m * a.ldx + k);
        if (norm) pre.wn4 = *(const s2p_u32x4*)(a.norm_w + k);
    }
}

template <bool COH>
S2P_DEV void st_act16(uint16_t* p, uint16_t v) {
    if constexpr (COH) coh_st16(p, v);
    else *p = v;
}

/* Work geometry of workgroup p of P and of one of its waves. */
struct Gv3Geo {
    int nw, units, tiles, niter;
    int j, sp, gb, gn, nch, T;
};

template <int WFMT>
S2P_DEV Gv3Geo gv3_geo(const GemvArgs& a, int p, int P, int wave) {
    Gv3Geo g;
    const int G = a.K >> 5, ks = a.ks, rt = a.rt;
    const bool swiglu = a.epi == GEMV_EPI_SWIGLU;
    g.nw = rt * ks;
    g.units = swiglu ? rt >> 1 : rt;                       /* output tiles per group */
    g.tiles = swiglu ? (a.N >> 1) >> 4 : (a.N + 15) >> 4;  /* output tiles */
    const int ngroups = (g.tiles + g.units - 1) / g.units;
    g.niter = p < ngroups ? (ngroups - p + P - 1) / P : 0;
    g.j = wave / ks;                                        /* tile of the group */
    g.sp = wave - g.j * ks;                                 /* K slice */
    g.gb = g.sp * a.gps;
    g.gn = min(G, g.gb + a.gps) - g.gb;
    g.nch = (g.gn + gv_chg(WFMT) - 1) / gv_chg(WFMT);
    g.T = g.niter * g.nch;
    return g;
}

/* weight row of lane row r of this wave in tile group tg */
S2P_DEV int gv3_wrow(const GemvArgs& a, const Gv3Geo& g, int tg, int r) {
    int base;
    if (a.epi == GEMV_EPI_SWIGLU) {
        const int h = g.units;
        const int t = tg * h + (g.j < h ? g.j : g.j - h);
        base = (g.j < h ? 0 : a.N >> 1) + t * 16;
    } else {
        base = (tg * g.units + g.j) * 16;
    }
    return min(base + r, a.N - 1);
}

/* INT4 at one column tile runs the transposed tile (gv_compute TR), except
 * in the persistent kernel (NOTR), whose register budget the untransposed
 * tile fits, and in layer launches shaped like it (the test hook that
 * compares the two) */
static __host__ __device__ constexpr bool gv3_tr(int wfmt, int mt, bool notr) {
    return wfmt == GEMV_W_INT4 && mt == 1 && !notr;
}

/* chunk t of the wave's flattened (tile group, chunk) stream */
template <int WFMT, int MT, bool NOTR>
S2P_DEV void gv3_load(GvBuf& B, const GemvArgs& a, const Gv3Geo& g, int p, int P, int t) {
    constexpr int CHG = gv_chg(WFMT);
    const int lane = threadIdx.x & 63;
    const int it = g.nch == 1 ? t : t / g.nch, c = t - it * g.nch;
    gv_load<WFMT, gv3_tr(WFMT, MT, NOTR)>(B, a, gv3_wrow(a, g, p + it * P, lane & 15), g.gb + c * CHG,
                  min(CHG, g.gn - c * CHG), lane >> 4);
}

/* The first weight chunk of workgroup p, issued ahead (the persistent kernel
 * issues it before the barrier that precedes the GEMV). */
template <int WFMT, int MT = 1>
S2P_DEV void gv3_prefetch(const GemvArgs& a, int p, int P, GvBuf& b0, GvBuf& b1) {
    const Gv3Geo g = gv3_geo<WFMT>(a, p, P, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    /* both buffers defined on every path: their old contents are dead */
    if (g.T > 0) {
        gv3_load<WFMT, MT, true>(b0, a, g, p, P, 0);
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) b0.w[i] = 0u;
        b0.s = (s2p_u32x2){0u, 0u};
    }
    if (g.T > 1) {
        gv3_load<WFMT, MT, true>(b1, a, g, p, P, 1);
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) b1.w[i] = 0u;
        b1.s = (s2p_u32x2){0u, 0u};
    }
}

/* PRE: b0 and b1 already hold (or are loading) the first two chunks
 * (gv3_prefetch). */
/* COH: activation loads bypass the L2 (their producer ran in this launch
 * and the L2 was not invalidated since); WT: outputs written through. */
template <int WFMT, int MT, bool COH, bool PRE = false, bool WT = COH, bool NOTR = PRE>
__device__ void gv3_block(const GemvArgs& a, int p, int P, LDS(unsigned char)* smem,
                          uint16_t* Y, GvBuf& b0, GvBuf& b1) {
#pragma clang fp contract(off)
    constexpr int CHG = gv_chg(WFMT);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, r = lane & 15;
    const int M = a.M, ks = a.ks, gps = a.gps;
    const Gv3Geo geo = gv3_geo<WFMT>(a, p, P, wave);
    const int nw = geo.nw, units = geo.units, tiles = geo.tiles, niter = geo.niter;
    if (niter == 0) return; /* uniform over the workgroup */
    const bool swiglu = a.epi == GEMV_EPI_SWIGLU;
    const int F = a.N >> 1;
    const int sp = geo.sp, gb = geo.gb, gn = geo.gn;
    (void)r;
#ifdef S2P_DIAG
    uint64_t* const probe = a.probe ? a.probe + (size_t)blockIdx.x * 8 : nullptr;
#else
    uint64_t* const probe = nullptr; /* stage clocks: diagnostics build only */
#endif
    auto stamp = [&](int i) __attribute__((always_inline)) {
        if (probe && tid == 0) probe[i] = wall_clock64();
    };
    stamp(0);

    /* carve */
    const size_t sb = gv3_slice_bytes(M, gps, WFMT);
    LDS(unsigned char)* slice = smem + (size_t)sp * sb;
    GvLds L;
    L.xs = gps * 32 + GV_XPAD;
    L.xg = gv_round32(gps) + 8;
    L.x = (LDS(uint16_t)*)slice;
    uint32_t off = (uint32_t)M * L.xs * 2;
    L.X3 = (LDS(uint16_t)*)(slice + off);
    off = (off + (uint32_t)M * 3 * L.xg * 2 + 15) & ~15u;
    L.xtot = (LDS(float)*)(slice + off);
    size_t o2 = (size_t)ks * sb;
    L.sc = (LDS(float)*)(smem + o2 + (size_t)wave * 1024);
    if (WFMT == GEMV_W_INT4) o2 += (size_t)nw * 1024;
    L.inv = (LDS(float)*)(smem + o2);
    o2 += GEMV_MAX_M * 4;
    L.flag = nullptr;
    LDS(s2p_f32x4)* red = (LDS(s2p_f32x4)*)(smem + o2);

    const int nch = geo.nch, T = geo.T;
    auto load_t = [&](GvBuf& B, int t) __attribute__((always_inline)) {
        gv3_load<WFMT, MT, NOTR>(B, a, geo, p, P, t);
    };

    Gv3Pre pre;
    gv3_pre_issue<COH>(a, pre, geo.j == 0, wave, lane, gb, gn);
    if constexpr (!PRE) load_t(b0, 0); /* in flight during the staging */
    if (a.xmode == GEMV_X_NORM) {
        /* inverse RMS per row: lanes take the producer's blocks, fixed-order
         * wave reduction */
        for (int m = wave; m < M; m += nw) {
            float s = 0.f;
            if (m == wave && a.ssq_in_blocks <= 192) {
#pragma unroll
                for (int i = 0; i < 3; i++)
                    if (lane + 64 * i < a.ssq_in_blocks) s += pre.ssq[i];
            } else {
                for (int b = lane; b < a.ssq_in_blocks; b += 64)
                    s += ld_actf<COH>(a.ssq_in + (size_t)b * GEMV_MAX_M + m);
            }
            s = wave_sum_down(s);
            if (lane == 0) L.inv[m] = rsqrt_rule(s / (float)a.K + a.norm_eps);
        }
        __syncthreads();
    }
    stamp(1);
    if (geo.j == 0) {
        /* the slice's stager: rows < 8 of the first 64 column blocks from
         * the registers, the rest loaded here */
        const int nb8 = gn * 4;
        const int wnp = gv_round32(gn);
        for (int row = lane >> 5; row < M * 3; row += 2)
            if ((lane & 31) < wnp - gn) L.X3[row * L.xg + gn + (lane & 31)] = 0;
#pragma unroll
        for (int m = 0; m < 8; m++)
            if (m < M) gv_stage_one<WFMT>(a, L, m, lane, lane < nb8, pre.raw[m], pre.wn4);
        for (int bb = 0; bb < nb8; bb += 64) {
            const int b = bb + lane;
            const bool valid = b < nb8;
            const int k = gb * 32 + b * 8;
            s2p_u32x4 wn4 = {0u, 0u, 0u, 0u};
            if (valid && a.xmode == GEMV_X_NORM) wn4 = *(const s2p_u32x4*)(a.norm_w + k);
            for (int m0 = bb == 0 ? 8 : 0; m0 < M; m0 += 4) {
                s2p_u32x4 raw[4];
#pragma unroll
                for (int jj = 0; jj < 4; jj++)
                    raw[jj] = (valid && m0 + jj < M)
                                  ? ld_act128<COH>(a.x + (size_t)(m0 + jj) * a.ldx + k)
                                  : (s2p_u32x4){0u, 0u, 0u, 0u};
#pragma unroll
                for (int jj = 0; jj < 4; jj++)
                    if (m0 + jj < M) gv_stage_one<WFMT>(a, L, m0 + jj, b, valid, raw[jj], wn4);
            }
        }
        if (WFMT == GEMV_W_INT8) {
            wave_lds_sync();
            for (int m = 0; m < M; m++) {
                float s = 0.f;
                for (int g = lane; g < gn; g += 64)
                    s += bf2f(L.X3[(m * 3 + 0) * L.xg + g]) + bf2f(L.X3[(m * 3 + 1) * L.xg + g]) +
                         bf2f(L.X3[(m * 3 + 2) * L.xg + g]);
                s = wave_sum_down(s);
                if (lane == 0) L.xtot[m] = s;
            }
        }
    }
    __syncthreads();
    stamp(2);
    if (probe) { /* diagnostics: weights arrived */
        vm_drain();
        stamp(6);
    }

    s2p_f32x4 acc[MT], corr[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) {
        acc[t] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
        corr[t] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
    }

    /* end of tile group it: partial tile to LDS, barrier, sum + epilogue */
    auto finish = [&](int it) __attribute__((always_inline)) {
        LDS(s2p_f32x4)* rb = red + (size_t)(it & 1) * nw * MT * 64;
#pragma unroll
        for (int t = 0; t < MT; t++) {
            s2p_f32x4 v;
#pragma unroll
            for (int i = 0; i < 4; i++)
                v[i] = WFMT == GEMV_W_INT4   ? 16.0f * acc[t][i] - 24.0f * corr[t][i]
                       : WFMT == GEMV_W_INT8 ? fmaf(-128.0f, L.xtot[min(t * 16 + r, M - 1)],
                                                    acc[t][i])
                                             : acc[t][i];
            rb[(wave * MT + t) * 64 + lane] = v;
            acc[t] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
            corr[t] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
        }
        if (it == 0) stamp(3);
        __syncthreads();
        if (it == 0) stamp(4);
        if constexpr (NOTR) {
            /* output (row rho of unit u, column m): element rho % 4 of lane
             * (rho / 4) * 16 + m % 16, column tile m / 16, of the unit's waves */
            const LDS(float)* rf = (const LDS(float)*)rb;
            const int g = p + it * P;
            auto tsum = [&](int jw, int rho, int m) __attribute__((always_inline)) {
                const int src = ((m >> 4) * 64 + (rho >> 2) * 16 + (m & 15)) * 4 + (rho & 3);
                float v = 0.f;
                for (int s = 0; s < ks; s++) v += rf[(size_t)(jw * ks + s) * MT * 256 + src];
                return v;
            };
            for (int u = 0; u < units; u++)
            for (int base = 0; base < M * 16; base += nw * 64) {
                const int idx = base + tid;
                const int rho = idx & 15, m = idx >> 4;
                const int tile = g * units + u;
                const int n = tile * 16 + rho;
                const bool ok = m < M && tile < tiles;
                if (swiglu) {
                    if (ok) {
                        float gv = tsum(u, rho, m), uv = tsum(units + u, rho, m);
                        if (WFMT == GEMV_W_INT8) {
                            gv *= ((const float*)a.s)[n];
                            uv *= ((const float*)a.s)[F + n];
                        }
                        st_act16<WT>(Y + (size_t)m * a.ldy + n, silu_mul_bf16(f2bf(gv), f2bf(uv)));
                    }
                    continue;
                }
                float ssq = 0.f;
                if (ok && n < a.N) {
                    float v = tsum(u, rho, m);
                    if (WFMT == GEMV_W_INT8) v *= ((const float*)a.s)[n];
                    const uint16_t yb = f2bf(v);
                    uint16_t* yp = Y + (size_t)m * a.ldy + n;
                    if (a.epi == GEMV_EPI_RESID) {
                        const uint16_t xo = f2bf(__fadd_rn(bf2f(ld_act16<COH>(yp)), bf2f(yb)));
                        st_act16<WT>(yp, xo);
                        const float xv = bf2f(xo);
                        ssq = xv * xv;
                    } else {
                        st_act16<WT>(yp, yb);
                    }
                }
                if (a.epi == GEMV_EPI_RESID && a.ssq_out) {
                    const float tot = sum_lanes16(ssq); /* the 16 rows of (tile, m) */
                    if (rho == 0 && ok) coh_stf(a.ssq_out + (size_t)tile * GEMV_MAX_M + m, tot);
                }
            }
        } else {
            /* Unit u (a 16-row output tile; SWIGLU: its gate and up tiles) is
             * reduced by its own waves, lane-locally: a lane sums its elements
             * over the ks K-slice partials in slice order (deterministic), then
             * runs the epilogue.  Element i of lane (q, r) in column tile t is
             * (m, n) = (16t + 4q + i, r) for the transposed INT4 tile, and
             * (16t + r, 4q + i) otherwise.  Transposed: element i is handled by
             * the unit's slice wave i % ks (the per-column sums of squares are
             * per element); otherwise slice wave 0 takes all four. */
            constexpr bool TRN = gv3_tr(WFMT, MT, NOTR);
            const int u = geo.j, sl0 = geo.sp;
            const int tile = (p + it * P) * units + u;
            if (u < units && tile < tiles && (TRN || sl0 == 0)) { /* uniform */
                const int n0 = tile * 16;
                const LDS(float)* rf = (const LDS(float)*)rb;
    #pragma unroll 1
                for (int t = 0; t < MT; t++) {
                    float sq4 = 0.f;
    #pragma unroll
                    for (int i = 0; i < 4; i++) {
                        if (TRN && i % ks != sl0) continue; /* uniform */
                        float v = 0.f, w = 0.f;
                        for (int sl = 0; sl < ks; sl++)
                            v += rf[(((u * ks + sl) * MT + t) * 64 + lane) * 4 + i];
                        if (swiglu)
                            for (int sl = 0; sl < ks; sl++)
                                w += rf[((((units + u) * ks + sl) * MT + t) * 64 + lane) * 4 + i];
                        const int m = TRN ? t * 16 + 4 * q + i : t * 16 + r;
                        const int n = n0 + (TRN ? r : 4 * q + i);
                        const bool ok = m < M;
                        if (swiglu) {
                            if (ok) {
                                float gv = v, uv = w;
                                if (WFMT == GEMV_W_INT8) {
                                    gv *= ((const float*)a.s)[n];
                                    uv *= ((const float*)a.s)[F + n];
                                }
                                st_act16<WT>(Y + (size_t)m * a.ldy + n,
                                             silu_mul_bf16(f2bf(gv), f2bf(uv)));
                            }
                            continue;
                        }
                        float sq = 0.f;
                        if (ok && n < a.N) {
                            if (WFMT == GEMV_W_INT8) v *= ((const float*)a.s)[n];
                            const uint16_t yb = f2bf(v);
                            uint16_t* yp = Y + (size_t)m * a.ldy + n;
                            if (a.epi == GEMV_EPI_RESID) {
                                const uint16_t xo = f2bf(__fadd_rn(bf2f(ld_act16<COH>(yp)), bf2f(yb)));
                                st_act16<WT>(yp, xo);
                                const float xv = bf2f(xo);
                                sq = xv * xv;
                            } else {
                                st_act16<WT>(yp, yb);
                            }
                        }
                        if (a.epi == GEMV_EPI_RESID && a.ssq_out) {
                            if (TRN) {
                                /* over the tile's 16 rows n = r of column m */
                                const float tot = sum_lanes16(sq);
                                if (r == 0 && ok)
                                    coh_stf(a.ssq_out + (size_t)tile * GEMV_MAX_M + m, tot);
                            } else {
                                sq4 += sq;
                            }
                        }
                    }
                    if (!TRN && !swiglu && a.epi == GEMV_EPI_RESID && a.ssq_out) {
                        float tot = sq4;
                        tot += __shfl_xor(tot, 16, 64);
                        tot += __shfl_xor(tot, 32, 64);
                        const int m = t * 16 + r;
                        if (q == 0 && m < M)
                            coh_stf(a.ssq_out + (size_t)tile * GEMV_MAX_M + m, tot);
                    }
                }
            }
        }
    };
    auto step = [&](const GvBuf& B, int t) __attribute__((always_inline)) {
        const int it = nch == 1 ? t : t / nch, c = t - it * nch;
        gv_compute<WFMT, MT, gv3_tr(WFMT, MT, NOTR)>(B, L, c * CHG, min(CHG, gn - c * CHG), M, 0, q, r, acc, corr);
        if (c == nch - 1) finish(it);
    };
    int t = 0;
    if constexpr (!PRE) {
        /* one chunk ahead: b1 is loaded while b0 is multiplied; every path
         * into a step has the same loads outstanding, and no load is issued
         * past the end */
        for (; t + 2 < T; t += 2) {
            load_t(b1, t + 1);
            step(b0, t);
            load_t(b0, t + 2);
            step(b1, t + 1);
        }
        if (T - t == 2) {
            load_t(b1, t + 1);
            step(b0, t);
            step(b1, t + 1);
        } else {
            step(b0, t);
        }
    } else {
    /* b0 holds chunk t and b1 chunk t + 1 (both issued before the barrier):
     * two chunks in flight, every load in the loop unconditional, no load
     * issued past the end */
    for (; t + 3 < T; t += 2) {
        step(b0, t);
        load_t(b0, t + 2);
        step(b1, t + 1);
        load_t(b1, t + 3);
    }
    if (T - t == 3) {
        step(b0, t);
        load_t(b0, t + 2);
        step(b1, t + 1);
        step(b0, t + 2);
    } else if (T - t == 2) {
        step(b0, t);
        step(b1, t + 1);
    } else {
        step(b0, t);
    }
    }
    if (probe) {
        vm_drain();
        stamp(5);
    }
}

#endif