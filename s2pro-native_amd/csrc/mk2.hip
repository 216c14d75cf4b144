/* s2pro MI355X — persistent verify kernel: the K-token verify forward of the
 * 36-layer slow-AR backbone and the lm head in ONE launch (reference
 * run_layer, src/slowar/slowar.c:156-260, and the head projection
 * slowar.c:503-565, restated per row), for plans of at most MK2_MAX_ROWS
 * rows over bf16 session caches with INT4-g32 weights.
 *
 * Why one launch: on this part every dependent kernel costs a few
 * microseconds of dispatch, ramp and drain, and the weight stream of a
 * kernel cannot start before its predecessor ends.  Here the weights do not
 * wait for the activations at all:
 *
 *   - one workgroup per CU (MK2_NWG = 256, co-resident), 8 waves: waves 0..6
 *     compute, wave 7 ("IO wave") moves activations and synchronises;
 *   - the compute waves stream every weight byte through a ring of NSLOT
 *     register slots over the fixed per-layer sequence of their work units
 *     (wqkv | wo | gate_up | w2, then the head): consuming unit k issues the
 *     load of unit k + NSLOT.  The loads are issued from inline asm, so the
 *     compiler does not serialise them behind the activations; every wait is
 *     an explicit vmcnt(2 * (NSLOT - 1)) (the schedule is static: NSLOT - 1
 *     refills of two loads each lie between a unit's load and its use).
 *     Nothing else on those waves issues vector memory loads between
 *     prefetches except the attention phase, whose own (compiler-counted)
 *     waits can only wait longer, never shorter;
 *   - phases depend on each other through flags (one 32-bit word per
 *     producing workgroup or attention unit, each in its own 64-byte line,
 *     holding a per-launch epoch): a consumer polls exactly the producers
 *     it reads (attention: the owners of its kv head's 48 qkv tiles), no
 *     grid-wide barrier.  Outputs are written through (sc1) and read
 *     back with sc1 loads, so no cache maintenance is needed (the 8 XCD L2s
 *     are not coherent with each other inside a kernel);
 *   - every wait is bounded: a timeout sets a sticky error flag and every
 *     later wait returns at once, so the grid always drains.
 *
 * Per unit (one 16-row tile x 4 groups of 32 k, 1152 B): the packed nibbles
 * become bf16 128 + n = 136 + w with one v_and_or_b32 per two weights (the
 * +8 bias is applied at pack time); activations are the MFMA A operand
 * (row m), the weights B (column n), so each lane's four outputs share one
 * group scale, applied by v_fma_mix straight from the f16.  The 136 x (sum
 * of the group's activations) bias is removed exactly inside the MFMA: its
 * C operand is MFMA(x, -136).  Units are tile-major and every wave owns a
 * contiguous unit range, so a wave touches at most two tiles; the waves'
 * per-tile partials meet in LDS and are summed in wave order
 * (deterministic).
 *
 * The RMSNorm (rule roundings, kernels.cu:46-80) is applied to the staged
 * rows in LDS with the inverse RMS from the producer's per-16-column sums of
 * squares; SwiGLU and the residual adds are fused into the reductions. */
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <utility>

#include "coh.h"
#include "common.h"
#include "attn_dev.h"
#include "gemv_dev.h"
#include "mk2_internal.h"
#include "prims_dev.h"

#define NWAVE 8
#define CW 7 /* compute waves */
#define NTH (64 * NWAVE)
#ifndef NSLOT
#define NSLOT 8 /* measured: 8 slots beat 20 and 10 (less queueing in front of the exchanges); 5 is 0.7% slower, 4 within 1% */
#endif
#define LDSP(T) __attribute__((address_space(3))) T

typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef const __attribute__((address_space(1))) s2p_u32x4 G4;

enum { PQ = 0, PO = 1, PG = 2, PD = 3 };

/* Build with -DMK2_TRACE for per-workgroup phase clocks (diagnostics; not
 * in the product build): g_mk2_tr[wg][layer][event], s2p_mk2_trace copies
 * them out. */
#ifdef MK2_TRACE
#define TR_L 40
#define TR_E 32
__device__ uint64_t g_mk2_tr[MK2_NWG][TR_L][TR_E];

#define TRACE(l, e)                                                                    \
    do {                                                                               \
        if ((threadIdx.x & 63) == 0 && (l) < TR_L) g_mk2_tr[blockIdx.x][l][e] = wall_clock64(); \
    } while (0)
#else
#define TRACE(l, e) \
    do {            \
    } while (0)
#endif

/* ---- static geometry of the four layer GEMVs ---- */
constexpr int phT(int P) { return P == PQ ? 384 : P == PO ? 160 : P == PG ? 1216 : 160; } /* 16-row tiles */
constexpr int phNB(int P) { return P == PQ ? 20 : P == PO ? 32 : P == PG ? 20 : 76; }    /* 4-group blocks */
constexpr size_t phOFF(int P) {
    return P == PQ ? 0 : P == PO ? (size_t)MK2_BLK_Q * MK2_BLK
                                 : P == PG ? (size_t)(MK2_BLK_Q + MK2_BLK_O) * MK2_BLK
                                           : (size_t)(MK2_BLK_Q + MK2_BLK_O + MK2_BLK_G) * MK2_BLK;
}
constexpr size_t LAYER_BYTES = (size_t)MK2_LAYER_BLKS * MK2_BLK;
/* units per compute wave at most (gate_up: 15, padded so that the layer
 * sequence tiles the ring), and the per-layer unit sequence */
constexpr int maxu(int P) { return P == PQ ? 6 : P == PO ? 5 : P == PG ? 18 : 11; }
constexpr int LSEQ = 40;
constexpr int seq_base(int P) { return P == PQ ? 0 : P == PO ? 6 : P == PG ? 11 : 29; }
constexpr int seq_phase(int k) { return k < 6 ? PQ : k < 11 ? PO : k < 29 ? PG : PD; }
constexpr int WAITN = 2 * (NSLOT - 1);
static_assert(LSEQ % NSLOT == 0, "the ring must tile the layer sequence");
static_assert(maxu(PQ) + maxu(PO) + maxu(PG) + maxu(PD) == LSEQ, "sequence length");

/* opaque copy: keeps per-unit address arithmetic inside the layer loop
 * (hoisted, it would pin dozens of SGPRs for the whole kernel) */
S2P_DEV int opq(int v) {
    v = __builtin_amdgcn_readfirstlane(v); /* wave-uniform by construction */
    asm volatile("" : "+s"(v));
    return v;
}
/* opaque thread index: lane-dependent addresses of a phase are computed in
 * that phase (hoisted out of the layer loop, they would hold VGPRs across
 * every other phase) */
S2P_DEV int tid_opq() {
    int v = threadIdx.x;
    asm volatile("" : "+v"(v));
    return v;
}

template <typename F, int... I>
S2P_DEV void sfor_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
S2P_DEV void sfor(F&& f) {
    sfor_impl(f, std::make_integer_sequence<int, N>{});
}

/* workgroup wg's 16-row tiles and compute wave cw's units */
struct Geo {
    int t0, np, nt, u0, nu;
};
/* gate_up splits its units 9:8 between waves 0-3 and waves 4-6: a wave
 * 4-6 shares its SIMD with an older wave and runs its loop ~0.7 us slower
 * (at 4 or 5 tiles, 12 or 15 units at most) */
static_assert(CW == 7, "the weighted split is written for seven compute waves");
S2P_DEV int wave_cut(int U, int cw, bool weighted) {
    if (!weighted) return U - (CW - cw) * U / CW; /* uneven shares: the shorter ones to the last waves */
    const int cum = cw <= 4 ? 9 * cw : 36 + 8 * (cw - 4);
    return U * cum / 60;
}
S2P_DEV Geo geo_of(int T, int nb, bool weighted, int wg, int cw) {
    Geo g;
    g.t0 = wg * T / MK2_NWG;
    g.np = (wg + 1) * T / MK2_NWG - g.t0;
    g.nt = g.np;
    const int U = g.nt * nb;
    g.u0 = wave_cut(U, cw, weighted);
    g.nu = wave_cut(U, cw + 1, weighted) - g.u0;
    return g;
}
template <int P>
S2P_DEV Geo geoP(int wg, int cw) {
    return geo_of(phT(P), phNB(P), P == PG, opq(wg), cw);
}
/* a compute wave's packed units: start .. last (contiguous in the packed
 * layout), nu of them; units j >= jb lie in its second local tile */
struct WG {
    int start, last, nu, jb, lt0;
};
S2P_DEV WG wg_of(const Geo& g, int nb, bool pairs) {
    WG w;
    const int tp0 = pairs ? 2 * g.t0 : g.t0;
    w.nu = g.nu;
    w.start = g.nu > 0 ? tp0 * nb + g.u0 : 0;
    w.last = g.nu > 0 ? w.start + g.nu - 1 : 0;
    w.lt0 = g.u0 / nb;
    w.jb = nb - (g.u0 - w.lt0 * nb);
    return w;
}

/* ---- register slots ---- */
struct Slot {
    s2p_u32x4 w;
    u32x2 s;
};
S2P_DEV void slot_issue(Slot& S, const uint8_t* p, uint32_t vw, uint32_t vs) {
    asm volatile("global_load_dwordx4 %0, %1, %2 nt ; SLOTLOAD" : "=a"(S.w) : "v"(vw), "s"(p) : "memory");
    asm volatile("global_load_dwordx2 %0, %1, %2 nt ; SLOTLOAD" : "=a"(S.s) : "v"(vs), "s"(p) : "memory");
}
template <int N>
S2P_DEV void slot_wait(Slot& S) {
    asm volatile("s_waitcnt vmcnt(%2) ; SLOTWAIT %0 %1" : "+a"(S.w), "+a"(S.s) : "n"(N) : "memory");
}
S2P_DEV void unit_issue(Slot& S, const uint8_t* blk, int start, int last, int u) {
    const uint8_t* p = blk + (size_t)min(opq(start) + u, opq(last)) * MK2_BLK;
    const uint32_t lane = threadIdx.x & 63;
    slot_issue(S, p, 16 * lane, 1024 + 8 * (lane & 15));
}

struct Ctx {
    WG w[4];      /* per layer phase */
    WG hw;        /* head */
    int head_t0, head_nt;
};

/* refill the slot of sequence position K (layer l) with position K + NSLOT:
 * a unit of the same or the next layer, or past the last layer a head unit */
template <int K>
S2P_DEV void refill(Slot (&S)[NSLOT], const Mk2Args& A, int l, const Ctx& C) {
    constexpr int k2 = K + NSLOT;
    constexpr int kk = k2 % LSEQ;
    constexpr int tp = seq_phase(kk);
    constexpr int tu = kk - seq_base(tp);
    const int tl = l + k2 / LSEQ;
    /* one issue point (a branch would merge the asm outputs through copies
     * of registers whose loads are still in flight): selects only.  Past the
     * last layer the position is head unit kk. */
    const bool hd = tl >= A.n_layers;
    const uint8_t* b = hd ? A.hpack : A.wpack + (size_t)tl * LAYER_BYTES + phOFF(tp);
    const int st = hd ? C.hw.start : C.w[tp].start;
    const int la = hd ? C.hw.last : C.w[tp].last;
    unit_issue(S[K % NSLOT], b, st, la, hd ? kk : tu);
}

S2P_DEV s2p_f32x4 mfma32(s2p_u32x4 a, s2p_u32x4 b, s2p_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(s2p_bf16x8, a),
                                                   __builtin_bit_cast(s2p_bf16x8, b), c, 0, 0, 0);
}

/* one unit: 4 groups of the slot against the staged rows at xa (lane (q, r)
 * reads row min(r, M - 1); rows >= M of the MFMA output are never used),
 * the code bias of each group from the table at nb (lane's rows 4q..4q+3,
 * q taken mod 2: rows >= 8 are never used).  All LDS reads first, then four
 * independent MFMAs. */
S2P_DEV s2p_f32x4 unit_mul(const Slot& S, const LDSP(uint16_t)* xa, const LDSP(float)* nb, uint32_t mask,
                           uint32_t one) {
#pragma clang fp contract(off)
    s2p_u32x4 ag[4];
    s2p_f32x4 bias[4];
#pragma unroll
    for (int gg = 0; gg < 4; gg++) {
        ag[gg] = *(const LDSP(s2p_u32x4)*)(xa + gg * 32);
        bias[gg] = *(const LDSP(s2p_f32x4)*)(nb + gg * 8);
    }
    const uint32_t wd[4] = {S.w.x, S.w.y, S.w.z, S.w.w};
    s2p_f32x4 D[4];
#pragma unroll
    for (int gg = 0; gg < 4; gg++) {
        const uint32_t d = wd[gg];
        s2p_u32x4 wv;
        wv.x = (d & mask) | one;
        wv.y = ((d >> 4) & mask) | one;
        wv.z = ((d >> 8) & mask) | one;
        wv.w = ((d >> 12) & mask) | one;
        D[gg] = mfma32(ag[gg], wv, bias[gg]);
    }
    s2p_f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int gg = 0; gg < 4; gg++) {
        const uint32_t sw = gg < 2 ? S.s.x : S.s.y;
        const _Float16 sh =
            __builtin_bit_cast(_Float16, (uint16_t)((gg & 1) ? (sw >> 16) : (sw & 0xFFFFu)));
        const float sf = (float)sh;
#pragma unroll
        for (int i = 0; i < 4; i++) t[i] = fmaf(sf, D[gg][i], t[i]);
    }
    return t;
}

/* ---- LDS carve-up (bytes) ----
 * layer GEMVs: staged rows [M][XRS(K)] bf16 at 0 (w2 at M = 6: 117.1 KB),
 *              partials [tile][cw][M][16] f32 at L_PART (6 tiles: 16 KB);
 * head:        staged rows at 0 (31.1 KB), partials at L_HPART (39 tiles:
 *              105 KB);
 * attention:   its own carve-up from 0 (< 100 KB);
 * small state from L_INV up (all phases). */
#define L_XS 0
/* staged row stride (elements): K + 32 puts consecutive rows 16 banks apart,
 * so the units' 16-byte row reads (lane (q, r): row r, offset 16 q bytes)
 * hit distinct banks for rows 0..3 */
constexpr int XRS(int K) { return K + 32; }
#define L_PART (117 * 1024)
#define L_HPART (32 * 1024)
#define L_INV (140 * 1024)       /* [M] inverse RMS */
#define L_OUTB (L_INV + 256)     /* [M][96] bf16 outputs of the workgroup's tiles */
#define L_XOLD (L_OUTB + 1280)   /* [M][16] bf16 residual before the add */
#define L_SSQO (L_XOLD + 256)    /* [M][16] f32 sums of squares of the new residual */
#define L_FLAG (L_SSQO + 512)    /* [16] int broadcast words */
#define L_NW (L_FLAG + 64)       /* (5120 B) weighted outputs, their sums, next-norm weights: */
#define L_OUTW L_NW              /*   [M][96] bf16 bf16(new residual x next norm weight) */
#define L_HS (L_NW + 1280)       /*   [M][8] f32 per-tile sums of L_OUTW (w2/wo) or of h (gate_up) */
#define L_NWT (L_NW + 1536)      /*   [96] bf16 next-norm weights of the workgroup's columns */
#define L_BIAS (L_NW + 5120)     /* [NB][4 groups][8 rows] f32: -136 x the group's row sums */
#define L_TOTAL (L_BIAS + 76 * 4 * 8 * 4)
static_assert(MK2_MAX_ROWS * XRS(9728) * 2 <= L_PART && L_PART + 608 * 8 * 4 <= L_INV && MK2_MAX_ROWS * XRS(2560) * 2 <= L_HPART &&
                  L_TOTAL <= 160 * 1024,
              "LDS carve-up");

/* ---- shared (all waves) pieces of a GEMV phase ----
 * The RMSNorm is split between producer and consumer: the producer of a
 * residual tile also writes bf16(x * w) with the weight of the norm that
 * follows, and the per-16-column sums of those values; the consumer stages
 * the weighted rows as they are, builds the code-bias table from the sums,
 * and scales its dot products by the row's inverse RMS in the reduction.
 * (The reference rounds x * inv * w to bf16 before the GEMV, kernels.cu:
 * 46-80; here x * w is rounded and inv applied to the f32 dot product:
 * one rounding of the same product, at another point.) */

/* sum of the waves' partials of local tile lt, element (m, n) */
S2P_DEV float tile_sum(const LDSP(float)* part, int lt, int m, int n, int M) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < CW; w++) s += part[((lt * CW + w) * M + m) * 16 + n];
    return s;
}

/* reduce + epilogue into the LDS output rows (all waves) */
template <int P>
S2P_DEV void reduce_phase(LDSP(unsigned char)* smem, int M, int wg) {
#pragma clang fp contract(off)
    const LDSP(float)* part = (const LDSP(float)*)(smem + L_PART);
    const LDSP(uint16_t)* xold = (const LDSP(uint16_t)*)(smem + L_XOLD);
    const LDSP(float)* inv = (const LDSP(float)*)(smem + L_INV);
    const LDSP(uint16_t)* nwt = (const LDSP(uint16_t)*)(smem + L_NWT);
    LDSP(uint16_t)* outb = (LDSP(uint16_t)*)(smem + L_OUTB);
    LDSP(uint16_t)* outw = (LDSP(uint16_t)*)(smem + L_OUTW);
    LDSP(float)* ssqo = (LDSP(float)*)(smem + L_SSQO);
    LDSP(float)* hs = (LDSP(float)*)(smem + L_HS);
    const Geo g0 = geoP<P>(wg, 0);
    if constexpr (P == PG) {
        /* tile k holds gate rows (n < 8) and up rows (n >= 8) of h columns
         * 8 (t0 + k) + n; per tile and row the sum of its 8 h values */
        const int ncol = g0.np * 8;
        LDSP(float)* ts = ssqo; /* [M][8] tile sums (free in this phase) */
        for (int i = threadIdx.x; i < ncol * M; i += NTH) {
            const int n = i & 7, rest = i >> 3;
            const int m = rest % M, k = rest / M;
            const float iv = inv[m];
            const uint16_t o = silu_mul_bf16(f2bf(__fmul_rn(iv, tile_sum(part, k, m, n, M))),
                                             f2bf(__fmul_rn(iv, tile_sum(part, k, m, n + 8, M))));
            outb[m * 96 + k * 8 + n] = o;
            float t = bf2f(o); /* 8 aligned lanes: quads, then the other quad of the half-row */
            t += dpp_f<0xB1>(t);
            t += dpp_f<0x4E>(t);
            t += dpp_f<0x141>(t);
            if (n == 0) ts[m * 8 + k] = t;
        }
        __syncthreads();
        /* the w2 code-bias terms: for each 32-column group of h that meets
         * this workgroup's columns, -136 x the sum of its tile sums here */
        const int gf = g0.t0 / 4, ng = (g0.t0 + g0.np - 1) / 4 - gf + 1;
        if ((int)threadIdx.x < M * ng) {
            const int m = threadIdx.x % M, gi = threadIdx.x / M;
            float t = 0.f;
            for (int k = max(0, 4 * (gf + gi) - g0.t0); k < min(g0.np, 4 * (gf + gi + 1) - g0.t0); k++) t += ts[m * 8 + k];
            hs[m * 8 + gi] = -136.f * t;
        }
        __syncthreads();
        return;
    }
    const int ncol = g0.np * 16;
    for (int i = threadIdx.x; i < ncol * M; i += NTH) {
        const int n = i & 15, rest = i >> 4;
        const int m = rest % M, k = rest / M;
        const int c = k * 16 + n;
        uint16_t o;
        if (P == PO || P == PD) {
            o = f2bf(__fadd_rn(bf2f(xold[m * 16 + c]), bf2f(f2bf(tile_sum(part, k, m, n, M)))));
            const float v = bf2f(o);
            const float t = sum_lanes16(v * v); /* the tile's sum of squares of the new residual */
            if (n == 0) ssqo[m * 16 + k] = t;
            const uint16_t xw = f2bf(__fmul_rn(v, bf2f(nwt[c])));
            outw[m * 96 + c] = xw;
            const float tw = sum_lanes16(bf2f(xw)); /* and of its weighted values: a code-bias term */
            if (n == 0) hs[m * 8 + k] = -136.f * tw;
        } else {
            o = f2bf(__fmul_rn(inv[m], tile_sum(part, k, m, n, M)));
        }
        outb[m * 96 + c] = o;
    }
    __syncthreads();
}

/* compute waves: one GEMV phase over the ring */
template <int P>
S2P_DEV void c_gemv(Slot (&S)[NSLOT], const Mk2Args& A, int l, int cw, const Ctx& C,
                    LDSP(unsigned char)* smem, int M) {
    constexpr int NU = maxu(P), NB = phNB(P), RS = XRS(NB * 128);
    /* opaque per phase: the unit addresses below are recomputed in every
     * layer instead of being hoisted into dozens of live registers */
    WG w = C.w[P];
    w.start = opq(w.start);
    w.nu = opq(w.nu);
    w.jb = opq(w.jb);
    const int lane = threadIdx.x & 63, q = lane >> 4, r = lane & 15;
    const LDSP(uint16_t)* xs = (const LDSP(uint16_t)*)(smem + L_XS) + min(r, M - 1) * RS + q * 8;
    const LDSP(float)* nbt = (const LDSP(float)*)(smem + L_BIAS) + 4 * (q & 1);
    uint32_t mask = 0x000F000Fu, one = 0x43004300u;
    asm volatile("" : "+v"(mask), "+v"(one));
    /* partials [lt][cw][m][16]: the wave's first local tile is written when
     * its units cross into the second (at j == jb), the last one at the end */
    LDSP(float)* part = (LDSP(float)*)(smem + L_PART);
    auto put = [&](int lt, const s2p_f32x4& v) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = 4 * q + i;
            if (m < M) part[((lt * CW + cw) * M + m) * 16 + r] = v[i];
        }
    };
    s2p_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#ifdef MK2_TRACE
    uint64_t tw = 0, tr = 0;
    if (cw == 0) TRACE(l, P == PD ? 30 : 17 + P);
#endif
    sfor<NU>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        constexpr int K = seq_base(P) + j;
#ifdef MK2_TRACE
        const uint64_t t0 = wall_clock64();
        slot_wait<WAITN>(S[K % NSLOT]);
        asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(mask) : "a"(S[K % NSLOT].s.x)); /* make the wait observable */
        mask = (mask & 0u) | 0x000F000Fu;
        tw += wall_clock64() - t0 + (__builtin_amdgcn_readfirstlane(mask) & 0u);
#else
        slot_wait<WAITN>(S[K % NSLOT]);
#endif
        if (j < w.nu) {
            if (j == w.jb) {
                put(w.lt0, acc);
                acc = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
            }
            const int b = (w.start + j) % NB;
            acc += unit_mul(S[K % NSLOT], xs + b * 128, nbt + b * 32, mask, one);
        }
#ifdef MK2_TRACE
        __builtin_amdgcn_sched_barrier(0);
        const uint64_t t1 = wall_clock64();
        refill<K>(S, A, l, C);
        asm volatile("s_nop 0" ::: "memory");
        tr += wall_clock64() - t1;
#else
        refill<K>(S, A, l, C);
#endif
        __builtin_amdgcn_sched_barrier(0);
    });
#ifdef MK2_TRACE
    if (cw == 0 && (threadIdx.x & 63) == 0 && l < TR_L) g_mk2_tr[blockIdx.x][l][26 + P] = tw;
    if (P == PG && cw == 0 && (threadIdx.x & 63) == 0 && l < TR_L) g_mk2_tr[blockIdx.x][l][31] = tr;
#endif
    /* the last touched tile, then zeros for the workgroup's tiles this wave
     * did not touch */
    const int ntouch = w.nu == 0 ? 0 : (w.nu > w.jb ? 2 : 1);
    if (ntouch > 0) put(w.lt0 + ntouch - 1, acc);
    const Geo g = geoP<P>(blockIdx.x, cw);
    for (int lt = 0; lt < g.nt; lt++)
        if (lt < w.lt0 || lt >= w.lt0 + ntouch) put(lt, (s2p_f32x4){0.f, 0.f, 0.f, 0.f});
}

/* ---- flags ---- */
/* distinct per (launch, layer, kind) and never 0 (the flags' initial value) */
S2P_DEV uint32_t flag_val(uint32_t epoch, int l, int kind) {
    return epoch * 2048u + (uint32_t)((l + 2) * 8 + kind);
}
/* flag i of a kind: word (i / 2) MK2_FSTR + i % 2, two producers per 64-byte
 * line (a hop probe over 256 workgroups: one flag per line 2.9 us, two per
 * line polled with one 8-byte load 1.95 us, sixteen per line 3.7 us) */
S2P_DEV uint32_t* flag_at(const Mk2Args& A, int kind, int i) {
    return A.flags + kind + (i >> 1) * MK2_FSTR + (i & 1);
}

/* one wave: wait until the flags of up to three ranges [i0, i0 + n) all read
 * want, one poll over all of them at a time: one 8-byte load per flag pair
 * (fewer than 64 * NLD pairs in total).  (Deeper polling, several polls in
 * flight, measured slower: the extra reads of the flag lines delay the
 * producers more than they shorten the detection.) */
template <int NLD>
S2P_DEV void flags_poll(const Mk2Args& A, int kind, int ia, int na, int ib, int nb, int ic, int nc,
                        uint32_t want) {
    const int lane = threadIdx.x & 63;
    if (coh_ld32(A.err)) return;
    const int pa = na ? ((ia + na - 1) >> 1) - (ia >> 1) + 1 : 0;
    const int pb = nb ? ((ib + nb - 1) >> 1) - (ib >> 1) + 1 : 0;
    const int pc = nc ? ((ic + nc - 1) >> 1) - (ic >> 1) + 1 : 0;
    const int n = pa + pb + pc; /* < 64 * NLD: slot n reads the error word */
    const uint64_t* ptr[NLD];
    bool lo[NLD], hi[NLD], errw[NLD];
#pragma unroll
    for (int j = 0; j < NLD; j++) {
        const int e = lane + 64 * j;
        int i0 = ia, i1 = ia + na, p = (ia >> 1) + e;
        if (e >= pa) { i0 = ib; i1 = ib + nb; p = (ib >> 1) + (e - pa); }
        if (e >= pa + pb) { i0 = ic; i1 = ic + nc; p = (ic >> 1) + (e - pa - pb); }
        const bool in = e < n;
        lo[j] = in && 2 * p >= i0 && 2 * p < i1;
        hi[j] = in && 2 * p + 1 >= i0 && 2 * p + 1 < i1;
        errw[j] = e == n;
        ptr[j] = e == n ? (const uint64_t*)A.err : (const uint64_t*)flag_at(A, kind, in ? 2 * p : 0);
    }
    for (unsigned spins = 0; spins < A.spin_limit; spins++) {
        uint64_t r[NLD];
#pragma unroll
        for (int j = 0; j < NLD; j++) r[j] = coh_ld64(ptr[j]);
        bool o = true, er = false;
#pragma unroll
        for (int j = 0; j < NLD; j++) {
            o = o && (!lo[j] || (uint32_t)r[j] == want) && (!hi[j] || (uint32_t)(r[j] >> 32) == want);
            er = er || (errw[j] && (uint32_t)r[j] != 0u);
        }
        if (__any(er) || __all(o)) return;
        __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) __hip_atomic_store(A.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
S2P_DEV void flags_wait3(const Mk2Args& A, int kind, int ia, int na, int ib, int nb, int ic, int nc,
                         uint32_t want) {
    const int n = (na + nb + nc) / 2 + 3; /* pairs, at most */
    if (n < 64) flags_poll<1>(A, kind, ia, na, ib, nb, ic, nc, want);
    else if (n < 192) flags_poll<3>(A, kind, ia, na, ib, nb, ic, nc, want);
    else
        for (int c = 0; c < na; c += 1024) /* one range of 378 flags or more */
            flags_poll<9>(A, kind, ia + c, min(1024, na - c), 0, 0, 0, 0, want);
}
S2P_DEV void flags_wait(const Mk2Args& A, int kind, int i0, int n, uint32_t want) {
    flags_wait3(A, kind, i0, n, 0, 0, 0, 0, want);
}
/* one wave: publish flags f[i0 .. i0 + n) = val once this wave's stores completed */
S2P_DEV void flags_set(const Mk2Args& A, int kind, int i0, int n, uint32_t val) {
    vm_drain();
    const int lane = threadIdx.x & 63;
    for (int i = lane; i < n; i += 64) coh_st32(flag_at(A, kind, i0 + i), val);
}

/* ---- IO wave pieces of a GEMV phase ---- */
/* stage M rows of K activations (sc1 loads straight to LDS) and the code-bias
 * table from the producers' terms gs ([block][8 rows]: per 32 columns, or when
 * half two terms per 32 columns, summed in pairs: per 16 columns for the
 * residual, per producing workgroup for h); NORM: the rows' inverse RMS; RESID:
 * the residual's old values of this workgroup's tiles and the next norm's
 * weights of its columns (nwn) */
template <int K, bool NORM, bool RESID, bool HALF>
S2P_DEV void io_stage(const Mk2Args& A, const uint16_t* src, const float* gs, const uint16_t* nwn,
                      int M, LDSP(unsigned char)* smem, int t0, int np) {
    const int lane = threadIdx.x & 63;
    constexpr int RS = XRS(K), NG = K / 32;
    LDSP(uint16_t)* xs = (LDSP(uint16_t)*)(smem + L_XS);
    for (int m = 0; m < M; m++)
#pragma unroll 4
        for (int c = 0; c < K / 512; c++)
            __builtin_amdgcn_global_load_lds((const void*)(src + (size_t)m * K + c * 512 + lane * 8),
                                             (LDSP(void)*)(xs + m * RS + c * 512), 16, 0, 16);
    /* the bias terms straight into LDS, 1 KB per load: into the table, or
     * (HALF) into the partials' space, free until the GEMV */
    LDSP(float)* tb = (LDSP(float)*)(smem + L_BIAS);
    LDSP(float)* gsr = HALF ? (LDSP(float)*)(smem + L_PART) : tb;
    {
        constexpr int tot = (HALF ? 2 : 1) * NG * 8 * 4;
#pragma unroll 4
        for (int c = 0; c * 1024 < tot; c++)
            __builtin_amdgcn_global_load_lds((const void*)((const char*)gs + min(c * 1024 + lane * 16, tot - 16)),
                                             (LDSP(void)*)((LDSP(unsigned char)*)gsr + c * 1024), 16, 0, 16);
    }
    if (NORM) {
        /* inverse RMS from the [M][160] per-16-column sums of squares */
        s2p_u32x4 v[MK2_MAX_ROWS];
#pragma unroll
        for (int m = 0; m < MK2_MAX_ROWS; m++)
            v[m] = (m < M && lane < 40) ? coh_ld128(A.ssq + m * 160 + lane * 4)
                                        : (s2p_u32x4){0u, 0u, 0u, 0u};
        LDSP(float)* inv = (LDSP(float)*)(smem + L_INV);
#pragma unroll
        for (int m = 0; m < MK2_MAX_ROWS; m++) {
            if (m >= M) break;
            float s = (__uint_as_float(v[m].x) + __uint_as_float(v[m].y)) +
                      (__uint_as_float(v[m].z) + __uint_as_float(v[m].w));
            s = wave_sum_down(s);
            if (lane == 0) inv[m] = rsqrt_rule(s / 2560.0f + A.eps);
        }
    }
    if (RESID && np > 0) {
        /* (np <= 1 here) 4-byte loads straight to LDS, lane l at + 4 l: the
         * tile's old residual [M][16] and its next-norm weights [16] */
        if (lane < 8 * M)
            __builtin_amdgcn_global_load_lds((const void*)(A.x + (size_t)(lane >> 3) * 2560 + t0 * 16 + 2 * (lane & 7)),
                                             (LDSP(void)*)(smem + L_XOLD), 4, 0, 16);
        if (lane < 8)
            __builtin_amdgcn_global_load_lds((const void*)(nwn + t0 * 16 + 2 * lane), (LDSP(void)*)(smem + L_NWT), 4, 0, 0);
    }
    vm_drain();
}

/* all waves, after the staging barrier (HALF inputs): table[group][row] =
 * the sum of the group's two 16-column terms, 4 rows per thread; then a
 * barrier */
template <int K>
S2P_DEV void bias_pairs(LDSP(unsigned char)* smem) {
    constexpr int NG = K / 32;
    const LDSP(s2p_f32x4)* r4 = (const LDSP(s2p_f32x4)*)(smem + L_PART);
    LDSP(s2p_f32x4)* t4 = (LDSP(s2p_f32x4)*)(smem + L_BIAS);
    for (int j = threadIdx.x; j < NG * 2; j += NTH) {
        const int g2 = j >> 1, h = j & 1;
        t4[j] = r4[4 * g2 + h] + r4[4 * g2 + 2 + h];
    }
    __syncthreads();
}

/* write the workgroup's output columns [t0 * 16, (t0 + np) * 16) of M rows
 * (and, for the residual, the tiles' sums of squares), then the flags */
S2P_DEV void io_store(const Mk2Args& A, LDSP(unsigned char)* smem, uint16_t* dst, int ldd,
                      int t0, int np, int M, bool resid, float* gs, int kind, uint32_t val, int l,
                      bool half = false) {
    const int lane = threadIdx.x & 63;
    const LDSP(uint16_t)* outb = (const LDSP(uint16_t)*)(smem + L_OUTB);
    const LDSP(uint16_t)* outw = (const LDSP(uint16_t)*)(smem + L_OUTW);
    const int tw = half ? 8 : 16; /* columns per tile (gate_up: 8 h columns) */
    const int nch = np * tw / 8;  /* 16-byte chunks per row */
#ifdef MK2_TRACE
    const int trk = kind == MK2_F_Q ? 0 : kind == MK2_F_O ? 1 : kind == MK2_F_G ? 2 : 3;
    uint64_t tst0 = wall_clock64();
#endif
    for (int i = lane; i < M * nch; i += 64) {
        const int m = i / nch, c = i - m * nch;
        coh_st128(dst + (size_t)m * ldd + t0 * tw + c * 8, *(const LDSP(s2p_u32x4)*)(outb + m * 96 + c * 8));
        if (resid)
            coh_st128(A.xw + (size_t)m * 2560 + t0 * 16 + c * 8, *(const LDSP(s2p_u32x4)*)(outw + m * 96 + c * 8));
    }
    if (resid && np > 0 && lane < M)
        coh_stf(A.ssq + lane * 160 + t0, ((const LDSP(float)*)(smem + L_SSQO))[lane * 16]);
    if (gs && half) { /* h: [32-column group][part][row], part 1 if the group began in an earlier workgroup */
        const int gf = t0 / 4, ng = (t0 + np - 1) / 4 - gf + 1;
        for (int i = lane; i < M * ng; i += 64) {
            const int m = i % M, gi = i / M, g = gf + gi;
            coh_stf(gs + (2 * g + (4 * g >= t0 ? 0 : 1)) * 8 + m, ((const LDSP(float)*)(smem + L_HS))[m * 8 + gi]);
        }
    } else if (gs) /* the tiles' code-bias terms, [tile][row] */
        for (int i = lane; i < M * np; i += 64) {
            const int m = i / np, k = i - m * np;
            coh_stf(gs + (t0 + k) * 8 + m, ((const LDSP(float)*)(smem + L_HS))[m * 8 + k]);
        }
#ifdef MK2_TRACE
    vm_drain();
    if (lane == 0 && l == 18) {
        g_mk2_tr[blockIdx.x][39][trk * 3 + 0] = tst0;
        g_mk2_tr[blockIdx.x][39][trk * 3 + 1] = wall_clock64();
    }
#endif
    flags_set(A, kind, blockIdx.x, 1, val); /* one flag per workgroup, tiles or none */
}

/* ---- attention: one (segment, kv head, 128-position split) unit per
 * workgroup, all 8 waves.  Every global read of the phase is the IO wave's
 * (direct-to-LDS loads): the unit's old K/V rows (before waiting for this
 * step's qkv tiles), the raw q / k / v vectors of its items, their RoPE rows
 * and the visibility masks; the compute waves work from LDS only.  qk-norm +
 * RoPE of the unit's q vectors and new K rows use the rule arithmetic of
 * prims_dev.h; new K/V rows are appended to the cache by the split that
 * holds them.  Wave w owns positions 16w..16w+15 of the split for the
 * scores and dims 16w..16w+15 of the output for PV.  Every split writes its
 * partial (m, l, O), waits until all splits of its (segment, kv head) have
 * arrived, and merges its share of the outputs. */
#define A_SQ 0                     /* [32][128] bf16 roped q vectors, chunk k of row v at slot k ^ (v & 15) */
#define A_SK (8 * 1024)            /* [128][128] bf16 K: chunk k of row t at slot k ^ (t & 15) */
#define A_SV (40 * 1024)           /* [128][128] bf16 V, SVX swizzle */
#define A_SP (72 * 1024)           /* P hi [32][136] bf16 */
#define A_SPL (81 * 1024)          /* P lo [32][136] bf16 */
#define A_SM (90 * 1024)           /* [32 q][8 waves] f32 row maxima */
#define A_SL (91 * 1024)           /* [32 q][8 waves] f32 row sums */
#define A_SO (92 * 1024)           /* [32][128] f32 O */
#define A_RAW (108 * 1024)         /* raw items: q vectors [32][128] bf16, then new slots [8][k, v][128] */
#define A_ROPE (123 * 1024)        /* items [30][128] f32 (cos, sin) of the item's row */
#define A_VIS (138 * 1024)         /* [8] u64 visibility masks of the segment's rows */
#define A_SEG (A_VIS + 64)         /* the segment record */
#define A_NW (A_VIS + 256)         /* q-norm then k-norm weights [2][128] bf16 */
#define A_PST 136
/* INT8 caches: the split's old rows as loaded (free until the scores) */
#define A_R8K A_SP                 /* [128][128] int8 K codes */
#define A_R8V (A_SP + 16 * 1024)   /* [128][128] int8 V codes */
#define A_R8KS (A_SP + 32 * 1024)  /* [128][4] f16 K group scales */
#define A_R8VS (A_SP + 33 * 1024)  /* [128][4] f16 V group scales */
/* INT8 caches, kept through the unit in the GEMV bias table's space (free
 * during attention): every row's group scales as f32, and the new slots'
 * codes and scales as appended */
#define A_KS8 L_BIAS               /* [128][4] f32 */
#define A_VS8 (L_BIAS + 2048)      /* [128][4] f32 */
#define A_NEW8 (L_BIAS + 4096)     /* [8 slots][K, V][128] int8 */
#define A_NEW8S (L_BIAS + 6144)    /* [8 slots][K, V][4] f16 */
#define SVX(t, d) ((t) * 128 + ((((d) >> 3) ^ (((t) >> 2) & 6)) << 3) + ((d) & 7))
#define SKX(t, ch) ((t) * 128 + (((ch) ^ ((t) & 15)) << 3))
static_assert(A_NW + 512 <= L_INV && sizeof(S2pAttnSeg) <= 192, "attention LDS overlaps the shared state");
static_assert(A_R8VS + 1024 <= A_RAW && A_NEW8S + 128 <= L_TOTAL, "INT8 attention LDS");

/* Quantise elements (lane, lane + 64) of one 128-wide K or V row as the
 * INT8 / INT4 append does (reference kernels.cu:541-579, this build's
 * s2pk_kv_append8): per 32-element group, scale = f16(max|x| / QMAX), code =
 * rint(x / scale) clamped to +-QMAX (127 / 7).  Returns the two codes; lanes 0 and 32
 * write the group scales of elements lane and lane + 64 (groups lane / 32
 * and 2 + lane / 32) into hs[4]. */
template <int QMAX>
S2P_DEV void q8_row(float x0, float x1, int lane, int* c0, int* c1, LDSP(uint16_t)* hs) {
#pragma clang fp contract(off)
    const float xs[2] = {x0, x1};
    int cs[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        float a = fabsf(xs[h]);
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
        const uint16_t hv = f2h(__fdiv_rn(a, (float)QMAX));
        const float sc = h2f(hv);
        int q = sc > 0.f ? (int)rintf(__fdiv_rn(xs[h], sc)) : 0;
        cs[h] = max(-QMAX, min(QMAX, q));
        if ((lane & 31) == 0) hs[2 * h + (lane >> 5)] = hv;
    }
    *c0 = cs[0];
    *c1 = cs[1];
}

/* direct-to-LDS 16-byte load of lane's chunk (LDS base is wave-uniform:
 * lane l lands at base + 16 l) */
S2P_DEV void dma16(const void* g, LDSP(void)* base, bool coherent) {
    if (coherent) __builtin_amdgcn_global_load_lds(g, base, 16, 0, 16);
    else __builtin_amdgcn_global_load_lds(g, base, 16, 0, 0);
}

template <bool IO, int KVB>
S2P_DEV void attn_unit(const Mk2Args& A, int l, int seg, int kvh, int sp, uint32_t epoch,
                       LDSP(unsigned char)* smem) {
#pragma clang fp contract(off)
    const int tidx = tid_opq();
    const int lane = tidx & 63, wave = tidx >> 6;
    const int qq = lane >> 4, c = lane & 15;
    constexpr bool io = IO;
#ifdef MK2_TRACE
#define ATRACE(e)                                                                                  \
    do {                                                                                           \
        asm volatile("; ATRACE %0 IO %1" ::"n"(e), "n"((int)IO));                                   \
        if (l == 18 && lane == 0) g_mk2_tr[blockIdx.x][37 + ((e) >> 2)][wave * 4 + ((e) & 3)] = wall_clock64(); \
    } while (0)
#else
#define ATRACE(e) \
    do {          \
    } while (0)
#endif
    ATRACE(0);
    LDSP(uint16_t)* s_q = (LDSP(uint16_t)*)(smem + A_SQ);
    LDSP(uint16_t)* s_k = (LDSP(uint16_t)*)(smem + A_SK);
    LDSP(uint16_t)* s_v = (LDSP(uint16_t)*)(smem + A_SV);
    LDSP(uint16_t)* s_p = (LDSP(uint16_t)*)(smem + A_SP);
    LDSP(uint16_t)* s_pl = (LDSP(uint16_t)*)(smem + A_SPL);
    LDSP(float)* s_m = (LDSP(float)*)(smem + A_SM);
    LDSP(float)* s_l = (LDSP(float)*)(smem + A_SL);
    LDSP(float)* s_o = (LDSP(float)*)(smem + A_SO);
    LDSP(uint16_t)* s_raw = (LDSP(uint16_t)*)(smem + A_RAW);
    LDSP(float)* s_rope = (LDSP(float)*)(smem + A_ROPE);
    LDSP(uint64_t)* s_vis = (LDSP(uint64_t)*)(smem + A_VIS);
    LDSP(uint32_t)* s_seg = (LDSP(uint32_t)*)(smem + A_SEG); /* the segment record's words */
    LDSP(uint16_t)* s_nw = (LDSP(uint16_t)*)(smem + A_NW);
    const int ns = A.nsplit;

    /* 1. IO wave: the segment record, the split's old K/V rows (independent
     * of this step's outputs), then the unit's qkv tiles, its items' raw
     * vectors, RoPE rows and visibility masks */
    if (io) {
        const S2pAttnSeg g = A.segs[seg];
        const uint16_t* kvb = (const uint16_t*)g.kv + (size_t)l * A.plan.layer_stride;
        const uint16_t* kp = kvb + (size_t)kvh * A.plan.max_seq * 128;
        const uint16_t* vp = kvb + (size_t)(8 + kvh) * A.plan.max_seq * 128;
        const int p0 = sp * A.split_pos, p1 = min(p0 + A.split_pos, g.span);
        const int oend = min(p1, g.L);
        if (KVB != 16 && oend > p0) {
            /* INT8 / INT4: codes (EL = 128 / 64 B a row) and group scales
             * (8 B a row) of K and V, rows past the old range clamped (their
             * LDS rows are overwritten by the new slots or zeroed) */
            constexpr int EL = KVB == 8 ? 128 : 64, RPL = 1024 / EL; /* rows a 1 KB load */
            const size_t pk = ((size_t)l * 16 + kvh) * A.plan.max_seq, pv = pk + (size_t)8 * A.plan.max_seq;
            const int8_t* cb = (const int8_t*)g.kv;
            const uint16_t* sb = (const uint16_t*)A.plan.kvs[g.sess];
            for (int i = 0; i < 128 / RPL; i++) {
                const int pos = min(p0 + RPL * i + lane / (EL / 16), oend - 1);
                const int off = 16 * (lane % (EL / 16));
                dma16(cb + (pk + pos) * EL + off, (LDSP(void)*)(smem + A_R8K + i * 1024), false);
                dma16(cb + (pv + pos) * EL + off, (LDSP(void)*)(smem + A_R8V + i * 1024), false);
            }
            const int pr = min(p0 + 2 * lane, oend - 1); /* rows 2 lane, 2 lane + 1 */
            dma16(sb + (pk + pr) * 4, (LDSP(void)*)(smem + A_R8KS), false);
            dma16(sb + (pv + pr) * 4, (LDSP(void)*)(smem + A_R8VS), false);
        } else if (oend > p0) {
            for (int i = 0; i < 32; i++) { /* rows 4i .. 4i + 3 */
                const int t = 4 * i + (lane >> 4);
                const int pos = min(p0 + t, oend - 1);
                dma16(kp + (size_t)pos * 128 + 8 * ((lane & 15) ^ (t & 15)), (LDSP(void)*)(s_k + 4 * i * 128), false);
                dma16(vp + (size_t)pos * 128 + 8 * ((lane & 15) ^ ((t >> 2) & 6)), (LDSP(void)*)(s_v + 4 * i * 128), false);
            }
        }
        if (lane < (int)(sizeof(S2pAttnSeg) / 4)) s_seg[lane] = ((const uint32_t*)(A.segs + seg))[lane];
        /* q-norm and k-norm weights are adjacent: 512 B */
        if (lane < 32) dma16(A.norms + (size_t)l * MK2_NORM_STRIDE + MK2_NORM_Q + 8 * lane, (LDSP(void)*)s_nw, false);
        const uint32_t want = flag_val(epoch, l, MK2_F_Q);
        /* the workgroups that own the kv head's 32 q, 8 k and 8 v tiles (tile t
         * of the 384 is owned by workgroup ((t + 1) 256 - 1) / 384) */
        auto own = [](int t) { return ((t + 1) * MK2_NWG - 1) / 384; };
        const int qa = own(32 * kvh), ka = own(256 + 8 * kvh), va = own(320 + 8 * kvh);
        flags_wait3(A, MK2_F_Q, qa, own(32 * kvh + 31) - qa + 1, ka, own(263 + 8 * kvh) - ka + 1, va,
                    own(327 + 8 * kvh) - va + 1, want);
        const int s0 = max(p0, g.L), nq = g.nrows * 4, nnew = max(0, p1 - s0);
        /* q items: the row's 4 q heads of kv head kvh are 1 KB contiguous */
        for (int rl = 0; rl < g.nrows; rl++) {
            const int row = g.row0 + rl;
            dma16(A.qkv + (size_t)row * 6144 + 512 * kvh + 8 * lane, (LDSP(void)*)(s_raw + 4 * rl * 128), true);
        }
        /* new-slot items: k head then v head (32 lanes) */
        for (int j = 0; j < nnew; j++) {
            const int row = g.first + (s0 + j - g.L);
            const uint16_t* src = A.qkv + (size_t)row * 6144 + (lane < 16 ? 4096 + 128 * kvh + 8 * lane
                                                                          : 5120 + 128 * kvh + 8 * (lane - 16));
            if (lane < 32) dma16(src, (LDSP(void)*)(s_raw + 32 * 128 + j * 256), true);
        }
        /* RoPE rows of the items (512 B each, 32 lanes) */
        for (int it = 0; it < nq + nnew; it++) {
            const int row = it < nq ? g.row0 + (it >> 2) : g.first + (s0 + (it - nq) - g.L);
            if (lane < 32) dma16(A.rope_tab + (size_t)row * 128 + 4 * lane, (LDSP(void)*)(s_rope + it * 128), false);
        }
        if (lane < g.nrows) s_vis[lane] = A.plan.vis[g.row0 + lane];
        vm_drain();
    }
    ATRACE(1);
    __syncthreads();
    ATRACE(2);
    S2pAttnSeg g;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(S2pAttnSeg) / 4); i++) ((uint32_t*)&g)[i] = s_seg[i];
    const int L = g.L, span = g.span, nrows = g.nrows;
    const int p0 = sp * A.split_pos, p1 = min(p0 + A.split_pos, span);
    const int s0 = max(p0, L);       /* new positions [s0, p1) */
    const int nq = nrows * 4, nnew = max(0, p1 - s0), nit = nq + nnew;
    TRACE(l, 20);
    /* 2. items: qk-norm + RoPE from LDS into the q rows and the K / V
     * tiles; rows past the split's end zeroed (their P is 0, stale LDS could
     * be Inf / NaN).  INT8 caches: the old rows' codes into the tiles as
     * bf16 (exact) and their scales as f32; the new slots quantised as the
     * append does, their codes into the tiles and the append staging. */
    constexpr bool q8 = KVB != 16;
    constexpr int EL8 = KVB == 8 ? 128 : 64; /* code bytes a row */
    LDSP(float)* s_ks8 = (LDSP(float)*)(smem + A_KS8);
    LDSP(float)* s_vs8 = (LDSP(float)*)(smem + A_VS8);
    if (q8) {
        const int nold = max(0, min(p1, L) - p0);
        for (int i = tidx; i < nold * 32; i += NTH) { /* 8 codes of K or V a thread */
            const int isv = i >= nold * 16, j = isv ? i - nold * 16 : i;
            const int tr = j >> 4, ch = j & 15;
            uint32_t o[4];
            if constexpr (KVB == 8) {
                const uint64_t w = *(const LDSP(uint64_t)*)(smem + (isv ? A_R8V : A_R8K) + tr * 128 + ch * 8);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float lo = (float)(int8_t)(w >> (16 * e)), hi = (float)(int8_t)(w >> (16 * e + 8));
                    o[e] = (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
                }
            } else {
                /* element 2b in the low nibble of byte b, both nibbles the
                 * two's complement the append writes */
                const uint32_t w = *(const LDSP(uint32_t)*)(smem + (isv ? A_R8V : A_R8K) + tr * 64 + ch * 4);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int8_t by = (int8_t)(w >> (8 * e));
                    const float lo = (float)((int8_t)(by << 4) >> 4), hi = (float)(by >> 4);
                    o[e] = (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
                }
            }
            const s2p_u32x4 v = {o[0], o[1], o[2], o[3]};
            if (isv) *(LDSP(s2p_u32x4)*)(s_v + SVX(tr, 8 * ch)) = v;
            else *(LDSP(s2p_u32x4)*)(s_k + SKX(tr, ch)) = v;
        }
        /* scales: the old rows', zeros past the split's end; the new slots'
         * rows [nold, p1 - p0) are written by their items below */
        const int nend = max(p1, p0) - p0;
        for (int i = tidx; i < 128 * 8; i += NTH) {
            const int isv = i >= 512, j = i & 511, tr = j >> 2;
            if (tr < nold) (isv ? s_vs8 : s_ks8)[j] = h2f(((const LDSP(uint16_t)*)(smem + (isv ? A_R8VS : A_R8KS)))[j]);
            else if (tr >= nend) (isv ? s_vs8 : s_ks8)[j] = 0.f;
        }
    }
    for (int it = wave; it < nit; it += NWAVE) {
        const bool isq = it < nq;
        const LDSP(uint16_t)* rv = isq ? s_raw + it * 128 : s_raw + 32 * 128 + (it - nq) * 256;
        const LDSP(float)* rp = s_rope + it * 128;
        const float v0 = bf2f(rv[lane]), v1 = bf2f(rv[lane + 64]);
        const float c0 = rp[(lane >> 1) * 2], sn0 = rp[(lane >> 1) * 2 + 1];
        const float c1 = rp[((lane + 64) >> 1) * 2], sn1 = rp[((lane + 64) >> 1) * 2 + 1];
        const LDSP(uint16_t)* nw = s_nw + (isq ? 0 : 128);
        float o0, o1;
        qkrope_math(v0, v1, nw[lane], nw[lane + 64], c0, sn0, c1, sn1, A.eps, lane, &o0, &o1);
        const uint16_t b0 = f2bf(o0), b1 = f2bf(o1);
        if (isq) {
            s_q[SKX(it, lane >> 3) + (lane & 7)] = b0;
            s_q[SKX(it, (lane + 64) >> 3) + (lane & 7)] = b1;
        } else if (q8) {
            const int t = s0 + (it - nq) - p0, j = it - nq;
            LDSP(int8_t)* nc = (LDSP(int8_t)*)(smem + A_NEW8) + j * 256;
            LDSP(uint16_t)* ns8 = (LDSP(uint16_t)*)(smem + A_NEW8S) + j * 8;
            constexpr int QMAX = KVB == 8 ? 127 : 7;
            /* codes as stored: INT8 one a byte; INT4 element 2b in the low
             * nibble of byte b (the pair's high element from the next lane) */
            auto put = [&](LDSP(int8_t)* row, int e, int c) __attribute__((always_inline)) {
                if constexpr (KVB == 8) {
                    row[e] = (int8_t)c;
                } else {
                    const int hi = __shfl_down(c, 1, 64);
                    if ((e & 1) == 0) row[e >> 1] = (int8_t)((c & 0xF) | ((hi & 0xF) << 4));
                }
            };
            int c0, c1;
            q8_row<QMAX>(bf2f(b0), bf2f(b1), lane, &c0, &c1, ns8);
            s_k[SKX(t, lane >> 3) + (lane & 7)] = f2bf((float)c0);
            s_k[SKX(t, (lane + 64) >> 3) + (lane & 7)] = f2bf((float)c1);
            put(nc, lane, c0);
            put(nc, lane + 64, c1);
            q8_row<QMAX>(bf2f(rv[128 + lane]), bf2f(rv[128 + lane + 64]), lane, &c0, &c1, ns8 + 4);
            s_v[SVX(t, lane)] = f2bf((float)c0);
            s_v[SVX(t, lane + 64)] = f2bf((float)c1);
            put(nc + 128, lane, c0);
            put(nc + 128, lane + 64, c1);
            if (lane < 4) {
                s_ks8[t * 4 + lane] = h2f(ns8[lane]);
                s_vs8[t * 4 + lane] = h2f(ns8[4 + lane]);
            }
        } else {
            const int t = s0 + (it - nq) - p0;
            s_k[SKX(t, lane >> 3) + (lane & 7)] = b0;
            s_k[SKX(t, (lane + 64) >> 3) + (lane & 7)] = b1;
            s_v[SVX(t, lane)] = rv[128 + lane];
            s_v[SVX(t, lane + 64)] = rv[128 + lane + 64];
        }
    }
    for (int i = tidx; i < (p0 + 128 - max(p1, p0)) * 128; i += NTH) {
        const int t = max(p1, p0) - p0 + (i >> 7), d = i & 127;
        s_v[SVX(t, d)] = 0;
        s_k[t * 128 + d] = 0;
    }
    ATRACE(3);
    __syncthreads();
    ATRACE(4);
    if (io) {
        /* the new slots' K / V rows appended to the cache; split 0 keeps an
         * inspection copy of the roped q rows */
        uint16_t* kvb = (uint16_t*)g.kv + (size_t)l * A.plan.layer_stride;
        if (q8) {
            /* codes (16 B a lane: K then V, EL8 / 16 lanes each) and scales
             * (the next two lanes) */
            constexpr int CL = EL8 / 16;
            const size_t pk = ((size_t)l * 16 + kvh) * A.plan.max_seq, pv = pk + (size_t)8 * A.plan.max_seq;
            int8_t* cb = (int8_t*)g.kv;
            uint16_t* sb = (uint16_t*)A.plan.kvs[g.sess];
            for (int j = 0; j < nnew; j++) {
                const size_t slot = (size_t)(s0 + j);
                if (lane < 2 * CL) {
                    const bool isv = lane >= CL;
                    const int c16 = 16 * (lane % CL);
                    coh_st128(cb + ((isv ? pv : pk) + slot) * EL8 + c16,
                              *(const LDSP(s2p_u32x4)*)(smem + A_NEW8 + j * 256 + (isv ? 128 : 0) + c16));
                } else if (lane < 2 * CL + 2) {
                    const bool isv = lane == 2 * CL + 1;
                    coh_st64(sb + ((isv ? pv : pk) + slot) * 4,
                             *(const LDSP(uint64_t)*)(smem + A_NEW8S + j * 16 + (isv ? 8 : 0)));
                }
            }
        }
        for (int j = 0; j < (q8 ? 0 : nnew); j++) {
            const int slot = s0 + j, t = slot - p0;
            if (lane < 32) {
                const int ch = lane & 15;
                const bool isv = lane >= 16;
                const s2p_u32x4 v = *(const LDSP(s2p_u32x4)*)(isv ? s_v + SVX(t, 8 * ch) : s_k + SKX(t, ch));
                coh_st128(kvb + ((size_t)((isv ? 8 : 0) + kvh) * A.plan.max_seq + slot) * 128 + 8 * ch, v);
            }
        }
        if (sp == 0)
            for (int idx = lane; idx < nq * 16; idx += 64) {
                const int qv = idx >> 4, ch = idx & 15;
                coh_st128(A.q + (size_t)(g.row0 + (qv >> 2)) * 4096 + (4 * kvh + (qv & 3)) * 128 + 8 * ch,
                          *(const LDSP(s2p_u32x4)*)(s_q + SKX(qv, ch)));
            }
    }
    TRACE(l, 21);
    /* 3. scores of this wave's 16 positions for the 32 q vectors */
    const int t = 16 * wave + c, pos = p0 + t;
    const float scale = 0.08838834764831845f;
    s2p_f32x4 sc[2];
    if (q8) {
        /* one MFMA per 32-dim group (the codes are exact in bf16), then the
         * group scales of the position in group order:
         * s = sum_g ks[t][g] (q_g . k_g) (kernels.cu:625-700's order) */
        const s2p_f32x4 kst = *(const LDSP(s2p_f32x4)*)(s_ks8 + t * 4);
#pragma unroll
        for (int qt = 0; qt < 2; qt++) {
            s2p_f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ch = 0; ch < 4; ch++) {
                const s2p_u32x4 qa = *(const LDSP(s2p_u32x4)*)(s_q + SKX(16 * qt + c, 4 * ch + qq));
                const s2p_u32x4 kb = *(const LDSP(s2p_u32x4)*)(s_k + SKX(t, 4 * ch + qq));
                const s2p_f32x4 pg = mfma16x16x32(qa, kb, (s2p_f32x4){0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int i = 0; i < 4; i++) d[i] = fmaf(pg[i], kst[ch], d[i]);
            }
            sc[qt] = d;
        }
    } else {
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        s2p_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ch = 0; ch < 4; ch++) {
            const s2p_u32x4 qa = *(const LDSP(s2p_u32x4)*)(s_q + SKX(16 * qt + c, 4 * ch + qq));
            const s2p_u32x4 kb = *(const LDSP(s2p_u32x4)*)(s_k + SKX(t, 4 * ch + qq));
            acc = mfma16x16x32(qa, kb, acc);
        }
        sc[qt] = acc;
    }
    }
    /* visibility: lane (qq, c) element i is q vector 16 qt + 4 qq + i (row
     * 4 qt + qq), position pos */
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        const int rl = 4 * qt + qq;
        bool vis = rl < nrows && pos < p1;
        if (vis && pos >= L) {
            const int bb = pos - L;
            vis = bb < 64 && ((s_vis[rl] >> bb) & 1ull);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float tv = vis ? sc[qt][i] * scale : -INFINITY;
            sc[qt][i] = tv;
            const float mx = max16(tv);
            if (c == 0) s_m[(16 * qt + 4 * qq + i) * 8 + wave] = mx;
        }
    }
    ATRACE(5);
    __syncthreads();
    /* 4. P = e^(s - M) (M over the split), row sums, P as bf16 hi + lo */
#pragma unroll
    for (int qt = 0; qt < 2; qt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int qv = 16 * qt + 4 * qq + i;
            const s2p_f32x4 ma = *(const LDSP(s2p_f32x4)*)(s_m + qv * 8);
            const s2p_f32x4 mb = *(const LDSP(s2p_f32x4)*)(s_m + qv * 8 + 4);
            const float M = fmaxf(fmaxf(fmaxf(ma[0], ma[1]), fmaxf(ma[2], ma[3])),
                                  fmaxf(fmaxf(mb[0], mb[1]), fmaxf(mb[2], mb[3])));
            const float Ms = M == -INFINITY ? 0.f : M;
            const float p = __expf(sc[qt][i] - Ms);
            const float ps = sum16(p);
            if (c == 0) s_l[qv * 8 + wave] = ps;
            const uint16_t h = f2bf(p);
            s_p[qv * A_PST + t] = h;
            s_pl[qv * A_PST + t] = f2bf(p - bf2f(h));
        }
    ATRACE(6);
    __syncthreads();
    /* 5. O[:, 16 wave .. 16 wave + 15] = P V */
    s2p_f32x4 o[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int ch = 0; ch < 4; ch++) {
        uint32_t bw[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int tt = 32 * ch + 8 * qq + 2 * e;
            bw[e] = (uint32_t)s_v[SVX(tt, 16 * wave + c)] | ((uint32_t)s_v[SVX(tt + 1, 16 * wave + c)] << 16);
        }
        const s2p_u32x4 bv = {bw[0], bw[1], bw[2], bw[3]};
#pragma unroll
        for (int qt = 0; qt < 2; qt++) {
            s2p_u32x4 pa = *(const LDSP(s2p_u32x4)*)(s_p + (16 * qt + c) * A_PST + 32 * ch + 8 * qq);
            s2p_u32x4 pl = *(const LDSP(s2p_u32x4)*)(s_pl + (16 * qt + c) * A_PST + 32 * ch + 8 * qq);
            if (q8) {
                /* the V group scale rides in P: p' = (hi + lo) x vs[t][g] for this
                 * wave's output group g = wave / 2, split again into bf16 hi + lo */
                const int g8 = wave >> 1, t0 = 32 * ch + 8 * qq;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t hw = pa[e], lw = pl[e];
                    float v2[2];
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const float pv = bf2f((uint16_t)(hw >> (16 * h))) + bf2f((uint16_t)(lw >> (16 * h)));
                        v2[h] = pv * s_vs8[(t0 + 2 * e + h) * 4 + g8];
                    }
                    const uint16_t h0 = f2bf(v2[0]), h1 = f2bf(v2[1]);
                    pa[e] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                    pl[e] = (uint32_t)f2bf(v2[0] - bf2f(h0)) | ((uint32_t)f2bf(v2[1] - bf2f(h1)) << 16);
                }
            }
            o[qt] = mfma16x16x32(pl, bv, o[qt]);
            o[qt] = mfma16x16x32(pa, bv, o[qt]);
        }
    }
#pragma unroll
    for (int qt = 0; qt < 2; qt++)
#pragma unroll
        for (int i = 0; i < 4; i++) s_o[(16 * qt + 4 * qq + i) * 128 + 16 * wave + c] = o[qt][i];
    ATRACE(7);
    __syncthreads();
    TRACE(l, 22);
    /* this unit's share of the (segment, kv head)'s outputs: q vectors
     * [v0s, v1s) x 128 dims */
    const int per = (nq + ns - 1) / ns;
    const int v0s = min(nq, sp * per), v1s = min(nq, v0s + per), nv = v1s - v0s;
    float* part = A.attn_part;
    float* po = part + (size_t)A.rows * 32 * ns * 2;
    auto pidx = [&](int qv, int s2) __attribute__((always_inline)) {
        return ((size_t)(g.row0 + (qv >> 2)) * 32 + 4 * kvh + (qv & 3)) * ns + s2;
    };
    if (ns > 1) {
        /* 6. partial (m, l, O) of this split; arrival; wait for every split;
         * the share's partials of all splits into LDS (K / V tiles' space) */
        LDSP(float)* s_po = (LDSP(float)*)(smem + A_SK); /* [nv][ns][128] */
        LDSP(float)* s_ml = (LDSP(float)*)(smem + A_SP); /* [nv][ns][2] */
        if (io) {
            for (int idx = lane; idx < nq * 32; idx += 64) {
                const int qv = idx >> 5, d4 = (idx & 31) * 4;
                const size_t pi = pidx(qv, sp);
                coh_st128(po + pi * 128 + d4, *(const LDSP(s2p_u32x4)*)(s_o + qv * 128 + d4));
                if (d4 == 0) {
                    const s2p_f32x4 ma = *(const LDSP(s2p_f32x4)*)(s_m + qv * 8);
                    const s2p_f32x4 mb = *(const LDSP(s2p_f32x4)*)(s_m + qv * 8 + 4);
                    const s2p_f32x4 la = *(const LDSP(s2p_f32x4)*)(s_l + qv * 8);
                    const s2p_f32x4 lb = *(const LDSP(s2p_f32x4)*)(s_l + qv * 8 + 4);
                    const float Mx = fmaxf(fmaxf(fmaxf(ma[0], ma[1]), fmaxf(ma[2], ma[3])),
                                           fmaxf(fmaxf(mb[0], mb[1]), fmaxf(mb[2], mb[3])));
                    const float ls = ((la[0] + la[1]) + (la[2] + la[3])) + ((lb[0] + lb[1]) + (lb[2] + lb[3]));
                    coh_st64(part + pi * 2, (uint64_t)__float_as_uint(Mx) | ((uint64_t)__float_as_uint(ls) << 32));
                }
            }
            /* this split's partials are written: its flag, then every split's
             * flag of the group (the flags' own lines; an arrival counter's
             * atomics queue up on one line) */
            const int u0 = (seg * 8 + kvh) * ns;
            flags_set(A, MK2_F_PART, u0 + sp, 1, flag_val(epoch, l, MK2_F_PART));
            flags_wait(A, MK2_F_PART, u0, ns, flag_val(epoch, l, MK2_F_PART));
            /* every split's partial of the share: 512 B each, two per load */
            for (int i = 0; 2 * i < nv * ns; i++) {
                const int e = 2 * i + (lane >> 5);
                const int k = e / ns, s2 = e - k * ns;
                const int ec = min(e, nv * ns - 1), kc = ec / ns, sc2 = ec - kc * ns;
                (void)k;
                (void)s2;
                dma16(po + pidx(v0s + kc, sc2) * 128 + 4 * (lane & 31), (LDSP(void)*)(s_po + 2 * i * 128), true);
            }
            for (int e = lane; e < nv * ns; e += 64) {
                const int k = e / ns, s2 = e - k * ns;
                const uint64_t ml = coh_ld64(part + pidx(v0s + k, s2) * 2);
                s_ml[2 * e] = __uint_as_float((uint32_t)ml);
                s_ml[2 * e + 1] = __uint_as_float((uint32_t)(ml >> 32));
            }
            vm_drain();
        }
        __syncthreads();
        TRACE(l, 23);
        /* 7. merge of the share: split weights e^(m_s - M), denominators */
        LDSP(float)* s_w = (LDSP(float)*)(smem + A_SPL); /* [nv][ns] weights, [nv] denominators */
        if (tidx < nv) {
            const int k = tidx;
            float Mx = -INFINITY;
#pragma unroll 8
            for (int s2 = 0; s2 < ns; s2++) Mx = fmaxf(Mx, s_ml[2 * (k * ns + s2)]);
            const float Ms = Mx == -INFINITY ? 0.f : Mx;
            float lsum = 0.f;
#pragma unroll 8
            for (int s2 = 0; s2 < ns; s2++) {
                const float w = __expf(s_ml[2 * (k * ns + s2)] - Ms);
                lsum = fmaf(s_ml[2 * (k * ns + s2) + 1], w, lsum);
                s_w[k * ns + s2] = w;
            }
            s_w[nv * ns + k] = lsum;
        }
        __syncthreads();
        for (int idx = tidx; idx < nv * 128; idx += NTH) {
            const int k = idx >> 7, d = idx & 127;
            float acc = 0.f;
            /* unrolled: the loads of a batch issue together, the sum keeps split order */
#pragma unroll 8
            for (int s2 = 0; s2 < ns; s2++) acc = fmaf(s_po[(k * ns + s2) * 128 + d], s_w[k * ns + s2], acc);
            s_o[(v0s + k) * 128 + d] = acc / s_w[nv * ns + k];
        }
        __syncthreads();
    } else {
        /* one split: normalise in place */
        for (int idx = tidx; idx < nq * 128; idx += NTH) {
            const int qv = idx >> 7;
            const s2p_f32x4 la = *(const LDSP(s2p_f32x4)*)(s_l + qv * 8);
            const s2p_f32x4 lb = *(const LDSP(s2p_f32x4)*)(s_l + qv * 8 + 4);
            const float ls = ((la[0] + la[1]) + (la[2] + la[3])) + ((lb[0] + lb[1]) + (lb[2] + lb[3]));
            s_o[idx] = s_o[idx] / ls;
        }
        __syncthreads();
    }
    if (io) {
        /* the share of attn[row][(4 kvh + g) * 128 + d] as bf16, then its flag */
        for (int idx = lane; idx < nv * 16; idx += 64) {
            const int qv = v0s + (idx >> 4), d = (idx & 15) * 8;
            const LDSP(float)* sv = s_o + qv * 128 + d;
            s2p_u32x4 ob;
            ob.x = (uint32_t)f2bf(sv[0]) | ((uint32_t)f2bf(sv[1]) << 16);
            ob.y = (uint32_t)f2bf(sv[2]) | ((uint32_t)f2bf(sv[3]) << 16);
            ob.z = (uint32_t)f2bf(sv[4]) | ((uint32_t)f2bf(sv[5]) << 16);
            ob.w = (uint32_t)f2bf(sv[6]) | ((uint32_t)f2bf(sv[7]) << 16);
            coh_st128(A.attn + (size_t)(g.row0 + (qv >> 2)) * 4096 + (4 * kvh + (qv & 3)) * 128 + d, ob);
            /* the sum of each 32 columns (4 lanes) of the stored values: the
             * wo code bias */
            float t = ((bf2f_lo(ob.x) + bf2f_hi(ob.x)) + (bf2f_lo(ob.y) + bf2f_hi(ob.y))) +
                      ((bf2f_lo(ob.z) + bf2f_hi(ob.z)) + (bf2f_lo(ob.w) + bf2f_hi(ob.w)));
            t += __shfl_xor(t, 1, 64);
            t += __shfl_xor(t, 2, 64);
            if ((idx & 3) == 0) /* [32-column block][row] */
                coh_stf(A.gsa + ((4 * kvh + (qv & 3)) * 4 + (idx & 15) / 4) * 8 + g.row0 + (qv >> 2), -136.f * t);
        }
        flags_set(A, MK2_F_ATT, (seg * 8 + kvh) * ns + sp, 1, flag_val(epoch, l, MK2_F_ATT));
        TRACE(l, 24);
    }
    __syncthreads();
}

/* attention phase of layer l: this workgroup's units.  A split waits for
 * every split of its (segment, kv head), so the splits of one group are
 * handed out in the same round of workgroups: a round holds
 * floor(gridDim / nsplit) whole groups, split sp of the round's group i on
 * workgroup i * nsplit + sp. */
template <bool IO, int KVB>
S2P_DEV void attn_phase(const Mk2Args& A, int l, uint32_t epoch, LDSP(unsigned char)* smem) {
    const int ns = A.nsplit, ng = A.n_seg * 8, gpr = (int)gridDim.x / ns;
    const int gi = (int)blockIdx.x / ns, sp = (int)blockIdx.x - gi * ns;
    if (gi >= gpr) return;
    for (int grp = gi; grp < ng; grp += gpr) attn_unit<IO, KVB>(A, l, grp % A.n_seg, grp / A.n_seg, sp, epoch, smem);
}

/* ---- head: the ring continues over this wave's head units ---- */
S2P_DEV void c_head(Slot (&S)[NSLOT], const Mk2Args& A, int cw, const Ctx& C,
                    LDSP(unsigned char)* smem, int M) {
    constexpr int RS = XRS(2560);
    const WG& w = C.hw;
    const int lane = threadIdx.x & 63, q = lane >> 4, r = lane & 15;
    const LDSP(uint16_t)* xs = (const LDSP(uint16_t)*)(smem + L_XS) + min(r, M - 1) * RS + q * 8;
    LDSP(float)* part = (LDSP(float)*)(smem + L_HPART);
    const LDSP(float)* nbt = (const LDSP(float)*)(smem + L_BIAS) + 4 * (q & 1);
    uint32_t mask = 0x000F000Fu, one = 0x43004300u;
    asm volatile("" : "+v"(mask), "+v"(one));
    /* the wave's units are tiles (start / 20) .. (last / 20) of the packed
     * head, local tile = tile - head_t0 */
    s2p_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    int cur = w.start / 20;
    auto flush = [&]() __attribute__((always_inline)) {
        const int lt = cur - C.head_t0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = 4 * q + i;
            if (m < M) part[((lt * CW + cw) * M + m) * 16 + r] = acc[i];
        }
        acc = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
    };
    for (int r0 = 0; r0 < w.nu; r0 += NSLOT) {
        sfor<NSLOT>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            slot_wait<WAITN>(S[j]);
            const int u = r0 + j;
            if (u < w.nu) {
                const int pu = w.start + u;
                const int tile = pu / 20, b = pu - tile * 20;
                if (tile != cur) {
                    flush();
                    cur = tile;
                }
                acc += unit_mul(S[j], xs + b * 128, nbt + b * 32, mask, one);
            }
            unit_issue(S[j], A.hpack, w.start, w.last, u + NSLOT);
            __builtin_amdgcn_sched_barrier(0);
        });
    }
    if (w.nu > 0) flush();
}

/* head reduction: logits[m][n] of this workgroup's tiles (all waves); a
 * tile's partials come from the waves whose unit range meets it, summed in
 * wave order */
S2P_DEV void head_reduce(const Mk2Args& A, const Ctx& C, LDSP(unsigned char)* smem, int M) {
    const LDSP(float)* part = (const LDSP(float)*)(smem + L_HPART);
    const LDSP(float)* inv = (const LDSP(float)*)(smem + L_INV);
    const int nout = C.head_nt * 16 * M;
    const int U = C.head_nt * 20;
    for (int i = threadIdx.x; i < nout; i += NTH) {
        const int n = i & 15, rest = i >> 4;
        const int m = rest % M, lt = rest / M;
        const int row = (C.head_t0 + lt) * 16 + n;
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < CW; w++) {
            const int u0 = wave_cut(U, w, false), u1 = wave_cut(U, w + 1, false); /* as geo_of splits */
            if (u0 < (lt + 1) * 20 && u1 > lt * 20) s += part[((lt * CW + w) * M + m) * 16 + n];
        }
        if (row < A.head_n) A.logits[(size_t)m * A.head_n + row] = f2bf(__fmul_rn(inv[m], s));
    }
}

/* ---- the kernel ---- */
/* KVB: the sessions' caches, bf16 (16) or INT8 / INT4 codes with f16 group
 * scales (8 / 4, A.kvb) */
template <int KVB>
__global__ __launch_bounds__(NTH) void k_mk2(const Mk2Args A) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    LDSP(unsigned char)* smem = (LDSP(unsigned char)*)smem_raw;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int M = A.rows, NL = A.n_layers;
    const int wg = blockIdx.x;
    const uint32_t epoch = coh_ld32(A.state);

    if (wave < CW) {
        /* ================= compute waves ================= */
        asm volatile("; CPATH_BEGIN");
        const int cw = wave;
        Ctx C;
        C.w[PQ] = wg_of(geoP<PQ>(wg, cw), phNB(PQ), false);
        C.w[PO] = wg_of(geoP<PO>(wg, cw), phNB(PO), false);
        C.w[PG] = wg_of(geoP<PG>(wg, cw), phNB(PG), false);
        C.w[PD] = wg_of(geoP<PD>(wg, cw), phNB(PD), false);
        {
            const Geo gh = geo_of(A.head_tiles, 20, false, wg, cw);
            C.hw = wg_of(gh, 20, false);
            C.head_t0 = gh.t0;
            C.head_nt = gh.nt;
        }
        Slot S[NSLOT];
        sfor<NSLOT>([&](auto kc) {
            constexpr int k = decltype(kc)::value;
            constexpr int tp = seq_phase(k);
            const bool hd = NL == 0;
            unit_issue(S[k], hd ? A.hpack : A.wpack + phOFF(tp), hd ? C.hw.start : C.w[tp].start,
                       hd ? C.hw.last : C.w[tp].last, hd ? k : k - seq_base(tp));
        });
        __syncthreads(); /* (init) */
        for (int l = 0; l < NL; l++) {
            /* Q */
            __syncthreads();
            bias_pairs<2560>(smem);
            c_gemv<PQ>(S, A, l, cw, C, smem, M);
            if (cw == 0) TRACE(l, 13);
            __syncthreads();
            reduce_phase<PQ>(smem, M, wg);
            /* attention */
            attn_phase<false, KVB>(A, l, epoch, smem);
            /* O */
            __syncthreads();
            c_gemv<PO>(S, A, l, cw, C, smem, M);
            if (cw == 0) TRACE(l, 14);
            __syncthreads();
            reduce_phase<PO>(smem, M, wg);
            /* G */
            __syncthreads();
            bias_pairs<2560>(smem);
            c_gemv<PG>(S, A, l, cw, C, smem, M);
#ifdef MK2_TRACE
            if (l == 18 && (threadIdx.x & 63) == 0) g_mk2_tr[blockIdx.x][39][19 + cw] = wall_clock64();
#endif
            if (cw == 0) TRACE(l, 15);
            __syncthreads();
            reduce_phase<PG>(smem, M, wg);
            /* D */
            __syncthreads();
            bias_pairs<9728>(smem);
            c_gemv<PD>(S, A, l, cw, C, smem, M);
#ifdef MK2_TRACE
            if (l == 18 && (threadIdx.x & 63) == 0) g_mk2_tr[blockIdx.x][39][12 + cw] = wall_clock64();
#endif
            if (cw == 0) TRACE(l, 16);
            __syncthreads();
            reduce_phase<PD>(smem, M, wg);
        }
        /* head */
        __syncthreads();
        bias_pairs<2560>(smem);
        c_head(S, A, cw, C, smem, M);
        if (cw == 0) TRACE(NL, 2);
        __syncthreads();
        head_reduce(A, C, smem, M);
        /* drain this wave's remaining (clamped, unused) prefetches */
        vm_drain();
    } else {
        /* ================= IO wave ================= */
        asm volatile("; IOPATH_BEGIN");
        /* residual stream init: x = x_in for this workgroup's 16-column
         * tile (the w2 geometry), its sums of squares, its values weighted by
         * the first norm and their sums */
        const Geo gd = geoP<PD>(wg, 0);
        {
            const uint16_t* nw0 = NL > 0 ? A.norms + MK2_NORM_ATTN : A.final_norm;
            for (int i = lane; i < M * 16 * gd.np; i += 64) {
                const int m = i / 16, cc = i & 15;
                const size_t ix = (size_t)m * 2560 + gd.t0 * 16 + cc;
                const uint16_t v = A.x_in[ix];
                coh_st16(A.x + ix, v);
                const float f = bf2f(v);
                const float t = sum_lanes16(f * f);
                if (cc == 0) coh_stf(A.ssq + m * 160 + gd.t0, t);
                const uint16_t xw = f2bf(__fmul_rn(f, bf2f(nw0[gd.t0 * 16 + cc])));
                coh_st16(A.xw + ix, xw);
                const float tw = sum_lanes16(bf2f(xw));
                if (cc == 0) coh_stf(A.gsx + gd.t0 * 8 + m, -136.f * tw);
            }
            flags_set(A, MK2_F_INIT, wg, 1, flag_val(epoch, -1, MK2_F_INIT));
        }
        __syncthreads(); /* (init) */
        const Geo gq = geoP<PQ>(wg, 0), go = geoP<PO>(wg, 0), gg = geoP<PG>(wg, 0);
        for (int l = 0; l < NL; l++) {
            const uint16_t* nl = A.norms + (size_t)l * MK2_NORM_STRIDE;
            /* Q: x (previous w2, or the init) -> qkv */
            if (l == 0) flags_wait(A, MK2_F_INIT, 0, MK2_NWG, flag_val(epoch, -1, MK2_F_INIT));
            else flags_wait(A, MK2_F_D, 0, MK2_NWG, flag_val(epoch, l - 1, MK2_F_D));
            TRACE(l, 0);
            io_stage<2560, true, false, true>(A, A.xw, A.gsx, nullptr, M, smem, gq.t0, gq.np);
            TRACE(l, 1);
            __syncthreads();
            bias_pairs<2560>(smem);
            __syncthreads();
            reduce_phase<PQ>(smem, M, wg);
            io_store(A, smem, A.qkv, 6144, gq.t0, gq.np, M, false, nullptr, MK2_F_Q,
                     flag_val(epoch, l, MK2_F_Q), l);
            TRACE(l, 2);
            /* attention */
            attn_phase<true, KVB>(A, l, epoch, smem);
            TRACE(l, 3);
            /* O: attn -> x += wo attn */
            flags_wait(A, MK2_F_ATT, 0, A.n_seg * 8 * A.nsplit, flag_val(epoch, l, MK2_F_ATT));
            TRACE(l, 4);
            io_stage<4096, false, true, false>(A, A.attn, A.gsa, nl + MK2_NORM_FFN, M, smem, go.t0, go.np);
            TRACE(l, 5);
            __syncthreads();
            __syncthreads();
            reduce_phase<PO>(smem, M, wg);
            io_store(A, smem, A.x, 2560, go.t0, go.np, M, true, A.gsx, MK2_F_O,
                     flag_val(epoch, l, MK2_F_O), l);
            TRACE(l, 6);
            /* G: x -> h */
            flags_wait(A, MK2_F_O, 0, MK2_NWG, flag_val(epoch, l, MK2_F_O));
            TRACE(l, 7);
            io_stage<2560, true, false, true>(A, A.xw, A.gsx, nullptr, M, smem, gg.t0, gg.np);
            TRACE(l, 8);
            __syncthreads();
            bias_pairs<2560>(smem);
            __syncthreads();
            reduce_phase<PG>(smem, M, wg);
            io_store(A, smem, A.h, 9728, gg.t0, gg.np, M, false, A.gsh, MK2_F_G,
                     flag_val(epoch, l, MK2_F_G), l, true);
            TRACE(l, 9);
            /* D: h -> x += w2 h */
            flags_wait(A, MK2_F_G, 0, MK2_NWG, flag_val(epoch, l, MK2_F_G));
            TRACE(l, 10);
            io_stage<9728, false, true, true>(A, A.h, A.gsh,
                                        l + 1 < NL ? nl + MK2_NORM_STRIDE + MK2_NORM_ATTN : A.final_norm, M,
                                        smem, gd.t0, gd.np);
            TRACE(l, 11);
            __syncthreads();
            bias_pairs<9728>(smem);
            __syncthreads();
            reduce_phase<PD>(smem, M, wg);
            io_store(A, smem, A.x, 2560, gd.t0, gd.np, M, true, A.gsx, MK2_F_D,
                     flag_val(epoch, l, MK2_F_D), l);
            TRACE(l, 12);
        }
        /* head: final RMSNorm of x */
        if (NL == 0) flags_wait(A, MK2_F_INIT, 0, MK2_NWG, flag_val(epoch, -1, MK2_F_INIT));
        else flags_wait(A, MK2_F_D, 0, MK2_NWG, flag_val(epoch, NL - 1, MK2_F_D));
        TRACE(NL, 0);
        io_stage<2560, true, false, true>(A, A.xw, A.gsx, nullptr, M, smem, 0, 0);
        TRACE(NL, 1);
        __syncthreads();
        bias_pairs<2560>(smem);
        __syncthreads();
        {
            const Geo gh = geo_of(A.head_tiles, 20, false, wg, 0);
            Ctx C;
            C.head_t0 = gh.t0;
            C.head_nt = gh.nt;
            head_reduce(A, C, smem, M);
        }
        TRACE(NL, 3);
        /* launch bookkeeping: the last workgroup to finish advances the epoch */
        vm_drain();
        if (lane == 0) {
            const uint32_t done = __hip_atomic_fetch_add(A.state + 1, 1u, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            if (done + 1 == (epoch + 1) * (uint32_t)gridDim.x)
                __hip_atomic_store(A.state, epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

/* ---- packing ---- */
/* one thread per (tile, block, lane): 16 bytes of codes (4 groups of the
 * lane's row and quarter) and, lanes 0..15, the row's 4 group scales */
__global__ void k_mk2_pack(const uint8_t* __restrict__ w, const uint16_t* __restrict__ sc, int N,
                           int K, int pairs, uint8_t* __restrict__ dst) {
    const int nb = K / 128;
    const int T = (N + 15) / 16;
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int lane = (int)(gid & 63);
    const long tb = gid >> 6;
    if (tb >= (long)T * nb) return;
    const int t = (int)(tb / nb), b = (int)(tb % nb);
    const int q = lane >> 4, r = lane & 15;
    /* packed tile t row r -> source row; gate_up (pairs): rows 0..7 gate
     * rows 8t.., rows 8..15 the matching up rows N/2 + 8t.. */
    const int n = !pairs ? t * 16 + r : r < 8 ? 8 * t + r : N / 2 + 8 * t + (r - 8);
    uint32_t o[4];
#pragma unroll
    for (int gg = 0; gg < 4; gg++) {
        const int grp = 4 * b + gg;
        uint32_t d = 0x88888888u; /* padding rows: code 8 = weight 0 */
        if (n < N) {
            const uint32_t s = *(const uint32_t*)(w + (size_t)n * (K / 2) + grp * 16 + 4 * q);
            /* source nibble p = weight k = 8q + p; target nibble j = k 8q + 2j,
             * nibble 4 + j = k 8q + 2j + 1, each biased by 8 */
            d = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t lo = ((s >> (8 * j)) & 0xFu) ^ 8u;
                const uint32_t hi = ((s >> (8 * j + 4)) & 0xFu) ^ 8u;
                d |= lo << (4 * j);
                d |= hi << (16 + 4 * j);
            }
        }
        o[gg] = d;
    }
    uint8_t* blk = dst + ((size_t)t * nb + b) * MK2_BLK;
    *(s2p_u32x4*)(blk + 16 * lane) = (s2p_u32x4){o[0], o[1], o[2], o[3]};
    if (lane < 16) {
        uint16_t s4[4];
#pragma unroll
        for (int gg = 0; gg < 4; gg++) s4[gg] = n < N ? sc[(size_t)n * (K / 32) + 4 * b + gg] : 0;
        uint16_t* sd = (uint16_t*)(blk + 1024) + r * 4;
#pragma unroll
        for (int gg = 0; gg < 4; gg++) sd[gg] = s4[gg];
    }
}

extern "C" hipError_t s2p_mk2_pack(const void* w_pack, const void* scales, int N, int K, int pairs,
                                   void* dst, hipStream_t st) {
    if (!w_pack || !scales || !dst || N <= 0 || (K % 128) || (pairs && (N % 32)))
        return hipErrorInvalidValue;
    const long threads = (long)((N + 15) / 16) * (K / 128) * 64;
    hipLaunchKernelGGL(k_mk2_pack, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                       (const uint8_t*)w_pack, (const uint16_t*)scales, N, K, pairs, (uint8_t*)dst);
    return hipGetLastError();
}

#ifdef MK2_TRACE
extern "C" int s2p_mk2_trace(void* host, size_t bytes) {
    if (bytes < sizeof(g_mk2_tr)) return -1;
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_mk2_tr), sizeof(g_mk2_tr)) == hipSuccess ? 0 : -1;
}
#endif

/* ---- launch ---- */
static int g_mk2_ok = -1;

extern "C" int s2p_mk2_supported(void) {
    if (g_mk2_ok >= 0) return g_mk2_ok ? 0 : -1;
    int dev = 0, cus = 0, per_cu = 0;
    bool ok = hipGetDevice(&dev) == hipSuccess &&
              hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
              cus == MK2_NWG &&
              hipFuncSetAttribute((const void*)k_mk2<16>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)L_TOTAL) == hipSuccess &&
              hipFuncSetAttribute((const void*)k_mk2<8>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)L_TOTAL) == hipSuccess &&
              hipFuncSetAttribute((const void*)k_mk2<4>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)L_TOTAL) == hipSuccess;
    for (const void* f : {(const void*)k_mk2<16>, (const void*)k_mk2<8>, (const void*)k_mk2<4>})
        ok = ok && hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, NTH, L_TOTAL) == hipSuccess &&
             per_cu >= 1;
    (void)hipGetLastError();
    g_mk2_ok = ok ? 1 : 0;
    return ok ? 0 : -1;
}

extern "C" hipError_t s2p_mk2_launch(const Mk2Args* args, hipStream_t st) {
    if (s2p_mk2_supported() != 0) return hipErrorNotSupported;
    if (!args || args->rows < 1 || args->rows > MK2_MAX_ROWS || args->n_seg > 8 ||
        args->nsplit < 1 || args->nsplit > MK2_MAX_SPLIT ||
        args->n_seg * 8 * args->nsplit > MK2_ATT_MAX || args->n_layers > MK2_MAX_LAYERS ||
        args->head_tiles > 39 * MK2_NWG || (args->kvb != 16 && args->kvb != 8 && args->kvb != 4) ||
        (args->kvb != 16 && !args->plan.kvs))
        return hipErrorInvalidValue;
    if (args->kvb == 8) hipLaunchKernelGGL(k_mk2<8>, dim3(MK2_NWG), dim3(NTH), L_TOTAL, st, *args);
    else if (args->kvb == 4) hipLaunchKernelGGL(k_mk2<4>, dim3(MK2_NWG), dim3(NTH), L_TOTAL, st, *args);
    else hipLaunchKernelGGL(k_mk2<16>, dim3(MK2_NWG), dim3(NTH), L_TOTAL, st, *args);
    return hipGetLastError();
}
