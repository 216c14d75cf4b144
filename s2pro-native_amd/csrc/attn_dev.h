/* s2pro MI355X — device code of the decode / verify attention (see
 * attention.hip for the design), shared by k_attn and the persistent verify
 * kernel.  q, outputs and split partials go through the coherent accessors
 * of coh.h; the KV cache is read with plain streaming loads (rows written in
 * the same launch are written through before they are first read). */
#ifndef S2P_ATTN_DEV_H
#define S2P_ATTN_DEV_H

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "coh.h"
#include "common.h"
#include "prims_dev.h"
#include "prims_internal.h"

#define AT_HD 128
#define AT_TILE 32
#define AT_WAVES 4
#define AT_SEG_ROWS 8
#define AT_VSTRIDE 136
#define AT_PSTRIDE 40
#define LDS(T) __attribute__((address_space(3))) T
/* LDS carve-up of one attention block of W waves (bytes) */
#define AT_SV_BYTES_W(W) ((W) * AT_TILE * AT_VSTRIDE * 2)
#define AT_SP_BYTES_W(W) ((W) * 32 * AT_PSTRIDE * 2)
#define AT_SML_BYTES_W(W) ((W) * 32 * 2 * 4)
#define AT_SQ_BYTES (32 * AT_HD * 2) /* fused path: the block's q vectors */
#define AT_LDS_BYTES_W(W) \
    (AT_SV_BYTES_W(W) + 2 * AT_SP_BYTES_W(W) + AT_SML_BYTES_W(W) + 16 + AT_SQ_BYTES)
#define AT_SV_BYTES AT_SV_BYTES_W(AT_WAVES)
#define AT_LDS_BYTES AT_LDS_BYTES_W(AT_WAVES)

enum { AM_CONTIG = 0, AM_PTRS = 1, AM_PLAN = 2 };

struct AttnArgs {
    int mode;
    const uint16_t* q;
    uint16_t* out;
    int rows;
    int qh, kvh_n;
    /* CONTIG */
    const uint16_t* kc;
    const uint16_t* vc;
    int pos0;
    int max_seq;
    /* PTRS */
    const uint16_t* const* kcs;
    const uint16_t* const* vcs;
    const int32_t* pos;
    /* PLAN */
    S2pRowPlan plan;
    const S2pAttnSeg* segs;
    int layer;
    /* splitting: nseg segments x kvh_n kv heads x nsplit position splits */
    int nseg;
    int nsplit;
    int split_pos;
    float* part;
    /* non-NULL: the last split to finish a (segment, kv head) merges the
     * splits itself (persistent kernel); NULL: k_attn_combine does */
    unsigned* counters;
#ifdef S2P_DIAG
    uint64_t* probe; /* diagnostics build: [grid][8] stage clocks */
#endif
    /* PLAN, fused qk-norm + RoPE + KV append (qkv != NULL): q is computed
     * from the raw fused qkv rows into q (written, then read back by the
     * same block), and the blocks whose positions cover a segment's new
     * slots append that segment's K/V of their kv head first */
    const uint16_t* qkv;
    const uint16_t* qn_w;
    const uint16_t* kn_w;
    const float* rope_tab; /* [rows][64][cos, sin] of the plan's positions */
    float eps;
};

struct SegInfo {
    const uint16_t* kp;
    const uint16_t* vp;
    int L, row0, nrows, span, first;
    const uint64_t* vis; /* NULL: causal */
};

/* MODE is a compile-time constant: each caller kind gets its own kernel,
 * with no run-time branch over the modes */
template <int MODE>
S2P_DEV SegInfo resolve(const AttnArgs& a, int seg, int kvh) {
    SegInfo s;
    s.vis = nullptr;
    s.first = 0;
    if constexpr (MODE == AM_CONTIG) {
        s.row0 = seg * AT_SEG_ROWS;
        s.nrows = min(AT_SEG_ROWS, a.rows - s.row0);
        s.L = a.pos0 + s.row0;
        s.span = min(s.L + s.nrows, a.max_seq); /* never read past the cache */
        s.kp = a.kc + (size_t)kvh * a.max_seq * AT_HD;
        s.vp = a.vc + (size_t)kvh * a.max_seq * AT_HD;
    } else if constexpr (MODE == AM_PTRS) {
        s.row0 = seg;
        s.L = a.pos[seg];
        /* a position outside the cache attends nothing (and reads nothing) */
        s.nrows = (s.L >= 0 && s.L < a.max_seq) ? 1 : 0;
        s.span = s.nrows ? s.L + 1 : 0;
        s.kp = a.kcs[seg] + (size_t)kvh * a.max_seq * AT_HD;
        s.vp = a.vcs[seg] + (size_t)kvh * a.max_seq * AT_HD;
    } else {
        const S2pAttnSeg g = a.segs[seg];
        s.row0 = g.row0;
        s.nrows = g.nrows;
        s.L = g.L;
        s.span = g.span;
        s.first = g.first;
        const uint16_t* kv = (const uint16_t*)g.kv + (size_t)a.layer * a.plan.layer_stride;
        s.kp = kv + (size_t)kvh * a.plan.max_seq * AT_HD;
        s.vp = kv + (size_t)(a.kvh_n + kvh) * a.plan.max_seq * AT_HD;
        s.vis = a.plan.vis;
    }
    return s;
}

/* ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
 * i % 4 of the 8-byte chunks addressed by lanes i / 4, 4 + i / 4, 8 + i / 4,
 * 12 + i / 4 (a 4 x 4 transpose of 16-bit elements per group of lanes;
 * measured on the part with an index pattern) */
S2P_DEV s2p_u32x2 ds_read_tr16(const LDS(uint16_t)* p) {
    typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4;
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS(s16x4)*)p);
    return __builtin_bit_cast(s2p_u32x2, v);
}

/* may row rl see slot j: the prefix, then the causal chain or the row's
 * tree mask word vw = s.vis[row0 + rl], which the caller loads once (any
 * value when s.vis is NULL), so the tile loop makes no memory access */
S2P_DEV bool visible_w(const SegInfo& s, uint64_t vw, int rl, int j) {
    if (rl >= s.nrows || j >= s.span) return false;
    if (j < s.L) return true;
    const int b = j - s.L;
    if (!s.vis) return b <= rl;
    return b < 64 && ((vw >> b) & 1ull);
}


S2P_DEV float max16(float v) {
    /* every lane of the 16-lane row gets the max (DPP moves; max is exact,
     * so the rotations' order is immaterial) */
    v = fmaxf(v, dpp_f<0xB1>(v)); /* quad_perm [1,0,3,2] */
    v = fmaxf(v, dpp_f<0x4E>(v)); /* quad_perm [2,3,0,1] */
    v = fmaxf(v, dpp_f<0x124>(v)); /* row_ror:4 */
    v = fmaxf(v, dpp_f<0x128>(v)); /* row_ror:8 */
    return v;
}
S2P_DEV float sum16(float v) {
    /* lane 0 of each 16-lane row gets the xor-butterfly total ((q0 + q1) +
     * (q2 + q3)) of its quad sums q (DPP moves; the other lanes get partial
     * rotations, unused) */
    v = quad_sum(v);
    v += dpp_f<0x124>(v); /* row_ror:4 */
    v += dpp_f<0x128>(v); /* row_ror:8 */
    return v;
}

/* max / sum over the lanes c, c + 16, c + 32, c + 48 (row swaps, VALU);
 * every lane gets the result */
S2P_DEV float xg_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
S2P_DEV float xg_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
/* two floats as a bf16 pair (RNE), the first in the low half */
S2P_DEV uint32_t pk_bf(float lo, float hi) {
    return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}

S2P_DEV void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* merge the split partials of (row, head h, dim d):
 * out = sum_s e^(m_s - M) O_s / sum_s e^(m_s - M) l_s, in split order */
template <bool COH>
S2P_DEV float ld_f(const float* p) {
    if constexpr (COH) return coh_ldf(p);
    else return *p;
}

template <bool COH = true>
S2P_DEV void attn_merge_one(const float* part, uint16_t* out, int rows, int qh, int nsplit,
                            int row, int h, int d) {
    const size_t p0 = ((size_t)row * qh + h) * nsplit;
    const float* po = part + (size_t)rows * qh * nsplit * 2;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; s++) M = fmaxf(M, ld_f<COH>(part + (p0 + s) * 2));
    const float Ms = M == -INFINITY ? 0.f : M;
    float lt = 0.f, acc = 0.f;
    for (int s0 = 0; s0 < nsplit; s0 += 8) {
        float mv[8], lv[8], ov[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const bool ok = s0 + j < nsplit;
            mv[j] = ok ? ld_f<COH>(part + (p0 + s0 + j) * 2) : 0.f;
            lv[j] = ok ? ld_f<COH>(part + (p0 + s0 + j) * 2 + 1) : 0.f;
            ov[j] = ok ? ld_f<COH>(po + (p0 + s0 + j) * AT_HD + d) : 0.f;
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (s0 + j >= nsplit) break;
            const float w = __expf(mv[j] - Ms);
            lt = fmaf(lv[j], w, lt);
            acc = fmaf(ov[j], w, acc);
        }
    }
    coh_st16(out + ((size_t)row * qh + h) * AT_HD + d, f2bf(acc / lt));
}

/* One (segment, kv head, position split) attention block; smem holds
 * AT_LDS_BYTES.  Body of k_attn, also run by the persistent verify kernel.
 * Returns true (uniformly) when this block wrote final outputs: a single
 * split, or the last split to arrive, which merged all of them. */
/* COH: the q / qkv / RoPE-table reads bypass the L2 (the persistent
 * kernel, where their producer ran in the same launch); the layer kernel
 * reads them through the caches */
template <int MQT, int W, bool COH, int MODE>
__device__ bool attn_block(const AttnArgs& a, int seg, int kvh, int sp, LDS(unsigned char)* smem) {
    constexpr int SVB = AT_SV_BYTES_W(W), SPB = AT_SP_BYTES_W(W), SMLB = AT_SML_BYTES_W(W);
    LDS(uint16_t)* s_v = (LDS(uint16_t)*)smem;
    LDS(uint16_t)* s_p = (LDS(uint16_t)*)(smem + SVB);
    LDS(float)* s_ml = (LDS(float)*)(smem + SVB + 2 * SPB);
    LDS(int)* s_flag = (LDS(int)*)(smem + SVB + 2 * SPB + SMLB);
/* V tile of wave w: 32 positions x 16 chunks of 16 bytes (8 dims), chunk
 * (t, k) stored at slot k ^ vsw(t) of row t (rows of 256 B).  The Vt
 * operand is read with transposing loads (ds_read_b64_tr_b16): a read
 * touches 16 rows (4 G + k, or 16 + 4 G + k; G, k < 4) at the same two
 * chunks, and vsw spreads them over 8 slot pairs (2-way at most). */
#define VSW(t) (((t) & 7) << 1)
#define SVOFF(w, t, d) ((w) * (AT_TILE * 128) + (t) * 128 + ((((d) >> 3) ^ VSW(t)) << 3) + ((d) & 7))
#define SML(w, qv, k) s_ml[((w) * 32 + (qv)) * 2 + (k)]

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int qq = lane >> 4, c = lane & 15;
    const SegInfo S = resolve<MODE>(a, seg, kvh);
    /* the mask words of this lane's query rows 4 qt + c / 4 (query vector
     * 16 qt + c), loaded once and first (every later load is then younger,
     * so the tile loop's waits can count the prefetches in flight) */
    uint64_t vw[MQT];
#pragma unroll
    for (int qt = 0; qt < MQT; qt++) {
        const int rl = 4 * qt + (c >> 2);
        vw[qt] = S.vis && rl < S.nrows ? S.vis[S.row0 + rl] : 0ull;
    }
    const int p_begin = sp * a.split_pos;
    const int p_end = min(p_begin + a.split_pos, S.span);
    const float scale = 0.08838834764831845f;
    const int qrow_stride = a.qh * AT_HD;
#ifdef S2P_DIAG
    uint64_t* const probe =
        a.probe ? a.probe + ((size_t)(sp * a.kvh_n + kvh) * a.nseg + seg) * 8 : nullptr;
#else
    uint64_t* const probe = nullptr; /* stage clocks: diagnostics build only */
#endif
    auto stamp = [&](int i) __attribute__((always_inline)) {
        if (probe && threadIdx.x == 0) probe[i] = wall_clock64();
    };
    stamp(0);

    /* one tile of K (registers) and V (straight to this wave's LDS: lane l
     * of load i fills bytes 16 l of the load's 1 KB = slot l % 16 of row
     * 4 i + l / 16) */
    s2p_u32x4 kr[2][4];
    auto issue_k = [&](int tb) __attribute__((always_inline)) {
#pragma unroll
        for (int ps = 0; ps < 2; ps++) {
            const int pos = min(tb + 16 * ps + c, p_end - 1);
#pragma unroll
            for (int ch = 0; ch < 4; ch++)
                kr[ps][ch] = gld_nt128(S.kp + (size_t)pos * AT_HD + 32 * ch + 8 * qq);
        }
    };
    /* V into registers (lane l of load i holds the 16 bytes that go to
     * bytes 16 l of the wave's 1 KB row group i in LDS), written to LDS just
     * before its P V: loads the compiler counts, so the tile loop's waits
     * leave the next tile's loads in flight */
    s2p_u32x4 vt[8];
    auto issue_v = [&](int tb) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int t = 4 * i + (lane >> 4);
            const int pos = min(tb + t, p_end - 1);
            vt[i] = gld_nt128(S.vp + (size_t)pos * AT_HD + 8 * (lane & 15));
        }
    };
    auto issue_tile = [&](int tb) __attribute__((always_inline)) {
        issue_k(tb);
        issue_v(tb);
    };
    const int tb0 = p_begin + wave * AT_TILE;
    bool early = false; /* first tile issued before the fused prologue */

    /* Q operands: A row i = c -> query vector qv = 16 qt + c */
    s2p_u32x4 qa[MQT][4];
    if (MODE == AM_PLAN && a.qkv) {
        /* fused qk-norm + RoPE + K/V append, one wave per (row, head) item:
         * the block's 4 q heads of its segment's rows (to LDS), then the k/v
         * of every new slot of the session inside the block's positions (a
         * tree's ancestors may sit in another segment: each block appends
         * what it reads itself; blocks that overlap write identical values).
         * Every load of a batch of items is issued before any is used. */
        LDS(uint16_t)* s_q = (LDS(uint16_t)*)(smem + SVB + 2 * SPB + SMLB + 16);
        const int first = S.first; /* the session's row at slot L */
        const int s0 = max(p_begin, S.L), s1 = min(p_end, S.span);
        const int nq = S.nrows * 4, nit = nq + max(0, s1 - s0);
        const bool appends = s1 > s0;
        early = !appends && tb0 < p_end;
        constexpr int IB = 8; /* every item of a 4-wave block in one batch at M <= 5 */
        /* the norm weights of this lane's two elements, once per wave (q and k) */
        const bool qkn = a.qn_w != nullptr; /* no norm weights: RoPE only */
        const uint16_t qw0 = qkn ? a.qn_w[lane] : 0, qw1 = qkn ? a.qn_w[lane + 64] : 0;
        const uint16_t kw0 = qkn ? a.kn_w[lane] : 0, kw1 = qkn ? a.kn_w[lane + 64] : 0;
        for (int base = wave; base < nit; base += IB * W) {
            float v0[IB], v1[IB], cs[IB][4];
            uint16_t x0[IB], x1[IB];
#pragma unroll
            for (int j = 0; j < IB; j++) {
                const int it = base + j * W;
                if (it >= nit) break; /* uniform */
                const bool isq = it < nq;
                const int row = isq ? S.row0 + (it >> 2) : first + (s0 - S.L) + (it - nq);
                const int head = isq ? 4 * kvh + (it & 3) : 32 + kvh;
                const uint16_t* src = a.qkv + (size_t)row * 6144 + head * AT_HD;
                v0[j] = bf2f(COH ? coh_ld16(src + lane) : src[lane]);
                v1[j] = bf2f(COH ? coh_ld16(src + lane + 64) : src[lane + 64]);
                /* (cos, sin) of the lane's two pairs, 8 bytes each */
                const float* tab = a.rope_tab + (size_t)row * 128;
                const float* t0 = tab + (lane >> 1) * 2;
                const float* t1 = tab + ((lane + 64) >> 1) * 2;
                if (COH) {
                    cs[j][0] = coh_ldf(t0);
                    cs[j][1] = coh_ldf(t0 + 1);
                    cs[j][2] = coh_ldf(t1);
                    cs[j][3] = coh_ldf(t1 + 1);
                } else {
                    const float2 c0 = *(const float2*)t0, c1 = *(const float2*)t1;
                    cs[j][0] = c0.x;
                    cs[j][1] = c0.y;
                    cs[j][2] = c1.x;
                    cs[j][3] = c1.y;
                }
                if (!isq) { /* the v head rides along */
                    x0[j] = COH ? coh_ld16(src + 8 * AT_HD + lane) : src[8 * AT_HD + lane];
                    x1[j] = COH ? coh_ld16(src + 8 * AT_HD + lane + 64) : src[8 * AT_HD + lane + 64];
                }
            }
            /* the first K/V tile goes out behind the first batch's loads, so
             * the item arithmetic below waits for those loads only */
            if (early && base == wave) issue_tile(tb0);
#pragma unroll
            for (int j = 0; j < IB; j++) {
                const int it = base + j * W;
                if (it >= nit) break;
                float o0, o1;
                const bool isq = it < nq;
                qkrope_math(v0[j], v1[j], isq ? qw0 : kw0, isq ? qw1 : kw1, cs[j][0], cs[j][1],
                            cs[j][2], cs[j][3], a.eps, lane, &o0, &o1, qkn);
                if (it < nq) {
                    LDS(uint16_t)* dq = s_q + it * AT_HD; /* q vector (rl, g) = it */
                    const uint16_t q0 = f2bf(o0), q1 = f2bf(o1);
                    dq[lane] = q0;
                    dq[lane + 64] = q1;
                    if (sp == 0) { /* the q rows also land in q (inspection) */
                        uint16_t* gq = (uint16_t*)a.q + (size_t)(S.row0 + (it >> 2)) * qrow_stride +
                                       (4 * kvh + (it & 3)) * AT_HD;
                        gq[lane] = q0;
                        gq[lane + 64] = q1;
                    }
                } else {
                    const size_t slot = (size_t)(s0 + (it - nq)); /* row first + slot - L */
                    uint16_t* kd = (uint16_t*)S.kp + slot * AT_HD;
                    uint16_t* vd = (uint16_t*)S.vp + slot * AT_HD;
                    coh_st16(kd + lane, f2bf(o0));
                    coh_st16(kd + lane + 64, f2bf(o1));
                    coh_st16(vd + lane, x0[j]);
                    coh_st16(vd + lane + 64, x1[j]);
                }
            }
        }
        if (early && nit <= wave) issue_tile(tb0); /* a wave with no item */
        if (appends) vm_drain(); /* the appended K/V before any tile load */
        __syncthreads();
#pragma unroll
        for (int qt = 0; qt < MQT; qt++) {
            const int qv = 16 * qt + c;
#pragma unroll
            for (int ch = 0; ch < 4; ch++)
                qa[qt][ch] = (qv >> 2) < S.nrows
                                 ? *(const LDS(s2p_u32x4)*)(s_q + qv * AT_HD + 32 * ch + 8 * qq)
                                 : (s2p_u32x4){0u, 0u, 0u, 0u};
        }
    } else {
#pragma unroll
        for (int qt = 0; qt < MQT; qt++) {
            const int qv = 16 * qt + c;
            const int rl = qv >> 2, g = qv & 3;
#pragma unroll
            for (int ch = 0; ch < 4; ch++) {
                if (rl < S.nrows) {
                    const uint16_t* qp = a.q + (size_t)(S.row0 + rl) * qrow_stride +
                                         (4 * kvh + g) * AT_HD + 32 * ch + 8 * qq;
                    qa[qt][ch] = COH ? coh_ld128(qp) : *(const s2p_u32x4*)qp;
                } else {
                    qa[qt][ch] = (s2p_u32x4){0u, 0u, 0u, 0u};
                }
            }
        }
    }

    /* The scores are computed transposed, S^T = K Q^T: lane (qq, c) holds
     * query vector 16 qt + c at positions 16 ps + 4 qq + v, so a query's
     * softmax runs over its own 8 values and then the lanes c + 16 G, and
     * the 8 values, packed, are the B operand of O^T = V^T P^T (k slot
     * 8 qq + 4 ps + v <-> position 16 ps + 4 qq + v): P never goes through
     * LDS.  m, l per query vector (l: this lane's positions, summed at the
     * end); o[qt][dt]: O^T, dims 16 dt + 4 qq + v of query vector 16 qt + c */
    float m[MQT], l[MQT];
    s2p_f32x4 o[MQT][8];
#pragma unroll
    for (int qt = 0; qt < MQT; qt++) {
        m[qt] = -INFINITY;
        l[qt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < 8; dt++) o[qt][dt] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
    }
    const int open_end = min(S.L, p_end); /* tiles below it need no mask */

    /* software pipeline over this wave's tiles: the next tile's K loads
     * (into kr, free once the scores are issued) fly during this tile's
     * softmax and P V, its V loads (into vt, free once this tile's V is in
     * LDS) during this P V and the next scores and softmax */
    if (!early && tb0 < p_end) issue_tile(tb0);
    auto tile_step = [&](int tb, auto nxt_c) __attribute__((always_inline)) {
        constexpr bool nxt = decltype(nxt_c)::value; /* a next tile follows */
        const int tn = tb + W * AT_TILE;
        if (probe && tb == p_begin) stamp(1); /* prologue done, first scores next */
        /* scores */
        s2p_f32x4 sc[MQT][2];
#pragma unroll
        for (int qt = 0; qt < MQT; qt++)
#pragma unroll
            for (int ps = 0; ps < 2; ps++) {
                s2p_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ch = 0; ch < 4; ch++) acc = mfma16x16x32(kr[ps][ch], qa[qt][ch], acc);
                sc[qt][ps] = acc;
            }
        if constexpr (nxt) issue_k(tn);
        /* online softmax of query vector 16 qt + c over positions
         * tb + 16 ps + 4 qq + v.  O is rescaled only when some query of the
         * wave raised its maximum: otherwise every factor is e^0 = 1 exactly
         * and the products would change nothing (past the first tiles of a
         * split, the usual case) */
        const bool open = tb + AT_TILE <= open_end;
        float corr[MQT];
        s2p_u32x4 ph[MQT], pl[MQT];
        bool raised = false;
#pragma unroll
        for (int qt = 0; qt < MQT; qt++) {
            const int rl = 4 * qt + (c >> 2);
            float t[2][4];
            float tm = -INFINITY;
#pragma unroll
            for (int ps = 0; ps < 2; ps++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int pos = tb + 16 * ps + 4 * qq + v;
                    const bool vis = open || (visible_w(S, vw[qt], rl, pos) && pos < p_end);
                    t[ps][v] = vis ? sc[qt][ps][v] * scale : -INFINITY;
                    tm = fmaxf(tm, t[ps][v]);
                }
            tm = xg_max(tm);
            const float mn = fmaxf(m[qt], tm);
            const float ms = mn == -INFINITY ? 0.f : mn;
            corr[qt] = __expf(m[qt] - ms);
            raised |= corr[qt] != 1.0f;
            float ls = 0.f;
            float p[2][4], lo[2][4];
#pragma unroll
            for (int ps = 0; ps < 2; ps++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    p[ps][v] = __expf(t[ps][v] - ms);
                    ls += p[ps][v];
                    /* P = hi + lo, both bf16: 16 significant bits into the MFMA */
                    lo[ps][v] = p[ps][v] - bf2f(f2bf(p[ps][v]));
                }
            l[qt] = l[qt] * corr[qt] + ls;
            m[qt] = mn;
            ph[qt] = (s2p_u32x4){pk_bf(p[0][0], p[0][1]), pk_bf(p[0][2], p[0][3]),
                                 pk_bf(p[1][0], p[1][1]), pk_bf(p[1][2], p[1][3])};
            pl[qt] = (s2p_u32x4){pk_bf(lo[0][0], lo[0][1]), pk_bf(lo[0][2], lo[0][3]),
                                 pk_bf(lo[1][0], lo[1][1]), pk_bf(lo[1][2], lo[1][3])};
        }
        if (__any(raised)) {
#pragma unroll
            for (int qt = 0; qt < MQT; qt++)
#pragma unroll
                for (int dt = 0; dt < 8; dt++)
#pragma unroll
                    for (int v = 0; v < 4; v++) o[qt][dt][v] *= corr[qt];
        }
        /* this tile's V into the wave's LDS buffer (free: the previous
         * tile's P V has read it), then the next tile's V loads */
#pragma unroll
        for (int i = 0; i < 8; i++)
            *(LDS(s2p_u32x4)*)(s_v + SVOFF(wave, 4 * i + (lane >> 4), 8 * (lane & 15))) = vt[i];
        if constexpr (nxt) issue_v(tn);
        wave_sync_lds();
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            /* A operand (row c = dim 16 dt + c, k slots 8 qq + j = positions
             * 4 qq + j, then 16 + 4 qq + j) by two transposing reads: lane
             * 4 k + m of a 16-lane group supplies the 4 dims 16 dt + 4 m.. of
             * row 4 qq + k (+ 16), and lane c receives dim 16 dt + c of the
             * group's 4 rows */
            const int k4 = c >> 2, m4 = c & 3;
            const s2p_u32x2 b0 = ds_read_tr16(s_v + SVOFF(wave, 4 * qq + k4, 16 * dt + 4 * m4));
            const s2p_u32x2 b1 = ds_read_tr16(s_v + SVOFF(wave, 16 + 4 * qq + k4, 16 * dt + 4 * m4));
            const s2p_u32x4 va = {b0.x, b0.y, b1.x, b1.y};
#pragma unroll
            for (int qt = 0; qt < MQT; qt++) {
                o[qt][dt] = mfma16x16x32(va, pl[qt], o[qt][dt]);
                o[qt][dt] = mfma16x16x32(va, ph[qt], o[qt][dt]);
            }
        }
        wave_sync_lds();
    };
    /* the tiles with a successor run in a loop whose every iteration issues
     * the next tile's loads (so the compiler's waits count them), the last
     * tile after it */
    if (tb0 < p_end) {
        int tb = tb0;
        for (; tb + W * AT_TILE < p_end; tb += W * AT_TILE)
            tile_step(tb, std::integral_constant<bool, true>{});
        tile_step(tb, std::integral_constant<bool, false>{});
    }

    stamp(2);
    /* ---- merge the W waves ---- */
#pragma unroll
    for (int qt = 0; qt < MQT; qt++) {
        l[qt] = xg_sum(l[qt]);
        if (qq == 0) {
            SML(wave, 16 * qt + c, 0) = m[qt];
            SML(wave, 16 * qt + c, 1) = l[qt];
        }
    }
    __syncthreads();
    float ltot[MQT], mtot[MQT];
#pragma unroll
    for (int qt = 0; qt < MQT; qt++) {
        const int qv = 16 * qt + c;
        float M = -INFINITY;
#pragma unroll 4
        for (int w = 0; w < W; w++) M = fmaxf(M, SML(w, qv, 0));
        const float Ms = M == -INFINITY ? 0.f : M;
        float lt = 0.f;
#pragma unroll 4
        for (int w = 0; w < W; w++) lt += __expf(SML(w, qv, 0) - Ms) * SML(w, qv, 1);
        const float f = __expf(m[qt] - Ms);
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int v = 0; v < 4; v++) o[qt][dt][v] *= f;
        ltot[qt] = lt;
        mtot[qt] = M;
    }
    /* sum O over waves through LDS (reusing the V tiles: 2 x 16 KB) */
    LDS(float)* s_o = (LDS(float)*)s_v;
    /* O of the 32 query vectors as [q vector][dim] */
    auto put = [&]() {
#pragma unroll
        for (int qt = 0; qt < MQT; qt++)
#pragma unroll
            for (int dt = 0; dt < 8; dt++)
                *(LDS(s2p_f32x4)*)(s_o + (16 * qt + c) * AT_HD + 16 * dt + 4 * qq) = o[qt][dt];
    };
    /* the tree's hand-offs in a lane-major layout ([slot][qt][dt][lane] of
     * 16 bytes): one ds_write_b128 / ds_read_b128 per register quad,
     * conflict-free */
    static_assert((W / 2) * MQT * 8 * 64 * 16 <= SVB, "merge slots exceed the V tiles");
    LDS(s2p_f32x4)* s_o4 = (LDS(s2p_f32x4)*)s_v;
    auto put4 = [&](int slot) {
#pragma unroll
        for (int qt = 0; qt < MQT; qt++)
#pragma unroll
            for (int dt = 0; dt < 8; dt++) s_o4[((slot * MQT + qt) * 8 + dt) * 64 + lane] = o[qt][dt];
    };
    auto add4 = [&](int slot) {
#pragma unroll
        for (int qt = 0; qt < MQT; qt++)
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                const s2p_f32x4 t = s_o4[((slot * MQT + qt) * 8 + dt) * 64 + lane];
#pragma unroll
                for (int v = 0; v < 4; v++) o[qt][dt][v] += t[v];
            }
    };
    /* pairwise tree: wave w += wave w + half for half = W/2 .. 2, then wave
     * 0 += wave 1 below */
#pragma unroll
    for (int half = W / 2; half >= 2; half /= 2) {
        __syncthreads();
        if (wave >= half && wave < 2 * half) put4(wave - half);
        __syncthreads();
        if (wave < half) add4(wave);
    }
    __syncthreads();
    if (wave == 1) put4(0);
    __syncthreads();
    stamp(3);
    if (wave == 0) add4(0);
    if (a.nsplit == 1) {
        if (wave == 0) {
#pragma unroll
            for (int qt = 0; qt < MQT; qt++) {
                const int qv = 16 * qt + c;
                const int rl = qv >> 2, g = qv & 3;
                if (rl >= S.nrows) continue;
                const int row = S.row0 + rl;
                const int h = 4 * kvh + g;
                const float inv = 1.0f / ltot[qt];
#pragma unroll
                for (int dt = 0; dt < 8; dt++) {
                    const s2p_f32x4 y = o[qt][dt];
                    coh_st64(a.out + (size_t)row * qrow_stride + h * AT_HD + 16 * dt + 4 * qq,
                             (uint64_t)pk_bf(y[0] * inv, y[1] * inv) |
                                 ((uint64_t)pk_bf(y[2] * inv, y[3] * inv) << 32));
                }
            }
        }
    } else {
        /* partial (m, l, O) of this split: O through LDS ([q vector][dim]), then
         * 16-byte write-through stores by the whole block */
        LDS(float)* s_mlw = (LDS(float)*)s_p; /* [32][2], free after the tiles */
        if (wave == 0) {
            put();
            if (qq == 0) {
#pragma unroll
                for (int qt = 0; qt < MQT; qt++) {
                    s_mlw[(16 * qt + c) * 2] = mtot[qt];
                    s_mlw[(16 * qt + c) * 2 + 1] = ltot[qt];
                }
            }
        }
        __syncthreads();
        for (int idx = threadIdx.x; idx < S.nrows * 4 * (AT_HD / 4); idx += W * 64) {
            const int qv = idx >> 5, d4 = (idx & 31) * 4;
            const int row = S.row0 + (qv >> 2), h = 4 * kvh + (qv & 3);
            const size_t pi = ((size_t)row * a.qh + h) * a.nsplit + sp;
            float* po = a.part + (size_t)a.rows * a.qh * a.nsplit * 2 + pi * AT_HD;
            coh_st128(po + d4, *(const LDS(s2p_u32x4)*)(s_o + qv * AT_HD + d4));
            if (d4 == 0)
                coh_st64(a.part + pi * 2, (uint64_t)__float_as_uint(s_mlw[qv * 2]) |
                                              ((uint64_t)__float_as_uint(s_mlw[qv * 2 + 1]) << 32));
        }
    }
    if (probe) {
        vm_drain();
        stamp(4);
    }
    if (a.nsplit == 1) return true;
    if (!a.counters) return false;
    /* last split of this (segment, kv head) to finish merges the splits */
    vm_drain();
    __syncthreads();
    const int cidx = seg * a.kvh_n + kvh;
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_fetch_add(a.counters + cidx, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        *s_flag = prev == (unsigned)(a.nsplit - 1);
    }
    __syncthreads();
    if (*s_flag && 2 * S.nrows * 4 * a.nsplit + S.nrows * 4 > SVB / 4) {
        /* too many splits for the LDS merge: one output at a time */
        for (int idx = threadIdx.x; idx < S.nrows * 4 * AT_HD; idx += W * 64) {
            const int rl = idx >> 9, g = (idx >> 7) & 3, d = idx & (AT_HD - 1);
            attn_merge_one(a.part, a.out, a.rows, a.qh, a.nsplit, S.row0 + rl, 4 * kvh + g, d);
        }
        if (threadIdx.x == 0)
            __hip_atomic_store(a.counters + cidx, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (*s_flag) {
        /* merge (same arithmetic and order as attn_merge_one): split weights
         * e^(m_s - M) and the denominators per (row, head) once, in LDS
         * (the V tiles' space), then every output with all of its split
         * loads in flight */
        const int npair = S.nrows * 4, ns = a.nsplit;
        LDS(float)* wm = (LDS(float)*)s_v;   /* [npair][ns] m, then weights */
        LDS(float)* wl = wm + npair * ns;    /* [npair][ns] l */
        LDS(float)* lt = wl + npair * ns;    /* [npair] */
        for (int idx = threadIdx.x; idx < npair * ns; idx += W * 64) {
            const int pr = idx / ns, sp2 = idx - pr * ns;
            const size_t pi = ((size_t)(S.row0 + (pr >> 2)) * a.qh + 4 * kvh + (pr & 3)) * ns + sp2;
            wm[idx] = coh_ldf(a.part + pi * 2);
            wl[idx] = coh_ldf(a.part + pi * 2 + 1);
        }
        __syncthreads();
        if ((int)threadIdx.x < npair) {
            const int pr = threadIdx.x;
            float M = -INFINITY;
            for (int k = 0; k < ns; k++) M = fmaxf(M, wm[pr * ns + k]);
            const float Ms = M == -INFINITY ? 0.f : M;
            float l = 0.f;
            for (int k = 0; k < ns; k++) {
                const float w = __expf(wm[pr * ns + k] - Ms);
                l = fmaf(wl[pr * ns + k], w, l);
                wm[pr * ns + k] = w;
            }
            lt[pr] = l;
        }
        __syncthreads();
        const float* po = a.part + (size_t)a.rows * a.qh * ns * 2;
        /* item = (pair, 4 dims): 16-byte partial loads, 8 splits in flight */
        for (int idx = threadIdx.x; idx < npair * (AT_HD / 4); idx += W * 64) {
            const int pr = idx >> 5, d = (idx & 31) * 4;
            const int row = S.row0 + (pr >> 2), h = 4 * kvh + (pr & 3);
            const size_t p0 = ((size_t)row * a.qh + h) * ns;
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            for (int k0 = 0; k0 < ns; k0 += 8) {
                s2p_u32x4 ov[8];
#pragma unroll
                for (int j = 0; j < 8; j++)
                    ov[j] = k0 + j < ns ? coh_ld128(po + (p0 + k0 + j) * AT_HD + d)
                                        : (s2p_u32x4){0u, 0u, 0u, 0u};
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    if (k0 + j >= ns) break;
                    const float w = wm[pr * ns + k0 + j];
                    acc[0] = fmaf(__uint_as_float(ov[j].x), w, acc[0]);
                    acc[1] = fmaf(__uint_as_float(ov[j].y), w, acc[1]);
                    acc[2] = fmaf(__uint_as_float(ov[j].z), w, acc[2]);
                    acc[3] = fmaf(__uint_as_float(ov[j].w), w, acc[3]);
                }
            }
            const float lp = lt[pr];
            const uint64_t o4 = (uint64_t)f2bf(acc[0] / lp) | ((uint64_t)f2bf(acc[1] / lp) << 16) |
                                ((uint64_t)f2bf(acc[2] / lp) << 32) |
                                ((uint64_t)f2bf(acc[3] / lp) << 48);
            coh_st64(a.out + ((size_t)row * a.qh + h) * AT_HD + d, o4);
        }
        if (threadIdx.x == 0)
            __hip_atomic_store(a.counters + cidx, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (probe && *s_flag) {
        vm_drain();
        stamp(5);
    }
    const bool merged = *s_flag != 0;
    __syncthreads();
    return merged;
#undef SVOFF
#undef VSW
#undef SP
#undef SPL
#undef SML
}

#endif
