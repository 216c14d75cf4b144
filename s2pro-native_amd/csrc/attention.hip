/* s2pro MI355X — decode / verify GQA attention over the bf16 KV cache.
 *
 * Replaces the reference's causal single-pass attention (kernels.cu:234-339)
 * and split-K flash-decode (kernels.cu:341-508), and adds the tree mask the
 * verify pass needs.  One kernel serves three callers:
 *   CONTIG  s2pk_attention: one contiguous cache, rows at positions pos..;
 *   PTRS    s2pk_attention_ptrs / _decode: per-row caches and positions;
 *   PLAN    the verify forward: sessions x rows with per-row visibility
 *           masks (causal chain or draft tree) relative to the prefix L.
 *
 * Block = (segment of <= 8 rows, kv head, position split).  The 4 query heads
 * of the GQA group x the segment's rows form up to 32 query vectors, i.e. two
 * 16-row MFMA tiles that stay in registers.  The 4 waves take 32-position
 * tiles round-robin; per tile:
 *   S = Q K^T    v_mfma_f32_16x16x32_bf16, K read straight from HBM with one
 *                16-byte load per lane per (16 positions x 32 dims);
 *   online softmax in fp32 (max across the 16 lanes of a row group);
 *   O += P V     P re-laid out through LDS as the A operand, V staged in LDS
 *                and gathered per 16-dim column tile as the B operand.
 * The waves merge through LDS; a block writes its (m, l, O) partial, and a
 * combine kernel merges splits (log-sum-exp) unless there is one split.
 * Scores are (q . k) * 1/sqrt(128) with q, k bf16 exact products and fp32
 * sums; P enters the PV product as a bf16 hi + lo pair (two MFMAs), so the
 * PV sum sees P to ~2^-16 relative.  Parity is by tolerance
 * against the reference order (oracle or_attention / or_attention_split).
 */
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "common.h"
#include "prims_internal.h"
#include "s2pro/kernels.h"
#include "s2pro/slowar_kernels.h"

#define AT_HD 128
#define AT_TILE 32
#define AT_WAVES 4
#define AT_SEG_ROWS 8
#define AT_VSTRIDE 136
#define AT_PSTRIDE 40

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
    /* splitting */
    int nsplit;
    int split_pos;
    float* part;
};

struct SegInfo {
    const uint16_t* kp;
    const uint16_t* vp;
    int L, row0, nrows, span;
    const uint64_t* vis; /* NULL: causal */
};

S2P_DEV SegInfo resolve(const AttnArgs& a, int seg, int kvh) {
    SegInfo s;
    s.vis = nullptr;
    if (a.mode == AM_CONTIG) {
        s.row0 = seg * AT_SEG_ROWS;
        s.nrows = min(AT_SEG_ROWS, a.rows - s.row0);
        s.L = a.pos0 + s.row0;
        s.span = min(s.L + s.nrows, a.max_seq); /* never read past the cache */
        s.kp = a.kc + (size_t)kvh * a.max_seq * AT_HD;
        s.vp = a.vc + (size_t)kvh * a.max_seq * AT_HD;
    } else if (a.mode == AM_PTRS) {
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
        const uint16_t* kv =
            (const uint16_t*)a.plan.kv[g.sess] + (size_t)a.layer * a.plan.layer_stride;
        s.kp = kv + (size_t)kvh * a.plan.max_seq * AT_HD;
        s.vp = kv + (size_t)(a.kvh_n + kvh) * a.plan.max_seq * AT_HD;
        s.vis = a.plan.vis;
    }
    return s;
}

S2P_DEV bool visible(const SegInfo& s, int rl, int j) {
    if (rl >= s.nrows || j >= s.span) return false;
    if (j < s.L) return true;
    const int b = j - s.L;
    if (!s.vis) return b <= rl;
    return b < 64 && ((s.vis[s.row0 + rl] >> b) & 1ull);
}

S2P_DEV float max16(float v) {
    v = fmaxf(v, __shfl_xor(v, 1, 16));
    v = fmaxf(v, __shfl_xor(v, 2, 16));
    v = fmaxf(v, __shfl_xor(v, 4, 16));
    v = fmaxf(v, __shfl_xor(v, 8, 16));
    return v;
}
S2P_DEV float sum16(float v) {
    v += __shfl_xor(v, 1, 16);
    v += __shfl_xor(v, 2, 16);
    v += __shfl_xor(v, 4, 16);
    v += __shfl_xor(v, 8, 16);
    return v;
}

S2P_DEV void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int MQT>
__global__ __launch_bounds__(256) void k_attn(AttnArgs a) {
    __shared__ __align__(16) uint16_t s_v[AT_WAVES][AT_TILE][AT_VSTRIDE];
    __shared__ __align__(16) uint16_t s_p[AT_WAVES][32][AT_PSTRIDE];
    __shared__ __align__(16) uint16_t s_pl[AT_WAVES][32][AT_PSTRIDE];
    __shared__ float s_ml[AT_WAVES][32][2];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int qq = lane >> 4, c = lane & 15;
    const int seg = blockIdx.x, kvh = blockIdx.y, sp = blockIdx.z;
    const SegInfo S = resolve(a, seg, kvh);
    const int p_begin = sp * a.split_pos;
    const int p_end = min(p_begin + a.split_pos, S.span);
    const float scale = 0.08838834764831845f;
    const int qrow_stride = a.qh * AT_HD;

    /* Q operands: A row i = c -> query vector qv = 16 qt + c */
    s2p_u32x4 qa[MQT][4];
#pragma unroll
    for (int qt = 0; qt < MQT; qt++) {
        const int qv = 16 * qt + c;
        const int rl = qv >> 2, g = qv & 3;
#pragma unroll
        for (int ch = 0; ch < 4; ch++) {
            if (rl < S.nrows) {
                qa[qt][ch] = *(const s2p_u32x4*)(a.q + (size_t)(S.row0 + rl) * qrow_stride +
                                                 (4 * kvh + g) * AT_HD + 32 * ch + 8 * qq);
            } else {
                qa[qt][ch] = (s2p_u32x4){0u, 0u, 0u, 0u};
            }
        }
    }

    float m[MQT][4], l[MQT][4];
    s2p_f32x4 o[MQT][8];
#pragma unroll
    for (int qt = 0; qt < MQT; qt++) {
#pragma unroll
        for (int v = 0; v < 4; v++) {
            m[qt][v] = -INFINITY;
            l[qt][v] = 0.f;
        }
#pragma unroll
        for (int dt = 0; dt < 8; dt++) o[qt][dt] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
    }

    for (int tb = p_begin + wave * AT_TILE; tb < p_end; tb += AT_WAVES * AT_TILE) {
        /* K: 2 position subtiles x 4 dim chunks, one 16-byte load each */
        s2p_u32x4 kr[2][4];
#pragma unroll
        for (int ps = 0; ps < 2; ps++) {
            const int pos = min(tb + 16 * ps + c, p_end - 1);
#pragma unroll
            for (int ch = 0; ch < 4; ch++)
                kr[ps][ch] = __builtin_nontemporal_load(
                    (const s2p_u32x4*)(S.kp + (size_t)pos * AT_HD + 32 * ch + 8 * qq));
        }
        /* V tile -> LDS [pos][dim] */
        s2p_u32x4 vr[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int idx = i * 64 + lane;
            const int pos = min(tb + (idx >> 4), p_end - 1);
            vr[i] = __builtin_nontemporal_load(
                (const s2p_u32x4*)(S.vp + (size_t)pos * AT_HD + 8 * (idx & 15)));
        }
        /* scores */
        s2p_f32x4 sc[MQT][2];
#pragma unroll
        for (int qt = 0; qt < MQT; qt++)
#pragma unroll
            for (int ps = 0; ps < 2; ps++) {
                s2p_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ch = 0; ch < 4; ch++) acc = mfma16x16x32(qa[qt][ch], kr[ps][ch], acc);
                sc[qt][ps] = acc;
            }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int idx = i * 64 + lane;
            *(s2p_u32x4*)&s_v[wave][idx >> 4][8 * (idx & 15)] = vr[i];
        }
        /* online softmax; lane (qq, c) holds rows 4 qq + v of each q tile */
#pragma unroll
        for (int qt = 0; qt < MQT; qt++) {
            const int rl = 4 * qt + qq;
            const bool vis0 = visible(S, rl, tb + c) && tb + c < p_end;
            const bool vis1 = visible(S, rl, tb + 16 + c) && tb + 16 + c < p_end;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float t0 = vis0 ? sc[qt][0][v] * scale : -INFINITY;
                const float t1 = vis1 ? sc[qt][1][v] * scale : -INFINITY;
                const float tm = max16(fmaxf(t0, t1));
                const float mn = fmaxf(m[qt][v], tm);
                const float ms = mn == -INFINITY ? 0.f : mn;
                const float corr = __expf(m[qt][v] - ms);
                const float p0 = __expf(t0 - ms), p1 = __expf(t1 - ms);
                l[qt][v] = l[qt][v] * corr + p0 + p1;
                m[qt][v] = mn;
#pragma unroll
                for (int dt = 0; dt < 8; dt++) o[qt][dt][v] *= corr;
                /* P = hi + lo, both bf16: 16 significant bits into the PV MFMA */
                const uint16_t h0 = f2bf(p0), h1 = f2bf(p1);
                s_p[wave][16 * qt + 4 * qq + v][c] = h0;
                s_p[wave][16 * qt + 4 * qq + v][16 + c] = h1;
                s_pl[wave][16 * qt + 4 * qq + v][c] = f2bf(p0 - bf2f(h0));
                s_pl[wave][16 * qt + 4 * qq + v][16 + c] = f2bf(p1 - bf2f(h1));
            }
        }
        wave_sync_lds();
        s2p_u32x4 pa[MQT], pl[MQT];
#pragma unroll
        for (int qt = 0; qt < MQT; qt++) {
            pa[qt] = *(const s2p_u32x4*)&s_p[wave][16 * qt + c][8 * qq];
            pl[qt] = *(const s2p_u32x4*)&s_pl[wave][16 * qt + c][8 * qq];
        }
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            uint32_t b[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                b[e] = (uint32_t)s_v[wave][8 * qq + 2 * e][16 * dt + c] |
                       ((uint32_t)s_v[wave][8 * qq + 2 * e + 1][16 * dt + c] << 16);
            const s2p_u32x4 bv = {b[0], b[1], b[2], b[3]};
#pragma unroll
            for (int qt = 0; qt < MQT; qt++) {
                o[qt][dt] = mfma16x16x32(pl[qt], bv, o[qt][dt]);
                o[qt][dt] = mfma16x16x32(pa[qt], bv, o[qt][dt]);
            }
        }
        wave_sync_lds();
    }

    /* ---- merge the 4 waves ---- */
#pragma unroll
    for (int qt = 0; qt < MQT; qt++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            l[qt][v] = sum16(l[qt][v]);
            if (c == 0) {
                s_ml[wave][16 * qt + 4 * qq + v][0] = m[qt][v];
                s_ml[wave][16 * qt + 4 * qq + v][1] = l[qt][v];
            }
        }
    __syncthreads();
    float ltot[MQT][4], mtot[MQT][4];
#pragma unroll
    for (int qt = 0; qt < MQT; qt++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int qv = 16 * qt + 4 * qq + v;
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < AT_WAVES; w++) M = fmaxf(M, s_ml[w][qv][0]);
            const float Ms = M == -INFINITY ? 0.f : M;
            float lt = 0.f;
#pragma unroll
            for (int w = 0; w < AT_WAVES; w++) lt += __expf(s_ml[w][qv][0] - Ms) * s_ml[w][qv][1];
            const float f = __expf(m[qt][v] - Ms);
#pragma unroll
            for (int dt = 0; dt < 8; dt++) o[qt][dt][v] *= f;
            ltot[qt][v] = lt;
            mtot[qt][v] = M;
        }
    /* sum O over waves through LDS (reusing the V tiles: 2 x 16 KB) */
    float* s_o = (float*)&s_v[0][0][0];
    const int ostride = 32 * AT_HD;
    auto put = [&](int slot) {
#pragma unroll
        for (int qt = 0; qt < MQT; qt++)
#pragma unroll
            for (int dt = 0; dt < 8; dt++)
#pragma unroll
                for (int v = 0; v < 4; v++)
                    s_o[slot * ostride + (16 * qt + 4 * qq + v) * AT_HD + 16 * dt + c] = o[qt][dt][v];
    };
    auto add = [&](int slot) {
#pragma unroll
        for (int qt = 0; qt < MQT; qt++)
#pragma unroll
            for (int dt = 0; dt < 8; dt++)
#pragma unroll
                for (int v = 0; v < 4; v++)
                    o[qt][dt][v] += s_o[slot * ostride + (16 * qt + 4 * qq + v) * AT_HD + 16 * dt + c];
    };
    __syncthreads();
    if (wave >= 2) put(wave - 2);
    __syncthreads();
    if (wave < 2) add(wave);
    __syncthreads();
    if (wave == 1) put(0);
    __syncthreads();
    if (wave != 0) return;
    add(0);

    /* ---- write ---- */
#pragma unroll
    for (int qt = 0; qt < MQT; qt++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int qv = 16 * qt + 4 * qq + v;
            const int rl = qv >> 2, g = qv & 3;
            if (rl >= S.nrows) continue;
            const int row = S.row0 + rl;
            const int h = 4 * kvh + g;
            if (a.nsplit == 1) {
                const float inv = 1.0f / ltot[qt][v];
#pragma unroll
                for (int dt = 0; dt < 8; dt++)
                    a.out[(size_t)row * qrow_stride + h * AT_HD + 16 * dt + c] =
                        f2bf(o[qt][dt][v] * inv);
            } else {
                const size_t pi = ((size_t)row * a.qh + h) * a.nsplit + sp;
                float* po = a.part + (size_t)a.rows * a.qh * a.nsplit * 2 + pi * AT_HD;
#pragma unroll
                for (int dt = 0; dt < 8; dt++) po[16 * dt + c] = o[qt][dt][v];
                if (c == 0) {
                    a.part[pi * 2] = mtot[qt][v];
                    a.part[pi * 2 + 1] = ltot[qt][v];
                }
            }
        }
}

/* merge split partials: out = sum_s e^(m_s - M) O_s / sum_s e^(m_s - M) l_s */
__global__ __launch_bounds__(128) void k_attn_combine(const float* __restrict__ part,
                                                      uint16_t* __restrict__ out, int rows,
                                                      int qh, int nsplit) {
    const int row = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
    const size_t p0 = ((size_t)row * qh + h) * nsplit;
    const float* po = part + (size_t)rows * qh * nsplit * 2;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; s++) M = fmaxf(M, part[(p0 + s) * 2]);
    const float Ms = M == -INFINITY ? 0.f : M;
    float lt = 0.f, acc = 0.f;
    for (int s = 0; s < nsplit; s++) {
        const float w = __expf(part[(p0 + s) * 2] - Ms);
        lt = fmaf(part[(p0 + s) * 2 + 1], w, lt);
        acc = fmaf(po[(p0 + s) * AT_HD + d], w, acc);
    }
    out[((size_t)row * qh + h) * AT_HD + d] = f2bf(acc / lt);
}

static int64_t part_floats(int rows, int qh, int nsplit) {
    return (int64_t)rows * qh * nsplit * (AT_HD + 2);
}

static hipError_t attn_run(AttnArgs a, int n_seg, int max_nrows, int max_span,
                           int64_t part_cap, hipStream_t st) {
    const int tiles = (max_span + AT_TILE * AT_WAVES - 1) / (AT_TILE * AT_WAVES);
    int tpw = 1; /* tiles per wave per split */
    if (a.part && part_cap > 0) {
        while ((int64_t)n_seg * a.kvh_n * ((tiles + tpw - 1) / tpw) > 4096) tpw *= 2;
        int nsplit = (tiles + tpw - 1) / tpw;
        while (nsplit > 1 && part_floats(a.rows, a.qh, nsplit) > part_cap) {
            tpw *= 2;
            nsplit = (tiles + tpw - 1) / tpw;
        }
    } else {
        tpw = tiles > 0 ? tiles : 1;
    }
    a.split_pos = tpw * AT_TILE * AT_WAVES;
    a.nsplit = (max_span + a.split_pos - 1) / a.split_pos;
    if (a.nsplit < 1) a.nsplit = 1;
    dim3 grid((unsigned)n_seg, (unsigned)a.kvh_n, (unsigned)a.nsplit);
    if (max_nrows <= 4)
        hipLaunchKernelGGL(k_attn<1>, grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL(k_attn<2>, grid, dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit == 1) return e;
    hipLaunchKernelGGL(k_attn_combine, dim3(a.rows, a.qh), dim3(AT_HD), 0, st, a.part, a.out,
                       a.rows, a.qh, a.nsplit);
    return hipGetLastError();
}

extern "C" hipError_t s2pk_attention(const s2p_bf16* q, const s2p_bf16* k_cache,
                                     const s2p_bf16* v_cache, s2p_bf16* out, int rows,
                                     int q_heads, int kv_heads, int head_dim, int pos,
                                     int max_seq, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (head_dim != AT_HD || q_heads != 4 * kv_heads) return hipErrorInvalidValue;
    AttnArgs a = {};
    a.mode = AM_CONTIG;
    a.q = (const uint16_t*)q;
    a.out = (uint16_t*)out;
    a.rows = rows;
    a.qh = q_heads;
    a.kvh_n = kv_heads;
    a.kc = (const uint16_t*)k_cache;
    a.vc = (const uint16_t*)v_cache;
    a.pos0 = pos;
    a.max_seq = max_seq;
    const int n_seg = (rows + AT_SEG_ROWS - 1) / AT_SEG_ROWS;
    return attn_run(a, n_seg, rows < AT_SEG_ROWS ? rows : AT_SEG_ROWS, pos + rows, 0, st);
}

extern "C" hipError_t s2pk_attention_ptrs(const s2p_bf16* q, const s2p_bf16* const* k_caches,
                                          const s2p_bf16* const* v_caches, s2p_bf16* out,
                                          int rows, int q_heads, int kv_heads, int head_dim,
                                          const int32_t* pos, int max_seq, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (head_dim != AT_HD || q_heads != 4 * kv_heads) return hipErrorInvalidValue;
    /* the split count needs the host-known max length; without it the whole
     * cache capacity bounds the work */
    AttnArgs a = {};
    a.mode = AM_PTRS;
    a.q = (const uint16_t*)q;
    a.out = (uint16_t*)out;
    a.rows = rows;
    a.qh = q_heads;
    a.kvh_n = kv_heads;
    a.kcs = (const uint16_t* const*)k_caches;
    a.vcs = (const uint16_t* const*)v_caches;
    a.pos = pos;
    a.max_seq = max_seq;
    return attn_run(a, rows, 1, max_seq, 0, st);
}

extern "C" int64_t s2pk_attention_part_floats(int rows, int q_heads, int max_len) {
    const int nsplit = (max_len + AT_TILE * AT_WAVES - 1) / (AT_TILE * AT_WAVES);
    return part_floats(rows, q_heads, nsplit < 1 ? 1 : nsplit);
}

extern "C" hipError_t s2pk_attention_decode(const s2p_bf16* q, const s2p_bf16* const* k_caches,
                                            const s2p_bf16* const* v_caches, s2p_bf16* out,
                                            int rows, int q_heads, int kv_heads, int head_dim,
                                            const int32_t* pos, int max_seq, int max_len,
                                            float* part, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (head_dim != AT_HD || q_heads != 4 * kv_heads || !part || max_len <= 0)
        return hipErrorInvalidValue;
    AttnArgs a = {};
    a.mode = AM_PTRS;
    a.q = (const uint16_t*)q;
    a.out = (uint16_t*)out;
    a.rows = rows;
    a.qh = q_heads;
    a.kvh_n = kv_heads;
    a.kcs = (const uint16_t* const*)k_caches;
    a.vcs = (const uint16_t* const*)v_caches;
    a.pos = pos;
    a.max_seq = max_seq;
    a.part = part;
    return attn_run(a, rows, 1, max_len, s2pk_attention_part_floats(rows, q_heads, max_len), st);
}

extern "C" int64_t s2p_attn_plan_part_floats(int rows, int max_span) {
    return s2pk_attention_part_floats(rows, 32, max_span);
}

extern "C" hipError_t s2p_attn_plan_launch(const void* q, void* out, const S2pRowPlan* plan,
                                           const S2pAttnSeg* segs, int n_seg, int rows,
                                           int layer, int max_span, float* part,
                                           hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    AttnArgs a = {};
    a.mode = AM_PLAN;
    a.q = (const uint16_t*)q;
    a.out = (uint16_t*)out;
    a.rows = rows;
    a.qh = 32;
    a.kvh_n = 8;
    a.plan = *plan;
    a.segs = segs;
    a.layer = layer;
    a.part = part;
    return attn_run(a, n_seg, AT_SEG_ROWS, max_span, s2p_attn_plan_part_floats(rows, max_span),
                    st);
}
