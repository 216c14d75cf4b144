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

#include "attn_dev.h"
#include "s2pro/kernels.h"
#include "s2pro/slowar_kernels.h"

/* Position splits are sized so that the grid stays within AT_MAX_BLOCKS
 * blocks (two per CU): a block's fixed costs (q load or the fused prologue,
 * the wave merge, the partial store) are paid once per block, so at configs
 * 4 / 5 (8 x 4096 / 4 x 8192 positions) 512 blocks ran the layer's
 * attention in 34 / 85 us against 54 / 112 us with 4096. */
#ifndef AT_MAX_BLOCKS
#define AT_MAX_BLOCKS 512
#endif

/* Blocks are numbered (segment fastest, then kv head, then split) and the
 * numbering is laid over the 8 XCDs in contiguous chunks: workgroup i runs
 * on XCD i % 8 and takes the (i / 8)-th block of chunk i % 8.  The
 * segments of one session (a draft tree of more than 8 rows has several)
 * read the same K/V positions of a kv head; this way they run together on
 * one XCD and the second and third reads hit its L2. */
#ifdef S2P_DIAG
/* diagnostics build: wall clock per block (logical number) at the stages of
 * attn_block, for the last launch */
__device__ uint64_t g_at_probe[4096 * 8];
extern "C" hipError_t s2p_at_probe_get(uint64_t* host, int n) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_at_probe), (size_t)n * 8, 0, hipMemcpyDeviceToHost);
}
#endif

template <int MQT, int W, int MODE>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2))) void k_attn(AttnArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const int lin = (int)blockIdx.x;
    const int total = a.nseg * a.kvh_n * a.nsplit;
    /* chunk x of the numbering (the first total % 8 chunks one block
     * longer) goes to XCD x; bijective for lin < total */
    const int q = total >> 3, r = total & 7, xcd = lin & 7, j = lin >> 3;
    const int b = xcd < r ? xcd * (q + 1) + j : r * (q + 1) + (xcd - r) * q + j;
    const int seg = b % a.nseg, rest = b / a.nseg;
#ifdef S2P_DIAG
    a.probe = b < 4096 ? g_at_probe : nullptr;
#endif
    attn_block<MQT, W, false, MODE>(a, seg, rest % a.kvh_n, rest / a.kvh_n,
                                    (LDS(unsigned char)*)smem_raw);
}

/* merge split partials (one thread per output element) */
__global__ __launch_bounds__(128) void k_attn_combine(const float* __restrict__ part,
                                                      uint16_t* __restrict__ out, int rows,
                                                      int qh, int nsplit) {
    /* the partials come from the previous launch: plain (cached) loads */
    attn_merge_one<false>(part, out, rows, qh, nsplit, blockIdx.x, blockIdx.y, threadIdx.x);
}

/* ---- tree segments: one block per (session, kv head, split) ----
 * A draft tree of R > 8 rows per session (config 5: 17) in 8-row segments
 * has every segment read its session's K/V again.  Here one block takes all
 * R <= 32 rows of the session's GQA group (4 query heads): waves 0..3 take
 * rows 0..15 of one head each, wave 4 + e rows 16 + 4 e .. + 3 of all four
 * heads (so a 17-row tree runs 5 waves, not 8 half-empty q tiles).  The
 * waves share each 32-position K/V tile through LDS, so the K/V are read
 * once.  The q rows come roped from the q buffer (k_qkrope_append ran
 * before).
 * The scores are computed transposed, S^T = K Q^T: lane (G, c) (G = lane /
 * 16, c = lane % 16) holds query vector c at positions 16 ps + 4 G + v,
 * so a query's softmax runs in its own lanes (8 values each, then the 4
 * lanes c + 16 G) and the 8 values are, packed, the B operand of
 * O^T = V^T P^T (k slot 8 G + 4 ps + v <-> position 16 ps + 4 G + v): P
 * never goes through LDS.  P is split hi + lo, both bf16 (16 significant
 * bits into the MFMA).  V comes by transposing LDS reads.  Every query
 * vector ends with its (m, l, O) over the split: the partial, merged by
 * k_attn_combine. */
#define TR_KOFF(t, ch) ((t) * 128 + ((((ch) ^ ((t) & 15))) << 3))
/* a transposing V read touches rows 4 G + k (or 16 + 4 G + k), G, k < 4, at
 * two adjacent 16-byte chunks: the swizzle gives the 16 rows 8 distinct
 * chunk pairs (2-way, the minimum for 512 bytes) */
#define TR_VSW(t) (((t) & 7) << 1)
#define TR_VOFF(t, d) ((t) * 128 + ((((d) >> 3) ^ TR_VSW(t)) << 3) + ((d) & 7))
#define TR_LDS_BYTES (4 * AT_TILE * 128 * 2)

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void k_attn_tree(AttnArgs a) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) unsigned char smem_raw[];
    LDS(unsigned char)* smem = (LDS(unsigned char)*)smem_raw;
    LDS(uint16_t)* s_k = (LDS(uint16_t)*)smem;                           /* [2][32][128] */
    LDS(uint16_t)* s_v = s_k + 2 * AT_TILE * 128;                         /* [2][32][128] */
    const int lin = (int)blockIdx.x;
    const int total = a.nseg * a.kvh_n * a.nsplit;
    const int qd = total >> 3, rd = total & 7, xcd = lin & 7, jd = lin >> 3;
    const int b = xcd < rd ? xcd * (qd + 1) + jd : rd * (qd + 1) + (xcd - rd) * qd + jd;
    const int seg = b % a.nseg, rest = b / a.nseg;
    const int kvh = rest % a.kvh_n, sp = rest / a.kvh_n;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nthr = (int)blockDim.x;
    const int qq = lane >> 4, c = lane & 15;
    const SegInfo S = resolve<AM_PLAN>(a, seg, kvh);
    /* this lane's query vector: waves 0..3 rows c of head 4 kvh + wave;
     * wave 4 + e rows 16 + 4 e + c / 4 of head 4 kvh + c % 4 */
    const int r = wave < 4 ? c : 16 + 4 * (wave - 4) + (c >> 2);
    const int h = 4 * kvh + (wave < 4 ? wave : (c & 3));
    const int p_begin = sp * a.split_pos;
    const int p_end = min(p_begin + a.split_pos, S.span);
    const float scale = 0.08838834764831845f;

    /* mask word and Q operand (B: query vector c, dims 32 ch + 8 qq .. + 7) */
    const uint64_t vw = S.vis && r < S.nrows ? S.vis[S.row0 + r] : 0ull;
    s2p_u32x4 qb[4];
#pragma unroll
    for (int ch = 0; ch < 4; ch++)
        qb[ch] = r < S.nrows ? *(const s2p_u32x4*)(a.q + (size_t)(S.row0 + r) * (a.qh * AT_HD) +
                                                    h * AT_HD + 32 * ch + 8 * qq)
                             : (s2p_u32x4){0u, 0u, 0u, 0u};

    /* the block's K/V tile loads: chunks i = tid, tid + nthr (< 512) of the
     * tile's 512 16-byte chunks (row i / 16, chunk i % 16) of K, then of V */
    s2p_u32x4 ld[4];
    auto load_tile = [&](int tb) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int i = tid + nthr * j, t = (i >> 4) & 31, ch = i & 15;
            const int pos = min(tb + t, p_end - 1);
            if (i < 512) {
                ld[j] = gld_nt128(S.kp + (size_t)pos * AT_HD + 8 * ch);
                ld[2 + j] = gld_nt128(S.vp + (size_t)pos * AT_HD + 8 * ch);
            }
        }
    };
    auto store_tile = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int i = tid + nthr * j, t = (i >> 4) & 31, ch = i & 15;
            if (i < 512) {
                *(LDS(s2p_u32x4)*)(s_k + buf * AT_TILE * 128 + TR_KOFF(t, ch)) = ld[j];
                *(LDS(s2p_u32x4)*)(s_v + buf * AT_TILE * 128 + TR_VOFF(t, 8 * ch)) = ld[2 + j];
            }
        }
    };

    /* m, l of the query (l: this lane's positions only, summed at the end);
     * o[dt]: O^T, dims 16 dt + 4 qq + v of the query */
    float m = -INFINITY, l = 0.f;
    s2p_f32x4 o[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++) o[dt] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};

    const int ntile = p_end > p_begin ? (p_end - p_begin + AT_TILE - 1) / AT_TILE : 0;
    /* tiles wholly inside the prefix (and the split) need no mask */
    const int open_end = min(S.L, p_end);
    if (ntile > 0) {
        load_tile(p_begin);
        store_tile(0);
        if (ntile > 1) load_tile(p_begin + AT_TILE);
    }
    __syncthreads();
    for (int ti = 0; ti < ntile; ti++) {
        const int tb = p_begin + ti * AT_TILE, buf = ti & 1;
        const LDS(uint16_t)* kt = s_k + buf * AT_TILE * 128;
        const LDS(uint16_t)* vt = s_v + buf * AT_TILE * 128;
        /* S^T: K operand (A) = row 16 ps + c, dims 32 ch + 8 qq .. */
        s2p_f32x4 sc[2];
#pragma unroll
        for (int ps = 0; ps < 2; ps++) {
            s2p_u32x4 ka[4];
#pragma unroll
            for (int ch = 0; ch < 4; ch++)
                ka[ch] = *(const LDS(s2p_u32x4)*)(kt + TR_KOFF(16 * ps + c, 4 * ch + qq));
            s2p_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ch = 0; ch < 4; ch++) acc = mfma16x16x32(ka[ch], qb[ch], acc);
            sc[ps] = acc;
        }
        const bool open = tb + AT_TILE <= open_end;
        /* online softmax of the query over positions tb + 16 ps + 4 qq + v */
        float t[2][4];
        float tm = -INFINITY;
#pragma unroll
        for (int ps = 0; ps < 2; ps++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int pos = tb + 16 * ps + 4 * qq + v;
                const bool vis = open || (visible_w(S, vw, r, pos) && pos < p_end);
                t[ps][v] = vis ? sc[ps][v] * scale : -INFINITY;
                tm = fmaxf(tm, t[ps][v]);
            }
        tm = xg_max(tm);
        const float mn = fmaxf(m, tm);
        const float ms = mn == -INFINITY ? 0.f : mn;
        const float corr = __expf(m - ms);
        float ls = 0.f;
        float p[2][4], lo[2][4];
#pragma unroll
        for (int ps = 0; ps < 2; ps++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                p[ps][v] = __expf(t[ps][v] - ms);
                ls += p[ps][v];
                lo[ps][v] = p[ps][v] - bf2f(f2bf(p[ps][v]));
            }
        l = l * corr + ls;
        m = mn;
        const s2p_u32x4 ph = {pk_bf(p[0][0], p[0][1]), pk_bf(p[0][2], p[0][3]),
                              pk_bf(p[1][0], p[1][1]), pk_bf(p[1][2], p[1][3])};
        const s2p_u32x4 pl = {pk_bf(lo[0][0], lo[0][1]), pk_bf(lo[0][2], lo[0][3]),
                              pk_bf(lo[1][0], lo[1][1]), pk_bf(lo[1][2], lo[1][3])};
        if (__any(corr != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < 8; dt++)
#pragma unroll
                for (int v = 0; v < 4; v++) o[dt][v] *= corr;
        }
        /* O^T += V^T P^T: A row c = dim 16 dt + c, k slots 8 qq + j =
         * positions 4 qq + j (j < 4), 16 + 4 qq + j - 4 */
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const int k4 = c >> 2, m4 = c & 3;
            const s2p_u32x2 b0 = ds_read_tr16(vt + TR_VOFF(4 * qq + k4, 16 * dt + 4 * m4));
            const s2p_u32x2 b1 = ds_read_tr16(vt + TR_VOFF(16 + 4 * qq + k4, 16 * dt + 4 * m4));
            const s2p_u32x4 va = {b0.x, b0.y, b1.x, b1.y};
            o[dt] = mfma16x16x32(va, pl, o[dt]);
            o[dt] = mfma16x16x32(va, ph, o[dt]);
        }
        /* the next tile into the other buffer (its previous tile was read
         * before the last barrier), then the one after into registers */
        if (ti + 1 < ntile) store_tile(buf ^ 1);
        __syncthreads();
        if (ti + 2 < ntile) load_tile(tb + 2 * AT_TILE);
    }

    /* the partial of this lane's query: (m, l) and the unnormalised O */
    const float lt = xg_sum(l);
    if (r >= S.nrows) return;
    const size_t pi = ((size_t)(S.row0 + r) * a.qh + h) * a.nsplit + sp;
    float* po = a.part + (size_t)a.rows * a.qh * a.nsplit * 2 + pi * AT_HD;
#pragma unroll
    for (int dt = 0; dt < 8; dt++)
        coh_st128(po + 16 * dt + 4 * qq, __builtin_bit_cast(s2p_u32x4, o[dt]));
    if (qq == 0)
        coh_st64(a.part + pi * 2, (uint64_t)__float_as_uint(m) | ((uint64_t)__float_as_uint(lt) << 32));
}

extern "C" hipError_t s2p_attn_tree_launch(const void* q, void* out, const S2pRowPlan* plan,
                                           const S2pAttnSeg* segs, int n_seg, int rows,
                                           int max_nrows, int layer, int max_span, float* part,
                                           int64_t part_cap, hipStream_t st) {
    if (rows <= 0 || n_seg <= 0) return hipSuccess;
    if (max_nrows < 1 || max_nrows > 32 || max_span <= 0) return hipErrorInvalidValue;
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
    /* splits of whole 32-position tiles, as many as keep the grid within
     * AT_MAX_BLOCKS blocks and the partials within part_cap floats */
    const int tiles = (max_span + AT_TILE - 1) / AT_TILE;
    int ns = (int)(AT_MAX_BLOCKS / ((int64_t)n_seg * 8));
    if (ns < 1) ns = 1;
    if (ns > tiles) ns = tiles;
    while (ns > 1 && (int64_t)rows * 32 * ns * (AT_HD + 2) > part_cap) ns--;
    const int tps = (tiles + ns - 1) / ns;
    a.split_pos = tps * AT_TILE;
    a.nsplit = (max_span + a.split_pos - 1) / a.split_pos;
    a.nseg = n_seg;
    const int total = n_seg * 8 * a.nsplit;
    /* 4 waves (rows 0..15 of the 4 heads), then a wave per 4 more rows */
    const int waves = 4 + (max_nrows > 16 ? (max_nrows - 16 + 3) / 4 : 0);
    static const hipError_t attr = hipFuncSetAttribute(
        (const void*)k_attn_tree, hipFuncAttributeMaxDynamicSharedMemorySize, TR_LDS_BYTES);
    (void)attr;
    hipLaunchKernelGGL(k_attn_tree, dim3((unsigned)total), dim3(64 * waves), TR_LDS_BYTES, st, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_combine, dim3(a.rows, a.qh), dim3(AT_HD), 0, st, a.part, a.out,
                       a.rows, a.qh, a.nsplit);
    return hipGetLastError();
}

/* the split merge for other attention kernels with the same partial layout
 * (the INT8 / INT4 KV decode) */
extern "C" hipError_t s2p_attn_combine_launch(const float* part, uint16_t* out, int rows, int qh,
                                              int nsplit, hipStream_t st) {
    hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)rows, (unsigned)qh), dim3(AT_HD), 0, st,
                       part, out, rows, qh, nsplit);
    return hipGetLastError();
}

static int64_t part_floats(int rows, int qh, int nsplit) {
    return (int64_t)rows * qh * nsplit * (AT_HD + 2);
}

template <int MQT, int W, int MODE>
static void attn_launch(const AttnArgs& a, dim3 grid, hipStream_t st) {
    /* once per instantiation (thread-safe static initialisation) */
    static const hipError_t attr =
        hipFuncSetAttribute((const void*)k_attn<MQT, W, MODE>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, AT_LDS_BYTES_W(W));
    (void)attr;
    hipLaunchKernelGGL((k_attn<MQT, W, MODE>), grid, dim3(64 * W), AT_LDS_BYTES_W(W), st, a);
}

template <int MQT, int W>
static void attn_launch_mode(const AttnArgs& a, dim3 grid, hipStream_t st) {
    if (a.mode == AM_CONTIG) attn_launch<MQT, W, AM_CONTIG>(a, grid, st);
    else if (a.mode == AM_PTRS) attn_launch<MQT, W, AM_PTRS>(a, grid, st);
    else attn_launch<MQT, W, AM_PLAN>(a, grid, st);
}

static hipError_t attn_run(AttnArgs a, int n_seg, int max_nrows, int max_span,
                           int64_t part_cap, hipStream_t st) {
    constexpr int W = AT_WAVES;
    const int tiles = (max_span + AT_TILE * W - 1) / (AT_TILE * W);
    int tpw = 1; /* tiles per wave per split */
    if (a.part && part_cap > 0) {
        while ((int64_t)n_seg * a.kvh_n * ((tiles + tpw - 1) / tpw) > AT_MAX_BLOCKS) tpw *= 2;
        int nsplit = (tiles + tpw - 1) / tpw;
        while (nsplit > 1 && part_floats(a.rows, a.qh, nsplit) > part_cap) {
            tpw *= 2;
            nsplit = (tiles + tpw - 1) / tpw;
        }
    } else {
        tpw = tiles > 0 ? tiles : 1;
    }
    a.split_pos = tpw * AT_TILE * W;
    a.nsplit = (max_span + a.split_pos - 1) / a.split_pos;
    if (a.nsplit < 1) a.nsplit = 1;
    a.nseg = n_seg;
    const int total = n_seg * a.kvh_n * a.nsplit;
    const dim3 grid((unsigned)total);
    if (max_nrows <= 4) attn_launch_mode<1, W>(a, grid, st);
    else attn_launch_mode<2, W>(a, grid, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit == 1 || a.counters) return e;
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

extern "C" hipError_t s2p_attn_plan_fused_launch(void* q, void* out, const S2pRowPlan* plan,
                                                 const S2pAttnSeg* segs, int n_seg, int rows,
                                                 int layer, int max_span, float* part,
                                                 const void* qkv, const void* qn_w,
                                                 const void* kn_w, const float* rope_tab,
                                                 float eps, unsigned* counters, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (!qkv || !rope_tab || (!qn_w) != (!kn_w)) return hipErrorInvalidValue; /* both or no norm */
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
    a.counters = counters;
    a.qkv = (const uint16_t*)qkv;
    a.qn_w = (const uint16_t*)qn_w;
    a.kn_w = (const uint16_t*)kn_w;
    a.rope_tab = rope_tab;
    a.eps = eps;
    return attn_run(a, n_seg, AT_SEG_ROWS, max_span, s2p_attn_plan_part_floats(rows, max_span),
                    st);
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
