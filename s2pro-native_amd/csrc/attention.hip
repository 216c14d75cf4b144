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
#ifdef AT_NO_XCD
    const int b = lin;
#else
    /* chunk x of the numbering (the first total % 8 chunks one block
     * longer) goes to XCD x; bijective for lin < total */
    const int q = total >> 3, r = total & 7, xcd = lin & 7, j = lin >> 3;
    const int b = xcd < r ? xcd * (q + 1) + j : r * (q + 1) + (xcd - r) * q + j;
#endif
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
