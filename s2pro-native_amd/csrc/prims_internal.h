/* s2pro MI355X — internal launch descriptors of the fused verify kernels
 * (prims.hip, attention.hip), shared with the C host code.  Not public ABI. */
#ifndef S2P_PRIMS_INTERNAL_H
#define S2P_PRIMS_INTERNAL_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Per-row plan of one verify call (device arrays). */
typedef struct {
    const int32_t*  pos;          /* [rows] RoPE position */
    const int32_t*  slot;         /* [rows] KV cache slot written by the row */
    const int32_t*  sess;         /* [rows] session index */
    const uint64_t* vis;          /* [rows] visible node slots relative to L */
    void* const*    kv;           /* [n_sess] KV base, [layers][2*8][max_seq][128] (bf16),
                                   * or the INT8 / INT4 codes [layers][2*8][max_seq][128 | 64] */
    void* const*    kvs;          /* [n_sess] INT8 / INT4 caches: f16 group scales
                                   * [layers][2*8][max_seq][4] */
    int64_t         layer_stride; /* elements per layer in a session KV */
    int             max_seq;
} S2pRowPlan;

/* Attention segment: up to 8 consecutive rows sharing one cache. */
typedef struct {
    int32_t sess;   /* session index (KV base in plan.kv) */
    int32_t L;      /* prefix length: slots [0, L) visible to every row */
    int32_t row0;   /* first row */
    int32_t nrows;  /* rows in this segment (<= 8) */
    int32_t span;   /* slots [0, span) may be visible to some row */
    int32_t first;  /* the session's first row (its node 0, KV slot L) */
    const void* kv; /* the session's KV base (plan.kv[sess]), so the kernel has it at hand */
} S2pAttnSeg;

/* The fused qkv rows as the wqkv GEMM left them when its K-split merge was
 * deferred (splits > 0): fp32 partials [splits][M][nrb][64], element (row,
 * n) at part[((k * M + row) * nrb + n / 64) * 64 + n % 64]; a consumer sums
 * them in split order from 0 and rounds to bf16 (the merge's value) and
 * stores the result into the qkv rows as the merge would have.  splits = 0:
 * the qkv rows hold the merged values. */
typedef struct {
    const float* part;
    int splits, M, nrb;
} S2pQkvParts;

/* s2p_qkrope_append_launch with (cos, sin) from a RoPE table [rows][64][2]
 * (s2p_rope_tab_launch of the same plan) */
hipError_t s2p_qkrope_append_tab_launch(const void* qkv, void* q_out, const void* qn_w,
                                        const void* kn_w, const S2pRowPlan* plan, int rows,
                                        int layer, float eps, const float* rope_tab,
                                        hipStream_t st);
/* the same over the wqkv GEMM's deferred partials (qkv receives the merged rows) */
hipError_t s2p_qkrope_append_tab_parts_launch(void* qkv, const S2pQkvParts* parts, void* q_out,
                                              const void* qn_w, const void* kn_w,
                                              const S2pRowPlan* plan, int rows, int layer,
                                              float eps, const float* rope_tab, hipStream_t st);
hipError_t s2p_qkrope_append_launch(const void* qkv, void* q_out, const void* qn_w,
                                    const void* kn_w, const S2pRowPlan* plan, int rows,
                                    int layer, float eps, float base, hipStream_t st);
/* Fast-AR: step input x[r] = table[clamp(ids[r])] plus its sums of squares
 * ([width/16][128]); the 10-codebook VQ embedding added onto rows. */
hipError_t s2p_fa_embed_ssq_launch(const void* table, const int32_t* ids, int n_ids, void* x,
                                   float* ssq, int rows, int width, hipStream_t st);
hipError_t s2p_fa_vq_embed_add_launch(const void* table, const int32_t* codes, int T, void* rows,
                                      int dim, hipStream_t st);
/* Draft step prologue: the one-row plan (pos/slot/sess/vis/kv arrays behind
 * the plan's pointers) and segment at position pos over the cache at kv,
 * the RoPE row into tab [64][2], zeros into x [nx] bf16 and ctr [nctr].
 * pos_dev != NULL: the position is *pos_dev + pos, read on the device and
 * clamped to [0, pos_max). */
hipError_t s2p_draft_prologue_launch(const S2pRowPlan* plan, S2pAttnSeg* seg, void* kv, int pos,
                                     const int32_t* pos_dev, int pos_max, float base,
                                     float* tab, void* x, int nx, unsigned* ctr, int nctr,
                                     hipStream_t st);
/* Move accepted tree nodes' K/V from slot L + node to L + depth. */
hipError_t s2p_kv_commit_launch(const S2pRowPlan* plan, const int32_t* path,
                                const int32_t* n_acc, int n_sess, int R, int n_layers,
                                hipStream_t st);
hipError_t s2p_resid_init_launch(const void* xin, void* x, float* ssq, int rows,
                                 int width, hipStream_t st);
/* (cos, sin) of every row's position and pair i < 64: tab [rows][64][2] */
hipError_t s2p_rope_tab_launch(const S2pRowPlan* plan, int rows, float base, float* tab,
                               hipStream_t st);

/* Verify-plan attention over the per-layer caches of the plan's sessions.
 * segs: device [n_seg]; max_span: host bound of max(span) (grid sizing);
 * part: scratch of s2p_attn_plan_part_floats(rows, max_span) floats. */
hipError_t s2p_attn_plan_launch(const void* q, void* out, const S2pRowPlan* plan,
                                const S2pAttnSeg* segs, int n_seg, int rows, int layer,
                                int max_span, float* part, hipStream_t st);
/* The same, fused with qk-norm + RoPE + KV append (q is the scratch the q
 * rows are written to) and, with counters ([n_seg * 8], zero between calls),
 * with the split merge done by the last split of each block. */
/* qn_w = kn_w = NULL: RoPE without qk-norm (a model without qk-norm) */
/* Tree attention over bf16 caches (csrc/attention.hip): segs [n_seg] hold
 * one segment a session of max_nrows <= 32 rows; q holds the roped rows
 * (k_qkrope_append ran); partials in part (part_cap floats), merged into
 * out by k_attn_combine. */
hipError_t s2p_attn_tree_launch(const void* q, void* out, const S2pRowPlan* plan,
                                const S2pAttnSeg* segs, int n_seg, int rows, int max_nrows,
                                int layer, int max_span, float* part, int64_t part_cap,
                                hipStream_t st);
hipError_t s2p_attn_plan_fused_launch(void* q, void* out, const S2pRowPlan* plan,
                                      const S2pAttnSeg* segs, int n_seg, int rows, int layer,
                                      int max_span, float* part, const void* qkv,
                                      const void* qn_w, const void* kn_w, const float* rope_tab,
                                      float eps, unsigned* counters, hipStream_t st);
int64_t    s2p_attn_plan_part_floats(int rows, int max_span);

/* The verify plan over INT8 / INT4 (bw 8 / 4) session caches (kv8.hip): codes
 * plan.kv[s] [layers][16][max_seq][bw == 8 ? 128 : 64] (K heads, then V) and
 * f16 scales plan.kvs[s] [layers][16][max_seq][4]. */
int64_t    s2p_attn8_plan_part_floats(int rows, int max_span);
/* qk-norm + RoPE (positions from rope_tab) + quantise-on-append */
hipError_t s2p_qkrope_append8_launch(const void* qkv, void* q_out, const void* qn_w,
                                     const void* kn_w, const S2pRowPlan* plan, int rows,
                                     int layer, float eps, const float* rope_tab, int bw,
                                     hipStream_t st);
/* split attention over the plan's segments (matrix cores) + the combine
 * into out; part holds s2p_attn8_plan_part_floats(rows, max_span) floats */
hipError_t s2p_attn8_plan_launch(const void* q, void* out, const S2pRowPlan* plan,
                                 const S2pAttnSeg* segs, int n_seg, int rows, int layer,
                                 int max_span, float* part, int bw, hipStream_t st);
hipError_t s2p_kv_commit8_launch(const S2pRowPlan* plan, const int32_t* path,
                                 const int32_t* n_acc, int n_sess, int R, int n_layers, int bw,
                                 hipStream_t st);

/* the chain condition of speculative frames (verify.c s2p_verify_chain):
 * gather each drafted node's parent hidden row and semantic code; compare
 * the fast-AR codes (stage [9][n_sess (R - 1)]) with the drafted ones */
/* *out = *word (0: the forward completed, else a bounded wait timed out; a
 * NULL word reads 0); clear != 0 also resets the word */
hipError_t s2p_word_status_launch(int* word, int32_t* out, int clear, hipStream_t st);
hipError_t s2p_chain_prep_launch(const int32_t* parent, const int64_t* tok, const void* hidden,
                                 void* par_hidden, int32_t* sem, int n_sess, int R, int dim,
                                 hipStream_t st);
hipError_t s2p_chain_check_launch(const int32_t* stage, const int32_t* draft_codes,
                                  const int64_t* tok, uint8_t* chain_ok, int32_t* codes_out,
                                  int n_sess, int R, hipStream_t st);

#ifdef __cplusplus
}
#endif
#endif
