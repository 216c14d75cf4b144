/* s2pro MI355X — speculative verify pass for the slow-AR backbone.
 *
 * New API (the reference designed but never built this stage:
 * docs/SPECULATIVE.md:249-256).  It follows the reference contract
 * conventions: s2p_status returns, device pointers, an explicit stream, no
 * host synchronisation or allocation inside the per-step calls, so a whole
 * verify step can be captured in one hipGraph and replayed.
 *
 * A verify step takes n_sess sessions that share one draft shape of R rows:
 * row 0 is the root (the last accepted token, whose K/V is not in the cache
 * yet) and rows 1..R-1 are drafted nodes with parent[i] < i (a chain
 * parent[i] = i-1 for K-token drafts, or a tree).  For session s with kv_len
 * L tokens in its cache, node i is written to KV slot L + i, has RoPE
 * position L + depth(i), and attends slots [0, L) plus the slots of its
 * ancestors and itself.  This is the reference's decode contract extended to
 * rows: s2pk_kv_append(rows=K+1, pos=L) + s2pk_attention(rows=K+1, pos=L)
 * (kernels.cu:172-209, 250) for the chain.  After acceptance the cache holds
 * the accepted path at L + 1 .. L + n (s2p_verify_kv_commit moves tree nodes
 * there) and the session's kv_len advances by 1 + n_accepted: rejected slots
 * are simply overwritten later (rollback by length, slowar.c:751).
 */
#ifndef S2P_VERIFY_H
#define S2P_VERIFY_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#include "s2pro/gemm.h"
#include "s2pro/slowar_kernels.h"
#include "s2pro/status.h"
#include "s2pro/tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

#define S2P_DIM 2560
#define S2P_Q_HEADS 32
#define S2P_KV_HEADS 8
#define S2P_HEAD_DIM 128
#define S2P_QKV_WIDTH 6144
#define S2P_FFN_DIM 9728
#define S2P_VOCAB 155776
#define S2P_HEAD_SLICE 4097 /* 4096 semantic rows + EOS */
#define S2P_VERIFY_MAX_ROWS 64 /* R per session (visibility masks are 64-bit) */

/* One backbone layer (reference src/slowar/slowar_internal.h:72-81). */
typedef struct {
    s2p_linear wqkv;    /* [6144, 2560] fused q,k,v */
    s2p_linear wo;      /* [2560, 4096] */
    s2p_linear gate_up; /* [19456, 2560] = w1 rows then w3 rows */
    s2p_linear w2;      /* [2560, 9728] */
    s2p_tensor attn_norm, ffn_norm; /* [2560] bf16 */
    s2p_tensor q_norm, k_norm;      /* [128] bf16 */
} s2p_slow_layer;

typedef enum { S2P_WQ_INT4_G32 = 0, S2P_WQ_INT8 = 1 } s2p_weight_q;

typedef struct {
    int          n_layers;      /* 36 for the S2-Pro backbone */
    s2p_weight_q quant;         /* backbone linears */
    s2p_weight_q head_quant;    /* lm head */
    int          head_rows;     /* S2P_VOCAB (full head) or S2P_HEAD_SLICE */
    int          max_rows;      /* rows per verify call: sessions x R (<= 128) */
    int          max_sessions;
    int          ctx_len;       /* per-session KV capacity (slots) */
    int          kv_bits;       /* KV cache: 0 or 16 = bf16; 8 / 4 = INT8 / INT4 with
                                 * f16 scales per 32 dims (kernels.cu:510-946) */
} s2p_backbone_opts;

typedef struct s2p_backbone s2p_backbone;

/* Random-init backbone (synthetic workloads): INT4-g32 codes uniform in
 * [-8,7] with f16 group scales |N(0, sigma)|, or INT8 codes uniform with f32
 * row scales |N(0, sigma)|, sigma chosen so the weights have rms 1/sqrt(in)
 * (the scale of trained projections); norm weights bf16 1 + N(0,0.02).
 * Calls s2p_gemm_init.  Synchronises `st`. */
s2p_status s2p_backbone_create_random(const s2p_backbone_opts* opts, uint64_t seed,
                                      hipStream_t st, s2p_backbone** out);
void       s2p_backbone_free(s2p_backbone* b);
s2p_slow_layer* s2p_backbone_layer(s2p_backbone* b, int layer);
s2p_linear*     s2p_backbone_head(s2p_backbone* b);
void*           s2p_backbone_final_norm(s2p_backbone* b);
/* bytes of one session's KV: [n_layers][2 * 8][ctx_len][128] bf16, or with
 * kv_bits 8 / 4 the codes [n_layers][2 * 8][ctx_len][128 or 64] int8 */
size_t          s2p_backbone_kv_bytes(const s2p_backbone* b);
/* bytes of one session's f16 group scales [n_layers][2 * 8][ctx_len][4]
 * (kv_bits 8 / 4; 0 for a bf16 cache) */
size_t          s2p_backbone_kv_scale_bytes(const s2p_backbone* b);
/* weight bytes streamed by one verify step (backbone + head) */
size_t          s2p_backbone_weight_bytes(const s2p_backbone* b);

typedef struct {
    int            n_sess;
    int            rows;     /* R */
    const int32_t* parent;   /* host [R]; parent[0] = -1 */
    void* const*   kv;       /* host [n_sess] device KV bases: bf16 [layers][16][ctx][128];
                              * INT8 / INT4 codes [layers][16][ctx][128 | 64] */
    const int32_t* kv_len;   /* host [n_sess] */
    void* const*   kv_scales;/* host [n_sess] device bases of the INT8 / INT4 caches' f16
                              * group scales [layers][16][ctx][4] (the reference session's
                              * separate kvs tensor, slowar_internal.h:177-179, 208-225);
                              * NULL for a bf16 cache */
} s2p_verify_batch;

/* Upload the per-row plan (positions, slots, visibility) and per-session KV
 * bases.  Host -> device copy; call outside graph capture, before each step
 * whose plan changed.  Fails with S2P_ERR_FULL if a session would overflow
 * ctx_len. */
s2p_status s2p_verify_plan(s2p_backbone* b, const s2p_verify_batch* vb, hipStream_t st);

/* Re-plan the current shape (same sessions, caches and draft shape) from
 * device KV lengths kv_len_dev [n_sess]: every row's position and slot,
 * each segment's prefix and the RoPE table, on the device.  Asynchronous,
 * capturable, no host copy: consecutive verify steps replayed from one graph
 * can advance their sessions (kv_len += 1 + n_accepted) without a host round
 * trip.  Lengths must stay within the span the last s2p_verify_plan sized
 * its launches for (the largest L + R of that plan rounded up to 512, at
 * most ctx_len): a session with L + R beyond it keeps its previous plan and
 * sets *overflow = 1 (overflow may be NULL); re-plan on the host before
 * that. */
s2p_status s2p_verify_plan_device(s2p_backbone* b, const int32_t* kv_len_dev, int32_t* overflow,
                                  hipStream_t st);

/* Verify forward over the planned rows: x_in [n_sess*R, 2560] bf16 input
 * embeddings (read only); logits [n_sess*R, head_rows] bf16.  Appends every
 * row's K/V to its slot.  Asynchronous, capturable.
 *
 * Plans of at most 6 rows over bf16 caches with INT4 weights run as ONE
 * persistent launch of one workgroup per CU whose workgroups exchange data
 * through flags in memory.  That needs every workgroup resident at once:
 * while the forward runs, no other kernel may occupy the device's CUs (do
 * not overlap it with work on another stream, e.g. a draft step).  Each wait
 * is bounded; if one gives up (its producers were not resident), the launch
 * still completes but its logits are not valid and the backbone's error word
 * is set: s2p_verify_step then reports out_n_acc = -1 for every session, and
 * s2p_verify_status reads the word.  The word stays set (every later forward
 * also drains without waiting) until s2p_verify_status clears it or a new
 * plan is uploaded. */
s2p_status s2p_verify_forward(s2p_backbone* b, const void* x_in, void* logits, hipStream_t st);

/* Status of the forwards since the word was last cleared, written to out
 * (device or pinned host memory): 0 = every forward completed, 1 = a bounded
 * wait of the persistent kernel timed out (logits invalid).  clear != 0
 * resets the word.  Asynchronous (no host sync), capturable; with the
 * layer-by-layer forward it always writes 0. */
s2p_status s2p_verify_status(s2p_backbone* b, int32_t* out, int clear, hipStream_t st);

/* Workspace of s2p_verify_accept. */
size_t s2p_verify_accept_work_bytes(int n_sess, int rows);

/* Acceptance (device).  tgt/drf rows follow s2pk_sample's layout (full vocab
 * with eos == NULL, else 4096 semantic logits + eos[row]); draft row i holds
 * the draft logits whose samples are node i's children; parent [R] and tok
 * [n_sess*R] (drafted vocab ids, entry 0 of each session unused) and states
 * [n_sess] are device arrays.  Writes the accepted node ids (out_path
 * [n_sess*R]), their count, the emitted vocab ids (out_emit [n_sess*(R+1)]:
 * accepted drafts then the corrected or bonus token) and their count, and
 * advances each state.  Asynchronous, capturable. */
s2p_status s2p_verify_accept(const void* tgt_logits, const void* tgt_eos, const void* drf_logits,
                             const void* drf_eos, int64_t row_stride, const int32_t* parent,
                             const int64_t* tok, s2ps_dev_state* const* states, int n_sess,
                             int rows, int32_t* out_path, int32_t* out_n_acc, int64_t* out_emit,
                             int32_t* out_n_emit, void* work, hipStream_t st);

/* The chain condition of speculative frames (reference docs/SPECULATIVE.md:
 * 26-41: a drafted frame survives only if its semantic token is accepted AND
 * the nine greedy residual codes the fast-AR gives on the true hidden equal
 * the codes the draft built the next input from).  For every drafted node
 * (row s*R + i, i >= 1) of the current plan: the greedy fast-AR frame on the
 * final-normed hidden of its parent's row from the last forward (the
 * backbone's final RMSNorm of its residual rows) with the node's semantic
 * code (tok - 151678; 0 for EOS); parent [R] and tok [n_sess*R] as for
 * s2p_verify_accept (device).  chain_ok [n_sess*R] (device): 1 for
 * roots, EOS nodes, and nodes whose codes equal draft_codes [n_sess*R][9]
 * (device); codes_out [n_sess*R][9] (device): the fast-AR codes of every
 * drafted node (the emitted frame's codes), zeros for roots.  Needs
 * n_sess*(R-1) <= the decoder's max_b.  Asynchronous, capturable. */
typedef struct s2pfa s2pfa;
s2p_status s2p_verify_chain(s2p_backbone* b, s2pfa* fa, const int32_t* parent, const int64_t* tok,
                            const int32_t* draft_codes, uint8_t* chain_ok, int32_t* codes_out,
                            hipStream_t st);

/* s2p_verify_accept under the chain condition: chain_ok as written by
 * s2p_verify_chain (NULL: every node passes).  An accepted node whose frame
 * failed ends the walk: its token is the last emitted id, the node is not in
 * out_path (its forward row had the wrong input, so its K/V is not
 * committed) and no bonus token is drawn. */
s2p_status s2p_verify_accept_chain(const void* tgt_logits, const void* tgt_eos,
                                   const void* drf_logits, const void* drf_eos,
                                   int64_t row_stride, const int32_t* parent, const int64_t* tok,
                                   s2ps_dev_state* const* states, int n_sess, int rows,
                                   const uint8_t* chain_ok, int32_t* out_path, int32_t* out_n_acc,
                                   int64_t* out_emit, int32_t* out_n_emit, void* work,
                                   hipStream_t st);

/* Move the K/V of accepted tree nodes from slot L + node to L + depth for
 * every layer (no-op for chains).  Uses the current plan. */
s2p_status s2p_verify_kv_commit(s2p_backbone* b, const int32_t* out_path,
                                const int32_t* out_n_acc, hipStream_t st);

/* One verify step (forward + acceptance) replayed from a hipGraph captured
 * on first use for the current plan shape; falls back to eager launches
 * when use_graph == 0.  When the forward's error word is set (see
 * s2p_verify_forward) the acceptance decides nothing: out_n_acc[s] = -1,
 * out_n_emit[s] = 0 and the sampler states are left unchanged. */
typedef struct {
    const void* x_in;
    void* logits;                       /* target logits out */
    const void* drf_logits;             /* draft rows, layout of the target logits */
    int64_t drf_stride;                 /* == head rows */
    const int32_t* parent_dev;
    const int64_t* tok_dev;
    s2ps_dev_state* const* states_dev;
    int32_t* out_path;
    int32_t* out_n_acc;
    int64_t* out_emit;
    int32_t* out_n_emit;
    void* work;
} s2p_verify_step_io;

s2p_status s2p_verify_step(s2p_backbone* b, const s2p_verify_step_io* io, int use_graph,
                           hipStream_t st);

#ifdef __cplusplus
}
#endif
#endif
