/* s2pro MI355X — speculative-decoding draft model (the proposal producer).
 *
 * Drop-in for the reference src/draft/draft.h:22-62 (names, struct fields,
 * argument order and status conventions kept; cudaStream_t -> hipStream_t).
 * One backbone-shaped block behind a fuse linear predicts the next
 * final-normed hidden from [h_t ; e_{t+1}] (draft.h:1-8).  Weights are the
 * trainer's bf16 draft.safetensors; the forward runs the same contract
 * kernels as the backbone (s2pk_rms_norm, s2pk_qk_norm, s2pk_rope,
 * s2pk_kv_append, s2pk_attention, s2pk_silu_mul, s2pk_add) and
 * s2p_gemm_bf16, whose bf16-weight path is this build's MFMA GEMV engine.
 * RoPE positions are per-session frame indices: a state resets with its
 * session (draft.h:54).
 */
#ifndef S2P_DRAFT_H
#define S2P_DRAFT_H

#include <hip/hip_runtime_api.h>

#include "s2pro/status.h"
#include "s2pro/tensor.h"
#include "s2pro/gemm.h"

#ifdef __cplusplus
extern "C" {
#endif

#define S2P_DRAFT_DIM 2560
#define S2P_DRAFT_FFN 9728
#define S2P_DRAFT_CTX 4096

/* reference draft.h:25-42 */
typedef struct s2p_draft_model {
    /* device bf16 weights, engine layout [out, in] */
    s2p_tensor fuse;                      /* [2560, 5120] */
    s2p_tensor wqkv;                      /* [6144, 2560] */
    s2p_tensor wo;                        /* [2560, 4096] */
    s2p_tensor w1, w3;                    /* [9728, 2560] */
    s2p_tensor w2;                        /* [2560, 9728] */
    s2p_tensor q_norm, k_norm;            /* [128] */
    s2p_tensor attn_norm, ffn_norm;       /* [2560] */
    s2p_tensor final_norm;                /* [2560] */
    /* scratch, single row */
    s2p_tensor xcat;                      /* [1, 5120] */
    s2p_tensor x, a;                      /* [1, 2560] */
    s2p_tensor qkv;                       /* [1, 6144] */
    s2p_tensor attn;                      /* [1, 4096] */
    s2p_tensor gu;                        /* [1, 2*9728] */
    s2p_tensor ffn;                       /* [1, 9728] */
} s2p_draft_model;

/* reference draft.h:44-47 */
typedef struct s2p_draft_state {
    s2p_tensor kc, vc; /* bf16 [8, S2P_DRAFT_CTX, 128] each */
    int pos;           /* frames consumed (draft rope position) */
} s2p_draft_state;

/* Load draft.safetensors (the trainer's fixed tensor names, dtype BF16,
 * shapes checked); reference draft.h:50, draft.c:73-139.  S2P_ERR_IO for an
 * unreadable file, S2P_ERR_INVALID for a missing or mis-shaped tensor. */
s2p_status s2p_draft_load(s2p_draft_model* m, const char* path);
void       s2p_draft_free(s2p_draft_model* m);

s2p_status s2p_draft_state_init(s2p_draft_state* s);
void       s2p_draft_state_free(s2p_draft_state* s);
static inline void s2p_draft_state_reset(s2p_draft_state* s) { s->pos = 0; }

/* One step (reference draft.h:56-61, draft.c:157-202): consume (h [2560
 * bf16], e [2560 bf16]) at the state's next position, emit the predicted
 * next final-normed hidden into out [2560 bf16].  All pointers
 * device-resident; asynchronous on st; advances s->pos.  S2P_ERR_INVALID
 * once the state holds S2P_DRAFT_CTX frames. */
s2p_status s2p_draft_step(s2p_draft_model* m, s2p_draft_state* s,
                          const void* h, const void* e, void* out,
                          hipStream_t st);

/* Semantic token rows of the tied head (reference config.h:45-49). */
#define S2P_TOK_EOS 151645
#define S2P_TOK_SEMANTIC_START 151678
#define S2P_DRAFT_HEAD_ROWS 4097 /* 4096 semantic rows + EOS */

/* The draft's q logits: the frozen tied-head slice scores the draft's output
 * (the predicted final-normed hidden), reference docs/SPECULATIVE.md:55-56,
 * with the slice of slowar.c:519-541 (semantic rows S2P_TOK_SEMANTIC_START
 * .. +4095, then EOS).  head is the backbone's lm head as a quantised linear
 * (INT4-g32 packed or per-channel INT8): either the 4,097-row slice itself
 * (out_features == S2P_DRAFT_HEAD_ROWS, one GEMV) or the full head
 * (out_features > S2P_TOK_SEMANTIC_START + 4095: the slice's rows are read in
 * place, two GEMVs).  hidden [rows][2560] bf16, logits [rows][4097] bf16,
 * 1 <= rows <= 16; device pointers, asynchronous on st; needs s2p_gemm_init. */
s2p_status s2p_draft_head(const s2p_linear* head, const void* hidden, void* logits, int rows,
                          hipStream_t st);

#ifdef __cplusplus
}
#endif
#endif
