/* s2pro MI355X — the fast-AR residual-codebook decoder, run on each accepted
 * frame after verification.
 *
 * Replaces the reference's src/fastar/fastar.h:23-83 (its pinned cross-module
 * API: s2pfa_decode_frame_batch{,_dev}, s2pfa_vq_embed_add{,_dev}) with the
 * same per-frame loop (fastar.cu:726-789): prime the depth-11 KV cache at
 * position 0 on the backbone's FINAL-NORMED hidden (logits discarded), then
 * nine greedy steps, each fed embeddings(previous code) (the 4,096-row table;
 * step 1 takes the sampled semantic code) at position cb: 4 layers (dim 2560,
 * GQA 32/8, head_dim 128, no qk-norm, RoPE base 1e6, SwiGLU 9728), final
 * RMSNorm, the untied head Linear(2560, 4096), argmax (lowest index on ties).
 * Here the layers run on the verify engine: RMSNorm fused into GEMV staging,
 * residual adds and SwiGLU into GEMV epilogues, RoPE + K/V append +
 * attention as one plan-mode launch over every row's own cache; the plan of
 * each position is built once, so a frame is a fixed launch sequence (graph
 * capturable).  Weights are quantised linears (INT4-g32 or INT8) prepared
 * by the caller with the gemm.h API, or random (tests, benchmarks).
 * Not thread-safe: one s2pfa per stream; needs s2p_gemm_init. */
#ifndef S2P_FASTAR_H
#define S2P_FASTAR_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#include "s2pro/gemm.h"
#include "s2pro/status.h"
#include "s2pro/tensor.h"
#include "s2pro/verify.h"

#ifdef __cplusplus
extern "C" {
#endif

#define S2P_FA_LAYERS 4
#define S2P_FA_NCB 10   /* semantic + 9 residual codebooks */
#define S2P_FA_CB 4096  /* codes per codebook */
#define S2P_FA_SEQ 11   /* KV depth per frame */

typedef struct {
    s2p_linear wqkv;        /* [6144, 2560] */
    s2p_linear wo;          /* [2560, 4096] */
    s2p_linear w13;         /* [2 * 9728, 2560]: w1 rows, then w3 rows */
    s2p_linear w2;          /* [2560, 9728] */
    s2p_tensor attn_norm;   /* [2560] bf16 */
    s2p_tensor ffn_norm;    /* [2560] bf16 */
} s2pfa_layer;

typedef struct {
    s2pfa_layer layers[S2P_FA_LAYERS];
    s2p_tensor  norm;       /* final RMSNorm [2560] bf16 */
    s2p_linear  output;     /* untied head [4096, 2560] */
    s2p_tensor  cb_emb;     /* codebook_embeddings [10 * 4096, 2560] bf16 */
    s2p_tensor  emb;        /* embeddings [4096, 2560] bf16 */
} s2pfa_weights;

typedef struct s2pfa s2pfa;

/* A decoder over the caller's weights (kept, not copied or freed) for up to
 * max_b rows per frame batch. */
s2p_status s2pfa_create(s2pfa** out, const s2pfa_weights* w, int max_b, hipStream_t st);
/* The same with random weights of the model's shapes (owned, freed by
 * s2pfa_free). */
s2p_status s2pfa_create_random(s2pfa** out, s2p_weight_q quant, int max_b, uint64_t seed,
                               hipStream_t st);
void s2pfa_free(s2pfa* f);
const s2pfa_weights* s2pfa_weights_of(const s2pfa* f);

/* reference fastar.h:66-75.  hidden [B, 2560] device bf16 (final-normed),
 * sem_ids [B] HOST (0..4095); writes out_codes[b * 10 + 1 .. 9] (HOST),
 * leaves out_codes[b * 10] untouched; synchronises the stream. */
s2p_status s2pfa_decode_frame_batch(s2pfa* f, const void* hidden, const int32_t* sem_ids, int B,
                                    int32_t* out_codes, hipStream_t st);
/* reference fastar.h:77-83.  sem_dev [B] device; no sync: *stage_dev points
 * at the residual codes [9][B] (device, step-major), valid until the next
 * call. */
s2p_status s2pfa_decode_frame_batch_dev(s2pfa* f, const void* hidden, const int32_t* sem_dev,
                                        int B, const int32_t** stage_dev, hipStream_t st);
/* Test seam, no reference counterpart: the same, also writing every step's
 * head logits into logits [9][B][4096] bf16 (device). */
s2p_status s2pfa_decode_frame_logits_dev(s2pfa* f, const void* hidden, const int32_t* sem_dev,
                                         int B, const int32_t** stage_dev, void* logits,
                                         hipStream_t st);

/* reference fastar.h:46-56.  codes [10][T] codebook-major (device for _dev,
 * HOST otherwise); adds the summed 10-codebook embedding of frame t onto
 * rows[t] (device [T, 2560] bf16): f32 sum in codebook order, one bf16
 * rounding, then one bf16 add. */
s2p_status s2pfa_vq_embed_add_dev(s2pfa* f, const int32_t* codes_dev, int T, void* rows,
                                  hipStream_t st);
s2p_status s2pfa_vq_embed_add(s2pfa* f, const int32_t* codes, int T, void* rows,
                              hipStream_t st);

#ifdef __cplusplus
}
#endif
#endif
