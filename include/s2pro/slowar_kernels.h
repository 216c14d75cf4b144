/* s2pro MI355X — batched-decode launchers and the device sampler.
 *
 * Mirrors the reference private header src/slowar/slowar_kernels.h:29-173 for
 * the functions on the verify path (qkv_split, rope_pos, kv_append_ptrs,
 * attention_ptrs, attention_decode, the device sampler state and
 * s2pk_sample).  Conventions as in kernels.h. */
#ifndef S2P_SLOWAR_KERNELS_H
#define S2P_SLOWAR_KERNELS_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>
#include "s2pro/kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

/* fused qkv [rows, q_width + 2*kv_width] -> q, k, v (kernels.cu:1368-1395) */
hipError_t s2pk_qkv_split(const s2p_bf16* qkv, s2p_bf16* q, s2p_bf16* k,
                          s2p_bf16* v, int rows, int q_width, int kv_width,
                          hipStream_t st);

/* RoPE with per-row positions pos[rows] (kernels.cu:162-168) */
hipError_t s2pk_rope_pos(s2p_bf16* q, s2p_bf16* k, int rows, int q_heads,
                         int kv_heads, int head_dim, const int32_t* pos,
                         float rope_base, hipStream_t st);

/* row r writes k/v at position pos[r] of k_caches[r]/v_caches[r]
 * (kernels.cu:211-222) */
hipError_t s2pk_kv_append_ptrs(const s2p_bf16* k, const s2p_bf16* v,
                               s2p_bf16* const* k_caches,
                               s2p_bf16* const* v_caches, int rows,
                               int kv_heads, int head_dim, const int32_t* pos,
                               int max_seq, hipStream_t st);

/* row r attends cache[0..pos[r]] of its own caches (kernels.cu:313-330) */
hipError_t s2pk_attention_ptrs(const s2p_bf16* q,
                               const s2p_bf16* const* k_caches,
                               const s2p_bf16* const* v_caches, s2p_bf16* out,
                               int rows, int q_heads, int kv_heads,
                               int head_dim, const int32_t* pos, int max_seq,
                               hipStream_t st);

/* split-K flash-decode variant (kernels.cu:491-508).  max_len = max over
 * rows of pos[r]+1; part = device scratch of at least
 * s2pk_attention_part_floats(rows, q_heads, max_len) floats. */
hipError_t s2pk_attention_decode(const s2p_bf16* q,
                                 const s2p_bf16* const* k_caches,
                                 const s2p_bf16* const* v_caches,
                                 s2p_bf16* out, int rows, int q_heads,
                                 int kv_heads, int head_dim,
                                 const int32_t* pos, int max_seq, int max_len,
                                 float* part, hipStream_t st);
/* scratch size (floats) required by s2pk_attention_decode */
int64_t s2pk_attention_part_floats(int rows, int q_heads, int max_len);

/* INT8 / INT4 KV cache (reference slowar_kernels.h:76-120, kernels.cu:510-946).
 * Payload [kv_heads][max_seq][bw == 8 ? head_dim : head_dim / 2] bytes
 * (bw 4: element 2b in the low nibble), scales f16 [kv_heads][max_seq]
 * [head_dim / 32]; head_dim 128, bw 8 or 4.  Quantise-on-append: per
 * 32-group scale f16(absmax / QMAX), values rint(x / scale) clamped to
 * +-QMAX (127 or 7).  Scale pointers cross the ABI as void* (f16). */
/* rows at positions pos..pos+rows-1 of one cache (kernels.cu:583-600) */
hipError_t s2pk_kv_append8(const s2p_bf16* k, const s2p_bf16* v, int8_t* k_cache,
                           int8_t* v_cache, void* k_scale, void* v_scale, int rows,
                           int kv_heads, int head_dim, int pos, int max_seq, int bw,
                           hipStream_t st);
/* row r at position pos[r] of its own caches (kernels.cu:602-620) */
hipError_t s2pk_kv_append8_ptrs(const s2p_bf16* k, const s2p_bf16* v,
                                int8_t* const* k_caches, int8_t* const* v_caches,
                                void* const* k_scales, void* const* v_scales, int rows,
                                int kv_heads, int head_dim, const int32_t* pos, int max_seq,
                                int bw, hipStream_t st);
/* causal single pass over one quantised cache, rows at pos.. (kernels.cu:724-746) */
hipError_t s2pk_attention8(const s2p_bf16* q, const int8_t* k_cache, const int8_t* v_cache,
                           const void* k_scale, const void* v_scale, s2p_bf16* out, int rows,
                           int q_heads, int kv_heads, int head_dim, int pos, int max_seq, int bw,
                           hipStream_t st);
/* split decode, row r attends its caches [0..pos[r]]; part holds
 * s2pk_attention_part_floats(rows, q_heads, max_len) floats (kernels.cu:751-946) */
hipError_t s2pk_attention8_decode(const s2p_bf16* q, const int8_t* const* k_caches,
                                  const int8_t* const* v_caches, const void* const* k_scales,
                                  const void* const* v_scales, s2p_bf16* out, int rows,
                                  int q_heads, int kv_heads, int head_dim, const int32_t* pos,
                                  int max_seq, int max_len, float* part, int bw,
                                  hipStream_t st);

/* Per-session sampler state, device resident; byte layout of the reference
 * s2ps_dev_state (slowar_kernels.h:132-142). */
typedef struct {
    int64_t  prev[64];       /* repetition/RAS window, oldest first */
    uint64_t count;          /* uncapped emitted count == step counter */
    uint64_t rng[4];         /* xoshiro256** state (unseeded path) */
    float    temperature, top_p, rep_penalty;
    int32_t  window, seeded;
    uint32_t seed31;
    uint32_t pad_;
} s2ps_dev_state;

/* One block per row: the reference two-softmax semantic sampler
 * (sampling.c:119-282, kernels.cu:979-1181) with the rule's exp/log of
 * s2p_fmath.h, so draws are bit-identical to the host rule.  eos_logits ==
 * NULL: rows are full-vocab (stride vocab_stride), candidates gathered at
 * their vocab ids; else rows hold the 4096 semantic logits and
 * eos_logits[r] the EOS logit.  Writes out_tok (i64), out_sem (i32),
 * out_codes[r*10] (i32, may be NULL), out_eos (u8) and advances the state. */
hipError_t s2pk_sample(const s2p_bf16* logits, int64_t vocab_stride,
                       const s2p_bf16* eos_logits,
                       s2ps_dev_state* const* states, int rows,
                       int64_t* out_tok, int32_t* out_sem, int32_t* out_codes,
                       uint8_t* out_eos, hipStream_t st);

#ifdef __cplusplus
}
#endif
#endif
