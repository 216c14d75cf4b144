/* s2pro MI355X — transformer primitive launchers on the verify path.
 *
 * Same names, argument order and semantics as the reference contract
 * include/s2pro/kernels.h:19-58 (rms_norm, qk_norm, rope, kv_append,
 * attention, silu_mul, add).  All pointers are device pointers; launchers are
 * asynchronous on `st`, never synchronise or allocate (hipGraph-capturable),
 * return the HIP error code, and treat rows <= 0 as success.
 * bf16 tensors are passed as s2p_bf16 (one 16-bit bit pattern per element;
 * only pointers cross the ABI). */
#ifndef S2P_KERNELS_H
#define S2P_KERNELS_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct { uint16_t x; } s2p_bf16;

/* y = bf16(x * rsqrt(mean(x^2) + eps) * w), fp32 math (kernels.cu:46-77) */
hipError_t s2pk_rms_norm(const s2p_bf16* x, const s2p_bf16* w, s2p_bf16* y,
                         int rows, int width, float eps, hipStream_t st);

/* in-place per-head RMSNorm on [rows, heads, head_dim]; w == NULL is a
 * no-op (kernels.cu:81-109) */
hipError_t s2pk_qk_norm(s2p_bf16* qk, const s2p_bf16* w, int rows, int heads,
                        int head_dim, float eps, hipStream_t st);

/* in-place interleaved RoPE on q and k, positions pos..pos+rows-1, cos/sin
 * rounded through bf16 (kernels.cu:114-160) */
hipError_t s2pk_rope(s2p_bf16* q, s2p_bf16* k, int rows, int q_heads,
                     int kv_heads, int head_dim, int pos, float rope_base,
                     hipStream_t st);

/* k,v [rows, kv_heads*head_dim] -> caches [kv_heads, max_seq, head_dim] at
 * positions pos..pos+rows-1 (kernels.cu:172-209) */
hipError_t s2pk_kv_append(const s2p_bf16* k, const s2p_bf16* v,
                          s2p_bf16* k_cache, s2p_bf16* v_cache, int rows,
                          int kv_heads, int head_dim, int pos, int max_seq,
                          hipStream_t st);

/* causal GQA attention: row r sees cache positions 0..pos+r
 * (kernels.cu:234-311).  head_dim must be 128, q_heads = 4*kv_heads. */
hipError_t s2pk_attention(const s2p_bf16* q, const s2p_bf16* k_cache,
                          const s2p_bf16* v_cache, s2p_bf16* out, int rows,
                          int q_heads, int kv_heads, int head_dim, int pos,
                          int max_seq, hipStream_t st);

/* h = bf16(bf16(silu(gate)) * up), gu = [gate || up] (kernels.cu:1216-1238) */
hipError_t s2pk_silu_mul(const s2p_bf16* gu, s2p_bf16* h, int rows, int ffn,
                         hipStream_t st);

/* y = bf16(y + x) over n elements (kernels.cu:1242-1254) */
hipError_t s2pk_add(s2p_bf16* y, const s2p_bf16* x, int64_t n, hipStream_t st);

/* logits bf16 [vocab] -> fp32 scratch [vocab], exact widening: the sampler
 * contract's device staging (kernels.h:65-66, kernels.cu:1315-1322) */
hipError_t s2pk_sample_prepare(const s2p_bf16* logits, float* scratch, int vocab,
                               hipStream_t st);

/* Gather rows of an embedding table: out[i] = table[ids[i]] (reference
 * kernels.h:58-60). */
hipError_t s2pk_embed(const s2p_bf16* table, const int64_t* ids, s2p_bf16* out, int rows,
                      int dim, hipStream_t st);

/* argmax over logits [rows, vocab] -> ids[rows]; the lowest index among
 * equal maxima (reference kernels.h:68-70, the fast-AR residuals). */
hipError_t s2pk_argmax(const s2p_bf16* logits, int32_t* ids, int rows, int vocab,
                       hipStream_t st);

#ifdef __cplusplus
}
#endif
#endif
