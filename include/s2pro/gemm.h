/* s2pro MI355X — quantised linear layers and raw weight-only GEMV primitives.
 *
 * Drop-in for the reference contract include/s2pro/gemm.h (names, argument
 * order, layouts and error behaviour kept).  Convention (row-major):
 * x [M, in] bf16, w [out, in], y [M, out] bf16, y = x * w^T, fp32 accumulate.
 *
 * Differences from the reference, all MI355X-side:
 *  - one GEMV engine (MFMA with in-register dequantisation) serves every M;
 *    the reference's M > 16 dequant + cuBLAS fallback (gemm.c:467-490) is not
 *    needed and s2p_linear_forward runs the same kernel for M up to
 *    S2P_GEMV_MAX_M_MFMA;
 *  - the FP8 path (fish-scales-ops, gemm.h:13-27) is out of scope and
 *    s2p_linear_forward returns S2P_ERR_UNSUPPORTED for S2P_GEMM_FP8;
 *  - loaders from safetensors are out of scope; linears are created from
 *    device bf16 weights (then quantised) or generated directly in the
 *    quantised format (s2p_linear_init_random_*).
 * Streams are hipStream_t; bf16/f16 tensors cross the ABI as void*.
 */
#ifndef S2P_GEMM_H
#define S2P_GEMM_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>
#include "s2pro/status.h"
#include "s2pro/tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    S2P_GEMM_BF16 = 0,   /* unquantised bf16 weights (s2p_gemm_bf16) */
    S2P_GEMM_FP8  = 1,   /* out of scope */
    S2P_GEMM_INT8 = 2,   /* weight-only INT8 per channel / INT4 group-wise */
} s2p_gemm_mode;

/* Largest M accepted by s2p_int8_gemv / s2p_int4p_gemv / s2p_intq_gemv
 * (reference gemm.h:32-34). */
#define S2P_INT8_GEMV_MAX_M 16
/* Largest M served by s2p_linear_forward / s2p_int4p_gemm_tc. */
#define S2P_GEMV_MAX_M_MFMA 128

/* Process-wide GEMV context: split-K partial buffers and arrival counters
 * (reference gemm.c:57-73).  Must be called once before any GEMV, with the
 * stream-ordering rule that GEMV calls issued on different streams must not
 * overlap in time (they share the split-K scratch), as the reference
 * serialises its shared scratch behind one mutex.  max_m is a sizing hint. */
s2p_status s2p_gemm_init(int max_m);
void       s2p_gemm_shutdown(void);

typedef struct {
    int        in_features;
    int        out_features;
    s2p_tensor w_bf16;        /* [out, in] bf16, dropped after quantisation */
    s2p_tensor w_fp8;         /* unused (FP8 out of scope); kept for layout */
    s2p_tensor w_scales;      /* unused */
    int        fp8_ready;
    s2p_tensor w_int8;        /* [out, in] int8 (per-channel, or container) */
    s2p_tensor w_iscale;      /* q_group==0: [out] f32; >0: [out, in/G] f16 */
    s2p_tensor w_pack;        /* [out, in/2] packed nibbles (q_packed only) */
    int        int8_ready;
    int        q_group;       /* 0 = per-channel INT8, else group size */
    int        q_packed;      /* 1 = two 4-bit weights per byte */
} s2p_linear;

typedef enum {
    S2P_QSITE_BACKBONE = 0,
    S2P_QSITE_FASTAR   = 1,
} s2p_qsite;

/* Wrap an existing device bf16 weight [out, in] (ownership moves to lin). */
s2p_status s2p_linear_from_device_bf16(s2p_linear* lin, void* w_bf16,
                                       int in_features, int out_features);
/* Quantise w_bf16 -> per-channel INT8 sidecar, free w_bf16
 * (reference gemm.c:267-304).  Synchronises `stream`. */
s2p_status s2p_linear_prepare_int8(s2p_linear* lin, hipStream_t stream);
/* Policy variant (reference gemm.c:369-373): backbone -> INT4-g32 packed
 * with the MSE clip search, fast-AR -> per-channel INT8. */
s2p_status s2p_linear_prepare_int8_site(s2p_linear* lin, s2p_qsite site,
                                        hipStream_t stream);
s2p_status s2p_linear_forward(const s2p_linear* lin, const void* x_bf16,
                              void* y_bf16, int M, s2p_gemm_mode mode,
                              hipStream_t stream);
void       s2p_linear_free(s2p_linear* lin);

/* Random-init linears directly in the quantised formats (synthetic
 * workloads): INT4 values uniform in [-7,7] (the quantiser's symmetric code
 * range, zero mean), f16 group scales |N(0,sigma)|;
 * or INT8 values uniform in [-127,127] with f32 row scales |N(0,sigma)|.
 * Deterministic in (seed). */
s2p_status s2p_linear_init_random_int4(s2p_linear* lin, int in_features,
                                       int out_features, int G, float sigma,
                                       uint64_t seed, hipStream_t stream);
s2p_status s2p_linear_init_random_int8(s2p_linear* lin, int in_features,
                                       int out_features, float sigma,
                                       uint64_t seed, hipStream_t stream);

/* Raw bf16 GEMM for non-quantised matmuls (reference gemm.h:93-96, cuBLAS
 * there): y[M,N] = x[M,K] * w[N,K]^T, bf16 in/out, fp32 accumulate. */
s2p_status s2p_gemm_bf16(const void* x, const void* w, void* y, int M, int N,
                         int K, hipStream_t stream);

/* ---- raw primitives (reference src/sched/int8_gemv.cu) ------------------ */

/* w_i8[N,K], scales[N] = per-row absmax/127 RTN (int8_gemv.cu:32-58). */
s2p_status s2p_int8_quant(void* w_i8, float* scales, const void* w_bf16,
                          int N, int K, hipStream_t stream);
/* y[M,N] = x[M,K] * (w_i8 * scales)^T; M <= 16, K % 512 == 0
 * (int8_gemv.cu:964-986). */
s2p_status s2p_int8_gemv(void* y_bf16, const void* x_bf16, const void* w_i8,
                         const float* scales, int M, int N, int K,
                         hipStream_t stream);
s2p_status s2p_int8_dequant(void* w_bf16, const void* w_i8,
                            const float* scales, int N, int K,
                            hipStream_t stream);

/* Group-wise symmetric quantiser with optional per-group MSE clip search
 * (int8_gemv.cu:135-195, 752-770). */
s2p_status s2p_intq_quant(void* w_i8, void* scales_f16, const void* w_bf16,
                          int N, int K, int G, int levels, int mse,
                          hipStream_t stream);
s2p_status s2p_intq_gemv(void* y_bf16, const void* x_bf16, const void* w_i8,
                         const void* scales_f16, int M, int N, int K, int G,
                         hipStream_t stream);
s2p_status s2p_intq_dequant(void* w_bf16, const void* w_i8,
                            const void* scales_f16, int N, int K, int G,
                            hipStream_t stream);

/* Packed INT4: byte i of a row holds k=2i (low nibble) and k=2i+1 (high),
 * two's complement (int8_gemv.cu:255-277). */
s2p_status s2p_int4_pack(void* w_pack, const void* w_i8, int N, int K,
                         hipStream_t stream);
/* M <= 16, K % 512 == 0, G power of two >= 16 dividing K
 * (int8_gemv.cu:836-902). */
s2p_status s2p_int4p_gemv(void* y_bf16, const void* x_bf16,
                          const void* w_pack, const void* scales_f16, int M,
                          int N, int K, int G, hipStream_t stream);
/* Same GEMV for 1 <= M <= 128, K % 64 == 0 (int8_gemv.cu:907-929). */
s2p_status s2p_int4p_gemm_tc(void* y_bf16, const void* x_bf16,
                             const void* w_pack, const void* scales_f16,
                             int M, int N, int K, int G, hipStream_t stream);
/* Test seam, no counterpart in the reference: one INT4-g32 (wfmt 0: packed
 * codes, f16 scales [N][K/32]) or INT8 (wfmt 1: f32 per-row scales) GEMV,
 * 1 <= M <= 128, K % 512 == 0, with the engine chosen per call (0: the
 * launcher's choice, 2: the split-K engine only), so that the split-K engine
 * is exercised on shapes the launcher gives to another engine. */
s2p_status s2p_gemv_engine_run(int engine, int wfmt, void* y_bf16,
                               const void* x_bf16, const void* w,
                               const void* scales, int M, int N, int K,
                               hipStream_t stream);
/* No counterpart in the reference: s2p_int4p_gemm_tc for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  G == 32, K % 128 == 0,
 * 1 <= M <= 128, N <= 262144.  The split partials (8 MiB) and arrival
 * counters live in a fixed per-GPU device array instead of the context
 * scratch, so s2p_gemm_init is not needed and nothing is allocated; sizes
 * beyond the array return S2P_ERR_INVALID with a message.  Calls that overlap
 * on one GPU share the array and race: serialise them. */
s2p_status s2p_int4p_gemm_tc_noalloc(void* y_bf16, const void* x_bf16,
                                     const void* w_pack, const void* scales_f16,
                                     int M, int N, int K, int G,
                                     hipStream_t stream);
s2p_status s2p_int4p_dequant(void* w_bf16, const void* w_pack,
                             const void* scales_f16, int N, int K, int G,
                             hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
