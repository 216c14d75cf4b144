/* s2pro MI355X — quantised linear layers (reference src/sched/gemm.c) and
 * the raw GEMV entry points of include/s2pro/gemm.h.
 *
 * One process-wide context (reference gemm.c:42-73) owns the split-K partial
 * buffer and the per-row-block arrival counters of the GEMV engine; GEMVs
 * issued on one stream reuse them in order.  The split count of each call is
 * chosen so that about 4 workgroups per CU stream the weights while each
 * split covers at least 8 groups of 32 k. */
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "s2pro/gemm.h"
#include "../gemv_internal.h"
#include "../synth_internal.h"

#define CTX_PART_FLOATS (16u << 20) /* 64 MiB of split-K partials */
#define CTX_COUNTERS (1u << 16)

static struct {
    int inited;
    pthread_mutex_t mu;
    int max_m;
    float* part;
    unsigned* counters;
} g = {0, PTHREAD_MUTEX_INITIALIZER, 0, NULL, NULL};

s2p_status s2p_gemm_init(int max_m) {
    pthread_mutex_lock(&g.mu);
    if (g.inited) {
        pthread_mutex_unlock(&g.mu);
        return S2P_OK;
    }
    s2p_status rc = S2P_OK;
    if (hipMalloc((void**)&g.part, sizeof(float) * CTX_PART_FLOATS) != hipSuccess ||
        hipMalloc((void**)&g.counters, sizeof(unsigned) * CTX_COUNTERS) != hipSuccess) {
        rc = S2P_ERR_OOM;
    } else if (hipMemset(g.counters, 0, sizeof(unsigned) * CTX_COUNTERS) != hipSuccess ||
               hipDeviceSynchronize() != hipSuccess) {
        rc = S2P_ERR_CUDA;
    }
    if (rc != S2P_OK) {
        if (g.part) (void)hipFree(g.part);
        if (g.counters) (void)hipFree(g.counters);
        g.part = NULL;
        g.counters = NULL;
        pthread_mutex_unlock(&g.mu);
        return rc;
    }
    g.max_m = max_m > 0 ? max_m : 16;
    g.inited = 1;
    pthread_mutex_unlock(&g.mu);
    return S2P_OK;
}

void s2p_gemm_shutdown(void) {
    pthread_mutex_lock(&g.mu);
    if (g.inited) {
        (void)hipDeviceSynchronize();
        (void)hipFree(g.part);
        (void)hipFree(g.counters);
        g.part = NULL;
        g.counters = NULL;
        g.inited = 0;
    }
    pthread_mutex_unlock(&g.mu);
}

/* internal accessors for the verify forward (same scratch, same rules) */
float* s2p_gemm_ctx_part(void) { return g.part; }
int64_t s2p_gemm_ctx_part_cap(void) { return CTX_PART_FLOATS; }
unsigned* s2p_gemm_ctx_counters(void) { return g.counters; }
int s2p_gemm_ctx_ready(void) { return g.inited; }

/* Fill the descriptor of a plain GEMV on the context scratch. */
void s2p_gemv_args_plain(GemvArgs* a, int wfmt, const void* w, const void* s, const void* x,
                         void* y, int M, int N, int K) {
    memset(a, 0, sizeof(*a));
    a->w = (const uint8_t*)w;
    a->s = s;
    a->x = (const uint16_t*)x;
    a->ldx = K;
    a->y = (uint16_t*)y;
    a->ldy = N;
    a->M = M;
    a->N = N;
    a->K = K;
    a->wfmt = wfmt;
    a->gps = 0; /* the launcher sizes the splits */
    a->xmode = GEMV_X_PLAIN;
    a->epi = GEMV_EPI_STORE;
    a->part = g.part;
    a->part_cap = CTX_PART_FLOATS;
    a->counters = g.counters;
}

static s2p_status run_gemv(const GemvArgs* a, hipStream_t st) {
    hipError_t e = s2p_gemv_launch(a, st);
    if (e != hipSuccess) {
        fprintf(stderr, "[s2pro] gemv launch (M=%d,N=%d,K=%d): %s\n", a->M, a->N, a->K,
                hipGetErrorString(e));
        return S2P_ERR_CUDA;
    }
    return S2P_OK;
}

static int gshift_of(int G) {
    if (G < 16 || (G & (G - 1)) != 0) return -1;
    int s = 0;
    while ((1 << s) < G) s++;
    return s;
}

/* ------------------------------------------------------------ raw GEMVs */

s2p_status s2p_gemm_bf16(const void* x, const void* w, void* y, int M, int N, int K,
                         hipStream_t stream) {
    if (!x || !w || !y || M <= 0 || N <= 0 || K <= 0) return S2P_ERR_INVALID;
    if (!g.inited) return S2P_ERR_STATE;
    hipError_t e = hipSuccess;
    if (K % 128 == 0) {
        /* whole-K engine, in row chunks whose activations fit in LDS */
        int mc = M < GEMV_MAX_M ? M : GEMV_MAX_M;
        for (int m0 = 0; m0 < M;) {
            const int rows = M - m0 < mc ? M - m0 : mc;
            GemvArgs a;
            s2p_gemv_args_plain(&a, GEMV_W_BF16, w, NULL, (const uint16_t*)x + (size_t)m0 * K,
                                (uint16_t*)y + (size_t)m0 * N, rows, N, K);
            e = s2p_gemv_launch(&a, stream);
            if (e == hipErrorNotSupported && mc > 1) {
                mc = (mc + 1) / 2;
                continue;
            }
            if (e != hipSuccess) break;
            m0 += rows;
        }
        if (e == hipSuccess) return S2P_OK;
        if (e != hipErrorNotSupported) {
            fprintf(stderr, "[s2pro] gemm_bf16 (M=%d,N=%d,K=%d): %s\n", M, N, K,
                    hipGetErrorString(e));
            return S2P_ERR_CUDA;
        }
    }
    e = s2p_gemv_bf16_generic_launch(w, x, y, M, N, K, stream);
    return e == hipSuccess ? S2P_OK : S2P_ERR_CUDA;
}

s2p_status s2p_int8_gemv(void* y_bf16, const void* x_bf16, const void* w_i8, const float* scales,
                         int M, int N, int K, hipStream_t stream) {
    if (!y_bf16 || !x_bf16 || !w_i8 || !scales || M <= 0 || N <= 0 || K <= 0)
        return S2P_ERR_INVALID;
    if (M > S2P_INT8_GEMV_MAX_M || K % 512 != 0) return S2P_ERR_INVALID;
    if (!g.inited) return S2P_ERR_STATE;
    GemvArgs a;
    s2p_gemv_args_plain(&a, GEMV_W_INT8, w_i8, scales, x_bf16, y_bf16, M, N, K);
    return run_gemv(&a, stream);
}

static s2p_status int4p_any_m(void* y, const void* x, const void* w, const void* sc, int M, int N,
                              int K, int G, hipStream_t stream) {
    if (!g.inited) return S2P_ERR_STATE;
    if (G == 32 && K % 128 == 0) {
        GemvArgs a;
        s2p_gemv_args_plain(&a, GEMV_W_INT4, w, sc, x, y, M, N, K);
        return run_gemv(&a, stream);
    }
    hipError_t e = s2p_gemv_generic_launch(0, w, sc, x, y, M, N, K, gshift_of(G), stream);
    return e == hipSuccess ? S2P_OK : S2P_ERR_CUDA;
}

s2p_status s2p_gemv_engine_run(int engine, int wfmt, void* y_bf16, const void* x_bf16,
                               const void* w, const void* scales, int M, int N, int K,
                               hipStream_t stream) {
    if (!y_bf16 || !x_bf16 || !w || !scales || M <= 0 || M > GEMV_MAX_M || N <= 0 ||
        K <= 0 || K % 512 != 0 || (engine != GEMV_ENGINE_AUTO && engine != GEMV_ENGINE_SPLITK) ||
        (wfmt != GEMV_W_INT4 && wfmt != GEMV_W_INT8))
        return S2P_ERR_INVALID;
    if (!g.inited) return S2P_ERR_STATE;
    GemvArgs a;
    s2p_gemv_args_plain(&a, wfmt, w, scales, x_bf16, y_bf16, M, N, K);
    a.engine = engine;
    return run_gemv(&a, stream);
}

s2p_status s2p_int4p_gemv(void* y_bf16, const void* x_bf16, const void* w_pack,
                          const void* scales_f16, int M, int N, int K, int G,
                          hipStream_t stream) {
    if (!y_bf16 || !x_bf16 || !w_pack || !scales_f16 || M <= 0 || N <= 0 || K <= 0)
        return S2P_ERR_INVALID;
    const int gs = gshift_of(G);
    if (M > S2P_INT8_GEMV_MAX_M || K % 512 != 0 || gs < 0 || K % G != 0) return S2P_ERR_INVALID;
    return int4p_any_m(y_bf16, x_bf16, w_pack, scales_f16, M, N, K, G, stream);
}

s2p_status s2p_int4p_gemm_tc(void* y_bf16, const void* x_bf16, const void* w_pack,
                             const void* scales_f16, int M, int N, int K, int G,
                             hipStream_t stream) {
    const int gs = gshift_of(G);
    if (!y_bf16 || !x_bf16 || !w_pack || !scales_f16 || M <= 0 || M > S2P_GEMV_MAX_M_MFMA ||
        N <= 0 || K <= 0 || K % 64 != 0 || gs < 0 || K % G != 0)
        return S2P_ERR_INVALID;
    return int4p_any_m(y_bf16, x_bf16, w_pack, scales_f16, M, N, K, G, stream);
}

s2p_status s2p_intq_gemv(void* y_bf16, const void* x_bf16, const void* w_i8,
                         const void* scales_f16, int M, int N, int K, int G,
                         hipStream_t stream) {
    if (!y_bf16 || !x_bf16 || !w_i8 || !scales_f16 || M <= 0 || N <= 0 || K <= 0)
        return S2P_ERR_INVALID;
    const int gs = gshift_of(G);
    if (M > S2P_INT8_GEMV_MAX_M || K % 512 != 0 || gs < 0 || K % G != 0) return S2P_ERR_INVALID;
    if (!g.inited) return S2P_ERR_STATE;
    hipError_t e = s2p_gemv_generic_launch(1, w_i8, scales_f16, x_bf16, y_bf16, M, N, K, gs,
                                           stream);
    return e == hipSuccess ? S2P_OK : S2P_ERR_CUDA;
}

/* ------------------------------------------------------------- linears */

s2p_status s2p_linear_from_device_bf16(s2p_linear* lin, void* w_bf16, int in_features,
                                       int out_features) {
    if (!lin || !w_bf16 || in_features <= 0 || out_features <= 0) return S2P_ERR_INVALID;
    memset(lin, 0, sizeof(*lin));
    lin->in_features = in_features;
    lin->out_features = out_features;
    lin->w_bf16.data = w_bf16;
    lin->w_bf16.dtype = S2P_DT_BF16;
    lin->w_bf16.ndim = 2;
    lin->w_bf16.shape[0] = out_features;
    lin->w_bf16.shape[1] = in_features;
    lin->w_bf16.bytes = (size_t)in_features * out_features * 2;
    lin->w_bf16.on_device = 1;
    return S2P_OK;
}

/* reference gemm.c:267-304 */
s2p_status s2p_linear_prepare_int8(s2p_linear* lin, hipStream_t stream) {
    if (!lin) return S2P_ERR_INVALID;
    if (lin->int8_ready) return S2P_OK;
    if (!lin->w_bf16.data) return S2P_ERR_INVALID;
    const int N = lin->out_features, K = lin->in_features;
    if (K % 512 != 0) return S2P_OK; /* not servable; stays bf16 (reference behaviour) */
    int64_t qshape[2] = {N, K};
    S2P_TRY(s2p_tensor_device_alloc(&lin->w_int8, S2P_DT_I8, 2, qshape));
    int64_t sshape[1] = {N};
    s2p_status rc = s2p_tensor_device_alloc(&lin->w_iscale, S2P_DT_F32, 1, sshape);
    if (rc == S2P_OK)
        rc = s2p_int8_quant(lin->w_int8.data, (float*)lin->w_iscale.data, lin->w_bf16.data, N, K,
                            stream);
    if (rc == S2P_OK && hipStreamSynchronize(stream) != hipSuccess) rc = S2P_ERR_CUDA;
    if (rc != S2P_OK) {
        s2p_tensor_free(&lin->w_int8);
        s2p_tensor_free(&lin->w_iscale);
        return rc;
    }
    lin->int8_ready = 1;
    lin->q_group = 0;
    s2p_tensor_free(&lin->w_bf16);
    return S2P_OK;
}

/* reference gemm.c:308-373: backbone -> INT4-g32 packed with MSE clip */
s2p_status s2p_linear_prepare_int8_site(s2p_linear* lin, s2p_qsite site, hipStream_t stream) {
    if (!lin) return S2P_ERR_INVALID;
    if (site == S2P_QSITE_FASTAR) return s2p_linear_prepare_int8(lin, stream);
    if (lin->int8_ready) return S2P_OK;
    if (!lin->w_bf16.data) return S2P_ERR_INVALID;
    const int N = lin->out_features, K = lin->in_features, G = 32;
    if (K % 512 != 0 || K % G != 0) return S2P_OK;
    int64_t qshape[2] = {N, K};
    S2P_TRY(s2p_tensor_device_alloc(&lin->w_int8, S2P_DT_I8, 2, qshape));
    int64_t sshape[1] = {(int64_t)N * (K / G)};
    s2p_status rc = s2p_tensor_device_alloc(&lin->w_iscale, S2P_DT_F16, 1, sshape);
    if (rc == S2P_OK)
        rc = s2p_intq_quant(lin->w_int8.data, lin->w_iscale.data, lin->w_bf16.data, N, K, G, 7, 1,
                            stream);
    int64_t pshape[2] = {N, K / 2};
    if (rc == S2P_OK) rc = s2p_tensor_device_alloc(&lin->w_pack, S2P_DT_U8, 2, pshape);
    if (rc == S2P_OK) rc = s2p_int4_pack(lin->w_pack.data, lin->w_int8.data, N, K, stream);
    if (rc == S2P_OK && hipStreamSynchronize(stream) != hipSuccess) rc = S2P_ERR_CUDA;
    if (rc != S2P_OK) {
        s2p_tensor_free(&lin->w_int8);
        s2p_tensor_free(&lin->w_iscale);
        s2p_tensor_free(&lin->w_pack);
        return rc;
    }
    s2p_tensor_free(&lin->w_int8);
    lin->q_packed = 1;
    lin->int8_ready = 1;
    lin->q_group = G;
    s2p_tensor_free(&lin->w_bf16);
    return S2P_OK;
}

/* reference gemm.c:424-501; every M up to S2P_GEMV_MAX_M_MFMA runs the GEMV
 * engine (no dequant round trip) */
s2p_status s2p_linear_forward(const s2p_linear* lin, const void* x_bf16, void* y_bf16, int M,
                              s2p_gemm_mode mode, hipStream_t stream) {
    if (!lin || !x_bf16 || !y_bf16 || M <= 0) return S2P_ERR_INVALID;
    if (!g.inited) return S2P_ERR_STATE;
    if (mode == S2P_GEMM_BF16 || (mode == S2P_GEMM_INT8 && !lin->int8_ready)) {
        /* bf16 weights (reference gemm.c:493-500: also the fallback for
         * layers without a quantised copy) */
        if (!lin->w_bf16.data) return S2P_ERR_STATE;
        return s2p_gemm_bf16(x_bf16, lin->w_bf16.data, y_bf16, M, lin->out_features,
                             lin->in_features, stream);
    }
    if (mode != S2P_GEMM_INT8) return S2P_ERR_UNSUPPORTED;
    if (M > S2P_GEMV_MAX_M_MFMA) return S2P_ERR_INVALID;
    const int N = lin->out_features, K = lin->in_features;
    if (lin->q_packed)
        return int4p_any_m(y_bf16, x_bf16, lin->w_pack.data, lin->w_iscale.data, M, N, K,
                           lin->q_group, stream);
    if (lin->q_group > 0) {
        hipError_t e = s2p_gemv_generic_launch(1, lin->w_int8.data, lin->w_iscale.data, x_bf16,
                                               y_bf16, M, N, K, gshift_of(lin->q_group), stream);
        return e == hipSuccess ? S2P_OK : S2P_ERR_CUDA;
    }
    GemvArgs a;
    s2p_gemv_args_plain(&a, GEMV_W_INT8, lin->w_int8.data, lin->w_iscale.data, x_bf16, y_bf16, M,
                        N, K);
    return run_gemv(&a, stream);
}

void s2p_linear_free(s2p_linear* lin) {
    if (!lin) return;
    s2p_tensor_free(&lin->w_bf16);
    s2p_tensor_free(&lin->w_fp8);
    s2p_tensor_free(&lin->w_scales);
    s2p_tensor_free(&lin->w_int8);
    s2p_tensor_free(&lin->w_iscale);
    s2p_tensor_free(&lin->w_pack);
    lin->fp8_ready = 0;
    lin->int8_ready = 0;
    lin->q_group = 0;
    lin->q_packed = 0;
}

s2p_status s2p_linear_init_random_int4(s2p_linear* lin, int in_features, int out_features, int G,
                                       float sigma, uint64_t seed, hipStream_t stream) {
    if (!lin || in_features <= 0 || out_features <= 0 || gshift_of(G) < 0 || in_features % G)
        return S2P_ERR_INVALID;
    memset(lin, 0, sizeof(*lin));
    lin->in_features = in_features;
    lin->out_features = out_features;
    int64_t pshape[2] = {out_features, in_features / 2};
    S2P_TRY(s2p_tensor_device_alloc(&lin->w_pack, S2P_DT_U8, 2, pshape));
    int64_t sshape[1] = {(int64_t)out_features * (in_features / G)};
    s2p_status rc = s2p_tensor_device_alloc(&lin->w_iscale, S2P_DT_F16, 1, sshape);
    if (rc == S2P_OK &&
        (s2p_synth_int4(lin->w_pack.data, (int64_t)lin->w_pack.bytes, seed, stream) != hipSuccess ||
         s2p_synth_f16_absnormal(lin->w_iscale.data, sshape[0], sigma, seed ^ 0x5CA1E5ULL,
                                 stream) != hipSuccess))
        rc = S2P_ERR_CUDA;
    if (rc != S2P_OK) {
        s2p_linear_free(lin);
        return rc;
    }
    lin->int8_ready = 1;
    lin->q_group = G;
    lin->q_packed = 1;
    return S2P_OK;
}

s2p_status s2p_linear_init_random_int8(s2p_linear* lin, int in_features, int out_features,
                                       float sigma, uint64_t seed, hipStream_t stream) {
    if (!lin || in_features <= 0 || out_features <= 0) return S2P_ERR_INVALID;
    memset(lin, 0, sizeof(*lin));
    lin->in_features = in_features;
    lin->out_features = out_features;
    int64_t qshape[2] = {out_features, in_features};
    S2P_TRY(s2p_tensor_device_alloc(&lin->w_int8, S2P_DT_I8, 2, qshape));
    int64_t sshape[1] = {out_features};
    s2p_status rc = s2p_tensor_device_alloc(&lin->w_iscale, S2P_DT_F32, 1, sshape);
    if (rc == S2P_OK &&
        (s2p_synth_int8(lin->w_int8.data, (int64_t)lin->w_int8.bytes, seed, stream) != hipSuccess ||
         s2p_synth_f32_absnormal(lin->w_iscale.data, out_features, sigma, seed ^ 0x5CA1E5ULL,
                                 stream) != hipSuccess))
        rc = S2P_ERR_CUDA;
    if (rc != S2P_OK) {
        s2p_linear_free(lin);
        return rc;
    }
    lin->int8_ready = 1;
    lin->q_group = 0;
    return S2P_OK;
}
