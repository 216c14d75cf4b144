/* s2pro MI355X — internal launch descriptor of the GEMV engine (gemv.hip),
 * shared by the C host code (gemm.c, verify.c).  Not part of the public ABI. */
#ifndef S2P_GEMV_INTERNAL_H
#define S2P_GEMV_INTERNAL_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GEMV_MAX_M 128         /* rows per call (8 MFMA column tiles) */
#define GEMV_SSQ_COLS 16       /* columns per sum-of-squares block */

enum { GEMV_W_INT4 = 0, GEMV_W_INT8 = 1, GEMV_W_BF16 = 2 }; /* weight formats */
enum { GEMV_X_PLAIN = 0, GEMV_X_NORM = 1 };            /* activation staging */
/* STORE: y = bf16(W x); RESID: y = bf16(y + bf16(W x)) plus per-16-column
 * sums of squares; SWIGLU: W = [gate; up] (2F rows), y[m][F] =
 * silu(bf16(gate)) * bf16(up) with the rule's roundings. */
enum { GEMV_EPI_STORE = 0, GEMV_EPI_RESID = 1, GEMV_EPI_SWIGLU = 2 };
enum { GEMV_ENGINE_AUTO = 0, GEMV_ENGINE_SPLITK = 2 };

typedef struct {
    const uint8_t*  w;       /* INT4: packed [N][K/2]; INT8: [N][K]; BF16: bf16 [N][K] */
    const void*     s;       /* INT4: f16 [N][K/32]; INT8: f32 [N]; BF16: unused */
    const uint16_t* x;       /* bf16 activations, row stride ldx */
    int             ldx;
    uint16_t*       y;       /* bf16 output (or residual stream), stride ldy */
    int             ldy;
    int             M, N, K;
    int             wfmt;
    int             gps;     /* 32-k groups per split (multiple of 4); 0 = auto */
    int             splits;  /* derived by the launcher */
    int             win;     /* derived: staged groups per LDS window */
    int             nrb;     /* derived: 64-row blocks */
    int             ks;      /* derived (whole-K engine): K slices = waves per 16-row tile */
    int             rt;      /* derived (whole-K engine): 16-row tiles per tile group */
    int             xmode;
    const uint16_t* norm_w;  /* NORM: bf16 [K] */
    float           norm_eps;
    const float*    ssq_in;  /* NORM: [ssq_in_blocks][GEMV_MAX_M] */
    int             ssq_in_blocks;
    int             epi;
    float*          ssq_out; /* RESID: [ceil(N/16)][GEMV_MAX_M] (may be NULL) */
    float*          part;    /* [splits][M][nrb][64] fp32 */
    int64_t         part_cap;/* floats available at part */
    unsigned*       counters;/* [ceil(N/64)], zero between calls */
    int             engine;  /* GEMV_ENGINE_AUTO, or GEMV_ENGINE_SPLITK: the split-K engine only */
    const float*    inv_in;  /* NORM (k_gemm4): the rows' inverse RMS, [M], when the producer
                              * wrote it (NULL: computed here) */
    float*          inv_out; /* RESID: also write the output rows' inverse RMS, [M] (NULL: no) */
    float           inv_eps; /* RESID with inv_out: the epsilon of the norm that follows */
    int*            deferred;/* STORE (host pointer, may be NULL): a K-split k_gemm4 launch
                              * leaves its partials [splits][M][ceil(N/64)][64] in part
                              * unmerged and stores the split count here, else 0; the
                              * consumer sums them in split order (the merge's values) */
#ifdef S2P_DIAG
    uint64_t*       probe;   /* diagnostics build (whole-K engine): [grid][8] stage clocks */
#endif
} GemvArgs;

hipError_t s2p_gemv_launch(const GemvArgs* a, hipStream_t st);
/* INT4, 16 < M <= 96 (gemm4.hip); hipErrorNotSupported outside that range */
hipError_t s2p_gemm4_launch(const GemvArgs* a, hipStream_t st);
/* inv[m] = the rule's inverse RMS of row m < M from per-16-column sums of
 * squares ssq [blocks][GEMV_MAX_M] of rows of K values (gemm4.hip) */
hipError_t s2p_g4_rms_launch(const float* ssq, int blocks, int M, int K, float eps, float* inv,
                             hipStream_t st);
/* resident-workgroup target the split-K engine plans for (4 per CU) */
int s2p_gemv_slots(void);
/* compute units of the current device, queried once per device */
int s2p_cu_count(void);
hipError_t s2p_gemv_bf16_generic_launch(const void* w, const void* x, void* y, int M, int N,
                                         int K, hipStream_t st);
hipError_t s2p_gemv_generic_launch(int fmt, const void* w, const void* sc,
                                   const void* x, void* y, int M, int N, int K,
                                   int gshift, hipStream_t st);

#ifdef __cplusplus
}
/* work decomposition for `slots` resident workgroups (gemv.hip) */
extern "C" hipError_t s2p_gemv_plan(GemvArgs* a, int slots, dim3* grid, size_t* lds);
#endif
#endif
