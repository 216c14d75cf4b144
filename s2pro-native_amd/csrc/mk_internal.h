/* s2pro MI355X — descriptors of the persistent verify kernel (verify_mk.hip),
 * shared with the C host code (verify.c).  Not public ABI. */
#ifndef S2P_MK_INTERNAL_H
#define S2P_MK_INTERNAL_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#include "gemv_internal.h"
#include "prims_internal.h"

#ifdef __cplusplus
extern "C" {
#endif

/* one GEMV of the step, planned for the kernel's grid: virtual grid (P, S) */
typedef struct {
    GemvArgs a;
    int P, S;
} MkGemv;

typedef struct {
    MkGemv g[4]; /* wqkv (NORM attn_norm, STORE qkv), wo (RESID x), gate_up (NORM
                    ffn_norm, SWIGLU h), w2 (RESID x) */
    const uint16_t* q_norm;
    const uint16_t* k_norm;
} MkLayer;

#define MK_MAX_GROUPS 64
/* barrier state (uint64 words, monotonic across launches): per group an
 * arrival counter and a release word, plus the top counter; every word on
 * its own 4 KiB stride so that they spread over memory channels */
#define MK_BAR_STRIDE 512
#define MK_BAR_WORDS ((2 * MK_MAX_GROUPS + 1) * MK_BAR_STRIDE)

typedef struct {
    const MkLayer* layers; /* device [n_layers] */
    int n_layers;
    const MkGemv* head;    /* device */
    int wfmt;
    uint16_t* x;           /* residual stream [rows][2560] */
    float* ssq_a;          /* sums of squares of x, [160][128] */
    float* ssq_b;
    uint16_t* qkv;
    uint16_t* q;
    uint16_t* attn;
    float* rope_tab;       /* [rows][64][cos, sin] of the plan's positions */
    int rows;
    float eps, rope_base;
    /* attention */
    S2pRowPlan plan;
    const S2pAttnSeg* segs;
    int n_seg;
    int nsplit, split_pos;
    int attn_mqt2;           /* some segment has > 4 rows: two 16-query tiles */
    float* attn_part;
    unsigned* attn_counters; /* [n_seg * 8], zero between calls */
    /* synchronisation */
    uint64_t* bar;           /* MK_BAR_WORDS */
    uint64_t* ts;            /* optional [2 + 6 n_layers]: wall clock after each phase */
    uint64_t* ts_wg;         /* optional [barriers][2][nwg]: per-workgroup arrival and
                                departure wall clock (diagnostics) */
    int dbg_attn_twice;
    uint64_t* probe;         /* diagnostics: [nwg][8] GEMV stage clocks of phase probe_phase */
    int probe_phase;      /* diagnostics: run the attention phase twice (the second
                                pass stamps the slot of the following barrier) */
    int* err;                /* sticky: a barrier wait timed out */
} MkArgs;

/* grid of the persistent kernel on the current device: workgroups that are
 * co-resident, and the dynamic LDS bytes; 0 on success */
int s2p_mk_grid(int* nwg, size_t* lds);
/* plan one GEMV for `nwg` workgroups; fails if it would need LDS windows */
hipError_t s2p_mk_plan_gemv(const GemvArgs* a, int nwg, size_t lds_cap, MkGemv* out);
/* args_dev: the MkArgs in device memory (read by the kernel) */
hipError_t s2p_mk_launch(const MkArgs* args_dev, int wfmt, const void* x_in, void* logits,
                         int nwg, size_t lds, hipStream_t st);

#ifdef __cplusplus
}
#endif
#endif
