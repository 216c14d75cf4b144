/* s2pro MI355X — launchers of the speculative tick's device bookkeeping
 * (spec.hip), shared with the C host code.  Not public ABI. */
#ifndef S2P_SPEC_INTERNAL_H
#define S2P_SPEC_INTERNAL_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#include "prims_internal.h"
#include "s2pro/slowar_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int n_sess, R;
    const int32_t* n_acc;     /* [n] */
    const int32_t* n_emit;    /* [n] */
    const int64_t* emit;      /* [n][R+1] */
    const int32_t* path;      /* [n][R] */
    const int32_t* tail;      /* [n][2] (k_accept_walk) */
    const int32_t* codes_out; /* [n*R][9] chain condition's fast-AR codes */
    const int32_t* stage;     /* [9][n] the bonus frames' residual codes */
    const uint16_t* hidden;   /* [n*R][2560] final-normed verify rows */
    int32_t* frames;          /* [n][R+1][10] out */
    int32_t* kv_len;          /* [n] in/out */
    int64_t* prev_tok;        /* [n] in/out */
    int32_t* prev_codes;      /* [n][10] in/out */
    void* prev_hidden;        /* [n][2560] in/out */
    uint8_t* done;            /* [n] in/out */
} SpecAdvanceArgs;

hipError_t s2p_plan_device_launch(int32_t* pos, int32_t* slot, S2pAttnSeg* segs, int n_seg,
                                  const int32_t* kv_len, const int32_t* depth, int n_sess, int R,
                                  int cap, int32_t* overflow, hipStream_t st);
hipError_t s2p_spec_begin_launch(const void* table, const void* cb, const int64_t* prev_tok,
                                 const int32_t* prev_codes, void* x, int n_sess, int R, float scale,
                                 s2ps_dev_state* const* states, s2ps_dev_state* dstates,
                                 hipStream_t st);
hipError_t s2p_spec_frame_launch(const void* table, const void* cb, const int64_t* tok_d,
                                 const int32_t* stage, int n_sess, int R, int i, int64_t* tok,
                                 int32_t* draft_codes, void* x, float scale, hipStream_t st);
hipError_t s2p_spec_pick_launch(const int32_t* tail, const int64_t* emit, const int32_t* n_emit,
                                const void* hidden, int n_sess, int R, void* bonus_hidden,
                                int32_t* bonus_sem, hipStream_t st);
hipError_t s2p_spec_advance_launch(const SpecAdvanceArgs* a, hipStream_t st);

#ifdef __cplusplus
}
#endif
#endif
