/* s2pro MI355X — internal launch descriptor of the acceptance kernels
 * (sample.hip), shared with the C host code.  Not public ABI. */
#ifndef S2P_SAMPLE_INTERNAL_H
#define S2P_SAMPLE_INTERNAL_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>
#include "s2pro/slowar_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    const uint16_t* tgt;       /* target logits rows [n_sess*R][row_stride] */
    const uint16_t* tgt_eos;   /* NULL: full-vocab rows; else [n_sess*R] EOS logits */
    const uint16_t* drf;       /* draft logits rows, same layout */
    const uint16_t* drf_eos;
    int64_t         row_stride;
    int64_t         tgt_eos_stride; /* elements between rows' EOS logits */
    int64_t         drf_eos_stride;
    const int32_t*  parent;    /* [R] tree shape, parent[0] = -1, parent[i] < i */
    const int64_t*  tok;       /* [n_sess*R] drafted vocab ids (entry 0 unused) */
    s2ps_dev_state* const* states; /* [n_sess] */
    int             n_sess, R;
    int32_t*        out_path;  /* [n_sess*R] accepted nodes */
    int32_t*        out_n_acc; /* [n_sess] */
    int64_t*        out_emit;  /* [n_sess*(R+1)] emitted vocab ids */
    int32_t*        out_n_emit;/* [n_sess] */
    void*           work;      /* s2p_accept_work_bytes(n_sess, R) */
    const uint8_t*  chain_ok;  /* NULL, or [n_sess*R]: 0 = the node's drafted frame failed
                                  the chain condition (its token ends the walk, its row is
                                  not accepted) */
    const int*      fwd_err;   /* NULL, or the forward's error word: when it is set the
                                  logits are not trustworthy, so every session gets
                                  out_n_acc = -1, out_n_emit = 0 and its state is left
                                  as it was */
    int32_t*        out_tail;  /* NULL, or [n_sess][2]: the node whose row ended the walk
                                  (the last accepted node, or the root; its hidden produced
                                  the last emitted token unless that token is an accepted
                                  EOS node's own) and the chain-failed node whose token was
                                  emitted last (-1 if none) */
} AcceptArgs;

size_t     s2p_accept_work_bytes(int n_sess, int rows);
hipError_t s2p_accept_launch(const AcceptArgs* a, hipStream_t st);

#ifdef __cplusplus
}
#endif
#endif
