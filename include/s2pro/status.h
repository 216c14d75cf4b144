/* s2pro MI355X — status codes and error macros.
 * Same enum values as the reference contract include/s2pro/status.h:11-22,
 * so callers compiled against the reference map errors identically. */
#ifndef S2P_STATUS_H
#define S2P_STATUS_H

#include <stdio.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    S2P_OK              = 0,
    S2P_ERR_INVALID     = -1,  /* bad argument / precondition */
    S2P_ERR_CUDA        = -2,  /* GPU runtime error (name kept for ABI parity) */
    S2P_ERR_IO          = -3,
    S2P_ERR_OOM         = -4,  /* host or device allocation failed */
    S2P_ERR_FORMAT      = -5,
    S2P_ERR_STATE       = -6,  /* API misuse / wrong lifecycle state */
    S2P_ERR_UNSUPPORTED = -7,
    S2P_ERR_INTERNAL    = -8,
    S2P_ERR_FULL        = -9,  /* capacity exhausted */
} s2p_status;

const char* s2p_status_str(s2p_status s);

#define S2P_TRY(expr)                                                          \
    do {                                                                       \
        s2p_status _s = (expr);                                                \
        if (_s != S2P_OK) return _s;                                           \
    } while (0)

/* Wrap a HIP runtime call; logs file:line on failure
 * (reference: S2P_CUDA_TRY, include/s2pro/status.h:33-41). */
#define S2P_HIP_TRY(expr)                                                      \
    do {                                                                       \
        hipError_t _e = (expr);                                                \
        if (_e != hipSuccess) {                                                \
            fprintf(stderr, "[s2pro] HIP error %s:%d: %s\n", __FILE__,         \
                    __LINE__, hipGetErrorString(_e));                          \
            return S2P_ERR_CUDA;                                               \
        }                                                                      \
    } while (0)

#ifdef __cplusplus
}
#endif
#endif
