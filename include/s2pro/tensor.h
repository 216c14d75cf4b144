/* s2pro MI355X — minimal device-buffer type used by s2p_linear.
 * Field layout of the reference include/s2pro/tensor.h:13-31. */
#ifndef S2P_TENSOR_H
#define S2P_TENSOR_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>
#include "s2pro/status.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    S2P_DT_BF16 = 0,
    S2P_DT_F32  = 1,
    S2P_DT_F16  = 2,
    S2P_DT_I8   = 3,
    S2P_DT_I32  = 4,
    S2P_DT_I64  = 5,
    S2P_DT_U8   = 6,
} s2p_dtype;

size_t s2p_dtype_size(s2p_dtype dt);

typedef struct {
    void*     data;
    s2p_dtype dtype;
    int       ndim;
    int64_t   shape[4];
    size_t    bytes;
    int       on_device;
} s2p_tensor;

int64_t    s2p_tensor_numel(const s2p_tensor* t);
s2p_status s2p_tensor_device_alloc(s2p_tensor* t, s2p_dtype dt, int ndim,
                                   const int64_t* shape);
void       s2p_tensor_free(s2p_tensor* t);

#ifdef __cplusplus
}
#endif
#endif
