/* s2pro MI355X — device buffers (reference src/core/tensor.c:1-127). */
#include <string.h>

#include "s2pro/tensor.h"

size_t s2p_dtype_size(s2p_dtype dt) {
    switch (dt) {
        case S2P_DT_BF16: return 2;
        case S2P_DT_F32: return 4;
        case S2P_DT_F16: return 2;
        case S2P_DT_I8: return 1;
        case S2P_DT_I32: return 4;
        case S2P_DT_I64: return 8;
        case S2P_DT_U8: return 1;
    }
    return 0;
}

int64_t s2p_tensor_numel(const s2p_tensor* t) {
    int64_t n = 1;
    for (int i = 0; i < t->ndim; i++) n *= t->shape[i];
    return n;
}

s2p_status s2p_tensor_device_alloc(s2p_tensor* t, s2p_dtype dt, int ndim, const int64_t* shape) {
    if (!t || ndim < 1 || ndim > 4) return S2P_ERR_INVALID;
    memset(t, 0, sizeof(*t));
    t->dtype = dt;
    t->ndim = ndim;
    for (int i = 0; i < ndim; i++) {
        if (shape[i] <= 0) return S2P_ERR_INVALID;
        t->shape[i] = shape[i];
    }
    t->bytes = (size_t)s2p_tensor_numel(t) * s2p_dtype_size(dt);
    if (hipMalloc(&t->data, t->bytes) != hipSuccess) {
        t->data = NULL;
        return S2P_ERR_OOM;
    }
    t->on_device = 1;
    return S2P_OK;
}

void s2p_tensor_free(s2p_tensor* t) {
    if (!t) return;
    if (t->data && t->on_device) (void)hipFree(t->data);
    memset(t, 0, sizeof(*t));
}
