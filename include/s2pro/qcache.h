/* s2pro MI355X — prequantized-weight sidecar cache.
 *
 * Drop-in for the reference include/s2pro/qcache.h (names, argument order,
 * status conventions and the on-disk layout of src/sched/qcache.c:1-16 kept;
 * cudaStream_t -> hipStream_t).  The cache stores the final quantised
 * device tensors of the linears (per-channel INT8, packed INT4-g32, INT4 in
 * an int8 container) so that later starts upload them instead of
 * re-quantising: same bytes in GPU memory.  A file written by either build
 * is read by the other.
 *
 * Staleness guard: FNV-1a 64 over the quantisation config string (mode and
 * the S2P_INT4* knobs) and the sorted (name, size, mtime) of the model
 * directory's *.safetensors.  A mismatch, or any read error, leaves the cache
 * in write mode (the caller quantises live and the file is rewritten).
 *
 * Env: S2P_QCACHE=0 disables; S2P_QCACHE_DIR overrides the cache location
 * (default: the model directory). */
#ifndef S2P_QCACHE_H
#define S2P_QCACHE_H

#include <hip/hip_runtime_api.h>

#include "s2pro/gemm.h"
#include "s2pro/status.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct s2p_qcache s2p_qcache;

/* reference qcache.h:31-33.  *out == NULL (S2P_OK) when caching is disabled
 * or the mode carries no quantised tensors; a valid matching file puts the
 * cache in read mode, otherwise it collects entries for s2p_qcache_finish. */
s2p_status s2p_qcache_open(const char* model_dir, s2p_gemm_mode mode, s2p_qcache** out);

/* reference qcache.h:35 */
int s2p_qcache_reading(const s2p_qcache* qc);

/* reference qcache.h:39-42.  Read mode: 1 = hit (lin populated, quant flags
 * set), 0 = miss or any error.  Write mode: 0. */
int s2p_qcache_try_load(s2p_qcache* qc, const char* name, int in_features, int out_features,
                        s2p_linear* lin, hipStream_t stream);

/* reference qcache.h:46-47.  Write mode: snapshot a prepared linear (syncs
 * the stream, copies device -> host).  Read mode or unquantised: no-op. */
s2p_status s2p_qcache_put_linear(s2p_qcache* qc, const char* name, const s2p_linear* lin,
                                 hipStream_t stream);

/* reference qcache.h:51.  Read mode: release the file mapping (after the
 * stream's uploads complete).  Write mode: write the entries atomically. */
s2p_status s2p_qcache_finish(s2p_qcache* qc, hipStream_t stream);

/* reference qcache.h:53 */
void s2p_qcache_free(s2p_qcache* qc);

#ifdef __cplusplus
}
#endif
#endif
