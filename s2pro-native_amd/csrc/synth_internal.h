/* s2pro MI355X — synthetic-data launchers (synth.hip), exported for tests and
 * benchmarks that build random-init workloads on the device. */
#ifndef S2P_SYNTH_INTERNAL_H
#define S2P_SYNTH_INTERNAL_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

hipError_t s2p_synth_bytes(void* p, int64_t n, uint64_t seed, hipStream_t st);
/* packed INT4 codes: both nibbles of each byte uniform over -7..7 (the
 * symmetric code range of the reference quantiser, zero mean) */
hipError_t s2p_synth_int4(void* p, int64_t n, uint64_t seed, hipStream_t st);
hipError_t s2p_synth_int8(void* p, int64_t n, uint64_t seed, hipStream_t st);
hipError_t s2p_synth_f16_absnormal(void* p, int64_t n, float sigma, uint64_t seed,
                                   hipStream_t st);
hipError_t s2p_synth_f32_absnormal(void* p, int64_t n, float sigma, uint64_t seed,
                                   hipStream_t st);
hipError_t s2p_synth_bf16_normal(void* p, int64_t n, float mean, float sd, uint64_t seed,
                                 hipStream_t st);

#ifdef __cplusplus
}
#endif
#endif
