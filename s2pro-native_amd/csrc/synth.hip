/* s2pro MI355X — deterministic synthetic data on the device (random-init
 * weights, activations, KV caches of the benchmark workloads).  Every value
 * is a function of (seed, element index) through splitmix64, so a buffer is
 * reproducible independently of the launch shape. */
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "common.h"
#include "synth_internal.h"

S2P_DEV uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
S2P_DEV uint64_t h64(uint64_t seed, uint64_t i, uint64_t lane) {
    return mix64(seed * 0x9E3779B97F4A7C15ULL + i * 0xD1B54A32D192ED03ULL + lane * 0x8CB92BA72F3D8DD7ULL + 1);
}
/* standard normal from two hashed uniforms (Box-Muller, binary64) */
S2P_DEV double normal_of(uint64_t seed, uint64_t i) {
    const double u1 = ((double)(h64(seed, i, 0) >> 11) + 1.0) * 0x1.0p-53; /* (0, 1] */
    const double u2 = (double)(h64(seed, i, 1) >> 11) * 0x1.0p-53;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925 * u2);
}

enum { SY_BYTES = 0, SY_INT8 = 1, SY_F16_ABSN = 2, SY_F32_ABSN = 3, SY_BF16_N = 4, SY_INT4 = 5 };

__global__ __launch_bounds__(256) void k_synth(void* p, int64_t n, int kind, float a, float b,
                                               uint64_t seed) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        switch (kind) {
            case SY_BYTES: {
                ((uint8_t*)p)[i] = (uint8_t)(h64(seed, (uint64_t)i, 2) >> 56);
                break;
            }
            case SY_INT4: { /* two nibbles, each uniform over -7..7 (zero mean) */
                const uint64_t h = h64(seed, (uint64_t)i, 3);
                const int lo = (int)((h >> 8) % 15ULL) - 7, hi = (int)((h >> 40) % 15ULL) - 7;
                ((uint8_t*)p)[i] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
                break;
            }
            case SY_INT8: {
                ((int8_t*)p)[i] = (int8_t)((int)(h64(seed, (uint64_t)i, 2) % 255ULL) - 127);
                break;
            }
            case SY_F16_ABSN:
                ((uint16_t*)p)[i] = f2h((float)fabs(normal_of(seed, (uint64_t)i) * (double)a));
                break;
            case SY_F32_ABSN:
                ((float*)p)[i] = (float)fabs(normal_of(seed, (uint64_t)i) * (double)a);
                break;
            default: /* bf16 normal(mean a, sd b) */
                ((uint16_t*)p)[i] = f2bf((float)((double)a + (double)b * normal_of(seed, (uint64_t)i)));
                break;
        }
    }
}

static hipError_t run(void* p, int64_t n, int kind, float a, float b, uint64_t seed,
                      hipStream_t st) {
    if (n <= 0) return hipSuccess;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_synth, dim3((unsigned)blocks), dim3(256), 0, st, p, n, kind, a, b, seed);
    return hipGetLastError();
}

extern "C" hipError_t s2p_synth_bytes(void* p, int64_t n, uint64_t seed, hipStream_t st) {
    return run(p, n, SY_BYTES, 0.f, 0.f, seed, st);
}
extern "C" hipError_t s2p_synth_int4(void* p, int64_t n, uint64_t seed, hipStream_t st) {
    return run(p, n, SY_INT4, 0.f, 0.f, seed, st);
}
extern "C" hipError_t s2p_synth_int8(void* p, int64_t n, uint64_t seed, hipStream_t st) {
    return run(p, n, SY_INT8, 0.f, 0.f, seed, st);
}
extern "C" hipError_t s2p_synth_f16_absnormal(void* p, int64_t n, float sigma, uint64_t seed,
                                              hipStream_t st) {
    return run(p, n, SY_F16_ABSN, sigma, 0.f, seed, st);
}
extern "C" hipError_t s2p_synth_f32_absnormal(void* p, int64_t n, float sigma, uint64_t seed,
                                              hipStream_t st) {
    return run(p, n, SY_F32_ABSN, sigma, 0.f, seed, st);
}
extern "C" hipError_t s2p_synth_bf16_normal(void* p, int64_t n, float mean, float sd,
                                            uint64_t seed, hipStream_t st) {
    return run(p, n, SY_BF16_N, mean, sd, seed, st);
}
