/* s2pro MI355X — device-coherent accesses for data exchanged between
 * workgroups of one launch (the persistent verify kernel and split-K
 * handoffs).
 *
 * MI355X has one L2 per XCD and the eight L2s are not coherent with each
 * other inside a kernel.  Activations that one workgroup writes and another
 * reads later in the same launch (and buffers reused layer after layer) are
 * therefore written through to memory and read around the L2: relaxed
 * agent-scope atomic loads / stores, which the compiler emits as ordinary
 * vector memory instructions with the sc1 bit and tracks for s_waitcnt.
 * Nothing here writes through the scalar data cache.
 */
#ifndef S2P_COH_H
#define S2P_COH_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

S2P_DEV uint64_t coh_ld64(const void* p) {
    return __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
S2P_DEV uint32_t coh_ld32(const void* p) {
    return __hip_atomic_load((const uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
S2P_DEV float coh_ldf(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
S2P_DEV uint16_t coh_ld16(const uint16_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
/* 16 bytes (8 bf16) as two 8-byte coherent loads; p 16-byte aligned */
S2P_DEV s2p_u32x4 coh_ld128(const void* p) {
    const uint64_t a = coh_ld64(p), b = coh_ld64((const char*)p + 8);
    return (s2p_u32x4){(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
}

S2P_DEV void coh_st16(uint16_t* p, uint16_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
S2P_DEV void coh_stf(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
S2P_DEV void coh_st32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
S2P_DEV void coh_st64(void* p, uint64_t v) {
    __hip_atomic_store((uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
/* 16 bytes written through as two 8-byte agent-scope stores (p 16-byte
 * aligned).  The stores stay visible to the compiler: a store hidden in
 * inline asm escapes its hazard tracking, and a VALU write of the store's
 * data registers issued right after a 16-byte store can then replace data
 * the store has not read yet (seen as a corrupted first element of some
 * lanes' stores). */
S2P_DEV void coh_st128(void* p, s2p_u32x4 v) {
    coh_st64(p, (uint64_t)v.x | ((uint64_t)v.y << 32));
    coh_st64((char*)p + 8, (uint64_t)v.z | ((uint64_t)v.w << 32));
}

/* wait for this wave's outstanding vector memory operations (stores
 * included) to complete */
S2P_DEV void vm_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

#endif
