/* s2pro MI355X — device helpers shared by the HIP kernels (gfx950 only). */
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define S2P_DEV static __device__ __forceinline__

typedef __attribute__((ext_vector_type(8))) __bf16 s2p_bf16x8;
typedef __attribute__((ext_vector_type(4))) float s2p_f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t s2p_u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t s2p_u32x2;

/* 16-byte streaming load through a global-address-space pointer (a generic
 * pointer would compile to flat_load, which also counts against lgkmcnt and
 * serialises with LDS traffic) */
S2P_DEV s2p_u32x4 gld_nt128(const void* p) {
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) s2p_u32x4*)p);
}

/* bf16 bit pattern -> float (exact) */
S2P_DEV float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
S2P_DEV float bf2f_lo(uint32_t w) { return __uint_as_float(w << 16); }
S2P_DEV float bf2f_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

/* float -> bf16 bit pattern, round to nearest even (NaN stays NaN) */
S2P_DEV uint16_t f2bf(float f) {
    /* v_cvt_pk_bf16_f32: round to nearest even, NaN quieted (the rule:
     * u + 0x7FFF + lsb, NaN -> (u >> 16) | 0x40; pinned by a GPU test) */
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

/* IEEE f16 bit pattern <-> float (hardware conversions, RNE) */
S2P_DEV float h2f(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}
S2P_DEV uint16_t f2h(float f) {
    /* materialise f as a float first: without the barrier the compiler may
     * fold a preceding multiply and this conversion into one v_fma_mix
     * (a single rounding where the reference rounds to f32, then to f16) */
    asm volatile("" : "+v"(f));
    return __half_as_ushort(__float2half_rn(f));
}

/* 1/sqrt(v) as two correctly rounded operations: the rule's rsqrt value for
 * every norm in this build (the reference calls the approximate rsqrtf). */
S2P_DEV float rsqrt_rule(float v) { return 1.0f / __fsqrt_rn(v); }

S2P_DEV s2p_bf16x8 as_bf16x8(s2p_u32x4 v) { return __builtin_bit_cast(s2p_bf16x8, v); }

/* D = A(16x32) * B(32x16) + C, bf16 in, f32 accumulate (v_mfma_f32_16x16x32_bf16).
 * Lane l supplies A row (l % 16) and B column (l % 16), 8 k-slots each from
 * k-group (l / 16); D row 4*(l/16)+i, column l % 16 lands in C[i]. */
S2P_DEV s2p_f32x4 mfma16x16x32(s2p_u32x4 a, s2p_u32x4 b, s2p_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

/* lane permutation within 16-lane rows (DPP control CTRL), a VALU move */
template <int CTRL>
S2P_DEV float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
/* v + (v of lane ^ 1) + (... of lane ^ 2): the 4-lane butterfly of
 * __shfl_xor 1 then 2, with quad_perm moves */
S2P_DEV float quad_sum(float v) {
    v += dpp_f<0xB1>(v); /* quad_perm [1,0,3,2] */
    v += dpp_f<0x4E>(v); /* quad_perm [2,3,0,1] */
    return v;
}
/* Wave-wide (64 lanes) reductions through cross-lane shuffles.  The sum
 * follows the shuffle-down tree (offsets 32,16,...,1): lane 0 ends with
 * ((x0+x32)+(x16+x48))+... */
S2P_DEV float wave_sum_down(float v) {
    /* the same tree in lane 0, with cross-lane moves that stay in the VALU
     * (no LDS round trip): halves and 16-lane rows by permlane swaps, then
     * row rotations (lane i < 16 - off reads lane i + off) */
    v += __uint_as_float(
        __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false)[1]);
    v += __uint_as_float(
        __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false)[1]);
    v += dpp_f<0x128>(v); /* row_ror:8 */
    v += dpp_f<0x124>(v); /* row_ror:4 */
    v += dpp_f<0x122>(v); /* row_ror:2 */
    v += dpp_f<0x121>(v); /* row_ror:1 */
    return v;
}
/* sum over each aligned group of 16 lanes (fixed-order butterfly; every
 * lane of the group gets the total) */
S2P_DEV float sum_lanes16(float v) {
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
S2P_DEV float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
