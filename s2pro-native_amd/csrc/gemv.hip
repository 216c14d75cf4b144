/* s2pro MI355X — weight-only INT4 / INT8 GEMV engine for decode / verify M.
 *
 * Replaces the reference's packed-INT4 and per-channel INT8 GEMVs
 * (src/sched/int8_gemv.cu:60-104, 279-324, 836-902, 964-986) and its M > 16
 * dequant + cuBLAS / WMMA paths (gemm.c:444-490, int8_gemv.cu:535-618) with
 * one MI355X kernel.
 *
 * Work decomposition.  The N output rows form 64-row blocks, K forms S
 * splits.  The grid is (P, S): workgroup (p, s) stages the activations of
 * split s in LDS once and then streams the weights of row blocks p, p+P,
 * p+2P, ...; P is sized so the grid is about one resident round of
 * workgroups, so the staging is paid once per workgroup, not once per block.
 * Wave w owns rows 16w..16w+15 of the current block and runs its own weight
 * stream, double buffered (the next chunk's 16-byte loads are in flight
 * while the current chunk is multiplied), with no workgroup barrier between
 * chunks.
 *
 * MFMA mapping (v_mfma_f32_16x16x32_bf16).  Lane (q, r) = (lane / 16,
 * lane % 16) issues coalesced 16-byte loads: INT4 one 32-weight group of row
 * r, INT8 half a group.  A 4 x 4 transpose across lane quarters
 * (v_permlane32_swap, v_permlane16_swap) turns four such loads into the A
 * operands of four MFMAs, 16 rows x 32 k each.  The B operand (16 activation
 * rows x 32 k) comes from LDS; columns beyond M read row M-1 and are dropped.
 *
 * INT4 -> bf16 in registers: nibbles XOR 8 are OR-ed into the top mantissa
 * bits of bf16 1.0, giving 1.5 + w/16 exactly.  Per group the MFMA yields
 * raw_g = 1.5 X_g + (w . x)_g / 16 with X_g the activation group sum; the f16
 * group scale is applied in fp32 (acc += s_g raw_g, as the reference's
 * acc += s * gs, int8_gemv.cu:312) and the bias sum_g s_g X_g is two extra
 * MFMAs per 32 groups per split part on exact bf16 splits of s (hi + lo) and
 * X (hi + mid + lo): result = 16 acc - 24 corr.  The per-group VALU work is
 * then independent of M.
 * INT8 per channel: bytes XOR 0x80 via v_cvt_f32_ubyte*, 128 + w exact in
 * bf16; result = s_n (acc - 128 sum_k x_k).
 *
 * Staging applies the consuming layer's RMSNorm (row inverse RMS from the
 * producer epilogue's per-64-column sums of squares) with the rule's
 * roundings.  Epilogues: bf16 store; residual add y = bf16(y + bf16(acc))
 * (kernels.cu:1242-1247) with sums of squares for the next RMSNorm; or
 * SwiGLU, where a block holds 32 gate rows and the 32 matching up rows and
 * the epilogue writes silu(bf16 g) * bf16 u (kernels.cu:1216-1229).
 *
 * Split-K partials go to a device scratch; the last workgroup to arrive at a
 * row block (self-resetting counter) sums the partials in split order
 * (deterministic) and runs the epilogue.
 */
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <atomic>

#include "gemv_dev.h"
#include "s2pro/gemm.h"

/* whole-K workgroups of up to 16 waves (MT = 1) or 8 waves */
template <int WFMT, int MT, bool NOTR = false>
__global__ __launch_bounds__(MT == 1 ? 1024 : 512) void k_gemv3(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem3[];
    /* every argument in one round of scalar loads: left to itself the
     * compiler issues them next to their first uses, three dependent
     * kernarg round trips before the first weight load */
    asm volatile("" ::"s"(a.w), "s"(a.s), "s"(a.x), "s"(a.y), "s"(a.norm_w), "s"(a.ssq_in),
                 "s"(a.ssq_out), "s"(a.ldx), "s"(a.ldy), "s"(a.M), "s"(a.N),
                 "s"(a.K), "s"(a.gps), "s"(a.ks), "s"(a.rt), "s"(a.xmode), "s"(a.epi),
                 "s"(a.ssq_in_blocks), "s"(a.norm_eps), "s"(gridDim.x));
    GvBuf b0, b1;
    gv3_block<WFMT, MT, false, false, false, NOTR>(a, blockIdx.x, gridDim.x,
                                                  (LDS(unsigned char)*)smem3, a.y, b0, b1);
}

template <int WFMT, int MT, bool WIN1>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(MT == 1 ? 4 : (MT == 2 ? 3 : 2)))) void k_gemv(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    gv_block<WFMT, MT, WIN1, false>(a, blockIdx.x, gridDim.x, blockIdx.y,
                             (LDS(unsigned char)*)smem_raw);
}

/* Generic one-wave-per-row GEMV for group sizes other than 32 and the
 * int8-container group-wise format (s2p_intq_gemv); off the verify path.
 * Lane l covers 16-k tiles l*16 + 1024 i; wave tree reduction. */
template <int FMT>
__global__ __launch_bounds__(256) void k_gemv_generic(const uint8_t* __restrict__ w,
                                                      const void* __restrict__ sc,
                                                      const uint16_t* __restrict__ x,
                                                      uint16_t* __restrict__ y, int M,
                                                      int N, int K, int gshift) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;
    for (int m = 0; m < M; m++) {
        float acc = 0.f;
        for (int k0 = lane * 16; k0 < K; k0 += 1024) {
            float s = 0.f;
            for (int j = 0; j < 16; j++) {
                const int k = k0 + j;
                int wv;
                if (FMT == 0) { /* packed int4 */
                    const uint8_t b = w[(size_t)n * (K >> 1) + (k >> 1)];
                    wv = (k & 1) ? ((int)(int8_t)b >> 4) : ((int)(int8_t)(uint8_t)(b << 4) >> 4);
                } else {        /* int8 container */
                    wv = (int)(int8_t)w[(size_t)n * K + k];
                }
                s = fmaf((float)wv, bf2f(x[(size_t)m * K + k]), s);
            }
            const float g = h2f(((const uint16_t*)sc)[(size_t)n * (K >> gshift) + (k0 >> gshift)]);
            acc = fmaf(s, g, acc);
        }
        acc = wave_sum_down(acc);
        if (lane == 0) y[(size_t)m * N + n] = f2bf(acc);
    }
}

/* bf16-weight fallback for K not a multiple of 128: one wave per output,
 * lanes stride K, fp32 sums, fixed-order wave reduction. */
__global__ __launch_bounds__(256) void k_gemv_bf16_generic(const uint16_t* __restrict__ w,
                                                           const uint16_t* __restrict__ x,
                                                           uint16_t* __restrict__ y, int M, int N,
                                                           int K) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;
    for (int m = 0; m < M; m++) {
        float acc = 0.f;
        for (int k = lane; k < K; k += 64)
            acc = fmaf(bf2f(w[(size_t)n * K + k]), bf2f(x[(size_t)m * K + k]), acc);
        acc = wave_sum_down(acc);
        if (lane == 0) y[(size_t)m * N + n] = f2bf(acc);
    }
}

extern "C" hipError_t s2p_gemv_bf16_generic_launch(const void* w, const void* x, void* y, int M,
                                                   int N, int K, hipStream_t st) {
    hipLaunchKernelGGL(k_gemv_bf16_generic, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st,
                       (const uint16_t*)w, (const uint16_t*)x, (uint16_t*)y, M, N, K);
    return hipGetLastError();
}

/* ------------------------------------------------------------- launchers */

extern "C" int s2p_cu_count(void) {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
        v = 256;
    cache[dev].store(v, std::memory_order_relaxed);
    return v;
}

extern "C" int s2p_gemv_slots(void) { return 4 * s2p_cu_count(); }

template <int WFMT, int MT, bool WIN1>
static hipError_t gv_launch_w(const GemvArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    /* once per instantiation (thread-safe static initialisation) */
    static const hipError_t attr = hipFuncSetAttribute((const void*)k_gemv<WFMT, MT, WIN1>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       GV_LDS_MAX);
    (void)attr;
    hipLaunchKernelGGL((k_gemv<WFMT, MT, WIN1>), grid, dim3(256), lds, st, a);
    return hipGetLastError();
}

template <int WFMT, int MT>
static hipError_t gv_launch_mt(const GemvArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    if (a.win >= a.gps) return gv_launch_w<WFMT, MT, true>(a, grid, lds, st);
    return gv_launch_w<WFMT, MT, false>(a, grid, lds, st);
}

/* Work decomposition of one GEMV for a target of `slots` resident
 * workgroups: fills a->nrb, gps, splits, win and returns the grid and the
 * dynamic LDS bytes. */
static hipError_t s2p_gemv_plan_check(const GemvArgs* ap) {
    const GemvArgs& a = *ap;
    if (a.M <= 0 || a.M > GEMV_MAX_M || a.N <= 0 || a.K <= 0 || (a.K & 127))
        return hipErrorInvalidValue;
    if (a.gps < 0 || (a.gps & 3)) return hipErrorInvalidValue;
    if (a.epi == GEMV_EPI_SWIGLU && ((a.N & 1) || ((a.N >> 1) & 31))) return hipErrorInvalidValue;
    if (a.xmode == GEMV_X_NORM && (!a.norm_w || !a.ssq_in || a.ssq_in_blocks <= 0))
        return hipErrorInvalidValue;
    return hipSuccess;
}

extern "C" hipError_t s2p_gemv_plan(GemvArgs* ap, int slots, dim3* grid_out, size_t* lds_out) {
    GemvArgs& a = *ap;
    const hipError_t ce = s2p_gemv_plan_check(ap);
    if (ce != hipSuccess) return ce;
    const int G = a.K >> 5;
    a.nrb = a.epi == GEMV_EPI_SWIGLU ? (a.N >> 1) / 32 : (a.N + 63) / 64;
    const bool autos = a.gps == 0;
    int gps = a.gps;
    if (autos) {
        int S = a.nrb >= slots ? 1 : (slots + a.nrb - 1) / a.nrb;
        int smax = G / 8;
        if (smax < 1) smax = 1;
        if (S > smax) S = smax;
        if (S > GV_SMAX) S = GV_SMAX;
        gps = (((G + S - 1) / S) + 3) & ~3;
    }
    if (gps > G) gps = G;
    a.splits = (G + gps - 1) / gps;
    const bool handoff = a.splits > 1 || a.epi != GEMV_EPI_STORE;
    if (handoff) {
        if (!a.part || !a.counters || a.nrb > GV_COUNTERS) return hipErrorInvalidValue;
        while ((int64_t)a.splits * a.M * a.nrb * 64 > a.part_cap || a.splits > GV_SMAX) {
            if (!autos || a.splits == 1) return hipErrorInvalidValue;
            gps += 4;
            a.splits = (G + gps - 1) / gps;
        }
    }
    /* prefer more splits over LDS windows (restaging per block) */
    while (autos && gps > 4 && gv_lds_bytes(a.M, gps, a.wfmt) > GV_LDS_BUDGET) {
        const int g2 = gps - 4, s2 = (G + g2 - 1) / g2;
        if (s2 > GV_SMAX || (int64_t)s2 * a.M * a.nrb * 64 > a.part_cap || !a.part || !a.counters)
            break;
        gps = g2;
        a.splits = s2;
    }
    a.gps = gps;
    int win = gps;
    while (win > 4 && gv_lds_bytes(a.M, win, a.wfmt) > GV_LDS_BUDGET) win -= 4;
    const size_t lds = gv_lds_bytes(a.M, win, a.wfmt);
    if (lds > GV_LDS_MAX) return hipErrorInvalidValue;
    a.win = win;
    int P = (slots + a.splits - 1) / a.splits;
    if (P > a.nrb) P = a.nrb;
    *grid_out = dim3((unsigned)P, (unsigned)a.splits);
    *lds_out = lds;
    return hipSuccess;
}

#define GV3_LDS_MAX (160 * 1024)

/* Whole-K plan: K slices of whole 16-group chunks where possible (at most 16
 * waves), then as many tiles per group as the waves allow, fewer when the
 * launch would not cover every CU; the grid is one resident round.  Returns
 * hipErrorNotSupported when the activations do not fit in LDS (the split-K
 * engine runs instead). */
extern "C" hipError_t s2p_gemv3_plan(GemvArgs* a, dim3* grid, dim3* block, size_t* lds_out) {
    const int G = a->K >> 5;
    const int mt = (a->M + 15) / 16;
    const bool swiglu = a->epi == GEMV_EPI_SWIGLU;
    const int tiles = swiglu ? (a->N >> 1) / 16 : (a->N + 15) / 16;
    const int nwmax = mt == 1 ? 16 : 8;
    const int chg = gv_chg(a->wfmt);
    const int cus = s2p_cu_count();
    const int kmax = swiglu ? nwmax / 2 : nwmax;
    int gps = chg;
    while ((G + gps - 1) / gps > kmax) gps += 4;
    int ks = (G + gps - 1) / gps;
    /* units: output tiles per group (SWIGLU: a unit is a gate + up pair) */
    const int per = swiglu ? 2 : 1;
    int units = nwmax / (per * ks);
    if (units < 1) units = 1;
    while (units > 1 && (tiles + units - 1) / units < cus) units--;
    /* still fewer groups than CUs: thinner K slices */
    while ((tiles + units - 1) / units < cus && per * units * (ks + 1) <= nwmax && gps > 4) {
        const int g2 = ((G + ks) / (ks + 1) + 3) & ~3;
        if ((G + g2 - 1) / g2 <= ks) break;
        gps = g2;
        ks = (G + gps - 1) / gps;
    }
    for (;;) {
        const int rt = per * units, nw = rt * ks;
        const int ngroups = (tiles + units - 1) / units;
        /* resident workgroups per CU: LDS, and waves at this kernel's
         * register budget (16 waves per CU at MT = 1, else 8) */
        const size_t lds1 = gv3_lds_bytes(a->M, gps, a->wfmt, ks, nw, 1);
        int per_cu = (int)(GV3_LDS_MAX / lds1);
        const int wcap = nwmax / nw;
        if (per_cu > wcap) per_cu = wcap;
        if (per_cu < 1) per_cu = 1;
        int P = cus * per_cu;
        if (P > ngroups) P = ngroups;
        const size_t lds = gv3_lds_bytes(a->M, gps, a->wfmt, ks, nw, ngroups > P ? 2 : 1);
        if (lds <= GV3_LDS_MAX) {
            a->gps = gps;
            a->ks = ks;
            a->rt = rt;
            a->splits = 1;
            *grid = dim3((unsigned)P);
            *block = dim3((unsigned)(64 * nw));
            *lds_out = lds;
            return hipSuccess;
        }
        if (units == 1) return hipErrorNotSupported;
        units--;
    }
}

template <int WFMT, int MT, bool NOTR>
static hipError_t gv3_launch_k(const GemvArgs& a, dim3 grid, dim3 block, size_t lds,
                               hipStream_t st) {
    /* once per instantiation (thread-safe static initialisation) */
    static const hipError_t attr = hipFuncSetAttribute((const void*)k_gemv3<WFMT, MT, NOTR>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       GV3_LDS_MAX);
    (void)attr;
    hipLaunchKernelGGL((k_gemv3<WFMT, MT, NOTR>), grid, block, lds, st, a);
    return hipGetLastError();
}

template <int WFMT, int MT>
static hipError_t gv3_launch_mt(const GemvArgs& a, dim3 grid, dim3 block, size_t lds,
                                hipStream_t st) {
    return gv3_launch_k<WFMT, MT, false>(a, grid, block, lds, st);
}

template <int WFMT>
static hipError_t gv3_launch(const GemvArgs& a, dim3 grid, dim3 block, size_t lds,
                             hipStream_t st) {
    switch ((a.M + 15) / 16) {
        case 1: return gv3_launch_mt<WFMT, 1>(a, grid, block, lds, st);
        case 2: return gv3_launch_mt<WFMT, 2>(a, grid, block, lds, st);
        case 3: return gv3_launch_mt<WFMT, 3>(a, grid, block, lds, st);
        case 4: return gv3_launch_mt<WFMT, 4>(a, grid, block, lds, st);
        case 5: return gv3_launch_mt<WFMT, 5>(a, grid, block, lds, st);
        case 6: return gv3_launch_mt<WFMT, 6>(a, grid, block, lds, st);
        case 7: return gv3_launch_mt<WFMT, 7>(a, grid, block, lds, st);
        default: return gv3_launch_mt<WFMT, 8>(a, grid, block, lds, st);
    }
}

static hipError_t gemv_engines(const GemvArgs* ap, hipStream_t st) {
    GemvArgs a = *ap;
    dim3 grid;
    size_t lds = 0;
    if (a.engine != GEMV_ENGINE_SPLITK && a.gps == 0) {
        GemvArgs a3 = a;
        dim3 block;
        const hipError_t e3 = s2p_gemv_plan_check(&a3);
        if (e3 != hipSuccess) return e3;
        const hipError_t pe3 = s2p_gemv3_plan(&a3, &grid, &block, &lds);
        if (pe3 == hipSuccess) {
            switch (a3.wfmt) {
                case GEMV_W_INT4: return gv3_launch<GEMV_W_INT4>(a3, grid, block, lds, st);
                case GEMV_W_INT8: return gv3_launch<GEMV_W_INT8>(a3, grid, block, lds, st);
                default: return gv3_launch<GEMV_W_BF16>(a3, grid, block, lds, st);
            }
        }
    }
    if (a.wfmt == GEMV_W_BF16) return hipErrorNotSupported; /* whole-K engine only */
    const hipError_t pe = s2p_gemv_plan(&a, s2p_gemv_slots(), &grid, &lds);
    if (pe != hipSuccess) return pe;
    const int mt = (a.M + 15) / 16;
    if (a.wfmt == GEMV_W_INT4) {
        switch (mt) {
            case 1: return gv_launch_mt<GEMV_W_INT4, 1>(a, grid, lds, st);
            case 2: return gv_launch_mt<GEMV_W_INT4, 2>(a, grid, lds, st);
            case 3: return gv_launch_mt<GEMV_W_INT4, 3>(a, grid, lds, st);
            case 4: return gv_launch_mt<GEMV_W_INT4, 4>(a, grid, lds, st);
            case 5: return gv_launch_mt<GEMV_W_INT4, 5>(a, grid, lds, st);
            case 6: return gv_launch_mt<GEMV_W_INT4, 6>(a, grid, lds, st);
            case 7: return gv_launch_mt<GEMV_W_INT4, 7>(a, grid, lds, st);
            default: return gv_launch_mt<GEMV_W_INT4, 8>(a, grid, lds, st);
        }
    }
    switch (mt) {
        case 1: return gv_launch_mt<GEMV_W_INT8, 1>(a, grid, lds, st);
        case 2: return gv_launch_mt<GEMV_W_INT8, 2>(a, grid, lds, st);
        case 3: return gv_launch_mt<GEMV_W_INT8, 3>(a, grid, lds, st);
        case 4: return gv_launch_mt<GEMV_W_INT8, 4>(a, grid, lds, st);
        case 5: return gv_launch_mt<GEMV_W_INT8, 5>(a, grid, lds, st);
        case 6: return gv_launch_mt<GEMV_W_INT8, 6>(a, grid, lds, st);
        case 7: return gv_launch_mt<GEMV_W_INT8, 7>(a, grid, lds, st);
        default: return gv_launch_mt<GEMV_W_INT8, 8>(a, grid, lds, st);
    }
}

extern "C" hipError_t s2p_gemv_launch(const GemvArgs* ap, hipStream_t st) {
    if (ap->deferred) *ap->deferred = 0; /* merged, unless k_gemm4 defers below */
    /* INT4 at 16 < M <= 96: the row-split GEMM with streamed activation
     * windows (gemm4.hip), which writes inv_out itself */
    if (ap->engine == GEMV_ENGINE_AUTO && ap->gps == 0 && ap->wfmt == GEMV_W_INT4 && ap->M > 16) {
        const hipError_t e4 = s2p_gemm4_launch(ap, st);
        if (e4 != hipErrorNotSupported) return e4;
    }
    const hipError_t e = gemv_engines(ap, st);
    if (e != hipSuccess || !ap->inv_out || ap->epi != GEMV_EPI_RESID || !ap->ssq_out) return e;
    return s2p_g4_rms_launch(ap->ssq_out, (ap->N + 15) / 16, ap->M, ap->N, ap->inv_eps,
                             ap->inv_out, st);
}

extern "C" hipError_t s2p_gemv_generic_launch(int fmt, const void* w, const void* sc,
                                              const void* x, void* y, int M, int N, int K,
                                              int gshift, hipStream_t st) {
    dim3 grid((unsigned)((N + 3) / 4));
    if (fmt == 0)
        hipLaunchKernelGGL((k_gemv_generic<0>), grid, dim3(256), 0, st, (const uint8_t*)w, sc,
                           (const uint16_t*)x, (uint16_t*)y, M, N, K, gshift);
    else
        hipLaunchKernelGGL((k_gemv_generic<1>), grid, dim3(256), 0, st, (const uint8_t*)w, sc,
                           (const uint16_t*)x, (uint16_t*)y, M, N, K, gshift);
    return hipGetLastError();
}
