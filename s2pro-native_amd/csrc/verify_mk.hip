/* s2pro MI355X — persistent verify kernel: the whole K-token verify forward
 * (36 layers + lm head, slowar.c:156-260 / 503-565 restated per row) in one
 * launch.
 *
 * Why: every kernel on this part costs ~4-5 us of dispatch / ramp / drain
 * even back to back inside a hipGraph, and the layer-by-layer forward needs
 * ~250 of them per step.  Here one grid of co-resident workgroups (a normal,
 * graph-capturable launch sized to the occupancy of the device) walks the
 * phases of every layer and separates them with device-wide barriers:
 *
 *   x = x_in (+ sums of squares)                                   | barrier
 *   per layer:  wqkv GEMV (RMSNorm staged, split-K fixup -> qkv)   | barrier
 *               qk-norm + RoPE + KV append (wave per row x head)   | barrier
 *               attention (segment x kv head x split blocks, the
 *               last split of a block merges)                      | barrier
 *               wo GEMV + residual (+ sums of squares)             | barrier
 *               gate_up GEMV (RMSNorm staged) + SwiGLU             | barrier
 *               w2 GEMV + residual (+ sums of squares)             | barrier
 *   lm head GEMV (final RMSNorm staged)
 *
 * Each phase runs the same device code as the layer-by-layer kernels
 * (gemv_dev.h, attn_dev.h, prims_dev.h) over the same work decomposition,
 * so both paths produce identical bits.  Data written in one phase and read
 * in another go through device-coherent accesses (coh.h): the XCD L2s are
 * not coherent inside a kernel.
 *
 * Barrier: two levels of monotonic 64-bit counters (groups of 16 workgroups,
 * then one top counter) plus one release word per group, each on its own
 * 4 KiB stride; a workgroup's first thread arrives after the whole workgroup
 * drained its stores; the last arrival overall writes the release words and
 * every workgroup polls only its group's word (s_sleep between polls), so no
 * word sees more than 16 pollers.  Counters never reset: each launch derives
 * its base from the value it reads at entry (at most one barrier's worth of
 * arrivals can precede that read).  Every wait is bounded:
 * a timeout sets a sticky error flag, and every later wait returns at once,
 * so the grid always drains (the host reports the flag as an error).
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_dev.h"
#include "coh.h"
#include "gemv_dev.h"
#include "mk_internal.h"
#include "prims_dev.h"

#define MK_WAVES 8
#define MK_THREADS (64 * MK_WAVES)
#define MK_GROUP 16
#define MK_SPIN_LIMIT (1u << 20)

struct MkBar {
    uint64_t* grp;  /* this group's arrival counter */
    uint64_t* rel;  /* release words: [g * MK_BAR_STRIDE], g < ngroups */
    uint64_t* top;
    uint64_t gbase, tbase, rbase;
    unsigned g, gsz, ngroups, k;
    int* err;
};

S2P_DEV uint64_t ld64_coh(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* per-launch base of the counters; nbar = barriers per launch */
__device__ MkBar mk_bar_init(uint64_t* bar, int* err, int nbar) {
    MkBar b;
    const unsigned wg = blockIdx.x, nwg = gridDim.x;
    b.g = wg / MK_GROUP;
    b.ngroups = (nwg + MK_GROUP - 1) / MK_GROUP;
    b.gsz = min((unsigned)MK_GROUP, nwg - b.g * MK_GROUP);
    b.grp = bar + (size_t)b.g * MK_BAR_STRIDE;
    b.rel = bar + (size_t)MK_MAX_GROUPS * MK_BAR_STRIDE;
    b.top = bar + (size_t)2 * MK_MAX_GROUPS * MK_BAR_STRIDE;
    b.err = err;
    b.k = 0;
    __shared__ uint64_t s_base[3];
    if (threadIdx.x == 0) {
        /* arrivals of this launch that can precede these reads: fewer than
         * one barrier's worth, so rounding down to a multiple of the
         * per-launch increment gives this launch's base */
        const uint64_t gv = ld64_coh(b.grp), tv = ld64_coh(b.top);
        const uint64_t rv = ld64_coh(b.rel + (size_t)b.g * MK_BAR_STRIDE);
        s_base[0] = gv - gv % ((uint64_t)nbar * b.gsz);
        s_base[1] = tv - tv % ((uint64_t)nbar * b.ngroups);
        s_base[2] = rv - rv % (uint64_t)nbar;
    }
    __syncthreads();
    b.gbase = s_base[0];
    b.tbase = s_base[1];
    b.rbase = s_base[2];
    __syncthreads();
    return b;
}

/* Arrive: group counter; the group's last arrival bumps the top counter;
 * the last arrival overall writes every group's release word.  Wait: poll
 * the own group's release word (16 pollers per word). */
__device__ void mk_bar_sync(MkBar& b, uint64_t* ts_wg) {
    vm_drain();
    __syncthreads();
    b.k++;
    if (threadIdx.x < 64) { /* wave 0 */
        const int lane = threadIdx.x;
        if (ts_wg && lane == 0)
            ts_wg[((size_t)(b.k - 1) * 2) * gridDim.x + blockIdx.x] = wall_clock64();
        int last_all = 0;
        if (lane == 0) {
            const uint64_t old = __hip_atomic_fetch_add(b.grp, (uint64_t)1, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
            if (old + 1 - b.gbase == (uint64_t)b.k * b.gsz) {
                const uint64_t t = __hip_atomic_fetch_add(b.top, (uint64_t)1, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT);
                last_all = t + 1 - b.tbase == (uint64_t)b.k * b.ngroups;
            }
        }
        last_all = __shfl(last_all, 0, 64);
        if (last_all && (unsigned)lane < b.ngroups) /* one store instruction for all groups */
            __hip_atomic_store(b.rel + (size_t)lane * MK_BAR_STRIDE, b.rbase + b.k,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0) {
            const uint64_t target = b.rbase + b.k;
            const uint64_t* mine = b.rel + (size_t)b.g * MK_BAR_STRIDE;
            unsigned spins = 0;
            if (!coh_ld32(b.err)) {
                while ((int64_t)(ld64_coh(mine) - target) < 0) {
                    __builtin_amdgcn_s_sleep(8); /* ~0.2 us: keeps polling traffic low */
                    if ((++spins & 255) == 0 && coh_ld32(b.err)) break;
                    if (spins > MK_SPIN_LIMIT) {
                        __hip_atomic_store(b.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                }
            }
            if (ts_wg) ts_wg[((size_t)(b.k - 1) * 2 + 1) * gridDim.x + blockIdx.x] = wall_clock64();
        }
        /* acquire: drop this CU's L1 and this XCD's L2 lines from before the
         * barrier, so the next phase may read activations through the caches
         * (every store of the phase was written through before arrival) */
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
}

/* barriers per launch for n_layers */
static __host__ __device__ int mk_nbar(int n_layers) { return 1 + 6 * n_layers; }

__device__ __forceinline__ void mk_phase_init(const MkArgs* A, const uint16_t* x_in) {
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * (MK_THREADS / 64) + (threadIdx.x >> 6);
    const int nw = gridDim.x * (MK_THREADS / 64);
    /* residual stream x = x_in and its sums of squares */
    for (int it = gw; it < 40 * A->rows; it += nw)
        resid_init_item(x_in, A->x, A->ssq_a, 2560, it % 40, it / 40, lane);
    /* RoPE table of the plan's positions (the same for every layer) */
    const int gt = blockIdx.x * MK_THREADS + threadIdx.x;
    for (int it = gt; it < A->rows * 64; it += gridDim.x * MK_THREADS)
        rope_tab_item(A->plan, A->rope_base, A->rope_tab, it / 64, it % 64);
}

__device__ __forceinline__ void mk_phase_qkrope(const MkArgs* A, int l) {
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * (MK_THREADS / 64) + (threadIdx.x >> 6);
    const int nw = gridDim.x * (MK_THREADS / 64);
    const MkLayer* L = A->layers + l;
    for (int it = gw; it < A->rows * 40; it += nw)
        qkrope_item_t<true>(A->qkv, A->q, L->q_norm, L->k_norm, A->plan, l, A->eps,
                            A->rope_base, it / 40, it % 40, lane, A->rope_tab);
}

__device__ __forceinline__ void mk_phase_attn(const MkArgs* A, int l,
                                              LDS(unsigned char)* smem) {
    AttnArgs at = {};
    at.mode = 2; /* AM_PLAN */
    at.q = A->q;
    at.out = A->attn;
    at.rows = A->rows;
    at.qh = 32;
    at.kvh_n = 8;
    at.plan = A->plan;
    at.segs = A->segs;
    at.layer = l;
    at.nsplit = A->nsplit;
    at.split_pos = A->split_pos;
    at.part = A->attn_part;
    at.counters = A->attn_counters;
    if (A->probe && A->probe_phase == 1000 + l) at.probe = A->probe;
    const int nseg = A->n_seg;
    const int nb = nseg * 8 * A->nsplit;
    for (int vb = blockIdx.x; vb < nb; vb += gridDim.x)
        attn_block<2, MK_WAVES>(at, vb % nseg, (vb / nseg) % 8, vb / (nseg * 8), smem);
}

/* GEMV i of a layer (0 wqkv, 1 wo, 2 gate_up, 3 w2) or the head (l == n) */
S2P_DEV const MkGemv* mk_gemv(const MkArgs* A, int l, int i) {
    return l == A->n_layers ? A->head : &A->layers[l].g[i];
}

/* Phase sequence: resid init | per layer: wqkv | qk-norm + RoPE + append |
 * attention | wo | gate_up | w2 | and the head.  Every GEMV's first weight
 * chunk is issued before the barrier that precedes it (weights do not
 * depend on the previous phase), so the barrier wait and the weight latency
 * overlap. */
template <int WFMT>
__global__ __launch_bounds__(MK_THREADS) __attribute__((amdgpu_waves_per_eu(2))) void k_verify_mk(
    const MkArgs* __restrict__ A, const uint16_t* __restrict__ x_in, uint16_t* logits) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    LDS(unsigned char)* smem = (LDS(unsigned char)*)smem_raw;
    const int n_layers = A->n_layers;
    MkBar bar = mk_bar_init(A->bar, A->err, mk_nbar(n_layers));
    uint64_t* ts = A->ts;
    int tsi = 0;
    auto stamp = [&]() __attribute__((always_inline)) {
        tsi++;
        if (ts && blockIdx.x == 0 && threadIdx.x == 0) ts[tsi] = wall_clock64();
    };
    if (ts && blockIdx.x == 0 && threadIdx.x == 0) ts[0] = wall_clock64();
    GvBuf pre, pre1;
    mk_phase_init(A, x_in);
    {
        const GemvArgs g0 = mk_gemv(A, 0, 0)->a;
        gv3_prefetch<WFMT>(g0, blockIdx.x, gridDim.x, pre, pre1);
    }
    mk_bar_sync(bar, A->ts_wg);
    stamp();
    for (int l = 0; l <= n_layers; l++) {
        for (int i = 0; i < 4; i++) {
            if (l < n_layers && i == 1) {
                mk_phase_qkrope(A, l);
                mk_bar_sync(bar, A->ts_wg);
                stamp();
                mk_phase_attn(A, l, smem);
                const GemvArgs gn = mk_gemv(A, l, 1)->a;
                gv3_prefetch<WFMT>(gn, blockIdx.x, gridDim.x, pre, pre1);
                mk_bar_sync(bar, A->ts_wg);
                stamp();
            }
            const bool head = l == n_layers;
            /* a copy in registers: read through a pointer, every field would
             * be reloaded after each store the phase makes */
            const GemvArgs ga = mk_gemv(A, l, i)->a;
            /* activations through the L2 (invalidated at the barrier),
             * outputs written through */
            gv3_block<WFMT, 1, false, true, true>(ga, blockIdx.x, gridDim.x, smem,
                                                  head ? logits : ga.y, pre, pre1);
            if (head) break;
            if (i != 0) { /* the next GEMV follows directly */
                const int nl = i == 3 ? l + 1 : l, ni = i == 3 ? 0 : i + 1;
                const GemvArgs gn = mk_gemv(A, nl, ni)->a;
                gv3_prefetch<WFMT>(gn, blockIdx.x, gridDim.x, pre, pre1);
            }
            mk_bar_sync(bar, A->ts_wg);
            stamp();
        }
    }
}

/* ------------------------------------------------------------------ host */

/* one workgroup per CU: the whole LDS (the whole-K GEMVs stage up to
 * M x 9728 activations; attention needs AT_LDS_BYTES_W(8)) */
static size_t mk_lds_bytes(void) { return 160 * 1024 - 256; /* static LDS: barrier state */ }

extern "C" int s2p_mk_grid(int* nwg, size_t* lds) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return -1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return -1;
    const size_t sb = mk_lds_bytes();
    (void)hipFuncSetAttribute((const void*)k_verify_mk<0>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)sb);
    (void)hipFuncSetAttribute((const void*)k_verify_mk<1>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)sb);
    if (hipGetLastError() != hipSuccess) return -1;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)k_verify_mk<0>,
                                                     MK_THREADS, sb) != hipSuccess)
        return -1;
    int per_cu8 = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu8, (const void*)k_verify_mk<1>,
                                                     MK_THREADS, sb) != hipSuccess)
        return -1;
    if (per_cu8 < per_cu) per_cu = per_cu8;
    if (per_cu > 1) per_cu = 1;
    if (per_cu < 1) return -1;
    int n = cus * per_cu;
    if (n > MK_MAX_GROUPS * MK_GROUP) n = MK_MAX_GROUPS * MK_GROUP;
    *nwg = n;
    *lds = sb;
    return 0;
}

extern "C" hipError_t s2p_mk_plan_gemv(const GemvArgs* ap, int nwg, size_t lds_cap, MkGemv* out) {
    MkGemv g;
    g.a = *ap;
    size_t lds = 0;
    if (g.a.M > 16) return hipErrorInvalidValue;
    const hipError_t e = s2p_gemv3_plan_nw(&g.a, MK_WAVES, lds_cap, &lds);
    if (e != hipSuccess) return e;
    g.P = nwg;
    g.S = 1;
    *out = g;
    return hipSuccess;
}

extern "C" hipError_t s2p_mk_launch(const MkArgs* args_dev, int wfmt, const void* x_in,
                                     void* logits, int nwg, size_t lds, hipStream_t st) {
    static bool attr0 = false, attr1 = false;
    if (wfmt == GEMV_W_INT4) {
        if (!attr0) {
            (void)hipFuncSetAttribute((const void*)k_verify_mk<0>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            attr0 = true;
        }
        hipLaunchKernelGGL(k_verify_mk<0>, dim3(nwg), dim3(MK_THREADS), lds, st, args_dev,
                           (const uint16_t*)x_in, (uint16_t*)logits);
    } else {
        if (!attr1) {
            (void)hipFuncSetAttribute((const void*)k_verify_mk<1>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            attr1 = true;
        }
        hipLaunchKernelGGL(k_verify_mk<1>, dim3(nwg), dim3(MK_THREADS), lds, st, args_dev,
                           (const uint16_t*)x_in, (uint16_t*)logits);
    }
    return hipGetLastError();
}
