/* s2pro MI355X — INT4-g32 weight GEMM for the batched / tree verify rows
 * (16 < M <= 96: configs 4 and 5 of the verify path).
 *
 * Replaces the reference's M > 16 path (dequant + cuBLAS, gemm.c:467-490, or
 * the WMMA kernel int8_gemv.cu:535-618) for packed INT4 weights.
 *
 * The whole-K GEMV engine stages all M x K activations of a workgroup in LDS,
 * which stops fitting past M ~ 16 (M = 68 x K = 2560 is 348 KB).  Here the
 * waves of a workgroup split ROWS, not K, and share one activation window:
 *   - a workgroup of 8 waves owns 8 row tiles of 16 (SWIGLU: 4 gate tiles and
 *     the 4 matching up tiles), every wave one tile, over the whole of K;
 *   - K advances in windows of 16 groups (512 k): the workgroup stages the
 *     window's M x 512 activations in LDS (RMSNorm with the rule's roundings,
 *     the INT4 k-slot order and the group sums of the bias correction, as the
 *     GEMV staging does), then every wave multiplies its tile's 16-group chunk
 *     of weights against it (MT = ceil(M / 16) MFMA column tiles, the GEMV
 *     engine's untransposed INT4 tile), accumulating over the windows;
 *   - the next chunk's weights are in flight while a window is staged and
 *     multiplied; two waves per SIMD hide each other's latencies;
 *   - when the row blocks are too few to fill the chip, K is split over
 *     workgroups, which store partials; a second launch (k_g4_merge, every
 *     CU) sums the splits in order and runs the epilogue.
 * Per group the dequantisation (9 VALU per 8 weights) is shared by the MT
 * column tiles, so at M = 68 the MFMA work, not the weight stream, sets the
 * pace.  Accumulation order per output is fixed (window by window, group by
 * group): deterministic.  The epilogues are the GEMV engine's: bf16 store,
 * residual add with per-16-column sums of squares, SwiGLU. */
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "gemv_dev.h"

#define G4_WAVES 8
#define G4_WIN 16 /* groups per window = one weight chunk (GV_CHG_INT4) */
#define G4_MAX_M 96 /* six column tiles */
#ifndef G4_PIPE
#define G4_PIPE(MT) ((MT) != 5) /* five tiles: no registers left for it */
#endif

static __host__ __device__ size_t g4_xs() { return (size_t)G4_WIN * 32 + GV_XPAD; }
static __host__ __device__ size_t g4_xg() { return (size_t)gv_round32(G4_WIN) + 8; }
/* x [M][xs] bf16 (two of them up to four column tiles: the next window's
 * rows land in the second while the first multiplies) | X3 [M][3][xg] bf16 |
 * scale staging [waves][16][16] f32 | inverse RMS [GEMV_MAX_M] f32 */
static __host__ __device__ bool g4_dbuf(int M) { return (M + 15) / 16 <= 4; }
static __host__ __device__ size_t g4_xbytes(int M) { return ((size_t)M * g4_xs() * 2 + 15) & ~(size_t)15; }
static __host__ __device__ size_t g4_lds_bytes(int M) {
    const size_t x = g4_xbytes(M) * (g4_dbuf(M) ? 2 : 1);
    const size_t x3 = ((size_t)M * 3 * g4_xg() * 2 + 15) & ~(size_t)15;
    return x + x3 + G4_WAVES * 1024 + GEMV_MAX_M * 4 + 16;
}

#ifdef S2P_DIAG
/* diagnostics build: wall clock per workgroup at the stages of the kernel
 * (start, staged, first window, multiplied) */
__device__ uint64_t g4_probe[4096 * 8];
extern "C" hipError_t s2p_g4_probe_get(uint64_t* host, int n) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g4_probe), (size_t)n * 8, 0, hipMemcpyDeviceToHost);
}
#define G4_STAMP(i) \
    if (threadIdx.x == 0) g4_probe[(blockIdx.y * gridDim.x + blockIdx.x) * 8 + (i)] = wall_clock64();
#else
#define G4_STAMP(i)
#endif

/* inverse RMS of activation row m from the producer's per-block sums of
 * squares: lane l sums blocks l, l + 64, ... in order, then the wave's tree
 * (the GEMV engine's order); every lane returns it */
static __device__ float g4_inv_rms(const GemvArgs& a, int m, int lane) {
#pragma clang fp contract(off)
    float s = 0.f;
    for (int b = lane; b < a.ssq_in_blocks; b += 64) s += a.ssq_in[(size_t)b * GEMV_MAX_M + m];
    s = wave_sum_down(s);
    return rsqrt_rule(s / (float)a.K + a.norm_eps);
}

/* the rows' inverse RMS once per launch into inv_out (a k_gemm4 workgroup
 * otherwise computes all M of them itself: a chain of a load round and
 * M / 8 trees a wave, ~7 us at M = 68 in every workgroup).  Workgroup g
 * takes rows 4 g .. 4 g + 3: their block sums come in as one 16-byte load
 * per block (coalesced; GEMV_MAX_M is a multiple of 4), then wave w sums
 * row 4 g + w in the GEMV engine's order from LDS */
#define G4_RMS_BLOCKS 1024
__global__ __launch_bounds__(256) void k_g4_rms(GemvArgs a, float* inv_out) {
#pragma clang fp contract(off)
    __shared__ s2p_f32x4 sb[G4_RMS_BLOCKS];
    const int m0 = blockIdx.x * 4, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = a.ssq_in_blocks;
    for (int b = threadIdx.x; b < nb; b += 256)
        sb[b] = *(const s2p_f32x4*)(a.ssq_in + (size_t)b * GEMV_MAX_M + m0);
    __syncthreads();
    const int m = m0 + wave;
    if (m >= a.M) return; /* uniform per wave */
    float s = 0.f;
    for (int b = lane; b < nb; b += 64) s += sb[b][wave];
    s = wave_sum_down(s);
    if (lane == 0) inv_out[m] = rsqrt_rule(s / (float)a.K + a.norm_eps);
}

template <int MT>
__global__ __launch_bounds__(64 * G4_WAVES) void k_gemm4(GemvArgs a) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) unsigned char smem4[];
    LDS(unsigned char)* smem = (LDS(unsigned char)*)smem4;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    G4_STAMP(0);
    const int q = lane >> 4, r = lane & 15;
    const int M = a.M, G = a.K >> 5;
    const bool swiglu = a.epi == GEMV_EPI_SWIGLU;
    const int F = a.N >> 1;

    /* this wave's tile: rows wbase .. wbase + 15 of W */
    int tile, wbase, tiles;
    if (swiglu) {
        tiles = F >> 4;
        tile = blockIdx.x * 4 + (wave & 3);
        wbase = (wave < 4 ? 0 : F) + tile * 16;
    } else {
        tiles = (a.N + 15) >> 4;
        tile = blockIdx.x * G4_WAVES + wave;
        wbase = tile * 16;
    }
    const bool active = tile < tiles; /* uniform; idle waves still stage */
    const int nrow = min(wbase + r, a.N - 1);

    GvLds L;
    L.xs = (int)g4_xs();
    L.xg = (int)g4_xg();
    constexpr bool DB = MT <= 4; /* g4_dbuf */
    L.x = (LDS(uint16_t)*)smem;
    size_t off = g4_xbytes(M) * (DB ? 2 : 1);
    L.X3 = (LDS(uint16_t)*)(smem + off);
    off += ((size_t)M * 3 * L.xg * 2 + 15) & ~(size_t)15;
    L.sc = (LDS(float)*)(smem + off + (size_t)wave * 1024);
    off += G4_WAVES * 1024;
    L.inv = (LDS(float)*)(smem + off);
    off += GEMV_MAX_M * 4;
    L.xtot = nullptr;
    L.flag = (LDS(int)*)(smem + off);

    GvBuf b0, b1;
    const int nch_all = (G + G4_WIN - 1) / G4_WIN;
    /* K split sp of a.splits: chunks [c0, c0 + nch) (a.win chunks a split) */
    const int sp = blockIdx.y;
    const int c0 = sp * a.win;
    const int nch = min(a.win, nch_all - c0);
    auto load_c = [&](GvBuf& B, int c) __attribute__((always_inline)) {
        gv_load<GEMV_W_INT4, false>(B, a, nrow, c * G4_WIN, min(G4_WIN, G - c * G4_WIN), q);
    };
    load_c(b0, c0); /* in flight during the inverse RMS and the first staging */

    if (a.xmode == GEMV_X_NORM) {
        if (a.inv_in) { /* written before this launch (the residual producer's merge, or k_g4_rms) */
            if (tid < M) L.inv[tid] = a.inv_in[tid];
        } else {
            for (int m = wave; m < M; m += G4_WAVES) L.inv[m] = g4_inv_rms(a, m, lane);
        }
    }

    /* window c of the activations into LDS, transformed there (RMSNorm with
     * the rule's roundings, k-slot order, group sums: a group's 4 blocks sit
     * in adjacent lanes).  Two ways to bring the raw rows in:
     * - stage_lds: straight to their LDS slots at staging time (16-byte
     *   direct-to-LDS loads, one per row and wave, all in flight together),
     *   then every lane transforms its 8-element block b = lane in place;
     * - stage_regs (five column tiles, M = 65..80): wave w holds rows w,
     *   w + 8, ... of the window in registers, loaded one window ahead by
     *   prefetch() so they land while the previous window multiplies
     *   (measured 38.3 -> 35.8 us per launch at M = 68).  At six tiles no
     *   registers are left for them, and at three tiles it measured slower
     *   (26.4 -> 29.3 us at M = 40). */
    constexpr bool PF = MT == 5;
    constexpr int RPW = PF ? 2 * MT : 1; /* rows per wave: M <= 16 MT */
    s2p_u32x4 raw[RPW];
    s2p_u32x4 wn4p = {0u, 0u, 0u, 0u};
    auto zero_tail = [&](int gn) __attribute__((always_inline)) {
        if (gn < G4_WIN)
            for (int i = tid; i < M * 3 * (G4_WIN - gn); i += 64 * G4_WAVES) {
                const int row = i / (G4_WIN - gn), g = gn + i % (G4_WIN - gn);
                L.X3[row * L.xg + g] = 0;
            }
    };
    auto prefetch = [&](int c) __attribute__((always_inline)) {
        if constexpr (PF) {
            const int nb = min(G4_WIN, G - c * G4_WIN) * 4;
            const size_t k0 = (size_t)c * G4_WIN * 32;
#pragma unroll
            for (int j = 0; j < RPW; j++) {
                const int m = wave + G4_WAVES * j;
                raw[j] = (m < M && lane < nb) ? *(const s2p_u32x4*)(a.x + (size_t)m * a.ldx + k0 + lane * 8)
                                              : (s2p_u32x4){0u, 0u, 0u, 0u};
            }
            if (a.xmode == GEMV_X_NORM && lane < nb) wn4p = *(const s2p_u32x4*)(a.norm_w + k0 + lane * 8);
        }
    };
    auto stage_regs = [&](int c) __attribute__((always_inline)) {
        const int gn = min(G4_WIN, G - c * G4_WIN);
        const int nb = gn * 4;
        __syncthreads(); /* the previous window is no longer read */
        zero_tail(gn);
        vm_drain(); /* this wave's rows (and the weights issued before) landed */
#pragma unroll
        for (int j = 0; j < RPW; j++) {
            const int m = wave + G4_WAVES * j;
            if (m < M) gv_stage_one<GEMV_W_INT4>(a, L, m, lane, lane < nb, raw[j], wn4p);
        }
        __syncthreads();
    };
    auto stage_lds = [&](int c) __attribute__((always_inline)) {
        const int gn = min(G4_WIN, G - c * G4_WIN);
        const int nb = gn * 4;
        const size_t k0 = (size_t)c * G4_WIN * 32;
        __syncthreads(); /* the previous window is no longer read */
        for (int m = wave; m < M; m += G4_WAVES)
            if (lane < nb)
                __builtin_amdgcn_global_load_lds(
                    (const void*)(a.x + (size_t)m * a.ldx + k0 + lane * 8),
                    (LDS(void)*)(L.x + m * L.xs), 16, 0, 0);
        s2p_u32x4 wn4 = {0u, 0u, 0u, 0u};
        if (a.xmode == GEMV_X_NORM && lane < nb) wn4 = *(const s2p_u32x4*)(a.norm_w + k0 + lane * 8);
        zero_tail(gn);
        vm_drain(); /* this wave's rows (and the weights issued before) landed */
        __syncthreads();
        for (int m = wave; m < M; m += G4_WAVES) {
            const bool ok = lane < nb;
            const s2p_u32x4 raw = ok ? *(const LDS(s2p_u32x4)*)(L.x + m * L.xs + lane * 8)
                                     : (s2p_u32x4){0u, 0u, 0u, 0u};
            gv_stage_one<GEMV_W_INT4>(a, L, m, lane, ok, raw, wn4);
        }
        __syncthreads();
    };
    auto stage = [&](int c) __attribute__((always_inline)) {
        if constexpr (PF)
            stage_regs(c);
        else
            stage_lds(c);
    };
    prefetch(c0);

    s2p_f32x4 acc[MT], corr[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) {
        acc[t] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
        corr[t] = (s2p_f32x4){0.f, 0.f, 0.f, 0.f};
    }
    auto mult = [&](const GvBuf& B, int c) __attribute__((always_inline)) {
        gv_compute<GEMV_W_INT4, MT, false, G4_PIPE(MT)>(B, L, 0, min(G4_WIN, G - c * G4_WIN), M, 0, q, r, acc,
                                           corr);
    };
    const int ce = c0 + nch;
    G4_STAMP(1);
    if constexpr (DB) {
        /* double-buffered windows: the raw rows of window c + 1 go to the
         * other x buffer (direct-to-LDS) right after window c is staged, so
         * they land while c multiplies; staging then only waits, transforms
         * in place and publishes */
        GvLds Lb[2] = {L, L};
        Lb[1].x = (LDS(uint16_t)*)(smem + g4_xbytes(M));
        s2p_u32x4 wnb[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
        auto issue = [&](int c, int bsel) __attribute__((always_inline)) {
            const int nb = min(G4_WIN, G - c * G4_WIN) * 4;
            const size_t k0 = (size_t)c * G4_WIN * 32;
            for (int m = wave; m < M; m += G4_WAVES)
                if (lane < nb)
                    __builtin_amdgcn_global_load_lds(
                        (const void*)(a.x + (size_t)m * a.ldx + k0 + lane * 8),
                        (LDS(void)*)(Lb[bsel].x + m * L.xs), 16, 0, 0);
            if (a.xmode == GEMV_X_NORM && lane < nb)
                wnb[bsel] = *(const s2p_u32x4*)(a.norm_w + k0 + lane * 8);
        };
        auto stage_db = [&](int c, int bsel) __attribute__((always_inline)) {
            const int gn = min(G4_WIN, G - c * G4_WIN);
            const int nb = gn * 4;
            __syncthreads(); /* the previous window (and its X3) is no longer read */
            zero_tail(gn);
            vm_drain(); /* this wave's rows of window c (and the weights issued before) landed */
            __syncthreads();
            for (int m = wave; m < M; m += G4_WAVES) {
                const bool ok = lane < nb;
                const s2p_u32x4 rw = ok ? *(const LDS(s2p_u32x4)*)(Lb[bsel].x + m * L.xs + lane * 8)
                                        : (s2p_u32x4){0u, 0u, 0u, 0u};
                gv_stage_one<GEMV_W_INT4>(a, Lb[bsel], m, lane, ok, rw, wnb[bsel]);
            }
            __syncthreads();
        };
        auto mult_db = [&](const GvBuf& B, int c, int bsel) __attribute__((always_inline)) {
            gv_compute<GEMV_W_INT4, MT, false, G4_PIPE(MT)>(B, Lb[bsel], 0, min(G4_WIN, G - c * G4_WIN), M, 0, q,
                                               r, acc, corr);
        };
        issue(c0, 0);
        for (int c = c0; c < ce; c += 2) {
            stage_db(c, 0);
            if (c == c0) G4_STAMP(2);
            if (c + 1 < ce) {
                issue(c + 1, 1);
                load_c(b1, c + 1);
            }
            mult_db(b0, c, 0);
            if (c + 1 >= ce) break;
            stage_db(c + 1, 1);
            if (c + 2 < ce) {
                issue(c + 2, 0);
                load_c(b0, c + 2);
            }
            mult_db(b1, c + 1, 1);
        }
    } else
    for (int c = c0; c < ce; c += 2) {
        stage(c);
        if (c == c0) G4_STAMP(2);
        if (c + 1 < ce) {
            prefetch(c + 1);
            load_c(b1, c + 1);
        }
        mult(b0, c);
        if (c + 1 >= ce) break;
        stage(c + 1);
        if (c + 2 < ce) {
            prefetch(c + 2);
            load_c(b0, c + 2);
        }
        mult(b1, c + 1);
    }

    /* epilogue: element i of lane (q, r) in column tile t is
     * (n, m) = (wbase + 4q + i, 16t + r) */
    s2p_f32x4 v[MT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) v[t][i] = 16.0f * acc[t][i] - 24.0f * corr[t][i];
    G4_STAMP(3);
    uint16_t* Y = a.y;
    if (a.splits > 1) {
        /* K split: this split's partial rows in the 64-row block layout of
         * the merge (wave w holds rows 16w..16w+15, SWIGLU gate rows then up
         * rows), plain stores; k_g4_merge, the next launch, sums the splits
         * in order and runs the epilogue.  The workgroup's 128 rows are two
         * 64-row blocks: block h holds tiles 4h..4h+3, or (SWIGLU) gate
         * tiles 2h, 2h+1 then the matching up tiles */
        const int h = swiglu ? (wave & 3) >> 1 : wave >> 2;
        const int row = swiglu ? (wave >= 4 ? 32 : 0) + (wave & 1) * 16 : (wave & 3) * 16;
        const int rb = blockIdx.x * 2 + h;
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int m = t * 16 + r;
            if (m >= M || rb >= a.nrb) continue;
            float* dst = &a.part[(((size_t)sp * M + m) * a.nrb + rb) * 64 + row + q * 4];
            *(s2p_f32x4*)dst = v[t];
        }
        return;
    }
    if (swiglu) {
        /* gate wave w and up wave w + 4 hold the two halves of the same
         * outputs: each takes half the column tiles (the gate wave the first
         * TH, the up wave the rest) and hands the other half of its values
         * over through LDS, so both halves of the SiLU work run at once */
        constexpr int TH = (MT + 1) / 2;
        __syncthreads(); /* the last window is no longer read: reuse x for the exchange */
        LDS(s2p_f32x4)* ex = (LDS(s2p_f32x4)*)smem;
        const int pw = wave & 3;
#pragma unroll
        for (int t = 0; t < MT; t++)
            if ((wave >= 4) == (t < TH)) ex[(pw * MT + t) * 64 + lane] = v[t];
        __syncthreads();
        if (active) {
#pragma unroll
            for (int t = 0; t < MT; t++) {
                if ((wave >= 4) != (t >= TH)) continue; /* uniform */
                const s2p_f32x4 o = ex[(pw * MT + t) * 64 + lane];
                const s2p_f32x4 gv = wave < 4 ? v[t] : o, uv = wave < 4 ? o : v[t];
                const int m = t * 16 + r;
                if (m >= M) continue;
                uint16_t h[4];
#pragma unroll
                for (int i = 0; i < 4; i++) h[i] = silu_mul_bf16(f2bf(gv[i]), f2bf(uv[i]));
                /* outputs tile * 16 + 4 q .. + 3 of row m: one 8-byte store
                 * where aligned (F is a multiple of 32) */
                uint16_t* yp = Y + (size_t)m * a.ldy + tile * 16 + 4 * q;
                if (((uintptr_t)yp & 7) == 0) {
                    *(uint64_t*)yp = (uint64_t)h[0] | ((uint64_t)h[1] << 16) |
                                     ((uint64_t)h[2] << 32) | ((uint64_t)h[3] << 48);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i++) yp[i] = h[i];
                }
            }
        }
        return;
    }
    if (!active) return;
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const int m = t * 16 + r;
        float sq = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = wbase + 4 * q + i;
            if (m >= M || n >= a.N) continue;
            const uint16_t yb = f2bf(v[t][i]);
            uint16_t* yp = Y + (size_t)m * a.ldy + n;
            if (a.epi == GEMV_EPI_RESID) {
                const uint16_t xo = f2bf(__fadd_rn(bf2f(*yp), bf2f(yb)));
                *yp = xo;
                const float xv = bf2f(xo);
                sq += xv * xv;
            } else {
                *yp = yb;
            }
        }
        if (a.epi == GEMV_EPI_RESID && a.ssq_out) {
            /* the tile's 16 rows of column m: 4 per lane, then across q */
            sq += __shfl_xor(sq, 16, 64);
            sq += __shfl_xor(sq, 32, 64);
            if (q == 0 && m < M) coh_stf(a.ssq_out + (size_t)tile * GEMV_MAX_M + m, sq);
        }
    }
}

/* the K-split merge: 64-row block blockIdx.x, its items (4 adjacent
 * outputs of one row m) blockIdx.y * G4_MERGE_T + tid, then every
 * gridDim.y * G4_MERGE_T (every split's partials in flight together, summed
 * in split order, then the epilogue) */
#ifndef G4_MERGE_T
#define G4_MERGE_T 256
#endif
__global__ __launch_bounds__(G4_MERGE_T) void k_g4_merge(GemvArgs a) {
    gv_fixup4<1, GEMV_W_INT4, false, true>(a, blockIdx.x, a.y, threadIdx.x, blockIdx.y * G4_MERGE_T,
                                           gridDim.y * G4_MERGE_T);
}

/* the split merge of a RESID GEMM whose rows' inverse RMS the next GEMM
 * wants (inv_out): workgroup m takes all of row m, so after the outputs
 * (the same sums in split order and epilogue as k_g4_merge) it has every
 * 16-column sum of squares of the row and writes inv_out[m] (the order and
 * arithmetic of k_g4_rms) — no separate launch for it */
__global__ __launch_bounds__(1024) void k_g4_merge_rows(GemvArgs a) {
#pragma clang fp contract(off)
    __shared__ float sblk[G4_RMS_BLOCKS];
    const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int nit = a.N >> 2, S = a.splits;
    const size_t stride = (size_t)a.M * a.nrb * 64;
    uint16_t* Y = a.y;
    for (int i0 = 0; i0 < nit; i0 += (int)blockDim.x) {
        const int i = i0 + tid;
        const bool ok = i < nit;
        const int n0 = 4 * min(i, nit - 1), rb = n0 >> 6, l4 = n0 & 63;
        const float* p0 = a.part + ((size_t)m * a.nrb + rb) * 64 + l4;
        uint16_t* yp = Y + (size_t)m * a.ldy + n0;
        uint16_t yold[4];
#pragma unroll
        for (int e = 0; e < 4; e++) yold[e] = yp[e];
        s2p_f32x4 g = {0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < S; k0 += 8) {
            s2p_f32x4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++)
                v[j] = *(const s2p_f32x4*)(p0 + (size_t)min(k0 + j, S - 1) * stride);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                if (k0 + j >= S) break;
#pragma unroll
                for (int e = 0; e < 4; e++) g[e] += v[j][e];
            }
        }
        float ssq = 0.f;
        uint16_t ov[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint16_t xo = f2bf(__fadd_rn(bf2f(yold[e]), bf2f(f2bf(g[e]))));
            ov[e] = xo;
            const float xv = bf2f(xo);
            ssq += xv * xv;
        }
        if (ok)
            *(uint64_t*)yp = (uint64_t)ov[0] | ((uint64_t)ov[1] << 16) | ((uint64_t)ov[2] << 32) |
                             ((uint64_t)ov[3] << 48);
        /* a 16-column block is 4 adjacent lanes */
        ssq += __shfl_xor(ssq, 1, 64);
        ssq += __shfl_xor(ssq, 2, 64);
        if ((lane & 3) == 0 && ok) {
            if (a.ssq_out) a.ssq_out[(size_t)(n0 >> 4) * GEMV_MAX_M + m] = ssq;
            sblk[n0 >> 4] = ssq;
        }
    }
    __syncthreads();
    if (tid < 64) {
        float s = 0.f;
        for (int b = lane; b < (a.N >> 4); b += 64) s += sblk[b];
        s = wave_sum_down(s);
        if (lane == 0) a.inv_out[m] = rsqrt_rule(s / (float)a.N + a.inv_eps);
    }
}

extern "C" hipError_t s2p_g4_rms_launch(const float* ssq, int blocks, int M, int K, float eps,
                                        float* inv, hipStream_t st) {
    if (blocks > G4_RMS_BLOCKS || M > GEMV_MAX_M || (GEMV_MAX_M & 3)) return hipErrorInvalidValue;
    GemvArgs r;
    memset(&r, 0, sizeof(r));
    r.ssq_in = ssq;
    r.ssq_in_blocks = blocks;
    r.M = M;
    r.K = K;
    r.norm_eps = eps;
    hipLaunchKernelGGL(k_g4_rms, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, st, r, inv);
    return hipGetLastError();
}

template <int MT>
static hipError_t g4_launch_mt(const GemvArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    /* once per instantiation (thread-safe static initialisation) */
    static const hipError_t attr = hipFuncSetAttribute(
        (const void*)k_gemm4<MT>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    (void)attr;
    hipLaunchKernelGGL((k_gemm4<MT>), grid, dim3(64 * G4_WAVES), lds, st, a);
    return hipGetLastError();
}

/* INT4 weights, 16 < M <= 96, any epilogue; hipErrorNotSupported otherwise
 * (the caller falls back to the split-K GEMV engine). */
extern "C" hipError_t s2p_gemm4_launch(const GemvArgs* ap, hipStream_t st) {
    const GemvArgs& a = *ap;
    if (a.wfmt != GEMV_W_INT4 || a.M <= 16 || a.M > G4_MAX_M || (a.K & 127) || a.N <= 0)
        return hipErrorNotSupported;
    if (a.epi == GEMV_EPI_SWIGLU && ((a.N & 1) || ((a.N >> 1) & 31))) return hipErrorInvalidValue;
    if (a.xmode == GEMV_X_NORM && (!a.norm_w || !a.ssq_in || a.ssq_in_blocks <= 0))
        return hipErrorInvalidValue;
    const size_t lds = g4_lds_bytes(a.M);
    if (lds > 160 * 1024) return hipErrorNotSupported;
    GemvArgs b = a;
    /* NORM: the rows' inverse RMS as the producer wrote it (inv_in), else
     * by k_g4_rms first, into the last GEMV_MAX_M floats of the split
     * scratch (kept out of the partials) */
    float* inv_buf = nullptr;
    if (a.xmode == GEMV_X_NORM && !a.inv_in && a.part && a.part_cap >= 4 * GEMV_MAX_M &&
        a.ssq_in_blocks <= G4_RMS_BLOCKS && (GEMV_MAX_M & 3) == 0) {
        const int64_t at = (a.part_cap - GEMV_MAX_M) & ~(int64_t)63;
        inv_buf = a.part + at;
        b.part_cap = at;
    }
    /* workgroups of 8 row tiles (SWIGLU: 4 gate + 4 up tiles) */
    const unsigned nblk = a.epi == GEMV_EPI_SWIGLU
                              ? (unsigned)(((a.N >> 1) / 16 + 3) / 4)
                              : (unsigned)(((a.N + 15) / 16 + G4_WAVES - 1) / G4_WAVES);
    /* 64-row blocks of the split merge (SWIGLU: 32 gate + 32 up) */
    const int nrb = a.epi == GEMV_EPI_SWIGLU ? (a.N >> 1) / 32 : (a.N + 63) / 64;
    /* too few row blocks to fill the chip: split K over at most one
     * workgroup per CU (needs the caller's split-K scratch for the
     * partials).  One workgroup fits a CU, so a grid past the CU count runs
     * in two rounds: gate_up (152 row blocks) split in two took 44.5 us at
     * M = 40, unsplit (five windows a workgroup, no handoff) about half */
    const int nch = ((a.K >> 5) + G4_WIN - 1) / G4_WIN;
    const int cus = s2p_cu_count();
    int ks = (int)((unsigned)cus / nblk);
    if (ks > nch) ks = nch;
    if (ks < 1) ks = 1;
    int cps = (nch + ks - 1) / ks;
    ks = (nch + cps - 1) / cps;
    b.nrb = nrb;
    if (ks > 1 && (!a.part || (int64_t)ks * a.M * nrb * 64 > b.part_cap)) {
        ks = 1;
        cps = nch;
    }
    b.splits = ks;
    b.win = cps;
    const dim3 grid(nblk, (unsigned)ks);
    if (inv_buf) {
        hipLaunchKernelGGL(k_g4_rms, dim3((unsigned)((a.M + 3) / 4)), dim3(256), 0, st, b, inv_buf);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        b.inv_in = inv_buf;
    }
    hipError_t err;
    switch ((a.M + 15) / 16) {
        case 2: err = g4_launch_mt<2>(b, grid, lds, st); break;
        case 3: err = g4_launch_mt<3>(b, grid, lds, st); break;
        case 4: err = g4_launch_mt<4>(b, grid, lds, st); break;
        case 5: err = g4_launch_mt<5>(b, grid, lds, st); break;
        default: err = g4_launch_mt<6>(b, grid, lds, st); break;
    }
    if (err != hipSuccess) return err;
    if (ks > 1 && a.deferred && a.epi == GEMV_EPI_STORE) { /* the consumer merges */
        *a.deferred = ks;
        return hipSuccess;
    }
    const bool want_inv = a.inv_out && a.epi == GEMV_EPI_RESID && a.ssq_out;
    if (ks == 1) /* the kernel's epilogue wrote the sums of squares */
        return want_inv ? s2p_g4_rms_launch(a.ssq_out, (a.N + 15) / 16, a.M, a.N, a.inv_eps,
                                            a.inv_out, st)
                        : hipSuccess;
    if (want_inv && (a.N & 15) == 0 && a.N / 16 <= G4_RMS_BLOCKS && (a.ldy & 3) == 0 &&
        ((uintptr_t)a.y & 7) == 0) { /* k_g4_merge_rows stores four outputs at once */
        const int nit = a.N >> 2;
        const unsigned th = (unsigned)(nit >= 1024 ? 1024 : ((nit + 63) / 64) * 64);
        hipLaunchKernelGGL(k_g4_merge_rows, dim3((unsigned)a.M), dim3(th), 0, st, b);
        return hipGetLastError();
    }
    const int items = a.M * (a.epi == GEMV_EPI_SWIGLU ? 8 : 16);
    const unsigned ny = (unsigned)((items + G4_MERGE_T - 1) / G4_MERGE_T);
    hipLaunchKernelGGL(k_g4_merge, dim3((unsigned)nrb, ny), dim3(G4_MERGE_T), 0, st, b);
    err = hipGetLastError();
    if (err != hipSuccess || !want_inv) return err;
    return s2p_g4_rms_launch(a.ssq_out, (a.N + 15) / 16, a.M, a.N, a.inv_eps, a.inv_out, st);
}
