/* s2pro MI355X — device sampler and speculative acceptance.
 *
 * Compiled with FP contraction off: every float operation of the rule is one
 * IEEE rounding, in the order of the reference sampler (sampling.c:119-282),
 * and exp/log are the rule's s2p_expf/s2p_logf (binary64 evaluation, one
 * rounding), so sampled ids and accept/reject decisions are bit-identical to
 * the host restatement for the same state and logits.
 *
 * k_transform: one workgroup per (row, target|draft).
 *   1. sampler state of the row: the session state plus, for a verify tree
 *      node, the drafted tokens on its root path pushed as emitted tokens
 *      (sampling.c:269-281), so node i sees the history with d_1..d_i;
 *   2. gather the 4096 semantic logits + EOS (bf16 -> f32, exact);
 *   3. RAS detect and repetition penalty on one lane (gather then scatter);
 *   4. top-30 by value desc / index asc: a 4-pass 8-bit radix select finds
 *      the 30th largest value, ties at the threshold are taken in index
 *      order through a block prefix count, and the 30 survivors are ranked;
 *   5. top-p over the un-tempered softmax and the temperature softmax: the
 *      exps are elementwise across lanes, every sum is sequential on lane 0.
 *   s2pk_sample then draws (seeded hash-Gumbel or xoshiro inverse CDF,
 *   sampling.c:221-262) and updates the state; the verify path writes the
 *   30 (candidate, probability) pairs to the workspace.
 * k_accept: one wave per session walks the draft tree root-first
 *   (Leviathan et al. 2211.17192; SpecInfer multi-candidate form for
 *   siblings): child c of node v with drafted id d is accepted iff
 *   u * q_v(d) < p_v(d) (u a 24-bit uniform, compared exactly in binary64);
 *   on rejection p_v <- norm(max(0, p_v - q_v)) and the next sibling is
 *   tried; when no child is accepted the corrected token is drawn from the
 *   residual, and at an accepted leaf the bonus token is drawn from p exactly
 *   as s2ps_sample would.  An accepted EOS ends generation.  The state
 *   advances over every emitted non-EOS id.
 */
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "common.h"
#include "s2pro/s2p_fmath.h"
#include "s2pro/slowar_kernels.h"
#include "sample_internal.h"

#define N_SEM 4096
#define N_CAND 4097
#define CAND_EOS 4096
#define TOP_K 30
#define TOK_EOS 151645LL
#define SEM_START 151678LL
#define SEM_END 155773LL
#define TX_THREADS 256

/* ------------------------------------------------------------ RNG pieces */

S2P_DEV uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
S2P_DEV uint64_t xoshiro_next(uint64_t* s) {
    const uint64_t result = rotl64(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}

/* reference seeded draw, sampling.c:221-243 */
S2P_DEV int gumbel_draw(const s2ps_dev_state* sp, const float* prob) {
    const uint64_t step_seed = ((uint64_t)sp->seed31 * 19349663ULL) ^ (sp->count * 73856093ULL);
    float best = -INFINITY;
    int choice = 0;
    for (int j = 0; j < TOP_K; j++) {
        const uint64_t hashed = (step_seed * 8589934591ULL) ^ ((uint64_t)j * 479001599ULL);
        float u = (float)(uint32_t)(hashed & 0xFFFFFFULL) / 16777216.0f;
        if (u < 1e-10f) u = 1e-10f;
        const float g = -s2p_logf(-s2p_logf(u));
        const float pert = s2p_logf(prob[j] + 1e-10f) + g;
        if (pert > best) {
            best = pert;
            choice = j;
        }
    }
    return choice;
}

/* reference unseeded draw, sampling.c:244-262 */
S2P_DEV int xoshiro_draw(s2ps_dev_state* sp, const float* prob) {
    const double r = (double)(xoshiro_next(sp->rng) >> 11) * 0x1.0p-53;
    double cum2 = 0.0;
    int lastnz = 0, choice = -1;
    for (int j = 0; j < TOP_K; j++) {
        if (prob[j] <= 0.f) continue;
        lastnz = j;
        cum2 += (double)prob[j];
        if (r < cum2) {
            choice = j;
            break;
        }
    }
    return choice < 0 ? lastnz : choice;
}

/* acceptance-rule uniform: splitmix64 finaliser of (seed31, count, slot) */
S2P_DEV uint32_t rule_u24(const s2ps_dev_state* sp, uint32_t slot) {
    uint64_t z = ((uint64_t)sp->seed31 * 0x9E3779B97F4A7C15ULL) ^
                 (sp->count * 0xBF58476D1CE4E5B9ULL) ^
                 ((uint64_t)(slot + 1) * 0x94D049BB133111EBULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    z ^= z >> 31;
    return (uint32_t)(z >> 40);
}

S2P_DEV int residual_draw(s2ps_dev_state* sp, const float* prob) {
    if (!sp->seeded) return xoshiro_draw(sp, prob);
    float best = -INFINITY;
    int choice = 0;
    for (int j = 0; j < TOP_K; j++) {
        if (!(prob[j] > 0.f)) continue;
        float u = (float)rule_u24(sp, (uint32_t)j) / 16777216.0f;
        if (u < 1e-10f) u = 1e-10f;
        const float g = -s2p_logf(-s2p_logf(u));
        const float pert = s2p_logf(prob[j] + 1e-10f) + g;
        if (pert > best) {
            best = pert;
            choice = j;
        }
    }
    return choice;
}

S2P_DEV void state_push(s2ps_dev_state* sp, int64_t tok) {
    if (tok == TOK_EOS) return;
    if (sp->count < (uint64_t)sp->window) {
        sp->prev[sp->count] = tok;
    } else {
        for (int j = 0; j < sp->window - 1; j++) sp->prev[j] = sp->prev[j + 1];
        sp->prev[sp->window - 1] = tok;
    }
    sp->count++;
}

/* state_push by the 64 lanes of one wave (wave-uniform arguments): the
 * window shift is one LDS read and one write per lane instead of a serial
 * loop; a wave's read completes for all lanes before its write */
S2P_DEV void state_push_wave(s2ps_dev_state* sp, int64_t tok, int lane) {
    if (tok == TOK_EOS) return;
    const int W = sp->window;
    if (sp->count < (uint64_t)W) {
        if (lane == 0) sp->prev[sp->count] = tok;
    } else {
        const int64_t nx = lane < W - 1 ? sp->prev[lane + 1] : 0;
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
        if (lane < W - 1) sp->prev[lane] = nx;
        if (lane == 0) sp->prev[W - 1] = tok;
    }
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) sp->count++;
    __builtin_amdgcn_wave_barrier();
}

S2P_DEV int64_t cand_to_vocab(int ci) { return ci == CAND_EOS ? TOK_EOS : SEM_START + ci; }
S2P_DEV int vocab_to_cand(int64_t t) {
    if (t >= SEM_START && t <= SEM_END) return (int)(t - SEM_START);
    if (t == TOK_EOS) return CAND_EOS;
    return -1;
}

/* orderable key of a float (-0 folded onto +0): unsigned order == value order */
S2P_DEV uint32_t okey(float v) {
    uint32_t u = __float_as_uint(v + 0.0f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* --------------------------------------------------------------- transform */

struct TxShared {
    float cand[N_CAND];
    s2ps_dev_state st;
    unsigned hist[4][256]; /* one histogram per wave (LDS atomics contend less) */
    uint32_t prefix;
    int need;       /* survivors still to take at the threshold key */
    int n_gt;       /* collected strictly above the threshold */
    int eq_base[TX_THREADS];
    float tv[32];
    int ti[32];
    float e[32];
    float p2[32];
    int greedy;
    float temp, topp, m, sum, t, m2, s2;
    int masked[32];
    /* the tree (accept transform): parents, drafted tokens, a root path */
    int par[64];
    int64_t tks[64];
    int path[64];
    int npath;
};

/* Sampler transform of one logits row into sh.ti / sh.p2 (ranks 0..29). */
__device__ void transform_row(TxShared& sh, const uint16_t* lrow, const uint16_t* eos_ptr) {
    const int tid = threadIdx.x;
    /* gather: every load of the thread issued before the first is waited
     * for (a load-store loop would wait out one memory round trip per
     * element) */
    {
        constexpr int PG = N_SEM / TX_THREADS;
        static_assert(N_SEM % TX_THREADS == 0, "gather split");
        const uint16_t* src = eos_ptr ? lrow : lrow + SEM_START;
        uint16_t r[PG];
#pragma unroll
        for (int j = 0; j < PG; j++) r[j] = src[tid + j * TX_THREADS];
        const uint16_t re = *(eos_ptr ? eos_ptr : lrow + TOK_EOS); /* every thread: one more load in the batch */
#pragma unroll
        for (int j = 0; j < PG; j++) sh.cand[tid + j * TX_THREADS] = bf2f(r[j]);
        if (tid == 0) sh.cand[CAND_EOS] = bf2f(re);
    }
    __syncthreads();
    /* RAS detection (sampling.c:129-174) on lane 0, then the repetition penalty */
    if (tid == 0) {
        const s2ps_dev_state* sp = &sh.st;
        const int greedy = sp->temperature == 0.0f;
        const int capped = sp->count < (uint64_t)sp->window ? (int)sp->count : sp->window;
        int use_ras = 0;
        if (!greedy && capped >= 4) {
            int64_t last4[4];
            for (int r = 0; r < 4; r++) {
                int idx = capped - (4 - r);
                if (idx < 0) idx = 0;
                last4[r] = sp->prev[idx];
            }
            for (int a = 0; a < 3; a++)
                for (int b = a + 1; b < 4; b++)
                    if (last4[b] < last4[a]) {
                        const int64_t t = last4[a];
                        last4[a] = last4[b];
                        last4[b] = t;
                    }
            for (int a = 0; a < 3; a++)
                if (last4[a] == last4[a + 1]) use_ras = 1;
        }
        sh.greedy = greedy;
        sh.temp = use_ras ? 1.0f : sp->temperature;
        sh.topp = use_ras ? 0.9f : sp->top_p;
    }
    {
        /* repetition penalty, one window entry per thread: every entry's
         * value is read before any is written (the rule's gather, then its
         * scatter; repeated tokens write the same value) */
        const s2ps_dev_state* sp = &sh.st;
        const int capped = sp->count < (uint64_t)sp->window ? (int)sp->count : sp->window;
        int ci = -1;
        float rv = 0.f;
        if (tid < capped && tid < 64) {
            ci = vocab_to_cand(sp->prev[tid]);
            if (ci >= 0) {
                const float v = sh.cand[ci];
                rv = v < 0.f ? v * sp->rep_penalty : v / sp->rep_penalty;
            }
        }
        __syncthreads();
        if (ci >= 0) sh.cand[ci] = rv;
    }
    __syncthreads();
    /* this thread's keys (a contiguous index range) stay in registers */
    constexpr int PER = (N_CAND + TX_THREADS - 1) / TX_THREADS; /* 17 */
    const int i0 = tid * PER;
    uint32_t kk[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) kk[j] = i0 + j < N_CAND ? okey(sh.cand[i0 + j]) : 0u;
    if (tid == 0) {
        sh.prefix = 0;
        sh.need = TOP_K;
    }
    __syncthreads();
    /* radix select of the 30th largest key, 8 bits per pass from the top */
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;
        const uint32_t hmask = pass == 0 ? 0u : (0xFFFFFFFFu << (shift + 8));
#pragma unroll
        for (int w = 0; w < 4; w++) sh.hist[w][tid] = 0;
        __syncthreads();
        const uint32_t pre = sh.prefix;
        unsigned* hw = sh.hist[tid >> 6];
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (i0 + j < N_CAND && (kk[j] & hmask) == pre) atomicAdd(&hw[(kk[j] >> shift) & 0xFFu], 1u);
        __syncthreads();
        if (tid < 64) {
            /* lane l owns bins 255-4l .. 252-4l (descending) */
            unsigned b4[4], own = 0;
            for (int i = 0; i < 4; i++) {
                const int bin = 255 - 4 * tid - i;
                b4[i] = sh.hist[0][bin] + sh.hist[1][bin] + sh.hist[2][bin] + sh.hist[3][bin];
                own += b4[i];
            }
            /* exclusive prefix over lanes in descending-bin order */
            unsigned incl = own;
            for (int off = 1; off < 64; off <<= 1) {
                const unsigned o = __shfl_up(incl, off, 64);
                if (tid >= off) incl += o;
            }
            const unsigned excl = incl - own;
            const int need = sh.need;
            if (excl < (unsigned)need && incl >= (unsigned)need) {
                unsigned cum = excl;
                for (int i = 0; i < 4; i++) {
                    if (cum + b4[i] >= (unsigned)need) {
                        const uint32_t bin = 255u - 4u * tid - i;
                        sh.prefix = pre | (bin << shift);
                        sh.need = need - (int)cum;
                        break;
                    }
                    cum += b4[i];
                }
            }
        }
        __syncthreads();
    }
    /* collect: keys above the threshold, then the first `need` equal keys in
     * index order (contiguous index ranges per thread + block prefix count) */
    const uint32_t T = sh.prefix;
    const int need = sh.need;
    if (tid == 0) sh.n_gt = 0;
    int n_eq = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PER; j++) {
        if (i0 + j >= N_CAND) break;
        const uint32_t k = kk[j];
        if (k > T) {
            const int s = atomicAdd(&sh.n_gt, 1);
            sh.ti[s] = i0 + j;
        } else if (k == T) {
            n_eq++;
        }
    }
    {
        /* exclusive prefix of the per-thread tie counts in thread order
         * (integers: any association gives the same result) */
        const int lane = tid & 63, wv = tid >> 6;
        int inc = n_eq;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int o = __shfl_up(inc, off, 64);
            if (lane >= off) inc += o;
        }
        if (lane == 63) sh.eq_base[wv] = inc; /* wave totals, read below */
        __syncthreads();
        int base = 0;
        for (int w = 0; w < wv; w++) base += sh.eq_base[w];
        __syncthreads();
        sh.eq_base[tid] = base + inc - n_eq;
    }
    __syncthreads();
    {
        int r = sh.eq_base[tid];
        const int ngt = TOP_K - need; /* == sh.n_gt */
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (i0 + j < N_CAND && r < need && kk[j] == T) {
                sh.ti[ngt + r] = i0 + j;
                r++;
            }
    }
    __syncthreads();
    /* rank the 30 survivors: value desc, index asc */
    int my_i = 0, rank = 0;
    float my_v = 0.f;
    if (tid < TOP_K) {
        my_i = sh.ti[tid];
        my_v = sh.cand[my_i];
        const uint32_t mk = okey(my_v);
#pragma unroll
        for (int j = 0; j < TOP_K; j++) {
            const int oi = sh.ti[j];
            const uint32_t ok = okey(sh.cand[oi]);
            rank += (ok > mk) || (ok == mk && oi < my_i);
        }
    }
    __syncthreads();
    if (tid < TOP_K) {
        sh.tv[rank] = my_v;
        sh.ti[rank] = my_i;
    }
    __syncthreads();
    /* two softmaxes (sampling.c:196-219) */
    if (sh.greedy) {
        if (tid < 32) sh.p2[tid] = tid == 0 ? 1.0f : 0.0f;
        __syncthreads();
        return;
    }
    if (tid < TOP_K) sh.e[tid] = s2p_expf(sh.tv[tid] - sh.tv[0]);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < TOP_K; j++) sum += sh.e[j];
        float cum = 0.f;
#pragma unroll
        for (int j = 0; j < TOP_K; j++) {
            cum += sh.e[j] / sum;
            sh.masked[j] = (j > 0 && cum > sh.topp) ? 1 : 0;
        }
        const float t = sh.temp < 1e-5f ? 1e-5f : sh.temp;
        sh.t = t;
        sh.m2 = sh.tv[0] / t;
    }
    __syncthreads();
    if (tid < TOP_K) sh.p2[tid] = sh.masked[tid] ? 0.f : s2p_expf(sh.tv[tid] / sh.t - sh.m2);
    __syncthreads();
    if (tid == 0) {
        float s2 = 0.f;
#pragma unroll
        for (int j = 0; j < TOP_K; j++) s2 += sh.p2[j];
        sh.s2 = s2;
    }
    __syncthreads();
    if (tid < TOP_K) sh.p2[tid] = sh.p2[tid] / sh.s2;
    __syncthreads();
}

/* ------------------------------------------------------------ s2pk_sample */

__global__ __launch_bounds__(TX_THREADS) void k_sample(const uint16_t* __restrict__ logits,
                                                       int64_t vocab_stride,
                                                       const uint16_t* __restrict__ eos_logits,
                                                       s2ps_dev_state* const* states,
                                                       int64_t* out_tok, int32_t* out_sem,
                                                       int32_t* out_codes, uint8_t* out_eos) {
    __shared__ TxShared sh;
    const int row = blockIdx.x;
    s2ps_dev_state* sp = states[row];
    {
        const uint32_t* src = (const uint32_t*)sp;
        uint32_t* dst = (uint32_t*)&sh.st;
        for (int i = threadIdx.x; i < (int)(sizeof(sh.st) / 4); i += TX_THREADS) dst[i] = src[i];
    }
    __syncthreads();
    transform_row(sh, logits + (size_t)row * vocab_stride, eos_logits ? eos_logits + row : nullptr);
    if (threadIdx.x != 0) return;
    int choice = 0;
    if (!sh.greedy) choice = sh.st.seeded ? gumbel_draw(&sh.st, sh.p2) : xoshiro_draw(&sh.st, sh.p2);
    const int ci = sh.ti[choice];
    const int64_t tok = cand_to_vocab(ci);
    out_tok[row] = tok;
    if (tok == TOK_EOS) {
        out_sem[row] = 0;
        if (out_codes) out_codes[(size_t)row * 10] = 0;
        out_eos[row] = 1;
    } else {
        out_sem[row] = ci;
        if (out_codes) out_codes[(size_t)row * 10] = ci;
        out_eos[row] = 0;
        state_push(&sh.st, tok);
    }
    *sp = sh.st;
}

extern "C" hipError_t s2pk_sample(const s2p_bf16* logits, int64_t vocab_stride,
                                  const s2p_bf16* eos_logits, s2ps_dev_state* const* states,
                                  int rows, int64_t* out_tok, int32_t* out_sem,
                                  int32_t* out_codes, uint8_t* out_eos, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_sample, dim3(rows), dim3(TX_THREADS), 0, st, (const uint16_t*)logits,
                       vocab_stride, (const uint16_t*)eos_logits, states, out_tok, out_sem,
                       out_codes, out_eos);
    return hipGetLastError();
}

/* ------------------------------------------------------------- acceptance */

/* workspace entry per (session, node, target|draft) */
struct TxOut {
    int32_t ti[32];
    float p[32];
    int32_t greedy;
    int32_t pad_[31];
};
static_assert(sizeof(TxOut) % 16 == 0 && offsetof(TxOut, greedy) == 64 * 4, "the walk copies TxOut words 0..67 as 17 16-byte chunks");

__global__ __launch_bounds__(TX_THREADS) void k_accept_transform(AcceptArgs a) {
    __shared__ TxShared sh;
    const int gr = blockIdx.x;          /* global node row s * R + v */
    const int which = blockIdx.y;       /* 0 target, 1 draft */
    const int s = gr / a.R, v = gr - s * a.R;
    /* a forward whose bounded wait timed out: its logits are not read (the
     * walk reports the session as undecided) */
    if (a.fwd_err && *(const volatile int*)a.fwd_err != 0) return;
    /* the state and the tree in one batch of loads */
    {
        const uint32_t* src = (const uint32_t*)a.states[s];
        uint32_t* dst = (uint32_t*)&sh.st;
        for (int i = threadIdx.x; i < (int)(sizeof(sh.st) / 4); i += TX_THREADS) dst[i] = src[i];
        if (threadIdx.x < a.R) {
            sh.par[threadIdx.x] = a.parent[threadIdx.x];
            sh.tks[threadIdx.x] = a.tok[(size_t)s * a.R + threadIdx.x];
        }
    }
    __syncthreads();
    /* leaves need no draft transform */
    if (which == 1) {
        bool has_child = false;
        for (int c = v + 1; c < a.R; c++) has_child |= sh.par[c] == v;
        if (!has_child) return;
    }
    if (threadIdx.x == 0) {
        /* root path (root excluded); parent indices are validated (parent[u]
         * in [0, u)) so a malformed tree ends the walk */
        int n = 0;
        for (int u = v; u > 0 && u < a.R && n < 64;) {
            sh.path[n++] = u;
            const int p = sh.par[u];
            if (p < 0 || p >= u) break;
            u = p;
        }
        sh.npath = n;
    }
    __syncthreads();
    /* push the path's drafted tokens, root side first (wave 0) */
    if (threadIdx.x < 64)
        for (int i = sh.npath - 1; i >= 0; i--) state_push_wave(&sh.st, sh.tks[sh.path[i]], threadIdx.x);
    __syncthreads();
    const uint16_t* base = which ? a.drf : a.tgt;
    const uint16_t* eos = which ? a.drf_eos : a.tgt_eos;
    const int64_t es = which ? a.drf_eos_stride : a.tgt_eos_stride;
    transform_row(sh, base + (size_t)gr * a.row_stride, eos ? eos + (size_t)gr * es : nullptr);
    TxOut* o = (TxOut*)a.work + ((size_t)gr * 2 + which);
    if (threadIdx.x < 32) {
        o->ti[threadIdx.x] = threadIdx.x < TOP_K ? sh.ti[threadIdx.x] : -1;
        o->p[threadIdx.x] = threadIdx.x < TOP_K ? sh.p2[threadIdx.x] : 0.f;
    }
    if (threadIdx.x == 0) o->greedy = sh.greedy;
}

/* p of the first j with ti[j] == ci, else 0: a branchless scan from the end
 * (its reads are independent, so they issue together instead of one LDS
 * round trip per step) */
S2P_DEV float prob_of(const int32_t* ti, const float* p, int ci) {
    float r = 0.f;
#pragma unroll
    for (int j = TOP_K - 1; j >= 0; j--) r = ti[j] == ci ? p[j] : r;
    return r;
}

/* argmax over the wave with the sequential rule's tie order: the first
 * (lowest) index among equal maxima; NaN never wins (the sequential loop's
 * `pert > best` is false for NaN); all -inf -> index 0 */
S2P_DEV int wave_argmax_first(float v, int idx) {
    if (v != v) v = -INFINITY;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
    return idx;
}

/* perturbed log-probability of candidate j of a seeded draw: the loop
 * bodies of gumbel_draw (plain sample / bonus token, residual == false)
 * and residual_draw (residual == true), one candidate per lane */
S2P_DEV float draw_pert(const s2ps_dev_state* sp, const float* prob, int j, bool residual) {
    if (j >= TOP_K) return -INFINITY;
    float u;
    if (residual) {
        if (!(prob[j] > 0.f)) return -INFINITY;
        u = (float)rule_u24(sp, (uint32_t)j) / 16777216.0f;
    } else {
        const uint64_t step_seed = ((uint64_t)sp->seed31 * 19349663ULL) ^ (sp->count * 73856093ULL);
        const uint64_t hashed = (step_seed * 8589934591ULL) ^ ((uint64_t)j * 479001599ULL);
        u = (float)(uint32_t)(hashed & 0xFFFFFFULL) / 16777216.0f;
    }
    if (u < 1e-10f) u = 1e-10f;
    const float g = -s2p_logf(-s2p_logf(u));
    return s2p_logf(prob[j] + 1e-10f) + g;
}

/* One wave per session.  Control flow is uniform: every lane reads the same
 * state (in LDS) and takes the same decisions; lane 0 alone mutates the
 * state; the per-candidate work of the seeded draws and of the residual
 * (two logs per candidate, the dominant cost) runs one candidate per lane,
 * with the sequential rule's sums and tie order kept. */
__global__ __launch_bounds__(64) void k_accept_walk(AcceptArgs a) {
    __shared__ s2ps_dev_state st;
    __shared__ float p[TOP_K], qp[TOP_K], rsd[TOP_K];
    __shared__ int32_t pti[TOP_K], qti[TOP_K];
    __shared__ uint32_t bcast;
    /* the (target, draft) transforms of every node: the first 68 words
     * (ti, p, greedy) of each TxOut entry */
    __shared__ uint32_t wk[64 * 2 * 68];
    __shared__ int32_t par[64];
    __shared__ int64_t tks[64];
    __shared__ uint8_t cok[64];
    const int s = blockIdx.x, lane = threadIdx.x;
    const int R = a.R;
    if (a.fwd_err && *(const volatile int*)a.fwd_err != 0) {
        /* the forward that produced the logits did not complete (a bounded
         * wait of the persistent kernel timed out): decide nothing */
        if (lane == 0) {
            a.out_n_acc[s] = -1;
            a.out_n_emit[s] = 0;
        }
        return;
    }
    {
        /* everything the walk reads, in one batch of loads (the walk itself
         * then runs from LDS: a load per node would put a memory round trip
         * on every step of it) */
        const uint32_t* src = (const uint32_t*)a.states[s];
        uint32_t* dst = (uint32_t*)&st;
#pragma unroll 4
        for (int i = lane; i < (int)(sizeof(st) / 4); i += 64) dst[i] = src[i];
        if (lane < R) {
            par[lane] = a.parent[lane];
            tks[lane] = a.tok[(size_t)s * R + lane];
            cok[lane] = a.chain_ok ? a.chain_ok[(size_t)s * R + lane] : (uint8_t)1;
        }
        const s2p_u32x4* ws = (const s2p_u32x4*)((const TxOut*)a.work + (size_t)s * R * 2);
        s2p_u32x4* wd = (s2p_u32x4*)wk;
        const int n = R * 2 * 17;
#pragma unroll 4
        for (int i = lane; i < n; i += 64) {
            const int e = i / 17, c = i - e * 17;
            wd[i] = ws[e * (int)(sizeof(TxOut) / 16) + c];
        }
    }
    __syncthreads();
    const int64_t* tok = tks;
    int32_t* path = a.out_path + (size_t)s * R;
    int64_t* emit = a.out_emit + (size_t)s * (R + 1);
    int n_acc = 0, n_emit = 0;
    int v = 0, tail_node = -1;
    for (;;) {
        const uint32_t* tp = wk + (v * 2 + 0) * 68;
        const uint32_t* tq = wk + (v * 2 + 1) * 68;
        if (lane < TOP_K) {
            p[lane] = __uint_as_float(tp[32 + lane]);
            pti[lane] = (int32_t)tp[lane];
            qp[lane] = __uint_as_float(tq[32 + lane]);
            qti[lane] = (int32_t)tq[lane];
        }
        __syncthreads();
        const int greedy = (int)tp[64];
        int accepted = -1, rejected_any = 0, j = 0;
        for (int c = v + 1; c < R && accepted < 0; c++) {
            if (par[c] != v) continue;
            const int ci = vocab_to_cand(tok[c]);
            const float pc = ci < 0 ? 0.f : prob_of(pti, p, ci);
            const float qc = ci < 0 ? 0.f : prob_of(qti, qp, ci);
            uint32_t u;
            if (greedy) {
                u = 0u;
            } else if (st.seeded) {
                u = rule_u24(&st, 64u + (uint32_t)j);
            } else {
                if (lane == 0) bcast = (uint32_t)(xoshiro_next(st.rng) >> 40);
                __syncthreads();
                u = bcast;
                __syncthreads();
            }
            if ((double)u * (double)qc < (double)pc * 16777216.0) {
                accepted = c;
                break;
            }
            rejected_any = 1;
            if (lane < TOP_K) {
                const float d = p[lane] - prob_of(qti, qp, pti[lane]);
                rsd[lane] = d > 0.f ? d : 0.f;
            }
            __syncthreads();
            float z = 0.f;
#pragma unroll
            for (int k = 0; k < TOP_K; k++) z += rsd[k]; /* the rule's order */
            if (z > 0.f && lane < TOP_K) p[lane] = rsd[lane] / z;
            __syncthreads();
            j++;
        }
        if (accepted >= 0 && !cok[accepted]) {
            /* the drafted frame failed the chain condition: its token is
             * emitted, its row is not accepted, no bonus draw */
            tail_node = accepted;
            if (lane == 0) emit[n_emit] = tok[accepted];
            state_push_wave(&st, tok[accepted], lane);
            n_emit++;
            __syncthreads();
            break;
        }
        if (accepted >= 0) {
            if (lane == 0) {
                path[n_acc] = accepted;
                emit[n_emit] = tok[accepted];
            }
            n_acc++;
            n_emit++;
            if (tok[accepted] == TOK_EOS) {
                v = accepted; /* the EOS node's own row ends the walk */
                break;
            }
            state_push_wave(&st, tok[accepted], lane);
            __syncthreads();
            v = accepted;
            continue;
        }
        int choice = 0;
        if (greedy) {
            for (int k = 1; k < TOP_K; k++)
                if (p[k] > p[choice]) choice = k;
        } else if (st.seeded) {
            choice = wave_argmax_first(draw_pert(&st, p, lane, rejected_any != 0), lane);
        } else {
            if (lane == 0) bcast = (uint32_t)xoshiro_draw(&st, p);
            __syncthreads();
            choice = (int)bcast;
        }
        const int64_t t = cand_to_vocab(pti[choice]);
        if (lane == 0) emit[n_emit] = t;
        state_push_wave(&st, t, lane);
        n_emit++;
        __syncthreads();
        break;
    }
    if (lane == 0) {
        a.out_n_acc[s] = n_acc;
        a.out_n_emit[s] = n_emit;
        if (a.out_tail) {
            a.out_tail[2 * s] = v;
            a.out_tail[2 * s + 1] = tail_node;
        }
    }
    __syncthreads();
    {
        uint32_t* dst = (uint32_t*)a.states[s];
        const uint32_t* src = (const uint32_t*)&st;
        for (int i = lane; i < (int)(sizeof(st) / 4); i += 64) dst[i] = src[i];
    }
}

extern "C" size_t s2p_accept_work_bytes(int n_sess, int rows) {
    return (size_t)n_sess * rows * 2 * sizeof(TxOut);
}

extern "C" hipError_t s2p_accept_launch(const AcceptArgs* ap, hipStream_t st) {
    const AcceptArgs a = *ap;
    if (a.n_sess <= 0) return hipSuccess;
    if (a.R < 1 || a.R > 64 || !a.work) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_accept_transform, dim3(a.n_sess * a.R, 2), dim3(TX_THREADS), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_accept_walk, dim3(a.n_sess), dim3(64), 0, st, a);
    return hipGetLastError();
}
