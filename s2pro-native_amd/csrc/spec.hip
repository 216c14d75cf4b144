/* s2pro MI355X — device bookkeeping of the composed speculative tick
 * (csrc/host/spec.c): the verify plan advanced from device KV lengths, the
 * input embeddings of drafted and emitted frames, and the per-session state
 * carried from one tick to the next.  Each kernel is small and runs once or
 * a few times per tick; together they keep every per-tick decision on the
 * device, so consecutive ticks replay one graph with no host round trip.
 *
 * Frame embedding (reference decode tick, slowar.c:478-496): the token's
 * row of the bf16 embedding table (s2pk_embed); for a semantic token, plus
 * the bf16-rounded f32 sum of its frame's ten codebook rows in codebook
 * order (s2pfa_vq_embed_add, one bf16 add), then x 1/sqrt(11) rounded to
 * bf16 (s2pk_scale_rows_masked, kernels.cu:1413-1421).  Other tokens (EOS)
 * keep the plain table row. */
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"
#include "prims_dev.h"
#include "spec_internal.h"

#define SPEC_DIM 2560
#define SPEC_SEM0 151678LL
#define SPEC_EOS 151645LL
#define SPEC_VOCAB 155776LL

S2P_DEV int sem_code(int64_t t) {
    return (t >= SPEC_SEM0 && t < SPEC_SEM0 + 4096) ? (int)(t - SPEC_SEM0) : 0;
}

/* one block of 256 threads: out = frame embedding of (id, codes[0..9]) */
S2P_DEV void frame_embed(const uint16_t* __restrict__ table, const uint16_t* __restrict__ cb,
                         int64_t id, const int32_t* codes, uint16_t* __restrict__ out,
                         float scale) {
    const bool sem = id >= SPEC_SEM0 && id < SPEC_SEM0 + 4096;
    id = id < 0 ? 0 : (id >= SPEC_VOCAB ? SPEC_VOCAB - 1 : id);
    size_t rowc[10];
#pragma unroll
    for (int c = 0; c < 10; c++) {
        int v = codes[c];
        v = v < 0 ? 0 : (v > 4095 ? 4095 : v);
        rowc[c] = (size_t)(c * 4096 + v) * SPEC_DIM;
    }
    const uint16_t* trow = table + (size_t)id * SPEC_DIM;
    for (int d = threadIdx.x; d < SPEC_DIM; d += 256) {
        uint16_t x = trow[d];
        if (sem) {
            float acc = 0.f;
#pragma unroll
            for (int c = 0; c < 10; c++) acc += bf2f(cb[rowc[c] + d]);
            x = f2bf(__fadd_rn(bf2f(x), bf2f(f2bf(acc))));
            x = f2bf(__fmul_rn(bf2f(x), scale));
        }
        out[d] = x;
    }
}

/* The verify plan of the current device KV lengths: rows s*R + i of session
 * s at position L + depth[i], slot L + i; each segment's prefix and span.
 * A session whose L + R exceeds cap (the span the plan's launches were
 * sized for) keeps its previous plan and raises *overflow. */
__global__ __launch_bounds__(256) void k_plan_device(int32_t* __restrict__ pos, int32_t* __restrict__ slot,
                                                     S2pAttnSeg* __restrict__ segs, int n_seg,
                                                     const int32_t* __restrict__ kv_len,
                                                     const int32_t* __restrict__ depth, int n_sess,
                                                     int R, int cap, int32_t* __restrict__ overflow) {
    for (int r = threadIdx.x; r < n_sess * R; r += 256) {
        const int s = r / R, i = r - s * R, L = kv_len[s];
        if (L < 0 || L + R > cap) {
            if (overflow) *overflow = 1;
            continue;
        }
        pos[r] = L + depth[i];
        slot[r] = L + i;
    }
    for (int g = threadIdx.x; g < n_seg; g += 256) {
        const int L = kv_len[segs[g].sess];
        if (L < 0 || L + R > cap) continue;
        segs[g].L = L;
        segs[g].span = L + R;
    }
}

extern "C" hipError_t s2p_plan_device_launch(int32_t* pos, int32_t* slot, S2pAttnSeg* segs, int n_seg,
                                             const int32_t* kv_len, const int32_t* depth,
                                             int n_sess, int R, int cap, int32_t* overflow,
                                             hipStream_t st) {
    if (n_sess < 1 || R < 1 || n_seg < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_plan_device, dim3(1), dim3(256), 0, st, pos, slot, segs, n_seg, kv_len, depth,
                       n_sess, R, cap, overflow);
    return hipGetLastError();
}

/* tick start, block s: the root row's input (the previous frame's
 * embedding) and a copy of the session's sampler state for drafting */
__global__ __launch_bounds__(256) void k_spec_begin(const uint16_t* __restrict__ table,
                                                    const uint16_t* __restrict__ cb,
                                                    const int64_t* __restrict__ prev_tok,
                                                    const int32_t* __restrict__ prev_codes,
                                                    uint16_t* __restrict__ x, int R, float scale,
                                                    s2ps_dev_state* const* __restrict__ states,
                                                    s2ps_dev_state* __restrict__ dstates) {
    const int s = blockIdx.x;
    frame_embed(table, cb, prev_tok[s], prev_codes + (size_t)s * 10, x + (size_t)s * R * SPEC_DIM,
                scale);
    const uint32_t* src = (const uint32_t*)states[s];
    uint32_t* dst = (uint32_t*)(dstates + s);
    for (int i = threadIdx.x; i < (int)(sizeof(s2ps_dev_state) / 4); i += 256) dst[i] = src[i];
}

extern "C" hipError_t s2p_spec_begin_launch(const void* table, const void* cb, const int64_t* prev_tok,
                                            const int32_t* prev_codes, void* x, int n_sess, int R,
                                            float scale, s2ps_dev_state* const* states,
                                            s2ps_dev_state* dstates, hipStream_t st) {
    if (n_sess < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_spec_begin, dim3((unsigned)n_sess), dim3(256), 0, st, (const uint16_t*)table,
                       (const uint16_t*)cb, prev_tok, prev_codes, (uint16_t*)x, R, scale, states,
                       dstates);
    return hipGetLastError();
}

/* a drafted frame at depth i, block s: its token (sampled), its nine
 * residual codes (the fast-AR on the draft's hidden, stage [9][n]) into the
 * chain condition's draft codes, and its embedding as verify row s*R + i */
__global__ __launch_bounds__(256) void k_spec_frame(const uint16_t* __restrict__ table,
                                                    const uint16_t* __restrict__ cb,
                                                    const int64_t* __restrict__ tok_d,
                                                    const int32_t* __restrict__ stage, int n_sess,
                                                    int R, int i, int64_t* __restrict__ tok,
                                                    int32_t* __restrict__ draft_codes,
                                                    uint16_t* __restrict__ x, float scale) {
    const int s = blockIdx.x, row = s * R + i;
    const int64_t t = tok_d[s];
    __shared__ int32_t codes[10];
    if (threadIdx.x < 10) {
        const int c = threadIdx.x;
        codes[c] = c == 0 ? sem_code(t) : stage[(size_t)(c - 1) * n_sess + s];
        if (c > 0) draft_codes[(size_t)row * 9 + c - 1] = codes[c];
    }
    if (threadIdx.x == 0) tok[row] = t;
    __syncthreads();
    frame_embed(table, cb, t, codes, x + (size_t)row * SPEC_DIM, scale);
}

extern "C" hipError_t s2p_spec_frame_launch(const void* table, const void* cb, const int64_t* tok_d,
                                            const int32_t* stage, int n_sess, int R, int i,
                                            int64_t* tok, int32_t* draft_codes, void* x, float scale,
                                            hipStream_t st) {
    if (n_sess < 1 || i < 1 || i >= R) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_spec_frame, dim3((unsigned)n_sess), dim3(256), 0, st, (const uint16_t*)table,
                       (const uint16_t*)cb, tok_d, stage, n_sess, R, i, tok, draft_codes,
                       (uint16_t*)x, scale);
    return hipGetLastError();
}

/* after acceptance, block s: the hidden whose frame is still to be decoded
 * (the row that ended the walk) and the semantic code of the last emitted
 * token, for one fast-AR batch over the sessions */
__global__ __launch_bounds__(64) void k_spec_pick(const int32_t* __restrict__ tail,
                                                  const int64_t* __restrict__ emit,
                                                  const int32_t* __restrict__ n_emit,
                                                  const uint16_t* __restrict__ hidden, int R,
                                                  uint16_t* __restrict__ bonus_hidden,
                                                  int32_t* __restrict__ bonus_sem) {
    const int s = blockIdx.x;
    int v = tail[2 * s];
    v = v < 0 ? 0 : (v >= R ? R - 1 : v);
    const int ne = n_emit[s];
    const int64_t t = ne > 0 ? emit[(size_t)s * (R + 1) + ne - 1] : 0;
    const uint16_t* src = hidden + (size_t)(s * R + v) * SPEC_DIM;
    for (int c = threadIdx.x * 8; c < SPEC_DIM; c += 64 * 8)
        *(s2p_u32x4*)(bonus_hidden + (size_t)s * SPEC_DIM + c) = *(const s2p_u32x4*)(src + c);
    if (threadIdx.x == 0) bonus_sem[s] = sem_code(t);
}

extern "C" hipError_t s2p_spec_pick_launch(const int32_t* tail, const int64_t* emit, const int32_t* n_emit,
                                           const void* hidden, int n_sess, int R, void* bonus_hidden,
                                           int32_t* bonus_sem, hipStream_t st) {
    if (n_sess < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_spec_pick, dim3((unsigned)n_sess), dim3(64), 0, st, tail, emit, n_emit,
                       (const uint16_t*)hidden, R, (uint16_t*)bonus_hidden, bonus_sem);
    return hipGetLastError();
}

/* tick end, block s: the emitted frames' codes, the session's next root
 * frame and hidden, and its KV length.  A session whose forward did not
 * complete (n_acc < 0) or that already emitted EOS keeps everything. */
__global__ __launch_bounds__(64) void k_spec_advance(const SpecAdvanceArgs a) {
    const int s = blockIdx.x, R = a.R;
    const int na = a.n_acc[s], ne = a.n_emit[s];
    if (na < 0 || a.done[s]) return;
    const int64_t* em = a.emit + (size_t)s * (R + 1);
    const int v = a.tail[2 * s], c = a.tail[2 * s + 1];
    const int64_t last = ne > 0 ? em[ne - 1] : 0;
    /* frames: accepted nodes carry their chain-checked codes; the last one,
     * when not an accepted node, the failed node's or the bonus decode's */
    for (int j = threadIdx.x; j < ne * 10; j += 64) {
        const int f = j / 10, cbk = j - f * 10;
        const int64_t t = em[f];
        int32_t code;
        if (cbk == 0) {
            code = sem_code(t);
        } else if (f < na) {
            const int node = a.path[(size_t)s * R + f];
            code = a.codes_out[((size_t)s * R + node) * 9 + cbk - 1];
        } else if (c >= 0) {
            code = a.codes_out[((size_t)s * R + c) * 9 + cbk - 1];
        } else {
            code = a.stage[(size_t)(cbk - 1) * a.n_sess + s];
        }
        if (t == SPEC_EOS) code = 0; /* an EOS frame carries no codes */
        a.frames[((size_t)s * (R + 1) + f) * 10 + cbk] = code;
    }
    __syncthreads();
    if (ne > 0) {
        for (int cbk = threadIdx.x; cbk < 10; cbk += 64)
            a.prev_codes[(size_t)s * 10 + cbk] = a.frames[((size_t)s * (R + 1) + ne - 1) * 10 + cbk];
        const uint16_t* src = a.hidden + (size_t)(s * R + (v < 0 ? 0 : v)) * SPEC_DIM;
        for (int k = threadIdx.x * 8; k < SPEC_DIM; k += 64 * 8)
            *(s2p_u32x4*)((uint16_t*)a.prev_hidden + (size_t)s * SPEC_DIM + k) =
                *(const s2p_u32x4*)(src + k);
    }
    if (threadIdx.x == 0) {
        a.kv_len[s] += 1 + na;
        if (ne > 0) a.prev_tok[s] = last;
        if (last == SPEC_EOS) a.done[s] = 1;
    }
}

extern "C" hipError_t s2p_spec_advance_launch(const SpecAdvanceArgs* a, hipStream_t st) {
    if (a->n_sess < 1 || a->R < 2) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_spec_advance, dim3((unsigned)a->n_sess), dim3(64), 0, st, *a);
    return hipGetLastError();
}
