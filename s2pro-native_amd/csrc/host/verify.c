/* s2pro MI355X — the speculative verify pass (C11 host side).
 *
 * Per backbone layer the forward issues (reference run_layer,
 * src/slowar/slowar.c:156-260, with its elementwise ops fused):
 *   1. GEMV wqkv    staging = RMSNorm(attn_norm) of the residual stream
 *   2. qk-norm + RoPE + KV append of every row (one launch)
 *   3. attention over each session's cache with the row visibility masks
 *      (+ split combine)
 *   4. GEMV wo      epilogue = residual add, sums of squares for the next norm
 *   5. GEMV gate_up staging = RMSNorm(ffn_norm)
 *   6. GEMV w2      staging = silu(gate) * up, epilogue = residual add
 * then the final RMSNorm is fused into the head GEMV.  The plan (per-row
 * positions, slots, visibility; per-session KV bases; attention segments)
 * lives in device memory, so a captured graph replays for any plan of the
 * same shape.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "s2pro/verify.h"
#include "s2pro/fastar.h"
#include "../gemv_internal.h"
#include "../mk2_internal.h"
#include "../prims_internal.h"
#include "../sample_internal.h"
#include "../spec_internal.h"
#include "../synth_internal.h"

float* s2p_gemm_ctx_part(void);
int64_t s2p_gemm_ctx_part_cap(void);
unsigned* s2p_gemm_ctx_counters(void);

#define NORM_EPS 1e-6f
#define ROPE_BASE 1000000.0f
#define SPAN_BUCKET 512

struct s2p_backbone {
    s2p_backbone_opts o;
    s2p_slow_layer* layers;
    s2p_tensor final_norm;
    s2p_linear head;
    /* activations */
    void* x;      /* [max_rows][2560] residual stream */
    void* qkv;    /* [max_rows][6144] */
    void* q;      /* [max_rows][4096] */
    void* attn;   /* [max_rows][4096] */
    void* gu;     /* [max_rows][9728] SwiGLU output h */
    float* ssq;   /* [2][S2P_DIM / GEMV_SSQ_COLS][GEMV_MAX_M] per-block sums of squares */
    float* attn_part;
    int64_t attn_part_floats;
    /* plan (device + pinned host staging) */
    int32_t* d_pos;
    int32_t* d_slot;
    int32_t* d_sess;
    int32_t* d_depth;      /* [S2P_VERIFY_MAX_ROWS] node depths of the plan's shape */
    uint64_t* d_vis;
    void** d_kv;
    void** d_kvs;          /* [max_sessions] scale bases (INT8 / INT4 caches) */
    S2pAttnSeg* d_segs;
    /* bf16 caches, 8 < R <= 32 rows a session: one segment a session for the
     * tree attention kernel (every segment of <= 8 rows would read the
     * session's K/V again) */
    S2pAttnSeg* d_tsegs;
    int tree;
    void* h_stage;
    size_t stage_bytes;
    int planned, rows, n_sess, R, n_seg, max_span;
    int kvb;               /* KV cache bits: 16 (bf16), 8 or 4 */
    int seg_rows_max;
    float* d_rope;         /* [max_rows][64][2] RoPE table of the plan */
    /* persistent verify kernel (mk2.hip): one launch per forward */
    uint8_t* d_wpack;      /* tile-packed layer weights (packed at the first eligible plan) */
    uint8_t* d_hpack;      /* tile-packed head */
    uint16_t* d_norms;     /* [n_layers][MK2_NORM_STRIDE] norm weights */
    uint32_t* d_mk2;       /* flags, launch state, error flag, attention counters */
    void* d_chain_hidden;  /* [max_rows][2560] bf16: final-normed hidden (chain condition) */
    void* d_chain_par;     /* [max_rows][2560] bf16: the drafted nodes' parent rows */
    int32_t* d_chain_sem;  /* [max_rows] their semantic codes */
    Mk2Args mk2;           /* launch arguments of the current plan */
    int mk2_enabled;       /* off: layer-by-layer launches (env S2P_VERIFY_MK2=0) */
    int mk2_ready;         /* the current plan runs on the persistent kernel */
    unsigned mk2_spin;     /* polls per flag wait (0: MK2_SPIN_LIMIT); tests shorten it */
    /* graph of one verify step */
    hipGraphExec_t gexec;
    int g_rows, g_nseg, g_span, g_valid;
    s2p_verify_step_io g_io;
};

static s2p_status hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fprintf(stderr, "[s2pro] %s: %s\n", what, hipGetErrorString(e));
        return S2P_ERR_CUDA;
    }
    return S2P_OK;
}

static uint64_t seed_of(uint64_t base, int layer, int which) {
    uint64_t z = base ^ (0x9E3779B97F4A7C15ULL * (uint64_t)(layer * 16 + which + 1));
    z = (z ^ (z >> 31)) * 0xBF58476D1CE4E5B9ULL;
    return z ^ (z >> 29);
}

static s2p_status norm_weight(s2p_tensor* t, int n, uint64_t seed, hipStream_t st) {
    int64_t shape[1] = {n};
    S2P_TRY(s2p_tensor_device_alloc(t, S2P_DT_BF16, 1, shape));
    return hip_ok(s2p_synth_bf16_normal(t->data, n, 1.0f, 0.02f, seed, st), "norm init");
}

/* Random weights at rms 1/sqrt(in), the scale of trained projections, so a
 * synthetic stack keeps activations O(1) layer to layer.  The scale sigma is
 * the group / row scale; the code rms is sqrt(56/3) ~ 4.32 for nibbles
 * uniform over -7..7 and ~73.9 for uniform bytes over -127..127. */
static s2p_status rand_linear(s2p_linear* l, s2p_weight_q q, int in, int out, uint64_t seed,
                              hipStream_t st) {
    const float w_rms = 1.0f / sqrtf((float)in);
    if (q == S2P_WQ_INT4_G32)
        return s2p_linear_init_random_int4(l, in, out, 32, w_rms / 4.32f, seed, st);
    return s2p_linear_init_random_int8(l, in, out, w_rms / 73.9f, seed, st);
}

static s2p_status dalloc(void** p, size_t bytes) {
    if (hipMalloc(p, bytes) != hipSuccess) {
        *p = NULL;
        return S2P_ERR_OOM;
    }
    return S2P_OK;
}

s2p_status s2p_backbone_create_random(const s2p_backbone_opts* opts, uint64_t seed,
                                      hipStream_t st, s2p_backbone** out) {
    if (!opts || !out || opts->n_layers <= 0 || opts->max_rows <= 0 ||
        opts->max_rows > GEMV_MAX_M || opts->max_sessions <= 0 || opts->ctx_len <= 0 ||
        opts->head_rows <= 0 ||
        (opts->kv_bits != 0 && opts->kv_bits != 16 && opts->kv_bits != 8 && opts->kv_bits != 4))
        return S2P_ERR_INVALID;
    S2P_TRY(s2p_gemm_init(opts->max_rows));
    s2p_backbone* b = (s2p_backbone*)calloc(1, sizeof(*b));
    if (!b) return S2P_ERR_OOM;
    b->o = *opts;
    b->kvb = opts->kv_bits == 0 ? 16 : opts->kv_bits;
    b->layers = (s2p_slow_layer*)calloc((size_t)opts->n_layers, sizeof(s2p_slow_layer));
    s2p_status rc = b->layers ? S2P_OK : S2P_ERR_OOM;
    for (int l = 0; l < opts->n_layers && rc == S2P_OK; l++) {
        s2p_slow_layer* L = &b->layers[l];
        rc = rand_linear(&L->wqkv, opts->quant, S2P_DIM, S2P_QKV_WIDTH, seed_of(seed, l, 0), st);
        if (rc == S2P_OK)
            rc = rand_linear(&L->wo, opts->quant, S2P_Q_HEADS * S2P_HEAD_DIM, S2P_DIM,
                             seed_of(seed, l, 1), st);
        if (rc == S2P_OK)
            rc = rand_linear(&L->gate_up, opts->quant, S2P_DIM, 2 * S2P_FFN_DIM,
                             seed_of(seed, l, 2), st);
        if (rc == S2P_OK)
            rc = rand_linear(&L->w2, opts->quant, S2P_FFN_DIM, S2P_DIM, seed_of(seed, l, 3), st);
        if (rc == S2P_OK) rc = norm_weight(&L->attn_norm, S2P_DIM, seed_of(seed, l, 4), st);
        if (rc == S2P_OK) rc = norm_weight(&L->ffn_norm, S2P_DIM, seed_of(seed, l, 5), st);
        if (rc == S2P_OK) rc = norm_weight(&L->q_norm, S2P_HEAD_DIM, seed_of(seed, l, 6), st);
        if (rc == S2P_OK) rc = norm_weight(&L->k_norm, S2P_HEAD_DIM, seed_of(seed, l, 7), st);
    }
    if (rc == S2P_OK) rc = norm_weight(&b->final_norm, S2P_DIM, seed_of(seed, 999, 0), st);
    if (rc == S2P_OK)
        rc = rand_linear(&b->head, opts->head_quant, S2P_DIM, opts->head_rows,
                         seed_of(seed, 999, 1), st);
    const size_t R = (size_t)opts->max_rows;
    if (rc == S2P_OK) rc = dalloc(&b->x, R * S2P_DIM * 2);
    if (rc == S2P_OK) rc = dalloc(&b->qkv, R * S2P_QKV_WIDTH * 2);
    if (rc == S2P_OK) rc = dalloc(&b->q, R * S2P_Q_HEADS * S2P_HEAD_DIM * 2);
    if (rc == S2P_OK) rc = dalloc(&b->attn, R * S2P_Q_HEADS * S2P_HEAD_DIM * 2);
    if (rc == S2P_OK) rc = dalloc(&b->gu, R * 2 * S2P_FFN_DIM * 2);
    /* two sums-of-squares buffers, then the two rows' inverse RMS arrays */
    if (rc == S2P_OK)
        rc = dalloc((void**)&b->ssq, sizeof(float) * 2 * ((S2P_DIM / GEMV_SSQ_COLS) * GEMV_MAX_M + GEMV_MAX_M));
    b->attn_part_floats = s2p_attn_plan_part_floats((int)R, opts->ctx_len);
    if (b->kvb != 16) {
        const int64_t p8 = s2p_attn8_plan_part_floats((int)R, opts->ctx_len);
        if (p8 > b->attn_part_floats) b->attn_part_floats = p8;
    }
    if (rc == S2P_OK) rc = dalloc((void**)&b->attn_part, sizeof(float) * b->attn_part_floats);
    const int S = opts->max_sessions;
    const int nseg_max = (int)R + S; /* segments of <= 8 rows per session */
    if (rc == S2P_OK) rc = dalloc((void**)&b->d_pos, R * 4);
    if (rc == S2P_OK) rc = dalloc((void**)&b->d_slot, R * 4);
    if (rc == S2P_OK) rc = dalloc((void**)&b->d_sess, R * 4);
    if (rc == S2P_OK) rc = dalloc((void**)&b->d_depth, S2P_VERIFY_MAX_ROWS * 4);
    if (rc == S2P_OK) rc = dalloc((void**)&b->d_vis, R * 8);
    if (rc == S2P_OK) rc = dalloc((void**)&b->d_kv, (size_t)S * sizeof(void*));
    if (rc == S2P_OK) rc = dalloc((void**)&b->d_kvs, (size_t)S * sizeof(void*));
    if (rc == S2P_OK) rc = dalloc((void**)&b->d_segs, (size_t)nseg_max * sizeof(S2pAttnSeg));
    if (rc == S2P_OK) rc = dalloc((void**)&b->d_tsegs, (size_t)S * sizeof(S2pAttnSeg));
    b->stage_bytes = R * (4 + 4 + 4 + 8) + (size_t)2 * S * sizeof(void*) +
                     (size_t)nseg_max * sizeof(S2pAttnSeg) + 64 + S2P_VERIFY_MAX_ROWS * 4 +
                     (size_t)S * sizeof(S2pAttnSeg) + 64;
    if (rc == S2P_OK) rc = dalloc((void**)&b->d_rope, R * 64 * 2 * sizeof(float));
    if (rc == S2P_OK) rc = dalloc((void**)&b->d_mk2, MK2_AUX_OFF + MK2_AUX_BYTES);
    if (rc == S2P_OK) rc = dalloc(&b->d_chain_hidden, R * S2P_DIM * 2);
    if (rc == S2P_OK) rc = dalloc(&b->d_chain_par, R * S2P_DIM * 2);
    if (rc == S2P_OK) rc = dalloc((void**)&b->d_chain_sem, R * sizeof(int32_t));
    if (rc == S2P_OK) /* flags, epoch and counters start at zero once; the kernel keeps them */
        rc = hip_ok(hipMemsetAsync(b->d_mk2, 0, MK2_STATE_WORDS * sizeof(uint32_t), st), "mk2 init");
    if (rc == S2P_OK) {
        const char* e = getenv("S2P_VERIFY_MK2");
        b->mk2_enabled = !(e && e[0] == '0') && s2p_mk2_supported() == 0;
    }
    if (rc == S2P_OK && hipHostMalloc(&b->h_stage, b->stage_bytes, 0) != hipSuccess) {
        b->h_stage = NULL;
        rc = S2P_ERR_OOM;
    }
    if (rc == S2P_OK) rc = hip_ok(hipStreamSynchronize(st), "backbone init sync");
    if (rc != S2P_OK) {
        s2p_backbone_free(b);
        return rc;
    }
    *out = b;
    return S2P_OK;
}

void s2p_backbone_free(s2p_backbone* b) {
    if (!b) return;
    (void)hipDeviceSynchronize();
    if (b->g_valid) (void)hipGraphExecDestroy(b->gexec);
    if (b->layers) {
        for (int l = 0; l < b->o.n_layers; l++) {
            s2p_slow_layer* L = &b->layers[l];
            s2p_linear_free(&L->wqkv);
            s2p_linear_free(&L->wo);
            s2p_linear_free(&L->gate_up);
            s2p_linear_free(&L->w2);
            s2p_tensor_free(&L->attn_norm);
            s2p_tensor_free(&L->ffn_norm);
            s2p_tensor_free(&L->q_norm);
            s2p_tensor_free(&L->k_norm);
        }
        free(b->layers);
    }
    s2p_tensor_free(&b->final_norm);
    s2p_linear_free(&b->head);
    void* bufs[] = {b->x,        b->qkv,       b->q,           b->attn,          b->gu,
                    b->ssq,      b->attn_part, b->d_pos,       b->d_slot,        b->d_sess,
                    b->d_depth,  b->d_vis,    (void*)b->d_kv, (void*)b->d_kvs, (void*)b->d_segs, (void*)b->d_rope,
                    (void*)b->d_tsegs,
                    (void*)b->d_wpack, (void*)b->d_hpack, (void*)b->d_norms, (void*)b->d_mk2,
                    b->d_chain_hidden, b->d_chain_par, (void*)b->d_chain_sem};
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++)
        if (bufs[i]) (void)hipFree(bufs[i]);
    if (b->h_stage) (void)hipHostFree(b->h_stage);
    free(b);
}

s2p_slow_layer* s2p_backbone_layer(s2p_backbone* b, int layer) {
    if (!b || layer < 0 || layer >= b->o.n_layers) return NULL;
    return &b->layers[layer];
}
s2p_linear* s2p_backbone_head(s2p_backbone* b) { return b ? &b->head : NULL; }
void* s2p_backbone_final_norm(s2p_backbone* b) { return b ? b->final_norm.data : NULL; }

size_t s2p_backbone_kv_bytes(const s2p_backbone* b) {
    if (b->kvb != 16)
        return (size_t)b->o.n_layers * 2 * S2P_KV_HEADS * (size_t)b->o.ctx_len *
               (b->kvb == 8 ? S2P_HEAD_DIM : S2P_HEAD_DIM / 2);
    return (size_t)b->o.n_layers * 2 * S2P_KV_HEADS * (size_t)b->o.ctx_len * S2P_HEAD_DIM * 2;
}

size_t s2p_backbone_kv_scale_bytes(const s2p_backbone* b) {
    if (b->kvb == 16) return 0;
    return (size_t)b->o.n_layers * 2 * S2P_KV_HEADS * (size_t)b->o.ctx_len * 4 * 2;
}

static size_t lin_bytes(const s2p_linear* l) {
    return l->w_pack.bytes + l->w_int8.bytes + l->w_iscale.bytes;
}

size_t s2p_backbone_weight_bytes(const s2p_backbone* b) {
    size_t t = lin_bytes(&b->head);
    for (int l = 0; l < b->o.n_layers; l++) {
        const s2p_slow_layer* L = &b->layers[l];
        t += lin_bytes(&L->wqkv) + lin_bytes(&L->wo) + lin_bytes(&L->gate_up) + lin_bytes(&L->w2);
    }
    return t;
}

/* Activation buffers of the last forward (diagnostics and stage-level parity
 * tests; not part of the public header). */
void s2p_backbone_debug_ptrs(s2p_backbone* b, void** x, void** qkv, void** q, void** attn,
                             void** gu) {
    if (x) *x = b->x;
    if (qkv) *qkv = b->qkv;
    if (q) *q = b->q;
    if (attn) *attn = b->attn;
    if (gu) *gu = b->gu;
}

/* Persistent-kernel controls for tests (not in the public header): enable /
 * disable it for later plans; report whether the current plan runs on it
 * (1), on the layer-by-layer kernels (0), or whether a flag wait of the last
 * launches timed out (-1, synchronises and clears the flag). */
void s2p_backbone_set_mk(s2p_backbone* b, int on) {
    b->mk2_enabled = on && s2p_mk2_supported() == 0;
}

/* Test hook: polls per flag wait of later plans (0 = the default).  A tiny
 * limit makes the waits give up early, which is how the tests reach the
 * timeout path with every kernel still exiting normally. */
void s2p_backbone_set_mk_spin(s2p_backbone* b, unsigned spins) {
    b->mk2_spin = spins;
    if (b->mk2_ready) b->mk2.spin_limit = spins ? spins : MK2_SPIN_LIMIT;
    if (b->g_valid) { /* the captured step holds the old limit in its kernel arguments */
        (void)hipGraphExecDestroy(b->gexec);
        b->g_valid = 0;
    }
}

s2p_status s2p_verify_status(s2p_backbone* b, int32_t* out, int clear, hipStream_t st) {
    if (!b || !out) return S2P_ERR_INVALID;
    if (!b->planned) return S2P_ERR_STATE;
    /* the layer-by-layer forward has no bounded waits: always complete */
    return hip_ok(s2p_word_status_launch(b->mk2_ready ? b->mk2.err : NULL, out, clear, st),
                  "status");
}

int s2p_backbone_mk_status(s2p_backbone* b) {
    if (!b->mk2_ready) return 0;
    int err = 0;
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(&err, b->d_mk2 + MK2_ERR_WORD, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    if (err) {
        (void)hipMemset(b->d_mk2 + MK2_ERR_WORD, 0, sizeof(int));
        return -1;
    }
    return 1;
}

/* ------------------------------------------------------------------ plan */

static int mk2_build(s2p_backbone* b, hipStream_t st);
static S2pRowPlan row_plan(const s2p_backbone* b);

s2p_status s2p_verify_plan(s2p_backbone* b, const s2p_verify_batch* vb, hipStream_t st) {
    if (!b || !vb || vb->n_sess <= 0 || vb->rows <= 0 || vb->rows > S2P_VERIFY_MAX_ROWS ||
        !vb->parent || !vb->kv || !vb->kv_len)
        return S2P_ERR_INVALID;
    const int n = vb->n_sess, R = vb->rows, rows = n * R;
    if (n > b->o.max_sessions || rows > b->o.max_rows) return S2P_ERR_INVALID;
    if (vb->parent[0] != -1) return S2P_ERR_INVALID;
    int depth[S2P_VERIFY_MAX_ROWS];
    uint64_t anc[S2P_VERIFY_MAX_ROWS];
    depth[0] = 0;
    anc[0] = 1ull;
    for (int i = 1; i < R; i++) {
        const int p = vb->parent[i];
        if (p < 0 || p >= i) return S2P_ERR_INVALID;
        depth[i] = depth[p] + 1;
        anc[i] = anc[p] | (1ull << i);
    }
    unsigned char* h = (unsigned char*)b->h_stage;
    int32_t* pos = (int32_t*)h;
    int32_t* slot = pos + rows;
    int32_t* sess = slot + rows;
    uint64_t* vis = (uint64_t*)(((uintptr_t)(sess + rows) + 7) & ~(uintptr_t)7);
    void** kv = (void**)(vis + rows);
    void** kvs = kv + n;
    S2pAttnSeg* segs = (S2pAttnSeg*)(kvs + n);
    if (b->kvb != 16 && !vb->kv_scales) return S2P_ERR_INVALID;
    int nseg = 0, max_span = 0;
    for (int s = 0; s < n; s++) {
        const int L = vb->kv_len[s];
        if (L < 0 || !vb->kv[s]) return S2P_ERR_INVALID;
        if (b->kvb != 16 && !vb->kv_scales[s]) return S2P_ERR_INVALID;
        if (L + R > b->o.ctx_len) return S2P_ERR_FULL;
        kv[s] = vb->kv[s];
        kvs[s] = b->kvb != 16 ? vb->kv_scales[s] : NULL;
        for (int i = 0; i < R; i++) {
            const int r = s * R + i;
            pos[r] = L + depth[i];
            slot[r] = L + i;
            sess[r] = s;
            vis[r] = anc[i];
        }
        for (int r0 = 0; r0 < R; r0 += 8) {
            S2pAttnSeg* g = &segs[nseg++];
            g->sess = s;
            g->L = L;
            g->row0 = s * R + r0;
            g->nrows = R - r0 < 8 ? R - r0 : 8;
            g->span = L + R;
            g->first = s * R;
            g->kv = vb->kv[s];
        }
        if (L + R > max_span) max_span = L + R;
    }
    S2P_TRY(hip_ok(hipMemcpyAsync(b->d_pos, pos, (size_t)rows * 4, hipMemcpyHostToDevice, st), "plan"));
    S2P_TRY(hip_ok(hipMemcpyAsync(b->d_slot, slot, (size_t)rows * 4, hipMemcpyHostToDevice, st), "plan"));
    S2P_TRY(hip_ok(hipMemcpyAsync(b->d_sess, sess, (size_t)rows * 4, hipMemcpyHostToDevice, st), "plan"));
    S2P_TRY(hip_ok(hipMemcpyAsync(b->d_vis, vis, (size_t)rows * 8, hipMemcpyHostToDevice, st), "plan"));
    S2P_TRY(hip_ok(hipMemcpyAsync(b->d_kv, kv, (size_t)n * sizeof(void*), hipMemcpyHostToDevice, st), "plan"));
    S2P_TRY(hip_ok(hipMemcpyAsync(b->d_kvs, kvs, (size_t)n * sizeof(void*), hipMemcpyHostToDevice, st), "plan"));
    S2P_TRY(hip_ok(hipMemcpyAsync(b->d_segs, segs, (size_t)nseg * sizeof(S2pAttnSeg),
                                  hipMemcpyHostToDevice, st), "plan"));
    {
        int32_t* hd = (int32_t*)(segs + nseg);
        memcpy(hd, depth, (size_t)R * sizeof(int32_t));
        S2P_TRY(hip_ok(hipMemcpyAsync(b->d_depth, hd, (size_t)R * 4, hipMemcpyHostToDevice, st),
                       "plan"));
        b->tree = b->kvb == 16 && R > 8 && R <= 32;
        if (b->tree) {
            S2pAttnSeg* ts = (S2pAttnSeg*)(((uintptr_t)(hd + R) + 63) & ~(uintptr_t)63);
            for (int s = 0; s < n; s++) {
                ts[s] = segs[0];
                ts[s].sess = s;
                ts[s].L = vb->kv_len[s];
                ts[s].row0 = s * R;
                ts[s].nrows = R;
                ts[s].span = vb->kv_len[s] + R;
                ts[s].first = s * R;
                ts[s].kv = vb->kv[s];
            }
            S2P_TRY(hip_ok(hipMemcpyAsync(b->d_tsegs, ts, (size_t)n * sizeof(S2pAttnSeg),
                                          hipMemcpyHostToDevice, st), "plan"));
        }
    }
    S2P_TRY(hip_ok(hipStreamSynchronize(st), "plan sync"));
    b->planned = 1;
    b->rows = rows;
    b->n_sess = n;
    b->R = R;
    b->n_seg = nseg;
    /* bucketed so that a graph captured for one span serves nearby spans */
    b->max_span = ((max_span + SPAN_BUCKET - 1) / SPAN_BUCKET) * SPAN_BUCKET;
    if (b->max_span > b->o.ctx_len) b->max_span = b->o.ctx_len;
    {
        /* the RoPE table of the plan's positions, used by every layer */
        const S2pRowPlan rp = row_plan(b);
        S2P_TRY(hip_ok(s2p_rope_tab_launch(&rp, rows, ROPE_BASE, b->d_rope, st), "rope table"));
        S2P_TRY(hip_ok(hipStreamSynchronize(st), "rope table sync"));
    }
    b->mk2_ready = mk2_build(b, st);
    return S2P_OK;
}

static S2pRowPlan row_plan(const s2p_backbone* b) {
    S2pRowPlan p;
    p.pos = b->d_pos;
    p.slot = b->d_slot;
    p.sess = b->d_sess;
    p.vis = b->d_vis;
    p.kv = b->d_kv;
    p.kvs = b->d_kvs;
    p.layer_stride = (int64_t)2 * S2P_KV_HEADS * b->o.ctx_len * S2P_HEAD_DIM;
    p.max_seq = b->o.ctx_len;
    return p;
}

s2p_status s2p_verify_plan_device(s2p_backbone* b, const int32_t* kv_len_dev, int32_t* overflow,
                                  hipStream_t st) {
    if (!b || !kv_len_dev) return S2P_ERR_INVALID;
    if (!b->planned) return S2P_ERR_STATE;
    S2P_TRY(hip_ok(s2p_plan_device_launch(b->d_pos, b->d_slot, b->d_segs, b->n_seg, kv_len_dev,
                                          b->d_depth, b->n_sess, b->R, b->max_span, overflow, st),
                   "device plan"));
    if (b->tree) /* the per-session segments too (positions rewritten alike) */
        S2P_TRY(hip_ok(s2p_plan_device_launch(b->d_pos, b->d_slot, b->d_tsegs, b->n_sess,
                                              kv_len_dev, b->d_depth, b->n_sess, b->R,
                                              b->max_span, overflow, st),
                       "device plan"));
    const S2pRowPlan rp = row_plan(b);
    return hip_ok(s2p_rope_tab_launch(&rp, b->rows, ROPE_BASE, b->d_rope, st), "rope table");
}

/* Internal helpers of the speculative tick (csrc/host/spec.c). */
const void* s2p_backbone_chain_hidden(const s2p_backbone* b) { return b->d_chain_hidden; }
int s2p_backbone_plan_span(const s2p_backbone* b) { return b->planned ? b->max_span : 0; }
int s2p_backbone_ctx_len(const s2p_backbone* b) { return b->o.ctx_len; }

/* --------------------------------------------------------------- forward */

static void gemv_args(GemvArgs* ap, const s2p_linear* lin, int M, const void* x, int ldx, void* y,
                      int ldy, int xmode, const void* norm_w, const float* ssq_in, int epi,
                      float* ssq_out) {
    GemvArgs a;
    memset(&a, 0, sizeof(a));
    a.wfmt = lin->q_packed ? GEMV_W_INT4 : GEMV_W_INT8;
    a.w = (const uint8_t*)(lin->q_packed ? lin->w_pack.data : lin->w_int8.data);
    a.s = lin->w_iscale.data;
    a.x = (const uint16_t*)x;
    a.ldx = ldx;
    a.y = (uint16_t*)y;
    a.ldy = ldy;
    a.M = M;
    a.N = lin->out_features;
    a.K = lin->in_features;
    a.gps = 0;
    a.xmode = xmode;
    a.norm_w = (const uint16_t*)norm_w;
    a.norm_eps = NORM_EPS;
    a.ssq_in = ssq_in;
    a.ssq_in_blocks = S2P_DIM / GEMV_SSQ_COLS;
    a.epi = epi;
    a.ssq_out = ssq_out;
    a.part = s2p_gemm_ctx_part();
    a.part_cap = s2p_gemm_ctx_part_cap();
    a.counters = s2p_gemm_ctx_counters();
    *ap = a;
}

/* inv_out / inv_in: the output rows' inverse RMS written by a residual GEMV
 * for the normed GEMV that reads them next (the row-split INT4 GEMM at
 * 16 < M <= 96 only: elsewhere the consumer computes its own) */
static s2p_status gemv_ex(const s2p_linear* lin, int M, const void* x, int ldx, void* y,
                          int ldy, int xmode, const void* norm_w, const float* ssq_in, int epi,
                          float* ssq_out, const float* inv_in, float* inv_out,
                          S2pQkvParts* parts, hipStream_t st) {
    GemvArgs a;
    gemv_args(&a, lin, M, x, ldx, y, ldy, xmode, norm_w, ssq_in, epi, ssq_out);
    int deferred = 0;
    if (M > 16 && M <= 96) {
        a.inv_in = inv_in;
        a.inv_out = inv_out;
        a.inv_eps = NORM_EPS;
        if (parts) a.deferred = &deferred;
    }
    S2P_TRY(hip_ok(s2p_gemv_launch(&a, st), "verify gemv"));
    if (parts) {
        parts->part = a.part;
        parts->splits = deferred;
        parts->M = M;
        parts->nrb = (a.N + 63) / 64;
    }
    return S2P_OK;
}

static s2p_status gemv(const s2p_linear* lin, int M, const void* x, int ldx, void* y, int ldy,
                       int xmode, const void* norm_w, const float* ssq_in, int epi, float* ssq_out,
                       const float* inv_in, float* inv_out, hipStream_t st) {
    return gemv_ex(lin, M, x, ldx, y, ldy, xmode, norm_w, ssq_in, epi, ssq_out, inv_in, inv_out,
                   NULL, st);
}

/* Pack the weights into the persistent kernel's tile layout (once per
 * backbone): every layer's four GEMVs, the norm weights and the head. */
static s2p_status mk2_pack_all(s2p_backbone* b, hipStream_t st) {
    const int NL = b->o.n_layers;
    const size_t lb = (size_t)MK2_LAYER_BLKS * MK2_BLK;
    const int ht = (b->head.out_features + 15) / 16;
    S2P_TRY(dalloc((void**)&b->d_wpack, lb * NL));
    S2P_TRY(dalloc((void**)&b->d_hpack, (size_t)ht * 20 * MK2_BLK));
    S2P_TRY(dalloc((void**)&b->d_norms, (size_t)NL * MK2_NORM_STRIDE * 2));
    for (int l = 0; l < NL; l++) {
        const s2p_slow_layer* L = &b->layers[l];
        uint8_t* base = b->d_wpack + lb * l;
        const struct {
            const s2p_linear* lin;
            size_t off;
            int pairs;
        } g[4] = {{&L->wqkv, 0, 0},
                  {&L->wo, (size_t)MK2_BLK_Q * MK2_BLK, 0},
                  {&L->gate_up, (size_t)(MK2_BLK_Q + MK2_BLK_O) * MK2_BLK, 1},
                  {&L->w2, (size_t)(MK2_BLK_Q + MK2_BLK_O + MK2_BLK_G) * MK2_BLK, 0}};
        for (int i = 0; i < 4; i++)
            S2P_TRY(hip_ok(s2p_mk2_pack(g[i].lin->w_pack.data, g[i].lin->w_iscale.data,
                                        g[i].lin->out_features, g[i].lin->in_features, g[i].pairs,
                                        base + g[i].off, st),
                           "mk2 pack"));
        uint16_t* nd = b->d_norms + (size_t)l * MK2_NORM_STRIDE;
        S2P_TRY(hip_ok(hipMemcpyAsync(nd + MK2_NORM_ATTN, L->attn_norm.data, S2P_DIM * 2,
                                      hipMemcpyDeviceToDevice, st), "mk2 norms"));
        S2P_TRY(hip_ok(hipMemcpyAsync(nd + MK2_NORM_FFN, L->ffn_norm.data, S2P_DIM * 2,
                                      hipMemcpyDeviceToDevice, st), "mk2 norms"));
        S2P_TRY(hip_ok(hipMemcpyAsync(nd + MK2_NORM_Q, L->q_norm.data, S2P_HEAD_DIM * 2,
                                      hipMemcpyDeviceToDevice, st), "mk2 norms"));
        S2P_TRY(hip_ok(hipMemcpyAsync(nd + MK2_NORM_K, L->k_norm.data, S2P_HEAD_DIM * 2,
                                      hipMemcpyDeviceToDevice, st), "mk2 norms"));
    }
    S2P_TRY(hip_ok(s2p_mk2_pack(b->head.w_pack.data, b->head.w_iscale.data, b->head.out_features,
                                b->head.in_features, 0, b->d_hpack, st),
                   "mk2 pack head"));
    return hip_ok(hipStreamSynchronize(st), "mk2 pack sync");
}

/* Set up the persistent kernel for the current plan; returns 0 if the plan
 * is not served by it (the layer-by-layer path runs instead): more than
 * MK2_MAX_ROWS rows, quantised caches, INT8 weights. */
static int mk2_build(s2p_backbone* b, hipStream_t st) {
    if (!b->mk2_enabled || b->rows > MK2_MAX_ROWS ||
        b->o.quant != S2P_WQ_INT4_G32 || b->o.head_quant != S2P_WQ_INT4_G32 ||
        b->head.out_features > 39 * 16 * MK2_NWG || b->n_seg > 8 ||
        b->o.n_layers > MK2_MAX_LAYERS)
        return 0;
    const int split_pos = 128;
    const int nsplit = (b->max_span + split_pos - 1) / split_pos;
    if ((int64_t)b->rows * 32 * nsplit * (2 + S2P_HEAD_DIM) > b->attn_part_floats ||
        nsplit > MK2_MAX_SPLIT || b->n_seg * 8 * nsplit > MK2_ATT_MAX)
        return 0;
    if (!b->d_wpack && mk2_pack_all(b, st) != S2P_OK) return 0;
    /* a fresh state block per plan: flags, launch epoch, error word */
    if (hipMemsetAsync(b->d_mk2, 0, MK2_STATE_WORDS * sizeof(uint32_t), st) != hipSuccess ||
        hipMemsetAsync((unsigned char*)b->d_mk2 + MK2_AUX_OFF, 0, MK2_AUX_BYTES, st) != hipSuccess)
        return 0;
    Mk2Args* A = &b->mk2;
    memset(A, 0, sizeof(*A));
    A->wpack = b->d_wpack;
    A->hpack = b->d_hpack;
    A->head_tiles = (b->head.out_features + 15) / 16;
    A->head_n = b->head.out_features;
    A->norms = b->d_norms;
    A->final_norm = (const uint16_t*)b->final_norm.data;
    A->n_layers = b->o.n_layers;
    A->rows = b->rows;
    A->x = (uint16_t*)b->x;
    A->qkv = (uint16_t*)b->qkv;
    A->q = (uint16_t*)b->q;
    A->attn = (uint16_t*)b->attn;
    A->h = (uint16_t*)b->gu;
    A->ssq = b->ssq;
    {
        unsigned char* aux = (unsigned char*)b->d_mk2 + MK2_AUX_OFF;
        A->xw = (uint16_t*)(aux + MK2_AUX_XW);
        A->gsx = (float*)(aux + MK2_AUX_GSX);
        A->gsh = (float*)(aux + MK2_AUX_GSH);
        A->gsa = (float*)(aux + MK2_AUX_GSA);
    }
    A->flags = b->d_mk2;
    A->state = b->d_mk2 + MK2_STATE_WORD;
    A->err = (int*)(b->d_mk2 + MK2_ERR_WORD);
    A->spin_limit = b->mk2_spin ? b->mk2_spin : MK2_SPIN_LIMIT;
    A->kvb = b->kvb;
    A->plan = row_plan(b);
    A->segs = b->d_segs;
    A->n_seg = b->n_seg;
    A->nsplit = nsplit;
    A->split_pos = split_pos;
    A->attn_part = b->attn_part;
    A->rope_tab = b->d_rope;
    A->eps = NORM_EPS;
    return 1;
}

s2p_status s2p_verify_forward(s2p_backbone* b, const void* x_in, void* logits, hipStream_t st) {
    if (!b || !x_in || !logits) return S2P_ERR_INVALID;
    if (!b->planned) return S2P_ERR_STATE;
    if (b->mk2_ready) {
        Mk2Args A = b->mk2;
        A.x_in = (const uint16_t*)x_in;
        A.logits = (uint16_t*)logits;
        return hip_ok(s2p_mk2_launch(&A, st), "verify kernel");
    }
    const int M = b->rows;
    const S2pRowPlan plan = row_plan(b);
    float* ssq_a = b->ssq;
    float* ssq_b = b->ssq + (S2P_DIM / GEMV_SSQ_COLS) * GEMV_MAX_M;
    float* inv_a = b->ssq + 2 * (S2P_DIM / GEMV_SSQ_COLS) * GEMV_MAX_M;
    float* inv_b = inv_a + GEMV_MAX_M;
    S2P_TRY(hip_ok(s2p_resid_init_launch(x_in, b->x, ssq_a, M, S2P_DIM, st), "resid init"));
    for (int l = 0; l < b->o.n_layers; l++) {
        const s2p_slow_layer* L = &b->layers[l];
        /* trees over bf16 caches: the qk-norm / RoPE / append kernel merges
         * wqkv's K-split partials itself (one launch fewer; the fused
         * attention prologue of the other plans measured slower reading them:
         * every split's blocks reread the partials) */
        S2pQkvParts qp = {NULL, 0, 0, 0};
        S2P_TRY(gemv_ex(&L->wqkv, M, b->x, S2P_DIM, b->qkv, S2P_QKV_WIDTH, GEMV_X_NORM,
                        L->attn_norm.data, ssq_a, GEMV_EPI_STORE, NULL, l > 0 ? inv_a : NULL,
                        NULL, b->kvb == 16 && b->tree ? &qp : NULL, st));
        if (b->kvb != 16) {
            /* quantised caches: prologue + quantise-on-append, then the
             * split attention and its combine */
            S2P_TRY(hip_ok(s2p_qkrope_append8_launch(b->qkv, b->q, L->q_norm.data,
                                                     L->k_norm.data, &plan, M, l, NORM_EPS,
                                                     b->d_rope, b->kvb, st),
                           "qk-norm / rope / append8"));
            S2P_TRY(hip_ok(s2p_attn8_plan_launch(b->q, b->attn, &plan, b->d_segs, b->n_seg, M, l,
                                                 b->max_span, b->attn_part, b->kvb, st),
                           "attention8"));
        } else if (b->tree) {
            /* trees of 9..32 rows: qk-norm + RoPE + append, then one block
             * per (session, kv head, split) */
            S2P_TRY(hip_ok(s2p_qkrope_append_tab_parts_launch(b->qkv, &qp, b->q, L->q_norm.data,
                                                              L->k_norm.data, &plan, M, l,
                                                              NORM_EPS, b->d_rope, st),
                           "qk-norm / rope / append"));
            S2P_TRY(hip_ok(s2p_attn_tree_launch(b->q, b->attn, &plan, b->d_tsegs, b->n_sess, M, b->R,
                                                l, b->max_span, b->attn_part, b->attn_part_floats, st),
                           "tree attention"));
        } else
        S2P_TRY(hip_ok(s2p_attn_plan_fused_launch(b->q, b->attn, &plan, b->d_segs, b->n_seg, M, l,
                                                  b->max_span, b->attn_part, b->qkv,
                                                  L->q_norm.data, L->k_norm.data, b->d_rope,
                                                  NORM_EPS, NULL, st),
                       "attention"));
        S2P_TRY(gemv(&L->wo, M, b->attn, S2P_Q_HEADS * S2P_HEAD_DIM, b->x, S2P_DIM, GEMV_X_PLAIN,
                     NULL, NULL, GEMV_EPI_RESID, ssq_b, NULL, inv_b, st));
        S2P_TRY(gemv(&L->gate_up, M, b->x, S2P_DIM, b->gu, S2P_FFN_DIM, GEMV_X_NORM,
                     L->ffn_norm.data, ssq_b, GEMV_EPI_SWIGLU, NULL, inv_b, NULL, st));
        S2P_TRY(gemv(&L->w2, M, b->gu, S2P_FFN_DIM, b->x, S2P_DIM, GEMV_X_PLAIN, NULL, NULL,
                     GEMV_EPI_RESID, ssq_a, NULL, inv_a, st));
    }
    return gemv(&b->head, M, b->x, S2P_DIM, logits, b->head.out_features, GEMV_X_NORM,
                b->final_norm.data, ssq_a, GEMV_EPI_STORE, NULL, b->o.n_layers > 0 ? inv_a : NULL,
                NULL, st);
}

/* ------------------------------------------------------------ acceptance */

size_t s2p_verify_accept_work_bytes(int n_sess, int rows) {
    return s2p_accept_work_bytes(n_sess, rows);
}

static s2p_status accept_run(const void* tgt, const void* tgt_eos, int64_t tgt_eos_stride,
                             int64_t tgt_stride, const void* drf, const void* drf_eos,
                             int64_t drf_eos_stride, int64_t drf_stride, const int32_t* parent,
                             const int64_t* tok, s2ps_dev_state* const* states, int n_sess,
                             int rows, int32_t* out_path, int32_t* out_n_acc, int64_t* out_emit,
                             int32_t* out_n_emit, void* work, const uint8_t* chain_ok,
                             const int* fwd_err, int32_t* out_tail, hipStream_t st) {
    if (tgt_stride != drf_stride) return S2P_ERR_INVALID;
    AcceptArgs a;
    memset(&a, 0, sizeof(a));
    a.chain_ok = chain_ok;
    a.fwd_err = fwd_err;
    a.out_tail = out_tail;
    a.tgt = (const uint16_t*)tgt;
    a.tgt_eos = (const uint16_t*)tgt_eos;
    a.drf = (const uint16_t*)drf;
    a.drf_eos = (const uint16_t*)drf_eos;
    a.row_stride = tgt_stride;
    a.tgt_eos_stride = tgt_eos_stride;
    a.drf_eos_stride = drf_eos_stride;
    a.parent = parent;
    a.tok = tok;
    a.states = states;
    a.n_sess = n_sess;
    a.R = rows;
    a.out_path = out_path;
    a.out_n_acc = out_n_acc;
    a.out_emit = out_emit;
    a.out_n_emit = out_n_emit;
    a.work = work;
    return hip_ok(s2p_accept_launch(&a, st), "accept");
}

s2p_status s2p_verify_accept(const void* tgt_logits, const void* tgt_eos, const void* drf_logits,
                             const void* drf_eos, int64_t row_stride, const int32_t* parent,
                             const int64_t* tok, s2ps_dev_state* const* states, int n_sess,
                             int rows, int32_t* out_path, int32_t* out_n_acc, int64_t* out_emit,
                             int32_t* out_n_emit, void* work, hipStream_t st) {
    if (!tgt_logits || !drf_logits || !parent || !tok || !states || !out_path || !out_n_acc ||
        !out_emit || !out_n_emit || !work || n_sess <= 0 || rows <= 0 ||
        rows > S2P_VERIFY_MAX_ROWS || (!tgt_eos) != (!drf_eos))
        return S2P_ERR_INVALID;
    if (!tgt_eos && row_stride < 155774) return S2P_ERR_INVALID;
    if (tgt_eos && row_stride < 4096) return S2P_ERR_INVALID;
    return accept_run(tgt_logits, tgt_eos, 1, row_stride, drf_logits, drf_eos, 1, row_stride,
                      parent, tok, states, n_sess, rows, out_path, out_n_acc, out_emit, out_n_emit,
                      work, NULL, NULL, NULL, st);
}

s2p_status s2p_verify_accept_chain(const void* tgt_logits, const void* tgt_eos,
                                   const void* drf_logits, const void* drf_eos,
                                   int64_t row_stride, const int32_t* parent, const int64_t* tok,
                                   s2ps_dev_state* const* states, int n_sess, int rows,
                                   const uint8_t* chain_ok, int32_t* out_path, int32_t* out_n_acc,
                                   int64_t* out_emit, int32_t* out_n_emit, void* work,
                                   hipStream_t st) {
    if (!tgt_logits || !drf_logits || !parent || !tok || !states || !out_path || !out_n_acc ||
        !out_emit || !out_n_emit || !work || n_sess <= 0 || rows <= 0 ||
        rows > S2P_VERIFY_MAX_ROWS || (!tgt_eos) != (!drf_eos))
        return S2P_ERR_INVALID;
    if (!tgt_eos && row_stride < 155774) return S2P_ERR_INVALID;
    if (tgt_eos && row_stride < 4096) return S2P_ERR_INVALID;
    return accept_run(tgt_logits, tgt_eos, 1, row_stride, drf_logits, drf_eos, 1, row_stride,
                      parent, tok, states, n_sess, rows, out_path, out_n_acc, out_emit, out_n_emit,
                      work, chain_ok, NULL, NULL, st);
}

/* Acceptance of the current plan's rows on the backbone's logits layout,
 * with the chain condition, the forward's error word and the walk's tail
 * (internal: the speculative tick). */
s2p_status s2p_verify_accept_tail(s2p_backbone* b, const void* logits, const void* drf,
                                  const int32_t* parent, const int64_t* tok,
                                  s2ps_dev_state* const* states, const uint8_t* chain_ok,
                                  int32_t* path, int32_t* n_acc, int64_t* emit, int32_t* n_emit,
                                  int32_t* tail, void* work, hipStream_t st) {
    const int sliced = b->head.out_features == S2P_HEAD_SLICE;
    const uint16_t* lg = (const uint16_t*)logits;
    const uint16_t* dg = (const uint16_t*)drf;
    const int64_t ts = b->head.out_features;
    return accept_run(lg, sliced ? lg + 4096 : NULL, ts, ts, dg, sliced ? dg + 4096 : NULL, ts, ts,
                      parent, tok, states, b->n_sess, b->R, path, n_acc, emit, n_emit, work,
                      chain_ok, b->mk2_ready ? b->mk2.err : NULL, tail, st);
}

s2p_status s2p_verify_chain(s2p_backbone* b, s2pfa* fa, const int32_t* parent, const int64_t* tok,
                            const int32_t* draft_codes, uint8_t* chain_ok, int32_t* codes_out,
                            hipStream_t st) {
    if (!b || !fa || !parent || !tok || !draft_codes || !chain_ok || !codes_out) return S2P_ERR_INVALID;
    if (!b->planned) return S2P_ERR_STATE;
    const int n = b->n_sess, R = b->R;
    if (R < 2) return S2P_ERR_INVALID; /* no drafted node */
    const int rows = n * R, B = n * (R - 1);
    S2P_TRY(hip_ok(s2pk_rms_norm((const s2p_bf16*)b->x, (const s2p_bf16*)b->final_norm.data,
                                 (s2p_bf16*)b->d_chain_hidden, rows, S2P_DIM, NORM_EPS, st),
                   "chain final norm"));
    S2P_TRY(hip_ok(s2p_chain_prep_launch(parent, tok, b->d_chain_hidden, b->d_chain_par,
                                         b->d_chain_sem, n, R, S2P_DIM, st),
                   "chain prep"));
    const int32_t* stage = NULL;
    S2P_TRY(s2pfa_decode_frame_batch_dev(fa, b->d_chain_par, b->d_chain_sem, B, &stage, st));
    return hip_ok(s2p_chain_check_launch(stage, draft_codes, tok, chain_ok, codes_out, n, R, st),
                  "chain check");
}

s2p_status s2p_verify_kv_commit(s2p_backbone* b, const int32_t* out_path,
                                const int32_t* out_n_acc, hipStream_t st) {
    if (!b || !out_path || !out_n_acc) return S2P_ERR_INVALID;
    if (!b->planned) return S2P_ERR_STATE;
    const S2pRowPlan plan = row_plan(b);
    if (b->kvb != 16)
        return hip_ok(s2p_kv_commit8_launch(&plan, out_path, out_n_acc, b->n_sess, b->R,
                                            b->o.n_layers, b->kvb, st),
                      "kv commit");
    return hip_ok(s2p_kv_commit_launch(&plan, out_path, out_n_acc, b->n_sess, b->R,
                                       b->o.n_layers, st), "kv commit");
}

/* ------------------------------------------------------------------ step */

static s2p_status step_enqueue(s2p_backbone* b, const s2p_verify_step_io* io, hipStream_t st) {
    S2P_TRY(s2p_verify_forward(b, io->x_in, io->logits, st));
    const int sliced = b->head.out_features == S2P_HEAD_SLICE;
    const uint16_t* lg = (const uint16_t*)io->logits;
    const int64_t ts = b->head.out_features;
    const uint16_t* dg = (const uint16_t*)io->drf_logits;
    return accept_run(lg, sliced ? lg + 4096 : NULL, ts, ts, dg, sliced ? dg + 4096 : NULL, ts,
                      io->drf_stride, io->parent_dev, io->tok_dev,
                      io->states_dev, b->n_sess, b->R, io->out_path, io->out_n_acc,
                      io->out_emit, io->out_n_emit, io->work, NULL,
                      b->mk2_ready ? b->mk2.err : NULL, NULL, st);
}

s2p_status s2p_verify_step(s2p_backbone* b, const s2p_verify_step_io* io, int use_graph,
                           hipStream_t st) {
    if (!b || !io) return S2P_ERR_INVALID;
    if (!b->planned) return S2P_ERR_STATE;
    if (io->drf_stride != b->head.out_features) return S2P_ERR_INVALID;
    if (!use_graph) return step_enqueue(b, io, st);
    const int same = b->g_valid && b->g_rows == b->rows && b->g_nseg == b->n_seg &&
                     b->g_span == b->max_span && memcmp(&b->g_io, io, sizeof(*io)) == 0;
    if (!same) {
        if (b->g_valid) {
            (void)hipGraphExecDestroy(b->gexec);
            b->g_valid = 0;
        }
        hipGraph_t graph;
        S2P_TRY(hip_ok(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "capture"));
        s2p_status rc = step_enqueue(b, io, st);
        hipError_t ce = hipStreamEndCapture(st, &graph);
        if (rc != S2P_OK) return rc;
        S2P_TRY(hip_ok(ce, "end capture"));
        ce = hipGraphInstantiate(&b->gexec, graph, NULL, NULL, 0);
        (void)hipGraphDestroy(graph);
        S2P_TRY(hip_ok(ce, "graph instantiate"));
        b->g_valid = 1;
        b->g_rows = b->rows;
        b->g_nseg = b->n_seg;
        b->g_span = b->max_span;
        b->g_io = *io;
    }
    return hip_ok(hipGraphLaunch(b->gexec, st), "graph launch");
}
