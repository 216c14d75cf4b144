/* s2pro MI355X — the fast-AR residual-codebook decoder (include/s2pro/fastar.h).
 *
 * The reference loop (src/fastar/fastar.cu:726-789) on the verify engine:
 * every row b of a frame batch is a one-row attention segment over its own
 * depth-11 cache (per row [4 layers][16 planes][11][128] bf16, the verify
 * path's cache layout), so RoPE + K/V append + attention of all rows is one
 * plan-mode launch per layer with qk-norm off.  The plans of positions 0..9
 * (row positions, slots, visibility, segments, RoPE rows) are written once at
 * creation.  Per layer: wqkv with the attention RMSNorm in its staging; the
 * attention; wo with the residual add (and the sums of squares of the new
 * residual) in its epilogue; w13 with the FFN RMSNorm in its staging and
 * SwiGLU in its epilogue; w2 with the residual add.  The step input and the
 * prime pass's hidden enter through a gather / copy that also writes the
 * sums of squares.  Launches per frame: 1 + 4 x 5 (prime) and 9 x (1 + 4 x 5
 * + head + argmax). */
#include "s2pro/fastar.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "s2pro/kernels.h"
#include "../gemv_internal.h"
#include "../prims_internal.h"
#include "../synth_internal.h"

float* s2p_gemm_ctx_part(void);
int64_t s2p_gemm_ctx_part_cap(void);
unsigned* s2p_gemm_ctx_counters(void);

#define FA_DIM 2560
#define FA_FFN 9728
#define FA_QKV 6144
#define FA_Q 4096
#define FA_PLANE ((size_t)S2P_FA_SEQ * 128)           /* elements of one cache plane */
#define FA_LSTRIDE ((int64_t)16 * FA_PLANE)           /* elements of one layer of a row */
#define FA_ROWKV ((size_t)S2P_FA_LAYERS * FA_LSTRIDE) /* elements of a row's cache */
#define FA_EPS 1e-6f
#define FA_ROPE_BASE 1000000.0f
#define FA_NPOS 10 /* positions 0 (prime) .. 9 */

struct s2pfa {
    s2pfa_weights w;
    int owns;
    int max_b;
    /* device workspace for max_b rows */
    uint16_t *x, *qkv, *q, *attn, *ffn, *logits;
    float *ssq_a, *ssq_b, *part;
    unsigned* counters;
    int32_t* stage;   /* [9][max_b] */
    int32_t* sem_dev; /* [max_b] (host-pointer entry point) */
    uint16_t* kv;     /* [max_b][FA_ROWKV] */
    /* per position p: the plan arrays, segments and RoPE rows */
    int32_t* d_pos;   /* [FA_NPOS][max_b]: p */
    int32_t* d_slot;  /* [FA_NPOS][max_b]: p */
    int32_t* d_sess;  /* [max_b]: b */
    uint64_t* d_vis;  /* [max_b]: 1 */
    void** d_kv;      /* [max_b]: row b's cache */
    S2pAttnSeg* d_seg; /* [FA_NPOS][max_b] */
    float* d_rope;    /* [FA_NPOS][max_b][64][2] */
    int32_t* codes_dev; /* host-codes VQ entry point, grown on demand */
    int codes_cap;
    int32_t* stage_host;
};

#define HIPCHK(x)                                                                    \
    do {                                                                             \
        hipError_t e_ = (x);                                                         \
        if (e_ != hipSuccess) {                                                      \
            fprintf(stderr, "[s2pro] fastar: %s: %s\n", #x, hipGetErrorString(e_)); \
            return S2P_ERR_CUDA;                                                     \
        }                                                                            \
    } while (0)
#define TRY(x)                            \
    do {                                  \
        s2p_status rc_ = (x);             \
        if (rc_ != S2P_OK) return rc_;    \
    } while (0)

static s2p_status dalloc(void* pp, size_t bytes) {
    void** p = (void**)pp;
    if (hipMalloc(p, bytes ? bytes : 1) != hipSuccess) {
        *p = NULL;
        return S2P_ERR_OOM;
    }
    return S2P_OK;
}

static S2pRowPlan plan_of(const s2pfa* f, int p) {
    S2pRowPlan pl;
    memset(&pl, 0, sizeof(pl));
    pl.pos = f->d_pos + (size_t)p * f->max_b;
    pl.slot = f->d_slot + (size_t)p * f->max_b;
    pl.sess = f->d_sess;
    pl.vis = f->d_vis;
    pl.kv = (void* const*)f->d_kv;
    pl.kvs = NULL;
    pl.layer_stride = FA_LSTRIDE;
    pl.max_seq = S2P_FA_SEQ;
    return pl;
}

/* workspace and the per-position plans (host tables uploaded once) */
static s2p_status build(s2pfa* f, hipStream_t st) {
    const int B = f->max_b, NP = FA_NPOS;
    TRY(dalloc(&f->x, (size_t)B * FA_DIM * 2));
    TRY(dalloc(&f->qkv, (size_t)B * FA_QKV * 2));
    TRY(dalloc(&f->q, (size_t)B * FA_Q * 2));
    TRY(dalloc(&f->attn, (size_t)B * FA_Q * 2));
    TRY(dalloc(&f->ffn, (size_t)B * FA_FFN * 2));
    TRY(dalloc(&f->logits, (size_t)B * S2P_FA_CB * 2));
    TRY(dalloc(&f->ssq_a, (size_t)(FA_DIM / GEMV_SSQ_COLS) * GEMV_MAX_M * 4));
    TRY(dalloc(&f->ssq_b, (size_t)(FA_DIM / GEMV_SSQ_COLS) * GEMV_MAX_M * 4));
    TRY(dalloc(&f->part, (size_t)s2p_attn_plan_part_floats(B, S2P_FA_SEQ) * 4));
    TRY(dalloc(&f->counters, (size_t)B * 8 * 4));
    TRY(dalloc(&f->stage, (size_t)(S2P_FA_NCB - 1) * B * 4));
    TRY(dalloc(&f->sem_dev, (size_t)B * 4));
    TRY(dalloc(&f->kv, (size_t)B * FA_ROWKV * 2));
    TRY(dalloc(&f->d_pos, (size_t)NP * B * 4));
    TRY(dalloc(&f->d_slot, (size_t)NP * B * 4));
    TRY(dalloc(&f->d_sess, (size_t)B * 4));
    TRY(dalloc(&f->d_vis, (size_t)B * 8));
    TRY(dalloc(&f->d_kv, (size_t)B * sizeof(void*)));
    TRY(dalloc(&f->d_seg, (size_t)NP * B * sizeof(S2pAttnSeg)));
    TRY(dalloc(&f->d_rope, (size_t)NP * B * 128 * 4));
    if (hipHostMalloc((void**)&f->stage_host, (size_t)(S2P_FA_NCB - 1) * B * 4, 0) != hipSuccess) {
        f->stage_host = NULL;
        return S2P_ERR_OOM;
    }
    int32_t* pos = (int32_t*)malloc((size_t)NP * B * 4);
    int32_t* sess = (int32_t*)malloc((size_t)B * 4);
    uint64_t* vis = (uint64_t*)malloc((size_t)B * 8);
    void** kv = (void**)malloc((size_t)B * sizeof(void*));
    S2pAttnSeg* seg = (S2pAttnSeg*)malloc((size_t)NP * B * sizeof(S2pAttnSeg));
    s2p_status rc = pos && sess && vis && kv && seg ? S2P_OK : S2P_ERR_OOM;
    if (rc == S2P_OK) {
        for (int b = 0; b < B; b++) {
            sess[b] = b;
            vis[b] = 1ull; /* a row sees its own slot and the prefix before it */
            kv[b] = f->kv + (size_t)b * FA_ROWKV;
        }
        for (int p = 0; p < NP; p++)
            for (int b = 0; b < B; b++) {
                pos[p * B + b] = p;
                S2pAttnSeg* g = &seg[p * B + b];
                g->sess = b;
                g->L = p;
                g->row0 = b;
                g->nrows = 1;
                g->span = p + 1;
                g->first = b;
                g->kv = kv[b];
            }
        if (hipMemcpy(f->d_pos, pos, (size_t)NP * B * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(f->d_slot, pos, (size_t)NP * B * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(f->d_sess, sess, (size_t)B * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(f->d_vis, vis, (size_t)B * 8, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(f->d_kv, kv, (size_t)B * sizeof(void*), hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(f->d_seg, seg, (size_t)NP * B * sizeof(S2pAttnSeg), hipMemcpyHostToDevice) !=
                hipSuccess ||
            hipMemset(f->counters, 0, (size_t)B * 8 * 4) != hipSuccess)
            rc = S2P_ERR_CUDA;
    }
    free(pos);
    free(sess);
    free(vis);
    free(kv);
    free(seg);
    if (rc != S2P_OK) return rc;
    for (int p = 0; p < NP; p++) {
        const S2pRowPlan pl = plan_of(f, p);
        HIPCHK(s2p_rope_tab_launch(&pl, B, FA_ROPE_BASE, f->d_rope + (size_t)p * B * 128, st));
    }
    HIPCHK(hipStreamSynchronize(st));
    return S2P_OK;
}

s2p_status s2pfa_create(s2pfa** out, const s2pfa_weights* w, int max_b, hipStream_t st) {
    if (!out || !w || max_b < 1 || max_b > GEMV_MAX_M) return S2P_ERR_INVALID;
    *out = NULL;
    s2pfa* f = (s2pfa*)calloc(1, sizeof(*f));
    if (!f) return S2P_ERR_OOM;
    f->w = *w;
    f->max_b = max_b;
    s2p_status rc = build(f, st);
    if (rc != S2P_OK) {
        s2pfa_free(f);
        return rc;
    }
    *out = f;
    return S2P_OK;
}

static s2p_status rand_lin(s2p_linear* l, s2p_weight_q q, int in, int out, uint64_t seed,
                           hipStream_t st) {
    const float w_rms = 1.0f / sqrtf((float)in);
    if (q == S2P_WQ_INT4_G32) return s2p_linear_init_random_int4(l, in, out, 32, w_rms / 4.32f, seed, st);
    return s2p_linear_init_random_int8(l, in, out, w_rms / 73.9f, seed, st);
}

static s2p_status rand_bf16(s2p_tensor* t, int64_t rows, int64_t cols, float mean, float sd,
                            uint64_t seed, hipStream_t st) {
    const int64_t sh[2] = {rows, cols};
    TRY(s2p_tensor_device_alloc(t, S2P_DT_BF16, cols ? 2 : 1, sh));
    HIPCHK(s2p_synth_bf16_normal(t->data, rows * (cols ? cols : 1), mean, sd, seed, st));
    return S2P_OK;
}

static void free_weights(s2pfa_weights* w) {
    for (int l = 0; l < S2P_FA_LAYERS; l++) {
        s2pfa_layer* L = &w->layers[l];
        s2p_linear_free(&L->wqkv);
        s2p_linear_free(&L->wo);
        s2p_linear_free(&L->w13);
        s2p_linear_free(&L->w2);
        s2p_tensor_free(&L->attn_norm);
        s2p_tensor_free(&L->ffn_norm);
    }
    s2p_tensor_free(&w->norm);
    s2p_linear_free(&w->output);
    s2p_tensor_free(&w->cb_emb);
    s2p_tensor_free(&w->emb);
}

s2p_status s2pfa_create_random(s2pfa** out, s2p_weight_q quant, int max_b, uint64_t seed,
                               hipStream_t st) {
    if (!out) return S2P_ERR_INVALID;
    *out = NULL;
    s2pfa_weights w;
    memset(&w, 0, sizeof(w));
    s2p_status rc = S2P_OK;
    uint64_t s = seed * 0x9E3779B97F4A7C15ull + 1;
    for (int l = 0; l < S2P_FA_LAYERS && rc == S2P_OK; l++) {
        s2pfa_layer* L = &w.layers[l];
        rc = rand_lin(&L->wqkv, quant, FA_DIM, FA_QKV, ++s, st);
        if (rc == S2P_OK) rc = rand_lin(&L->wo, quant, FA_Q, FA_DIM, ++s, st);
        if (rc == S2P_OK) rc = rand_lin(&L->w13, quant, FA_DIM, 2 * FA_FFN, ++s, st);
        if (rc == S2P_OK) rc = rand_lin(&L->w2, quant, FA_FFN, FA_DIM, ++s, st);
        if (rc == S2P_OK) rc = rand_bf16(&L->attn_norm, FA_DIM, 0, 1.0f, 0.02f, ++s, st);
        if (rc == S2P_OK) rc = rand_bf16(&L->ffn_norm, FA_DIM, 0, 1.0f, 0.02f, ++s, st);
    }
    if (rc == S2P_OK) rc = rand_bf16(&w.norm, FA_DIM, 0, 1.0f, 0.02f, ++s, st);
    if (rc == S2P_OK) rc = rand_lin(&w.output, quant, FA_DIM, S2P_FA_CB, ++s, st);
    if (rc == S2P_OK) rc = rand_bf16(&w.cb_emb, (int64_t)S2P_FA_NCB * S2P_FA_CB, FA_DIM, 0.0f, 1.0f, ++s, st);
    if (rc == S2P_OK) rc = rand_bf16(&w.emb, S2P_FA_CB, FA_DIM, 0.0f, 1.0f, ++s, st);
    if (rc == S2P_OK) rc = s2pfa_create(out, &w, max_b, st);
    if (rc != S2P_OK) {
        free_weights(&w);
        return rc;
    }
    (*out)->owns = 1;
    return S2P_OK;
}

void s2pfa_free(s2pfa* f) {
    if (!f) return;
    void* ps[] = {f->x,     f->qkv,    f->q,     f->attn,   f->ffn,  f->logits,
                  f->ssq_a, f->ssq_b,  f->part,  f->counters, f->stage, f->sem_dev,
                  f->kv,    f->d_pos,  f->d_slot, f->d_sess, f->d_vis, f->d_kv,
                  f->d_seg, f->d_rope, f->codes_dev};
    for (size_t i = 0; i < sizeof(ps) / sizeof(ps[0]); i++)
        if (ps[i]) (void)hipFree(ps[i]);
    if (f->stage_host) (void)hipHostFree(f->stage_host);
    if (f->owns) free_weights(&f->w);
    free(f);
}

const s2pfa_weights* s2pfa_weights_of(const s2pfa* f) { return f ? &f->w : NULL; }

static s2p_status gemv(const s2p_linear* lin, int M, const void* x, void* y, int ldy, int xmode,
                       const void* norm_w, const float* ssq_in, int epi, float* ssq_out,
                       hipStream_t st) {
    GemvArgs a;
    memset(&a, 0, sizeof(a));
    if (lin->q_packed) {
        a.wfmt = GEMV_W_INT4;
        a.w = (const uint8_t*)lin->w_pack.data;
    } else {
        a.wfmt = GEMV_W_INT8;
        a.w = (const uint8_t*)lin->w_int8.data;
    }
    a.s = lin->w_iscale.data;
    a.x = (const uint16_t*)x;
    a.ldx = lin->in_features;
    a.y = (uint16_t*)y;
    a.ldy = ldy;
    a.M = M;
    a.N = lin->out_features;
    a.K = lin->in_features;
    a.xmode = xmode;
    a.norm_w = (const uint16_t*)norm_w;
    a.norm_eps = FA_EPS;
    a.ssq_in = ssq_in;
    a.ssq_in_blocks = FA_DIM / GEMV_SSQ_COLS;
    a.epi = epi;
    a.ssq_out = ssq_out;
    a.part = s2p_gemm_ctx_part();
    a.part_cap = s2p_gemm_ctx_part_cap();
    a.counters = s2p_gemm_ctx_counters();
    HIPCHK(s2p_gemv_launch(&a, st));
    return S2P_OK;
}

/* the 4 layers on x (sums of squares in ssq_a) at position p, K/V at slot p */
static s2p_status run_layers(s2pfa* f, int B, int p, hipStream_t st) {
    const S2pRowPlan pl = plan_of(f, p);
    const S2pAttnSeg* seg = f->d_seg + (size_t)p * f->max_b;
    const float* rope = f->d_rope + (size_t)p * f->max_b * 128;
    for (int l = 0; l < S2P_FA_LAYERS; l++) {
        const s2pfa_layer* L = &f->w.layers[l];
        TRY(gemv(&L->wqkv, B, f->x, f->qkv, FA_QKV, GEMV_X_NORM, L->attn_norm.data, f->ssq_a,
                 GEMV_EPI_STORE, NULL, st));
        HIPCHK(s2p_attn_plan_fused_launch(f->q, f->attn, &pl, seg, B, B, l, p + 1, f->part, f->qkv,
                                          NULL, NULL, rope, FA_EPS, f->counters, st));
        TRY(gemv(&L->wo, B, f->attn, f->x, FA_DIM, GEMV_X_PLAIN, NULL, NULL, GEMV_EPI_RESID,
                 f->ssq_b, st));
        TRY(gemv(&L->w13, B, f->x, f->ffn, FA_FFN, GEMV_X_NORM, L->ffn_norm.data, f->ssq_b,
                 GEMV_EPI_SWIGLU, NULL, st));
        TRY(gemv(&L->w2, B, f->ffn, f->x, FA_DIM, GEMV_X_PLAIN, NULL, NULL, GEMV_EPI_RESID,
                 f->ssq_a, st));
    }
    return S2P_OK;
}

static s2p_status frame(s2pfa* f, const void* hidden, const int32_t* sem_dev, int B,
                        uint16_t* logits_all, hipStream_t st) {
    /* prime: K/V at position 0 from the final-normed hidden; its logits are
     * never read (the reference computes and discards them) */
    HIPCHK(s2p_resid_init_launch(hidden, f->x, f->ssq_a, B, FA_DIM, st));
    TRY(run_layers(f, B, 0, st));
    for (int cb = 1; cb < S2P_FA_NCB; cb++) {
        const int32_t* ids = cb == 1 ? sem_dev : f->stage + (size_t)(cb - 2) * B;
        HIPCHK(s2p_fa_embed_ssq_launch(f->w.emb.data, ids, S2P_FA_CB, f->x, f->ssq_a, B, FA_DIM, st));
        TRY(run_layers(f, B, cb, st));
        uint16_t* lg = logits_all ? logits_all + (size_t)(cb - 1) * B * S2P_FA_CB : f->logits;
        TRY(gemv(&f->w.output, B, f->x, lg, S2P_FA_CB, GEMV_X_NORM, f->w.norm.data, f->ssq_a,
                 GEMV_EPI_STORE, NULL, st));
        HIPCHK(s2pk_argmax((const s2p_bf16*)lg, f->stage + (size_t)(cb - 1) * B, B, S2P_FA_CB, st));
    }
    return S2P_OK;
}

static int ready(const s2pfa* f, int B) {
    return f && B >= 1 && B <= f->max_b && s2p_gemm_ctx_part() != NULL;
}

s2p_status s2pfa_decode_frame_logits_dev(s2pfa* f, const void* hidden, const int32_t* sem_dev,
                                         int B, const int32_t** stage_dev, void* logits,
                                         hipStream_t st) {
    if (!f || !hidden || !sem_dev || !stage_dev) return S2P_ERR_INVALID;
    if (!ready(f, B)) return B >= 1 && f && B <= f->max_b ? S2P_ERR_STATE : S2P_ERR_INVALID;
    *stage_dev = f->stage;
    return frame(f, hidden, sem_dev, B, (uint16_t*)logits, st);
}

s2p_status s2pfa_decode_frame_batch_dev(s2pfa* f, const void* hidden, const int32_t* sem_dev,
                                        int B, const int32_t** stage_dev, hipStream_t st) {
    return s2pfa_decode_frame_logits_dev(f, hidden, sem_dev, B, stage_dev, NULL, st);
}

s2p_status s2pfa_decode_frame_batch(s2pfa* f, const void* hidden, const int32_t* sem_ids, int B,
                                    int32_t* out_codes, hipStream_t st) {
    if (!f || !hidden || !sem_ids || !out_codes) return S2P_ERR_INVALID;
    if (!ready(f, B)) return B >= 1 && B <= f->max_b ? S2P_ERR_STATE : S2P_ERR_INVALID;
    HIPCHK(hipMemcpyAsync(f->sem_dev, sem_ids, (size_t)B * 4, hipMemcpyHostToDevice, st));
    const int32_t* stage = NULL;
    TRY(frame(f, hidden, f->sem_dev, B, NULL, st));
    stage = f->stage;
    HIPCHK(hipMemcpyAsync(f->stage_host, stage, (size_t)(S2P_FA_NCB - 1) * B * 4,
                          hipMemcpyDeviceToHost, st));
    HIPCHK(hipStreamSynchronize(st));
    for (int b = 0; b < B; b++)
        for (int cb = 1; cb < S2P_FA_NCB; cb++)
            out_codes[(size_t)b * S2P_FA_NCB + cb] = f->stage_host[(size_t)(cb - 1) * B + b];
    return S2P_OK;
}

s2p_status s2pfa_vq_embed_add_dev(s2pfa* f, const int32_t* codes_dev, int T, void* rows,
                                  hipStream_t st) {
    if (!f || !codes_dev || !rows || T < 0) return S2P_ERR_INVALID;
    HIPCHK(s2p_fa_vq_embed_add_launch(f->w.cb_emb.data, codes_dev, T, rows, FA_DIM, st));
    return S2P_OK;
}

s2p_status s2pfa_vq_embed_add(s2pfa* f, const int32_t* codes, int T, void* rows, hipStream_t st) {
    if (!f || !codes || !rows || T < 0) return S2P_ERR_INVALID;
    if (T == 0) return S2P_OK;
    if (T > f->codes_cap) {
        if (f->codes_dev) (void)hipFree(f->codes_dev);
        f->codes_dev = NULL;
        f->codes_cap = 0;
        TRY(dalloc(&f->codes_dev, (size_t)S2P_FA_NCB * T * 4));
        f->codes_cap = T;
    }
    HIPCHK(hipMemcpyAsync(f->codes_dev, codes, (size_t)S2P_FA_NCB * T * 4, hipMemcpyHostToDevice, st));
    return s2pfa_vq_embed_add_dev(f, f->codes_dev, T, rows, st);
}
