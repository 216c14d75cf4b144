/* s2pro MI355X — draft model: safetensors loader and the one-row forward.
 *
 * Same contract as the reference src/draft/draft.c (loader :73-139, state
 * :149-155, step :157-202), with the step built on this build's fused verify
 * engine instead of the reference's standalone launchers:
 *   - the five GEMVs are the MFMA engine's bf16 path with their neighbours
 *     fused in: RMSNorm in the activation staging (attn / ffn norms, from the
 *     sums of squares the previous epilogue wrote), the residual adds and
 *     the next norm's sums of squares in the epilogues, SiLU(w1 x) * (w3 x)
 *     as one gate+up GEMV over w1 and w3 stored back to back;
 *   - qk-norm, RoPE, the K/V append and the attention over the state's
 *     cache are the verify path's fused plan-mode attention (one launch, the
 *     position splits merged in-kernel), on a one-row plan that a prologue
 *     kernel writes on the stream from the step's position;
 *   - every launch takes its arguments by value and allocates nothing, so
 *     the step can be captured into a graph (the position is an argument:
 *     one graph per position).
 * Launches per step: two copies ([h ; e]), the prologue, five GEMVs, the
 * attention and the final RMSNorm (ten; the reference issues seventeen).
 * The arithmetic is the reference rule's: the same bf16 roundings at the
 * same points (norm, GEMV outputs, residual adds, SwiGLU). */
#include "s2pro/draft.h"

#include <ctype.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "s2pro/gemm.h"
#include "s2pro/kernels.h"
#include "../gemv_internal.h"
#include "../prims_internal.h"

float* s2p_gemm_ctx_part(void);
int64_t s2p_gemm_ctx_part_cap(void);
unsigned* s2p_gemm_ctx_counters(void);

#define D_DIM S2P_DRAFT_DIM
#define D_FFN S2P_DRAFT_FFN
#define D_QH 32
#define D_KVH 8
#define D_HD 128
#define D_EPS 1e-6f
#define D_ROPE_BASE 1000000.0f

#define TRY(x)                                  \
    do {                                        \
        s2p_status rc_ = (x);                   \
        if (rc_ != S2P_OK) return rc_;          \
    } while (0)
#define HIPTRY(x)                                                           \
    do {                                                                    \
        hipError_t e_ = (x);                                                \
        if (e_ != hipSuccess) {                                             \
            fprintf(stderr, "[draft] HIP: %s\n", hipGetErrorString(e_));    \
            return S2P_ERR_CUDA;                                            \
        }                                                                   \
    } while (0)

/* The step's device workspace, held in the model's scratch tensor `a` (a
 * [1, 2560] temporary in the reference sequence, which the fused step does
 * not need): sums of squares [160][GEMV_MAX_M] f32 twice (ping-pong), the
 * one-row attention plan, its RoPE row, the split counters and partials. */
#define WS_SSQ_A 0
#define WS_SSQ_B (WS_SSQ_A + (size_t)(D_DIM / GEMV_SSQ_COLS) * GEMV_MAX_M * 4)
#define WS_PLAN (WS_SSQ_B + (size_t)(D_DIM / GEMV_SSQ_COLS) * GEMV_MAX_M * 4)
#define WS_PL_POS (WS_PLAN + 0)
#define WS_PL_SLOT (WS_PLAN + 4)
#define WS_PL_SESS (WS_PLAN + 8)
#define WS_PL_VIS (WS_PLAN + 16)
#define WS_PL_KV (WS_PLAN + 24)
#define WS_PL_SEG (WS_PLAN + 64)
#define WS_ROPE (WS_PLAN + 256)
#define WS_CTR (WS_ROPE + 64 * 2 * 4)
#define WS_NCTR 64
#define WS_PART (WS_CTR + WS_NCTR * 4)
static size_t ws_bytes(void) {
    return WS_PART + (size_t)s2p_attn_plan_part_floats(1, S2P_DRAFT_CTX) * 4;
}

/* w3 (and the state's vc) are views into the allocation of w1 (kc): the
 * gate+up GEMV reads [w1 ; w3] as one [2F][D] matrix, the fused attention
 * reads K then V planes of one cache */
static int is_view_after(const s2p_tensor* base, const s2p_tensor* v) {
    return base->data && v->data && (const char*)v->data == (const char*)base->data + base->bytes;
}

/* ---- safetensors header ------------------------------------------------ */

static const char* skip_ws(const char* p) {
    while (*p && isspace((unsigned char)*p)) p++;
    return p;
}

/* The entry object of tensor `name` in the header JSON: [*beg, *end). */
static int st_entry(const char* json, const char* name, const char** beg, const char** end) {
    const size_t nl = strlen(name);
    for (const char* p = strchr(json, '"'); p; p = strchr(p + 1, '"')) {
        if (strncmp(p + 1, name, nl) != 0 || p[1 + nl] != '"') continue;
        const char* q = skip_ws(p + 2 + nl);
        if (*q != ':') continue;
        q = skip_ws(q + 1);
        if (*q != '{') return -1;
        const char* e = strchr(q, '}');
        if (!e) return -1;
        *beg = q;
        *end = e;
        return 0;
    }
    return -1;
}

/* integers of the JSON array following key `key` inside [beg, end) */
static int st_ints(const char* beg, const char* end, const char* key, long long* v, int maxn) {
    char k[32];
    snprintf(k, sizeof(k), "\"%s\"", key);
    const char* p = strstr(beg, k);
    if (!p || p >= end) return -1;
    p = skip_ws(p + strlen(k));
    if (*p != ':') return -1;
    p = skip_ws(p + 1);
    if (*p != '[') return -1;
    p++;
    int n = 0;
    for (;;) {
        p = skip_ws(p);
        if (*p == ']') break;
        char* q;
        const long long x = strtoll(p, &q, 10);
        if (q == p || n >= maxn) return -1;
        v[n++] = x;
        p = skip_ws(q);
        if (*p == ',') p++;
        else if (*p != ']') return -1;
    }
    return n;
}

static int st_is_bf16(const char* beg, const char* end) {
    const char* p = strstr(beg, "\"dtype\"");
    if (!p || p >= end) return 0;
    p = skip_ws(p + 7);
    if (*p != ':') return 0;
    p = skip_ws(p + 1);
    return strncmp(p, "\"BF16\"", 6) == 0;
}

static s2p_status load_one(s2p_tensor* t, const char* json, FILE* f, long data0,
                           const char* name, int ndim, const int64_t* shape) {
    const char *beg, *end;
    if (st_entry(json, name, &beg, &end) != 0) {
        fprintf(stderr, "[draft] missing tensor %s\n", name);
        return S2P_ERR_INVALID;
    }
    long long sh[4], off[2];
    const int n = st_ints(beg, end, "shape", sh, 4);
    if (!st_is_bf16(beg, end) || n != ndim || st_ints(beg, end, "data_offsets", off, 2) != 2) {
        fprintf(stderr, "[draft] %s: not a bf16 tensor of rank %d\n", name, ndim);
        return S2P_ERR_INVALID;
    }
    for (int i = 0; i < ndim; i++)
        if (sh[i] != shape[i]) {
            fprintf(stderr, "[draft] %s: dim %d is %lld, want %lld\n", name, i, sh[i],
                    (long long)shape[i]);
            return S2P_ERR_INVALID;
        }
    TRY(s2p_tensor_device_alloc(t, S2P_DT_BF16, ndim, shape));
    if (off[1] - off[0] != (long long)t->bytes || off[0] < 0) {
        fprintf(stderr, "[draft] %s: %lld bytes, want %zu\n", name, off[1] - off[0], t->bytes);
        return S2P_ERR_INVALID;
    }
    void* host = malloc(t->bytes);
    if (!host) return S2P_ERR_OOM;
    s2p_status rc = S2P_OK;
    if (fseek(f, data0 + (long)off[0], SEEK_SET) != 0 || fread(host, 1, t->bytes, f) != t->bytes)
        rc = S2P_ERR_IO;
    else if (hipMemcpy(t->data, host, t->bytes, hipMemcpyHostToDevice) != hipSuccess)
        rc = S2P_ERR_CUDA;
    free(host);
    return rc;
}

s2p_status s2p_draft_load(s2p_draft_model* m, const char* path) {
    if (!m || !path) return S2P_ERR_INVALID;
    memset(m, 0, sizeof(*m));
    FILE* f = fopen(path, "rb");
    if (!f) return S2P_ERR_IO;
    unsigned char hl[8];
    if (fread(hl, 1, 8, f) != 8) {
        fclose(f);
        return S2P_ERR_IO;
    }
    unsigned long long jlen = 0;
    for (int i = 7; i >= 0; i--) jlen = (jlen << 8) | hl[i];
    if (jlen == 0 || jlen > (1ull << 26)) {
        fclose(f);
        return S2P_ERR_FORMAT;
    }
    char* json = (char*)malloc((size_t)jlen + 1);
    if (!json || fread(json, 1, (size_t)jlen, f) != jlen) {
        free(json);
        fclose(f);
        return S2P_ERR_IO;
    }
    json[jlen] = '\0';
    const long data0 = 8 + (long)jlen;

    const int64_t D = D_DIM, F = D_FFN;
    struct {
        s2p_tensor* t;
        const char* n;
        int nd;
        int64_t s[2];
    } spec[] = {
        {&m->fuse, "fuse.weight", 2, {D, 2 * D}}, {&m->wqkv, "wqkv.weight", 2, {6144, D}},
        {&m->wo, "wo.weight", 2, {D, 4096}},     {&m->w1, "w1.weight", 2, {F, D}},
        {&m->w3, "w3.weight", 2, {F, D}},        {&m->w2, "w2.weight", 2, {D, F}},
        {&m->q_norm, "q_norm", 1, {D_HD, 0}},    {&m->k_norm, "k_norm", 1, {D_HD, 0}},
        {&m->attn_norm, "attn_norm", 1, {D, 0}}, {&m->ffn_norm, "ffn_norm", 1, {D, 0}},
        {&m->final_norm, "final_norm", 1, {D, 0}},
    };
    s2p_status rc = S2P_OK;
    for (size_t i = 0; i < sizeof(spec) / sizeof(spec[0]) && rc == S2P_OK; i++)
        rc = load_one(spec[i].t, json, f, data0, spec[i].n, spec[i].nd, spec[i].s);
    free(json);
    fclose(f);
    if (rc == S2P_OK) { /* w1 and w3 back to back: [w1 ; w3] is the gate+up matrix */
        s2p_tensor gu;
        const int64_t sh[2] = {2 * F, D};
        rc = s2p_tensor_device_alloc(&gu, S2P_DT_BF16, 2, sh);
        if (rc == S2P_OK &&
            (hipMemcpy(gu.data, m->w1.data, m->w1.bytes, hipMemcpyDeviceToDevice) != hipSuccess ||
             hipMemcpy((char*)gu.data + m->w1.bytes, m->w3.data, m->w3.bytes,
                       hipMemcpyDeviceToDevice) != hipSuccess)) {
            s2p_tensor_free(&gu);
            rc = S2P_ERR_CUDA;
        }
        if (rc == S2P_OK) {
            const size_t half = m->w1.bytes;
            s2p_tensor_free(&m->w1);
            s2p_tensor_free(&m->w3);
            m->w1 = gu;
            m->w1.shape[0] = F;
            m->w1.bytes = half;
            m->w3 = m->w1;
            m->w3.data = (char*)gu.data + half;
        }
    }
    if (rc == S2P_OK) {
        struct {
            s2p_tensor* t;
            int64_t w;
        } scr[] = {
            {&m->xcat, 2 * D}, {&m->x, D},       {&m->a, (int64_t)(ws_bytes() / 2)},
            {&m->qkv, 6144},   {&m->attn, 4096}, {&m->gu, 2 * F},  {&m->ffn, F},
        };
        for (size_t i = 0; i < sizeof(scr) / sizeof(scr[0]) && rc == S2P_OK; i++) {
            const int64_t sh[2] = {1, scr[i].w};
            rc = s2p_tensor_device_alloc(scr[i].t, S2P_DT_BF16, 2, sh);
        }
    }
    if (rc != S2P_OK) s2p_draft_free(m);
    return rc;
}

void s2p_draft_free(s2p_draft_model* m) {
    if (!m) return;
    if (is_view_after(&m->w1, &m->w3)) memset(&m->w3, 0, sizeof(m->w3)); /* freed with w1 */
    s2p_tensor* ts[] = {&m->fuse,      &m->wqkv,     &m->wo,        &m->w1,   &m->w3,
                        &m->w2,        &m->q_norm,   &m->k_norm,    &m->attn_norm,
                        &m->ffn_norm,  &m->final_norm, &m->xcat,    &m->x,    &m->a,
                        &m->qkv,       &m->attn,     &m->gu,        &m->ffn};
    for (size_t i = 0; i < sizeof(ts) / sizeof(ts[0]); i++) s2p_tensor_free(ts[i]);
}

s2p_status s2p_draft_state_init(s2p_draft_state* s) {
    if (!s) return S2P_ERR_INVALID;
    memset(s, 0, sizeof(*s));
    /* K planes then V planes in one allocation ([16][ctx][128], the verify
     * path's per-layer cache layout); vc views the second half */
    const int64_t sh2[3] = {2 * D_KVH, S2P_DRAFT_CTX, D_HD};
    s2p_status rc = s2p_tensor_device_alloc(&s->kc, S2P_DT_BF16, 3, sh2);
    if (rc != S2P_OK) return rc;
    s->kc.shape[0] = D_KVH;
    s->kc.bytes /= 2;
    s->vc = s->kc;
    s->vc.data = (char*)s->kc.data + s->kc.bytes;
    return S2P_OK;
}

void s2p_draft_state_free(s2p_draft_state* s) {
    if (!s) return;
    if (is_view_after(&s->kc, &s->vc)) memset(&s->vc, 0, sizeof(s->vc)); /* freed with kc */
    s2p_tensor_free(&s->kc);
    s2p_tensor_free(&s->vc);
}

#define BF(t) ((s2p_bf16*)(t).data)

/* one bf16-weight GEMV of the step: y = W · x (x staged plain, or RMSNormed
 * with norm_w from ssq_in), epilogue store / residual add (+ sums of squares
 * into ssq_out) / SwiGLU */
static s2p_status draft_gemv(const s2p_tensor* w, int N, int K, const void* x, void* y, int xmode,
                             const void* norm_w, const float* ssq_in, int epi, float* ssq_out,
                             hipStream_t st) {
    GemvArgs a;
    memset(&a, 0, sizeof(a));
    a.wfmt = GEMV_W_BF16;
    a.w = (const uint8_t*)w->data;
    a.x = (const uint16_t*)x;
    a.ldx = K;
    a.y = (uint16_t*)y;
    a.ldy = epi == GEMV_EPI_SWIGLU ? N / 2 : N;
    a.M = 1;
    a.N = N;
    a.K = K;
    a.xmode = xmode;
    a.norm_w = (const uint16_t*)norm_w;
    a.norm_eps = D_EPS;
    a.ssq_in = ssq_in;
    a.ssq_in_blocks = D_DIM / GEMV_SSQ_COLS;
    a.epi = epi;
    a.ssq_out = ssq_out;
    a.part = s2p_gemm_ctx_part();
    a.part_cap = s2p_gemm_ctx_part_cap();
    a.counters = s2p_gemm_ctx_counters();
    HIPTRY(s2p_gemv_launch(&a, st));
    return S2P_OK;
}

/* The step at a host position (pos_dev == NULL: pos, attention span pos + 1)
 * or at the device position *pos_dev + pos, clamped below span_max, with
 * the attention launched for span_max slots. */
static s2p_status draft_step_at(s2p_draft_model* m, s2p_draft_state* s, const void* h,
                                const void* e, void* out, const int32_t* pos_dev, int pos,
                                int span_max, hipStream_t st) {
    if (!m || !s || !h || !e || !out || !m->fuse.data || !s->kc.data) return S2P_ERR_INVALID;
    if (!is_view_after(&m->w1, &m->w3) || !is_view_after(&s->kc, &s->vc) ||
        m->a.bytes < ws_bytes())
        return S2P_ERR_STATE; /* not made by s2p_draft_load / s2p_draft_state_init */
    if (!s2p_gemm_ctx_part()) return S2P_ERR_STATE; /* s2p_gemm_init not called */
    const int D = D_DIM, F = D_FFN;
    unsigned char* ws = (unsigned char*)m->a.data;
    float* ssq_a = (float*)(ws + WS_SSQ_A);
    float* ssq_b = (float*)(ws + WS_SSQ_B);
    /* the one-row plan: row 0 at slot pos of the state's cache, seeing
     * slots [0, pos] */
    S2pRowPlan plan;
    memset(&plan, 0, sizeof(plan));
    plan.pos = (const int32_t*)(ws + WS_PL_POS);
    plan.slot = (const int32_t*)(ws + WS_PL_SLOT);
    plan.sess = (const int32_t*)(ws + WS_PL_SESS);
    plan.vis = (const uint64_t*)(ws + WS_PL_VIS);
    plan.kv = (void* const*)(ws + WS_PL_KV);
    plan.kvs = NULL;
    plan.layer_stride = (int64_t)2 * D_KVH * S2P_DRAFT_CTX * D_HD;
    plan.max_seq = S2P_DRAFT_CTX;
    S2pAttnSeg* seg = (S2pAttnSeg*)(ws + WS_PL_SEG);
    /* [h ; e] */
    HIPTRY(hipMemcpyAsync(BF(m->xcat), h, (size_t)D * 2, hipMemcpyDeviceToDevice, st));
    HIPTRY(hipMemcpyAsync(BF(m->xcat) + D, e, (size_t)D * 2, hipMemcpyDeviceToDevice, st));
    /* plan, RoPE row, x = 0, counters = 0 */
    HIPTRY(s2p_draft_prologue_launch(&plan, seg, s->kc.data, pos, pos_dev, span_max, D_ROPE_BASE,
                                     (float*)(ws + WS_ROPE), m->x.data, D,
                                     (unsigned*)(ws + WS_CTR), WS_NCTR, st));
    /* x = 0 + fuse · [h ; e], and its sums of squares */
    TRY(draft_gemv(&m->fuse, D, 2 * D, m->xcat.data, m->x.data, GEMV_X_PLAIN, NULL, NULL,
                   GEMV_EPI_RESID, ssq_a, st));
    /* qkv = wqkv · RMSNorm(x; attn_norm) */
    TRY(draft_gemv(&m->wqkv, 6144, D, m->x.data, m->qkv.data, GEMV_X_NORM, m->attn_norm.data,
                   ssq_a, GEMV_EPI_STORE, NULL, st));
    /* qk-norm, RoPE, K/V append at slot pos and attention over [0, pos]
     * (the normed q rows land in xcat, no longer needed) */
    HIPTRY(s2p_attn_plan_fused_launch(m->xcat.data, m->attn.data, &plan, seg, 1, 1, 0, span_max,
                                      (float*)(ws + WS_PART), m->qkv.data, m->q_norm.data,
                                      m->k_norm.data, (const float*)(ws + WS_ROPE), D_EPS,
                                      (unsigned*)(ws + WS_CTR), st));
    /* x += wo · attn */
    TRY(draft_gemv(&m->wo, D, 4096, m->attn.data, m->x.data, GEMV_X_PLAIN, NULL, NULL,
                   GEMV_EPI_RESID, ssq_b, st));
    /* ffn = SiLU(w1 · n) * (w3 · n), n = RMSNorm(x; ffn_norm) */
    TRY(draft_gemv(&m->w1, 2 * F, D, m->x.data, m->ffn.data, GEMV_X_NORM, m->ffn_norm.data, ssq_b,
                   GEMV_EPI_SWIGLU, NULL, st));
    /* x += w2 · ffn */
    TRY(draft_gemv(&m->w2, D, F, m->ffn.data, m->x.data, GEMV_X_PLAIN, NULL, NULL, GEMV_EPI_RESID,
                   NULL, st));
    /* the predicted next final-normed hidden */
    HIPTRY(s2pk_rms_norm(BF(m->x), BF(m->final_norm), (s2p_bf16*)out, 1, D, D_EPS, st));
    return S2P_OK;
}

s2p_status s2p_draft_step(s2p_draft_model* m, s2p_draft_state* s, const void* h, const void* e,
                          void* out, hipStream_t st) {
    if (!s || s->pos < 0 || s->pos >= S2P_DRAFT_CTX) return S2P_ERR_INVALID;
    TRY(draft_step_at(m, s, h, e, out, NULL, s->pos, s->pos + 1, st));
    s->pos++;
    return S2P_OK;
}

/* Internal (the speculative tick): the step at position *pos_dev + pos_add
 * read on the device, attention launched for span_max <= S2P_DRAFT_CTX slots
 * (the position is clamped below it); s->pos is not used or advanced. */
s2p_status s2p_draft_step_dev(s2p_draft_model* m, s2p_draft_state* s, const void* h,
                              const void* e, void* out, const int32_t* pos_dev, int pos_add,
                              int span_max, hipStream_t st) {
    if (!pos_dev || span_max < 1 || span_max > S2P_DRAFT_CTX) return S2P_ERR_INVALID;
    return draft_step_at(m, s, h, e, out, pos_dev, pos_add, span_max, st);
}

/* One GEMV over rows [r0, r0 + n) of a quantised linear, outputs into
 * columns of y with row stride ldy. */
static s2p_status head_rows(const s2p_linear* lin, int r0, int n, const void* x, int M, void* y,
                            int ldy, hipStream_t st) {
    const int K = lin->in_features;
    GemvArgs a;
    memset(&a, 0, sizeof(a));
    if (lin->q_packed) {
        if (lin->q_group != 32) return S2P_ERR_INVALID;
        a.wfmt = GEMV_W_INT4;
        a.w = (const uint8_t*)lin->w_pack.data + (size_t)r0 * (K / 2);
        a.s = (const uint16_t*)lin->w_iscale.data + (size_t)r0 * (K / 32);
    } else {
        if (lin->q_group != 0 || !lin->int8_ready) return S2P_ERR_INVALID;
        a.wfmt = GEMV_W_INT8;
        a.w = (const uint8_t*)lin->w_int8.data + (size_t)r0 * K;
        a.s = (const float*)lin->w_iscale.data + r0;
    }
    a.x = (const uint16_t*)x;
    a.ldx = K;
    a.y = (uint16_t*)y;
    a.ldy = ldy;
    a.M = M;
    a.N = n;
    a.K = K;
    a.xmode = GEMV_X_PLAIN;
    a.epi = GEMV_EPI_STORE;
    a.part = s2p_gemm_ctx_part();
    a.part_cap = s2p_gemm_ctx_part_cap();
    a.counters = s2p_gemm_ctx_counters();
    HIPTRY(s2p_gemv_launch(&a, st));
    return S2P_OK;
}

/* Internal (the speculative tick): q logits of rows hidden rows written into
 * rows of a target-logits layout: ldy elements apart, width W = the head's
 * out_features (the 4,097-row slice, or the full vocabulary with the slice's
 * rows at their vocabulary columns; the other columns are not written). */
s2p_status s2p_draft_head_into(const s2p_linear* head, const void* hidden, int rows, void* y,
                               int64_t ldy, hipStream_t st) {
    if (!head || !hidden || !y || rows < 1 || rows > 16 || head->in_features != D_DIM)
        return S2P_ERR_INVALID;
    if (!s2p_gemm_ctx_part()) return S2P_ERR_STATE;
    uint16_t* o = (uint16_t*)y;
    if (head->out_features == S2P_DRAFT_HEAD_ROWS)
        return head_rows(head, 0, S2P_DRAFT_HEAD_ROWS, hidden, rows, o, (int)ldy, st);
    if (head->out_features < S2P_TOK_SEMANTIC_START + 4096) return S2P_ERR_INVALID;
    TRY(head_rows(head, S2P_TOK_SEMANTIC_START, 4096, hidden, rows, o + S2P_TOK_SEMANTIC_START,
                  (int)ldy, st));
    return head_rows(head, S2P_TOK_EOS, 1, hidden, rows, o + S2P_TOK_EOS, (int)ldy, st);
}

s2p_status s2p_draft_head(const s2p_linear* head, const void* hidden, void* logits, int rows,
                          hipStream_t st) {
    if (!head || !hidden || !logits || rows < 1 || rows > 16 || head->in_features != D_DIM)
        return S2P_ERR_INVALID;
    if (!s2p_gemm_ctx_part()) return S2P_ERR_STATE;
    const int W = S2P_DRAFT_HEAD_ROWS;
    if (head->out_features == W) return head_rows(head, 0, W, hidden, rows, logits, W, st);
    if (head->out_features < S2P_TOK_SEMANTIC_START + 4096 || head->out_features <= S2P_TOK_EOS)
        return S2P_ERR_INVALID;
    TRY(head_rows(head, S2P_TOK_SEMANTIC_START, 4096, hidden, rows, logits, W, st));
    return head_rows(head, S2P_TOK_EOS, 1, hidden, rows, (uint16_t*)logits + 4096, W, st);
}
