/* s2pro MI355X — draft model: safetensors loader and the one-row forward.
 *
 * Same contract as the reference src/draft/draft.c (loader :73-139, state
 * :149-155, step :157-202): the step is the reference's op sequence over
 * this build's launchers, so its numerics are those of the contract
 * kernels, and s2p_gemm_bf16 runs the bf16 path of the MFMA GEMV engine.
 */
#include "s2pro/draft.h"

#include <ctype.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "s2pro/gemm.h"
#include "s2pro/kernels.h"

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
    if (rc == S2P_OK) {
        struct {
            s2p_tensor* t;
            int64_t w;
        } scr[] = {
            {&m->xcat, 2 * D}, {&m->x, D},       {&m->a, D},       {&m->qkv, 6144},
            {&m->attn, 4096},  {&m->gu, 2 * F},  {&m->ffn, F},
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
    s2p_tensor* ts[] = {&m->fuse,      &m->wqkv,     &m->wo,        &m->w1,   &m->w3,
                        &m->w2,        &m->q_norm,   &m->k_norm,    &m->attn_norm,
                        &m->ffn_norm,  &m->final_norm, &m->xcat,    &m->x,    &m->a,
                        &m->qkv,       &m->attn,     &m->gu,        &m->ffn};
    for (size_t i = 0; i < sizeof(ts) / sizeof(ts[0]); i++) s2p_tensor_free(ts[i]);
}

s2p_status s2p_draft_state_init(s2p_draft_state* s) {
    if (!s) return S2P_ERR_INVALID;
    memset(s, 0, sizeof(*s));
    const int64_t sh[3] = {D_KVH, S2P_DRAFT_CTX, D_HD};
    s2p_status rc = s2p_tensor_device_alloc(&s->kc, S2P_DT_BF16, 3, sh);
    if (rc == S2P_OK) rc = s2p_tensor_device_alloc(&s->vc, S2P_DT_BF16, 3, sh);
    if (rc != S2P_OK) s2p_draft_state_free(s);
    return rc;
}

void s2p_draft_state_free(s2p_draft_state* s) {
    if (!s) return;
    s2p_tensor_free(&s->kc);
    s2p_tensor_free(&s->vc);
}

#define BF(t) ((s2p_bf16*)(t).data)

s2p_status s2p_draft_step(s2p_draft_model* m, s2p_draft_state* s, const void* h, const void* e,
                          void* out, hipStream_t st) {
    if (!m || !s || !h || !e || !out || !m->fuse.data || !s->kc.data) return S2P_ERR_INVALID;
    const int D = D_DIM, F = D_FFN;
    if (s->pos >= S2P_DRAFT_CTX) return S2P_ERR_INVALID;
    /* xcat = [h ; e] */
    HIPTRY(hipMemcpyAsync(BF(m->xcat), h, (size_t)D * 2, hipMemcpyDeviceToDevice, st));
    HIPTRY(hipMemcpyAsync(BF(m->xcat) + D, e, (size_t)D * 2, hipMemcpyDeviceToDevice, st));
    /* x = fuse(xcat): the residual stream */
    TRY(s2p_gemm_bf16(BF(m->xcat), BF(m->fuse), BF(m->x), 1, D, 2 * D, st));
    /* attention */
    HIPTRY(s2pk_rms_norm(BF(m->x), BF(m->attn_norm), BF(m->a), 1, D, D_EPS, st));
    TRY(s2p_gemm_bf16(BF(m->a), BF(m->wqkv), BF(m->qkv), 1, 6144, D, st));
    s2p_bf16* q = BF(m->qkv);
    s2p_bf16* k = q + D_QH * D_HD;
    s2p_bf16* v = k + D_KVH * D_HD;
    HIPTRY(s2pk_qk_norm(q, BF(m->q_norm), 1, D_QH, D_HD, D_EPS, st));
    HIPTRY(s2pk_qk_norm(k, BF(m->k_norm), 1, D_KVH, D_HD, D_EPS, st));
    HIPTRY(s2pk_rope(q, k, 1, D_QH, D_KVH, D_HD, s->pos, D_ROPE_BASE, st));
    HIPTRY(s2pk_kv_append(k, v, BF(s->kc), BF(s->vc), 1, D_KVH, D_HD, s->pos, S2P_DRAFT_CTX, st));
    HIPTRY(s2pk_attention(q, BF(s->kc), BF(s->vc), BF(m->attn), 1, D_QH, D_KVH, D_HD, s->pos,
                          S2P_DRAFT_CTX, st));
    TRY(s2p_gemm_bf16(BF(m->attn), BF(m->wo), BF(m->a), 1, D, 4096, st));
    HIPTRY(s2pk_add(BF(m->x), BF(m->a), D, st));
    /* ffn */
    HIPTRY(s2pk_rms_norm(BF(m->x), BF(m->ffn_norm), BF(m->a), 1, D, D_EPS, st));
    TRY(s2p_gemm_bf16(BF(m->a), BF(m->w1), BF(m->gu), 1, F, D, st));
    TRY(s2p_gemm_bf16(BF(m->a), BF(m->w3), BF(m->gu) + F, 1, F, D, st));
    HIPTRY(s2pk_silu_mul(BF(m->gu), BF(m->ffn), 1, F, st));
    TRY(s2p_gemm_bf16(BF(m->ffn), BF(m->w2), BF(m->a), 1, D, F, st));
    HIPTRY(s2pk_add(BF(m->x), BF(m->a), D, st));
    /* predicted next final-normed hidden */
    HIPTRY(s2pk_rms_norm(BF(m->x), BF(m->final_norm), (s2p_bf16*)out, 1, D, D_EPS, st));
    s->pos++;
    return S2P_OK;
}
