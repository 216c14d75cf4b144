/* s2pro MI355X — the composed speculative tick (include/s2pro/spec.h).
 *
 * The tick is one fixed launch sequence over buffers owned here and the
 * caller's device state, so it is captured once into a hipGraph and
 * replayed; everything that changes from tick to tick (KV lengths, the
 * previous frame, sampler states) lives in device memory and is read by the
 * kernels themselves (csrc/spec.hip), never by the host. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "s2pro/spec.h"
#include "../spec_internal.h"

/* internal entry points of verify.c and draft.c */
s2p_status s2p_verify_accept_tail(s2p_backbone* b, const void* logits, const void* drf,
                                  const int32_t* parent, const int64_t* tok,
                                  s2ps_dev_state* const* states, const uint8_t* chain_ok,
                                  int32_t* path, int32_t* n_acc, int64_t* emit, int32_t* n_emit,
                                  int32_t* tail, void* work, hipStream_t st);
const void* s2p_backbone_chain_hidden(const s2p_backbone* b);
int s2p_backbone_plan_span(const s2p_backbone* b);
int s2p_backbone_ctx_len(const s2p_backbone* b);
s2p_status s2p_draft_step_dev(s2p_draft_model* m, s2p_draft_state* s, const void* h,
                              const void* e, void* out, const int32_t* pos_dev, int pos_add,
                              int span_max, hipStream_t st);
s2p_status s2p_draft_head_into(const s2p_linear* head, const void* hidden, int rows, void* y,
                               int64_t ldy, hipStream_t st);

#define DIM 2560
#define SQRT11 3.3166247903554

struct s2p_spec {
    s2p_spec_model m;
    s2p_spec_sessions ss;
    s2p_spec_out o;
    void* kv_host[S2P_SPEC_MAX_SESSIONS];
    int n, K, R, rows, W;
    int bound[S2P_SPEC_MAX_SESSIONS]; /* upper bound of each kv_len at the next tick */
    int span;                         /* the current plan's span */
    int replans;
    /* device buffers of the tick */
    uint16_t *logits, *drf, *x, *hid[2], *bonus_hidden;
    int64_t *tok, *tok_d;
    int32_t *draft_codes, *codes_out, *path, *tail, *sem_d, *codes_d, *bonus_sem, *overflow,
        *parent;
    uint8_t *chain_ok, *eos_d;
    void* work;
    s2ps_dev_state* dstates;
    s2ps_dev_state** dstate_ptrs;
    /* graph */
    hipGraphExec_t gexec;
    int g_valid;
};

static s2p_status hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fprintf(stderr, "[s2pro] spec tick: %s: %s\n", what, hipGetErrorString(e));
        return S2P_ERR_CUDA;
    }
    return S2P_OK;
}

static s2p_status dev(void* p, size_t bytes) {
    void** pp = (void**)p;
    if (hipMalloc(pp, bytes ? bytes : 1) != hipSuccess) {
        *pp = NULL;
        return S2P_ERR_OOM;
    }
    return S2P_OK;
}

/* host re-plan from the current device lengths (synchronises st) */
static s2p_status replan(s2p_spec* sp, const int32_t* kv_len_host, hipStream_t st) {
    int32_t lens[S2P_SPEC_MAX_SESSIONS];
    if (kv_len_host) {
        memcpy(lens, kv_len_host, sizeof(int32_t) * (size_t)sp->n);
    } else {
        S2P_TRY(hip_ok(hipStreamSynchronize(st), "sync"));
        S2P_TRY(hip_ok(hipMemcpy(lens, sp->ss.kv_len, sizeof(int32_t) * (size_t)sp->n,
                                 hipMemcpyDeviceToHost), "kv_len readback"));
    }
    int32_t parent[S2P_VERIFY_MAX_ROWS];
    for (int i = 0; i < sp->R; i++) parent[i] = i - 1;
    for (int s = 0; s < sp->n; s++) {
        /* the draft's cache holds S2P_DRAFT_CTX frames */
        if (lens[s] < 0 || lens[s] + sp->R > S2P_DRAFT_CTX) return S2P_ERR_FULL;
    }
    const s2p_verify_batch vb = {sp->n, sp->R, parent, sp->kv_host, lens, NULL};
    S2P_TRY(s2p_verify_plan(sp->m.bb, &vb, st));
    sp->span = s2p_backbone_plan_span(sp->m.bb);
    if (sp->span > S2P_DRAFT_CTX) sp->span = S2P_DRAFT_CTX;
    for (int s = 0; s < sp->n; s++) sp->bound[s] = lens[s];
    if (sp->g_valid) {
        (void)hipGraphExecDestroy(sp->gexec);
        sp->g_valid = 0;
    }
    sp->replans++;
    return S2P_OK;
}

s2p_status s2p_spec_create(s2p_spec** out, const s2p_spec_model* m, const s2p_spec_sessions* ss,
                           const int32_t* kv_len_host, const s2p_spec_out* o, hipStream_t st) {
    if (!out || !m || !ss || !kv_len_host || !o) return S2P_ERR_INVALID;
    *out = NULL;
    if (!m->bb || !m->draft || !m->draft_states || !m->fa || !m->embed || m->n_sess < 1 ||
        m->n_sess > S2P_SPEC_MAX_SESSIONS || m->K < 1 || m->K + 1 > S2P_VERIFY_MAX_ROWS)
        return S2P_ERR_INVALID;
    if (!ss->kv || !ss->kv_len || !ss->prev_tok || !ss->prev_codes || !ss->prev_hidden ||
        !ss->states || !ss->done || !o->n_acc || !o->n_emit || !o->emit || !o->frames)
        return S2P_ERR_INVALID;
    if (s2p_backbone_kv_scale_bytes(m->bb) != 0) return S2P_ERR_INVALID; /* bf16 caches only */
    const s2pfa_weights* fw = s2pfa_weights_of(m->fa);
    if (!fw || !fw->cb_emb.data) return S2P_ERR_INVALID;
    s2p_spec* sp = (s2p_spec*)calloc(1, sizeof(*sp));
    if (!sp) return S2P_ERR_OOM;
    sp->m = *m;
    sp->ss = *ss;
    sp->o = *o;
    sp->n = m->n_sess;
    sp->K = m->K;
    sp->R = m->K + 1;
    sp->rows = sp->n * sp->R;
    sp->W = s2p_backbone_head(m->bb)->out_features;
    for (int s = 0; s < sp->n; s++) sp->kv_host[s] = ss->kv[s];
    const size_t rows = (size_t)sp->rows, n = (size_t)sp->n, W = (size_t)sp->W;
    s2p_status rc = S2P_OK;
    if (rc == S2P_OK) rc = dev(&sp->logits, rows * W * 2);
    if (rc == S2P_OK) rc = dev(&sp->drf, rows * W * 2);
    if (rc == S2P_OK) rc = dev(&sp->x, rows * DIM * 2);
    if (rc == S2P_OK) rc = dev(&sp->hid[0], n * DIM * 2);
    if (rc == S2P_OK) rc = dev(&sp->hid[1], n * DIM * 2);
    if (rc == S2P_OK) rc = dev(&sp->bonus_hidden, n * DIM * 2);
    if (rc == S2P_OK) rc = dev(&sp->tok, rows * 8);
    if (rc == S2P_OK) rc = dev(&sp->tok_d, n * 8);
    if (rc == S2P_OK) rc = dev(&sp->draft_codes, rows * 9 * 4);
    if (rc == S2P_OK) rc = dev(&sp->codes_out, rows * 9 * 4);
    if (rc == S2P_OK) rc = dev(&sp->path, rows * 4);
    if (rc == S2P_OK) rc = dev(&sp->tail, n * 2 * 4);
    if (rc == S2P_OK) rc = dev(&sp->sem_d, n * 4);
    if (rc == S2P_OK) rc = dev(&sp->codes_d, n * 10 * 4);
    if (rc == S2P_OK) rc = dev(&sp->bonus_sem, n * 4);
    if (rc == S2P_OK) rc = dev(&sp->overflow, 4);
    if (rc == S2P_OK) rc = dev(&sp->parent, (size_t)sp->R * 4);
    if (rc == S2P_OK) rc = dev(&sp->chain_ok, rows);
    if (rc == S2P_OK) rc = dev(&sp->eos_d, n);
    if (rc == S2P_OK) rc = dev(&sp->work, s2p_verify_accept_work_bytes(sp->n, sp->R));
    if (rc == S2P_OK) rc = dev(&sp->dstates, n * sizeof(s2ps_dev_state));
    if (rc == S2P_OK) rc = dev(&sp->dstate_ptrs, n * sizeof(void*));
    if (rc == S2P_OK) {
        int32_t parent[S2P_VERIFY_MAX_ROWS];
        s2ps_dev_state* ptrs[S2P_SPEC_MAX_SESSIONS];
        for (int i = 0; i < sp->R; i++) parent[i] = i - 1;
        for (int s = 0; s < sp->n; s++) ptrs[s] = sp->dstates + s;
        rc = hip_ok(hipMemcpyAsync(sp->parent, parent, (size_t)sp->R * 4, hipMemcpyHostToDevice, st),
                    "upload");
        if (rc == S2P_OK)
            rc = hip_ok(hipMemcpyAsync(sp->dstate_ptrs, ptrs, n * sizeof(void*),
                                       hipMemcpyHostToDevice, st), "upload");
        if (rc == S2P_OK)
            rc = hip_ok(hipMemsetAsync(sp->overflow, 0, 4, st), "clear");
        /* tokens and draft logits rows no tick writes (the roots', the
         * leaves') read as zeros */
        if (rc == S2P_OK) rc = hip_ok(hipMemsetAsync(sp->tok, 0, rows * 8, st), "clear");
        if (rc == S2P_OK) rc = hip_ok(hipMemsetAsync(sp->draft_codes, 0, rows * 9 * 4, st), "clear");
        if (rc == S2P_OK) rc = hip_ok(hipMemsetAsync(sp->path, 0, rows * 4, st), "clear");
        if (rc == S2P_OK) rc = hip_ok(hipMemsetAsync(sp->drf, 0, rows * W * 2, st), "clear");
        if (rc == S2P_OK) rc = hip_ok(hipStreamSynchronize(st), "create sync");
    }
    if (rc == S2P_OK) rc = replan(sp, kv_len_host, st);
    if (rc != S2P_OK) {
        s2p_spec_free(sp);
        return rc;
    }
    sp->replans = 0;
    *out = sp;
    return S2P_OK;
}

static s2p_status tick_enqueue(s2p_spec* sp, hipStream_t st) {
    const s2p_spec_model* m = &sp->m;
    const s2p_spec_sessions* ss = &sp->ss;
    const int n = sp->n, R = sp->R, W = sp->W;
    const float scale = (float)(1.0 / SQRT11);
    const void* cb = s2pfa_weights_of(m->fa)->cb_emb.data;
    const s2p_linear* head = s2p_backbone_head(m->bb);
    /* 1-2: plan from the device lengths; the roots' inputs; draft states */
    S2P_TRY(s2p_verify_plan_device(m->bb, ss->kv_len, sp->overflow, st));
    S2P_TRY(hip_ok(s2p_spec_begin_launch(m->embed, cb, ss->prev_tok, ss->prev_codes, sp->x, n, R,
                                         scale, ss->states, sp->dstates, st), "begin"));
    /* 3: K draft steps */
    for (int i = 1; i < R; i++) {
        uint16_t* hout = sp->hid[i & 1];
        for (int s = 0; s < n; s++) {
            const void* h_in = i == 1 ? (const uint16_t*)ss->prev_hidden + (size_t)s * DIM
                                      : sp->hid[(i - 1) & 1] + (size_t)s * DIM;
            S2P_TRY(s2p_draft_step_dev(m->draft, &m->draft_states[s], h_in,
                                       sp->x + (size_t)(s * R + i - 1) * DIM, hout + (size_t)s * DIM,
                                       ss->kv_len + s, i - 1, sp->span, st));
        }
        S2P_TRY(s2p_draft_head_into(head, hout, n, sp->drf + (size_t)(i - 1) * W, (int64_t)R * W, st));
        for (int s = 0; s < n; s++) {
            const uint16_t* row = sp->drf + (size_t)(s * R + i - 1) * W;
            const int sliced = W == S2P_HEAD_SLICE;
            S2P_TRY(hip_ok(s2pk_sample((const s2p_bf16*)row, W,
                                       sliced ? (const s2p_bf16*)(row + 4096) : NULL,
                                       sp->dstate_ptrs + s, 1, sp->tok_d + s, sp->sem_d + s,
                                       sp->codes_d + (size_t)s * 10, sp->eos_d + s, st),
                           "draft sample"));
        }
        const int32_t* stage = NULL;
        S2P_TRY(s2pfa_decode_frame_batch_dev(m->fa, hout, sp->sem_d, n, &stage, st));
        S2P_TRY(hip_ok(s2p_spec_frame_launch(m->embed, cb, sp->tok_d, stage, n, R, i, sp->tok,
                                             sp->draft_codes, sp->x, scale, st), "frame"));
    }
    /* 4-5: verify, chain condition, acceptance */
    S2P_TRY(s2p_verify_forward(m->bb, sp->x, sp->logits, st));
    S2P_TRY(s2p_verify_chain(m->bb, m->fa, sp->parent, sp->tok, sp->draft_codes, sp->chain_ok,
                             sp->codes_out, st));
    S2P_TRY(s2p_verify_accept_tail(m->bb, sp->logits, sp->drf, sp->parent, sp->tok, ss->states,
                                   sp->chain_ok, sp->path, sp->o.n_acc, sp->o.emit, sp->o.n_emit,
                                   sp->tail, sp->work, st));
    /* 6: the last frame's codes, the sessions' next state */
    const void* hidden = s2p_backbone_chain_hidden(m->bb);
    S2P_TRY(hip_ok(s2p_spec_pick_launch(sp->tail, sp->o.emit, sp->o.n_emit, hidden, n, R,
                                        sp->bonus_hidden, sp->bonus_sem, st), "pick"));
    const int32_t* stage = NULL;
    S2P_TRY(s2pfa_decode_frame_batch_dev(m->fa, sp->bonus_hidden, sp->bonus_sem, n, &stage, st));
    SpecAdvanceArgs a;
    memset(&a, 0, sizeof(a));
    a.n_sess = n;
    a.R = R;
    a.n_acc = sp->o.n_acc;
    a.n_emit = sp->o.n_emit;
    a.emit = sp->o.emit;
    a.path = sp->path;
    a.tail = sp->tail;
    a.codes_out = sp->codes_out;
    a.stage = stage;
    a.hidden = (const uint16_t*)hidden;
    a.frames = sp->o.frames;
    a.kv_len = ss->kv_len;
    a.prev_tok = ss->prev_tok;
    a.prev_codes = ss->prev_codes;
    a.prev_hidden = ss->prev_hidden;
    a.done = ss->done;
    return hip_ok(s2p_spec_advance_launch(&a, st), "advance");
}

s2p_status s2p_spec_tick(s2p_spec* sp, int use_graph, hipStream_t st) {
    if (!sp) return S2P_ERR_INVALID;
    int need = 0;
    for (int s = 0; s < sp->n; s++) need |= sp->bound[s] + sp->R > sp->span;
    if (need) S2P_TRY(replan(sp, NULL, st));
    if (!use_graph) {
        S2P_TRY(tick_enqueue(sp, st));
    } else {
        if (!sp->g_valid) {
            hipGraph_t g;
            S2P_TRY(hip_ok(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "capture"));
            const s2p_status rc = tick_enqueue(sp, st);
            hipError_t ce = hipStreamEndCapture(st, &g);
            if (rc != S2P_OK) {
                if (ce == hipSuccess) (void)hipGraphDestroy(g);
                return rc;
            }
            S2P_TRY(hip_ok(ce, "end capture"));
            ce = hipGraphInstantiate(&sp->gexec, g, NULL, NULL, 0);
            (void)hipGraphDestroy(g);
            S2P_TRY(hip_ok(ce, "graph instantiate"));
            sp->g_valid = 1;
        }
        S2P_TRY(hip_ok(hipGraphLaunch(sp->gexec, st), "graph launch"));
    }
    for (int s = 0; s < sp->n; s++) sp->bound[s] += sp->R;
    return S2P_OK;
}

s2p_status s2p_spec_buffers_of(const s2p_spec* sp, s2p_spec_buffers* out) {
    if (!sp || !out) return S2P_ERR_INVALID;
    out->logits = sp->logits;
    out->drf_logits = sp->drf;
    out->x = sp->x;
    out->tok = sp->tok;
    out->draft_codes = sp->draft_codes;
    out->codes_out = sp->codes_out;
    out->path = sp->path;
    out->tail = sp->tail;
    out->chain_ok = sp->chain_ok;
    out->head_rows = sp->W;
    out->replans = sp->replans;
    return S2P_OK;
}

void s2p_spec_free(s2p_spec* sp) {
    if (!sp) return;
    (void)hipDeviceSynchronize();
    if (sp->g_valid) (void)hipGraphExecDestroy(sp->gexec);
    void* bufs[] = {sp->logits,   sp->drf,         sp->x,         sp->hid[0],   sp->hid[1],
                    sp->bonus_hidden, sp->tok,     sp->tok_d,     sp->draft_codes, sp->codes_out,
                    sp->path,     sp->tail,        sp->sem_d,     sp->codes_d,  sp->bonus_sem,
                    sp->overflow, sp->parent,      sp->chain_ok,  sp->eos_d,    sp->work,
                    sp->dstates,  sp->dstate_ptrs};
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++)
        if (bufs[i]) (void)hipFree(bufs[i]);
    free(sp);
}
