/* s2pro MI355X — the composed speculative tick.
 *
 * New API (no reference counterpart: the reference's per-tick entry is the
 * non-speculative s2p_model_batch_next_frame, src/slowar/slowar.c:609-826,
 * which embeds the previous frame, runs the backbone, samples and decodes
 * the frame's codes in one captured graph; its speculative stage was
 * designed but never built, docs/SPECULATIVE.md:249-256).  One tick does,
 * for n_sess sessions with K-token drafts (R = K + 1 verify rows each):
 *   1. the verify plan from the device KV lengths (s2p_verify_plan_device);
 *   2. row 0 of each session: the embedding of its previous frame;
 *   3. K draft steps: draft forward on [h ; e], q logits over the tied-head
 *      slice, a token sampled from them with a copy of the session's
 *      sampler state, the fast-AR codes of that drafted frame on the draft's
 *      hidden, and the frame's embedding as the next verify row;
 *   4. the verify forward over the n_sess x R rows;
 *   5. the chain condition (fast-AR on each drafted node's parent's true
 *      hidden, docs/SPECULATIVE.md:26-41) and acceptance under it;
 *   6. the codes of the last emitted token's frame (fast-AR on the true
 *      hidden of the row that produced it, unless the chain condition
 *      already decoded it), and each session's next root frame, hidden and
 *      KV length (kv_len += 1 + n_accepted).
 * Every step runs on the device, so consecutive ticks replay ONE captured
 * hipGraph with no host round trip.  The host only keeps an upper bound of
 * each session's length (R per tick); when a session could outgrow the span
 * the plan's launches were sized for (512-slot buckets), s2p_spec_tick
 * synchronises once, re-plans and re-captures.
 *
 * Draft positions: the draft step of depth i runs at frame index
 * kv_len + i - 1 of the session's draft cache (rollback by length, as the
 * backbone's cache).  A session that emits EOS is finished: its done flag is
 * set and later ticks leave its length and frame untouched (its rows are
 * still computed; drop it at the next s2p_spec_create).  A tick whose
 * forward did not complete (see s2p_verify_forward) reports n_acc = -1 and
 * changes no session. */
#ifndef S2P_SPEC_H
#define S2P_SPEC_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#include "s2pro/draft.h"
#include "s2pro/fastar.h"
#include "s2pro/status.h"
#include "s2pro/verify.h"

#ifdef __cplusplus
extern "C" {
#endif

#define S2P_SPEC_MAX_SESSIONS 16

typedef struct {
    s2p_backbone*     bb;           /* max_rows >= n_sess * (K + 1), bf16 KV caches */
    s2p_draft_model*  draft;
    s2p_draft_state*  draft_states; /* [n_sess]: each session's draft KV cache */
    s2pfa*            fa;           /* max_b >= n_sess * K */
    const void*       embed;        /* [155776][2560] bf16 token embedding (the tied head's
                                     * table, reference s2pk_embed) */
    int               n_sess, K;
} s2p_spec_model;

/* Per-session state, device memory owned by the caller, read and advanced
 * by every tick. */
typedef struct {
    void* const*      kv;          /* host [n_sess]: the sessions' backbone KV bases */
    int32_t*          kv_len;      /* [n_sess] cached tokens */
    int64_t*          prev_tok;    /* [n_sess] the last emitted token */
    int32_t*          prev_codes;  /* [n_sess][10] its frame: semantic code, 9 residual codes */
    void*             prev_hidden; /* [n_sess][2560] bf16: the final-normed hidden that
                                    * produced it (the draft's first h) */
    s2ps_dev_state* const* states; /* [n_sess] device array of the sessions' sampler states */
    uint8_t*          done;        /* [n_sess] 1 once the session emitted EOS */
} s2p_spec_sessions;

/* Per-tick outputs (device memory owned by the caller, rewritten by every
 * tick). */
typedef struct {
    int32_t* n_acc;   /* [n_sess] accepted drafted frames, -1: the forward did not complete */
    int32_t* n_emit;  /* [n_sess] frames emitted this tick */
    int64_t* emit;    /* [n_sess][K + 2] their tokens */
    int32_t* frames;  /* [n_sess][K + 2][10] their codes (semantic code first; zeros for EOS) */
} s2p_spec_out;

typedef struct s2p_spec s2p_spec;

/* Bind the model, sessions and outputs (all kept by reference) and plan the
 * first tick from the host lengths kv_len_host [n_sess].  Allocates the
 * tick's buffers; synchronises st. */
s2p_status s2p_spec_create(s2p_spec** out, const s2p_spec_model* m, const s2p_spec_sessions* ss,
                           const int32_t* kv_len_host, const s2p_spec_out* o, hipStream_t st);

/* One tick: replayed from a hipGraph captured at the first call for the
 * current plan (use_graph = 1), or launched eagerly (use_graph = 0).  No
 * host synchronisation except the occasional re-plan described above. */
s2p_status s2p_spec_tick(s2p_spec* sp, int use_graph, hipStream_t st);

/* The tick's intermediate device buffers (tests, instrumentation):
 * target logits [n_sess*R][head_rows], draft logits (same layout), drafted
 * tokens [n_sess*R] (entry 0 of a session unused), drafted residual codes
 * [n_sess*R][9], chain flags [n_sess*R], chain codes [n_sess*R][9], accepted
 * path [n_sess*R], walk tail [n_sess][2], verify inputs [n_sess*R][2560]. */
typedef struct {
    void *logits, *drf_logits, *x;
    int64_t* tok;
    int32_t *draft_codes, *codes_out, *path, *tail;
    uint8_t* chain_ok;
    int head_rows;
    int replans;   /* host re-plans so far */
} s2p_spec_buffers;
s2p_status s2p_spec_buffers_of(const s2p_spec* sp, s2p_spec_buffers* out);

void s2p_spec_free(s2p_spec* sp);

#ifdef __cplusplus
}
#endif
#endif
