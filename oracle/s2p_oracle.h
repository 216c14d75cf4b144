/* s2pro MI355X — CPU oracle for the speculative-verify path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a scalar C restatement of the reference
 * algorithms on the verify path (luka-loehr/s2pro-native), used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker.
 * Nothing in the shipped library links, loads or calls it.
 *
 * Each function cites the reference file:line it restates.  Where the
 * reference's result depends on nvcc's default FMA contraction of `a*b + c`
 * (--fmad=true), the restatement uses an explicit fmaf; where the reference
 * calls a CUDA approximate intrinsic (rsqrtf, powf, cosf, sinf, expf) the
 * restatement uses the correctly rounded value (see the notes per function);
 * the transcendental functions of the sampling rule are the ones specified in
 * include/s2pro/s2p_fmath.h.
 *
 * Pinning status (what checks each function beyond the restatement itself)
 * is listed in tests/test_oracle.py; every function here is pinned by at
 * least one closed form, invariant, brute-force or golden-vector check.
 *
 * All arrays are host memory.  bf16 and f16 values are passed as uint16_t
 * bit patterns.
 */
#ifndef S2P_ORACLE_H
#define S2P_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions ------------------------------------------------ */
float    or_bf2f(uint16_t h);
uint16_t or_f2bf(float f);          /* round to nearest even */
float    or_h2f(uint16_t h);
uint16_t or_f2h(float f);           /* round to nearest even */
void     or_bf16_to_f32(const uint16_t* in, float* out, int64_t n);
void     or_f32_to_bf16(const float* in, uint16_t* out, int64_t n);

/* ---- weight formats (src/sched/int8_gemv.cu) --------------------------- */
void or_int8_quant(int8_t* q, float* scales, const uint16_t* w, int N, int K);
void or_intq_quant(int8_t* q, uint16_t* scales_f16, const uint16_t* w, int N,
                   int K, int G, int levels, int mse);
void or_int4_pack(uint8_t* p, const int8_t* q, int N, int K);
void or_int8_dequant(uint16_t* o, const int8_t* w, const float* sc, int N, int K);
void or_intq_dequant(uint16_t* o, const int8_t* w, const uint16_t* sc, int N,
                     int K, int G);
void or_int4p_dequant(uint16_t* o, const uint8_t* w, const uint16_t* sc, int N,
                      int K, int G);

/* ---- GEMVs in the reference's per-lane order ------------------------------ */
void or_int8_gemv(uint16_t* y, const uint16_t* x, const int8_t* w,
                  const float* sc, int M, int N, int K);
void or_intq_gemv(uint16_t* y, const uint16_t* x, const int8_t* w,
                  const uint16_t* sc, int M, int N, int K, int G);
void or_int4p_gemv(uint16_t* y, const uint16_t* x, const uint8_t* w,
                   const uint16_t* sc, int M, int N, int K, int G);
/* exact (binary64) dot products, no output rounding: ground truth */
void or_int8_gemv_f64(double* y, const uint16_t* x, const int8_t* w,
                      const float* sc, int M, int N, int K);
void or_int4p_gemv_f64(double* y, const uint16_t* x, const uint8_t* w,
                       const uint16_t* sc, int M, int N, int K, int G);

/* ---- transformer primitives (src/slowar/kernels.cu) ----------------------- */
void or_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* y, int rows,
                 int width, float eps);
void or_qk_norm(uint16_t* qk, const uint16_t* w, int rows, int heads,
                int head_dim, float eps);
void or_rope(uint16_t* x, int rows, int heads, int head_dim, int pos0,
             const int32_t* pos_arr, float base);
void or_kv_append(const uint16_t* k, const uint16_t* v, uint16_t* kc,
                  uint16_t* vc, int rows, int kv_heads, int head_dim,
                  int pos0, const int32_t* slot_arr, int max_seq);
void or_qkv_split(const uint16_t* qkv, uint16_t* q, uint16_t* k, uint16_t* v,
                  int rows, int q_width, int kv_width);
void or_silu_mul(const uint16_t* gu, uint16_t* h, int rows, int ffn);
void or_add(uint16_t* y, const uint16_t* x, int64_t n);

/* Attention over one session's cache [kv_heads, max_seq, head_dim].
 * Visibility of row r: cache slots [0, prefix) plus slot prefix+b for every
 * b < rows with bit b set in vis[r] (vis == NULL: causal, b <= r).
 * or_attention follows k_attention's tile order; or_attention_split follows
 * k_attn_split + k_attn_combine; or_attention_f64 is the binary64 ground
 * truth (unrounded output). */
void or_attention(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                  uint16_t* out, int rows, int q_heads, int kv_heads,
                  int head_dim, int prefix, const uint64_t* vis, int max_seq);
void or_attention_split(const uint16_t* q, const uint16_t* kc,
                        const uint16_t* vc, uint16_t* out, int rows,
                        int q_heads, int kv_heads, int head_dim, int prefix,
                        int max_seq);
void or_attention_f64(const uint16_t* q, const uint16_t* kc,
                      const uint16_t* vc, double* out, int rows, int q_heads,
                      int kv_heads, int head_dim, int prefix,
                      const uint64_t* vis, int max_seq);

/* INT8 / INT4 KV cache (kernels.cu:510-946): payload [kv_heads][max_seq]
 * [bw == 8 ? 128 : 64] bytes, f16 scales [kv_heads][max_seq][4].  Caches are
 * passed as pointer arrays: slot_arr == NULL appends rows at pos0.. of cache
 * 0, else row r at slot slot_arr[r] of cache r. */
void or_kv_append8(const uint16_t* k, const uint16_t* v, int8_t* const* kcs,
                   int8_t* const* vcs, uint16_t* const* kss, uint16_t* const* vss,
                   int rows, int kv_heads, int pos0, const int32_t* slot_arr,
                   int max_seq, int bw);
void or_attention8(const uint16_t* q, const int8_t* kc, const int8_t* vc,
                   const uint16_t* ks, const uint16_t* vs, uint16_t* out, int rows,
                   int q_heads, int kv_heads, int pos0, int max_seq, int bw);
/* the same with the verify visibility (vis[r] bit b: slot prefix + b), or
 * causal rows at prefix.. when vis is NULL */
void or_attention8_vis(const uint16_t* q, const int8_t* kc, const int8_t* vc,
                       const uint16_t* ks, const uint16_t* vs, uint16_t* out, int rows,
                       int q_heads, int kv_heads, int prefix, const uint64_t* vis, int max_seq,
                       int bw);
void or_attention8_f64(const uint16_t* q, const int8_t* const* kcs, const int8_t* const* vcs,
                       const uint16_t* const* kss, const uint16_t* const* vss, double* out,
                       int rows, int q_heads, int kv_heads, const int32_t* pos, int max_seq,
                       int bw);

/* ---- sampler (src/slowar/sampling.c) ------------------------------------ */
/* Device sampler state, byte layout of src/slowar/slowar_kernels.h:132-142. */
typedef struct {
    int64_t  prev[64];
    uint64_t count;
    uint64_t rng[4];
    float    temperature, top_p, rep_penalty;
    int32_t  window, seeded;
    uint32_t seed31;
    uint32_t pad_;
} or_state;

/* s2ps_sampler_init + s2p_sampling_defaults (sampling.c:83-112). */
void or_state_init(or_state* st, float temperature, float top_p,
                   float rep_penalty, int window, uint64_t seed,
                   uint64_t entropy);
/* 1 = libm expf/logf (the reference's calls), 0 = the rule's s2p_expf/logf */
void or_set_libm(int on);

/* The sampler transform T of sampling.c:119-219: candidate gather, RAS,
 * repetition penalty, top-30, top-p, temperature softmax.  row_bf16 is a
 * logits row; eos_bf16 == NULL means row_bf16 spans the full vocabulary and
 * the semantic slice / EOS are gathered at their vocab ids; otherwise row_bf16
 * holds the 4096 semantic logits and *eos_bf16 the EOS logit.
 * Outputs: ti[30] candidate indices (0..4095 semantic, 4096 EOS), tv[30]
 * penalised values, p2[30] final probabilities; returns 1 if greedy. */
int or_transform(const or_state* st, const uint16_t* row_bf16,
                 const uint16_t* eos_bf16, int ti[30], float tv[30],
                 float p2[30]);
/* s2ps_sample (sampling.c:119-282): transform + draw + history update.
 * Returns the raw vocab id. */
int64_t or_sample(or_state* st, const uint16_t* row_bf16,
                  const uint16_t* eos_bf16, int32_t* out_sem, int* out_eos);
/* Test hooks: splitmix64 step (sampling.c:54-59), xoshiro256** step
 * (sampling.c:65-75), the seeded hash-Gumbel draw (sampling.c:221-243) and the
 * unseeded inverse-CDF draw (sampling.c:244-262) over prob[0..29] with the
 * state as is (no history update), and the acceptance rule's counter-based
 * 24-bit uniform. */
uint64_t or_splitmix64_next(uint64_t* s);
uint64_t or_xoshiro_next(uint64_t s[4]);
int or_gumbel_draw(const or_state* st, const float* prob);
int or_xoshiro_draw(or_state* st, const float* prob);
uint32_t or_rule_u24(const or_state* st, uint32_t slot);
/* history update of sampling.c:269-281 for an emitted vocab id */
void or_state_push(or_state* st, int64_t tok);

/* ---- acceptance (build-defined rule, Leviathan et al. 2211.17192; tree
 * form of SpecInfer) ------------------------------------------------------- */
/* One session.  Nodes 0..R-1, node 0 = root (the last accepted token);
 * parent[i] < i for i >= 1.  tgt row i = target logits after node i; drf row
 * i = draft logits whose samples are node i's children; tok[i] = node i's
 * drafted vocab id (i >= 1).  Rows use the or_transform layout with
 * row_stride elements per row and optional per-row eos arrays.
 * Outputs: path[] accepted node ids (root excluded), *n_acc, emitted[] vocab
 * ids (accepted tokens then the corrected/bonus token unless an accepted EOS
 * ended generation), *n_emit.  The state advances over emitted non-EOS ids.
 */
void or_accept_tree(or_state* st, const uint16_t* tgt, const uint16_t* tgt_eos,
                    const uint16_t* drf, const uint16_t* drf_eos,
                    int64_t row_stride, const int32_t* parent,
                    const int64_t* tok, int R, int32_t* path, int* n_acc,
                    int64_t* emitted, int* n_emit, const uint8_t* chain);

/* ---- the verify forward (src/slowar/slowar.c:156-260, 503-565) --------- */
typedef struct {
    /* packed INT4-g32 (q_group > 0) or per-channel INT8 (q_group == 0) */
    const void* w;        /* [N, K/2] u8 (int4) or [N, K] i8 (int8) */
    const void* s;        /* [N, K/G] f16 (int4) or [N] f32 (int8) */
    int N, K, G;
} or_linear;

typedef struct {
    or_linear wqkv, wo, gate_up, w2;
    const uint16_t* attn_norm; /* [dim] */
    const uint16_t* ffn_norm;  /* [dim] */
    const uint16_t* q_norm;    /* [head_dim] */
    const uint16_t* k_norm;    /* [head_dim] */
} or_layer_w;

void or_linear_fwd(const or_linear* L, const uint16_t* x, uint16_t* y, int M);

/* One backbone layer over `rows` rows of one session: x [rows, dim] in/out;
 * kc/vc this layer's cache planes [kv_heads, max_seq, head_dim]; row r has
 * RoPE position pos[r], KV slot prefix + r, visibility vis (NULL = causal). */
void or_layer(const or_layer_w* lw, uint16_t* x, int rows, uint16_t* kc,
              uint16_t* vc, int max_seq, int prefix, const int32_t* pos,
              const uint64_t* vis);
/* the same over one layer's INT8 / INT4 KV cache (payload [8][max_seq][128
 * or 64], f16 scales [8][max_seq][4]); rows append at slots prefix + r
 * (append != 0) or find their codes there already (append == 0) */
void or_layer8(const or_layer_w* lw, uint16_t* x, int rows, int8_t* kc, int8_t* vc,
               uint16_t* ks, uint16_t* vs, int max_seq, int prefix, const int32_t* pos,
               const uint64_t* vis, int bw, int append);

/* ---- the fast-AR frame (src/fastar/fastar.cu:726-789) ------------------ */
typedef struct {
    or_layer_w layers[4];     /* q_norm = k_norm = NULL: no qk-norm */
    const uint16_t* norm;     /* final RMSNorm [2560] */
    or_linear output;         /* untied head [4096, 2560] */
    const uint16_t* emb;      /* embeddings [4096, 2560] */
} or_fa_w;

/* One frame of one row: codes[0..8] the nine residual codes; logits (may be
 * NULL) [9][4096] the head outputs of the nine steps. */
void or_fastar_frame(const or_fa_w* w, const uint16_t* hidden, int sem, int32_t* codes,
                     uint16_t* logits);
/* codes [10][T] codebook-major; rows [T, 2560] bf16 in/out */
void or_vq_embed_add(const uint16_t* cb_emb, const int32_t* codes, int T, uint16_t* rows);

/* ---- the draft model (src/draft/draft.c:157-202) ---------------------- */
/* y[M,N] = bf16(sum_k w[n,k] x[m,k]) with an fp32 sum in increasing k: the
 * contract of s2p_gemm_bf16 (reference gemm.h:93-96, cuBLAS there, whose
 * summation order is not published: pinned against the binary64 dot only). */
void or_gemm_bf16(const uint16_t* x, const uint16_t* w, uint16_t* y, int M, int N, int K);
void or_gemm_bf16_f64(const uint16_t* x, const uint16_t* w, double* y, int M, int N, int K);

typedef struct {
    const uint16_t* fuse;   /* [2560, 5120] */
    const uint16_t* wqkv;   /* [6144, 2560] */
    const uint16_t* wo;     /* [2560, 4096] */
    const uint16_t* w1;     /* [9728, 2560] */
    const uint16_t* w3;     /* [9728, 2560] */
    const uint16_t* w2;     /* [2560, 9728] */
    const uint16_t* q_norm; /* [128] */
    const uint16_t* k_norm; /* [128] */
    const uint16_t* attn_norm, *ffn_norm, *final_norm; /* [2560] */
} or_draft_w;

/* One draft step at position pos: consumes h, e [2560], appends K/V at slot
 * pos of kc/vc [8, max_seq, 128], writes out [2560] (final-normed). */
void or_draft_step(const or_draft_w* d, uint16_t* kc, uint16_t* vc, int max_seq, int pos,
                   const uint16_t* h, const uint16_t* e, uint16_t* out);

#ifdef __cplusplus
}
#endif
#endif
