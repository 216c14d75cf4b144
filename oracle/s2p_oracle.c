/* s2pro MI355X — CPU oracle (TEST INFRASTRUCTURE ONLY; see s2p_oracle.h).
 *
 * Scalar restatement of the reference verify-path arithmetic.  Built by
 * oracle/Makefile with -O2 -ffp-contract=off so that every a*b+c below is
 * two roundings unless written as fmaf().
 */
#include "s2p_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "s2pro/s2p_fmath.h"

/* ----------------------------------------------------------- conversions */

float or_bf2f(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t or_f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu))
        return (uint16_t)((u >> 16) | 0x0040u); /* quiet nan */
    const uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}

float or_h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    uint32_t u;
    if (e == 0) {
        if (m == 0) {
            u = s;
        } else { /* subnormal: value m * 2^-24, exact in float */
            float f = (float)m * 5.9604644775390625e-08f;
            memcpy(&u, &f, 4);
            u |= s;
        }
    } else if (e == 31) {
        u = s | 0x7F800000u | (m << 13);
    } else {
        u = s | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t or_f2h(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint16_t s = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) /* inf / nan */
        return (uint16_t)(s | 0x7C00u | (a > 0x7F800000u ? 0x200u : 0u));
    if (a >= 0x477FF000u) return (uint16_t)(s | 0x7C00u); /* rounds to inf */
    if (a < 0x38800000u) { /* result subnormal or zero: units of 2^-24 */
        float af;
        memcpy(&af, &a, 4);
        /* af * 2^24 is exact (power-of-two scale); round to int, ties even */
        float t = af * 16777216.0f;
        float r = nearbyintf(t);
        return (uint16_t)(s | (uint16_t)r);
    }
    uint32_t e = ((a >> 23) - 112u) << 10;
    uint32_t m = (a >> 13) & 0x3FFu;
    uint32_t h = e | m;
    const uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(s | h);
}

void or_bf16_to_f32(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = or_bf2f(in[i]);
}
void or_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = or_f2bf(in[i]);
}

static int gshift_of(int G) {
    int s = 0;
    while ((1 << s) < G) s++;
    return s;
}

/* ------------------------------------------------------- weight formats */

/* k_quant (int8_gemv.cu:32-58): per-row absmax/127, RTN (ties even),
 * clamp to +-127.  The absmax reduction is order-insensitive. */
void or_int8_quant(int8_t* q, float* scales, const uint16_t* w, int N, int K) {
    for (int n = 0; n < N; n++) {
        const uint16_t* row = w + (size_t)n * K;
        float amax = 0.f;
        for (int k = 0; k < K; k++) amax = fmaxf(amax, fabsf(or_bf2f(row[k])));
        const float scale = amax > 0.f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / scale;
        scales[n] = scale;
        for (int k = 0; k < K; k++) {
            int v = (int)nearbyintf(or_bf2f(row[k]) * inv);
            v = v > 127 ? 127 : (v < -127 ? -127 : v);
            q[(size_t)n * K + k] = (int8_t)v;
        }
    }
}

/* k_quant_g (int8_gemv.cu:135-195), launched with min(G,256) threads per
 * group (int8_gemv.cu:760-763).  The MSE error is reduced per thread then by
 * the shared-memory tree of :176-179; nvcc contracts `v - qi*s` and
 * `err += d*d` into FMAs. */
void or_intq_quant(int8_t* q, uint16_t* scales_f16, const uint16_t* w, int N,
                   int K, int G, int levels, int mse) {
    const int ng = K / G;
    const int T = G < 256 ? G : 256;
    float* red = (float*)malloc(sizeof(float) * (size_t)T);
    for (int n = 0; n < N; n++) {
        for (int g = 0; g < ng; g++) {
            const uint16_t* wp = w + (size_t)n * K + (size_t)g * G;
            float amax = 0.f;
            for (int k = 0; k < G; k++) amax = fmaxf(amax, fabsf(or_bf2f(wp[k])));
            const float base = amax > 0.f ? amax / (float)levels : 1.0f;
            float scale = or_h2f(or_f2h(base));
            if (mse && amax > 0.f) {
                float best_err = 3.4e38f, best_s = scale;
                for (int c = 0; c < 32; c++) {
                    const float s = or_h2f(or_f2h(
                        base * (1.0f - (float)c / (2.0f * 32))));
                    const float inv = 1.0f / s;
                    for (int t = 0; t < T; t++) {
                        float err = 0.f;
                        for (int k = t; k < G; k += T) {
                            const float v = or_bf2f(wp[k]);
                            int qi = (int)nearbyintf(v * inv);
                            qi = qi > levels ? levels : (qi < -levels ? -levels : qi);
                            const float d = fmaf(-(float)qi, s, v);
                            err = fmaf(d, d, err);
                        }
                        red[t] = err;
                    }
                    for (int r = T / 2; r > 0; r >>= 1)
                        for (int t = 0; t < r; t++) red[t] += red[t + r];
                    if (red[0] < best_err) {
                        best_err = red[0];
                        best_s = s;
                    }
                }
                scale = best_s;
            }
            scales_f16[(size_t)n * ng + g] = or_f2h(scale);
            const float inv = 1.0f / scale;
            for (int k = 0; k < G; k++) {
                int v = (int)nearbyintf(or_bf2f(wp[k]) * inv);
                v = v > levels ? levels : (v < -levels ? -levels : v);
                q[(size_t)n * K + (size_t)g * G + k] = (int8_t)v;
            }
        }
    }
    free(red);
}

/* k_pack_nib (int8_gemv.cu:265-269): low nibble = even k. */
void or_int4_pack(uint8_t* p, const int8_t* q, int N, int K) {
    const size_t n = (size_t)N * (size_t)(K / 2);
    for (size_t i = 0; i < n; i++)
        p[i] = (uint8_t)((q[2 * i] & 0xF) | ((q[2 * i + 1] & 0xF) << 4));
}

static inline int nib(const uint8_t* row, int k) {
    const uint8_t b = row[k >> 1];
    return (k & 1) ? (int)((int8_t)b >> 4) : (int)((int8_t)(uint8_t)(b << 4) >> 4);
}

void or_int8_dequant(uint16_t* o, const int8_t* w, const float* sc, int N, int K) {
    for (int n = 0; n < N; n++)
        for (int k = 0; k < K; k++)
            o[(size_t)n * K + k] = or_f2bf((float)w[(size_t)n * K + k] * sc[n]);
}

void or_intq_dequant(uint16_t* o, const int8_t* w, const uint16_t* sc, int N,
                     int K, int G) {
    const int gs = gshift_of(G);
    for (int n = 0; n < N; n++)
        for (int k = 0; k < K; k++)
            o[(size_t)n * K + k] = or_f2bf((float)w[(size_t)n * K + k] *
                                          or_h2f(sc[(size_t)n * (K >> gs) + (k >> gs)]));
}

/* k_dequant_p (int8_gemv.cu:731-744) */
void or_int4p_dequant(uint16_t* o, const uint8_t* w, const uint16_t* sc, int N,
                      int K, int G) {
    const int gs = gshift_of(G);
    for (int n = 0; n < N; n++) {
        const uint8_t* row = w + (size_t)n * (K / 2);
        for (int k = 0; k < K; k++)
            o[(size_t)n * K + k] = or_f2bf(
                (float)nib(row, k) * or_h2f(sc[(size_t)n * (K >> gs) + (k >> gs)]));
    }
}

/* ---------------------------------------------------------------- GEMVs */

/* 32-lane __shfl_down_sync tree (int8_gemv.cu:97-100): lane 0's result. */
static float warp_reduce32(float* lane) {
    float tmp[32];
    for (int off = 16; off > 0; off >>= 1) {
        for (int l = 0; l < 32; l++)
            tmp[l] = lane[l] + (l + off < 32 ? lane[l + off] : lane[l]);
        memcpy(lane, tmp, sizeof(tmp));
    }
    return lane[0];
}

/* k_gemv (int8_gemv.cu:60-104).  int8 x bf16 products are exact in fp32, so
 * contraction of `s += w*x` does not change s. */
void or_int8_gemv(uint16_t* y, const uint16_t* x, const int8_t* w,
                  const float* sc, int M, int N, int K) {
    float lane[32];
    for (int n = 0; n < N; n++) {
        const int8_t* wrow = w + (size_t)n * K;
        for (int m = 0; m < M; m++) {
            for (int l = 0; l < 32; l++) {
                float acc = 0.f;
                for (int k0 = l * 16; k0 < K; k0 += 512) {
                    float s = 0.f;
                    for (int j = 0; j < 16; j++)
                        s = fmaf((float)wrow[k0 + j], or_bf2f(x[(size_t)m * K + k0 + j]), s);
                    acc += s;
                }
                lane[l] = acc;
            }
            y[(size_t)m * N + n] = or_f2bf(warp_reduce32(lane) * sc[n]);
        }
    }
}

/* k_gemv_g (int8_gemv.cu:197-242): acc = fma(s, gs, acc). */
void or_intq_gemv(uint16_t* y, const uint16_t* x, const int8_t* w,
                  const uint16_t* sc, int M, int N, int K, int G) {
    const int gs = gshift_of(G);
    float lane[32];
    for (int n = 0; n < N; n++) {
        const int8_t* wrow = w + (size_t)n * K;
        const uint16_t* srow = sc + (size_t)n * (K >> gs);
        for (int m = 0; m < M; m++) {
            for (int l = 0; l < 32; l++) {
                float acc = 0.f;
                for (int k0 = l * 16; k0 < K; k0 += 512) {
                    const float g = or_h2f(srow[k0 >> gs]);
                    float s = 0.f;
                    for (int j = 0; j < 16; j++)
                        s = fmaf((float)wrow[k0 + j], or_bf2f(x[(size_t)m * K + k0 + j]), s);
                    acc = fmaf(s, g, acc);
                }
                lane[l] = acc;
            }
            y[(size_t)m * N + n] = or_f2bf(warp_reduce32(lane));
        }
    }
}

/* k_gemv_p (int8_gemv.cu:279-324): the packed-INT4 decode GEMV. */
void or_int4p_gemv(uint16_t* y, const uint16_t* x, const uint8_t* w,
                   const uint16_t* sc, int M, int N, int K, int G) {
    const int gs = gshift_of(G);
    float lane[32];
    float* xf = (float*)malloc(sizeof(float) * (size_t)M * K);
    or_bf16_to_f32(x, xf, (int64_t)M * K);
    for (int n = 0; n < N; n++) {
        const uint8_t* wrow = w + (size_t)n * (K / 2);
        const uint16_t* srow = sc + (size_t)n * (K >> gs);
        for (int m = 0; m < M; m++) {
            const float* xr = xf + (size_t)m * K;
            for (int l = 0; l < 32; l++) {
                float acc = 0.f;
                for (int k0 = l * 16; k0 < K; k0 += 512) {
                    const float g = or_h2f(srow[k0 >> gs]);
                    float s = 0.f;
                    for (int j = 0; j < 16; j++)
                        s = fmaf((float)nib(wrow, k0 + j), xr[k0 + j], s);
                    acc = fmaf(s, g, acc);
                }
                lane[l] = acc;
            }
            y[(size_t)m * N + n] = or_f2bf(warp_reduce32(lane));
        }
    }
    free(xf);
}

void or_int8_gemv_f64(double* y, const uint16_t* x, const int8_t* w,
                      const float* sc, int M, int N, int K) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            double a = 0.0;
            for (int k = 0; k < K; k++)
                a += (double)w[(size_t)n * K + k] * (double)or_bf2f(x[(size_t)m * K + k]);
            y[(size_t)m * N + n] = a * (double)sc[n];
        }
}

void or_int4p_gemv_f64(double* y, const uint16_t* x, const uint8_t* w,
                       const uint16_t* sc, int M, int N, int K, int G) {
    const int gs = gshift_of(G);
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            const uint8_t* wrow = w + (size_t)n * (K / 2);
            double a = 0.0;
            for (int k = 0; k < K; k++)
                a += (double)nib(wrow, k) *
                     (double)or_h2f(sc[(size_t)n * (K >> gs) + (k >> gs)]) *
                     (double)or_bf2f(x[(size_t)m * K + k]);
            y[(size_t)m * N + n] = a;
        }
}

/* --------------------------------------------------------------- norms */

/* 1/sqrt(v) as two correctly rounded float operations.  The reference uses
 * the approximate rsqrtf (kernels.cu:62, :97); this rule fixes its value. */
static inline float rsqrt_rule(float v) { return 1.0f / sqrtf(v); }

/* k_rms_norm (kernels.cu:46-77), 256 threads: per-thread strided sum of
 * squares (contracted to fma), shared-memory tree, y = bf16((v*inv)*w). */
void or_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* y, int rows,
                 int width, float eps) {
    float red[256];
    for (int r = 0; r < rows; r++) {
        const uint16_t* xr = x + (size_t)r * width;
        for (int t = 0; t < 256; t++) {
            float s = 0.f;
            for (int i = t; i < width; i += 256) {
                const float v = or_bf2f(xr[i]);
                s = fmaf(v, v, s);
            }
            red[t] = s;
        }
        for (int off = 128; off > 0; off >>= 1)
            for (int t = 0; t < off; t++) red[t] += red[t + off];
        const float inv = rsqrt_rule(red[0] / (float)width + eps);
        for (int i = 0; i < width; i++)
            y[(size_t)r * width + i] = or_f2bf(or_bf2f(xr[i]) * inv * or_bf2f(w[i]));
    }
}

/* k_qk_norm (kernels.cu:81-109), 128 threads = one element each. */
void or_qk_norm(uint16_t* qk, const uint16_t* w, int rows, int heads,
                int head_dim, float eps) {
    float red[256];
    for (int b = 0; b < rows * heads; b++) {
        uint16_t* p = qk + (size_t)b * head_dim;
        for (int t = 0; t < 128; t++) {
            float s = 0.f;
            for (int i = t; i < head_dim; i += 128) {
                const float v = or_bf2f(p[i]);
                s = fmaf(v, v, s);
            }
            red[t] = s;
        }
        for (int off = 64; off > 0; off >>= 1)
            for (int t = 0; t < off; t++) red[t] += red[t + off];
        const float inv = rsqrt_rule(red[0] / (float)head_dim + eps);
        for (int i = 0; i < head_dim; i++)
            p[i] = or_f2bf(or_bf2f(p[i]) * inv * or_bf2f(w[i]));
    }
}

/* k_rope (kernels.cu:114-168).  inv = 1/powf(base, 2i/dim), ang = p*inv,
 * cos/sin rounded through bf16, butterfly with per-op rounding.  powf, cosf
 * and sinf take their correctly rounded values here (binary64 libm rounded
 * once to float). */
void or_rope(uint16_t* x, int rows, int heads, int head_dim, int pos0,
             const int32_t* pos_arr, float base) {
    const int pairs = head_dim / 2;
    for (int r = 0; r < rows; r++) {
        const int p = pos_arr ? pos_arr[r] : pos0 + r;
        for (int i = 0; i < pairs; i++) {
            const float ex = (float)(2 * i) / (float)head_dim;
            const float pw = (float)pow((double)base, (double)ex);
            const float inv = 1.0f / pw;
            const float ang = (float)p * inv;
            const float c = or_bf2f(or_f2bf((float)cos((double)ang)));
            const float s = or_bf2f(or_f2bf((float)sin((double)ang)));
            for (int h = 0; h < heads; h++) {
                const size_t o = ((size_t)r * heads + h) * head_dim + 2 * i;
                const float x0 = or_bf2f(x[o]);
                const float x1 = or_bf2f(x[o + 1]);
                const float a = x0 * c, b = x1 * s;
                const float d = x1 * c, e = x0 * s;
                x[o] = or_f2bf(a - b);
                x[o + 1] = or_f2bf(d + e);
            }
        }
    }
}

/* k_kv_append (kernels.cu:172-222); slot_arr == NULL -> slot pos0 + r. */
void or_kv_append(const uint16_t* k, const uint16_t* v, uint16_t* kc,
                  uint16_t* vc, int rows, int kv_heads, int head_dim,
                  int pos0, const int32_t* slot_arr, int max_seq) {
    for (int r = 0; r < rows; r++) {
        const int p = slot_arr ? slot_arr[r] : pos0 + r;
        for (int h = 0; h < kv_heads; h++)
            for (int d = 0; d < head_dim; d++) {
                const size_t src = ((size_t)r * kv_heads + h) * head_dim + d;
                const size_t dst = ((size_t)h * max_seq + p) * head_dim + d;
                kc[dst] = k[src];
                vc[dst] = v[src];
            }
    }
}

/* k_qkv_split (kernels.cu:1368-1384) */
void or_qkv_split(const uint16_t* qkv, uint16_t* q, uint16_t* k, uint16_t* v,
                  int rows, int q_width, int kv_width) {
    const int w = q_width + 2 * kv_width;
    for (int r = 0; r < rows; r++) {
        memcpy(q + (size_t)r * q_width, qkv + (size_t)r * w, 2 * (size_t)q_width);
        memcpy(k + (size_t)r * kv_width, qkv + (size_t)r * w + q_width, 2 * (size_t)kv_width);
        memcpy(v + (size_t)r * kv_width, qkv + (size_t)r * w + q_width + kv_width,
               2 * (size_t)kv_width);
    }
}

/* k_silu_mul (kernels.cu:1216-1229): sig = 1/(1+exp(-g)), silu rounded to
 * bf16, times up rounded to bf16.  exp is the rule's s2p_expf. */
void or_silu_mul(const uint16_t* gu, uint16_t* h, int rows, int ffn) {
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < ffn; c++) {
            const float g = or_bf2f(gu[(size_t)r * 2 * ffn + c]);
            const float u = or_bf2f(gu[(size_t)r * 2 * ffn + ffn + c]);
            const float sig = 1.0f / (1.0f + s2p_expf(-g));
            const float sil = or_bf2f(or_f2bf(g * sig));
            h[(size_t)r * ffn + c] = or_f2bf(sil * u);
        }
}

/* k_add (kernels.cu:1242-1247) */
void or_add(uint16_t* y, const uint16_t* x, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = or_f2bf(or_bf2f(y[i]) + or_bf2f(x[i]));
}

/* ----------------------------------------------------------- attention */

static const float ATTN_SCALE_128 = 0.0883883461356163025f; /* RN(1/sqrt(128)) */

static int visible(int prefix, const uint64_t* vis, int r, int j) {
    if (j < prefix) return 1;
    const int b = j - prefix;
    if (vis) return (int)((vis[r] >> b) & 1u);
    return b <= r;
}

/* k_attention (kernels.cu:234-339): tiles of 128 positions, per-position
 * fmaf dot over e, tree max / tree sum over 128 lanes, l = fma(l, corr,
 * tsum), acc = fma(p, v, acc*corr).  Masked positions inside the window
 * contribute p = 0 exactly like out-of-range ones.  exp is s2p_expf. */
void or_attention(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                  uint16_t* out, int rows, int q_heads, int kv_heads,
                  int head_dim, int prefix, const uint64_t* vis, int max_seq) {
    const int group = q_heads / kv_heads;
    float sq[128], sp[128], red[128], acc[128];
    for (int r = 0; r < rows; r++) {
        int len = prefix + r + 1;
        if (vis)
            for (int b = 0; b < 64; b++)
                if ((vis[r] >> b) & 1u) len = prefix + b + 1 > len ? prefix + b + 1 : len;
        for (int h = 0; h < q_heads; h++) {
            const int kvh = h / group;
            const uint16_t* kb = kc + (size_t)kvh * max_seq * head_dim;
            const uint16_t* vb = vc + (size_t)kvh * max_seq * head_dim;
            for (int e = 0; e < head_dim; e++)
                sq[e] = or_bf2f(q[((size_t)r * q_heads + h) * head_dim + e]) * ATTN_SCALE_128;
            float m = -INFINITY, l = 0.f;
            for (int d = 0; d < head_dim; d++) acc[d] = 0.f;
            for (int t0 = 0; t0 < len; t0 += 128) {
                float s[128];
                for (int t = 0; t < 128; t++) {
                    const int j = t0 + t;
                    s[t] = -INFINITY;
                    if (j < len && visible(prefix, vis, r, j)) {
                        float d = 0.f;
                        for (int e = 0; e < head_dim; e++)
                            d = fmaf(sq[e], or_bf2f(kb[(size_t)j * head_dim + e]), d);
                        s[t] = d;
                    }
                }
                float tmax = -INFINITY;
                for (int t = 0; t < 128; t++) tmax = fmaxf(tmax, s[t]);
                const float m_new = fmaxf(m, tmax);
                const float corr = (m == -INFINITY) ? 0.f : s2p_expf(m - m_new);
                for (int t = 0; t < 128; t++) {
                    sp[t] = (s[t] == -INFINITY) ? 0.f : s2p_expf(s[t] - m_new);
                    red[t] = sp[t];
                }
                for (int off = 64; off > 0; off >>= 1)
                    for (int t = 0; t < off; t++) red[t] += red[t + off];
                l = fmaf(l, corr, red[0]);
                const int lim = len - t0 < 128 ? len - t0 : 128;
                for (int d = 0; d < head_dim; d++) {
                    float a = acc[d] * corr;
                    for (int j2 = 0; j2 < lim; j2++)
                        a = fmaf(sp[j2], or_bf2f(vb[(size_t)(t0 + j2) * head_dim + d]), a);
                    acc[d] = a;
                }
                m = m_new;
            }
            for (int d = 0; d < head_dim; d++)
                out[((size_t)r * q_heads + h) * head_dim + d] = or_f2bf(acc[d] / l);
        }
    }
}

/* k_attn_split + k_attn_combine (kernels.cu:351-489): 64-position splits,
 * per-split tree max/sum over 128 lanes, LSE combine in split order.
 * Causal only (the reference decode path). */
void or_attention_split(const uint16_t* q, const uint16_t* kc,
                        const uint16_t* vc, uint16_t* out, int rows,
                        int q_heads, int kv_heads, int head_dim, int prefix,
                        int max_seq) {
    const int group = q_heads / kv_heads;
    for (int r = 0; r < rows; r++) {
        const int len = prefix + r + 1;
        const int ns = (len + 63) / 64;
        for (int h = 0; h < q_heads; h++) {
            const int kvh = h / group;
            const uint16_t* kb = kc + (size_t)kvh * max_seq * head_dim;
            const uint16_t* vb = vc + (size_t)kvh * max_seq * head_dim;
            float sq[128];
            for (int e = 0; e < head_dim; e++)
                sq[e] = or_bf2f(q[((size_t)r * q_heads + h) * head_dim + e]) * ATTN_SCALE_128;
            float* pm = (float*)malloc(sizeof(float) * ns);
            float* pl = (float*)malloc(sizeof(float) * ns);
            float* pa = (float*)malloc(sizeof(float) * ns * 128);
            for (int sp = 0; sp < ns; sp++) {
                const int start = sp * 64;
                const int cnt = len - start < 64 ? len - start : 64;
                float sc[64], red[128];
                for (int t = 0; t < cnt; t++) {
                    float d = 0.f;
                    for (int e = 0; e < head_dim; e++)
                        d = fmaf(sq[e], or_bf2f(kb[(size_t)(start + t) * head_dim + e]), d);
                    sc[t] = d;
                }
                float mx = -INFINITY;
                for (int t = 0; t < cnt; t++) mx = fmaxf(mx, sc[t]);
                for (int t = 0; t < 128; t++) red[t] = t < cnt ? s2p_expf(sc[t] - mx) : 0.f;
                for (int t = 0; t < cnt; t++) sc[t] = red[t];
                for (int off = 64; off > 0; off >>= 1)
                    for (int t = 0; t < off; t++) red[t] += red[t + off];
                pm[sp] = mx;
                pl[sp] = red[0];
                for (int d = 0; d < head_dim; d++) {
                    float a = 0.f;
                    for (int j = 0; j < cnt; j++)
                        a = fmaf(sc[j], or_bf2f(vb[(size_t)(start + j) * head_dim + d]), a);
                    pa[(size_t)sp * 128 + d] = a;
                }
            }
            float M = -INFINITY;
            for (int sp = 0; sp < ns; sp++) M = fmaxf(M, pm[sp]);
            for (int d = 0; d < head_dim; d++) {
                float l = 0.f, a = 0.f;
                for (int sp = 0; sp < ns; sp++) {
                    if (pl[sp] == 0.f) continue;
                    const float wgt = s2p_expf(pm[sp] - M);
                    l = fmaf(pl[sp], wgt, l);
                    a = fmaf(pa[(size_t)sp * 128 + d], wgt, a);
                }
                out[((size_t)r * q_heads + h) * head_dim + d] = or_f2bf(a / l);
            }
            free(pm);
            free(pl);
            free(pa);
        }
    }
}

void or_attention_f64(const uint16_t* q, const uint16_t* kc,
                      const uint16_t* vc, double* out, int rows, int q_heads,
                      int kv_heads, int head_dim, int prefix,
                      const uint64_t* vis, int max_seq) {
    const int group = q_heads / kv_heads;
    const int maxlen = prefix + 64;
    double* s = (double*)malloc(sizeof(double) * (size_t)maxlen);
    for (int r = 0; r < rows; r++)
        for (int h = 0; h < q_heads; h++) {
            const int kvh = h / group;
            const uint16_t* kb = kc + (size_t)kvh * max_seq * head_dim;
            const uint16_t* vb = vc + (size_t)kvh * max_seq * head_dim;
            double mx = -INFINITY;
            const int lim = prefix + (vis ? 64 : r + 1);
            for (int j = 0; j < lim && j < max_seq; j++) {
                s[j] = -INFINITY;
                if (!visible(prefix, vis, r, j)) continue;
                double d = 0.0;
                for (int e = 0; e < head_dim; e++)
                    d += (double)or_bf2f(q[((size_t)r * q_heads + h) * head_dim + e]) *
                         (double)or_bf2f(kb[(size_t)j * head_dim + e]);
                s[j] = d / sqrt((double)head_dim);
                if (s[j] > mx) mx = s[j];
            }
            double l = 0.0;
            for (int d = 0; d < head_dim; d++) out[((size_t)r * q_heads + h) * head_dim + d] = 0.0;
            for (int j = 0; j < lim && j < max_seq; j++) {
                if (s[j] == -INFINITY) continue;
                const double p = exp(s[j] - mx);
                l += p;
                for (int d = 0; d < head_dim; d++)
                    out[((size_t)r * q_heads + h) * head_dim + d] +=
                        p * (double)or_bf2f(vb[(size_t)j * head_dim + d]);
            }
            for (int d = 0; d < head_dim; d++) out[((size_t)r * q_heads + h) * head_dim + d] /= l;
        }
    free(s);
}

/* ---- INT8 / INT4 KV cache (kernels.cu:510-946) ---------------------------
 * Cache: payload [kv_heads][max_seq][bw == 8 ? 128 : 64] bytes, scales f16
 * [kv_heads][max_seq][4] (one per 32-element group). */

/* k_kv_append8 (kernels.cu:516-581): per 32-group absmax / QMAX rounded
 * through f16, values x / scale rounded to nearest even and clamped to
 * +-QMAX (QMAX 127 for bw 8, 7 for bw 4; bw 4 packs element 2b in the low
 * nibble).  slot_arr == NULL: row r goes to slot pos0 + r of one cache;
 * else to slot slot_arr[r] of cache r (caches given as a pointer array). */
void or_kv_append8(const uint16_t* k, const uint16_t* v, int8_t* const* kcs,
                   int8_t* const* vcs, uint16_t* const* kss, uint16_t* const* vss,
                   int rows, int kv_heads, int pos0, const int32_t* slot_arr,
                   int max_seq, int bw) {
    const int hd = 128, el = bw == 8 ? 128 : 64, qmax = bw == 8 ? 127 : 7;
    for (int r = 0; r < rows; r++) {
        const int c = slot_arr ? r : 0;
        const int p = slot_arr ? slot_arr[r] : pos0 + r;
        for (int h = 0; h < kv_heads; h++)
            for (int kv = 0; kv < 2; kv++) {
                const uint16_t* src = (kv ? v : k) + ((size_t)r * kv_heads + h) * hd;
                int8_t* pay = (kv ? vcs : kcs)[c] + ((size_t)h * max_seq + p) * el;
                uint16_t* sc = (kv ? vss : kss)[c] + ((size_t)h * max_seq + p) * 4;
                for (int g = 0; g < 4; g++) {
                    float a = 0.f;
                    for (int e = 0; e < 32; e++) a = fmaxf(a, fabsf(or_bf2f(src[g * 32 + e])));
                    const uint16_t hs = or_f2h(a / (float)qmax);
                    const float s = or_h2f(hs);
                    int qv[32];
                    for (int e = 0; e < 32; e++) {
                        int q = s > 0.f ? (int)rintf(or_bf2f(src[g * 32 + e]) / s) : 0;
                        qv[e] = q < -qmax ? -qmax : (q > qmax ? qmax : q);
                    }
                    if (bw == 8) {
                        for (int e = 0; e < 32; e++) pay[g * 32 + e] = (int8_t)qv[e];
                    } else {
                        for (int e = 0; e < 32; e += 2)
                            pay[(g * 32 + e) / 2] = (int8_t)((qv[e] & 0xF) | ((qv[e + 1] & 0xF) << 4));
                    }
                    sc[g] = hs;
                }
            }
    }
}

/* element e of a cached row.  bw 4: the two's complement nibble the append
 * wrote (element 2b low).  The reference's decode expression
 * (int8_t)((nib << 4) >> 4) (kernels.cu:675, 717, 845, 906) sign-extends
 * only high nibbles: a negative low nibble reads back as 9..15.  The rule
 * here, and the GPU kernels, decode both nibbles as written. */
static float kv8_val(const int8_t* row, int e, int bw) {
    if (bw == 8) return (float)row[e];
    const uint8_t b = (uint8_t)row[e >> 1];
    const int nib = (e & 1) ? (b >> 4) : (b & 0xF);
    return (float)(nib >= 8 ? nib - 16 : nib);
}

/* k_attention8 (kernels.cu:614-722): causal single pass, row r attends
 * slots 0..pos0+r; per 128-slot tile the scores are sum_g fma(pp_g, ks_g)
 * with pp_g the in-order fma dot of the group, the tile max and sum are the
 * 128-lane trees, and V is dequantised as (p * vs_g) * v.  The rule's
 * s2p_expf replaces expf; l * corr + sum as one fma (nvcc contracts it). */
/* Slots visible to row r: [0, prefix) and the node slots of vis[r] (bit b =
 * slot prefix + b; its highest bit is the row itself), or, with vis NULL,
 * causal rows at prefix.. (kernels.cu:724-746).  The arithmetic of every
 * visible slot is the reference's; an invisible slot scores -inf, as one
 * beyond the length does. */
void or_attention8_vis(const uint16_t* q, const int8_t* kc, const int8_t* vc,
                       const uint16_t* ks, const uint16_t* vs, uint16_t* out, int rows,
                       int q_heads, int kv_heads, int prefix, const uint64_t* vis, int max_seq,
                       int bw) {
    const int hd = 128, el = bw == 8 ? 128 : 64, group = q_heads / kv_heads;
    float sq[128], sp[128], red[128], acc[128];
    for (int r = 0; r < rows; r++) {
        const int len = !vis ? prefix + r + 1 : (vis[r] ? prefix + 64 - __builtin_clzll(vis[r]) : prefix);
        for (int h = 0; h < q_heads; h++) {
            const int kvh = h / group;
            const int8_t* kb = kc + (size_t)kvh * max_seq * el;
            const int8_t* vb = vc + (size_t)kvh * max_seq * el;
            const uint16_t* ksb = ks + (size_t)kvh * max_seq * 4;
            const uint16_t* vsb = vs + (size_t)kvh * max_seq * 4;
            for (int e = 0; e < hd; e++)
                sq[e] = or_bf2f(q[((size_t)r * q_heads + h) * hd + e]) * ATTN_SCALE_128;
            float m = -INFINITY, l = 0.f;
            for (int d = 0; d < hd; d++) acc[d] = 0.f;
            for (int t0 = 0; t0 < len; t0 += 128) {
                float s[128];
                for (int t = 0; t < 128; t++) {
                    const int j = t0 + t;
                    s[t] = -INFINITY;
                    if (j < len && visible(prefix, vis, r, j)) {
                        float d = 0.f;
                        for (int g = 0; g < 4; g++) {
                            float pp = 0.f;
                            for (int e = 0; e < 32; e++)
                                pp = fmaf(sq[g * 32 + e], kv8_val(kb + (size_t)j * el, g * 32 + e, bw), pp);
                            d = fmaf(pp, or_h2f(ksb[(size_t)j * 4 + g]), d);
                        }
                        s[t] = d;
                    }
                }
                float tmax = -INFINITY;
                for (int t = 0; t < 128; t++) tmax = fmaxf(tmax, s[t]);
                const float m_new = fmaxf(m, tmax);
                const float corr = (m == -INFINITY) ? 0.f : s2p_expf(m - m_new);
                for (int t = 0; t < 128; t++) {
                    sp[t] = (s[t] == -INFINITY) ? 0.f : s2p_expf(s[t] - m_new);
                    red[t] = sp[t];
                }
                for (int off = 64; off > 0; off >>= 1)
                    for (int t = 0; t < off; t++) red[t] += red[t + off];
                l = fmaf(l, corr, red[0]);
                const int lim = len - t0 < 128 ? len - t0 : 128;
                for (int d = 0; d < hd; d++) {
                    float a = acc[d] * corr;
                    for (int j2 = 0; j2 < lim; j2++) {
                        const size_t j = (size_t)(t0 + j2);
                        a = fmaf(sp[j2] * or_h2f(vsb[j * 4 + (d >> 5)]), kv8_val(vb + j * el, d, bw), a);
                    }
                    acc[d] = a;
                }
                m = m_new;
            }
            for (int d = 0; d < hd; d++)
                out[((size_t)r * q_heads + h) * hd + d] = or_f2bf(acc[d] / l);
        }
    }
}

/* k_attention8 (kernels.cu:625-728): causal rows at pos0.. of one cache */
void or_attention8(const uint16_t* q, const int8_t* kc, const int8_t* vc,
                   const uint16_t* ks, const uint16_t* vs, uint16_t* out, int rows,
                   int q_heads, int kv_heads, int pos0, int max_seq, int bw) {
    or_attention8_vis(q, kc, vc, ks, vs, out, rows, q_heads, kv_heads, pos0, NULL, max_seq, bw);
}

/* Binary64 attention over the dequantised INT8 / INT4 cache (ground truth
 * for both the single-pass and the split decode kernels): row r of cache c
 * attends slots 0..len_c - 1, len_c = pos[r] + 1. */
void or_attention8_f64(const uint16_t* q, const int8_t* const* kcs, const int8_t* const* vcs,
                       const uint16_t* const* kss, const uint16_t* const* vss, double* out,
                       int rows, int q_heads, int kv_heads, const int32_t* pos, int max_seq,
                       int bw) {
    const int hd = 128, el = bw == 8 ? 128 : 64, group = q_heads / kv_heads;
    for (int r = 0; r < rows; r++) {
        const int len = pos[r] + 1;
        double* s = (double*)malloc((size_t)len * sizeof(double));
        for (int h = 0; h < q_heads; h++) {
            const int kvh = h / group;
            const int8_t* kb = kcs[r] + (size_t)kvh * max_seq * el;
            const int8_t* vb = vcs[r] + (size_t)kvh * max_seq * el;
            const uint16_t* ksb = kss[r] + (size_t)kvh * max_seq * 4;
            const uint16_t* vsb = vss[r] + (size_t)kvh * max_seq * 4;
            double mx = -INFINITY;
            for (int j = 0; j < len; j++) {
                double d = 0.0;
                for (int e = 0; e < hd; e++)
                    d += (double)or_bf2f(q[((size_t)r * q_heads + h) * hd + e]) *
                         kv8_val(kb + (size_t)j * el, e, bw) * or_h2f(ksb[(size_t)j * 4 + (e >> 5)]);
                s[j] = d / sqrt(128.0);
                if (s[j] > mx) mx = s[j];
            }
            double l = 0.0;
            for (int j = 0; j < len; j++) { s[j] = exp(s[j] - mx); l += s[j]; }
            for (int d = 0; d < hd; d++) {
                double a = 0.0;
                for (int j = 0; j < len; j++)
                    a += s[j] * kv8_val(vb + (size_t)j * el, d, bw) * or_h2f(vsb[(size_t)j * 4 + (d >> 5)]);
                out[((size_t)r * q_heads + h) * hd + d] = a / l;
            }
        }
        free(s);
    }
}


/* ------------------------------------------------------------- sampler */

#define N_SEM 4096
#define N_CAND 4097
#define CAND_EOS 4096
#define TOP_K 30
#define TOK_EOS 151645
#define SEM_START 151678
#define SEM_END 155773

static int g_libm = 0;
void or_set_libm(int on) { g_libm = on; }
static inline float rexp(float x) { return g_libm ? expf(x) : s2p_expf(x); }
static inline float rlog(float x) { return g_libm ? logf(x) : s2p_logf(x); }

static uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
static uint64_t xoshiro_next(uint64_t s[4]) {
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

/* s2p_sampling_defaults + s2ps_sampler_init (sampling.c:83-112) */
void or_state_init(or_state* st, float temperature, float top_p,
                   float rep_penalty, int window, uint64_t seed,
                   uint64_t entropy) {
    memset(st, 0, sizeof(*st));
    st->temperature = temperature < 0.f ? 0.f : temperature;
    st->top_p = (top_p <= 0.f || top_p > 1.f) ? 1.f : top_p;
    st->rep_penalty = rep_penalty > 0.f ? rep_penalty : 1.f;
    st->window = window > 0 ? window : 16;
    if (st->window > 64) st->window = 64;
    st->seeded = seed != 0;
    st->seed31 = (uint32_t)(seed & 0x7FFFFFFFULL);
    uint64_t sm = entropy ^ 0xD1B54A32D192ED03ULL;
    for (int i = 0; i < 4; i++) st->rng[i] = splitmix64(&sm);
}

static void gather_cand(float* cand, const uint16_t* row, const uint16_t* eos) {
    if (eos) {
        for (int i = 0; i < N_SEM; i++) cand[i] = or_bf2f(row[i]);
        cand[CAND_EOS] = or_bf2f(*eos);
    } else {
        for (int i = 0; i < N_SEM; i++) cand[i] = or_bf2f(row[SEM_START + i]);
        cand[CAND_EOS] = or_bf2f(row[TOK_EOS]);
    }
}

/* sampling.c:119-219 (everything up to the draw) */
int or_transform(const or_state* sp, const uint16_t* row_bf16,
                 const uint16_t* eos_bf16, int ti[30], float tv[30],
                 float p2[30]) {
    float cand[N_CAND];
    gather_cand(cand, row_bf16, eos_bf16);
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
                    int64_t t = last4[a];
                    last4[a] = last4[b];
                    last4[b] = t;
                }
        for (int a = 0; a < 3; a++)
            if (last4[a] == last4[a + 1]) use_ras = 1;
    }
    const float temp = use_ras ? 1.0f : sp->temperature;
    const float topp = use_ras ? 0.9f : sp->top_p;

    if (capped > 0) {
        int ridx[64];
        float rval[64];
        int rn = 0;
        for (int j = 0; j < capped; j++) {
            const int64_t tok = sp->prev[j];
            int ci;
            if (tok >= SEM_START && tok <= SEM_END) ci = (int)(tok - SEM_START);
            else if (tok == TOK_EOS) ci = CAND_EOS;
            else continue;
            const float v = cand[ci];
            ridx[rn] = ci;
            rval[rn] = v < 0.f ? v * sp->rep_penalty : v / sp->rep_penalty;
            rn++;
        }
        for (int j = 0; j < rn; j++) cand[ridx[j]] = rval[j];
    }

    int tn = 0;
    for (int i = 0; i < N_CAND; i++) {
        const float v = cand[i];
        if (tn == TOP_K && v <= tv[TOP_K - 1]) continue;
        int p = tn < TOP_K ? tn : TOP_K - 1;
        while (p > 0 && v > tv[p - 1]) {
            tv[p] = tv[p - 1];
            ti[p] = ti[p - 1];
            p--;
        }
        tv[p] = v;
        ti[p] = i;
        if (tn < TOP_K) tn++;
    }

    if (greedy) {
        for (int j = 0; j < TOP_K; j++) p2[j] = j == 0 ? 1.0f : 0.0f;
        return 1;
    }
    float e[TOP_K], sum = 0.f;
    const float m = tv[0];
    for (int j = 0; j < tn; j++) {
        e[j] = rexp(tv[j] - m);
        sum += e[j];
    }
    int masked[TOP_K] = {0};
    float cum = 0.f;
    for (int j = 0; j < tn; j++) {
        cum += e[j] / sum;
        if (j > 0 && cum > topp) masked[j] = 1;
    }
    const float t = temp < 1e-5f ? 1e-5f : temp;
    float s2 = 0.f;
    const float m2 = tv[0] / t;
    for (int j = 0; j < tn; j++) {
        p2[j] = masked[j] ? 0.f : rexp(tv[j] / t - m2);
        s2 += p2[j];
    }
    for (int j = 0; j < tn; j++) p2[j] /= s2;
    return 0;
}

/* seeded hash-Gumbel draw (sampling.c:221-243) over prob[0..29] */
static int gumbel_draw(const or_state* sp, const float* prob) {
    const uint64_t step_seed = ((uint64_t)sp->seed31 * 19349663ULL) ^ (sp->count * 73856093ULL);
    float best = -INFINITY;
    int choice = 0;
    for (int j = 0; j < TOP_K; j++) {
        const uint64_t hashed = (step_seed * 8589934591ULL) ^ ((uint64_t)j * 479001599ULL);
        float u = (float)(uint32_t)(hashed & 0xFFFFFFULL) / 16777216.0f;
        if (u < 1e-10f) u = 1e-10f;
        const float g = -rlog(-rlog(u));
        const float pert = rlog(prob[j] + 1e-10f) + g;
        if (pert > best) {
            best = pert;
            choice = j;
        }
    }
    return choice;
}

/* unseeded inverse-CDF draw (sampling.c:244-262) */
static int xoshiro_draw(or_state* sp, const float* prob) {
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

static int64_t cand_to_vocab(int ci) {
    return ci == CAND_EOS ? (int64_t)TOK_EOS : (int64_t)(SEM_START + ci);
}

static int vocab_to_cand(int64_t tok) {
    if (tok >= SEM_START && tok <= SEM_END) return (int)(tok - SEM_START);
    if (tok == TOK_EOS) return CAND_EOS;
    return -1;
}

/* sampling.c:269-281 */
void or_state_push(or_state* sp, int64_t tok) {
    if (tok == TOK_EOS) return;
    if (sp->count < (uint64_t)sp->window) {
        sp->prev[sp->count] = tok;
    } else {
        memmove(sp->prev, sp->prev + 1, (size_t)(sp->window - 1) * sizeof(int64_t));
        sp->prev[sp->window - 1] = tok;
    }
    sp->count++;
}

/* Test hooks: the draw primitives and both draws, exposed so that the tests
 * pin them against published vectors and hand-derived values. */
uint64_t or_splitmix64_next(uint64_t* s) { return splitmix64(s); }
uint64_t or_xoshiro_next(uint64_t s[4]) { return xoshiro_next(s); }
int or_gumbel_draw(const or_state* sp, const float* prob) { return gumbel_draw(sp, prob); }
int or_xoshiro_draw(or_state* sp, const float* prob) { return xoshiro_draw(sp, prob); }

int64_t or_sample(or_state* sp, const uint16_t* row_bf16,
                  const uint16_t* eos_bf16, int32_t* out_sem, int* out_eos) {
    int ti[TOP_K];
    float tv[TOP_K], p2[TOP_K];
    const int greedy = or_transform(sp, row_bf16, eos_bf16, ti, tv, p2);
    int choice = 0;
    if (!greedy) choice = sp->seeded ? gumbel_draw(sp, p2) : xoshiro_draw(sp, p2);
    const int64_t tok = cand_to_vocab(ti[choice]);
    if (tok == TOK_EOS) {
        *out_sem = 0;
        *out_eos = 1;
        return tok;
    }
    *out_sem = ti[choice];
    *out_eos = 0;
    or_state_push(sp, tok);
    return tok;
}

/* ----------------------------------------------------------- acceptance */

/* Counter-based uniform of the acceptance rule: splitmix64's finaliser of a
 * key built from (seed31, step count, slot), top 24 bits.  Slots: 64 + j for
 * the accept test of the j-th sibling tried at a node, 0..29 for the Gumbel
 * noise of a residual draw.  (The reference's own seeded hash derives all 30
 * Gumbel uniforms of a step from one 24-bit value, which does not sample p
 * without bias; it is kept only where the rule reproduces a reference draw.) */
static uint32_t rule_u24(const or_state* sp, uint32_t slot) {
    uint64_t z = ((uint64_t)sp->seed31 * 0x9E3779B97F4A7C15ULL) ^
                 (sp->count * 0xBF58476D1CE4E5B9ULL) ^
                 ((uint64_t)(slot + 1) * 0x94D049BB133111EBULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    z ^= z >> 31;
    return (uint32_t)(z >> 40);
}

uint32_t or_rule_u24(const or_state* sp, uint32_t slot) { return rule_u24(sp, slot); }

/* accept-test uniform: seeded -> rule_u24(slot 64 + j); unseeded -> top 24
 * bits of the next xoshiro output; greedy -> 0 */
static uint32_t accept_u24(or_state* sp, int j, int greedy) {
    if (greedy) return 0u;
    if (sp->seeded) return rule_u24(sp, 64u + (uint32_t)j);
    return (uint32_t)(xoshiro_next(sp->rng) >> 40);
}

/* residual draw: Gumbel-max over the nonzero entries (seeded, rule_u24
 * noise) or inverse CDF on xoshiro (unseeded) */
static int residual_draw(or_state* sp, const float* prob) {
    if (!sp->seeded) return xoshiro_draw(sp, prob);
    float best = -INFINITY;
    int choice = 0;
    for (int j = 0; j < TOP_K; j++) {
        if (!(prob[j] > 0.f)) continue;
        float u = (float)rule_u24(sp, (uint32_t)j) / 16777216.0f;
        if (u < 1e-10f) u = 1e-10f;
        const float g = -rlog(-rlog(u));
        const float pert = rlog(prob[j] + 1e-10f) + g;
        if (pert > best) {
            best = pert;
            choice = j;
        }
    }
    return choice;
}

static float prob_of(const int* ti, const float* p, int ci) {
    for (int j = 0; j < TOP_K; j++)
        if (ti[j] == ci) return p[j];
    return 0.f;
}

void or_accept_tree(or_state* st, const uint16_t* tgt, const uint16_t* tgt_eos,
                    const uint16_t* drf, const uint16_t* drf_eos,
                    int64_t row_stride, const int32_t* parent,
                    const int64_t* tok, int R, int32_t* path, int* n_acc,
                    int64_t* emitted, int* n_emit, const uint8_t* chain) {
    int v = 0;
    *n_acc = 0;
    *n_emit = 0;
    for (;;) {
        int pti[TOP_K], qti[TOP_K];
        float ptv[TOP_K], p[TOP_K], qtv[TOP_K], q[TOP_K];
        const int greedy = or_transform(st, tgt + (size_t)v * row_stride,
                                        tgt_eos ? tgt_eos + v : NULL, pti, ptv, p);
        int nchild = 0;
        for (int c = v + 1; c < R; c++)
            if (parent[c] == v) nchild++;
        int accepted = -1, rejected_any = 0;
        if (nchild > 0) {
            or_transform(st, drf + (size_t)v * row_stride, drf_eos ? drf_eos + v : NULL,
                         qti, qtv, q);
            int j = 0;
            for (int c = v + 1; c < R && accepted < 0; c++) {
                if (parent[c] != v) continue;
                const int ci = vocab_to_cand(tok[c]);
                const float pc = ci < 0 ? 0.f : prob_of(pti, p, ci);
                const float qc = ci < 0 ? 0.f : prob_of(qti, q, ci);
                const uint32_t u = accept_u24(st, j, greedy);
                /* u/2^24 * qc < pc, evaluated exactly in binary64 */
                if ((double)u * (double)qc < (double)pc * 16777216.0) {
                    accepted = c;
                    break;
                }
                /* reject: p <- normalize(max(0, p - q)) over p's ranks */
                rejected_any = 1;
                float rsd[TOP_K], z = 0.f;
                for (int k = 0; k < TOP_K; k++) {
                    const float d = p[k] - prob_of(qti, q, pti[k]);
                    rsd[k] = d > 0.f ? d : 0.f;
                    z += rsd[k];
                }
                if (z > 0.f)
                    for (int k = 0; k < TOP_K; k++) p[k] = rsd[k] / z;
                j++;
            }
        }
        if (accepted >= 0 && chain && !chain[accepted]) {
            /* the chain condition (docs/SPECULATIVE.md:26-41): the drafted
             * frame's residual codes differ from the fast-AR's on the true
             * hidden, so the node's own forward row is void: its token is
             * emitted (a valid sample of the target at that position), its
             * row is not committed and the walk ends without a bonus draw */
            emitted[(*n_emit)++] = tok[accepted];
            if (tok[accepted] != TOK_EOS) or_state_push(st, tok[accepted]);
            return;
        }
        if (accepted >= 0) {
            path[(*n_acc)++] = accepted;
            emitted[(*n_emit)++] = tok[accepted];
            if (tok[accepted] == TOK_EOS) return; /* generation ended */
            or_state_push(st, tok[accepted]);
            v = accepted;
            continue;
        }
        /* no child accepted: draw the corrected token from the residual; at
         * a leaf draw the bonus token exactly as s2ps_sample would */
        int choice = 0;
        if (greedy) {
            for (int k = 1; k < TOP_K; k++)
                if (p[k] > p[choice]) choice = k;
        } else if (rejected_any) {
            choice = residual_draw(st, p);
        } else {
            choice = st->seeded ? gumbel_draw(st, p) : xoshiro_draw(st, p);
        }
        const int64_t t = cand_to_vocab(pti[choice]);
        emitted[(*n_emit)++] = t;
        or_state_push(st, t);
        return;
    }
}

/* ------------------------------------------------------------- layer */

void or_linear_fwd(const or_linear* L, const uint16_t* x, uint16_t* y, int M) {
    if (L->G > 0)
        or_int4p_gemv(y, x, (const uint8_t*)L->w, (const uint16_t*)L->s, M, L->N, L->K, L->G);
    else
        or_int8_gemv(y, x, (const int8_t*)L->w, (const float*)L->s, M, L->N, L->K);
}

/* run_layer (slowar.c:156-260), single-session path with per-row RoPE
 * positions and KV slots prefix + r. */
void or_layer(const or_layer_w* lw, uint16_t* x, int rows, uint16_t* kc,
              uint16_t* vc, int max_seq, int prefix, const int32_t* pos,
              const uint64_t* vis) {
    const int dim = lw->wqkv.K;
    const int qw = 4096, kvw = 1024, ffn = lw->w2.K;
    const float eps = 1e-6f;
    uint16_t* xn = (uint16_t*)malloc(2 * (size_t)rows * dim);
    uint16_t* qkv = (uint16_t*)malloc(2 * (size_t)rows * (qw + 2 * kvw));
    uint16_t* q = (uint16_t*)malloc(2 * (size_t)rows * qw);
    uint16_t* k = (uint16_t*)malloc(2 * (size_t)rows * kvw);
    uint16_t* v = (uint16_t*)malloc(2 * (size_t)rows * kvw);
    uint16_t* att = (uint16_t*)malloc(2 * (size_t)rows * qw);
    uint16_t* proj = (uint16_t*)malloc(2 * (size_t)rows * dim);
    uint16_t* gu = (uint16_t*)malloc(2 * (size_t)rows * 2 * ffn);
    uint16_t* h = (uint16_t*)malloc(2 * (size_t)rows * ffn);
    int32_t* slots = (int32_t*)malloc(sizeof(int32_t) * rows);
    for (int r = 0; r < rows; r++) slots[r] = prefix + r;

    or_rms_norm(x, lw->attn_norm, xn, rows, dim, eps);
    or_linear_fwd(&lw->wqkv, xn, qkv, rows);
    or_qkv_split(qkv, q, k, v, rows, qw, kvw);
    if (lw->q_norm) { /* NULL: a layer without qk-norm (the fast-AR, fastar.cu:654) */
        or_qk_norm(q, lw->q_norm, rows, 32, 128, eps);
        or_qk_norm(k, lw->k_norm, rows, 8, 128, eps);
    }
    or_rope(q, rows, 32, 128, 0, pos, 1000000.0f);
    or_rope(k, rows, 8, 128, 0, pos, 1000000.0f);
    or_kv_append(k, v, kc, vc, rows, 8, 128, 0, slots, max_seq);
    or_attention(q, kc, vc, att, rows, 32, 8, 128, prefix, vis, max_seq);
    or_linear_fwd(&lw->wo, att, proj, rows);
    or_add(x, proj, (int64_t)rows * dim);
    or_rms_norm(x, lw->ffn_norm, xn, rows, dim, eps);
    or_linear_fwd(&lw->gate_up, xn, gu, rows);
    or_silu_mul(gu, h, rows, ffn);
    or_linear_fwd(&lw->w2, h, proj, rows);
    or_add(x, proj, (int64_t)rows * dim);

    free(xn); free(qkv); free(q); free(k); free(v); free(att);
    free(proj); free(gu); free(h); free(slots);
}

/* run_layer with the INT8 / INT4 KV cache (slowar.c:156-260 with the
 * quantised-cache kernels of kernels.cu:510-946): K (after qk-norm and RoPE,
 * rounded to bf16) and V are quantised on append at slots prefix + r, and
 * the attention reads the quantised cache with the rows' visibility.
 * append == 0 keeps the cache as given (slots prefix + r already hold codes
 * made elsewhere, e.g. by the GPU, so that a forward can be checked on the
 * same cache contents: a code that rounds the other way moves the result by
 * a whole quantisation step). */
void or_layer8(const or_layer_w* lw, uint16_t* x, int rows, int8_t* kc, int8_t* vc,
               uint16_t* ks, uint16_t* vs, int max_seq, int prefix, const int32_t* pos,
               const uint64_t* vis, int bw, int append) {
    const int dim = lw->wqkv.K;
    const int qw = 4096, kvw = 1024, ffn = lw->w2.K;
    const float eps = 1e-6f;
    uint16_t* xn = (uint16_t*)malloc(2 * (size_t)rows * dim);
    uint16_t* qkv = (uint16_t*)malloc(2 * (size_t)rows * (qw + 2 * kvw));
    uint16_t* q = (uint16_t*)malloc(2 * (size_t)rows * qw);
    uint16_t* k = (uint16_t*)malloc(2 * (size_t)rows * kvw);
    uint16_t* v = (uint16_t*)malloc(2 * (size_t)rows * kvw);
    uint16_t* att = (uint16_t*)malloc(2 * (size_t)rows * qw);
    uint16_t* proj = (uint16_t*)malloc(2 * (size_t)rows * dim);
    uint16_t* gu = (uint16_t*)malloc(2 * (size_t)rows * 2 * ffn);
    uint16_t* h = (uint16_t*)malloc(2 * (size_t)rows * ffn);

    or_rms_norm(x, lw->attn_norm, xn, rows, dim, eps);
    or_linear_fwd(&lw->wqkv, xn, qkv, rows);
    or_qkv_split(qkv, q, k, v, rows, qw, kvw);
    or_qk_norm(q, lw->q_norm, rows, 32, 128, eps);
    or_qk_norm(k, lw->k_norm, rows, 8, 128, eps);
    or_rope(q, rows, 32, 128, 0, pos, 1000000.0f);
    or_rope(k, rows, 8, 128, 0, pos, 1000000.0f);
    if (append) or_kv_append8(k, v, &kc, &vc, &ks, &vs, rows, 8, prefix, NULL, max_seq, bw);
    or_attention8_vis(q, kc, vc, ks, vs, att, rows, 32, 8, prefix, vis, max_seq, bw);
    or_linear_fwd(&lw->wo, att, proj, rows);
    or_add(x, proj, (int64_t)rows * dim);
    or_rms_norm(x, lw->ffn_norm, xn, rows, dim, eps);
    or_linear_fwd(&lw->gate_up, xn, gu, rows);
    or_silu_mul(gu, h, rows, ffn);
    or_linear_fwd(&lw->w2, h, proj, rows);
    or_add(x, proj, (int64_t)rows * dim);

    free(xn); free(qkv); free(q); free(k); free(v); free(att);
    free(proj); free(gu); free(h);
}

/* ---- the draft model ------------------------------------------------------ */

void or_gemm_bf16(const uint16_t* x, const uint16_t* w, uint16_t* y, int M, int N, int K) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.f;
            for (int k = 0; k < K; k++)
                acc = fmaf(or_bf2f(w[(size_t)n * K + k]), or_bf2f(x[(size_t)m * K + k]), acc);
            y[(size_t)m * N + n] = or_f2bf(acc);
        }
}

void or_gemm_bf16_f64(const uint16_t* x, const uint16_t* w, double* y, int M, int N, int K) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            double acc = 0.0;
            for (int k = 0; k < K; k++)
                acc += (double)or_bf2f(w[(size_t)n * K + k]) * (double)or_bf2f(x[(size_t)m * K + k]);
            y[(size_t)m * N + n] = acc;
        }
}

/* Op order of src/draft/draft.c:167-199: fuse, RMSNorm, wqkv, qk-norm (q, k),
 * RoPE at the state's position, KV append, causal attention over slots
 * 0..pos, wo + residual, RMSNorm, w1 / w3, SiLU-mul, w2 + residual, final
 * RMSNorm. */
void or_draft_step(const or_draft_w* d, uint16_t* kc, uint16_t* vc, int max_seq, int pos,
                   const uint16_t* h, const uint16_t* e, uint16_t* out) {
    const int D = 2560, F = 9728, QW = 4096, KVW = 1024;
    const float eps = 1e-6f;
    uint16_t* xcat = (uint16_t*)malloc(2 * (size_t)2 * D);
    uint16_t* x = (uint16_t*)malloc(2 * (size_t)D);
    uint16_t* a = (uint16_t*)malloc(2 * (size_t)D);
    uint16_t* qkv = (uint16_t*)malloc(2 * (size_t)(QW + 2 * KVW));
    uint16_t* att = (uint16_t*)malloc(2 * (size_t)QW);
    uint16_t* gu = (uint16_t*)malloc(2 * (size_t)2 * F);
    uint16_t* ffn = (uint16_t*)malloc(2 * (size_t)F);
    memcpy(xcat, h, 2 * (size_t)D);
    memcpy(xcat + D, e, 2 * (size_t)D);
    or_gemm_bf16(xcat, d->fuse, x, 1, D, 2 * D);
    or_rms_norm(x, d->attn_norm, a, 1, D, eps);
    or_gemm_bf16(a, d->wqkv, qkv, 1, QW + 2 * KVW, D);
    uint16_t* q = qkv;
    uint16_t* k = qkv + QW;
    uint16_t* v = k + KVW;
    or_qk_norm(q, d->q_norm, 1, 32, 128, eps);
    or_qk_norm(k, d->k_norm, 1, 8, 128, eps);
    or_rope(q, 1, 32, 128, pos, NULL, 1000000.0f);
    or_rope(k, 1, 8, 128, pos, NULL, 1000000.0f);
    or_kv_append(k, v, kc, vc, 1, 8, 128, pos, NULL, max_seq);
    or_attention(q, kc, vc, att, 1, 32, 8, 128, pos, NULL, max_seq);
    or_gemm_bf16(att, d->wo, a, 1, D, QW);
    or_add(x, a, D);
    or_rms_norm(x, d->ffn_norm, a, 1, D, eps);
    or_gemm_bf16(a, d->w1, gu, 1, F, D);
    or_gemm_bf16(a, d->w3, gu + F, 1, F, D);
    or_silu_mul(gu, ffn, 1, F);
    or_gemm_bf16(ffn, d->w2, a, 1, D, F);
    or_add(x, a, D);
    or_rms_norm(x, d->final_norm, out, 1, D, eps);
    free(xcat); free(x); free(a); free(qkv); free(att); free(gu); free(ffn);
}

/* ---- the fast-AR frame (src/fastar/fastar.cu:726-789, fa_run_layers
 * :647-723): prime the depth-11 cache at position 0 on the final-normed
 * hidden (logits discarded), then for cb = 1..9: x = emb[code] (the previous
 * code, clamped to 0..4095; cb 1 takes the semantic code), the 4 layers at
 * position cb (no qk-norm), RMSNorm, the untied head, argmax (largest
 * value, lowest index on ties, kernels.cu:1326-1357). ---- */
void or_fastar_frame(const or_fa_w* w, const uint16_t* hidden, int sem, int32_t* codes,
                     uint16_t* logits) {
    const int dim = 2560, seq = 11, ncb = 10, cbs = 4096;
    uint16_t* kc = (uint16_t*)calloc((size_t)4 * 8 * seq * 128, 2);
    uint16_t* vc = (uint16_t*)calloc((size_t)4 * 8 * seq * 128, 2);
    uint16_t* x = (uint16_t*)malloc((size_t)dim * 2);
    uint16_t* xn = (uint16_t*)malloc((size_t)dim * 2);
    uint16_t* lg = (uint16_t*)malloc((size_t)cbs * 2);
    const size_t plane = (size_t)8 * seq * 128;
    memcpy(x, hidden, (size_t)dim * 2);
    for (int p = 0; p < ncb; p++) {
        if (p > 0) {
            int c = p == 1 ? sem : codes[p - 2];
            c = c < 0 ? 0 : (c >= cbs ? cbs - 1 : c);
            memcpy(x, w->emb + (size_t)c * dim, (size_t)dim * 2);
        }
        const int32_t pos = p;
        for (int l = 0; l < 4; l++)
            or_layer(&w->layers[l], x, 1, kc + l * plane, vc + l * plane, seq, p, &pos, NULL);
        if (p == 0) continue;
        or_rms_norm(x, w->norm, xn, 1, dim, 1e-6f);
        or_linear_fwd(&w->output, xn, lg, 1);
        int best = 0;
        float bv = or_bf2f(lg[0]);
        for (int i = 1; i < cbs; i++) {
            const float v = or_bf2f(lg[i]);
            if (v > bv) {
                bv = v;
                best = i;
            }
        }
        codes[p - 1] = best;
        if (logits) memcpy(logits + (size_t)(p - 1) * cbs, lg, (size_t)cbs * 2);
    }
    free(kc);
    free(vc);
    free(x);
    free(xn);
    free(lg);
}

/* s2pfa_vq_embed_add (fastar.cu:104-127): rows[t] += bf16(f32 sum over the
 * ten codebooks, in order, of cb_emb[cb * 4096 + clamp(code)]). */
void or_vq_embed_add(const uint16_t* cb_emb, const int32_t* codes, int T, uint16_t* rows) {
    const int dim = 2560, ncb = 10, cbs = 4096;
    for (int t = 0; t < T; t++)
        for (int d = 0; d < dim; d++) {
            float acc = 0.f;
            for (int cb = 0; cb < ncb; cb++) {
                int c = codes[(size_t)cb * T + t];
                c = c < 0 ? 0 : (c >= cbs ? cbs - 1 : c);
                acc += or_bf2f(cb_emb[((size_t)cb * cbs + c) * dim + d]);
            }
            uint16_t* o = rows + (size_t)t * dim + d;
            *o = or_f2bf(or_bf2f(*o) + or_bf2f(or_f2bf(acc)));
        }
}
