/* s2pro MI355X — per-wave bodies of the fused verify primitives, shared by
 * the prims.hip kernels and the persistent verify kernel.  Activations and
 * the appended K/V go through the coherent accessors of coh.h (the K/V rows
 * are read by other workgroups of the same launch).  Rounding points follow
 * kernels.cu:4-17 (see prims.hip). */
#ifndef S2P_PRIMS_DEV_H
#define S2P_PRIMS_DEV_H

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "coh.h"
#include "common.h"
#include "prims_internal.h"

/* cos/sin (bf16-rounded, as float) of pair i at position p */
S2P_DEV void rope_cs(int p, int i, int head_dim, float base, float* c, float* s) {
#pragma clang fp contract(off)
    const float ex = __fdiv_rn((float)(2 * i), (float)head_dim);
    const float pw = (float)pow((double)base, (double)ex);
    const float inv = __fdiv_rn(1.0f, pw);
    const float ang = __fmul_rn((float)p, inv);
    *c = bf2f(f2bf((float)cos((double)ang)));
    *s = bf2f(f2bf((float)sin((double)ang)));
}

/* qk-norm + RoPE arithmetic of one (row, head), lane = elements lane and
 * lane + 64 (v0, v1) with norm weights w0, w1 and the (cos, sin) of their
 * pairs; the partner of element e (e ^ 1) lives in lane ^ 1.  norm false:
 * RoPE of the values as they are (a model without qk-norm, the fast-AR). */
S2P_DEV void qkrope_math(float v0, float v1, uint16_t w0, uint16_t w1, float c0, float s0,
                         float c1, float s1, float eps, int lane, float* o0, float* o1,
                         bool norm = true) {
#pragma clang fp contract(off)
    if (norm) {
        float s = fmaf(v0, v0, 0.f) + fmaf(v1, v1, 0.f);
        s = wave_sum_down(s);
        s = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(s), 0)); /* lane 0's total */
        const float inv = rsqrt_rule(s / 128.0f + eps);
        v0 = bf2f(f2bf(__fmul_rn(__fmul_rn(v0, inv), bf2f(w0))));
        v1 = bf2f(f2bf(__fmul_rn(__fmul_rn(v1, inv), bf2f(w1))));
    }
    const float pv0 = dpp_f<0xB1>(v0), pv1 = dpp_f<0xB1>(v1); /* lane ^ 1 */
    if ((lane & 1) == 0) {
        *o0 = __fsub_rn(__fmul_rn(v0, c0), __fmul_rn(pv0, s0)); /* x0' */
        *o1 = __fsub_rn(__fmul_rn(v1, c1), __fmul_rn(pv1, s1));
    } else {
        *o0 = __fadd_rn(__fmul_rn(v0, c0), __fmul_rn(pv0, s0)); /* x1' */
        *o1 = __fadd_rn(__fmul_rn(v1, c1), __fmul_rn(pv1, s1));
    }
}

/* element n of fused qkv row `row` (the row width is 6144): the merged
 * bf16 value, from the rows or summed from the deferred partials */
template <bool COH>
S2P_DEV uint16_t qkv_elem(const uint16_t* qkv, const S2pQkvParts& p, int row, int n) {
#pragma clang fp contract(off)
    if (p.splits > 0) {
        const float* e = p.part + ((size_t)row * p.nrb + (n >> 6)) * 64 + (n & 63);
        const size_t stride = (size_t)p.M * p.nrb * 64;
        float s = 0.f;
        if (p.splits <= 8) { /* every load in flight before the first add */
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = e[(size_t)min(k, p.splits - 1) * stride];
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (k < p.splits) s += v[k];
        } else {
            for (int k = 0; k < p.splits; k++) s += e[(size_t)k * stride];
        }
        return f2bf(s);
    }
    return COH ? coh_ld16(qkv + (size_t)row * 6144 + n) : qkv[(size_t)row * 6144 + n];
}

/* qk-norm + RoPE of one (row, head) of the fused qkv output, one wave:
 * q heads 0..31 go to q_out, k heads 32..39 (with the matching v head) to
 * the row's KV slot of `layer` (kernels.cu:81-109, 114-168, 172-222). */
template <bool TAB>
S2P_DEV void qkrope_item_t(const uint16_t* qkv, uint16_t* q_out, const uint16_t* qn_w,
                           const uint16_t* kn_w, const S2pRowPlan& plan, int layer, float eps,
                           float base, int row, int head, int lane, const float* rope_tab,
                           S2pQkvParts parts = S2pQkvParts{nullptr, 0, 0, 0}) {
#pragma clang fp contract(off)
    const int QH = 32, KVH = 8, HD = 128;
    const int qkv_w = (QH + 2 * KVH) * HD;
    const bool is_q = head < QH;
    const int kh = head - QH;
    const int n0 = is_q ? head * HD : QH * HD + kh * HD;
    const uint16_t* nw = is_q ? qn_w : kn_w;
    const uint16_t r0 = qkv_elem<true>(qkv, parts, row, n0 + lane);
    const uint16_t r1 = qkv_elem<true>(qkv, parts, row, n0 + lane + 64);
    if (parts.splits > 0) { /* the merged row, as the merge would have stored it */
        coh_st16((uint16_t*)qkv + (size_t)row * qkv_w + n0 + lane, r0);
        coh_st16((uint16_t*)qkv + (size_t)row * qkv_w + n0 + lane + 64, r1);
    }
    const float v0 = bf2f(r0), v1 = bf2f(r1);
    /* RoPE: element e = lane + 64*slot, pair e >> 1 */
    float cs[2][2];
#pragma unroll
    for (int slot = 0; slot < 2; slot++) {
        const int e = lane + 64 * slot;
        if constexpr (TAB) { /* (cos, sin) of (row, pair), precomputed with rope_cs */
            cs[slot][0] = coh_ldf(rope_tab + ((size_t)row * 64 + (e >> 1)) * 2);
            cs[slot][1] = coh_ldf(rope_tab + ((size_t)row * 64 + (e >> 1)) * 2 + 1);
        } else {
            rope_cs(plan.pos[row], e >> 1, HD, base, &cs[slot][0], &cs[slot][1]);
        }
    }
    float o[2];
    qkrope_math(v0, v1, nw[lane], nw[lane + 64], cs[0][0], cs[0][1], cs[1][0], cs[1][1], eps,
                lane, &o[0], &o[1]);
    if (is_q) {
        uint16_t* dst = q_out + (size_t)row * QH * HD + head * HD;
        coh_st16(dst + lane, f2bf(o[0]));
        coh_st16(dst + lane + 64, f2bf(o[1]));
    } else {
        uint16_t* kvb = (uint16_t*)plan.kv[plan.sess[row]] + (size_t)layer * plan.layer_stride;
        const size_t slot = (size_t)plan.slot[row];
        uint16_t* kd = kvb + ((size_t)kh * plan.max_seq + slot) * HD;
        uint16_t* vd = kvb + ((size_t)(KVH + kh) * plan.max_seq + slot) * HD;
        coh_st16(kd + lane, f2bf(o[0]));
        coh_st16(kd + lane + 64, f2bf(o[1]));
        const int nv = (QH + KVH) * HD + kh * HD;
        const uint16_t w0 = qkv_elem<true>(qkv, parts, row, nv + lane);
        const uint16_t w1 = qkv_elem<true>(qkv, parts, row, nv + lane + 64);
        if (parts.splits > 0) {
            coh_st16((uint16_t*)qkv + (size_t)row * qkv_w + nv + lane, w0);
            coh_st16((uint16_t*)qkv + (size_t)row * qkv_w + nv + lane + 64, w1);
        }
        coh_st16(vd + lane, w0);
        coh_st16(vd + lane + 64, w1);
    }
}

/* cos/sin computed in place (TAB = false) or read from the plan's table */
S2P_DEV void qkrope_item(const uint16_t* qkv, uint16_t* q_out, const uint16_t* qn_w,
                         const uint16_t* kn_w, const S2pRowPlan& plan, int layer, float eps,
                         float base, int row, int head, int lane) {
    qkrope_item_t<false>(qkv, q_out, qn_w, kn_w, plan, layer, eps, base, row, head, lane, nullptr);
}

/* RoPE table entry (row, pair i) for head_dim 128: the rule's cos/sin of
 * position pos[row], layer-independent, so computed once per forward. */
S2P_DEV void rope_tab_item(const S2pRowPlan& plan, float base, float* tab, int row, int i) {
    float c, sn;
    rope_cs(plan.pos[row], i, 128, base, &c, &sn);
    coh_stf(tab + ((size_t)row * 64 + i) * 2, c);
    coh_stf(tab + ((size_t)row * 64 + i) * 2 + 1, sn);
}

/* Residual stream init of one 64-column block of row m: x = x_in and the
 * sums of squares of its four 16-column blocks (layout [width/16][GEMV_MAX_M
 * = 128]). */
S2P_DEV void resid_init_item(const uint16_t* xin, uint16_t* x, float* ssq, int width, int blk,
                             int m, int lane) {
    const size_t i = (size_t)m * width + blk * 64 + lane;
    const uint16_t v = xin[i];
    coh_st16(x + i, v);
    const float f = bf2f(v);
    const float t = sum_lanes16(f * f);
    if ((lane & 15) == 0) coh_stf(ssq + (size_t)(blk * 4 + (lane >> 4)) * 128 + m, t);
}

#endif
