"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker.  The shipped library never loads
it.  All arrays are numpy; bf16/f16 travel as uint16 bit patterns.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

P = ctypes.c_void_p
I = ctypes.c_int
I64 = ctypes.c_int64
F = ctypes.c_float
U64 = ctypes.c_uint64


class OrState(ctypes.Structure):
    """Byte layout of s2ps_dev_state (reference src/slowar/slowar_kernels.h:132-142)."""
    _fields_ = [("prev", ctypes.c_int64 * 64), ("count", ctypes.c_uint64),
                ("rng", ctypes.c_uint64 * 4), ("temperature", F), ("top_p", F),
                ("rep_penalty", F), ("window", ctypes.c_int32),
                ("seeded", ctypes.c_int32), ("seed31", ctypes.c_uint32),
                ("pad_", ctypes.c_uint32)]


_SIGS = {
    "or_bf2f": (F, [ctypes.c_uint16]),
    "or_f2bf": (ctypes.c_uint16, [F]),
    "or_h2f": (F, [ctypes.c_uint16]),
    "or_f2h": (ctypes.c_uint16, [F]),
    "or_bf16_to_f32": (None, [P, P, I64]),
    "or_f32_to_bf16": (None, [P, P, I64]),
    "or_int8_quant": (None, [P, P, P, I, I]),
    "or_intq_quant": (None, [P, P, P, I, I, I, I, I]),
    "or_int4_pack": (None, [P, P, I, I]),
    "or_int8_dequant": (None, [P, P, P, I, I]),
    "or_intq_dequant": (None, [P, P, P, I, I, I]),
    "or_int4p_dequant": (None, [P, P, P, I, I, I]),
    "or_int8_gemv": (None, [P, P, P, P, I, I, I]),
    "or_intq_gemv": (None, [P, P, P, P, I, I, I, I]),
    "or_int4p_gemv": (None, [P, P, P, P, I, I, I, I]),
    "or_int8_gemv_f64": (None, [P, P, P, P, I, I, I]),
    "or_int4p_gemv_f64": (None, [P, P, P, P, I, I, I, I]),
    "or_rms_norm": (None, [P, P, P, I, I, F]),
    "or_qk_norm": (None, [P, P, I, I, I, F]),
    "or_rope": (None, [P, I, I, I, I, P, F]),
    "or_kv_append": (None, [P, P, P, P, I, I, I, I, P, I]),
    "or_qkv_split": (None, [P, P, P, P, I, I, I]),
    "or_silu_mul": (None, [P, P, I, I]),
    "or_add": (None, [P, P, I64]),
    "or_attention": (None, [P, P, P, P, I, I, I, I, I, P, I]),
    "or_attention_split": (None, [P, P, P, P, I, I, I, I, I, I]),
    "or_attention_f64": (None, [P, P, P, P, I, I, I, I, I, P, I]),
    "or_kv_append8": (None, [P, P, P, P, P, P, I, I, I, P, I, I]),
    "or_attention8": (None, [P, P, P, P, P, P, I, I, I, I, I, I]),
    "or_attention8_f64": (None, [P, P, P, P, P, P, I, I, I, P, I, I]),
    "or_attention8_vis": (None, [P, P, P, P, P, P, I, I, I, I, P, I, I]),
    "or_state_init": (None, [P, F, F, F, I, U64, U64]),
    "or_set_libm": (None, [I]),
    "or_transform": (I, [P, P, P, P, P, P]),
    "or_sample": (ctypes.c_int64, [P, P, P, P, P]),
    "or_state_push": (None, [P, ctypes.c_int64]),
    "or_splitmix64_next": (U64, [P]),
    "or_xoshiro_next": (U64, [P]),
    "or_gumbel_draw": (I, [P, P]),
    "or_xoshiro_draw": (I, [P, P]),
    "or_rule_u24": (ctypes.c_uint32, [P, ctypes.c_uint32]),
    "or_accept_tree": (None, [P, P, P, P, P, I64, P, P, I, P, P, P, P, P]),
    "or_linear_fwd": (None, [P, P, P, I]),
    "or_layer": (None, [P, P, I, P, P, I, I, P, P]),
    "or_layer8": (None, [P, P, I, P, P, P, P, I, I, P, P, I, I]),
    "or_gemm_bf16": (None, [P, P, P, I, I, I]),
    "or_gemm_bf16_f64": (None, [P, P, P, I, I, I]),
    "or_draft_step": (None, [P, P, P, I, I, P, P, P]),
    "or_fastar_frame": (None, [P, P, I, P, P]),
    "or_vq_embed_add": (None, [P, P, I, P]),
}


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            subprocess.check_call(["make", "-s", "-C", _HERE])
        _LIB = ctypes.CDLL(path)
        for name, (res, args) in _SIGS.items():
            fn = getattr(_LIB, name)
            fn.restype = res
            fn.argtypes = args
    return _LIB


def ptr(a):
    if a is None:
        return None
    if isinstance(a, ctypes.Structure):
        return ctypes.addressof(a)
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


# ---------------------------------------------------------------- numerics
def f32_to_bf16(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().or_f32_to_bf16(ptr(a), ptr(out), a.size)
    return out


def bf16_to_f32(a):
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, np.float32)
    lib().or_bf16_to_f32(ptr(a), ptr(out), a.size)
    return out


def f16_bits_to_f32(a):
    return np.ascontiguousarray(a, np.uint16).view(np.float16).astype(np.float32)


# ---------------------------------------------------------------- formats
def int8_quant(w_bf16, N, K):
    q = np.empty((N, K), np.int8)
    s = np.empty(N, np.float32)
    lib().or_int8_quant(ptr(q), ptr(s), ptr(w_bf16), N, K)
    return q, s


def intq_quant(w_bf16, N, K, G=32, levels=7, mse=1):
    q = np.empty((N, K), np.int8)
    s = np.empty((N, K // G), np.uint16)
    lib().or_intq_quant(ptr(q), ptr(s), ptr(w_bf16), N, K, G, levels, mse)
    return q, s


def int4_pack(q, N, K):
    p = np.empty((N, K // 2), np.uint8)
    lib().or_int4_pack(ptr(p), ptr(np.ascontiguousarray(q, np.int8)), N, K)
    return p


def int4p_dequant(p, s, N, K, G=32):
    o = np.empty((N, K), np.uint16)
    lib().or_int4p_dequant(ptr(o), ptr(p), ptr(s), N, K, G)
    return o


# ---------------------------------------------------------------- GEMVs
def int4p_gemv(x, p, s, M, N, K, G=32):
    y = np.empty((M, N), np.uint16)
    lib().or_int4p_gemv(ptr(y), ptr(x), ptr(p), ptr(s), M, N, K, G)
    return y


def intq_gemv(x, q, s, M, N, K, G=32):
    y = np.empty((M, N), np.uint16)
    lib().or_intq_gemv(ptr(y), ptr(x), ptr(q), ptr(s), M, N, K, G)
    return y


def int8_gemv(x, q, s, M, N, K):
    y = np.empty((M, N), np.uint16)
    lib().or_int8_gemv(ptr(y), ptr(x), ptr(q), ptr(s), M, N, K)
    return y


def int4p_gemv_f64(x, p, s, M, N, K, G=32):
    y = np.empty((M, N), np.float64)
    lib().or_int4p_gemv_f64(ptr(y), ptr(x), ptr(p), ptr(s), M, N, K, G)
    return y


def int8_gemv_f64(x, q, s, M, N, K):
    y = np.empty((M, N), np.float64)
    lib().or_int8_gemv_f64(ptr(y), ptr(x), ptr(q), ptr(s), M, N, K)
    return y


# ---------------------------------------------------------------- primitives
def rms_norm(x, w, rows, width, eps=1e-6):
    y = np.empty((rows, width), np.uint16)
    lib().or_rms_norm(ptr(x), ptr(w), ptr(y), rows, width, eps)
    return y


def qk_norm(qk, w, rows, heads, hd=128, eps=1e-6):
    out = np.array(qk, np.uint16, copy=True, order="C")
    lib().or_qk_norm(ptr(out), ptr(w), rows, heads, hd, eps)
    return out


def rope(x, rows, heads, hd, pos0=0, pos=None, base=1000000.0):
    out = np.array(x, np.uint16, copy=True, order="C")
    pa = None if pos is None else np.ascontiguousarray(pos, np.int32)
    lib().or_rope(ptr(out), rows, heads, hd, pos0, ptr(pa), base)
    return out


def silu_mul(gu, rows, ffn):
    h = np.empty((rows, ffn), np.uint16)
    lib().or_silu_mul(ptr(gu), ptr(h), rows, ffn)
    return h


def add(y, x):
    out = np.array(y, np.uint16, copy=True, order="C")
    lib().or_add(ptr(out), ptr(np.ascontiguousarray(x, np.uint16)), out.size)
    return out


def attention(q, kc, vc, rows, qh, kvh, hd, prefix, max_seq, vis=None):
    out = np.empty((rows, qh * hd), np.uint16)
    va = None if vis is None else np.ascontiguousarray(vis, np.uint64)
    lib().or_attention(ptr(q), ptr(kc), ptr(vc), ptr(out), rows, qh, kvh, hd, prefix,
                       ptr(va), max_seq)
    return out


def attention_split(q, kc, vc, rows, qh, kvh, hd, prefix, max_seq):
    out = np.empty((rows, qh * hd), np.uint16)
    lib().or_attention_split(ptr(q), ptr(kc), ptr(vc), ptr(out), rows, qh, kvh, hd,
                             prefix, max_seq)
    return out


def attention_f64(q, kc, vc, rows, qh, kvh, hd, prefix, max_seq, vis=None):
    out = np.empty((rows, qh * hd), np.float64)
    va = None if vis is None else np.ascontiguousarray(vis, np.uint64)
    lib().or_attention_f64(ptr(q), ptr(kc), ptr(vc), ptr(out), rows, qh, kvh, hd, prefix,
                           ptr(va), max_seq)
    return out


# ------------------------------------------------------ INT8 / INT4 KV cache
def _parr(arrs):
    return (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])


def kv_append8(k, v, kcs, vcs, kss, vss, rows, kvh, pos0, slots, max_seq, bw):
    """In place on the host caches (lists of numpy arrays: int8 payloads,
    uint16 f16 scales); slots None: rows at pos0.. of cache 0."""
    sa = None if slots is None else np.ascontiguousarray(slots, np.int32)
    lib().or_kv_append8(ptr(k), ptr(v), _parr(kcs), _parr(vcs), _parr(kss), _parr(vss), rows,
                        kvh, pos0, ptr(sa), max_seq, bw)


def attention8(q, kc, vc, ks, vs, rows, qh, kvh, pos0, max_seq, bw):
    out = np.empty((rows, qh * 128), np.uint16)
    lib().or_attention8(ptr(q), ptr(kc), ptr(vc), ptr(ks), ptr(vs), ptr(out), rows, qh, kvh,
                        pos0, max_seq, bw)
    return out


def attention8_vis(q, kc, vc, ks, vs, rows, qh, kvh, prefix, vis, max_seq, bw):
    out = np.empty((rows, qh * 128), np.uint16)
    va = None if vis is None else np.ascontiguousarray(vis, np.uint64)
    lib().or_attention8_vis(ptr(q), ptr(kc), ptr(vc), ptr(ks), ptr(vs), ptr(out), rows, qh, kvh,
                            prefix, ptr(va), max_seq, bw)
    return out


def attention8_f64(q, kcs, vcs, kss, vss, rows, qh, kvh, pos, max_seq, bw):
    out = np.empty((rows, qh * 128), np.float64)
    pa = np.ascontiguousarray(pos, np.int32)
    lib().or_attention8_f64(ptr(q), _parr(kcs), _parr(vcs), _parr(kss), _parr(vss), ptr(out),
                            rows, qh, kvh, ptr(pa), max_seq, bw)
    return out


# ---------------------------------------------------------------- sampler
def state(temperature=0.8, top_p=0.8, rep_penalty=1.1, window=16, seed=0, entropy=0):
    st = OrState()
    lib().or_state_init(ptr(st), temperature, top_p, rep_penalty, window, seed, entropy)
    return st


def copy_state(st):
    c = OrState()
    ctypes.memmove(ctypes.addressof(c), ctypes.addressof(st), ctypes.sizeof(OrState))
    return c


def set_libm(on):
    lib().or_set_libm(1 if on else 0)


def transform(st, row, eos=None):
    ti = np.empty(30, np.int32)
    tv = np.empty(30, np.float32)
    p2 = np.empty(30, np.float32)
    e = None if eos is None else np.ascontiguousarray([eos], np.uint16)
    g = lib().or_transform(ptr(st), ptr(np.ascontiguousarray(row, np.uint16)), ptr(e),
                           ptr(ti), ptr(tv), ptr(p2))
    return ti, tv, p2, g


def sample(st, row, eos=None):
    sem = ctypes.c_int32()
    iseos = ctypes.c_int()
    e = None if eos is None else np.ascontiguousarray([eos], np.uint16)
    tok = lib().or_sample(ptr(st), ptr(np.ascontiguousarray(row, np.uint16)), ptr(e),
                          ctypes.addressof(sem), ctypes.addressof(iseos))
    return tok, sem.value, iseos.value


def state_push(st, tok):
    lib().or_state_push(ptr(st), int(tok))


def accept_tree(st, tgt, drf, parent, tok, tgt_eos=None, drf_eos=None, chain=None):
    """tgt/drf: [R, stride] uint16; parent/tok: [R]; returns (path, emitted)."""
    tgt = np.ascontiguousarray(tgt, np.uint16)
    drf = np.ascontiguousarray(drf, np.uint16)
    R = tgt.shape[0]
    assert tgt.shape == drf.shape
    par = np.ascontiguousarray(parent, np.int32)
    tk = np.ascontiguousarray(tok, np.int64)
    path = np.zeros(R, np.int32)
    emitted = np.zeros(R + 1, np.int64)
    nacc = ctypes.c_int()
    nemit = ctypes.c_int()
    te = None if tgt_eos is None else np.ascontiguousarray(tgt_eos, np.uint16)
    de = None if drf_eos is None else np.ascontiguousarray(drf_eos, np.uint16)
    ch = None if chain is None else np.ascontiguousarray(chain, np.uint8)
    lib().or_accept_tree(ptr(st), ptr(tgt), ptr(te), ptr(drf), ptr(de), tgt.shape[1],
                         ptr(par), ptr(tk), R, ptr(path), ctypes.addressof(nacc),
                         ptr(emitted), ctypes.addressof(nemit), ptr(ch))
    return path[: nacc.value].copy(), emitted[: nemit.value].copy()


# ---------------------------------------------------------------- layer
class OrLinear(ctypes.Structure):
    _fields_ = [("w", P), ("s", P), ("N", I), ("K", I), ("G", I)]


class OrLayerW(ctypes.Structure):
    _fields_ = [("wqkv", OrLinear), ("wo", OrLinear), ("gate_up", OrLinear),
                ("w2", OrLinear), ("attn_norm", P), ("ffn_norm", P), ("q_norm", P),
                ("k_norm", P)]


def make_linear(w, s, N, K, G):
    return OrLinear(ptr(w), ptr(s), N, K, G)


def linear_fwd(lin, x, M):
    y = np.empty((M, lin.N), np.uint16)
    lib().or_linear_fwd(ctypes.addressof(lin), ptr(x), ptr(y), M)
    return y


def layer(lw, x, rows, kc, vc, max_seq, prefix, pos, vis=None):
    """In place on x, kc, vc."""
    pa = np.ascontiguousarray(pos, np.int32)
    va = None if vis is None else np.ascontiguousarray(vis, np.uint64)
    lib().or_layer(ctypes.addressof(lw), ptr(x), rows, ptr(kc), ptr(vc), max_seq, prefix,
                   ptr(pa), ptr(va))


def layer8(lw, x, rows, kc, vc, ks, vs, max_seq, prefix, pos, vis, bw, append=True):
    """In place on x and the quantised caches (kc, vc int8; ks, vs uint16);
    append=False reads the rows' codes from the cache instead of writing them."""
    pa = np.ascontiguousarray(pos, np.int32)
    va = None if vis is None else np.ascontiguousarray(vis, np.uint64)
    lib().or_layer8(ctypes.addressof(lw), ptr(x), rows, ptr(kc), ptr(vc), ptr(ks), ptr(vs),
                    max_seq, prefix, ptr(pa), ptr(va), bw, 1 if append else 0)


class OrFaW(ctypes.Structure):
    _fields_ = [("layers", OrLayerW * 4), ("norm", P), ("output", OrLinear), ("emb", P)]


def fastar_frame(faw, hidden, sem):
    """One fast-AR frame of one row (the oracle's or_fastar_frame): returns
    (codes [9] int32, logits [9, 4096] uint16 bf16 bits)."""
    h = np.ascontiguousarray(hidden, np.uint16)
    codes = np.zeros(9, np.int32)
    lg = np.zeros((9, 4096), np.uint16)
    lib().or_fastar_frame(ctypes.addressof(faw), ptr(h), int(sem), ptr(codes), ptr(lg))
    return codes, lg


def vq_embed_add(cb_emb, codes, rows):
    """In place on rows [T, 2560]; codes [10, T]."""
    c = np.ascontiguousarray(codes, np.int32)
    lib().or_vq_embed_add(ptr(cb_emb), ptr(c), c.shape[1], ptr(rows))


def gemm_bf16(x, w, M, N, K):
    y = np.empty((M, N), np.uint16)
    lib().or_gemm_bf16(ptr(x), ptr(w), ptr(y), M, N, K)
    return y


def gemm_bf16_f64(x, w, M, N, K):
    y = np.empty((M, N), np.float64)
    lib().or_gemm_bf16_f64(ptr(x), ptr(w), ptr(y), M, N, K)
    return y


class OrDraft(ctypes.Structure):
    """or_draft_w: bf16 weight pointers in the order of s2p_oracle.h."""
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("fuse", "wqkv", "wo", "w1", "w3", "w2", "q_norm", "k_norm", "attn_norm",
                 "ffn_norm", "final_norm")]


def make_draft(w):
    """w: dict of contiguous uint16 arrays keyed by the OrDraft field names
    (kept alive by the caller)."""
    return OrDraft(*[ptr(w[n]) for n, _ in OrDraft._fields_])


def draft_step(d, kc, vc, max_seq, pos, h, e):
    """In place on kc, vc; returns the step's output [2560] bf16 bits."""
    out = np.empty(2560, np.uint16)
    lib().or_draft_step(ctypes.addressof(d), ptr(kc), ptr(vc), max_seq, pos, ptr(h), ptr(e),
                        ptr(out))
    return out
