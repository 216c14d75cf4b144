"""Fast-AR residual decoder on the GPU (include/s2pro/fastar.h) against the
oracle's frame (or_fastar_frame, restating src/fastar/fastar.cu:726-789),
plus the two step primitives it uses from kernels.h (s2pk_embed,
s2pk_argmax) and the VQ-embedding sum (s2pfa_vq_embed_add).

Tolerance (north star: 1e-2 relative): each step's head logits against the
oracle's under the verify path's logits rule (test_gpu_verify.check_logits:
1e-2 L2 per row, 2x that in the max norm, a named exception up to 2e-2 only
where the GPU is at least as close to the binary64 forward as the oracle,
and GPU rms error vs binary64 at most 1.25x the oracle's).  The GPU feeds its
own argmax into the next step, so steps are compared while the two code
sequences agree; the codes must agree at every step where the oracle's top-2
margin exceeds 2e-2 of the row's max (a smaller margin is a tie at this
tolerance, after which the sequences may diverge legitimately).
The embedding gather, the argmax and the VQ sum are bit-exact."""
import ctypes

import numpy as np
import pytest
import torch

import f64_forward as f64
import pyoracle as po
import s2pamd
from test_gpu_verify import check_logits
from gpu_util import P, S, bf16_bits, bf16_vals, d2h, empty, sync, to_dev, to_host

pytestmark = pytest.mark.gpu

DIM, CB = 2560, 4096


@pytest.fixture(scope="module")
def lib():
    lib = s2pamd.load()
    s2pamd.check(lib.s2p_gemm_init(128), "gemm init")
    return lib


def host_linear(lin):
    if lin.q_packed:
        w = d2h(lin.w_pack.data, lin.w_pack.bytes, np.uint8)
        s = d2h(lin.w_iscale.data, lin.w_iscale.bytes, np.uint16)
        return po.make_linear(w, s, lin.out_features, lin.in_features, 32), (w, s)
    w = d2h(lin.w_int8.data, lin.w_int8.bytes, np.int8)
    s = d2h(lin.w_iscale.data, lin.w_iscale.bytes, np.float32)
    return po.make_linear(w, s, lin.out_features, lin.in_features, 0), (w, s)


def host_weights(W):
    """The oracle's view of a decoder's weights (arrays kept alive in keep)."""
    keep = []
    layers = []
    for l in range(4):
        L = W.layers[l]
        lins = []
        for name in ("wqkv", "wo", "w13", "w2"):
            li, k = host_linear(getattr(L, name))
            lins.append(li)
            keep.append(k)
        an = d2h(L.attn_norm.data, L.attn_norm.bytes, np.uint16)
        fn = d2h(L.ffn_norm.data, L.ffn_norm.bytes, np.uint16)
        keep += [an, fn]
        layers.append(po.OrLayerW(lins[0], lins[1], lins[2], lins[3], po.ptr(an), po.ptr(fn),
                                  None, None))
    norm = d2h(W.norm.data, W.norm.bytes, np.uint16)
    out, k = host_linear(W.output)
    emb = d2h(W.emb.data, W.emb.bytes, np.uint16)
    keep += [norm, k, emb]
    faw = po.OrFaW((po.OrLayerW * 4)(*layers), po.ptr(norm), out, po.ptr(emb))
    return faw, keep


@pytest.fixture(scope="module", params=[0, 1], ids=["int4", "int8"])
def decoder(lib, request):
    f = ctypes.c_void_p()
    s2pamd.check(lib.s2pfa_create_random(ctypes.byref(f), request.param, 4, 77 + request.param,
                                         S()), "fastar create")
    sync()
    yield f
    lib.s2pfa_free(f)


def run_frame(lib, f, hidden, sem):
    B = hidden.shape[0]
    stage = ctypes.c_void_p()
    lg = empty((9, B, CB))
    s2pamd.check(lib.s2pfa_decode_frame_logits_dev(f, P(to_dev(hidden)),
                                                   P(to_dev(np.asarray(sem, np.int32))), B,
                                                   ctypes.byref(stage), P(lg), S()), "frame")
    sync()
    codes = d2h(stage.value, 9 * B * 4, np.int32).reshape(9, B)
    return codes, bf16_vals(to_host(lg, np.uint16)).astype(np.float64)


def final_normed(r, B):
    """A final-normed hidden: unit-rms rows times a norm-like weight."""
    h = r.standard_normal((B, DIM)).astype(np.float32)
    h /= np.sqrt(np.mean(h * h, axis=1, keepdims=True))
    return bf16_bits(h * (1 + 0.02 * r.standard_normal(DIM).astype(np.float32)))


def f64_weights(W):
    layers = []
    for l in range(4):
        L = W.layers[l]
        d = {}
        for name, key in (("wqkv", "wqkv"), ("wo", "wo"), ("w13", "gate_up"), ("w2", "w2")):
            lin = getattr(L, name)
            _, (w, s) = host_linear(lin)
            d[key] = f64.dequant(w, s, lin.out_features, lin.in_features)
        for n in ("attn_norm", "ffn_norm"):
            t = getattr(L, n)
            d[n] = f64.bf(d2h(t.data, t.bytes, np.uint16))
        layers.append(d)
    _, (w, s) = host_linear(W.output)
    head = f64.dequant(w, s, W.output.out_features, W.output.in_features)
    return layers, f64.bf(d2h(W.norm.data, W.norm.bytes, np.uint16)), head


def test_fastar_frame_vs_oracle(lib, decoder):
    W = lib.s2pfa_weights_of(decoder).contents
    faw, keep = host_weights(W)
    emb = keep[-1].reshape(CB, DIM)
    r = np.random.default_rng(3)
    B = 3
    hidden = final_normed(r, B)
    sem = [0, 4095, int(r.integers(1, 4095))]
    codes, logits = run_frame(lib, decoder, hidden, sem)
    fl, fnorm, fhead = f64_weights(W)
    got, want, truth = [], [], []
    n_diff_codes = 0
    for b in range(B):
        want_codes, want_lg = po.fastar_frame(faw, hidden[b], sem[b])
        n_diff_codes += len(set(want_codes.tolist()))
        seq = emb[[sem[b]] + [int(c) for c in want_codes]]
        for s in range(9):
            w = bf16_vals(want_lg[s]).astype(np.float64)
            got.append(logits[s, b])
            want.append(want_lg[s])
            truth.append(f64.fastar_step(fl, fnorm, fhead, hidden[b], seq, s + 1)[0])
            if codes[s, b] != want_codes[s]:
                top2 = np.sort(w)[-2:]
                scale = np.max(np.abs(w))
                assert top2[1] - top2[0] <= 2e-2 * scale, \
                    f"row {b} step {s + 1}: code {codes[s, b]} vs {want_codes[s]} " \
                    f"at margin {(top2[1] - top2[0]) / scale:.3g}"
                print(f"row {b}: codes diverge at step {s + 1} on a near-tie")
                break  # the sequences diverge here, legitimately
    check_logits(np.array(got), np.array(want), np.array(truth), "fast-AR step logits")
    # the synthetic decoder is not degenerate: codes vary within a frame
    assert n_diff_codes >= 2 * B, n_diff_codes


def test_fastar_host_entry_point_and_determinism(lib, decoder):
    """s2pfa_decode_frame_batch (host codes, [B][10] with column 0 kept)
    equals the device entry point's stage, and a frame repeats bit-exactly
    (the cache of the previous frame is never read)."""
    r = np.random.default_rng(9)
    B = 4
    hidden = final_normed(r, B)
    sem = r.integers(0, 4096, B).astype(np.int32)
    c1, l1 = run_frame(lib, decoder, hidden, sem)
    out = np.full((B, 10), -7, np.int32)
    s2pamd.check(lib.s2pfa_decode_frame_batch(decoder, P(to_dev(hidden)),
                                              sem.ctypes.data_as(ctypes.c_void_p), B,
                                              out.ctypes.data_as(ctypes.c_void_p), S()), "host")
    assert np.all(out[:, 0] == -7)
    assert np.array_equal(out[:, 1:], c1.T)
    c2, l2 = run_frame(lib, decoder, hidden, sem)
    assert np.array_equal(c1, c2) and np.array_equal(l1, l2)
    # a row alone gives its step-1 logits of the batch (to the tolerance:
    # another M may take another GEMV split)
    c3, l3 = run_frame(lib, decoder, hidden[1:2], sem[1:2])
    np.testing.assert_allclose(l3[0, 0], l1[0, 1], rtol=0, atol=1e-2 * np.max(np.abs(l1[0, 1])))


def test_fastar_frame_graph_replay(lib, decoder):
    r = np.random.default_rng(11)
    B = 2
    hd = to_dev(final_normed(r, B))
    sd = to_dev(np.array([5, 4000], np.int32))
    c0, l0 = None, None
    stage = ctypes.c_void_p()
    lg = empty((9, B, CB))
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        s2pamd.check(lib.s2pfa_decode_frame_logits_dev(decoder, P(hd), P(sd), B,
                                                       ctypes.byref(stage), P(lg),
                                                       ctypes.c_void_p(s.cuda_stream)), "eager")
    s.synchronize()
    c0 = d2h(stage.value, 9 * B * 4, np.int32).copy()
    l0 = to_host(lg, np.uint16).copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        s2pamd.check(lib.s2pfa_decode_frame_logits_dev(decoder, P(hd), P(sd), B,
                                                       ctypes.byref(stage), P(lg),
                                                       ctypes.c_void_p(s.cuda_stream)), "capture")
    for i in range(3):
        lg.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(d2h(stage.value, 9 * B * 4, np.int32), c0), f"replay {i} codes"
        assert np.array_equal(to_host(lg, np.uint16), l0), f"replay {i} logits"


def test_fastar_vq_embed_add_vs_oracle(lib, decoder):
    W = lib.s2pfa_weights_of(decoder).contents
    cb = d2h(W.cb_emb.data, W.cb_emb.bytes, np.uint16)
    r = np.random.default_rng(4)
    T = 5
    codes = r.integers(0, 4096, (10, T)).astype(np.int32)
    codes[0, 0], codes[3, 1], codes[9, 4] = -5, 4096, 99999  # clamped
    rows = bf16_bits(r.standard_normal((T, DIM)).astype(np.float32))
    want = rows.copy()
    po.vq_embed_add(cb, codes, want)
    d = to_dev(rows)
    s2pamd.check(lib.s2pfa_vq_embed_add_dev(decoder, P(to_dev(codes)), T, P(d), S()), "vq dev")
    assert np.array_equal(to_host(d, np.uint16), want)
    d = to_dev(rows)
    s2pamd.check(lib.s2pfa_vq_embed_add(decoder, codes.ctypes.data_as(ctypes.c_void_p), T, P(d),
                                        S()), "vq host")
    assert np.array_equal(to_host(d, np.uint16), want)
    assert lib.s2pfa_vq_embed_add_dev(decoder, None, T, P(d), S()) == -1
    assert lib.s2pfa_vq_embed_add(decoder, codes.ctypes.data_as(ctypes.c_void_p), 0, P(d),
                                  S()) == 0


def test_fastar_argument_errors(lib, decoder):
    st = ctypes.c_void_p()
    h = empty((1, DIM))
    sd = to_dev(np.zeros(1, np.int32))
    assert lib.s2pfa_decode_frame_batch_dev(decoder, P(h), P(sd), 0, ctypes.byref(st), S()) == -1
    assert lib.s2pfa_decode_frame_batch_dev(decoder, P(h), P(sd), 5, ctypes.byref(st), S()) == -1
    assert lib.s2pfa_decode_frame_batch_dev(decoder, None, P(sd), 1, ctypes.byref(st), S()) == -1
    f = ctypes.c_void_p()
    assert lib.s2pfa_create_random(ctypes.byref(f), 0, 0, 1, S()) == -1


def test_embed_gather_exact(lib):
    r = np.random.default_rng(1)
    table = bf16_bits(r.standard_normal((300, 2560)).astype(np.float32))
    ids = np.array([0, 299, 17, 17, 150], np.int64)
    out = empty((5, 2560))
    assert lib.s2pk_embed(P(to_dev(table)), P(to_dev(ids)), P(out), 5, 2560, S()) == 0
    assert np.array_equal(to_host(out, np.uint16), table[ids])
    assert lib.s2pk_embed(None, P(to_dev(ids)), P(out), 5, 2560, S()) != 0


def test_argmax_ties_nan(lib):
    """Largest value, lowest index among equal maxima, NaN never chosen
    (kernels.cu:1326-1357): brute force over crafted rows."""
    r = np.random.default_rng(2)
    V = 4096
    x = r.standard_normal((6, V)).astype(np.float32)
    x[1, [3000, 7, 4095]] = 50.0                   # a tie: index 7
    x[2, :] = 1.0                                  # all equal: index 0
    x[3, 10] = np.nan
    x[3, 11] = 60.0                                # NaN beside the max
    x[4, :] = np.nan
    x[4, 2049] = -3.0                              # one real value among NaNs
    x[5, 4095] = np.inf
    bits = bf16_bits(x)
    vals = bf16_vals(bits).astype(np.float64)
    ids = empty((6,), torch.int32)
    assert lib.s2pk_argmax(P(to_dev(bits)), P(ids), 6, V, S()) == 0
    got = to_host(ids, np.int32)
    for i in range(6):
        v = np.where(np.isnan(vals[i]), -np.inf, vals[i])
        want = int(np.flatnonzero(v == v.max())[0])
        assert got[i] == want, f"row {i}: {got[i]} vs {want}"
    assert got[1] == 7 and got[2] == 0 and got[3] == 11 and got[4] == 2049 and got[5] == 4095
