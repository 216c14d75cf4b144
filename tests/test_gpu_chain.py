"""The chain condition of speculative frames on the GPU (s2p_verify_chain,
reference docs/SPECULATIVE.md:26-41): after a verify forward, the fast-AR
frame of every drafted node on its parent row's final-normed hidden, and the
comparison with the codes the draft used.

Checked against the pieces it composes, each pinned elsewhere: the final
RMSNorm of the GPU's residual rows by the oracle (bit-exact rule), then the
decoder's own host entry point s2pfa_decode_frame_batch on those rows
(deterministic: the same codes), and the per-node comparison by numpy."""
import ctypes

import numpy as np
import pytest
import torch

import pyoracle as po
import s2pamd
from gpu_util import P, S, bf16_bits, d2h, empty, sync, to_dev, to_host
from test_gpu_verify import TREE16, make_backbone, new_kv, plan

pytestmark = pytest.mark.gpu

EOS, SEM0 = 151645, 151678


@pytest.fixture(scope="module")
def lib():
    lib = s2pamd.load()
    s2pamd.check(lib.s2p_gemm_init(128), "gemm init")
    return lib


@pytest.fixture(scope="module")
def decoder(lib):
    f = ctypes.c_void_p()
    s2pamd.check(lib.s2pfa_create_random(ctypes.byref(f), 0, 64, 5, S()), "fastar")
    sync()
    yield f
    lib.s2pfa_free(f)


@pytest.mark.parametrize("parent,n_sess", [([-1, 0, 1, 2, 3], 1), (TREE16, 2)])
def test_verify_chain_codes_and_flags(lib, decoder, parent, n_sess):
    R = len(parent)
    ctx = 1024
    bb = make_backbone(lib, 2, s2pamd.WQ_INT4, s2pamd.S2P_HEAD_SLICE, n_sess * R, n_sess, ctx, 91)
    try:
        kvs = [new_kv(lib, bb, 10 + s) for s in range(n_sess)]
        plan(lib, bb, parent, kvs, [300 + 17 * s for s in range(n_sess)])
        rows = n_sess * R
        r = np.random.default_rng(R)
        x = bf16_bits(r.standard_normal((rows, 2560)).astype(np.float32))
        logits = empty((rows, s2pamd.S2P_HEAD_SLICE))
        s2pamd.check(lib.s2p_verify_forward(bb, P(to_dev(x)), P(logits), S()))
        tok = (SEM0 + r.integers(0, 4096, rows)).astype(np.int64)
        tok[::R] = 0
        tok[2] = EOS  # an EOS node passes whatever its codes
        # the expected codes: oracle final norm of the GPU's residual rows,
        # parents gathered, the decoder's host entry point
        ptrs = [ctypes.c_void_p() for _ in range(5)]
        lib.s2p_backbone_debug_ptrs.restype = None
        lib.s2p_backbone_debug_ptrs.argtypes = [ctypes.c_void_p] + [ctypes.c_void_p] * 5
        lib.s2p_backbone_debug_ptrs(bb, *[ctypes.byref(p) for p in ptrs])
        g_x = d2h(ptrs[0].value, rows * 2560 * 2, np.uint16).reshape(rows, 2560)
        fnorm = d2h(lib.s2p_backbone_final_norm(bb), 2560 * 2, np.uint16)
        hid = po.rms_norm(g_x, fnorm, rows, 2560)
        nodes = [(s, i) for s in range(n_sess) for i in range(1, R)]
        par = np.stack([hid[s * R + parent[i]] for s, i in nodes])
        sem = np.array([(t - SEM0) if 0 <= t - SEM0 < 4096 else 0
                        for t in (tok[s * R + i] for s, i in nodes)], np.int32)
        out = np.zeros((len(nodes), 10), np.int32)
        s2pamd.check(lib.s2pfa_decode_frame_batch(decoder, P(to_dev(par)),
                                                  sem.ctypes.data_as(ctypes.c_void_p), len(nodes),
                                                  out.ctypes.data_as(ctypes.c_void_p), S()), "host")
        want = np.zeros((rows, 9), np.int32)
        for b, (s, i) in enumerate(nodes):
            want[s * R + i] = out[b, 1:]
        # drafted codes: right for some nodes, one code off for the others
        draft = want.copy()
        wrong = r.random(rows) < 0.4
        wrong[::R] = False
        draft[wrong, r.integers(0, 9)] += 1
        chain = torch.zeros(rows, dtype=torch.uint8, device="cuda")
        codes = torch.zeros((rows, 9), dtype=torch.int32, device="cuda")
        d_parent = to_dev(np.asarray(parent, np.int32))
        d_tok, d_draft = to_dev(tok), to_dev(draft)
        s2pamd.check(lib.s2p_verify_chain(bb, decoder, P(d_parent), P(d_tok), P(d_draft),
                                          P(chain), P(codes), S()), "chain")
        got_codes = to_host(codes, np.int32)
        assert np.array_equal(got_codes, want)
        ok = ~wrong
        ok[tok == EOS] = True
        assert np.array_equal(to_host(chain, np.uint8).astype(bool), ok)
        assert wrong.any() and ok[1:].any()
        # graph capture replays the same
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            s2pamd.check(lib.s2p_verify_chain(bb, decoder, P(d_parent), P(d_tok), P(d_draft),
                                              P(chain), P(codes), ctypes.c_void_p(s.cuda_stream)),
                         "capture")
        for _ in range(2):
            codes.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(to_host(codes, np.int32), want)
    finally:
        lib.s2p_backbone_free(bb)


def test_verify_chain_argument_errors(lib, decoder):
    z = ctypes.c_void_p(0)
    assert lib.s2p_verify_chain(None, decoder, z, z, z, z, z, S()) == -1
