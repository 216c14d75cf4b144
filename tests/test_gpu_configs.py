"""Configs 4 and 5 of the verify path through the C ABI, on 2-layer backbones
at the configs' batch shapes and KV lengths (the 36-layer depth adds nothing
the per-layer checks do not see; config 3 covers full depth).

Config 4: a lockstep batch of 8 sessions x K=4 (M = 40 rows: three MFMA column
tiles in every GEMV), per-session KV lengths drawn uniformly from 256..4096,
per-session acceptance with independent seeds.
Config 5: a 16-node draft tree (+ root) per session, batch 4 (M = 68: five
column tiles), KV context 8192, acceptance along the longest accepted root
path with residual resampling.

Logits follow the tolerance of test_gpu_verify (north star: 1e-2 relative
to the oracle's reference-order forward per row; over all sessions' rows no
less accurate than it against binary64); acceptance decisions, emitted ids
and sampler states are bit-exact against the host rule applied to the logits
the GPU produced."""
import numpy as np
import pytest

import f64_forward as f64
import pyoracle as po
import s2pamd
from gpu_util import P, S, bf16_bits, bf16_vals, empty, to_dev, to_host
from test_gpu_sample import draft_tokens, run_accept
from test_gpu_verify import (TREE16, check_logits, check_rms, f64_weights, make_backbone,
                             new_kv, oracle_forward, plan)

pytestmark = pytest.mark.gpu

N_LAYERS = 2


@pytest.fixture(scope="module")
def lib():
    return s2pamd.load()


def run_config(lib, parent, lens, ctx, seed):
    """Forward of len(lens) sessions sharing `parent`, checked per session
    against the oracle and binary64; then device acceptance of drafts drawn
    from target + N(0, 0.5) logits, checked against the host rule."""
    n = len(lens)
    R = len(parent)
    head_rows = s2pamd.S2P_HEAD_SLICE
    bb = make_backbone(lib, N_LAYERS, s2pamd.WQ_INT4, head_rows, n * R, n, ctx, seed)
    try:
        kvs = [new_kv(lib, bb, seed + 10 + s) for s in range(n)]
        hosts = [to_host(k, np.uint16).copy() for k in kvs]
        print(f"config: {n} sessions x {R} rows, lens {list(lens)}, ctx {ctx}", flush=True)
        plan(lib, bb, parent, kvs, [int(v) for v in lens])
        rng = np.random.default_rng(seed)
        x = bf16_bits(rng.standard_normal((n * R, 2560)).astype(np.float32))
        logits = empty((n * R, head_rows))
        s2pamd.check(lib.s2p_verify_forward(bb, P(to_dev(x)), P(logits), S()), "forward")
        got_bits = to_host(logits, np.uint16)
        got = bf16_vals(got_bits)
        W, fn, head = f64_weights(lib, bb, N_LAYERS)
        wants, truths = [], []
        for s in range(n):
            rows = slice(s * R, (s + 1) * R)
            want, _ = oracle_forward(lib, bb, N_LAYERS, x[rows], hosts[s], ctx, int(lens[s]),
                                     parent, head_rows)
            truth = f64.forward(W, fn, head, x[rows],
                                hosts[s].reshape(N_LAYERS, 16, ctx, 128), int(lens[s]), parent)
            check_logits(got[rows], want, truth, f"session {s} (L={lens[s]})", rms=False)
            wants.append(bf16_vals(want))
            truths.append(truth)
        # the accuracy criterion over all sessions' rows (5 rows alone are too
        # few for an rms comparison of two rounding orders)
        check_rms(got, np.concatenate(wants), np.concatenate(truths), "all sessions")
    finally:
        lib.s2p_backbone_free(bb)

    # acceptance on the produced logits: 4096 semantic columns + EOS
    tgt = np.ascontiguousarray(got_bits[:, :4096])
    te = np.ascontiguousarray(got_bits[:, 4096])
    noisy = bf16_vals(got_bits) + 0.5 * rng.standard_normal(got_bits.shape).astype(np.float32)
    drf_full = bf16_bits(noisy)
    drf = np.ascontiguousarray(drf_full[:, :4096])
    de = np.ascontiguousarray(drf_full[:, 4096])
    states = [po.state(temperature=0.8, top_p=0.8, seed=1000 + 17 * s, entropy=s)
              for s in range(n)]
    tok = draft_tokens(states, drf, de, parent, R)
    path, nacc, emit, nemit, new_states = run_accept(lib, states, tgt, drf, te, de, parent, tok,
                                                     n, R)
    for s in range(n):
        rows = slice(s * R, (s + 1) * R)
        st = po.copy_state(states[s])
        p_ref, e_ref = po.accept_tree(st, tgt[rows], drf[rows], parent, tok[rows], te[rows],
                                      de[rows])
        assert nacc[s] == len(p_ref) and list(path[s, :nacc[s]]) == list(p_ref), s
        assert nemit[s] == len(e_ref) and list(emit[s, :nemit[s]]) == list(e_ref), s
        assert bytes(new_states[s]) == bytes(st), s
    return nacc


def test_config4_batch8_chains(lib):
    """8 sessions x K=4 chain, KV lengths ~ U[256, 4096] (fixed seed)."""
    lens = np.random.default_rng(4).integers(256, 4097, 8)
    nacc = run_config(lib, [-1, 0, 1, 2, 3], lens, 4096 + 64, 404)
    assert len(nacc) == 8


def test_config5_tree_batch4(lib):
    """4 sessions x 16-node tree (+ root), KV context 8192."""
    nacc = run_config(lib, TREE16, [8192] * 4, 8192 + 64, 505)
    assert len(nacc) == 4
