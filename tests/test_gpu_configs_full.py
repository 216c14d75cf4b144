"""Configs 4 and 5 at full depth (36 INT4-g32 layers, full 155,776-row
head): the batch of 8 chain sessions (M = 40, KV lengths ~ U[256, 4096])
and 4 sixteen-node trees (M = 68, KV 8192).  The forward is deterministic
and finite; the captured step replayed twice equals the eager step (logits
bit for bit, acceptance outputs); each session's device acceptance equals
the host rule on the same logits.  (Their numerics against the oracle are
checked at two layers in test_gpu_configs.py.)"""
import ctypes

import numpy as np
import pytest
import torch

import pyoracle as po
import s2pamd
from gpu_util import P, S, bf16_bits, bf16_vals, empty, to_dev, to_host
from test_gpu_verify import TREE16, make_backbone, new_kv, plan

pytestmark = pytest.mark.gpu

CONFIGS = {
    "config4": ([-1, 0, 1, 2, 3],
                [int(v) for v in np.random.default_rng(4).integers(256, 4097, 8)]),
    "config5": (TREE16, [8192] * 4),
}


@pytest.fixture(scope="module")
def lib():
    lib = s2pamd.load()
    s2pamd.check(lib.s2p_gemm_init(128), "gemm init")
    return lib


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_full_depth_step(lib, name):
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        _body(lib, *CONFIGS[name], name)
    torch.cuda.synchronize()


def _body(lib, parent, lens, name):
    NS, R = len(lens), len(parent)
    M = NS * R
    ctx = max(lens) + 64
    print(f"{name}: {NS} sessions x {R} rows, ctx {ctx}", flush=True)
    bb = make_backbone(lib, 36, s2pamd.WQ_INT4, s2pamd.S2P_VOCAB, max(16, M), NS, ctx, 17)
    try:
        kvs = [new_kv(lib, bb, 30 + s) for s in range(NS)]
        plan(lib, bb, parent, kvs, lens)
        x = to_dev(bf16_bits(np.random.default_rng(2).standard_normal((M, 2560)).astype(np.float32)))
        l1, l2 = empty((M, s2pamd.S2P_VOCAB)), empty((M, s2pamd.S2P_VOCAB))
        s2pamd.check(lib.s2p_verify_forward(bb, P(x), P(l1), S()))
        s2pamd.check(lib.s2p_verify_forward(bb, P(x), P(l2), S()))
        a, b = to_host(l1, np.uint16), to_host(l2, np.uint16)
        assert np.array_equal(a, b), "forward is not deterministic"
        v = bf16_vals(a)
        assert np.all(np.isfinite(v)) and v.std() > 0.1
        drf = to_dev(bf16_bits(v + np.random.default_rng(3).standard_normal(
            a.shape).astype(np.float32) * 0.5))
        dv = to_host(drf, np.uint16)
        states = [po.state(temperature=0.8, top_p=0.8, seed=s, entropy=s) for s in range(NS)]
        # drafted ids: each node sampled from its parent's draft row
        tok = np.zeros(M, np.int64)
        for s in range(NS):
            sd = po.copy_state(states[s])
            for i in range(1, R):
                tok[s * R + i] = po.sample(sd, dv[s * R + parent[i]])[0]
        outs = []
        for use_graph in (0, 1, 1):
            d_states = [to_dev(np.frombuffer(bytes(st), np.uint8).copy()) for st in states]
            d_ptrs = to_dev(np.array([t.data_ptr() for t in d_states], np.int64))
            work = torch.empty(lib.s2p_verify_accept_work_bytes(NS, R), dtype=torch.uint8,
                               device="cuda")
            path = torch.zeros(M, dtype=torch.int32, device="cuda")
            nacc = torch.zeros(NS, dtype=torch.int32, device="cuda")
            emit = torch.zeros(NS * (R + 1), dtype=torch.int64, device="cuda")
            nemit = torch.zeros(NS, dtype=torch.int32, device="cuda")
            logits = empty((M, s2pamd.S2P_VOCAB))
            d_par, d_tok = to_dev(np.array(parent, np.int32)), to_dev(tok)
            io = s2pamd.StepIO(x.data_ptr(), logits.data_ptr(), drf.data_ptr(), s2pamd.S2P_VOCAB,
                               d_par.data_ptr(), d_tok.data_ptr(), d_ptrs.data_ptr(),
                               path.data_ptr(), nacc.data_ptr(), emit.data_ptr(),
                               nemit.data_ptr(), work.data_ptr())
            s2pamd.check(lib.s2p_verify_step(bb, ctypes.byref(io), use_graph, S()), "step")
            lg = to_host(logits, np.uint16)
            assert np.array_equal(lg, a), f"use_graph={use_graph}: logits differ"
            na, ne, em = to_host(nacc), to_host(nemit), to_host(emit)
            got = [(int(na[s]), list(em[s * (R + 1):s * (R + 1) + int(ne[s])])) for s in range(NS)]
            for s in range(NS):
                p_ref, e_ref = po.accept_tree(po.copy_state(states[s]), lg[s * R:(s + 1) * R],
                                              dv[s * R:(s + 1) * R], parent, tok[s * R:(s + 1) * R])
                assert got[s] == (len(p_ref), list(e_ref)), f"session {s}"
            outs.append(got)
            del d_states, work, d_par, d_tok
        assert outs[0] == outs[1] == outs[2]
    finally:
        lib.s2p_backbone_free(bb)
