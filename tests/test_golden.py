"""Golden fixtures (tests/golden/, written by make_golden.py from BASELINE
config 1's recipe): the oracle reproduces them on the CPU, and the device
path reproduces them through the C ABI (-m gpu).  GEMV: within 1e-2 of the
binary64 dot; acceptance: bit-exact paths, emitted ids and state bytes."""
import ctypes
import os

import numpy as np
import pytest

import pyoracle as po

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return dict(np.load(os.path.join(HERE, name), allow_pickle=False))


def test_gemv_golden_oracle():
    g = load("gemv_cfg1.npz")
    M, K = g["x"].shape
    N = g["w"].shape[0]
    y = po.int4p_gemv(g["x"], g["w"], g["s"], M, N, K)
    assert np.array_equal(y, g["y_ref"])
    yf = po.bf16_to_f32(y).astype(np.float64)
    rel = np.linalg.norm(yf - g["y_f64"], axis=1) / np.linalg.norm(g["y_f64"], axis=1)
    assert rel.max() < 1e-2


def states_of(arr):
    out = []
    for row in arr:
        s = po.OrState()
        ctypes.memmove(ctypes.addressof(s), row.tobytes(), ctypes.sizeof(po.OrState))
        out.append(s)
    return out


@pytest.mark.parametrize("name", ["accept_cfg1.npz", "accept_tree.npz"])
def test_accept_golden_oracle(name):
    g = load(name)
    parent = list(g["parent"])
    R = len(parent)
    for si, st in enumerate(states_of(g["states_in"])):
        sl = slice(si * R, (si + 1) * R)
        p, e = po.accept_tree(st, g["tgt"][sl], g["drf"][sl], parent, g["tok"][sl],
                              g["tgt_eos"][sl], g["drf_eos"][sl])
        assert list(p) == list(g["path"][si, :g["n_acc"][si]])
        assert list(e) == list(g["emit"][si, :g["n_emit"][si]])
        assert bytes(st) == g["states_out"][si].tobytes()


@pytest.mark.gpu
def test_gemv_golden_device():
    import s2pamd
    from gpu_util import P, S, empty, to_dev, to_host
    lib = s2pamd.load()
    s2pamd.check(lib.s2p_gemm_init(128))
    g = load("gemv_cfg1.npz")
    M, K = g["x"].shape
    N = g["w"].shape[0]
    y = empty((M, N))
    s2pamd.check(lib.s2p_int4p_gemv(P(y), P(to_dev(g["x"])), P(to_dev(g["w"])), P(to_dev(g["s"])),
                                    M, N, K, 32, S()))
    yf = po.bf16_to_f32(to_host(y, np.uint16)).astype(np.float64)
    rel = np.linalg.norm(yf - g["y_f64"], axis=1) / np.linalg.norm(g["y_f64"], axis=1)
    assert rel.max() < 1e-2, rel


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["accept_cfg1.npz", "accept_tree.npz"])
def test_accept_golden_device(name):
    import torch
    import s2pamd
    from gpu_util import P, S, to_dev, to_host
    lib = s2pamd.load()
    g = load(name)
    R = len(g["parent"])
    n = len(g["states_in"])
    d_states = to_dev(np.ascontiguousarray(g["states_in"]).reshape(-1))
    sb = g["states_in"].shape[1]
    d_ptrs = to_dev(np.array([d_states.data_ptr() + i * sb for i in range(n)], np.int64))
    work = torch.empty(lib.s2p_verify_accept_work_bytes(n, R), dtype=torch.uint8, device="cuda")
    path = torch.full((n * R,), -1, dtype=torch.int32, device="cuda")
    nacc = torch.zeros(n, dtype=torch.int32, device="cuda")
    emit = torch.zeros(n * (R + 1), dtype=torch.int64, device="cuda")
    nemit = torch.zeros(n, dtype=torch.int32, device="cuda")
    s2pamd.check(lib.s2p_verify_accept(P(to_dev(g["tgt"])), P(to_dev(g["tgt_eos"])),
                                       P(to_dev(g["drf"])), P(to_dev(g["drf_eos"])), 4096,
                                       P(to_dev(g["parent"])), P(to_dev(g["tok"])), P(d_ptrs), n, R,
                                       P(path), P(nacc), P(emit), P(nemit), P(work), S()))
    assert np.array_equal(to_host(nacc), g["n_acc"])
    assert np.array_equal(to_host(nemit), g["n_emit"])
    p = to_host(path).reshape(n, R)
    e = to_host(emit).reshape(n, R + 1)
    for si in range(n):
        assert list(p[si, :g["n_acc"][si]]) == list(g["path"][si, :g["n_acc"][si]])
        assert list(e[si, :g["n_emit"][si]]) == list(g["emit"][si, :g["n_emit"][si]])
    assert to_host(d_states).tobytes() == np.ascontiguousarray(g["states_out"]).tobytes()
