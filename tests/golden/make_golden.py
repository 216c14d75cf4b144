"""Writes the golden fixtures of the verify path (tests/golden/*.npz).

The reference ships no fixtures for this path (its tests/test_draft.c needs
external fix_*.f32 files), so these are generated here from BASELINE
config 1's recipe and seeds:
  gemv_cfg1.npz   INT4-g32 linear 2560 -> 9728 (a 64-row slice), M=5:
                  codes uniform [-8,7], f16 scales |N(0,0.02)|, x bf16 N(0,1);
                  y_f64 = binary64 dot (numpy, independent of the oracle),
                  y_ref = the reference-order oracle (bf16).
  accept_cfg1.npz acceptance over 4096-way logits, K=4, T0.8 p0.8:
                  target N(0,2), draft = target + N(0,0.5); 8 sessions
                  (seeded and unseeded); drafted ids from the draft rows;
                  expected path / emitted ids / final sampler state bytes
                  from the oracle's rule (regression vectors).
  accept_tree.npz the same for the 16-node tree of config 5, 2 sessions.
Run: python tests/golden/make_golden.py  (needs oracle/liboracle.so)
"""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import pyoracle as po  # noqa: E402

SEM0 = 151678
TREE16 = [-1, 0, 0, 1, 1, 2, 2, 3, 3, 4, 5, 6, 6, 7, 8, 10, 11]


def bf16(a):
    return po.f32_to_bf16(np.asarray(a, np.float32))


def gemv_cfg1():
    r = np.random.default_rng(0)
    N, K, M = 64, 2560, 5
    q = r.integers(-8, 8, (N, K), dtype=np.int8)
    w = po.int4_pack(q, N, K)
    s = np.abs(r.standard_normal((N, K // 32)) * 0.02).astype(np.float16).view(np.uint16)
    x = bf16(r.standard_normal((M, K)))
    xf = po.bf16_to_f32(x).astype(np.float64)
    wf = q.astype(np.float64) * np.repeat(s.view(np.float16).astype(np.float64), 32, axis=1)
    y_f64 = xf @ wf.T
    y_ref = po.int4p_gemv(x, w, s, M, N, K)
    np.savez_compressed(os.path.join(HERE, "gemv_cfg1.npz"), w=w, s=s, x=x, y_f64=y_f64,
                        y_ref=y_ref)


def draft_ids(states, drf, de, parent, R):
    tok = np.zeros(len(states) * R, np.int64)
    for si, st in enumerate(states):
        for i in range(1, R):
            sd = po.copy_state(st)
            path, u = [], parent[i]
            while u > 0:
                path.append(u)
                u = parent[u]
            for u in reversed(path):
                po.state_push(sd, tok[si * R + u])
            row, eos = drf[si * R + parent[i]], int(de[si * R + parent[i]])
            first = min(c for c in range(1, R) if parent[c] == parent[i]) == i
            if first:
                tok[si * R + i] = po.sample(sd, row, eos)[0]
            else:
                ti = po.transform(sd, row, eos)[0]
                tok[si * R + i] = SEM0 + int(ti[(i * 7) % 30])
    return tok


def accept_case(name, parent, n_sess, seed):
    r = np.random.default_rng(seed)
    R = len(parent)
    tgt = r.standard_normal((n_sess * R, 4096)) * 2
    drf = tgt + r.standard_normal((n_sess * R, 4096)) * 0.5
    te = r.standard_normal(n_sess * R) - 6
    de = r.standard_normal(n_sess * R) - 6
    tgt, drf, te, de = bf16(tgt), bf16(drf), bf16(te), bf16(de)
    states = []
    for si in range(n_sess):
        st = po.state(temperature=0.8, top_p=0.8, seed=0 if si % 2 == 0 else 100 + si,
                      entropy=si)
        for t in r.integers(0, 4096, si % 7):
            po.state_push(st, SEM0 + int(t))
        states.append(st)
    tok = draft_ids(states, drf, de, parent, R)
    paths = np.full((n_sess, R), -1, np.int32)
    emits = np.full((n_sess, R + 1), -1, np.int64)
    nacc = np.zeros(n_sess, np.int32)
    nemit = np.zeros(n_sess, np.int32)
    st_in, st_out = [], []
    for si, st in enumerate(states):
        st_in.append(np.frombuffer(bytes(st), np.uint8).copy())
        sc = po.copy_state(st)
        p, e = po.accept_tree(sc, tgt[si * R:(si + 1) * R], drf[si * R:(si + 1) * R], parent,
                              tok[si * R:(si + 1) * R], te[si * R:(si + 1) * R],
                              de[si * R:(si + 1) * R])
        paths[si, :len(p)] = p
        emits[si, :len(e)] = e
        nacc[si], nemit[si] = len(p), len(e)
        st_out.append(np.frombuffer(bytes(sc), np.uint8).copy())
    np.savez_compressed(os.path.join(HERE, name), parent=np.asarray(parent, np.int32), tgt=tgt,
                        drf=drf, tgt_eos=te, drf_eos=de, tok=tok, states_in=np.stack(st_in),
                        path=paths, n_acc=nacc, emit=emits, n_emit=nemit,
                        states_out=np.stack(st_out))


if __name__ == "__main__":
    gemv_cfg1()
    accept_case("accept_cfg1.npz", [-1, 0, 1, 2, 3], 8, 1)
    accept_case("accept_tree.npz", TREE16, 2, 2)
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
