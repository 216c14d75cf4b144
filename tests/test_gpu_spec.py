"""The composed speculative tick (s2p_spec_tick, include/s2pro/spec.h) on the
GPU: consecutive ticks replayed from one captured graph, checked tick for
tick against the host rule applied to the tick's own intermediate buffers.

Per tick and session:
- the verify inputs are the frame embeddings of the previous frame (row 0)
  and of the drafted frames (rows 1..K), bit for bit (numpy restatement of
  s2pk_embed + s2pfa_vq_embed_add + the 1/sqrt(11) scale, slowar.c:478-496);
- the drafted tokens are the oracle sampler's draws from the draft logits
  rows with a copy of the session's state, in order;
- the chain flags say whether the chain condition's codes equal the
  drafted codes (EOS nodes pass);
- acceptance equals the oracle's rule (path, emitted ids, advanced state
  bytes) on the tick's target and draft logits under those flags;
- kv_len advances by 1 + n_accepted; the emitted frames carry the chain
  codes of accepted nodes and, for the last token, the failed node's codes
  or the decoder's own frame on the hidden of the row that produced it;
- the next tick's previous frame / hidden are the last emitted ones.
The graph replays equal eager ticks bit for bit, and a session that outgrows
the plan's span triggers one host re-plan with everything still consistent.
"""
import ctypes

import numpy as np
import pytest
import torch

import draft_util as du
import gpu_util
import pyoracle as po
import s2pamd
from gpu_util import P, S, d2h, h2d_raw, sync, to_dev, to_host
from test_gpu_verify import make_backbone, new_kv

pytestmark = pytest.mark.gpu

EOS, SEM0, VOCAB, DIM = 151645, 151678, 155776, 2560
SCALE = np.float32(1.0 / 3.3166247903554)


@pytest.fixture(scope="module")
def lib():
    lib = s2pamd.load()
    s2pamd.check(lib.s2p_gemm_init(128), "gemm init")
    return lib


def f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf(x):
    """float32 -> bf16 bits, round to nearest even"""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def frame_embed(table_row, cb_rows, tok):
    """table_row [2560] bits, cb_rows [10][2560] bits (the frame's codebook
    rows in codebook order)"""
    x = np.asarray(table_row, np.uint16)
    if not (SEM0 <= tok < SEM0 + 4096):
        return x
    acc = np.zeros(DIM, np.float32)
    for c in range(10):
        acc = (acc + f32(cb_rows[c])).astype(np.float32)
    x = bf(f32(x) + f32(bf(acc)))
    return bf(f32(x) * SCALE)


class Tick:
    """One tick model + sessions + outputs, all device buffers kept alive."""

    def __init__(self, lib, tmp_path, n, K, lens, seed, near_identity=False):
        """near_identity: every backbone layer's group scales set to the
        smallest normal f16 (the layers then barely move the residual
        stream) and a draft whose fuse passes e through unchanged with zero
        block weights and the backbone's final norm: its predicted hidden is
        then close to the backbone's true hidden, so drafts are mostly
        accepted and the chain condition mostly holds."""
        self.lib, self.n, self.K, self.R = lib, n, K, K + 1
        R = self.R
        self.bb = make_backbone(lib, 2, s2pamd.WQ_INT4, s2pamd.S2P_HEAD_SLICE, n * R, n, 1024, 61)
        w = du.make_weights(3)
        if near_identity:
            for l in range(2):
                layer = lib.s2p_backbone_layer(self.bb, l).contents
                for name in ("wqkv", "wo", "gate_up", "w2"):
                    sc = getattr(layer, name).w_iscale
                    h2d_raw(np.full(sc.bytes // 2, 0x0400, np.uint16), sc.data)
            fuse = np.zeros((DIM, 2 * DIM), np.float32)
            fuse[:, DIM:] = np.eye(DIM, dtype=np.float32)
            w["fuse.weight"] = du.bf16_bits(fuse)
            for name in ("wqkv.weight", "wo.weight", "w1.weight", "w3.weight", "w2.weight"):
                w[name] = np.zeros_like(w[name])
            w["final_norm"] = d2h(lib.s2p_backbone_final_norm(self.bb), DIM * 2, np.uint16)
        self.fa = ctypes.c_void_p()
        s2pamd.check(lib.s2pfa_create_random(ctypes.byref(self.fa), 0, n * K, 17, S()), "fastar")
        path = tmp_path / "draft.safetensors"
        du.write_safetensors(path, w)
        self.dm = s2pamd.DraftModel()
        s2pamd.check(lib.s2p_draft_load(ctypes.byref(self.dm), str(path).encode()), "draft")
        self.dst = (s2pamd.DraftState * n)()
        hip = gpu_util.hip()
        hip.hipMemset.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
        for s in range(n):
            s2pamd.check(lib.s2p_draft_state_init(ctypes.byref(self.dst[s])), "draft state")
            # a draft cache with no history: zeros (its slots below kv_len are attended)
            assert hip.hipMemset(self.dst[s].kc.data, 0, 2 * self.dst[s].kc.bytes) == 0
        self.embed = torch.empty(VOCAB * DIM, dtype=torch.int16, device="cuda")
        s2pamd.hip_check(lib.s2p_synth_bf16_normal(P(self.embed), self.embed.numel(), 0.0, 0.05,
                                                   23, S()))
        self.kvs = [new_kv(lib, self.bb, 40 + s) for s in range(n)]
        r = np.random.default_rng(seed)
        self.kv_len = to_dev(np.array(lens, np.int32))
        self.prev_tok = to_dev((SEM0 + r.integers(0, 4096, n)).astype(np.int64))
        self.prev_codes = to_dev(r.integers(0, 4096, (n, 10)).astype(np.int32))
        h = r.standard_normal((n, DIM)).astype(np.float32)
        self.prev_hidden = to_dev(bf(h / np.sqrt(np.mean(h * h, axis=1, keepdims=True))))
        self.st_bufs = [to_dev(np.frombuffer(bytes(po.state(0.8, 0.8, seed=s + 1, entropy=s)),
                                             np.uint8).copy()) for s in range(n)]
        self.states = to_dev(np.array([t.data_ptr() for t in self.st_bufs], np.int64))
        self.done = to_dev(np.zeros(n, np.uint8))
        self.n_acc = to_dev(np.zeros(n, np.int32))
        self.n_emit = to_dev(np.zeros(n, np.int32))
        self.emit = to_dev(np.zeros((n, R + 1), np.int64))
        self.frames = to_dev(np.zeros((n, R + 1, 10), np.int32))
        self.kvp = (ctypes.c_void_p * n)(*[k.data_ptr() for k in self.kvs])
        self.cb = lib.s2pfa_weights_of(self.fa).contents.cb_emb
        m = s2pamd.SpecModel(self.bb, ctypes.addressof(self.dm), ctypes.addressof(self.dst),
                             self.fa, self.embed.data_ptr(), n, K)
        ss = s2pamd.SpecSessions(ctypes.addressof(self.kvp), self.kv_len.data_ptr(),
                                 self.prev_tok.data_ptr(), self.prev_codes.data_ptr(),
                                 self.prev_hidden.data_ptr(), self.states.data_ptr(),
                                 self.done.data_ptr())
        o = s2pamd.SpecOut(self.n_acc.data_ptr(), self.n_emit.data_ptr(), self.emit.data_ptr(),
                           self.frames.data_ptr())
        self.sp = ctypes.c_void_p()
        lens_h = np.array(lens, np.int32)
        s2pamd.check(lib.s2p_spec_create(ctypes.byref(self.sp), ctypes.byref(m), ctypes.byref(ss),
                                         lens_h.ctypes.data, ctypes.byref(o), S()), "spec create")
        self.buf = s2pamd.SpecBuffers()
        s2pamd.check(lib.s2p_spec_buffers_of(self.sp, ctypes.byref(self.buf)))

    def tick(self, use_graph):
        s2pamd.check(self.lib.s2p_spec_tick(self.sp, use_graph, S()), "tick")
        sync()

    def snapshot(self):
        n, R, W = self.n, self.R, self.buf.head_rows
        b = self.buf
        return dict(
            kv_len=to_host(self.kv_len).copy(), prev_tok=to_host(self.prev_tok).copy(),
            prev_codes=to_host(self.prev_codes).copy(),
            prev_hidden=to_host(self.prev_hidden, np.uint16).copy(),
            states=[to_host(t, np.uint8).copy() for t in self.st_bufs],
            done=to_host(self.done).copy(), n_acc=to_host(self.n_acc).copy(),
            n_emit=to_host(self.n_emit).copy(), emit=to_host(self.emit).copy(),
            frames=to_host(self.frames).copy(),
            logits=d2h(b.logits, n * R * W * 2, np.uint16).reshape(n * R, W),
            drf=d2h(b.drf_logits, n * R * W * 2, np.uint16).reshape(n * R, W),
            x=d2h(b.x, n * R * DIM * 2, np.uint16).reshape(n * R, DIM),
            tok=d2h(b.tok, n * R * 8, np.int64),
            draft_codes=d2h(b.draft_codes, n * R * 9 * 4, np.int32).reshape(n * R, 9),
            codes_out=d2h(b.codes_out, n * R * 9 * 4, np.int32).reshape(n * R, 9),
            chain_ok=d2h(b.chain_ok, n * R, np.uint8),
            tail=d2h(b.tail, n * 2 * 4, np.int32).reshape(n, 2))

    def free(self):
        sync()
        self.lib.s2p_spec_free(self.sp)
        for s in range(self.n):
            self.lib.s2p_draft_state_free(ctypes.byref(self.dst[s]))
        self.lib.s2p_draft_free(ctypes.byref(self.dm))
        self.lib.s2pfa_free(self.fa)
        self.lib.s2p_backbone_free(self.bb)


def table_row(t, tok):
    return d2h(t.embed.data_ptr() + int(tok) * DIM * 2, DIM * 2, np.uint16)


def cb_rows(t, codes):
    return np.stack([d2h(t.cb.data + (c * 4096 + int(codes[c])) * DIM * 2, DIM * 2, np.uint16)
                     for c in range(10)])


def check_tick(lib, t, pre, post):
    n, R, K = t.n, t.R, t.K
    parent = [-1] + list(range(R - 1))
    for s in range(n):
        if pre["done"][s]:
            continue
        rows = slice(s * R, (s + 1) * R)
        # row 0: the previous frame's embedding
        want = frame_embed(table_row(t, pre["prev_tok"][s]), cb_rows(t, pre["prev_codes"][s]),
                           pre["prev_tok"][s])
        assert np.array_equal(post["x"][s * R], want), f"session {s}: root input"
        # drafted tokens: the sampler on the draft rows with a copy of the state
        st = po.OrState()
        ctypes.memmove(ctypes.addressof(st), pre["states"][s].ctypes.data, ctypes.sizeof(st))
        sd = po.copy_state(st)
        drf = post["drf"][rows]
        tok = post["tok"][rows].copy()
        for i in range(1, R):
            tk = po.sample(sd, drf[i - 1, :4096], int(drf[i - 1, 4096]))[0]
            assert tok[i] == tk, f"session {s} depth {i}: drafted {tok[i]} vs rule {tk}"
            codes = np.concatenate([[tk - SEM0 if SEM0 <= tk < SEM0 + 4096 else 0],
                                    post["draft_codes"][s * R + i]])
            want = frame_embed(table_row(t, tk), cb_rows(t, codes), tk)
            assert np.array_equal(post["x"][s * R + i], want), f"session {s}: row {i} input"
        # chain flags
        for i in range(1, R):
            ok = np.array_equal(post["codes_out"][s * R + i], post["draft_codes"][s * R + i])
            assert post["chain_ok"][s * R + i] == int(ok or tok[i] == EOS), (s, i)
        # acceptance under the chain condition
        tgt = post["logits"][rows]
        p_ref, e_ref = po.accept_tree(st, np.ascontiguousarray(tgt[:, :4096]),
                                      np.ascontiguousarray(drf[:, :4096]), parent, tok,
                                      np.ascontiguousarray(tgt[:, 4096]),
                                      np.ascontiguousarray(drf[:, 4096]),
                                      chain=post["chain_ok"][rows])
        na, ne = int(post["n_acc"][s]), int(post["n_emit"][s])
        assert na == len(p_ref) and list(post["emit"][s][:ne]) == list(e_ref), \
            (s, na, list(post["emit"][s][:ne]), p_ref, e_ref)
        assert np.array_equal(post["states"][s], np.frombuffer(bytes(st), np.uint8)), \
            f"session {s}: sampler state"
        assert post["kv_len"][s] == pre["kv_len"][s] + 1 + na
        # frames and the next root
        v, c = post["tail"][s]
        last = int(e_ref[-1])
        fr = post["frames"][s]
        for j in range(na):
            node = p_ref[j]
            if e_ref[j] != EOS:
                assert np.array_equal(fr[j, 1:], post["codes_out"][s * R + node]), (s, j)
        if ne > na and last != EOS:
            if c >= 0:
                assert np.array_equal(fr[ne - 1, 1:], post["codes_out"][s * R + c])
            else:
                # the decoder's own frame on the hidden of row v (now prev_hidden)
                codes = np.zeros(10, np.int32)
                sem = np.array([last - SEM0 if SEM0 <= last < SEM0 + 4096 else 0], np.int32)
                s2pamd.check(lib.s2pfa_decode_frame_batch(
                    t.fa, ctypes.c_void_p(t.prev_hidden.data_ptr() + s * DIM * 2),
                    sem.ctypes.data, 1, codes.ctypes.data, S()), "decode")
                assert np.array_equal(fr[ne - 1, 1:], codes[1:]), (s, fr[ne - 1], codes)
        assert post["prev_tok"][s] == last
        assert np.array_equal(post["prev_codes"][s], fr[ne - 1])
        assert bool(post["done"][s]) == (last == EOS)


@pytest.mark.timeout(300)
def test_spec_ticks_graph_vs_host_rule(lib, tmp_path):
    """Two sessions x K=4, eight ticks from one graph; session 0 starts 12
    slots below its 512-slot span bucket, so a host re-plan (and re-capture)
    happens on the way."""
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        t = Tick(lib, tmp_path, 2, 4, [495, 301], seed=7)
        try:
            pre = t.snapshot()
            accepted = 0
            for k in range(8):
                print(f"tick {k}", flush=True)
                t.tick(1)
                post = t.snapshot()
                check_tick(lib, t, pre, post)
                accepted += int(np.maximum(post["n_acc"], 0).sum())
                pre = post
            s2pamd.check(lib.s2p_spec_buffers_of(t.sp, ctypes.byref(t.buf)))
            assert t.buf.replans >= 1, "the span bucket was never crossed"
            print("accepted drafted frames over 8 ticks:", accepted, "replans:", t.buf.replans)
        finally:
            t.free()
    torch.cuda.synchronize()


@pytest.mark.timeout(300)
def test_spec_ticks_high_acceptance(lib, tmp_path):
    """A near-identity backbone and a pass-through draft (Tick near_identity):
    drafts are mostly accepted, so the accepted-frame, bonus and chain
    bookkeeping of the tick is exercised; six graph ticks, each checked
    against the host rule."""
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        t = Tick(lib, tmp_path, 2, 4, [200, 333], seed=11, near_identity=True)
        try:
            pre = t.snapshot()
            accepted, chain_failed, ticks = 0, 0, 0
            for k in range(6):
                t.tick(1)
                post = t.snapshot()
                check_tick(lib, t, pre, post)
                live = pre["done"] == 0
                accepted += int(np.maximum(post["n_acc"][live], 0).sum())
                chain_failed += int((post["tail"][live, 1] >= 0).sum())
                ticks += int(live.sum())
                pre = post
            print(f"accepted drafted frames: {accepted} over {ticks} session-ticks of K=4; "
                  f"last token from a chain-failed node: {chain_failed}")
            assert accepted >= ticks, "drafts were not accepted"
        finally:
            t.free()
    torch.cuda.synchronize()


@pytest.mark.timeout(300)
def test_spec_graph_equals_eager(lib, tmp_path):
    """The same three ticks replayed from the graph and launched eagerly,
    from the same starting state, give identical outputs and states."""
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    runs = []
    with torch.cuda.stream(side):
        for use_graph in (1, 0):
            t = Tick(lib, tmp_path, 1, 4, [200], seed=9)
            try:
                out = []
                for _ in range(3):
                    t.tick(use_graph)
                    snap = t.snapshot()
                    out.append({k: v for k, v in snap.items()})
                runs.append(out)
            finally:
                t.free()
    torch.cuda.synchronize()
    R = 5
    for a, b in zip(*runs):
        for k in a:
            va, vb = a[k], b[k]
            if k == "tok":  # entry 0 of a session (the root) is not a drafted token
                va, vb = va.reshape(-1, R)[:, 1:], vb.reshape(-1, R)[:, 1:]
            if k == "drf":  # a session's last draft row (a leaf's) is never written
                va, vb = va.reshape(-1, R, va.shape[-1])[:, :R - 1], vb.reshape(-1, R, vb.shape[-1])[:, :R - 1]
            if isinstance(va, list):
                assert all(np.array_equal(x, y) for x, y in zip(va, vb)), k
            else:
                assert np.array_equal(va, vb), k
