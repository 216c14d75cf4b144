"""Verify-step benchmark of the MI355X speculative verify path.

Workload (the north-star metric): one session, K=4
draft tokens (M = 5 verify rows) through the 36-layer INT4-g32 slow-AR
backbone against a bf16 KV cache of 2048 tokens, the INT4 lm head
2560 -> 155,776, then device acceptance sampling (T 0.8, top-p 0.8) of the 4
drafted tokens against draft logits = target logits + N(0, 0.5).  Random-init
weights, synthetic inputs resident in HBM before the timed region.  A step is
one replay of the captured hipGraph (forward + acceptance).

Prints one JSON line (see README of the driver contract): value = verify
steps/s, plus `roofline` for the dominant kernel timed with HIP events on its
own stream (the persistent verify kernel k_mk2, the whole forward in one
launch, when the plan runs on it; otherwise the INT4 GEMV engine's 145 weight
GEMVs of a step), and `cpu_baseline` (the scalar C oracle on one host core
over a bounded sample: one backbone layer + 1/8 of the head GEMV,
extrapolated to 36 layers and the full head).

`--workload config4|config5` runs the batch (8 sessions x K=4, M = 40) and tree
(4 sessions x 16-node tree, M = 68, KV 8192) configurations the same way; their
lines are reported beside the headline, which stays config 3.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "s2pro-native_amd"))

import numpy as np  # noqa: E402

METRIC = "verify steps/s (36L INT4, K=4, b=1) + achieved HBM GB/s vs peak"
PEAK_GBS = 8000.0
N_LAYERS, CTX, K = 36, 2048, 4
# algorithmic bytes of one config-3 step (weights + KV + activations + logits)
W_LAYER = [(6144, 2560), (2560, 4096), (19456, 2560), (2560, 9728)]


def int4_bytes(N, Kd):
    return N * Kd // 2 + 2 * N * Kd // 32


TREE16 = [-1, 0, 0, 1, 1, 2, 2, 3, 3, 4, 5, 6, 6, 7, 8, 10, 11]
# sessions, per-session parent array, KV lengths, cache capacity
WORKLOADS = {
    "config3": dict(parent=[-1, 0, 1, 2, 3], lens=[CTX],
                    desc="config3: 36L INT4-g32 backbone + INT4 head 2560->155776, K=4 chain "
                         "(M=5), b=1, bf16 KV 2048, device acceptance T0.8 p0.8"),
    "config4": dict(parent=[-1, 0, 1, 2, 3],
                    lens=[int(v) for v in np.random.default_rng(4).integers(256, 4097, 8)],
                    desc="config4: 8 sessions x K=4 chain (M=40), 36L INT4-g32 + INT4 head, "
                         "KV lengths ~ U[256, 4096] (seed 4), per-session acceptance"),
    "config5": dict(parent=TREE16, lens=[8192] * 4,
                    desc="config5: 4 sessions x 16-node draft tree (M=68), 36L INT4-g32 + INT4 "
                         "head, KV 8192, tree acceptance"),
}


def kv_token_bytes(kv_bits=16):
    """Bytes of one cached token of one layer: K and V of 8 heads x 128 dims,
    bf16 (4,096 B), or INT8 / INT4 codes plus four f16 group scales per head
    (2,176 / 1,152 B)."""
    if kv_bits == 16:
        return 2 * 8 * 128 * 2
    return 2 * 8 * (128 * kv_bits // 8 + 8)


def step_alg_bytes(lens=(CTX,), rows=K + 1, kv_bits=16):
    """Weights and scales once, each cached KV token once (4,096 B per layer
    for bf16), activations and logits per row (3,887,360 B: 17,879,040 +
    1,557,760 at M = 5)."""
    w = N_LAYERS * sum(int4_bytes(n, k) for n, k in W_LAYER) + int4_bytes(155776, 2560)
    kv = N_LAYERS * kv_token_bytes(kv_bits) * sum(lens)
    act = rows * 3_887_360
    return w, kv, w + kv + act


TRAFFIC_FILES = {"gemv": "gemv_int4_config3_traffic.md", "mk2": "mk2_config3_traffic.md"}


def measured_traffic(kind):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (copy-calibrated); None if the
    summary is absent."""
    try:
        for line in open(os.path.join(ROOT, "profiles", TRAFFIC_FILES[kind])):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(budget_s=20.0):
    """Scalar C oracle (one core): one layer (4 GEMVs in the reference lane
    order, norms, RoPE, attention over 2048 slots, SwiGLU) plus the head GEMV,
    extrapolated as 36 x layer + head."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as po
    r = np.random.default_rng(0)
    M = K + 1
    lins, keep = [], []
    for n, k in W_LAYER:
        w = r.integers(0, 256, (n, k // 2), dtype=np.uint8)
        s = np.abs(r.standard_normal((n, k // 32)) * 0.02).astype(np.float16).view(np.uint16)
        keep.append((w, s))
        lins.append(po.make_linear(w, s, n, k, 32))
    norms = [po.f32_to_bf16(np.ones(d, np.float32)) for d in (2560, 2560, 128, 128)]
    lw = po.OrLayerW(*lins, *(po.ptr(x) for x in norms))
    kc = po.f32_to_bf16(r.standard_normal((8, CTX + M, 128)).astype(np.float32))
    vc = po.f32_to_bf16(r.standard_normal((8, CTX + M, 128)).astype(np.float32))
    x = po.f32_to_bf16(r.standard_normal((M, 2560)).astype(np.float32))
    pos = np.arange(CTX, CTX + M, dtype=np.int32)
    t0 = time.perf_counter()
    po.layer(lw, x, M, kc, vc, CTX + M, CTX, pos)
    t_layer = time.perf_counter() - t0
    hw = r.integers(0, 256, (155776 // 8, 1280), dtype=np.uint8)  # 1/8 of the head rows
    hs = np.abs(r.standard_normal((155776 // 8, 80)) * 0.02).astype(np.float16).view(np.uint16)
    t0 = time.perf_counter()
    po.int4p_gemv(x, hw, hs, M, 155776 // 8, 2560)
    t_head = (time.perf_counter() - t0) * 8
    step = N_LAYERS * t_layer + t_head
    return {"value": round(1.0 / step, 6), "unit": "steps/s", "cores": 1, "kind": "port",
            "host_cpus_online": os.sysconf("SC_NPROCESSORS_ONLN"), "host_cpu_model": _cpu_model(),
            "sample": f"1 of 36 layers ({t_layer:.2f} s) + 1/8 of the head GEMV, scalar C "
                      f"oracle at -O2, extrapolated to 36 layers + full head "
                      f"({step:.1f} s per step)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--workload", default="config3", choices=sorted(WORKLOADS) + ["tick"],
                    help="config3 (the headline metric), the batch / tree configs 4, 5, or "
                         "tick: the composed speculative tick on the config-3 backbone")
    ap.add_argument("--kv-bits", type=int, default=16, choices=[16, 8, 4],
                    help="session KV cache: bf16 (16) or the INT8 / INT4 quantised cache")
    ap.add_argument("--copy-calib", action="store_true",
                    help="only run a plain 256 MiB device copy (3 launches): the reference "
                         "dispatch that scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one MI355X; --gpus must be 1 "
                          "(sessions shard across GPUs with no collectives: one process per GPU, "
                          "each on its own sessions)"}))
        sys.exit(2)

    import torch
    if args.copy_calib:
        a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        a.fill_(1)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes_read": a.numel(), "copy_calib_bytes_written": b.numel(),
                          "launches": 3}))
        return
    import s2pamd
    lib = s2pamd.load()
    if args.workload == "tick":
        tick_bench(lib, args)
        return
    dev = torch.device("cuda:0")
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        S = s2pamd.stream_ptr()
        wl = WORKLOADS[args.workload]
        parent = np.array(wl["parent"], np.int32)
        lens = wl["lens"]
        NS, R = len(lens), len(parent)
        M = NS * R
        ctx = max(lens) + 64
        opts = s2pamd.BackboneOpts(N_LAYERS, s2pamd.WQ_INT4, s2pamd.WQ_INT4, s2pamd.S2P_VOCAB,
                                   max(16, M), NS, ctx, args.kv_bits)
        bb = ctypes.c_void_p()
        s2pamd.check(lib.s2p_backbone_create_random(ctypes.byref(opts), 2026, S, ctypes.byref(bb)))
        kvs, scs = [], []
        for s_ in range(NS):
            kv = torch.empty(lib.s2p_backbone_kv_bytes(bb) // 2, dtype=torch.int16, device=dev)
            s2pamd.hip_check(lib.s2p_synth_bf16_normal(s2pamd.dptr(kv), kv.numel(), 0.0, 1.0,
                                                       5 + s_, S))
            kvs.append(kv)
            if args.kv_bits != 16:
                # quantised cache: random codes, every group scale f16 0.01
                sc = torch.full((lib.s2p_backbone_kv_scale_bytes(bb) // 2,), 0x211F,
                                dtype=torch.int16, device=dev)
                scs.append(sc)
        kvp = (ctypes.c_void_p * NS)(*[k.data_ptr() for k in kvs])
        scp = (ctypes.c_void_p * NS)(*[c.data_ptr() for c in scs]) if scs else None
        ln = np.array(lens, np.int32)
        vb = s2pamd.VerifyBatch(NS, R, parent.ctypes.data, ctypes.addressof(kvp), ln.ctypes.data,
                                ctypes.addressof(scp) if scp is not None else None)
        s2pamd.check(lib.s2p_verify_plan(bb, ctypes.byref(vb), S))
        x = torch.empty((M, 2560), dtype=torch.int16, device=dev)
        s2pamd.hip_check(lib.s2p_synth_bf16_normal(s2pamd.dptr(x), x.numel(), 0.0, 1.0, 9, S))
        logits = torch.empty((M, s2pamd.S2P_VOCAB), dtype=torch.int16, device=dev)
        s2pamd.check(lib.s2p_verify_forward(bb, s2pamd.dptr(x), s2pamd.dptr(logits), S))
        # draft logits: target + N(0, 0.5); drafted ids by the device sampler
        noise = torch.empty_like(logits)
        s2pamd.hip_check(lib.s2p_synth_bf16_normal(s2pamd.dptr(noise), noise.numel(), 0.0, 0.5,
                                                   13, S))
        drf = (logits.view(torch.bfloat16).float() + noise.view(torch.bfloat16).float()).to(
            torch.bfloat16).view(torch.int16)
        # per-session sampler states (seeds differ); drafted ids: the device
        # sampler on each node's parent draft row
        d_states, d_drafts = [], []
        for s_ in range(NS):
            st = StateBytes.make(0.8, 0.8, 1.1, 16, seed=s_, entropy=s_)
            d_states.append(torch.from_numpy(np.frombuffer(bytes(st), np.uint8).copy()).to(dev))
            d_drafts.append(d_states[-1].clone())
        d_sptr = torch.tensor([t.data_ptr() for t in d_states], dtype=torch.int64, device=dev)
        tok = torch.zeros(M, dtype=torch.int64, device=dev)
        sem = torch.zeros(1, dtype=torch.int32, device=dev)
        eos = torch.zeros(1, dtype=torch.uint8, device=dev)
        for s_ in range(NS):
            d_dptr = torch.tensor([d_drafts[s_].data_ptr()], dtype=torch.int64, device=dev)
            for i in range(1, R):
                s2pamd.hip_check(lib.s2pk_sample(s2pamd.dptr(drf[s_ * R + int(parent[i])]),
                                                 s2pamd.S2P_VOCAB, None, s2pamd.dptr(d_dptr), 1,
                                                 ctypes.c_void_p(tok.data_ptr() +
                                                                 8 * (s_ * R + i)),
                                                 s2pamd.dptr(sem), None, s2pamd.dptr(eos), S))
            side.synchronize()
        d_parent = torch.from_numpy(parent).to(dev)
        work = torch.empty(lib.s2p_verify_accept_work_bytes(NS, R), dtype=torch.uint8,
                           device=dev)
        path = torch.zeros(M, dtype=torch.int32, device=dev)
        nacc = torch.zeros(NS, dtype=torch.int32, device=dev)
        emit = torch.zeros(NS * (R + 1), dtype=torch.int64, device=dev)
        nemit = torch.zeros(NS, dtype=torch.int32, device=dev)
        io = s2pamd.StepIO(x.data_ptr(), logits.data_ptr(), drf.data_ptr(), s2pamd.S2P_VOCAB,
                           d_parent.data_ptr(), tok.data_ptr(), d_sptr.data_ptr(), path.data_ptr(),
                           nacc.data_ptr(), emit.data_ptr(), nemit.data_ptr(), work.data_ptr())

        def step():
            s2pamd.check(lib.s2p_verify_step(bb, ctypes.byref(io), 1, S), "verify step")

        for _ in range(args.warmup):
            step()
        side.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(side)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        e1.record(side)
        side.synchronize()
        wall = time.perf_counter() - t0
        ms = e0.elapsed_time(e1) / args.steps

        # the timed steps must all have completed: a bounded flag wait of the
        # persistent kernel that gave up makes a launch drain early (faster and
        # wrong), so such a run reports no number
        mk_status = lib.s2p_backbone_mk_status(bb)
        n_acc_last = nacc.cpu().numpy()
        if mk_status < 0 or np.any(n_acc_last < 0):
            print(json.dumps({"error": "a flag wait of the persistent verify kernel timed out "
                              "during the timed steps; no number is reported",
                              "mk_status": int(mk_status)}), flush=True)
            sys.exit(3)
        mk2 = mk_status == 1
        if mk2:
            # dominant kernel: the persistent verify kernel k_mk2, the whole forward
            # (36 layers + head) in one launch; back-to-back launches on this stream,
            # bracketed by HIP events
            reps = 50
            g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            g0.record(side)
            for _ in range(reps):
                s2pamd.check(lib.s2p_verify_forward(bb, s2pamd.dptr(x), s2pamd.dptr(logits), S))
            g1.record(side)
            side.synchronize()
            avg_launch_s = g0.elapsed_time(g1) / 1e3 / reps
            if lib.s2p_backbone_mk_status(bb) != 1:
                print(json.dumps({"error": "a flag wait of the persistent verify kernel timed "
                                  "out during the roofline launches; no number is reported"}),
                      flush=True)
                sys.exit(3)
            _, _, per_launch = step_alg_bytes(lens, M, args.kv_bits)
            kern_gbs = per_launch / avg_launch_s / 1e9
            kern_name = "k_mk2 (persistent verify forward: 36 layers + head, one launch)"
        # otherwise the GEMV engine is the dominant kernel: every weight GEMV of one
        # step (36 x {wqkv, wo, gate_up, w2} + head at the step's M), replayed as one
        # graph on this stream and bracketed by HIP events
        if not mk2:
            lins = []
            for l in range(N_LAYERS):
                L = lib.s2p_backbone_layer(bb, l).contents
                lins += [L.wqkv, L.wo, L.gate_up, L.w2]
            lins.append(lib.s2p_backbone_head(bb).contents)
            ybuf = torch.empty((M, s2pamd.S2P_VOCAB), dtype=torch.int16, device=dev)
            xbuf = torch.empty((M, 9728), dtype=torch.int16, device=dev)
            s2pamd.hip_check(lib.s2p_synth_bf16_normal(s2pamd.dptr(xbuf), xbuf.numel(), 0.0, 1.0, 3, S))

            def gemvs():
                for lin in lins:
                    s2pamd.check(lib.s2p_linear_forward(ctypes.byref(lin), s2pamd.dptr(xbuf),
                                                        s2pamd.dptr(ybuf), M, 2, S), "gemv")
            gemvs()
            side.synchronize()
            # the 145 launches captured once and replayed: the events then time
            # the kernels back to back, not the host's per-launch call overhead
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                gemvs()
            graph.replay()
            side.synchronize()
            reps = 5
            g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            g0.record(side)
            for _ in range(reps):
                graph.replay()
            g1.record(side)
            side.synchronize()
            del graph
            n_launch = reps * len(lins)
            avg_launch_s = g0.elapsed_time(g1) / 1e3 / n_launch
            wbytes = sum(lin.w_pack.bytes + lin.w_iscale.bytes for lin in lins)
            abytes = sum(2 * M * (lin.in_features + lin.out_features) for lin in lins)
            per_launch = (wbytes + abytes) / len(lins)
            kern_gbs = per_launch / avg_launch_s / 1e9
            # M <= 16 rows run on the GEMV engine, 16 < M <= 96 on k_gemm4
            mt = (M + 15) // 16
            kern_name = ((f"k_gemv3<INT4, MT={mt}>" if M <= 16 else f"k_gemm4<MT={mt}>") +
                         " (all 145 weight GEMVs of a step, layer path)")
        lib.s2p_backbone_free(bb)

    w, kvb, alg = step_alg_bytes(lens, M, args.kv_bits)
    step_gbs = alg / (ms / 1e3) / 1e9
    headline = args.workload == "config3" and args.kv_bits == 16
    kvname = "" if args.kv_bits == 16 else f", INT{args.kv_bits} KV"
    out = {
        "metric": METRIC if headline else f"verify steps/s ({args.workload}, 36L INT4{kvname})",
        "value": round(1e3 / ms, 3),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init INT4-g32 weights, N(0,1) KV cache and inputs)",
        "config": {"workload": wl["desc"] + kvname, "global_batch": NS, "seq_len": max(lens),
                   "parallelism": "single GPU"},
        "step_alg_bytes": alg,
        "step_hbm_gbs": round(step_gbs, 1),
        "step_frac_of_peak": round(step_gbs / PEAK_GBS, 4),
        "wall_s_timed": round(wall, 3),
        # 1: the step ran on the persistent kernel and no bounded wait timed out
        # (checked after the timed region); 0: the layer-by-layer forward
        "mk_status": int(mk_status),
        "roofline": {"bound": "hbm", "achieved": round(kern_gbs, 1), "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": round(kern_gbs / PEAK_GBS, 4),
                     "traffic": measured_traffic("mk2" if mk2 else "gemv") if headline else None,
                     "traffic_source": ("profiles/" + TRAFFIC_FILES["mk2" if mk2 else "gemv"])
                     if headline else None,
                     "kernel": kern_name,
                     "avg_launch_us": round(avg_launch_s * 1e6, 3),
                     "alg_bytes_per_launch": int(per_launch)},
    }
    if headline and not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


def tick_bench(lib, args):
    """The composed speculative tick (s2p_spec_tick) on config 3's backbone
    (36L INT4-g32, full head, bf16 KV 2048, one session, K = 4) with a random
    draft model (bf16, the trainer's shapes), a random INT4 fast-AR decoder
    and a random bf16 token embedding: draft steps + draft head + draft
    sampling + drafted frames' fast-AR codes, the verify forward, the chain
    condition, acceptance, the last frame's codes and the session update,
    replayed from one graph.  Reported beside the headline, not as it."""
    import tempfile
    import torch
    import s2pamd
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import draft_util as du
    dev = torch.device("cuda:0")
    K_, L0 = K, CTX
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        S = s2pamd.stream_ptr()
        opts = s2pamd.BackboneOpts(N_LAYERS, s2pamd.WQ_INT4, s2pamd.WQ_INT4, s2pamd.S2P_VOCAB,
                                   16, 1, 4096, 16)
        bb = ctypes.c_void_p()
        s2pamd.check(lib.s2p_backbone_create_random(ctypes.byref(opts), 2026, S, ctypes.byref(bb)))
        fa = ctypes.c_void_p()
        s2pamd.check(lib.s2pfa_create_random(ctypes.byref(fa), s2pamd.WQ_INT4, 16, 17, S))
        with tempfile.TemporaryDirectory() as td:
            path = os.path.join(td, "draft.safetensors")
            du.write_safetensors(path, du.make_weights(3))
            dm = s2pamd.DraftModel()
            s2pamd.check(lib.s2p_draft_load(ctypes.byref(dm), path.encode()), "draft")
        dst = (s2pamd.DraftState * 1)()
        s2pamd.check(lib.s2p_draft_state_init(ctypes.byref(dst[0])))
        embed = torch.empty(155776 * 2560, dtype=torch.int16, device=dev)
        s2pamd.hip_check(lib.s2p_synth_bf16_normal(s2pamd.dptr(embed), embed.numel(), 0.0, 0.05,
                                                   23, S))
        kv = torch.empty(lib.s2p_backbone_kv_bytes(bb) // 2, dtype=torch.int16, device=dev)
        s2pamd.hip_check(lib.s2p_synth_bf16_normal(s2pamd.dptr(kv), kv.numel(), 0.0, 1.0, 5, S))
        r = np.random.default_rng(0)
        kv_len = torch.tensor([L0], dtype=torch.int32, device=dev)
        prev_tok = torch.tensor([151678 + 17], dtype=torch.int64, device=dev)
        prev_codes = torch.from_numpy(r.integers(0, 4096, (1, 10)).astype(np.int32)).to(dev)
        prev_hidden = torch.empty(2560, dtype=torch.int16, device=dev)
        s2pamd.hip_check(lib.s2p_synth_bf16_normal(s2pamd.dptr(prev_hidden), 2560, 0.0, 1.0, 7, S))
        st = StateBytes.make(0.8, 0.8, 1.1, 16, seed=1, entropy=1)
        st_buf = torch.from_numpy(np.frombuffer(bytes(st), np.uint8).copy()).to(dev)
        states = torch.tensor([st_buf.data_ptr()], dtype=torch.int64, device=dev)
        done = torch.zeros(1, dtype=torch.uint8, device=dev)
        n_acc = torch.zeros(1, dtype=torch.int32, device=dev)
        n_emit = torch.zeros(1, dtype=torch.int32, device=dev)
        emit = torch.zeros(K_ + 2, dtype=torch.int64, device=dev)
        frames = torch.zeros((K_ + 2) * 10, dtype=torch.int32, device=dev)
        kvp = (ctypes.c_void_p * 1)(kv.data_ptr())
        m = s2pamd.SpecModel(bb, ctypes.addressof(dm), ctypes.addressof(dst), fa,
                             embed.data_ptr(), 1, K_)
        ss = s2pamd.SpecSessions(ctypes.addressof(kvp), kv_len.data_ptr(), prev_tok.data_ptr(),
                                 prev_codes.data_ptr(), prev_hidden.data_ptr(),
                                 states.data_ptr(), done.data_ptr())
        o = s2pamd.SpecOut(n_acc.data_ptr(), n_emit.data_ptr(), emit.data_ptr(),
                           frames.data_ptr())
        sp = ctypes.c_void_p()
        lens = np.array([L0], np.int32)
        s2pamd.check(lib.s2p_spec_create(ctypes.byref(sp), ctypes.byref(m), ctypes.byref(ss),
                                         lens.ctypes.data, ctypes.byref(o), S), "spec create")
        for _ in range(max(2, args.warmup // 5)):
            s2pamd.check(lib.s2p_spec_tick(sp, 1, S), "tick")
        side.synchronize()
        steps = max(5, args.steps // 10)
        emitted = 0
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(side)
        for _ in range(steps):
            s2pamd.check(lib.s2p_spec_tick(sp, 1, S), "tick")
        e1.record(side)
        side.synchronize()
        ms = e0.elapsed_time(e1) / steps
        emitted = int(kv_len.cpu()[0]) - L0  # frames advanced over warmup + timed ticks
        mk_status = lib.s2p_backbone_mk_status(bb)
        buf = s2pamd.SpecBuffers()
        s2pamd.check(lib.s2p_spec_buffers_of(sp, ctypes.byref(buf)))
        lib.s2p_spec_free(sp)
        lib.s2p_draft_state_free(ctypes.byref(dst[0]))
        lib.s2p_draft_free(ctypes.byref(dm))
        lib.s2pfa_free(fa)
        lib.s2p_backbone_free(bb)
    if mk_status < 0:
        print(json.dumps({"error": "a flag wait timed out during the ticks"}), flush=True)
        sys.exit(3)
    total = steps + max(2, args.warmup // 5)
    print(json.dumps({
        "metric": "speculative ticks/s (config-3 backbone, K=4, draft + fast-AR chain)",
        "value": round(1e3 / ms, 3), "unit": "ticks/s", "n_gpus": 1, "steps": steps,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init backbone, draft, fast-AR and embedding)",
        "config": {"workload": "tick: 36L INT4-g32 + full INT4 head, bf16 KV from 2048, b=1, "
                               "K=4 drafts (random draft model), chain condition, T0.8 p0.8",
                   "global_batch": 1, "seq_len": L0, "parallelism": "single GPU"},
        "frames_per_tick": round(emitted / total, 3), "host_replans": buf.replans,
        "mk_status": int(mk_status)}), flush=True)


class StateBytes(ctypes.Structure):
    """s2ps_dev_state byte layout (include/s2pro/slowar_kernels.h)."""
    _fields_ = [("prev", ctypes.c_int64 * 64), ("count", ctypes.c_uint64),
                ("rng", ctypes.c_uint64 * 4), ("temperature", ctypes.c_float),
                ("top_p", ctypes.c_float), ("rep_penalty", ctypes.c_float),
                ("window", ctypes.c_int32), ("seeded", ctypes.c_int32),
                ("seed31", ctypes.c_uint32), ("pad_", ctypes.c_uint32)]

    @classmethod
    def make(cls, temperature, top_p, rep_penalty, window, seed, entropy):
        """Initial sampler state (reference sampling.c:95-112)."""
        st = cls()
        st.temperature, st.top_p, st.rep_penalty = temperature, top_p, rep_penalty
        st.window = window
        st.seeded = 1 if seed else 0
        st.seed31 = seed & 0x7FFFFFFF
        sm = (entropy ^ 0xD1B54A32D192ED03) & (2 ** 64 - 1)
        for i in range(4):
            sm = (sm + 0x9E3779B97F4A7C15) & (2 ** 64 - 1)
            z = sm
            z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2 ** 64 - 1)
            z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2 ** 64 - 1)
            st.rng[i] = z ^ (z >> 31)
        return st


if __name__ == "__main__":
    main()
