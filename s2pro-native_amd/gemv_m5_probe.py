"""Timing driver for the M = 5 INT4-g32 GEMV of the verify step (config 3:
the four layer shapes of the 36-layer backbone), used to compare the
product library with its measurement variant `libs2pamd_dot2.so`
(`make dot2`: the main product of the transposed tile on the VALU with
v_dot2_f32_bf16 instead of the MFMA).  Run it under rocprofv3 for kernel
durations and instruction counters:

    python s2pro-native_amd/gemv_m5_probe.py [--lib PATH] [--reps N]

Random weights and activations; prints one line per shape with the mean
time per GEMV from HIP events and a checksum of the outputs."""
import argparse
import ctypes
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SHAPES = [(6144, 2560), (2560, 4096), (19456, 2560), (2560, 9728)]  # wqkv, wo, gate_up, w2


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib", default=None, help="library to load (default: the in-tree build)")
    ap.add_argument("--reps", type=int, default=200)
    args = ap.parse_args()
    if args.lib:
        os.environ["S2PAMD_LIB"] = os.path.abspath(args.lib)
    sys.path.insert(0, HERE)
    import torch
    import s2pamd
    lib = s2pamd.load()
    s2pamd.check(lib.s2p_gemm_init(128), "gemm init")
    dev = torch.device("cuda:0")
    S = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    M = 5
    g = torch.Generator(device="cpu").manual_seed(5)
    for N, K in SHAPES:
        w = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, generator=g).to(dev)
        sc = (torch.randn((N, K // 32), generator=g).abs() * 0.02).to(torch.float16).to(dev)
        x = torch.randn((M, K), generator=g).to(torch.bfloat16).to(dev)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

        def run():
            s2pamd.check(lib.s2p_int4p_gemv(y.data_ptr(), x.data_ptr(), w.data_ptr(), sc.data_ptr(),
                                            M, N, K, 32, S), "gemv")
        for _ in range(10):
            run()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.reps):
            run()
        e1.record()
        torch.cuda.synchronize()
        print(f"M={M} N={N} K={K}: {e0.elapsed_time(e1) * 1e3 / args.reps:.2f} us per GEMV, "
              f"checksum {y.float().abs().sum().item():.6e}", flush=True)


if __name__ == "__main__":
    main()
