"""Profiling driver for rocprofv3 runs of the tb.matmul gfx950 kernels.

Runs, on one stream and in this order:
  1. `--copy-reps` device-to-device copies of a `--copy-mib` MiB buffer
     (torch's copy kernel; known bytes read and written, used to calibrate
     the FETCH_SIZE / WRITE_SIZE counters into HBM bytes);
  2. `--reps` launches of the workload's GEMM through the C ABI.

Usage (under rocprofv3, the program after `--`):
  rocprofv3 --pmc FETCH_SIZE -d out/pmc -- \
      python3 -m mini_triton_nvgpu_v1_amd.profiling --workload gemm_4096
"""
from __future__ import annotations

import argparse
import sys


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="gemm_4096")
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--copy-mib", type=int, default=256)
    ap.add_argument("--copy-reps", type=int, default=3)
    ap.add_argument("--hipblaslt", action="store_true",
                    help="also run torch.matmul on the same operands")
    args = ap.parse_args()

    import torch

    import mini_triton_nvgpu_v1_amd as tb
    from mini_triton_nvgpu_v1_amd import configs

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    n = args.copy_mib * 1024 * 1024
    src = torch.ones(n, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(args.copy_reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"profiling: {args.copy_reps} copies of {args.copy_mib} MiB", flush=True)

    w = configs.BY_NAME[args.workload]
    desc = tb.plan_from_mlir(w.mlir())
    A = torch.empty((w.M, w.K), dtype=torch.float16, device=dev)
    B = torch.empty((w.K, w.N), dtype=torch.float16, device=dev)
    C = torch.zeros((w.M, w.N), dtype=torch.float32 if w.c_f32 else torch.float16,
                    device=dev)
    ws = (torch.empty(desc.workspace_bytes, dtype=torch.uint8, device=dev)
          if desc.workspace_bytes else None)
    tb.fill_seeded_f16(A, w.M, w.K, w.seed, w.dist, w.scale, stream=stream)
    tb.fill_seeded_f16(B, w.K, w.N, w.seed_b, w.dist, w.scale, stream=stream)
    bias = None
    if w.bias:  # fused bias step: N seeded values
        bias = torch.empty((1, w.N), dtype=torch.float16, device=dev)
        tb.fill_seeded_f16(bias, 1, w.N, w.seed ^ 0xB1A5, 0, 1.0, stream=stream)
        if w.bias == "f32":
            bias = bias.float()
    for _ in range(args.reps):
        desc.launch(A, B, C, ws, stream=stream, bias=bias)
    torch.cuda.synchronize()
    print(f"profiling: {args.reps} launches of {desc.kernel_name} ({w.name})", flush=True)
    if args.hipblaslt and not w.c_f32:
        # the vendor library on the same operands, for side-by-side counters
        for _ in range(args.reps):
            torch.matmul(A, B, out=C)
        torch.cuda.synchronize()
        print(f"profiling: {args.reps} torch.matmul (hipBLASLt) launches", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
