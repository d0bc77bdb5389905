"""Profiling driver for rocprofv3 runs of the tb.matmul gfx950 kernels.

Runs, on one stream and in this order:
  1. `--copy-reps` device-to-device copies of a `--copy-mib` MiB buffer
     (torch's copy kernel; known bytes read and written, used to calibrate
     the FETCH_SIZE / WRITE_SIZE counters into HBM bytes);
  2. `--reps` launches of the workload's GEMM through the C ABI.

Usage (under rocprofv3, the program after `--`):
  rocprofv3 --pmc FETCH_SIZE -d out/pmc -- \
      python3 -m mini_triton_nvgpu_v1_amd.profiling --workload gemm_4096

`--small-tiles` instead launches single-tile problems of the reference's
small cases (64x64, 64x128 and 128x64 tiles on the wave counts its configs
name, the 64x64 tile on 4 waves beside its 1, and 128x128 on both MFMA
shapes) as f16 C, plain f32 C and f32 C += A*B, `--reps` times each, back to
back: a kernel trace of it shows what the output mode, the wave count and
the MFMA shape cost at the size where a launch is all latency.
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
    ap.add_argument("--small-tiles", action="store_true",
                    help="single-tile problems of the reference's small cases")
    args = ap.parse_args()

    import torch

    import mini_triton_nvgpu_v1_amd as tb
    from mini_triton_nvgpu_v1_amd import configs

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    if args.small_tiles:
        return small_tiles(tb, torch, dev, stream, args.reps)
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


# (M, N, K, block_m, block_n, block_k, wave grid m, wave grid n, MFMA
# 16x16x32): one tile each
SMALL_TILES = [(64, 64, 32, 64, 64, 32, 1, 1, False), (64, 64, 32, 64, 64, 32, 2, 2, False),
               (64, 64, 64, 64, 64, 32, 1, 1, False), (64, 64, 64, 64, 64, 64, 1, 1, False),
               (128, 64, 32, 128, 64, 32, 4, 1, False), (64, 128, 32, 64, 128, 32, 1, 4, False),
               (128, 128, 32, 128, 128, 32, 2, 2, True), (128, 128, 32, 128, 128, 32, 2, 2, False),
               (128, 128, 64, 128, 128, 64, 2, 2, True), (128, 128, 64, 128, 128, 64, 2, 2, False)]


def small_tiles(tb, torch, dev, stream, reps) -> int:
    for (M, N, K, bm, bn, bk, gm, gn, m16) in SMALL_TILES:
        A = torch.empty((M, K), dtype=torch.float16, device=dev)
        B = torch.empty((K, N), dtype=torch.float16, device=dev)
        tb.fill_seeded_f16(A, M, K, 0x5EED0A00 + K, 0, 1.0, stream=stream)
        tb.fill_seeded_f16(B, K, N, 0x5EED0B00 + N, 0, 1.0, stream=stream)
        for out in (0, 1, 2):  # f16 C, plain f32 C, f32 C += A*B
            cfg = tb.GemmConfig(
                m=M, n=N, k=K, lda=K, ldb=N, ldc=N,
                c_dtype=tb.DTYPE_F16 if out == 0 else tb.DTYPE_F32,
                acc_init=tb.ACC_INIT_LOAD_C if out == 2 else tb.ACC_INIT_ZERO,
                block_m=bm, block_n=bn, block_k=bk, num_waves=gm * gn, wave_grid_m=gm,
                wave_grid_n=gn, stages=2, mapping=tb.MAP_TILE, group_m=1, split_k=1,
                reduction=tb.RED_NONE, num_programs=1, xcd_remap=0,
                mfma=tb.MFMA_16X16X32 if m16 else tb.MFMA_32X32X16)
            desc = tb.GemmDesc.from_config(cfg)
            C = torch.zeros((M, N), dtype=torch.float16 if out == 0 else torch.float32,
                            device=dev)
            for _ in range(reps):
                desc.launch(A, B, C, stream=stream)
            torch.cuda.synchronize()
            print(f"profiling: {reps} launches of {desc.kernel_name} ({M}x{N}x{K})",
                  flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
