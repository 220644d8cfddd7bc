"""fp16 GEMM sweep on one GPU: the tuned gfx950 kernel (the C ABI's gemm_f16 with the tile
mma.matmul picks from tune_table.json)
against torch.matmul (hipBLASLt on ROCm) on the same inputs, for the square sweep 1024..16384 and
the reference tests' K=256 shapes (test_mma.py). Inputs U[-1, 1] fp16, seeded; each figure is the
median per-launch time of back-to-back batches (about 2 ms of work per sample, 7 samples; the two
libraries alternate twice and each keeps its best), with the
relative Frobenius error of ours against an fp32 product.

Usage: python gemm_sweep.py [--json out.json]
"""
from __future__ import annotations

import argparse
import json
import statistics
import sys

import torch

import gfx950_configs as cfgs
import hip_lib

SHAPES = [(n, n, n) for n in (1024, 2048, 4096, 8192, 16384)] + [(1024, 1024, 256), (8192, 8192, 256)]


def _time(fn, batch_ms: float = 2.0, samples: int = 7) -> float:
    for _ in range(3):
        fn()
    torch.cuda.synchronize()

    def sample(n: int) -> float:
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(n):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / n

    n = max(1, min(200, round(batch_ms / max(sample(1), 1e-3))))
    return statistics.median(sample(n) for _ in range(samples))


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--json", default=None)
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("gemm_sweep.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    rows = []
    for M, N, K in SHAPES:
        g = torch.Generator().manual_seed(M * 31 + K)
        a = (torch.rand(M, K, generator=g) * 2 - 1).half().to(dev)
        b = (torch.rand(K, N, generator=g) * 2 - 1).half().to(dev)
        c = torch.empty(M, N, dtype=torch.float16, device=dev)
        flops = 2.0 * M * N * K
        tile = cfgs.choose_gemm_tile_any(M, N, K)  # what mma.matmul launches
        gt = hip_lib.GemmTile(*tile)
        # alternate the two measurements (power and clock drift between them) and keep each best
        ms_ours = ms_torch = float("inf")
        for _ in range(2):
            ms_ours = min(ms_ours, _time(lambda: hip_lib.gemm_f16(a, b, c, gt)))
            ms_torch = min(ms_torch, _time(lambda: torch.matmul(a, b)))
        ref = a.float() @ b.float()
        rel = ((c.float() - ref).norm() / ref.norm()).item()
        row = {"M": M, "N": N, "K": K, "tile": list(tile), "ms": round(ms_ours, 4),
               "tflops": round(flops / ms_ours / 1e9, 1), "ms_torch": round(ms_torch, 4),
               "tflops_torch": round(flops / ms_torch / 1e9, 1), "ratio_vs_torch": round(ms_torch / ms_ours, 3),
               "rel_fro": rel}
        rows.append(row)
        print(f"[gemm_sweep] {M}x{N}x{K} tile={tile}: ours {row['tflops']} TFLOP/s, torch.matmul "
              f"{row['tflops_torch']} TFLOP/s ({row['ratio_vs_torch']}x), rel_fro={rel:.1e}", flush=True)
        del a, b, c, ref
        torch.cuda.empty_cache()
    if args.json:
        with open(args.json, "w") as fh:
            json.dump(rows, fh, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
