"""Attention pipeline cases in the reference test's `[case]` log format.

The reference's pipeline test (test_flash_atten.py:86-115, 270-305) times its kernels and torch's
SDPA backends on large shapes and writes one line per case:

    [case] status=ok B=1 H=28 S=8192 D=128 causal=False | cpu_sdpa mean=n/a p50=n/a | gpu_math_sdpa
    mean=...ms p50=...ms | ... | triton_flash_block_d_nomask mean=...ms p50=...ms | ...

Its plot helpers parse those lines by series name (KERNEL_RUNTIME_SERIES keys). This script runs the
same cases on the MI355X with the gfx950 kernels under the reference's series names
(triton_flash_basic / triton_flash_opt_shared_mem / triton_flash_block_d_nomask = the basic,
optimized and sliced variants here) and torch's math / efficient / flash SDPA backends, and writes
lines the reference's `_parse_flash_atten_kernel_pipeline_rows` reads unchanged. Backends that are
unavailable, or would need more than --math-limit-gb of scores (the math backend materialises
B*H*S*S fp32), are reported as n/a, as the reference does for skipped kernels.

Usage: python case_log.py [--log pipeline.log] [--cases large|small]
"""
from __future__ import annotations

import argparse
import statistics
import sys

import torch
import torch.nn.functional as F

import flash_atten
import tuner

# the reference's PIPELINE_CASES (test_flash_atten.py:83-88): (B, H, D, S, causal)
LARGE_CASES = [(1, 28, 128, s, False) for s in (1024, 8192, 16384, 32768, 65536)] + \
              [(1, 16, 256, s, False) for s in (1024, 8192, 16384, 32768, 65536)]
SMALL_CASES = [(1, 4, 64, s, c) for s in (128, 512) for c in (False, True)]

SERIES = ["cpu_sdpa", "gpu_math_sdpa", "gpu_efficient_sdpa", "gpu_flash_sdpa", "triton_flash_basic",
          "triton_flash_opt_shared_mem", "triton_flash_block_d_nomask"]
VARIANT_BY_SERIES = {"triton_flash_basic": "basic", "triton_flash_opt_shared_mem": "optimized",
                     "triton_flash_block_d_nomask": "sliced"}


def _stats(fn, warmup: int, iters: int) -> dict[str, float]:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(iters):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        torch.cuda.synchronize()
        times.append(s.elapsed_time(e))
    return {"mean_ms": statistics.mean(times), "p50_ms": statistics.median(times)}


def run_case(case, *, warmup: int, iters: int, math_limit_gb: float, seed: int = 20260328) -> str:
    from torch.nn.attention import SDPBackend, sdpa_kernel

    B, H, D, S, causal = case
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, H, S, D, generator=g, dtype=torch.float16).to(dev) for _ in range(3))
    stats: dict[str, dict | None] = {name: None for name in SERIES}
    details: dict[str, str] = {}
    ref = None
    for name in SERIES:
        if name == "cpu_sdpa":
            continue  # the host path is the bench's cpu_baseline leg; too slow at these sizes
        if name in VARIANT_BY_SERIES:
            # launch spec built once (as the reference test does), then only the launch is timed
            cls = {"basic": tuner.FlashAttentionTuner, "optimized": tuner.FlashAttentionOptimizeSharedMemTuner,
                   "sliced": tuner.FlashAttentionBlockDNomaskTuner}[VARIANT_BY_SERIES[name]]
            spec = cls(tuple(q.shape), tuple(k.shape), tuple(v.shape), q.element_size(), causal=causal,
                       return_lse=False).build_flash_attention_launch_spec(q, k, v)
            fn = lambda spec=spec: flash_atten.flash_attention(spec)  # noqa: E731
        else:
            if name == "gpu_math_sdpa" and B * H * S * S * 4 * 3 / 2 ** 30 > math_limit_gb:
                details[name] = "skipped(size)"
                continue
            backend = {"gpu_math_sdpa": SDPBackend.MATH, "gpu_efficient_sdpa": SDPBackend.EFFICIENT_ATTENTION,
                       "gpu_flash_sdpa": SDPBackend.FLASH_ATTENTION}[name]

            def fn(backend=backend):
                with sdpa_kernel(backend):
                    return F.scaled_dot_product_attention(q, k, v, is_causal=causal)
        try:
            out = fn()
            torch.cuda.synchronize()
        except RuntimeError as exc:  # backend not available for this shape / build
            details[name] = "unavailable"
            print(f"[case_log] {name} B={B} H={H} S={S} D={D}: {str(exc).splitlines()[0][:100]}", file=sys.stderr)
            continue
        if ref is None:
            ref = out.float()
        else:
            details[name] = f"max_abs_diff={(out.float() - ref).abs().max().item():.2e}"
        stats[name] = _stats(fn, warmup, iters)
    del q, k, v, ref
    torch.cuda.empty_cache()
    return format_case_line(case, stats, details)


def format_case_line(case, stats: dict, details: dict) -> str:
    """One `[case]` line (the layout of test_flash_atten.py:98-115): per series `name [detail]
    mean=Xms p50=Yms` or `mean=n/a p50=n/a`, then speed ratios and TFLOP/s of the gfx950 kernels."""
    B, H, D, S, causal = case
    summary = []
    for name in SERIES:
        label = f"{name} {details[name]}" if name in details else name
        st = stats.get(name)
        summary.append(f"{label} mean={st['mean_ms']:.3f}ms p50={st['p50_ms']:.3f}ms" if st else f"{label} mean=n/a p50=n/a")
    ours = stats.get("triton_flash_opt_shared_mem")
    ratios = []
    for other in ("gpu_flash_sdpa", "gpu_efficient_sdpa", "gpu_math_sdpa"):
        if ours and stats.get(other):
            ratios.append(f"opt_shared_mem_vs_{other}={stats[other]['mean_ms'] / ours['mean_ms']:.2f}x")
    flops = 4.0 * B * H * D * (S * (S + 1) / 2 if causal else S * S)
    statuses = [f"{name}_tflops={flops / st['mean_ms'] / 1e9:.1f}" for name, st in stats.items()
                if st and name in VARIANT_BY_SERIES]
    return (f"[case] status=ok B={B} H={H} S={S} D={D} causal={causal} | " + " | ".join(summary + ratios + statuses))


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--log", default=None, help="append the [case] lines to this file")
    ap.add_argument("--cases", choices=["large", "small"], default="large")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--iters", type=int, default=10)
    ap.add_argument("--math-limit-gb", type=float, default=48.0)
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("case_log.py needs a GPU (gfx950)", file=sys.stderr)
        return 1
    cases = LARGE_CASES if args.cases == "large" else SMALL_CASES
    for case in cases:
        line = run_case(case, warmup=args.warmup, iters=args.iters, math_limit_gb=args.math_limit_gb)
        print(line, flush=True)
        if args.log:
            with open(args.log, "a") as fh:
                fh.write(line + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
