"""Decode-shaped attention on MI355X: a few query rows against a long KV cache, through the sliced
variant (split-KV + LSE merge, GQA heads packed per kv head).

Decode reads every K/V element once and does ~2 FLOP per element per query head, so the bound is
HBM bandwidth: algorithmic bytes = |K| + |V| + |Q| + |O| (+ the fp32 split partials the merge pass
reads back, reported separately), peak 8 TB/s. torch's scaled_dot_product_attention (its default
ROCm backend, GQA via enable_gqa) on the same inputs is timed beside it.

Usage: python decode_bench.py [--json out.json]
"""
from __future__ import annotations

import argparse
import json
import statistics
import sys

import torch
import torch.nn.functional as F

import flash_atten

HBM_PEAK_GBS = 8000.0

# (label, B, H, H_kv, M, N, D, dtype)
CASES = [
    ("llama3-8b B1 N8k", 1, 32, 8, 1, 8192, 128, torch.bfloat16),
    ("llama3-8b B1 N32k", 1, 32, 8, 1, 32768, 128, torch.bfloat16),
    ("llama3-8b B1 N128k", 1, 32, 8, 1, 131072, 128, torch.bfloat16),
    ("llama3-8b B8 N32k", 8, 32, 8, 1, 32768, 128, torch.bfloat16),
    ("llama3-8b B32 N8k", 32, 32, 8, 1, 8192, 128, torch.bfloat16),
    ("llama3-8b B8 N32k M4 (spec)", 8, 32, 8, 4, 32768, 128, torch.bfloat16),
    ("qwen2.5-1.5b B1 N32k", 1, 12, 2, 1, 32768, 128, torch.bfloat16),
    ("qwen2.5-1.5b B16 N16k", 16, 12, 2, 1, 16384, 128, torch.bfloat16),
    ("fp16 D64 B4 N64k", 4, 16, 2, 1, 65536, 64, torch.float16),
]


def _time(fn, warmup: int = 3, iters: int = 20) -> float:
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
    return statistics.median(times)


def _time_graph(fn, iters: int = 20, batch: int = 20) -> tuple[float, torch.Tensor]:
    """Per-step time of replaying one call captured in a HIP graph (torch.cuda.CUDAGraph), as a
    decode loop runs it: `batch` back-to-back replays between two events, median over `iters`
    such samples. This is the GPU time of the split and merge launches without the host's per-call
    launch cost, which dominates a single eager decode step. Returns (ms, the graph's output)."""
    side = torch.cuda.Stream()  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(iters):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(batch):
            graph.replay()
        e.record()
        torch.cuda.synchronize()
        times.append(s.elapsed_time(e) / batch)
    return statistics.median(times), out


def run_case(label, B, H, Hkv, M, N, D, dtype, seed: int = 0) -> dict:
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(B, H, M, D, generator=g).to(dtype).to(dev)
    k = torch.randn(B, Hkv, N, D, generator=g).to(dtype).to(dev)
    v = torch.randn(B, Hkv, N, D, generator=g).to(dtype).to(dev)
    ours = lambda: flash_atten.sdpa(q, k, v, is_causal=False, scale=D ** -0.5, variant="sliced")  # noqa: E731
    out = ours()
    ref = F.scaled_dot_product_attention(q, k, v, scale=D ** -0.5, enable_gqa=True)
    torch.cuda.synchronize()
    err = (out.float() - ref.float()).abs().max().item()
    ms = _time(ours)
    ms_graph, out_graph = _time_graph(ours)
    graph_diff = (out_graph.float() - out.float()).abs().max().item()
    ms_torch = _time(lambda: F.scaled_dot_product_attention(q, k, v, scale=D ** -0.5, enable_gqa=True))
    elt = q.element_size()
    kv_bytes = 2 * B * Hkv * N * D * elt
    io_bytes = kv_bytes + 2 * B * H * M * D * elt
    flops = 4.0 * B * H * M * N * D
    row = {
        "case": label, "B": B, "H": H, "H_kv": Hkv, "M": M, "N": N, "D": D, "dtype": str(dtype).replace("torch.", ""),
        "ms": round(ms, 4), "ms_torch_sdpa": round(ms_torch, 4), "speedup_vs_torch": round(ms_torch / ms, 2),
        "algorithmic_bytes": io_bytes, "GBs": round(io_bytes / ms / 1e6, 1),
        "hbm_frac": round(io_bytes / ms / 1e6 / HBM_PEAK_GBS, 4), "TFLOPs": round(flops / ms / 1e9, 1),
        "ms_graph": round(ms_graph, 4), "GBs_graph": round(io_bytes / ms_graph / 1e6, 1),
        "hbm_frac_graph": round(io_bytes / ms_graph / 1e6 / HBM_PEAK_GBS, 4), "graph_vs_eager_max_abs": graph_diff,
        "max_abs_vs_torch": err,
    }
    print(f"[decode] {label}: {ms:.4f} ms = {row['GBs']:.0f} GB/s ({100 * row['hbm_frac']:.1f}% of 8 TB/s); "
          f"graph replay {ms_graph:.4f} ms = {row['GBs_graph']:.0f} GB/s ({100 * row['hbm_frac_graph']:.1f}%); "
          f"torch SDPA {ms_torch:.4f} ms ({row['speedup_vs_torch']:.2f}x), max|diff|={err:.2e}", flush=True)
    del q, k, v, out, ref, out_graph
    torch.cuda.empty_cache()
    return row


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--json", default=None)
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("decode_bench.py needs a GPU (gfx950)", file=sys.stderr)
        return 1
    rows = [run_case(*c) for c in CASES]
    if args.json:
        with open(args.json, "w") as fh:
            json.dump(rows, fh, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
