"""Timed launch-configuration sweep for gfx950; writes tune_table.json.

The reference's tuner compiles every candidate and keeps the feasible one with the largest resource
footprint, without timing (tuner.py:489-560; mma.py:63-81 is a fixed table). Here every built tile
that fits the device is timed on the device with HIP events, per shape bucket, and the winner is
persisted; FlashAttentionTuner* and _select_2d_contiguous_config read the table
(gfx950_configs.choose_fa_tile / choose_gemm_tile).

  * attention: tiles (block_m, block_n, waves, stages) x variant (basic / optimized / sliced) x dtype x D x
    causal, per (B*H, M, N) power-of-two bucket;
  * GEMM: tiles (block_m, block_n, block_k, waves) x GROUP_M in {4, 8, 16}, per (M, N, K) bucket.

Usage: python gfx950_tune.py [--quick] [--out tune_table.json]
"""
from __future__ import annotations

import argparse
import json
import statistics
import sys
import time

import torch

import gfx950_configs as cfgs
import hip_lib

VARIANTS = {"basic": hip_lib.FA_VARIANT_BASIC, "optimized": hip_lib.FA_VARIANT_OPT,
            "sliced": hip_lib.FA_VARIANT_SLICED}

# (name, dtype, B, H, H_kv, M, N, D, causal, variants) -- the benchmark configurations, plus
# decode shapes (a few query rows against a long KV cache) for the sliced variant
FA_SWEEP = (
    [("fp16_d128", torch.float16, 4, 32, 32, n, n, 128, c, ("basic", "optimized", "sliced"))
     for n in (1024, 2048, 4096, 8192, 16384) for c in (False, True)]
    + [("bf16_d256", torch.bfloat16, 2, 16, 16, n, n, 256, False, ("basic", "optimized", "sliced"))
       for n in (1024, 2048, 4096, 8192)]
    + [("fp16_d64_cfg1", torch.float16, 1, 4, 4, 512, 512, 64, False, ("basic", "optimized", "sliced"))]
    + [(f"ttft_{name}_gqa", dt, 1, 12, 2, n, n, 128, True, ("sliced", "optimized"))
       for name, dt in (("bf16", torch.bfloat16), ("fp16", torch.float16)) for n in (4096, 16384, 65536)]
    + [("decode_bf16_gqa", torch.bfloat16, b, 32, 8, 1, n, 128, False, ("sliced",))
       for b, n in ((1, 8192), (1, 32768), (1, 131072), (8, 32768), (32, 8192))]
)
GEMM_SWEEP = ([(n, n, n) for n in (1024, 2048, 4096, 8192, 16384)]
              + [(8192, 8192, 256), (1024, 1024, 256), (4096, 4096, 512)])
GROUP_MS = (4, 8, 16)


GRAPH_BELOW_MS = 0.25


def _time(fn, warmup: int, iters: int, batch_ms: float = 1.0) -> float:
    """Median per-launch time (ms) of back-to-back launches: each of `iters` samples times a batch
    of launches lasting about `batch_ms`, so short kernels are ranked by their steady rate rather
    than by one launch from an idle queue. A launch shorter than GRAPH_BELOW_MS is timed as a
    replay of the batch captured in a HIP graph: eager launches of a few microseconds are paced by
    the host's per-call cost (~6 us here), not by the kernel, which would tie every tile."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()

    def sample(run, n: int) -> float:
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        run()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / n

    def eager(n: int):
        def run():
            for _ in range(n):
                fn()
        return run

    one = sample(eager(1), 1)
    batch = max(1, min(64, round(batch_ms / max(one, 1e-3))))
    if one < GRAPH_BELOW_MS:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(batch):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        return statistics.median(sample(graph.replay, batch) for _ in range(iters))
    return statistics.median(sample(eager(batch), batch) for _ in range(iters))


REFINE_TOP = 3
REFINE_ROUNDS = 5
REFINE_BATCH_MS = 8.0


def _refine(fns: dict, results: dict, top: int = REFINE_TOP, rounds: int = REFINE_ROUNDS, iters: int = 3) -> dict:
    """Re-time the `top` fastest candidates of a first pass in `rounds` interleaved rounds and
    return their medians: tiles within a few percent of each other are then ranked under the same
    clock and thermal conditions rather than by one pass each, minutes apart. Each sample is a
    batch of ~REFINE_BATCH_MS of back-to-back launches (a 2 ms kernel timed one launch per sample
    ranked two tiles 2% apart the wrong way round)."""
    best = sorted(results, key=results.get)[:top]
    if len(best) < 2:
        return {}
    samples: dict = {k: [] for k in best}
    for _ in range(rounds):
        for k in best:
            samples[k].append(_time(fns[k], 1, iters, batch_ms=REFINE_BATCH_MS))
    return {k: round(statistics.median(v), 4) for k, v in samples.items()}


def tune_attention(table: dict, sweep=FA_SWEEP, warmup: int = 2, iters: int = 5, log=print) -> None:
    dev = torch.device("cuda:0")
    for name, dtype, B, H, Hkv, M, N, D, causal, variants in sweep:
        q = torch.randn(B, H, M, D, device=dev, dtype=dtype)
        k = torch.randn(B, Hkv, N, D, device=dev, dtype=dtype)
        v = torch.randn(B, Hkv, N, D, device=dev, dtype=dtype)
        o = torch.empty_like(q)
        flops = 4.0 * B * H * D * (N * (N + 1) / 2 if causal and M == N else M * N)
        for vname in variants:
            variant = VARIANTS[vname]
            results, fns = {}, {}
            for cand in cfgs.fa_candidates(variant, dtype, D):
                splits = 1
                ws = None
                if variant == hip_lib.FA_VARIANT_SLICED:
                    splits = cfgs.choose_splits(
                        B, H, M, N, cand.block_m, cand.block_n, H_kv=Hkv, causal=causal,
                        resident_per_cu=cfgs.split_residency(dtype, D, cand.block_m, cand.block_n, cand.waves,
                                                             cand.stages))
                    need = hip_lib.workspace_bytes(B, H, M, D, splits)
                    ws = torch.empty(need, dtype=torch.uint8, device=dev) if need else None
                tile = cfgs.FaTileChoice(cand.block_m, cand.block_n, cand.waves, cand.stages, splits).to_c()
                key = f"{cand.block_m}x{cand.block_n}x{cand.waves}x{cand.stages}"
                fns[key] = (lambda tile=tile, ws=ws, variant=variant: hip_lib.fa_fwd(
                    q, k, v, o, None, sm_scale=D ** -0.5, causal=causal, variant=variant, tile=tile, workspace=ws))
                results[key] = round(_time(fns[key], warmup, iters), 4)
            refined = _refine(fns, results)
            pool = refined or results
            best = min(pool, key=pool.get)
            key = cfgs.fa_table_key(variant, dtype, D, causal, B, H, M, N)
            table["fa"][key] = {
                "tile": [int(x) for x in best.split("x")],
                "ms": pool[best],
                "tflops": round(flops / pool[best] / 1e9, 1),
                "timed": results,
                **({"refined": refined} if refined else {}),
            }
            log(f"[tune] attention {name} B={B} M={M} N={N} causal={causal} {vname}: best {best} "
                f"{pool[best]:.3f} ms ({flops / pool[best] / 1e9:.0f} TFLOP/s) of {len(results)}")
        del q, k, v, o
        torch.cuda.empty_cache()


def tune_gemm(table: dict, sweep=GEMM_SWEEP, warmup: int = 2, iters: int = 5, log=print) -> None:
    dev = torch.device("cuda:0")
    for M, N, K in sweep:
        a = (torch.rand(M, K, device=dev) * 2 - 1).half()
        b = (torch.rand(K, N, device=dev) * 2 - 1).half()
        c = torch.empty(M, N, device=dev, dtype=torch.float16)
        results, fns = {}, {}
        for t in cfgs.gemm_candidates():
            if M % t[0] or N % t[1] or K % t[2]:
                continue
            for gm in GROUP_MS:
                gt = hip_lib.GemmTile(t[0], t[1], t[2], t[3], gm)
                key = f"{t[0]}x{t[1]}x{t[2]}x{t[3]}g{gm}"
                fns[key] = lambda gt=gt: hip_lib.gemm_f16(a, b, c, gt)
                results[key] = round(_time(fns[key], warmup, iters), 4)
        if not results:
            continue
        refined = _refine(fns, results)
        pool = refined or results
        best = min(pool, key=pool.get)
        tile_part, gm_part = best.split("g")
        table["gemm"][cfgs.gemm_table_key(M, N, K)] = {
            "tile": [int(x) for x in tile_part.split("x")],
            "group_m": int(gm_part),
            "ms": pool[best],
            "tflops": round(2.0 * M * N * K / pool[best] / 1e9, 1),
            "timed": results,
            **({"refined": refined} if refined else {}),
        }
        log(f"[tune] gemm {M}x{N}x{K}: best {best} {pool[best]:.3f} ms "
            f"({2.0 * M * N * K / pool[best] / 1e9:.0f} TFLOP/s) of {len(results)}")
        del a, b, c
        torch.cuda.empty_cache()


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out", default=str(cfgs.TUNE_TABLE_PATH))
    ap.add_argument("--quick", action="store_true", help="fewer timed launches per candidate")
    ap.add_argument("--only", choices=["fa", "gemm"], default=None)
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("gfx950_tune.py needs a GPU", file=sys.stderr)
        return 1
    table = {"fa": {}, "gemm": {}}
    if args.only is not None:
        # a partial sweep keeps the other half of the table at --out, or else of the installed one
        for path in (args.out, str(cfgs.TUNE_TABLE_PATH)):
            try:
                with open(path) as fh:
                    old = json.load(fh)
            except (OSError, ValueError):
                continue
            table = {"fa": old.get("fa", {}), "gemm": old.get("gemm", {})}
            break
        table[args.only] = {}
    t0 = time.time()
    iters = 3 if args.quick else 5
    if args.only in (None, "fa"):
        tune_attention(table, iters=iters, log=lambda m: print(m, flush=True))
    if args.only in (None, "gemm"):
        tune_gemm(table, iters=iters, log=lambda m: print(m, flush=True))
    table["meta"] = {"device": torch.cuda.get_device_name(0), "seconds": round(time.time() - t0, 1),
                     "torch": torch.__version__, "iters": iters}
    with open(args.out, "w") as fh:
        json.dump(table, fh, indent=1, sort_keys=True)
        fh.write("\n")
    print(f"[tune] wrote {args.out}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
