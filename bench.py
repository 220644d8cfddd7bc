"""Headline benchmark: FlashAttention forward (fp16, B=4, H=32, N=8192, D=128, non-causal) and the
fp16 GEMM at 8192^3 on one MI355X, through the drop-in API (tuner -> flash_attention, and
_matmul_contiguous_kernel), i.e. the hand-written HIP kernels in libfa_gfx950.so.

Prints ONE JSON line. `value` is the attention forward throughput in TFLOP/s (4*B*H*N^2*D per
launch, test_flash_atten.py:234-240) with inputs resident in HBM; the GEMM figure (2*M*N*K,
test_mma.py:78-83) is reported in the `gemm` object. Each launch is timed with HIP events recorded
on the stream the kernels are launched on (torch's current stream), and the mean launch duration
feeds `roofline.achieved`. The CPU baseline is the reference's own CPU path (torch SDPA math
backend on fp32 CPU copies, test_flash_atten.py:459-461, 498-499; CPU torch.matmul, test_mma.py:
260-261), measured on the box's host cores: attention on one (b, h) slice of the headline and on
config 1, the GEMM in fp32 at 8192^3 and in fp16 at the reference's published 8192x8192x256.
Beside each kernel, AMD's own implementation on the same GPU (torch.matmul -> hipBLASLt; torch's
scaled_dot_product_attention) is timed in alternating rounds with ours (`vendor`).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-vendor] [--variant optimized]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import threading
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "flash-attn-economical-gpu_amd"
for _p in (str(PKG), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_FP16_TFLOPS = 2516.6  # MI355X dense fp16/bf16 MFMA: 256 CU x 4096 FLOP/clk x 2.4 GHz
PEAK_HBM_GBS = 8000.0
# HBM bytes per launch of each attention workload and of the 8192^3 GEMM, from rocprofv3 --pmc
# FETCH_SIZE / WRITE_SIZE passes over this script's own warmed launches (`--counters-summarize
# ... --traffic-out`).
TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_fa_fwd_configs_gemm8192.json"
SEED = 20260328  # the reference's constant (test_flash_atten.py:33)
FA_SHAPE = dict(B=4, H=32, N=8192, D=128)
# Attention workloads of the BASELINE configurations: the headline (default line) and, for
# separate measurement, config 3's causal case at N=8192 and config 4's largest case.
FA_CONFIGS = {
    "headline": dict(B=4, H=32, N=8192, D=128, dtype="fp16", causal=False, variant="optimized", input_scale=1.0),
    "fp16_d128_causal": dict(B=4, H=32, N=8192, D=128, dtype="fp16", causal=True, variant="optimized",
                             input_scale=1.0),
    "bf16_d256": dict(B=2, H=16, N=8192, D=256, dtype="bf16", causal=False, variant="sliced", input_scale=0.5),
}
GEMM_SHAPE = dict(M=8192, N=8192, K=8192)
GEMM_K256_SHAPE = dict(M=8192, N=8192, K=256)


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _clock_warmup(torch, fn, ms: float) -> int:
    """Run `fn` back to back until at least `ms` of GPU time has passed (batches timed with HIP
    events); returns the launch count. After the GPU has idled (host-side input setup), MI355X
    takes ~30 ms of load to reach its steady clock: the 8192^3 GEMM measured 1030 TFLOP/s over its
    first 5 launches, 1282 over launches 10-40 and 1345 from launch 40 on. The reference warms the
    clock before timing too (torch.cuda._sleep, test_flash_atten.py:502-506)."""
    done, n, spent = 0, 1, 0.0
    while spent < ms:
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(n):
            fn()
        e.record()
        torch.cuda.synchronize()
        spent += s.elapsed_time(e)
        done += n
        n = min(2 * n, 64)
    return done


class ClockSampler:
    """The graphics clock of this process's GPU under a given load: amdsmi's GPU metrics (the
    XCDs' current gfx clocks, averaged), matched to torch's device by PCI bus. The firmware
    refreshes those metrics about once a second (a 1 s GEMM burst saw one change, from idle to
    1.67-1.77 GHz), so measure() runs the launch back to back for a few seconds and averages the
    readings of the burst's second half. Reading only; None where amdsmi, the device match or the
    metric is unavailable (the bench then reports no clock)."""

    def __init__(self, torch, dev):
        self.amdsmi = self.handle = None
        try:
            import amdsmi

            amdsmi.amdsmi_init()
            props = torch.cuda.get_device_properties(dev)
            bus, domain = getattr(props, "pci_bus_id", None), getattr(props, "pci_domain_id", 0)
            if bus is None:
                return
            for h in amdsmi.amdsmi_get_processor_handles():
                bdf = amdsmi.amdsmi_get_gpu_device_bdf(h)  # "dddd:bb:dd.f"
                dom, b = (int(x, 16) for x in bdf.split(":")[:2])
                if b == bus and dom == domain:
                    self.amdsmi, self.handle = amdsmi, h
                    break
            if self.handle is not None and self._read() is None:
                self.handle = None
        except Exception:  # no amdsmi, no permission, no such metric: no clock in the line
            self.handle = None

    def _read(self) -> float | None:
        m = self.amdsmi.amdsmi_get_gpu_metrics_info(self.handle)
        vals = [x for x in (m.get("current_gfxclks") or []) if isinstance(x, (int, float)) and 0 < x < 10000]
        if not vals and isinstance(m.get("current_gfxclk"), (int, float)) and 0 < m["current_gfxclk"] < 10000:
            vals = [m["current_gfxclk"]]
        return sum(vals) / len(vals) if vals else None

    def measure(self, torch, fn, seconds: float = 2.5) -> float | None:
        """Mean clock (GHz) while `fn` runs back to back for `seconds` (batches of ~20 ms)."""
        if self.handle is None:
            return None
        samples: list[tuple[float, float]] = []
        stop = threading.Event()
        t0 = time.perf_counter()

        def loop():
            while not stop.is_set():
                try:
                    v = self._read()
                except Exception:
                    v = None
                if v:
                    samples.append((time.perf_counter() - t0, v))
                stop.wait(0.01)

        thread = threading.Thread(target=loop, daemon=True)
        thread.start()
        n = 1
        try:
            while time.perf_counter() - t0 < seconds:
                b0 = time.perf_counter()
                for _ in range(n):
                    fn()
                torch.cuda.synchronize()
                if time.perf_counter() - b0 < 0.02:
                    n = min(2 * n, 256)
        finally:
            stop.set()
            thread.join()
        late = [v for t, v in samples if t >= seconds / 2]
        return round(statistics.mean(late) / 1000.0, 3) if late else None


def _time_launches(torch, fn, steps: int, warmup: int, clock_warmup_ms: float = 0.0):
    """Warm the clock (`clock_warmup_ms` of back-to-back launches), do `warmup` untimed launches,
    then time exactly `steps` launches; per-launch HIP events on the current stream."""
    if clock_warmup_ms > 0:
        _clock_warmup(torch, fn, clock_warmup_ms)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    outer_s, outer_e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    outer_s.record()
    for s, e in events:
        s.record()
        fn()
        e.record()
    outer_e.record()
    torch.cuda.synchronize()
    per = [s.elapsed_time(e) for s, e in events]
    return outer_s.elapsed_time(outer_e), per


def _cpu_threads(torch) -> dict:
    return {"cores": torch.get_num_threads(), "affinity_cores": len(os.sched_getaffinity(0)),
            "torch_threads": torch.get_num_threads()}


def _time_cpu(fn, warmup: int, runs: int, label: str) -> list[float]:
    for _ in range(warmup):
        fn()
    times = []
    for i in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        _log(f"cpu {label} run {i + 1}/{runs}: {times[-1] * 1e3:.1f} ms")
    return times


def _cpu_baseline_attention(torch, B, H, N, D):
    """The reference's CPU path for attention (its oracle, test_flash_atten.py:459-461, 498-499):
    torch SDPA, math backend, on fp32 copies of fp16 N(0,1) inputs.
      * headline: one (b, h) slice [1,1,N,D] of the workload, measured; the whole workload is that
        time x B*H (stated as extrapolated, never as measured);
      * config 1 [1,4,512,64], 3 warm-ups + 10 timed runs, mean and p50 (test_flash_atten.py:549-571)."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    g = torch.Generator().manual_seed(SEED)

    def inputs(shape):
        return tuple(torch.randn(shape, generator=g, dtype=torch.float16).float() for _ in range(3))

    with sdpa_kernel(SDPBackend.MATH):
        q, k, v = inputs((1, 1, N, D))
        t_slice = _time_cpu(lambda: F.scaled_dot_product_attention(q, k, v), 1, 3, f"sdpa [1,1,{N},{D}]")
        q1, k1, v1 = inputs((1, 4, 512, 64))
        t_cfg1 = _time_cpu(lambda: F.scaled_dot_product_attention(q1, k1, v1), 3, 10, "sdpa config1 [1,4,512,64]")
    slice_s = statistics.mean(t_slice)
    slice_flops = 4.0 * N * N * D
    cfg1_flops = 4.0 * 1 * 4 * 512 * 512 * 64
    cfg1_mean, cfg1_p50 = statistics.mean(t_cfg1), statistics.median(t_cfg1)
    return {
        "value": slice_flops / slice_s / 1e12,
        "unit": "TFLOP/s",
        **_cpu_threads(torch),
        "kind": "reference",
        "sample": (f"torch CPU SDPA math backend on fp32 copies of fp16 inputs (the reference's oracle path), one "
                   f"(b,h) slice [1,1,{N},{D}] of the headline: 1 warm-up + 3 runs, mean {slice_s * 1e3:.1f} ms "
                   f"(measured); the whole B={B} H={H} workload would take {slice_s * B * H:.1f} s "
                   f"(extrapolated x{B * H})"),
        "config1": {"shape": [1, 4, 512, 64], "warmup": 3, "runs": 10, "mean_ms": round(cfg1_mean * 1e3, 3),
                    "p50_ms": round(cfg1_p50 * 1e3, 3), "tflops_mean": cfg1_flops / cfg1_mean / 1e12,
                    "note": "measured; BASELINE configs[0], test_flash_atten.py:549-571 protocol"},
    }


def _cpu_baseline_gemm(torch, M, N, K, fp16_runs: int = 1):
    """The reference's CPU GEMM path (CPU torch.matmul, test_mma.py:260-261): fp32 at M x K x N (the
    headline shape; 1 warm-up + 2 runs, measured) and fp16 on a 2048-row block of the reference's
    published 8192x8192x256 (test_mma.py:42-45; `fp16_runs` runs, no warm-up). CPU fp16 GEMM runs at
    ~1 GFLOP/s, so the whole published shape would take ~50 s; output rows are independent, so the
    whole shape's time is the block's x 4, stated as such."""
    g = torch.Generator().manual_seed(SEED)
    a32 = torch.rand(M, K, generator=g) * 2 - 1
    b32 = torch.rand(K, N, generator=g) * 2 - 1
    t32 = _time_cpu(lambda: torch.matmul(a32, b32), 1, 2, f"matmul fp32 {M}x{K}x{N}")
    del a32, b32
    pm, pk, pn = 2048, 256, 8192
    a16 = (torch.rand(pm, pk, generator=g) * 2 - 1).half()
    b16 = (torch.rand(pk, pn, generator=g) * 2 - 1).half()
    t16 = _time_cpu(lambda: torch.matmul(a16, b16), 0, fp16_runs, f"matmul fp16 {pm}x{pk}x{pn}")
    s32, s16 = statistics.mean(t32), statistics.mean(t16)
    return {
        "value": 2.0 * M * N * K / s32 / 1e12,
        "unit": "TFLOP/s",
        **_cpu_threads(torch),
        "kind": "reference",
        "sample": (f"CPU torch.matmul fp32 {M}x{K} @ {K}x{N} (the headline shape in fp32; fp16 CPU GEMM at that "
                   f"shape would run for ~15 min): 1 warm-up + 2 runs, mean {s32:.3f} s, measured"),
        "fp16_8192x8192x256": {"block_rows_measured": pm, "block_mean_s": round(s16, 3), "runs": fp16_runs,
                               "tflops": 2.0 * pm * pn * pk / s16 / 1e12,
                               "whole_shape_s_extrapolated": round(s16 * 8192 / pm, 1),
                               "note": "the reference's CPU path at its published shape (test_mma.py:42-45, "
                                       "260-261): a 2048x256 @ 256x8192 row block measured, the whole "
                                       "8192-row shape = 4 such blocks"},
    }


def _alternating(torch, fns: dict, rounds: int, per_round: int) -> dict:
    """Median launch time (ms) of each callable, timed in alternating rounds on the current stream so
    clock and thermal drift hit every entry alike."""
    times = {name: [] for name in fns}
    for _ in range(rounds):
        for name, fn in fns.items():
            fn()
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(per_round):
                fn()
            e.record()
            torch.cuda.synchronize()
            times[name].append(s.elapsed_time(e) / per_round)
    return {name: statistics.median(v) for name, v in times.items()}


# Counter passes for `--counters-summarize` (each within one pass's hardware limits: at most 8 SQ,
# 4 TCC and 2 GRBM counters). Each pass profiles one `bench.py --counter-run` process.
COUNTER_PASSES = {
    "p1": "GRBM_GUI_ACTIVE SQ_BUSY_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA SQ_INSTS_VALU SQ_INSTS_LDS "
          "SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_WAVE_CYCLES",
    "p2": "GRBM_GUI_ACTIVE SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS SQ_WAIT_INST_LDS SQ_WAIT_INST_ANY SQ_INSTS_SALU "
          "SQ_ACTIVE_INST_MISC SQ_INSTS_SMEM SQ_WAVES",
    "p3": "GRBM_GUI_ACTIVE SQ_WAIT_ANY SQ_ACTIVE_INST_ANY SQ_VALU_MFMA_COEXEC_CYCLES SQ_INSTS_VALU_TRANS_F32 "
          "SQ_LDS_DATA_FIFO_FULL SQ_LDS_CMD_FIFO_FULL SQ_BUSY_CU_CYCLES SQ_INSTS_BRANCH",
    "fetch": "FETCH_SIZE",
    "write": "WRITE_SIZE",
}
# Calibration launches of `--counter-run`: out = in + 1 over fp32 tensors of these sizes, the first
# add kernels of the process (each reads and writes exactly its size once).
CALIBRATION_MIB = (64, 256, 1024)


def counters_command(fa_config: str, out_dir: str, fa_tile: str | None = None) -> str:
    tile = f" --fa-tile {fa_tile}" if fa_tile else ""
    runs = [f"rocprofv3 --pmc {c} --output-format csv -d {out_dir} -o {name} -- python -u bench.py --counter-run "
            f"--fa-config {fa_config}{tile}" for name, c in COUNTER_PASSES.items()]
    return " && ".join(["export TMPDIR=/tmp", *runs,
                        f"python bench.py --counters-summarize {out_dir} --fa-config {fa_config}{tile}"])


def _calibration_launches(torch, dev) -> None:
    for mib in CALIBRATION_MIB:
        src = torch.ones(mib * 1024 * 1024 // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.add(src, 1.0, out=dst)
        torch.cuda.synchronize()
        del src, dst
    torch.cuda.empty_cache()


def _counters_summarize(directory: str, fa_config: str, steps: int, fa_tile: str | None = None,
                        traffic_out: str | None = None) -> int:
    """Markdown summary of the counter passes over `bench.py --counter-run --fa-config <cfg>`: per
    kernel, the mean over its last `steps` dispatches (the bench's timed launches, after its
    warm-up), clock and MFMA utilisation, instruction mix, LDS conflicts and calibrated HBM bytes."""
    import csv
    import glob

    passes: dict[str, list[dict]] = {}
    for path in sorted(glob.glob(os.path.join(directory, "*_counter_collection.csv"))):
        name = os.path.basename(path)[: -len("_counter_collection.csv")]
        disp: dict[int, dict] = {}
        with open(path) as fh:
            for r in csv.DictReader(fh):
                d = disp.setdefault(int(r["Dispatch_Id"]), {"kernel": r["Kernel_Name"], "c": {},
                                                           "ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"])})
                d["c"][r["Counter_Name"]] = d["c"].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        passes[name] = [disp[k] for k in sorted(disp)]
    missing = set(COUNTER_PASSES) - set(passes)
    if missing:
        raise SystemExit(f"counter passes missing in {directory}: {sorted(missing)}")

    def calib(rows, counter):
        # torch.add's kernel (the fills that create the tensors are separate dispatches)
        cal = [r for r in rows if "_add<" in r["kernel"]][: len(CALIBRATION_MIB)]
        if len(cal) != len(CALIBRATION_MIB):
            raise SystemExit("calibration dispatches not found")
        return [mib * 1024 * 1024 / (r["c"][counter] * 1024) for mib, r in zip(CALIBRATION_MIB, cal)]

    f_factors, w_factors = calib(passes["fetch"], "FETCH_SIZE"), calib(passes["write"], "WRITE_SIZE")
    f_factor, w_factor = statistics.mean(f_factors), statistics.mean(w_factors)

    cfg = FA_CONFIGS[fa_config]
    B, H, N, D = cfg["B"], cfg["H"], cfg["N"], cfg["D"]
    fa_flops = 4.0 * B * H * D * (N * (N + 1) / 2 if cfg["causal"] else N * N)
    M_, Ng, K = GEMM_SHAPE["M"], GEMM_SHAPE["N"], GEMM_SHAPE["K"]
    kernels = {
        "attention": ("fa_fwd", fa_flops, 4 * B * H * N * D * 2),  # fa_fwd_kernel or fa_fwd16_kernel
        "gemm": ("gemm_f16", 2.0 * M_ * Ng * K, 2 * (M_ * K + K * Ng + M_ * Ng)),
        # hipBLASLt's kernel for the same GEMM (torch.matmul in the alternating vendor rounds; the
        # fp32 product of the parity check is a Cijk_..._S_B_ kernel and is skipped)
        "gemm hipBLASLt": ("Cijk_", 2.0 * M_ * Ng * K, 2 * (M_ * K + K * Ng + M_ * Ng)),
    }

    def is_kernel(name: str, needle: str) -> bool:
        if needle == "fa_fwd":
            return "fa_fwd_kernel" in name or "fa_fwd16_kernel" in name
        return needle in name and not (needle == "Cijk_" and "_S_B_" in name)

    def mfma_flop(name: str) -> int:
        """FLOP per MFMA instruction of a kernel: 16x16x32 (our fa_fwd16 kernels, GEMM tiles built
        with MI = 16, hipBLASLt's MI16x16 kernels) or 32x32x16."""
        if "fa_fwd16_kernel" in name or "MI16x16" in name:
            return 16384
        if "gemm_f16" in name and "<" in name:
            args = [a.strip() for a in name.split("<", 1)[1].split(">", 1)[0].split(",")]
            if len(args) >= 6 and args[5] == "16":
                return 16384
        return 32768

    out = {}
    for key, (needle, flops, algo_bytes) in kernels.items():
        per_pass = {}
        for name, rows in passes.items():
            hits = [r for r in rows if is_kernel(r["kernel"], needle)][-steps:]
            if not hits:
                break
            per_pass[name] = None
        if len(per_pass) != len(passes):
            if key.endswith("hipBLASLt"):
                continue  # vendor rounds not in these passes
            raise SystemExit(f"no {needle} dispatch in some pass")
        for name, rows in passes.items():
            hits = [r for r in rows if is_kernel(r["kernel"], needle)][-steps:]
            per_pass[name] = {"kernel": hits[0]["kernel"], "n": len(hits),
                              "ns": statistics.mean(r["ns"] for r in hits),
                              "c": {c: statistics.mean(r["c"][c] for r in hits) for c in hits[0]["c"]}}
        p1, p2, p3 = per_pass["p1"], per_pass["p2"], per_pass["p3"]
        c1, c2, c3 = p1["c"], p2["c"], p3["c"]
        secs = p1["ns"] * 1e-9
        cycles = c1["GRBM_GUI_ACTIVE"] / 8  # summed over the 8 XCDs
        rd = per_pass["fetch"]["c"]["FETCH_SIZE"] * 1024 * f_factor
        wr = per_pass["write"]["c"]["WRITE_SIZE"] * 1024 * w_factor
        out[key] = {
            "kernel": p1["kernel"], "dispatches_averaged": p1["n"],
            "duration_ms_p1": p1["ns"] * 1e-6, "duration_ms_p2": p2["ns"] * 1e-6,
            "tflops_at_p1_duration": flops / secs / 1e12,
            "clock_ghz": cycles / secs / 1e9,
            "mfma_busy": c1["SQ_VALU_MFMA_BUSY_CYCLES"] / (1024 * cycles),
            "mfma_insts": c1["SQ_INSTS_MFMA"],
            "mfma_flop_per_inst": mfma_flop(p1["kernel"]),
            "valu_per_mfma": c1["SQ_INSTS_VALU"] / c1["SQ_INSTS_MFMA"],
            "lds_per_mfma": c1["SQ_INSTS_LDS"] / c1["SQ_INSTS_MFMA"],
            "lds_bank_conflict_rate": c1["SQ_LDS_BANK_CONFLICT"] / max(c1["SQ_LDS_IDX_ACTIVE"], 1.0),
            "valu_active_per_wave_cycle": c2["SQ_ACTIVE_INST_VALU"] / c1["SQ_WAVE_CYCLES"],
            "lds_wait_per_wave_cycle": c2["SQ_WAIT_INST_LDS"] / c1["SQ_WAVE_CYCLES"],
            "any_wait_per_wave_cycle": c2["SQ_WAIT_INST_ANY"] / c1["SQ_WAVE_CYCLES"],
            "salu_per_mfma": c2["SQ_INSTS_SALU"] / c1["SQ_INSTS_MFMA"],
            "wait_any_per_wave_cycle": c3["SQ_WAIT_ANY"] / c1["SQ_WAVE_CYCLES"],
            "issue_any_per_wave_cycle": c3["SQ_ACTIVE_INST_ANY"] / c1["SQ_WAVE_CYCLES"],
            "valu_mfma_coexec_of_mfma_busy": c3["SQ_VALU_MFMA_COEXEC_CYCLES"] / max(c1["SQ_VALU_MFMA_BUSY_CYCLES"], 1.0),
            "trans_per_mfma": c3["SQ_INSTS_VALU_TRANS_F32"] / c1["SQ_INSTS_MFMA"],
            "lds_fifo_full_per_cu_cycle": (c3["SQ_LDS_DATA_FIFO_FULL"] + c3["SQ_LDS_CMD_FIFO_FULL"]) / (256 * cycles),
            "branches_per_mfma": c3["SQ_INSTS_BRANCH"] / c1["SQ_INSTS_MFMA"],
            "hbm_read_bytes": rd, "hbm_write_bytes": wr, "hbm_bytes": rd + wr,
            "algorithmic_bytes": algo_bytes, "hbm_ratio_to_algorithmic": (rd + wr) / algo_bytes,
        }
    lines = [f"# Counters on warmed launches: attention `{fa_config}` and the 8192³ GEMM", "",
             "Command (repository root, one MI355X):", "", "```", counters_command(fa_config, directory, fa_tile), "```", "",
             f"Each pass is one `bench.py --counter-run` process: {len(CALIBRATION_MIB)} calibration launches "
             f"(out = in + 1 over fp32 tensors of {', '.join(f'{m} MiB' for m in CALIBRATION_MIB)}), then the bench's "
             f"own warm-up and timed launches of the attention forward and the GEMM. Figures are means over "
             f"each kernel's last {steps} dispatches (the timed ones); durations are the counter passes' own "
             f"(kernels run one at a time under counter collection).", "",
             f"HBM calibration: FETCH_SIZE x 1024 x {f_factor:.3f} and WRITE_SIZE x 1024 x {w_factor:.3f} bytes "
             f"(per-size factors: read {', '.join(f'{x:.3f}' for x in f_factors)}; "
             f"write {', '.join(f'{x:.3f}' for x in w_factors)}).", "",
             "| | " + " | ".join(out) + " |", "|---|" + "---|" * len(out)]
    fields = [("kernel", "kernel", "{}"), ("duration (ms, pass 1 / 2)", None, None),
              ("TFLOP/s at that duration", "tflops_at_p1_duration", "{:.0f}"), ("clock (GHz)", "clock_ghz", "{:.2f}"),
              ("MFMA busy (of SIMD-cycles)", "mfma_busy", "{:.3f}"), ("MFMA instructions", "mfma_insts", "{:.4g}"),
              ("FLOP per MFMA instruction (16x16x32: 16384, 32x32x16: 32768)", "mfma_flop_per_inst", "{}"),
              ("VALU instructions per MFMA (MFMA included)", "valu_per_mfma", "{:.2f}"),
              ("LDS instructions per MFMA", "lds_per_mfma", "{:.2f}"), ("SALU per MFMA", "salu_per_mfma", "{:.2f}"),
              ("LDS bank-conflict cycles / LDS active", "lds_bank_conflict_rate", "{:.4f}"),
              ("VALU active per wave-cycle", "valu_active_per_wave_cycle", "{:.3f}"),
              ("waiting on LDS per wave-cycle", "lds_wait_per_wave_cycle", "{:.3f}"),
              ("waiting (any) per wave-cycle", "any_wait_per_wave_cycle", "{:.3f}"),
              ("SQ_WAIT_ANY per wave-cycle (waitcnt and barrier waits)", "wait_any_per_wave_cycle", "{:.3f}"),
              ("instruction issued per wave-cycle", "issue_any_per_wave_cycle", "{:.3f}"),
              ("MFMA cycles with a VALU op co-executing", "valu_mfma_coexec_of_mfma_busy", "{:.3f}"),
              ("transcendental (exp, log, rcp) per MFMA", "trans_per_mfma", "{:.2f}"),
              ("LDS FIFO-full cycles per CU-cycle", "lds_fifo_full_per_cu_cycle", "{:.4f}"),
              ("branches per MFMA", "branches_per_mfma", "{:.3f}"),
              ("HBM read / write (GB)", None, None),
              ("HBM bytes / algorithmic bytes", "hbm_ratio_to_algorithmic", "{:.3f}")]
    for label, key, fmt in fields:
        cells = []
        for v in out.values():
            if label.startswith("duration"):
                cells.append(f"{v['duration_ms_p1']:.4f} / {v['duration_ms_p2']:.4f}")
            elif label.startswith("HBM read"):
                cells.append(f"{v['hbm_read_bytes'] / 1e9:.4f} / {v['hbm_write_bytes'] / 1e9:.4f}")
            elif key == "kernel":
                name = v["kernel"]
                cells.append(f"`{name if len(name) < 90 else name[:87] + '...'}`")
            else:
                cells.append(fmt.format(v[key]))
        lines.append(f"| {label} | " + " | ".join(cells) + " |")
    lines += ["", "```json", json.dumps(out, indent=1, default=float), "```", ""]
    print("\n".join(lines))
    if traffic_out:
        path = Path(traffic_out)
        doc = json.loads(path.read_text()) if path.exists() else {}
        doc["note"] = ("HBM bytes per launch: FETCH_SIZE x 1024 x fetch_factor + WRITE_SIZE x 1024 x write_factor, means "
                       "over the bench's timed launches under rocprofv3 --pmc; the factors make out = in + 1 over fp32 "
                       f"tensors of {', '.join(f'{m} MiB' for m in CALIBRATION_MIB)} read and write exactly their size.")
        doc[f"calibration_{fa_config}"] = {"fetch_factor": round(f_factor, 4), "write_factor": round(w_factor, 4),
                                           "fetch_factors_per_size": [round(x, 4) for x in f_factors],
                                           "write_factors_per_size": [round(x, 4) for x in w_factors]}
        for key, name in (("attention", f"fa_fwd_{fa_config}"), ("gemm", "gemm_f16_8192cube")):
            v = out[key]
            rd_b, wr_b = int(v["hbm_read_bytes"]), int(v["hbm_write_bytes"])
            doc[name] = {"kernel": v["kernel"], "command": counters_command(fa_config, directory, fa_tile),
                         "bytes_read": rd_b, "bytes_written": wr_b, "bytes_per_launch": rd_b + wr_b,
                         "algorithmic_bytes_per_launch": v["algorithmic_bytes"],
                         "ratio_to_algorithmic": round(v["hbm_ratio_to_algorithmic"], 4)}
        path.write_text(json.dumps(doc, indent=2, sort_keys=True) + "\n")
    return 0


def _bench_gemm_k256(torch, args, g, dev, vendor_rounds) -> dict:
    """The reference's own GEMM test and chart shape (test_mma.py:42-45), 8192x8192x256, through the same
    drop-in launcher: 128 MiB of C against 8 MiB of A and B, so its roofline is HBM (142.6 MB per launch,
    17.8 us at 8 TB/s). Beside it: torch's fill of the same C (a pure 128 MiB write stream) and
    hipBLASLt in alternating rounds."""
    import mma

    Mk, Nk, Kk = GEMM_K256_SHAPE["M"], GEMM_K256_SHAPE["N"], GEMM_K256_SHAPE["K"]
    a = (torch.rand(Mk, Kk, generator=g) * 2 - 1).half().to(dev)
    b = (torch.rand(Kk, Nk, generator=g) * 2 - 1).half().to(dev)
    c = torch.empty(Mk, Nk, dtype=torch.float16, device=dev)
    bm2, bn2, bk2, group_m2, warps2, stages2 = mma._select_2d_contiguous_config(Mk, Nk, Kk)
    grid2 = (math.ceil(Mk / bm2) * math.ceil(Nk / bn2),)

    def gemm_k256():
        mma._matmul_contiguous_kernel[grid2](a, b, c, Mk, Nk, Kk, BLOCK_M=bm2, BLOCK_N=bn2, BLOCK_K=bk2,
                                             GROUP_M=group_m2, USE_CACHE_EVICTION_HINTS=True, num_warps=warps2,
                                             num_stages=stages2)

    # back-to-back launches between one pair of events: at ~55 us per launch, events recorded between
    # launches would add several microseconds each
    k_steps = max(args.steps, 100)
    if args.clock_warmup_ms > 0:
        _clock_warmup(torch, gemm_k256, args.clock_warmup_ms)
    for _ in range(args.warmup):
        gemm_k256()
    torch.cuda.synchronize()
    ks, ke = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ks.record()
    for _ in range(k_steps):
        gemm_k256()
    ke.record()
    torch.cuda.synchronize()
    k_total = ks.elapsed_time(ke)
    k_ms = k_total / k_steps
    k_bytes = 2 * (Mk * Kk + Kk * Nk + Mk * Nk)
    ref = a.float() @ b.float()
    k_rel = ((c.float() - ref).norm() / ref.norm()).item()
    del ref
    fill_med = _alternating(torch, {"fill": lambda: c.fill_(1.0)}, rounds=3, per_round=20)["fill"]
    k_vendor = None
    if not args.no_vendor:
        med = _alternating(torch, {"ours": gemm_k256, "hipblaslt": lambda: torch.matmul(a, b, out=c)},
                           rounds=vendor_rounds[0], per_round=4 * vendor_rounds[1])
        k_vendor = {"library": "torch.matmul (hipBLASLt)", "us": round(med["hipblaslt"] * 1e3, 2),
                    "ours_same_rounds_us": round(med["ours"] * 1e3, 2),
                    "speedup": round(med["hipblaslt"] / med["ours"], 3)}
    gemm_k256_obj = {
        "metric": "GEMM fp16 8192x8192x256 (the reference's test and chart shape)",
        "us_per_step": round(k_total / k_steps * 1e3, 2),
        "tflops": round(2.0 * Mk * Nk * Kk / (k_total / k_steps * 1e-3) / 1e12, 2),
        "steps": k_steps,
        "timing": "back-to-back launches between one pair of HIP events",
        "tile": {"block_m": bm2, "block_n": bn2, "block_k": bk2, "waves": warps2, "group_m": group_m2},
        "rel_fro": k_rel,
        "roofline": {"bound": "hbm", "achieved": round(k_bytes / (k_ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(k_bytes / (k_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                     "kernel_us": round(k_ms * 1e3, 2), "algorithmic_bytes_per_launch": k_bytes,
                     "algorithmic_flop_per_launch": 2.0 * Mk * Nk * Kk},
        "c_fill_us": round(fill_med * 1e3, 2),
        "vendor": k_vendor,
    }
    _log(f"gemm 8192x8192x256: {gemm_k256_obj['us_per_step']} us/step ({gemm_k256_obj['roofline']['frac']:.3f} of HBM "
         f"peak), fill of C {gemm_k256_obj['c_fill_us']} us, vendor {k_vendor}")
    del a, b, c
    torch.cuda.empty_cache()
    return gemm_k256_obj


# The rest of the attention sweeps of BASELINE configs 3 (fp16 B4 H32 D128, N 1024..16384, causal and
# not; the headline is the non-causal N=8192 case) and 4 (bf16 B2 H16 D256 sliced, N 1024..8192).
FA_SWEEP = ([dict(B=4, H=32, N=n, D=128, dtype="fp16", causal=c, variant="optimized", input_scale=1.0)
             for n in (1024, 2048, 4096, 8192, 16384) for c in (False, True) if (n, c) != (8192, False)]
            + [dict(B=2, H=16, N=n, D=256, dtype="bf16", causal=False, variant="sliced", input_scale=0.5)
               for n in (1024, 2048, 4096, 8192)])


def _bench_fa_sweep(torch, dev, rounds: int = 3) -> dict:
    """Each FA_SWEEP case through its reference tuner class -> flash_attention (the tuned tile), timed
    beside torch's scaled_dot_product_attention (its fused flash / memory-efficient backends; a case
    neither backend takes gets no vendor figure) in alternating rounds of back-to-back launches, with
    16 sampled output rows checked against fp32 math."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    import flash_atten
    import tuner

    gen = torch.Generator(device=dev).manual_seed(SEED)
    rows_out = []
    for cfg in FA_SWEEP:
        B, H, N, D, causal = cfg["B"], cfg["H"], cfg["N"], cfg["D"], cfg["causal"]
        dt = {"fp16": torch.float16, "bf16": torch.bfloat16}[cfg["dtype"]]
        q, k, v = ((torch.randn(B, H, N, D, generator=gen, device=dev) * cfg["input_scale"]).to(dt) for _ in range(3))
        tuner_cls = {"optimized": tuner.FlashAttentionOptimizeSharedMemTuner,
                     "sliced": tuner.FlashAttentionBlockDNomaskTuner}[cfg["variant"]]
        spec = tuner_cls(tuple(q.shape), tuple(k.shape), tuple(v.shape), q.element_size(), causal=causal,
                         return_lse=False).build_flash_attention_launch_spec(q, k, v)
        flops = 4.0 * B * H * D * (N * (N + 1) / 2 if causal else N * N)
        ours = lambda: flash_atten.flash_attention(spec)
        ours()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        ours()
        e.record()
        torch.cuda.synchronize()
        per_round = max(2, min(32, int(4.0 / max(s.elapsed_time(e), 1e-3))))
        fns = {"ours": ours}

        def sdpa():
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                return F.scaled_dot_product_attention(q, k, v, is_causal=causal)

        try:
            sdpa()
            torch.cuda.synchronize()
            fns["sdpa"] = sdpa
        except RuntimeError:
            pass
        med = _alternating(torch, fns, rounds=rounds, per_round=per_round)
        # 16 sampled rows against fp32 math
        o = spec.kernel_args[3]
        pick = torch.randint(0, B * H * N, (16,), generator=torch.Generator().manual_seed(N + D + causal))
        bh, m = pick // N, pick % N
        qs, ks, vs = (t.reshape(B * H, N, D)[idx].float() for t, idx in ((q, (bh, m)), (k, bh), (v, bh)))
        sc = torch.bmm(ks, qs[:, :, None])[:, :, 0] * D ** -0.5
        if causal:
            sc = sc.masked_fill(torch.arange(N, device=dev)[None, :] > m.to(dev)[:, None], float("-inf"))
        ref = torch.bmm(torch.softmax(sc, dim=-1)[:, None, :], vs)[:, 0, :]
        err = (o.reshape(B * H, N, D)[bh, m].float() - ref).abs().max().item()
        row = {"dtype": cfg["dtype"], "variant": cfg["variant"], "B": B, "H": H, "N": N, "D": D, "causal": causal,
               "ms": round(med["ours"], 4), "tflops": round(flops / (med["ours"] * 1e-3) / 1e12, 1),
               "peak_frac": round(flops / (med["ours"] * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4),
               "tile": {"block_m": spec.kernel_kwargs["BLOCK_M"], "block_n": spec.kernel_kwargs["BLOCK_N"],
                        "waves": spec.kernel_kwargs["num_warps"], "stages": spec.kernel_kwargs["num_stages"]},
               "max_abs_err_16_rows": err,
               "vendor_ms": round(med["sdpa"], 4) if "sdpa" in med else None,
               "speedup_vs_vendor": round(med["sdpa"] / med["ours"], 3) if "sdpa" in med else None}
        rows_out.append(row)
        _log(f"attention {cfg['dtype']} D{D} N{N} {'causal' if causal else 'non-causal'}: {row['ms']} ms "
             f"({row['tflops']} TFLOP/s), SDPA {row['vendor_ms']} ms, max err {err:.2e}")
        del q, k, v, spec, o, qs, ks, vs, sc, ref, fns
        torch.cuda.empty_cache()
    return {"metric": "FA forward sweeps of BASELINE configs 3 and 4 (the headline case is the main line)",
            "protocol": f"{rounds} alternating rounds of back-to-back launches (~4 ms each), median per launch",
            "vendor_library": "torch.nn.functional.scaled_dot_product_attention (flash / memory-efficient backends)",
            "rows": rows_out}


GEMM_SWEEP_SIZES = (1024, 2048, 4096, 16384)


def _bench_gemm_sweep(torch, g, dev, rounds: int = 3) -> dict:
    """The rest of the square GEMM sweep of BASELINE config 2 (8192^3 is the `gemm` object): each
    size through the drop-in launcher and through torch.matmul (hipBLASLt), both timed as replays
    of a HIP graph holding a batch of back-to-back launches (GPU time: an eager call of either
    costs several microseconds of host time, more than a 1024^3 product takes), in alternating
    rounds. A vendor graph whose replay does not reproduce the eager product (a library call may
    record memset nodes) is timed eagerly instead, and says so."""
    import mma

    rows = []
    for n in GEMM_SWEEP_SIZES:
        a = (torch.rand(n, n, generator=g) * 2 - 1).half().to(dev)
        b = (torch.rand(n, n, generator=g) * 2 - 1).half().to(dev)
        c = torch.empty(n, n, dtype=torch.float16, device=dev)
        c2 = torch.empty(n, n, dtype=torch.float16, device=dev)
        bm, bn, bk, group_m, warps, stages = mma._select_2d_contiguous_config(n, n, n)
        grid = (math.ceil(n / bm) * math.ceil(n / bn),)

        def ours():
            mma._matmul_contiguous_kernel[grid](a, b, c, n, n, n, BLOCK_M=bm, BLOCK_N=bn, BLOCK_K=bk,
                                                GROUP_M=group_m, USE_CACHE_EVICTION_HINTS=True,
                                                num_warps=warps, num_stages=stages)

        def vendor():
            torch.matmul(a, b, out=c2)

        ours()
        vendor()
        torch.cuda.synchronize()
        ref = a.float() @ b.float()
        rel = ((c.float() - ref).norm() / ref.norm()).item()
        eager_vendor = c2.clone()
        del ref
        batch = max(2, min(64, int(4e-3 / (2.0 * n ** 3 / 1.2e15))))  # ~4 ms of work per replay
        graphs, protocol = {}, {}
        for key, fn in (("ours", ours), ("vendor", vendor)):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for _ in range(batch):
                    fn()
            gr.replay()
            torch.cuda.synchronize()
            graphs[key] = gr.replay
            protocol[key] = "graph"
        if ((c2.float() - eager_vendor.float()).norm() / eager_vendor.float().norm()).item() > 1e-3:
            graphs["vendor"] = lambda: [vendor() for _ in range(batch)]
            protocol["vendor"] = "eager (its graph replay differed from the eager product)"
        times = {k: [] for k in graphs}
        for _ in range(rounds):
            for key, run in graphs.items():
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                run()
                e.record()
                torch.cuda.synchronize()
                times[key].append(s.elapsed_time(e) / batch)
        us = {k: statistics.median(v) * 1e3 for k, v in times.items()}
        flop = 2.0 * n ** 3
        rows.append({"M": n, "N": n, "K": n, "us": round(us["ours"], 2),
                     "tflops": round(flop / (us["ours"] * 1e-6) / 1e12, 1),
                     "peak_frac": round(flop / (us["ours"] * 1e-6) / 1e12 / PEAK_FP16_TFLOPS, 4),
                     "tile": {"block_m": bm, "block_n": bn, "block_k": bk, "waves": warps, "group_m": group_m},
                     "rel_fro": rel, "vendor_us": round(us["vendor"], 2),
                     "speedup_vs_vendor": round(us["vendor"] / us["ours"], 3), "vendor_timing": protocol["vendor"]})
        _log(f"gemm {n}^3: {rows[-1]['us']} us ({rows[-1]['tflops']} TFLOP/s), hipBLASLt {rows[-1]['vendor_us']} us "
             f"({rows[-1]['speedup_vs_vendor']}x), rel_fro {rel:.2e}")
        del a, b, c, c2, eager_vendor, graphs
        torch.cuda.empty_cache()
    return {"metric": "GEMM fp16 square sweep (BASELINE config 2), GPU time per launch",
            "protocol": f"HIP-graph replays of batched back-to-back launches, {rounds} alternating rounds, median",
            "vendor_library": "torch.matmul (hipBLASLt)", "rows": rows}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # at least 10 warm-up and 30 timed launches, median and mean reported (the reference's timing
    # protocol, test_flash_atten.py:502-545)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--fa-config", default="headline", choices=sorted(FA_CONFIGS),
                    help="attention workload of the line (the default is the headline the metric names)")
    ap.add_argument("--variant", default=None, choices=["basic", "optimized", "sliced"],
                    help="attention variant (default: the workload's own)")
    ap.add_argument("--fa-tile", default=None, metavar="BM,BN,WAVES,STAGES",
                    help="attention tile as the reference's tune arguments (BLOCK_M, BLOCK_N, NUM_WARPS, "
                         "NUM_STAGES) instead of the tuning table's choice")
    ap.add_argument("--no-vendor", action="store_true", help="skip the alternating vendor-library timings")
    ap.add_argument("--no-clock", action="store_true",
                    help="skip the clock bursts after the timed launches (kernel-trace runs: the trace's last "
                         "launches of each kernel are then the timed ones)")
    ap.add_argument("--clock-warmup-ms", type=float, default=200.0,
                    help="GPU time of back-to-back launches before each kernel's warm-up launches, so the timed "
                         "launches run at the steady clock (0 disables)")
    ap.add_argument("--counter-run", action="store_true",
                    help="for rocprofv3 --pmc passes: calibration launches first, then 10 warm-up + 10 timed "
                         "launches of each kernel, no CPU or vendor legs")
    ap.add_argument("--counters-summarize", metavar="DIR",
                    help="summarise the counter passes in DIR (see COUNTER_PASSES) as markdown and exit")
    ap.add_argument("--traffic-out", metavar="JSON",
                    help="with --counters-summarize: also record the HBM bytes per launch in this file (the bench "
                         "line's roofline.traffic reads profiles/hbm_traffic_fa_fwd_configs_gemm8192.json)")
    args = ap.parse_args()
    if args.counters_summarize:
        return _counters_summarize(args.counters_summarize, args.fa_config, steps=10, fa_tile=args.fa_tile,
                                   traffic_out=args.traffic_out)
    if args.counter_run:
        args.steps, args.warmup, args.no_cpu = 10, 10, True
    # alternating vendor rounds: (rounds, launches per round); fewer under counter collection
    vendor_rounds = (2, 5) if args.counter_run else (5, 10)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one MI355X only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "the attention/GEMM path is single-GPU here (it would shard B*H, or KV splits, one share per GPU).",
              file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (gfx950)", file=sys.stderr)
        return 1
    import flash_atten
    import hip_lib
    import mma
    import tuner

    dev = torch.device("cuda:0")
    if args.counter_run:
        _calibration_launches(torch, dev)
    limits = hip_lib.device_limits(0)
    _log(f"device gfx{limits['gcn_arch']} CUs={limits['cu_count']} clock={limits['clock_khz'] / 1e6:.2f} GHz")

    # ---- attention forward ----------------------------------------------------------------------
    fa_cfg = FA_CONFIGS[args.fa_config]
    variant = args.variant or fa_cfg["variant"]
    causal = fa_cfg["causal"]
    fa_dtype = {"fp16": torch.float16, "bf16": torch.bfloat16}[fa_cfg["dtype"]]
    B, H, N, D = fa_cfg["B"], fa_cfg["H"], fa_cfg["N"], fa_cfg["D"]
    g = torch.Generator().manual_seed(SEED)
    q, k, v = ((torch.randn(B, H, N, D, generator=g) * fa_cfg["input_scale"]).to(fa_dtype).to(dev) for _ in range(3))
    tuner_cls = {
        "basic": tuner.FlashAttentionTuner,
        "optimized": tuner.FlashAttentionOptimizeSharedMemTuner,
        "sliced": tuner.FlashAttentionBlockDNomaskTuner,
    }[variant]
    tune_args = None
    if args.fa_tile:
        bm_, bn_, w_, st_ = (int(x) for x in args.fa_tile.split(","))
        tune_args = tuner.FlashAttenTuneArguments(BLOCK_M=bm_, BLOCK_N=bn_, BLOCK_N_PAD=bn_, NUM_WARPS=w_,
                                                  NUM_STAGES=st_)
    spec = tuner_cls(tuple(q.shape), tuple(k.shape), tuple(v.shape), q.element_size(), causal=causal,
                     return_lse=False, tune_args=tune_args).build_flash_attention_launch_spec(q, k, v)
    if tune_args is not None and spec.launch_context.get("tune_args_relaxed"):
        raise SystemExit(f"--fa-tile {args.fa_tile} is not built for this workload "
                         f"(relaxed: {spec.launch_context['tune_args_relaxed']})")
    # the reference's FLOP count (test_flash_atten.py:234-240): causal counts N(N+1)/2 scores per (b, h)
    fa_flops = 4.0 * B * H * D * (N * (N + 1) / 2 if causal else N * N)
    _log(f"attention {args.fa_config} {variant}: tile {spec.kernel_kwargs['BLOCK_M']}x{spec.kernel_kwargs['BLOCK_N']} "
         f"waves={spec.kernel_kwargs['num_warps']} stages={spec.kernel_kwargs['num_stages']}")
    total_ms, per = _time_launches(torch, lambda: flash_atten.flash_attention(spec), args.steps, args.warmup,
                                   args.clock_warmup_ms)
    # the clock under the same launches, after the timed ones (none beside counter passes)
    clock = ClockSampler(torch, dev) if not (args.counter_run or args.no_clock) else None
    fa_clock = clock.measure(torch, lambda: flash_atten.flash_attention(spec)) if clock else None
    fa_launch_ms = statistics.mean(per)
    fa_tflops_launch = fa_flops / (fa_launch_ms * 1e-3) / 1e12
    fa_ms_per_step = total_ms / args.steps
    fa_tflops = fa_flops / (fa_ms_per_step * 1e-3) / 1e12
    _log(f"attention: {fa_ms_per_step:.3f} ms/step, {fa_tflops:.1f} TFLOP/s "
         f"({100 * fa_tflops / PEAK_FP16_TFLOPS:.1f}% of dense fp16 peak)")

    # parity spot check on 64 sampled rows against fp32 math on the GPU
    o = spec.kernel_args[3]
    rows = torch.randint(0, B * H * N, (64,), generator=torch.Generator().manual_seed(1))
    bh, m = rows // N, rows % N
    qs = q.reshape(B * H, N, D)[bh, m].float()
    ks = k.reshape(B * H, N, D)[bh].float()
    vs = v.reshape(B * H, N, D)[bh].float()
    sc = torch.einsum("rd,rnd->rn", qs.to(dev), ks) * D ** -0.5
    if causal:  # top-left: row m sees keys j <= m
        sc = sc.masked_fill(torch.arange(N, device=dev)[None, :] > m.to(dev)[:, None], float("-inf"))
    p = torch.softmax(sc, dim=-1)
    ref = torch.einsum("rn,rnd->rd", p, vs)
    fa_err = (o.reshape(B * H, N, D)[bh, m].float() - ref).abs().max().item()
    del qs, ks, vs, sc, p, ref
    fa_vendor = None
    if not args.no_vendor:
        import torch.nn.functional as F

        med = _alternating(torch, {"ours": lambda: flash_atten.flash_attention(spec),
                                   "torch_sdpa": lambda: F.scaled_dot_product_attention(q, k, v, is_causal=causal)},
                           rounds=vendor_rounds[0], per_round=4)
        fa_vendor = {"library": "torch.nn.functional.scaled_dot_product_attention (default ROCm backend)",
                     "value": round(fa_flops / (med["torch_sdpa"] * 1e-3) / 1e12, 2),
                     "ours_same_rounds": round(fa_flops / (med["ours"] * 1e-3) / 1e12, 2),
                     "speedup": round(med["torch_sdpa"] / med["ours"], 3),
                     "protocol": f"{vendor_rounds[0]} alternating rounds of 4 back-to-back launches each, median "
                                 "per launch"}
        _log(f"attention vs torch SDPA: {fa_vendor}")
    del q, k, v, spec, o
    torch.cuda.empty_cache()

    # ---- GEMM ---------------------------------------------------------------------------------------
    M, Ng, K = GEMM_SHAPE["M"], GEMM_SHAPE["N"], GEMM_SHAPE["K"]
    a = (torch.rand(M, K, generator=g) * 2 - 1).half().to(dev)
    b = (torch.rand(K, Ng, generator=g) * 2 - 1).half().to(dev)
    c = torch.empty(M, Ng, dtype=torch.float16, device=dev)
    bm, bn, bk, group_m, warps, stages = mma._select_2d_contiguous_config(M, Ng, K)
    grid = (math.ceil(M / bm) * math.ceil(Ng / bn),)

    def gemm():
        mma._matmul_contiguous_kernel[grid](a, b, c, M, Ng, K, BLOCK_M=bm, BLOCK_N=bn, BLOCK_K=bk, GROUP_M=group_m,
                                            USE_CACHE_EVICTION_HINTS=True, num_warps=warps, num_stages=stages)

    g_total, g_per = _time_launches(torch, gemm, args.steps, args.warmup, args.clock_warmup_ms)
    gemm_clock = clock.measure(torch, gemm) if clock else None
    gemm_flops = 2.0 * M * Ng * K
    gemm_launch_ms = statistics.mean(g_per)
    gemm_tflops = gemm_flops / (g_total / args.steps * 1e-3) / 1e12
    ref = a.float() @ b.float()
    gemm_rel = ((c.float() - ref).norm() / ref.norm()).item()
    _log(f"gemm {bm}x{bn}x{bk} waves={warps} group_m={group_m}: {g_total / args.steps:.3f} ms, {gemm_tflops:.1f} TFLOP/s, rel_fro={gemm_rel:.2e}")
    del ref
    gemm_vendor = None
    if not args.no_vendor:
        med = _alternating(torch, {"ours": gemm, "hipblaslt": lambda: torch.matmul(a, b, out=c)},
                           rounds=vendor_rounds[0], per_round=vendor_rounds[1])
        gemm_vendor = {"library": "torch.matmul (hipBLASLt)",
                       "clock_ghz": clock.measure(torch, lambda: torch.matmul(a, b, out=c)) if clock else None,
                       "value": round(gemm_flops / (med["hipblaslt"] * 1e-3) / 1e12, 2),
                       "ours_same_rounds": round(gemm_flops / (med["ours"] * 1e-3) / 1e12, 2),
                       "speedup": round(med["hipblaslt"] / med["ours"], 3),
                       "protocol": f"{vendor_rounds[0]} alternating rounds of {vendor_rounds[1]} back-to-back "
                                   "launches each, median per launch"}
        _log(f"gemm vs hipBLASLt: {gemm_vendor}")
    del a, b, c
    torch.cuda.empty_cache()

    # ---- GEMM at the reference's own test and chart shape (test_mma.py:42-45) ------------------------
    # 8192x8192x256: 128 MiB of C against 8 MiB of A and B, so the roofline is HBM (142.6 MB per launch,
    # 17.8 us at 8 TB/s); beside it, torch's fill of the same C (a pure 128 MiB write stream) on this GPU.
    # (not in counter runs: their summaries take each kernel's last dispatches as the 8192^3 launches)
    gemm_k256_obj = None if args.counter_run else _bench_gemm_k256(torch, args, g, dev, vendor_rounds)
    # ---- the rest of config 2's square sweep, beside hipBLASLt in GPU time (not in counter or trace runs)
    gemm_sweep_obj = None if (args.counter_run or args.no_vendor) else _bench_gemm_sweep(torch, g, dev)
    # ---- the rest of configs 3 and 4's attention sweeps, beside torch SDPA (same runs skip it)
    fa_sweep_obj = None if (args.counter_run or args.no_vendor) else _bench_fa_sweep(torch, dev)

    # ---- CPU baseline (reference CPU path, bounded sample) ---------------------------------------
    cpu_fa = cpu_gemm = None
    if not args.no_cpu:
        _log("timing the CPU baseline (the reference's CPU path on this host)")
        cpu_fa = _cpu_baseline_attention(torch, B, H, N, D)
        cpu_gemm = _cpu_baseline_gemm(torch, M, Ng, K)

    traffic = gemm_traffic = None
    if TRAFFIC_FILE.exists() and not args.fa_tile and args.variant is None:
        try:
            recorded = json.loads(TRAFFIC_FILE.read_text())
            # recorded for each workload's own variant and tuned tile
            traffic = recorded.get(f"fa_fwd_{args.fa_config}", {}).get("bytes_per_launch")
            gemm_traffic = recorded.get("gemm_f16_8192cube", {}).get("bytes_per_launch")
        except (ValueError, OSError):
            traffic = gemm_traffic = None

    line = {
        "metric": "FA fwd TFLOP/s + % fp16 MFMA peak (D=128,N=8k); GEMM TFLOP/s at 8192^3",
        "value": round(fa_tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(fa_ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": fa_cfg["dtype"],
        "data": (f"synthetic (torch.randn x {fa_cfg['input_scale']} rounded to {fa_cfg['dtype']}, seed 20260328)"),
        "config": {"workload": (f"FlashAttention forward, {variant} variant, {'causal' if causal else 'non-causal'}, "
                                f"sm_scale=1/sqrt(D)"),
                   "B": B, "H": H, "N": N, "D": D, "causal": causal},
        "mfma_peak_frac": round(fa_tflops / PEAK_FP16_TFLOPS, 4),
        "clock_ghz": fa_clock,
        "roofline": {
            "bound": "mfma",
            "achieved": round(fa_tflops_launch, 2),
            "peak": PEAK_FP16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(fa_tflops_launch / PEAK_FP16_TFLOPS, 4),
            "traffic": traffic,
            "kernel_ms": round(fa_launch_ms, 4),
            "kernel_ms_median": round(statistics.median(per), 4),
            "algorithmic_flop_per_launch": fa_flops,
            "algorithmic_bytes_per_launch": 4 * B * H * N * D * 2,
        },
        "cpu_baseline": cpu_fa,
        "vendor": fa_vendor,
        "parity": {"fa_max_abs_err_64_rows": fa_err, "gemm_rel_fro": gemm_rel},
        "gemm": {
            "metric": "GEMM fp16 TFLOP/s at 8192^3",
            "value": round(gemm_tflops, 2),
            "ms_per_step": round(g_total / args.steps, 4),
            "tile": {"block_m": bm, "block_n": bn, "block_k": bk, "waves": warps, "group_m": group_m},
            "clock_ghz": gemm_clock,
            "roofline": {
                "bound": "mfma",
                "achieved": round(gemm_flops / (gemm_launch_ms * 1e-3) / 1e12, 2),
                "peak": PEAK_FP16_TFLOPS,
                "unit": "TFLOP/s",
                "frac": round(gemm_flops / (gemm_launch_ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4),
                "traffic": gemm_traffic,
                "kernel_ms": round(gemm_launch_ms, 4),
                "kernel_ms_median": round(statistics.median(g_per), 4),
                "algorithmic_flop_per_launch": gemm_flops,
                "algorithmic_bytes_per_launch": 2 * (M * K + K * Ng + M * Ng),
            },
            "cpu_baseline": cpu_gemm,
            "vendor": gemm_vendor,
        },
        "gemm_k256": gemm_k256_obj,
        "gemm_sweep": gemm_sweep_obj,
        "fa_sweep": fa_sweep_obj,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
