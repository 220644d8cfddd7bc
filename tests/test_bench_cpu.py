"""Host logic of bench.py (no GPU): the one-GPU guard and the summary of the rocprofv3 counter
passes (warmed dispatches only; FETCH_SIZE / WRITE_SIZE in KiB per dispatch calibrated into HBM
bytes per launch)."""
from __future__ import annotations

import csv
import importlib.util
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=120)
    assert proc.returncode == 2
    assert "one MI355X only" in proc.stderr
    assert proc.stdout == ""  # no JSON line for a configuration that was not measured


def _pass_csv(path: Path, dispatches: list[tuple[str, dict[str, float], int]]) -> None:
    """rocprofv3 counter_collection layout: one row per (dispatch, counter), with timestamps."""
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value",
                                           "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for i, (name, counters, ns) in enumerate(dispatches, start=1):
            for c, v in counters.items():
                w.writerow({"Dispatch_Id": i, "Kernel_Name": name, "Counter_Name": c, "Counter_Value": v,
                            "Start_Timestamp": 1000 * i, "End_Timestamp": 1000 * i + ns})


def test_counter_summary_and_traffic_calibration(tmp_path):
    """Synthetic passes: the three calibration adds read half (FETCH_SIZE) and all (WRITE_SIZE) of
    their bytes, so the factors are 2 and 1 at every size; per-kernel figures are the means over the
    last 10 dispatches (the 10 warm-up ones carry other values and must not count)."""
    bench = _bench()
    add = "void at::native::vectorized_elementwise_kernel<4, at::native::CUDAFunctorOnSelf_add<float>>(...)"
    fill = "void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<float>>(...)"
    fa = "void fa::fa_fwd_kernel<fa::f16_t, 128, 4, 1, 64, 3, false>(fa::FwdParams)"
    gemm = "void fa::gemm_f16_kernel<256, 256, 64, 2, 4>(fa::GemmParams)"
    ns_fa, ns_gemm = 4_000_000, 1_000_000
    for name, counters in bench.COUNTER_PASSES.items():
        names = counters.split()
        rows = []
        for mib in bench.CALIBRATION_MIB:
            kib = mib * 1024
            rows.append((fill, {c: (kib if c == "WRITE_SIZE" else 1.0) for c in names}, 1000))
            rows.append((add, {c: (kib / 2 if c == "FETCH_SIZE" else kib if c == "WRITE_SIZE" else 1.0)
                               for c in names}, 1000))
        for warm in (True, False):
            for _ in range(10):
                v_fa = {c: 7.0 for c in names}
                v_fa.update({"GRBM_GUI_ACTIVE": 8 * 6.0e6, "SQ_VALU_MFMA_BUSY_CYCLES": 1024 * 3.0e6,
                             "SQ_INSTS_MFMA": 1.342e8, "SQ_INSTS_VALU": 5.0 * 1.342e8, "SQ_WAVE_CYCLES": 1.0e9,
                             "FETCH_SIZE": 393216.0, "WRITE_SIZE": 262144.0})
                if warm:
                    v_fa = {c: 99.0 for c in names}
                rows.append((fa, {c: v_fa.get(c, 7.0) for c in names}, ns_fa))
                rows.append((gemm, {c: (1.0e6 if c == "FETCH_SIZE" else 131072.0 if c == "WRITE_SIZE" else 3.0)
                                    for c in names}, ns_gemm))
        _pass_csv(tmp_path / f"{name}_counter_collection.csv", rows)
    out = tmp_path / "traffic.json"
    assert bench._counters_summarize(str(tmp_path), "headline", steps=10, traffic_out=str(out)) == 0
    t = json.loads(out.read_text())
    cal = t["calibration_headline"]
    assert cal["fetch_factors_per_size"] == [2.0, 2.0, 2.0] and cal["write_factors_per_size"] == [1.0, 1.0, 1.0]
    fa_t = t["fa_fwd_headline"]
    assert fa_t["bytes_read"] == 393216 * 1024 * 2 and fa_t["bytes_written"] == 262144 * 1024  # Q+K+V, O
    assert fa_t["algorithmic_bytes_per_launch"] == 4 * 4 * 32 * 8192 * 128 * 2  # |Q|+|K|+|V|+|O| fp16
    assert fa_t["ratio_to_algorithmic"] == pytest.approx(1.0)
    g = t["gemm_f16_8192cube"]
    assert g["bytes_per_launch"] == g["bytes_read"] + g["bytes_written"]
    assert g["algorithmic_bytes_per_launch"] == 2 * 3 * 8192 * 8192


def test_committed_traffic_file_matches_the_summary_schema():
    t = json.loads((ROOT / "profiles" / "hbm_traffic_fa_fwd_configs_gemm8192.json").read_text())
    for key in ("fa_fwd_headline", "fa_fwd_fp16_d128_causal", "fa_fwd_bf16_d256", "gemm_f16_8192cube"):
        e = t[key]
        assert e["bytes_per_launch"] == e["bytes_read"] + e["bytes_written"]
        assert e["bytes_per_launch"] >= e["algorithmic_bytes_per_launch"] * 0.99
        assert "bench.py --counter-run" in e["command"]
