"""Host logic of bench.py (no GPU): the one-GPU guard and the calibration that turns the two
rocprofv3 counter passes (FETCH_SIZE, WRITE_SIZE in KiB per dispatch) into HBM bytes per launch."""
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


def _counter_csv(path: Path, rows: list[tuple[int, str, list[float]]]) -> None:
    """rocprofv3 counter_collection layout: one row per counter instance of a dispatch."""
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for dispatch, name, values in rows:
            for v in values:
                w.writerow({"Dispatch_Id": dispatch, "Kernel_Name": name, "Counter_Name": "X", "Counter_Value": v})


def test_traffic_calibration(tmp_path):
    bench = _bench()
    copy = "void at::native::elementwise_kernel<copy>(...)"
    fa = "void fa::fa_fwd_kernel<fa::f16_t, 128, 4, 1, 64, 3, false>(fa::FwdParams)"
    gemm = "void fa::gemm_f16_kernel<256, 256, 64, 2, 4>(fa::GemmParams)"
    copy_kib = 256 * 1024  # the 256 MiB calibration copy
    # FETCH_SIZE reads half of the copy's bytes (factor 2), split over two counter instances;
    # WRITE_SIZE reads them exactly (factor 1)
    _counter_csv(tmp_path / "fetch.csv", [(1, copy, [copy_kib / 4, copy_kib / 4]), (2, fa, [1000.0, 500.0]),
                                          (3, gemm, [3000.0])])
    _counter_csv(tmp_path / "write.csv", [(1, copy, [copy_kib]), (2, fa, [256.0]), (3, gemm, [128.0, 128.0])])
    out = tmp_path / "traffic.json"
    assert bench._traffic_summarize(str(tmp_path / "fetch.csv"), str(tmp_path / "write.csv"), out) == 0
    t = json.loads(out.read_text())
    assert t["calibration"]["fetch_factor"] == 2.0 and t["calibration"]["write_factor"] == 1.0
    fa_t = t["fa_fwd_b4h32n8192d128_f16"]
    assert fa_t["bytes_read"] == 1500 * 1024 * 2 and fa_t["bytes_written"] == 256 * 1024
    assert fa_t["algorithmic_bytes_per_launch"] == 4 * 4 * 32 * 8192 * 128 * 2  # |Q|+|K|+|V|+|O| fp16
    g = t["gemm_f16_8192cube"]
    assert g["bytes_per_launch"] == 3000 * 1024 * 2 + 256 * 1024
    assert g["algorithmic_bytes_per_launch"] == 2 * 3 * 8192 * 8192
    assert g["ratio_to_algorithmic"] == pytest.approx(g["bytes_per_launch"] / g["algorithmic_bytes_per_launch"],
                                                      abs=1e-4)


def test_committed_traffic_file_matches_the_summary_schema():
    t = json.loads((ROOT / "profiles" / "hbm_traffic_fa_b4h32n8192d128_gemm8192.json").read_text())
    for key in ("fa_fwd_b4h32n8192d128_f16", "gemm_f16_8192cube"):
        e = t[key]
        assert e["bytes_per_launch"] == e["bytes_read"] + e["bytes_written"]
        assert e["bytes_per_launch"] >= e["algorithmic_bytes_per_launch"] * 0.99
