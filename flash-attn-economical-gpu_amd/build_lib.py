"""Build libfa_gfx950.so (the C-ABI HIP library) in-tree with hipcc for gfx950.

Usage: python build_lib.py [--jobs N]

Each csrc/*.hip file is compiled to an object in _build/ (in parallel), then linked into
libfa_gfx950.so next to this file. The compiler's kernel-resource-usage remarks are parsed into
kernel_resources.json (VGPR/AGPR/SGPR counts, LDS bytes, scratch, occupancy per kernel symbol), which
the tuner's resource filter and the resource report read on hosts without a GPU. Measurement
programs under probes/ (not part of the library) are built into executables next to their sources.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import json
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
PROBES = HERE / "probes"
LIB = HERE / "libfa_gfx950.so"
RESOURCES = HERE / "kernel_resources.json"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # Packed fp32 VALU ops stay off: plain float code only.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # No kernel produces or tests NaN (masked scores are -inf, kept: infinities stay honoured), so
    # fmaxf needs no operand canonicalisation and v_max3 applies directly to MFMA results.
    "-fno-honor-nans",
    "-mno-amdgpu-ieee",
    "-Rpass-analysis=kernel-resource-usage",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


_REMARK_RE = re.compile(r"^(\S+):(\d+):\d+: remark: (.*?) \[-Rpass-analysis=kernel-resource-usage\]")


def _parse_resources(stderr: str) -> dict[str, dict[str, object]]:
    """Parse `-Rpass-analysis=kernel-resource-usage` remarks into {kernel: {field: value}}."""
    kernels: dict[str, dict[str, object]] = {}
    current: str | None = None
    for line in stderr.splitlines():
        m = _REMARK_RE.search(line)
        if not m:
            continue
        text = m.group(3).strip()
        if text.startswith("Function Name:"):
            current = text.split(":", 1)[1].strip()
            kernels[current] = {}
            continue
        if current is None or ":" not in text:
            continue
        key, value = (part.strip() for part in text.split(":", 1))
        try:
            kernels[current][key] = int(value.split()[0])
        except ValueError:
            kernels[current][key] = value
    return kernels


def _compile(src: Path) -> tuple[Path, dict[str, dict[str, object]]]:
    obj = BUILD / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stderr)
        raise RuntimeError(f"hipcc failed for {src.name} (exit {proc.returncode})")
    return obj, _parse_resources(proc.stderr)


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, min(16, os.cpu_count() or 1)))
    resources: dict[str, dict[str, object]] = {}
    objects: list[Path] = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        for obj, res in pool.map(_compile, sources):
            objects.append(obj)
            resources.update(res)
            if verbose:
                print(f"[build] compiled {obj.name}", flush=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stderr)
        raise RuntimeError("link of libfa_gfx950.so failed")
    os.replace(tmp, LIB)
    RESOURCES.write_text(json.dumps(resources, indent=1, sort_keys=True) + "\n")
    if verbose:
        print(f"[build] linked {LIB} ({len(resources)} kernels with resource data)", flush=True)
    for exe in build_probes():
        if verbose:
            print(f"[build] probe {exe}", flush=True)
    return LIB


def build_probes() -> list[Path]:
    """Standalone measurement programs (probes/*.hip -> probes/<name>); not part of the library."""
    built = []
    for src in sorted(PROBES.glob("*.hip")):
        exe = PROBES / src.stem
        cmd = [_hipcc(), *(f for f in HIPCC_FLAGS if not f.startswith("-Rpass") and f != "-fPIC"), "-o", str(exe),
               str(src)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            sys.stderr.write(proc.stderr)
            raise RuntimeError(f"hipcc failed for probe {src.name} (exit {proc.returncode})")
        built.append(exe)
    return built


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    build(args.jobs)
