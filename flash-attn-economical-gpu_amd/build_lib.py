"""Build libfa_gfx950.so (the C-ABI HIP library) in-tree with hipcc for gfx950.

Usage: python build_lib.py [--jobs N]

Each csrc/*.hip file is compiled to an object in _build/ (in parallel), then linked into
libfa_gfx950.so next to this file. The compiler's kernel-resource-usage remarks are parsed into
kernel_resources.json (VGPR/AGPR/SGPR counts, LDS bytes, scratch, occupancy per kernel symbol), which
the tuner's resource filter and the resource report read on hosts without a GPU. Each file is also
compiled to device assembly (_build/*.s) and checked for the gfx9 hazards the compiler leaves to
hand-written asm (asm_hazards); a hit fails the build.
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


_SGPR_RE = re.compile(r"\bs\[(\d+):(\d+)\]|\bs(\d+)\b")


def _sgprs(text: str) -> set[int]:
    out: set[int] = set()
    for m in _SGPR_RE.finditer(text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def _valu_sgpr_defs(instr: str) -> set[int]:
    """SGPRs a vector-ALU instruction writes: the destination of v_readfirstlane / v_readlane, the
    mask of a VOP3 compare, the carry-out of a VOP3 *_co_* add."""
    op, _, rest = instr.partition(" ")
    if not op.startswith("v_"):
        return set()
    operands = [o.strip() for o in rest.split(",")]
    if op.startswith(("v_readfirstlane", "v_readlane")) or (op.startswith("v_cmp") and op.endswith("_e64")):
        return _sgprs(operands[0]) if operands else set()
    if "_co_" in op and op.endswith("_e64") and len(operands) > 1:
        return _sgprs(operands[1])
    return set()


def asm_hazards(asm: str) -> list[str]:
    """Hazards the compiler does not cover around the kernels' inline-asm memory instructions (gfx9):
    a vector-memory instruction reading an SGPR within 5 wait states of a VALU write to it, and a
    store of more than 8 bytes whose asm block does not end in an s_nop (a VALU write to its data
    VGPRs needs 1 wait state after it)."""
    lines = asm.splitlines()
    found: list[str] = []
    func = "?"
    in_asm = False
    for k, line in enumerate(lines):
        t = line.strip()
        if re.match(r"^_Z\w+:", line):
            func = line.split(":")[0]
        if t.startswith(";;#ASMSTART"):
            in_asm, block_start = True, k
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not in_asm or not t.startswith(("buffer_load", "buffer_store")):
            continue
        op, _, rest = t.partition(" ")
        if op.startswith("buffer_store") and op.endswith(("dwordx3", "dwordx4")):
            nxt = next((lines[j].strip() for j in range(k + 1, len(lines)) if lines[j].strip()), "")
            if not nxt.startswith("s_nop"):
                found.append(f"{func}: asm {op} without a following s_nop")
        used = _sgprs(rest)
        waits, j = 0, k - 1
        while j >= 0 and waits < 5:
            u = lines[j].strip()
            j -= 1
            if not u or u.startswith((";", ".")):
                continue
            if u.startswith("s_nop"):
                waits += int(u.split()[1], 0) + 1
                continue
            if _valu_sgpr_defs(u) & used:
                found.append(f"{func}: '{u}' writes an SGPR that asm '{op}' reads {waits} wait states later")
                break
            waits += 1
    return found


def _compile(src: Path) -> tuple[Path, dict[str, dict[str, object]]]:
    obj = BUILD / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stderr)
        raise RuntimeError(f"hipcc failed for {src.name} (exit {proc.returncode})")
    # the same device code as assembly, checked for hazards around the inline-asm memory instructions
    asm = BUILD / (src.stem + ".s")
    flags = [f for f in HIPCC_FLAGS if not f.startswith("-Rpass")]
    aproc = subprocess.run([_hipcc(), *flags, "--cuda-device-only", "-S", str(src), "-o", str(asm)],
                           capture_output=True, text=True)
    if aproc.returncode != 0:
        sys.stderr.write(aproc.stderr)
        raise RuntimeError(f"hipcc -S failed for {src.name} (exit {aproc.returncode})")
    hazards = asm_hazards(asm.read_text())
    if hazards:
        raise RuntimeError(f"{src.name}: {len(hazards)} inline-asm hazard(s), first: {hazards[0]}")
    return obj, _parse_resources(proc.stderr)


# Remark fields -> KernelResourceRow fields (csrc/fa_kernels.h), in declaration order.
_ROW_FIELDS = (("VGPRs", "vgprs"), ("AGPRs", "agprs"), ("TotalSGPRs", "sgprs"), ("LDS Size [bytes/block]", "lds_bytes"),
               ("ScratchSize [bytes/lane]", "scratch_bytes"), ("Occupancy [waves/SIMD]", "occupancy"))


def resource_table_source(resources: dict[str, dict[str, object]]) -> str:
    """C++ source of fa::kKernelResourceRows: one row per compiled kernel, from its remarks."""
    rows = []
    for sym in sorted(resources):
        vals = []
        for key, _ in _ROW_FIELDS:
            v = resources[sym].get(key)
            if not isinstance(v, int):
                raise RuntimeError(f"resource remark {key!r} missing for {sym}")
            vals.append(str(v))
        rows.append(f'    {{"{sym}", {", ".join(vals)}}},')
    return "\n".join([
        "// Generated by build_lib.py from the compiler's kernel-resource-usage remarks.",
        '#include "../csrc/fa_kernels.h"',
        "namespace fa {",
        "const KernelResourceRow kKernelResourceRows[] = {",
        *rows,
        "};",
        "const int kKernelResourceRowCount = (int)(sizeof(kKernelResourceRows) / sizeof(kKernelResourceRows[0]));",
        "}  // namespace fa",
        "",
    ])


def _compile_resource_table(resources: dict[str, dict[str, object]]) -> Path:
    src = BUILD / "kernel_resource_table.cpp"
    obj = BUILD / "kernel_resource_table.o"
    src.write_text(resource_table_source(resources))
    # plain host C++ (no device code): the system compiler
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stderr)
        raise RuntimeError("compile of the kernel resource table failed")
    return obj


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
    objects.append(_compile_resource_table(resources))
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
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    build(args.jobs)
