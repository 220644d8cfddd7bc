"""Input generation and comparison helpers shared by the tests (oracle-side code only)."""
from __future__ import annotations

import numpy as np
import torch

import oracle

# Tolerances from the north star: attention max-abs error vs the fp32-accumulated oracle.
ATOL = {torch.float16: 2e-2, torch.bfloat16: 3e-2}
GEMM_REL_FRO = 1e-3

ORACLE_DTYPE = {torch.float16: oracle.DTYPE_F16, torch.bfloat16: oracle.DTYPE_BF16}


def make_qkv(seed: int, B: int, H: int, Hkv: int, M: int, N: int, D: int, dtype: torch.dtype, scale: float = 1.0):
    """Seeded q [B,H,M,D], k/v [B,Hkv,N,D] (N(0,1)*scale, rounded to dtype) as float32 numpy arrays."""
    od = ORACLE_DTYPE[dtype]
    q = oracle.round_to(oracle.portable_normal(seed, (B, H, M, D)) * scale, od)
    k = oracle.round_to(oracle.portable_normal(seed + 1, (B, Hkv, N, D)) * scale, od)
    v = oracle.round_to(oracle.portable_normal(seed + 2, (B, Hkv, N, D)) * scale, od)
    return q, k, v


def to_device(a: np.ndarray, dtype: torch.dtype, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype=dtype).to(device)


def max_abs(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - b)))


def rel_fro(actual, expected) -> float:
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    return float(np.linalg.norm(actual - expected) / max(np.linalg.norm(expected), 1e-30))


def oracle_rows_threaded(q, k, v, rows, *, causal: bool, scale: float | None = None, threads: int | None = None):
    """oracle.attention_rows over `rows` (flattened (b*H + h)*M + m) split across host threads.

    The C oracle runs without the GIL, so the chunks run in parallel; at most 16 threads (the GPU
    box's CPU share)."""
    import os
    from concurrent.futures import ThreadPoolExecutor

    rows = np.asarray(rows, dtype=np.int64)
    n = threads or max(1, min(16, len(os.sched_getaffinity(0))))
    chunks = [c for c in np.array_split(rows, n) if c.size]
    with ThreadPoolExecutor(len(chunks)) as ex:
        parts = list(ex.map(lambda c: oracle.attention_rows(q, k, v, c, causal=causal, scale=scale), chunks))
    return np.concatenate([p[0] for p in parts]), np.concatenate([p[1] for p in parts])
