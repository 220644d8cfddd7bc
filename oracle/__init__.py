"""CPU oracle for the attention / GEMM hot path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, and
only as the checker (or the timed CPU baseline). The product path (libfa_gfx950.so and the
modules beside it) never imports it.

Contents:
  * ``portable_normal`` / ``portable_uniform``: seeded input generators whose streams are fixed
    by this file (splitmix64 + Box-Muller), so CPU fixtures and GPU tests see identical inputs on
    any numpy version.
  * ctypes wrappers of oracle.c (``attention``, ``attention_rows``, ``attention_online``,
    ``lse_merge``, ``gemm``, ``gemm_entries``, ``round_to``).
  * ``attention_np`` / ``gemm_np``: numpy float64 restatements used to cross-check the C code.

Reference citations (relative to the reference repository) are in oracle.c.
"""
from __future__ import annotations

import ctypes
import math
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    """Compile oracle.c with gcc (Makefile beside this file)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    f32p = ctypes.POINTER(ctypes.c_float)
    f64p = ctypes.POINTER(ctypes.c_double)
    i64p = ctypes.POINTER(ctypes.c_int64)
    i32 = ctypes.c_int
    lib.oracle_attention.argtypes = [f32p, f32p, f32p, f32p, f32p, i32, i32, i32, i32, i32, i32,
                                     ctypes.c_double, i32]
    lib.oracle_attention_rows.argtypes = [f32p, f32p, f32p, i64p, ctypes.c_int64, f32p, f32p, i32, i32, i32,
                                          i32, i32, i32, ctypes.c_double, i32]
    lib.oracle_attention_online.argtypes = [f32p, f32p, f32p, f32p, f32p, i32, i32, i32, i32, i32, i32,
                                            ctypes.c_float, i32, i32, i32]
    lib.oracle_lse_merge.argtypes = [f32p, f32p, i32, ctypes.c_int64, i32, f32p, f32p]
    lib.oracle_gemm.argtypes = [f32p, f32p, f32p, i32, i32, i32]
    lib.oracle_gemm_entries.argtypes = [f32p, f32p, i64p, i64p, ctypes.c_int64, f64p, i32, i32, i32]
    lib.oracle_round_array.argtypes = [f32p, f32p, ctypes.c_int64, i32]
    for name in ("oracle_attention", "oracle_attention_rows", "oracle_attention_online", "oracle_lse_merge",
                 "oracle_gemm", "oracle_gemm_entries"):
        getattr(lib, name).restype = ctypes.c_int
    lib.oracle_round_array.restype = None
    _lib = lib
    return lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _ptr(a: np.ndarray, ctype=ctypes.c_float):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _check(code: int, what: str) -> None:
    if code != 0:
        raise ValueError(f"{what} failed with code {code}")


# ---- portable seeded generators -----------------------------------------------------------------

_MASK64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix64(seed: int, n: int) -> np.ndarray:
    """n outputs of splitmix64 (Steele, Lea, Flood 2014) started at `seed`."""
    with np.errstate(over="ignore"):
        idx = np.arange(1, n + 1, dtype=np.uint64)
        z = (np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * np.uint64(0x9E3779B97F4A7C15)) & _MASK64
        z = ((z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)) & _MASK64
        z = ((z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)) & _MASK64
        return z ^ (z >> np.uint64(31))


def portable_uniform(seed: int, shape, low: float = 0.0, high: float = 1.0) -> np.ndarray:
    """Uniform [low, high) float64 with 53-bit resolution; stream fixed by this file."""
    n = int(np.prod(shape)) if len(shape) else 1
    u = (_splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    return (low + (high - low) * u).reshape(shape)


def portable_normal(seed: int, shape) -> np.ndarray:
    """Standard normal float64 by Box-Muller over portable_uniform pairs."""
    n = int(np.prod(shape)) if len(shape) else 1
    m = (n + 1) // 2
    u = portable_uniform(seed, (2 * m,))
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * math.pi * u2)
    z[1::2] = r * np.sin(2.0 * math.pi * u2)
    return z[:n].reshape(shape)


# ---- rounding ---------------------------------------------------------------------------------

DTYPE_F16, DTYPE_BF16 = 0, 1


def round_to(x, dtype: int) -> np.ndarray:
    """Round float32 values to binary16 (dtype 0) or bfloat16 (dtype 1), RNE; returned as float32."""
    a = _f32(x)
    out = np.empty_like(a)
    _load().oracle_round_array(_ptr(a), _ptr(out), a.size, dtype)
    return out


# ---- attention ----------------------------------------------------------------------------------

def attention(q, k, v, *, scale: float | None = None, causal: bool = False):
    """Exact attention in double precision. q [B,H,M,D], k/v [B,Hkv,N,D] -> (o fp32, lse fp32)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, M, D = q.shape
    _, Hkv, N, _ = k.shape
    scale = D ** -0.5 if scale is None else scale
    o = np.empty((B, H, M, D), dtype=np.float32)
    lse = np.empty((B, H, M), dtype=np.float32)
    _check(_load().oracle_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), B, H, Hkv, M, N, D,
                                    float(scale), int(causal)), "oracle_attention")
    return o, lse


def attention_rows(q, k, v, rows, *, scale: float | None = None, causal: bool = False):
    """Exact attention for selected flattened rows (b*H + h)*M + m -> (o [n,D], lse [n])."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, M, D = q.shape
    _, Hkv, N, _ = k.shape
    scale = D ** -0.5 if scale is None else scale
    rows = np.ascontiguousarray(np.asarray(rows, dtype=np.int64))
    o = np.empty((rows.size, D), dtype=np.float32)
    lse = np.empty((rows.size,), dtype=np.float32)
    _check(_load().oracle_attention_rows(_ptr(q), _ptr(k), _ptr(v), _ptr(rows, ctypes.c_int64), rows.size,
                                         _ptr(o), _ptr(lse), B, H, Hkv, M, N, D, float(scale), int(causal)),
           "oracle_attention_rows")
    return o, lse


def attention_online(q, k, v, *, scale: float | None = None, causal: bool = False, block_n: int = 64,
                     dtype: int = DTYPE_F16):
    """The reference kernel's blocked fp32 online softmax with P rounded to `dtype`."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, M, D = q.shape
    _, Hkv, N, _ = k.shape
    scale = D ** -0.5 if scale is None else scale
    o = np.empty((B, H, M, D), dtype=np.float32)
    lse = np.empty((B, H, M), dtype=np.float32)
    _check(_load().oracle_attention_online(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), B, H, Hkv, M, N, D,
                                           float(scale), int(causal), int(block_n), int(dtype)),
           "oracle_attention_online")
    return o, lse


def lse_merge(o_parts, lse_parts):
    """o_parts [S, rows, D], lse_parts [S, rows] -> (o [rows, D], lse [rows])."""
    o_parts, lse_parts = _f32(o_parts), _f32(lse_parts)
    S, R, D = o_parts.shape
    o = np.empty((R, D), dtype=np.float32)
    lse = np.empty((R,), dtype=np.float32)
    _check(_load().oracle_lse_merge(_ptr(o_parts), _ptr(lse_parts), S, R, D, _ptr(o), _ptr(lse)), "oracle_lse_merge")
    return o, lse


def attention_np(q, k, v, *, scale: float | None = None, causal: bool = False):
    """numpy float64 restatement (cross-check of the C oracle)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, H, M, D = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    scale = D ** -0.5 if scale is None else scale
    kk = np.repeat(k, H // Hkv, axis=1)
    vv = np.repeat(v, H // Hkv, axis=1)
    s = np.einsum("bhmd,bhnd->bhmn", q, kk) * scale
    if causal:
        mask = np.arange(N)[None, :] > np.arange(M)[:, None]
        s = np.where(mask, -np.inf, s)
    mx = s.max(axis=-1, keepdims=True)
    p = np.exp(s - mx)
    l = p.sum(axis=-1, keepdims=True)
    o = np.einsum("bhmn,bhnd->bhmd", p / l, vv)
    return o, (mx + np.log(l))[..., 0]


# ---- GEMM ---------------------------------------------------------------------------------------

def gemm(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    M, K = a.shape
    _, N = b.shape
    c = np.empty((M, N), dtype=np.float32)
    _check(_load().oracle_gemm(_ptr(a), _ptr(b), _ptr(c), M, N, K), "oracle_gemm")
    return c


def gemm_entries(a, b, ii, jj) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    M, K = a.shape
    _, N = b.shape
    ii = np.ascontiguousarray(np.asarray(ii, dtype=np.int64))
    jj = np.ascontiguousarray(np.asarray(jj, dtype=np.int64))
    out = np.empty(ii.size, dtype=np.float64)
    _check(_load().oracle_gemm_entries(_ptr(a), _ptr(b), _ptr(ii, ctypes.c_int64), _ptr(jj, ctypes.c_int64), ii.size,
                                       _ptr(out, ctypes.c_double), M, N, K), "oracle_gemm_entries")
    return out


def gemm_np(a, b) -> np.ndarray:
    return np.asarray(a, dtype=np.float64) @ np.asarray(b, dtype=np.float64)


def attention_flops(B: int, H: int, M: int, N: int, D: int, causal: bool) -> float:
    """FLOP convention of the reference (test_flash_atten.py:234-240): 4*B*H*D*scores, where
    scores = S*(S+1)/2 when causal (square) else M*N."""
    if causal:
        scores = M * (M + 1) / 2 if M == N else sum(min(m + 1, N) for m in range(M))
    else:
        scores = M * N
    return 4.0 * B * H * D * scores


def gemm_flops(M: int, N: int, K: int) -> float:
    """2*M*K*N (test_mma.py:78-83)."""
    return 2.0 * M * N * K
