"""fp16 GEMM on MI355X (gfx950): the reference's `mma.py` surface over a hand-written HIP kernel.

  * ``_matmul_contiguous_kernel[grid](a, b, c, M, N, K, BLOCK_M=, BLOCK_N=, BLOCK_K=, GROUP_M=,
    USE_CACHE_EVICTION_HINTS=, num_warps=, num_stages=)`` writes C = A @ B (fp32 accumulation,
    fp16 result) into the caller's ``c``, as mma.py:8-52 does. The BLOCK_* values are hints: a
    built gfx950 tile with those sizes that divides the problem is used, otherwise the tuned tile
    for (M, N, K). The grid argument is accepted (and may be a callable) but the launch computes
    its own grid for the chosen tile.
  * ``_select_2d_contiguous_config(m, n, k)`` returns (BLOCK_M, BLOCK_N, BLOCK_K, GROUP_M,
    num_warps, num_stages) for gfx950 (num_warps = wavefronts per workgroup, num_stages = LDS
    buffers) and raises ValueError for exactly the shapes the reference rejects (mma.py:63-81).
  * ``_supports_contiguous_cache_eviction_hints(device)`` keeps the reference contract
    (mma.py:55-60): True when a GPU with compute capability major >= 8 is present (gfx950 reports
    9.5). The hint is accepted by the launcher; the gfx950 kernel's loads already stream through
    L2 with the XCD-grouped tile order.
"""
from __future__ import annotations

import functools
import logging

import torch

import gfx950_configs as cfgs
import hip_lib
from tuner import get_architecture

logger = logging.getLogger(__name__)


@functools.lru_cache(maxsize=1024)
def _gemm_tile(M: int, N: int, K: int, hint: tuple[int, int, int] | None, group_m: int | None):
    try:
        bm, bn, bk, waves, gm = cfgs.choose_gemm_tile(M, N, K, hint)
    except ValueError:
        # no built tile divides the shape: the kernel masks partial tiles (K % 8, N % 4 suffice)
        bm, bn, bk, waves, gm = cfgs.choose_gemm_tile_any(M, N, K)
    return hip_lib.GemmTile(bm, bn, bk, waves, int(group_m) if group_m else gm)


class _HipMatmulKernel:
    """``kernel[grid](a, b, c, M, N, K, **meta)`` launcher (mma.py:8-21 layout)."""

    __name__ = "_matmul_contiguous_kernel"
    _META = {"BLOCK_M", "BLOCK_N", "BLOCK_K", "GROUP_M", "USE_CACHE_EVICTION_HINTS", "num_warps", "num_stages",
             "debug"}

    def __repr__(self) -> str:
        return "<gfx950 HIP kernel _matmul_contiguous_kernel>"

    def __getitem__(self, grid):
        def launch(*args, **kwargs):
            return self._launch(grid, args, kwargs)

        return launch

    def _launch(self, grid, args, kwargs):
        if len(args) != 6:
            raise TypeError(f"_matmul_contiguous_kernel takes (a, b, c, M, N, K), got {len(args)} arguments")
        unknown = set(kwargs) - self._META
        if unknown:
            raise TypeError(f"_matmul_contiguous_kernel got unexpected keyword arguments {sorted(unknown)}")
        a, b, c = args[0:3]
        M, N, K = (int(x) for x in args[3:6])
        if callable(grid):
            grid(kwargs)
        for name, t, shape in (("a", a, (M, K)), ("b", b, (K, N)), ("c", c, (M, N))):
            if not isinstance(t, torch.Tensor) or tuple(t.shape) != shape:
                raise ValueError(f"{name} must have shape {shape}")
            if t.dtype != torch.float16:
                raise ValueError(f"{name} must be float16 (got {t.dtype})")
            if not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous row-major (mma.py indexes it as such)")
        hint = None
        if all(kwargs.get(key) is not None for key in ("BLOCK_M", "BLOCK_N", "BLOCK_K")):
            hint = (int(kwargs["BLOCK_M"]), int(kwargs["BLOCK_N"]), int(kwargs["BLOCK_K"]))
            if kwargs.get("num_warps") is not None:
                hint = (*hint, int(kwargs["num_warps"]))
        tile = _gemm_tile(M, N, K, hint, kwargs.get("GROUP_M"))
        hip_lib.gemm_f16(a, b, c, tile)


_matmul_contiguous_kernel = _HipMatmulKernel()


def _supports_contiguous_cache_eviction_hints(device=None) -> bool:
    if not torch.cuda.is_available():
        return False
    major, _ = torch.cuda.get_device_capability(device)
    return major >= 8


def _select_2d_contiguous_config(m: int, n: int, k: int) -> tuple[int, int, int, int, int, int]:
    get_architecture()
    bm, bn, bk, waves, group_m = cfgs.choose_gemm_tile(int(m), int(n), int(k))
    return bm, bn, bk, group_m, waves, 2


def matmul(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """C = A @ B through the gfx950 kernel (convenience entry). Unlike the reference selector it
    accepts shapes no tile divides (K % 8 == 0 and N % 4 == 0; partial tiles are masked). The
    kernel reads B rows in 16-byte chunks, so B's row pitch must be a multiple of 8 elements: when
    N % 8 == 4, B is first copied into rows of N + 4 elements (its last 4 columns are never
    stored to C)."""
    a = a.contiguous()
    b = b.contiguous()
    M, K = a.shape
    _, N = b.shape
    c = torch.empty((M, N), device=a.device, dtype=torch.float16) if out is None else out
    bm, bn, bk, waves, group_m = cfgs.choose_gemm_tile_any(M, N, K)
    if N % 8:
        pitch = N + (-N) % 8
        b_rows = torch.zeros((K, pitch), device=b.device, dtype=b.dtype)
        b_rows[:, :N].copy_(b)
        hip_lib.gemm_f16(a, b_rows[:, :N], c, hip_lib.GemmTile(bm, bn, bk, waves, group_m))
        return c
    _matmul_contiguous_kernel[(-(-M // bm) * -(-N // bn),)](
        a, b, c, M, N, K, BLOCK_M=bm, BLOCK_N=bn, BLOCK_K=bk, GROUP_M=group_m,
        USE_CACHE_EVICTION_HINTS=_supports_contiguous_cache_eviction_hints(a.device),
        num_warps=waves, num_stages=2,
    )
    return c


__all__ = [
    "_select_2d_contiguous_config",
    "_supports_contiguous_cache_eviction_hints",
    "_matmul_contiguous_kernel",
]
