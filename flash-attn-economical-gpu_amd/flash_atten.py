"""FlashAttention forward on MI355X (gfx950): kernel objects and the unified entrance.

Same surface as the reference's `flash_atten.py` (flash_atten.py:364-389):
  * ``_flash_attn_fwd_kernel_basic``, ``_flash_attn_fwd_kernel_optimize_shared_mem`` and
    ``_flash_attn_fwd_kernel_block_d_nomask_contiguous`` are launchable objects used as
    ``kernel[grid](*args, **kwargs)`` with the reference's positional layouts
    (basic/optimized: 29 arguments, flash_atten.py:15-50; sliced: 9 arguments,
    flash_atten.py:262-275). Each launch is one call into libfa_gfx950.so (hand-written HIP for
    gfx950), on the current HIP stream.
  * ``flash_attention_kernel_mapping`` maps the three reference kernel names to them.
  * ``flash_attention(launch_spec)`` launches a spec built by the tuners and returns ``o`` or
    ``(o, lse)``; an unknown kernel name raises NameError (flash_atten.py:370-383).

Variant meaning on gfx950: basic = single-buffered K/V LDS tiles; optimized = the software-
pipelined kernel (K/V rings filled by LDS-DMA, exp work of one tile under the MFMAs of the next;
the double-buffered kernel where a tile asks for it); sliced = split-KV partials with an LSE merge
pass (the reference's "sliced" split the head dimension instead; all three compute the same
attention).
"""
from __future__ import annotations

import functools
import logging

import torch

import gfx950_configs as cfgs
import hip_lib
from tuner import FlashAttentionLaunchSpec

logger = logging.getLogger(__name__)

_TILE_KWARGS = {"BLOCK_M", "BLOCK_N", "BLOCK_N_PAD", "BLOCK_DMODEL", "BLOCK_DMODEL_OUTER", "num_warps",
                "num_stages", "debug"}


def _resolve_grid(grid, kwargs):
    return grid(kwargs) if callable(grid) else tuple(grid)


def _tile_for(variant: int, dtype: torch.dtype, D: int, causal: bool, B: int, H: int, M: int, N: int,
              kwargs: dict) -> cfgs.FaTileChoice:
    return _tile_for_cached(variant, dtype, D, causal, B, H, M, N, kwargs.get("BLOCK_M"), kwargs.get("BLOCK_N"),
                            kwargs.get("num_warps"), kwargs.get("num_stages"))


@functools.lru_cache(maxsize=4096)
def _tile_for_cached(variant, dtype, D, causal, B, H, M, N, block_m, block_n, num_warps, num_stages):
    cands = cfgs.fa_candidates(variant, dtype, D)
    if not cands:
        raise hip_lib.FaUnsupportedError(
            f"attention head dim D={D} with dtype {dtype} is not built for gfx950 (D in 64/128/256, fp16/bf16)"
        )
    hints = {"BLOCK_M": block_m, "BLOCK_N": block_n, "NUM_WARPS": num_warps, "NUM_STAGES": num_stages}
    matched, _ = cfgs.filter_by_hints(cands, hints)
    return cfgs.choose_fa_tile(variant, dtype, D, causal, B, H, M, N, matched)


class _HipAttentionKernel:
    """``kernel[grid](*args, **kwargs)`` launcher for one reference kernel name."""

    def __init__(self, name: str, variant: int, layout: str) -> None:
        self.__name__ = name
        self.name = name
        self.variant = variant
        self.layout = layout  # "strided" (29 args) or "contiguous" (9 args)

    def __repr__(self) -> str:
        return f"<gfx950 HIP kernel {self.name}>"

    def __getitem__(self, grid):
        def launch(*args, **kwargs):
            return self._launch(grid, args, kwargs)

        return launch

    def _launch(self, grid, args, kwargs):
        if self.layout == "strided":
            return self._launch_strided(grid, args, kwargs)
        return self._launch_contiguous(grid, args, kwargs)

    def _launch_strided(self, grid, args, kwargs):
        if len(args) != 29:
            raise TypeError(f"{self.name} takes 29 positional arguments (flash_atten.py:15-43), got {len(args)}")
        unknown = set(kwargs) - _TILE_KWARGS - {"causal", "HAS_LSE"}
        if unknown:
            raise TypeError(f"{self.name} got unexpected keyword arguments {sorted(unknown)}")
        q, k, v, o, lse = args[0:5]
        strides = [int(s) for s in args[5:24]]
        H, M, N, D = (int(x) for x in args[24:28])
        sm_scale = float(args[28])
        causal = bool(kwargs.get("causal", False))
        has_lse = bool(kwargs.get("HAS_LSE", False)) and isinstance(lse, torch.Tensor)
        self._check_shapes(q, k, v, o, H, M, N, D)
        _resolve_grid(grid, kwargs)
        q_v = q.as_strided(q.shape, strides[0:4])
        k_v = k.as_strided(k.shape, strides[4:8])
        v_v = v.as_strided(v.shape, strides[8:12])
        o_v = o.as_strided(o.shape, strides[12:16])
        lse_v = lse.as_strided(lse.shape, strides[16:19]) if has_lse else None
        tile = _tile_for(self.variant, q.dtype, D, causal, q.shape[0], H, M, N, kwargs)
        hip_lib.fa_fwd(q_v, k_v, v_v, o_v, lse_v, sm_scale=sm_scale, causal=causal, variant=self.variant,
                       tile=tile.to_c())

    def _launch_contiguous(self, grid, args, kwargs):
        if len(args) != 9:
            raise TypeError(f"{self.name} takes 9 positional arguments (flash_atten.py:262-270), got {len(args)}")
        unknown = set(kwargs) - _TILE_KWARGS - {"causal", "SPLITS", "lse", "workspace"}
        if unknown:
            raise TypeError(f"{self.name} got unexpected keyword arguments {sorted(unknown)}")
        q, k, v, o = args[0:4]
        H, M, N, D = (int(x) for x in args[4:8])
        sm_scale = float(args[8])
        self._check_shapes(q, k, v, o, H, M, N, D)
        for name, t in (("q", q), ("k", k), ("v", v), ("o", o)):
            if not t.is_contiguous():
                raise ValueError(f"{self.name} requires contiguous [B, H, S, D] tensors ({name} is not)")
        _resolve_grid(grid, kwargs)
        causal = bool(kwargs.get("causal", False))
        lse = kwargs.get("lse")
        B = q.shape[0]
        tile = _tile_for(self.variant, q.dtype, D, causal, B, H, M, N, kwargs)
        splits = kwargs.get("SPLITS")
        if splits is None:
            splits = cfgs.choose_splits(B, H, M, N, tile.block_m, tile.block_n, H_kv=k.shape[1], causal=causal,
                                        resident_per_cu=cfgs.split_residency(q.dtype, D, tile.block_m, tile.block_n,
                                                                             tile.waves, tile.stages))
        splits = int(splits)
        workspace = kwargs.get("workspace")
        need = hip_lib.workspace_bytes(B, H, M, D, splits)
        if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
            workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
        choice = cfgs.FaTileChoice(tile.block_m, tile.block_n, tile.waves, tile.stages, max(1, splits))
        hip_lib.fa_fwd(q, k, v, o, lse, sm_scale=sm_scale, causal=causal, variant=self.variant,
                       tile=choice.to_c(), workspace=workspace)

    @staticmethod
    def _check_shapes(q, k, v, o, H, M, N, D):
        for name, t in (("q", q), ("k", k), ("v", v), ("o", o)):
            if not isinstance(t, torch.Tensor) or t.dim() != 4:
                raise ValueError(f"{name} must be a 4-D tensor [batch, heads, seq, head_dim]")
        if tuple(q.shape[1:]) != (H, M, D) or tuple(o.shape) != tuple(q.shape):
            raise ValueError(f"q/o shape {tuple(q.shape)} does not match H={H} M={M} D={D}")
        if k.shape[2] != N or v.shape[2] != N or k.shape[3] != D or v.shape[3] != D:
            raise ValueError(f"k/v shapes {tuple(k.shape)}/{tuple(v.shape)} do not match N={N} D={D}")


_flash_attn_fwd_kernel_basic = _HipAttentionKernel(
    "_flash_attn_fwd_kernel_basic", hip_lib.FA_VARIANT_BASIC, "strided")
_flash_attn_fwd_kernel_optimize_shared_mem = _HipAttentionKernel(
    "_flash_attn_fwd_kernel_optimize_shared_mem", hip_lib.FA_VARIANT_OPT, "strided")
_flash_attn_fwd_kernel_block_d_nomask_contiguous = _HipAttentionKernel(
    "_flash_attn_fwd_kernel_block_d_nomask_contiguous", hip_lib.FA_VARIANT_SLICED, "contiguous")

flash_attention_kernel_mapping = {
    "_flash_attn_fwd_kernel_basic": _flash_attn_fwd_kernel_basic,
    "_flash_attn_fwd_kernel_optimize_shared_mem": _flash_attn_fwd_kernel_optimize_shared_mem,
    "_flash_attn_fwd_kernel_block_d_nomask_contiguous": _flash_attn_fwd_kernel_block_d_nomask_contiguous,
}


def flash_attention(
    launch_spec: FlashAttentionLaunchSpec,
) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
    """FlashAttention-2 style forward, hand-written HIP for gfx950 (unified entrance)."""
    if launch_spec.function_name in flash_attention_kernel_mapping:
        flash_attention_kernel_mapping[launch_spec.function_name][launch_spec.grid](
            *launch_spec.kernel_args, **launch_spec.kernel_kwargs
        )
    else:
        raise NameError(f"No such kernel named {launch_spec.function_name}.")
    o = launch_spec.kernel_args[3]
    lse = launch_spec.kernel_args[4] if isinstance(launch_spec.kernel_args[4], torch.Tensor) else None
    return (o, lse) if lse is not None else o


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = False,
              sm_scale: float | None = None, return_lse: bool = False, variant: str = "optimized"):
    """Convenience entry: tune, launch and return o (or (o, lse)); k/v may have fewer heads (GQA)."""
    import tuner

    cls = {
        "basic": tuner.FlashAttentionTuner,
        "optimized": tuner.FlashAttentionOptimizeSharedMemTuner,
        "sliced": tuner.FlashAttentionBlockDNomaskTuner,
    }[variant]
    spec = cls(tuple(q.shape), tuple(k.shape), tuple(v.shape), q.element_size(), causal=causal,
               return_lse=return_lse).build_flash_attention_launch_spec(q, k, v, sm_scale=sm_scale)
    out = flash_attention(spec)
    if variant == "sliced" and return_lse:
        return out, spec.kernel_kwargs["lse"]
    return out


def sdpa(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *, is_causal: bool = False,
         scale: float | None = None, variant: str = "sliced") -> torch.Tensor:
    """scaled_dot_product_attention-shaped entry for model code (no mask, no dropout).

    q [B, H, M, D] and k/v [B, H_kv, N, D] are read through their strides (any batch/head/row
    strides with a unit head-dim stride, e.g. the transposed projection views a decoder layer
    passes), so no contiguous copies are made. H_kv may divide H (GQA). The result is a [B, H, M, D]
    view of memory laid out [B, M, H, D], which is what a decoder's following
    `.transpose(1, 2).contiguous()` wants (that copy becomes a no-op)."""
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        raise ValueError("sdpa expects 4-D [batch, heads, seq, head_dim] tensors")
    B, H, M, D = query.shape
    variant_code = {"basic": hip_lib.FA_VARIANT_BASIC, "optimized": hip_lib.FA_VARIANT_OPT,
                    "sliced": hip_lib.FA_VARIANT_SLICED}[variant]
    sm_scale = D ** -0.5 if scale is None else float(scale)
    out = torch.empty((B, M, H, D), device=query.device, dtype=query.dtype).transpose(1, 2)
    N = key.shape[2]
    tile = _tile_for(variant_code, query.dtype, D, bool(is_causal), B, H, M, N, {})
    splits = 1
    workspace = None
    if variant_code == hip_lib.FA_VARIANT_SLICED:
        splits = cfgs.choose_splits(B, H, M, N, tile.block_m, tile.block_n, H_kv=key.shape[1],
                                    causal=bool(is_causal),
                                    resident_per_cu=cfgs.split_residency(query.dtype, D, tile.block_m, tile.block_n,
                                                                         tile.waves, tile.stages))
        need = hip_lib.workspace_bytes(B, H, M, D, splits)
        if need:
            workspace = torch.empty(need, dtype=torch.uint8, device=query.device)
    choice = cfgs.FaTileChoice(tile.block_m, tile.block_n, tile.waves, tile.stages, splits)
    hip_lib.fa_fwd(query, key, value, out, None, sm_scale=sm_scale, causal=bool(is_causal), variant=variant_code,
                   tile=choice.to_c(), workspace=workspace)
    return out


__all__ = [
    "flash_attention_kernel_mapping",
    "flash_attention",
]
