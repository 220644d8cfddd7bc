"""Launch specs and launch-configuration tuners for the gfx950 attention kernels.

Same public surface as the reference's `tuner.py` (tuner.py:19-108, 117-748): ``LaunchSpec``,
``Tuner``, ``FlashAttentionLaunchSpec`` (+``update_data``), ``FlashAttenTuneArguments`` (identical
validation errors), ``FlashAttentionTuner`` / ``FlashAttentionOptimizeSharedMemTuner`` /
``FlashAttentionBlockDNomaskTuner`` with the same constructor, ``build_launch_spec``,
``build_flash_attention_launch_spec``, ``build_compiling_context``, ``evaluate_candidate`` and the
same positional kernel-argument layouts, so callers written against the reference run unchanged.

What differs, by design (all gfx950-first):
  * Candidates are the tiles built into libfa_gfx950.so (gfx950_configs.FA_TILE_SPACE); resources
    come from the compiler's resource table for this library instead of Triton JIT compiles, and
    ranking uses the timed MI355X tuning table instead of "largest footprint".
  * Caller tune args are validated exactly as the reference does, then treated as hints (see
    gfx950_configs); relaxed hints are recorded in ``launch_context["tune_args_relaxed"]``.
  * Grouped-query attention: k/v may have H_kv heads with H % H_kv == 0 (the reference requires
    equal heads, tuner.py:134-135); batch sizes must still match.
  * The sliced tuner honours ``causal`` and ``return_lse`` (the reference silently drops them,
    tuner.py:640-658) and is a split-KV kernel with an LSE merge; its 9-argument layout is kept and
    the extra inputs travel as kernel keyword arguments.
  * The config cache is keyed per tuner class and on every tune argument (the reference's key omits
    BLOCK_DMODEL_OUTER and the kernel name, tuner.py:159-176).
"""
from __future__ import annotations

import math
from abc import ABC, abstractmethod
from dataclasses import dataclass

import torch

import gfx950_configs as cfgs
import hip_lib
from exceptions import OutOfResourcesWithDetail, get_sm_resource_limits


def get_architecture():
    """(major, minor) compute capability; gfx950 reports (9, 5)."""
    if torch.cuda.is_available():
        major, minor = torch.cuda.get_device_capability(torch.cuda.current_device())
        return major, minor
    return 9, 5


@dataclass(frozen=True)
class LaunchSpec:
    grid: tuple[int, ...]
    kernel_args: tuple[object, ...]
    kernel_kwargs: dict[str, object]
    launch_context: dict[str, object]


class Tuner(ABC):
    @abstractmethod
    def build_launch_spec(self, *data: torch.Tensor, **kwargs: object) -> LaunchSpec:
        """Build a fully materialized launch spec from runtime tensors."""

    @abstractmethod
    def build_compiling_context(self, **kwargs: object) -> dict[str, object]:
        """Build resource context for a candidate launch."""

    @abstractmethod
    def evaluate_candidate(self, *data: torch.Tensor, **kwargs: object) -> tuple[bool, LaunchSpec]:
        """Evaluate a candidate launch and return feasibility plus its launch spec."""


def _next_power_of_two(x: int) -> int:
    if x <= 0:
        raise ValueError("x must be positive")
    return 1 << (x - 1).bit_length()


def _get_max_shared_mem_bytes() -> int:
    return int(get_sm_resource_limits()["available_shared_memory_bytes_per_sm"])


@dataclass(frozen=True)
class FlashAttentionLaunchSpec(LaunchSpec):
    function_name: str
    tune_args: "FlashAttenTuneArguments"
    input_shapes: dict[str, tuple[int, ...] | None]

    def update_data(self, data):
        """Swap in new q, k, v (same shapes/strides); o, lse and workspace are reused."""
        q, k, v = data
        object.__setattr__(self, "kernel_args", (q, k, v, *self.kernel_args[3:]))


@dataclass(frozen=True)
class FlashAttenTuneArguments:
    BLOCK_N: int | None = None
    BLOCK_M: int | None = None
    BLOCK_N_PAD: int | None = None
    BLOCK_DMODEL: int | None = None
    BLOCK_DMODEL_OUTER: int | None = None
    NUM_WARPS: int | None = None
    NUM_STAGES: int | None = None

    def __post_init__(self) -> None:
        if self.BLOCK_N is not None and self.BLOCK_N <= 0:
            raise ValueError("BLOCK_N must be positive when provided")
        for name in ("BLOCK_M", "BLOCK_N_PAD", "BLOCK_DMODEL", "BLOCK_DMODEL_OUTER"):
            value = getattr(self, name)
            if value is None:
                continue
            if value <= 0:
                raise ValueError(f"{name} must be positive when provided")
            if _next_power_of_two(value) != value:
                raise ValueError(f"{name} must be a power of 2 when provided")
        if self.NUM_WARPS is not None and self.NUM_WARPS <= 0:
            raise ValueError("NUM_WARPS must be positive when provided")
        if self.NUM_STAGES is not None and self.NUM_STAGES <= 0:
            raise ValueError("NUM_STAGES must be positive when provided")


def _resource_context(limits: dict, threads: int, res: dict | None) -> dict[str, object]:
    context: dict[str, object] = dict(limits)
    context["threads_per_block"] = int(threads)
    if res is None:
        context["resource_introspection_error"] = "kernel missing from kernel_resources.json"
        return context
    regs = res["vgprs"] + res["agprs"]
    context["compiled_shared_memory_bytes_per_block"] = res["lds_bytes"]
    context["attempted_shared_memory_bytes_per_block"] = res["lds_bytes"]
    context["attempted_registers_per_thread"] = regs
    context["attempted_registers_per_block"] = regs * int(threads)
    context["attempted_register_file_size_bytes_per_block"] = regs * int(threads) * 4
    context["compiled_vgprs"] = res["vgprs"]
    context["compiled_agprs"] = res["agprs"]
    context["compiled_scratch_bytes_per_lane"] = res["scratch_bytes_per_lane"]
    context["compiled_waves_per_simd"] = res["waves_per_simd"]
    return context


def _fits(context: dict, limits: dict) -> bool:
    """LDS within the CU and every SIMD's share of waves within its 512-register lane file."""
    if "compiled_shared_memory_bytes_per_block" not in context:
        return False
    if int(context["compiled_shared_memory_bytes_per_block"]) > int(limits["available_shared_memory_bytes_per_sm"]):
        return False
    regs = int(context.get("attempted_registers_per_thread", 0))
    waves = int(context["threads_per_block"]) // int(limits["warp_size"])
    simds = int(limits.get("simds_per_cu", 4))
    per_simd_lane = int(limits.get("vgprs_per_simd_lane", 512))
    waves_per_simd = max(1, math.ceil(waves / simds))
    granule = 8
    regs_alloc = math.ceil(regs / granule) * granule
    if waves_per_simd * regs_alloc > per_simd_lane:
        return False
    return int(context.get("attempted_register_file_size_bytes_per_block", 0)) <= int(
        limits["available_register_file_size_bytes_per_sm"]
    )


class FlashAttentionTuner(Tuner):
    KERNEL_NAME = "_flash_attn_fwd_kernel_basic"
    _config_cache: dict[tuple[object, ...], tuple[dict[str, int | bool], dict[str, object]]] = {}

    def __init__(
        self,
        q_shape: tuple[int, int, int, int],
        k_shape: tuple[int, int, int, int],
        v_shape: tuple[int, int, int, int],
        dtype_size: int,
        *,
        causal: bool,
        return_lse: bool,
        tune_args: FlashAttenTuneArguments | None = None,
    ) -> None:
        if len(q_shape) != 4 or len(k_shape) != 4 or len(v_shape) != 4:
            raise ValueError("q_shape, k_shape, and v_shape must all be 4D")
        heads_ok = (
            q_shape[0] == k_shape[0] == v_shape[0]
            and k_shape[1] == v_shape[1]
            and k_shape[1] > 0
            and q_shape[1] % k_shape[1] == 0
        )
        if not heads_ok:
            raise ValueError("Batch and head dimensions must match across q_shape, k_shape, and v_shape")
        if q_shape[3] != k_shape[3] or q_shape[3] != v_shape[3]:
            raise ValueError("Last dimension must match across q_shape, k_shape, and v_shape")
        if k_shape[2] != v_shape[2]:
            raise ValueError("k_shape and v_shape sequence lengths must match")
        self.q_shape = tuple(int(v) for v in q_shape)
        self.k_shape = tuple(int(v) for v in k_shape)
        self.v_shape = tuple(int(v) for v in v_shape)
        self.dtype_size = dtype_size
        self.causal = causal
        self.return_lse = return_lse
        self.tune_args = tune_args or FlashAttenTuneArguments()
        self.B, self.H, self.M, self.D = self.q_shape
        _, self.H_kv, self.N, _ = self.k_shape
        if (
            self.tune_args.BLOCK_DMODEL is not None
            and self.tune_args.BLOCK_DMODEL < self.D
            and not self._allow_block_dmodel_smaller_than_d()
        ):
            raise ValueError("BLOCK_DMODEL must be >= D when provided")
        if self.tune_args.BLOCK_N_PAD is not None and self.tune_args.BLOCK_N is not None:
            if self.tune_args.BLOCK_N > self.tune_args.BLOCK_N_PAD:
                raise ValueError("BLOCK_N cannot exceed BLOCK_N_PAD")
        self.sm_limits = get_sm_resource_limits()
        max_warps = max(1, int(self.sm_limits.get("max_warps_per_block", 1)))
        if self.tune_args.NUM_WARPS is not None and self.tune_args.NUM_WARPS > max_warps:
            raise ValueError(f"NUM_WARPS must be <= {max_warps} for the current device")

    # -- identity -------------------------------------------------------------------------------

    @property
    def variant(self) -> int:
        return cfgs.VARIANT_BY_KERNEL[self.KERNEL_NAME]

    def _cache_key(self, q: torch.Tensor) -> tuple[object, ...]:
        ta = self.tune_args
        return (
            type(self).__name__,
            self.KERNEL_NAME,
            str(q.device),
            str(q.dtype),
            self.B, self.H, self.H_kv, self.M, self.N, self.D,
            self.causal, self.return_lse,
            ta.BLOCK_N, ta.BLOCK_M, ta.BLOCK_N_PAD, ta.BLOCK_DMODEL, ta.BLOCK_DMODEL_OUTER,
            ta.NUM_WARPS, ta.NUM_STAGES,
        )

    def _allow_block_dmodel_smaller_than_d(self) -> bool:
        return False

    # -- resources ------------------------------------------------------------------------------

    def estimate_flash_fwd_shared_bytes(self, *, block_m: int, block_n_pad: int, block_dmodel: int,
                                        element_size: int, stages: int | None = None,
                                        num_warps: int | None = None) -> int:
        """LDS of one gfx950 workgroup. stages 1/2: per buffer a K tile [block_n][D+8] and a V tile
        [block_n][D+32] (the pads are bank skews). stages 3: a ring of 3 (8 waves) or 2 (fewer)
        unpadded K and V tiles. block_m does not enter: Q stays in registers."""
        stages = cfgs.stages_for(self.variant) if stages is None else stages
        del block_m
        if stages == 3:
            ring = 3 if (num_warps or 0) >= 8 else 2
            return ring * element_size * 2 * block_n_pad * block_dmodel
        return stages * element_size * (block_n_pad * (block_dmodel + 8) + block_n_pad * (block_dmodel + 32))

    def _dtype_from_size(self, q: torch.Tensor | None = None) -> torch.dtype:
        if q is not None:
            return q.dtype
        return torch.float16

    def _candidate_configs(self, dtype: torch.dtype = torch.float16) -> list[dict[str, int | bool]]:
        """Built gfx950 tiles for this variant/dtype/D that satisfy the tune-arg hints."""
        cands = cfgs.fa_candidates(self.variant, dtype, self.D)
        if not cands:
            return []
        hints = {
            "BLOCK_M": self.tune_args.BLOCK_M,
            "BLOCK_N": self.tune_args.BLOCK_N,
            "NUM_WARPS": self.tune_args.NUM_WARPS,
            "NUM_STAGES": self.tune_args.NUM_STAGES,
        }
        matched, relaxed = cfgs.filter_by_hints(cands, hints)
        best = cfgs.choose_fa_tile(self.variant, dtype, self.D, self.causal, self.B, self.H, self.M, self.N, matched)
        ordered = [best] + [c for c in matched if c != best]
        out = []
        for c in ordered:
            out.append(
                {
                    "BLOCK_M": c.block_m,
                    "BLOCK_N": c.block_n,
                    "BLOCK_N_PAD": c.block_n,
                    "BLOCK_DMODEL": self.D,
                    "BLOCK_DMODEL_OUTER": self.D,
                    "num_warps": c.waves,
                    "num_stages": c.stages,
                    "relaxed": ",".join(relaxed),
                }
            )
        return out

    def _choice(self, config: dict) -> cfgs.FaTileChoice:
        return cfgs.FaTileChoice(int(config["BLOCK_M"]), int(config["BLOCK_N"]), int(config["num_warps"]),
                                 int(config["num_stages"]), int(config.get("splits", 1)))

    def build_compiling_context(
        self,
        *,
        grid: tuple[int, ...],
        kernel_args: tuple[object, ...],
        kernel_kwargs: dict[str, object],
        attempted_shared_memory_bytes_per_block: int,
        dtype: torch.dtype = torch.float16,
        config: dict | None = None,
    ) -> dict[str, object]:
        del grid, kernel_args
        threads = int(kernel_kwargs.get("num_warps", 1)) * int(self.sm_limits["warp_size"])
        res = None
        if config is not None:
            res = cfgs.fa_resources(self.variant, dtype, self.D, self._choice(config))
        context = _resource_context(self.sm_limits, threads, res)
        context.setdefault("attempted_shared_memory_bytes_per_block", attempted_shared_memory_bytes_per_block)
        return context

    # -- launch layout ----------------------------------------------------------------------------

    def _build_candidate_launch(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        *,
        sm_scale: float,
        o: torch.Tensor,
        lse: torch.Tensor | None,
        config: dict[str, int | bool],
        launch_context: dict[str, object] | None = None,
    ) -> FlashAttentionLaunchSpec:
        grid = (math.ceil(self.M / int(config["BLOCK_M"])), self.B * self.H)
        kernel_args = (
            q, k, v, o,
            lse if lse is not None else 0,
            q.stride(0), q.stride(1), q.stride(2), q.stride(3),
            k.stride(0), k.stride(1), k.stride(2), k.stride(3),
            v.stride(0), v.stride(1), v.stride(2), v.stride(3),
            o.stride(0), o.stride(1), o.stride(2), o.stride(3),
            (lse.stride(0) if lse is not None else 0),
            (lse.stride(1) if lse is not None else 0),
            (lse.stride(2) if lse is not None else 0),
            self.H, self.M, self.N, self.D,
            sm_scale,
        )
        kernel_kwargs = {
            "causal": self.causal,
            "HAS_LSE": self.return_lse,
            "BLOCK_M": int(config["BLOCK_M"]),
            "BLOCK_N": int(config["BLOCK_N"]),
            "BLOCK_N_PAD": int(config["BLOCK_N_PAD"]),
            "BLOCK_DMODEL": int(config["BLOCK_DMODEL"]),
            "num_warps": int(config["num_warps"]),
            "num_stages": int(config["num_stages"]),
        }
        if launch_context is None:
            launch_context = self.build_compiling_context(
                grid=grid,
                kernel_args=kernel_args,
                kernel_kwargs=kernel_kwargs,
                attempted_shared_memory_bytes_per_block=self.estimate_flash_fwd_shared_bytes(
                    block_m=int(config["BLOCK_M"]),
                    block_n_pad=int(config["BLOCK_N_PAD"]),
                    block_dmodel=self.D,
                    element_size=q.element_size(),
                    stages=int(config["num_stages"]),
                    num_warps=int(config["num_warps"]),
                ),
                dtype=q.dtype,
                config=config,
            )
            if config.get("relaxed"):
                launch_context["tune_args_relaxed"] = config["relaxed"]
        return FlashAttentionLaunchSpec(
            grid=grid,
            kernel_args=kernel_args,
            kernel_kwargs=kernel_kwargs,
            launch_context=launch_context,
            function_name=self.KERNEL_NAME,
            tune_args=FlashAttenTuneArguments(
                BLOCK_N=int(config["BLOCK_N"]),
                BLOCK_M=int(config["BLOCK_M"]),
                BLOCK_N_PAD=int(config["BLOCK_N_PAD"]),
                BLOCK_DMODEL=int(config["BLOCK_DMODEL"]),
                NUM_WARPS=int(config["num_warps"]),
                NUM_STAGES=int(config["num_stages"]),
            ),
            input_shapes={
                "q": tuple(int(dim) for dim in q.shape),
                "k": tuple(int(dim) for dim in k.shape),
                "v": tuple(int(dim) for dim in v.shape),
                "o": tuple(int(dim) for dim in o.shape),
                "lse": (tuple(int(dim) for dim in lse.shape) if lse is not None else None),
            },
        )

    def evaluate_candidate(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        *,
        sm_scale: float,
        o: torch.Tensor,
        lse: torch.Tensor | None,
        config: dict[str, int | bool],
    ) -> tuple[bool, FlashAttentionLaunchSpec]:
        launch_spec = self._build_candidate_launch(q, k, v, sm_scale=sm_scale, o=o, lse=lse, config=config)
        return _fits(launch_spec.launch_context, self.sm_limits), launch_spec

    def _validate_runtime_tensors(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
        if tuple(q.shape) != self.q_shape or tuple(k.shape) != self.k_shape or tuple(v.shape) != self.v_shape:
            raise ValueError("Runtime tensor shapes do not match the tuner shapes")

    def build_launch_spec(
        self,
        *data: torch.Tensor,
        sm_scale: float,
        o: torch.Tensor,
        lse: torch.Tensor | None,
    ) -> FlashAttentionLaunchSpec:
        if len(data) != 3:
            raise ValueError("FlashAttentionTuner.build_launch_spec expects (q, k, v)")
        q, k, v = data
        self._validate_runtime_tensors(q, k, v)
        if q.dtype not in (torch.float16, torch.bfloat16):
            raise ValueError(f"unsupported dtype {q.dtype}: the gfx950 kernels take float16 or bfloat16")
        if not (q.dtype == k.dtype == v.dtype):
            raise ValueError("q, k and v must share one dtype")

        key = self._cache_key(q)
        cached = self._config_cache.get(key)
        if cached is not None:
            selected_config, selected_context = cached
            return self._build_candidate_launch(
                q, k, v, sm_scale=sm_scale, o=o, lse=lse,
                config=dict(selected_config), launch_context=dict(selected_context),
            )

        candidates = self._candidate_configs(q.dtype)
        if not candidates:
            raise ValueError(
                f"{self.KERNEL_NAME}: head dim D={self.D} with dtype {q.dtype} is not built for gfx950 "
                "(D in {64, 128, 256}, float16/bfloat16)"
            )
        fallback_spec: FlashAttentionLaunchSpec | None = None
        for config in candidates:
            feasible, launch_spec = self.evaluate_candidate(q, k, v, sm_scale=sm_scale, o=o, lse=lse, config=config)
            fallback_spec = launch_spec
            if feasible:
                self._config_cache[key] = (dict(config), dict(launch_spec.launch_context))
                return launch_spec

        context = dict(fallback_spec.launch_context) if fallback_spec is not None else dict(self.sm_limits)
        register_bytes = int(context.get("attempted_register_file_size_bytes_per_block", 0))
        if register_bytes > int(self.sm_limits["available_register_file_size_bytes_per_sm"]) or (
            "compiled_shared_memory_bytes_per_block" in context
            and int(context["compiled_shared_memory_bytes_per_block"])
            <= int(self.sm_limits["available_shared_memory_bytes_per_sm"])
        ):
            raise OutOfResourcesWithDetail(
                int(context.get("attempted_registers_per_block", 0)),
                int(self.sm_limits["available_registers_per_sm"]),
                "registers",
                kernel_name=self.KERNEL_NAME,
                launch_context=context,
                extra_detail="No candidate flash-attention block fit the per-SIMD register-file limit",
            )
        raise OutOfResourcesWithDetail(
            int(context.get("attempted_shared_memory_bytes_per_block", 0)),
            int(self.sm_limits["available_shared_memory_bytes_per_sm"]),
            "shared memory",
            kernel_name=self.KERNEL_NAME,
            launch_context=context,
            extra_detail="No candidate flash-attention block fit the per-CU LDS (shared memory) limit",
        )

    def build_flash_attention_launch_spec(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        *,
        sm_scale: float | None = None,
    ) -> FlashAttentionLaunchSpec:
        q = q.contiguous()
        k = k.contiguous()
        v = v.contiguous()
        if sm_scale is None:
            sm_scale = q.shape[-1] ** -0.5
        o = torch.empty_like(q)
        lse = (
            torch.empty((q.shape[0], q.shape[1], q.shape[2]), device=q.device, dtype=torch.float32)
            if self.return_lse
            else None
        )
        return self.build_launch_spec(q, k, v, sm_scale=sm_scale, o=o, lse=lse)


class FlashAttentionOptimizeSharedMemTuner(FlashAttentionTuner):
    KERNEL_NAME = "_flash_attn_fwd_kernel_optimize_shared_mem"


class FlashAttentionBlockDNomaskTuner(FlashAttentionTuner):
    """The "sliced" variant: split-KV partial passes plus an LSE merge (one pass when the grid
    already fills the GPU). Keeps the reference's 9-argument layout (tuner.py:640-650)."""

    KERNEL_NAME = "_flash_attn_fwd_kernel_block_d_nomask_contiguous"

    def _allow_block_dmodel_smaller_than_d(self) -> bool:
        return True

    def _candidate_configs(self, dtype: torch.dtype = torch.float16) -> list[dict[str, int | bool]]:
        out = super()._candidate_configs(dtype)
        for config in out:
            config["BLOCK_DMODEL"] = int(self.tune_args.BLOCK_DMODEL or self.D)
            config["BLOCK_DMODEL_OUTER"] = int(self.tune_args.BLOCK_DMODEL_OUTER or self.D)
            resident = cfgs.split_residency(dtype, self.D, int(config["BLOCK_M"]), int(config["BLOCK_N"]),
                                            int(config["num_warps"]), int(config["num_stages"]))
            config["splits"] = cfgs.choose_splits(self.B, self.H, self.M, self.N, int(config["BLOCK_M"]),
                                                  int(config["BLOCK_N"]), H_kv=self.H_kv, causal=self.causal,
                                                  resident_per_cu=resident)
        return out

    def _build_candidate_launch(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        *,
        sm_scale: float,
        o: torch.Tensor,
        lse: torch.Tensor | None,
        config: dict[str, int | bool],
        launch_context: dict[str, object] | None = None,
    ) -> FlashAttentionLaunchSpec:
        grid = (math.ceil(self.M / int(config["BLOCK_M"])), self.B * self.H)
        kernel_args = (q, k, v, o, self.H, self.M, self.N, self.D, sm_scale)
        splits = int(config.get("splits", 1))
        workspace = None
        nbytes = hip_lib.workspace_bytes(self.B, self.H, self.M, self.D, splits)
        if nbytes:
            workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
        kernel_kwargs = {
            "BLOCK_M": int(config["BLOCK_M"]),
            "BLOCK_N": int(config["BLOCK_N"]),
            "BLOCK_DMODEL": int(config["BLOCK_DMODEL"]),
            "BLOCK_DMODEL_OUTER": int(config["BLOCK_DMODEL_OUTER"]),
            "num_warps": int(config["num_warps"]),
            "num_stages": int(config["num_stages"]),
            "causal": self.causal,
            "SPLITS": splits,
            "lse": lse,
            "workspace": workspace,
        }
        if launch_context is None:
            launch_context = self.build_compiling_context(
                grid=grid,
                kernel_args=kernel_args,
                kernel_kwargs=kernel_kwargs,
                attempted_shared_memory_bytes_per_block=self.estimate_flash_fwd_shared_bytes(
                    block_m=int(config["BLOCK_M"]),
                    block_n_pad=int(config["BLOCK_N_PAD"]),
                    block_dmodel=self.D,
                    element_size=self.dtype_size,
                    stages=int(config["num_stages"]),
                    num_warps=int(config["num_warps"]),
                ),
                dtype=q.dtype,
                config=config,
            )
            launch_context["kv_splits"] = splits
            if config.get("relaxed"):
                launch_context["tune_args_relaxed"] = config["relaxed"]
        return FlashAttentionLaunchSpec(
            grid=grid,
            kernel_args=kernel_args,
            kernel_kwargs=kernel_kwargs,
            launch_context=launch_context,
            function_name=self.KERNEL_NAME,
            tune_args=FlashAttenTuneArguments(
                BLOCK_N=int(config["BLOCK_N"]),
                BLOCK_M=int(config["BLOCK_M"]),
                BLOCK_N_PAD=int(config["BLOCK_N_PAD"]),
                BLOCK_DMODEL=int(config["BLOCK_DMODEL"]),
                BLOCK_DMODEL_OUTER=int(config["BLOCK_DMODEL_OUTER"]),
                NUM_WARPS=int(config["num_warps"]),
                NUM_STAGES=int(config["num_stages"]),
            ),
            input_shapes={
                "q": tuple(int(dim) for dim in q.shape),
                "k": tuple(int(dim) for dim in k.shape),
                "v": tuple(int(dim) for dim in v.shape),
                "o": tuple(int(dim) for dim in o.shape),
                "lse": (tuple(int(dim) for dim in lse.shape) if lse is not None else None),
            },
        )


__all__ = [
    "FlashAttenTuneArguments",
    "FlashAttentionLaunchSpec",
    "FlashAttentionTuner",
    "FlashAttentionOptimizeSharedMemTuner",
    "FlashAttentionBlockDNomaskTuner",
    "LaunchSpec",
    "Tuner",
    "_get_max_shared_mem_bytes",
    "_next_power_of_two",
    "get_architecture",
]
