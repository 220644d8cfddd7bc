"""Resource limits, out-of-resources errors and the resource report for the gfx950 kernels.

Mirrors the reference's `exceptions.py` surface used by its callers and tuners:
  * ``get_sm_resource_limits()`` (exceptions.py:760-775): same keys, filled from the HIP device
    properties of an MI355X (gfx950). The "per SM" keys describe one CU: 160 KiB LDS and
    4 SIMDs x 512 VGPR+AGPR x 64 lanes of 32-bit registers.
  * ``OutOfResources`` / ``OutOfResourcesWithDetail`` (exceptions.py:695-757): same constructor,
    fields (required, limit, name, kernel_name, launch_context, extra_detail,
    original_exception), ``from_out_of_resources``, hint text and ``__str__`` layout. The base class
    is defined here (the reference subclasses Triton's; this build has no Triton).
  * ``_resource_usage_summary`` (exceptions.py:633-685): same report layout
    (``<name> tuner resources: shared=a/b ..., register_file=..., registers=...`` plus optional
    tune_args / input_shapes), fed from this library's own code-object metadata. The reference's
    TTGIR/PTX transfer analysis (exceptions.py:44-631) inspects NVIDIA compiler output and is not
    rebuilt; the report instead appends the gfx950 VGPR/AGPR/scratch figures when known.
  * ``_format_tune_args`` / ``_format_input_shapes`` (exceptions.py:17-42): identical formatting.
"""
from __future__ import annotations

from collections.abc import Mapping
from dataclasses import asdict, is_dataclass
from typing import Any, Callable

# gfx950 (MI355X) per-CU limits used when no GPU is visible (CPU tuning/validation) and checked
# against the live device when one is.
GFX950_LIMITS = {
    "lds_bytes_per_cu": 160 * 1024,
    "vgprs_per_simd_lane": 512,  # unified VGPR + AGPR file per lane at one wave per SIMD
    "simds_per_cu": 4,
    "wavefront_size": 64,
    "max_threads_per_block": 1024,
    "cu_count": 256,
    "clock_khz": 2_400_000,
    "gcn_arch": 950,
}


def _format_tune_args(tune_args: Any | None) -> str | None:
    if tune_args is None:
        return None
    if is_dataclass(tune_args):
        values = asdict(tune_args)
    elif isinstance(tune_args, Mapping):
        values = dict(tune_args)
    else:
        values = {key: getattr(tune_args, key) for key in dir(tune_args) if key.isupper() and not key.startswith("_")}
    formatted = ", ".join(f"{key}={value}" for key, value in values.items() if value is not None)
    return formatted or None


def _format_input_shapes(input_shapes: Any | None) -> str | None:
    if input_shapes is None:
        return None
    values = dict(input_shapes) if isinstance(input_shapes, Mapping) else {"input_shapes": input_shapes}
    formatted = ", ".join(f"{key}={value}" for key, value in values.items() if value is not None)
    return formatted or None


def _resource_usage_summary(
    name: str,
    launch_context: Mapping[str, Any] | None,
    tune_args: Any | None = None,
    input_shapes: Any | None = None,
) -> str:
    launch_context = launch_context or {}
    shared_used = int(
        launch_context.get(
            "compiled_shared_memory_bytes_per_block",
            launch_context.get("attempted_shared_memory_bytes_per_block", 0),
        )
    )
    shared_total = int(launch_context.get("available_shared_memory_bytes_per_sm", 0))
    register_file_used = int(launch_context.get("attempted_register_file_size_bytes_per_block", 0))
    register_file_total = int(launch_context.get("available_register_file_size_bytes_per_sm", 0))
    registers_used = int(launch_context.get("attempted_registers_per_block", 0))
    registers_total = int(launch_context.get("available_registers_per_sm", 0))
    summary = (
        f"{name} tuner resources: \n"
        f"shared={shared_used}/{shared_total} bytes per block/SM, \n"
        f"register_file={register_file_used}/{register_file_total} bytes per block/SM, \n"
        f"registers={registers_used}/{registers_total} per block/SM "
    )
    if "compiled_vgprs" in launch_context:
        summary += (
            f", \ngfx950=vgpr:{launch_context.get('compiled_vgprs')} agpr:{launch_context.get('compiled_agprs')} "
            f"scratch:{launch_context.get('compiled_scratch_bytes_per_lane')}B/lane "
            f"occupancy:{launch_context.get('compiled_waves_per_simd')} waves/SIMD"
        )
    formatted_tune_args = _format_tune_args(tune_args)
    if formatted_tune_args:
        summary += f", \ntune_args={formatted_tune_args}"
    formatted_input_shapes = _format_input_shapes(input_shapes)
    if formatted_input_shapes:
        summary += f", \ninput_shapes={formatted_input_shapes}"
    return summary


class OutOfResources(Exception):
    """A launch configuration needs more of a per-CU resource than the hardware has."""

    def __init__(self, required: int, limit: int, name: str) -> None:
        self.required = required
        self.limit = limit
        self.name = name
        super().__init__(required, limit, name)

    def __str__(self) -> str:
        return f"out of resource: {self.name}; required {self.required}, hardware limit {self.limit}."

    def __reduce__(self):
        return (type(self), (self.required, self.limit, self.name))


class OutOfResourcesWithDetail(OutOfResources):
    """Resource error with kernel and block-launch context (the reference's contract)."""

    def __init__(
        self,
        required: int,
        limit: int,
        name: str,
        *,
        kernel_name: str | None = None,
        launch_context: Mapping[str, Any] | None = None,
        extra_detail: str | None = None,
        original_exception: BaseException | None = None,
    ) -> None:
        super().__init__(required, limit, name)
        self.kernel_name = kernel_name
        self.launch_context = dict(launch_context or {})
        self.extra_detail = extra_detail
        self.original_exception = original_exception

    @classmethod
    def from_out_of_resources(
        cls,
        exc: OutOfResources,
        *,
        kernel_name: str | None = None,
        launch_context: Mapping[str, Any] | None = None,
        extra_detail: str | None = None,
    ) -> "OutOfResourcesWithDetail":
        return cls(
            exc.required,
            exc.limit,
            exc.name,
            kernel_name=kernel_name,
            launch_context=launch_context,
            extra_detail=extra_detail,
            original_exception=exc,
        )

    def _resource_hint(self) -> str:
        resource = str(self.name).lower()
        if "register" in resource:
            return "The block likely needs more register file capacity per CU than the hardware can provide."
        if "shared" in resource:
            return "The block likely needs more LDS (shared memory) per CU than the hardware can provide."
        return "The block likely exceeds a per-CU hardware resource limit for this launch configuration."

    def _format_context(self) -> str | None:
        if not self.launch_context:
            return None
        return "\n".join(f"{key}={value}" for key, value in self.launch_context.items())

    def __str__(self) -> str:
        parts = [super().__str__(), self._resource_hint()]
        if self.kernel_name:
            parts.append(f"Kernel: {self.kernel_name}.")
        context = self._format_context()
        if context:
            parts.append(f"Launch context: {context}.")
        if self.extra_detail:
            parts.append(self.extra_detail.rstrip(".") + ".")
        return " ".join(parts)


# ---- device limits ----------------------------------------------------------------------------

_limits_provider: Callable[[], dict[str, Any]] | None = None


def set_device_limits_provider(provider: Callable[[], dict[str, Any]] | None) -> None:
    """Install a function returning get_sm_resource_limits()-style dicts (tests use fake limits)."""
    global _limits_provider
    _limits_provider = provider


def _limits_from_raw(lds: int, regs_per_simd_lane: int, simds: int, wave: int, max_threads: int, cus: int) -> dict:
    registers = regs_per_simd_lane * wave * simds  # 32-bit registers per CU
    return {
        "available_shared_memory_bytes_per_sm": int(lds),
        "available_registers_per_sm": int(registers),
        "available_register_file_size_bytes_per_sm": int(registers * 4),
        "warp_size": int(wave),
        "max_threads_per_block": int(max_threads),
        "max_warps_per_block": max(1, int(max_threads) // max(1, int(wave))),
        "multiprocessor_count": int(cus),
        # gfx950 extras used by the tuner's per-SIMD check
        "vgprs_per_simd_lane": int(regs_per_simd_lane),
        "simds_per_cu": int(simds),
    }


def gfx950_static_limits() -> dict[str, Any]:
    g = GFX950_LIMITS
    return _limits_from_raw(g["lds_bytes_per_cu"], g["vgprs_per_simd_lane"], g["simds_per_cu"], g["wavefront_size"],
                            g["max_threads_per_block"], g["cu_count"])


def get_sm_resource_limits() -> dict[str, Any]:
    """Per-CU limits of the current device (exceptions.py:760-775 keys).

    With a visible GPU the values come from hipGetDeviceProperties through libfa_gfx950.so and the
    device must be gfx950; without one the gfx950 table above is returned (host-side tuning and
    validation)."""
    if _limits_provider is not None:
        return dict(_limits_provider())
    import torch

    if not torch.cuda.is_available():
        return gfx950_static_limits()
    import hip_lib

    dev = hip_lib.device_limits(torch.cuda.current_device())
    if dev["gcn_arch"] != GFX950_LIMITS["gcn_arch"]:
        raise RuntimeError(f"libfa_gfx950 needs a gfx950 (MI355X) device, found gfx{dev['gcn_arch']}")
    return _limits_from_raw(
        dev["lds_bytes_per_cu"],
        GFX950_LIMITS["vgprs_per_simd_lane"],
        GFX950_LIMITS["simds_per_cu"],
        dev["wavefront_size"],
        dev["max_threads_per_block"],
        dev["cu_count"],
    )


__all__ = [
    "OutOfResources",
    "OutOfResourcesWithDetail",
    "_format_input_shapes",
    "_format_tune_args",
    "_resource_usage_summary",
    "get_sm_resource_limits",
    "gfx950_static_limits",
    "set_device_limits_provider",
]
