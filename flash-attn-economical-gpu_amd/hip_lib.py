"""ctypes binding of libfa_gfx950.so (C ABI declared in include/fa_gfx950.h).

This is the only module that talks to the native library. Tensors are passed as raw device
pointers plus sizes and element strides; launches go to the caller's current HIP stream
(torch.cuda.current_stream().cuda_stream). There is no fallback: if the library is missing or was
built for another ABI, every entry point raises RuntimeError.
"""
from __future__ import annotations

import ctypes
import functools
import json
import threading
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libfa_gfx950.so"
RESOURCES_PATH = HERE / "kernel_resources.json"
ABI_VERSION = 4

FA_OK, FA_EINVAL, FA_ENOTSUP, FA_EHIP, FA_EWORKSPACE = 0, 1, 2, 3, 4
FA_DTYPE_F16, FA_DTYPE_BF16 = 0, 1
FA_VARIANT_BASIC, FA_VARIANT_OPT, FA_VARIANT_SLICED = 0, 1, 2

_DTYPE_CODES = {torch.float16: FA_DTYPE_F16, torch.bfloat16: FA_DTYPE_BF16}


class FaTile(ctypes.Structure):
    _fields_ = [
        ("block_m", ctypes.c_int32),
        ("block_n", ctypes.c_int32),
        ("waves", ctypes.c_int32),
        ("stages", ctypes.c_int32),
        ("splits", ctypes.c_int32),
    ]


class FaFwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_int64),
        ("q_stride", ctypes.c_int64 * 4),
        ("k_stride", ctypes.c_int64 * 4),
        ("v_stride", ctypes.c_int64 * 4),
        ("o_stride", ctypes.c_int64 * 4),
        ("lse_stride", ctypes.c_int64 * 3),
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("H_kv", ctypes.c_int32),
        ("M", ctypes.c_int32),
        ("N", ctypes.c_int32),
        ("D", ctypes.c_int32),
        ("sm_scale", ctypes.c_float),
        ("dtype", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("variant", ctypes.c_int32),
        ("tile", FaTile),
    ]


class GemmTile(ctypes.Structure):
    _fields_ = [
        ("block_m", ctypes.c_int32),
        ("block_n", ctypes.c_int32),
        ("block_k", ctypes.c_int32),
        ("waves", ctypes.c_int32),
        ("group_m", ctypes.c_int32),
    ]


class FaResources(ctypes.Structure):
    _fields_ = [
        ("vgprs", ctypes.c_int32),
        ("agprs", ctypes.c_int32),
        ("sgprs", ctypes.c_int32),
        ("lds_bytes", ctypes.c_int32),
        ("scratch_bytes", ctypes.c_int32),
        ("threads", ctypes.c_int32),
        ("max_threads", ctypes.c_int32),
        ("occupancy", ctypes.c_int32),
    ]


class FaDeviceLimits(ctypes.Structure):
    _fields_ = [
        ("lds_bytes_per_cu", ctypes.c_int32),
        ("registers_per_simd", ctypes.c_int32),
        ("register_file_bytes_per_simd", ctypes.c_int32),
        ("wavefront_size", ctypes.c_int32),
        ("max_threads_per_block", ctypes.c_int32),
        ("cu_count", ctypes.c_int32),
        ("clock_khz", ctypes.c_int32),
        ("gcn_arch", ctypes.c_int32),
    ]


# Every symbol include/fa_gfx950.h declares, with its ctypes signature.
SIGNATURES = {
    "fa_abi_version": (ctypes.c_int, []),
    "fa_last_error": (ctypes.c_char_p, []),
    "fa_fwd": (ctypes.c_int, [ctypes.POINTER(FaFwdArgs), ctypes.c_void_p]),
    "fa_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(FaFwdArgs), ctypes.c_void_p]),
    "fa_fwd_workspace_bytes": (
        ctypes.c_int64,
        [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32],
    ),
    "fa_fwd_pack_group": (ctypes.c_int32, [ctypes.c_int32] * 6),
    "fa_fwd_supported": (ctypes.c_int, [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(FaTile)]),
    "gemm_f16": (
        ctypes.c_int,
        [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.POINTER(GemmTile), ctypes.c_void_p,
        ],
    ),
    "gemm_f16_supported": (ctypes.c_int, [ctypes.POINTER(GemmTile)]),
    "fa_kernel_resources": (
        ctypes.c_int,
        [
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            ctypes.POINTER(FaTile), ctypes.POINTER(GemmTile), ctypes.POINTER(FaResources),
        ],
    ),
    "fa_kernel_symbol": (
        ctypes.c_int,
        [
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            ctypes.POINTER(FaTile), ctypes.POINTER(GemmTile), ctypes.c_char_p, ctypes.c_int32,
        ],
    ),
    "fa_device_limits": (ctypes.c_int, [ctypes.c_int32, ctypes.POINTER(FaDeviceLimits)]),
}


class FaLibraryError(RuntimeError):
    """The native library is missing, stale, or a HIP call inside it failed."""


class FaUnsupportedError(ValueError):
    """The requested head dim / dtype / tile is not built into the library."""


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load libfa_gfx950.so once (after torch, so it binds to torch's HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise FaLibraryError(
                f"{LIB_PATH} is missing: build it with `python {HERE / 'build_lib.py'}` "
                "(or __graft_entry__.build()); there is no non-HIP fallback"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.fa_abi_version()
        if version != ABI_VERSION:
            raise FaLibraryError(f"{LIB_PATH} has ABI version {version}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def last_error() -> str:
    msg = load().fa_last_error()
    return msg.decode() if msg else ""


def check(code: int, what: str) -> None:
    if code == FA_OK:
        return
    msg = f"{what}: {last_error()}"
    if code == FA_ENOTSUP:
        raise FaUnsupportedError(msg)
    if code in (FA_EINVAL, FA_EWORKSPACE):
        raise ValueError(msg)
    raise FaLibraryError(msg)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise FaUnsupportedError(f"dtype {dtype} is not supported (float16, bfloat16)") from None


# torch's raw current-stream query (what its own generated launchers call) skips building a Stream
# object: a few microseconds per launch, which single-sequence decode steps pay on the host.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_ptr(device: torch.device) -> int:
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


_I64x4 = ctypes.c_int64 * 4


def _strides4(t: torch.Tensor):
    return _I64x4(*t.stride())


def make_tile(block_m: int, block_n: int, waves: int, stages: int, splits: int = 1) -> FaTile:
    return FaTile(int(block_m), int(block_n), int(waves), int(stages), int(splits))


@functools.lru_cache(maxsize=4096)
def workspace_bytes(B: int, H: int, M: int, D: int, splits: int) -> int:
    return int(load().fa_fwd_workspace_bytes(B, H, M, D, splits))


@functools.lru_cache(maxsize=4096)
def pack_group(H: int, H_kv: int, M: int, causal: bool, block_m: int, splits: int) -> int:
    """Query heads fa_fwd packs into one tile's rows (1 = none); see fa_fwd_pack_group."""
    return int(load().fa_fwd_pack_group(H, H_kv, M, int(bool(causal)), block_m, splits))


def fa_fwd_supported(variant: int, dtype: torch.dtype, D: int, tile: FaTile) -> bool:
    return load().fa_fwd_supported(variant, dtype_code(dtype), D, ctypes.byref(tile)) == FA_OK


def _fwd_args(q, k, v, o, lse, *, sm_scale, causal, variant, tile, workspace) -> FaFwdArgs:
    for name, t in (("q", q), ("k", k), ("v", v), ("o", o)):
        if t.dim() != 4:
            raise ValueError(f"{name} must be 4-D [batch, heads, seq, head_dim], got {tuple(t.shape)}")
        if t.device.type != "cuda":
            raise ValueError(f"{name} must be a GPU tensor, got device {t.device}")
    if not (q.dtype == k.dtype == v.dtype == o.dtype):
        raise ValueError(f"q/k/v/o dtypes differ: {q.dtype} {k.dtype} {v.dtype} {o.dtype}")
    B, H, M, D = q.shape
    Bk, Hkv, N, Dk = k.shape
    if tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} shapes differ")
    if Bk != B or Dk != D or tuple(o.shape) != tuple(q.shape):
        raise ValueError(f"incompatible shapes q={tuple(q.shape)} k={tuple(k.shape)} o={tuple(o.shape)}")
    args = FaFwdArgs()
    args.q, args.k, args.v, args.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
    if lse is not None:
        if lse.dtype != torch.float32 or tuple(lse.shape) != (B, H, M) or lse.device != q.device:
            raise ValueError(f"lse must be float32 [{B}, {H}, {M}] on {q.device}")
        args.lse = lse.data_ptr()
        args.lse_stride = (ctypes.c_int64 * 3)(*[int(s) for s in lse.stride()])
    if workspace is not None:
        args.workspace = workspace.data_ptr()
        args.workspace_bytes = workspace.numel() * workspace.element_size()
    args.q_stride, args.k_stride = _strides4(q), _strides4(k)
    args.v_stride, args.o_stride = _strides4(v), _strides4(o)
    args.B, args.H, args.H_kv, args.M, args.N, args.D = B, H, Hkv, M, N, D
    args.sm_scale = float(sm_scale)
    args.dtype = dtype_code(q.dtype)
    args.causal = 1 if causal else 0
    args.variant = int(variant)
    args.tile = tile
    return args


def fa_fwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor,
    lse: torch.Tensor | None,
    *,
    sm_scale: float,
    causal: bool,
    variant: int,
    tile: FaTile,
    workspace: torch.Tensor | None = None,
) -> None:
    """Launch one attention forward: o (and lse) are written in place on the current stream."""
    lib = load()
    args = _fwd_args(q, k, v, o, lse, sm_scale=sm_scale, causal=causal, variant=variant, tile=tile,
                     workspace=workspace)
    check(lib.fa_fwd(ctypes.byref(args), _stream_ptr(q.device)), "fa_fwd")


# Size of the static device array fa_fwd_noalloc keeps its split-KV partials in
# (FA_NOALLOC_SCRATCH_BYTES in include/fa_gfx950.h).
NOALLOC_SCRATCH_BYTES = 64 << 20


def fa_fwd_noalloc(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor,
    lse: torch.Tensor | None,
    *,
    sm_scale: float,
    causal: bool,
    variant: int,
    tile: FaTile,
) -> None:
    """fa_fwd with the split-KV partials in the library's static per-GPU scratch array (no device
    allocation by the library or here). Calls on one GPU share that array: overlapping calls race.
    Raises ValueError when the partials need more than NOALLOC_SCRATCH_BYTES."""
    lib = load()
    args = _fwd_args(q, k, v, o, lse, sm_scale=sm_scale, causal=causal, variant=variant, tile=tile, workspace=None)
    check(lib.fa_fwd_noalloc(ctypes.byref(args), _stream_ptr(q.device)), "fa_fwd_noalloc")


def gemm_f16(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, tile: GemmTile) -> None:
    """C = A @ B (fp16, fp32 accumulation) written into c on the current stream."""
    lib = load()
    for name, t in (("a", a), ("b", b), ("c", c)):
        if t.dim() != 2 or t.device.type != "cuda" or t.dtype != torch.float16:
            raise ValueError(f"{name} must be a 2-D float16 GPU tensor")
        if t.stride(1) != 1:
            raise ValueError(f"{name} must be row-major (unit column stride)")
    M, K = a.shape
    K2, N = b.shape
    if K2 != K or tuple(c.shape) != (M, N):
        raise ValueError(f"incompatible GEMM shapes a={tuple(a.shape)} b={tuple(b.shape)} c={tuple(c.shape)}")
    code = lib.gemm_f16(
        a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K,
        a.stride(0), b.stride(0), c.stride(0), ctypes.byref(tile), _stream_ptr(a.device),
    )
    check(code, "gemm_f16")


def gemm_supported(tile: GemmTile) -> bool:
    return load().gemm_f16_supported(ctypes.byref(tile)) == FA_OK


def kernel_resources_live(op: int, *, variant: int = 0, dtype: torch.dtype = torch.float16, D: int = 0,
                          tile: FaTile | None = None, gtile: GemmTile | None = None) -> dict[str, int]:
    """Resources of one built kernel (needs a GPU): registers, scratch and occupancy from the
    compiler's table linked into the library, LDS and the workgroup limit from the loaded kernel."""
    out = FaResources()
    code = load().fa_kernel_resources(
        op, variant, dtype_code(dtype), D,
        ctypes.byref(tile) if tile is not None else None,
        ctypes.byref(gtile) if gtile is not None else None,
        ctypes.byref(out),
    )
    check(code, "fa_kernel_resources")
    return {name: int(getattr(out, name)) for name, _ in FaResources._fields_}


def device_limits(device: int = 0) -> dict[str, int]:
    out = FaDeviceLimits()
    check(load().fa_device_limits(device, ctypes.byref(out)), "fa_device_limits")
    return {name: int(getattr(out, name)) for name, _ in FaDeviceLimits._fields_}


_resource_table: dict[str, dict[str, object]] | None = None


def compiled_resources() -> dict[str, dict[str, object]]:
    """Per-kernel resource table written by build_lib.py from the compiler's resource remarks."""
    global _resource_table
    if _resource_table is None:
        if not RESOURCES_PATH.exists():
            raise FaLibraryError(f"{RESOURCES_PATH} is missing: rebuild with build_lib.py")
        _resource_table = json.loads(RESOURCES_PATH.read_text())
    return _resource_table


def _kernel_symbol(op: int, variant: int, dtype: torch.dtype, D: int, tile: FaTile | None,
                   gtile: GemmTile | None) -> str:
    buf = ctypes.create_string_buffer(512)
    code = load().fa_kernel_symbol(
        op, variant, dtype_code(dtype), D,
        ctypes.byref(tile) if tile is not None else None,
        ctypes.byref(gtile) if gtile is not None else None,
        buf, len(buf),
    )
    check(code, "fa_kernel_symbol")
    return buf.value.decode()


def fwd_kernel_symbol(variant: int, dtype: torch.dtype, D: int, tile: FaTile) -> str:
    """Mangled name of the attention kernel a tile resolves to (the key of kernel_resources.json),
    as the library resolves it; needs no device."""
    return _kernel_symbol(0, variant, dtype, D, tile, None)


def gemm_kernel_symbol(tile: GemmTile) -> str:
    """Mangled name of the GEMM kernel a tile runs (its default deep-ring kernel); needs no device."""
    return _kernel_symbol(1, 0, torch.float16, 0, None, tile)
