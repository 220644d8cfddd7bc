"""The C ABI library loads without a GPU, exports every symbol include/fa_gfx950.h declares, and
rejects bad arguments before any launch (no compute calls here)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

import hip_lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "fa_gfx950.h"


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = hip_lib.load()
    names = _declared_functions()
    assert set(names) == set(hip_lib.SIGNATURES), names
    for name in names:
        assert getattr(lib, name) is not None


def test_abi_version_and_struct_layout_match_the_header(tmp_path):
    """ctypes mirrors must have the C compiler's sizes and field offsets for every ABI struct."""
    import subprocess

    assert hip_lib.load().fa_abi_version() == hip_lib.ABI_VERSION
    structs = {
        "fa_fwd_args": hip_lib.FaFwdArgs, "fa_tile": hip_lib.FaTile, "gemm_tile": hip_lib.GemmTile,
        "fa_resources": hip_lib.FaResources, "fa_device_limits_t": hip_lib.FaDeviceLimits,
    }
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'  printf("{cname} %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'  printf("{cname}.{field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    out = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                              check=True).stdout.splitlines())
    for cname, cls in structs.items():
        assert int(out[cname]) == ctypes.sizeof(cls), cname
        for field, _ in cls._fields_:
            assert int(out[f"{cname}.{field}"]) == getattr(cls, field).offset, f"{cname}.{field}"


def test_workspace_bytes_formula():
    assert hip_lib.workspace_bytes(1, 2, 100, 128, 1) == 0
    rows = 4 * 1 * 2 * 100
    o_bytes = rows * 128 * 4
    assert hip_lib.workspace_bytes(1, 2, 100, 128, 4) == ((o_bytes + 255) // 256) * 256 + rows * 4


def test_supported_tiles():
    t = hip_lib.make_tile(256, 64, 8, 2, 1)
    assert hip_lib.fa_fwd_supported(hip_lib.FA_VARIANT_OPT, torch.float16, 128, t)
    assert not hip_lib.fa_fwd_supported(hip_lib.FA_VARIANT_OPT, torch.float16, 96, t)
    assert not hip_lib.fa_fwd_supported(hip_lib.FA_VARIANT_OPT, torch.float16, 128, hip_lib.make_tile(512, 64, 8, 2))
    assert hip_lib.gemm_supported(hip_lib.GemmTile(256, 256, 64, 4, 8))
    assert not hip_lib.gemm_supported(hip_lib.GemmTile(96, 256, 64, 4, 8))


def test_kernel_symbols_key_the_resource_table():
    """fa_kernel_symbol names the kernel a tile resolves to, without a device: each built GEMM tile
    and a pipelined attention tile map to a row of the compiler's resource table; a buffer too small
    for the name is rejected, an unbuilt tile is unsupported."""
    table = hip_lib.compiled_resources()
    for t in ((256, 256, 64, 8), (256, 256, 32, 8), (256, 256, 64, 4), (128, 128, 32, 4), (64, 256, 32, 4)):
        sym = hip_lib.gemm_kernel_symbol(hip_lib.GemmTile(*t, 8))
        assert sym.startswith(f"_ZN2fa15gemm_f16_kernelILi{t[0]}ELi{t[1]}ELi{t[2]}E") and sym in table, sym
    fsym = hip_lib.fwd_kernel_symbol(hip_lib.FA_VARIANT_OPT, torch.float16, 128, hip_lib.make_tile(128, 64, 4, 3))
    assert fsym in table and "ELi64ELi3ELb0E" in fsym
    lib = hip_lib.load()
    small = ctypes.create_string_buffer(8)
    tile = hip_lib.GemmTile(256, 256, 64, 8, 8)
    assert lib.fa_kernel_symbol(1, 0, 0, 0, None, ctypes.byref(tile), small, len(small)) == hip_lib.FA_EINVAL
    assert lib.fa_kernel_symbol(1, 0, 0, 0, None, ctypes.byref(hip_lib.GemmTile(96, 256, 64, 4, 8)), small,
                                len(small)) == hip_lib.FA_ENOTSUP


def _args(**over):
    a = hip_lib.FaFwdArgs()
    a.q = a.k = a.v = a.o = 256  # never dereferenced: every case below fails validation first
    for s in ("q_stride", "k_stride", "v_stride", "o_stride"):
        setattr(a, s, (ctypes.c_int64 * 4)(64 * 64 * 2, 64 * 64, 64, 1))
    a.B, a.H, a.H_kv, a.M, a.N, a.D = 1, 2, 2, 64, 64, 64
    a.sm_scale = 0.125
    a.dtype, a.causal, a.variant = 0, 0, hip_lib.FA_VARIANT_OPT
    a.tile = hip_lib.make_tile(128, 64, 4, 2, 1)
    for k, v in over.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "over,code,needle",
    [
        ({"D": 96}, hip_lib.FA_ENOTSUP, "head dim"),
        ({"dtype": 7}, hip_lib.FA_ENOTSUP, "dtype"),
        ({"variant": 9}, hip_lib.FA_EINVAL, "variant"),
        ({"H_kv": 3, "H": 4}, hip_lib.FA_EINVAL, "multiple of kv heads"),
        ({"M": -1}, hip_lib.FA_EINVAL, "invalid sizes"),
        ({"sm_scale": float("nan")}, hip_lib.FA_EINVAL, "sm_scale"),
        ({"q_stride": (ctypes.c_int64 * 4)(1, 1, 1, 2)}, hip_lib.FA_EINVAL, "head-dim stride"),
        ({"q": 258}, hip_lib.FA_EINVAL, "16-byte aligned"),
        ({"tile": hip_lib.make_tile(128, 64, 4, 2, 4)}, hip_lib.FA_EINVAL, "sliced"),
        ({"variant": hip_lib.FA_VARIANT_SLICED, "tile": hip_lib.make_tile(128, 64, 4, 2, 4)},
         hip_lib.FA_EWORKSPACE, "workspace"),
        ({"tile": hip_lib.make_tile(96, 64, 4, 2, 1)}, hip_lib.FA_ENOTSUP, "not built"),
    ],
)
def test_fa_fwd_rejects_before_launch(over, code, needle):
    lib = hip_lib.load()
    assert lib.fa_fwd(ctypes.byref(_args(**over)), None) == code
    assert needle in hip_lib.last_error()


def test_fa_fwd_empty_problem_is_a_no_op():
    lib = hip_lib.load()
    assert lib.fa_fwd(ctypes.byref(_args(M=0)), None) == hip_lib.FA_OK
    assert lib.fa_fwd(ctypes.byref(_args(B=0)), None) == hip_lib.FA_OK


@pytest.mark.parametrize(
    "dims,code",
    [((256, 256, 100), hip_lib.FA_EINVAL), ((256, 254, 256), hip_lib.FA_EINVAL), ((256, 256, 0), hip_lib.FA_EINVAL),
     ((0, 256, 256), hip_lib.FA_OK)],
)
def test_gemm_rejects_before_launch(dims, code):
    lib = hip_lib.load()
    M, N, K = dims
    tile = hip_lib.GemmTile(256, 256, 64, 4, 8)
    assert lib.gemm_f16(256, 256, 256, M, N, K, max(K, 8), N, N, ctypes.byref(tile), None) == code


def test_python_wrappers_raise_mapped_errors():
    with pytest.raises(hip_lib.FaUnsupportedError):
        hip_lib.check(hip_lib.FA_ENOTSUP, "x")
    with pytest.raises(ValueError):
        hip_lib.check(hip_lib.FA_EINVAL, "x")
    with pytest.raises(hip_lib.FaLibraryError):
        hip_lib.check(hip_lib.FA_EHIP, "x")


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(hip_lib, "_lib", None)
    monkeypatch.setattr(hip_lib, "LIB_PATH", tmp_path / "libfa_gfx950.so")
    with pytest.raises(hip_lib.FaLibraryError, match="missing"):
        hip_lib.load()


_ASM_LOAD = """_ZN2fa6kernelEv:
{pre}
	;;#ASMSTART
{guard}	s_mov_b32 m0, s20
	buffer_load_dwordx4 v163, s[12:15], 0 offen offset:0 lds
	;;#ASMEND
	s_endpgm
"""


@pytest.mark.parametrize("pre,guard,hits", [
    ("\tv_readlane_b32 s15, v166, 7", "", 1),             # VALU writes the descriptor, load 0 wait states later
    ("\tv_readfirstlane_b32 s13, v2\n\ts_mov_b32 s1, 0\n\ts_mov_b32 s2, 0", "", 1),  # 2 wait states
    ("\tv_readlane_b32 s15, v166, 7", "\ts_nop 4\n", 0),  # the guard: 5 wait states
    ("\tv_readfirstlane_b32 s13, v2\n" + "\ts_add_u32 s0, s0, 1\n" * 5, "", 0),  # 5 instructions between
    ("\ts_mov_b32 s15, s3", "", 0),                        # a scalar write is no hazard
    ("\tv_readlane_b32 s30, v166, 7", "", 0),              # an SGPR the load does not read
])
def test_build_asm_hazard_check_loads(pre, guard, hits):
    """The build's assembly check (build_lib.asm_hazards) flags a VALU write to an SGPR that an
    inline-asm vector-memory instruction reads within 5 wait states, and nothing else."""
    import build_lib
    asm = _ASM_LOAD.format(pre=pre, guard=guard)
    assert len(build_lib.asm_hazards(asm)) == hits


@pytest.mark.parametrize("inside,hits", [("", 1), ("\ts_nop 1\n", 0)])
def test_build_asm_hazard_check_wide_stores(inside, hits):
    """An inline-asm store of 16 bytes must end in an s_nop: a VALU write to its data registers right
    after it corrupts the stored data (seen in the persistent GEMM's first version)."""
    import build_lib
    asm = ("_ZN2fa6kernelEv:\n\t;;#ASMSTART\n\tbuffer_store_dwordx4 v[24:27], v29, s[8:11], 0 offen\n"
           + inside + "\t;;#ASMEND\n\tv_add_u32_e32 v24, v23, v30\n")
    assert len(build_lib.asm_hazards(asm)) == hits
