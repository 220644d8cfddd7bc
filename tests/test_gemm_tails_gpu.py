"""GEMM shapes no tile divides (tails): the gfx950 kernel masks partial tiles in M, N
and K (K % 8 == 0, N % 4 == 0). Checked against the exact oracle, with NaN in the row padding of A
(past K) and B (past N) to show those elements never reach valid outputs, and a sentinel in C's
padding to show nothing is stored outside [M, N)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import gfx950_configs as cfgs
import hip_lib
import mma
import oracle
from helpers import to_device

pytestmark = pytest.mark.gpu

# every built tile (16x16 and 32x32 MFMAs; compiler-scheduled and pipelined loops)
TILES = [(256, 256, 64, 8), (256, 256, 32, 8), (256, 128, 64, 8), (128, 256, 64, 8), (256, 256, 64, 4),
         (256, 256, 32, 4), (128, 128, 64, 4), (128, 128, 32, 4), (128, 64, 32, 4), (64, 256, 32, 4),
         (128, 128, 32, 8), (128, 64, 32, 8), (128, 64, 32, 16), (64, 64, 32, 8)]
# K from 1 to 32 slabs: up to 8 slabs the 128x128, 128x64 and 64x256 tiles launch their
# shallow-ring kernels (K=256 is the last such for BK=32, K=264 the first deep one).
SHAPES = [(100, 200, 72), (257, 260, 520), (33, 4, 8), (1000, 1004, 1000), (300, 512, 136), (260, 392, 256),
          (260, 392, 264)]


def _padded(x: np.ndarray, cols: int, fill: float) -> torch.Tensor:
    rows, n = x.shape
    buf = np.full((rows, cols), fill, dtype=np.float32)
    buf[:, :n] = x
    t = to_device(buf, torch.float16, "cuda:0")
    return t[:, :n]  # row-major view with leading dimension `cols`


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in SHAPES])
def test_gemm_tails_all_tiles(gpu, shape):
    M, N, K = shape
    print(f"[gemm_tails] M={M} N={N} K={K}", flush=True)
    a = oracle.round_to(oracle.portable_uniform(21, (M, K), -1, 1), 0)
    b = oracle.round_to(oracle.portable_uniform(22, (K, N), -1, 1), 0)
    ref = oracle.gemm(a, b)
    ad = _padded(a, K + 24, np.nan)                 # NaN past K in every A row (lda % 8 == 0)
    bd = _padded(b, -(-N // 8) * 8 + 8, np.nan)     # NaN past N in every B row (ldb % 8 == 0)
    sentinel = 1234.0
    cbuf = torch.full((M, N + 8), sentinel, dtype=torch.float16, device="cuda:0")
    cd = cbuf[:, :N]
    for tile in TILES:
        cbuf.fill_(sentinel)
        hip_lib.gemm_f16(ad, bd, cd, hip_lib.GemmTile(*tile, 4))
        torch.cuda.synchronize()
        c = cd.float().cpu().numpy()
        assert np.isfinite(c).all(), tile
        rel = float(np.linalg.norm(c - ref) / np.linalg.norm(ref))
        assert rel <= 1e-3, (tile, rel)
        assert bool((cbuf[:, N:] == sentinel).all()), tile


@pytest.mark.parametrize("shape", [(777, 1032, 264), (300, 100, 64), (65, 1028, 520)],
                         ids=["n_mod8_0", "n_mod8_4", "n_mod8_4_deep"])
def test_gemm_tails_convenience_entry(gpu, shape):
    """mma.matmul takes tail shapes (the reference selector still raises for them), N % 8 == 4
    included (B is restaged into rows of a multiple of 8 elements)."""
    M, N, K = shape
    print(f"[gemm_tails] mma.matmul {M}x{N}x{K}", flush=True)
    with pytest.raises(ValueError):
        mma._select_2d_contiguous_config(M, N, K)
    a = oracle.round_to(oracle.portable_uniform(31, (M, K), -1, 1), 0)
    b = oracle.round_to(oracle.portable_uniform(32, (K, N), -1, 1), 0)
    c = mma.matmul(to_device(a, torch.float16, "cuda:0"), to_device(b, torch.float16, "cuda:0"))
    torch.cuda.synchronize()
    assert c.is_contiguous() and tuple(c.shape) == (M, N)
    ref = oracle.gemm(a, b)
    assert float(np.linalg.norm(c.float().cpu().numpy() - ref) / np.linalg.norm(ref)) <= 1e-3
    assert cfgs.choose_gemm_tile_any(M, N, K)[:3] != ()


def test_gemm_rejects_unaligned_tails(gpu):
    a = torch.zeros(64, 12, dtype=torch.float16, device="cuda:0")
    b = torch.zeros(12, 64, dtype=torch.float16, device="cuda:0")
    c = torch.zeros(64, 64, dtype=torch.float16, device="cuda:0")
    with pytest.raises(ValueError, match="multiple of 8"):
        hip_lib.gemm_f16(a, b, c, hip_lib.GemmTile(128, 128, 32, 4, 4))
