"""GPU parity of the attention kernels, called directly through the C ABI (fa_fwd), against the
oracle (exact double-precision attention) on identical seeded inputs.

Tolerance (north star): max |O - O_oracle| <= 2e-2 for fp16, <= 3e-2 for bf16; LSE within 1e-3
(absolute, natural log units).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import hip_lib
import oracle
from helpers import ATOL, make_qkv, max_abs, to_device

pytestmark = pytest.mark.gpu

F16, BF16 = torch.float16, torch.bfloat16
BASIC, OPT, SLICED = hip_lib.FA_VARIANT_BASIC, hip_lib.FA_VARIANT_OPT, hip_lib.FA_VARIANT_SLICED

# (variant, block_m, block_n, waves, stages)
TILES = {
    "basic128": (BASIC, 128, 64, 4, 1),
    "opt128": (OPT, 128, 64, 4, 2),
    "opt256w4": (OPT, 256, 64, 4, 2),
    "opt256w8": (OPT, 256, 64, 8, 2),
    # software-pipelined kernel (stages=3): LDS-DMA ring of 2 tiles (4 waves) or 3 tiles (8 waves)
    "pipe128": (OPT, 128, 64, 4, 3),
    "pipe256": (OPT, 256, 64, 8, 3),
    "pipe128n32": (OPT, 128, 32, 4, 3),  # D = 256 pipelined (32-key tiles)
    # two-tile-ahead pipeline (stages=4): ring of 2 tiles (D <= 128) or 3 (D = 256)
    "pipe4_128": (OPT, 128, 64, 4, 4),
    "pipe4_128n32": (OPT, 128, 32, 4, 4),
    # one tile per step, two waves per SIMD (stages=5; D = 256)
    "lean128n32": (OPT, 128, 32, 4, 5),
    # the stages=5 pipeline with 16x16x32 MFMA tiles (stages=6)
    "m16_128": (OPT, 128, 64, 4, 6),
    "m16_128n32": (OPT, 128, 32, 4, 6),
    # 16x16x32 MFMAs with the stages=3 software pipeline (stages=7; D <= 128)
    "m16p_128": (OPT, 128, 64, 4, 7),
    "m16p_128n32": (OPT, 128, 32, 4, 7),
    # ping-pong (stages=8): 8 waves in two groups one phase apart, 256 rows, 16x16x32 MFMAs
    "pp_256": (OPT, 256, 64, 8, 8),
    # the ping-pong kernel in a persistent grid (stages=9): one workgroup per CU walks query blocks
    "ppp_256": (OPT, 256, 64, 8, 9),
}


def run_fa(q, k, v, *, variant, tile, causal, scale=None, with_lse=True, dtype=F16, device="cuda:0", splits=1):
    qd, kd, vd = (to_device(x, dtype, device) for x in (q, k, v))
    B, H, M, D = qd.shape
    o = torch.empty_like(qd)
    lse = torch.empty((B, H, M), dtype=torch.float32, device=device) if with_lse else None
    scale = D ** -0.5 if scale is None else scale
    var, bm, bn, waves, stages = tile
    t = hip_lib.make_tile(bm, bn, waves, stages, splits)
    ws = None
    nbytes = hip_lib.workspace_bytes(B, H, M, D, splits)
    if nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    hip_lib.fa_fwd(qd, kd, vd, o, lse, sm_scale=scale, causal=causal, variant=variant if variant is not None else var,
                   tile=t, workspace=ws)
    torch.cuda.synchronize()
    return o.float().cpu().numpy(), (lse.cpu().numpy() if lse is not None else None)


CASES = [
    # name, B, H, Hkv, M, N, D, dtype, causal, tile
    ("cfg1_d64", 1, 4, 4, 512, 512, 64, F16, False, "basic128"),
    ("cfg1_d64_opt", 1, 4, 4, 512, 512, 64, F16, False, "opt128"),
    ("d128_noncausal", 1, 2, 2, 512, 512, 128, F16, False, "opt128"),
    ("d128_causal", 1, 2, 2, 512, 512, 128, F16, True, "opt128"),
    ("d128_causal_basic", 1, 2, 2, 384, 384, 128, F16, True, "basic128"),
    ("d128_w4r2", 2, 2, 2, 512, 512, 128, F16, False, "opt256w4"),
    ("d128_w8", 2, 2, 2, 512, 512, 128, F16, True, "opt256w8"),
    ("d256_bf16", 1, 2, 2, 256, 256, 256, BF16, False, "opt128"),
    ("d256_f16_basic", 1, 2, 2, 256, 320, 256, F16, False, "basic128"),
    ("gqa_6to1_causal", 1, 12, 2, 256, 256, 128, BF16, True, "opt128"),
    ("ragged_m_n", 2, 3, 3, 200, 333, 64, F16, False, "opt128"),
    ("ragged_causal", 1, 2, 1, 190, 190, 128, F16, True, "opt256w8"),
    ("tiny", 1, 1, 1, 1, 1, 64, F16, False, "basic128"),
    ("m_ne_n_causal", 1, 2, 2, 100, 260, 64, BF16, True, "opt128"),
    ("pipe_d128", 1, 2, 2, 512, 512, 128, F16, False, "pipe128"),
    ("pipe_d128_bf16_causal", 1, 2, 2, 512, 512, 128, BF16, True, "pipe128"),
    ("pipe_d64", 2, 2, 2, 256, 448, 64, F16, False, "pipe128"),
    ("pipe_w8_d128_causal", 2, 2, 2, 512, 512, 128, F16, True, "pipe256"),
    ("pipe_w8_d64_bf16", 1, 3, 3, 256, 576, 64, BF16, False, "pipe256"),
    ("pipe_gqa_causal", 1, 12, 2, 256, 256, 128, BF16, True, "pipe128"),
    ("pipe_ragged", 2, 3, 3, 200, 333, 128, F16, False, "pipe128"),
    ("pipe_w8_ragged_causal", 1, 2, 1, 190, 190, 128, F16, True, "pipe256"),
    ("pipe_tiny", 1, 1, 1, 1, 1, 128, F16, False, "pipe256"),
    ("pipe_d256_bf16", 1, 2, 2, 256, 300, 256, BF16, False, "pipe128n32"),
    ("pipe_d256_f16_causal", 2, 2, 1, 200, 200, 256, F16, True, "pipe128n32"),
    ("pipe_d256_one_tile", 1, 1, 1, 40, 17, 256, BF16, False, "pipe128n32"),
    ("pipe4_d128", 1, 2, 2, 512, 512, 128, F16, False, "pipe4_128"),
    ("pipe4_d128_bf16_causal", 1, 2, 2, 512, 512, 128, BF16, True, "pipe4_128"),
    ("pipe4_d64", 2, 2, 2, 256, 448, 64, F16, False, "pipe4_128"),
    ("pipe4_d128_causal_b2", 2, 2, 2, 512, 512, 128, F16, True, "pipe4_128"),
    ("pipe4_d64_bf16", 1, 3, 3, 256, 576, 64, BF16, False, "pipe4_128"),
    ("pipe4_gqa_causal", 1, 12, 2, 256, 256, 128, BF16, True, "pipe4_128"),
    ("pipe4_ragged", 2, 3, 3, 200, 333, 128, F16, False, "pipe4_128"),
    ("pipe4_ragged_causal", 1, 2, 1, 190, 190, 128, F16, True, "pipe4_128"),
    ("pipe4_tiny", 1, 1, 1, 1, 1, 128, F16, False, "pipe4_128"),
    ("pipe4_d256_bf16", 1, 2, 2, 256, 300, 256, BF16, False, "pipe4_128n32"),
    ("pipe4_d256_f16_causal", 2, 2, 1, 200, 200, 256, F16, True, "pipe4_128n32"),
    ("pipe4_d256_one_tile", 1, 1, 1, 40, 17, 256, BF16, False, "pipe4_128n32"),
    ("pipe4_d256_long_causal", 1, 2, 2, 700, 700, 256, BF16, True, "pipe4_128n32"),
    ("lean_d256_bf16", 1, 2, 2, 256, 300, 256, BF16, False, "lean128n32"),
    ("lean_d256_f16_causal", 2, 2, 1, 200, 200, 256, F16, True, "lean128n32"),
    ("lean_d256_one_tile", 1, 1, 1, 40, 17, 256, BF16, False, "lean128n32"),
    ("lean_d256_long_causal_gqa", 1, 4, 2, 700, 700, 256, BF16, True, "lean128n32"),
    ("m16_d128", 1, 2, 2, 512, 512, 128, F16, False, "m16_128"),
    ("m16_d128_bf16_causal", 1, 2, 2, 512, 512, 128, BF16, True, "m16_128"),
    ("m16_d64", 2, 2, 2, 256, 448, 64, F16, False, "m16_128"),
    ("m16_d64_bf16_causal", 1, 3, 3, 256, 576, 64, BF16, True, "m16_128"),
    ("m16_gqa_causal", 1, 12, 2, 256, 256, 128, BF16, True, "m16_128"),
    ("m16_ragged", 2, 3, 3, 200, 333, 128, F16, False, "m16_128"),
    ("m16_ragged_causal", 1, 2, 1, 190, 190, 128, F16, True, "m16_128"),
    ("m16_tiny", 1, 1, 1, 1, 1, 128, F16, False, "m16_128"),
    ("m16n32_d128", 1, 2, 2, 512, 448, 128, F16, False, "m16_128n32"),
    ("m16n32_d128_bf16_causal_ragged", 2, 2, 1, 300, 300, 128, BF16, True, "m16_128n32"),
    ("m16n32_d256_bf16", 1, 2, 2, 256, 300, 256, BF16, False, "m16_128n32"),
    ("m16n32_d256_f16_causal", 2, 2, 1, 200, 200, 256, F16, True, "m16_128n32"),
    ("m16n32_d256_one_tile", 1, 1, 1, 40, 17, 256, BF16, False, "m16_128n32"),
    ("m16n32_d256_long_causal_gqa", 1, 4, 2, 700, 700, 256, BF16, True, "m16_128n32"),
    ("m16p_d128", 1, 2, 2, 512, 512, 128, F16, False, "m16p_128"),
    ("m16p_d128_bf16_causal", 1, 2, 2, 512, 512, 128, BF16, True, "m16p_128"),
    ("m16p_d64", 2, 2, 2, 256, 448, 64, F16, False, "m16p_128"),
    ("m16p_d64_bf16_causal", 1, 3, 3, 256, 576, 64, BF16, True, "m16p_128"),
    ("m16p_gqa_causal", 1, 12, 2, 256, 256, 128, BF16, True, "m16p_128"),
    ("m16p_ragged", 2, 3, 3, 200, 333, 128, F16, False, "m16p_128"),
    ("m16p_ragged_causal", 1, 2, 1, 190, 190, 128, F16, True, "m16p_128"),
    ("m16p_tiny", 1, 1, 1, 1, 1, 128, F16, False, "m16p_128"),
    ("m16pn32_d128", 1, 2, 2, 512, 448, 128, F16, False, "m16p_128n32"),
    ("m16pn32_d128_bf16_causal_ragged", 2, 2, 1, 300, 300, 128, BF16, True, "m16p_128n32"),
    ("m16pn32_d64_causal", 1, 2, 2, 333, 333, 64, F16, True, "m16p_128n32"),
    ("pp_d128", 1, 2, 2, 512, 512, 128, F16, False, "pp_256"),
    ("pp_d128_bf16_causal", 1, 2, 2, 512, 512, 128, BF16, True, "pp_256"),
    ("pp_d64", 2, 2, 2, 256, 448, 64, F16, False, "pp_256"),
    ("pp_d64_bf16_causal", 1, 3, 3, 300, 576, 64, BF16, True, "pp_256"),
    ("pp_gqa_causal", 1, 12, 2, 256, 256, 128, BF16, True, "pp_256"),
    ("pp_ragged", 2, 3, 3, 200, 333, 128, F16, False, "pp_256"),
    ("pp_ragged_causal", 1, 2, 1, 290, 290, 128, F16, True, "pp_256"),
    ("pp_idle_waves", 1, 2, 2, 40, 700, 128, F16, False, "pp_256"),  # waves 2-7 hold no rows
    ("pp_tiny", 1, 1, 1, 1, 1, 128, F16, False, "pp_256"),
    ("ppp_d128", 1, 2, 2, 512, 512, 128, F16, False, "ppp_256"),
    ("ppp_d128_bf16_causal", 1, 2, 2, 512, 512, 128, BF16, True, "ppp_256"),
    ("ppp_d64", 2, 2, 2, 256, 448, 64, F16, False, "ppp_256"),
    ("ppp_d64_bf16_causal", 1, 3, 3, 300, 576, 64, BF16, True, "ppp_256"),
    ("ppp_gqa_causal", 1, 12, 2, 256, 256, 128, BF16, True, "ppp_256"),
    ("ppp_ragged", 2, 3, 3, 200, 333, 128, F16, False, "ppp_256"),
    ("ppp_ragged_causal", 1, 2, 1, 290, 290, 128, F16, True, "ppp_256"),
    ("ppp_idle_waves", 1, 2, 2, 40, 700, 128, F16, False, "ppp_256"),
    ("ppp_tiny", 1, 1, 1, 1, 1, 128, F16, False, "ppp_256"),
]


@pytest.mark.parametrize("tile_name", ["pipe128", "pipe256", "pipe4_128", "pipe4_128n32", "lean128n32", "m16_128",
                                       "m16_128n32", "m16p_128", "pp_256", "ppp_256"])
@pytest.mark.parametrize("n", [1, 64, 65, 128, 192, 256, 320, 384, 448, 512])
def test_fa_pipelined_tile_counts(gpu, tile_name, n):
    """1..8 KV tiles: the pipelined loops' prologues, unrolled pairs, peeled tails (stages=4: 1, 2
    or 3 trailing steps) and the LDS-DMA rings (2 or 3 slots) at every length parity, with a
    partial last tile."""
    print(f"[fa_abi] pipelined tile counts {tile_name} N={n}", flush=True)
    B, H, M = 1, 2, 96
    D = 256 if TILES[tile_name][2] == 32 else 128  # 32-key tiles are the D = 256 ones
    q, k, v = make_qkv(300 + n, B, H, H, M, n, D, F16)
    o, lse = run_fa(q, k, v, variant=None, tile=TILES[tile_name], causal=False)
    o_ref, lse_ref = oracle.attention(q, k, v, causal=False)
    assert max_abs(o, o_ref) <= ATOL[F16]
    assert max_abs(lse, lse_ref) <= 1e-3


@pytest.mark.parametrize("tile_name", ["opt256w8", "pipe128", "pipe256", "pp_256", "ppp_256"])
def test_fa_strided_bshd_layout(gpu, tile_name):
    """q/k/v/o as [B, S, H, D] memory viewed as [B, H, S, D] (row stride H*D): buffer ranges and
    DMA offsets of the pipelined kernel follow the strides."""
    B, H, M, N, D = 2, 4, 160, 300, 128
    print(f"[fa_abi] strided BSHD {tile_name}", flush=True)
    q, k, v = make_qkv(911, B, H, H, M, N, D, F16)
    dev = "cuda:0"
    qd, kd, vd = (to_device(np.ascontiguousarray(x.transpose(0, 2, 1, 3)), F16, dev).transpose(1, 2) for x in (q, k, v))
    od = torch.empty((B, M, H, D), dtype=F16, device=dev).transpose(1, 2)
    lse = torch.empty((B, H, M), dtype=torch.float32, device=dev)
    var, bm, bn, waves, stages = TILES[tile_name]
    hip_lib.fa_fwd(qd, kd, vd, od, lse, sm_scale=D ** -0.5, causal=True, variant=var,
                   tile=hip_lib.make_tile(bm, bn, waves, stages, 1))
    torch.cuda.synchronize()
    o_ref, lse_ref = oracle.attention(q, k, v, causal=True)
    assert max_abs(od.float().cpu().numpy(), o_ref) <= ATOL[F16]
    assert max_abs(lse.cpu().numpy(), lse_ref) <= 1e-3


@pytest.mark.parametrize("splits", [2, 5])
@pytest.mark.parametrize("causal", [False, True])
def test_fa_sliced_pipelined_split_kv(gpu, splits, causal):
    B, H, Hkv, M, N, D, dtype = 1, 4, 2, 256, 1000, 128, BF16
    print(f"[fa_abi] sliced pipelined splits={splits} causal={causal}", flush=True)
    q, k, v = make_qkv(78, B, H, Hkv, M, N, D, dtype)
    for tile_name in ("pipe128", "pipe256", "pipe4_128", "m16_128", "m16p_128", "pp_256", "ppp_256"):
        o, lse = run_fa(q, k, v, variant=SLICED, tile=TILES[tile_name], causal=causal, dtype=dtype, splits=splits)
        o_ref, lse_ref = oracle.attention(q, k, v, causal=causal)
        assert max_abs(o, o_ref) <= ATOL[dtype], tile_name
        assert max_abs(lse, lse_ref) <= 1e-3, tile_name


@pytest.mark.parametrize("stages", [8, 9])
@pytest.mark.parametrize("causal", [False, True])
def test_fa_ping_pong_offset_moves(gpu, stages, causal):
    """Large and climbing logits through the ping-pong kernels, whose lazy rescale moves a row's
    exponent offset only when a score rises more than 8 (log2 units) above it. Keys whose norm grows
    along the sequence make every row's maximum climb tile after tile (many moves), and a large scale
    puts the logits at tens of units; a causal launch adds rows whose first tiles are masked. The
    logits are formed in fp32 from the binary16 inputs, so the LSE error stays at the fp32 level
    relative to its magnitude (a variant that folded the scale into Q, rounded to binary16, was
    8x less accurate at |LSE| ~ 70 and is not used)."""
    B, H, Hkv, M, N, D, dtype = 1, 4, 2, 512, 1536, 128, F16
    print(f"[fa_abi] ping-pong offset moves stages={stages} causal={causal}", flush=True)
    q, k, v = make_qkv(91, B, H, Hkv, M, N, D, dtype)
    ramp = np.linspace(0.25, 2.5, N, dtype=np.float32)[None, None, :, None]
    k = oracle.round_to(k * ramp, oracle.DTYPE_F16)
    for scale in (None, 0.6):
        o, lse = run_fa(q, k, v, variant=OPT, tile=(OPT, 256, 64, 8, stages), causal=causal, dtype=dtype, scale=scale)
        o_ref, lse_ref = oracle.attention(q, k, v, causal=causal, scale=scale)
        assert np.isfinite(o).all() and np.isfinite(lse).all(), scale
        assert max_abs(o, o_ref) <= ATOL[dtype], scale
        assert max_abs(lse, lse_ref) <= 1e-3 * max(1.0, float(np.abs(lse_ref).max()) / 8), scale


# Persistent grid (stages=9) with several work items per workgroup (more query blocks than CUs):
# name, B, H, Hkv, M, N, D, dtype, causal, splits
PERSISTENT_CASES = [
    ("items_x2", 2, 32, 32, 2048, 2048, 128, F16, False, 1),
    ("items_causal_snake", 2, 32, 32, 4096, 4096, 128, F16, True, 1),  # 4..64 tiles per item
    ("items_one_tile", 4, 32, 32, 2048, 64, 128, F16, False, 1),       # T = 1: the next K_0 from the prologue
    ("items_two_tiles", 4, 32, 32, 2048, 100, 128, BF16, False, 1),
    ("items_three_tiles_d64", 2, 32, 32, 2048, 130, 64, F16, False, 1),
    ("items_gqa_causal_ragged", 3, 24, 8, 1000, 777, 128, BF16, True, 1),
    ("items_split_causal", 1, 32, 8, 2048, 2048, 128, BF16, True, 4),  # empty split items (causal)
    ("items_not_multiple_of_8", 1, 37, 37, 1800, 300, 64, F16, False, 1),
]


@pytest.mark.parametrize("case", PERSISTENT_CASES, ids=[c[0] for c in PERSISTENT_CASES])
def test_fa_persistent_items(gpu, case):
    """stages=9 walks several query blocks per workgroup, fetching the next block's Q/K/V during the
    current block's last steps; its per-block arithmetic is stages=8's, so outputs and LSE must be
    bit-identical to the per-workgroup ping-pong kernel, and sampled rows match the oracle."""
    name, B, H, Hkv, M, N, D, dtype, causal, splits = case
    print(f"[fa_abi] persistent {name} B={B} H={H} Hkv={Hkv} M={M} N={N} D={D} {dtype} causal={causal} "
          f"splits={splits}", flush=True)
    q, k, v = make_qkv(4242 + M + N, B, H, Hkv, M, N, D, dtype)
    variant = SLICED if splits > 1 else OPT
    outs = {}
    for stages in (8, 9):
        outs[stages] = run_fa(q, k, v, variant=variant, tile=(variant, 256, 64, 8, stages), causal=causal,
                              dtype=dtype, splits=splits)
    o8, lse8 = outs[8]
    o9, lse9 = outs[9]
    assert np.array_equal(o9, o8), name
    assert np.array_equal(lse9, lse8), name
    rows = np.unique(np.random.default_rng(M + N).integers(0, B * H * M, 48))
    o_ref, lse_ref = oracle.attention_rows(q, k, v, rows, causal=causal)
    assert max_abs(o9.reshape(-1, D)[rows], o_ref) <= ATOL[dtype], name
    assert max_abs(lse9.reshape(-1)[rows], lse_ref) <= 1e-3, name


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_fa_parity(gpu, case):
    name, B, H, Hkv, M, N, D, dtype, causal, tile_name = case
    print(f"[fa_abi] {name} B={B} H={H} Hkv={Hkv} M={M} N={N} D={D} {dtype} causal={causal} tile={tile_name}",
          flush=True)
    q, k, v = make_qkv(1000 + len(name), B, H, Hkv, M, N, D, dtype)
    o, lse = run_fa(q, k, v, variant=None, tile=TILES[tile_name], causal=causal, dtype=dtype)
    o_ref, lse_ref = oracle.attention(q, k, v, causal=causal)
    assert np.isfinite(o).all()
    err = max_abs(o, o_ref)
    assert err <= ATOL[dtype], f"max abs error {err}"
    assert max_abs(lse, lse_ref) <= 1e-3


@pytest.mark.parametrize("splits", [2, 3, 8])
@pytest.mark.parametrize("causal", [False, True])
def test_fa_sliced_split_kv(gpu, splits, causal):
    B, H, Hkv, M, N, D, dtype = 1, 4, 2, 256, 1000, 128, F16
    print(f"[fa_abi] sliced splits={splits} causal={causal}", flush=True)
    q, k, v = make_qkv(77, B, H, Hkv, M, N, D, dtype)
    o, lse = run_fa(q, k, v, variant=SLICED, tile=TILES["opt128"], causal=causal, dtype=dtype, splits=splits)
    o_ref, lse_ref = oracle.attention(q, k, v, causal=causal)
    assert max_abs(o, o_ref) <= ATOL[dtype]
    assert max_abs(lse, lse_ref) <= 1e-3


def test_fa_matches_reference_online_algorithm(gpu):
    """Against the reference kernel's own blocked algorithm (P rounded to fp16): tighter bound."""
    B, H, M, N, D = 1, 2, 256, 256, 64
    q, k, v = make_qkv(5, B, H, H, M, N, D, F16)
    o, _ = run_fa(q, k, v, variant=None, tile=TILES["opt128"], causal=False)
    o_ref, _ = oracle.attention_online(q, k, v, block_n=64, dtype=oracle.DTYPE_F16)
    assert max_abs(o, o_ref) <= 4e-3


def test_gemm_parity(gpu):
    for (M, N, K, tile) in [(256, 256, 256, (256, 256, 64, 4, 8)), (512, 384, 320, (128, 128, 64, 4, 8)),
                            (1024, 1024, 256, (128, 256, 64, 8, 8)), (512, 512, 512, (256, 256, 32, 8, 8)),
                            (768, 512, 640, (256, 256, 64, 8, 3)), (256, 192, 96, (128, 64, 32, 4, 2)),
                            (128, 512, 64, (64, 256, 32, 4, 1)), (256, 256, 1024, (128, 128, 32, 8, 4)),
                            (384, 192, 992, (128, 64, 32, 8, 2)), (256, 128, 1056, (128, 64, 32, 16, 8))]:
        print(f"[gemm_abi] M={M} N={N} K={K} tile={tile}", flush=True)
        if M % tile[0] or N % tile[1] or K % tile[2]:
            continue
        a = oracle.round_to(oracle.portable_uniform(11, (M, K), -1, 1), 0)
        b = oracle.round_to(oracle.portable_uniform(12, (K, N), -1, 1), 0)
        ad = to_device(a, F16, "cuda:0")
        bd = to_device(b, F16, "cuda:0")
        cd = torch.empty((M, N), dtype=F16, device="cuda:0")
        hip_lib.gemm_f16(ad, bd, cd, hip_lib.GemmTile(*tile))
        torch.cuda.synchronize()
        ref = oracle.gemm(a, b)
        c = cd.float().cpu().numpy()
        rel = float(np.linalg.norm(c - ref) / np.linalg.norm(ref))
        assert rel <= 1e-3, rel


def _strided_kv(x: np.ndarray, row_stride: int, dtype, device) -> torch.Tensor:
    """[1, 1, N, D] device view whose rows sit row_stride elements apart (row_stride < D overlaps
    neighbouring rows; those rows then hold what the later row wrote, mirrored in the returned
    host copy)."""
    _, _, N, D = x.shape
    base = torch.zeros((N - 1) * row_stride + D, dtype=dtype, device=device)
    view = base.as_strided((1, 1, N, D), (N * row_stride, N * row_stride, row_stride, 1))
    for n in range(N):  # row by row, so overlapping rows end up as the last writer left them
        view[0, 0, n].copy_(torch.from_numpy(np.ascontiguousarray(x[0, 0, n])).to(dtype))
    return view


@pytest.mark.parametrize("why", ["short_row_stride", "span_over_4gib"])
@pytest.mark.parametrize("D,tile_name,dtype", [(128, "pipe128", F16), (256, "pipe128n32", BF16),
                                               (128, "pipe4_128", F16), (256, "pipe4_128n32", BF16),
                                               (256, "lean128n32", BF16), (128, "m16_128", F16),
                                               (256, "m16_128n32", BF16), (128, "m16p_128", F16),
                                               (128, "pp_256", BF16)])
@pytest.mark.parametrize("splits", [1, 2])
def test_fa_pipelined_fallback(gpu, why, D, tile_name, dtype, splits):
    """A pipelined (stages=3) tile whose addressing rules a launch breaks runs the double-buffered
    kernel instead: K/V row stride below D (overlapping rows), and a (batch, kv-head) span of
    (N + block_n) * row stride * 2 bytes beyond 2^32. Both against the oracle on the same data."""
    N, M = (40, 64) if why == "span_over_4gib" else (300, 96)
    row_stride = 48 * 1024 * 1024 if why == "span_over_4gib" else D // 2
    print(f"[fa_abi] pipelined fallback {why} D={D} {dtype} splits={splits} N={N} stride={row_stride}", flush=True)
    var, bm, bn, waves, stages = TILES[tile_name]
    assert (N + bn) * row_stride * 2 > 2 ** 32 or row_stride < D
    q, k, v = make_qkv(4242 + D, 1, 1, 1, M, N, D, dtype)
    dev = "cuda:0"
    kd, vd = _strided_kv(k, row_stride, dtype, dev), _strided_kv(v, row_stride, dtype, dev)
    # what the kernel reads: the device rows as they ended up (overlaps resolved by the last row)
    k_seen, v_seen = (t.float().cpu().numpy() for t in (kd, vd))
    qd = to_device(q, dtype, dev)
    o = torch.empty_like(qd)
    lse = torch.empty((1, 1, M), dtype=torch.float32, device=dev)
    ws = None
    nbytes = hip_lib.workspace_bytes(1, 1, M, D, splits)
    if nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    hip_lib.fa_fwd(qd, kd, vd, o, lse, sm_scale=D ** -0.5, causal=False, variant=SLICED if splits > 1 else OPT,
                   tile=hip_lib.make_tile(bm, bn, waves, stages, splits), workspace=ws)
    torch.cuda.synchronize()
    o_ref, lse_ref = oracle.attention(q, k_seen, v_seen, causal=False)
    assert max_abs(o.float().cpu().numpy(), o_ref) <= ATOL[dtype]
    assert max_abs(lse.cpu().numpy(), lse_ref) <= 1e-3
    del kd, vd
    torch.cuda.empty_cache()


def test_kernel_resources_live_match_compiled_table(gpu):
    """fa_kernel_resources for every built attention tile and GEMM tile: registers, scratch and
    occupancy from the table linked into the library, LDS and the workgroup limit from the loaded
    kernel; both must agree with kernel_resources.json (the same compiler remarks)."""
    import gfx950_configs

    table = hip_lib.compiled_resources()
    checked = 0
    for variant in (BASIC, OPT, SLICED):
        for dtype in (F16, BF16):
            for D in (64, 128, 256):
                for bm, bn, waves, stages in gfx950_configs.FA_TILE_SPACE:
                    for splits in ((1, 4) if variant == SLICED else (1,)):
                        t = hip_lib.make_tile(bm, bn, waves, stages, splits)
                        if not hip_lib.fa_fwd_supported(variant, dtype, D, t):
                            continue
                        live = hip_lib.kernel_resources_live(0, variant=variant, dtype=dtype, D=D, tile=t)
                        raw = table[hip_lib.fwd_kernel_symbol(variant, dtype, D, t)]
                        _compare_resources(live, raw, waves)
                        checked += 1
    for bm, bn, bk, waves in gfx950_configs.GEMM_TILE_SPACE:
        g = hip_lib.GemmTile(bm, bn, bk, waves, 8)
        if not hip_lib.gemm_supported(g):
            continue
        live = hip_lib.kernel_resources_live(1, gtile=g)
        _compare_resources(live, table[hip_lib.gemm_kernel_symbol(g)], waves)
        checked += 1
    print(f"[fa_abi] kernel resources checked for {checked} launches", flush=True)
    assert checked >= 40


def _compare_resources(live: dict, raw: dict, waves: int) -> None:
    assert live["vgprs"] == raw["VGPRs"]
    assert live["agprs"] == raw["AGPRs"]
    assert live["sgprs"] == raw["TotalSGPRs"]
    assert live["scratch_bytes"] == raw["ScratchSize [bytes/lane]"]
    assert live["occupancy"] == raw["Occupancy [waves/SIMD]"]
    assert live["lds_bytes"] == raw["LDS Size [bytes/block]"]
    assert live["threads"] == waves * 64 <= live["max_threads"]


# Shapes that run the persistent short-K GEMM kernel of the 256x128x64 8-wave tile (whole tiles,
# 4..16 K slabs, a tile count divisible by 8): many tiles per workgroup, an uneven share (272 tiles
# over 256 workgroups), one tile each, an odd slab count, the longest K it takes, GROUP_M 1 / 4 / 8.
PERSIST_GEMM_CASES = [(8192, 8192, 256, 8), (4352, 2048, 256, 4), (2048, 1024, 256, 8), (4096, 1024, 320, 1),
                      (1024, 2048, 1024, 8), (4096, 4096, 512, 4)]


@pytest.mark.parametrize("M,N,K,gm", PERSIST_GEMM_CASES)
def test_gemm_persistent_matches_per_tile_kernel(gpu, M, N, K, gm):
    """The persistent kernel (16-byte aligned C) against the same tile's one-workgroup-per-tile
    kernel (C 8 bytes off 16-byte alignment, which the persistent kernel does not take): identical
    accumulation order and rounding, so the results must be bit-identical."""
    print(f"[gemm_abi] persistent M={M} N={N} K={K} group_m={gm}", flush=True)
    g = torch.Generator(device="cuda:0").manual_seed(M + N + K)
    a = (torch.rand((M, K), generator=g, device="cuda:0") * 2 - 1).half()
    b = (torch.rand((K, N), generator=g, device="cuda:0") * 2 - 1).half()
    tile = hip_lib.GemmTile(256, 128, 64, 8, gm)
    c = torch.full((M, N), float("nan"), dtype=F16, device="cuda:0")
    assert c.data_ptr() % 16 == 0
    hip_lib.gemm_f16(a, b, c, tile)
    raw = torch.full((M * N + 4,), float("nan"), dtype=F16, device="cuda:0")
    c8 = raw[4:].view(M, N)
    assert c8.data_ptr() % 16 == 8
    hip_lib.gemm_f16(a, b, c8, tile)
    torch.cuda.synchronize()
    assert not torch.isnan(c).any()
    assert torch.equal(c, c8)


def test_gemm_persistent_against_oracle(gpu):
    """The persistent kernel on a small shape against the exact oracle product."""
    M, N, K = 2048, 1024, 320
    print(f"[gemm_abi] persistent oracle M={M} N={N} K={K}", flush=True)
    a = oracle.round_to(oracle.portable_uniform(21, (M, K), -1, 1), 0)
    b = oracle.round_to(oracle.portable_uniform(22, (K, N), -1, 1), 0)
    cd = torch.empty((M, N), dtype=F16, device="cuda:0")
    hip_lib.gemm_f16(to_device(a, F16, "cuda:0"), to_device(b, F16, "cuda:0"), cd, hip_lib.GemmTile(256, 128, 64, 8, 8))
    torch.cuda.synchronize()
    ref = oracle.gemm(a, b)
    c = cd.float().cpu().numpy()
    assert float(np.linalg.norm(c - ref) / np.linalg.norm(ref)) <= 1e-3
