"""Seeded randomized parity sweeps against the exact oracle. Attention: every built tile of every
variant, fp16/bf16, head dims 64/128/256, GQA groups, causal, ragged M and N (M != N included),
split counts beyond the KV tile count, with and without LSE. GEMM: every built tile, ragged M,
N % 4 == 0, K % 8 == 0 from one slab to many (so both the shallow and the deep LDS ring run).
Each case is drawn from its own seed, so a failure names a reproducible case."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import gfx950_configs as cfgs
import hip_lib
import oracle
from helpers import ATOL, make_qkv, max_abs, to_device

pytestmark = pytest.mark.gpu

N_CASES = 120
N_GEMM_CASES = 40
SEED0 = 20261201


def draw_case(i: int) -> dict:
    rng = np.random.RandomState(SEED0 + i)
    variant = int(rng.choice([hip_lib.FA_VARIANT_BASIC, hip_lib.FA_VARIANT_OPT, hip_lib.FA_VARIANT_SLICED]))
    dtype = [torch.float16, torch.bfloat16][rng.randint(2)]
    D = int(rng.choice([64, 128, 256]))
    cands = cfgs.fa_candidates(variant, dtype, D)
    tile = cands[rng.randint(len(cands))]
    limit = 160 if D == 256 else 300
    Hkv = int(rng.randint(1, 3))
    return {
        "variant": variant, "dtype": dtype, "D": D, "tile": tile,
        "B": int(rng.randint(1, 3)), "Hkv": Hkv, "H": Hkv * int(rng.randint(1, 4)),
        "M": int(rng.randint(1, limit)), "N": int(rng.randint(1, limit + 100)),
        "causal": bool(rng.randint(2)),
        "splits": int(rng.choice([1, 2, 3, 5, 8])) if variant == hip_lib.FA_VARIANT_SLICED else 1,
        "with_lse": bool(rng.randint(2)),
        "scale": float(rng.choice([0.5, 1.0])),
    }


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_case_matches_oracle(gpu, i):
    c = draw_case(i)
    t = c["tile"]
    print(f"[random_parity] case {i}: variant={c['variant']} {c['dtype']} D={c['D']} tile={t.block_m}x{t.block_n}"
          f"x{t.waves} st={t.stages} B={c['B']} H={c['H']}/{c['Hkv']} M={c['M']} N={c['N']} causal={c['causal']} "
          f"splits={c['splits']} lse={c['with_lse']}", flush=True)
    q, k, v = make_qkv(SEED0 + 97 * i, c["B"], c["H"], c["Hkv"], c["M"], c["N"], c["D"], c["dtype"], c["scale"])
    dev = "cuda:0"
    qd, kd, vd = (to_device(x, c["dtype"], dev) for x in (q, k, v))
    o = torch.full_like(qd, float("nan"))
    lse = (torch.full((c["B"], c["H"], c["M"]), float("nan"), dtype=torch.float32, device=dev)
           if c["with_lse"] else None)
    ws = None
    need = hip_lib.workspace_bytes(c["B"], c["H"], c["M"], c["D"], c["splits"])
    if need:
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
    ctile = cfgs.FaTileChoice(t.block_m, t.block_n, t.waves, t.stages, c["splits"]).to_c()
    hip_lib.fa_fwd(qd, kd, vd, o, lse, sm_scale=c["D"] ** -0.5, causal=c["causal"], variant=c["variant"],
                   tile=ctile, workspace=ws)
    torch.cuda.synchronize()
    o_ref, lse_ref = oracle.attention(q, k, v, causal=c["causal"])
    got = o.float().cpu().numpy()
    assert np.isfinite(got).all(), "unwritten or non-finite output"
    assert max_abs(got, o_ref) <= ATOL[c["dtype"]]
    if lse is not None:
        assert max_abs(lse.cpu().numpy(), lse_ref) <= 1e-3


def draw_gemm_case(i: int) -> dict:
    rng = np.random.RandomState(SEED0 + 100000 + i)
    cands = cfgs.gemm_candidates()
    t = cands[rng.randint(len(cands))]
    return {"tile": t, "group_m": int(rng.choice([1, 4, 8, 16])), "M": int(rng.randint(1, 700)),
            "N": 4 * int(rng.randint(1, 180)), "K": 8 * int(rng.randint(1, 160))}


@pytest.mark.parametrize("i", range(N_GEMM_CASES))
def test_random_gemm_case_matches_oracle(gpu, i):
    c = draw_gemm_case(i)
    t = c["tile"]
    M, N, K = c["M"], c["N"], c["K"]
    print(f"[random_parity] gemm case {i}: tile={t} group_m={c['group_m']} M={M} N={N} K={K}", flush=True)
    a = oracle.round_to(oracle.portable_uniform(SEED0 + 3 * i, (M, K), -1, 1), oracle.DTYPE_F16)
    b = oracle.round_to(oracle.portable_uniform(SEED0 + 3 * i + 1, (K, N), -1, 1), oracle.DTYPE_F16)
    # B rows need 16-byte alignment: pad its leading dimension to a multiple of 8 when N % 8 != 0
    ldb = -(-N // 8) * 8
    bbuf = torch.zeros((K, ldb), dtype=torch.float16, device="cuda:0")
    bbuf[:, :N] = to_device(b, torch.float16, "cuda:0")
    cd = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda:0")
    hip_lib.gemm_f16(to_device(a, torch.float16, "cuda:0"), bbuf[:, :N], cd, hip_lib.GemmTile(*t, c["group_m"]))
    torch.cuda.synchronize()
    ref = oracle.gemm(a, b)
    got = cd.float().cpu().numpy()
    assert np.isfinite(got).all(), "unwritten or non-finite output"
    assert float(np.linalg.norm(got - ref) / np.linalg.norm(ref)) <= 1e-3
