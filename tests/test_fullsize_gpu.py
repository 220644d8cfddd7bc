"""The benchmark configurations at full size (GPU; fp16 B4 H32 N8192 D128, bf16 B2 H16 D256, the
GQA 12:2 prefill, GEMM 1024..16384 squares): sampled rows against the oracle plus
size-independent properties (first causal row copies V[0]; native GQA equals the expanded
computation bit for bit; KV-split invariance; finite outputs), and the 8192^3 GEMM against an fp32
product and sampled exact entries."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import hip_lib
import mma
import oracle
from flash_atten import attention
from helpers import ATOL, oracle_rows_threaded

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _randn(shape, seed, dtype, scale=1.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=DEV, dtype=torch.float32) * scale).to(dtype)


def _check_rows(q, k, v, out, causal, heads, rows_per_head=24, scale=None, tol=2e-2, seed=0):
    """Oracle on `rows_per_head` random rows of each listed (b, h)."""
    B, H, M, D = q.shape
    Hkv = k.shape[1]
    rng = np.random.default_rng(seed)
    worst = 0.0
    for b, h in heads:
        hk = h // (H // Hkv)
        rows = np.sort(rng.choice(M, size=min(rows_per_head, M), replace=False))
        rows[0] = 0
        rows[-1] = M - 1
        qs = q[b, h].float().cpu().numpy()[None, None]
        ks = k[b, hk].float().cpu().numpy()[None, None]
        vs = v[b, hk].float().cpu().numpy()[None, None]
        o_ref, _ = oracle.attention_rows(qs, ks, vs, rows, causal=causal, scale=scale)
        got = out[b, h].float().cpu().numpy()[rows]
        worst = max(worst, float(np.abs(got - o_ref).max()))
    assert worst <= tol, worst
    return worst


# (b, h) pairs sampled at B=4, H=32: both ends of the batch and head ranges, the last pair included
B4H32_HEADS = [(0, 0), (0, 31), (1, 5), (1, 17), (2, 9), (2, 24), (3, 3), (3, 31)]


@pytest.mark.parametrize("N", [1024, 2048, 4096, 8192, 16384])
@pytest.mark.parametrize("variant", ["optimized", "basic", "sliced"])
@pytest.mark.parametrize("causal", [False, True])
def test_config3_fa_fp16_b4h32d128(gpu, variant, causal, N):
    """BASELINE configs[2] (N = 8192 is the headline): fp16 B=4 H=32 D=128, N swept 1024..16384,
    non-causal and causal, all three variants through the tuning table's tile for that size."""
    print(f"[fullsize] fa fp16 4x32x{N}x128 causal={causal} {variant}", flush=True)
    B, H, D = 4, 32, 128
    q, k, v = (_randn((B, H, N, D), N + s, torch.float16) for s in (1, 2, 3))
    out = attention(q, k, v, causal=causal, variant=variant)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    _check_rows(q, k, v, out, causal, B4H32_HEADS, rows_per_head=16, seed=N + int(causal))
    if causal:
        assert torch.equal(out[:, :, 0], v[:, :, 0])  # row 0 attends only key 0: O = V[0] exactly


def _block_rows(B, H, M, block, seed):
    """One flattened row (b*H + h)*M + m in every `block`-row query block of every (b, h), at a
    random offset inside the block (so the rows land in every wave and lane position), plus the
    last row of every (b, h)."""
    rng = np.random.default_rng(seed)
    nb = -(-M // block)
    base = (np.arange(B * H, dtype=np.int64)[:, None] * M + np.arange(nb, dtype=np.int64)[None, :] * block)
    m_in = np.minimum(rng.integers(0, block, size=base.shape), M - 1 - np.arange(nb)[None, :] * block)
    last = np.arange(B * H, dtype=np.int64) * M + M - 1
    return np.unique(np.concatenate([(base + m_in).ravel(), last]))


# Tiles the config-3 workgroup sweep runs, besides the tuning table's choice: the ping-pong
# 256-row kernel and the 128-row pipelined kernels (16x16 and 32x32 MFMA tiles).
CONFIG3_TILES = [None, (256, 64, 8, 8), (128, 64, 4, 7), (128, 64, 4, 3)]


@pytest.mark.parametrize("causal", [False, True])
def test_config3_every_workgroup(gpu, causal):
    """BASELINE configs[2] at N = 8192 (the headline shape, and its causal case): one oracle row in
    every 128-row query block of every (b, h) -- 8192 rows, so every workgroup of every tile's grid
    (XCD remap, causal heaviest-first order, both ping-pong wave groups) is checked -- for the
    table's tile and each listed tile, through the C ABI."""
    B, H, N, D = 4, 32, 8192, 128
    print(f"[fullsize] every workgroup fp16 4x32x8192x128 causal={causal}", flush=True)
    q, k, v = (_randn((B, H, N, D), 40 + s + 10 * int(causal), torch.float16) for s in range(3))
    rows = _block_rows(B, H, N, 128, seed=7 + int(causal))
    assert rows.size >= B * H * (N // 128)
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    o_ref, lse_ref = oracle_rows_threaded(qn, kn, vn, rows, causal=causal)
    del qn, kn, vn
    rows_t = torch.from_numpy(rows).to(DEV)
    for t in CONFIG3_TILES:
        print(f"[fullsize]   tile {t or 'tuned'}", flush=True)
        if t is None:
            out, lse = attention(q, k, v, causal=causal, variant="optimized", return_lse=True)
        else:
            out = torch.empty_like(q)
            lse = torch.empty((B, H, N), device=DEV, dtype=torch.float32)
            hip_lib.fa_fwd(q, k, v, out, lse, sm_scale=D ** -0.5, causal=causal, variant=hip_lib.FA_VARIANT_OPT,
                           tile=hip_lib.make_tile(*t, 1))
        got = out.reshape(-1, D)[rows_t].float().cpu().numpy()
        got_lse = lse.reshape(-1)[rows_t].cpu().numpy()
        err = float(np.abs(got - o_ref).max())
        err_lse = float(np.abs(got_lse - lse_ref).max())
        print(f"[fullsize]   tile {t or 'tuned'}: max|dO| {err:.3e} max|dLSE| {err_lse:.3e}", flush=True)
        assert err <= ATOL[torch.float16], (t, err)
        assert err_lse <= 1e-3, (t, err_lse)
        del out, lse


# The reference's own pipeline cases at long sequence (test_flash_atten.py:82-88): B=1, H28 D128
# and H16 D256, fp16, non-causal, S = 32768 and 65536; all three variants.
@pytest.mark.parametrize("S", [32768, 65536])
@pytest.mark.parametrize("H,D", [(28, 128), (16, 256)])
def test_reference_long_sequence_cases(gpu, H, D, S):
    print(f"[fullsize] reference pipeline case B1 H{H} D{D} S{S}", flush=True)
    q, k, v = (_randn((1, H, S, D), 60 + s + S // 1024, torch.float16) for s in range(3))
    rng = np.random.default_rng(S + D)
    # per head: 8 random rows, the first and the last
    rows = np.unique(np.concatenate([h * S + np.concatenate([[0, S - 1], rng.integers(0, S, 8)])
                                     for h in range(H)]).astype(np.int64))
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    o_ref, _ = oracle_rows_threaded(qn, kn, vn, rows, causal=False)
    del qn, kn, vn
    rows_t = torch.from_numpy(rows).to(DEV)
    for variant in ("basic", "optimized", "sliced"):
        out = attention(q, k, v, causal=False, variant=variant)
        got = out.reshape(-1, D)[rows_t].float().cpu().numpy()
        assert torch.isfinite(out).all()
        err = float(np.abs(got - o_ref).max())
        print(f"[fullsize]   {variant}: max|dO| {err:.3e}", flush=True)
        assert err <= ATOL[torch.float16], (variant, err)
        del out


@pytest.mark.parametrize("N", [1024, 2048, 4096, 8192])
def test_bf16_d256_b2h16_sliced(gpu, N):
    """bf16, D=256, B=2, H=16, inputs N(0,1)*0.5, sliced split-KV + LSE merge."""
    print(f"[fullsize] fa bf16 d256 N={N}", flush=True)
    B, H, D = 2, 16, 256
    q, k, v = (_randn((B, H, N, D), 10 + s, torch.bfloat16, 0.5) for s in range(3))
    out, lse = attention(q, k, v, causal=False, variant="sliced", return_lse=True)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    _check_rows(q, k, v, out, False, [(0, 0), (0, 9), (1, 4), (1, 15)], tol=ATOL[torch.bfloat16])


def test_split_invariance_and_lse(gpu):
    """Sliced output is invariant (to fp16 output rounding) to the number of KV splits."""
    B, H, M, N, D = 1, 8, 512, 8192, 128
    q, k, v = (_randn((B, H, s_len, D), 20 + i, torch.float16) for i, s_len in enumerate((M, N, N)))
    outs, lses = [], []
    for splits in (1, 4, 16):
        o = torch.empty_like(q)
        lse = torch.empty((B, H, M), device=DEV, dtype=torch.float32)
        ws_bytes = hip_lib.workspace_bytes(B, H, M, D, splits)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
        hip_lib.fa_fwd(q, k, v, o, lse, sm_scale=D ** -0.5, causal=False, variant=hip_lib.FA_VARIANT_SLICED,
                       tile=hip_lib.make_tile(256, 64, 8, 2, splits), workspace=ws if ws_bytes else None)
        outs.append(o.float())
        lses.append(lse)
    torch.cuda.synchronize()
    for o, lse in zip(outs[1:], lses[1:]):
        assert (o - outs[0]).abs().max().item() <= 2e-3
        assert (lse - lses[0]).abs().max().item() <= 1e-4


def test_ttft_shape_gqa_bf16_causal(gpu):
    """BASELINE configs[4] attention shape: [1,12,S,128] queries, 2 KV heads, bf16, causal."""
    for S in (4096, 16384):
        print(f"[fullsize] ttft-shape S={S}", flush=True)
        q = _randn((1, 12, S, 128), 30, torch.bfloat16)
        k = _randn((1, 2, S, 128), 31, torch.bfloat16)
        v = _randn((1, 2, S, 128), 32, torch.bfloat16)
        out = attention(q, k, v, causal=True, variant="sliced")
        out_x = attention(q, k.repeat_interleave(6, dim=1), v.repeat_interleave(6, dim=1), causal=True,
                          variant="sliced")
        torch.cuda.synchronize()
        assert torch.equal(out, out_x)
        _check_rows(q, k, v, out, True, [(0, 0), (0, 7), (0, 11)], tol=ATOL[torch.bfloat16])


@pytest.mark.parametrize("n", [1024, 2048, 4096, 8192, 16384])
def test_gemm_square_sweep(gpu, n):
    """fp16 A,B ~ U[-1,1], fp32 accumulation; relative Frobenius <= 1e-3."""
    print(f"[fullsize] gemm {n}^3", flush=True)
    g = torch.Generator(device=DEV).manual_seed(n)
    a = (torch.rand((n, n), generator=g, device=DEV) * 2 - 1).half()
    b = (torch.rand((n, n), generator=g, device=DEV) * 2 - 1).half()
    c = mma.matmul(a, b)
    ref = a.float() @ b.float()
    torch.cuda.synchronize()
    rel = ((c.float() - ref).norm() / ref.norm()).item()
    assert rel <= 1e-3, rel
    del ref
    rng = np.random.default_rng(n)
    ii, jj = rng.integers(0, n, 256), rng.integers(0, n, 256)
    a_rows = a[torch.from_numpy(ii).to(DEV)].float().cpu().numpy()
    b_cols = b[:, torch.from_numpy(jj).to(DEV)].float().cpu().numpy()
    exact = np.einsum("tk,kt->t", a_rows.astype(np.float64), b_cols.astype(np.float64))
    got = c[torch.from_numpy(ii).to(DEV), torch.from_numpy(jj).to(DEV)].float().cpu().numpy()
    assert np.abs(got - exact).max() <= 2e-3 * np.sqrt(n / 1024) * 8 + np.abs(exact).max() * 2 ** -10
