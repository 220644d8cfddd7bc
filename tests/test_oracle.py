"""Pins the CPU oracle (oracle/) before it is trusted as the checker of the HIP kernels.

Each check is chosen so that a plausible oracle mistake (dropped scale, wrong causal offset,
transposed operand, wrong GQA head mapping, wrong LSE base) fails at least one of them:
  * golden fixtures from torch's CPU SDPA / matmul in float64 (the reference tests' own oracle path,
    test_flash_atten.py:498-499, test_mma.py:260-261);
  * torch CPU SDPA directly on fresh inputs, including GQA (enable_gqa) and top-left causal;
  * closed forms: one-hot values, identical keys, a single key, the first causal row, softmax shift
    invariance, q/scale reciprocity, causal prefix truncation, GQA == repeat_interleave, and
    merge(split(KV)) == full;
  * GEMM identities (identity, permutation, integer-valued exactness);
  * the IEEE rounding helpers against numpy float16 / torch bfloat16 casts.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
META = json.loads((GOLDEN / "golden.json").read_text())


def _golden_inputs(meta):
    od = meta["dtype"]
    s = meta["input_scale"]
    q = oracle.round_to(oracle.portable_normal(meta["seed"], (meta["B"], meta["H"], meta["M"], meta["D"])) * s, od)
    k = oracle.round_to(oracle.portable_normal(meta["seed"] + 1, (meta["B"], meta["Hkv"], meta["N"], meta["D"])) * s, od)
    v = oracle.round_to(oracle.portable_normal(meta["seed"] + 2, (meta["B"], meta["Hkv"], meta["N"], meta["D"])) * s, od)
    return q, k, v


def _digest(*arrays):
    import hashlib

    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a, dtype=np.float32).tobytes())
    return h.hexdigest()


# ---- portable generator -----------------------------------------------------------------------

def test_portable_rng_stream_is_pinned():
    u = oracle.portable_uniform(1, (4,))
    z = oracle.portable_normal(20260328, (3,))
    # splitmix64 first output for state 1 (Vigna's reference implementation, seed=1): 0x910a2dec89025cc1
    assert int(oracle._splitmix64(1, 1)[0]) == 0x910A2DEC89025CC1
    assert np.all((u >= 0) & (u < 1))
    assert z.shape == (3,) and np.all(np.isfinite(z))


def test_portable_normal_moments():
    z = oracle.portable_normal(7, (200_000,))
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01


# ---- rounding -------------------------------------------------------------------------------------

def test_round_f16_matches_numpy_rne():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0,
        rng.standard_normal(2000).astype(np.float32) * 1e-5,  # subnormal range
        np.array([65504.0, 65519.0, 65520.0, 70000.0, -65520.0, 0.0, -0.0, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11,
                  np.inf, -np.inf, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26], dtype=np.float32),
    ])
    ours = oracle.round_to(vals, oracle.DTYPE_F16)
    ref = vals.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(ours, ref)


def test_round_bf16_matches_torch():
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 100.0,
                           np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 3.4e38, -0.0], dtype=np.float32)])
    ours = oracle.round_to(vals, oracle.DTYPE_BF16)
    ref = torch.from_numpy(vals).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ours, ref)


# ---- golden fixtures ------------------------------------------------------------------------------

@pytest.mark.parametrize("name", sorted(META["attention"]))
def test_attention_oracle_matches_golden(name):
    meta = META["attention"][name]
    q, k, v = _golden_inputs(meta)
    assert _digest(q, k, v) == meta["inputs_sha256"], "portable generator stream changed"
    ref = np.load(GOLDEN / f"{name}.npz")
    o, lse = oracle.attention(q, k, v, causal=meta["causal"])
    np.testing.assert_allclose(o, ref["o"], atol=2e-6, rtol=1e-5)
    np.testing.assert_allclose(lse, ref["lse"], atol=2e-6, rtol=1e-6)


@pytest.mark.parametrize("name", sorted(META["gemm"]))
def test_gemm_oracle_matches_golden(name):
    meta = META["gemm"][name]
    a = oracle.round_to(oracle.portable_uniform(meta["seed"], (meta["M"], meta["K"]), -1, 1), oracle.DTYPE_F16)
    b = oracle.round_to(oracle.portable_uniform(meta["seed"] + 1, (meta["K"], meta["N"]), -1, 1), oracle.DTYPE_F16)
    assert _digest(a, b) == meta["inputs_sha256"]
    np.testing.assert_allclose(oracle.gemm(a, b), np.load(GOLDEN / f"{name}.npz")["c"], atol=1e-5, rtol=1e-6)


# ---- against torch SDPA (the reference tests' oracle) on fresh inputs ----------------------------

@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(2, 4, 4, 37, 37, 64), (1, 6, 2, 33, 71, 128), (1, 2, 1, 50, 20, 256)])
def test_attention_oracle_matches_torch_sdpa(shape, causal):
    B, H, Hkv, M, N, D = shape
    q = oracle.portable_normal(101, (B, H, M, D))
    k = oracle.portable_normal(102, (B, Hkv, N, D))
    v = oracle.portable_normal(103, (B, Hkv, N, D))
    o, lse = oracle.attention(q, k, v, causal=causal)
    qt, kt, vt = (torch.from_numpy(x) for x in (q, k, v))
    ref = F.scaled_dot_product_attention(qt, kt, vt, is_causal=causal, enable_gqa=H != Hkv).numpy()
    np.testing.assert_allclose(o, ref, atol=2e-6, rtol=1e-5)
    o2, lse2 = oracle.attention_np(q, k, v, causal=causal)
    np.testing.assert_allclose(o, o2, atol=2e-6)
    np.testing.assert_allclose(lse, lse2, atol=2e-6)


# ---- closed forms ---------------------------------------------------------------------------------

def _softmax_rows(s):
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    return e / e.sum(axis=-1, keepdims=True)


def test_one_hot_values_give_softmax_rows():
    D = N = 64
    q = oracle.portable_normal(1, (1, 1, 16, D))
    k = oracle.portable_normal(2, (1, 1, N, D))
    v = np.eye(N, D, dtype=np.float64)[None, None]
    o, lse = oracle.attention(q, k, v)
    s = (q[0, 0] @ k[0, 0].T) * D ** -0.5
    np.testing.assert_allclose(o[0, 0], _softmax_rows(s), atol=1e-6)
    np.testing.assert_allclose(lse[0, 0], np.log(np.exp(s).sum(-1)), atol=1e-5)


def test_identical_keys_average_values():
    D, N = 128, 40
    q = oracle.portable_normal(3, (1, 2, 8, D))
    k = np.repeat(oracle.portable_normal(4, (1, 2, 1, D)), N, axis=2)
    v = oracle.portable_normal(5, (1, 2, N, D))
    o, _ = oracle.attention(q, k, v)
    np.testing.assert_allclose(o, np.broadcast_to(v.mean(axis=2, keepdims=True), o.shape), atol=1e-6)


def test_single_key_copies_value_and_lse_is_scaled_logit():
    D = 64
    q = oracle.portable_normal(6, (1, 3, 5, D))
    k = oracle.portable_normal(7, (1, 3, 1, D))
    v = oracle.portable_normal(8, (1, 3, 1, D))
    o, lse = oracle.attention(q, k, v, scale=0.3)
    np.testing.assert_allclose(o, np.broadcast_to(v, o.shape), atol=1e-6)
    np.testing.assert_allclose(lse, 0.3 * np.einsum("bhmd,bhd->bhm", q, k[:, :, 0]), atol=1e-5)


def test_causal_rows_equal_truncated_noncausal():
    D, S = 64, 24
    q = oracle.portable_normal(9, (1, 2, S, D))
    k = oracle.portable_normal(10, (1, 2, S, D))
    v = oracle.portable_normal(11, (1, 2, S, D))
    o, lse = oracle.attention(q, k, v, causal=True)
    np.testing.assert_allclose(o[:, :, 0], v[:, :, 0], atol=1e-6)  # first row sees only key 0
    for m in (1, 7, S - 1):
        o_m, lse_m = oracle.attention(q[:, :, m:m + 1], k[:, :, :m + 1], v[:, :, :m + 1])
        np.testing.assert_allclose(o[:, :, m], o_m[:, :, 0], atol=1e-6)
        np.testing.assert_allclose(lse[:, :, m], lse_m[:, :, 0], atol=1e-5)


def test_softmax_shift_and_scale_invariance():
    D = 128
    q = oracle.portable_normal(12, (1, 2, 10, D))
    k = oracle.portable_normal(13, (1, 2, 30, D))
    v = oracle.portable_normal(14, (1, 2, 30, D))
    c = oracle.portable_normal(15, (1, 2, 1, D))
    o, lse = oracle.attention(q, k, v)
    o_shift, lse_shift = oracle.attention(q, k + c, v)
    np.testing.assert_allclose(o, o_shift, atol=1e-5)
    np.testing.assert_allclose(lse_shift - lse, D ** -0.5 * np.einsum("bhmd,bhd->bhm", q, c[:, :, 0]), atol=1e-4)
    o_sc, lse_sc = oracle.attention(q * 2.0, k, v, scale=D ** -0.5 / 2.0)
    np.testing.assert_allclose(o, o_sc, atol=1e-6)
    np.testing.assert_allclose(lse, lse_sc, atol=1e-5)


def test_gqa_equals_repeat_interleave():
    q = oracle.portable_normal(16, (2, 6, 12, 64))
    k = oracle.portable_normal(17, (2, 2, 20, 64))
    v = oracle.portable_normal(18, (2, 2, 20, 64))
    o, lse = oracle.attention(q, k, v, causal=True)
    o_x, lse_x = oracle.attention(q, np.repeat(k, 3, axis=1), np.repeat(v, 3, axis=1), causal=True)
    np.testing.assert_allclose(o, o_x, atol=0)
    np.testing.assert_allclose(lse, lse_x, atol=0)


@pytest.mark.parametrize("bounds", [(0, 17, 40), (0, 5, 6, 40), (0, 40)])
def test_lse_merge_of_kv_splits_equals_full(bounds):
    D, M = 64, 9
    q = oracle.portable_normal(19, (1, 1, M, D))
    k = oracle.portable_normal(20, (1, 1, 40, D))
    v = oracle.portable_normal(21, (1, 1, 40, D))
    o, lse = oracle.attention(q, k, v)
    parts = [oracle.attention(q, k[:, :, a:b], v[:, :, a:b]) for a, b in zip(bounds[:-1], bounds[1:])]
    o_parts = np.stack([p[0].reshape(M, D) for p in parts])
    lse_parts = np.stack([p[1].reshape(M) for p in parts])
    o_m, lse_m = oracle.lse_merge(o_parts, lse_parts)
    np.testing.assert_allclose(o_m, o.reshape(M, D), atol=1e-6)
    np.testing.assert_allclose(lse_m, lse.reshape(M), atol=1e-6)


def test_lse_merge_ignores_empty_splits():
    o_parts = np.stack([np.ones((2, 4)), np.zeros((2, 4))]).astype(np.float32)
    lse_parts = np.array([[0.5, 1.0], [-np.inf, -np.inf]], dtype=np.float32)
    o, lse = oracle.lse_merge(o_parts, lse_parts)
    np.testing.assert_allclose(o, 1.0)
    np.testing.assert_allclose(lse, [0.5, 1.0])


def test_rows_variant_matches_full():
    q = oracle.portable_normal(22, (2, 3, 17, 64))
    k = oracle.portable_normal(23, (2, 1, 29, 64))
    v = oracle.portable_normal(24, (2, 1, 29, 64))
    o, lse = oracle.attention(q, k, v, causal=True)
    rows = np.array([0, 5, 16, 17, 50, 2 * 3 * 17 - 1])
    o_r, lse_r = oracle.attention_rows(q, k, v, rows, causal=True)
    np.testing.assert_allclose(o_r, o.reshape(-1, 64)[rows], atol=0)
    np.testing.assert_allclose(lse_r, lse.reshape(-1)[rows], atol=0)


def test_online_blocked_algorithm_close_to_exact():
    """The reference kernel's own blocked algorithm (P rounded to fp16) stays within a few 1e-3."""
    q = oracle.round_to(oracle.portable_normal(25, (1, 2, 64, 64)), 0)
    k = oracle.round_to(oracle.portable_normal(26, (1, 2, 200, 64)), 0)
    v = oracle.round_to(oracle.portable_normal(27, (1, 2, 200, 64)), 0)
    for causal in (False, True):
        o, lse = oracle.attention(q, k, v, causal=causal)
        o_on, lse_on = oracle.attention_online(q, k, v, causal=causal, block_n=64)
        assert np.abs(o - o_on).max() < 3e-3
        assert np.abs(lse - lse_on).max() < 1e-4


def test_checks_catch_planted_mistakes():
    """Plausible oracle bugs, planted in numpy restatements, fail the closed-form checks."""
    D = 64
    q = oracle.portable_normal(28, (1, 1, 6, D))
    k = oracle.portable_normal(29, (1, 1, 6, D))
    v = oracle.portable_normal(30, (1, 1, 6, D))
    good, _ = oracle.attention(q, k, v, causal=True)

    def attn(qq, kk, vv, scale, causal_offset):
        s = (qq[0, 0] @ kk[0, 0].T) * scale
        mask = np.arange(6)[None, :] > np.arange(6)[:, None] + causal_offset
        s = np.where(mask, -np.inf, s)
        return (_softmax_rows(s) @ vv[0, 0])[None, None]

    assert np.abs(attn(q, k, v, D ** -0.5, 0) - good).max() < 1e-5  # correct restatement agrees
    assert np.abs(attn(q, k, v, 1.0, 0) - good).max() > 1e-2  # dropped scale
    assert np.abs(attn(q, k, v, D ** -0.5, 1) - good).max() > 1e-2  # off-by-one causal mask
    assert np.abs(attn(q, v, k, D ** -0.5, 0) - good).max() > 1e-2  # swapped K/V operands


# ---- GEMM ---------------------------------------------------------------------------------------

def test_gemm_identity_permutation_and_integers():
    a = oracle.portable_uniform(31, (48, 64), -1, 1)
    eye = np.eye(64)
    np.testing.assert_allclose(oracle.gemm(a, eye), a.astype(np.float32), atol=0)
    perm = np.eye(64)[np.roll(np.arange(64), 5)]
    np.testing.assert_allclose(oracle.gemm(a, perm), (a @ perm).astype(np.float32), atol=0)
    ai = np.floor(oracle.portable_uniform(32, (40, 256), -8, 8))
    bi = np.floor(oracle.portable_uniform(33, (256, 24), -8, 8))
    np.testing.assert_array_equal(oracle.gemm(ai, bi), (ai @ bi).astype(np.float32))
    entries = oracle.gemm_entries(ai, bi, [0, 39, 7], [0, 23, 11])
    np.testing.assert_array_equal(entries, (ai @ bi)[[0, 39, 7], [0, 23, 11]])


def test_gemm_matches_torch_matmul():
    a = oracle.portable_uniform(34, (96, 160), -1, 1)
    b = oracle.portable_uniform(35, (160, 72), -1, 1)
    ref = (torch.from_numpy(a) @ torch.from_numpy(b)).numpy()
    np.testing.assert_allclose(oracle.gemm(a, b), ref, atol=1e-5)


def test_flop_conventions():
    # test_flash_atten.py:234-240 and test_mma.py:78-83
    assert oracle.attention_flops(4, 32, 8192, 8192, 128, False) == 4 * 4 * 32 * 128 * 8192 * 8192
    assert oracle.attention_flops(1, 1, 8, 8, 64, True) == 4 * 64 * 8 * 9 / 2
    assert oracle.gemm_flops(8192, 8192, 8192) == 2 * 8192 ** 3
