"""TTFT harness: the SDPA replacement's contract on the CPU, and on the GPU a
small Qwen2-architecture decoder whose every attention call runs the gfx950 kernel, checked
against torch's own SDPA the way the reference's verify_against_flash does (ttft.py:415-446)."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import flash_atten
import oracle
import ttft_qwen
from helpers import max_abs, to_device

SMALL = dict(vocab_size=2048, num_hidden_layers=2)


def test_architecture_numbers_match_baseline():
    a = ttft_qwen.QWEN25_1P5B
    assert (a["num_hidden_layers"], a["hidden_size"], a["num_attention_heads"], a["num_key_value_heads"]) == (
        28, 1536, 12, 2)
    assert a["hidden_size"] // a["num_attention_heads"] == 128
    assert (a["intermediate_size"], a["rope_theta"], a["vocab_size"]) == (8960, 1e6, 151936)


def test_patch_rejects_unsupported_calls_and_restores():
    original = F.scaled_dot_product_attention
    q = torch.zeros(1, 2, 4, 64)
    with ttft_qwen.patched_sdpa_with_gfx950(allow_causal=False):
        assert F.scaled_dot_product_attention is not original
        with pytest.raises(RuntimeError, match="dropout"):
            F.scaled_dot_product_attention(q, q, q, dropout_p=0.1)
        with pytest.raises(RuntimeError, match="attn_mask"):
            F.scaled_dot_product_attention(q, q, q, attn_mask=torch.ones(4, 4, dtype=torch.bool))
        with pytest.raises(RuntimeError, match="is_causal"):
            F.scaled_dot_product_attention(q, q, q, is_causal=True)
    with ttft_qwen.patched_sdpa_with_gfx950():
        with pytest.raises(RuntimeError, match="tensors on cpu"):
            F.scaled_dot_product_attention(q, q, q)
    assert F.scaled_dot_product_attention is original


def test_small_model_builds_on_cpu():
    model = ttft_qwen.build_model(seed=1, device="cpu", dtype=torch.float32,
                                  overrides=dict(SMALL, hidden_size=256, intermediate_size=512, num_attention_heads=4,
                                                 num_key_value_heads=2))
    ids = ttft_qwen.make_prompt(9, model.config.vocab_size, device="cpu")
    assert ttft_qwen.prefill_logits(model, ids).shape == (1, model.config.vocab_size)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_sdpa_entry_strided_gqa_causal(gpu, dtype):
    """flash_atten.sdpa on the transposed projection views a decoder passes ([B,S,H,D] memory)."""
    B, S, H, Hkv, D = 1, 300, 12, 2, 128
    od = oracle.DTYPE_BF16 if dtype == torch.bfloat16 else oracle.DTYPE_F16
    q = oracle.round_to(oracle.portable_normal(51, (B, S, H, D)), od)
    k = oracle.round_to(oracle.portable_normal(52, (B, Hkv, S, D)), od)
    v = oracle.round_to(oracle.portable_normal(53, (B, Hkv, S, D)), od)
    qd = to_device(q, dtype, "cuda:0").transpose(1, 2)  # [B,H,S,D] view, row stride H*D
    kd, vd = to_device(k, dtype, "cuda:0"), to_device(v, dtype, "cuda:0")
    for variant in ("basic", "optimized", "sliced"):
        out = flash_atten.sdpa(qd, kd, vd, is_causal=True, scale=D ** -0.5, variant=variant)
        torch.cuda.synchronize()
        assert out.transpose(1, 2).is_contiguous()
        ref, _ = oracle.attention(q.transpose(0, 2, 1, 3), k, v, causal=True)
        assert max_abs(out.float().cpu().numpy(), ref) <= (3e-2 if dtype == torch.bfloat16 else 2e-2), variant


@pytest.mark.gpu
def test_small_qwen2_prefill_matches_torch_sdpa(gpu):
    print("[ttft] small qwen2 prefill", flush=True)
    model = ttft_qwen.build_model(seed=3, dtype=torch.bfloat16, overrides=SMALL)
    ids = ttft_qwen.make_prompt(1024, model.config.vocab_size, seed=5)
    check = ttft_qwen.verify_against_torch(model, ids)
    assert check["kernel_calls"] == model.config.num_hidden_layers
    assert check["allclose_rtol_atol_0p1"], check
    assert check["argmax_match"], check
    assert np.isfinite(check["max_abs_diff"])
