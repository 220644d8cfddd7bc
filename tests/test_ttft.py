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


def test_fp32_attention_yardstick_is_float32_sdpa_and_restores():
    """fp32_attention() computes every SDPA call in float32 (GQA and causal passed through) and
    returns the caller's dtype; F.scaled_dot_product_attention is restored afterwards."""
    original = F.scaled_dot_product_attention
    g = torch.Generator().manual_seed(4)
    q = torch.randn((1, 4, 33, 16), generator=g).to(torch.bfloat16)
    k = torch.randn((1, 2, 33, 16), generator=g).to(torch.bfloat16)
    v = torch.randn((1, 2, 33, 16), generator=g).to(torch.bfloat16)
    with ttft_qwen.fp32_attention():
        out = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
    assert F.scaled_dot_product_attention is original
    kr, vr = (t.float().repeat_interleave(2, dim=1) for t in (k, v))
    s = (q.float() @ kr.transpose(-1, -2)) * 16 ** -0.5
    s = s.masked_fill(torch.ones(33, 33, dtype=torch.bool).triu(1), float("-inf"))
    ref = torch.softmax(s, dim=-1) @ vr
    assert out.dtype == torch.bfloat16
    assert torch.allclose(out.float(), ref.to(torch.bfloat16).float(), atol=1e-2, rtol=0)


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


def _layer_rows_vs_oracle(rec: dict, *, heads=(0, 5, 11), rows_per_head: int = 16, seed: int = 0) -> float:
    """Max |O - O_oracle| over sampled rows of a captured attention call (first and last row of
    each listed head included). q is [1, H, S, D] (a strided view of the projection), k/v carry
    the kv heads; query head h reads kv head h // (H // H_kv)."""
    q, k, v, out = (rec[n] for n in ("q", "k", "v", "out"))
    _, H, S, D = q.shape
    group = H // k.shape[1]
    rng = np.random.default_rng(seed)
    worst = 0.0
    for h in heads:
        rows = np.sort(rng.choice(S, size=rows_per_head, replace=False))
        rows[0], rows[-1] = 0, S - 1
        qs = q[0, h].float().cpu().numpy()[None, None]
        ks = k[0, h // group].float().cpu().numpy()[None, None]
        vs = v[0, h // group].float().cpu().numpy()[None, None]
        o_ref, _ = oracle.attention_rows(qs, ks, vs, rows, causal=bool(rec["is_causal"]), scale=rec["scale"])
        got = out[0, h].float().cpu().numpy()[rows]
        worst = max(worst, max_abs(got, o_ref))
    return worst


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_qwen25_1p5b_full_prefill_layers_vs_oracle(gpu, dtype):
    """BASELINE configs[4] at full size: the 28-layer, vocab-151936 Qwen2.5-1.5B architecture (random
    init), causal prefill of 4096 and 16384 seeded tokens (fp16 also 65536) with every attention call
    on the gfx950 kernel, in bf16 (the configuration) and in fp16 (the reference harness's dtype,
    ttft.py:34).
    Asserted: the attention output of the first, a middle and the last layer against the oracle on
    sampled rows of three heads (bound 3e-2 bf16, 2e-2 fp16), one kernel call per layer, the
    final-token argmax against torch's own SDPA, and in fp16 the reference's full pass rule,
    allclose(rtol=atol=0.1) on the final logits (ttft.py:415-446). Recorded (printed as one JSON line
    per prompt): that rule in bf16, where two of torch's own backends already fail it, the same
    comparison between torch's default and math SDPA backends, and both paths (ours, torch's default)
    against the model with float32 attention."""
    import json

    print(f"[ttft] building the 28-layer Qwen2.5-1.5B-architecture model ({dtype})", flush=True)
    model = ttft_qwen.build_model(seed=0, dtype=dtype)
    assert model.config.num_hidden_layers == 28 and model.config.vocab_size == 151936
    layers = model.config.num_hidden_layers
    bound = 3e-2 if dtype == torch.bfloat16 else 2e-2
    # fp16 adds the reference's 64k prompt (README.md:42-44); its math / fp32 yardsticks are skipped there
    for S in ((4096, 16384, 65536) if dtype == torch.float16 else (4096, 16384)):
        print(f"[ttft] full prefill S={S} {dtype}", flush=True)
        ids = ttft_qwen.make_prompt(S, model.config.vocab_size, seed=S)
        cap = ttft_qwen.SdpaCapture(calls=(0, layers // 2, layers - 1))
        check = ttft_qwen.verify_against_torch(model, ids, capture=cap)
        layer_err = {i: _layer_rows_vs_oracle(cap.records[i], seed=S + i) for i in cap.calls}
        print("[ttft] " + json.dumps({"prompt_len": S, "dtype": str(dtype), "layer_max_abs_vs_oracle": layer_err,
                                      **check}), flush=True)
        del cap
        torch.cuda.empty_cache()
        assert check["kernel_calls"] == layers
        assert all(err <= bound for err in layer_err.values()), layer_err
        assert check["argmax_match"], check
        if dtype == torch.float16:
            assert check["passed"], check
