"""Host logic of the drop-in surface (no GPU): tune-argument validation, tuner validation, launch
layouts, config selection, resource errors, and the resource report. Restates the reference's
rules (tuner.py:72-157, 252-339, 563-590, 597-734; mma.py:63-81; exceptions.py:633-757)."""
from __future__ import annotations

import itertools

import pytest
import torch

import exceptions
import flash_atten
import gfx950_configs as cfgs
import hip_lib
import mma
import tuner
from tuner import (
    FlashAttenTuneArguments,
    FlashAttentionBlockDNomaskTuner,
    FlashAttentionOptimizeSharedMemTuner,
    FlashAttentionTuner,
)

# ---- FlashAttenTuneArguments (tuner.py:82-108) ----------------------------------------------------


@pytest.mark.parametrize(
    "kwargs,message",
    [
        ({"BLOCK_N": 0}, "BLOCK_N must be positive when provided"),
        ({"BLOCK_M": -4}, "BLOCK_M must be positive when provided"),
        ({"BLOCK_M": 96}, "BLOCK_M must be a power of 2 when provided"),
        ({"BLOCK_N_PAD": 0}, "BLOCK_N_PAD must be positive when provided"),
        ({"BLOCK_N_PAD": 48}, "BLOCK_N_PAD must be a power of 2 when provided"),
        ({"BLOCK_DMODEL": 0}, "BLOCK_DMODEL must be positive when provided"),
        ({"BLOCK_DMODEL": 80}, "BLOCK_DMODEL must be a power of 2 when provided"),
        ({"BLOCK_DMODEL_OUTER": -1}, "BLOCK_DMODEL_OUTER must be positive when provided"),
        ({"BLOCK_DMODEL_OUTER": 24}, "BLOCK_DMODEL_OUTER must be a power of 2 when provided"),
        ({"NUM_WARPS": 0}, "NUM_WARPS must be positive when provided"),
        ({"NUM_STAGES": 0}, "NUM_STAGES must be positive when provided"),
    ],
)
def test_tune_argument_validation(kwargs, message):
    with pytest.raises(ValueError, match=message):
        FlashAttenTuneArguments(**kwargs)


def test_tune_arguments_accept_non_power_of_two_block_n():
    assert FlashAttenTuneArguments(BLOCK_N=48).BLOCK_N == 48  # only BLOCK_N skips the power-of-2 rule


# ---- tuner constructor (tuner.py:132-157) ----------------------------------------------------------

Q = (1, 4, 256, 64)


@pytest.mark.parametrize(
    "shapes,tune,message",
    [
        (((1, 4, 256), Q, Q), None, "must all be 4D"),
        ((Q, (2, 4, 256, 64), Q), None, "Batch and head dimensions must match"),
        ((Q, (1, 3, 256, 64), (1, 3, 256, 64)), None, "Batch and head dimensions must match"),
        ((Q, (1, 2, 256, 64), (1, 4, 256, 64)), None, "Batch and head dimensions must match"),
        ((Q, (1, 4, 256, 32), Q), None, "Last dimension must match"),
        ((Q, (1, 4, 128, 64), Q), None, "sequence lengths must match"),
        ((Q, Q, Q), FlashAttenTuneArguments(BLOCK_DMODEL=32), "BLOCK_DMODEL must be >= D"),
        ((Q, Q, Q), FlashAttenTuneArguments(BLOCK_N=128, BLOCK_N_PAD=64), "BLOCK_N cannot exceed BLOCK_N_PAD"),
        ((Q, Q, Q), FlashAttenTuneArguments(NUM_WARPS=64), "NUM_WARPS must be <= 16"),
    ],
)
def test_tuner_validation(shapes, tune, message):
    with pytest.raises(ValueError, match=message):
        FlashAttentionTuner(*shapes, 2, causal=False, return_lse=False, tune_args=tune)


def test_gqa_shapes_accepted_and_sliced_allows_small_block_dmodel():
    FlashAttentionTuner(Q, (1, 2, 300, 64), (1, 2, 300, 64), 2, causal=True, return_lse=True)
    FlashAttentionBlockDNomaskTuner(Q, Q, Q, 2, causal=False, return_lse=False,
                                    tune_args=FlashAttenTuneArguments(BLOCK_DMODEL=32))


# ---- launch layouts (tuner.py:264-305, 639-658) ------------------------------------------------------


def _cpu_qkv(B=1, H=4, M=256, N=256, D=64, Hkv=None, dtype=torch.float16):
    Hkv = H if Hkv is None else Hkv
    return (torch.zeros(B, H, M, D, dtype=dtype), torch.zeros(B, Hkv, N, D, dtype=dtype),
            torch.zeros(B, Hkv, N, D, dtype=dtype))


@pytest.mark.parametrize("cls", [FlashAttentionTuner, FlashAttentionOptimizeSharedMemTuner])
@pytest.mark.parametrize("return_lse", [False, True])
def test_strided_launch_layout(cls, return_lse):
    q, k, v = _cpu_qkv()
    spec = cls(tuple(q.shape), tuple(k.shape), tuple(v.shape), 2, causal=True, return_lse=return_lse
               ).build_flash_attention_launch_spec(q, k, v)
    assert spec.function_name == cls.KERNEL_NAME
    assert len(spec.kernel_args) == 29
    assert spec.kernel_args[24:28] == (4, 256, 256, 64)
    assert spec.kernel_args[28] == pytest.approx(64 ** -0.5)
    assert spec.kernel_args[5:9] == q.stride()
    assert isinstance(spec.kernel_args[4], torch.Tensor) == return_lse
    assert set(spec.kernel_kwargs) == {"causal", "HAS_LSE", "BLOCK_M", "BLOCK_N", "BLOCK_N_PAD", "BLOCK_DMODEL",
                                       "num_warps", "num_stages"}
    assert spec.kernel_kwargs["causal"] is True and spec.kernel_kwargs["HAS_LSE"] is return_lse
    assert spec.grid == (-(-256 // spec.kernel_kwargs["BLOCK_M"]), 4)
    assert spec.tune_args.BLOCK_M == spec.kernel_kwargs["BLOCK_M"]
    assert spec.input_shapes["q"] == (1, 4, 256, 64)
    assert spec.input_shapes["lse"] == ((1, 4, 256) if return_lse else None)
    ctx = spec.launch_context
    assert ctx["compiled_shared_memory_bytes_per_block"] <= ctx["available_shared_memory_bytes_per_sm"]


def test_sliced_launch_layout_and_update_data():
    q, k, v = _cpu_qkv(M=128, N=512, D=128, Hkv=2)
    spec = FlashAttentionBlockDNomaskTuner(tuple(q.shape), tuple(k.shape), tuple(v.shape), 2, causal=False,
                                           return_lse=False).build_flash_attention_launch_spec(q, k, v, sm_scale=0.5)
    assert len(spec.kernel_args) == 9
    assert spec.kernel_args[4:] == (4, 128, 512, 128, 0.5)
    assert {"BLOCK_M", "BLOCK_N", "BLOCK_DMODEL", "BLOCK_DMODEL_OUTER", "num_warps", "num_stages"} <= set(
        spec.kernel_kwargs)
    o = spec.kernel_args[3]
    q2, k2, v2 = _cpu_qkv(M=128, N=512, D=128, Hkv=2)
    spec.update_data((q2, k2, v2))
    assert spec.kernel_args[0] is q2 and spec.kernel_args[3] is o  # o reused (tuner.py:56-69)
    assert spec.launch_context["kv_splits"] == spec.kernel_kwargs["SPLITS"]


def test_config_cache_is_per_class_and_reused():
    q, k, v = _cpu_qkv()
    a = FlashAttentionTuner(tuple(q.shape), tuple(k.shape), tuple(v.shape), 2, causal=False, return_lse=False)
    spec1 = a.build_flash_attention_launch_spec(q, k, v)
    spec2 = a.build_flash_attention_launch_spec(q, k, v)
    assert spec1.kernel_kwargs == spec2.kernel_kwargs
    b = FlashAttentionOptimizeSharedMemTuner(tuple(q.shape), tuple(k.shape), tuple(v.shape), 2, causal=False,
                                             return_lse=False)
    assert b._cache_key(q) != a._cache_key(q)


def test_tune_args_are_hints_with_recorded_relaxation():
    q, k, v = _cpu_qkv(D=128)
    ta = FlashAttenTuneArguments(BLOCK_N=64, BLOCK_M=128, BLOCK_N_PAD=64, BLOCK_DMODEL=128, NUM_WARPS=8,
                                 NUM_STAGES=1)
    spec = FlashAttentionTuner(tuple(q.shape), tuple(k.shape), tuple(v.shape), 2, causal=False, return_lse=False,
                               tune_args=ta).build_flash_attention_launch_spec(q, k, v)
    assert spec.kernel_kwargs["BLOCK_M"] == 128 and spec.kernel_kwargs["BLOCK_N"] == 64
    assert spec.kernel_kwargs["num_stages"] == 1
    assert "NUM_WARPS" in spec.launch_context.get("tune_args_relaxed", "")


def test_unknown_kernel_name_raises_name_error():
    q, k, v = _cpu_qkv()
    spec = FlashAttentionTuner(tuple(q.shape), tuple(k.shape), tuple(v.shape), 2, causal=False,
                               return_lse=False).build_flash_attention_launch_spec(q, k, v)
    bad = tuner.FlashAttentionLaunchSpec(grid=spec.grid, kernel_args=spec.kernel_args,
                                         kernel_kwargs=spec.kernel_kwargs, launch_context={},
                                         function_name="_no_such_kernel", tune_args=spec.tune_args,
                                         input_shapes=spec.input_shapes)
    with pytest.raises(NameError, match="No such kernel named _no_such_kernel"):
        flash_atten.flash_attention(bad)


def test_unsupported_head_dim_and_dtype():
    q, k, v = _cpu_qkv(D=96)
    with pytest.raises(ValueError, match="not built"):
        FlashAttentionTuner(tuple(q.shape), tuple(k.shape), tuple(v.shape), 2, causal=False,
                            return_lse=False).build_flash_attention_launch_spec(q, k, v)
    q, k, v = _cpu_qkv(dtype=torch.float32)
    with pytest.raises(ValueError, match="dtype"):
        FlashAttentionTuner(tuple(q.shape), tuple(k.shape), tuple(v.shape), 4, causal=False,
                            return_lse=False).build_flash_attention_launch_spec(q, k, v)


# ---- resource errors are host-forcible (exceptions.py:695-757, tuner.py:519-554) -------------------------


def _fake_limits(lds):
    def provider():
        lim = exceptions.gfx950_static_limits()
        lim["available_shared_memory_bytes_per_sm"] = lds
        return lim

    return provider


def test_out_of_resources_with_detail_when_lds_too_small():
    exceptions.set_device_limits_provider(_fake_limits(1024))
    FlashAttentionTuner._config_cache.clear()  # the class cache is keyed on shapes, not limits
    try:
        q, k, v = _cpu_qkv()
        with pytest.raises(exceptions.OutOfResourcesWithDetail) as info:
            FlashAttentionTuner(tuple(q.shape), tuple(k.shape), tuple(v.shape), 2, causal=False,
                                return_lse=False).build_flash_attention_launch_spec(q, k, v)
        err = info.value
        assert err.name == "shared memory" and err.limit == 1024 and err.required > 1024
        assert err.kernel_name == "_flash_attn_fwd_kernel_basic"
        text = str(err)
        assert "Kernel: _flash_attn_fwd_kernel_basic." in text and "LDS" in text
    finally:
        exceptions.set_device_limits_provider(None)
        FlashAttentionTuner._config_cache.clear()


def test_out_of_resources_registers_when_register_file_too_small():
    def provider():
        lim = exceptions.gfx950_static_limits()
        lim["vgprs_per_simd_lane"] = 64
        return lim

    exceptions.set_device_limits_provider(provider)
    FlashAttentionTuner._config_cache.clear()
    try:
        q, k, v = _cpu_qkv()
        with pytest.raises(exceptions.OutOfResourcesWithDetail) as info:
            FlashAttentionOptimizeSharedMemTuner(tuple(q.shape), tuple(k.shape), tuple(v.shape), 2, causal=False,
                                                 return_lse=False).build_flash_attention_launch_spec(q, k, v)
        assert info.value.name == "registers"
    finally:
        exceptions.set_device_limits_provider(None)
        FlashAttentionTuner._config_cache.clear()


def test_out_of_resources_from_base_and_pickle():
    import pickle

    base = exceptions.OutOfResources(10, 5, "shared memory")
    detail = exceptions.OutOfResourcesWithDetail.from_out_of_resources(base, kernel_name="k",
                                                                       launch_context={"a": 1})
    assert detail.original_exception is base and detail.launch_context == {"a": 1}
    assert pickle.loads(pickle.dumps(base)).required == 10


def test_resource_usage_summary_format():
    ctx = {"compiled_shared_memory_bytes_per_block": 100, "available_shared_memory_bytes_per_sm": 200,
           "attempted_register_file_size_bytes_per_block": 3, "available_register_file_size_bytes_per_sm": 4,
           "attempted_registers_per_block": 5, "available_registers_per_sm": 6}
    text = exceptions._resource_usage_summary("kern", ctx, tune_args=FlashAttenTuneArguments(BLOCK_M=64),
                                               input_shapes={"q": (1, 2), "lse": None})
    assert text.startswith("kern tuner resources: \nshared=100/200 bytes per block/SM, ")
    assert "register_file=3/4" in text and "registers=5/6" in text
    assert "tune_args=BLOCK_M=64" in text and "input_shapes=q=(1, 2)" in text
    assert exceptions._format_tune_args(None) is None and exceptions._format_input_shapes({"x": None}) is None


# ---- GEMM config selection (mma.py:63-81) ----------------------------------------------------------


def _reference_accepts(m, n, k):
    if k % 32:
        return False
    return (m % 128 == 0 and n % 64 == 0) or (m % 64 == 0 and n % 256 == 0)


def test_gemm_selector_accepts_exactly_the_reference_shapes():
    sizes = [64, 96, 128, 192, 256, 320, 512, 768, 1024]
    for m, n, k in itertools.product(sizes, sizes, [32, 48, 64, 256]):
        if _reference_accepts(m, n, k):
            bm, bn, bk, group_m, warps, stages = mma._select_2d_contiguous_config(m, n, k)
            assert m % bm == 0 and n % bn == 0 and k % bk == 0 and group_m >= 1 and stages == 2
        else:
            with pytest.raises(ValueError):
                mma._select_2d_contiguous_config(m, n, k)


def test_gemm_selector_prefers_large_tiles_and_hints():
    assert mma._select_2d_contiguous_config(8192, 8192, 8192)[:3] in [(256, 256, 64), (256, 256, 32),
                                                                     (256, 128, 64), (128, 256, 64)]
    assert cfgs.choose_gemm_tile(1024, 1024, 256, hint=(128, 128, 64))[:3] == (128, 128, 64)
    # block sizes + wave count narrow the candidates; a wave count that is not built keeps the sizes
    assert cfgs.choose_gemm_tile(8192, 8192, 8192, hint=(256, 256, 64, 4))[:4] == (256, 256, 64, 4)
    assert cfgs.choose_gemm_tile(8192, 8192, 8192, hint=(256, 256, 64, 8))[:4] == (256, 256, 64, 8)
    assert cfgs.choose_gemm_tile(8192, 8192, 8192, hint=(256, 256, 64, 2))[:3] == (256, 256, 64)


def test_gemm_launch_hints_keep_the_tuned_tile():
    """BLOCK_* hints equal to the tuned tile's sizes (what _select_2d_contiguous_config returns and
    test_mma.py passes back) must launch the tuned tile, wave count included."""
    bm, bn, bk, group_m, warps, _ = mma._select_2d_contiguous_config(8192, 8192, 8192)
    assert cfgs.choose_gemm_tile(8192, 8192, 8192, hint=(bm, bn, bk))[:4] == (bm, bn, bk, warps)
    assert cfgs.choose_gemm_tile(8192, 8192, 8192, hint=(bm, bn, bk, warps))[:4] == (bm, bn, bk, warps)


def test_cache_eviction_hint_false_without_gpu():
    assert mma._supports_contiguous_cache_eviction_hints() is torch.cuda.is_available()


# ---- gfx950 selection helpers ---------------------------------------------------------------------------


def test_filter_by_hints_relaxes_minimally():
    cands = [cfgs.FaTileChoice(128, 64, 4, 1), cfgs.FaTileChoice(256, 64, 8, 1)]
    got, relaxed = cfgs.filter_by_hints(cands, {"BLOCK_M": 128, "NUM_WARPS": 8, "NUM_STAGES": 1})
    assert relaxed == ["NUM_WARPS"] and got == [cands[0]]
    got, relaxed = cfgs.filter_by_hints(cands, {"BLOCK_M": 256, "NUM_WARPS": 8})
    assert relaxed == [] and got == [cands[1]]
    got, relaxed = cfgs.filter_by_hints(cands, {"BLOCK_M": 512})
    assert relaxed == ["BLOCK_M"] and got == cands


def test_choose_splits():
    assert cfgs.choose_splits(4, 32, 8192, 8192, 256, 64) == 1  # grid already fills the GPU
    # prefill-shaped grids (full query tiles) split only below a quarter of the CUs
    assert cfgs.choose_splits(1, 12, 4096, 4096, 256, 64) == 1  # 192 workgroups
    assert cfgs.choose_splits(1, 28, 1024, 1024, 128, 64) == 1  # 224 workgroups
    assert cfgs.choose_splits(1, 2, 256, 65536, 256, 64) == cfgs.PREFILL_SPLIT_CUS // 2
    s = cfgs.choose_splits(1, 4, 512, 8192, 128, 64)              # 16 workgroups
    assert s == cfgs.PREFILL_SPLIT_CUS // 16
    # decode-shaped grids (a few rows per tile) split up to the resident capacity
    assert cfgs.choose_splits(1, 1, 1, 100000, 256, 64) == cfgs.MAX_SPLITS
    assert cfgs.choose_splits(8, 32, 1, 32768, 128, 64) == 2  # 256 single-row tiles, 2 per CU
    assert cfgs.choose_splits(1, 1, 64, 128, 256, 64) == 1  # too few KV tiles to split


def test_split_residency_follows_the_resource_table():
    # D=128 4-wave split kernels keep two workgroups per CU; the D=256 pipelined kernel (one wave
    # per SIMD) and 8-wave kernels keep one
    assert cfgs.split_residency(torch.float16, 128, 128, 64, 4, 3) == 2
    assert cfgs.split_residency(torch.bfloat16, 256, 128, 32, 4, 3) == 1
    assert cfgs.split_residency(torch.float16, 128, 256, 128, 8, 2) == 1
    # decode shapes fill the resident capacity: 128 single-row tiles split in two when one split
    # workgroup fits a CU, in four when two do
    assert cfgs.choose_splits(1, 128, 1, 32768, 128, 32, resident_per_cu=1) == 2
    assert cfgs.choose_splits(1, 128, 1, 32768, 128, 32, resident_per_cu=2) == 4


def test_every_candidate_has_compiled_resources():
    for variant in (0, 1, 2):
        for dtype in (torch.float16, torch.bfloat16):
            for D in (64, 128, 256):
                cands = cfgs.fa_candidates(variant, dtype, D)
                assert cands, (variant, dtype, D)
                for c in cands:
                    res = cfgs.fa_resources(variant, dtype, D, c)
                    assert res is not None and res["lds_bytes"] <= 160 * 1024
                    # the resources are those of the candidate's own pipeline
                    sym = hip_lib.fwd_kernel_symbol(variant, dtype, D, c.to_c())
                    if c.stages >= 6:  # the 16x16x32-MFMA kernels: PIPE 0, 1, 2 (stages 6, 7, 8)
                        assert "fa_fwd16_kernel" in sym and f"ELi{c.waves}ELi{c.block_n}ELi{c.stages - 6}ELb" in sym, (
                            sym, c)
                    else:
                        assert f"ELi{c.block_n}ELi{c.stages}ELb" in sym, (sym, c)
    for t in cfgs.gemm_candidates():
        assert cfgs.gemm_resources(t) is not None


def test_refine_reranks_the_top_candidates_by_interleaved_medians(monkeypatch):
    """gfx950_tune._refine re-times only the fastest three of a first pass, in interleaved rounds,
    and ranks them by their medians (a one-pass outlier does not win the table)."""
    import gfx950_tune
    first = {"a": 1.00, "b": 1.01, "c": 1.02, "d": 1.50}
    later = {"a": [1.10, 1.09, 1.11, 1.10, 1.30], "b": [1.00, 1.01, 1.00, 0.99, 1.00], "c": [1.05] * 5}
    calls = []

    def fake_time(fn, warmup, iters, batch_ms=1.0):
        key = fn()
        calls.append(key)
        return later[key][sum(1 for k in calls if k == key) - 1]

    monkeypatch.setattr(gfx950_tune, "_time", fake_time)
    fns = {k: (lambda k=k: k) for k in first}
    refined = gfx950_tune._refine(fns, first)
    assert set(refined) == {"a", "b", "c"} and "d" not in calls
    assert calls[:3] == ["a", "b", "c"]  # interleaved, not candidate after candidate
    assert min(refined, key=refined.get) == "b" and refined["a"] == 1.10
    assert gfx950_tune._refine({"a": fns["a"]}, {"a": 1.0}) == {}
