"""Persisted tuning table (the gfx950 replacement for the reference's untimed candidate ranking,
tuner.py:489-560 and mma.py:63-81): the committed table only names built tiles, selection honours
it, a missing table falls back to the preference order, and on the GPU a small live sweep writes
entries that selection then returns."""
from __future__ import annotations

import json

import pytest
import torch

import gfx950_configs as cfgs
import gfx950_tune
import hip_lib
import mma

_DTYPES = {"f16": torch.float16, "bf16": torch.bfloat16}


def _parse_fa_key(key: str):
    v, dt, d, c, bh, m, n = key.split("|")
    return int(v[1:]), _DTYPES[dt], int(d[1:]), bool(int(c[1:])), int(bh[2:]), int(m[1:]), int(n[1:])


@pytest.fixture
def fresh_table_cache():
    cfgs.reset_tune_table_cache()
    yield
    cfgs.reset_tune_table_cache()


def test_committed_table_names_only_built_tiles(fresh_table_cache):
    table = cfgs.load_tune_table()
    assert table["fa"] and table["gemm"], "tune_table.json is missing or empty"
    for key, entry in table["fa"].items():
        variant, dtype, D, _causal, _bh, _m, _n = _parse_fa_key(key)
        tiles = {(c.block_m, c.block_n, c.waves, c.stages) for c in cfgs.fa_candidates(variant, dtype, D)}
        assert tuple(entry["tile"]) in tiles, key
        # the winner is the fastest of the re-timed top candidates (their interleaved medians), or
        # of the single pass when nothing was re-timed
        timed = entry.get("refined") or entry["timed"]
        best = "x".join(map(str, entry["tile"]))
        assert timed[best] == entry["ms"] == min(timed.values()), key
        if "refined" in entry:  # the re-timed ones are the fastest of the first pass
            first = entry["timed"]
            cut = max(first[k] for k in entry["refined"])
            assert len(entry["refined"]) == min(gfx950_tune.REFINE_TOP, len(first)), key
            assert all(first[k] >= cut for k in first if k not in entry["refined"]), key
    gemm_tiles = set(cfgs.gemm_candidates())
    for key, entry in table["gemm"].items():
        assert tuple(entry["tile"]) in gemm_tiles, key
        assert entry["group_m"] in gfx950_tune.GROUP_MS
        assert entry["ms"] == min((entry.get("refined") or entry["timed"]).values()), key


def test_selection_returns_the_table_winner(fresh_table_cache):
    table = cfgs.load_tune_table()
    for key, entry in table["fa"].items():
        variant, dtype, D, causal, bh, m, n = _parse_fa_key(key)
        cands = cfgs.fa_candidates(variant, dtype, D)
        got = cfgs.choose_fa_tile(variant, dtype, D, causal, 1, bh, m, n, cands)
        assert [got.block_m, got.block_n, got.waves, got.stages] == entry["tile"], key
    for key, entry in table["gemm"].items():
        M, N, K = (int(p[1:]) for p in key.split("|"))
        try:
            bm, bn, bk, waves, gm = cfgs.choose_gemm_tile(M, N, K)
        except ValueError:
            continue
        assert [bm, bn, bk, waves] == entry["tile"] and gm == entry["group_m"], key
        # the drop-in selector reports the same tile (reference tuple order)
        assert mma._select_2d_contiguous_config(M, N, K)[:4] == (bm, bn, bk, gm)


def test_table_timed_every_current_candidate(fresh_table_cache):
    """Each entry was swept with every tile the library now builds for its (variant, dtype, D):
    a table older than a newly built tile would never select it."""
    table = cfgs.load_tune_table()
    for key, entry in table["fa"].items():
        variant, dtype, D, _causal, _bh, _m, _n = _parse_fa_key(key)
        built = {f"{c.block_m}x{c.block_n}x{c.waves}x{c.stages}" for c in cfgs.fa_candidates(variant, dtype, D)}
        assert built <= set(entry["timed"]), (key, sorted(built - set(entry["timed"])))
    for key, entry in table["gemm"].items():
        M, N, K = (int(p[1:]) for p in key.split("|"))
        built = {f"{t[0]}x{t[1]}x{t[2]}x{t[3]}g{gm}" for t in cfgs.gemm_candidates()
                 if M % t[0] == 0 and N % t[1] == 0 and K % t[2] == 0 for gm in gfx950_tune.GROUP_MS}
        assert built <= set(entry["timed"]), (key, sorted(built - set(entry["timed"])))


def test_selected_tiles_do_not_spill(fresh_table_cache):
    """Every kernel the table selects (and, for the sliced variant, its split instantiation)
    compiles without scratch: a spill inside the KV loop costs HBM traffic on every step."""
    table = cfgs.load_tune_table()
    for key, entry in table["fa"].items():
        variant, dtype, D, _causal, _bh, _m, _n = _parse_fa_key(key)
        for splits in ((1, 2) if variant == hip_lib.FA_VARIANT_SLICED else (1,)):
            res = cfgs.fa_resources(variant, dtype, D, cfgs.FaTileChoice(*entry["tile"], splits))
            assert res is not None, (key, splits)
            assert res["scratch_bytes_per_lane"] == 0, (key, splits, res)
    for key, entry in table["gemm"].items():
        res = cfgs.gemm_resources(tuple(entry["tile"]))
        assert res is not None and res["scratch_bytes_per_lane"] == 0, (key, res)


def test_shapes_in_one_bucket_share_an_entry():
    k1 = cfgs.fa_table_key(hip_lib.FA_VARIANT_OPT, torch.float16, 128, False, 4, 32, 8192, 8192)
    k2 = cfgs.fa_table_key(hip_lib.FA_VARIANT_OPT, torch.float16, 128, False, 2, 64, 5000, 7000)
    k3 = cfgs.fa_table_key(hip_lib.FA_VARIANT_OPT, torch.float16, 128, True, 4, 32, 8192, 8192)
    assert k1 == k2 != k3
    assert cfgs.gemm_table_key(8192, 8192, 8192) == cfgs.gemm_table_key(5000, 8000, 4097)


def test_missing_table_falls_back_to_preference_order(tmp_path, monkeypatch, fresh_table_cache):
    monkeypatch.setattr(cfgs, "TUNE_TABLE_PATH", tmp_path / "absent.json")
    cands = cfgs.fa_candidates(hip_lib.FA_VARIANT_BASIC, torch.float16, 128)
    got = cfgs.choose_fa_tile(hip_lib.FA_VARIANT_BASIC, torch.float16, 128, False, 4, 32, 8192, 8192, cands)
    assert got == cands[0]
    assert cfgs.choose_gemm_tile(8192, 8192, 8192) == (*cfgs.gemm_candidates()[0], cfgs.GEMM_DEFAULT_GROUP_M)


def test_shape_without_bucket_takes_nearest_swept_bucket(tmp_path, monkeypatch, fresh_table_cache):
    """A shape whose bucket was not swept (the reference's B=1 H=28 pipeline cases) runs the tile
    of the nearest swept bucket of the same variant, dtype, head dim and causality; with no such
    bucket it falls back to the preference order."""
    opt, f16 = hip_lib.FA_VARIANT_OPT, torch.float16
    near = cfgs.fa_table_key(opt, f16, 128, False, 4, 32, 8192, 8192)   # BH128 M8192 N8192
    far = cfgs.fa_table_key(opt, f16, 128, False, 1, 4, 512, 512)       # BH4 M512 N512
    path = tmp_path / "t.json"
    path.write_text(json.dumps({"fa": {near: {"tile": [128, 64, 4, 7]}, far: {"tile": [128, 64, 4, 5]}}, "gemm": {}}))
    monkeypatch.setattr(cfgs, "TUNE_TABLE_PATH", path)
    cands = cfgs.fa_candidates(opt, f16, 128)
    got = cfgs.choose_fa_tile(opt, f16, 128, False, 1, 28, 8192, 8192, cands)   # BH32: 2 octaves from `near`
    assert (got.block_m, got.block_n, got.waves, got.stages) == (128, 64, 4, 7)
    got = cfgs.choose_fa_tile(opt, f16, 128, False, 1, 4, 700, 700, cands)      # next to `far`
    assert (got.block_m, got.block_n, got.waves, got.stages) == (128, 64, 4, 5)
    # causal (or another dtype / head dim) has no swept bucket here: preference order
    assert cfgs.choose_fa_tile(opt, f16, 128, True, 1, 28, 8192, 8192, cands) == cands[0]
    assert cfgs.choose_fa_tile(opt, torch.bfloat16, 128, False, 1, 28, 8192, 8192,
                               cfgs.fa_candidates(opt, torch.bfloat16, 128)) == cfgs.fa_candidates(opt, torch.bfloat16, 128)[0]


def test_gemm_shape_without_bucket_takes_nearest_swept_bucket(tmp_path, monkeypatch, fresh_table_cache):
    """A GEMM shape between the swept buckets runs the winner of the nearest one (sum of |log2|
    distances in M, N, K); when that winner does not divide the shape, the fastest tile it timed
    that does."""
    small, big = cfgs.gemm_table_key(1024, 1024, 1024), cfgs.gemm_table_key(8192, 8192, 8192)
    path = tmp_path / "t.json"
    path.write_text(json.dumps({"fa": {}, "gemm": {
        small: {"tile": [128, 64, 32, 4], "group_m": 8,
                "timed": {"128x64x32x4g8": 0.0106, "128x128x32x4g4": 0.0107, "256x256x64x8g8": 0.0231}},
        big: {"tile": [256, 256, 64, 8], "group_m": 8, "timed": {"256x256x64x8g8": 0.8, "128x128x32x4g4": 1.1}},
    }}))
    monkeypatch.setattr(cfgs, "TUNE_TABLE_PATH", path)
    # 1024x4096x1024: two octaves from `small`, five from `big`
    assert cfgs.choose_gemm_tile(1024, 4096, 1024) == (128, 64, 32, 4, 8)
    assert cfgs.choose_gemm_tile(16384, 8192, 4096) == (256, 256, 64, 8, 8)
    # N = 1152 (bucket 2048) is nearest `small`, whose winner 128x64 divides it
    assert cfgs.choose_gemm_tile(1024, 1152, 1024) == (128, 64, 32, 4, 8)
    # M = 1152 (bucket 2048) with N = K = 8192 is nearest `big`, whose winner 256x256 does not
    # divide M: the next tile `big` timed, 128x128 with its GROUP_M, does
    assert cfgs.choose_gemm_tile(1152, 8192, 8192) == (128, 128, 32, 4, 4)
    # ragged shapes take the same ranking without the divisibility filter
    assert cfgs.choose_gemm_tile_any(1000, 4000, 1000)[:4] == (128, 64, 32, 4)


def test_table_entry_for_unbuilt_tile_is_ignored(tmp_path, monkeypatch, fresh_table_cache):
    key = cfgs.fa_table_key(hip_lib.FA_VARIANT_OPT, torch.float16, 128, False, 4, 32, 8192, 8192)
    path = tmp_path / "t.json"
    path.write_text(json.dumps({"fa": {key: {"tile": [512, 512, 16]}},
                                "gemm": {cfgs.gemm_table_key(8192, 8192, 8192): {"tile": [1, 2, 3, 4], "group_m": 4}}}))
    monkeypatch.setattr(cfgs, "TUNE_TABLE_PATH", path)
    cands = cfgs.fa_candidates(hip_lib.FA_VARIANT_OPT, torch.float16, 128)
    assert cfgs.choose_fa_tile(hip_lib.FA_VARIANT_OPT, torch.float16, 128, False, 4, 32, 8192, 8192, cands) == cands[0]
    assert cfgs.choose_gemm_tile(8192, 8192, 8192)[:4] == cfgs.gemm_candidates()[0]


def test_sliced_candidates_have_split_kernels():
    for dtype in (torch.float16, torch.bfloat16):
        for D in (64, 128, 256):
            for c in cfgs.fa_candidates(hip_lib.FA_VARIANT_SLICED, dtype, D):
                split = cfgs.FaTileChoice(c.block_m, c.block_n, c.waves, c.stages, 4).to_c()
                assert hip_lib.fa_fwd_supported(hip_lib.FA_VARIANT_SLICED, dtype, D, split), (dtype, D, c)


@pytest.mark.gpu
def test_live_sweep_writes_selectable_entries(gpu, tmp_path, monkeypatch, fresh_table_cache):
    print("[tune] live sweep: fp16 D=64 B1 H4 N=512, gemm 256x256x256", flush=True)
    table = {"fa": {}, "gemm": {}}
    sweep = [("t", torch.float16, 1, 4, 4, 512, 512, 64, False, ("basic", "sliced"))]
    gfx950_tune.tune_attention(table, sweep=sweep, warmup=1, iters=2, log=lambda m: None)
    gfx950_tune.tune_gemm(table, sweep=[(256, 256, 256)], warmup=1, iters=2, log=lambda m: None)
    assert len(table["fa"]) == 2 and len(table["gemm"]) == 1
    path = tmp_path / "t.json"
    path.write_text(json.dumps(table))
    monkeypatch.setattr(cfgs, "TUNE_TABLE_PATH", path)
    for key, entry in table["fa"].items():
        variant, dtype, D, causal, bh, m, n = _parse_fa_key(key)
        got = cfgs.choose_fa_tile(variant, dtype, D, causal, 1, bh, m, n, cfgs.fa_candidates(variant, dtype, D))
        assert [got.block_m, got.block_n, got.waves, got.stages] == entry["tile"]
    assert list(cfgs.choose_gemm_tile(256, 256, 256)[:4]) == table["gemm"][cfgs.gemm_table_key(256, 256, 256)]["tile"]


def test_case_log_lines_parse_like_the_reference_log():
    """case_log.py writes the `[case]` layout the reference's pipeline-log parser reads
    (test_flash_atten.py:270-305): shape fields, then `<series> ... mean=<ms>ms` per series, n/a for
    series that did not run. The two patterns below are that parser's, applied to our line."""
    import re

    import case_log

    stats = {"triton_flash_basic": {"mean_ms": 1.5, "p50_ms": 1.4},
             "triton_flash_opt_shared_mem": {"mean_ms": 1.25, "p50_ms": 1.2},
             "triton_flash_block_d_nomask": {"mean_ms": 1.0, "p50_ms": 0.9},
             "gpu_flash_sdpa": {"mean_ms": 2.5, "p50_ms": 2.4}}
    line = case_log.format_case_line((1, 28, 128, 8192, False), stats,
                                     {"gpu_math_sdpa": "skipped(size)", "triton_flash_basic": "max_abs_diff=1.00e-03"})
    assert line.startswith("[case]")
    shape = re.search(r"\bB=(\d+)\s+H=(\d+)\s+S=(\d+)\s+D=(\d+)\s+causal=(True|False)\b", line)
    assert shape.groups() == ("1", "28", "8192", "128", "False")
    got = {}
    for name in case_log.SERIES:
        m = re.search(rf"(?:^|\|\s*){re.escape(name)}(?:\s+[^|]*?)?\s+mean=(n/a|[0-9.]+)ms\b", line)
        got[name] = None if m is None or m.group(1) == "n/a" else float(m.group(1))
    assert got == {"cpu_sdpa": None, "gpu_math_sdpa": None, "gpu_efficient_sdpa": None, "gpu_flash_sdpa": 2.5,
                   "triton_flash_basic": 1.5, "triton_flash_opt_shared_mem": 1.25, "triton_flash_block_d_nomask": 1.0}
