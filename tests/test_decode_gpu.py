"""Decode-shaped split-KV (small M, long N): the sliced variant with KV splits, where the query
heads of a GQA group are packed into one tile's rows (fa_fwd_pack_group) so K/V are read once per
kv head. Parity against the exact oracle, as the other C-ABI tests."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import flash_atten
import gfx950_configs as cfgs
import hip_lib
import oracle
from helpers import ATOL, make_qkv, max_abs, to_device

F16, BF16 = torch.float16, torch.bfloat16
SLICED = hip_lib.FA_VARIANT_SLICED


def test_pack_rule():
    # packs only split launches, non-causal, grouped, when the whole group fits one tile
    assert hip_lib.pack_group(32, 8, 1, False, 128, 16) == 4
    assert hip_lib.pack_group(32, 8, 32, False, 128, 16) == 4
    assert hip_lib.pack_group(32, 8, 33, False, 128, 16) == 1
    assert hip_lib.pack_group(32, 8, 1, True, 128, 16) == 1
    assert hip_lib.pack_group(32, 8, 1, False, 128, 1) == 1
    assert hip_lib.pack_group(32, 32, 1, False, 128, 16) == 1
    assert hip_lib.pack_group(12, 2, 1, False, 128, 16) == 6
    # the split count then targets the packed grid: one workgroup per (batch, kv head, split)
    s = cfgs.choose_splits(1, 32, 1, 32768, 128, 64, H_kv=8)
    assert s == 64  # 8 packed tiles x 64 splits = 512 workgroups, two per CU
    assert cfgs.choose_splits(1, 32, 1, 32768, 128, 64, H_kv=32) < s
    assert cfgs.choose_splits(1, 12, 1, 32768, 128, 64, H_kv=2) == cfgs.MAX_SPLITS == 128


def _run(q, k, v, *, dtype, tile, splits, causal=False, lse=True):
    dev = "cuda:0"
    qd, kd, vd = (to_device(x, dtype, dev) for x in (q, k, v))
    B, H, M, D = qd.shape
    o = torch.empty_like(qd)
    l = torch.empty((B, H, M), dtype=torch.float32, device=dev) if lse else None
    nbytes = hip_lib.workspace_bytes(B, H, M, D, splits)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes else None
    bm, bn, waves, stages = tile
    hip_lib.fa_fwd(qd, kd, vd, o, l, sm_scale=D ** -0.5, causal=causal, variant=SLICED,
                   tile=hip_lib.make_tile(bm, bn, waves, stages, splits), workspace=ws)
    torch.cuda.synchronize()
    return o.float().cpu().numpy(), (l.cpu().numpy() if lse else None)


DECODE = [
    # name, B, H, Hkv, M, N, D, dtype, tile (bm, bn, waves, stages), splits
    ("llama_m1", 2, 32, 8, 1, 2000, 128, F16, (128, 64, 4, 3), 16),
    ("llama_m4_bf16", 1, 32, 8, 4, 1500, 128, BF16, (128, 64, 4, 3), 8),
    ("qwen_m1", 1, 12, 2, 1, 4096, 128, BF16, (128, 64, 4, 3), 32),
    ("qwen_m7_ragged", 1, 12, 2, 7, 777, 128, F16, (128, 64, 4, 3), 5),
    ("g8_d64", 3, 8, 1, 3, 1000, 64, F16, (128, 64, 4, 3), 6),
    ("w8_tile", 1, 16, 2, 9, 900, 128, BF16, (256, 64, 8, 3), 4),
    ("double_buffered", 2, 32, 8, 2, 1200, 128, F16, (128, 64, 4, 2), 8),
    ("group_exceeds_tile", 1, 16, 1, 9, 640, 64, F16, (128, 64, 4, 3), 4),  # 16*9 > 128: no packing
    # more splits than a wave has lanes: the merge takes split weights 64 at a time; 36 splits empty
    ("many_splits", 1, 8, 2, 1, 8192, 128, BF16, (128, 64, 4, 3), 100),
    ("many_splits_d256", 1, 4, 4, 2, 4000, 256, F16, (128, 32, 4, 3), 70),
    # the 16x16x32 MFMA split kernels (stages 6-9; a stages=9 tile packing query heads runs stages 8)
    ("m16_lean", 1, 32, 8, 1, 8192, 128, BF16, (128, 64, 4, 6), 64),
    ("m16_pipelined_n32", 2, 32, 8, 1, 5000, 128, F16, (128, 32, 4, 7), 48),
    ("m16_ping_pong", 1, 16, 2, 3, 3000, 128, BF16, (256, 64, 8, 8), 16),
    ("m16_persistent_tile", 1, 32, 8, 1, 4096, 128, F16, (256, 64, 8, 9), 32),  # packs: runs stages 8
    ("m16_d256_many_splits", 1, 8, 2, 1, 4000, 256, F16, (128, 32, 4, 6), 70),  # 64+ splits, 7 empty
    ("m16_d64_unpacked", 2, 4, 4, 5, 2500, 64, BF16, (128, 64, 4, 7), 9),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", DECODE, ids=[c[0] for c in DECODE])
def test_decode_split_kv_parity(gpu, case):
    name, B, H, Hkv, M, N, D, dtype, tile, splits = case
    print(f"[decode] {name} B={B} H={H} Hkv={Hkv} M={M} N={N} D={D} {dtype} tile={tile} splits={splits} "
          f"pack={hip_lib.pack_group(H, Hkv, M, False, tile[0], splits)}", flush=True)
    q, k, v = make_qkv(4000 + len(name), B, H, Hkv, M, N, D, dtype)
    o, lse = _run(q, k, v, dtype=dtype, tile=tile, splits=splits)
    o_ref, lse_ref = oracle.attention(q, k, v, causal=False)
    assert np.isfinite(o).all()
    assert max_abs(o, o_ref) <= ATOL[dtype]
    assert max_abs(lse, lse_ref) <= 1e-3


@pytest.mark.gpu
def test_decode_packed_equals_unpacked(gpu):
    """Packing changes which workgroup computes a row; it matches the same split launch with one
    query head per kv head (H_kv = H, K/V expanded) up to the rounding of P (the lazy-rescale
    offset is decided per wave, and a wave now holds rows of several heads)."""
    B, H, Hkv, M, N, D = 1, 32, 8, 2, 3000, 128
    print("[decode] packed vs expanded", flush=True)
    q, k, v = make_qkv(4242, B, H, Hkv, M, N, D, F16)
    ke, ve = (np.repeat(x, H // Hkv, axis=1) for x in (k, v))
    o1, l1 = _run(q, k, v, dtype=F16, tile=(128, 64, 4, 3), splits=16)
    o2, l2 = _run(q, ke, ve, dtype=F16, tile=(128, 64, 4, 3), splits=16)
    assert hip_lib.pack_group(H, Hkv, M, False, 128, 16) == 4 and hip_lib.pack_group(H, H, M, False, 128, 16) == 1
    assert max_abs(o1, o2) <= 2e-3
    assert max_abs(l1, l2) <= 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 3])
def test_decode_through_sdpa_entry(gpu, M):
    """flash_atten.sdpa (sliced) picks the split count and packing itself."""
    B, H, Hkv, N, D = 2, 12, 2, 5000, 128
    print(f"[decode] sdpa entry M={M}", flush=True)
    q, k, v = make_qkv(77 + M, B, H, Hkv, M, N, D, BF16)
    qd, kd, vd = (to_device(x, BF16, "cuda:0") for x in (q, k, v))
    out = flash_atten.sdpa(qd, kd, vd, is_causal=False, scale=D ** -0.5, variant="sliced")
    torch.cuda.synchronize()
    o_ref, _ = oracle.attention(q, k, v, causal=False)
    assert max_abs(out.float().cpu().numpy(), o_ref) <= ATOL[BF16]


@pytest.mark.gpu
def test_decode_step_replays_in_a_hip_graph(gpu):
    """A decode step (split pass + merge pass, workspace from torch's allocator) captured in a HIP
    graph replays correctly: between replays the query changes in place (eager work on the same
    stream), and every replay must match an eager call on the new query."""
    B, H, Hkv, M, N, D = 1, 32, 8, 1, 6000, 128
    print("[decode] HIP graph capture and replays", flush=True)
    q, k, v = make_qkv(9090, B, H, Hkv, M, N, D, BF16)
    qd, kd, vd = (to_device(x, BF16, "cuda:0") for x in (q, k, v))

    def step():
        return flash_atten.sdpa(qd, kd, vd, is_causal=False, scale=D ** -0.5, variant="sliced")

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    g = torch.Generator().manual_seed(5)
    for rep in range(4):
        qd.copy_(torch.randn(qd.shape, generator=g).to(BF16))
        eager = step()
        graph.replay()
        torch.cuda.synchronize()
        diff = (out.float() - eager.float()).abs().max().item()
        assert diff == 0.0, (rep, diff)
    o_ref, _ = oracle.attention(qd.float().cpu().numpy(), k, v, causal=False)
    assert max_abs(out.float().cpu().numpy(), o_ref) <= ATOL[BF16]


def _garbage(nbytes, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 256, (nbytes,), generator=g, dtype=torch.uint8).to("cuda:0")


@pytest.mark.gpu
@pytest.mark.parametrize("stages", [6, 7, 8])
def test_split_workspace_needs_no_clearing(gpu, stages):
    """A workspace of random bytes (never cleared), reused by calls with other split counts (so
    each call's partials overlay another layout's), must give the oracle's result every time, and
    a repeated call the same bits."""
    B, H, Hkv, M, N, D, dtype = 2, 16, 4, 2, 4500, 128, F16
    bm, bn, waves = (256, 64, 8) if stages == 8 else (128, 64, 4)
    print(f"[decode] stale workspace reused across split counts, stages={stages}", flush=True)
    q, k, v = make_qkv(606 + stages, B, H, Hkv, M, N, D, dtype)
    qd, kd, vd = (to_device(x, dtype, "cuda:0") for x in (q, k, v))
    o_ref, lse_ref = oracle.attention(q, k, v, causal=False)
    ws = _garbage(max(hip_lib.workspace_bytes(B, H, M, D, s) for s in (24, 7, 70)), 31 + stages)
    first = None
    for splits in (24, 7, 70, 24):
        o = torch.full_like(qd, float("nan"))
        lse = torch.full((B, H, M), float("nan"), dtype=torch.float32, device="cuda:0")
        hip_lib.fa_fwd(qd, kd, vd, o, lse, sm_scale=D ** -0.5, causal=False, variant=SLICED,
                       tile=hip_lib.make_tile(bm, bn, waves, stages, splits), workspace=ws)
        torch.cuda.synchronize()
        on, ln = o.float().cpu().numpy(), lse.cpu().numpy()
        assert np.isfinite(on).all() and np.isfinite(ln).all(), splits
        assert max_abs(on, o_ref) <= ATOL[dtype], splits
        assert max_abs(ln, lse_ref) <= 1e-3, splits
        if splits == 24:
            if first is None:
                first = (on, ln)
            else:
                assert np.array_equal(on, first[0]) and np.array_equal(ln, first[1])


@pytest.mark.gpu
@pytest.mark.parametrize("stages", [6, 8])
def test_split_workspace_shared_by_graph_and_eager_calls(gpu, stages):
    """One workspace serves a captured decode step and eager calls in turn: replays right after an
    eager call and back-to-back replays must both match the eager result bit for bit, with the
    query changed in place between rounds."""
    B, H, Hkv, M, N, D, dtype, splits = 1, 32, 8, 1, 6000, 128, BF16, 40
    bm, bn, waves = (256, 64, 8) if stages == 8 else (128, 64, 4)
    print(f"[decode] graph and eager calls on one workspace, stages={stages}", flush=True)
    q, k, v = make_qkv(7070 + stages, B, H, Hkv, M, N, D, dtype)
    qd, kd, vd = (to_device(x, dtype, "cuda:0") for x in (q, k, v))
    ws = _garbage(hip_lib.workspace_bytes(B, H, M, D, splits), 5)
    tile = hip_lib.make_tile(bm, bn, waves, stages, splits)
    o_g, o_e = torch.empty_like(qd), torch.empty_like(qd)
    lse_g = torch.empty((B, H, M), dtype=torch.float32, device="cuda:0")
    lse_e = torch.empty_like(lse_g)

    def call(o, lse):
        hip_lib.fa_fwd(qd, kd, vd, o, lse, sm_scale=D ** -0.5, causal=False, variant=SLICED, tile=tile,
                       workspace=ws)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call(o_g, lse_g)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(o_g, lse_g)
    g = torch.Generator().manual_seed(6)
    for rep in range(3):
        qd.copy_(torch.randn(qd.shape, generator=g).to(dtype))
        call(o_e, lse_e)
        torch.cuda.synchronize()
        for back_to_back in range(2):
            o_g.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(o_g, o_e) and torch.equal(lse_g, lse_e), (rep, back_to_back)
    o_ref, lse_ref = oracle.attention(qd.float().cpu().numpy(), k, v, causal=False)
    assert max_abs(o_g.float().cpu().numpy(), o_ref) <= ATOL[dtype]
    assert max_abs(lse_g.cpu().numpy(), lse_ref) <= 1e-3
