"""fa_fwd_noalloc, through the C ABI: the split-KV partials live in the library's static per-GPU
scratch array instead of a caller workspace. The kernels are the same as fa_fwd's, so outputs and
LSE must be bit-identical to fa_fwd with a torch-allocated workspace; they are also checked against
the oracle. Calls run back to back, each smaller than the one before, so a call that read the
previous call's leftovers in the shared array would show up."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import hip_lib
import oracle
from helpers import ATOL, make_qkv, max_abs, to_device

pytestmark = pytest.mark.gpu

F16, BF16 = torch.float16, torch.bfloat16
SLICED, OPT = hip_lib.FA_VARIANT_SLICED, hip_lib.FA_VARIANT_OPT

# name, B, H, Hkv, M, N, D, dtype, causal, splits, (block_m, block_n, waves, stages); largest first
CASES = [
    ("prefill_causal_gqa", 2, 8, 2, 300, 2000, 128, BF16, True, 4, (128, 64, 4, 3)),
    ("smaller_noncausal", 1, 4, 4, 40, 700, 128, F16, False, 3, (128, 64, 4, 3)),
    ("decode_packed_gqa", 1, 12, 2, 1, 5000, 128, BF16, False, 16, (128, 64, 4, 3)),
    ("d256_double_buffered", 1, 2, 2, 17, 300, 256, F16, False, 2, (128, 64, 4, 2)),
]


def _inputs(case):
    name, B, H, Hkv, M, N, D, dtype, causal, splits, tile = case
    q, k, v = make_qkv(7000 + len(name) * 13 + M, B, H, Hkv, M, N, D, dtype)
    dev = "cuda:0"
    return (q, k, v), tuple(to_device(x, dtype, dev) for x in (q, k, v))


def _run(case, qd, kd, vd, *, noalloc: bool):
    name, B, H, Hkv, M, N, D, dtype, causal, splits, (bm, bn, waves, stages) = case
    o = torch.full_like(qd, float("nan"))
    lse = torch.full((B, H, M), float("nan"), dtype=torch.float32, device=qd.device)
    tile = hip_lib.make_tile(bm, bn, waves, stages, splits)
    kw = dict(sm_scale=D ** -0.5, causal=causal, variant=SLICED, tile=tile)
    if noalloc:
        hip_lib.fa_fwd_noalloc(qd, kd, vd, o, lse, **kw)
    else:
        ws = torch.empty(hip_lib.workspace_bytes(B, H, M, D, splits), dtype=torch.uint8, device=qd.device)
        hip_lib.fa_fwd(qd, kd, vd, o, lse, workspace=ws, **kw)
    torch.cuda.synchronize()
    return o, lse


def test_noalloc_matches_fa_fwd_on_successive_calls(gpu):
    for case in CASES:
        name, B, H, Hkv, M, N, D, dtype, causal, splits, tile = case
        print(f"[no_alloc] {name} B={B} H={H} Hkv={Hkv} M={M} N={N} D={D} {dtype} causal={causal} "
              f"splits={splits} tile={tile}", flush=True)
        assert 0 < hip_lib.workspace_bytes(B, H, M, D, splits) <= hip_lib.NOALLOC_SCRATCH_BYTES
        (q, k, v), (qd, kd, vd) = _inputs(case)
        o_ref_gpu, lse_ref_gpu = _run(case, qd, kd, vd, noalloc=False)
        o, lse = _run(case, qd, kd, vd, noalloc=True)
        assert torch.equal(o, o_ref_gpu), name
        assert torch.equal(lse, lse_ref_gpu), name
        o_ref, lse_ref = oracle.attention(q, k, v, causal=causal)
        assert max_abs(o.float().cpu().numpy(), o_ref) <= ATOL[dtype], name
        assert max_abs(lse.cpu().numpy(), lse_ref) <= 1e-3, name


def test_noalloc_without_splits_equals_fa_fwd(gpu):
    case = ("one_split", 1, 2, 2, 100, 260, 64, F16, True, 1, (128, 64, 4, 3))
    (q, k, v), (qd, kd, vd) = _inputs(case)
    o_a, lse_a = _run(case, qd, kd, vd, noalloc=False)
    o_b, lse_b = _run(case, qd, kd, vd, noalloc=True)
    assert torch.equal(o_a, o_b) and torch.equal(lse_a, lse_b)


def test_noalloc_replays_in_a_hip_graph(gpu):
    """A split launch of fa_fwd_noalloc captured in a HIP graph: after one eager call (the first
    call on a device resolves the scratch array's address, which the header requires outside
    capture), the captured split pass + merge replay with new q/k/v contents written in place by
    eager work between replays, and every replay equals an eager fa_fwd (torch workspace) on the
    same inputs bit for bit."""
    case = ("graph_split", 1, 8, 2, 64, 3000, 128, F16, False, 8, (128, 64, 4, 3))
    name, B, H, Hkv, M, N, D, dtype, causal, splits, (bm, bn, waves, stages) = case
    print(f"[no_alloc] graph capture B={B} H={H} Hkv={Hkv} M={M} N={N} D={D} splits={splits}", flush=True)
    _, (qd, kd, vd) = _inputs(case)
    _run(case, qd, kd, vd, noalloc=True)
    o = torch.empty_like(qd)
    lse = torch.empty((B, H, M), dtype=torch.float32, device=qd.device)
    kw = dict(sm_scale=D ** -0.5, causal=causal, variant=SLICED, tile=hip_lib.make_tile(bm, bn, waves, stages, splits))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        hip_lib.fa_fwd_noalloc(qd, kd, vd, o, lse, **kw)
    g = torch.Generator().manual_seed(11)
    for rep in range(4):
        for t in (qd, kd, vd):
            t.copy_(torch.randn(t.shape, generator=g).to(dtype))
        o_ref, lse_ref = _run(case, qd, kd, vd, noalloc=False)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref), rep
        assert torch.equal(lse, lse_ref), rep


def test_noalloc_rejects_oversized_partials_before_launch(gpu):
    B, H, M, N, D, splits = 4, 32, 2048, 4096, 128, 4
    need = hip_lib.workspace_bytes(B, H, M, D, splits)
    assert need > hip_lib.NOALLOC_SCRATCH_BYTES
    dev = "cuda:0"
    q = torch.zeros((B, H, M, D), dtype=F16, device=dev)
    k = torch.zeros((B, H, N, D), dtype=F16, device=dev)
    o = torch.full_like(q, 7.0)
    with pytest.raises(ValueError, match="exceed its static scratch"):
        hip_lib.fa_fwd_noalloc(q, k, k, o, None, sm_scale=D ** -0.5, causal=False, variant=SLICED,
                               tile=hip_lib.make_tile(128, 64, 4, 3, splits))
    torch.cuda.synchronize()
    assert bool((o == 7.0).all())  # nothing ran


def test_noalloc_rejects_a_workspace_argument(gpu):
    dev = "cuda:0"
    q = torch.zeros((1, 1, 8, 64), dtype=F16, device=dev)
    ws = torch.empty(hip_lib.workspace_bytes(1, 1, 8, 64, 2), dtype=torch.uint8, device=dev)
    args = hip_lib._fwd_args(q, q, q, torch.empty_like(q), None, sm_scale=0.125, causal=False, variant=SLICED,
                             tile=hip_lib.make_tile(128, 64, 4, 3, 2), workspace=ws)
    code = hip_lib.load().fa_fwd_noalloc(ctypes.byref(args), hip_lib._stream_ptr(q.device))
    assert code == hip_lib.FA_EINVAL
    assert "takes no workspace" in hip_lib.last_error()
