"""gfx950 launch-configuration search space, selection rules and the persisted tuning table.

This replaces the reference's candidate enumeration and ranking (tuner.py:181-235, 414-449,
503-517; mma.py:63-81). The reference compiles Triton candidates and ranks feasible ones by the
largest resource footprint without timing. Here the candidates are the tiles built into
libfa_gfx950.so; feasibility comes from the compiler's resource table (kernel_resources.json);
ranking comes from a timed sweep on an MI355X (``tune_table.json``, written by gfx950_tune.py),
with a fixed preference order when no measurement exists for a shape.

Tune arguments given by a caller (FlashAttenTuneArguments, or the BLOCK_* kwargs of a kernel
launch) are hints: a built tile that matches every given tile field is used; otherwise fields are
relaxed in the order NUM_STAGES, NUM_WARPS, BLOCK_N, BLOCK_M and the relaxation is recorded.
Tile choice never changes results, only speed.
"""
from __future__ import annotations

import functools
import json
import math
from dataclasses import dataclass
from pathlib import Path

import hip_lib

HERE = Path(__file__).resolve().parent
TUNE_TABLE_PATH = HERE / "tune_table.json"

VARIANT_BY_KERNEL = {
    "_flash_attn_fwd_kernel_basic": hip_lib.FA_VARIANT_BASIC,
    "_flash_attn_fwd_kernel_optimize_shared_mem": hip_lib.FA_VARIANT_OPT,
    "_flash_attn_fwd_kernel_block_d_nomask_contiguous": hip_lib.FA_VARIANT_SLICED,
}

# Attention tiles in preference order (used when the tuning table has no entry for a shape's variant,
# dtype, head dim and causality; the first ones are the fastest measured at large sizes):
# (block_m, block_n, waves, stages). stages selects the kernel pipeline:
#   1  one K/V buffer, two barriers per KV tile (the basic variant),
#   2  double-buffered K/V, one barrier per tile,
#   3  software-pipelined (QK of tile u+1 overlapped with the softmax of tile u inside each wave,
#      K/V brought into an LDS ring by LDS-DMA loads),
#   4  two-tile-ahead pipeline (QK of tile u+2 one for one with PV of tile u, the softmax of tile
#      u+1 spread over both; same LDS-DMA rings),
#   5  one tile per step in a 2-slot LDS-DMA ring, lean enough in registers for two waves per
#      SIMD at D = 256,
#   6  stages 5 with 16x16x32 MFMA tiles,
#   7  stages 3 with 16x16x32 MFMA tiles,
#   8  ping-pong: 8 waves in two groups of four that alternate MFMA phases and softmax phases
#      on the same SIMDs (16x16x32 MFMA tiles, 256 query rows per workgroup),
#   9  the ping-pong kernel in a persistent grid: one workgroup per CU walks a fixed sequence of
#      query blocks and fetches the next block's Q, K and V during the current block's last steps.
# The basic variant uses stages 1; optimized and sliced use 2 to 9.
FA_TILE_SPACE = [
    (256, 64, 8, 8),
    (128, 32, 4, 6),
    (128, 64, 4, 7),
    (256, 64, 8, 9),
    (128, 64, 4, 3),
    (256, 64, 8, 3),
    (128, 32, 4, 3),
    (128, 64, 4, 4),
    (128, 32, 4, 4),
    (128, 32, 4, 5),
    (128, 64, 4, 5),
    (128, 64, 4, 6),
    (128, 32, 4, 7),
    (256, 64, 8, 2),
    (256, 64, 4, 2),
    (128, 64, 4, 2),
    (256, 128, 8, 2),
    (128, 128, 4, 2),
    (256, 32, 8, 2),
    (128, 32, 4, 2),
    (256, 64, 8, 1),
    (256, 64, 4, 1),
    (128, 64, 4, 1),
    (256, 128, 8, 1),
    (128, 128, 4, 1),
    (256, 32, 8, 1),
    (128, 32, 4, 1),
]
STAGES_BY_VARIANT = {
    hip_lib.FA_VARIANT_BASIC: (1,),
    hip_lib.FA_VARIANT_OPT: (3, 4, 5, 6, 7, 8, 9, 2),
    hip_lib.FA_VARIANT_SLICED: (3, 4, 5, 6, 7, 8, 9, 2),
}

# GEMM tiles in preference order: (block_m, block_n, block_k, waves).
GEMM_TILE_SPACE = [
    (256, 256, 64, 8),
    (256, 256, 64, 4),
    (256, 256, 32, 8),
    (256, 256, 32, 4),
    (256, 128, 64, 8),
    (128, 256, 64, 8),
    (128, 128, 64, 4),
    (128, 128, 32, 4),
    (128, 64, 32, 4),
    (64, 256, 32, 4),
    # K groups: 2 or 4 groups of 4 waves split one tile's K loop (shapes with few tiles)
    (128, 128, 32, 8),
    (128, 64, 32, 8),
    (128, 64, 32, 16),
    (64, 64, 32, 8),
]
GEMM_DEFAULT_GROUP_M = 8

# The sliced variant splits KV until every CU holds as many workgroups as the kernel can keep
# resident (RESIDENT_DEFAULT when its resources are unknown); splitting further only adds merge
# traffic.
NUM_CUS = 256
RESIDENT_DEFAULT = 2
# Prefill-shaped sliced launches split only below this many workgroups (a quarter of the CUs).
PREFILL_SPLIT_CUS = NUM_CUS // 4
# A single sequence with two kv heads needs 128 splits to fill the resident capacity (Qwen2.5
# B1 N32k: 18.7 us with 128 splits against 21.0 with 64, HIP-graph replay).
MAX_SPLITS = 128
LDS_PER_CU = 160 * 1024


@dataclass(frozen=True)
class FaTileChoice:
    block_m: int
    block_n: int
    waves: int
    stages: int
    splits: int = 1

    def to_c(self) -> hip_lib.FaTile:
        return hip_lib.make_tile(self.block_m, self.block_n, self.waves, self.stages, self.splits)


def stages_for(variant: int) -> int:
    """Default pipeline of a variant when no tile is chosen (the double-buffered one for
    optimized and sliced: it is built for every head dim)."""
    return 1 if variant == hip_lib.FA_VARIANT_BASIC else 2


def fa_candidates(variant: int, dtype, D: int) -> list[FaTileChoice]:
    """Built attention tiles for (variant, dtype, D), in preference order."""
    out = []
    allowed = STAGES_BY_VARIANT.get(variant, ())
    for bm, bn, waves, stages in FA_TILE_SPACE:
        if stages not in allowed:
            continue
        choice = FaTileChoice(bm, bn, waves, stages, 1)
        if not hip_lib.fa_fwd_supported(variant, dtype, D, choice.to_c()):
            continue
        # the sliced variant may split KV at run time: its split instantiation must exist as well
        if variant == hip_lib.FA_VARIANT_SLICED and not hip_lib.fa_fwd_supported(
                variant, dtype, D, FaTileChoice(bm, bn, waves, stages, 2).to_c()):
            continue
        out.append(choice)
    return out


def gemm_candidates() -> list[tuple[int, int, int, int]]:
    return [t for t in GEMM_TILE_SPACE if hip_lib.gemm_supported(hip_lib.GemmTile(t[0], t[1], t[2], t[3], 1))]


# ---- hint resolution ----------------------------------------------------------------------------

_RELAX_ORDER = ("NUM_STAGES", "NUM_WARPS", "BLOCK_N", "BLOCK_M")


def _matches(choice: FaTileChoice, hints: dict[str, int]) -> bool:
    if "BLOCK_M" in hints and choice.block_m != hints["BLOCK_M"]:
        return False
    if "BLOCK_N" in hints and choice.block_n != hints["BLOCK_N"]:
        return False
    if "NUM_WARPS" in hints and choice.waves != hints["NUM_WARPS"]:
        return False
    if "NUM_STAGES" in hints and choice.stages != hints["NUM_STAGES"]:
        return False
    return True


def filter_by_hints(candidates: list[FaTileChoice], hints: dict[str, int | None]) -> tuple[list[FaTileChoice], list[str]]:
    """Candidates matching the given hints, relaxing hints in _RELAX_ORDER until some match.
    Returns (matching candidates, names of relaxed hints)."""
    active = {k: int(v) for k, v in hints.items() if v is not None and k in _RELAX_ORDER}
    relaxed: list[str] = []
    for key in _RELAX_ORDER:
        if any(_matches(c, active) for c in candidates):
            break
        if key in active:
            del active[key]
            relaxed.append(key)
    # Put back every dropped hint that some candidate still satisfies together with the rest.
    for key in list(relaxed):
        trial = dict(active)
        trial[key] = int(hints[key])
        if any(_matches(c, trial) for c in candidates):
            active = trial
            relaxed.remove(key)
    found = [c for c in candidates if _matches(c, active)]
    return (found or list(candidates)), relaxed


# ---- tuning table -------------------------------------------------------------------------------

_table_cache: dict | None = None


def load_tune_table(path: Path | None = None) -> dict:
    global _table_cache
    if path is None and _table_cache is not None:
        return _table_cache
    p = path or TUNE_TABLE_PATH
    table = json.loads(p.read_text()) if p.exists() else {"fa": {}, "gemm": {}}
    table.setdefault("fa", {})
    table.setdefault("gemm", {})
    if path is None:
        _table_cache = table
    return table


def reset_tune_table_cache() -> None:
    global _table_cache
    _table_cache = None


def _bucket(x: int) -> int:
    """Power-of-two bucket (>= 1) used to key shapes in the tuning table."""
    return 1 << max(0, math.ceil(math.log2(max(1, x))))


def fa_table_key(variant: int, dtype, D: int, causal: bool, B: int, H: int, M: int, N: int) -> str:
    dt = "bf16" if "bfloat16" in str(dtype) else "f16"
    return f"v{variant}|{dt}|D{D}|c{int(bool(causal))}|BH{_bucket(B * H)}|M{_bucket(M)}|N{_bucket(N)}"


def gemm_table_key(M: int, N: int, K: int) -> str:
    return f"M{_bucket(M)}|N{_bucket(N)}|K{_bucket(K)}"


def _nearest_fa_entry(table: dict, key: str) -> dict | None:
    """The entry for `key`, else the swept bucket of the same (variant, dtype, D, causal) nearest to
    it: smallest sum of |log2| distances in B*H, M and N (ties: more work, then key order). Shapes
    between the swept sizes (the reference's B=1 H=28 pipeline cases, say) then run the tile timed on
    their neighbours instead of the fixed preference order."""
    entry = table.get(key)
    if entry is not None:
        return entry
    prefix, rest = key.rsplit("|", 3)[0], key.rsplit("|", 3)[1:]
    want = [int(part.lstrip("BHMN")) for part in rest]
    best, best_rank = None, None
    for other, ent in sorted(table.items()):
        o_prefix, o_rest = other.rsplit("|", 3)[0], other.rsplit("|", 3)[1:]
        if o_prefix != prefix:
            continue
        have = [int(part.lstrip("BHMN")) for part in o_rest]
        dist = sum(abs(math.log2(a) - math.log2(b)) for a, b in zip(want, have))
        rank = (dist, -have[0] * have[1] * have[2])
        if best_rank is None or rank < best_rank:
            best, best_rank = ent, rank
    return best


def _nearest_gemm_entry(table: dict, key: str) -> dict | None:
    """The entry for `key` ("M..|N..|K.."), else the swept GEMM bucket nearest to it: smallest sum
    of |log2| distances in M, N and K (ties: more work, then key order). A shape between the swept
    sizes (1024x4096x1024, say) then runs a tile timed on a shape of its scale, not the first built
    tile -- a 256x256 tile there leaves three quarters of the CUs idle."""
    entry = table.get(key)
    if entry is not None:
        return entry
    want = [int(part.lstrip("MNK")) for part in key.split("|")]
    best, best_rank = None, None
    for other, ent in sorted(table.items()):
        have = [int(part.lstrip("MNK")) for part in other.split("|")]
        dist = sum(abs(math.log2(a) - math.log2(b)) for a, b in zip(want, have))
        rank = (dist, -have[0] * have[1] * have[2])
        if best_rank is None or rank < best_rank:
            best, best_rank = ent, rank
    return best


def _gemm_ranked_tiles(entry: dict) -> list[tuple[tuple[int, ...], int]]:
    """(tile, group_m) of a GEMM table entry, fastest first: the entry's winner, then every other
    timed (tile, GROUP_M) in order of its time."""
    ranked = [(tuple(entry["tile"]), int(entry.get("group_m", GEMM_DEFAULT_GROUP_M)))]
    timed = {**entry.get("timed", {}), **entry.get("refined", {})}
    for name in sorted(timed, key=timed.get):
        tile_part, _, gm_part = name.partition("g")
        try:
            item = (tuple(int(x) for x in tile_part.split("x")), int(gm_part))
        except ValueError:
            continue
        if item not in ranked:
            ranked.append(item)
    return ranked


def choose_fa_tile(variant: int, dtype, D: int, causal: bool, B: int, H: int, M: int, N: int,
                   candidates: list[FaTileChoice]) -> FaTileChoice:
    """Timed-table winner among candidates (the shape's bucket, else its nearest swept bucket of the
    same variant, dtype, head dim and causality), else the first candidate (preference order)."""
    entry = _nearest_fa_entry(load_tune_table()["fa"], fa_table_key(variant, dtype, D, causal, B, H, M, N))
    if entry is not None:
        want = tuple(entry["tile"])
        for c in candidates:
            if (c.block_m, c.block_n, c.waves, c.stages)[:len(want)] == want:
                return c
    return candidates[0]


@functools.lru_cache(maxsize=256)
def split_residency(dtype, D: int, block_m: int, block_n: int, waves: int, stages: int) -> int:
    """Workgroups of the sliced variant's split kernel one CU holds at once: the lower of the
    register bound (waves per SIMD x 4 SIMDs / waves per workgroup) and the LDS bound, from the
    compiler's resource table; RESIDENT_DEFAULT when the kernel is not in it."""
    tile = hip_lib.FaTile(block_m, block_n, waves, stages, 2)
    try:
        res = hip_lib.compiled_resources().get(hip_lib.fwd_kernel_symbol(hip_lib.FA_VARIANT_SLICED, dtype, D, tile))
    except (hip_lib.FaLibraryError, KeyError):
        res = None
    if not res:
        return RESIDENT_DEFAULT
    by_regs = max(1, int(res["Occupancy [waves/SIMD]"]) * 4 // waves)
    lds = int(res["LDS Size [bytes/block]"])
    by_lds = LDS_PER_CU // lds if lds else by_regs
    return max(1, min(by_regs, by_lds))


@functools.lru_cache(maxsize=4096)
def choose_splits(B: int, H: int, M: int, N: int, block_m: int, block_n: int, H_kv: int | None = None,
                  causal: bool = False, resident_per_cu: int = RESIDENT_DEFAULT) -> int:
    """KV splits for the sliced variant, keeping at least two KV tiles per split.

    Decode-shaped grids (M < block_m: a few query rows per tile, K/V streaming dominates) split
    until NUM_CUS x resident_per_cu workgroups (the split kernel's resident capacity,
    split_residency) are in flight; their fp32 partials are a few rows each. Prefill-shaped grids
    (full query tiles) write partials as large as the output and read them back in the merge, so
    they split only when they would occupy fewer than PREFILL_SPLIT_CUS CUs. Split launches of
    decode shapes pack the query heads of a GQA group into one tile (hip_lib.pack_group), so they
    count workgroups per kv head."""
    n_tiles = max(1, math.ceil(N / block_n))
    if n_tiles < 4:
        return 1
    target = PREFILL_SPLIT_CUS if M >= block_m else NUM_CUS * max(1, resident_per_cu)

    def splits_for(base: int) -> int:
        if base >= target:
            return 1
        return max(1, min(math.ceil(target / base), n_tiles // 2, MAX_SPLITS))

    H_kv = H if H_kv is None else H_kv
    group = hip_lib.pack_group(H, H_kv, M, causal, block_m, 2)
    if group > 1:
        packed = splits_for(max(1, math.ceil(M * group / block_m) * B * H_kv))
        if packed > 1:
            return packed
    return splits_for(max(1, math.ceil(M / block_m) * B * H))


def choose_gemm_tile(M: int, N: int, K: int, hint: tuple[int, int, int] | None = None) -> tuple[int, int, int, int, int]:
    """(block_m, block_n, block_k, waves, group_m) for a GEMM; ValueError when no built tile divides.

    Acceptance matches the reference selector (mma.py:63-81): K % 32 == 0 and either
    (M % 128 == 0 and N % 64 == 0) or (M % 64 == 0 and N % 256 == 0)."""
    if K % 32 != 0:
        raise ValueError("fast 2D contiguous matmul requires K % 32 == 0")
    # the reference's rule, stated here rather than left to the built tile set (a 64x64 tile
    # divides shapes the reference rejects)
    reference_ok = (M % 128 == 0 and N % 64 == 0) or (M % 64 == 0 and N % 256 == 0)
    cands = [t for t in gemm_candidates() if M % t[0] == 0 and N % t[1] == 0 and K % t[2] == 0] if reference_ok else []
    if not cands:
        raise ValueError(
            "fast 2D contiguous matmul requires a supported divisible tile: "
            "(M % 128 == 0 and N % 64 == 0), "
            "(M % 128 == 0 and N % 128 == 0), or "
            "(M % 64 == 0 and N % 256 == 0), with K % 32 == 0"
        )
    if hint is not None:
        # (block_m, block_n, block_k[, waves]) hints narrow the candidates; the table still ranks them
        hint = tuple(hint)
        hinted = [t for t in cands if t[:len(hint)] == hint]
        if not hinted and len(hint) > 3:  # no built tile with that wave count: keep the sizes
            hinted = [t for t in cands if t[:3] == hint[:3]]
        cands = hinted or cands
    # the bucket's (or nearest swept bucket's) winner when it divides, else its fastest timed tile
    # that does; the preference order only without a table
    entry = _nearest_gemm_entry(load_tune_table()["gemm"], gemm_table_key(M, N, K))
    if entry is not None:
        for tile, group_m in _gemm_ranked_tiles(entry):
            if tile in cands:
                return (*tile, group_m)
    t = cands[0]
    return (*t, _gemm_group_m(M, N, K, t))


def choose_gemm_tile_any(M: int, N: int, K: int) -> tuple[int, int, int, int, int]:
    """(block_m, block_n, block_k, waves, group_m) for any shape the kernel accepts (K % 8 == 0,
    N % 4 == 0; partial tiles in M, N and K are masked in the kernel): the divisible choice when
    there is one, else the tuned tile of the shape's bucket, else the first built tile no larger
    than the problem (rounded up to 64)."""
    if K % 8 != 0 or N % 4 != 0:
        raise ValueError(f"gfx950 GEMM needs K % 8 == 0 and N % 4 == 0 (got M={M} N={N} K={K})")
    try:
        return choose_gemm_tile(M, N, K)
    except ValueError:
        pass
    cands = gemm_candidates()
    entry = _nearest_gemm_entry(load_tune_table()["gemm"], gemm_table_key(M, N, K))
    if entry is not None:
        for tile, group_m in _gemm_ranked_tiles(entry):
            if tile in cands:
                return (*tile, group_m)
    fit = [t for t in cands if t[0] <= -(-M // 64) * 64 and t[1] <= -(-N // 64) * 64]
    t = (fit or [min(cands, key=lambda t: t[0] * t[1])])[0]
    return (*t, GEMM_DEFAULT_GROUP_M)


def _gemm_group_m(M: int, N: int, K: int, tile) -> int:
    entry = load_tune_table()["gemm"].get(gemm_table_key(M, N, K))
    if entry is not None and list(entry["tile"]) == list(tile):
        return int(entry.get("group_m", GEMM_DEFAULT_GROUP_M))
    return GEMM_DEFAULT_GROUP_M


# ---- compiled resources ---------------------------------------------------------------------------

def fa_resources(variant: int, dtype, D: int, choice: FaTileChoice) -> dict[str, int] | None:
    sym = hip_lib.fwd_kernel_symbol(variant, dtype, D, choice.to_c())
    return _resources(sym)


def gemm_resources(tile: tuple[int, int, int, int]) -> dict[str, int] | None:
    sym = hip_lib.gemm_kernel_symbol(hip_lib.GemmTile(tile[0], tile[1], tile[2], tile[3], 1))
    return _resources(sym)


def _resources(sym: str) -> dict[str, int] | None:
    raw = hip_lib.compiled_resources().get(sym)
    if raw is None:
        return None
    return {
        "vgprs": int(raw.get("VGPRs", 0)),
        "agprs": int(raw.get("AGPRs", 0)),
        "sgprs": int(raw.get("TotalSGPRs", 0)),
        "lds_bytes": int(raw.get("LDS Size [bytes/block]", 0)),
        "scratch_bytes_per_lane": int(raw.get("ScratchSize [bytes/lane]", 0)),
        "waves_per_simd": int(raw.get("Occupancy [waves/SIMD]", 0)),
    }
