"""Routing oracle: the router's top-k softmax, the sort by expert and the tile map (numpy).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""

import numpy as np


def topk_softmax(logits, k: int, renorm: bool = True):
    """(weights fp32 (T, k), indices int64 (T, k)) of the router.

    Follows TF:models/qwen3_moe/modeling_qwen3_moe.py:262-266: softmax in fp32, the k largest,
    renormalised over the k when `renorm`.  Order: descending probability; equal logits in
    ascending expert index (a stable sort of -logit).  Selection is done on the logits, which order
    the exact softmax probabilities the same way.
    Pinned by: torch.topk on tie-free inputs (identical indices) and a brute-force sort on inputs
    with ties (tests/test_oracle.py).
    """
    x = np.asarray(logits, dtype=np.float32)
    x = x + np.float32(0.0)  # -0.0 and +0.0 are one value
    order = np.argsort(-x, axis=-1, kind="stable")[:, :k]
    m = x.max(axis=-1, keepdims=True)
    e = np.exp((x - m).astype(np.float64))
    p = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
    w = np.take_along_axis(p, order, axis=-1)
    if renorm:
        w = (w / w.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    return w, order.astype(np.int64)


def sort_by_expert(ids, num_experts: int):
    """(perm int64, inv int64, offsets int32) of the flat expert ids.

    Follows src/meepsquared/_moe.py:77-87: perm orders the ids by expert (here the stable order:
    ascending flat index within an expert), offsets = cumsum of the per-expert counts (ids at or
    past num_experts are sentinels: they sort after every expert and are not counted).
    Pinned by: torch.sort(stable=True), torch.bincount (tests/test_oracle.py).
    """
    ids = np.asarray(ids, dtype=np.int64).reshape(-1)
    key = np.where((ids >= 0) & (ids < num_experts), ids, num_experts)
    perm = np.argsort(key, kind="stable").astype(np.int64)
    inv = np.empty_like(perm)
    inv[perm] = np.arange(perm.size, dtype=np.int64)
    counts = np.bincount(key, minlength=num_experts + 1)[:num_experts]
    offsets = np.cumsum(counts).astype(np.int32)
    return perm, inv, offsets


def max_tiles(rows: int, experts: int, block_m: int) -> int:
    """src/meepsquared/_grouped.py:83-85."""
    return rows // block_m + experts


def tile_map(offsets, rows: int, block_m: int):
    """(tile_expert int32, tile_row int32, tiles int) — src/meepsquared/_grouped.py:88-103.

    Pinned by: the reference's known answers (tests/test_grouped.py:18-31), copied as literals
    into tests/test_oracle.py, and a brute-force enumeration of tiles.
    """
    offsets = np.asarray(offsets, dtype=np.int64)
    experts = offsets.size
    starts = np.concatenate([[0], offsets[:-1]])
    tiles_per_expert = (offsets - starts + block_m - 1) // block_m
    tile_ends = np.cumsum(tiles_per_expert)
    t = np.arange(max_tiles(rows, experts, block_m), dtype=np.int64)
    tile_expert = np.minimum(np.searchsorted(tile_ends, t, side="right"), experts - 1)
    tile_row = starts[tile_expert] + (t - (tile_ends - tiles_per_expert)[tile_expert]) * block_m
    return tile_expert.astype(np.int32), tile_row.astype(np.int32), int(tile_ends[-1])
