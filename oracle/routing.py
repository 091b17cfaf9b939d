"""Routing oracle: the router's top-k softmax, the sort by expert and the tile map (numpy).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""

import numpy as np


BITONIC_WIDTH = 32  # torch sorts the k selected values of a row with a 32-wide bitonic network when k <= 32


def _bitonic_stages(width):
    """The compare-exchange stages of a bitonic sort of `width` (a power of two) positions: per stage the
    pairs (a, b = a + stride) and each pair's direction flag, as a network of width / 2 comparators
    (comparator t at a = 2t - (t mod stride)); merges of growing size, then one descending merge of all."""
    stages = []
    size = 2
    while size < width:
        stride = size // 2
        while stride:
            t = np.arange(width // 2)
            stages.append((2 * t - (t & (stride - 1)), stride, (t & (size // 2)) != 0))
            stride //= 2
        size *= 2
    stride = width // 2
    while stride:
        t = np.arange(width // 2)
        stages.append((2 * t - (t & (stride - 1)), stride, np.zeros(width // 2, dtype=bool)))
        stride //= 2
    return stages


def _torch_gpu_order(order, key, k):
    """The k selected experts of each row in the order torch.topk returns them on the GPU.

    torch gathers the selected values in expert order (those strictly above the k-th value first,
    then those equal to it) and, for k <= 32, sorts them descending with a bitonic network over 32
    positions (the k values, then empty positions): a comparator swaps its pair when "a above b and a
    present, or b empty" equals its direction flag, so equal values are exchanged whenever a comparator
    with flag false meets them.  For k > 32 the sort is stable (equal values stay in expert order).
    order (T, k): the selected experts, descending, equal values in ascending expert; key: their values.
    """
    T = order.shape[0]
    kth = key[:, k - 1:k]
    gather = np.argsort(np.where(key > kth, 0, 1) * (1 << 20) + order, axis=1, kind="stable")
    idx = np.take_along_axis(order, gather, 1)
    val = np.take_along_axis(key, gather, 1)
    if k > BITONIC_WIDTH:
        return order  # a stable descending sort of the expert-ordered values is `order` itself
    W = BITONIC_WIDTH
    K = np.zeros((T, W), dtype=np.float64)
    V = np.zeros((T, W), dtype=np.int64)
    ok = np.zeros((T, W), dtype=bool)
    K[:, :k], V[:, :k], ok[:, :k] = val, idx, True
    for a, stride, flag in _bitonic_stages(W):
        b = a + stride
        swap = ((K[:, a] > K[:, b]) & ok[:, a]) | ~ok[:, b]
        do = swap == flag[None, :]
        for arr in (K, V, ok):
            xa, xb = arr[:, a].copy(), arr[:, b].copy()
            arr[:, a] = np.where(do, xb, xa)
            arr[:, b] = np.where(do, xa, xb)
    return V[:, :k]


def topk_softmax(logits, k: int, renorm: bool = True):
    """(weights fp32 (T, k), indices int64 (T, k)) of the router.

    Follows TF:models/qwen3_moe/modeling_qwen3_moe.py:262-266: softmax in fp32, torch.topk of the
    probabilities, renormalised over the k when `renorm`.  Selection and ties follow torch.topk on the
    GPU, where the reference's router runs: equal probabilities at the k-th place are taken in
    ascending expert order, and the k are returned in torch's GPU order (_torch_gpu_order).  Equal
    probabilities are equal values of x - max(x) in fp32, the argument of the softmax's exponential.
    Pinned by: torch.topk on the GPU over bf16 logits with ties, k = 1 .. 40
    (tests/golden/topk_gpu.npz, indices bit-exact), torch.topk on tie-free logits (routing.npz), and a
    brute-force selection on ties (tests/test_oracle.py).
    """
    x = np.asarray(logits, dtype=np.float32)
    m = x.max(axis=-1, keepdims=True)
    d = (x - m).astype(np.float32) + np.float32(0.0)  # -0.0 and +0.0 are one value
    order = np.argsort(-d, axis=-1, kind="stable")[:, :k]
    if k > 1:
        order = _torch_gpu_order(order, np.take_along_axis(d, order, 1).astype(np.float64), k)
    e = np.exp(d.astype(np.float64))
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
