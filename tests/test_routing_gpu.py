"""Routing kernels against the oracle: indices, permutation, offsets and tile map bit-exact."""

import numpy as np
import pytest
import torch

from oracle import routing

pytestmark = pytest.mark.gpu


def test_topk_matches_the_golden_torch_topk(golden):
    from meepsquared_amd import topk_softmax

    g = golden("routing.npz")
    logits = torch.from_numpy(g["logits"]).cuda()
    w, idx = topk_softmax(logits, int(g["k"]), renormalize=True, weights_dtype=torch.float32)
    assert np.array_equal(idx.cpu().numpy(), g["topk_idx"])
    np.testing.assert_allclose(w.cpu().numpy(), g["topk_w"], rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("T,E,k,dtype", [
    (8192, 128, 8, torch.bfloat16),  # Qwen3-30B-A3B router, bf16 logits: ties are common
    (16384, 8, 2, torch.float32),    # Mixtral
    (333, 1000, 17, torch.bfloat16),  # E past 64 per lane slot boundaries, odd T
    (64, 64, 64, torch.float32),      # k = E
])
def test_topk_indices_are_bit_exact_with_ties(T, E, k, dtype):
    from meepsquared_amd import topk_softmax

    torch.manual_seed(0)
    logits = torch.randn(T, E, dtype=torch.float32)
    if dtype == torch.bfloat16:
        logits = (logits * 4).round() / 4  # force many exact ties
    logits = logits.to(dtype)
    w, idx = topk_softmax(logits.cuda(), k, renormalize=True, weights_dtype=torch.float32)
    ow, oidx = routing.topk_softmax(logits.float().numpy(), k)
    assert np.array_equal(idx.cpu().numpy(), oidx)
    np.testing.assert_allclose(w.cpu().numpy(), ow, rtol=1e-5, atol=1e-6)


def test_topk_matches_the_golden_gpu_torch_topk_with_ties(golden):
    """tests/golden/topk_gpu.npz (torch.topk on the GPU, bf16 logits with ties, k = 1 .. 40): indices
    bit-exact, in torch's order; renormalised fp32 weights to the last bits."""
    from meepsquared_amd import topk_softmax

    g = golden("topk_gpu.npz")
    for c, (T, E, k, seed, q) in enumerate(g["cases"]):
        logits = torch.from_numpy(g[f"logits_{c}"].view(np.int16)).view(torch.bfloat16).cuda()
        w, idx = topk_softmax(logits, int(k), renormalize=True, weights_dtype=torch.float32)
        assert np.array_equal(idx.cpu().numpy(), g[f"idx_{c}"].astype(np.int64)), (c, int(T), int(E), int(k))
        np.testing.assert_allclose(w.cpu().numpy(), g[f"w_{c}"], rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("q", [0.0, 4.0])
@pytest.mark.parametrize("weights_dtype", [torch.bfloat16, torch.float32])
def test_topk_matches_torch_topk_on_the_same_gpu(q, weights_dtype):
    """The reference's router on config 1's logits (T=8192, E=128, top-8, bf16 N(0,1), seed 0; q = 4: logits
    rounded to quarters, ties in most rows), run by torch on this GPU: softmax(fp32) -> topk -> renormalise
    -> cast (TF:models/qwen3_moe/modeling_qwen3_moe.py:262-266).  Indices bit-exact, ties included;
    weights within one rounding of the dtype."""
    from meepsquared_amd import topk_softmax

    g = torch.Generator().manual_seed(0)
    logits = torch.randn(8192, 128, generator=g)
    if q:
        logits = (logits * q).round() / q
    logits = logits.to(torch.bfloat16).cuda()
    probs = torch.softmax(logits, dim=-1, dtype=torch.float)
    vals, tidx = torch.topk(probs, 8, dim=-1)
    tw = (vals / vals.sum(dim=-1, keepdim=True)).to(weights_dtype)
    w, idx = topk_softmax(logits, 8, renormalize=True, weights_dtype=weights_dtype)
    assert torch.equal(idx, tidx)
    tol = dict(rtol=4e-3, atol=0) if weights_dtype == torch.bfloat16 else dict(rtol=2e-6, atol=1e-7)
    torch.testing.assert_close(w, tw, **tol)


def test_topk_without_renormalisation_and_bf16_weights():
    from meepsquared_amd import topk_softmax

    torch.manual_seed(1)
    logits = torch.randn(1000, 128, dtype=torch.bfloat16)
    w, idx = topk_softmax(logits.cuda(), 8, renormalize=False)
    assert w.dtype == torch.bfloat16
    ow, oidx = routing.topk_softmax(logits.float().numpy(), 8, renorm=False)
    assert np.array_equal(idx.cpu().numpy(), oidx)
    np.testing.assert_allclose(w.float().cpu().numpy(), ow, rtol=8e-3)


def test_sort_matches_the_golden_stable_sort_with_sentinels(golden):
    from meepsquared_amd import sort_by_expert

    g = golden("routing.npz")
    perm, inv, offsets = sort_by_expert(torch.from_numpy(g["ids"]).cuda(), int(g["num_experts"]))
    assert np.array_equal(perm.cpu().numpy(), g["perm"])
    assert np.array_equal(offsets.cpu().numpy(), g["offsets"])
    assert np.array_equal(inv.cpu().numpy()[g["perm"]], np.arange(g["perm"].size))


@pytest.mark.parametrize("S,E", [(65536, 128), (32768, 8), (540672, 128), (1, 1), (4097, 2048), (100, 3)])
def test_sort_is_bit_exact(S, E):
    from meepsquared_amd import sort_by_expert

    rng = np.random.default_rng(S + E)
    ids = rng.integers(0, E + 1, size=S)  # id E: a sentinel
    if E == 8:  # Zipf-skewed load
        ids = np.minimum(rng.zipf(1.2, size=S) - 1, E - 1)
    perm, inv, offsets = sort_by_expert(torch.from_numpy(ids).cuda(), E)
    operm, oinv, ooffsets = routing.sort_by_expert(ids, E)
    assert np.array_equal(perm.cpu().numpy(), operm)
    assert np.array_equal(inv.cpu().numpy(), oinv)
    assert np.array_equal(offsets.cpu().numpy(), ooffsets)


def test_sort_writes_the_tile_map_too():
    from meepsquared_amd import sort_by_expert

    rng = np.random.default_rng(7)
    ids = rng.integers(0, 16, size=5000)
    perm, inv, offsets, te, tr, tiles = sort_by_expert(torch.from_numpy(ids).cuda(), 16, block_m=128)
    ote, otr, otiles = routing.tile_map(offsets.cpu().numpy(), 5000, 128)
    assert tiles.item() == otiles
    assert np.array_equal(te.cpu().numpy(), ote) and np.array_equal(tr.cpu().numpy(), otr)


def test_tile_map_known_answers():
    # tests/test_grouped.py:18-31 of the reference
    from meepsquared_amd import max_tiles, tile_map
    from helpers import offsets_of

    tile_expert, tile_row, tiles = tile_map(offsets_of([5, 0, 130, 64]), rows=199, block_m=64)
    assert tiles.item() == 5
    assert tile_expert[:5].tolist() == [0, 2, 2, 2, 3]
    assert tile_row[:5].tolist() == [0, 5, 69, 133, 135]
    assert tile_expert.numel() == max_tiles(199, 4, 64) >= 5
    assert tile_expert.max() <= 3
    tile_expert, tile_row, tiles = tile_map(offsets_of([0, 0, 7]), rows=7, block_m=64)
    assert tiles.item() == 1 and tile_expert[0].item() == 2 and tile_row[0].item() == 0


@pytest.mark.parametrize("seed", range(3))
def test_tile_map_matches_the_oracle_everywhere(seed):
    from meepsquared_amd import tile_map

    rng = np.random.default_rng(seed)
    counts = rng.integers(0, 700, size=rng.integers(1, 300))
    offsets = np.cumsum(counts).astype(np.int32)
    rows = int(offsets[-1]) + int(rng.integers(0, 50))
    te, tr, tiles = tile_map(torch.from_numpy(offsets).cuda(), rows, 128)
    ote, otr, otiles = routing.tile_map(offsets, rows, 128)
    assert tiles.item() == otiles
    assert np.array_equal(te.cpu().numpy(), ote) and np.array_equal(tr.cpu().numpy(), otr)
