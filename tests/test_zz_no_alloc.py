"""mlora_route_sort_noalloc (the counting sort with its histograms in the library's own per-GPU scratch
array, for callers that cannot allocate) against mlora_route_sort (the caller's workspace): the same
perm, inv, offsets and tile map to the bit, on two calls in a row, the second smaller; sizes past the
array's 4 MiB are refused before any launch.  Called through the C ABI."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _sort(ids, E, block_m, noalloc):
    from meepsquared_amd import _grouped, _lib
    from meepsquared_amd._lib import ptr

    S = ids.numel()
    dev = ids.device
    perm = torch.full((S,), -1, device=dev, dtype=torch.int64)
    inv = torch.full((S,), -1, device=dev, dtype=torch.int64)
    offsets = torch.full((E,), -1, device=dev, dtype=torch.int32)
    n_tiles = _grouped.max_tiles(S, E, block_m)
    te = torch.full((n_tiles,), -1, device=dev, dtype=torch.int32)
    tr = torch.full((n_tiles,), -1, device=dev, dtype=torch.int32)
    tn = torch.full((), -1, device=dev, dtype=torch.int32)
    if noalloc:
        _lib.call("mlora_route_sort_noalloc", ptr(ids), S, E, ptr(perm), ptr(inv), ptr(offsets), block_m, ptr(te),
                  ptr(tr), ptr(tn), n_tiles, _lib.stream(dev))
    else:
        ws = torch.empty(int(_lib.lib.mlora_route_sort_workspace_bytes(S, E)), device=dev, dtype=torch.uint8)
        _lib.call("mlora_route_sort", ptr(ids), S, E, ptr(perm), ptr(inv), ptr(offsets), block_m, ptr(te), ptr(tr),
                  ptr(tn), n_tiles, ptr(ws), ws.numel(), _lib.stream(dev))
    torch.cuda.synchronize()
    return perm.cpu(), inv.cpu(), offsets.cpu(), te.cpu(), tr.cpu(), tn.cpu()


def test_the_sort_without_a_workspace_matches_the_sort_with_one_on_two_calls():
    # config 1's routing (65,536 ids over 128 experts, with sentinels), then a smaller call over fewer
    # experts: the second call reads only what it wrote itself in the shared scratch array
    for S, E, seed in ((65536, 128, 0), (5000, 16, 1)):
        rng = np.random.default_rng(seed)
        ids = torch.from_numpy(rng.integers(0, E + 1, size=S)).cuda()  # id E: a sentinel
        print(f"noalloc sort: S={S} E={E} seed={seed}", flush=True)
        got = _sort(ids, E, 128, noalloc=True)
        want = _sort(ids, E, 128, noalloc=False)
        for name, a, b in zip(("perm", "inv", "offsets", "tile_expert", "tile_row", "tiles"), got, want):
            assert torch.equal(a, b), (S, E, name)


def test_the_sort_without_a_workspace_refuses_sizes_past_its_scratch():
    from meepsquared_amd import _lib

    S, E = 1 << 22, 2048  # 16,384 chunks x 2049 bins x 4 bytes: far past 4 MiB
    assert _lib.lib.mlora_route_sort_workspace_bytes(S, E) > 4 << 20
    rc = _lib.lib.mlora_route_sort_noalloc(None, S, E, None, None, None, 0, None, None, None, 0, None)
    assert rc != 0
    assert "scratch" in _lib.lib.mlora_last_error().decode()
