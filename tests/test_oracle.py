"""The CPU oracle, pinned against the reference's known answers, torch's own operators, golden
fixtures and closed forms (CPU only)."""

import numpy as np
import pytest
import torch

from oracle import formats, grouped, moe, routing


# ---- tile map: the reference's known answers (tests/test_grouped.py:18-31) ----

def offsets_of(rows_per_expert):
    return np.cumsum(np.array(rows_per_expert, dtype=np.int32)).astype(np.int32)


def test_tile_map_known_answer_uneven_with_an_empty_expert():
    tile_expert, tile_row, tiles = routing.tile_map(offsets_of([5, 0, 130, 64]), rows=199, block_m=64)
    assert tiles == 5
    assert tile_expert[:5].tolist() == [0, 2, 2, 2, 3]
    assert tile_row[:5].tolist() == [0, 5, 69, 133, 135]
    assert tile_expert.size == routing.max_tiles(199, 4, 64) >= 5
    assert tile_expert.max() <= 3


def test_tile_map_known_answer_all_empty_but_one():
    tile_expert, tile_row, tiles = routing.tile_map(offsets_of([0, 0, 7]), rows=7, block_m=64)
    assert tiles == 1 and tile_expert[0] == 2 and tile_row[0] == 0


@pytest.mark.parametrize("seed", range(5))
def test_tile_map_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    counts = rng.integers(0, 300, size=rng.integers(1, 12))
    bm = int(rng.choice([16, 64, 128]))
    rows = int(counts.sum())
    te, tr, tiles = routing.tile_map(np.cumsum(counts), rows, bm)
    brute = [(e, int(np.cumsum(counts)[e] - counts[e] + j)) for e in range(counts.size) for j in range(0, counts[e], bm)]
    assert tiles == len(brute)
    assert list(zip(te[:tiles].tolist(), tr[:tiles].tolist())) == brute


# ---- router and sort: torch's operators, golden fixture, brute force on ties ----

def test_router_matches_torch_topk_on_the_golden_logits(golden):
    g = golden("routing.npz")
    w, idx = routing.topk_softmax(g["logits"], int(g["k"]))
    assert np.array_equal(idx, g["topk_idx"])
    np.testing.assert_allclose(w, g["topk_w"], rtol=1e-6, atol=1e-7)


def test_router_ties_at_the_kth_place_go_to_the_lower_expert():
    # brute force: the selected set is the k first of (value descending, expert ascending), returned in
    # non-increasing order of value (the order among equal values is torch's: pinned by topk_gpu.npz)
    rng = np.random.default_rng(0)
    x = rng.integers(-3, 4, size=(64, 32)).astype(np.float32)  # many ties
    for k in (5, 2, 32):
        w, idx = routing.topk_softmax(x, k)
        for r in range(64):
            brute = sorted(range(32), key=lambda e: (-x[r, e], e))[:k]
            assert sorted(idx[r].tolist()) == sorted(brute)
            assert np.all(np.diff(x[r, idx[r]]) <= 0)
        np.testing.assert_allclose(w.sum(axis=1), 1.0, rtol=1e-6)


def test_router_order_matches_torch_topk_on_the_gpu_with_ties(golden):
    """tests/golden/topk_gpu.npz: torch.topk on the GPU over softmax(bf16 logits) with ties inside the k
    and at its boundary, k = 1 .. 40: the oracle's indices bit-exact, in torch's order."""
    g = golden("topk_gpu.npz")
    for c, (T, E, k, seed, q) in enumerate(g["cases"]):
        x = (g[f"logits_{c}"].astype(np.uint32) << 16).view(np.float32)
        w, idx = routing.topk_softmax(x, int(k))
        assert np.array_equal(idx, g[f"idx_{c}"].astype(np.int64)), (c, int(T), int(E), int(k))
        np.testing.assert_allclose(w, g[f"w_{c}"], rtol=2e-6, atol=1e-7)


def test_a_mistake_in_the_tie_network_fails_the_golden(golden, monkeypatch):
    """The golden pins the order among ties: the network with its direction flags inverted fails it."""
    g = golden("topk_gpu.npz")
    stages = routing._bitonic_stages

    def flipped(width):
        return [(a, stride, ~flag) for a, stride, flag in stages(width)]

    monkeypatch.setattr(routing, "_bitonic_stages", flipped)
    x = (g["logits_1"].astype(np.uint32) << 16).view(np.float32)
    _, idx = routing.topk_softmax(x, 8)
    assert not np.array_equal(idx, g["idx_1"].astype(np.int64))


@pytest.mark.parametrize("T,E,k,q", [(4096, 128, 8, 0.0), (2048, 64, 6, 2.0), (4096, 8, 2, 0.0)])
def test_router_selection_matches_cpu_torch_topk_on_tied_bf16_logits(T, E, k, q):
    """torch.topk on the CPU (its order among equal values differs from the GPU's and is not pinned
    here): the probabilities of the oracle's experts are torch's top-k values, position by position,
    and the selected sets are equal wherever the k-th and (k+1)-th probabilities differ."""
    g = torch.Generator().manual_seed(T + E + k)
    logits = torch.randn(T, E, generator=g)
    if q:
        logits = (logits * q).round() / q
    logits = logits.to(torch.bfloat16).float()
    probs = torch.softmax(logits, dim=-1)
    vals, tidx = torch.topk(probs, k)
    _, idx = routing.topk_softmax(logits.numpy(), k)
    assert torch.equal(probs.gather(1, torch.from_numpy(idx)), vals)
    srt = probs.sort(dim=1, descending=True).values
    untied = (srt[:, k - 1] != srt[:, k]).numpy()
    assert np.array_equal(np.sort(idx[untied], 1), np.sort(tidx.numpy()[untied], 1))


def test_router_without_renormalisation_gives_the_softmax_probabilities():
    x = np.random.default_rng(1).standard_normal((8, 16)).astype(np.float32)
    w, idx = routing.topk_softmax(x, 3, renorm=False)
    p = torch.softmax(torch.from_numpy(x), -1).numpy()
    np.testing.assert_allclose(w, np.take_along_axis(p, idx, 1), rtol=1e-6)


def test_sort_matches_torch_stable_sort_and_bincount(golden):
    g = golden("routing.npz")
    perm, inv, offsets = routing.sort_by_expert(g["ids"], int(g["num_experts"]))
    assert np.array_equal(perm, g["perm"])
    assert np.array_equal(offsets, g["offsets"])
    assert np.array_equal(inv[perm], np.arange(perm.size))
    assert offsets[-1] < perm.size  # the sentinels sit past the last expert


# ---- products: golden fixture, closed forms, gradcheck ----

def test_reference_lora_matches_the_merged_weight_golden(golden):
    g = golden("lora.npz")
    offsets = np.cumsum(g["rows_per_expert"])
    x = torch.from_numpy(g["x"]).requires_grad_()
    lhs = torch.from_numpy(g["lhs"]).requires_grad_()
    rhs = torch.from_numpy(g["rhs"]).requires_grad_()
    out = grouped.reference_lora(x, torch.from_numpy(g["W"]), None, offsets, False, lhs, rhs, float(g["scaling"]),
                                 torch.from_numpy(g["bias"]), out_dtype=torch.float64)
    out.backward(torch.from_numpy(g["grad"]))
    np.testing.assert_allclose(out.detach().numpy(), g["out"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(x.grad.numpy(), g["grad_x"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lhs.grad.numpy(), g["grad_lhs"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(rhs.grad.numpy(), g["grad_rhs"], rtol=1e-5, atol=1e-6)


def test_reference_lora_rank_one_indicator_adapter_moves_one_column():
    torch.manual_seed(0)
    E, K, N = 2, 6, 5
    x = torch.randn(7, K)
    W = torch.randn(E, N, K) * 0.1
    lhs = torch.zeros(E, N, 1)
    rhs = torch.zeros(E, 1, K)
    lhs[1, 3, 0] = 1.0  # delta of expert 1 = unit at (out=3, in=2)
    rhs[1, 0, 2] = 1.0
    offsets = np.array([3, 7])
    out = grouped.reference_lora(x, W, None, offsets, False, lhs, rhs, 2.5)
    base = grouped.reference(x, W, offsets, False)
    expected = base.clone()
    expected[3:, 3] += 2.5 * x[3:, 2]
    torch.testing.assert_close(out, expected, rtol=1e-5, atol=1e-5)


def test_reference_lora_is_the_same_for_a_stack_and_its_transpose():
    torch.manual_seed(1)
    E, K, N, r = 3, 8, 6, 2
    x = torch.randn(10, K)
    W = torch.randn(E, N, K)
    lhs, rhs = torch.randn(E, N, r), torch.randn(E, r, K)
    scale = torch.rand(E, N) + 0.5  # per output row
    offsets = np.array([4, 4, 10])
    a = grouped.reference_lora(x, W, scale, offsets, False, lhs, rhs, 0.7)
    # transposed stack (E, in, out) with delta = lhs' @ rhs' = (lhs @ rhs)^T
    b = grouped.reference_lora(x, W.transpose(1, 2), scale, offsets, True, rhs.transpose(1, 2), lhs.transpose(1, 2), 0.7)
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


def test_reference_lora_gradients_pass_gradcheck():
    torch.manual_seed(2)
    E, K, N, r = 2, 4, 3, 2
    x = torch.randn(5, K, dtype=torch.float64, requires_grad=True)
    W = torch.randn(E, N, K, dtype=torch.float64)
    lhs = torch.randn(E, N, r, dtype=torch.float64, requires_grad=True)
    rhs = torch.randn(E, r, K, dtype=torch.float64, requires_grad=True)
    offsets = np.array([2, 5])
    f = lambda x, lhs, rhs: grouped.reference_lora(x, W, None, offsets, False, lhs, rhs, 1.3, out_dtype=torch.float64)
    assert torch.autograd.gradcheck(f, (x, lhs, rhs))


def test_reference_without_adapters_has_the_closed_form_input_gradient():
    # tests/test_grouped.py:146-157: out.sum() -> x.grad[row] = sum over n of W_e[n, :]
    torch.manual_seed(3)
    x = torch.randn(40, 64, requires_grad=True)
    W = torch.randn(2, 48, 64) * 0.05
    offsets = np.array([10, 40])
    grouped.reference_lora(x, W, None, offsets, False, None, None, 1.0).sum().backward()
    expected = W.sum(dim=1)[torch.repeat_interleave(torch.arange(2), torch.tensor([10, 30]))]
    torch.testing.assert_close(x.grad, expected, rtol=1e-5, atol=1e-5)


def test_one_expert_is_one_dense_product():
    torch.manual_seed(4)
    x, W = torch.randn(9, 32), torch.randn(1, 16, 32)
    torch.testing.assert_close(grouped.reference(x, W, np.array([9]), False), x @ W[0].t())


# ---- the layer: brute force per token ----

@pytest.mark.parametrize("is_transposed", [False, True])
def test_routed_forward_matches_the_per_token_loop(is_transposed):
    torch.manual_seed(5)
    T, H, I, E, k, r = 12, 16, 8, 5, 2, 3
    h = torch.randn(T, H)
    idx = torch.stack([torch.randperm(E)[:k] for _ in range(T)])
    idx[3, 1] = E  # a sentinel
    w = torch.softmax(torch.randn(T, k), -1)
    gu = torch.randn(E, 2 * I, H) * 0.2
    dn = torch.randn(E, H, I) * 0.2
    f = {"gate_up_proj": (torch.randn(E, 2 * I, r) * 0.3, torch.randn(E, r, H) * 0.3, 2.0),
         "down_proj": (torch.randn(E, H, r) * 0.3, torch.randn(E, r, I) * 0.3, 2.0)}
    if is_transposed:
        gu, dn = gu.transpose(1, 2).contiguous(), dn.transpose(1, 2).contiguous()
        f = {n: (b.transpose(1, 2), a.transpose(1, 2), s) for n, (a, b, s) in f.items()}
    got = moe.routed_forward(h, idx, w, gu, dn, f, E, is_transposed)
    want = moe.routed_forward_loop(h, idx, w, gu, dn, f, E, is_transposed)
    torch.testing.assert_close(got.double(), want, rtol=1e-4, atol=1e-5)


def test_swiglu_matches_the_elementwise_definition():
    g = torch.randn(3, 8)
    out = moe.swiglu(g)
    for i in range(3):
        for j in range(4):
            a, b = g[i, j].item(), g[i, 4 + j].item()
            assert abs(out[i, j].item() - a / (1 + np.exp(-a)) * b) < 1e-5


# ---- formats ----

def test_fp8_round_trip_stays_within_e4m3_precision_per_expert():
    # tests/test_fp8.py:122-131 of the reference
    torch.manual_seed(0)
    stack = torch.randn(4, 6, 8) * torch.tensor([0.01, 0.1, 1.0, 10.0]).view(4, 1, 1)
    q, scale = formats.fp8_quantize(stack)
    assert scale.shape == (4,)
    back = formats.fp8_dequantize(q, scale)
    for e in range(4):
        assert (back[e] - stack[e]).abs().max() <= stack[e].abs().max() * 0.07


def test_fp8_per_row_scales_bound_each_row():
    torch.manual_seed(1)
    stack = torch.randn(3, 5, 16) * torch.rand(3, 5, 1) * 10
    q, scale = formats.fp8_quantize(stack, per_row=True)
    assert scale.shape == (3, 5)
    back = formats.fp8_dequantize(q, scale)
    err = (back - stack).abs().amax(dim=2)
    assert (err <= stack.abs().amax(dim=2) * 0.07).all()
    qt, st = formats.fp8_quantize(stack.transpose(1, 2), per_row=True, is_transposed=True)
    torch.testing.assert_close(st, scale)
    torch.testing.assert_close(formats.fp8_dequantize(qt, st, True), back.transpose(1, 2))


def test_nf4_code_is_the_published_table():
    from meepsquared_amd._nf4 import NF4_CODE

    np.testing.assert_allclose(formats.nf4_code_from_definition(), NF4_CODE, atol=1e-6)


def test_nf4_round_trip_error_is_bounded_by_half_the_widest_code_gap():
    from meepsquared_amd._nf4 import NF4_CODE, dynamic_code

    rng = np.random.default_rng(0)
    x = (rng.standard_normal(64 * 300) * 0.02).astype(np.float32)
    packed, q, a2, off = formats.nf4_quantize(x, NF4_CODE, dynamic_code())
    back = formats.nf4_dequantize(packed, q, a2, off, NF4_CODE, dynamic_code())
    blocks = x.reshape(-1, 64)
    absmax = np.abs(blocks).max(axis=1)
    gap = np.diff(NF4_CODE).max() / 2
    # the absmax itself is 8-bit coded: allow its error on top of the code's half gap
    err = np.abs(back.reshape(-1, 64) - blocks).max(axis=1)
    assert (err <= absmax * (gap + 0.02) + 1e-7).all()
    assert packed.size == x.size // 2


def test_nf4_packs_the_first_value_in_the_high_nibble():
    from meepsquared_amd._nf4 import NF4_CODE, dynamic_code

    x = np.zeros(64, np.float32)
    x[0], x[1] = 1.0, -1.0  # codes 15 and 0
    packed, *_ = formats.nf4_quantize(x, NF4_CODE, dynamic_code())
    assert packed[0] == (15 << 4) | 0
    assert packed[1] == (7 << 4) | 7  # zeros


def test_fp8_row_quantisation_picks_the_smallest_power_of_two_scale():
    torch.manual_seed(3)
    x = torch.randn(40, 200) * torch.logspace(-3, 3, 40).unsqueeze(1)
    x[5] = 0.0
    x[7, :64] = 448.0  # exactly at the limit: e = 0
    x[8, :64] = 449.0  # just above: e = 1
    q, e8 = formats.fp8_rows_quantize(x)
    assert q.shape == (40, 256) and e8.shape == (4, 40)
    xp = torch.zeros(40, 256)
    xp[:, :200] = x
    for r in range(40):
        for b in range(4):
            amax = xp[r, 64 * b:64 * b + 64].abs().max().item()
            e = int(e8[b, r]) - 127
            if amax == 0:
                assert e == 0
            else:  # brute force: the smallest e with amax * 2^-e <= 448
                assert amax * 2.0 ** -e <= 448.0 and amax * 2.0 ** -(e - 1) > 448.0, (r, b, amax, e)
    assert int(e8[0, 7]) == 127 and int(e8[0, 8]) == 128
    back = formats.fp8_rows_dequantize(q, e8, 200)
    # e4m3 keeps 3 mantissa bits: every normal value within 2^-4 relative
    normal = back.abs() >= 2.0 ** -6 * torch.pow(2.0, e8.t().float() - 127).repeat_interleave(64, 1)[:, :200]
    assert ((back - x).abs() <= x.abs() * 2.0 ** -4 + 1e-30)[normal].all()
    assert not q[:, 200:].any()


def test_fp8_two_term_quantisation_is_hi_plus_the_quantised_exact_residual():
    """fp8_rows_quantize2: hi is the one-term quantisation; lo is the one-term quantisation of the
    residual x - hi·2^e1 computed in float64 (it equals the fp32 one: the subtraction is exact); the
    reconstruction is within 2^-7 of each block's amax (one term: 2^-4), on rows spanning six decades."""
    torch.manual_seed(4)
    x = (torch.randn(40, 200) * torch.logspace(-3, 3, 40).unsqueeze(1)).bfloat16().float()
    x[5] = 0.0
    q, words = formats.fp8_rows_quantize2(x)
    assert q.shape == (40, 512) and words.shape == (4, 40)
    hi1, e1 = formats.fp8_rows_quantize(x)
    qq = q.view(40, 4, 2, 64)
    assert torch.equal(qq[:, :, 0].reshape(40, 256), hi1) and torch.equal(words & 0xFF, e1)
    xp = torch.zeros(40, 256, dtype=torch.float64)
    xp[:, :200] = x.double()
    residual = xp - formats.fp8_rows_dequantize(hi1, e1, 256).double()
    assert torch.equal(residual.float().double(), residual)  # exact in fp32
    lo1, e2 = formats.fp8_rows_quantize(residual.float())
    assert torch.equal(qq[:, :, 1].reshape(40, 256), lo1) and torch.equal((words >> 8) & 0xFF, e2)
    rec = formats.fp8_rows_dequantize2(q, words, 200)
    err = (rec - x).abs().view(40, -1)
    for b in range(4):
        blk = slice(64 * b, min(64 * b + 64, 200))
        amax = x[:, blk].abs().amax(dim=1)
        assert torch.all((rec - x)[:, blk].abs().amax(dim=1) <= amax * 2.0 ** -7)
    one = formats.fp8_rows_dequantize(hi1, e1, 200)
    assert (rec - x).norm() < (one - x).norm() / 8  # the second term buys at least 3 bits


def test_dense_fp8_oracle_closed_forms():
    """fp8_tensor_quantize is fp8_quantize over one expert and keeps the reference's round-trip bound;
    fp8_scaled_mm of a diagonal weight scales x's columns; x @ W^T is (W @ x^T)^T; x @ W uses W untransposed."""
    torch.manual_seed(5)
    w = torch.randn(48, 32) * 0.3
    q, s = formats.fp8_tensor_quantize(w)
    q1, s1 = formats.fp8_quantize(w.unsqueeze(0))
    assert torch.equal(q.view(torch.uint8), q1[0].view(torch.uint8)) and torch.equal(s.reshape(1), s1)
    assert (q.float() * s - w).abs().max() <= 0.07 * w.abs().max()  # tests/test_fp8.py:122-131
    d = torch.tensor([1.0, 2.0, 0.5, -4.0, 0.25, 3.0, -1.0, 8.0])
    dq, ds = formats.fp8_tensor_quantize(torch.diag(d))
    x = torch.randn(5, 8)
    assert torch.allclose(formats.fp8_scaled_mm(x, dq, ds, True), x * (dq.float().diagonal() * ds), atol=1e-6)
    x = torch.randn(7, 32)
    y = formats.fp8_scaled_mm(x, q, s, True, bias=torch.ones(48))
    assert torch.allclose(y - 1, ((q.float() * s) @ x.t()).t(), atol=1e-5)
    g = torch.randn(7, 48)
    assert torch.allclose(formats.fp8_scaled_mm(g, q, s, False), g @ (q.float() * s), atol=1e-5)


def test_lora_mlp_oracle_equals_the_merged_weight_mlp():
    """oracle.grouped.lora_mlp_swiglu against the MLP on merged weights W + s·B·A in float64 (a different
    formulation: the adapters folded into the weights before the products)."""
    torch.manual_seed(6)
    H, I, r = 24, 40, 4
    def p(o, i, s):
        return torch.randn(o, i) * 0.1, torch.randn(r, i) * 0.2, torch.randn(o, r) * 0.2, s
    gate, up, down = p(I, H, 2.0), p(I, H, 0.5), p(H, I, 1.5)
    bias = (torch.randn(I), None, torch.randn(H))
    x = torch.randn(9, H)
    got = grouped.lora_mlp_swiglu(x, gate, up, down, bias)
    def merged(t):
        w, a, b, s = t
        return (w.double() + s * b.double() @ a.double())
    g = x.double() @ merged(gate).t() + bias[0].double()
    u = x.double() @ merged(up).t()
    want = (torch.nn.functional.silu(g) * u) @ merged(down).t() + bias[2].double()
    assert torch.allclose(got.double(), want, rtol=1e-4, atol=1e-5)
