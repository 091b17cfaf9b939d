"""The grouped product kernel against the per-expert float32 oracle (mirrors the reference's
tests/test_grouped.py), with the tolerances BASELINE states: relative Frobenius error <= 1e-2 for
bf16 stacks, <= 3e-2 for fp8/NF4 stacks (against the oracle on the dequantised weights)."""

import pytest
import torch

from helpers import offsets_of, rel
from oracle import formats
from oracle import grouped as ref

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
Q_TOL = 3e-2


@pytest.mark.parametrize("is_transposed", [False, True])
@pytest.mark.parametrize("rows_per_expert,K,N", [
    ([37, 0, 200, 64, 1], 96, 80),      # uneven groups, an empty one, sizes that are no multiples of the tiles
    ([300] * 8, 256, 128),              # even groups
    ([3], 2048, 1024),                  # one expert
    ([130, 0, 0, 257, 0], 2048, 1536),  # tiles cut mid-expert, trailing empty experts
])
def test_the_kernel_matches_one_product_per_expert(is_transposed, rows_per_expert, K, N):
    from meepsquared_amd import grouped_linear

    torch.manual_seed(0)
    rows, experts = sum(rows_per_expert), len(rows_per_expert)
    x = torch.randn(rows, K, device="cuda", dtype=torch.bfloat16)
    shape = (experts, K, N) if is_transposed else (experts, N, K)
    weight = torch.randn(shape, device="cuda", dtype=torch.bfloat16) * 0.05
    offsets = offsets_of(rows_per_expert)
    out = grouped_linear(x, weight, offsets, is_transposed)
    expected = ref.reference(x, weight, offsets.cpu(), is_transposed)
    torch.testing.assert_close(out.float(), expected.float(), atol=2e-2, rtol=2e-2)
    assert rel(out, ref.reference_lora(x, weight, None, offsets.cpu(), is_transposed, None, None, 1.0, out_dtype=torch.float32)) < BF16_TOL


@pytest.mark.parametrize("is_transposed", [False, True])
def test_the_kernel_takes_an_fp8_stack_as_weights_to_convert(is_transposed):
    from meepsquared_amd import grouped_linear

    torch.manual_seed(0)
    x = torch.randn(70, 64, device="cuda", dtype=torch.bfloat16)
    shape = (3, 64, 48) if is_transposed else (3, 48, 64)
    weight = (torch.randn(shape, device="cuda") * 0.05).to(torch.float8_e4m3fn)
    offsets = offsets_of([10, 40, 20])
    out = grouped_linear(x, weight, offsets, is_transposed, products_fp8=False)
    expected = ref.reference(x, weight.float(), offsets.cpu(), is_transposed)
    torch.testing.assert_close(out.float(), expected.float(), atol=2e-2, rtol=2e-2)


def test_rows_past_the_last_expert_are_left_alone():
    from meepsquared_amd import grouped_linear

    x = torch.randn(50, 64, device="cuda", dtype=torch.bfloat16)
    weight = torch.randn(2, 32, 64, device="cuda", dtype=torch.bfloat16)
    out = grouped_linear(x, weight, offsets_of([10, 20]), False)
    assert out.shape == (50, 32)
    expected = ref.reference(x[:30], weight, [10, 30], False)
    torch.testing.assert_close(out[:30].float(), expected.float(), atol=2e-2, rtol=2e-2)


def adapters(experts, K, N, rank, is_transposed):
    if is_transposed:
        lhs = torch.randn(experts, K, rank, device="cuda", dtype=torch.bfloat16) * 0.1
        rhs = torch.randn(experts, rank, N, device="cuda", dtype=torch.bfloat16) * 0.1
    else:
        lhs = torch.randn(experts, N, rank, device="cuda", dtype=torch.bfloat16) * 0.1
        rhs = torch.randn(experts, rank, K, device="cuda", dtype=torch.bfloat16) * 0.1
    return lhs.requires_grad_(), rhs.requires_grad_()


def run_both(x, weight, scale, offsets, is_transposed, lhs, rhs, scaling, bias, ref_weight=None, ref_scale="same",
             products_fp8=None):
    from meepsquared_amd import lora_linear

    out = lora_linear(x, weight, scale, offsets, is_transposed, lhs, rhs, scaling, bias, products_fp8)
    grad = torch.randn_like(out)
    out.backward(grad)
    got = (out.detach(), x.grad.clone(), lhs.grad.clone(), rhs.grad.clone())
    x.grad = lhs.grad = rhs.grad = None
    rw = weight if ref_weight is None else ref_weight
    rs = scale if ref_scale == "same" else ref_scale
    expected_out = ref.reference_lora(x, rw, rs, offsets.cpu(), is_transposed, lhs, rhs, scaling, bias, out_dtype=torch.float32)
    expected_out.backward(grad.float())
    expected = (expected_out.detach(), x.grad, lhs.grad, rhs.grad)
    x.grad = lhs.grad = rhs.grad = None
    return got, expected


@pytest.mark.parametrize("is_transposed", [False, True])
@pytest.mark.parametrize("fp8", [False, "expert", "row", "products", "products_row"])
@pytest.mark.parametrize("rank", [4, 16, 40])
def test_the_product_with_adapters_and_its_gradients_match_pytorch(is_transposed, fp8, rank):
    from meepsquared_amd import _fp8

    torch.manual_seed(0)
    rows_per_expert = [37, 0, 200, 64, 1]
    K, N = 96, 80
    experts = len(rows_per_expert)
    offsets = offsets_of(rows_per_expert)
    x = torch.randn(sum(rows_per_expert), K, device="cuda", dtype=torch.bfloat16).requires_grad_()
    shape = (experts, K, N) if is_transposed else (experts, N, K)
    weight = torch.randn(shape, device="cuda", dtype=torch.bfloat16) * 0.05
    scale = None
    if fp8:
        weight, scale = _fp8.quantize_stack(weight, per_row=fp8.endswith("row"), is_transposed=is_transposed)
    lhs, rhs = adapters(experts, K, N, rank, is_transposed)
    bias = torch.randn(experts, N, device="cuda", dtype=torch.bfloat16)
    products = bool(fp8) and fp8.startswith("products")
    got, expected = run_both(x, weight, scale, offsets, is_transposed, lhs, rhs, 2.0, bias,
                             ref_weight=weight.float() if fp8 else None, products_fp8=products)
    tol = Q_TOL if fp8 else BF16_TOL
    for name, a, b in zip(("out", "grad_x", "grad_lhs", "grad_rhs"), got, expected):
        assert a.shape == b.shape, name
        # with fp8 products the activations (and the output gradient) are two e4m3 terms per row and 64
        # columns: within BASELINE's 3e-2 like the stacks' own quantisation
        assert rel(a, b) < tol, (name, rel(a, b))
        # the reference's own bound (tests/test_grouped.py:141-143)
        torch.testing.assert_close(a.float(), b.float(), atol=1e-2 * b.float().abs().max().item(), rtol=0, msg=name)


@pytest.mark.parametrize("is_transposed", [False, True])
@pytest.mark.parametrize("N", [320, 4400])  # 4400: 18 column blocks, the items taken in groups of row tiles
def test_tall_items_match_one_product_per_expert(is_transposed, N):
    """Groups whose last tile holds at most 32 rows past a full one (257, 288, 513, 544, 800, 1300 rows) are
    run as one item of up to 288 rows; a remainder of at most 32 n rows past n >= 2 full tiles (545, 560, 576,
    801, 832, 864, 1100, 2000, 2100 rows) is spread over the last ceil(rem / 32) tiles, each of up to 288 rows;
    289, 577, 865 and 1535 rows keep a tile of their own.  Output, input gradient and both adapter gradients
    against the oracle, with a bias and a column block cut short (N = 320, and N = 4400, whose 18 column
    blocks the product takes in groups of row tiles)."""
    torch.manual_seed(0)
    rows_per_expert = [257, 288, 289, 0, 545, 544, 513, 256, 1, 800, 33, 290, 560, 576, 577, 801, 832, 833, 864,
                       865, 1100, 1300, 1535, 2000, 2100]
    K, rank = 160, 16
    experts = len(rows_per_expert)
    offsets = offsets_of(rows_per_expert)
    x = torch.randn(sum(rows_per_expert), K, device="cuda", dtype=torch.bfloat16).requires_grad_()
    shape = (experts, K, N) if is_transposed else (experts, N, K)
    weight = torch.randn(shape, device="cuda", dtype=torch.bfloat16) * 0.05
    lhs, rhs = adapters(experts, K, N, rank, is_transposed)
    bias = torch.randn(experts, N, device="cuda", dtype=torch.bfloat16)
    got, expected = run_both(x, weight, None, offsets, is_transposed, lhs, rhs, 2.0, bias)
    for name, a, b in zip(("out", "grad_x", "grad_lhs", "grad_rhs"), got, expected):
        assert rel(a, b) < BF16_TOL, (name, rel(a, b))
        torch.testing.assert_close(a.float(), b.float(), atol=1e-2 * b.float().abs().max().item(), rtol=0, msg=name)
    from meepsquared_amd import grouped_linear  # the base product alone (no adapters)

    out = grouped_linear(x.detach(), weight, offsets, is_transposed)
    want = ref.reference(x.detach(), weight, offsets.cpu(), is_transposed)
    assert rel(out, want) < BF16_TOL


@pytest.mark.parametrize("seed", range(6))
def test_random_groups_around_the_tile_boundaries_match_the_oracle(seed):
    """Seeded sweep: group sizes drawn around every tile boundary (0, 1, 31-33, 255-257, 287-289, 511-513,
    543-545, 575-577, 831-833 rows), random K and N (multiples of 8), both stack layouts, rank 0 / 8 / 16 /
    32, with or without a bias; output and all gradients against the oracle."""
    g = torch.Generator().manual_seed(100 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))]
    sizes = [0, 1, 31, 32, 33, 255, 256, 257, 287, 288, 289, 511, 512, 513, 543, 544, 545, 575, 576, 577, 600, 831,
             832, 833]
    experts = int(torch.randint(2, 9, (1,), generator=g))
    rows_per_expert = [pick(sizes) for _ in range(experts)]
    K, N = 8 * int(torch.randint(4, 40, (1,), generator=g)), 8 * int(torch.randint(4, 72, (1,), generator=g))
    rank, is_transposed, with_bias = pick([0, 8, 16, 32]), bool(seed % 2), seed % 3 != 0
    torch.manual_seed(seed)
    offsets = offsets_of(rows_per_expert)
    x = torch.randn(sum(rows_per_expert) + 5, K, device="cuda", dtype=torch.bfloat16)  # 5 rows past the last expert
    shape = (experts, K, N) if is_transposed else (experts, N, K)
    weight = torch.randn(shape, device="cuda", dtype=torch.bfloat16) * 0.05
    bias = torch.randn(experts, N, device="cuda", dtype=torch.bfloat16) if with_bias else None
    live = int(offsets[-1])
    case = (rows_per_expert, K, N, rank, is_transposed, with_bias)
    if rank == 0:
        from meepsquared_amd import grouped_linear

        out = grouped_linear(x, weight, offsets, is_transposed)
        want = ref.reference(x[:live], weight, offsets.cpu(), is_transposed)
        if live:
            assert rel(out[:live], want) < BF16_TOL, case
        return
    x = x[:live].clone().requires_grad_()
    lhs, rhs = adapters(experts, K, N, rank, is_transposed)
    got, expected = run_both(x, weight, None, offsets, is_transposed, lhs, rhs, 2.0, bias)
    for name, a, b in zip(("out", "grad_x", "grad_lhs", "grad_rhs"), got, expected):
        if b.float().norm() == 0:
            assert a.float().abs().max() == 0, (name, case)
            continue
        assert rel(a, b) < BF16_TOL, (name, rel(a, b), case)


def test_the_product_without_adapters_gives_the_base_and_its_input_gradient():
    from meepsquared_amd import lora_linear

    torch.manual_seed(0)
    offsets = offsets_of([10, 30])
    x = torch.randn(40, 64, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    weight = torch.randn(2, 48, 64, device="cuda", dtype=torch.bfloat16) * 0.05
    out = lora_linear(x, weight, None, offsets, False)
    out.sum().backward()
    torch.testing.assert_close(out.float(), ref.reference(x.detach(), weight, offsets.cpu(), False).float(), atol=2e-2, rtol=2e-2)
    expected = weight.sum(dim=1)[torch.repeat_interleave(torch.arange(2, device="cuda"), torch.tensor([10, 30], device="cuda"))]
    torch.testing.assert_close(x.grad.float(), expected.float(), atol=5e-2, rtol=3e-2)


@pytest.mark.parametrize("is_transposed", [False, True])
def test_an_nf4_stack_computes_what_its_dequantised_twin_computes(is_transposed):
    from meepsquared_amd import _nf4

    torch.manual_seed(0)
    rows_per_expert = [100, 0, 50, 170]
    K, N = 128, 192
    experts = len(rows_per_expert)
    offsets = offsets_of(rows_per_expert)
    x = torch.randn(sum(rows_per_expert), K, device="cuda", dtype=torch.bfloat16).requires_grad_()
    shape = (experts, K, N) if is_transposed else (experts, N, K)
    w = torch.randn(shape, device="cuda") * 0.02
    stack = _nf4.quantize_stack(w)
    twin = _nf4.dequantize_stack(stack, torch.float32)
    lhs, rhs = adapters(experts, K, N, 16, is_transposed)
    got, expected = run_both(x, stack, None, offsets, is_transposed, lhs, rhs, 2.0, None, ref_weight=twin)
    for name, a, b in zip(("out", "grad_x", "grad_lhs", "grad_rhs"), got, expected):
        assert rel(a, b) < Q_TOL, (name, rel(a, b))


@pytest.mark.parametrize("is_transposed", [False, True])
def test_an_empty_input_gives_an_empty_output_and_zero_adapter_gradients(is_transposed):
    """rows == 0 (src/meepsquared/_grouped.py:325-326): an empty output, an empty input gradient, and
    adapter gradients of zero (no row contributes)."""
    from meepsquared_amd import lora_linear

    E, K, N, r = 3, 64, 96, 16
    x = torch.zeros(0, K, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    offsets = torch.zeros(E, device="cuda", dtype=torch.int32)
    shape = (E, K, N) if is_transposed else (E, N, K)
    weight = torch.randn(shape, device="cuda", dtype=torch.bfloat16)
    lhs, rhs = adapters(E, K, N, r, is_transposed)
    out = lora_linear(x, weight, None, offsets, is_transposed, lhs, rhs, 2.0)
    assert out.shape == (0, N)
    out.backward(torch.zeros_like(out))
    assert x.grad.shape == (0, K)
    assert torch.count_nonzero(lhs.grad) == 0 and torch.count_nonzero(rhs.grad) == 0


def test_the_product_is_deterministic():
    from meepsquared_amd import lora_linear

    torch.manual_seed(3)
    offsets = offsets_of([500, 20, 700])
    x = torch.randn(1220, 256, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    weight = torch.randn(3, 384, 256, device="cuda", dtype=torch.bfloat16) * 0.05
    lhs, rhs = adapters(3, 256, 384, 16, False)
    grad = torch.randn(1220, 384, device="cuda", dtype=torch.bfloat16)
    results = []
    for _ in range(2):
        out = lora_linear(x, weight, None, offsets, False, lhs, rhs, 2.0)
        out.backward(grad)
        results.append((out.detach().clone(), x.grad.clone(), lhs.grad.clone(), rhs.grad.clone()))
        x.grad = lhs.grad = rhs.grad = None
    for a, b in zip(*results):
        assert torch.equal(a, b)


def test_qwen3_moe_sized_projection_stays_within_tolerance():
    """Config-1 shapes (E=128, ~512 rows per expert, gate_up 2048 -> 1536, rank 16, s = 2)."""
    from meepsquared_amd import lora_linear

    torch.manual_seed(4)
    E, K, N, r = 128, 2048, 1536, 16
    counts = torch.multinomial(torch.ones(E), 65536, replacement=True).bincount(minlength=E)
    offsets = torch.cumsum(counts, 0).to(torch.int32).cuda()
    x = torch.randn(65536, K, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    weight = torch.randn(E, N, K, device="cuda", dtype=torch.bfloat16) * 0.02
    lhs = (torch.randn(E, N, r, device="cuda") * 0.01).bfloat16().requires_grad_()
    rhs = ((torch.rand(E, r, K, device="cuda") * 2 - 1) / K ** 0.5).bfloat16().requires_grad_()
    got, expected = run_both(x, weight, None, offsets, False, lhs, rhs, 2.0, None)
    for name, a, b in zip(("out", "grad_x", "grad_lhs", "grad_rhs"), got, expected):
        assert rel(a, b) < BF16_TOL, (name, rel(a, b))


@pytest.mark.parametrize("E,A,B", [(3, 16, 200), (2, 130, 48), (1, 64, 64), (5, 1, 7), (4, 300, 16), (3, 32, 300),
                                   (2, 257, 32), (128, 16, 2048), (2, 12, 40), (3, 2048, 16), (2, 48, 136),
                                   (2, 32, 1000), (3, 1000, 32), (1, 136, 200)])
def test_the_batched_transpose_is_exact(E, A, B):
    """mlora_transpose (the adapters' roles in the input-gradient product): exact, any strides."""
    from meepsquared_amd._grouped import _transposed

    torch.manual_seed(E * 1000 + A + B)
    t = torch.randn(E, A, B, device="cuda").bfloat16()
    assert torch.equal(_transposed(t), t.transpose(1, 2).contiguous())
    s = torch.randn(E, B, A, device="cuda").bfloat16().transpose(1, 2)  # a strided view
    assert torch.equal(_transposed(s), s.transpose(1, 2).contiguous())


@pytest.mark.parametrize("rank,K,N", [(16, 2048, 1536), (12, 768, 2048), (20, 136, 200), (32, 40, 48)])
def test_the_swapped_adapters_in_one_launch_are_the_transposes(rank, K, N):
    """mlora_swap_adapters (both transposes of the input-gradient product's adapters in one launch, padded rank
    16 or 32) gives exactly the two transposes."""
    from meepsquared_amd import _grouped

    torch.manual_seed(rank + K + N)
    E = 7
    lhs, rhs = torch.randn(E, N, rank, device="cuda"), torch.randn(E, rank, K, device="cuda")
    a = _grouped._Adapters(lhs, rhs, False)
    sw = a.swapped()
    R = a.at.shape[1]
    assert sw.at.shape == (E, R, N) and sw.bt.shape == (E, K, R)
    assert torch.equal(sw.at, a.bt.transpose(1, 2)) and torch.equal(sw.bt, a.at.transpose(1, 2))


def test_two_projections_swapped_in_one_launch_are_the_transposes(monkeypatch):
    """mlora_swap_adapters_two: adapters paired as the layer pairs its down and gate_up adapters are both
    swapped by the first swapped() call, in one launch, exactly the transposes; the partner's result is
    taken once, and a later call swaps afresh."""
    from meepsquared_amd import _grouped

    torch.manual_seed(3)
    E = 5
    a = _grouped._Adapters(torch.randn(E, 2048, 16, device="cuda"), torch.randn(E, 16, 768, device="cuda"), False)
    b = _grouped._Adapters(torch.randn(E, 1536, 20, device="cuda"), torch.randn(E, 20, 2048, device="cuda"), False)
    a.partner = b
    names = []
    real_call = _grouped.call

    def call(name, *args):
        names.append(name)
        return real_call(name, *args)

    monkeypatch.setattr(_grouped, "call", call)
    sa = a.swapped()
    sb = b.swapped()
    assert names == ["mlora_swap_adapters_two"], names
    for x, sx in ((a, sa), (b, sb)):
        assert torch.equal(sx.at, x.bt.transpose(1, 2)) and torch.equal(sx.bt, x.at.transpose(1, 2))
    assert sb.padded == 32 and sb.rank == 20 and a.partner is None and b._swapped is None
    again = b.swapped()
    assert names[-1] == "mlora_swap_adapters" and again is not sb and torch.equal(again.at, sb.at)
    # a second projection of rank 8 (not padded to 16 or 32) is refused, naming which one
    from meepsquared_amd._lib import KernelError
    c = _grouped._Adapters(torch.randn(E, 64, 8, device="cuda"), torch.randn(E, 8, 64, device="cuda"), False)
    c.at, c.bt = c.at[:, :8].contiguous(), c.bt[:, :, :8].contiguous()
    sa, sc = a._empty_swapped(), c._empty_swapped()
    with pytest.raises(KernelError, match="second"):
        real_call("mlora_swap_adapters_two", *a._swap_args(sa), *c._swap_args(sc), None)


def test_the_swapped_adapters_take_each_others_roles():
    from meepsquared_amd import _grouped

    lhs, rhs = torch.randn(3, 10, 4, device="cuda"), torch.randn(3, 4, 12, device="cuda")
    a = _grouped._Adapters(lhs, rhs, False)
    sw = a.swapped()
    assert sw.at.shape == (3, 16, 10) and sw.bt.shape == (3, 12, 16) and sw.rank == 4
    assert torch.equal(sw.at, a.bt.transpose(1, 2)) and torch.equal(sw.bt, a.at.transpose(1, 2))


@pytest.mark.parametrize("is_transposed", [False, True])
@pytest.mark.parametrize("terms", [1, 2])
def test_the_fp8_product_quantizes_the_activations_per_row_and_stays_close(is_transposed, terms, monkeypatch):
    """Mirrors the reference's tests/test_grouped.py:68-81 (products_fp8=True) with its bounds for one e4m3
    term (the reference's single pass), and BASELINE's 3e-2 for the two terms this build uses by default."""
    from meepsquared_amd import grouped_linear

    monkeypatch.setenv("MEEPSQUARED_FP8_TERMS", str(terms))
    torch.manual_seed(0)
    x = torch.randn(300, 128, device="cuda", dtype=torch.bfloat16)
    x[::7] *= 20  # rows of different sizes: the scale is per row
    shape = (4, 128, 96) if is_transposed else (4, 96, 128)
    weight = (torch.randn(shape, device="cuda") * 0.05).to(torch.float8_e4m3fn)
    offsets = offsets_of([100, 0, 150, 50])
    expected = ref.reference(x, weight.float(), offsets.cpu(), is_transposed).float().cpu()
    out = grouped_linear(x, weight, offsets, is_transposed, products_fp8=True).float().cpu()
    if terms == 1:
        assert (out - expected).abs().max() <= 0.1 * expected.abs().max()
        assert (out - expected).norm() / expected.norm() < 0.06
    else:
        assert (out - expected).abs().max() <= 0.01 * expected.abs().max()
        assert (out - expected).norm() / expected.norm() < 3e-2


def test_the_fp8_products_switch_follows_the_environment(monkeypatch):
    from meepsquared_amd import _grouped

    w8 = torch.zeros(2, 16, 32, device="cuda").to(torch.float8_e4m3fn)
    wb = torch.zeros(2, 16, 32, device="cuda", dtype=torch.bfloat16)
    monkeypatch.delenv("MEEPSQUARED_FP8_PRODUCTS", raising=False)
    assert not _grouped._x_fp8(w8, None) and _grouped._x_fp8(w8, True) and not _grouped._x_fp8(wb, True)
    monkeypatch.setenv("MEEPSQUARED_FP8_PRODUCTS", "1")
    assert _grouped._x_fp8(w8, None) and not _grouped._x_fp8(w8, False)


@pytest.mark.parametrize("terms", [1, 2])
@pytest.mark.parametrize("K,colscale", [(208, False), (2048, False), (96, True)])
def test_the_fp8_activation_pass_is_bit_exact(K, colscale, terms):
    """mlora_fp8_prep against the oracle: e4m3 bytes (one term, or hi and lo) and E8M0 scales bit-exact;
    low = bf16(x · A_e)."""
    from meepsquared_amd import _lib

    torch.manual_seed(K)
    counts = [37, 0, 130, 64, 1]
    rows, E, R = sum(counts), len(counts), 16
    offsets = offsets_of(counts)
    x = (torch.randn(rows, K) * torch.logspace(-2, 2, rows).unsqueeze(1)).bfloat16().cuda()
    at = (torch.randn(E, R, K) * 0.1).bfloat16().cuda()
    cs = (torch.rand(E, K) + 0.5).cuda() if colscale else None
    nkb = (K + 63) // 64
    x8 = torch.empty(rows, terms * nkb * 64, dtype=torch.uint8, device="cuda")
    xs = torch.empty(nkb, rows, dtype=torch.int32, device="cuda")
    low = torch.empty(rows, R, dtype=torch.bfloat16, device="cuda")
    _lib.call("mlora_fp8_prep", _lib.ptr(x), x.stride(0), rows, K, terms, _lib.ptr(cs), cs.stride(0) if cs is not None else 0,
              _lib.ptr(x8), x8.stride(0), _lib.ptr(xs), xs.stride(0), _lib.ptr(at), at.stride(0), at.stride(1), R,
              _lib.ptr(low), low.stride(0), _lib.ptr(offsets), E, _lib.stream())
    torch.cuda.synchronize()
    expert = torch.repeat_interleave(torch.arange(E), torch.tensor(counts))
    xc = x.float().cpu()
    scaled = xc * cs.cpu()[expert] if colscale else xc
    q, e8 = formats.fp8_rows_quantize(scaled) if terms == 1 else formats.fp8_rows_quantize2(scaled)
    assert torch.equal(x8.cpu(), q)
    assert torch.equal(xs.cpu(), e8)
    low_ref = torch.einsum("rk,rjk->rj", xc.double(), at.cpu().double()[expert]).float()
    assert rel(low.float().cpu(), low_ref) < 1e-2


@pytest.mark.parametrize("kind", ["bf16", "fp8", "nf4"])
@pytest.mark.parametrize("is_transposed", [False, True])
@pytest.mark.parametrize("T", [300, 600])  # 600 tokens: ~300 rows per expert, tall items among them
def test_the_gathered_product_is_bit_identical_to_the_product_of_the_gathered_rows(is_transposed, T, kind):
    """lora_linear_gathered (rows read through perm, never materialised) against lora_linear on
    hidden[perm // k]: the same tiles and the same sums, so the same bits, gradients included; for bf16,
    fp8 (one scale per output row) and NF4 stacks."""
    from meepsquared_amd import _fp8, _grouped, _nf4, lora_linear, sort_by_expert
    from meepsquared_amd._moe import _Gather

    torch.manual_seed(5)
    k, E, K, N, r = 3, 6, 192, 128, 16
    idx = torch.randint(0, E, (T, k), device="cuda")
    idx[::11, 0] = E  # sentinel ids: rows after every expert
    perm, inv, offsets = sort_by_expert(idx, E)
    h = torch.randn(T, K, device="cuda", dtype=torch.bfloat16)
    weight = torch.randn((E, K, N) if is_transposed else (E, N, K), device="cuda", dtype=torch.bfloat16) * 0.05
    scale = None
    if kind == "fp8":
        weight, scale = _fp8.quantize_stack(weight, per_row=True, is_transposed=is_transposed)
    elif kind == "nf4":
        weight = _nf4.quantize_stack(weight)
    assert _grouped.gathered_product_fits(weight, False)
    lhs, rhs = adapters(E, K, N, r, is_transposed)
    bias = torch.randn(E, N, device="cuda", dtype=torch.bfloat16)
    grad = torch.randn(T * k, N, device="cuda", dtype=torch.bfloat16)
    live = int(offsets[-1])

    h1 = h.clone().requires_grad_()
    out1 = _grouped.lora_linear_gathered(h1, perm, inv, k, weight, scale, offsets, is_transposed, lhs, rhs, 2.0, bias)
    out1[:live].backward(grad[:live])
    g1 = (out1[:live].detach().clone(), h1.grad.clone(), lhs.grad.clone(), rhs.grad.clone())
    lhs.grad = rhs.grad = None

    h2 = h.clone().requires_grad_()
    sel = _Gather.apply(h2, perm, inv, offsets, k)  # the materialised rows, through the same gather kernel
    out2 = lora_linear(sel, weight, scale, offsets, is_transposed, lhs, rhs, 2.0, bias, products_fp8=False)
    out2[:live].backward(grad[:live])
    g2 = (out2[:live].detach(), h2.grad, lhs.grad, rhs.grad)
    for name, a, b in zip(("out", "grad_h", "grad_lhs", "grad_rhs"), g1, g2):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("kind", ["fp8", "nf4"])
@pytest.mark.parametrize("rank", [0, 16])
def test_a_quantised_stack_in_the_forward_product_is_bit_identical_to_its_decoded_twin(kind, rank):
    """fp8 e4m3 and NF4 stacks read with k contiguous are decoded in registers as the MFMA operands
    are read, inside the same product as a bf16 stack: the result is the product of the decoded bf16
    twin, to the bit (fp8 converted without a scale; NF4 blocks of 64 with their absmax)."""
    from meepsquared_amd import _nf4, grouped_linear, lora_linear

    torch.manual_seed(21 + rank)
    rows_per_expert = [100, 0, 300, 37]
    E, K, N = len(rows_per_expert), 256, 320
    offsets = offsets_of(rows_per_expert)
    x = torch.randn(sum(rows_per_expert), K, device="cuda").bfloat16()
    w = torch.randn(E, N, K, device="cuda") * 0.05
    if kind == "fp8":
        stack = w.to(torch.float8_e4m3fn)
        twin = stack.to(torch.bfloat16)
    else:
        stack = _nf4.quantize_stack(w)
        twin = _nf4.dequantize_stack(stack, torch.bfloat16)
    if rank == 0:
        got = grouped_linear(x, stack, offsets, False, products_fp8=False)
        want = grouped_linear(x, twin, offsets, False)
    else:
        lhs, rhs = torch.randn(E, N, rank, device="cuda").bfloat16() * 0.1, torch.randn(E, rank, K, device="cuda").bfloat16() * 0.1
        got = lora_linear(x, stack, None, offsets, False, lhs, rhs, 2.0, products_fp8=False)
        want = lora_linear(x, twin, None, offsets, False, lhs, rhs, 2.0)
    assert torch.equal(got, want)


@pytest.mark.parametrize("is_transposed", [False, True])
def test_the_input_gradient_through_an_fp8_stack_is_bit_identical_to_its_decoded_twin(is_transposed):
    """An fp8 stack with one scale per output row, products in bf16: the input-gradient product reads the
    stack with k contiguous (directly, or through its byte-transposed copy) and applies each row's scale
    along k in the decode, bf16(e4m3 · s): the gradient is that of the scaled bf16 twin, to the bit."""
    from meepsquared_amd import _fp8, lora_linear

    torch.manual_seed(5)
    rows_per_expert = [100, 0, 300, 37]
    E, K, N, r = len(rows_per_expert), 256, 320, 16
    offsets = offsets_of(rows_per_expert)
    w = (torch.randn((E, K, N) if is_transposed else (E, N, K), device="cuda") * 0.05).bfloat16()
    stack, scale = _fp8.quantize_stack(w, per_row=True, is_transposed=is_transposed)
    twin = (stack.float() * (scale[:, None, :] if is_transposed else scale[:, :, None])).bfloat16()
    if is_transposed:
        lhs, rhs = torch.randn(E, K, r, device="cuda") * 0.1, torch.randn(E, r, N, device="cuda") * 0.1
    else:
        lhs, rhs = torch.randn(E, N, r, device="cuda") * 0.1, torch.randn(E, r, K, device="cuda") * 0.1
    x = torch.randn(sum(rows_per_expert), K, device="cuda").bfloat16()
    dy = torch.randn(sum(rows_per_expert), N, device="cuda").bfloat16()
    grads = []
    for wt, sc in ((stack, scale), (twin, None)):
        xx = x.clone().requires_grad_()
        out = lora_linear(xx, wt, sc, offsets, is_transposed, lhs.bfloat16(), rhs.bfloat16(), 2.0, products_fp8=False)
        out.backward(dy)
        grads.append(xx.grad)
    assert torch.equal(grads[0], grads[1])


@pytest.mark.parametrize("is_transposed", [False, True])
def test_tall_items_of_an_fp8_stack_are_those_of_its_decoded_twin(is_transposed):
    """fp8 stacks take tall items too (a last tile of up to 288 rows, or a larger remainder spread over the
    last tiles, each of up to 288 rows): with one scale per output row and bf16 products, the output and the input gradient
    over groups at every tile boundary are those of the scaled bf16 twin, to the bit (the forward applies the
    row scale in the epilogue, so its check is to the oracle's bound instead)."""
    from meepsquared_amd import _fp8, lora_linear

    torch.manual_seed(13)
    rows_per_expert = [257, 288, 289, 545, 544, 560, 576, 577, 801, 832, 833, 40, 1100, 2000]
    E, K, N, r = len(rows_per_expert), 192, 320, 16
    offsets = offsets_of(rows_per_expert)
    w = (torch.randn((E, K, N) if is_transposed else (E, N, K), device="cuda") * 0.05).bfloat16()
    stack, scale = _fp8.quantize_stack(w, per_row=True, is_transposed=is_transposed)
    twin = (stack.float() * (scale[:, None, :] if is_transposed else scale[:, :, None])).bfloat16()
    if is_transposed:
        lhs, rhs = torch.randn(E, K, r, device="cuda") * 0.1, torch.randn(E, r, N, device="cuda") * 0.1
    else:
        lhs, rhs = torch.randn(E, N, r, device="cuda") * 0.1, torch.randn(E, r, K, device="cuda") * 0.1
    x = torch.randn(sum(rows_per_expert), K, device="cuda").bfloat16()
    dy = torch.randn(sum(rows_per_expert), N, device="cuda").bfloat16()
    res = []
    for wt, sc in ((stack, scale), (twin, None)):
        xx = x.clone().requires_grad_()
        out = lora_linear(xx, wt, sc, offsets, is_transposed, lhs.bfloat16(), rhs.bfloat16(), 2.0, products_fp8=False)
        out.backward(dy)
        res.append((out.detach(), xx.grad))
    assert torch.equal(res[0][1], res[1][1])
    assert rel(res[0][0], res[1][0]) < BF16_TOL


@pytest.mark.parametrize("is_transposed", [False, True])
@pytest.mark.parametrize("rows_per_expert", [[100, 0, 300, 37],
                                             [257, 288, 289, 545, 544, 560, 576, 577, 801, 832, 833, 40, 1100, 2000]])
def test_an_nf4_stack_read_the_other_way_is_bit_identical_to_its_decoded_twin(is_transposed, rows_per_expert):
    """The product that reads an NF4 stack with its blocks along n (the input gradient of a stack, or
    the forward of a transposed one) goes through the stack's transposed codes and absmax table: each
    value decodes as bf16(code · absmax) with the absmax of its own block, so the input gradient (and,
    for a transposed stack, the output) is that of the decoded bf16 twin, to the bit; the second group
    list puts a group at every tile boundary (the sizes bf16 and fp8 stacks take as tall items; NF4
    stacks run them as full tiles plus a partial one)."""
    from meepsquared_amd import _nf4, lora_linear

    torch.manual_seed(8)
    E, K, N, r = len(rows_per_expert), 256, 320, 16
    offsets = offsets_of(rows_per_expert)
    w = torch.randn((E, K, N) if is_transposed else (E, N, K), device="cuda") * 0.05
    stack = _nf4.quantize_stack(w)
    twin = _nf4.dequantize_stack(stack, torch.bfloat16)
    if is_transposed:
        lhs, rhs = torch.randn(E, K, r, device="cuda") * 0.1, torch.randn(E, r, N, device="cuda") * 0.1
    else:
        lhs, rhs = torch.randn(E, N, r, device="cuda") * 0.1, torch.randn(E, r, K, device="cuda") * 0.1
    x = torch.randn(sum(rows_per_expert), K, device="cuda").bfloat16()
    dy = torch.randn(sum(rows_per_expert), N, device="cuda").bfloat16()
    res = []
    for wt in (stack, twin):
        xx = x.clone().requires_grad_()
        out = lora_linear(xx, wt, None, offsets, is_transposed, lhs.bfloat16(), rhs.bfloat16(), 2.0)
        out.backward(dy)
        res.append((out.detach(), xx.grad))
    assert torch.equal(res[0][1], res[1][1])
    if is_transposed:
        assert torch.equal(res[0][0], res[1][0])


@pytest.mark.parametrize("is_transposed", [False, True])
def test_a_scale_of_the_wrong_shape_is_refused(is_transposed):
    """A per-row scale must be (experts, out rows of the stack): (E, in) or a wrong length is a
    ValueError naming the shape it needs, forward and backward alike."""
    from meepsquared_amd import _fp8, lora_linear

    E, K, N = 3, 64, 48
    w = torch.randn((E, K, N) if is_transposed else (E, N, K), device="cuda") * 0.05
    stack, scale = _fp8.quantize_stack(w, per_row=True, is_transposed=is_transposed)
    assert scale.shape == (E, N)
    x = torch.randn(30, K, device="cuda", dtype=torch.bfloat16)
    offsets = offsets_of([10, 10, 10])
    for bad in (torch.ones(E, K, device="cuda"), torch.ones(E, N + 8, device="cuda"), torch.ones(E + 1, device="cuda")):
        with pytest.raises(ValueError, match=f"\\({E}, {N}\\)|{E} values"):
            lora_linear(x, stack, bad, offsets, is_transposed, products_fp8=False)
    lora_linear(x, stack, scale, offsets, is_transposed, products_fp8=False)  # the right shape is taken


@pytest.mark.parametrize("kind", ["bf16", "fp8", "fp8_row", "nf4"])
@pytest.mark.parametrize("is_transposed", [False, True])
@pytest.mark.parametrize("rank", [0, 16])
def test_the_gathered_product_with_swiglu_is_the_product_then_swiglu(kind, is_transposed, rank, monkeypatch):
    """mlora_grouped_gemm_gather_swiglu: out and low carry the bits of mlora_grouped_gemm_gather_q's, and act
    those of mlora_swiglu(out), though each tile now holds 128 gate columns and the 128 up columns paired
    with them (I = 384: three tiles); experts of 1, 257 (tall), 288 (tall, full), 300, 0 and 545 rows and
    sentinel rows; a bias; bf16, fp8 (per expert, per output row) and NF4 stacks."""
    from meepsquared_amd import _fp8, _grouped, _lib, _nf4, sort_by_expert
    from meepsquared_amd._lib import call, ptr

    monkeypatch.setenv("MEEPSQUARED_FUSED_SWIGLU", "1")
    torch.manual_seed(31 + rank)
    counts = [1, 257, 288, 300, 0, 545, 40]
    E, k, K, I = len(counts), 3, 192, 384
    N = 2 * I
    ids = torch.repeat_interleave(torch.arange(E + 1), torch.tensor(counts + [3]))  # 3 sentinel rows
    idx = ids[torch.randperm(ids.numel())].reshape(-1, k).cuda()
    T = idx.shape[0]
    perm, inv, offsets = sort_by_expert(idx, E)
    offsets = offsets.to(torch.int32)
    h = torch.randn(T, K, device="cuda", dtype=torch.bfloat16)
    weight = torch.randn((E, K, N) if is_transposed else (E, N, K), device="cuda", dtype=torch.bfloat16) * 0.05
    scale = None
    if kind in ("fp8", "fp8_row"):
        weight, scale = _fp8.quantize_stack(weight, per_row=kind == "fp8_row", is_transposed=is_transposed)
    elif kind == "nf4":
        weight = _nf4.quantize_stack(weight)
    ad = _grouped._Adapters(*adapters(E, K, N, rank, is_transposed), is_transposed) if rank else None
    bias = torch.randn(E, N, device="cuda", dtype=torch.bfloat16)
    args = (h, perm, k, weight, scale, offsets, is_transposed, ad, 2.0, bias)
    out, low, act = _grouped._launch_gathered(*args, swiglu=True)
    out2, low2 = _grouped._launch_gathered(*args)
    act2 = torch.empty_like(act)
    call("mlora_swiglu", ptr(out2), out2.shape[0], I, ptr(act2), _lib.stream())
    torch.cuda.synchronize()
    live = int(offsets[-1])
    assert torch.equal(out[:live], out2[:live])
    if rank:
        assert torch.equal(low[:live], low2[:live])
    assert torch.equal(act[:live], act2[:live])
    assert act[:live].abs().sum() > 0


@pytest.mark.parametrize("rank", [0, 16])
def test_the_gathered_product_with_swiglu_over_more_experts_than_take_tall_items(rank, monkeypatch):
    """With more than 1024 experts the product runs without tall items (the launch's other instantiation):
    1100 experts, a few holding 257-300 rows (a full tile and a small one), the rest 0-40 rows; out, low and
    act as in the product then mlora_swiglu, to the bit."""
    from meepsquared_amd import _grouped, _lib, sort_by_expert
    from meepsquared_amd._lib import call, ptr

    monkeypatch.setenv("MEEPSQUARED_FUSED_SWIGLU", "1")
    torch.manual_seed(41 + rank)
    E, k, K, I = 1100, 2, 128, 128
    N = 2 * I
    counts = torch.randint(0, 41, (E,))
    counts[[3, 500, 1099]] = torch.tensor([257, 300, 290])
    total = int(counts.sum())
    pad = (-total) % k
    ids = torch.repeat_interleave(torch.arange(E + 1), torch.cat([counts, torch.tensor([pad])]))
    idx = ids[torch.randperm(ids.numel())].reshape(-1, k).cuda()
    T = idx.shape[0]
    perm, inv, offsets = sort_by_expert(idx, E)
    offsets = offsets.to(torch.int32)
    h = torch.randn(T, K, device="cuda", dtype=torch.bfloat16)
    weight = torch.randn(E, N, K, device="cuda", dtype=torch.bfloat16) * 0.05
    ad = _grouped._Adapters(*adapters(E, K, N, rank, False), False) if rank else None
    args = (h, perm, k, weight, None, offsets, False, ad, 2.0, None)
    out, low, act = _grouped._launch_gathered(*args, swiglu=True)
    out2, low2 = _grouped._launch_gathered(*args)
    act2 = torch.empty_like(act)
    call("mlora_swiglu", ptr(out2), out2.shape[0], I, ptr(act2), _lib.stream())
    torch.cuda.synchronize()
    live = int(offsets[-1])
    assert torch.equal(out[:live], out2[:live])
    if rank:
        assert torch.equal(low[:live], low2[:live])
    assert torch.equal(act[:live], act2[:live])


def test_the_gathered_product_with_swiglu_refuses_what_it_does_not_pair(monkeypatch):
    """N = 2 I must be a multiple of 256 (each tile pairs 128 gate and 128 up columns), the product a forward
    one and the adapters of rank 16 or none: the host refuses N = 400 and rank 32, and so does the C entry
    point."""
    from meepsquared_amd import _grouped, _lib, sort_by_expert
    from meepsquared_amd._lib import KernelError, ptr

    E, k, K, N, T = 2, 2, 64, 400, 16
    idx = torch.randint(0, E, (T, k), device="cuda")
    perm, inv, offsets = sort_by_expert(idx, E)
    offsets = offsets.to(torch.int32)
    h = torch.randn(T, K, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(E, N, K, device="cuda", dtype=torch.bfloat16)
    monkeypatch.setenv("MEEPSQUARED_FUSED_SWIGLU", "0")
    assert not _grouped.swiglu_fusable(512)  # the separate pass, asked for
    monkeypatch.delenv("MEEPSQUARED_FUSED_SWIGLU", raising=False)  # on by default
    assert not _grouped.swiglu_fusable(N) and _grouped.swiglu_fusable(512) and _grouped.swiglu_fusable(512, 16)
    assert not _grouped.swiglu_fusable(512, backward=True) and not _grouped.swiglu_fusable(512, 32)
    with pytest.raises(ValueError, match="N % 256"):
        _grouped._launch_gathered(h, perm, k, w, None, offsets, False, None, 1.0, None, swiglu=True)
    out = torch.empty(T * k, N, device="cuda", dtype=torch.bfloat16)
    act = torch.empty(T * k, N // 2, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(KernelError, match="multiple of 256"):
        _lib.call("mlora_grouped_gemm_gather_swiglu", ptr(h), K, T, ptr(perm), k, T * k, K, N, ptr(w), _lib.dtype_code(w.dtype),
                  w.stride(0), w.stride(2), w.stride(1), None, 0, 0, None, None, None, None, None,
                  None, 0, 0, None, 0, 0, 0, 1.0, None, 0, ptr(out), N, None, 0, ptr(act), N // 2,
                  ptr(offsets), E, _lib.stream())
    N = 512  # pairs, but rank 32 is not taken
    w = torch.randn(E, N, K, device="cuda", dtype=torch.bfloat16)
    at = torch.randn(E, 32, K, device="cuda", dtype=torch.bfloat16)
    bt = torch.randn(E, N, 32, device="cuda", dtype=torch.bfloat16)
    out = torch.empty(T * k, N, device="cuda", dtype=torch.bfloat16)
    act = torch.empty(T * k, N // 2, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(KernelError, match="rank 16 or none"):
        _lib.call("mlora_grouped_gemm_gather_swiglu", ptr(h), K, T, ptr(perm), k, T * k, K, N, ptr(w),
                  _lib.dtype_code(w.dtype), w.stride(0), w.stride(2), w.stride(1), None, 0, 0, None, None, None, None,
                  None, ptr(at), at.stride(0), at.stride(1), ptr(bt), bt.stride(0), bt.stride(1), 32, 1.0, None, 0,
                  ptr(out), N, None, 0, ptr(act), N // 2, ptr(offsets), E, _lib.stream())


def test_the_gathered_products_refuse_what_their_kernel_does_not_take():
    """The gathered product reads bf16, fp8 and NF4 stacks whose rows are whole 16-byte chunks (NF4: 64-code
    blocks) and applies a per-row stack scale along k only in the fp8 decode: an fp8 stack with rows of 72
    bytes and a float32 stack are TypeErrors, a bf16 stack's per-row scale in the input-gradient pass a
    ValueError (lora_linear takes all three)."""
    from meepsquared_amd import _fp8, _grouped, sort_by_expert

    E, K, N, k, T = 3, 72, 48, 2, 20
    idx = torch.randint(0, E, (T, k), device="cuda")
    perm, inv, offsets = sort_by_expert(idx, E)
    h = torch.randn(T, K, device="cuda", dtype=torch.bfloat16)
    w8, s8 = _fp8.quantize_stack(torch.randn(E, N, K, device="cuda") * 0.05, per_row=True)
    with pytest.raises(TypeError, match="16-byte chunks"):
        _grouped.lora_linear_gathered(h, perm, inv, k, w8, s8, offsets, False)
    with pytest.raises(TypeError, match="16-byte chunks"):
        _grouped.lora_linear_gathered(h, perm, inv, k, torch.randn(E, N, K, device="cuda"), None, offsets, False)
    K = 64
    h = torch.randn(T, K, device="cuda", dtype=torch.bfloat16)
    wb = torch.randn(E, N, K, device="cuda", dtype=torch.bfloat16)
    x = torch.randn(T * k, K, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    wts = torch.rand(T, k, device="cuda")
    out = _grouped.lora_linear_combined(x, wts, perm, inv, k, wb, torch.ones(E, N, device="cuda"), offsets, False)
    with pytest.raises(ValueError, match="per-output-row"):
        out.backward(torch.ones_like(out))


@pytest.mark.parametrize("is_transposed", [False, True])
def test_adapter_gradients_of_experts_split_into_parts(is_transposed):
    """Experts with more rows than a reduction part (here 9000 and 5000 rows, parts of 4096 at this mean)
    are summed in parts through the workspace and added in part order: the adapters' gradients match the
    oracle and are the same bits on a second run; an empty expert's gradients are zero."""
    from meepsquared_amd import lora_linear

    torch.manual_seed(17)
    rows_per_expert = [9000, 10, 0, 5000]
    E, K, N, r = len(rows_per_expert), 128, 96, 16
    offsets = offsets_of(rows_per_expert)
    x = torch.randn(sum(rows_per_expert), K, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    weight = torch.randn((E, K, N) if is_transposed else (E, N, K), device="cuda", dtype=torch.bfloat16) * 0.05
    lhs, rhs = adapters(E, K, N, r, is_transposed)
    got, expected = run_both(x, weight, None, offsets, is_transposed, lhs, rhs, 2.0, None)
    for name, a, b in zip(("out", "grad_x", "grad_lhs", "grad_rhs"), got, expected):
        assert rel(a, b) < BF16_TOL, (name, rel(a, b))
    assert torch.count_nonzero(got[2][2]) == 0 and torch.count_nonzero(got[3][2]) == 0
    grad = torch.randn_like(got[0])
    runs = []
    for _ in range(2):
        out = lora_linear(x, weight, None, offsets, is_transposed, lhs, rhs, 2.0)
        out.backward(grad)
        runs.append((lhs.grad.clone(), rhs.grad.clone()))
        x.grad = lhs.grad = rhs.grad = None
    assert torch.equal(runs[0][0], runs[1][0]) and torch.equal(runs[0][1], runs[1][1])


@pytest.mark.parametrize("seed", range(6))
def test_the_fused_adapter_gradient_matches_the_standalone_reduction(seed):
    """mlora_grouped_gemm_db against the product launch and mlora_grouped_reduce(_gather) over the same rows:
    the product and its low are the same bits; B's gradient (summed per 256-row tile on the MFMA, the tiles
    added in row order) within 5e-3 of the standalone reduction and 1e-2 of an fp32 sum, and the same bits
    on a second run.  Seeded group sizes around the tile boundaries (tall items of 513-544 rows included),
    K a multiple of 8 but not of 64, gathered rows with per-row weights, both output layouts."""
    from meepsquared_amd import _grouped

    g = torch.Generator().manual_seed(300 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))]
    sizes = [0, 1, 31, 33, 255, 256, 257, 288, 289, 511, 513, 530, 544, 545, 700]
    E = int(torch.randint(2, 9, (1,), generator=g))
    rows_per_expert = [pick(sizes) for _ in range(E)]
    K, N = 8 * int(torch.randint(4, 100, (1,), generator=g)), 8 * int(torch.randint(4, 72, (1,), generator=g))
    is_transposed, transposed_out, gathered = bool(seed % 2), bool(seed // 2 % 2), seed >= 3
    print("case", rows_per_expert, K, N, is_transposed, transposed_out, gathered, flush=True)
    torch.manual_seed(seed)
    offsets = offsets_of(rows_per_expert)
    rows = sum(rows_per_expert)
    weight = torch.randn((E, K, N) if is_transposed else (E, N, K), device="cuda", dtype=torch.bfloat16) * 0.05
    lhs, rhs = adapters(E, K, N, 16, is_transposed)
    ad = _grouped._Adapters(lhs.detach(), rhs.detach(), is_transposed)
    l = torch.randn(rows, 16, device="cuda", dtype=torch.bfloat16)
    if gathered:
        k = 4
        T = rows // k + 3
        src = torch.randn(T, K, device="cuda", dtype=torch.bfloat16)
        perm = torch.randperm(T * k, device="cuda")[:rows]
        w = torch.rand(T * k, device="cuda")
        out_r, low_r = _grouped._launch_gathered(src, perm, k, weight, None, offsets, is_transposed, ad, 2.0, None,
                                                 row_scale=w, backward=True)
        grad_r = _grouped._reduce(src, l, offsets, 2.0, transposed=transposed_out, gather=(perm, k), row_scale=(w, perm))
        fused = lambda: _grouped._launch_db(src, weight, None, offsets, is_transposed, ad, 2.0, l, transposed_out,
                                            gather=(perm, k), row_scale=w, db_weight=(w, perm))
        x = src[perm // k].float()
        lw = (l.float() * w[perm][:, None]).bfloat16().float()
    else:
        src = torch.randn(rows, K, device="cuda", dtype=torch.bfloat16)
        out_r, low_r = _grouped._launch(src, weight, None, offsets, is_transposed, ad, 2.0, None, True, backward=True)
        grad_r = _grouped._reduce(src, l, offsets, 2.0, transposed=transposed_out)
        fused = lambda: _grouped._launch_db(src, weight, None, offsets, is_transposed, ad, 2.0, l, transposed_out)
        x, lw = src.float(), l.float()
    out, low, grad = fused()
    assert torch.equal(out, out_r) and torch.equal(low, low_r)
    exact = torch.zeros(E, K, 16, device="cuda")
    starts = [0] + offsets.tolist()
    for e in range(E):
        a, b = starts[e], starts[e + 1]
        exact[e] = 2.0 * (x[a:b].T @ lw[a:b])
    if transposed_out:
        exact = exact.transpose(1, 2)
    assert rel(grad, grad_r) < 5e-3, rel(grad, grad_r)
    assert rel(grad, exact) < 1e-2, rel(grad, exact)
    for e, n in enumerate(rows_per_expert):
        if n == 0:
            assert torch.count_nonzero(grad[e]) == 0
    assert torch.equal(fused()[2], grad)
