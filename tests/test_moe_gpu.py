"""The routed MoE-LoRA layer (router -> sort -> gather -> gate_up -> SwiGLU -> down -> combine),
forward and backward, against the oracle's composition of the reference's fp32 per-expert path."""

import numpy as np
import pytest
import torch

from helpers import kaiming_uniform, rel
from oracle import moe as ref_moe

pytestmark = pytest.mark.gpu


def make_layer(T, H, I, E, k, r, alpha, seed=0, is_transposed=False, zipf=0.0):
    """Config-0 style synthetic inputs: x, logits ~ N(0,1), W ~ N(0, 0.02), A Kaiming-uniform, B ~ N(0, 0.01).
    zipf > 0 biases the logits by -zipf * ln(e + 1), so that expert e's load falls roughly as (e + 1)^-zipf."""
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(T, H, generator=g)
    logits = torch.randn(T, E, generator=g) - zipf * torch.log(torch.arange(1, E + 1, dtype=torch.float32))
    gu = torch.randn(E, 2 * I, H, generator=g) * 0.02
    dn = torch.randn(E, H, I, generator=g) * 0.02
    f = {"gate_up_proj": (torch.randn(E, 2 * I, r, generator=g) * 0.01, kaiming_uniform((E, r, H), H, g), alpha / r),
         "down_proj": (torch.randn(E, H, r, generator=g) * 0.01, kaiming_uniform((E, r, I), I, g), alpha / r)}
    if is_transposed:
        gu, dn = gu.transpose(1, 2).contiguous(), dn.transpose(1, 2).contiguous()
        f = {n: (b.transpose(1, 2).contiguous(), a.transpose(1, 2).contiguous(), s) for n, (a, b, s) in f.items()}
    return h, logits, gu, dn, f


def run_layer(T, H, I, E, k, r, alpha, is_transposed=False, sentinel_frac=0.0, seed=0, fp8=None, nf4=False,
              zipf=0.0, bias=False):
    from meepsquared_amd import Experts, _fp8, _nf4, routed_forward, topk_softmax

    h, logits, gu, dn, f = make_layer(T, H, I, E, k, r, alpha, seed, is_transposed, zipf)
    dev = "cuda"
    hb = h.to(dev, torch.bfloat16).requires_grad_()
    w, idx = topk_softmax(logits.to(dev, torch.bfloat16), k)
    if sentinel_frac:
        mask = torch.rand(idx.shape, generator=torch.Generator().manual_seed(9)) < sentinel_frac
        idx = torch.where(mask.to(dev), torch.full_like(idx, E), idx)
    w = w.detach().requires_grad_()
    gub, dnb = gu.to(dev, torch.bfloat16), dn.to(dev, torch.bfloat16)
    scales = {}
    if fp8:
        gub, s1 = _fp8.quantize_stack(gub, per_row=fp8 == "row", is_transposed=is_transposed)
        dnb, s2 = _fp8.quantize_stack(dnb, per_row=fp8 == "row", is_transposed=is_transposed)
        scales = {"gate_up_proj": s1, "down_proj": s2}
    if nf4:
        gub, dnb = _nf4.quantize_stack(gub), _nf4.quantize_stack(dnb)
    biases = {}
    if bias:  # bias stacks (experts, out), as gpt-oss's experts hold them
        bg = torch.Generator().manual_seed(seed + 7)
        biases = {"gate_up_proj": (torch.randn(E, 2 * I, generator=bg) * 0.1).to(dev, torch.bfloat16),
                  "down_proj": (torch.randn(E, H, generator=bg) * 0.1).to(dev, torch.bfloat16)}
    experts = Experts(gub, dnb, is_transposed, scales.get("gate_up_proj"), scales.get("down_proj"),
                      biases.get("gate_up_proj"), biases.get("down_proj"))
    fb = {n: (a.to(dev, torch.bfloat16).requires_grad_(), b.to(dev, torch.bfloat16).requires_grad_(), s)
          for n, (a, b, s) in f.items()}
    out = routed_forward(experts, hb, idx, w, fb)
    dy = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed + 1)).to(dev, torch.bfloat16)
    out.backward(dy)
    got = {"out": out.detach(), "dh": hb.grad, "dw": w.grad}
    for n, (a, b, _) in fb.items():
        got[n + ".lhs"], got[n + ".rhs"] = a.grad, b.grad

    # the oracle in float32 on the same (bf16-rounded) values, the fp8 stacks dequantised
    h32 = hb.detach().float().requires_grad_()
    w32 = w.detach().float().requires_grad_()
    if nf4:  # the oracle runs on the stacks' decoded values
        gu32, dn32 = _nf4.dequantize_stack(gub, torch.float32), _nf4.dequantize_stack(dnb, torch.float32)
    else:
        gu32, dn32 = gub.float(), dnb.float()
    f32 = {n: (a.detach().float().requires_grad_(), b.detach().float().requires_grad_(), s) for n, (a, b, s) in fb.items()}
    o32 = ref_moe.routed_forward(h32, idx, w32, gu32, dn32, f32, E, is_transposed, scales=scales,
                                 biases={n: b.float() for n, b in biases.items()})
    o32.backward(dy.float())
    want = {"out": o32.detach(), "dh": h32.grad, "dw": w32.grad}
    for n, (a, b, _) in f32.items():
        want[n + ".lhs"], want[n + ".rhs"] = a.grad, b.grad
    return got, want


@pytest.mark.parametrize("is_transposed", [False, True])
def test_config0_layer_forward_and_backward(is_transposed):
    # BASELINE config 0 shapes: T=512, H=256, I=512, E=8, top-2, r=8, alpha=16
    got, want = run_layer(512, 256, 512, 8, 2, 8, 16, is_transposed)
    for name in want:
        assert rel(got[name], want[name]) < 1e-2, (name, rel(got[name], want[name]))


@pytest.mark.parametrize("is_transposed", [False, True])
def test_layer_with_bias_stacks(is_transposed):
    # experts with a bias per output (gpt-oss): the down product keeps y for the combine weights' gradient
    got, want = run_layer(300, 128, 64, 8, 2, 16, 32, is_transposed, sentinel_frac=0.05, seed=6, bias=True)
    for name in want:
        assert rel(got[name], want[name]) < 1e-2, (name, rel(got[name], want[name]))


def test_layer_with_every_id_a_sentinel():
    # every (token, slot) routed to another rank (ids >= E): the layer adds nothing, and every
    # gradient is zero
    got, want = run_layer(64, 128, 64, 8, 2, 16, 32, sentinel_frac=1.0)
    for name in want:
        assert torch.count_nonzero(got[name]) == 0, name
        assert want[name] is None or torch.count_nonzero(want[name]) == 0, name  # (None: no path to it)


def test_layer_on_no_tokens():
    from meepsquared_amd import Experts, routed_forward, topk_softmax

    E, H, I, k, r = 8, 128, 64, 2, 16
    h = torch.zeros(0, H, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    w, idx = topk_softmax(torch.zeros(0, E, device="cuda", dtype=torch.bfloat16), k)
    assert w.shape == (0, k) and idx.shape == (0, k)
    gu = torch.randn(E, 2 * I, H, device="cuda").bfloat16()
    dn = torch.randn(E, H, I, device="cuda").bfloat16()
    f = {"gate_up_proj": (torch.zeros(E, 2 * I, r, device="cuda").bfloat16().requires_grad_(),
                          torch.zeros(E, r, H, device="cuda").bfloat16().requires_grad_(), 2.0),
         "down_proj": (torch.zeros(E, H, r, device="cuda").bfloat16().requires_grad_(),
                       torch.zeros(E, r, I, device="cuda").bfloat16().requires_grad_(), 2.0)}
    out = routed_forward(Experts(gu, dn), h, idx, w.requires_grad_(), f)
    assert out.shape == (0, H)
    out.backward(torch.zeros_like(out))
    assert h.grad.shape == (0, H)
    for a, b, _ in f.values():
        assert torch.count_nonzero(a.grad) == 0 and torch.count_nonzero(b.grad) == 0


def test_layer_with_sentinel_ids():
    got, want = run_layer(300, 128, 64, 8, 2, 16, 32, sentinel_frac=0.1)
    for name in want:
        assert rel(got[name], want[name]) < 1e-2, (name, rel(got[name], want[name]))


@pytest.mark.parametrize("fp8", ["expert", "row"])
def test_layer_with_fp8_stacks_matches_the_dequantised_twin(fp8):
    got, want = run_layer(512, 256, 512, 8, 2, 8, 16, fp8=fp8)
    for name in want:
        assert rel(got[name], want[name]) < 3e-2, (name, rel(got[name], want[name]))


def test_qwen3_sized_layer_at_a_quarter_of_the_tokens():
    # config 1 dims (H=2048, I=768, E=128, top-8, r=16, alpha=32) on 2048 tokens
    got, want = run_layer(2048, 2048, 768, 128, 8, 16, 32, seed=3)
    for name in want:
        assert rel(got[name], want[name]) < 1e-2, (name, rel(got[name], want[name]))


@pytest.mark.parametrize("is_transposed", [False, True])
def test_layer_whose_experts_take_tall_items(is_transposed):
    # 560 tokens, top-4 of 8 experts: rows per expert 262-290 with this seed, so six groups run as one
    # tall item (257-288 rows) beside two of 289 and 290; the combine's per-row weights ride on them
    got, want = run_layer(560, 256, 192, 8, 4, 16, 32, is_transposed, seed=11)
    for name in want:
        assert rel(got[name], want[name]) < 1e-2, (name, rel(got[name], want[name]))


@pytest.mark.parametrize("is_transposed", [False, True])
def test_layer_with_the_adapter_gradient_fused_into_the_input_gradient_products(is_transposed, monkeypatch):
    """MEEPSQUARED_FUSED_DB=1: B's gradient of both products formed by the input-gradient launches
    (mlora_grouped_gemm_db; the down product's with the combine weights on its rows): every output and
    gradient against the oracle, and the same as the standalone reductions give within bf16 rounding."""
    monkeypatch.setenv("MEEPSQUARED_FUSED_DB", "1")
    got, want = run_layer(560, 256, 192, 8, 4, 16, 32, is_transposed, seed=11)
    for name in want:
        assert rel(got[name], want[name]) < 1e-2, (name, rel(got[name], want[name]))
    monkeypatch.setenv("MEEPSQUARED_FUSED_DB", "0")
    plain, _ = run_layer(560, 256, 192, 8, 4, 16, 32, is_transposed, seed=11)
    for name in want:
        assert rel(got[name], plain[name]) < 5e-3, (name, rel(got[name], plain[name]))


def test_mixtral_shaped_layer_with_zipf_loaded_experts():
    # config 2's routing (E=8, top-2, r=16, Zipf(1.2)-biased logits) at reduced width: the groups are ragged
    got, want = run_layer(1024, 512, 1792, 8, 2, 16, 32, seed=5, zipf=1.2)
    for name in want:
        assert rel(got[name], want[name]) < 1e-2, (name, rel(got[name], want[name]))


@pytest.mark.parametrize("is_transposed", [False, True])
def test_layer_with_nf4_stacks_on_a_packed_varlen_batch(is_transposed):
    # config 4: config-1 dims, NF4 stacks, the tokens of 6 packed sequences with lengths U[64, 512]
    T = int(np.random.default_rng(4).integers(64, 513, size=6).sum())
    got, want = run_layer(T, 2048, 768, 128, 8, 16, 32, is_transposed, seed=4, nf4=True)
    for name in want:
        assert rel(got[name], want[name]) < 3e-2, (name, rel(got[name], want[name]))


@pytest.mark.parametrize("is_transposed", [False, True])
@pytest.mark.parametrize("weights_dtype", [torch.bfloat16, torch.float32])
def test_the_combined_down_product_matches_the_product_then_the_combine(is_transposed, weights_dtype):
    """lora_linear_combined (the down product and the combine in one Function, the backward reading the
    output gradient through perm) against lora_linear followed by the combine: the same output bits, the
    weights', input and adapter gradients within bf16 rounding of each other (the weights enter after
    different roundings; the weights' gradient sums its dot products in another order)."""
    from meepsquared_amd import _grouped, _moe, sort_by_expert, topk_softmax

    torch.manual_seed(11)
    T, I, H, E, k, r = 300, 128, 192, 8, 2, 16
    dev = "cuda"
    logits = torch.randn(T, E, device=dev)
    w, idx = topk_softmax(logits.to(torch.bfloat16), k, weights_dtype=weights_dtype)
    idx = torch.where(torch.rand(idx.shape, device=dev) < 0.05, torch.full_like(idx, E), idx)  # a few sentinels
    perm, inv, offsets = sort_by_expert(idx, E)
    act = torch.randn(T * k, I, device=dev).bfloat16()
    down = (torch.randn((E, I, H) if is_transposed else (E, H, I), device=dev) * 0.05).bfloat16()
    if is_transposed:
        lhs, rhs = torch.randn(E, I, r, device=dev) * 0.1, torch.randn(E, r, H, device=dev) * 0.1
    else:
        lhs, rhs = torch.randn(E, H, r, device=dev) * 0.1, torch.randn(E, r, I, device=dev) * 0.1
    dres = torch.randn(T, H, device=dev).bfloat16()

    def run(combined):
        a = act.clone().requires_grad_()
        ww = w.detach().clone().requires_grad_()
        l_, r_ = lhs.bfloat16().requires_grad_(), rhs.bfloat16().requires_grad_()
        if combined:
            out = _grouped.lora_linear_combined(a, ww, perm, inv, k, down, None, offsets, is_transposed, l_, r_, 2.0)
        else:
            y = _grouped.lora_linear(a, down, None, offsets, is_transposed, l_, r_, 2.0)
            out = _moe._Combine.apply(y, ww, inv, offsets, k)
        out.backward(dres)
        return out.detach(), ww.grad, a.grad, l_.grad, r_.grad

    got, want = run(True), run(False)
    assert torch.equal(got[0], want[0])
    assert rel(got[1], want[1]) < 1e-2  # the weights' gradient: the same dot products, summed in another order
    valid = int(offsets[-1])  # rows past it are sentinels' and take no gradient
    assert rel(got[2][:valid], want[2][:valid]) < 1e-2
    for i in (3, 4):
        assert rel(got[i], want[i]) < 1e-2


@pytest.mark.parametrize("is_transposed", [False, True])
@pytest.mark.parametrize("weights_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("I", [128, 8704])  # 8704: rows wider than 8 fit in the SwiGLU backward's LDS
def test_swiglu_and_the_combined_down_product_match_the_composed_steps(is_transposed, weights_dtype, I):
    """swiglu_lora_linear_combined (SwiGLU, the down product and the combine in one Function, the weights'
    gradient formed in the SwiGLU backward as <g, act>) against SwiGLU, lora_linear and the combine
    composed: the same output bits; the gradients within bf16 rounding of each other (<g, act> and
    <dout, y> are the same sum taken over other roundings; the weights enter the SwiGLU backward in
    fp32 instead of through bf16(w · dout))."""
    from meepsquared_amd import _grouped, _moe, sort_by_expert, topk_softmax

    torch.manual_seed(12)
    T, H, E, k, r = 300, 192, 8, 2, 16
    dev = "cuda"
    logits = torch.randn(T, E, device=dev)
    w, idx = topk_softmax(logits.to(torch.bfloat16), k, weights_dtype=weights_dtype)
    idx = torch.where(torch.rand(idx.shape, device=dev) < 0.05, torch.full_like(idx, E), idx)  # a few sentinels
    perm, inv, offsets = sort_by_expert(idx, E)
    gu = torch.randn(T * k, 2 * I, device=dev).bfloat16()
    down = (torch.randn((E, I, H) if is_transposed else (E, H, I), device=dev) * 0.05).bfloat16()
    if is_transposed:
        lhs, rhs = torch.randn(E, I, r, device=dev) * 0.1, torch.randn(E, r, H, device=dev) * 0.1
    else:
        lhs, rhs = torch.randn(E, H, r, device=dev) * 0.1, torch.randn(E, r, I, device=dev) * 0.1
    dres = torch.randn(T, H, device=dev).bfloat16()

    def run(fused):
        g = gu.clone().requires_grad_()
        ww = w.detach().clone().requires_grad_()
        l_, r_ = lhs.bfloat16().requires_grad_(), rhs.bfloat16().requires_grad_()
        if fused:
            out = _grouped.swiglu_lora_linear_combined(g, ww, perm, inv, k, down, None, offsets, is_transposed, l_,
                                                       r_, 2.0)
        else:
            y = _grouped.lora_linear(_moe._SwiGLU.apply(g), down, None, offsets, is_transposed, l_, r_, 2.0)
            out = _moe._Combine.apply(y, ww, inv, offsets, k)
        out.backward(dres)
        return out.detach(), ww.grad, g.grad, l_.grad, r_.grad

    got, want = run(True), run(False)
    assert torch.equal(got[0], want[0])
    assert rel(got[1], want[1]) < 1e-2
    sentinel = (idx.reshape(-1) == E).reshape(got[1].shape)
    assert torch.all(got[1][sentinel] == 0)
    valid = int(offsets[-1])  # rows past it are sentinels' and take no gradient
    assert rel(got[2][:valid], want[2][:valid]) < 1e-2
    assert torch.all(got[2][valid:] == 0)
    for i in (3, 4):
        assert rel(got[i], want[i]) < 1e-2


def test_config3_fp8_stacks_with_fp8_products_at_config1_dims(monkeypatch):
    """config-1 dims (H=2048, I=768, E=128, top-8, r=16, alpha=32) on 2048 tokens, fp8
    e4m3 stacks with one fp32 scale per output row and the products on the fp8 MFMA (activations and output
    gradients quantised to two e4m3 terms in the kernels' prep pass), against the fp32 oracle on the
    dequantised stacks: every output and gradient within BASELINE's 3e-2.  (One term, the reference's
    single pass, measured 4.7 % on out here.)"""
    monkeypatch.setenv("MEEPSQUARED_FP8_PRODUCTS", "1")
    got, want = run_layer(2048, 2048, 768, 128, 8, 16, 32, seed=3, fp8="row")
    errors = {name: rel(got[name], want[name]) for name in want}
    print("config 3 (fp8 products) relative errors:", {n: f"{v:.4f}" for n, v in errors.items()}, flush=True)
    for name, err in errors.items():
        assert err < 3e-2, (name, err)


def test_config2_mixtral_layer_at_full_width_with_zipf_loaded_experts():
    """BASELINE config 2 at its own shapes: T=16384, H=4096, I=14336, E=8, top-2, r=16, Zipf(1.2)-biased
    logits (the busiest expert takes thousands of rows: K=14336 in the down product, N=28672 in gate_up),
    forward and backward against the fp32 oracle, 1e-2."""
    got, want = run_layer(16384, 4096, 14336, 8, 2, 16, 32, seed=5, zipf=1.2)
    errors = {name: rel(got[name], want[name]) for name in want}
    print("config 2 relative errors:", {n: f"{v:.4f}" for n, v in errors.items()}, flush=True)
    for name, err in errors.items():
        assert err < 1e-2, (name, err)


def test_config4_nf4_layer_on_a_packed_batch_of_32_sequences():
    """BASELINE config 4's load: config-1 dims on the tokens of 32 packed sequences with lengths U[64, 2048]
    (~34k tokens, ~2.1k rows per expert: many full tiles per expert), NF4 stacks, against the fp32 oracle on
    the decoded stacks, 3e-2."""
    T = int(np.random.default_rng(40).integers(64, 2049, size=32).sum())
    got, want = run_layer(T, 2048, 768, 128, 8, 16, 32, seed=40, nf4=True)
    errors = {name: rel(got[name], want[name]) for name in want}
    print(f"config 4 (T={T}) relative errors:", {n: f"{v:.4f}" for n, v in errors.items()}, flush=True)
    for name, err in errors.items():
        assert err < 3e-2, (name, err)
