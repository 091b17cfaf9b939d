"""Frozen dense layers held as fp8 (meepsquared_amd._fp8: quantize, scaled_mm, Fp8Linear, convertible, apply;
the reference's src/meepsquared/_fp8.py:95-109, 198-293) against the oracle's float32 restatement of the
reference's own CPU path (oracle/formats.py: fp8_tensor_quantize, fp8_scaled_mm).  The products run on the
fp8 MFMA with the activations as two e4m3 terms; tolerance 3e-2 (fp8), measured errors are ~0.4 %."""

import pytest
import torch

from helpers import rel
from oracle import formats

pytestmark = pytest.mark.gpu
FP8_TOL = 3e-2


def test_quantize_is_bit_exact_against_the_oracle():
    from meepsquared_amd import _fp8

    torch.manual_seed(0)
    w = (torch.randn(768, 2048) * 0.02).bfloat16()
    q, s = _fp8.quantize(w.cuda())
    oq, os_ = formats.fp8_tensor_quantize(w.float())
    assert s.shape == () and torch.equal(s.cpu(), os_)
    assert torch.equal(q.cpu().view(torch.uint8), oq.view(torch.uint8))


@pytest.mark.parametrize("shape,out_features,bias", [((4, 33, 2048), 768, True), ((1, 256), 512, False),
                                                     ((700, 1024), 2048, True)])
def test_fp8_linear_forward_and_input_gradient_match_the_oracle(shape, out_features, bias):
    from meepsquared_amd import _fp8

    torch.manual_seed(1)
    lin = torch.nn.Linear(shape[-1], out_features, bias=bias).cuda().to(torch.bfloat16)
    lin.requires_grad_(False)
    layer = _fp8.Fp8Linear(lin)
    x = torch.randn(*shape, device="cuda").bfloat16().requires_grad_()
    y = layer(x)
    assert y.dtype == torch.bfloat16 and y.shape == (*shape[:-1], out_features)
    g = torch.randn_like(y)
    y.backward(g)
    x32 = x.detach().float().reshape(-1, shape[-1])
    want = formats.fp8_scaled_mm(x32, layer.weight, layer.weight_scale_inv, True,
                                 None if lin.bias is None else lin.bias.float())
    want_dx = formats.fp8_scaled_mm(g.float().reshape(-1, out_features), layer.weight, layer.weight_scale_inv, False)
    assert rel(y.reshape(-1, out_features), want) < FP8_TOL, rel(y.reshape(-1, out_features), want)
    assert rel(x.grad.reshape(-1, shape[-1]), want_dx) < FP8_TOL, rel(x.grad.reshape(-1, shape[-1]), want_dx)
    # a second backward reuses the weight's transposed copy
    x.grad = None
    layer(x).backward(g)
    assert rel(x.grad.reshape(-1, shape[-1]), want_dx) < FP8_TOL


def test_scaled_mm_refuses_what_it_does_not_take():
    from meepsquared_amd import _fp8

    w8, s = _fp8.quantize(torch.randn(64, 32, device="cuda"))
    with pytest.raises(TypeError):
        _fp8.scaled_mm(torch.randn(4, 32), w8, s, True)  # a CPU tensor: no CPU path
    with pytest.raises(TypeError):
        _fp8.scaled_mm(torch.randn(4, 32, device="cuda"), w8.float(), s, True)  # not an fp8 weight


def test_apply_holds_the_frozen_decoder_linears_and_expert_stacks_as_fp8():
    """apply on a tiny Qwen3-MoE: every frozen nn.Linear of the decoder layers whose sizes are multiples of
    16 becomes an Fp8Linear, routers (mlp.gate) and the output layer stay bf16, the experts' stacks become
    fp8 with `<name>_scale_inv` (src/meepsquared/_fp8.py:264-293); each converted layer matches the oracle
    on its own weights; applying again converts the same layers without quantizing them twice."""
    transformers = pytest.importorskip("transformers")
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM

    from meepsquared_amd import _fp8, experts

    cfg = Qwen3MoeConfig(vocab_size=64, hidden_size=128, intermediate_size=256, moe_intermediate_size=64,
                         num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                         num_experts=4, num_experts_per_tok=2)
    torch.manual_seed(2)
    model = Qwen3MoeForCausalLM(cfg).to("cuda", torch.bfloat16)
    model.requires_grad_(False)
    experts.use(model)
    n = _fp8.apply(model)
    layer = model.model.layers[0]
    assert isinstance(layer.self_attn.q_proj, _fp8.Fp8Linear) and isinstance(layer.self_attn.o_proj, _fp8.Fp8Linear)
    assert type(layer.mlp.gate).__name__ != "Fp8Linear" and type(model.lm_head) is torch.nn.Linear
    assert layer.mlp.experts.gate_up_proj.dtype == torch.float8_e4m3fn
    assert hasattr(layer.mlp.experts, "gate_up_proj_scale_inv")
    assert n == 2 * (4 + 2)  # per layer: q, k, v, o projections and the two expert stacks
    assert _fp8.apply(model) == n  # nothing quantized twice: the same layers are counted
    x = torch.randn(3, 17, 128, device="cuda").bfloat16()
    q = layer.self_attn.q_proj
    want = formats.fp8_scaled_mm(x.float().reshape(-1, 128), q.weight, q.weight_scale_inv, True)
    assert rel(q(x).reshape(-1, q.out_features), want) < FP8_TOL
