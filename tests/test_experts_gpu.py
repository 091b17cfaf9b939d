"""The routed forward as a Transformers experts implementation, on the GPU: a Qwen3-MoE sparse block
switched to "meepsquared_amd" against the same block run by Transformers' own eager experts loop in
float32 (TF:models/qwen3_moe/modeling_qwen3_moe.py:209-281), forward and input gradient; and LoRA
factors attached to the experts module against the CPU oracle.  Tolerance: relative Frobenius error
1e-2 (bf16)."""

import copy

import pytest
import torch

from helpers import rel
from oracle import moe as ref_moe

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")


def tiny_block(E=8, k=2, H=256, I=128, seed=0):
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock

    cfg = Qwen3MoeConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E, num_experts_per_tok=k,
                         norm_topk_prob=True, hidden_act="silu")
    torch.manual_seed(seed)
    block = Qwen3MoeSparseMoeBlock(cfg)
    with torch.no_grad():
        block.gate.weight.normal_(0, 0.05)
        block.experts.gate_up_proj.normal_(0, 0.02)
        block.experts.down_proj.normal_(0, 0.02)
    block.experts.gate_up_proj.requires_grad_(False)  # frozen stacks, as in LoRA training
    block.experts.down_proj.requires_grad_(False)
    return block, cfg


def test_a_qwen3_moe_block_switched_to_the_routed_forward_matches_transformers_eager():
    from meepsquared_amd import experts

    experts.register()
    block, cfg = tiny_block()
    ref_experts = copy.deepcopy(block.experts).float().cuda()  # Transformers' per-expert loop, in float32
    cfg_ref = copy.deepcopy(cfg)
    cfg_ref._experts_implementation = "eager"
    ref_experts.config = cfg_ref
    block = block.to("cuda", torch.bfloat16)
    cfg_ours = copy.deepcopy(cfg)
    cfg_ours._experts_implementation = experts.IMPLEMENTATION
    block.experts.config = cfg_ours
    assert experts.routed(block.experts) and not experts.routed(ref_experts)

    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 96, 256, generator=g).to("cuda", torch.bfloat16)
    dy = torch.randn(2, 96, 256, generator=g).to("cuda", torch.bfloat16)
    # the whole sparse block (router + experts) through the routed forward
    xb = x.clone().requires_grad_()
    out = block(xb)
    out.backward(dy)
    # the same routing into Transformers' eager experts in float32 (a near-tie of the router would
    # otherwise pick other experts in float32)
    _, w, idx = block.gate(x.view(-1, 256))
    w = w.detach()
    x32 = x.view(-1, 256).float().requires_grad_()
    out32 = ref_experts(x32, idx, w.float())
    out32.backward(dy.view(-1, 256).float())
    # the input gradient through the experts alone (the block's includes the router's part)
    xe = x.view(-1, 256).clone().requires_grad_()
    oute = block.experts(xe, idx, w)
    oute.backward(dy.view(-1, 256))
    assert torch.equal(out.view(-1, 256), oute.detach())  # the block ran exactly this
    assert rel(oute, out32) < 1e-2, rel(oute, out32)
    assert rel(xe.grad, x32.grad) < 1e-2, rel(xe.grad, x32.grad)
    assert xb.grad is not None and torch.isfinite(xb.grad.float()).all()


@pytest.mark.parametrize("k", [2, 8])
def test_adapters_attached_to_the_experts_module_match_the_oracle(k):
    from meepsquared_amd import experts, topk_softmax

    experts.register()
    E, H, I, r, T = 16, 256, 128, 16, 300
    block, cfg = tiny_block(E=E, k=k, H=H, I=I, seed=2)
    module = block.experts.to("cuda", torch.bfloat16)
    cfg._experts_implementation = experts.IMPLEMENTATION
    module.config = cfg
    g = torch.Generator().manual_seed(3)
    f = {"gate_up_proj": ((torch.randn(E, 2 * I, r, generator=g) * 0.05).to("cuda", torch.bfloat16).requires_grad_(),
                          (torch.randn(E, r, H, generator=g) * 0.05).to("cuda", torch.bfloat16).requires_grad_(), 2.0),
         "down_proj": ((torch.randn(E, H, r, generator=g) * 0.05).to("cuda", torch.bfloat16).requires_grad_(),
                       (torch.randn(E, r, I, generator=g) * 0.05).to("cuda", torch.bfloat16).requires_grad_(), 2.0)}
    experts.set_adapters(module, f)
    h = torch.randn(T, H, generator=g).to("cuda", torch.bfloat16).requires_grad_()
    w, idx = topk_softmax(torch.randn(T, E, generator=g).to("cuda", torch.bfloat16), k)
    out = module(h, idx, w)  # through Qwen3MoeExperts.forward and the ExpertsInterface
    dy = torch.randn(out.shape, generator=g).to("cuda", torch.bfloat16)
    out.backward(dy)

    h32 = h.detach().float().requires_grad_()
    f32 = {n: (a.detach().float().requires_grad_(), b.detach().float().requires_grad_(), s) for n, (a, b, s) in f.items()}
    o32 = ref_moe.routed_forward(h32, idx, w.float(), module.gate_up_proj.float(), module.down_proj.float(), f32, E)
    o32.backward(dy.float())
    assert rel(out, o32) < 1e-2, rel(out, o32)
    assert rel(h.grad, h32.grad) < 1e-2, rel(h.grad, h32.grad)
    for n in f:
        for i in range(2):
            assert rel(f[n][i].grad, f32[n][i].grad) < 1e-2, (n, i, rel(f[n][i].grad, f32[n][i].grad))


def _module_with_adapters(E=8, H=256, I=128, r=16, seed=4):
    from meepsquared_amd import experts

    block, cfg = tiny_block(E=E, k=2, H=H, I=I, seed=seed)
    module = block.experts.to("cuda", torch.bfloat16)
    cfg._experts_implementation = experts.IMPLEMENTATION
    module.config = cfg
    g = torch.Generator().manual_seed(seed + 1)
    f = {"gate_up_proj": ((torch.randn(E, 2 * I, r, generator=g) * 0.05).to("cuda", torch.bfloat16),
                          (torch.randn(E, r, H, generator=g) * 0.05).to("cuda", torch.bfloat16), 2.0),
         "down_proj": ((torch.randn(E, H, r, generator=g) * 0.05).to("cuda", torch.bfloat16),
                       (torch.randn(E, r, I, generator=g) * 0.05).to("cuda", torch.bfloat16), 2.0)}
    experts.set_adapters(module, f)
    return module, g


@pytest.mark.parametrize("stacks", ["bf16", "fp8_row", "nf4"])
def test_merged_stacks_compute_what_the_adapters_add(stacks):
    """The routed forward with adapters equals the forward on the merged stacks W + s lhs rhs without them
    (the reference's merged save, src/meepsquared/_save.py:79-95), for bf16, fp8 (per-row scales) and NF4 stacks."""
    from meepsquared_amd import _fp8, _nf4, experts, topk_softmax

    experts.register()
    module, g = _module_with_adapters()
    module.gate_up_proj.requires_grad_(False)
    module.down_proj.requires_grad_(False)
    if stacks == "fp8_row":
        assert _fp8.convert_stacks(module, per_row=True) == 2
    elif stacks == "nf4":
        assert _nf4.convert_stacks(module) == 2 and _nf4.convert_stacks(module) == 2  # idempotent
    T, E = 200, module.num_experts
    h = torch.randn(T, 256, generator=g).to("cuda", torch.bfloat16)
    w, idx = topk_softmax(torch.randn(T, E, generator=g).to("cuda", torch.bfloat16), 2)
    with torch.no_grad():
        with_adapters = module(h, idx, w)
        merged = copy.copy(module)
        merged.gate_up_proj = torch.nn.Parameter(experts.merged_stack(module, "gate_up_proj"), requires_grad=False)
        merged.down_proj = torch.nn.Parameter(experts.merged_stack(module, "down_proj"), requires_grad=False)
        experts.set_adapters(merged, {})
        without = merged(h, idx, w)
    assert rel(without, with_adapters) < 1e-2, rel(without, with_adapters)


def test_a_qwen3_moe_causal_lm_switched_to_the_routed_forward_matches_the_eager_one():
    """A whole (tiny, one-layer) Qwen3-MoE causal LM in bf16: the same model with Transformers' eager experts
    and with experts.use(model) gives the same logits and embedding gradient to bf16 tolerance (one MoE layer,
    so both runs route the same tokens to the same experts); the stacks are frozen as in LoRA training."""
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM

    from meepsquared_amd import experts

    cfg = Qwen3MoeConfig(vocab_size=128, hidden_size=256, intermediate_size=512, moe_intermediate_size=128,
                         num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                         num_experts=8, num_experts_per_tok=2, norm_topk_prob=True)
    torch.manual_seed(0)
    model = Qwen3MoeForCausalLM(cfg)
    with torch.no_grad():
        for name, prm in model.named_parameters():
            if prm.dim() > 1:
                prm.normal_(0, 0.05)
    for name, prm in model.named_parameters():
        if name.endswith("experts.gate_up_proj") or name.endswith("experts.down_proj"):
            prm.requires_grad_(False)
    model = model.to("cuda", torch.bfloat16)
    ours = copy.deepcopy(model)
    model.set_experts_implementation("eager")
    assert experts.use(ours) == 1
    ids = torch.randint(0, 128, (2, 80), generator=torch.Generator().manual_seed(1)).cuda()

    def run(m):
        m.zero_grad(set_to_none=True)
        out = m(input_ids=ids, labels=ids)
        out.loss.backward()
        return out.logits.detach().float(), m.model.embed_tokens.weight.grad.float(), out.loss.item()

    logits_e, grad_e, loss_e = run(model)
    logits_o, grad_o, loss_o = run(ours)
    assert rel(logits_o, logits_e) < 1e-2, rel(logits_o, logits_e)
    assert rel(grad_o, grad_e) < 2e-2, rel(grad_o, grad_e)
    assert abs(loss_o - loss_e) < 1e-2 * abs(loss_e), (loss_o, loss_e)


@pytest.mark.parametrize("with_adapters", [False, True])
def test_gpt_oss_experts_with_their_own_gate_match_transformers_eager(with_adapters):
    """GptOssExperts (transposed stacks with biases, interleaved gate/up columns, the clamped
    (up + 1) · gate · sigmoid(1.702 · gate) gate, TF:models/gpt_oss/modeling_gpt_oss.py:68-113) switched
    to the routed forward: the products run on the kernels and the gate is the module's own
    `_apply_gate`, as src/meepsquared/_moe.py:118 calls it.  Against Transformers' eager loop in
    float32 (with adapters: the eager loop on the merged stacks W + s·lhs@rhs), forward and input
    gradient, relative error 1e-2."""
    from transformers import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssExperts

    from meepsquared_amd import experts, topk_softmax

    experts.register()
    E, H, I, k, T, r, s = 8, 128, 64, 2, 200, 16, 2.0
    cfg = GptOssConfig(hidden_size=H, intermediate_size=I, num_local_experts=E, num_experts_per_tok=k)
    torch.manual_seed(3)
    module = GptOssExperts(cfg)
    with torch.no_grad():
        module.gate_up_proj.normal_(0, 0.1)  # gates reach the clamp at 7 now and then
        module.gate_up_proj_bias.normal_(0, 0.5)
        module.down_proj.normal_(0, 0.05)
        module.down_proj_bias.normal_(0, 0.1)
    for p in module.parameters():
        p.requires_grad_(False)
    ref = copy.deepcopy(module).float().cuda()
    cfg_ref = copy.deepcopy(cfg)
    cfg_ref._experts_implementation = "eager"
    ref.config = cfg_ref
    module = module.to("cuda", torch.bfloat16)
    cfg_ours = copy.deepcopy(cfg)
    cfg_ours._experts_implementation = experts.IMPLEMENTATION
    module.config = cfg_ours
    g = torch.Generator().manual_seed(4)
    x = torch.randn(T, H, generator=g).to("cuda", torch.bfloat16)
    dy = torch.randn(T, H, generator=g).to("cuda", torch.bfloat16)
    w, idx = topk_softmax(torch.randn(T, E, generator=g).to("cuda", torch.bfloat16), k)
    if with_adapters:  # transposed stacks: lhs (E, in, r), rhs (E, r, out)
        fa = {"gate_up_proj": ((torch.randn(E, H, r, generator=g) * 0.05).to("cuda", torch.bfloat16),
                               (torch.randn(E, r, 2 * I, generator=g) * 0.05).to("cuda", torch.bfloat16), s),
              "down_proj": ((torch.randn(E, I, r, generator=g) * 0.05).to("cuda", torch.bfloat16),
                            (torch.randn(E, r, H, generator=g) * 0.05).to("cuda", torch.bfloat16), s)}
        experts.set_adapters(module, fa)
        with torch.no_grad():
            for name, (lhs, rhs, sc) in fa.items():
                getattr(ref, name).add_(sc * (lhs.float() @ rhs.float()))
    xb = x.clone().requires_grad_()
    out = module(xb, idx, w)
    out.backward(dy)
    x32 = x.float().requires_grad_()
    out32 = ref(x32, idx, w.float())
    out32.backward(dy.float())
    assert rel(out, out32) < 1e-2, rel(out, out32)
    assert rel(xb.grad, x32.grad) < 1e-2, rel(xb.grad, x32.grad)
