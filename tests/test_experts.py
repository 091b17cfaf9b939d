"""The Transformers ExpertsInterface integration (meepsquared_amd._experts), host side: which stacks a
model exposes (the reference's expert_targets, src/meepsquared/_moe.py:163-182), the switch of a model's
experts modules to the routed forward, the adapters' layout checks, and that the dispatch reaches the
kernels with no CPU path.  Tiny models built from configs (random weights, nothing downloaded)."""

import pytest
import torch

transformers = pytest.importorskip("transformers")


def tiny_qwen3_moe(layers=2):
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM

    cfg = Qwen3MoeConfig(vocab_size=64, hidden_size=64, intermediate_size=128, moe_intermediate_size=32,
                         num_hidden_layers=layers, num_attention_heads=2, num_key_value_heads=1, head_dim=32,
                         num_experts=4, num_experts_per_tok=2)
    return Qwen3MoeForCausalLM(cfg)


def test_expert_targets_name_every_stack_inside_a_decoder_layer():
    from meepsquared_amd import experts

    assert experts.expert_targets(tiny_qwen3_moe(3)) == (["mlp.experts.down_proj", "mlp.experts.gate_up_proj"], 6)


def test_a_model_without_experts_has_no_targets():
    from transformers import Qwen3Config, Qwen3ForCausalLM

    from meepsquared_amd import experts

    cfg = Qwen3Config(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=2, num_key_value_heads=1, head_dim=32)
    assert experts.expert_targets(Qwen3ForCausalLM(cfg)) == ([], 0)


def test_use_switches_every_experts_module_to_the_routed_forward():
    from transformers.integrations.moe import ALL_EXPERTS_FUNCTIONS

    from meepsquared_amd import experts

    model = tiny_qwen3_moe(2)
    assert experts.use(model) == 2
    assert experts.IMPLEMENTATION in ALL_EXPERTS_FUNCTIONS
    assert model.config._experts_implementation == experts.IMPLEMENTATION
    assert all(experts.routed(layer.mlp.experts) for layer in model.model.layers)


def test_the_dispatch_reaches_the_kernels_and_refuses_cpu_tensors():
    from meepsquared_amd import experts

    model = tiny_qwen3_moe(1)
    experts.use(model)
    module = model.model.layers[0].mlp.experts
    with pytest.raises(TypeError, match="GPU"):
        module(torch.randn(3, 64), torch.zeros(3, 2, dtype=torch.long), torch.ones(3, 2))


@pytest.mark.parametrize("is_transposed", [False, True])
def test_set_adapters_checks_the_factors_against_the_stack_layout(is_transposed):
    from meepsquared_amd import Experts, experts

    E, H, I, r = 4, 64, 48, 8
    gu = torch.zeros((E, H, 2 * I) if is_transposed else (E, 2 * I, H))
    dn = torch.zeros((E, I, H) if is_transposed else (E, H, I))
    module = Experts(gu, dn, is_transposed)
    if is_transposed:  # (E, in, r) and (E, r, out)
        good = {"gate_up_proj": (torch.zeros(E, H, r), torch.zeros(E, r, 2 * I), 2.0),
                "down_proj": (torch.zeros(E, I, r), torch.zeros(E, r, H), 2.0)}
    else:  # (E, out, r) and (E, r, in)
        good = {"gate_up_proj": (torch.zeros(E, 2 * I, r), torch.zeros(E, r, H), 2.0),
                "down_proj": (torch.zeros(E, H, r), torch.zeros(E, r, I), 2.0)}
    experts.set_adapters(module, good)
    swapped = {"gate_up_proj": (good["gate_up_proj"][1].transpose(1, 2), good["gate_up_proj"][0].transpose(1, 2), 2.0)}
    with pytest.raises(ValueError, match="expected"):
        experts.set_adapters(module, swapped)
    with pytest.raises(ValueError, match="not a stack"):
        experts.set_adapters(module, {"up_proj": good["gate_up_proj"]})
    with pytest.raises(TypeError):
        experts.set_adapters(torch.nn.Linear(2, 2), good)


def test_the_fused_swiglu_is_taken_only_for_the_default_silu_gate():
    """gate_of: None (the SwiGLU kernel) for Transformers' default gate with SiLU and for this package's
    Experts container; the model's own gate function for gpt-oss (interleaved, clamped, sigmoid(1.702 g))
    and for a default gate whose act_fn is not SiLU."""
    from transformers import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssExperts

    from meepsquared_amd import Experts
    from meepsquared_amd._moe import gate_of

    qwen = tiny_qwen3_moe(1).model.layers[0].mlp.experts
    assert gate_of(qwen) is None
    assert gate_of(Experts(torch.zeros(2, 8, 4), torch.zeros(2, 4, 4))) is None
    oss = GptOssExperts(GptOssConfig(hidden_size=16, intermediate_size=8, num_local_experts=2))
    gate = gate_of(oss)
    assert gate is not None
    gu = torch.randn(5, 16)
    assert torch.equal(gate(gu), oss._apply_gate(gu))
    qwen.act_fn = torch.nn.GELU()
    gate = gate_of(qwen)
    g, u = gu.chunk(2, dim=-1)
    assert gate is not None and torch.equal(gate(gu), torch.nn.functional.gelu(g) * u)
