"""The routed MoE-LoRA layer as a Transformers experts implementation.

Transformers dispatches the forward of its experts modules (`@use_experts_implementation`, e.g.
`Qwen3MoeExperts`) through `ExpertsInterface` by `config._experts_implementation`
(TF:integrations/moe.py:481-506, 523-572).  `register()` adds this package's routed forward there
under the name "meepsquared_amd"; `use(model)` registers it and switches the model to it.  Each
experts module then runs `routed_forward` (router output in, combined tokens out) on its base stacks,
plus the LoRA factors attached to it with `set_adapters` — the change the reference adds per
projection, `scaling * lhs @ rhs` in the layout of the stack.

In the reference the same forward replaces PEFT's ParamWrapper forward (src/meepsquared/_moe.py:
129-144, 208-228), taking (lhs, rhs, scaling) from PEFT's lora_A/lora_B (`_delta_factors`,
src/meepsquared/_moe.py:147-160).  PEFT is not part of this build; a PEFT chain hands the factors its
`_delta_factors` builds to `set_adapters`, in the layout described there.

As in the reference, the stacks are frozen: the forward returns no gradient for them.
"""

import re

import torch

from meepsquared_amd._moe import routed_forward

IMPLEMENTATION = "meepsquared_amd"
# The attributes of a Transformers experts module (TF:integrations/moe.py:559-563)
EXPERTS_ATTRIBUTES = ("num_experts", "has_gate", "has_bias", "is_transposed")
# The stacks an experts module holds, by name (src/meepsquared/_moe.py:34-35)
STACKS = ("gate_up_proj", "up_proj", "down_proj")
_FACTORS = "_meepsquared_amd_factors"


def experts_forward(self, hidden_states: torch.Tensor, top_k_index: torch.Tensor,
                    top_k_weights: torch.Tensor) -> torch.Tensor:
    """The ExpertsInterface forward: the routed layer over this module's stacks and attached adapters."""
    return routed_forward(self, hidden_states, top_k_index, top_k_weights, getattr(self, _FACTORS, {}))


def register(name: str = IMPLEMENTATION) -> str:
    """Adds the routed forward to Transformers' ExpertsInterface under `name` (idempotent); returns the name."""
    from transformers.integrations.moe import ExpertsInterface

    ExpertsInterface.register(name, experts_forward)
    return name


def is_experts(module) -> bool:
    """Whether the module is a Transformers experts module (the attributes its decorator sets)."""
    return all(hasattr(module, attribute) for attribute in EXPERTS_ATTRIBUTES)


def use(model, name: str = IMPLEMENTATION) -> int:
    """Registers the routed forward and makes every experts module of the model run it; returns how many.

    The counterpart of the reference's `apply(model)` (src/meepsquared/_moe.py:208-228), which patches
    PEFT's wrappers instead.
    """
    register(name)
    model.set_experts_implementation(name)
    return sum(1 for module in model.modules() if is_experts(module))


def routed(module) -> bool:
    """Whether the experts module's forward dispatches to this implementation (src/meepsquared/_moe.py:203-205)."""
    config = getattr(module, "config", None)
    return is_experts(module) and getattr(config, "_experts_implementation", None) == IMPLEMENTATION


def _stack_dims(module, name):
    """(experts, in, out) of a stack: a tensor or an Nf4Stack (which keeps its logical shape)."""
    w = getattr(module, name)
    e = module.num_experts
    shape = tuple(getattr(w, "shape", ()))
    if len(shape) != 3 or shape[0] != e:
        raise ValueError(f"{name}: not a stack of {e} experts")
    n_in, n_out = (shape[1], shape[2]) if module.is_transposed else (shape[2], shape[1])
    return e, n_in, n_out


def set_adapters(module, factors: dict) -> None:
    """Attaches LoRA factors to an experts module: {stack name: (lhs, rhs, scaling)}.

    lhs/rhs in the stack's layout, as the reference's `_delta_factors` returns them: (E, out, r) and
    (E, r, in) for an (E, out, in) stack, (E, in, r) and (E, r, out) when `is_transposed`.  The tensors
    are kept by reference, so trained parameters are read at every forward; gradients reach them
    through the routed forward.  An empty dict removes the adapters.
    """
    if not is_experts(module):
        raise TypeError(f"{type(module).__name__} is not a Transformers experts module")
    checked = {}
    for name, value in factors.items():
        if name not in STACKS or not hasattr(module, name):
            raise ValueError(f"{name}: not a stack of {type(module).__name__}")
        lhs, rhs, scaling = value
        e, n_in, n_out = _stack_dims(module, name)
        rank = lhs.shape[-1]
        want_lhs = (e, n_in, rank) if module.is_transposed else (e, n_out, rank)
        want_rhs = (e, rank, n_out) if module.is_transposed else (e, rank, n_in)
        if tuple(lhs.shape) != want_lhs or tuple(rhs.shape) != want_rhs:
            raise ValueError(f"{name}: factors {tuple(lhs.shape)} / {tuple(rhs.shape)}, expected {want_lhs} / {want_rhs}")
        checked[name] = (lhs, rhs, float(scaling))
    setattr(module, _FACTORS, checked)


def expert_targets(model) -> tuple:
    """The target_parameters naming every expert stack of the model, and how many stacks they reach.

    As the reference (src/meepsquared/_moe.py:163-182): a name is the stack's path inside its
    decoder layer ("mlp.experts.gate_up_proj"); a model without experts modules gives ([], 0).
    """
    names, stacks = set(), 0
    for name, module in model.named_modules():
        if not is_experts(module):
            continue
        inside_layer = re.search(r"(?:^|\.)layers\.\d+\.(.+)$", name)
        if inside_layer is None:
            raise NotImplementedError(f"{name}: an experts module outside a numbered decoder layer")
        for stack in STACKS:
            if isinstance(getattr(module, stack, None), torch.nn.Parameter):
                names.add(f"{inside_layer.group(1)}.{stack}")
                stacks += 1
    return sorted(names), stacks


def merged_stack(module, name: str, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """A stack with its attached adapter merged, W + scaling * lhs @ rhs for every expert, in the stack's layout.

    As the reference's merged save (src/meepsquared/_save.py:79-95): the factors the training computes
    with, in float32; an fp8 stack dequantised with its scale first (and an NF4 stack decoded).  A stack
    without an adapter comes back dequantised.  For saving a merged model; not on the training path.
    """
    from meepsquared_amd import _fp8, _grouped, _nf4

    stack = getattr(module, name)
    if isinstance(stack, _grouped.Nf4Stack):
        weight = _nf4.dequantize_stack(stack, torch.float32)
    elif stack.dtype == torch.float8_e4m3fn:
        weight = _fp8.dequantize_stack(stack.detach(), getattr(module, name + _fp8.STACK_SCALE), torch.float32,
                                       bool(module.is_transposed))
    else:
        weight = stack.detach().float()
    factors = getattr(module, _FACTORS, {})
    if name in factors:
        lhs, rhs, scaling = factors[name]
        weight = weight + scaling * torch.bmm(lhs.detach().float().contiguous(), rhs.detach().float().contiguous())
    return weight.to(dtype)

