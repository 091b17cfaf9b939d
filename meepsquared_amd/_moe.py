"""The routed MoE-LoRA layer on MI355X: router top-k, counting sort, gather, the two grouped
products with their adapters, SwiGLU, and the weighted combine — every step a HIP kernel.

`routed_forward(experts, hidden_states, top_k_index, top_k_weights, factors)` keeps the contract of
the reference's `src/meepsquared/_moe.py:70-126` (`_routed_forward`): `experts` is a Transformers
experts module (or the `Experts` container below) holding `num_experts`, `has_gate`, `has_bias`,
`is_transposed`, the stacks `gate_up_proj` and `down_proj` (fp8 stacks with `<name>_scale_inv`),
and `factors` maps a stack's name to PEFT's `(lhs, rhs, scaling)`.  Expert ids at or past
`num_experts` are sentinels (expert parallelism): they sort to the tail, take no compute and add
nothing to the output.

Ordering: the reference sorts the expert ids with an unstable `torch.sort`; here the order within
an expert is the stable one (ascending flat index t·k + j).  The outputs do not depend on it; the
adapters' gradients depend on it only through the order of an fp32 sum.
"""

import torch

from meepsquared_amd import _grouped, _lib
from meepsquared_amd._lib import call, ptr


# ---------------------------------------------------------------------------------------------
# routing
# ---------------------------------------------------------------------------------------------

def topk_softmax(router_logits: torch.Tensor, top_k: int, renormalize: bool = True, weights_dtype=None):
    """(top_k_weights, top_k_index) of the router: softmax in fp32, the k largest, optionally renormalised.

    As TF:models/qwen3_moe/modeling_qwen3_moe.py:262-266 (weights cast to the logits' dtype) and
    TF:models/mixtral/modeling_mixtral.py:104-111 (weights_dtype=torch.float32).  The indices are
    those torch.topk gives on the GPU, ties included: equal probabilities at the k-th place are taken
    in ascending expert order, and the k come in torch's order (for k <= 32 that of its bitonic sort,
    which places equal values in an order of its own); int64.
    """
    _lib.require_gpu(router_logits)
    logits = router_logits.reshape(-1, router_logits.shape[-1])
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    T, E = logits.shape
    weights_dtype = weights_dtype or router_logits.dtype
    if weights_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"router weights in {weights_dtype}: bf16 or fp32")
    idx = torch.empty((T, top_k), device=logits.device, dtype=torch.int64)
    w = torch.empty((T, top_k), device=logits.device, dtype=weights_dtype)
    call("mlora_route_topk", ptr(logits), _lib.dtype_code(logits.dtype), logits.stride(0), T, E, top_k,
         int(renormalize), ptr(idx), ptr(w), _lib.dtype_code(weights_dtype), _lib.stream(logits.device))
    return w, idx


def sort_by_expert(top_k_index: torch.Tensor, num_experts: int, block_m: int = None):
    """(perm, inv, offsets[, tile_expert, tile_row, tiles]) of the (token, slot) pairs in expert order.

    perm (S,) int64 with expert_ids[perm] sorted (stable), inv its inverse, offsets (E,) int32 the
    end of each expert's rows (ids >= num_experts excluded).  With block_m, also the tile map of
    _grouped.tile_map.  Replaces src/meepsquared/_moe.py:77-87.
    """
    _lib.require_gpu(top_k_index)
    ids = top_k_index.reshape(-1)
    if ids.dtype != torch.int64:
        ids = ids.to(torch.int64)
    ids = ids.contiguous()
    S = ids.numel()
    dev = ids.device
    perm = torch.empty(S, device=dev, dtype=torch.int64)
    inv = torch.empty(S, device=dev, dtype=torch.int64)
    offsets = torch.empty(num_experts, device=dev, dtype=torch.int32)
    ws = torch.empty(int(_lib.lib.mlora_route_sort_workspace_bytes(S, num_experts)), device=dev, dtype=torch.uint8)
    tiles_out = ()
    te = tr = tn = None
    n_tiles = 0
    if block_m is not None:
        n_tiles = _grouped.max_tiles(S, num_experts, block_m)
        te = torch.empty(n_tiles, device=dev, dtype=torch.int32)
        tr = torch.empty(n_tiles, device=dev, dtype=torch.int32)
        tn = torch.empty((), device=dev, dtype=torch.int32)
        tiles_out = (te, tr, tn)
    call("mlora_route_sort", ptr(ids), S, num_experts, ptr(perm), ptr(inv), ptr(offsets), block_m or 0,
         ptr(te), ptr(tr), ptr(tn), n_tiles, ptr(ws), ws.numel(), _lib.stream(dev))
    return (perm, inv, offsets) + tiles_out


# ---------------------------------------------------------------------------------------------
# the steps around the products, as autograd Functions over the kernels
# ---------------------------------------------------------------------------------------------

class _Gather(torch.autograd.Function):
    """selected[p] = hidden[perm[p] // k] (zero past offsets[-1]); gradient: per token, the sum of its k rows."""

    @staticmethod
    def forward(ctx, hidden, perm, inv, offsets, k):
        hidden = hidden if hidden.stride(-1) == 1 and hidden.stride(0) % 8 == 0 else hidden.contiguous()
        T, H = hidden.shape
        S = perm.numel()
        out = torch.empty((S, H), device=hidden.device, dtype=hidden.dtype)
        call("mlora_gather_rows", ptr(hidden), hidden.stride(0), H, ptr(perm), S, k, ptr(offsets), offsets.numel(),
             ptr(out), _lib.stream(hidden.device))
        ctx.save_for_backward(inv, offsets)
        ctx.k, ctx.T = k, T
        return out

    @staticmethod
    def backward(ctx, grad):
        inv, offsets = ctx.saved_tensors
        grad = grad.to(torch.bfloat16).contiguous()
        H = grad.shape[1]
        dh = torch.empty((ctx.T, H), device=grad.device, dtype=torch.bfloat16)
        call("mlora_gather_rows_backward", ptr(grad), H, ptr(inv), ctx.T, ctx.k, ptr(offsets), offsets.numel(),
             ptr(dh), _lib.stream(grad.device))
        return dh, None, None, None, None


class _SwiGLU(torch.autograd.Function):
    """silu(gate) · up with gate the first half of each row (TF:integrations/moe.py:509-520)."""

    @staticmethod
    def forward(ctx, gu):
        gu = gu.contiguous()
        S, I2 = gu.shape
        act = torch.empty((S, I2 // 2), device=gu.device, dtype=gu.dtype)
        call("mlora_swiglu", ptr(gu), S, I2 // 2, ptr(act), _lib.stream(gu.device))
        ctx.save_for_backward(gu)
        return act

    @staticmethod
    def backward(ctx, dact):
        (gu,) = ctx.saved_tensors
        dact = dact.to(torch.bfloat16).contiguous()
        dgu = torch.empty_like(gu)
        call("mlora_swiglu_backward", ptr(gu), ptr(dact), gu.shape[0], gu.shape[1] // 2, ptr(dgu), _lib.stream(gu.device))
        return dgu


class _Combine(torch.autograd.Function):
    """out[t] = sum_j y[inv[t*k+j]] · w[t, j] (sentinel rows skipped); gradients for y and w."""

    @staticmethod
    def forward(ctx, y, weights, inv, offsets, k):
        y = y.contiguous()
        S, H = y.shape
        T = inv.numel() // k
        w = weights.reshape(-1).contiguous()
        out = torch.empty((T, H), device=y.device, dtype=y.dtype)
        call("mlora_combine", ptr(y), H, ptr(w), _lib.dtype_code(w.dtype), ptr(inv), T, k, ptr(offsets),
             offsets.numel(), ptr(out), _lib.stream(y.device))
        ctx.save_for_backward(y, w, inv, offsets)
        ctx.k, ctx.wshape = k, weights.shape
        return out

    @staticmethod
    def backward(ctx, dout):
        y, w, inv, offsets = ctx.saved_tensors
        dout = dout.to(torch.bfloat16).contiguous()
        T, H = dout.shape
        dy = torch.empty_like(y)
        dw = torch.empty_like(w)
        call("mlora_combine_backward", ptr(dout), ptr(y), H, ptr(w), _lib.dtype_code(w.dtype), ptr(inv), T, ctx.k,
             ptr(offsets), offsets.numel(), ptr(dy), ptr(dw), _lib.stream(dout.device))
        return dy, dw.view(ctx.wshape), None, None, None


# ---------------------------------------------------------------------------------------------
# the layer
# ---------------------------------------------------------------------------------------------

class Experts(torch.nn.Module):
    """A plain holder of expert stacks with the attributes of a Transformers experts module.

    gate_up_proj (E, 2I, H) and down_proj (E, H, I) (or transposed), frozen; SwiGLU gate.
    """

    def __init__(self, gate_up_proj, down_proj, is_transposed=False, gate_up_proj_scale_inv=None,
                 down_proj_scale_inv=None, gate_up_proj_bias=None, down_proj_bias=None):
        super().__init__()
        self.num_experts = gate_up_proj.shape[0]
        self.is_transposed = is_transposed
        self.has_gate = True
        self.has_bias = gate_up_proj_bias is not None
        self.gate_up_proj, self.down_proj = gate_up_proj, down_proj
        self.gate_up_proj_scale_inv, self.down_proj_scale_inv = gate_up_proj_scale_inv, down_proj_scale_inv
        self.gate_up_proj_bias, self.down_proj_bias = gate_up_proj_bias, down_proj_bias


def _stack_scale(experts, name):
    w = getattr(experts, name)
    if isinstance(w, torch.Tensor) and w.dtype == torch.float8_e4m3fn:
        return getattr(experts, name + "_scale_inv")
    return None


def _is_silu(act_fn) -> bool:
    return isinstance(act_fn, torch.nn.SiLU) or type(act_fn).__name__ in ("SiLU", "SiLUActivation")


def gate_of(experts):
    """None when the experts' gate is silu(first half) · second half — the SwiGLU the kernels fuse — else
    the callable that maps a gate_up output (S, 2I) to the activation (S, I) with PyTorch operations.

    The reference calls `experts._apply_gate` (src/meepsquared/_moe.py:118-119), which Transformers sets
    to `_default_apply_gate` (chunk, `act_fn(gate) * up`, TF:integrations/moe.py:509-520) unless the
    experts class defines its own: gpt-oss interleaves gate and up columns, clamps both and gates with
    `(up + 1) · gate · sigmoid(1.702 · gate)`; DeepSeek-V4 clamps.  Those, and a default gate whose act_fn
    is not SiLU, take the model's own gate function.
    """
    apply_gate = getattr(type(experts), "_apply_gate", None)
    default = apply_gate is None
    if apply_gate is not None:
        try:
            from transformers.integrations.moe import _default_apply_gate
        except ImportError:
            _default_apply_gate = None
        default = apply_gate is _default_apply_gate
    act_fn = getattr(experts, "act_fn", None)
    if default and (act_fn is None or _is_silu(act_fn)):
        return None
    if apply_gate is not None:
        return experts._apply_gate

    def gate(gate_up):
        g, u = gate_up.chunk(2, dim=-1)
        return act_fn(g) * u

    return gate


def routed_forward(experts, hidden_states, top_k_index, top_k_weights, factors):
    """The experts' forward with each adapter's change added per projection (src/meepsquared/_moe.py:70-126)."""
    if not getattr(experts, "has_gate", True):
        raise NotImplementedError("experts without a gate (up_proj alone) are not built: the kernels fuse SwiGLU")
    custom_gate = gate_of(experts)
    num_tokens = hidden_states.shape[0]
    k = top_k_index.shape[-1]
    perm, inv, offsets = sort_by_expert(top_k_index, experts.num_experts)

    def project(x, name, bias_name):
        weight = getattr(experts, name)
        lhs, rhs, scaling = factors.get(name, (None, None, 1.0))
        bias = getattr(experts, bias_name) if getattr(experts, "has_bias", False) else None
        return _grouped.lora_linear(x, weight, _stack_scale(experts, name), offsets, experts.is_transposed,
                                    lhs, rhs, scaling, bias)

    link = None
    down_bias = getattr(experts, "has_bias", False) and experts.down_proj_bias is not None
    swiglu_combined = custom_gate is None and _grouped.gathered_product_fits(experts.down_proj) and not down_bias
    if hidden_states.dtype == torch.bfloat16 and _grouped.gathered_product_fits(experts.gate_up_proj):
        # the gate_up product reads its rows straight from hidden_states through perm; the link hands the
        # SwiGLU it forms in its epilogue to the down Function below, and lets that Function's SwiGLU
        # backward form this product's B gradient from the dgu it writes
        lhs, rhs, scaling = factors.get("gate_up_proj", (None, None, 1.0))
        bias = experts.gate_up_proj_bias if getattr(experts, "has_bias", False) else None
        link = _grouped.GateUpLink(want_act=swiglu_combined)
        gate_up = _grouped.lora_linear_gathered(hidden_states, perm, inv, k, experts.gate_up_proj,
                                                _stack_scale(experts, "gate_up_proj"), offsets, experts.is_transposed,
                                                lhs, rhs, scaling, bias, link)
    else:
        gate_up = project(_Gather.apply(hidden_states, perm, inv, offsets, k), "gate_up_proj", "gate_up_proj_bias")
    if swiglu_combined:
        # SwiGLU, the down product and the combine as one Function: its backward reads the output
        # gradient through perm, and the SwiGLU backward applies the combine weights and forms their
        # gradient (y is not kept)
        lhs, rhs, scaling = factors.get("down_proj", (None, None, 1.0))
        result = _grouped.swiglu_lora_linear_combined(gate_up, top_k_weights, perm, inv, k, experts.down_proj,
                                                      _stack_scale(experts, "down_proj"), offsets,
                                                      experts.is_transposed, lhs, rhs, scaling, link)
        assert result.shape[0] == num_tokens
        return result.to(hidden_states.dtype)
    # the model's own gate (autograd through its PyTorch operations on the GPU), or the SwiGLU kernel
    act = custom_gate(gate_up) if custom_gate is not None else _SwiGLU.apply(gate_up)
    if act.dtype != gate_up.dtype:
        act = act.to(gate_up.dtype)
    if _grouped.gathered_product_fits(experts.down_proj):
        # the down product and the combine as one Function: its backward reads the output gradient
        # through perm, the combine weights applied per row, instead of a weighted copy of it
        lhs, rhs, scaling = factors.get("down_proj", (None, None, 1.0))
        bias = experts.down_proj_bias if getattr(experts, "has_bias", False) else None
        result = _grouped.lora_linear_combined(act, top_k_weights, perm, inv, k, experts.down_proj,
                                               _stack_scale(experts, "down_proj"), offsets, experts.is_transposed,
                                               lhs, rhs, scaling, bias)
    else:
        out = project(act, "down_proj", "down_proj_bias")
        result = _Combine.apply(out, top_k_weights, inv, offsets, k)
    assert result.shape[0] == num_tokens
    return result.to(hidden_states.dtype)
