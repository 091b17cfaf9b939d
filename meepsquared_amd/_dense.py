"""The dense SwiGLU MLP with LoRA on gate, up and down, on the grouped kernels with a single expert.

The counterpart of the reference's fused dense LoRA MLP (src/meepsquared/_vendor/axolotl/lora.py:398-830,
`LoRA_MLP` and `apply_lora_mlp_swiglu`):

    gate = X Wg^T + sg·(X Ag^T) Bg^T (+ bg),  up = X Wu^T + su·(X Au^T) Bu^T (+ bu)
    h = silu(gate) · up,                      out = h Wd^T + sd·(h Ad^T) Bd^T (+ bd)

with PEFT's factors A (r, in) (lora_A.weight) and B (out, r) (lora_B.weight), gradients for X and the six
factors, the base weights frozen.  Gate and up run as ONE product: their weights stacked [Wg; Wu] (made once
per frozen pair and kept), their adapters A = [Ag; Au] and B = blockdiag(Bg, Bu), so X is read once; then the
SwiGLU kernel; then the down product.  A base weight is a bf16 (out, in) tensor or an fp8 one given as
(weight8, scale) with one fp32 scale per tensor (meepsquared_amd._fp8.quantize / Fp8Linear), decoded in
registers inside the product.  Dropout on the adapters' input and DoRA are not built (refused).
"""

import torch

from meepsquared_amd import _grouped, _lib
from meepsquared_amd._moe import _SwiGLU


def _weight(w):
    """(tensor, scale or None) of a base weight: bf16 (out, in), or (fp8 (out, in), scale) with one scale."""
    if isinstance(w, tuple):
        w8, scale = w
        if w8.dtype != torch.float8_e4m3fn:
            raise TypeError(f"an fp8 base weight is given as (float8_e4m3fn tensor, scale), not {w8.dtype}")
        return w8, scale.reshape(()).float()
    if w.dtype not in (torch.bfloat16, torch.float8_e4m3fn):
        raise TypeError(f"a base weight in {w.dtype}: bf16, or (fp8, scale)")
    return w, None


def _stacked(wg, sg, wu, su):
    """([Wg; Wu] as a one-expert stack (1, 2I, H), its per-row scale (1, 2I) or None), kept on Wg."""
    key = (wu.data_ptr(), wg._version, wu._version, None if sg is None else (sg.data_ptr(), sg._version),
           None if su is None else (su.data_ptr(), su._version))
    held = getattr(wg, "_mlora_gate_up", None)
    if held is None or held[0] != key:
        stack = torch.cat([wg, wu], dim=0).unsqueeze(0)
        scale = None
        if sg is not None:
            scale = torch.cat([sg.expand(wg.shape[0]), su.expand(wu.shape[0])]).reshape(1, -1).contiguous()
        held = (key, stack, scale)
        wg._mlora_gate_up = held
    return held[1], held[2]


def _bias(b):
    return None if b is None else b.reshape(1, -1)


def lora_mlp_swiglu(X, gate_weight, gate_A, gate_B, gate_scale, up_weight, up_A, up_B, up_scale,
                    down_weight, down_A, down_B, down_scale, gate_bias=None, up_bias=None, down_bias=None):
    """The LoRA MLP's forward (differentiable in X and the factors): X (..., H) bf16 on the GPU; weights (out,
    in) bf16 or (fp8, scale); A (r, in), B (out, r) or None for a projection without adapters; scales
    alpha / r.  Returns (..., H) bf16.  As src/meepsquared/_vendor/axolotl/lora.py:398-830 without
    dropout or DoRA."""
    _lib.require_gpu(X)
    shape = X.shape
    x = X.reshape(-1, shape[-1])
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    rows = x.shape[0]
    offsets = torch.full((1,), rows, device=x.device, dtype=torch.int32)
    wg, sg = _weight(gate_weight)
    wu, su = _weight(up_weight)
    wd, sd = _weight(down_weight)
    if (sg is None) != (su is None) or wg.dtype != wu.dtype:
        raise TypeError("gate and up weights must be held alike (both bf16 or both fp8)")
    stack, row_scale = _stacked(wg, sg, wu, su)
    I = wg.shape[0]
    lhs = rhs = None
    scaling = 1.0
    if (gate_A is None) != (up_A is None):
        raise ValueError("LoRA on one of gate and up only is not built")
    if gate_A is not None:
        rg, ru = gate_A.shape[0], up_A.shape[0]
        if gate_scale == up_scale:
            scaling, bg, bu = gate_scale, gate_B, up_B
        else:  # different scalings: each B carries its own
            bg, bu = gate_B * gate_scale, up_B * up_scale
        # PEFT layout of the (out, in) stack: lhs = B (out, r), rhs = A (r, in); the joint B is block diagonal
        top = torch.cat([bg, bg.new_zeros(I, ru)], dim=1)
        bottom = torch.cat([bu.new_zeros(wu.shape[0], rg), bu], dim=1)
        lhs = torch.cat([top, bottom], dim=0).unsqueeze(0)
        rhs = torch.cat([gate_A, up_A], dim=0).unsqueeze(0)
    gb = None
    if gate_bias is not None or up_bias is not None:
        gb = torch.cat([gate_bias if gate_bias is not None else x.new_zeros(I),
                        up_bias if up_bias is not None else x.new_zeros(wu.shape[0])])
    gu = _grouped.lora_linear(x, stack, row_scale, offsets, False, lhs, rhs, scaling, _bias(gb), products_fp8=False)
    h = _SwiGLU.apply(gu)
    dstack = wd.unsqueeze(0)
    dl = None if down_A is None else down_B.unsqueeze(0)
    dr = None if down_A is None else down_A.unsqueeze(0)
    out = _grouped.lora_linear(h, dstack, None if sd is None else sd.reshape(1), offsets, False, dl, dr,
                               down_scale if down_A is not None else 1.0, _bias(down_bias), products_fp8=False)
    return out.reshape(*shape[:-1], out.shape[-1])


def _projection(module):
    """(weight, A, B, scaling, bias) of a projection: an nn.Linear (or Fp8Linear) with LoRA factors attached as
    `lora_A` (r, in), `lora_B` (out, r) and `lora_scaling`, or none."""
    from meepsquared_amd._fp8 import Fp8Linear

    if getattr(module, "lora_dropout_p", 0.0):
        raise NotImplementedError("LoRA dropout on the MLP's input is not built")
    if getattr(module, "lora_magnitude", None) is not None:
        raise NotImplementedError("DoRA is not built")
    weight = (module.weight, module.weight_scale_inv) if isinstance(module, Fp8Linear) else module.weight
    return (weight, getattr(module, "lora_A", None), getattr(module, "lora_B", None),
            getattr(module, "lora_scaling", 1.0), module.bias)


def apply_lora_mlp_swiglu(mlp, X):
    """The SwiGLU MLP module `mlp` (gate_proj, up_proj, down_proj) with its attached adapters over X, as
    src/meepsquared/_vendor/axolotl/lora.py:831-880 dispatches it."""
    gw, ga, gbm, gs, gbias = _projection(mlp.gate_proj)
    uw, ua, ub, us, ubias = _projection(mlp.up_proj)
    dw, da, db, ds, dbias = _projection(mlp.down_proj)
    return lora_mlp_swiglu(X, gw, ga, gbm, gs, uw, ua, ub, us, dw, da, db, ds, gbias, ubias, dbias)
