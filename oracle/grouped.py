"""Product oracle: the per-expert float32 loop of the reference, differentiable (PyTorch).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""

import torch


def reference(x, weight, offsets, is_transposed: bool):
    """The base product, one expert at a time, in float32 — src/meepsquared/_grouped.py:420-428.

    Pinned by: a single expert equals one dense product; the closed-form input gradient of
    out.sum() (tests/test_grouped.py:146-157) (tests/test_oracle.py).
    """
    out = torch.empty((x.shape[0], weight.shape[2] if is_transposed else weight.shape[1]), device=x.device,
                      dtype=x.dtype)
    start = 0
    for e, end in enumerate(torch.as_tensor(offsets).tolist()):
        w = weight[e].float()
        out[start:end] = (x[start:end].float() @ (w if is_transposed else w.t())).to(x.dtype)
        start = end
    return out


def reference_lora(x, weight, scale, offsets, is_transposed, lhs, rhs, scaling, bias=None, out_dtype=None):
    """The whole product with PyTorch operations, differentiable — src/meepsquared/_grouped.py:431-444.

    scale is (experts,) (the reference's fp8 stacks) or (experts, out) (one per output row).
    Rows past offsets[-1] are not produced (the result has offsets[-1] rows).
    Pinned by: rank-1 indicator adapters (closed form), the layout identity between a stack and
    its transpose, float64 gradcheck, and the no-adapter input gradient (tests/test_oracle.py).
    """
    cd = torch.float64 if x.dtype == torch.float64 else torch.float32  # float32, or float64 for gradcheck
    out = []
    start = 0
    for e, end in enumerate(torch.as_tensor(offsets).tolist()):
        w = weight[e].to(cd)
        if scale is not None:
            s = scale[e].to(cd)
            if s.dim() == 1:  # one scale per output row: rows of (out, in), columns of (in, out)
                s = s.view(1, -1) if is_transposed else s.view(-1, 1)
            w = w * s
        if lhs is not None:
            w = w + scaling * (lhs[e].to(cd) @ rhs[e].to(cd))
        y = x[start:end].to(cd) @ (w if is_transposed else w.t())
        if bias is not None:
            y = y + bias[e].to(cd)
        out.append(y)
        start = end
    return torch.cat(out).to(out_dtype or x.dtype)


def reference_lora_bf16_low(x, weight, scale, offsets, is_transposed, lhs, rhs, scaling, bias=None):
    """As reference_lora but with the low-rank product x·A rounded to bf16 before ·B, the rounding
    the reference's kernel (and this build's) apply (src/meepsquared/_grouped.py:211-214); fp32
    elsewhere.  Used to bound the kernel's error more tightly than against the merged-weight form."""
    out = []
    start = 0
    for e, end in enumerate(torch.as_tensor(offsets).tolist()):
        w = weight[e].float()
        if scale is not None:
            s = scale[e].float()
            if s.dim() == 1:
                s = s.view(1, -1) if is_transposed else s.view(-1, 1)
            w = w * s
        xe = x[start:end].float()
        y = xe @ (w if is_transposed else w.t())
        if lhs is not None:
            if is_transposed:
                low = (xe @ lhs[e].float()).to(torch.bfloat16).float()
                y = y + scaling * (low @ rhs[e].float())
            else:
                low = (xe @ rhs[e].float().t()).to(torch.bfloat16).float()
                y = y + scaling * (low @ lhs[e].float().t())
        if bias is not None:
            y = y + bias[e].float()
        out.append(y)
        start = end
    return torch.cat(out)


def lora_mlp_swiglu(x, gate, up, down, biases=(None, None, None)):
    """The dense SwiGLU MLP with LoRA on each projection, float32, differentiable — the forward of
    src/meepsquared/_vendor/axolotl/lora.py:398-830 (LoRA_MLP, no dropout, no DoRA): each projection
    (W (out, in), A (r, in) or None, B (out, r), s) as reference_lora over one expert, then
    silu(gate) · up.
    Pinned by: reference_lora (pinned above) and the SwiGLU oracle (tests/test_oracle.py)."""
    from oracle.moe import swiglu

    rows = x.shape[0]
    offsets = [rows]

    def proj(h, p, b):
        w, a, bb, s = p
        return reference_lora(h, w.float().unsqueeze(0), None, offsets, False,
                              None if a is None else bb.float().unsqueeze(0), None if a is None else a.float().unsqueeze(0),
                              s, None if b is None else b.float().unsqueeze(0), out_dtype=torch.float32)

    g = proj(x.float(), gate, biases[0])
    u = proj(x.float(), up, biases[1])
    return proj(swiglu(torch.cat([g, u], dim=-1)), down, biases[2])
