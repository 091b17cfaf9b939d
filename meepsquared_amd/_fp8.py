"""Expert stacks held as fp8 e4m3 with fp32 scales, converted on the GPU.

One scale per expert is the reference's format (src/meepsquared/_fp8.py:111-134: scale =
max(amax, 1e-12) / 448, q = e4m3(w / scale), registered as `<name>_scale_inv`).  One scale per
output row is this package's extension: an (experts, out) scale, which the grouped product applies
in its epilogue (forward) or in its weight decode (input gradient).
"""

import torch

from meepsquared_amd import _lib
from meepsquared_amd._lib import call, ptr

E4M3_MAX = 448.0
STACK_SCALE = "_scale_inv"


def _group(per_row: bool):
    return _lib.SCALE_ROW if per_row else _lib.SCALE_EXPERT


def quantize_stack(weight: torch.Tensor, per_row: bool = False, is_transposed: bool = False):
    """(w8, scale): the stack as e4m3 with one scale per expert (E,) or per output row (E, out).

    A stack (E, out, in) has its output rows on dim 1; a transposed stack (E, in, out) on dim 2.
    """
    _lib.require_gpu(weight)
    w = weight.detach()
    if w.dtype not in (torch.bfloat16, torch.float32):
        w = w.float()
    w = w.contiguous()
    E, R, C = w.shape
    q = torch.empty(w.shape, device=w.device, dtype=torch.float8_e4m3fn)
    if per_row:
        scale = torch.empty((E, C if is_transposed else R), device=w.device, dtype=torch.float32)
    else:
        scale = torch.empty((E,), device=w.device, dtype=torch.float32)
    call("mlora_fp8_quantize", ptr(w), _lib.dtype_code(w.dtype), E, R, C, _group(per_row), int(per_row and is_transposed),
         ptr(q), ptr(scale), _lib.stream(w.device))
    return q, scale


def dequantize_stack(weight8: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype, is_transposed: bool = False):
    """The stack back in a compute dtype (bf16/fp32), for comparisons and the reference's twin."""
    _lib.require_gpu(weight8, scale)
    E, R, C = weight8.shape
    per_row = scale.dim() == 2
    out = torch.empty(weight8.shape, device=weight8.device, dtype=dtype)
    call("mlora_fp8_dequantize", ptr(weight8.contiguous()), ptr(scale.float().contiguous()), E, R, C, _group(per_row),
         int(per_row and is_transposed), ptr(out), _lib.dtype_code(dtype), _lib.stream(weight8.device))
    return out


def convert_stacks(experts, per_row: bool = False) -> int:
    """Every frozen 3-D float stack of an experts module held as fp8, its scale as `<name>_scale_inv`.

    As src/meepsquared/_fp8.py:170-186 (one scale per expert), or one scale per output row.
    """
    converted = 0
    for name, parameter in list(experts.named_parameters(recurse=False)):
        if parameter.dim() != 3 or parameter.requires_grad or not parameter.is_floating_point():
            continue
        if parameter.dtype == torch.float8_e4m3fn and hasattr(experts, name + STACK_SCALE):
            converted += 1
            continue
        w8, scale = quantize_stack(parameter.detach(), per_row, bool(getattr(experts, "is_transposed", False)))
        setattr(experts, name, torch.nn.Parameter(w8, requires_grad=False))
        experts.register_buffer(name + STACK_SCALE, scale)
        converted += 1
    if converted:
        experts._meepsquared_fp8 = True
    return converted


# ---------------------------------------------------------------------------------------------
# Frozen dense layers held as fp8 (src/meepsquared/_fp8.py:95-109, 198-293): one scale per tensor, each
# product on the fp8 MFMA — the grouped product with a single expert, the activations quantised on the
# way in by its prep pass (per row and 64 columns, two e4m3 terms: see meepsquared_amd._grouped).
# ---------------------------------------------------------------------------------------------

# the routers of a mixture of experts keep their bf16 weights (src/meepsquared/_fp8.py:258-259)
ROUTERS = ("gate", "router")
# the products take in/out features that are multiples of this (src/meepsquared/_fp8.py:260-261)
SIZE_MULTIPLE = 16


def quantize(x: torch.Tensor):
    """(x8, scale): x as fp8 e4m3 with one fp32 scale for the whole tensor, x ≈ x8 · scale, scale =
    max(amax, 1e-12) / 448 (src/meepsquared/_fp8.py:95-109), on the GPU."""
    _lib.require_gpu(x)
    w = x.detach()
    if w.dtype not in (torch.bfloat16, torch.float32):
        w = w.float()
    w = w.contiguous()
    C = w.shape[-1] if w.dim() else 1
    R = w.numel() // max(C, 1)
    q = torch.empty(w.shape, device=w.device, dtype=torch.float8_e4m3fn)
    scale = torch.empty((1,), device=w.device, dtype=torch.float32)
    call("mlora_fp8_quantize", ptr(w), _lib.dtype_code(w.dtype), 1, R, C, _lib.SCALE_EXPERT, 0, ptr(q), ptr(scale),
         _lib.stream(w.device))
    return q, scale.reshape(())


def _as_stack(weight8: torch.Tensor) -> torch.Tensor:
    """The (out, in) fp8 weight as a one-expert stack (1, out, in), one view kept on the weight, so that the
    byte-transposed copy the input-gradient product reads is made once per weight and reused."""
    stack = getattr(weight8, "_mlora_stack", None)
    if stack is None or stack.data_ptr() != weight8.data_ptr():
        stack = weight8.view(1, *weight8.shape)
        weight8._mlora_stack = stack
    return stack


def scaled_mm(x: torch.Tensor, weight8: torch.Tensor, weight_scale: torch.Tensor, transpose_weight: bool,
              bias: torch.Tensor = None) -> torch.Tensor:
    """x @ W^T (transpose_weight) or x @ W with W ≈ weight8 · weight_scale, in bf16
    (src/meepsquared/_fp8.py:198-211); bias (out,) added in the product's epilogue.

    weight8 is (out, in) row-major; x (..., in) or (..., out).  The product is the grouped fp8 product over
    one expert: weight8 read with k contiguous as it lies for x @ W^T, through its byte-transposed copy for
    x @ W.  There is no CPU path: a CPU tensor is a TypeError.
    """
    from meepsquared_amd import _grouped

    _lib.require_gpu(x, weight8, weight_scale)
    if weight8.dtype != torch.float8_e4m3fn or weight8.dim() != 2:
        raise TypeError(f"weight8 must be a 2-D float8_e4m3fn tensor, not {weight8.dtype} {tuple(weight8.shape)}")
    x2 = x.reshape(-1, x.shape[-1])
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
    rows = x2.shape[0]
    stack = _as_stack(weight8)
    offsets = torch.full((1,), rows, device=x.device, dtype=torch.int32)
    scale = weight_scale.reshape(1).to(torch.float32)
    b = None if bias is None else bias.reshape(1, -1)
    out, _ = _grouped._launch_fp8(x2, stack, scale, offsets, not transpose_weight, None, 1.0, b, False,
                                  backward=not transpose_weight)
    return out.reshape(*x.shape[:-1], out.shape[-1])


class _Fp8Product(torch.autograd.Function):
    """y = x @ W^T (+ bias) with W in fp8; the backward gives x's gradient only, W and the bias frozen
    (src/meepsquared/_fp8.py:214-224)."""

    @staticmethod
    def forward(ctx, x, weight8, weight_scale, bias=None):
        ctx.weight8, ctx.weight_scale = weight8, weight_scale
        return scaled_mm(x, weight8, weight_scale, transpose_weight=True, bias=bias)

    @staticmethod
    def backward(ctx, grad_out):
        return scaled_mm(grad_out, ctx.weight8, ctx.weight_scale, transpose_weight=False), None, None, None


class Fp8Linear(torch.nn.Module):
    """A frozen linear layer held as fp8 with one scale; its bias, if any, stays as it was and is added in
    the product's epilogue (src/meepsquared/_fp8.py:227-255).

    weight is the fp8 tensor and weight_scale_inv its scale (W ≈ weight · weight_scale_inv).
    """

    def __init__(self, linear: torch.nn.Linear):
        super().__init__()
        self.in_features, self.out_features = linear.in_features, linear.out_features
        weight8, scale = quantize(linear.weight.detach())
        self.register_buffer("weight", weight8)
        self.register_buffer("weight_scale_inv", scale)
        self.bias = linear.bias
        self.dtype = linear.weight.dtype

    def forward(self, x):
        """bf16 out, as torch._scaled_mm gives the reference's (src/meepsquared/_fp8.py:243-248)."""
        bias = self.bias
        if bias is not None and bias.requires_grad:  # a trained bias takes its gradient through autograd
            return _Fp8Product.apply(x, self.weight, self.weight_scale_inv, None) + bias
        return _Fp8Product.apply(x, self.weight, self.weight_scale_inv, None if bias is None else bias.detach())

    def dequantized(self) -> torch.Tensor:
        """The weight back in its dtype, for a merged save."""
        return (self.weight.float() * self.weight_scale_inv).to(self.dtype)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, fp8 e4m3, one scale"


def convertible(module, name: str, trainable: set) -> bool:
    """A frozen nn.Linear of a decoder layer, not an adapter, not the output layer, not a router, its sizes
    multiples of 16 (src/meepsquared/_fp8.py:264-269)."""
    return (type(module) is torch.nn.Linear and module.weight.dim() == 2 and not module.weight.requires_grad
            and "lora_" not in name and not name.endswith("lm_head") and name not in trainable
            and name.rsplit(".", 1)[-1] not in ROUTERS
            and module.in_features % SIZE_MULTIPLE == 0 and module.out_features % SIZE_MULTIPLE == 0)


def decoder_layers(model):
    """The decoder layers of a Transformers model: the longest nn.ModuleList named `layers` (or `h`)."""
    best = None
    for name, module in model.named_modules():
        if isinstance(module, torch.nn.ModuleList) and name.rsplit(".", 1)[-1] in ("layers", "h"):
            if best is None or len(module) > len(best):
                best = module
    return list(best) if best is not None else []


def apply(model, per_row_stacks: bool = False) -> int:
    """Every frozen linear layer of the decoder layers held as fp8 (Fp8Linear), and every expert stack of an
    experts module routed by this package (convert_stacks); returns how many.  Applying again changes
    nothing.  As src/meepsquared/_fp8.py:272-293."""
    from meepsquared_amd import _experts

    trainable = {name.rsplit(".", 1)[0] for name, p in model.named_parameters() if p.requires_grad}
    converted = 0
    for layer in decoder_layers(model):
        for name, module in list(layer.named_modules()):
            if _experts.is_experts(module):
                converted += convert_stacks(module, per_row_stacks)
            if isinstance(module, Fp8Linear):  # held as fp8 already
                converted += 1
                continue
            if not convertible(module, name, trainable):
                continue
            parent = layer.get_submodule(name.rsplit(".", 1)[0]) if "." in name else layer
            setattr(parent, name.rsplit(".", 1)[-1], Fp8Linear(module).to(module.weight.device))
            converted += 1
    if not converted:
        raise ValueError("found no frozen linear layer to hold as fp8")
    return converted
