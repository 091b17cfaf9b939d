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
