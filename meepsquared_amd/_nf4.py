"""Expert stacks held as NF4 (4-bit NormalFloat, blocks of 64) with double quantisation, on the GPU.

The format is QLoRA's (Dettmers et al. 2023, "QLoRA: Efficient Finetuning of Quantized LLMs"):

* each block of 64 consecutive values (along the stack's contiguous axis) has an absmax; each value
  is stored as the 4-bit index of the nearest NF4 code to value / absmax, two per byte, the first
  value in the high nibble (the packing of bitsandbytes' 4-bit layout, which the reference uses
  for dense layers through src/meepsquared/_vendor/axolotl/quantize.py:52-101);
* double quantisation: offset = the mean of the absmaxes; (absmax - offset) is quantised to 8 bits
  with a signed dynamic code (CODE2) in groups of 256 blocks, each group with an fp32 absmax2;
  a block's absmax decodes as CODE2[q] * absmax2[block / 256] + offset.

The reference has no NF4 expert stack; interoperability with bitsandbytes' bytes is not claimed.
The grouped product decodes this format in registers in its main loop.
"""

import torch

from meepsquared_amd import _lib
from meepsquared_amd._grouped import Nf4Stack
from meepsquared_amd._lib import call, ptr

BLOCKSIZE = 64
BLOCKSIZE2 = 256

# The 16 NF4 values, as published in the QLoRA paper (Appendix E): quantiles of N(0, 1) normalised
# to [-1, 1] with an exact zero.  tests/ re-derive them from that definition.
NF4_CODE = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
)


def dynamic_code(max_exponent_bits: int = 7) -> list:
    """The signed 8-bit dynamic (tree) code: for each decade 10^(i-6), i = 0..6, 2^i linear steps
    between 0.1 and 1 of that decade (midpoints of 2^i + 1 boundaries), both signs, plus 0 and 1;
    256 values, ascending (Dettmers et al. 2022, "8-bit Optimizers via Block-wise Quantization")."""
    values = []
    for i in range(max_exponent_bits):
        n = 2 ** i + 1
        bounds = [0.1 + (1.0 - 0.1) * j / (n - 1) for j in range(n)]
        means = [(a + b) / 2.0 for a, b in zip(bounds[:-1], bounds[1:])]
        decade = 10.0 ** (-(max_exponent_bits - 1) + i)
        values += [decade * m for m in means] + [-decade * m for m in means]
    values += [0.0, 1.0]
    return sorted(values)


_CODES = {}


def codes(device):
    """(NF4 code, second-level code) as fp32 tensors on `device`."""
    key = str(device)
    if key not in _CODES:
        _CODES[key] = (torch.tensor(NF4_CODE, dtype=torch.float32, device=device),
                       torch.tensor(dynamic_code(), dtype=torch.float32, device=device))
    return _CODES[key]


def quantize_stack(weight: torch.Tensor) -> Nf4Stack:
    """The stack (E, a, b) as NF4: blocks of 64 along its last (contiguous) axis, b % 64 == 0."""
    _lib.require_gpu(weight)
    w = weight.detach()
    if w.dtype not in (torch.bfloat16, torch.float32):
        w = w.float()
    w = w.contiguous()
    if w.dim() != 3 or w.shape[2] % BLOCKSIZE:
        raise ValueError(f"an NF4 stack needs 3 dims and a last axis of a multiple of {BLOCKSIZE}: {tuple(w.shape)}")
    n = w.numel()
    nblocks = n // BLOCKSIZE
    dev = w.device
    code, code2 = codes(dev)
    packed = torch.empty(n // 2, device=dev, dtype=torch.uint8)
    absmax_q = torch.empty(nblocks, device=dev, dtype=torch.uint8)
    absmax2 = torch.empty((nblocks + BLOCKSIZE2 - 1) // BLOCKSIZE2, device=dev, dtype=torch.float32)
    offset = torch.empty(1, device=dev, dtype=torch.float32)
    ws = torch.empty(int(_lib.lib.mlora_nf4_workspace_bytes(n)), device=dev, dtype=torch.uint8)
    call("mlora_nf4_quantize", ptr(w), _lib.dtype_code(w.dtype), n, ptr(code), ptr(code2), ptr(packed), ptr(absmax_q),
         ptr(absmax2), ptr(offset), ptr(ws), ws.numel(), _lib.stream(dev))
    return Nf4Stack(packed, absmax_q, absmax2, offset, code, code2, w.shape)


def dequantize_stack(stack: Nf4Stack, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """The stack decoded to bf16 or fp32 (the twin the product is compared with)."""
    out = torch.empty(stack.shape, device=stack.device, dtype=dtype)
    call("mlora_nf4_dequantize", ptr(stack.packed), ptr(stack.absmax_q), ptr(stack.absmax2), ptr(stack.offset),
         ptr(stack.code), ptr(stack.code2), out.numel(), ptr(out), _lib.dtype_code(dtype), _lib.stream(stack.device))
    return out


def convert_stacks(experts) -> int:
    """Every frozen 3-D float stack of an experts module held as NF4 (QLoRA-style); returns how many.

    The NF4 counterpart of `_fp8.convert_stacks` (src/meepsquared/_fp8.py:170-186): the parameter is
    replaced by an `Nf4Stack` attribute, which the routed forward computes with (decoded in the grouped
    product).  Stacks already held as NF4 count as converted.
    """
    converted = 0
    for name in list(dict(experts.named_parameters(recurse=False))) + [
            n for n, v in vars(experts).items() if isinstance(v, Nf4Stack)]:
        value = getattr(experts, name)
        if isinstance(value, Nf4Stack):
            converted += 1
            continue
        if value.dim() != 3 or value.requires_grad or not value.is_floating_point():
            continue
        stack = quantize_stack(value.detach())
        delattr(experts, name)  # the parameter goes; the packed stack is a plain attribute
        setattr(experts, name, stack)
        converted += 1
    return converted
