"""The experts' products with their LoRA adapters, one kernel launch each, on MI355X (gfx950).

The rows of x are sorted by expert; offsets[e] is the end of expert e's rows.  For every expert e
and its rows x_e the forward computes

    out_e = c_e · x_e @ W_e^T + s · bf16(x_e @ A_e^T) @ B_e^T + bias_e

with the stack W as (experts, out, in) or, when is_transposed, (experts, in, out), in bf16, in
fp8 e4m3 with one scale per expert or per output row (c_e), or in NF4 (`meepsquared_amd._nf4`);
the adapters are PEFT's lhs and rhs factors in the stack's layout.  The kernel is
`csrc/grouped_gemm.hip`, reached through the C ABI of `include/mlora.h`.

This module keeps the interface of the reference's `src/meepsquared/_grouped.py`: BLOCK_M and
RANK_MULTIPLE (:51-52), max_tiles and tile_map (:83-103), the stack-stride check and its
ValueError (:264-272), the rank padding (:275-282), the adapters' roles (:285-310),
grouped_linear (:348-359), the autograd Function with its gradient tuple (:373-405) and
lora_linear (:408-417).  The per-expert float32 references (:420-444) are test oracles and live
in the repository's `oracle/` package, not here.
"""

import os

import torch

from meepsquared_amd import _lib
from meepsquared_amd._lib import call, ptr

BLOCK_M = 128
RANK_MULTIPLE = 16  # the kernel's low-rank MFMAs take the rank in blocks of 16

# For measurement only: when set, called as launch_observer(kernel, phase, info) with phase
# "before"/"after" around each product or reduction launch, on the launching thread (the launch
# goes to torch's current stream); info holds the launch's sizes.  None in normal use.
launch_observer = None


def max_tiles(rows: int, experts: int, block_m: int = BLOCK_M) -> int:
    """An upper bound on the tiles: every expert's last tile may be partial (_grouped.py:83-85)."""
    return rows // block_m + experts


def tile_map(offsets: torch.Tensor, rows: int, block_m: int = BLOCK_M):
    """(tile_expert, tile_row, tiles) for `rows` rows sorted by expert, computed on the GPU.

    offsets[e] is the end of expert e's rows (int32, on the device).  The two arrays have
    max_tiles entries; tiles, a 0-d int32 tensor on the device, says how many are real.  Entries
    beyond that hold the last expert.  Same values as src/meepsquared/_grouped.py:88-103.
    The product kernel derives this map itself; this function exposes it.
    """
    _lib.require_gpu(offsets)
    offsets = offsets.to(torch.int32).contiguous()
    experts = offsets.numel()
    n = max_tiles(rows, experts, block_m)
    tile_expert = torch.empty(n, device=offsets.device, dtype=torch.int32)
    tile_row = torch.empty(n, device=offsets.device, dtype=torch.int32)
    tiles = torch.empty((), device=offsets.device, dtype=torch.int32)
    call("mlora_tile_map", ptr(offsets), experts, rows, block_m, ptr(tile_expert), ptr(tile_row), ptr(tiles), n,
         _lib.stream(offsets.device))
    return tile_expert, tile_row, tiles


class Nf4Stack:
    """An expert stack held as NF4 with double quantisation (made by meepsquared_amd._nf4.quantize_stack)."""

    def __init__(self, packed, absmax_q, absmax2, offset, code, code2, shape, dtype=torch.bfloat16):
        self.packed, self.absmax_q, self.absmax2, self.offset = packed, absmax_q, absmax2, offset
        self.code, self.code2 = code, code2
        self.shape = torch.Size(shape)
        self.dtype = dtype  # the dtype it dequantises to

    @property
    def device(self):
        return self.packed.device

    @property
    def is_cuda(self):
        return self.packed.is_cuda

    def dim(self):
        return 3

    def stride(self, d=None):
        strides = (self.shape[1] * self.shape[2], self.shape[2], 1)
        return strides if d is None else strides[d]


def _nf4_transposed(stack: Nf4Stack):
    """(codes (E, C, R/2) uint8, absmax (E, C/64, R) fp32) of an NF4 stack (E, R, C): its transpose's codes
    packed along R and every block's decoded absmax, for the products that read it with R as k.  Made once by
    the library's mlora_nf4_transpose and kept on the stack (a frozen stack: made once, reused every step)."""
    held = getattr(stack, "_mlora_transposed", None)
    if held is None:
        E, R, C = stack.shape
        codes_t = torch.empty((E, C, R // 2), device=stack.device, dtype=torch.uint8)
        absmax_t = torch.empty((E, C // 64, R), device=stack.device, dtype=torch.float32)
        call("mlora_nf4_transpose", ptr(stack.packed), ptr(stack.absmax_q), ptr(stack.absmax2), ptr(stack.offset),
             ptr(stack.code2), E, R, C, ptr(codes_t), ptr(absmax_t), _lib.stream(stack.device))
        held = (codes_t, absmax_t)
        stack._mlora_transposed = held
    return held


def _stack_strides(weight, K: int, is_transposed: bool):
    """(N, stride_e, stride_k, stride_n) of a stack addressed as (k, n); src/meepsquared/_grouped.py:264-272."""
    if is_transposed:
        if weight.shape[1] != K:
            raise ValueError(f"a transposed stack (experts, in, out) with in={weight.shape[1]} does not take x with {K} columns")
        return weight.shape[2], weight.stride(0), weight.stride(1), weight.stride(2)
    if weight.shape[2] != K:
        raise ValueError(f"a stack (experts, out, in) with in={weight.shape[2]} does not take x with {K} columns")
    return weight.shape[1], weight.stride(0), weight.stride(2), weight.stride(1)


def _padded_rank(factor: torch.Tensor, dim: int) -> torch.Tensor:
    """The factor with its rank dimension padded with zeros to a multiple of RANK_MULTIPLE (_grouped.py:275-282)."""
    pad = -factor.shape[dim] % RANK_MULTIPLE
    if not pad:
        return factor
    shape = list(factor.shape)
    shape[dim] = pad
    return torch.cat([factor, factor.new_zeros(shape)], dim=dim)


class _Adapters:
    """PEFT's factors as the kernel reads them: A^T as (e, R, k) and B^T as (e, n, R), R the padded rank.

    delta = lhs @ rhs in the stack's layout: (out, in) means lhs (out, rank) and rhs (rank, in),
    so A = rhs^T and B = lhs^T; (in, out) means lhs (in, rank) and rhs (rank, out), so A = lhs and
    B = rhs.  Roles as in src/meepsquared/_grouped.py:285-310.
    """

    def __init__(self, lhs, rhs, is_transposed):
        self.rank = lhs.shape[2]
        if is_transposed:
            at, bt = lhs.transpose(1, 2), rhs.transpose(1, 2)
        else:
            at, bt = rhs, lhs
        self.at = _padded_rank(at, 1).to(torch.bfloat16).contiguous()  # (e, R, k)
        self.bt = _padded_rank(bt, 2).to(torch.bfloat16).contiguous()  # (e, n, R)
        self.padded = self.at.shape[1]
        self.partner = None  # another projection's adapters, swapped in the same launch as these
        self._swapped = None  # these adapters swapped by the partner's launch, not yet taken

    def _pairable(self):
        E, R, K = self.at.shape
        N = self.bt.shape[1]
        return R in (16, 32) and K > R and N > R and K % 8 == 0 and N % 8 == 0

    def _empty_swapped(self):
        other = object.__new__(_Adapters)
        other.rank, other.padded, other.partner, other._swapped = self.rank, self.padded, None, None
        E, R, K = self.at.shape
        other.at = torch.empty((E, R, self.bt.shape[1]), device=self.at.device, dtype=torch.bfloat16)
        other.bt = torch.empty((E, K, R), device=self.at.device, dtype=torch.bfloat16)
        return other

    def _swap_args(self, other):
        E, R, K = self.at.shape
        return (ptr(self.at), self.at.stride(0), self.at.stride(1), ptr(self.bt), self.bt.stride(0), self.bt.stride(1),
                E, R, K, self.bt.shape[1], ptr(other.at), ptr(other.bt))

    def swapped(self):
        """The adapters of the input-gradient product: B takes A's role and A B's (_grouped.py:304-310).  With
        a partner (the layer's other projection) whose swap is still to come, both are swapped in one launch
        and the partner keeps its result until its own backward takes it (once)."""
        if self._swapped is not None:
            other, self._swapped = self._swapped, None
            return other
        if self._pairable():  # both transposes in one launch
            other = self._empty_swapped()
            p = self.partner
            if (p is not None and p._swapped is None and p._pairable() and p.at.device == self.at.device):
                p_other = p._empty_swapped()
                call("mlora_swap_adapters_two", *self._swap_args(other), *p._swap_args(p_other),
                     _lib.stream(self.at.device))
                p._swapped, self.partner, p.partner = p_other, None, None
            else:
                call("mlora_swap_adapters", *self._swap_args(other), _lib.stream(self.at.device))
        else:
            other = object.__new__(_Adapters)
            other.rank, other.padded, other.partner, other._swapped = self.rank, self.padded, None, None
            other.at = _transposed(self.bt)  # (e, R, n): B's rows become the new k
            other.bt = _transposed(self.at)  # (e, k, R)
        return other


def _transposed(t: torch.Tensor) -> torch.Tensor:
    """A contiguous (E, b, a) copy of the bf16 (E, a, b) tensor t, by the library's transpose kernel."""
    E, A, B = t.shape
    out = torch.empty((E, B, A), device=t.device, dtype=t.dtype)
    call("mlora_transpose", ptr(t), E, A, B, t.stride(0), t.stride(1), t.stride(2), ptr(out), _lib.stream(t.device))
    return out


def _scale_args(scale, weight, backward: bool, is_transposed: bool):
    """(scale, kind, stride_e, on_k): one scale per expert (E,) or per output row (E, out) of the stack.

    is_transposed is the layout the launch reads the stack in; in the input-gradient pass (backward)
    that is the other one, and the stack's output rows run along k."""
    if scale is None:
        return None, _lib.SCALE_NONE, 0, 0
    _lib.require_gpu(scale)
    scale = scale.to(torch.float32).contiguous()
    if scale.dim() == 1:
        if scale.numel() != weight.shape[0]:
            raise ValueError(f"a per-expert scale needs {weight.shape[0]} values, got {scale.numel()}")
        return scale, _lib.SCALE_EXPERT, 0, 0
    stack_transposed = is_transposed != backward  # the stack's own layout: (E, in, out) when True
    out_rows = weight.shape[2] if stack_transposed else weight.shape[1]
    if scale.dim() == 2 and tuple(scale.shape) == (weight.shape[0], out_rows):
        return scale, _lib.SCALE_ROW, scale.stride(0), int(backward)
    raise ValueError(f"scale of shape {tuple(scale.shape)} is neither ({weight.shape[0]},) per expert nor "
                     f"({weight.shape[0]}, {out_rows}) per output row of the stack")


def _stack_operand(weight, K, N, is_transposed, scale, backward):
    """The stack as the kernels take it: (w_ptr, w_dtype, w_se, w_sk, w_sn, the five NF4 arguments, the scale
    arguments of _scale_args).  An NF4 stack read with n contiguous goes through its transposed codes, an fp8
    stack read so through its k-contiguous byte copy (both made once and kept on the stack)."""
    _, w_se, w_sk, w_sn = _stack_strides(weight, K, is_transposed)
    scale_args = _scale_args(scale, weight, backward, is_transposed)
    nf4 = (None,) * 5
    if isinstance(weight, Nf4Stack) and w_sk != 1:
        # read with n contiguous (blocks along n): the stack's transposed codes and absmax table, kept on it
        codes_t, absmax_t = _nf4_transposed(weight)
        w_ptr, w_dtype = ptr(codes_t), _lib.DT_NF4_KT
        w_se, w_sk, w_sn = codes_t.shape[1] * codes_t.shape[2] * 2, 1, codes_t.shape[2] * 2
        nf4 = (None, ptr(absmax_t), None, None, ptr(weight.code))
    elif isinstance(weight, Nf4Stack):
        w_ptr, w_dtype = ptr(weight.packed), _lib.DT_NF4
        nf4 = (ptr(weight.absmax_q), ptr(weight.absmax2), ptr(weight.code2), ptr(weight.offset), ptr(weight.code))
    else:
        _lib.require_gpu(weight)
        if weight.dtype not in (torch.bfloat16, torch.float8_e4m3fn):
            raise TypeError(f"a stack in {weight.dtype}: the kernel takes bf16, float8_e4m3fn or NF4")
        w_ptr, w_dtype = ptr(weight), _lib.dtype_code(weight.dtype)
        if weight.dtype == torch.float8_e4m3fn and w_sk != 1 and w_sn == 1:
            # an fp8 stack read with n contiguous: its k-contiguous byte copy (kept on the stack), which the
            # DMA-fed product decodes in registers
            w8, w_se, w_sn = _k_contiguous(weight, w_se, w_sk, w_sn, K, N)
            w_sk, w_ptr = 1, ptr(w8)
    return w_ptr, w_dtype, w_se, w_sk, w_sn, nf4, scale_args


def _launch(x, weight, scale, offsets, is_transposed, adapters, scaling, bias, store_low, backward=False,
            products_fp8=False):
    """One launch of the product kernel. Returns (out, low), low None without adapters or store_low.
    products_fp8: the fp8 products (only for an fp8 stack; resolved by the caller as _x_fp8 does)."""
    _lib.require_gpu(x, offsets)
    if x.dtype != torch.bfloat16:
        raise TypeError(f"x is {x.dtype}; the kernel computes in bf16")
    if products_fp8:
        return _launch_fp8(x, weight, scale, offsets, is_transposed, adapters, scaling, bias, store_low, backward)
    rows, K = x.shape
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    N = _stack_strides(weight, K, is_transposed)[0]
    out = torch.empty((rows, N), device=x.device, dtype=x.dtype)
    R = adapters.padded if adapters is not None else 0
    low = torch.empty((rows, R), device=x.device, dtype=torch.bfloat16) if (adapters is not None and store_low) else None
    if rows == 0:
        return out, low
    offsets = offsets if offsets.dtype == torch.int32 else offsets.to(torch.int32)
    offsets = offsets.contiguous()
    w_ptr, w_dtype, w_se, w_sk, w_sn, nf4, (scale, scale_kind, scale_se, scale_on_k) = _stack_operand(
        weight, K, N, is_transposed, scale, backward)
    if bias is not None:
        bias = bias.to(torch.bfloat16)
        if bias.stride(-1) != 1:
            bias = bias.contiguous()
    at = bt = None
    if adapters is not None:
        at, bt = adapters.at, adapters.bt
    info = {"rows": rows, "K": K, "N": N, "rank": adapters.rank if adapters is not None else 0}
    if launch_observer is not None:
        launch_observer("grouped_gemm", "before", info)
    call("mlora_grouped_gemm",
         ptr(x), x.stride(0), rows, K, N,
         w_ptr, w_dtype, w_se, w_sk, w_sn,
         ptr(scale), scale_kind, scale_se, scale_on_k,
         *nf4,
         ptr(at), at.stride(0) if at is not None else 0, at.stride(1) if at is not None else 0,
         ptr(bt), bt.stride(0) if bt is not None else 0, bt.stride(1) if bt is not None else 0,
         R, float(scaling),
         ptr(bias), bias.stride(0) if bias is not None else 0,
         ptr(out), out.stride(0), ptr(low), low.stride(0) if low is not None else 0,
         ptr(offsets), offsets.numel(), _lib.stream(x.device))
    if launch_observer is not None:
        launch_observer("grouped_gemm", "after", info)
    return out, low


def grouped_linear(x: torch.Tensor, weight, offsets: torch.Tensor, is_transposed: bool,
                   block_m: int = BLOCK_M, products_fp8=None) -> torch.Tensor:
    """x (rows, in) by the stack (experts, out, in), or (experts, in, out) when is_transposed, per expert group.

    offsets (experts,) int32 on the device: the end of each expert's rows.  Returns (rows, out) in
    x's dtype.  A stack in fp8 is converted in registers without a scale: the caller folds the
    scale in.  The base product alone (src/meepsquared/_grouped.py:348-359); block_m is accepted
    for the reference's signature, the kernel's own tiling is fixed.
    """
    return _launch(x, weight, None, offsets, is_transposed, None, 1.0, None, False,
                   products_fp8=_x_fp8(weight, products_fp8))[0]


def fp8_products(device=None) -> bool:
    """Whether an fp8 stack's products run on the fp8 MFMA with the activations quantised to e4m3 when
    the caller does not say: MEEPSQUARED_FP8_PRODUCTS=1, as src/meepsquared/_grouped.py:70-80."""
    return os.environ.get("MEEPSQUARED_FP8_PRODUCTS") == "1"


def fp8_product_terms() -> int:
    """The e4m3 terms the fp8 products quantise the activations into: 2 (x ≈ hi + lo, within 2^-7 of each
    64-column block's amax: the layer stays within 3e-2 of float32), or 1 with MEEPSQUARED_FP8_TERMS=1 (the
    reference's single pass, src/meepsquared/_grouped.py:191-194: ~4-5 % error at config 1)."""
    return 1 if os.environ.get("MEEPSQUARED_FP8_TERMS") == "1" else 2


def _x_fp8(weight, products_fp8) -> bool:
    """The reference's X_FP8 (src/meepsquared/_grouped.py:320): only an fp8 stack, and then the switch."""
    w_fp8 = isinstance(weight, torch.Tensor) and weight.dtype == torch.float8_e4m3fn
    return w_fp8 and (fp8_products() if products_fp8 is None else bool(products_fp8))


def _k_contiguous(weight, w_se, w_sk, w_sn, K, N):
    """The fp8 stack addressed W[e][n][k] with k contiguous: the stack itself, or a transposed copy
    made by the library's byte transpose and kept on the stack tensor for as long as the tensor
    lives and is not modified in place (the stacks are frozen: made once, reused every step)."""
    if w_sk == 1:
        return weight, w_se, w_sn
    key = (tuple(weight.shape), tuple(weight.stride()), weight.data_ptr(), weight._version, K, N)
    held = getattr(weight, "_mlora_k_contiguous", None)
    if held is None or held[0] != key:
        E = weight.shape[0]
        t = torch.empty((E, N, K), device=weight.device, dtype=torch.uint8)
        call("mlora_transpose_u8", ptr(weight), E, K, N, w_se, w_sk, w_sn, ptr(t), _lib.stream(weight.device))
        held = (key, t)
        weight._mlora_k_contiguous = held
    t = held[1]
    return t, t.stride(0), t.stride(1)


def _launch_fp8(x, weight, scale, offsets, is_transposed, adapters, scaling, bias, store_low, backward):
    """The fp8 products: one fp8_prep pass over x (e4m3 terms, power-of-two scales per row and 64
    columns, and low = bf16(x · A_e)), then the fp8 grouped product on the block-scaled MFMA, one MFMA
    per term."""
    rows, K = x.shape
    if K % 16:
        raise ValueError(f"the fp8 products need in={K} to be a multiple of 16")
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    N, w_se, w_sk, w_sn = _stack_strides(weight, K, is_transposed)
    out = torch.empty((rows, N), device=x.device, dtype=x.dtype)
    R = adapters.padded if adapters is not None else 0
    low = torch.empty((rows, R), device=x.device, dtype=torch.bfloat16) if adapters is not None else None
    if rows == 0:
        return out, (low if store_low else None)
    offsets = offsets if offsets.dtype == torch.int32 else offsets.to(torch.int32)
    offsets = offsets.contiguous()
    _lib.require_gpu(weight)
    scale, scale_kind, scale_se, scale_on_k = _scale_args(scale, weight, backward, is_transposed)
    colscale, cs_se = None, 0
    if scale_kind == _lib.SCALE_ROW and scale_on_k:  # a per-row stack scale along k: folded into x
        colscale, cs_se, scale, scale_kind, scale_se = scale, scale_se, None, _lib.SCALE_NONE, 0
    w8, w_se, w_sn = _k_contiguous(weight, w_se, w_sk, w_sn, K, N)
    nkb = (K + 63) // 64
    terms = fp8_product_terms()
    x8 = torch.empty((rows, terms * nkb * 64), device=x.device, dtype=torch.uint8)
    xs = torch.empty((nkb, rows), device=x.device, dtype=torch.int32)
    E = offsets.numel()
    if bias is not None:
        bias = bias.to(torch.bfloat16)
        if bias.stride(-1) != 1:
            bias = bias.contiguous()
    at = adapters.at if adapters is not None else None
    bt = adapters.bt if adapters is not None else None
    info = {"rows": rows, "K": K, "N": N, "rank": adapters.rank if adapters is not None else 0, "fp8": True,
            "terms": terms}
    if launch_observer is not None:
        launch_observer("grouped_gemm", "before", info)
    stream = _lib.stream(x.device)
    call("mlora_fp8_prep", ptr(x), x.stride(0), rows, K, terms, ptr(colscale), cs_se, ptr(x8), x8.stride(0), ptr(xs),
         xs.stride(0), ptr(at), at.stride(0) if at is not None else 0, at.stride(1) if at is not None else 0, R,
         ptr(low), low.stride(0) if low is not None else 0, ptr(offsets), E, stream)
    call("mlora_fp8_gemm", ptr(x8), x8.stride(0), ptr(xs), xs.stride(0), rows, K, terms, N, ptr(w8), w_se, w_sn,
         ptr(scale), scale_kind, scale_se, ptr(low), low.stride(0) if low is not None else 0,
         ptr(bt), bt.stride(0) if bt is not None else 0, bt.stride(1) if bt is not None else 0, R, float(scaling),
         ptr(bias), bias.stride(0) if bias is not None else 0, ptr(out), out.stride(0), ptr(offsets), E, stream)
    if launch_observer is not None:
        launch_observer("grouped_gemm", "after", info)
    return out, (low if store_low else None)


def _reduce_out(experts: int, N: int, R: int, transposed: bool, device):
    """The (experts, N, R) bf16 gradient, or (experts, R, N) when transposed, and its (se, sn, sr) strides."""
    if transposed:
        out = torch.empty((experts, R, N), device=device, dtype=torch.bfloat16)
        return out, (out.stride(0), out.stride(2), out.stride(1))
    out = torch.empty((experts, N, R), device=device, dtype=torch.bfloat16)
    return out, (out.stride(0), out.stride(1), out.stride(2))


def _reduce(g: torch.Tensor, low: torch.Tensor, offsets: torch.Tensor, scaling: float,
            transposed: bool = False, gather=None, row_scale=None) -> torch.Tensor:
    """(experts, N, R) bf16: scaling · sum over each expert's rows of g^T @ low (_grouped.py:362-370);
    (experts, R, N), written in that layout by the kernel, when transposed.  gather = (perm, k): the
    rows are g[perm // k] (g then has its own row count).  row_scale = (w, index): row r's term
    weighted by w[index[r]] (applied to low's row, rounded to bf16)."""
    experts = offsets.numel()
    N = g.shape[1]
    rows = low.shape[0] if gather is not None else g.shape[0]
    R = low.shape[1]
    if g.stride(1) != 1 or g.stride(0) % 8 or g.data_ptr() % 16:
        g = g.contiguous()
    if transposed:
        out = torch.empty((experts, R, N), device=g.device, dtype=torch.bfloat16)
        o_se, o_sn, o_sr = out.stride(0), out.stride(2), out.stride(1)
    else:
        out = torch.empty((experts, N, R), device=g.device, dtype=torch.bfloat16)
        o_se, o_sn, o_sr = out.stride(0), out.stride(1), out.stride(2)
    if rows == 0:  # a sum over no rows (an empty gather or scale index has no device pointer to pass)
        return out.zero_()
    info = {"rows": rows, "N": N, "R": R, "gathered": gather is not None, "scaled": row_scale is not None}
    ws = torch.empty(int(_lib.lib.mlora_grouped_reduce_workspace_bytes(rows, N, R, experts)), device=g.device,
                     dtype=torch.uint8)
    if launch_observer is not None:
        launch_observer("grouped_reduce", "before", info)
    if gather is None and row_scale is None:
        call("mlora_grouped_reduce", ptr(g), g.stride(0), ptr(low), low.stride(0), rows, N, R, float(scaling),
             ptr(offsets), experts, ptr(out), o_se, o_sn, o_sr, ptr(ws) if ws.numel() else None, ws.numel(),
             _lib.stream(g.device))
    else:
        perm, k = gather if gather is not None else (None, 1)
        w, index = row_scale if row_scale is not None else (None, None)
        call("mlora_grouped_reduce_gather", ptr(g), g.stride(0), ptr(perm), k, ptr(w),
             _lib.dtype_code(w.dtype) if w is not None else 0, ptr(index), ptr(low), low.stride(0), rows, N, R,
             float(scaling), ptr(offsets), experts, ptr(out), o_se, o_sn, o_sr, ptr(ws) if ws.numel() else None,
             ws.numel(), _lib.stream(g.device))
    if launch_observer is not None:
        launch_observer("grouped_reduce", "after", info)
    return out


class _LoraGroupedProduct(torch.autograd.Function):
    """The experts' product with the adapters; gradients for x and the adapters, none for the frozen stack."""

    @staticmethod
    def forward(ctx, x, weight, scale, offsets, is_transposed, lhs, rhs, scaling, bias, products_fp8):
        x_fp8 = _x_fp8(weight, products_fp8)
        offsets = offsets.to(torch.int32).contiguous()
        adapters = _Adapters(lhs, rhs, is_transposed) if lhs is not None else None
        out, low = _launch(x, weight, scale, offsets, is_transposed, adapters, scaling, bias, True, products_fp8=x_fp8)
        ctx.x_fp8 = x_fp8
        ctx.save_for_backward(x, offsets, *((low,) if low is not None else ()))
        ctx.weight = weight  # frozen: held as it is (an NF4 stack is not a tensor)
        ctx.adapters, ctx.scale, ctx.is_transposed, ctx.scaling = adapters, scale, is_transposed, scaling
        ctx.lhs_dtype = lhs.dtype if lhs is not None else None
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, offsets, *rest = ctx.saved_tensors
        adapters, weight = ctx.adapters, ctx.weight
        grad_out = grad_out.to(torch.bfloat16).contiguous()
        if adapters is None:
            grad_x, _ = _launch(grad_out, weight, ctx.scale, offsets, not ctx.is_transposed, None, 1.0, None, False,
                                backward=True, products_fp8=ctx.x_fp8)
            return grad_x, None, None, None, None, None, None, None, None, None
        low = rest[0]
        # grad_x = grad @ W (the stack read the other way) + scaling · bf16(grad @ B^T) @ A^T, with B's
        # gradient formed in the same pass where the kernel can (it reads grad's rows already)
        if _db_fits(weight, adapters, offsets, ctx.x_fp8):
            grad_x, low2, grad_b = _launch_db(grad_out, weight, ctx.scale, offsets, not ctx.is_transposed,
                                              adapters.swapped(), ctx.scaling, low, ctx.is_transposed)
        else:
            grad_x, low2 = _launch(grad_out, weight, ctx.scale, offsets, not ctx.is_transposed, adapters.swapped(),
                                   ctx.scaling, None, True, backward=True, products_fp8=ctx.x_fp8)
            grad_b = _reduce(grad_out, low, offsets, ctx.scaling, transposed=ctx.is_transposed)
        # A's gradient (k, r) and B's (n, r), each written by the kernel in the layout of the factor it
        # belongs to, so no copy follows
        rank = adapters.rank
        if ctx.is_transposed:  # A = lhs (in, rank), B = rhs (rank, out)
            grad_lhs = _reduce(x, low2, offsets, ctx.scaling)[:, :, :rank]
            grad_rhs = grad_b[:, :rank, :]
        else:  # A = rhs^T, B = lhs^T
            grad_rhs = _reduce(x, low2, offsets, ctx.scaling, transposed=True)[:, :rank, :]
            grad_lhs = grad_b[:, :, :rank]
        if ctx.lhs_dtype is not None and ctx.lhs_dtype != torch.bfloat16:
            grad_lhs, grad_rhs = grad_lhs.to(ctx.lhs_dtype), grad_rhs.to(ctx.lhs_dtype)
        return grad_x, None, None, None, None, grad_lhs, grad_rhs, None, None, None


def gathered_product_fits(weight, products_fp8=None) -> bool:
    """Whether the product can read its rows gathered from the layer's input: a bf16 or fp8 e4m3 stack tensor
    (bf16 products) or an NF4 stack, with rows the DMA-fed product takes (16-byte chunks; NF4: 64-code blocks)."""
    if isinstance(weight, Nf4Stack):
        return weight.shape[1] % 64 == 0 and weight.shape[2] % 64 == 0
    if not isinstance(weight, torch.Tensor) or _x_fp8(weight, products_fp8):
        return False
    if weight.dtype == torch.bfloat16:
        return True
    return (weight.dtype == torch.float8_e4m3fn and weight.is_contiguous() and weight.shape[1] % 16 == 0
            and weight.shape[2] % 16 == 0 and weight.data_ptr() % 16 == 0)


def swiglu_fusable(N, rank=0, row_scale=None, backward=False) -> bool:
    """Whether the gathered product of a gate_up stack (N = 2 I columns) forms SwiGLU in its epilogue
    (mlora_grouped_gemm_gather_swiglu): a forward product without row scale, N a multiple of 256, adapters
    padded to rank 16 or none, unless MEEPSQUARED_FUSED_SWIGLU=0 asks for the separate SwiGLU pass.  On MI355X
    the fused epilogue costs less than the pass it replaces (Qwen3-shaped layer: +30 us to the gate_up product
    against a 46 us pass, the step +0.4 %; Mixtral-shaped: +1 %)."""
    return (os.environ.get("MEEPSQUARED_FUSED_SWIGLU", "1") != "0" and not backward and row_scale is None
            and N % 256 == 0 and N > 0 and rank in (0, 16))


def _launch_gathered(src, perm, k, weight, scale, offsets, is_transposed, adapters, scaling, bias,
                     row_scale=None, backward=False, swiglu=False):
    """One launch of the product over the rows src[perm // k]: (out, low).  row_scale: output row r multiplied
    by row_scale[perm[r]] (low stays bf16 of the unscaled rows' x·A).  A bf16, fp8 (bf16 products) or NF4
    stack, as gathered_product_fits admits.  swiglu (swiglu_fusable must hold): (out, low, act), act = SwiGLU
    of out formed in the same launch, the values mlora_swiglu(out) gives."""
    _lib.require_gpu(src, perm, offsets)
    if not gathered_product_fits(weight, False):
        raise TypeError(f"the gathered product takes a bf16, fp8 e4m3 or NF4 stack with rows of whole 16-byte chunks, "
                        f"not {getattr(weight, 'dtype', type(weight))}: use lora_linear")
    src = src if src.stride(-1) == 1 and src.stride(0) % 8 == 0 and src.data_ptr() % 16 == 0 else src.contiguous()
    T, K = src.shape
    rows = perm.numel()
    N = _stack_strides(weight, K, is_transposed)[0]
    out = torch.empty((rows, N), device=src.device, dtype=torch.bfloat16)
    R = adapters.padded if adapters is not None else 0
    low = torch.empty((rows, R), device=src.device, dtype=torch.bfloat16) if adapters is not None else None
    if swiglu and not swiglu_fusable(N, R, row_scale, backward):
        raise ValueError(f"the gathered product forms SwiGLU for a forward product of N % 256 == 0 columns and "
                         f"adapters of rank 16 or none, not N={N}, rank {R}")
    act = torch.empty((rows, N // 2), device=src.device, dtype=torch.bfloat16) if swiglu else None
    if rows == 0:
        return (out, low, act) if swiglu else (out, low)
    if (isinstance(weight, torch.Tensor) and weight.dtype == torch.bfloat16
            and _scale_args(scale, weight, backward, is_transposed)[3]):
        # a per-row scale along k is applied by the fp8 decode only
        raise ValueError("the gathered product takes no per-output-row scale of a bf16 stack in the input-gradient "
                         "pass: use lora_linear")
    w_ptr, w_dtype, w_se, w_sk, w_sn, nf4, (scale_, scale_kind, scale_se, on_k) = _stack_operand(
        weight, K, N, is_transposed, scale, backward)
    if bias is not None:
        bias = bias.to(torch.bfloat16)
        bias = bias if bias.stride(-1) == 1 else bias.contiguous()
    at, bt = (adapters.at, adapters.bt) if adapters is not None else (None, None)
    info = {"rows": rows, "K": K, "N": N, "rank": adapters.rank if adapters is not None else 0}
    if launch_observer is not None:
        launch_observer("grouped_gemm", "before", info)
    if swiglu:
        call("mlora_grouped_gemm_gather_swiglu", ptr(src), src.stride(0), T, ptr(perm), k, rows, K, N,
             w_ptr, w_dtype, w_se, w_sk, w_sn, ptr(scale_), scale_kind, scale_se, *nf4,
             ptr(at), at.stride(0) if at is not None else 0, at.stride(1) if at is not None else 0,
             ptr(bt), bt.stride(0) if bt is not None else 0, bt.stride(1) if bt is not None else 0,
             R, float(scaling), ptr(bias), bias.stride(0) if bias is not None else 0,
             ptr(out), out.stride(0), ptr(low), low.stride(0) if low is not None else 0, ptr(act), act.stride(0),
             ptr(offsets), offsets.numel(), _lib.stream(src.device))
        if launch_observer is not None:
            launch_observer("grouped_gemm", "after", info)
        return out, low, act
    call("mlora_grouped_gemm_gather_q", ptr(src), src.stride(0), T, ptr(perm), k, ptr(row_scale),
         _lib.dtype_code(row_scale.dtype) if row_scale is not None else 0, rows, K, N,
         w_ptr, w_dtype, w_se, w_sk, w_sn, ptr(scale_), scale_kind, scale_se, on_k, *nf4,
         ptr(at), at.stride(0) if at is not None else 0, at.stride(1) if at is not None else 0,
         ptr(bt), bt.stride(0) if bt is not None else 0, bt.stride(1) if bt is not None else 0,
         R, float(scaling), ptr(bias), bias.stride(0) if bias is not None else 0,
         ptr(out), out.stride(0), ptr(low), low.stride(0) if low is not None else 0,
         ptr(offsets), offsets.numel(), _lib.stream(src.device))
    if launch_observer is not None:
        launch_observer("grouped_gemm", "after", info)
    return out, low


def _db_fits(weight, adapters, offsets, products_fp8=False) -> bool:
    """Whether the input-gradient product forms B's gradient itself (mlora_grouped_gemm_db): asked for with
    MEEPSQUARED_FUSED_DB=1, and a bf16 stack tensor, adapters of rank <= 16, at most 256 experts, bf16
    products.  Off by default: on MI355X at the Qwen3-shaped layer the fused pass costs the two input-gradient
    launches 0.10-0.14 ms per step, about what the standalone reductions it replaces take (0.12 ms)."""
    return (os.environ.get("MEEPSQUARED_FUSED_DB", "0") == "1" and adapters is not None and adapters.padded == 16
            and isinstance(weight, torch.Tensor) and weight.dtype == torch.bfloat16 and not products_fp8
            and offsets.numel() <= 256)


def _launch_db(src, weight, scale, offsets, is_transposed, adapters, scaling, l, transposed_out, gather=None,
               row_scale=None, db_weight=None):
    """The input-gradient product of _launch / _launch_gathered (backward, low stored), with B's gradient
    scaling · sum over each expert's rows of x[row]^T l'[row] formed in the same pass, x the product's input
    rows (src, or src[perm // k] with gather=(perm, k)): the reduction _reduce(x, l, ...) would make
    (src/meepsquared/_grouped.py:398-399), without reading x again.  row_scale: the product's output row
    scale (as _launch_gathered's); db_weight=(w, index): l's row r weighted by w[index[r]] (rounded to bf16,
    as _reduce weights it).  Returns (out, low, grad): grad (experts, K, 16), or (experts, 16, K) when
    transposed_out, K = x's columns."""
    _lib.require_gpu(src, offsets, weight, l)
    src = src if src.stride(-1) == 1 and src.stride(0) % 8 == 0 and src.data_ptr() % 16 == 0 else src.contiguous()
    l = l if l.stride(-1) == 1 and l.stride(0) % 8 == 0 and l.data_ptr() % 16 == 0 else l.contiguous()
    xrows, K = src.shape
    perm, k = gather if gather is not None else (None, 1)
    rows = perm.numel() if gather is not None else xrows
    E = offsets.numel()
    N, w_se, w_sk, w_sn = _stack_strides(weight, K, is_transposed)
    out = torch.empty((rows, N), device=src.device, dtype=torch.bfloat16)
    R = adapters.padded
    low = torch.empty((rows, R), device=src.device, dtype=torch.bfloat16)
    if transposed_out:
        grad = torch.empty((E, R, K), device=src.device, dtype=torch.bfloat16)
        o_se, o_sk, o_sr = grad.stride(0), grad.stride(2), grad.stride(1)
    else:
        grad = torch.empty((E, K, R), device=src.device, dtype=torch.bfloat16)
        o_se, o_sk, o_sr = grad.stride(0), grad.stride(1), grad.stride(2)
    if rows == 0:
        return out, low, grad.zero_()
    scale_, scale_kind, scale_se, on_k = _scale_args(scale, weight, True, is_transposed)
    if on_k:
        raise ValueError("the fused adapter gradient takes no per-output-row stack scale in the input-gradient pass")
    if db_weight is not None:  # l's rows weighted once, bf16(w[index[r]] · l[r]), as _reduce weights them
        w, index = db_weight
        w = w.reshape(-1)
        lw = torch.empty_like(l)
        call("mlora_scale_rows", ptr(l), l.stride(0), l.shape[0], l.shape[1], ptr(w), _lib.dtype_code(w.dtype), ptr(index),
             ptr(lw), lw.stride(0), _lib.stream(l.device))
        l = lw
    ws = torch.empty(int(_lib.lib.mlora_grouped_gemm_db_workspace_bytes(rows, K, E)), device=src.device,
                     dtype=torch.uint8)
    info = {"rows": rows, "K": K, "N": N, "rank": adapters.rank, "db_rank": R}
    if launch_observer is not None:
        launch_observer("grouped_gemm", "before", info)
    call("mlora_grouped_gemm_db", ptr(src), src.stride(0), xrows, ptr(perm), k, ptr(row_scale),
         _lib.dtype_code(row_scale.dtype) if row_scale is not None else 0, rows, K, N,
         ptr(weight), w_se, w_sk, w_sn, ptr(scale_), scale_kind, scale_se,
         ptr(adapters.at), adapters.at.stride(0), adapters.at.stride(1),
         ptr(adapters.bt), adapters.bt.stride(0), adapters.bt.stride(1),
         R, float(scaling), None, 0, ptr(out), out.stride(0), ptr(low), low.stride(0),
         ptr(l), l.stride(0),
         ptr(grad), o_se, o_sk, o_sr, ptr(ws), ws.numel(),
         ptr(offsets), E, _lib.stream(src.device))
    if launch_observer is not None:
        launch_observer("grouped_gemm", "after", info)
    return out, low, grad


class GateUpLink:
    """What the layer's two Functions share.  Forward: with want_act, the gate_up product forms SwiGLU in its
    epilogue and leaves act here, and the down Function takes it when its input is that very gu, unchanged
    (else it runs SwiGLU itself).  Backward, so that the SwiGLU backward also forms the gate_up adapter's B
    gradient (mlora_swiglu_backward_reduce): the gate_up product's forward leaves its low rows and scaling
    here, the down Function's backward leaves that gradient and the dgu it was formed from, and the gate_up
    backward takes it when its incoming gradient is that very dgu (else it reduces as usual).  The gate_up
    forward also leaves its adapters here; the down forward pairs its own with them, so the first backward
    swaps both projections' adapters in one launch (mlora_swap_adapters_two)."""

    __slots__ = ("low", "scaling", "transposed", "padded", "grad_b", "dgu", "dgu_version", "want_act", "act",
                 "act_of", "act_version", "adapters")

    def __init__(self, want_act=False):
        self.low = self.grad_b = self.dgu = self.act = self.act_of = self.adapters = None
        self.scaling, self.transposed, self.padded, self.dgu_version, self.act_version = 1.0, False, 0, -1, -1
        self.want_act = want_act

    def take_act(self, gu):
        """SwiGLU of gu formed by the gate_up product, or None."""
        act, of = self.act, self.act_of
        self.act = self.act_of = None
        if act is None or gu is not of or gu._version != self.act_version:
            return None
        return act

    def take(self, grad_out):
        """The B gradient formed for grad_out, or None."""
        grad_b, dgu = self.grad_b, self.dgu
        self.grad_b = self.dgu = None
        if grad_b is None or grad_out is not dgu or grad_out._version != self.dgu_version:
            return None
        return grad_b


class _GatheredLoraProduct(torch.autograd.Function):
    """lora_linear of x = hidden[perm // k] without materialising x: the product and A's gradient read
    the rows of hidden through perm (the fusion of src/meepsquared/_moe.py:80 into the gate_up product).
    Gradients for hidden (each token's k rows summed) and the adapters."""

    @staticmethod
    def forward(ctx, hidden, perm, inv, k, weight, scale, offsets, is_transposed, lhs, rhs, scaling, bias, link=None):
        _lib.require_gpu(hidden, perm, offsets, weight)
        hidden = hidden if hidden.stride(-1) == 1 and hidden.stride(0) % 8 == 0 and hidden.data_ptr() % 16 == 0 \
            else hidden.contiguous()
        offsets = offsets.to(torch.int32).contiguous()
        adapters = _Adapters(lhs, rhs, is_transposed) if lhs is not None else None
        N = _stack_strides(weight, hidden.shape[1], is_transposed)[0]
        if link is not None and link.want_act and swiglu_fusable(N, adapters.padded if adapters is not None else 0):
            out, low, act = _launch_gathered(hidden, perm, k, weight, scale, offsets, is_transposed, adapters, scaling,
                                             bias, swiglu=True)
            link.act, link.act_of, link.act_version = act, out, out._version
        else:
            out, low = _launch_gathered(hidden, perm, k, weight, scale, offsets, is_transposed, adapters, scaling,
                                        bias)
        ctx.save_for_backward(hidden, perm, inv, offsets, *((low,) if low is not None else ()))
        ctx.link = link
        if link is not None and adapters is not None:
            link.low, link.scaling, link.transposed, link.padded = low, scaling, is_transposed, adapters.padded
            link.adapters = adapters
        ctx.weight, ctx.adapters, ctx.scale = weight, adapters, scale
        ctx.is_transposed, ctx.scaling, ctx.k = is_transposed, scaling, k
        ctx.lhs_dtype = lhs.dtype if lhs is not None else None
        return out

    @staticmethod
    def backward(ctx, grad_out):
        hidden, perm, inv, offsets, *rest = ctx.saved_tensors
        adapters, weight, k = ctx.adapters, ctx.weight, ctx.k
        grad_out = grad_out.to(torch.bfloat16).contiguous()
        T, K = hidden.shape
        grad_lhs = grad_rhs = None
        if adapters is None:
            grad_sel, _ = _launch(grad_out, weight, ctx.scale, offsets, not ctx.is_transposed, None, 1.0, None, False,
                                  backward=True)
        else:
            low = rest[0]
            grad_b = ctx.link.take(grad_out) if ctx.link is not None else None  # formed by the SwiGLU backward
            if grad_b is None and _db_fits(weight, adapters, offsets):
                grad_sel, low2, grad_b = _launch_db(grad_out, weight, ctx.scale, offsets, not ctx.is_transposed,
                                                    adapters.swapped(), ctx.scaling, low, ctx.is_transposed)
            else:
                grad_sel, low2 = _launch(grad_out, weight, ctx.scale, offsets, not ctx.is_transposed,
                                         adapters.swapped(), ctx.scaling, None, True, backward=True)
                if grad_b is None:
                    grad_b = _reduce(grad_out, low, offsets, ctx.scaling, transposed=ctx.is_transposed)
            rank = adapters.rank
            gather = (perm, k)
            if ctx.is_transposed:
                grad_lhs = _reduce(hidden, low2, offsets, ctx.scaling, gather=gather)[:, :, :rank]
                grad_rhs = grad_b[:, :rank, :]
            else:
                grad_rhs = _reduce(hidden, low2, offsets, ctx.scaling, transposed=True, gather=gather)[:, :rank, :]
                grad_lhs = grad_b[:, :, :rank]
            if ctx.lhs_dtype is not None and ctx.lhs_dtype != torch.bfloat16:
                grad_lhs, grad_rhs = grad_lhs.to(ctx.lhs_dtype), grad_rhs.to(ctx.lhs_dtype)
        dh = torch.empty((T, K), device=grad_out.device, dtype=torch.bfloat16)
        call("mlora_gather_rows_backward", ptr(grad_sel), K, ptr(inv), T, k, ptr(offsets), offsets.numel(),
             ptr(dh), _lib.stream(grad_out.device))
        return dh, None, None, None, None, None, None, None, grad_lhs, grad_rhs, None, None, None


class _CombinedLoraProduct(torch.autograd.Function):
    """combine(lora_linear(x, ...), weights): the down product and the weighted sum of each token's k
    rows (src/meepsquared/_moe.py:88-126, the last product and :123-126).  The backward never writes
    the weighted gradient rows bf16(w · dout[t]): the input-gradient product reads dout through perm and
    multiplies each output row by its weight in the epilogue, and the adapters' reductions weight
    each row's term as they load it.  Gradients for x, the weights and the adapters."""

    @staticmethod
    def forward(ctx, x, weights, perm, inv, k, weight, scale, offsets, is_transposed, lhs, rhs, scaling, bias):
        offsets = offsets.to(torch.int32).contiguous()
        adapters = _Adapters(lhs, rhs, is_transposed) if lhs is not None else None
        y, low = _launch(x, weight, scale, offsets, is_transposed, adapters, scaling, bias, True)
        S, H = y.shape
        T = inv.numel() // k
        w = weights.reshape(-1).contiguous()
        if w.dtype not in (torch.bfloat16, torch.float32):
            w = w.float()
        out = torch.empty((T, H), device=y.device, dtype=y.dtype)
        call("mlora_combine", ptr(y), H, ptr(w), _lib.dtype_code(w.dtype), ptr(inv), T, k, ptr(offsets),
             offsets.numel(), ptr(out), _lib.stream(y.device))
        ctx.save_for_backward(x, y, w, perm, inv, offsets, *((low,) if low is not None else ()))
        ctx.weight, ctx.adapters, ctx.scale = weight, adapters, scale
        ctx.is_transposed, ctx.scaling, ctx.k = is_transposed, scaling, k
        ctx.lhs_dtype = lhs.dtype if lhs is not None else None
        ctx.wshape, ctx.wdtype = weights.shape, weights.dtype
        return out

    @staticmethod
    def backward(ctx, dout):
        x, y, w, perm, inv, offsets, *rest = ctx.saved_tensors
        adapters, weight, k = ctx.adapters, ctx.weight, ctx.k
        dout = dout.to(torch.bfloat16).contiguous()
        T, H = dout.shape
        dw = torch.empty_like(w)
        call("mlora_combine_backward", ptr(dout), ptr(y), H, ptr(w), _lib.dtype_code(w.dtype), ptr(inv), T, k,
             ptr(offsets), offsets.numel(), None, ptr(dw), _lib.stream(dout.device))
        grad_lhs = grad_rhs = None
        if adapters is None:
            grad_x, _ = _launch_gathered(dout, perm, k, weight, ctx.scale, offsets, not ctx.is_transposed, None, 1.0,
                                         None, row_scale=w, backward=True)
        else:
            low = rest[0]
            ws = (w, perm)  # row r's weight: w[perm[r]]
            if _db_fits(weight, adapters, offsets):
                grad_x, low2, grad_b = _launch_db(dout, weight, ctx.scale, offsets, not ctx.is_transposed,
                                                  adapters.swapped(), ctx.scaling, low, ctx.is_transposed,
                                                  gather=(perm, k), row_scale=w, db_weight=ws)
            else:
                grad_x, low2 = _launch_gathered(dout, perm, k, weight, ctx.scale, offsets, not ctx.is_transposed,
                                                adapters.swapped(), ctx.scaling, None, row_scale=w, backward=True)
                grad_b = _reduce(dout, low, offsets, ctx.scaling, transposed=ctx.is_transposed, gather=(perm, k),
                                 row_scale=ws)
            rank = adapters.rank
            if ctx.is_transposed:  # A = lhs (in, rank), B = rhs (rank, out)
                grad_lhs = _reduce(x, low2, offsets, ctx.scaling, row_scale=ws)[:, :, :rank]
                grad_rhs = grad_b[:, :rank, :]
            else:  # A = rhs^T, B = lhs^T
                grad_rhs = _reduce(x, low2, offsets, ctx.scaling, transposed=True, row_scale=ws)[:, :rank, :]
                grad_lhs = grad_b[:, :, :rank]
            if ctx.lhs_dtype is not None and ctx.lhs_dtype != torch.bfloat16:
                grad_lhs, grad_rhs = grad_lhs.to(ctx.lhs_dtype), grad_rhs.to(ctx.lhs_dtype)
        dw = dw.view(ctx.wshape)
        if dw.dtype != ctx.wdtype:
            dw = dw.to(ctx.wdtype)
        return grad_x, dw, None, None, None, None, None, None, None, grad_lhs, grad_rhs, None, None


class _SwigluCombinedLoraProduct(torch.autograd.Function):
    """combine(lora_linear(swiglu(gu), ...), weights) for a down stack without bias
    (TF:integrations/moe.py:509-520, then src/meepsquared/_moe.py:88-126 for the last product and
    :123-126).  The backward runs the input-gradient product on dout read through perm WITHOUT the
    combine weights (g), and one SwiGLU-backward pass applies each row's weight and forms the weights'
    gradient <dout[t], y[p]> as <g[p], act[p]>: y is neither kept nor read again.  Gradients for gu,
    the weights and the adapters."""

    @staticmethod
    def forward(ctx, gu, weights, perm, inv, k, weight, scale, offsets, is_transposed, lhs, rhs, scaling, link=None):
        offsets = offsets.to(torch.int32).contiguous()
        act = link.take_act(gu) if link is not None else None  # (formed by the gate_up product)
        gu = gu.contiguous()
        S, I2 = gu.shape
        if act is None:
            act = torch.empty((S, I2 // 2), device=gu.device, dtype=gu.dtype)
            call("mlora_swiglu", ptr(gu), S, I2 // 2, ptr(act), _lib.stream(gu.device))
        adapters = _Adapters(lhs, rhs, is_transposed) if lhs is not None else None
        if adapters is not None and link is not None and link.adapters is not None:
            adapters.partner, link.adapters = link.adapters, None  # swapped together in the first backward
        y, low = _launch(act, weight, scale, offsets, is_transposed, adapters, scaling, None, True)
        H = y.shape[1]
        T = inv.numel() // k
        w = weights.reshape(-1).contiguous()
        if w.dtype not in (torch.bfloat16, torch.float32):
            w = w.float()
        out = torch.empty((T, H), device=y.device, dtype=y.dtype)
        call("mlora_combine", ptr(y), H, ptr(w), _lib.dtype_code(w.dtype), ptr(inv), T, k, ptr(offsets),
             offsets.numel(), ptr(out), _lib.stream(y.device))
        ctx.save_for_backward(gu, act, w, perm, offsets, *((low,) if low is not None else ()))
        ctx.weight, ctx.adapters, ctx.scale = weight, adapters, scale
        ctx.is_transposed, ctx.scaling, ctx.k = is_transposed, scaling, k
        ctx.lhs_dtype = lhs.dtype if lhs is not None else None
        ctx.wshape, ctx.wdtype = weights.shape, weights.dtype
        ctx.link = link
        return out

    @staticmethod
    def backward(ctx, dout):
        gu, act, w, perm, offsets, *rest = ctx.saved_tensors
        adapters, weight, k = ctx.adapters, ctx.weight, ctx.k
        dout = dout.to(torch.bfloat16).contiguous()
        grad_lhs = grad_rhs = None
        grad_b = None
        ws = (w, perm)  # row r's weight: w[perm[r]]
        if adapters is None:
            g, _ = _launch_gathered(dout, perm, k, weight, ctx.scale, offsets, not ctx.is_transposed, None, 1.0, None,
                                    backward=True)
        elif _db_fits(weight, adapters, offsets):
            g, low2, grad_b = _launch_db(dout, weight, ctx.scale, offsets, not ctx.is_transposed, adapters.swapped(),
                                         ctx.scaling, rest[0], ctx.is_transposed, gather=(perm, k), db_weight=ws)
        else:
            g, low2 = _launch_gathered(dout, perm, k, weight, ctx.scale, offsets, not ctx.is_transposed,
                                       adapters.swapped(), ctx.scaling, None, backward=True)
        S, I = g.shape
        dgu = torch.empty_like(gu)
        dw = torch.empty_like(w)
        link = ctx.link
        grad_a = None  # A's gradient of the down adapter, (E, I, R) or (E, R, I) as _reduce lays it out
        if (adapters is not None and adapters.padded == 16 and link is not None and link.low is not None
                and link.padded == 16 and S > 0):
            # the SwiGLU backward with A's gradient of the down adapter and B's of the gate_up adapter
            E = offsets.numel()
            low2_ = low2 if low2.stride(1) == 1 else low2.contiguous()
            lowgu = link.low
            grad_a, a_strides = _reduce_out(E, I, 16, not ctx.is_transposed, gu.device)
            grad_bgu, b_strides = _reduce_out(E, 2 * I, 16, link.transposed, gu.device)
            ws_ = torch.empty(int(_lib.lib.mlora_swiglu_backward_reduce_workspace_bytes(S, I, E)), device=gu.device,
                              dtype=torch.uint8)
            call("mlora_swiglu_backward_reduce", ptr(gu), ptr(g), S, I, ptr(w), _lib.dtype_code(w.dtype), ptr(perm),
                 ptr(offsets), E, ptr(low2_), low2_.stride(0), float(ctx.scaling), ptr(grad_a), *a_strides,
                 ptr(lowgu), lowgu.stride(0), float(link.scaling), ptr(grad_bgu), *b_strides, ptr(dgu), ptr(dw),
                 ptr(ws_), ws_.numel(), _lib.stream(gu.device))
            link.grad_b, link.dgu, link.dgu_version = grad_bgu, dgu, dgu._version
        else:
            call("mlora_swiglu_backward_weighted", ptr(gu), ptr(g), S, I, ptr(w), _lib.dtype_code(w.dtype),
                 ptr(perm), ptr(offsets), offsets.numel(), ptr(dgu), ptr(dw), _lib.stream(gu.device))
        if adapters is not None:
            low = rest[0]
            rank = adapters.rank
            if grad_b is None:
                grad_b = _reduce(dout, low, offsets, ctx.scaling, transposed=ctx.is_transposed, gather=(perm, k),
                                 row_scale=ws)
            if grad_a is None:
                grad_a = _reduce(act, low2, offsets, ctx.scaling, transposed=not ctx.is_transposed, row_scale=ws)
            if ctx.is_transposed:  # A = lhs (in, rank), B = rhs (rank, out)
                grad_lhs = grad_a[:, :, :rank]
                grad_rhs = grad_b[:, :rank, :]
            else:  # A = rhs^T, B = lhs^T
                grad_rhs = grad_a[:, :rank, :]
                grad_lhs = grad_b[:, :, :rank]
            if ctx.lhs_dtype is not None and ctx.lhs_dtype != torch.bfloat16:
                grad_lhs, grad_rhs = grad_lhs.to(ctx.lhs_dtype), grad_rhs.to(ctx.lhs_dtype)
        dw = dw.view(ctx.wshape)
        if dw.dtype != ctx.wdtype:
            dw = dw.to(ctx.wdtype)
        return dgu, dw, None, None, None, None, None, None, None, grad_lhs, grad_rhs, None, None


def swiglu_lora_linear_combined(gu, weights, perm, inv, k, weight, scale, offsets, is_transposed, lhs=None, rhs=None,
                                scaling: float = 1.0, link: GateUpLink = None):
    """combine(lora_linear(swiglu(gu), ...), weights) of the layer's down product (a stack gathered_product_fits
    admits, no bias).  link: shared with the lora_linear_gathered call that produced gu, so that the SwiGLU
    backward forms that product's B gradient too."""
    return _SwigluCombinedLoraProduct.apply(gu, weights, perm, inv, k, weight, scale, offsets, is_transposed, lhs,
                                            rhs, scaling, link)


def lora_linear_combined(x, weights, perm, inv, k, weight, scale, offsets, is_transposed, lhs=None, rhs=None,
                         scaling: float = 1.0, bias=None):
    """combine(lora_linear(x, ...), weights) of the layer's down product (stacks gathered_product_fits admits), its backward
    reading the output gradient through perm instead of a weighted copy of it."""
    return _CombinedLoraProduct.apply(x, weights, perm, inv, k, weight, scale, offsets, is_transposed, lhs, rhs,
                                      scaling, bias)


def lora_linear_gathered(hidden, perm, inv, k, weight, scale, offsets, is_transposed, lhs=None, rhs=None,
                         scaling: float = 1.0, bias=None, link: GateUpLink = None):
    """lora_linear(hidden[perm // k], ...) with the gathered rows never materialised (bf16, fp8 or NF4 stacks,
    as gathered_product_fits admits).  link: see swiglu_lora_linear_combined."""
    return _GatheredLoraProduct.apply(hidden, perm, inv, k, weight, scale, offsets, is_transposed, lhs, rhs, scaling,
                                      bias, link)


def lora_linear(x, weight, scale, offsets, is_transposed: bool, lhs=None, rhs=None, scaling: float = 1.0, bias=None,
                products_fp8=None):
    """The experts' product of x with the stack, the adapters (PEFT's lhs, rhs, scaling) and the bias stack (experts, out).

    scale is the fp8 stack's scale: (experts,) as the reference holds it, or (experts, out), one per
    output row; None for a bf16 or NF4 stack.  Same signature and gradients as
    src/meepsquared/_grouped.py:408-417.
    """
    return _LoraGroupedProduct.apply(x, weight, scale, offsets, is_transposed, lhs, rhs, scaling, bias, products_fp8)
