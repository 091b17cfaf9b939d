"""Stack-format oracle: fp8 e4m3 (per expert or per output row) and NF4 with double quantisation.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""

import numpy as np
import torch

E4M3_MAX = 448.0


def fp8_quantize(w, per_row=False, is_transposed=False):
    """(q e4m3 tensor, scale fp32) — src/meepsquared/_fp8.py:122-128, scale = max(amax, 1e-12) / 448.

    per_row: one scale per output row (dim 1 of (E, out, in), dim 2 of (E, in, out)).
    Pinned by: torch's float8_e4m3fn cast (a library) and the round-trip bound of
    tests/test_fp8.py:122-131 (error <= 0.07 · amax of the group).
    """
    w = torch.as_tensor(w).float()
    if per_row:
        amax = w.abs().amax(dim=1 if is_transposed else 2)
        scale = torch.clamp(amax, min=1e-12) / E4M3_MAX
        s = scale.unsqueeze(1) if is_transposed else scale.unsqueeze(2)
    else:
        amax = w.abs().flatten(1).amax(dim=1)
        scale = torch.clamp(amax, min=1e-12) / E4M3_MAX
        s = scale.view(-1, 1, 1)
    return (w / s).to(torch.float8_e4m3fn), scale


def fp8_dequantize(q, scale, is_transposed=False):
    """q · scale in fp32 — src/meepsquared/_fp8.py:131-134 (per-row: broadcast along the row)."""
    q = q.float()
    if scale.dim() == 1:
        return q * scale.view(-1, 1, 1)
    return q * (scale.unsqueeze(1) if is_transposed else scale.unsqueeze(2))


def fp8_rows_quantize(x, block=64, colscale=None):
    """Activations for the fp8 products: per row and per `block` columns, the power of two 2^e with
    amax·2^-e <= 448 (e the smallest such integer; e = 0 for an all-zero block) and the values
    e4m3(x·2^-e) rounded to nearest even.  Returns (q uint8 (rows, K padded to block), e8m0 int32
    (blocks, rows) = 127 + e).  colscale (K,) multiplies the columns first.

    The reference quantises per row and per BLOCK_K tile with scale amax/448
    (src/meepsquared/_grouped.py:191-194); this is that rule with the scale rounded up to a power of
    two, the form the block-scaled fp8 MFMA applies.
    Pinned by: torch's float8_e4m3fn cast (a library) for the values and, for the exponent, the
    brute-force definition min{e : amax·2^-e <= 448} (tests/test_oracle.py).
    """
    x = torch.as_tensor(x).float()
    if colscale is not None:
        x = x * torch.as_tensor(colscale).float()
    rows, K = x.shape
    kp = -(-K // block) * block
    xp = torch.zeros(rows, kp)
    xp[:, :K] = x
    xb = xp.view(rows, kp // block, block)
    amax = xb.abs().amax(dim=2)
    e = torch.zeros_like(amax, dtype=torch.int64)
    nz = amax > 0
    # smallest integer e with amax * 2^-e <= 448: ceil(log2(amax / 448)), exact in float64
    e[nz] = torch.ceil(torch.log2(amax[nz].double() / E4M3_MAX)).to(torch.int64)
    # guard the float64 log2 at exact powers of two
    over = nz & (amax.double() * torch.pow(2.0, -e.double()) > E4M3_MAX)
    e[over] += 1
    q = (xb * torch.pow(2.0, -e.float()).unsqueeze(2)).to(torch.float8_e4m3fn).view(rows, kp)
    return q.view(torch.uint8), (127 + e).to(torch.int32).t().contiguous()


def fp8_rows_dequantize(q, e8m0, K):
    """q · 2^(e8m0 - 127) per row and block, the first K columns (float32)."""
    rows, kp = q.shape
    block = kp // e8m0.shape[0]
    v = q.view(torch.float8_e4m3fn).float().view(rows, kp // block, block)
    v = v * torch.pow(2.0, (e8m0.t().float() - 127)).unsqueeze(2)
    return v.view(rows, kp)[:, :K]


def fp8_rows_quantize2(x, block=64, colscale=None):
    """Two-term activations for the fp8 products: x ≈ hi·2^e1 + lo·2^e2 per row and `block` columns, hi
    the one-term quantisation (fp8_rows_quantize) and lo the same rule applied to the residual
    x - hi·2^e1, which is exact in fp32.  Returns (q uint8 (rows, 2 · K padded), per block b the hi bytes
    at [2b·block, (2b+1)·block) and the lo bytes after them; words int32 (blocks, rows) = (127 + e1) |
    (127 + e2) << 8).  No reference counterpart: the reference's fp8 products keep one term
    (src/meepsquared/_grouped.py:191-194, 4.1 % error by design/grouped-lora-kernel.md:3).
    Pinned by: hi is fp8_rows_quantize's result; lo is fp8_rows_quantize of the residual computed in
    float64 (which equals the fp32 one); the reconstruction is within 2^-7 of each block's amax
    (tests/test_oracle.py).
    """
    x = torch.as_tensor(x).float()
    if colscale is not None:
        x = x * torch.as_tensor(colscale).float()
    rows, K = x.shape
    hi, e1 = fp8_rows_quantize(x, block)
    kp = hi.shape[1]
    xp = torch.zeros(rows, kp)
    xp[:, :K] = x
    residual = xp - fp8_rows_dequantize(hi, e1, kp)
    lo, e2 = fp8_rows_quantize(residual, block)
    nb = kp // block
    q = torch.stack([hi.view(rows, nb, block), lo.view(rows, nb, block)], dim=2).reshape(rows, 2 * kp)
    return q, e1 | (e2 << 8)


def fp8_rows_dequantize2(q, words, K):
    """hi·2^e1 + lo·2^e2 per row and block (fp8_rows_quantize2's layout), the first K columns (float32)."""
    rows, kp2 = q.shape
    nb = words.shape[0]
    block = kp2 // (2 * nb)
    qq = q.view(rows, nb, 2, block)
    hi = fp8_rows_dequantize(qq[:, :, 0].reshape(rows, nb * block).contiguous(), words & 0xFF, nb * block)
    lo = fp8_rows_dequantize(qq[:, :, 1].reshape(rows, nb * block).contiguous(), (words >> 8) & 0xFF, nb * block)
    return (hi + lo)[:, :K]


def fp8_tensor_quantize(w):
    """(q e4m3, scale 0-d fp32): one scale for the whole tensor — src/meepsquared/_fp8.py:95-109 (its CPU
    branch, :106-108), scale = max(amax, 1e-12) / 448.
    Pinned by: fp8_quantize over one expert (the same rule, pinned by torch's e4m3 cast), and the
    round-trip bound of tests/test_fp8.py:122-131 (tests/test_oracle.py)."""
    w = torch.as_tensor(w).float()
    scale = torch.clamp(w.abs().amax(), min=1e-12) / E4M3_MAX
    return (w / scale).to(torch.float8_e4m3fn), scale


def fp8_scaled_mm(x, weight8, weight_scale, transpose_weight, bias=None):
    """x @ W^T (transpose_weight) or x @ W with W = weight8 · weight_scale, in float32 — the reference's
    own CPU path of scaled_mm (src/meepsquared/_fp8.py:205-207), without its final bf16 cast; bias added.
    Pinned by: a diagonal weight (x times the diagonal, a closed form) and the transpose identity
    (x @ W^T)^T = W @ x^T (tests/test_oracle.py)."""
    w = torch.as_tensor(weight8).float() * torch.as_tensor(weight_scale).float()
    y = torch.as_tensor(x).float() @ (w.t() if transpose_weight else w)
    return y if bias is None else y + torch.as_tensor(bias).float()


def nf4_code_from_definition():
    """The 16 NF4 values from QLoRA's definition (Dettmers et al. 2023, Appendix E): 8 positive
    quantiles of N(0,1) from the upper half (offset 0.9677 = 1/2 (1/(2·15) + 1/(2·16)) mapped to
    the tail), 7 negative ones, an exact zero, normalised by the largest magnitude."""
    from scipy.stats import norm

    offset = 0.9677083
    pos = norm.ppf(np.linspace(offset, 0.5, 9)[:-1]).tolist()
    neg = (-norm.ppf(np.linspace(offset, 0.5, 8)[:-1])).tolist()
    v = np.array(sorted(pos + [0.0] + neg))
    return v / np.abs(v).max()


def nearest_index(values, code):
    """Index of the nearest code entry, ties to the lower index (numpy argmin's first minimum)."""
    values = np.asarray(values, dtype=np.float32)[..., None]
    d = np.abs(values - np.asarray(code, dtype=np.float32))
    return d.argmin(axis=-1)


def nf4_quantize(x, code, code2, blocksize=64, blocksize2=256):
    """(packed uint8, absmax_q uint8, absmax2 fp32, offset fp32) of the flat values x.

    The double-quant NF4 format of src/meepsquared/_vendor/axolotl/quantize.py:202-235's fields
    (absmax per block, its 8-bit code with a second absmax and an offset): codes relative to each
    block's exact absmax; the first value of a pair in the high nibble.
    Pinned by: round-trip error bounds and code-boundary checks (tests/test_oracle.py); the
    reference has no NF4 stack, so this format's bytes are this build's own.
    """
    x = np.asarray(x, dtype=np.float32).reshape(-1)
    blocks = x.reshape(-1, blocksize)
    absmax = np.abs(blocks).max(axis=1)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = np.where(absmax > 0, np.float32(1.0) / absmax, np.float32(0.0)).astype(np.float32)
    idx = nearest_index(blocks * inv[:, None], code).astype(np.uint8).reshape(-1)
    packed = (idx[0::2] << 4) | idx[1::2]
    offset = np.float32(absmax.astype(np.float64).mean())
    centred = (absmax - offset).astype(np.float32)
    pad = -centred.size % blocksize2
    groups = np.concatenate([centred, np.zeros(pad, np.float32)]).reshape(-1, blocksize2)
    absmax2 = np.abs(groups).max(axis=1).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = np.where(absmax2[:, None] > 0, groups / absmax2[:, None], 0).astype(np.float32)
    absmax_q = nearest_index(ratio, code2).astype(np.uint8).reshape(-1)[: centred.size]
    return packed.astype(np.uint8), absmax_q, absmax2, offset


def nf4_dequantize(packed, absmax_q, absmax2, offset, code, code2, blocksize=64, blocksize2=256):
    """code[nibble] · (code2[absmax_q[b]] · absmax2[b / 256] + offset), fp32."""
    packed = np.asarray(packed, dtype=np.uint8)
    nib = np.stack([packed >> 4, packed & 0xF], axis=1).reshape(-1)
    b = np.arange(nib.size) // blocksize
    code, code2 = np.asarray(code, np.float32), np.asarray(code2, np.float32)
    absmax = (code2[np.asarray(absmax_q)[b]] * np.asarray(absmax2, np.float32)[b // blocksize2] + np.float32(offset)).astype(np.float32)
    return (code[nib] * absmax).astype(np.float32)
