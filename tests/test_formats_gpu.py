"""Stack conversion kernels against the oracle: fp8 bytes and scales bit-exact (torch's own e4m3
cast is the oracle's), NF4 decode bit-exact and its encode equal to the oracle's nearest-code rule."""

import numpy as np
import pytest
import torch

from oracle import formats

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("is_transposed", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fp8_quantisation_is_bit_exact(per_row, is_transposed, dtype):
    from meepsquared_amd import _fp8

    torch.manual_seed(0)
    w = (torch.randn(5, 48, 80) * torch.rand(5, 48, 1) * 3).to(dtype)
    q, scale = _fp8.quantize_stack(w.cuda(), per_row=per_row, is_transposed=is_transposed)
    oq, oscale = formats.fp8_quantize(w, per_row, is_transposed)
    assert torch.equal(scale.cpu(), oscale)
    assert torch.equal(q.cpu().view(torch.uint8), oq.view(torch.uint8))
    back = _fp8.dequantize_stack(q, scale, torch.float32, is_transposed)
    assert torch.equal(back.cpu(), formats.fp8_dequantize(oq, oscale, is_transposed))


def test_every_e4m3_byte_decodes_as_torch_does():
    from meepsquared_amd import _fp8

    codes = torch.arange(256, dtype=torch.uint8)
    codes = codes[(codes & 0x7F) != 0x7F]  # no NaNs
    q = codes.view(torch.float8_e4m3fn).view(1, 1, -1).cuda()
    back = _fp8.dequantize_stack(q, torch.ones(1, device="cuda"), torch.float32)
    assert torch.equal(back.cpu().view(-1), q.cpu().float().view(-1))


def test_nf4_codec_matches_the_oracle():
    from meepsquared_amd import _nf4

    torch.manual_seed(0)
    w = torch.randn(3, 64, 256) * 0.02
    stack = _nf4.quantize_stack(w.cuda())
    code, code2 = np.array(_nf4.NF4_CODE, np.float32), np.array(_nf4.dynamic_code(), np.float32)
    packed, q, a2, off = formats.nf4_quantize(w.numpy(), code, code2)
    assert abs(stack.offset.item() - off) <= 1e-7 * abs(off)
    np.testing.assert_allclose(stack.absmax2.cpu().numpy(), a2, rtol=1e-6)
    assert (stack.absmax_q.cpu().numpy() == q).mean() > 0.999
    assert np.array_equal(stack.packed.cpu().numpy(), packed)
    # decoding the kernel's own bytes: bit-exact with the oracle's decode
    dec = _nf4.dequantize_stack(stack, torch.float32).cpu().numpy().reshape(-1)
    odec = formats.nf4_dequantize(stack.packed.cpu().numpy(), stack.absmax_q.cpu().numpy(), stack.absmax2.cpu().numpy(),
                                  stack.offset.item(), code, code2)
    assert np.array_equal(dec, odec)
