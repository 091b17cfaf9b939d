"""The dense SwiGLU MLP with LoRA on gate, up and down (meepsquared_amd._dense; the reference's fused
LoRA_MLP, src/meepsquared/_vendor/axolotl/lora.py:398-880) against the oracle's float32 composition:
output, X's gradient and the six factors' gradients; bf16 weights within 1e-2, fp8 weights (one scale per
tensor, against the dequantised weights) within 3e-2."""

import pytest
import torch

from helpers import kaiming_uniform, rel
from oracle import grouped as ref

pytestmark = pytest.mark.gpu


def make(H, I, r, seed, fp8=False, bias=False, scales=(2.0, 2.0, 2.0)):
    from meepsquared_amd import _fp8

    g = torch.Generator().manual_seed(seed)
    dev = "cuda"

    def w(o, i):
        t = (torch.randn(o, i, generator=g) * 0.02).to(dev, torch.bfloat16)
        return _fp8.quantize(t) if fp8 else t

    def f(o, i):  # PEFT: A kaiming-uniform (r, in), B (out, r)
        return (kaiming_uniform((r, i), i, g).to(dev, torch.bfloat16).requires_grad_(),
                (torch.randn(o, r, generator=g) * 0.01).to(dev, torch.bfloat16).requires_grad_())

    p = {"gate": (w(I, H), *f(I, H), scales[0]), "up": (w(I, H), *f(I, H), scales[1]),
         "down": (w(H, I), *f(H, I), scales[2])}
    b = [(torch.randn(n, generator=g) * 0.1).to(dev, torch.bfloat16) if bias else None for n in (I, I, H)]
    return p, b


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("bias,scales", [(False, (2.0, 2.0, 2.0)), (True, (2.0, 1.0, 0.5))])
def test_lora_mlp_matches_the_oracle(fp8, bias, scales):
    from meepsquared_amd._dense import lora_mlp_swiglu

    H, I, r = 512, 1024, 16
    p, b = make(H, I, r, seed=3, fp8=fp8, bias=bias, scales=scales)
    x = torch.randn(3, 70, H, generator=torch.Generator().manual_seed(4)).to("cuda", torch.bfloat16).requires_grad_()
    out = lora_mlp_swiglu(x, *p["gate"], *p["up"], *p["down"], *b)
    dy = torch.randn(out.shape, generator=torch.Generator().manual_seed(5)).to("cuda", torch.bfloat16)
    out.backward(dy)
    got = {"out": out.detach(), "dx": x.grad}
    for n, (_, a, bb, _) in p.items():
        got[n + ".A"], got[n + ".B"] = a.grad, bb.grad

    def deq(w):
        return w[0].float() * w[1] if isinstance(w, tuple) else w.float()

    x32 = x.detach().float().reshape(-1, H).requires_grad_()
    p32 = {n: (deq(w), a.detach().float().requires_grad_(), bb.detach().float().requires_grad_(), s)
           for n, (w, a, bb, s) in p.items()}
    o32 = ref.lora_mlp_swiglu(x32, p32["gate"], p32["up"], p32["down"], [None if t is None else t.float() for t in b])
    o32.backward(dy.float().reshape(-1, H))
    want = {"out": o32.detach(), "dx": x32.grad}
    for n, (_, a, bb, _) in p32.items():
        want[n + ".A"], want[n + ".B"] = a.grad, bb.grad
    tol = 3e-2 if fp8 else 1e-2
    for name in want:
        a, b_ = got[name].reshape(want[name].shape), want[name]
        assert rel(a, b_) < tol, (name, rel(a, b_))


def test_apply_lora_mlp_swiglu_on_a_module_and_its_refusals():
    from meepsquared_amd import _dense

    H, I, r = 256, 512, 8
    mlp = torch.nn.Module()
    mlp.gate_proj, mlp.up_proj, mlp.down_proj = (torch.nn.Linear(H, I, bias=False), torch.nn.Linear(H, I, bias=False),
                                                 torch.nn.Linear(I, H, bias=False))
    mlp = mlp.to("cuda", torch.bfloat16).requires_grad_(False)
    for proj in (mlp.gate_proj, mlp.up_proj, mlp.down_proj):
        proj.lora_A = torch.nn.Parameter(torch.randn(r, proj.in_features, device="cuda", dtype=torch.bfloat16) * 0.05)
        proj.lora_B = torch.nn.Parameter(torch.randn(proj.out_features, r, device="cuda", dtype=torch.bfloat16) * 0.05)
        proj.lora_scaling = 2.0
    x = torch.randn(40, H, device="cuda", dtype=torch.bfloat16)
    out = _dense.apply_lora_mlp_swiglu(mlp, x)
    params = {n: (p.weight, p.lora_A.detach().float(), p.lora_B.detach().float(), 2.0)
              for n, p in (("gate", mlp.gate_proj), ("up", mlp.up_proj), ("down", mlp.down_proj))}
    want = ref.lora_mlp_swiglu(x.float(), params["gate"], params["up"], params["down"])
    assert rel(out, want) < 1e-2
    mlp.gate_proj.lora_dropout_p = 0.1
    with pytest.raises(NotImplementedError, match="dropout"):
        _dense.apply_lora_mlp_swiglu(mlp, x)
