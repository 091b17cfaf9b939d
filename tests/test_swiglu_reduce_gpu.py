"""mlora_swiglu_backward_reduce (the SwiGLU backward with A's gradient of the down adapter and B's gradient of
the gate_up adapter formed from the same registers) against the kernels it replaces, run one after the other:
mlora_swiglu_backward_weighted for dgu and the combine weights' gradient, mlora_grouped_reduce(_gather) for
the two adapter gradients (src/meepsquared/_grouped.py:362-370).  dgu, dA and dB carry the same bits; dw is
the same fp32 sum taken in another order."""

import pytest
import torch

from helpers import rel

pytestmark = pytest.mark.gpu


def _case(S, I, E, sizes, w_dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    dev = "cuda"
    gu = torch.randn(S, 2 * I, device=dev, generator=g).bfloat16()
    gr = torch.randn(S, I, device=dev, generator=g).bfloat16()
    w = torch.rand(S, device=dev, generator=g).to(w_dtype)
    perm = torch.randperm(S, device=dev, generator=g)
    offsets = torch.tensor(sizes, dtype=torch.int64).cumsum(0).to(dev, torch.int32)
    low2 = torch.randn(S, 16, device=dev, generator=g).bfloat16()
    lowgu = torch.randn(S, 16, device=dev, generator=g).bfloat16()
    return gu, gr, w, perm, offsets, low2, lowgu


def _separate(gu, gr, w, perm, offsets, low2, lowgu, s2, su, ta, tb):
    from meepsquared_amd import _grouped, _lib
    from meepsquared_amd._lib import call, ptr

    S, I = gr.shape
    st = _lib.stream()
    act = torch.empty(S, I, device="cuda", dtype=torch.bfloat16)
    call("mlora_swiglu", ptr(gu), S, I, ptr(act), st)
    dgu = torch.empty_like(gu)
    dw = torch.empty_like(w)
    call("mlora_swiglu_backward_weighted", ptr(gu), ptr(gr), S, I, ptr(w), _lib.dtype_code(w.dtype), ptr(perm),
         ptr(offsets), offsets.numel(), ptr(dgu), ptr(dw), st)
    da = _grouped._reduce(act, low2, offsets, s2, transposed=ta, row_scale=(w, perm))
    db = _grouped._reduce(dgu, lowgu, offsets, su, transposed=tb)
    return dgu, dw, da, db


def _fused(gu, gr, w, perm, offsets, low2, lowgu, s2, su, ta, tb):
    from meepsquared_amd import _grouped, _lib
    from meepsquared_amd._lib import call, ptr

    S, I = gr.shape
    E = offsets.numel()
    dgu = torch.empty_like(gu)
    dw = torch.empty_like(w)
    da, a_st = _grouped._reduce_out(E, I, 16, ta, "cuda")
    db, b_st = _grouped._reduce_out(E, 2 * I, 16, tb, "cuda")
    ws = torch.empty(int(_lib.lib.mlora_swiglu_backward_reduce_workspace_bytes(S, I, E)), device="cuda",
                     dtype=torch.uint8)
    call("mlora_swiglu_backward_reduce", ptr(gu), ptr(gr), S, I, ptr(w), _lib.dtype_code(w.dtype), ptr(perm),
         ptr(offsets), E, ptr(low2), low2.stride(0), s2, ptr(da), *a_st, ptr(lowgu), lowgu.stride(0), su, ptr(db),
         *b_st, ptr(dgu), ptr(dw), ptr(ws), ws.numel(), _lib.stream())
    return dgu, dw, da, db


CASES = {
    # S, I, E, rows per expert (their sum short of S: the rest are sentinel rows)
    "small experts, an empty one, sentinels": (700, 128, 8, [90, 0, 130, 33, 200, 7, 120, 100]),
    "columns past a 64-column block": (520, 72, 4, [100, 160, 0, 250]),
    "config-1 shape": (8192, 768, 128, [64] * 128),
    "experts split over workgroups": (20480, 64, 4, [13030, 4000, 2000, 1450]),
    "one expert, eight columns, rows not a multiple of 32": (77, 8, 1, [70]),
    "every row a sentinel": (96, 128, 3, [0, 0, 0]),
}


@pytest.mark.parametrize("case", list(CASES))
@pytest.mark.parametrize("w_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("layouts", [(False, False), (True, True), (True, False)])
def test_the_fused_swiglu_backward_matches_the_kernels_it_replaces(case, w_dtype, layouts):
    S, I, E, sizes = CASES[case]
    print(f"case {case}: S={S} I={I} E={E} w={w_dtype} layouts={layouts}", flush=True)
    args = _case(S, I, E, sizes, w_dtype, seed=len(case))
    ta, tb = layouts
    want = _separate(*args, 0.5, 2.0, ta, tb)
    got = _fused(*args, 0.5, 2.0, ta, tb)
    torch.cuda.synchronize()
    assert torch.equal(got[0], want[0]), "dgu"
    assert torch.equal(got[2], want[2]), "dA"
    assert torch.equal(got[3], want[3]), "dB"
    valid = int(args[4][-1])
    sentinel = torch.zeros(S, dtype=torch.bool, device="cuda")
    sentinel[args[3][valid:]] = True
    assert torch.all(got[1][sentinel] == 0)
    tol = 1e-5 if w_dtype == torch.float32 else 8e-3
    assert rel(got[1].float(), want[1].float()) < tol, "dw"


def test_the_layer_takes_the_fused_swiglu_backward_and_matches_the_two_reductions(monkeypatch):
    """The routed layer with both adapters at rank 16: the gate_up backward takes the B gradient the SwiGLU
    backward formed (one grouped_reduce launch fewer per projection) and the down Function the SwiGLU the
    gate_up product formed (no SwiGLU pass, the default), with the same output and
    gradients as the layer run without the link between its two Functions."""
    from meepsquared_amd import Experts, _grouped, routed_forward, topk_softmax

    torch.manual_seed(5)
    T, H, I, E, k, r = 512, 256, 128, 16, 4, 16
    dev = "cuda"
    h = torch.randn(T, H, device=dev).bfloat16()
    logits = torch.randn(T, E, device=dev).bfloat16()
    gu = (torch.randn(E, 2 * I, H, device=dev) * 0.05).bfloat16()
    dn = (torch.randn(E, H, I, device=dev) * 0.05).bfloat16()
    f = {"gate_up_proj": ((torch.randn(E, 2 * I, r, device=dev) * 0.1).bfloat16(),
                          (torch.randn(E, r, H, device=dev) * 0.1).bfloat16(), 2.0),
         "down_proj": ((torch.randn(E, H, r, device=dev) * 0.1).bfloat16(),
                       (torch.randn(E, r, I, device=dev) * 0.1).bfloat16(), 2.0)}
    dy = torch.randn(T, H, device=dev).bfloat16()
    counts = {}
    monkeypatch.delenv("MEEPSQUARED_FUSED_SWIGLU", raising=False)

    def observe(kind, phase, info):
        if phase == "before":
            counts[kind] = counts.get(kind, 0) + 1

    real_call = _grouped.call

    def call(name, *args):  # counts the standalone SwiGLU launches
        if name == "mlora_swiglu":
            counts[name] = counts.get(name, 0) + 1
        return real_call(name, *args)

    monkeypatch.setattr(_grouped, "call", call)

    def run(linked):
        hh = h.clone().requires_grad_()
        ff = {n: (a.clone().requires_grad_(), b.clone().requires_grad_(), s) for n, (a, b, s) in f.items()}
        w, idx = topk_softmax(logits, k)
        w = w.detach().requires_grad_()
        if not linked:
            monkeypatch.setattr(_grouped, "GateUpLink", lambda **kw: None)
        counts.clear()
        monkeypatch.setattr(_grouped, "launch_observer", observe)
        out = routed_forward(Experts(gu, dn), hh, idx, w, ff)
        out.backward(dy)
        monkeypatch.setattr(_grouped, "launch_observer", None)
        grads = [hh.grad, w.grad] + [t.grad for (a, b, _) in ff.values() for t in (a, b)]
        return out.detach(), grads, dict(counts)

    got_out, got, got_counts = run(True)
    want_out, want, want_counts = run(False)
    assert torch.equal(got_out, want_out)
    for i, (a, b) in enumerate(zip(got, want)):
        assert rel(a.float(), b.float()) < 1e-2, i
    assert got_counts.get("grouped_reduce", 0) == want_counts.get("grouped_reduce", 0) - 2, (got_counts, want_counts)
    # and SwiGLU formed in the gate_up product's epilogue: the same bits (out above), no SwiGLU pass
    assert got_counts.get("mlora_swiglu", 0) == 0 and want_counts.get("mlora_swiglu", 0) == 1, (got_counts, want_counts)


def _bf16_ulp(v):
    """The spacing of bf16 values at |v| (the smallest normal's spacing below it)."""
    a = v.abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def test_swiglu_and_its_backward_are_within_one_bf16_step_of_the_exact_values():
    """mlora_swiglu and mlora_swiglu_backward against silu(g)·u and its derivatives taken in float64 from
    the same bf16 inputs, then rounded to bf16 once (TF integrations/moe.py:509-520): every value within
    one bf16 step of the exact one, nearly all of them equal to it; gates from 0 and ±tiny to ±1e4, where
    the sigmoid saturates or e^-g overflows."""
    from meepsquared_amd import _lib
    from meepsquared_amd._lib import call, ptr

    g = torch.Generator(device="cuda").manual_seed(11)
    S, I = 4096, 256
    gate = torch.randn(S, I, device="cuda", generator=g) * 4
    special = torch.tensor([0.0, -0.0, 1e-30, -1e-30, 1e-3, -1e-3, 15.0, -15.0, 88.0, -88.0, 90.0, -90.0,
                            1e4, -1e4, 3.0, -3.0], device="cuda")
    gate[:, :special.numel()] = special
    gu = torch.cat([gate, torch.randn(S, I, device="cuda", generator=g) * 2], 1).bfloat16()
    d = torch.randn(S, I, device="cuda", generator=g).bfloat16()
    st = _lib.stream()
    act = torch.empty(S, I, device="cuda", dtype=torch.bfloat16)
    call("mlora_swiglu", ptr(gu), S, I, ptr(act), st)
    dgu = torch.empty_like(gu)
    call("mlora_swiglu_backward", ptr(gu), ptr(d), S, I, ptr(dgu), st)
    torch.cuda.synchronize()

    g64, u64, d64 = gu[:, :I].double(), gu[:, I:].double(), d.double()
    sg = torch.sigmoid(g64)
    want = {"act": g64 * sg * u64, "d_gate": d64 * u64 * sg * (1 + g64 * (1 - sg)), "d_up": d64 * g64 * sg}
    got = {"act": act, "d_gate": dgu[:, :I], "d_up": dgu[:, I:]}
    for name, w in want.items():
        ours = got[name].double()
        exact = w.bfloat16().double()
        off = (ours - exact).abs()
        # below 2^-100 fp32's e^-g has overflowed (g < -88.7): 0, as with libm's expf
        assert bool(((off <= _bf16_ulp(exact)) | (w.abs() < 2.0 ** -100)).all()), (name, off.max().item())
        # the random columns: a rounding of the fp32 chain lands past a bf16 midpoint only rarely
        assert (off[:, special.numel():] != 0).double().mean().item() < 2e-3, name


@pytest.mark.parametrize("stack", ["bf16", "nf4"])
def test_the_layer_with_swiglu_in_the_product_is_bit_identical_to_the_separate_pass(stack, monkeypatch):
    """SwiGLU formed in the gate_up product's epilogue (the default) and the separate mlora_swiglu pass
    (MEEPSQUARED_FUSED_SWIGLU=0) give the routed layer the same output and the same gradients, bit for bit:
    act is formed from the same stored bf16 gate and up values either way."""
    from meepsquared_amd import Experts, _grouped, _nf4, routed_forward, topk_softmax

    torch.manual_seed(9)
    T, H, I, E, k, r = 640, 256, 256, 8, 2, 16
    dev = "cuda"
    h = torch.randn(T, H, device=dev).bfloat16()
    logits = torch.randn(T, E, device=dev).bfloat16()
    gu = (torch.randn(E, 2 * I, H, device=dev) * 0.05).bfloat16()
    dn = (torch.randn(E, H, I, device=dev) * 0.05).bfloat16()
    if stack == "nf4":
        gu, dn = _nf4.quantize_stack(gu.float()), _nf4.quantize_stack(dn.float())
    f = {"gate_up_proj": ((torch.randn(E, 2 * I, r, device=dev) * 0.1).bfloat16(),
                          (torch.randn(E, r, H, device=dev) * 0.1).bfloat16(), 2.0),
         "down_proj": ((torch.randn(E, H, r, device=dev) * 0.1).bfloat16(),
                       (torch.randn(E, r, I, device=dev) * 0.1).bfloat16(), 2.0)}
    dy = torch.randn(T, H, device=dev).bfloat16()
    names = []
    real_call = _grouped.call

    def call(name, *args):
        names.append(name)
        return real_call(name, *args)

    monkeypatch.setattr(_grouped, "call", call)

    def run(fused):
        monkeypatch.setenv("MEEPSQUARED_FUSED_SWIGLU", "1" if fused else "0")
        names.clear()
        hh = h.clone().requires_grad_()
        ff = {n: (a.clone().requires_grad_(), b.clone().requires_grad_(), s) for n, (a, b, s) in f.items()}
        w, idx = topk_softmax(logits, k)
        w = w.detach().requires_grad_()
        out = routed_forward(Experts(gu, dn), hh, idx, w, ff)
        out.backward(dy)
        return [out.detach(), hh.grad, w.grad] + [t.grad for (a, b, _) in ff.values() for t in (a, b)], list(names)

    got, got_names = run(True)
    want, want_names = run(False)
    assert "mlora_grouped_gemm_gather_swiglu" in got_names and "mlora_swiglu" not in got_names
    assert "mlora_swiglu" in want_names and "mlora_grouped_gemm_gather_swiglu" not in want_names
    for i, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), i
