"""Writes the golden fixtures of tests/golden/ from PyTorch's own operators (a library, not this
build and not the reference), seeded, on the CPU:

  routing.npz  fp32 router logits without ties; torch.topk's indices and the renormalised softmax
               weights; torch.sort(stable=True)'s permutation and torch.bincount's offsets of the
               selected experts, with sentinel ids mixed in.
  lora.npz     a small grouped LoRA product and its gradients in float64, computed from the merged
               weights W_e + s·lhs_e@rhs_e of the whole stack with one batched torch.einsum
               (a different formulation from the oracle's per-expert loop).

    python tests/golden/make_golden.py
"""

from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def routing():
    g = torch.Generator().manual_seed(1234)
    T, E, k = 257, 40, 6
    logits = torch.randn(T, E, generator=g, dtype=torch.float32)
    probs = torch.softmax(logits, dim=-1)
    w, idx = torch.topk(probs, k, dim=-1)
    w = w / w.sum(dim=-1, keepdim=True)
    ids = idx.reshape(-1).clone()
    sentinel = torch.rand(ids.numel(), generator=g) < 0.05
    ids[sentinel] = E  # expert parallelism's sentinel id
    key = ids.clamp(max=E)
    _, perm = torch.sort(key, stable=True)
    counts = torch.bincount(key, minlength=E + 1)[:E]
    offsets = torch.cumsum(counts, 0).to(torch.int32)
    np.savez(HERE / "routing.npz", logits=logits.numpy(), k=k, topk_idx=idx.numpy(), topk_w=w.numpy(),
             ids=ids.numpy(), perm=perm.numpy(), offsets=offsets.numpy(), num_experts=E)


def lora():
    g = torch.Generator().manual_seed(99)
    rows_per_expert = [5, 0, 9, 3]
    E, K, N, r, s = len(rows_per_expert), 16, 12, 3, 1.5
    rows = sum(rows_per_expert)
    x = torch.randn(rows, K, generator=g, dtype=torch.float64, requires_grad=True)
    W = torch.randn(E, N, K, generator=g, dtype=torch.float64) * 0.1
    lhs = (torch.randn(E, N, r, generator=g, dtype=torch.float64) * 0.3).requires_grad_()
    rhs = (torch.randn(E, r, K, generator=g, dtype=torch.float64) * 0.3).requires_grad_()
    bias = torch.randn(E, N, generator=g, dtype=torch.float64)
    expert_of_row = torch.repeat_interleave(torch.arange(E), torch.tensor(rows_per_expert))
    merged = W + s * torch.einsum("enr,erk->enk", lhs, rhs)
    out = torch.einsum("mk,mnk->mn", x, merged[expert_of_row]) + bias[expert_of_row]
    grad = torch.randn(rows, N, generator=g, dtype=torch.float64)
    out.backward(grad)
    np.savez(HERE / "lora.npz", rows_per_expert=np.array(rows_per_expert), scaling=s, x=x.detach().numpy(),
             W=W.numpy(), lhs=lhs.detach().numpy(), rhs=rhs.detach().numpy(), bias=bias.numpy(),
             out=out.detach().numpy(), grad=grad.numpy(), grad_x=x.grad.numpy(), grad_lhs=lhs.grad.numpy(),
             grad_rhs=rhs.grad.numpy())


if __name__ == "__main__":
    routing()
    lora()
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))
