"""Layer oracle: the routed MoE-LoRA layer composed as the reference composes it (PyTorch fp32).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Also the CPU baseline that bench.py times.
"""

import numpy as np
import torch

from oracle import grouped, routing


def swiglu(gate_up):
    """silu(gate) * up, gate the first half — TF:integrations/moe.py:509-520.
    Pinned by: a brute-force elementwise loop (tests/test_oracle.py)."""
    gate, up = gate_up.chunk(2, dim=-1)
    return torch.nn.functional.silu(gate) * up


def routed_forward(hidden, top_k_index, top_k_weights, gate_up, down, factors, num_experts, is_transposed=False,
                   scales=None, dtype=torch.float32, biases=None):
    """The layer forward — src/meepsquared/_moe.py:70-126 with reference_lora per projection.

    factors: {"gate_up_proj": (lhs, rhs, s), "down_proj": (lhs, rhs, s)}; scales: the same names to
    fp8 scales (or absent).  Computed in `dtype` (float32 by default), differentiable in hidden,
    top_k_weights and the factors.  Sentinel ids (>= num_experts) contribute nothing.  biases: the
    same names to (experts, out) bias stacks (or absent), added per expert as the reference's
    lora_linear adds `bias` (src/meepsquared/_grouped.py:408-417).
    Pinned by: a per-token brute-force loop over its k experts (tests/test_oracle.py).
    """
    scales = scales or {}
    biases = biases or {}
    T, k = top_k_index.shape
    ids = top_k_index.reshape(-1)
    perm, _, offsets = routing.sort_by_expert(ids.cpu().numpy(), num_experts)
    perm_t = torch.as_tensor(perm, device=hidden.device)
    valid = int(offsets[-1])
    rows = perm_t[:valid]
    selected = hidden.to(dtype)[rows // k]

    def project(x, name, weight):
        lhs, rhs, s = factors.get(name, (None, None, 1.0))
        return grouped.reference_lora(x, weight, scales.get(name), offsets, is_transposed, lhs, rhs, s,
                                      biases.get(name), out_dtype=dtype)

    act = swiglu(project(selected, "gate_up_proj", gate_up))
    out = project(act, "down_proj", down)
    w = top_k_weights.reshape(-1)[rows].to(dtype)
    weighted = out * w.unsqueeze(-1)
    result = torch.zeros((T * k, hidden.shape[1]), device=hidden.device, dtype=dtype)
    result = result.index_copy(0, rows, weighted)
    return result.view(T, k, -1).sum(dim=1)


def routed_forward_loop(hidden, top_k_index, top_k_weights, gate_up, down, factors, num_experts, is_transposed=False):
    """The same layer, one token and one of its experts at a time (float64): the brute force that pins routed_forward."""
    T, k = top_k_index.shape
    out = torch.zeros((T, hidden.shape[1]), dtype=torch.float64)
    for t in range(T):
        for j in range(k):
            e = int(top_k_index[t, j])
            if e >= num_experts:
                continue
            x = hidden[t].double()

            def w_of(name, W):
                w = W[e].double()
                w = w if is_transposed else w.t()  # (in, out)
                lhs, rhs, s = factors.get(name, (None, None, 1.0))
                if lhs is not None:
                    d = lhs[e].double() @ rhs[e].double()
                    w = w + s * (d if is_transposed else d.t())
                return w

            gu = x @ w_of("gate_up_proj", gate_up)
            I = gu.shape[0] // 2
            a = gu[:I] * torch.sigmoid(gu[:I]) * gu[I:]
            out[t] += float(top_k_weights[t, j]) * (a @ w_of("down_proj", down))
    return out
