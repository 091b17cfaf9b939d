"""Shared helpers of the GPU tests."""

import torch


def rel(a, b):
    """Relative Frobenius error of a against b, in float64."""
    a, b = a.detach().double(), b.detach().double()
    return ((a - b).norm() / b.norm().clamp(min=1e-30)).item()


def offsets_of(rows_per_expert, device="cuda"):
    return torch.cumsum(torch.tensor(rows_per_expert, dtype=torch.int32, device=device), 0, dtype=torch.int32)


def kaiming_uniform(shape, fan_in, gen=None, device="cpu"):
    """PEFT's lora_A init (kaiming_uniform with a=sqrt(5)): U(-1/sqrt(fan_in), 1/sqrt(fan_in))."""
    bound = 1.0 / fan_in ** 0.5
    return (torch.rand(shape, generator=gen, device=device) * 2 - 1) * bound
