"""Writes tests/golden/topk_gpu.npz: torch.topk on the GPU (a library, not this build and not the
reference) over fp32 softmax probabilities of seeded bf16 router logits with many exact ties, as the
reference's router computes them on its GPU (TF:models/qwen3_moe/modeling_qwen3_moe.py:262-266:
softmax(logits, fp32) -> topk -> renormalise).  torch.topk's order of equal probabilities on the GPU
differs from its CPU order; this fixture records the GPU one.

    python tests/golden/make_golden_gpu.py OUT.npz     # on a machine with a GPU

Per case c (shapes in `cases`): logits_c (T, E) as bf16 bit patterns (uint16), idx_c (T, k) int16,
vals_c (T, k) fp32 (torch's top-k probabilities), w_c (T, k) fp32 (renormalised over the k).
"""

import sys

import numpy as np
import torch

# (T, E, k, seed, q): logits N(0,1), rounded to multiples of 1/q when q (more ties), then bf16
CASES = [
    (512, 128, 8, 0, 0.0),    # config 1's router: bf16 logits, natural ties
    (512, 128, 8, 1, 4.0),    # ties inside the k and at its boundary in most rows
    (2048, 8, 2, 2, 0.0),     # Mixtral's router
    (512, 64, 6, 3, 2.0),
    (256, 40, 32, 4, 1.0),    # k = 32: the largest k torch sorts with its bitonic network
    (64, 1000, 17, 5, 2.0),
    (128, 64, 40, 6, 1.0),    # k > 32: a stable sort
    (256, 16, 1, 7, 1.0),     # k = 1
]


def main(out):
    torch.manual_seed(0)
    arrays = {"cases": np.array(CASES, dtype=np.float64)}
    for c, (T, E, k, seed, q) in enumerate(CASES):
        g = torch.Generator().manual_seed(int(seed))
        logits = torch.randn(int(T), int(E), generator=g)
        if q:
            logits = (logits * q).round() / q
        logits = logits.to(torch.bfloat16)
        probs = torch.softmax(logits.cuda().float(), dim=-1)
        vals, idx = torch.topk(probs, int(k), dim=-1)
        w = vals / vals.sum(dim=-1, keepdim=True)
        arrays[f"logits_{c}"] = logits.view(torch.int16).numpy().view(np.uint16)
        arrays[f"idx_{c}"] = idx.cpu().numpy().astype(np.int16)
        arrays[f"vals_{c}"] = vals.cpu().numpy()
        arrays[f"w_{c}"] = w.cpu().numpy()
    np.savez_compressed(out, **arrays)
    print("wrote", out, "with", len(CASES), "cases")


if __name__ == "__main__":
    main(sys.argv[1])
