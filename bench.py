"""MoE-LoRA layer forward + backward throughput on one MI355X: BASELINE config 1 (Qwen3-30B-A3B shaped).

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline]
    python bench.py --copy-calibration MIB    # a plain device copy of known size, for PMC scaling
    python bench.py --config 3                # config 3: fp8 e4m3 stacks with per-row scales (bf16 products)
    python bench.py --config 3 --fp8-products # ... with the products on the fp8 MFMA (two e4m3 terms)
    python bench.py --config 2|4              # Mixtral-shaped, Zipf-loaded / packed varlen batch, NF4 stacks

A step is one forward and backward pass of the routed MoE-LoRA layer over one batch of synthetic
inputs already resident in HBM: router top-k softmax (from given logits), counting sort, gather,
gate_up grouped product with its LoRA, SwiGLU, down grouped product with its LoRA, weighted
combine; then the backward: combine, down dX with dA/dB, SwiGLU, gate_up dX with dA/dB, gather.
Shapes: T=8192 tokens, hidden 2048, moe_intermediate 768, 128 experts, top-8 (renormalised),
LoRA r=16, alpha=32 on gate_up and down, bf16.  Data: x, logits ~ N(0,1), W ~ N(0,0.02),
A ~ Kaiming-uniform U(+-1/sqrt(in)), B ~ N(0,0.01), dY ~ N(0,1), seed 0.

Prints one JSON line: tokens/s (whole job), ms/step, the grouped-product kernel's achieved
TFLOP/s against the MI355X dense bf16 peak (HIP events around each of its launches over K more steps
run right after the timed ones, on the launch stream), and the CPU baseline: the oracle's float32 per-expert path
(the reference's algorithm) on a bounded sample of the same workload on this host's cores.
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

T, H, I, E, K_TOP, R, ALPHA = 8192, 2048, 768, 128, 8, 16, 32
PEAK_BF16_TFLOPS = 2500.0
PEAK_FP8_TFLOPS = 5000.0
PROFILE_TRAFFIC = ROOT / "profiles" / "grouped_gemm_qwen3_traffic.txt"


def step_flops(T, H, I, k, r):
    """Algorithmic FLOP of one fwd+bwd: base products forward and dX (W frozen), LoRA forward, dX, dA, dB."""
    S = T * k
    base = 2 * S * (2 * H * 2 * I + 2 * I * H)
    lora_fwd = 2 * S * (H * r + r * 2 * I + I * r + r * H)
    lora_dx = 2 * S * (2 * I * r + r * H + H * r + r * I)
    lora_da = 2 * S * (r * H + r * I)
    lora_db = 2 * S * (2 * I * r + H * r)
    return base + lora_fwd + lora_dx + lora_da + lora_db


def gemm_launch_flops(info):
    """Algorithmic FLOP of one grouped-product launch: x W plus the LoRA x A and low B."""
    rows, K, N, r = info["rows"], info["K"], info["N"], info["rank"]
    # an input-gradient launch that also forms B's gradient sums x^T l over its rows: K x db_rank more MACs per row
    return 2 * rows * (K * N + K * r + r * N + K * info.get("db_rank", 0))


# the BASELINE configurations this bench can run (1 is the headline; 2-4 are reported beside it)
CONFIGS = {
    1: dict(T=T, H=H, I=I, E=E, k=K_TOP, r=R, alpha=ALPHA,
            name="BASELINE config 1: Qwen3-30B-A3B-shaped MoE-LoRA layer fwd+bwd"),
    2: dict(T=16384, H=4096, I=14336, E=8, k=2, r=16, alpha=32, zipf=1.2,
            name="BASELINE config 2: Mixtral-8x7B-shaped MoE-LoRA layer fwd+bwd, Zipf(1.2)-loaded experts"),
    3: dict(T=T, H=H, I=I, E=E, k=K_TOP, r=R, alpha=ALPHA, stack="fp8",
            name="BASELINE config 3: config 1 with fp8-e4m3 stacks (per-row scales)"),
    4: dict(H=H, I=I, E=E, k=K_TOP, r=R, alpha=ALPHA, stack="nf4", varlen=(64, 64, 2048),
            name="BASELINE config 4: config 1 fed from a packed varlen batch (64 sequences, lengths U[64, 2048]), "
                 "NF4 stacks (blocksize 64, double quant)"),
}


def config_tokens(c, seed=0):
    """T of a configuration: fixed, or the total length of its packed varlen batch (seeded)."""
    if "varlen" not in c:
        return c["T"]
    import numpy as np

    n, lo, hi = c["varlen"]
    return int(np.random.default_rng(seed).integers(lo, hi + 1, size=n).sum())


def make_inputs(device, seed=0, c=None):
    import torch

    c = c or CONFIGS[1]
    T, H, I, E, R, ALPHA = config_tokens(c, seed), c["H"], c["I"], c["E"], c["r"], c["alpha"]
    g = torch.Generator(device=device).manual_seed(seed)

    def randn(*shape, std=1.0):
        return torch.randn(*shape, generator=g, device=device) * std

    def kaiming(*shape, fan_in):
        return (torch.rand(*shape, generator=g, device=device) * 2 - 1) / fan_in ** 0.5

    bf = torch.bfloat16
    hidden = randn(T, H).to(bf).requires_grad_()
    logits = randn(T, E)
    if "zipf" in c:  # router logits biased so that expert e's share of the load falls as (e + 1)^-s
        logits = logits + (-c["zipf"] * torch.log(torch.arange(1, E + 1, device=device, dtype=torch.float32)))
    logits = logits.to(bf)
    gate_up = randn(E, 2 * I, H, std=0.02).to(bf)
    down = randn(E, H, I, std=0.02).to(bf)
    s = ALPHA / R
    factors = {"gate_up_proj": (randn(E, 2 * I, R, std=0.01).to(bf).requires_grad_(),
                                kaiming(E, R, H, fan_in=H).to(bf).requires_grad_(), s),
               "down_proj": (randn(E, H, R, std=0.01).to(bf).requires_grad_(),
                             kaiming(E, R, I, fan_in=I).to(bf).requires_grad_(), s)}
    dy = randn(T, H).to(bf)
    return hidden, logits, gate_up, down, factors, dy


def cpu_baseline(tokens: int):
    """The oracle's float32 per-expert path (src/meepsquared/_grouped.py:431-444 composed as
    src/meepsquared/_moe.py:70-126), fwd + bwd by autograd, on `tokens` tokens of the config-1
    layer, timed on this host's cores after a small warm-up."""
    import torch

    from oracle import moe as ref_moe

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    gu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).bfloat16()
    dn = (torch.randn(E, H, I, generator=g) * 0.02).bfloat16()
    f = {"gate_up_proj": ((torch.randn(E, 2 * I, R, generator=g) * 0.01).requires_grad_(),
                          ((torch.rand(E, R, H, generator=g) * 2 - 1) / H ** 0.5).requires_grad_(), ALPHA / R),
         "down_proj": ((torch.randn(E, H, R, generator=g) * 0.01).requires_grad_(),
                       ((torch.rand(E, R, I, generator=g) * 2 - 1) / I ** 0.5).requires_grad_(), ALPHA / R)}

    def run(t):
        h = torch.randn(t, H, generator=g).bfloat16().float().requires_grad_()
        probs = torch.softmax(torch.randn(t, E, generator=g), -1)
        w, idx = torch.topk(probs, K_TOP)
        w = (w / w.sum(-1, keepdim=True)).requires_grad_()
        out = ref_moe.routed_forward(h, idx, w, gu, dn, f, E)
        out.backward(torch.randn(t, H, generator=g))

    run(64)  # warm-up: thread pool, allocator
    t0 = time.perf_counter()
    run(tokens)
    dt = time.perf_counter() - t0
    return {"value": round(tokens / dt, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"config-1 layer (H={H}, I={I}, E={E}, top-{K_TOP}, r={R}) fwd+bwd on {tokens} of the {T} tokens, "
                      f"fp32 per-expert oracle, {dt:.2f} s"}


def read_traffic():
    """HBM bytes per launch of the grouped product from the committed rocprofv3 PMC summary, or None."""
    if not PROFILE_TRAFFIC.exists():
        return None
    for line in PROFILE_TRAFFIC.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def roofline(c, achieved, config):
    """The grouped product's achieved rate against the MFMA peak it runs on (traffic measured for config 1)."""
    if c.get("stack") == "fp8" and os.environ.get("MEEPSQUARED_FP8_PRODUCTS") == "0":
        return {"bound": "mfma", "kernel": "grouped_gemm_bf16_kernel, fp8 stacks decoded to bf16 in registers",
                "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None}
    if c.get("stack") == "fp8":
        return {"bound": "mfma", "kernel": f"fp8_prep + fp8_gemm_kernel, {_fp8_terms()} e4m3 term(s) (4 products per "
                                           "step, timed together)",
                "achieved": round(achieved, 2), "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_FP8_TFLOPS, 4), "traffic": None}
    kernel = ("grouped_gemm_bf16_kernel (DMA-fed, NF4 stacks decoded in registers; 4 launches per step)"
              if c.get("stack") == "nf4" else
              "grouped_gemm_bf16_kernel (4 launches per step; traffic = mean HBM bytes per launch, rocprofv3 PMC)")
    return {"bound": "mfma", "kernel": kernel, "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": read_traffic() if config == 1 else None}


def _fp8_terms():
    return 1 if os.environ.get("MEEPSQUARED_FP8_TERMS") == "1" else 2


def copy_calibration(mib: int, reps: int = 3):
    """Copy a buffer of `mib` MiB device to device `reps` times: under rocprofv3 --pmc, FETCH_SIZE and
    WRITE_SIZE of these dispatches against the known byte count give the counters' scale factor."""
    import torch

    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_dispatch": n, "dispatches": reps}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-tokens", type=int, default=CONFIGS[1]["T"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB")
    ap.add_argument("--config", type=int, default=1, choices=(1, 2, 3, 4),
                    help="1: the bf16 Qwen3-shaped layer (default, the headline); 2: Mixtral-shaped with Zipf-loaded "
                         "experts; 3: config 1 with fp8 e4m3 stacks (per-row scales) on the fp8 MFMA; 4: config 1 "
                         "shapes on a packed varlen batch with NF4 stacks")
    ap.add_argument("--fp8-products", action="store_true",
                    help="config 3 with the products on the fp8 MFMA, the activations quantised to two e4m3 terms "
                         "(MEEPSQUARED_FP8_TERMS=1: one term, the reference's single pass, ~4.7 %% error) instead of "
                         "in bf16 with the fp8 stack decoded in registers (the default: exact decode, faster here)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {a.gpus})", file=sys.stderr)
        sys.exit(2)
    if a.copy_calibration:
        copy_calibration(a.copy_calibration)
        return

    import torch

    from meepsquared_amd import Experts, _grouped, routed_forward, topk_softmax

    torch.backends.cuda.matmul.allow_tf32 = False
    device = "cuda:0"
    torch.cuda.set_device(0)
    c = CONFIGS[a.config]
    T, H, I, E, K_TOP, R = config_tokens(c), c["H"], c["I"], c["E"], c["k"], c["r"]
    hidden, logits, gate_up, down, factors, dy = make_inputs(device, c=c)
    if c.get("stack") == "fp8":
        from meepsquared_amd import _fp8

        gate_up8, gate_up_s = _fp8.quantize_stack(gate_up, per_row=True)
        down8, down_s = _fp8.quantize_stack(down, per_row=True)
        del gate_up, down
        experts = Experts(gate_up8, down8, gate_up_proj_scale_inv=gate_up_s, down_proj_scale_inv=down_s)
        os.environ["MEEPSQUARED_FP8_PRODUCTS"] = "1" if a.fp8_products else "0"
        c = dict(c, name=c["name"] + (f", products on the fp8 MFMA ({_fp8_terms()} e4m3 activation term(s))"
                                      if a.fp8_products else ", bf16 products (fp8 stacks decoded in registers)"))
    elif c.get("stack") == "nf4":
        from meepsquared_amd import _nf4

        experts = Experts(_nf4.quantize_stack(gate_up), _nf4.quantize_stack(down))
        del gate_up, down
    else:
        experts = Experts(gate_up, down)
    params = [hidden] + [t for (a_, b_, _) in factors.values() for t in (a_, b_)]

    def step():
        for p in params:
            p.grad = None
        w, idx = topk_softmax(logits, K_TOP)
        w.requires_grad_()
        out = routed_forward(experts, hidden, idx, w, factors)
        out.backward(dy)

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()

    # the timed region: K steps with one event on each side (per-launch events would add a few
    # microseconds of idle GPU per launch and are taken in the pass that follows)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(a.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    # K more steps with HIP events around every grouped-product and reduction launch, on the launch
    # stream: the kernels' own durations for the roofline
    launches = []  # (kind, info, start event, end event)

    def observer(kind, phase, info):
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        if phase == "before":
            launches.append([kind, dict(info), ev, None])
        else:
            launches[-1][3] = ev

    _grouped.launch_observer = observer
    istart, iend = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    istart.record()
    for _ in range(a.steps):
        step()
    iend.record()
    torch.cuda.synchronize()
    _grouped.launch_observer = None
    ms_instrumented = istart.elapsed_time(iend) / a.steps

    ms_per_step = start.elapsed_time(end) / a.steps
    tokens_per_s = T * a.steps / (ms_per_step * a.steps / 1e3)
    gemm = [(info, s.elapsed_time(e)) for kind, info, s, e in launches if kind == "grouped_gemm"]
    red = [(info, s.elapsed_time(e)) for kind, info, s, e in launches if kind == "grouped_reduce"]
    gemm_ms = sum(ms for _, ms in gemm)
    gemm_flops = sum(gemm_launch_flops(info) for info, _ in gemm)
    achieved = gemm_flops / (gemm_ms / 1e3) / 1e12
    flops = step_flops(T, H, I, K_TOP, R)
    per_shape, red_shape = {}, {}
    for info, ms in gemm:
        key = f"{info['K']}->{info['N']}"
        per_shape.setdefault(key, []).append(ms)
    for info, ms in red:
        key = f"{info['N']}x{info['R']}" + ("/gathered" if info.get("gathered") else "") + \
              ("/scaled" if info.get("scaled") else "")
        red_shape.setdefault(key, []).append(ms)
    record = {
        "metric": "MoE-LoRA layer fwd+bwd tokens/sec; achieved TFLOP/s vs MFMA peak",
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"fp8": "fp8-e4m3 products (activations as e4m3 terms, per-row fp32 stack scales)" if a.fp8_products
                  else "bf16 products (fp8-e4m3 stacks decoded in registers, per-row fp32 scales)",
                  "nf4": "bf16 products (NF4 stacks decoded in registers)"}.get(c.get("stack"), "bf16"),
        "data": "synthetic (seeded N(0,1) x and logits, N(0,0.02) W, Kaiming-uniform A, N(0,0.01) B)",
        "config": {"workload": c["name"], "tokens": T, "hidden": H, "moe_intermediate": I, "experts": E,
                   "top_k": K_TOP, "lora_rank": R, "lora_alpha": c["alpha"], "parallelism": "single GPU"},
        "step_tflops": round(flops / (ms_per_step / 1e3) / 1e12, 2),
        "step_frac_of_bf16_peak": round(flops / (ms_per_step / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "roofline": roofline(c, achieved, a.config),
        "kernel_ms_per_step": {"grouped_gemm": round(gemm_ms / a.steps, 4),
                               "grouped_reduce": round(sum(ms for _, ms in red) / a.steps, 4),
                               "rest": round(ms_per_step - (gemm_ms + sum(ms for _, ms in red)) / a.steps, 4),
                               "measured_over": f"{a.steps} steps after the timed ones, HIP events around each "
                                                f"launch ({ms_instrumented:.4f} ms/step with the events)"},
        "grouped_gemm_ms_by_shape": {k_: round(sum(v) / len(v), 4) for k_, v in per_shape.items()},
        "grouped_reduce_ms_by_shape": {k_: round(sum(v) / len(v), 4) for k_, v in red_shape.items()},
        "wall_s_timed": round(wall, 3),
    }
    if "zipf" in c or "varlen" in c:  # how ragged the expert groups were
        counts = torch.bincount(topk_softmax(logits, K_TOP)[1].flatten(), minlength=E)
        record["config"]["expert_rows"] = {"min": int(counts.min()), "max": int(counts.max()),
                                           "mean": round(float(counts.float().mean()), 1)}
        if "zipf" in c:
            record["config"]["expert_rows"]["all"] = counts.tolist()
        if "varlen" in c:
            record["config"]["sequences"] = c["varlen"][0]
    if not a.no_cpu_baseline and a.config == 1:
        record["cpu_baseline"] = cpu_baseline(a.cpu_tokens)
    else:
        record["cpu_baseline"] = None
    print(json.dumps(record))


if __name__ == "__main__":
    main()
