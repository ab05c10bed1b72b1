"""Throughput of the fused 4-bit AdamW step on one MI355X.

Default workload: a Llama-3-8B-shaped fp32 parameter set (hidden 4096, 32 layers,
GQA q/o 4096x4096 and k/v 1024x4096, FFN 14336x4096 / 4096x14336, untied
128256x4096 embedding and LM head, RMSNorm vectors of 4096: 291 tensors,
8,030,261,248 values) with synthetic Student-t(3) gradients scaled by per-row
log-normal(-7, 1) magnitudes.  One timed step = one ZE-EDEN step followed by one
ZIP-SR step over all tensors (each recipe keeps its own moment state), i.e. two
fused launches.

Prints one JSON line: Gelem/s over the timed steps, the HBM roofline of the dominant
fused kernel (the recipe with the longest launches: algorithmic bytes per launch /
mean launch time, HIP events recorded on the launch stream; measured HBM traffic per
launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary of the workload)
and a CPU baseline: the oracle's restatement of the reference's eager chunk update
timed on this host on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0
HERE = os.path.dirname(os.path.abspath(__file__))
RECIPE_KERNELS = {"ZE-EDEN": "step_kernel<RTN, RTN, F32>", "ZIP-SR": "step_kernel<RTN, UPDATE_SR, F32>"}


def llama3_8b_shapes():
    h, ffn, vocab, kv = 4096, 14336, 128256, 1024
    shapes = [(vocab, h)]
    for _ in range(32):
        shapes += [(h, h), (kv, h), (kv, h), (h, h), (ffn, h), (ffn, h), (h, ffn), (h,), (h,)]
    shapes += [(h,), (vocab, h)]
    return shapes


def gpt2_small_shapes():
    d = 768
    shapes = [(50257, d), (1024, d)]
    for _ in range(12):
        shapes += [(d,), (d,), (d, 3 * d), (3 * d,), (d, d), (d,), (d,), (d,), (d, 4 * d), (4 * d,), (4 * d, d), (d,)]
    shapes += [(d,), (d,)]
    return shapes


CONFIGS = {
    "llama3-8b": llama3_8b_shapes,
    "gpt2-small": gpt2_small_shapes,
    "1024x1024": lambda: [(1024, 1024)],
    "4096x4096": lambda: [(4096, 4096)],
}


def bytes_per_value(numel: int, param_bytes: int = 4, grad_bytes: int = 4) -> float:
    """Algorithmic HBM bytes per value of one step: p read+write, g read, and per moment
    either 4-bit codes read+write plus one fp32 scale per 128 values read+write, or fp32
    state read+write (tensors below 4096 values or not a multiple of 128)."""
    moment = 2 * 0.5 + 2 * 4 / 128 if (numel >= 4096 and numel % 128 == 0) else 8.0
    return 2 * param_bytes + grad_bytes + 2 * moment


def make_grads(shapes, device, seed):
    import torch

    gen = torch.Generator(device=device).manual_seed(seed)
    grads = []
    for s in shapes:
        z = torch.randn(s, generator=gen, device=device)
        chi2 = torch.zeros(s, device=device)
        for _ in range(3):
            chi2.addcmul_(*(2 * [torch.randn(s, generator=gen, device=device)]))
        z.div_(chi2.div_(3.0).sqrt_())
        rows = s[0] if len(s) > 1 else 1
        scale = torch.exp(torch.randn(rows, generator=gen, device=device) - 7.0)
        z.mul_(scale.view(-1, *([1] * (len(s) - 1))) if len(s) > 1 else scale)
        grads.append(z)
        del chi2
    return grads


def cpu_baseline(seconds_target: float = 12.0):
    """The oracle's eager chunk update (the reference's CPU path, op for op) on a bounded
    sample: ZE-EDEN steps of one fp32 4096x4096 tensor, on all host threads."""
    import torch

    from oracle import reference_step as ref

    gen = torch.Generator().manual_seed(0)
    shape = (4096, 4096)
    p = torch.randn(shape, generator=gen) * 0.02
    oracle = ref.Oracle([p], ref.Hyper(), ["nf4"], ["dyn4_nz"], [True])
    g = torch.randn(shape, generator=gen) * 1e-3
    oracle.step([g])  # state initialization outside the timed steps
    times = []
    start = time.perf_counter()
    while time.perf_counter() - start < seconds_target or len(times) < 3:
        t0 = time.perf_counter()
        oracle.step([g])
        times.append(time.perf_counter() - t0)
    per_step = statistics.median(times)
    n = p.numel()
    return {"value": n / per_step / 1e9, "unit": "Gelem/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle ZE-EDEN eager chunk update, fp32 4096x4096 (16.8M values), median of {len(times)} "
                      f"steps, {per_step * 1e3:.1f} ms/step, {torch.get_num_threads()} threads"}


def measured_traffic(config: str):
    """HBM bytes per launch of each recipe's kernel from the committed rocprofv3 summary of
    this workload (TCC FETCH_SIZE / WRITE_SIZE, scaled by a device copy of known size);
    None where no summary covers the workload."""
    path = os.path.join(HERE, "profiles", f"step_kernel_{config}_fp32_hbm_traffic.txt")
    if not os.path.exists(path):
        return None, None
    out = {}
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch "):
                _, recipe, value = line.split()
                out[recipe] = float(value)
    return out, os.path.relpath(path, HERE)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="llama3-8b", choices=sorted(CONFIGS))
    ap.add_argument("--recipes", default="zeeden,zipsr")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--copy-probe-gb", type=float, default=0.0,
                    help="also run plain device copies of this many GB (calibrates HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the optimizer step is replica-local "
              "and this build runs no multi-GPU configuration", file=sys.stderr)
        sys.exit(2)

    import torch

    import adamw4bit_amd as aw

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.copy_probe_gb > 0:
        # A plain copy of known size: its FETCH_SIZE / WRITE_SIZE per dispatch calibrate the
        # counters; copy and add timings give the streaming bandwidth torch's kernels reach.
        n = int(args.copy_probe_gb * 1e9) // 4
        src = torch.ones(n, device=device)
        dst = torch.empty_like(src)
        for name, fn, nbytes in (("copy", lambda: dst.copy_(src), 8 * n), ("add", lambda: dst.add_(src), 12 * n)):
            fn()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(5):
                fn()
            b.record()
            torch.cuda.synchronize()
            ms = a.elapsed_time(b) / 5
            print(f"[bench] {name} probe: {nbytes} bytes in {ms:.3f} ms = {nbytes / ms / 1e6:.0f} GB/s",
                  file=sys.stderr, flush=True)
        del src, dst
    shapes = CONFIGS[args.config]()
    numels = [math.prod(s) for s in shapes]
    total = sum(numels)
    algo_bytes = sum(n * bytes_per_value(n) for n in numels)

    print(f"[bench] {args.config}: {len(shapes)} tensors, {total:,} values, "
          f"{algo_bytes / 1e9:.2f} GB algorithmic per launch", file=sys.stderr, flush=True)
    gen = torch.Generator(device=device).manual_seed(1234)
    params = [torch.nn.Parameter(torch.randn(s, generator=gen, device=device) * 0.02) for s in shapes]
    grads = make_grads(shapes, device, seed=5678)
    for p, g in zip(params, grads):
        p.grad = g
    del grads
    recipes = []
    for r in args.recipes.split(","):
        if r == "zeeden":
            recipes.append(("ZE-EDEN", aw.ZEEDENAdamW4Bit(params, optimized=True)))
        elif r == "zipsr":
            recipes.append(("ZIP-SR", aw.ZIPSRAdamW4Bit(params, optimized=True, quant_rng_seed=0)))
        else:
            raise SystemExit(f"unknown recipe {r}")
    torch.cuda.synchronize()
    print(f"[bench] allocated {torch.cuda.memory_allocated() / 1e9:.1f} GB; warmup {args.warmup}",
          file=sys.stderr, flush=True)

    stream = torch.cuda.current_stream(device)
    for _ in range(args.warmup):
        for _, opt in recipes:
            opt.step()
    torch.cuda.synchronize()

    events = {name: [] for name, _ in recipes}
    t0 = time.perf_counter()
    for _ in range(args.steps):
        for name, opt in recipes:
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            opt.step()
            stop.record(stream)
            events[name].append((start, stop))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    launch_ms = {name: [a.elapsed_time(b) for a, b in ev] for name, ev in events.items()}
    per_recipe = {name: statistics.mean(v) for name, v in launch_ms.items()}
    # The dominant kernel is the recipe with the longest launches; its roofline is reported.
    dominant = max(per_recipe, key=per_recipe.get)
    achieved = algo_bytes / (per_recipe[dominant] * 1e-3) / 1e9
    traffic, traffic_source = measured_traffic(args.config)
    ms_per_step = wall * 1e3 / args.steps
    value = total * len(recipes) * args.steps / wall / 1e9
    print(f"[bench] timed {args.steps} steps in {wall:.3f} s; per-launch ms mean "
          f"{ {k: round(v, 3) for k, v in per_recipe.items()} } min "
          f"{ {k: round(min(v), 3) for k, v in launch_ms.items()} }", file=sys.stderr, flush=True)

    baseline = None
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        baseline = cpu_baseline(args.cpu_seconds)

    out = {
        "metric": "4-bit AdamW step Gelem/s + % of HBM peak BW, Llama-3-8B param set, 1 GPU",
        "value": round(value, 3),
        "unit": "Gelem/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: Student-t(3) x per-row log-normal(-7,1) gradients, N(0,0.02) parameters",
        "config": {
            "workload": f"{args.config} fp32 parameter set, one {' + one '.join(n for n, _ in recipes)} step "
                        f"per timed step ({len(recipes)} fused launches)",
            "tensors": len(shapes), "values": total, "recipes": [n for n, _ in recipes],
            "launch_ms": {k: round(v, 4) for k, v in per_recipe.items()},
            "gelem_s_per_recipe": {k: round(total / (v * 1e-3) / 1e9, 2) for k, v in per_recipe.items()},
            "hbm_frac_per_recipe": {k: round(algo_bytes / (v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
                                    for k, v in per_recipe.items()},
            "algorithmic_gb_per_launch": round(algo_bytes / 1e9, 4),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"{RECIPE_KERNELS.get(dominant, dominant)} ({dominant})",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": (round(traffic[dominant]) if traffic and dominant in traffic else None),
            "traffic_source": traffic_source,
        },
        "cpu_baseline": baseline,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
