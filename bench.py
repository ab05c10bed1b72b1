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
# --recipes names of the reference step's research m2 schemes -> (scheme, extra bytes per value)
RESEARCH_M2 = {
    "la": ("dyn4_la_upd_sr", 0.0), "proxy-la": ("dyn4_proxy_la_upd_sr", 0.0),
    "vproxy-la": ("dyn4_vproxy_la_upd_sr", 0.0), "upd-sr": ("dyn4_upd_sr", 0.0),
    "store-eden": ("dyn4_upd_sr_store_eden", 4.0),
}


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
    "llama3-8b-bf16-mixed": llama3_8b_shapes,
    "gpt2-small": gpt2_small_shapes,
    "1024x1024": lambda: [(1024, 1024)],
    "4096x4096": lambda: [(4096, 4096)],
}


def bytes_per_value(numel: int, param_bytes: int = 4, grad_bytes: int = 4, m1: str = "nf4", m2: str = "dyn4") -> float:
    """Algorithmic HBM bytes per value of one step: p read+write, g read, and per moment
    either 4-bit codes read+write plus one fp32 scale per 128 values read+write, or fp32
    state read+write (an fp32 scheme, or tensors below 4096 values or not a multiple of 128)."""
    eligible = numel >= 4096 and numel % 128 == 0
    moment = [2 * 0.5 + 2 * 4 / 128 if (eligible and m != "fp32") else 8.0 for m in (m1, m2)]
    return 2 * param_bytes + grad_bytes + sum(moment)


def mixed_bf16_groups(params):
    """The mixed-scheme stress case on the Llama-3-8B shapes: ZIP-SR schemes everywhere, every
    tenth tensor an ablation of QuantizedAdamW (alternately an fp32 second moment and ZIP-SR with
    EDEN on m2), the LM head's first moment stochastically rounded (nf4_sr)."""
    groups, schemes = [], []
    for i, p in enumerate(params):
        if i % 10 == 5:
            m2, eden = ("fp32", False) if (i // 10) % 2 == 0 else ("dyn4_upd_sr_fp32read", True)
        else:
            m2, eden = "dyn4_upd_sr_fp32read", False
        groups.append(dict(params=[p], m1_quant_scheme="nf4", m2_quant_scheme=m2, use_eden_m2=eden))
        schemes.append(["nf4", m2])
    schemes[-1][0] = "nf4_sr"  # LM head
    return groups, schemes


def make_grads(shapes, device, seed):
    import torch

    gen = torch.Generator(device=device).manual_seed(seed)
    grads = []
    for i, s in enumerate(shapes):
        if i and i % 64 == 0:
            print(f"[bench] gradients {i}/{len(shapes)}", file=sys.stderr, flush=True)
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


CPU_SHAPE = (4096, 4096)
SMALL_SHAPE, SMALL_WARMUP, SMALL_STEPS = (1024, 1024), 10, 100
CPU_RECIPES = {"ZE-EDEN": ("nf4", "dyn4_nz", True), "ZIP-SR": ("nf4", "dyn4_upd_sr_fp32read", False)}


def cpu_leg(seconds_target: float) -> dict:
    """One leg of the CPU baseline, in a process that never touches the GPU: the oracle's eager
    chunk update (the reference's CPU path, op for op) on one fp32 4096x4096 tensor per recipe,
    with the draws of ZIP-SR from torch's CPU generator as the reference takes them; the median
    step time of each recipe after one untimed step."""
    import torch

    from oracle import reference_step as ref

    if os.environ.get("OMP_NUM_THREADS"):
        # ATen sizes its pool from MKL's thread count when MKL is present, which can differ
        torch.set_num_threads(int(os.environ["OMP_NUM_THREADS"]))
    out = {"threads": torch.get_num_threads(), "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
           "ms_per_step": {}, "steps": {}}
    gen = torch.Generator().manual_seed(0)
    for name, (m1, m2, eden) in CPU_RECIPES.items():
        p = torch.randn(CPU_SHAPE, generator=gen) * 0.02
        oracle = ref.Oracle([p], ref.Hyper(), [m1], [m2], [eden], seed=0)
        g = torch.randn(CPU_SHAPE, generator=gen) * 1e-3
        oracle.step([g])  # state initialization outside the timed steps
        times = []
        start = time.perf_counter()
        while time.perf_counter() - start < seconds_target / len(CPU_RECIPES) or len(times) < 3:
            t0 = time.perf_counter()
            oracle.step([g])
            times.append(time.perf_counter() - t0)
        out["ms_per_step"][name] = statistics.median(times) * 1e3
        out["steps"][name] = len(times)
    # the single small tensor: ZE-EDEN on one fp32 1024x1024 parameter with fresh seeded
    # N(0, 1e-3) gradients each step, 10 untimed steps, then the median of 100
    p = torch.randn(SMALL_SHAPE, generator=gen) * 0.02
    oracle = ref.Oracle([p], ref.Hyper(), ["nf4"], ["dyn4_nz"], [True])
    grads = [torch.randn(SMALL_SHAPE, generator=gen) * 1e-3 for _ in range(SMALL_WARMUP + SMALL_STEPS)]
    times = []
    for k, g in enumerate(grads):
        t0 = time.perf_counter()
        oracle.step([g])
        if k >= SMALL_WARMUP:
            times.append(time.perf_counter() - t0)
    out["small_ms_per_step"] = statistics.median(times) * 1e3
    return out


def _protocol_minutes(legs) -> float:
    """Minutes that 110 steps (10 warmup + 100 timed) of each 4096x4096 recipe would take in every
    leg, at the measured step times."""
    return sum(110 * sum(leg["ms_per_step"].values()) for leg in legs) / 6e4


def cpu_baseline(seconds_target: float = 20.0):
    """The CPU baseline: the same sample timed in two fresh child processes, on all host threads
    and at OMP_NUM_THREADS=2 (the reference's CI setting, .github/workflows/ci.yml:17).  `value`
    is the all-threads rate over both recipes (values x recipes / time), the unit of the GPU
    figure; it is measured on a 16.8M-value tensor and quoted as a rate, not on the 8.03G-value
    parameter set."""
    import subprocess

    legs = []
    for threads in (None, 2):
        env = dict(os.environ)
        if threads is not None:
            env["OMP_NUM_THREADS"] = env["MKL_NUM_THREADS"] = str(threads)
        env["CUDA_VISIBLE_DEVICES"] = ""
        env["HIP_VISIBLE_DEVICES"] = ""
        proc = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-leg",
                               "--cpu-seconds", str(seconds_target / 2)],
                              env=env, capture_output=True, text=True, cwd=HERE, timeout=600)
        if proc.returncode != 0:
            raise RuntimeError(f"cpu baseline leg failed: {proc.stderr[-2000:]}")
        legs.append(json.loads(proc.stdout.strip().splitlines()[-1]))
    n = CPU_SHAPE[0] * CPU_SHAPE[1]
    cpu = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next(line.split(":", 1)[1].strip() for line in f if line.startswith("model name"))
    except (OSError, StopIteration):
        pass
    import torch

    def rate(leg):
        return n * len(CPU_RECIPES) / (sum(leg["ms_per_step"].values()) * 1e-3) / 1e9

    main_leg, ci_leg = legs
    detail = "; ".join(f"{leg['threads']} threads: " + ", ".join(f"{k} {v:.1f} ms/step ({leg['steps'][k]} steps)"
                                                                for k, v in leg["ms_per_step"].items())
                       for leg in legs)
    return {"value": rate(main_leg), "unit": "Gelem/s", "cores": main_leg["threads"], "kind": "port",
            "sample": f"oracle eager chunk update (the reference's CPU path), one fp32 4096x4096 tensor "
                      f"(16.8M values) per recipe, ZE-EDEN + ZIP-SR, in child processes off the GPU: the median "
                      f"of the steps that fit in about {seconds_target / 2 / len(CPU_RECIPES):.0f} s after one "
                      f"untimed step (not the median of 100 steps after 10 warmup steps, which would take "
                      f"about {_protocol_minutes(legs):.0f} min on these threads); the 1024x1024 ZE-EDEN leg "
                      f"(legs[].zeeden_1024x1024_ms_per_step) is the median of 100 steps after 10 warmup "
                      f"steps; {detail}; {cpu}, ATen {torch.backends.cpu.get_cpu_capability()}, "
                      f"os.cpu_count {os.cpu_count()}",
            "legs": [{"threads": leg["threads"], "omp_num_threads": leg["omp_num_threads"],
                      "ms_per_step": {k: round(v, 2) for k, v in leg["ms_per_step"].items()},
                      "zeeden_1024x1024_ms_per_step": round(leg["small_ms_per_step"], 3),
                      "gelem_s": round(rate(leg), 5)} for leg in legs],
            "ci_threads_value": rate(ci_leg)}


def copy_ceiling(device, gb: float = 4.0, reps: int = 10) -> float:
    """The streaming rate of a plain device copy (torch's copy kernel, ``gb`` GB read and written
    per copy) on this box, GB/s: the ceiling a read-and-write stream reaches here, against which
    the step's rate is also reported."""
    import torch

    n = int(gb * 1e9) // 4
    src = torch.ones(n, device=device)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    del src, dst
    return 8 * n / (ms * 1e-3) / 1e9


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


def build_workload(config: str, recipe_names: str, clip, device):
    """Parameters (with gradients) and optimizers of one workload: (shapes, params, recipes,
    algorithmic bytes per launch of each recipe, gradient bytes); recipes are (name, optimizer,
    algorithmic bytes)."""
    import torch

    import adamw4bit_amd as aw

    shapes = CONFIGS[config]()
    numels = [math.prod(s) for s in shapes]
    total = sum(numels)
    mixed = config == "llama3-8b-bf16-mixed"
    dtype = torch.bfloat16 if mixed else torch.float32
    esize = 2 if mixed else 4

    gen = torch.Generator(device=device).manual_seed(1234)
    params = [torch.nn.Parameter((torch.randn(s, generator=gen, device=device) * 0.02).to(dtype)) for s in shapes]
    grads = make_grads(shapes, device, seed=5678)
    for p, g in zip(params, grads):
        if mixed and g.numel() % 128 == 0:  # 1% of gradient blocks zero (dyn4 zero-inclusive path)
            nb = g.numel() // 128
            g.view(nb, 128)[torch.rand(nb, generator=gen, device=device) < 0.01] = 0.0
        p.grad = g.to(dtype)
    del grads
    recipes = []  # (name, optimizer, algorithmic bytes per launch)
    if mixed:
        groups, schemes = mixed_bf16_groups(params)
        opt = aw.QuantizedAdamW(groups, m1_quant_scheme="nf4", m2_quant_scheme="dyn4_upd_sr_fp32read",
                                optimized=True, quant_rng_seed=0)
        opt.set_m1_quant_scheme_for_parameters([params[-1]], "nf4_sr")
        algo = sum(n * bytes_per_value(n, esize, esize, *sc) for n, sc in zip(numels, schemes))
        recipes.append(("mixed", opt, algo))
    else:
        algo = sum(n * bytes_per_value(n) for n in numels)
        for r in recipe_names.split(","):
            if r == "zeeden":
                recipes.append(("ZE-EDEN", aw.ZEEDENAdamW4Bit(params, optimized=True), algo))
            elif r == "zipsr":
                recipes.append(("ZIP-SR", aw.ZIPSRAdamW4Bit(params, optimized=True, quant_rng_seed=0), algo))
            elif r in RESEARCH_M2:
                # the reference step's research m2 schemes (one generic-kernel instance), NF4 m1
                m2, extra = RESEARCH_M2[r]
                opt = aw.QuantizedAdamW(params, m1_quant_scheme="nf4", m2_quant_scheme=m2, optimized=True,
                                        quant_rng_seed=0)
                # the pending lookahead m2 is fp32 state; store-EDEN also writes 1 / denominator
                m2_kind = "fp32" if m2 == "dyn4_la_upd_sr" else "dyn4"
                research = sum(n * (bytes_per_value(n, m2=m2_kind) + (extra if n >= 4096 and n % 128 == 0 else 0))
                               for n in numels)
                recipes.append((m2, opt, research))
            else:
                raise SystemExit(f"unknown recipe {r}")
    algo_bytes = {name: a for name, _, a in recipes}
    grad_bytes = sum(p.grad.numel() * p.grad.element_size() for p in params)
    if clip is not None:  # the fused clip adds one read of every gradient
        algo_bytes = {name: a + grad_bytes for name, a in algo_bytes.items()}
    print(f"[bench] {config}: {len(shapes)} tensors, {total:,} values, "
          f"{ {k: round(v / 1e9, 2) for k, v in algo_bytes.items()} } GB algorithmic per launch",
          file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    print(f"[bench] allocated {torch.cuda.memory_allocated() / 1e9:.1f} GB", file=sys.stderr, flush=True)
    return shapes, params, recipes, algo_bytes, grad_bytes



def time_launches(recipes, steps: int, warmup: int, clip, stream):
    """``warmup`` untimed steps, then ``steps`` timed steps of every recipe: each launch bracketed
    by HIP events on the launch stream.  Returns the launch times (ms) per recipe, the wall time
    of the timed steps (s) and the event pairs around the fused clip prologues."""
    import torch

    for _ in range(warmup):
        for _, opt, _ in recipes:
            if clip is not None:
                opt.clip_grad_norm_(clip)
            opt.step()
    torch.cuda.synchronize()
    events = {name: [] for name, _, _ in recipes}
    norm_events = []
    t0 = time.perf_counter()
    for _ in range(steps):
        for name, opt, _ in recipes:
            start, mid, stop = (torch.cuda.Event(enable_timing=True) for _ in range(3))
            start.record(stream)
            if clip is not None:
                opt.clip_grad_norm_(clip)
            mid.record(stream)
            opt.step()
            stop.record(stream)
            events[name].append((start, stop))
            norm_events.append((start, mid))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return {name: [a.elapsed_time(b) for a, b in ev] for name, ev in events.items()}, wall, norm_events


def time_grad_scaler(recipes, steps: int, warmup: int, clip, stream, fused: bool) -> dict:
    """A trainer with loss scaling (torch.amp.GradScaler, scale 1.0 so the gradients keep their
    values when torch unscales them in place): per iteration the unscale and clip, then
    ``scaler.step`` (which reads found_inf on the host) and ``scaler.update``.  fused: the unscale
    folded into the fused clip's read of the gradients (``clip_grad_norm_(max_norm,
    grad_scaler=scaler)``); else torch's ``scaler.unscale_`` (a read and a write of every gradient)
    followed by the fused clip.  Returns the mean ms per iteration per recipe (HIP events around
    the whole iteration on the launch stream)."""
    import torch

    out = {}
    for name, opt, _ in recipes:
        scaler = torch.amp.GradScaler("cuda", init_scale=1.0, growth_interval=1 << 30)
        loss = torch.ones((), device=stream.device)
        ev = []
        for k in range(warmup + steps):
            scaler.scale(loss)
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            if fused:
                opt.clip_grad_norm_(clip, grad_scaler=scaler)
            else:
                scaler.unscale_(opt)
                opt.clip_grad_norm_(clip)
            scaler.step(opt)
            stop.record(stream)
            scaler.update()
            if k >= warmup:
                ev.append((start, stop))
        torch.cuda.synchronize()
        out[name] = statistics.mean(a.elapsed_time(b) for a, b in ev)
    return out


def time_blocks(recipes, steps: int, warmup: int, stream) -> dict:
    """Per recipe: ``warmup`` untimed steps, then ``steps`` steps back to back between one pair of
    HIP events on the launch stream; ms per step."""
    import torch

    out = {}
    for name, opt, _ in recipes:
        for _ in range(warmup):
            opt.step()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for _ in range(steps):
            opt.step()
        b.record(stream)
        torch.cuda.synchronize()
        out[name] = a.elapsed_time(b) / steps
    return out


def time_single_tensors(device, stream) -> dict:
    """The two single-tensor workloads, each timed through ``step()``: ZE-EDEN on one fp32
    1024x1024 parameter with fresh seeded N(0, 1e-3) gradients each step (100 timed steps after
    10 untimed ones, the reference's protocol for it), and ZIP-SR (quant_rng_seed=0) on one fp32
    4096x4096 parameter with the heavy-tailed gradients (100 timed steps after 100 untimed ones:
    its first tens of steps after a launch of another size run up to 10% slower).  The timed
    steps run back to back between one pair of HIP events on the launch stream (host time shows
    where it exceeds the kernel's; events between the steps would add their own work to them)
    and the wall clock; per step: their time / steps."""
    import torch

    import adamw4bit_amd as aw

    hyper = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True)
    out = {}
    gen = torch.Generator(device=device).manual_seed(7)
    for name, shape, make, warmup, steps, fresh in (
            ("zeeden_1024x1024", SMALL_SHAPE, lambda ps: aw.ZEEDENAdamW4Bit(ps, **hyper), SMALL_WARMUP, SMALL_STEPS,
             True),
            ("zipsr_4096x4096", (4096, 4096), lambda ps: aw.ZIPSRAdamW4Bit(ps, quant_rng_seed=0, **hyper), 100, 100,
             False)):
        p = torch.nn.Parameter(torch.randn(shape, generator=gen, device=device) * 0.02)
        opt = make([p])
        if fresh:
            grads = [torch.randn(shape, generator=gen, device=device) * 1e-3 for _ in range(warmup + steps)]
        else:
            grads = make_grads([shape], device, seed=11) * (warmup + steps)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        for k, g in enumerate(grads):
            if k == warmup:
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                a.record(stream)
            p.grad = g
            opt.step()
        b.record(stream)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / steps
        ms = a.elapsed_time(b) / steps
        algo = math.prod(shape) * bytes_per_value(math.prod(shape))
        out[name] = {"steps": steps, "warmup": warmup, "event_ms_per_step": round(ms, 4),
                     "wall_ms_per_step": round(wall * 1e3, 4),
                     "hbm_frac": round(algo / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del opt, p, grads
    return out


def time_unfused(recipes, params, steps: int, warmup: int, clip, stream):
    """The unfused path a trainer runs: torch's clip (norm pass + in-place multiply), then the
    step; mean ms per recipe."""
    import torch

    unfused = {}
    for name, opt, _ in recipes:
        for _ in range(warmup):
            torch.nn.utils.clip_grad_norm_(params, clip)
            opt.step()
        ev = []
        for _ in range(steps):
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            torch.nn.utils.clip_grad_norm_(params, clip)
            opt.step()
            stop.record(stream)
            ev.append((start, stop))
        torch.cuda.synchronize()
        unfused[name] = statistics.mean(a.elapsed_time(b) for a, b in ev)
    return unfused


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="llama3-8b", choices=sorted(CONFIGS))
    ap.add_argument("--recipes", default="zeeden,zipsr",
                    help="comma-separated: zeeden, zipsr, or a research m2 scheme: " + ", ".join(RESEARCH_M2))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-bf16-mixed", action="store_true",
                    help="with the default fp32 set, skip the bf16 mixed-scheme set and the single-tensor "
                         "cases measured after it")
    ap.add_argument("--cpu-leg", action="store_true", help=argparse.SUPPRESS)  # child process of the CPU baseline
    ap.add_argument("--clip-grad-norm", type=float, default=None, metavar="MAX_NORM",
                    help="clip the gradients to this global 2-norm before every step, fused into the step "
                         "(QuantizedAdamW.clip_grad_norm_), and also time torch.nn.utils.clip_grad_norm_ + step")
    ap.add_argument("--grad-scaler", action="store_true",
                    help="with --clip-grad-norm: also time a GradScaler loop, the loss-scale unscaling fused into "
                         "the clip (clip_grad_norm_(..., grad_scaler=)) against torch's scaler.unscale_ + fused clip")
    ap.add_argument("--copy-probe-gb", type=float, default=0.0,
                    help="also run plain device copies of this many GB (calibrates HBM byte counters)")
    args = ap.parse_args()
    if args.cpu_leg:
        print(json.dumps(cpu_leg(args.cpu_seconds)), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the optimizer step is replica-local "
              "and no multi-GPU configuration is measured here", file=sys.stderr)
        sys.exit(2)

    import torch

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
    clip = args.clip_grad_norm
    shapes, params, recipes, algo_bytes, grad_bytes = build_workload(args.config, args.recipes, clip, device)
    total = sum(math.prod(sh) for sh in shapes)
    mixed = args.config == "llama3-8b-bf16-mixed"
    stream = torch.cuda.current_stream(device)
    print(f"[bench] warmup {args.warmup}, timed steps {args.steps}", file=sys.stderr, flush=True)
    launch_ms, wall, norm_events = time_launches(recipes, args.steps, args.warmup, clip, stream)
    prologue = None
    if clip is not None:
        norm_ms = statistics.mean(a.elapsed_time(b) for a, b in norm_events)
        unfused = time_unfused(recipes, params, args.steps, args.warmup, clip, stream)
        scaled = None
        if args.grad_scaler:
            scaled = {
                "fused_unscale_clip_step_ms": {k: round(v, 4) for k, v in time_grad_scaler(
                    recipes, args.steps, args.warmup, clip, stream, fused=True).items()},
                "torch_unscale_then_fused_clip_step_ms": {k: round(v, 4) for k, v in time_grad_scaler(
                    recipes, args.steps, args.warmup, clip, stream, fused=False).items()},
            }
        prologue = {
            "max_grad_norm": clip,
            "fused_clip_and_step_ms": {k: round(statistics.mean(v), 4) for k, v in launch_ms.items()},
            "torch_clip_then_step_ms": {k: round(v, 4) for k, v in unfused.items()},
            "norm_pass_ms": round(norm_ms, 4),
            "norm_pass_gb": round(grad_bytes / 1e9, 3),
            "norm_pass_gb_s": round(grad_bytes / (norm_ms * 1e-3) / 1e9, 1),
            **({"grad_scaler": scaled} if scaled else {}),
        }
        print(f"[bench] clip prologue: {prologue}", file=sys.stderr, flush=True)
    per_recipe = {name: statistics.mean(v) for name, v in launch_ms.items()}
    names = [n for n, _, _ in recipes]
    ceiling = copy_ceiling(device)
    print(f"[bench] copy ceiling {ceiling:.0f} GB/s", file=sys.stderr, flush=True)
    # The dominant kernel is the recipe with the longest launches; its roofline is reported.
    dominant = max(per_recipe, key=per_recipe.get)
    achieved = algo_bytes[dominant] / (per_recipe[dominant] * 1e-3) / 1e9
    traffic, traffic_source = measured_traffic(args.config)
    ms_per_step = wall * 1e3 / args.steps
    value = total * len(names) * args.steps / wall / 1e9
    print(f"[bench] timed {args.steps} steps in {wall:.3f} s; per-launch ms mean "
          f"{ {k: round(v, 3) for k, v in per_recipe.items()} } min "
          f"{ {k: round(min(v), 3) for k, v in launch_ms.items()} }", file=sys.stderr, flush=True)

    bf16_mixed = None
    if args.config == "llama3-8b" and clip is None and not args.no_bf16_mixed:
        # The bf16 mixed-scheme set on the same shapes, measured in the same run after the fp32
        # set is freed: its launches per step and their share of the HBM roofline.
        recipes = params = None
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        _, mparams, mrecipes, malgo, _ = build_workload("llama3-8b-bf16-mixed", "", None, device)
        mlaunch, _, _ = time_launches(mrecipes, args.steps, args.warmup, None, stream)
        ms = statistics.mean(mlaunch["mixed"])
        bf16_mixed = {
            "workload": "llama3-8b-bf16-mixed: Llama-3-8B bf16 parameter set, ZIP-SR schemes, nf4_sr LM head, every "
                        "tenth tensor an fp32-m2 / EDEN-m2 ablation, 1% zero gradient blocks",
            "steps": args.steps, "warmup": args.warmup,
            "step_ms": round(ms, 4),
            "gelem_s": round(total / (ms * 1e-3) / 1e9, 2),
            "algorithmic_gb_per_step": round(malgo["mixed"] / 1e9, 4),
            "hbm_frac": round(malgo["mixed"] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        }
        print(f"[bench] bf16 mixed set: {bf16_mixed}", file=sys.stderr, flush=True)
        mrecipes = mparams = None

    single = gpt2 = None
    if args.config == "llama3-8b" and clip is None and not args.no_bf16_mixed:
        torch.cuda.empty_cache()
        single = time_single_tensors(device, stream)
        print(f"[bench] single tensors: {single}", file=sys.stderr, flush=True)
        # The GPT-2-small parameter list (148 tensors, 124M values; its vectors stay fp32 in the
        # same launch), both recipes.  Its first tens of steps after the set is built run up to
        # 10% slower than the later ones (blocks of ten steps: 0.379, 0.348, 0.344, 0.337 ms, then
        # 0.335 from the fiftieth on, ZE-EDEN), so 50 untimed steps precede the timed 50.
        gshapes, gparams, grecipes, galgo, _ = build_workload("gpt2-small", "zeeden,zipsr", None, device)
        gms = time_blocks(grecipes, 50, 50, stream)
        gpt2 = {
            "workload": "gpt2-small: 148 tensors, 124,439,808 fp32 values, ZE-EDEN and ZIP-SR, each recipe's "
                        "steps back to back between one pair of events",
            "steps": 50, "warmup": 50,
            "ms_per_step": {k: round(v, 4) for k, v in gms.items()},
            "hbm_frac": {k: round(galgo[k] / (v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4) for k, v in gms.items()},
        }
        print(f"[bench] gpt2-small: {gpt2}", file=sys.stderr, flush=True)
        grecipes = gparams = None

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
        "dtype": "bf16" if mixed else "f32",
        "data": "synthetic: Student-t(3) x per-row log-normal(-7,1) gradients, N(0,0.02) parameters"
                + (", 1% zero gradient blocks" if mixed else ""),
        "config": {
            "workload": (f"{args.config}: Llama-3-8B bf16 parameter set, ZIP-SR schemes, nf4_sr LM head, every "
                         "tenth tensor an fp32-m2 / EDEN-m2 ablation, one optimizer step per timed step"
                         if mixed else
                         f"{args.config} fp32 parameter set, one {' + one '.join(names)} step "
                         f"per timed step ({len(names)} fused launches)")
                        + (f", each after a fused gradient clip to norm {clip}" if clip is not None else ""),
            "tensors": len(shapes), "values": total, "recipes": names,
            "launch_ms": {k: round(v, 4) for k, v in per_recipe.items()},
            "gelem_s_per_recipe": {k: round(total / (v * 1e-3) / 1e9, 2) for k, v in per_recipe.items()},
            "hbm_frac_per_recipe": {k: round(algo_bytes[k] / (v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
                                    for k, v in per_recipe.items()},
            "algorithmic_gb_per_launch": {k: round(v / 1e9, 4) for k, v in algo_bytes.items()},
            **({"prologue": prologue} if prologue else {}),
            **({"bf16_mixed": bf16_mixed} if bf16_mixed else {}),
            **({"single_tensors": single} if single else {}),
            **({"gpt2_small": gpt2} if gpt2 else {}),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"{RECIPE_KERNELS.get(dominant, 'step_kernel launches')} ({dominant})",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": (round(traffic[dominant]) if traffic and dominant in traffic else None),
            "traffic_source": traffic_source,
            "copy_ceiling_gb_s": round(ceiling, 1),
            "frac_of_copy_ceiling": round(achieved / ceiling, 4),
        },
        "cpu_baseline": baseline,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
