"""Write golden fixtures for the 4-bit AdamW step from the reference implementation.

Run in the development container only (the reference is not present on GPU hosts):

    python tests/golden/make_golden.py [/root/reference/src]

It imports ``adamw4bit`` from the reference checkout, runs short multi-step
trajectories and codec calls that none of the reference's own tests pin
(composition of decode -> AdamW -> encode over several steps, the random-draw
consumption of the optimized backend versus the reference step, the chunk loop),
and stores inputs and outputs as ``.npz`` files next to this script.  Each file
holds plain arrays plus one JSON string ``config``; it loads with
``numpy.load(..., allow_pickle=False)``.  bf16/fp16 tensors are stored as their
int16 bit patterns.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF_SRC = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src"
sys.path.insert(0, REF_SRC)

import adamw4bit  # noqa: E402
from adamw4bit import QuantizedAdamW, ZEEDENAdamW4Bit, ZIPSRAdamW4Bit  # noqa: E402
from adamw4bit import _optimized_quantization as oq  # noqa: E402
from adamw4bit.quantization import QuantState  # noqa: E402

DTYPES = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().copy()
    return t.numpy().copy()


def heavy_tailed(shape, generator, row_mu=-7.0, row_sigma=1.0):
    """Student-t(3) values times per-row log-normal magnitudes."""
    z = torch.randn(shape, generator=generator)
    chi2 = (torch.randn((3,) + tuple(shape), generator=generator) ** 2).sum(0)
    t = z / torch.sqrt(chi2 / 3.0)
    rows = shape[0] if len(shape) > 1 else 1
    scale = torch.exp(row_mu + row_sigma * torch.randn(rows, generator=generator))
    return t * (scale.view(-1, *([1] * (len(shape) - 1))) if len(shape) > 1 else scale)


def snapshot(opt, params, prefix, out):
    for i, p in enumerate(params):
        out[f"{prefix}p{i}"] = to_np(p.data)
        st = opt.state[p]
        out[f"{prefix}p{i}_step"] = np.array(st["step"], dtype=np.int64)
        for m in ("m1", "m2"):
            if m == "m2" and "lookahead_pending_exp_avg_sq" in st:
                assert "m2" not in st and "m2_code" not in st
                out[f"{prefix}p{i}_m2_pending"] = to_np(st["lookahead_pending_exp_avg_sq"])
            elif f"{m}_code" in st:
                out[f"{prefix}p{i}_{m}_code"] = to_np(st[f"{m}_code"])
                qs = st[f"{m}_quant_state"]
                assert isinstance(qs, QuantState) and qs.packed
                out[f"{prefix}p{i}_{m}_scale"] = to_np(qs.absmax)
            else:
                out[f"{prefix}p{i}_{m}_fp32"] = to_np(st[m])
        if "m2_read_preconditioner" in st:
            out[f"{prefix}p{i}_m2_pre"] = to_np(st["m2_read_preconditioner"])


def trajectory(name, build, shapes, dtype, steps, *, grad_seed, snap_steps, m1_override=None,
               zero_block_frac=0.0, note="", grad_mu=-7.0):
    gen = torch.Generator().manual_seed(grad_seed)
    dt = DTYPES[dtype]
    params = [torch.nn.Parameter((torch.randn(s, generator=gen) * 0.02).to(dt)) for s in shapes]
    out = {}
    for i, p in enumerate(params):
        out[f"init_p{i}"] = to_np(p.data)
    opt, cfg = build(params)
    if m1_override:
        opt.set_m1_quant_scheme_for_parameters([params[j] for j in m1_override[0]], m1_override[1])
    for k in range(steps):
        for i, p in enumerate(params):
            g = heavy_tailed(tuple(p.shape), gen, row_mu=grad_mu)
            if zero_block_frac:
                flat = g.view(-1)
                nb = flat.numel() // 128
                mask = torch.rand(nb, generator=gen) < zero_block_frac
                flat.view(nb, 128)[mask] = 0.0
            p.grad = g.to(dt)
            out[f"grad_s{k}_p{i}"] = to_np(p.grad)
        opt.step()
        if (k + 1) in snap_steps:
            snapshot(opt, params, f"after{k + 1}_", out)
    cfg.update(dict(name=name, shapes=[list(s) for s in shapes], dtype=dtype, steps=steps,
                    snap_steps=sorted(snap_steps), m1_override=m1_override, note=note, grad_mu=grad_mu))
    out["config"] = np.array(json.dumps(cfg))
    np.savez_compressed(os.path.join(HERE, f"traj_{name}.npz"), **out)
    print("wrote", name, sum(v.nbytes for v in out.values()), "bytes raw")


HP = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


def recipe(cls, optimized=True, seed=None, chunk=None, **extra):
    def build(params):
        opt = cls(params, optimized=optimized, quant_rng_seed=seed, **HP, **extra)
        if chunk is not None:
            for g in opt.param_groups:
                g["max_chunk_numel"] = chunk
        per = [dict(m1=g["m1_quant_scheme"], m2=g["m2_quant_scheme"], eden=g["use_eden_m2"])
               for g in opt.param_groups for _ in g["params"]]
        return opt, dict(optimizer=cls.__name__, optimized=optimized, seed=seed,
                         chunk=chunk or (1 << 19), hyper=dict(HP, betas=list(HP["betas"])),
                         per_param=per)
    return build


def grouped(groups, optimized=True, seed=None):
    """QuantizedAdamW with one parameter group per (m1, m2, eden) entry."""
    def build(params):
        pg = [dict(params=[p], m1_quant_scheme=g[0], m2_quant_scheme=g[1], use_eden_m2=g[2])
              for p, g in zip(params, groups)]
        opt = QuantizedAdamW(pg, optimized=optimized, quant_rng_seed=seed,
                             m1_quant_scheme="nf4", m2_quant_scheme="dyn4_nz", **HP)
        per = [dict(m1=g[0], m2=g[1], eden=g[2]) for g in groups]
        return opt, dict(optimizer="QuantizedAdamW", optimized=optimized, seed=seed, chunk=1 << 19,
                         hyper=dict(HP, betas=list(HP["betas"])), per_param=per)
    return build


def codec_cases():
    """Chunk-codec vectors (_optimized_quantization.quantize) on crafted blocks."""
    gen = torch.Generator().manual_seed(2024)
    out = {}
    entries = []
    schemes = ["nf4", "nf4_sr", "sdyn4", "sdyn4_sr", "lin4", "lin4_sr", "lin4_nz", "dyn4",
               "dyn4_sr", "dyn4_nz", "dyn4_upd_sr_fp32read", "lin4_upd_sr_fp32read",
               "dyn4_lookahead_sr"]
    for mode in schemes:
        cb = oq._codebook(mode, torch.device("cpu"))
        signed = bool(cb[0] < 0)
        mids = (cb[:-1] + cb[1:]) / 2
        crafted = torch.cat([
            cb, mids, torch.nextafter(mids, torch.full_like(mids, 2.0)),
            torch.nextafter(mids, torch.full_like(mids, -2.0)),
            torch.nextafter(cb, torch.full_like(cb, 2.0)), torch.nextafter(cb, torch.full_like(cb, -2.0)),
        ]).clamp(-1.0 if signed else 0.0, 1.0)
        crafted = torch.cat([crafted, torch.zeros(128 - crafted.numel() % 128)])
        rnd = torch.rand(128 * 6, generator=gen) ** 3
        if signed:
            rnd = rnd * torch.sign(torch.randn(rnd.numel(), generator=gen))
        # exact levels (block scale 1), and a constant block small enough that the fp32
        # preconditioner 1/(sqrt(s*level/bias)+eps) is flat across neighbouring levels
        blocks = [crafted * 0.37, rnd * 3.0e-3, torch.zeros(128), rnd[:128] * 1e-30,
                  torch.full((128,), 2.5e-7), cb.repeat(8), torch.full((128,), 1e-32),
                  cb.abs().repeat(8) * 1e-33]
        values = torch.cat(blocks).float()
        update_sr = "upd_sr" in mode or "lookahead" in mode
        # With a large eps the fp32 preconditioner of neighbouring levels can coincide;
        # the endpoint guards then decide exact-level writes.
        variants = [(False, 1e-8), (True, 1e-8)] + ([(False, 1e3)] if update_sr else [])
        for eden, eps in variants:
            if eden and mode in ("lin4_sr", "dyn4_sr"):
                continue
            vals = values if eps < 1 else torch.cat([values, torch.full((128,), 1e-10)])
            draws = torch.rand((vals.numel() // 128, 128), generator=gen)
            stochastic = mode.endswith("_sr") or update_sr
            kwargs = dict(block_size=128, mode=mode, eden_correction=eden)
            if stochastic:
                kwargs.update(draws=draws, bias_correction=0.0975, eps=eps)
            codes, meta = oq.quantize(vals, **kwargs)
            key = f"{mode}_{'eden' if eden else 'plain'}" + ("_flat" if eps > 1 else "")
            values_out = vals
            out[f"{key}_values"] = values_out.numpy().copy()
            out[f"{key}_draws"] = draws.numpy().copy()
            out[f"{key}_codes"] = codes.numpy().copy()
            out[f"{key}_scales"] = meta.absmax.numpy().copy()
            entries.append(dict(key=key, mode=mode, eden=eden, stochastic=stochastic,
                                bias=0.0975, eps=eps))
    out["config"] = np.array(json.dumps(entries))
    np.savez_compressed(os.path.join(HERE, "codec_vectors.npz"), **out)
    print("wrote codec_vectors")


def checkpoint_case():
    """A reference state_dict after two ZIP-SR steps, saved with torch.save."""
    gen = torch.Generator().manual_seed(99)
    p = torch.nn.Parameter(torch.randn(64, 128, generator=gen) * 0.02)
    q = torch.nn.Parameter(torch.randn(768, generator=gen) * 0.02)
    opt = ZIPSRAdamW4Bit([p, q], quant_rng_seed=11, optimized=True, **HP)
    for _ in range(2):
        p.grad = heavy_tailed((64, 128), gen)
        q.grad = heavy_tailed((768,), gen)
        opt.step()
    sd = opt.state_dict()
    torch.save(sd, os.path.join(HERE, "zipsr_state_dict.pt"))
    torch.save({"p": p.detach().clone(), "q": q.detach().clone()},
               os.path.join(HERE, "zipsr_state_dict_params.pt"))
    print("wrote checkpoint", sorted(sd["state"][0].keys()), sd["_quant_rng_state"]["version"])


def main():
    torch.set_num_threads(4)
    print("reference:", adamw4bit.__file__)
    trajectory("zeeden_f32", recipe(ZEEDENAdamW4Bit), [(32, 128)], "float32", 6,
               grad_seed=1, snap_steps={1, 6})
    trajectory("zipsr_f32_seed0", recipe(ZIPSRAdamW4Bit, seed=0), [(32, 128)], "float32", 6,
               grad_seed=2, snap_steps={1, 6})
    trajectory("zipsr_bf16_nf4sr", recipe(ZIPSRAdamW4Bit, seed=43), [(4096,)], "bfloat16", 5,
               grad_seed=3, snap_steps={5}, m1_override=([0], "nf4_sr"))
    trajectory("zeeden_f16", recipe(ZEEDENAdamW4Bit), [(4096,)], "float16", 4,
               grad_seed=4, snap_steps={4})
    trajectory("zeeden_multi", recipe(ZEEDENAdamW4Bit), [(4096,), (768,), (4097,), (32, 256)],
               "float32", 3, grad_seed=5, snap_steps={3})
    trajectory("ablation_groups",
               grouped([("sdyn4_sr", "lin4_sr", False), ("fp32", "dyn4", True),
                        ("nf4", "lin4_nz", True), ("nf4", "dyn4_lookahead_sr", True),
                        ("nf4", "fp32", False), ("nf4_sr", "dyn4_upd_sr_fp32read", True),
                        ("sdyn4", "dyn4_sr", False), ("nf4", "lin4_upd_sr_fp32read", False)],
                       seed=7),
               [(4096,)] * 8, "float32", 3, grad_seed=6, snap_steps={3}, zero_block_frac=0.05)
    trajectory("zipsr_chunked", recipe(ZIPSRAdamW4Bit, seed=5, chunk=1024), [(8192,), (512,)],
               "float32", 4, grad_seed=7, snap_steps={4}, m1_override=([0], "nf4_sr"))
    trajectory("refstep_zipsr", recipe(ZIPSRAdamW4Bit, optimized=False, seed=0), [(32, 128)],
               "float32", 5, grad_seed=8, snap_steps={5}, m1_override=([0], "nf4_sr"))
    trajectory("refstep_zeeden_bf16", recipe(ZEEDENAdamW4Bit, optimized=False), [(4096,)],
               "bfloat16", 4, grad_seed=9, snap_steps={4})
    trajectory("sampled_read_groups",
               grouped([("nf4", "dyn4_upd_sr", False), ("nf4_sr", "lin4_upd_sr", True),
                        ("fp32", "dyn4_upd_sr_store_eden", False), ("sdyn4", "lin4_upd_sr_store_eden", False),
                        ("nf4", "dyn4_upd_sr", True)],
                       seed=11),
               [(4096,)] * 4 + [(64, 128)], "float32", 3, grad_seed=10, snap_steps={1, 3}, zero_block_frac=0.05)
    trajectory("sampled_read_bf16", grouped([("nf4", "dyn4_upd_sr_store_eden", False)], seed=12), [(4096,)],
               "bfloat16", 3, grad_seed=11, snap_steps={3})
    trajectory("lookahead_groups",
               grouped([("nf4", "dyn4_la_upd_sr", False), ("fp32", "dyn4_proxy_la_upd_sr", False),
                        ("nf4", "dyn4_vproxy_la_upd_sr", False), ("fp32", "dyn4_la_upd_sr", False),
                        ("nf4", "dyn4_proxy_la_upd_sr", False)],
                       seed=13),
               [(4096,)] * 4 + [(64, 128)], "float32", 3, grad_seed=12, snap_steps={1, 3}, zero_block_frac=0.05)
    trajectory("lookahead_bf16",
               grouped([("nf4", "dyn4_vproxy_la_upd_sr", False), ("nf4", "dyn4_la_upd_sr", False)], seed=14),
               [(4096,), (4096,)], "bfloat16", 3, grad_seed=13, snap_steps={3})
    # gradients near 1e-8: sqrt(m2 / bias) comparable to eps, so the bias corrections matter
    trajectory("lookahead_small_grad",
               grouped([("fp32", "dyn4_la_upd_sr", False), ("fp32", "dyn4_proxy_la_upd_sr", False),
                        ("fp32", "dyn4_vproxy_la_upd_sr", False)], seed=15),
               [(4096,)] * 3, "float32", 4, grad_seed=14, snap_steps={4}, grad_mu=-18.0)
    codec_cases()
    checkpoint_case()


if __name__ == "__main__":
    main()
