"""The CPU oracle reproduces the reference bit for bit on its golden trajectories and codec vectors.

Fixtures come from ``tests/golden/make_golden.py``, which runs the reference
implementation itself; here only the oracle runs.
"""

import numpy as np
import pytest
import torch

from oracle import reference_step as ref
from tests._fixtures import bits, load, tensor, trajectory_names


def run_oracle(cfg, arrays, record_draws=False):
    dtype = cfg["dtype"]
    n_params = len(cfg["shapes"])
    params = [tensor(arrays[f"init_p{i}"], dtype).clone().reshape(cfg["shapes"][i])
              for i in range(n_params)]
    per = cfg["per_param"]
    m1 = [e["m1"] for e in per]
    if cfg.get("m1_override"):
        idx, scheme = cfg["m1_override"]
        for j in idx:
            m1[j] = scheme
    hp = cfg["hyper"]
    oracle = ref.Oracle(params, ref.Hyper(hp["lr"], tuple(hp["betas"]), hp["eps"], hp["weight_decay"]),
                        m1, [e["m2"] for e in per], [e["eden"] for e in per], seed=cfg["seed"],
                        optimized=cfg["optimized"], chunk=cfg["chunk"], record_draws=record_draws)
    snaps = {}
    for k in range(cfg["steps"]):
        grads = [tensor(arrays[f"grad_s{k}_p{i}"], dtype).reshape(cfg["shapes"][i]) for i in range(n_params)]
        if cfg["seed"] is None:
            torch.manual_seed(0)  # no stochastic scheme draws from the global stream in these cases
        oracle.step(grads)
        if (k + 1) in cfg["snap_steps"]:
            snaps[k + 1] = [(p.clone(), _copy_state(st)) for p, st in zip(params, oracle.states)]
    return oracle, snaps


def _copy_state(st):
    out = {"step": st.step}
    for name in ("m1", "m2"):
        ms = getattr(st, name)
        if ms.scheme == "fp32":
            out[f"{name}_fp32"] = ms.values.clone()
        elif ms.scheme in ref.PENDING_LOOKAHEAD_SCHEMES:
            out[f"{name}_pending"] = ms.values.clone()
        else:
            out[f"{name}_code"] = ms.codes.clone()
            out[f"{name}_scale"] = ms.scales.clone()
    if st.read_preconditioner is not None:
        out["m2_pre"] = st.read_preconditioner.clone()
    return out


@pytest.mark.parametrize("name", trajectory_names())
def test_oracle_matches_reference_trajectory(name):
    cfg, arrays = load(name)
    _, snaps = run_oracle(cfg, arrays)
    for step, entries in snaps.items():
        for i, (p, st) in enumerate(entries):
            prefix = f"after{step}_p{i}"
            expect_p = tensor(arrays[prefix], cfg["dtype"]).reshape(p.shape)
            assert torch.equal(bits(p), bits(expect_p)), f"{name} step {step} param {i}"
            assert st["step"] == int(arrays[f"{prefix}_step"])
            for key in ("m1_code", "m2_code", "m1_scale", "m2_scale", "m1_fp32", "m2_fp32", "m2_pre", "m2_pending"):
                if f"{prefix}_{key}" in arrays:
                    expect = torch.from_numpy(arrays[f"{prefix}_{key}"])
                    assert key in st, f"{name}: oracle state lacks {key} for param {i}"
                    assert torch.equal(bits(st[key]), bits(expect)), f"{name} step {step} {key} p{i}"
                else:
                    assert key not in st


def test_codec_vectors():
    entries, arrays = load("codec_vectors.npz")
    assert len(entries) >= 20
    for e in entries:
        k = e["key"]
        values = torch.from_numpy(arrays[f"{k}_values"])
        draws = torch.from_numpy(arrays[f"{k}_draws"]) if e["stochastic"] else None
        codes, scales = ref.encode(values, e["mode"], eden=e["eden"], draws=draws, bias=e["bias"],
                                   eps=e["eps"])
        assert np.array_equal(codes.numpy(), arrays[f"{k}_codes"]), k
        assert torch.equal(bits(scales), bits(torch.from_numpy(arrays[f"{k}_scales"]))), k
