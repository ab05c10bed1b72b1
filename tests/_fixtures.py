"""Loading helpers for the golden fixtures written by ``tests/golden/make_golden.py``."""

from __future__ import annotations

import glob
import json
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DTYPES = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


def load(name: str):
    data = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    arrays = {k: data[k] for k in data.files if k != "config"}
    return json.loads(str(data["config"])), arrays


def trajectory_names():
    return sorted(os.path.basename(p) for p in glob.glob(os.path.join(GOLDEN, "traj_*.npz")))


def tensor(arr: np.ndarray, dtype: str) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(arr))
    if dtype in ("bfloat16", "float16"):
        return t.view(DTYPES[dtype])
    return t


def bits(t: torch.Tensor) -> torch.Tensor:
    """Integer view for bit-exact comparisons (NaN-safe)."""
    t = t.detach().cpu().contiguous()
    return t.view({4: torch.int32, 2: torch.int16, 1: torch.uint8, 8: torch.int64}[t.element_size()])
