"""Build the HIP library ``libadamw4bit_hip.so`` in-tree for gfx950.

``python -m adamw4bit_amd.build`` compiles ``csrc/fused_step.hip`` with hipcc
(no GPU needed: hipcc cross-compiles for ``--offload-arch=gfx950``).  The
library lands next to this file so it travels with the source tree.

Flags that are part of the numerical contract:
  -ffp-contract=off   no implicit multiply-add fusion; the kernel writes each
                      fused multiply-add the reference's ATen kernels perform
                      explicitly (lerp) and nothing else.
  (defaults kept)     correctly rounded fp32 division and sqrt, fp32 denormals on.
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      keep scalar fp32 VALU ops (no packed fp32 instructions).  The
                      host pass prints that it does not know the feature and ignores
                      it: clang's -Xarch_device forwards no -Xclang option, so the flag
                      reaches both passes (tests/test_device_code_rules.py checks that
                      the device code has no packed fp32 instruction).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCE = os.path.join(HERE, "csrc", "fused_step.hip")
INCLUDE = os.path.join(ROOT, "include")
LIBRARY = os.path.join(HERE, "libadamw4bit_hip.so")
ARCH = os.environ.get("AW4_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and os.path.exists(candidate):
            return candidate
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def command(output: str = LIBRARY, extra=()) -> list:
    return [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-function",
        f"-I{INCLUDE}", f"-I{os.path.dirname(SOURCE)}", SOURCE, "-o", output, *extra,
    ]


def build(verbose: bool = False) -> str:
    """Compile the library (always) and return its path."""
    tmp = LIBRARY + ".tmp"
    cmd = command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
