"""Build the HIP library ``libadamw4bit_hip.so`` in-tree for gfx950.

``python -m adamw4bit_amd.build`` compiles ``csrc/fused_step.hip`` with hipcc
(no GPU needed: hipcc cross-compiles for ``--offload-arch=gfx950``) twice: the
main object, and one with ``AW4_SCHED_ILP_TU`` that holds only the four-wave
update-SR kernels, scheduled by LLVM's max-ilp strategy; one link makes the
library.  It lands next to this file so it travels with the source tree.

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
import tempfile

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


# The second object: the same source with AW4_SCHED_ILP_TU, which emits only the four-wave
# update-SR kernels, scheduled by LLVM's max-ilp strategy (the source says why).
ILP_FLAGS = ("-DAW4_SCHED_ILP_TU", "-mllvm", "-amdgpu-sched-strategy=max-ilp")


def compile_command(output: str, ilp: bool = False, extra=()) -> list:
    """hipcc line for one object of the library (the main one, or with ilp the second)."""
    return [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-function",
        f"-I{INCLUDE}", f"-I{os.path.dirname(SOURCE)}", *(ILP_FLAGS if ilp else ()),
        # a fixed compile-unit id per object (clang derives one from the output path otherwise,
        # a temporary directory's), so that a rebuild gives the same library byte for byte
        f"-cuid=adamw4bit_{'ilp' if ilp else 'main'}",
        "-c", SOURCE, "-o", output, *extra,
    ]


def link_command(objects, output: str) -> list:
    return [hipcc(), "-shared", "-fPIC", *objects, "-o", output]


def assembly_commands(directory: str) -> list:
    """(hipcc line, output path) for the gfx950 assembly of both objects' device code."""
    out = []
    for ilp in (False, True):
        path = os.path.join(directory, "fused_step_ilp.s" if ilp else "fused_step.s")
        cmd = [a for a in compile_command(path, ilp) if a not in ("-fPIC", "-c")] + ["--cuda-device-only", "-S"]
        out.append((cmd, path))
    return out


def _run(cmds, verbose: bool) -> None:
    procs = []
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append(subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
    failed = None
    for proc in procs:
        out, err = proc.communicate()
        if proc.returncode != 0 and failed is None:
            sys.stderr.write(out + err)
            failed = proc.returncode
    if failed is not None:
        raise RuntimeError(f"hipcc failed with exit code {failed}")


def build(verbose: bool = False) -> str:
    """Compile the library (always) and return its path: two objects in parallel, then one link."""
    with tempfile.TemporaryDirectory() as tmpdir:
        objects = [os.path.join(tmpdir, "fused_step.o"), os.path.join(tmpdir, "fused_step_ilp.o")]
        _run([compile_command(objects[0]), compile_command(objects[1], ilp=True)], verbose)
        tmp = LIBRARY + ".tmp"
        _run([link_command(objects, tmp)], verbose)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
