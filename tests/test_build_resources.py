"""Register budgets of the specialised step kernels, read from the gfx950 assembly of the
library's own source (compiled here with the library's flags; no GPU needed).

Waves per SIMD follow from the VGPR count (512 per lane per SIMD, allocated in steps of
8): 128 or fewer VGPRs run 4 waves.  The memory-bound kernels are latency bound at their
occupancy, and small source changes can make hipcc copy the prefetched tile registers
instead of coalescing them (about 40 VGPRs), so each kernel's occupancy is pinned here.
"""

import re

import pytest

# (m1 spec, m2 spec, dtype) template arguments -> minimum waves per SIMD
# m1: 1 = NF4 round-to-nearest, 66 = value-space SR with guards;
# m2: 33 = round-to-nearest + EDEN, 67 = update-SR with guards, 99 = update-SR + EDEN, 0 = fp32,
# 259 = update-SR read back after its encode, 803 = the same with the store-EDEN flags,
# 4 = lookahead update-SR stored as codes, 2052 = the pending lookahead form (fp32 state);
# dtype: 0 = fp32, 1 = bf16.
MIN_WAVES = {
    (1, 33, 0): 4, (1, 67, 0): 4, (1, 33, 1): 4, (1, 67, 1): 4, (66, 67, 0): 3, (66, 67, 1): 4,
    (1, 0, 0): 4, (1, 0, 1): 4, (1, 99, 0): 3, (1, 99, 1): 3, (1, 259, 0): 3, (1, 803, 0): 2,
    (1, 4, 0): 3, (1, 2052, 0): 3,
}
# Kernels held to an occupancy with a few spilled registers (the occupancy pays for them).
SPILL_LIMIT = {(1, 2052, 0): 8}
# The generic research instance (any m1, any read-back or lookahead m2, run-time dtypes) is held to
# two waves per SIMD (235 VGPRs, no spills).
RESEARCH_GENERIC, RESEARCH_SPILL_LIMIT = (7, 263, 7), 0


def waves_per_simd(vgprs: int) -> int:
    granule = (vgprs + 7) // 8 * 8
    return min(8, 512 // granule)


@pytest.fixture(scope="module")
def kernel_vgprs(device_assembly):
    # one metadata section per object of the library
    metas = device_assembly.split("amdhsa.kernels")[1:]
    assert metas, "no kernel metadata"
    found = {}
    for block in (b for meta in metas for b in re.split(r"\n  - \.", meta)):
        name = re.search(r"\.name:\s+(\S+)", block)
        if not name or "step_kernel" not in name.group(1):
            continue
        # a kernel taking its launch table in its arguments (step_kernel_inline*) counts with the
        # regular instance of the same moment specs and dtype: the worse of the two
        args = re.search(r"step_kernel(?:_inline)?(?:_[234]w)?ILi(\d+)ELi(\d+)ELi(\d+)E", name.group(1))
        vgpr = re.search(r"\.vgpr_count:\s+(\d+)", block)
        spill = re.search(r"\.vgpr_spill_count:\s+(\d+)", block)
        key = tuple(int(x) for x in args.groups())
        this = (int(vgpr.group(1)), int(spill.group(1)))
        found[key] = tuple(map(max, found.get(key, this), this))
        if "step_kernel_inline" in name.group(1):
            INLINE_FOUND.add(key)
    return found


INLINE_FOUND = set()
# The recipes' kernels (ZE-EDEN and ZIP-SR, fp32 and bf16) have instances for small steps.
INLINE_EXPECTED = {(1, 33, 0), (1, 67, 0), (1, 33, 1), (1, 67, 1)}


def test_small_step_instances_exist(kernel_vgprs):
    assert INLINE_FOUND == INLINE_EXPECTED, INLINE_FOUND


def test_specialised_kernels_keep_their_occupancy(kernel_vgprs):
    for key, waves in MIN_WAVES.items():
        assert key in kernel_vgprs, f"kernel {key} not instantiated"
        vgprs, spills = kernel_vgprs[key]
        assert spills <= SPILL_LIMIT.get(key, 0), f"kernel {key} spills {spills} VGPRs"
        assert waves_per_simd(vgprs) >= waves, f"kernel {key}: {vgprs} VGPRs -> {waves_per_simd(vgprs)} waves < {waves}"


def test_generic_kernels_do_not_spill(kernel_vgprs):
    generic = [k for k in kernel_vgprs if k not in MIN_WAVES]
    assert generic and RESEARCH_GENERIC in generic, "generic kernels not found"
    for key in generic:
        vgprs, spills = kernel_vgprs[key]
        if key == RESEARCH_GENERIC:
            assert waves_per_simd(vgprs) >= 2 and spills <= RESEARCH_SPILL_LIMIT, (key, vgprs, spills)
        else:
            assert spills == 0, f"kernel {key} spills"


def test_no_flat_memory_instructions(device_assembly):
    """Every memory access of the library's device code names its address space: global_* for
    device memory and ds_* for LDS.  A flat instruction would wait on the LDS counter for
    outstanding global traffic, and an LDS index out of its object would address global memory
    instead of being dropped at the LDS bound (views of LDS handed through a function the
    compiler keeps out of line turn generic)."""
    fn = None
    found = {}
    for line in device_assembly.split("\n"):
        m = re.match(r"^(_Z\S+):", line)
        if m:
            fn = m.group(1)
            continue
        if re.match(r"\s+flat_(load|store|atomic)", line):
            found[fn] = found.get(fn, 0) + 1
    assert not found, found
