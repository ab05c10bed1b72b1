import os
import subprocess
import sys
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    # GPU tests are selected explicitly with ``-m gpu``; without a device they are skipped
    # rather than silently passing on a CPU path.
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def device_assembly():
    """The gfx950 assembly of the library's own source, both of its objects, compiled here with
    the library's flags (hipcc cross-compiles; no GPU needed).  One compile serves every test of
    the session."""
    from adamw4bit_amd import build

    hipcc = build.hipcc()
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as tmp:
        text = []
        for cmd, out in build.assembly_commands(tmp):
            proc = subprocess.run(cmd, capture_output=True, text=True)
            assert proc.returncode == 0, proc.stderr[-2000:]
            with open(out) as f:
                text.append(f.read())
        return "\n".join(text)
