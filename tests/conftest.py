"""pytest configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs on a CPU-only host (oracle, host logic, C-ABI surface);
``-m gpu`` runs the HIP parity tests and needs a gfx950 device.
"""

import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT / "geometric-nn-ops_amd", ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP (gfx950) device")
    config.addinivalue_line("markers", "large: large-N tests (minutes of CPU oracle time)")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="needs a HIP device")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
