import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built library")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(0)


def pytest_sessionfinish(session, exitstatus):
    """Write the measured parity errors next to the GPU run's other outputs."""
    from tests._util import RECORDS
    out_dir = os.path.join(ROOT, "gpurun_out")
    if RECORDS and torch.cuda.is_available() and os.path.isdir(out_dir):
        import json
        with open(os.path.join(out_dir, "parity_errors.json"), "w") as f:
            json.dump(RECORDS, f, indent=1)
