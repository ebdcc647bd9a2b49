"""Shared test setup: import paths, the `gpu` marker and small helpers."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "npu-flex-att_amd")
for path in (ROOT, PKG):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built libflexatt.so")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def pytest_sessionfinish(session, exitstatus):
    """Write the parity errors the GPU tests measured (gpu_helpers.RECORDS)
    as JSON lines to $FLEXATT_PARITY_LOG, or to parity_errors.jsonl in the
    repository's GPU-run output folder when that folder exists."""
    mod = sys.modules.get("gpu_helpers")
    recs = getattr(mod, "RECORDS", None)
    if not recs:
        return
    path = os.environ.get("FLEXATT_PARITY_LOG")
    if not path:
        out = os.path.join(ROOT, "gpurun_out")
        if not os.path.isdir(out):
            return
        path = os.path.join(out, "parity_errors.jsonl")
    import json

    with open(path, "w") as f:
        for r in recs:
            f.write(json.dumps(r) + "\n")
