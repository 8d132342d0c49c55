import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this process")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_sessionfinish(session, exitstatus):
    """With ATLAS_PARITY_REPORT=<path>, write every parity comparison's normwise relative error
    (name, error, tolerance) there: the margin behind each passing check."""
    path = os.environ.get("ATLAS_PARITY_REPORT")
    if not path:
        return
    try:
        from _cases import NORMWISE
    except Exception:  # pragma: no cover
        return
    if not NORMWISE:
        return
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "w") as f:
        f.write("# name  normwise_rel_err  tol  margin(tol/err)\n")
        for name, err, tol in NORMWISE:
            margin = tol / err if err > 0 else float("inf")
            f.write(f"{name}\t{err:.3e}\t{tol:g}\t{margin:.1f}\n")
