import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


def has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session", autouse=True)
def per_op_workspace():
    """The host-created scratch the per-op entry points draw from (the
    reference's host owns its kernels' buffers the same way), bound to the
    default stream the per-op tests launch on."""
    if not has_gpu():
        yield None
        return
    from autoresearch_amd import ops
    ws = ops.Workspace(3 << 30).bind()
    yield ws
    ws.close()


def pytest_collection_modifyitems(config, items):
    if has_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


def rel_err(a, b) -> float:
    """Norm-wise relative error ||a - b||_2 / ||b||_2 (0 when both are 0)."""
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    nb = np.linalg.norm(b)
    d = np.linalg.norm(a - b)
    if nb == 0.0:
        return float(d)
    return float(d / nb)


# Tolerances: fp32 rel-err <= 1e-5, bf16 <= 2e-2,
# bit-exact for gather / scatter / indexing.
TOL_FP32 = 1e-5
TOL_BF16 = 2e-2
