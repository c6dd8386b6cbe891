import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "ray-tracing-attention_amd", ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and librta.so")


def _has_gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def tolerance_ok(actual, expected, rel=1e-3, abs_=1e-5):
    """Peak-relative criterion: max|a - e| <= abs_ + rel * max|e| (per output tensor)."""
    import numpy as np
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    if a.shape != e.shape or not np.isfinite(a).all():
        return False, float("inf")
    err = float(np.max(np.abs(a - e), initial=0.0))
    peak = float(np.max(np.abs(e), initial=0.0))
    return err <= abs_ + rel * peak, err / max(peak, 1e-30)
