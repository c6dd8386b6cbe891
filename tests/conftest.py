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


def allclose_fraction(actual, expected, rel=1e-3, abs_=1e-5):
    """Fraction of elements with |a - e| <= abs_ + rel |e| (numpy.allclose's test, per element),
    reported beside the peak-relative bar."""
    import numpy as np
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    if a.shape != e.shape or a.size == 0:
        return 0.0 if a.shape != e.shape else 1.0
    return float(np.mean(np.abs(a - e) <= abs_ + rel * np.abs(e)))


def assert_close(got, ref, what, rel=1e-3, abs_=1e-5):
    """The float bar of every GPU parity test (peak-relative, per tensor); the message also
    gives the elementwise allclose(rel, abs_) pass fraction."""
    ok, frac = tolerance_ok(got, ref, rel, abs_)
    assert ok, (f"{what}: max|err|/peak = {frac:.3e}, elementwise allclose({rel:g}, {abs_:g}) pass fraction "
                f"{allclose_fraction(got, ref, rel, abs_):.5f}")


def check_margin_ids(logits_gpu, ids_gpu, logits_ref, margin):
    """ids equal the margin rule on the kernel's own logits, and the fp64 oracle's id unless
    a logit sits within rounding of the threshold."""
    import numpy as np
    import oracle as orc
    for b in range(logits_gpu.shape[0]):
        # the kernel's id is exactly the margin rule applied to its own logits
        assert int(ids_gpu[b]) == orc.argmax_margin_f32(logits_gpu[b], margin), b
        # and the oracle's id, unless a logit sits within rounding of the threshold
        ref = logits_ref[b]
        M = ref.max()
        T = M - margin * abs(M)
        ambiguous = np.any(np.abs(ref - T) <= 1e-5 * max(1.0, abs(M)))
        if not ambiguous:
            assert int(ids_gpu[b]) == orc.argmax_margin_f64(ref, margin), b
