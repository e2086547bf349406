"""Shared test setup: import paths, the `gpu` marker, parity helpers."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "ml-edsl_amd")
for p in (ROOT, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs through the C ABI")


def _gpu_present() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_present():
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def assert_f32_parity(got, ref, K: int, rel_fro: float = 1e-5, abs_scale: float = 1e-4):
    """fp32 parity bar: relative Frobenius error <= 1e-5 and
    max|delta| <= 1e-4 * sqrt(K); NaN positions must agree."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    gn, rn = np.isnan(got), np.isnan(ref)
    assert np.array_equal(gn, rn), f"NaN positions differ: {np.argwhere(gn != rn)[:5]}"
    finite = ~rn
    ginf, rinf = np.isinf(got) & finite, np.isinf(ref) & finite
    assert np.array_equal(ginf, rinf) and np.array_equal(got[rinf], ref[rinf]), "inf mismatch"
    mask = finite & ~rinf
    d = got[mask] - ref[mask]
    max_abs = float(np.max(np.abs(d))) if d.size else 0.0
    assert max_abs <= abs_scale * np.sqrt(max(K, 1)), f"max|delta|={max_abs:g} > {abs_scale}*sqrt({K})"
    rn2 = float(np.linalg.norm(ref[mask]))
    if rn2 > 0:
        rel = float(np.linalg.norm(d)) / rn2
        assert rel <= rel_fro, f"relative Frobenius error {rel:g} > {rel_fro:g}"


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    oracle.lib()
    return oracle
