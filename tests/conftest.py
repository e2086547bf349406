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
    """fp32 parity bar against the reference CPU JIT, whichever rounding chain
    it takes: `ref` is an oracle.F32Chains holding the result on the fma chain
    and on the mulf+addf chain. Each element's deviation is the larger of its
    deviations from the two, so the bar holds against either chain and against
    any per-element mix of them. Bar: relative Frobenius error <= 1e-5 and
    max|delta| <= 1e-4 * sqrt(K); NaN and inf positions must agree."""
    import oracle
    assert isinstance(ref, oracle.F32Chains), "an f32 result is checked against both oracle chains"
    got = np.asarray(got, dtype=np.float64)
    refs = [np.asarray(r, dtype=np.float64) for r in ref]
    worst = None
    norm = None
    for r in refs:
        assert got.shape == r.shape, (got.shape, r.shape)
        gn, rn = np.isnan(got), np.isnan(r)
        assert np.array_equal(gn, rn), f"NaN positions differ: {np.argwhere(gn != rn)[:5]}"
        finite = ~rn
        ginf, rinf = np.isinf(got) & finite, np.isinf(r) & finite
        assert np.array_equal(ginf, rinf) and np.array_equal(got[rinf], r[rinf]), "inf mismatch"
        mask = finite & ~rinf
        d = np.abs(got[mask] - r[mask])
        worst = d if worst is None else np.maximum(worst, d)
        n = float(np.linalg.norm(r[mask]))
        norm = n if norm is None else min(norm, n)
    max_abs = float(np.max(worst)) if worst.size else 0.0
    assert max_abs <= abs_scale * np.sqrt(max(K, 1)), f"max|delta|={max_abs:g} > {abs_scale}*sqrt({K})"
    if norm > 0:
        rel = float(np.linalg.norm(worst)) / norm
        assert rel <= rel_fro, f"relative Frobenius error {rel:g} > {rel_fro:g}"


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    oracle.lib()
    return oracle
