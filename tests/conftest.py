"""Shared test configuration. GPU tests carry @pytest.mark.gpu and run through the C ABI."""
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libmnn.so")


def close_report(got, ref, atol, rtol):
    """(ok, max_abs, max_rel) under |got - ref| <= atol + rtol * |ref| per element, the
    closeness rule of the reference's ReferenceTestUtils.swift:141-179."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, f"shape {got.shape} != {ref.shape}"
    err = np.abs(got - ref)
    ok = bool(np.all(err <= atol + rtol * np.abs(ref))) and bool(np.all(np.isfinite(got)))
    max_abs = float(err.max()) if err.size else 0.0
    max_rel = float((err / np.maximum(np.abs(ref), 1e-30)).max()) if err.size else 0.0
    return ok, max_abs, max_rel


def assert_close(got, ref, atol=1e-4, rtol=1e-3, what=""):
    ok, ma, mr = close_report(got, ref, atol, rtol)
    assert ok, f"{what}: max abs {ma:.3e}, max rel {mr:.3e} (atol {atol}, rtol {rtol})"
    return ma


def assert_rel_norm(got, ref, rtol, what=""):
    """bf16 bar: max |got - ref| <= rtol * max |ref| (normwise relative error)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = float(np.abs(got - ref).max())
    scale = float(np.abs(ref).max())
    assert np.all(np.isfinite(got)) and err <= rtol * scale, \
        f"{what}: max abs {err:.3e} vs {rtol} * {scale:.3e}"
    return err / scale


@pytest.fixture(scope="session")
def golden_dir():
    return ROOT / "tests" / "golden"
