"""Shared pytest setup: repo root on sys.path, the `gpu` marker, GPU helpers."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built libt2h.so")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from torch2vk_amd import _lib

    _lib.lib()  # fail loudly if the library is missing
    return torch.device("cuda:0")


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.linalg.norm(a) * np.linalg.norm(b)
    return float(a @ b / den) if den > 0 else float(np.array_equal(a, b))


def assert_close(got, ref, *, max_abs: float, min_cos: float = 0.999, what: str = "") -> None:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} != {ref.shape}"
    err = float(np.abs(got - ref).max()) if got.size else 0.0
    cos = cosine(got, ref)
    assert err <= max_abs, f"{what}: max-abs error {err:.3e} > {max_abs:.3e} (cos {cos:.6f})"
    assert cos >= min_cos, f"{what}: cosine {cos:.6f} < {min_cos}"
