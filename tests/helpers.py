"""Seeded synthetic inputs and comparison rules shared by the tests."""
from __future__ import annotations

import numpy as np

# Attention tolerance of the north star: max-abs 2e-3 and relative 1e-2
# (relative = ||a - b||_2 / ||b||_2) against the fp32 oracle.
ATOL = 2e-3
RTOL = 1e-2


def randn_f16(rng: np.random.Generator, shape) -> np.ndarray:
    """N(0, 1) drawn in float64, rounded to fp32, then to fp16 (round-to-nearest-even)."""
    return rng.standard_normal(shape).astype(np.float32).astype(np.float16)


def assert_attention_close(actual: np.ndarray, expected: np.ndarray, what: str = "") -> None:
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    assert np.all(np.isfinite(actual)), f"{what}: non-finite output"
    err = np.abs(actual - expected)
    max_abs = float(err.max()) if err.size else 0.0
    denom = float(np.linalg.norm(expected))
    rel = float(np.linalg.norm(actual - expected)) / denom if denom > 0 else max_abs
    assert max_abs <= ATOL and rel <= RTOL, f"{what}: max_abs={max_abs:.3e} rel={rel:.3e}"


def attention_errors(actual, expected):
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    err = np.abs(actual - expected)
    denom = float(np.linalg.norm(expected))
    return float(err.max()), float(np.linalg.norm(actual - expected)) / max(denom, 1e-30)
