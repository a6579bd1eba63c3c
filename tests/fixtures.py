"""Seeded inputs shared by the tests: the reference's convolution cases (tests/golden/conv_cases.json,
restating tests/cuda_fixtures.py:6-26 of the reference) and its inputs convention."""

import json
from pathlib import Path

import numpy as np

_GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "conv_cases.json").read_text())
CONV_CASES = tuple((c[0], tuple(c[1]), tuple(c[2]), tuple(c[3]), tuple(c[4])) for c in _GOLDEN["conv_cases"])
PERFORMANCE_CASES = tuple((c[0], tuple(c[1]), tuple(c[2]), tuple(c[3]), tuple(c[4])) for c in _GOLDEN["performance_cases"])
POOL_CASES = tuple((tuple(c[0]), tuple(c[1]), tuple(c[2]), tuple(c[3])) for c in _GOLDEN["pool_cases"])
EPS32 = float(np.finfo(np.float32).eps)


def conv_fixture(case, seed=0):
    """x, w, b, dy as float32 from default_rng(seed).normal in that order; T0 is arange(25) (*) ones."""
    name, x_shape, w_shape, stride, padding = case
    rng = np.random.default_rng(seed)
    out = (x_shape[0], w_shape[0], (x_shape[2] + 2 * padding[0] - w_shape[2]) // stride[0] + 1,
           (x_shape[3] + 2 * padding[1] - w_shape[3]) // stride[1] + 1)
    arrays = [rng.normal(size=s).astype(np.float32) for s in (x_shape, w_shape, (w_shape[0],), out)]
    if name == "T0":
        arrays[0] = np.arange(25, dtype=np.float32).reshape(x_shape)
        arrays[1] = np.ones(w_shape, dtype=np.float32)
        arrays[2] = np.zeros(w_shape[0], dtype=np.float32)
    return arrays


def assert_near(actual, expected, rel, name):
    """max |actual - expected| <= rel * max |expected| (the reference's _assert_near)."""
    actual = np.asarray(actual, dtype=np.float64)
    scale = max(float(np.abs(expected).max()), 1e-30)
    error = float(np.abs(actual - expected).max())
    assert error <= rel * scale, f"{name}: max error {error:.3e} > {rel:.1e} x {scale:.3e}"


def gamma_k(k):
    """Classical worst-case bound factor of a k-term FP32 dot product."""
    u = EPS32 / 2
    return k * u / (1 - k * u)
