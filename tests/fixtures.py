"""Seeded inputs shared by the tests.

The convolution cases are the reference's (tests/golden/conv_cases.json restates
tests/cuda_fixtures.py:6-26 and tests/test_cuda_native_kernels.py:20-24 of the reference), and so is
their input convention: one default_rng(seed) stream, normal draws for x, then the weight, then the
bias, then dy, each cast to float32; case T0 replaces x, w, b by the known-answer arange(25) and
ones(3x3) with a zero bias.
"""

import json
from pathlib import Path

import numpy as np

_CASES = json.loads((Path(__file__).resolve().parent / "golden" / "conv_cases.json").read_text())


def _case(row):
    name, x_shape, w_shape, stride, padding = row
    return name, tuple(x_shape), tuple(w_shape), tuple(stride), tuple(padding)


CONV_CASES = tuple(_case(row) for row in _CASES["conv_cases"])
PERFORMANCE_CASES = tuple(_case(row) for row in _CASES["performance_cases"])
POOL_CASES = tuple(tuple(tuple(part) for part in row) for row in _CASES["pool_cases"])
EPS32 = float(np.finfo(np.float32).eps)


def conv_output_shape(case):
    _, (n, _, h, w), (co, _, kh, kw), (sh, sw), (ph, pw) = case
    return n, co, (h + 2 * ph - kh) // sh + 1, (w + 2 * pw - kw) // sw + 1


def conv_fixture(case, seed=0):
    """(x, w, b, dy) float32 arrays of a convolution case."""
    generator = np.random.default_rng(seed)
    shapes = (case[1], case[2], (case[2][0],), conv_output_shape(case))
    x, w, b, dy = (generator.normal(size=shape).astype(np.float32) for shape in shapes)
    if case[0] == "T0":
        x = np.arange(25, dtype=np.float32).reshape(case[1])
        w = np.ones(case[2], dtype=np.float32)
        b = np.zeros(case[2][0], dtype=np.float32)
    return x, w, b, dy


def assert_near(actual, expected, rel, name):
    """Normwise check: max |actual - expected| <= rel * max |expected|."""
    worst = float(np.max(np.abs(np.asarray(actual, dtype=np.float64) - expected)))
    allowed = rel * max(float(np.max(np.abs(expected))), 1e-30)
    assert worst <= allowed, f"{name}: max error {worst:.3e} > {rel:.1e} x max|ref| = {allowed:.3e}"


def gamma_k(k):
    """gamma_k = k u / (1 - k u), u = 2^-24: the worst-case relative error factor of a k-term FP32
    dot product (Higham, Accuracy and Stability of Numerical Algorithms, 3.1)."""
    u = EPS32 / 2
    return k * u / (1 - k * u)
