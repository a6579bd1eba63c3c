"""Seeded parameter initialisers, restating ``utils/initializers.py:14-57`` of the reference.

Values are drawn in float64 from a NumPy Generator and cast by the caller, so a seeded model gets the
same weights as the reference model built with the same seed and the same layer order.
"""

from __future__ import annotations

import numpy as np


def compute_fans(shape):
    if len(shape) < 2:
        return 1, 1
    if len(shape) == 2:
        return int(shape[0]), int(shape[1])
    receptive = int(np.prod(shape[2:]))
    return max(1, int(shape[1] * receptive)), max(1, int(shape[0] * receptive))


def make_initializer(name=None, *, seed=None, value=0.0, mean=0.0, std=0.01):
    if callable(name):
        return name
    key = str(name or "kaiming_normal").strip().lower()
    rng = np.random.default_rng(seed)

    def init(shape):
        resolved = tuple(int(v) for v in shape)
        fan_in, fan_out = compute_fans(resolved)
        if key in ("default", "he", "he_normal", "kaiming", "kaiming_normal"):
            return rng.normal(0.0, np.sqrt(2.0 / fan_in), size=resolved)
        if key == "kaiming_uniform":
            limit = np.sqrt(6.0 / fan_in)
            return rng.uniform(-limit, limit, size=resolved)
        if key == "xavier_normal":
            return rng.normal(0.0, np.sqrt(2.0 / (fan_in + fan_out)), size=resolved)
        if key == "xavier_uniform":
            limit = np.sqrt(6.0 / (fan_in + fan_out))
            return rng.uniform(-limit, limit, size=resolved)
        if key == "normal":
            return rng.normal(float(mean), float(std), size=resolved)
        if key == "constant":
            return np.full(resolved, float(value), dtype=np.float64)
        raise ValueError(f"unknown initializer: {name!r}")

    return init
