"""Seeded parameter initialisers.

``make_initializer(name, seed=...)`` returns a callable ``shape -> float64 ndarray`` that draws from
one ``numpy.random.default_rng(seed)`` stream, so a model built layer by layer in the reference's
order gets exactly the reference's weights (``utils/initializers.py:14-57``: the same
distributions, fan rules and draw calls). The caller casts to float32.
"""

from __future__ import annotations

import math

import numpy as np


def compute_fans(shape):
    """(fan_in, fan_out): dense (in, out) or convolution (out, in, *receptive field)."""
    if len(shape) < 2:
        return 1, 1
    if len(shape) == 2:
        return int(shape[0]), int(shape[1])
    field = math.prod(int(v) for v in shape[2:])
    return max(1, int(shape[1]) * field), max(1, int(shape[0]) * field)


class _Draw:
    """One named distribution drawing from a shared generator."""

    def __init__(self, kind, rng, mean, std, value):
        self.kind, self.rng = kind, rng
        self.mean, self.std, self.value = float(mean), float(std), float(value)

    def __call__(self, shape):
        shape = tuple(int(v) for v in shape)
        fan_in, fan_out = compute_fans(shape)
        if self.kind == "kaiming_normal":
            return self.rng.normal(0.0, np.sqrt(2.0 / fan_in), size=shape)
        if self.kind == "kaiming_uniform":
            bound = np.sqrt(6.0 / fan_in)
            return self.rng.uniform(-bound, bound, size=shape)
        if self.kind == "xavier_normal":
            return self.rng.normal(0.0, np.sqrt(2.0 / (fan_in + fan_out)), size=shape)
        if self.kind == "xavier_uniform":
            bound = np.sqrt(6.0 / (fan_in + fan_out))
            return self.rng.uniform(-bound, bound, size=shape)
        if self.kind == "normal":
            return self.rng.normal(self.mean, self.std, size=shape)
        return np.full(shape, self.value, dtype=np.float64)  # constant


_ALIASES = {"default": "kaiming_normal", "he": "kaiming_normal", "he_normal": "kaiming_normal",
            "kaiming": "kaiming_normal", "kaiming_normal": "kaiming_normal", "kaiming_uniform": "kaiming_uniform",
            "xavier_normal": "xavier_normal", "xavier_uniform": "xavier_uniform", "normal": "normal",
            "constant": "constant"}


def make_initializer(name=None, *, seed=None, value=0.0, mean=0.0, std=0.01):
    """A shape -> ndarray initialiser; ``name`` defaults to Kaiming normal, a callable is returned
    unchanged."""
    if callable(name):
        return name
    key = str(name or "kaiming_normal").strip().lower()
    if key not in _ALIASES:
        raise ValueError(f"unknown initializer: {name!r}")
    return _Draw(_ALIASES[key], np.random.default_rng(seed), mean, std, value)
