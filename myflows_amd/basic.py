"""Add and the fused Linear operator (y = x @ W + b).

Restates ``ops/basic.py:5-164`` of the reference. ``Linear`` on ``hip_native`` runs its three GEMMs on
the MFMA engine: the forward with the bias fused in the epilogue, dX = g W^T as an NT GEMM and
dW = x^T g as a TN GEMM that read the transposed operands in place; ``hip_native_kahan`` and
``hip_native_dot2`` run the compensated lecture kernels instead. db is summed in FP64 and rounded
once; an input with ``requires_grad=False`` skips the dX GEMM.
"""

from __future__ import annotations

import torch

from .core import GradientOp
from . import native

LINEAR_BACKENDS = ("auto", "hip_native", "hip_native_kahan", "hip_native_dot2")


def _linear_backend(backend):
    if backend not in LINEAR_BACKENDS:
        raise ValueError(f"backend must be one of {', '.join(LINEAR_BACKENDS)}")
    return backend


def _reduce_to(grad, shape):
    """Sum over the broadcast axes in FP64, rounded once (ops/basic.py:67-73)."""
    lead = grad.ndim - len(shape)
    axes = tuple(range(lead)) + tuple(lead + i for i, (gd, bd) in enumerate(zip(grad.shape[lead:], shape))
                                      if bd == 1 and gd != 1)
    total = grad.sum(dim=axes, dtype=torch.float64) if axes else grad
    return total.reshape(shape).to(grad.dtype)


class Add(GradientOp):
    def forward(self, a, b):
        self.a_shape = tuple(a.shape)
        self.b_shape = tuple(b.shape)
        if a.ndim == 4 and b.ndim == 1:
            self.a_broadcast_shape = self.a_shape
            self.b_broadcast_shape = (1, b.shape[0], 1, 1)
            self.value = a + b.reshape(self.b_broadcast_shape)
        else:
            ndim = max(a.ndim, b.ndim)
            self.a_broadcast_shape = (1,) * (ndim - a.ndim) + self.a_shape
            self.b_broadcast_shape = (1,) * (ndim - b.ndim) + self.b_shape
            self.value = a + b

    def backward(self):
        a, b = self.parents
        if a.requires_grad:
            a.accumulate_grad(self._handle_broadcast(self.grad, self.a_broadcast_shape, self.a_shape))
        if b.requires_grad:
            b.accumulate_grad(self._handle_broadcast(self.grad, self.b_broadcast_shape, self.b_shape))

    @staticmethod
    def _handle_broadcast(grad, broadcast_shape, original_shape):
        if tuple(grad.shape) != tuple(broadcast_shape):
            axes = tuple(axis for axis, (gd, sd) in enumerate(zip(grad.shape, broadcast_shape)) if sd == 1 and gd != 1)
            if axes:
                grad = grad.sum(dim=axes, keepdim=True)
        return grad.reshape(original_shape)


class Linear(GradientOp):
    def __init__(self, x, w, b, name=None, backend="auto"):
        super().__init__(x, w, b, name=name)
        self.backend = _linear_backend(backend)

    def _spec(self):
        from .convolution import _resolve_backend

        _resolve_backend("hip_native", *(p.value for p in self.parents))
        return {"auto": "mfma", "hip_native": "mfma", "hip_native_kahan": "kahan", "hip_native_dot2": "dot2"}[self.backend]

    def forward(self, x, w, b):
        self.x_shape, self.w_shape, self.b_shape = tuple(x.shape), tuple(w.shape), tuple(b.shape)
        spec = self._spec()
        if x.ndim != 2:
            raise ValueError("Linear on hip_native expects 2-D inputs")
        bias = b.reshape(-1) if b.numel() == w.shape[1] else None
        if spec == "mfma":
            out = native.gemm(x, w, bias)
        else:
            out = native.matmul(x, w, bias, variant="register", accumulate=spec)
        self.value = out if bias is not None else out + b

    def _matmul(self, a, b, trans_a=False, trans_b=False):
        spec = self._spec()
        if spec == "mfma":
            return native.gemm(a, b, trans_a=trans_a, trans_b=trans_b)
        return native.matmul((a.t() if trans_a else a).contiguous(), (b.t() if trans_b else b).contiguous(),
                             variant="register", accumulate=spec)

    def backward(self):
        x, w, b = self.parents
        grad = self.grad
        if getattr(x, "requires_grad", True):
            x.accumulate_grad(self._matmul(grad, w.value, trans_b=True), owned=True)
        if w.requires_grad:
            w.accumulate_grad(self._matmul(x.value, grad, trans_a=True), owned=True)
        if b.requires_grad:
            b.accumulate_grad(_reduce_to(grad, tuple(b.value.shape)))
