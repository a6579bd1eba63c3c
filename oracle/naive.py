"""FP64 textbook loops: the independent references of the reference's own convolution tests.

TEST INFRASTRUCTURE ONLY. Nothing in ``myflows_amd`` imports this package; only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it, as the checker.

Restated from ``tests/test_convolution.py:17-147`` of the reference (``naive_conv_forward``,
``naive_conv_backward``, ``naive_maxpool_forward``, ``naive_maxpool_backward``, ``naive_im2col``,
``naive_col2im``): direct window loops with no index tricks, so a wrong index in the vectorised
oracle (``oracle.reference_path``) or in a HIP kernel shows up as a mismatch.
"""

from __future__ import annotations

import numpy as np


def _pad(x, padding, value=0.0):
    ph, pw = padding
    return np.pad(x, ((0, 0), (0, 0), (ph, ph), (pw, pw)), mode="constant", constant_values=value)


def conv_forward(x, kernel, stride=(1, 1), padding=(0, 0)):
    """y[n, co, i, j] = sum over (ci, kh, kw) of window * kernel[co]; test_convolution.py:17-37."""
    sh, sw = stride
    n, ci, _, _ = x.shape
    co, kci, kh, kw = kernel.shape
    if ci != kci:
        raise ValueError("kernel input channels must match x input channels")
    xp = _pad(x, padding)
    oh = (xp.shape[2] - kh) // sh + 1
    ow = (xp.shape[3] - kw) // sw + 1
    out = np.zeros((n, co, oh, ow), dtype=x.dtype)
    for i in range(oh):
        for j in range(ow):
            window = xp[:, :, i * sh:i * sh + kh, j * sw:j * sw + kw]
            for c in range(co):
                out[:, c, i, j] = np.sum(window * kernel[c], axis=(1, 2, 3))
    return out


def conv_backward(x, kernel, grad_y, stride=(1, 1), padding=(0, 0)):
    """(dx, dkernel) by scattering every window's contribution; test_convolution.py:40-63."""
    sh, sw = stride
    ph, pw = padding
    xp = _pad(x, padding)
    gxp = np.zeros_like(xp)
    gk = np.zeros_like(kernel)
    _, co, oh, ow = grad_y.shape
    _, _, kh, kw = kernel.shape
    for i in range(oh):
        for j in range(ow):
            window = xp[:, :, i * sh:i * sh + kh, j * sw:j * sw + kw]
            for c in range(co):
                local = grad_y[:, c, i, j][:, None, None, None]
                gk[c] += np.sum(window * local, axis=0)
                gxp[:, :, i * sh:i * sh + kh, j * sw:j * sw + kw] += kernel[c] * local
    return gxp[:, :, ph:ph + x.shape[2], pw:pw + x.shape[3]], gk


def maxpool_forward(x, kernel_size=(2, 2), stride=(2, 2)):
    """Window maximum; test_convolution.py:66-81."""
    kh, kw = kernel_size
    sh, sw = stride
    n, c, h, w = x.shape
    oh, ow = (h - kh) // sh + 1, (w - kw) // sw + 1
    out = np.zeros((n, c, oh, ow), dtype=x.dtype)
    for i in range(oh):
        for j in range(ow):
            out[:, :, i, j] = np.max(x[:, :, i * sh:i * sh + kh, j * sw:j * sw + kw], axis=(2, 3))
    return out


def maxpool_backward(x, grad_y, kernel_size=(2, 2), stride=(2, 2)):
    """Gradient to the first maximum (np.argmax) of each window; test_convolution.py:84-103."""
    kh, kw = kernel_size
    sh, sw = stride
    gx = np.zeros_like(x)
    n, c, _, _ = x.shape
    _, _, oh, ow = grad_y.shape
    for i in range(oh):
        for j in range(ow):
            window = x[:, :, i * sh:i * sh + kh, j * sw:j * sw + kw]
            flat = window.reshape(n, c, -1)
            mask = np.zeros_like(flat)
            mask[np.arange(n)[:, None], np.arange(c)[None, :], np.argmax(flat, axis=-1)] = 1.0
            gx[:, :, i * sh:i * sh + kh, j * sw:j * sw + kw] += mask.reshape(window.shape) * grad_y[:, :, i, j][:, :, None, None]
    return gx


def im2col(x, kernel_size, stride=(1, 1), padding=(0, 0)):
    """One row per output position, features in (ci, kh, kw) order; test_convolution.py:106-123."""
    kh, kw = kernel_size
    sh, sw = stride
    xp = _pad(x, padding)
    n, c, _, _ = x.shape
    oh = (xp.shape[2] - kh) // sh + 1
    ow = (xp.shape[3] - kw) // sw + 1
    rows = []
    for b in range(n):
        for i in range(oh):
            for j in range(ow):
                rows.append(xp[b, :, i * sh:i * sh + kh, j * sw:j * sw + kw].reshape(c * kh * kw))
    return np.array(rows)


def col2im(rows, input_shape, kernel_size, stride=(1, 1), padding=(0, 0)):
    """Adjoint of im2col; test_convolution.py:126-147."""
    kh, kw = kernel_size
    sh, sw = stride
    ph, pw = padding
    n, c, h, w = input_shape
    padded = np.zeros((n, c, h + 2 * ph, w + 2 * pw), dtype=rows.dtype)
    oh = (padded.shape[2] - kh) // sh + 1
    ow = (padded.shape[3] - kw) // sw + 1
    r = 0
    for b in range(n):
        for i in range(oh):
            for j in range(ow):
                padded[b, :, i * sh:i * sh + kh, j * sw:j * sw + kw] += rows[r].reshape(c, kh, kw)
                r += 1
    return padded[:, :, ph:ph + h, pw:pw + w]
