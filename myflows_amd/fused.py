"""Batch norm (+ residual + ReLU), ReLU backward and Adam on libmfhip.

Same names, arguments and results as the reference's ``ops/fused.py``: ``batchnorm2d_forward``
(:250-305), ``batchnorm2d_backward`` (:308-380), ``relu_backward_accumulate`` /
``leaky_relu_backward_accumulate`` (:50-77), ``adam_update`` (:514-533) and ``adam_update_many``
(:609-621). The head of the network runs here too: the global average pool
(``ops/batchnorm.py:110-123``), the MSE loss and its gradient (``ops/loss.py:94-113``) and a
Linear layer's bias gradient (``ops/basic.py:164``). Every tensor is a float32 GPU tensor; there is
no host path.
"""

from __future__ import annotations

from functools import lru_cache

import torch

from . import native


def _f32(value, name):
    return native._device_f32(value, name)


def on_libmfhip(value):
    """Whether an operator's tensor runs on libmfhip: a float32 GPU tensor. (Operators that also
    accept host tensors compute those with torch on the host, as before.)"""
    return isinstance(value, torch.Tensor) and value.is_cuda and value.dtype == torch.float32


@lru_cache(maxsize=256)
def _bn_workspace_doubles(n, c, hw):
    doubles = native._library().mfh_bn_workspace(n, c, hw)
    if doubles < 0:
        native._raise_for(2, native._library())
    return doubles


@lru_cache(maxsize=256)
def _bn_dims(shape):
    if len(shape) != 4:
        raise ValueError("batch norm expects an NCHW tensor")
    n, c, h, w = (int(v) for v in shape)
    native._within_int32(x=n * c * h * w)
    return n, c, h * w


def _bn_shape(x):
    return _bn_dims(x.shape)


def _channel_vector(value, c, name):
    value = _f32(value, name)
    if value.shape != (c,):
        raise ValueError(f"{name} must have shape (C,)")
    return value


# Positions per channel (N * H * W) up to which a training batch norm normalises a channel in one
# launch, and so can also form a deferred convolution output (mfh_bn_forward_split).
SPLIT_FORM_MAX_POSITIONS = 8192


def batchnorm2d_forward(x, gamma, beta, running_mean, running_var, *, momentum, eps, training,
                        unbiased_running_var=False, relu=False, residual=None):
    """(y, mean, inv_std); updates running_mean / running_var in place when training.

    mean has shape (2, C): the FP64 batch mean as the float pair mean[0] + mean[1], to be passed
    unchanged to batchnorm2d_backward. The normalisation uses the biased batch variance; with
    unbiased_running_var the running variance tracks count / (count - 1) times it.
    """
    x = _f32(x, "x")
    n, c, hw = _bn_shape(x)
    gamma, beta = _channel_vector(gamma, c, "gamma"), _channel_vector(beta, c, "beta")
    for name, stat in (("running_mean", running_mean), ("running_var", running_var)):
        if not (isinstance(stat, torch.Tensor) and stat.dtype == torch.float32 and stat.is_cuda
                and stat.is_contiguous() and tuple(stat.shape) == (c,)):
            raise ValueError(f"{name} must be a contiguous float32 GPU tensor of shape (C,)")
    if residual is not None:
        residual = _f32(residual, "residual")
        if residual.shape != x.shape:
            raise ValueError("residual must have x's shape")
    count = n * hw
    var_scale = count / (count - 1) if unbiased_running_var and count > 1 else 1.0
    y = torch.empty_like(x)
    mean = torch.empty((2, c), dtype=torch.float32, device=x.device)
    inv_std = torch.empty((c,), dtype=torch.float32, device=x.device)
    split = native.take_pending_split(x)
    if split is not None:  # x is a convolution output still in split-K slices: form it here
        if not training or count > SPLIT_FORM_MAX_POSITIONS:
            raise RuntimeError("a deferred convolution output reached a batch norm that cannot form it")
        partial, slices, bias, _block = split
        native._call("mfh_bn_forward_split", partial, slices, native._addr(bias), x.data_ptr(), gamma.data_ptr(),
                     beta.data_ptr(), running_mean.data_ptr(), running_var.data_ptr(), native._addr(residual),
                     y.data_ptr(), mean.data_ptr(), inv_std.data_ptr(), n, c, hw, int(bool(relu)), float(momentum),
                     float(eps), float(var_scale), native._stream())
        return y, mean, inv_std
    doubles = _bn_workspace_doubles(n, c, hw) if training else 0
    workspace = native.stream_workspace(doubles, torch.float64) if doubles else None
    native._call("mfh_bn_forward", x.data_ptr(), gamma.data_ptr(), beta.data_ptr(), running_mean.data_ptr(),
                 running_var.data_ptr(), native._addr(residual), y.data_ptr(), mean.data_ptr(), inv_std.data_ptr(),
                 native._addr(workspace), doubles, n, c, hw, int(bool(training)), int(bool(relu)), float(momentum),
                 float(eps), float(var_scale), native._stream())
    return y, mean, inv_std


def _gradient_buffer(value, like, name):
    if value is None:
        return None
    if not (isinstance(value, torch.Tensor) and value.dtype == torch.float32 and value.is_cuda
            and value.is_contiguous() and value.shape == like.shape):
        raise ValueError(f"{name} must be a contiguous float32 GPU tensor shaped like its forward value")
    return value


def batchnorm2d_backward(x, dy, gamma, mean, inv_std, *, training, x_grad, gamma_grad, beta_grad,
                         accumulate=(True, True, True), gate=None, residual_grad=None, add_residual=False):
    """Write (or add, per ``accumulate``) the requested gradients into x_grad, gamma_grad and beta_grad.

    With ``gate`` (the output of a fused ReLU) dy counts only where gate > 0, and that gated dy is
    also stored (or added, with add_residual) into ``residual_grad``. A dy that a convolution's
    backward left in split-K slices (native.conv2d_backward with defer_dx_positions) is formed and
    stored first, in the same launch.
    """
    x, dy = _f32(x, "x"), _f32(dy, "dy")
    n, c, hw = _bn_shape(x)
    if dy.shape != x.shape:
        raise ValueError("dy must have x's shape")
    gamma = _channel_vector(gamma, c, "gamma")
    mean, inv_std = _f32(mean, "mean"), _channel_vector(inv_std, c, "inv_std")
    if tuple(mean.shape) != (2, c):
        raise ValueError("mean must be the (2, C) pair from batchnorm2d_forward")
    x_grad = _gradient_buffer(x_grad, x, "x_grad")
    gamma_grad = _gradient_buffer(gamma_grad, gamma, "gamma_grad")
    beta_grad = _gradient_buffer(beta_grad, gamma, "beta_grad")
    if gate is not None:
        gate = _f32(gate, "gate")
        if gate.shape != x.shape:
            raise ValueError("gate must have x's shape")
    elif residual_grad is not None:
        raise ValueError("a residual gradient needs the fused ReLU's output as gate")
    residual_grad = _gradient_buffer(residual_grad, x, "residual_grad")
    split = native.take_pending_split(dy)
    if split is not None:  # dy is a convolution's input gradient still in split-K slices: form it here
        sums = gamma_grad is not None or beta_grad is not None or (training and x_grad is not None)
        if not sums or n * hw > SPLIT_FORM_MAX_POSITIONS:
            raise RuntimeError("a deferred convolution input gradient reached a batch norm that cannot form it")
    if x_grad is None and gamma_grad is None and beta_grad is None and residual_grad is None:
        return
    doubles = _bn_workspace_doubles(n, c, hw)
    workspace = native.stream_workspace(doubles, torch.float64)
    add_x, add_gamma, add_beta = (int(bool(a)) for a in accumulate)
    pointers = (x.data_ptr(), dy.data_ptr(), native._addr(gate), gamma.data_ptr(), mean.data_ptr(),
                inv_std.data_ptr(), native._addr(x_grad), native._addr(gamma_grad), native._addr(beta_grad),
                native._addr(residual_grad), workspace.data_ptr(), doubles, n, c, hw, int(bool(training)), add_x,
                add_gamma, add_beta, int(bool(add_residual)), native._stream())
    if split is not None:
        native._call("mfh_bn_backward_split", split[0], split[1], *pointers)
    else:
        native._call("mfh_bn_backward", *pointers)


def _pool_window(x, kernel_size, stride):
    kh, kw = (int(v) for v in kernel_size)
    sh, sw = (int(v) for v in stride)
    n, c, h, w = (int(v) for v in x.shape)
    if min(kh, kw, sh, sw) <= 0 or kh > h or kw > w:
        raise ValueError("max-pool window and stride must be positive and the window inside the input")
    return kh, kw, sh, sw, (h - kh) // sh + 1, (w - kw) // sw + 1


def batchnorm_relu_pool_supported(shape, kernel_size, stride):
    """Whether batchnorm2d_relu_pool_forward/backward take an NCHW input of this shape and this pool
    window (their LDS staging of one plane fits)."""
    n, c, h, w = (int(v) for v in shape)
    kh, kw = (int(v) for v in kernel_size)
    sh, sw = (int(v) for v in stride)
    return bool(native._library().mfh_bn_relu_pool_supported(n, c, h, w, kh, kw, sh, sw))


def batchnorm2d_relu_pool_forward(x, gamma, beta, running_mean, running_var, *, momentum, eps, training,
                                  kernel_size, stride, unbiased_running_var=False):
    """(pooled, argmax, mean, inv_std): batchnorm2d_forward(..., relu=True) followed by a max-pool
    without padding, in two launches that never store the ReLU output. argmax is the int32 flat index
    into x's shape (as maxpool2d_forward's into its input). Bit for bit the separate passes."""
    x = _f32(x, "x")
    if native.take_pending_split(x) is not None:
        raise RuntimeError("a deferred convolution output reached a unit that cannot form it")
    n, c, hw = _bn_shape(x)
    gamma, beta = _channel_vector(gamma, c, "gamma"), _channel_vector(beta, c, "beta")
    for name, stat in (("running_mean", running_mean), ("running_var", running_var)):
        if not (isinstance(stat, torch.Tensor) and stat.dtype == torch.float32 and stat.is_cuda
                and stat.is_contiguous() and tuple(stat.shape) == (c,)):
            raise ValueError(f"{name} must be a contiguous float32 GPU tensor of shape (C,)")
    kh, kw, sh, sw, oh, ow = _pool_window(x, kernel_size, stride)
    count = n * hw
    var_scale = count / (count - 1) if unbiased_running_var and count > 1 else 1.0
    pooled = torch.empty((n, c, oh, ow), dtype=torch.float32, device=x.device)
    argmax = torch.empty((n, c, oh, ow), dtype=torch.int32, device=x.device)
    mean = torch.empty((2, c), dtype=torch.float32, device=x.device)
    inv_std = torch.empty((c,), dtype=torch.float32, device=x.device)
    doubles = _bn_workspace_doubles(n, c, hw) if training else 0
    workspace = native.stream_workspace(doubles, torch.float64) if doubles else None
    native._call("mfh_bn_relu_pool_forward", x.data_ptr(), gamma.data_ptr(), beta.data_ptr(),
                 running_mean.data_ptr(), running_var.data_ptr(), pooled.data_ptr(), argmax.data_ptr(),
                 mean.data_ptr(), inv_std.data_ptr(), native._addr(workspace), doubles, n, c, int(x.shape[2]),
                 int(x.shape[3]), kh, kw, sh, sw, int(bool(training)), float(momentum), float(eps), float(var_scale),
                 native._stream())
    return pooled, argmax, mean, inv_std


def batchnorm2d_relu_pool_backward(x, pooled_grad, argmax, gamma, beta, mean, inv_std, *, training, kernel_size,
                                   stride, x_grad, gamma_grad, beta_grad, accumulate=(True, True, True)):
    """Gradients of batchnorm2d_relu_pool_forward from the pooled output's gradient: the max-pool
    backward, the ReLU gate (recomputed from x) and batchnorm2d_backward in two launches, written (or
    added, per ``accumulate``) into x_grad, gamma_grad and beta_grad."""
    x, pooled_grad = _f32(x, "x"), _f32(pooled_grad, "pooled_grad")
    n, c, hw = _bn_shape(x)
    kh, kw, sh, sw, oh, ow = _pool_window(x, kernel_size, stride)
    if tuple(pooled_grad.shape) != (n, c, oh, ow):
        raise ValueError("pooled_grad must have the pooled output's shape")
    if not (isinstance(argmax, torch.Tensor) and argmax.dtype == torch.int32 and argmax.is_cuda
            and argmax.is_contiguous() and argmax.shape == pooled_grad.shape):
        raise ValueError("argmax must be the contiguous int32 GPU tensor from batchnorm2d_relu_pool_forward")
    gamma, beta = _channel_vector(gamma, c, "gamma"), _channel_vector(beta, c, "beta")
    mean, inv_std = _f32(mean, "mean"), _channel_vector(inv_std, c, "inv_std")
    if tuple(mean.shape) != (2, c):
        raise ValueError("mean must be the (2, C) pair from batchnorm2d_relu_pool_forward")
    x_grad = _gradient_buffer(x_grad, x, "x_grad")
    gamma_grad = _gradient_buffer(gamma_grad, gamma, "gamma_grad")
    beta_grad = _gradient_buffer(beta_grad, gamma, "beta_grad")
    if x_grad is None and gamma_grad is None and beta_grad is None:
        return
    doubles = _bn_workspace_doubles(n, c, hw)
    workspace = native.stream_workspace(doubles, torch.float64)
    add_x, add_gamma, add_beta = (int(bool(a)) for a in accumulate)
    native._call("mfh_bn_relu_pool_backward", x.data_ptr(), pooled_grad.data_ptr(), argmax.data_ptr(),
                 gamma.data_ptr(), beta.data_ptr(), mean.data_ptr(), inv_std.data_ptr(), native._addr(x_grad),
                 native._addr(gamma_grad), native._addr(beta_grad), workspace.data_ptr(), doubles, n, c,
                 int(x.shape[2]), int(x.shape[3]), kh, kw, sh, sw, int(bool(training)), add_x, add_gamma, add_beta,
                 native._stream())


def relu_forward(x):
    """max(0, x) (NaN stays NaN)."""
    x = _f32(x, "x")
    y = torch.empty_like(x)
    native._call("mfh_relu_forward", x.data_ptr(), y.data_ptr(), x.numel(), native._stream())
    return y


def _relu_backward(x, grad, out, alpha):
    x, grad = _f32(x, "x"), _f32(grad, "grad")
    if grad.shape != x.shape:
        raise ValueError("grad must have x's shape")
    add = out is not None
    if out is None:
        out = torch.empty_like(x)
    elif not (isinstance(out, torch.Tensor) and out.dtype == torch.float32 and out.is_cuda and out.is_contiguous()
              and out.shape == x.shape):
        raise ValueError("out must be a contiguous float32 GPU tensor shaped like x")
    native._call("mfh_relu_backward", x.data_ptr(), grad.data_ptr(), out.data_ptr(), x.numel(), float(alpha),
                 int(add), native._stream())
    return out


def relu_backward_accumulate(x, grad, out):
    """out += grad where x > 0 (a new tensor when out is None)."""
    return _relu_backward(x, grad, out, 0.0)


def leaky_relu_backward_accumulate(x, grad, out, alpha):
    """out += grad where x > 0 and alpha * grad elsewhere (a new tensor when out is None)."""
    return _relu_backward(x, grad, out, float(alpha))


def _output(out, add, shape, device):
    """The buffer a result goes to: a new tensor when out is None (add must then be False), else
    `out`, a contiguous float32 GPU tensor of `shape`, overwritten (add False) or added to."""
    if out is None:
        if add:
            raise ValueError("add needs an out tensor")
        return torch.empty(tuple(shape), dtype=torch.float32, device=device)
    if not (isinstance(out, torch.Tensor) and out.dtype == torch.float32 and out.is_cuda and out.is_contiguous()
            and tuple(out.shape) == tuple(shape)):
        raise ValueError(f"out must be a contiguous float32 GPU tensor of shape {tuple(shape)}")
    return out


def global_avg_pool_forward(x):
    """(N, C, H, W) -> (N, C): FP64 mean over H, W rounded once to float32."""
    x = _f32(x, "x")
    if x.ndim != 4:
        raise ValueError("global average pool takes an (N, C, H, W) tensor")
    n, c, h, w = x.shape
    y = torch.empty((n, c), dtype=torch.float32, device=x.device)
    if h * w == 0:
        raise ValueError("global average pool needs H * W > 0")
    native._call("mfh_plane_mean", x.data_ptr(), y.data_ptr(), n * c, h * w, native._stream())
    return y


def global_avg_pool_backward(grad, in_shape, out=None, add=False):
    """dx = grad[n, c] / (H * W) broadcast over (H, W), written to (or, with add, added to) out."""
    grad = _f32(grad, "grad")
    n, c, h, w = (int(v) for v in in_shape)
    if grad.numel() != n * c or h * w == 0:
        raise ValueError("grad must hold one value per (n, c) plane of a non-empty input")
    buffer = _output(out, add, (n, c, h, w), grad.device)
    native._call("mfh_plane_mean_backward", grad.data_ptr(), buffer.data_ptr(), n * c, h * w, int(add),
                 native._stream())
    return buffer


def mse_loss_forward(pred, target):
    """FP64 mean of the float32 squared differences, rounded to a 0-d float32 tensor."""
    pred, target = _f32(pred, "pred"), _f32(target, "target")
    if pred.shape != target.shape:
        raise ValueError("pred and target must have the same shape")
    loss = torch.empty((), dtype=torch.float32, device=pred.device)
    native._call("mfh_mse_loss", pred.data_ptr(), target.data_ptr(), loss.data_ptr(), pred.numel(), native._stream())
    return loss


def mse_loss_backward(pred, target, seed, out=None, add=False):
    """seed * (2 * (pred - target) / pred.numel()), each step rounded to float32, written to (or,
    with add, added to) out."""
    pred, target, seed = _f32(pred, "pred"), _f32(target, "target"), _f32(seed, "seed")
    if pred.shape != target.shape or seed.numel() != 1:
        raise ValueError("pred and target must match and seed must hold one value")
    buffer = _output(out, add, pred.shape, pred.device)
    native._call("mfh_mse_loss_backward", pred.data_ptr(), target.data_ptr(), seed.data_ptr(), buffer.data_ptr(),
                 pred.numel(), int(add), native._stream())
    return buffer


def column_sums(grad):
    """FP64 sums over the rows of a 2-D tensor, rounded once: (rows, cols) -> (cols,)."""
    grad = _f32(grad, "grad")
    if grad.ndim != 2:
        raise ValueError("column sums take a 2-D tensor")
    rows, cols = grad.shape
    out = torch.empty((cols,), dtype=torch.float32, device=grad.device)
    native._call("mfh_column_sums", grad.data_ptr(), out.data_ptr(), rows, cols, native._stream())
    return out


def _adam_row(param, grad, m, v, lr, decay, step, beta1, beta2):
    # The scalars are formed in double precision and rounded once to float32 by the c_float fields.
    return native.AdamTensor(param.data_ptr(), grad.data_ptr(), m.data_ptr(), v.data_ptr(), param.numel(),
                             float(lr), float(decay), 1.0 - beta1 ** step, 1.0 - beta2 ** step)


def _adam_launch(rows, beta1, beta2, eps, grad_scale):
    if not rows:
        return
    table = (native.AdamTensor * len(rows))(*rows)
    native._call("mfh_adam_step", table, len(rows), float(grad_scale), float(beta1), 1.0 - beta1, float(beta2),
                 1.0 - beta2, float(eps), native._stream())


def adam_update(param, grad, m, v, *, lr, beta1, beta2, eps, step, grad_scale=1.0, weight_decay=0.0):
    """One Adam step (zero-initialised moments, bias-corrected) applied in place. param, m and v are
    float32 GPU tensors of one shape; a strided one is updated through a contiguous copy that is
    written back, and a strided gradient is read through a contiguous copy."""
    tensors = [_f32(t, name) for t, name in ((param, "param"), (grad, "grad"), (m, "m"), (v, "v"))]
    if any(t.shape != param.shape for t in tensors):
        raise ValueError("Adam updates tensors of the parameter's shape")
    _adam_launch([_adam_row(*tensors, lr, weight_decay, step, beta1, beta2)], beta1, beta2, eps, grad_scale)
    for original, updated in ((param, tensors[0]), (m, tensors[2]), (v, tensors[3])):
        if updated is not original:
            original.copy_(updated)


class _AdamTable:
    """The parameter side of the last multi-tensor Adam launch: the (param, m, v) tensors, checked
    once (float32 GPU, contiguous, same shape, no two overlapping), and a row table holding their
    pointers. A training loop hands the same tensors back every step, and then only the gradients
    (new tensors each step) are checked and written into the table. The tensors are held, so their
    ids stay theirs while the table is kept."""

    def __init__(self):
        self.key = None
        self.held = None
        self.shapes = None
        self.owners = None  # ids of the param / moment tensors and of the tensors they view
        self.table = None


_ADAM_TABLE = _AdamTable()


def _adam_param_key(updates):
    return tuple((id(p), id(m), id(v), p.data_ptr(), m.data_ptr(), v.data_ptr()) for p, g, m, v, *_ in updates)


def _multi_adam_fits(updates):
    """Whether one multi-tensor launch can update these (param, grad, m, v, ...) tuples: every
    param, m and v a contiguous float32 GPU tensor of its parameter's shape, and none of them
    overlapping another (the launch reads and writes each element once, in no set order). Otherwise
    the updates run one tensor after another, as the reference's multi-tensor Adam does
    (ops/fused.py:579-606)."""
    f32 = torch.float32
    spans = []
    for p, g, m, v, *_ in updates:
        for t in (p, m, v):
            if not (isinstance(t, torch.Tensor) and t.dtype is f32 and t.is_cuda and t.is_contiguous()
                    and t.shape == p.shape):
                return False
            if t.numel():
                spans.append((t.data_ptr(), t.data_ptr() + 4 * t.numel()))
    spans.sort()
    return all(start >= end for (_, end), (start, _) in zip(spans, spans[1:]))


def _adam_table_for(updates, beta1, beta2):
    """The cached row table for these (param, m, v) tensors, rebuilt (with every check) when they
    change; None when they cannot share one launch (_multi_adam_fits)."""
    cache = _ADAM_TABLE
    key = _adam_param_key(updates)
    if cache.key == key:
        return cache
    if not _multi_adam_fits(updates):
        return None
    rows = [_adam_row(p, p, m, v, lr, decay, step, beta1, beta2) for p, g, m, v, lr, decay, step in updates]
    cache.key = key
    cache.held = [(p, m, v) for p, g, m, v, *_ in updates]
    cache.shapes = [p.shape for p, *_ in updates]
    cache.owners = {id(t if t._base is None else t._base) for held in cache.held for t in held}
    cache.table = (native.AdamTensor * len(rows))(*rows)
    return cache


def adam_update_many(updates, *, beta1, beta2, eps, grad_scale):
    """Adam for (param, grad, m, v, lr, decay, step) tuples in one multi-tensor launch per 48 tensors.

    Tensors that one launch cannot take (a strided or overlapping param or moment, a strided
    gradient, a gradient that shares memory with a param or moment) are updated one after another
    with adam_update instead, in the order given.
    """
    updates = list(updates)
    if not updates:
        return
    cache = _adam_table_for(updates, beta1, beta2)
    if cache is not None:
        table, owners = cache.table, cache.owners
        f32 = torch.float32
        for i, ((p, g, m, v, lr, decay, step), shape) in enumerate(zip(updates, cache.shapes)):
            if not (isinstance(g, torch.Tensor) and g.dtype is f32 and g.is_cuda and g.is_contiguous()
                    and g.shape == shape and id(g if g._base is None else g._base) not in owners):
                cache = None
                break
            row = table[i]
            # The scalars are formed in double precision and rounded once to float32 by the fields.
            row.grad = g.data_ptr()
            row.lr, row.weight_decay = float(lr), float(decay)
            row.bias_correction1, row.bias_correction2 = 1.0 - beta1 ** step, 1.0 - beta2 ** step
    if cache is None:
        for p, g, m, v, lr, decay, step in updates:
            adam_update(p, g, m, v, lr=lr, beta1=beta1, beta2=beta2, eps=eps, step=step, grad_scale=grad_scale,
                        weight_decay=decay)
        return
    native._call("mfh_adam_step", table, len(updates), float(grad_scale), float(beta1), 1.0 - beta1, float(beta2),
                 1.0 - beta2, float(eps), native._stream())
