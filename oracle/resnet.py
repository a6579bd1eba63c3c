"""ResNet18(output_dim=2) training step on the NumPy path, written out as straight-line code.

TEST INFRASTRUCTURE ONLY (parity oracle and the timed CPU baseline); the product never imports it.

Follows the reference model and step:
  * parameters and their draw order: ``layers/resnet.py:199-259`` (stem conv, then per block conv1,
    conv2, downsample conv, then fc), Kaiming normal from one shared ``np.random.default_rng(seed)``
    stream drawn in float64 and cast to float32 (``utils/initializers.py:25-57``,
    ``layers/layer.py:117-119``); conv biases and BN beta start at 0, gamma at 1, running mean 0 and
    running var 1 (``layers/resnet.py:55-62``); ``compat="myflows"``: convs with bias, stem max-pool
    3x3/2 without padding (``layers/resnet.py:296-300``);
  * the block ``ReLU(BN(conv2(ReLU(BN(conv1(x))))) + shortcut(x))`` (``layers/resnet.py:170-188``);
  * GlobalAvgPool2d, Linear fc (``layers/resnet.py:319-328``), MSELoss (``ops/loss.py:94-113``);
  * backward in reverse graph order with the NumPy operator branches of ``oracle.reference_path``;
  * Adam with zero-initialised moments (``train/opt.py:227-281``, ``ops/fused.py:514-533``).
The graph engine of the product is not used here, so this is an independent check of its order
and gradient accumulation.
"""

from __future__ import annotations

import numpy as np

from . import reference_path as rp


def _kaiming(rng, shape):
    fan_in = shape[0] if len(shape) == 2 else shape[1] * int(np.prod(shape[2:]))
    return rng.normal(0.0, np.sqrt(2.0 / fan_in), size=shape).astype(np.float32)


def block_specs(base_width=64):
    """(name, in_c, out_c, stride) of the eight BasicBlocks."""
    widths = [base_width, base_width * 2, base_width * 4, base_width * 8]
    specs, in_c = [], widths[0]
    for stage, (out_c, stride) in enumerate(zip(widths, (1, 2, 2, 2)), start=1):
        for index in range(2):
            specs.append((f"layer{stage}.{index}", in_c, out_c, stride if index == 0 else 1))
            in_c = out_c
    return specs


def as_dtype(params, running, dtype):
    """Copies of the parameters and running statistics in another float dtype."""
    return ({k: v.astype(dtype) for k, v in params.items()},
            {k: (m.astype(dtype), v.astype(dtype)) for k, (m, v) in running.items()})


def init_params(in_channels=3, output_dim=2, base_width=64, seed=0):
    """Ordered dict of float32 parameters plus BN running statistics, in the reference's order."""
    rng = np.random.default_rng(seed)
    params, running = {}, {}

    def conv(name, ci, co, k):
        params[f"{name}.weight"] = _kaiming(rng, (co, ci, k, k))
        params[f"{name}.bias"] = np.zeros((co,), np.float32)

    def bn(name, c):
        params[f"{name}.gamma"] = np.ones((c,), np.float32)
        params[f"{name}.beta"] = np.zeros((c,), np.float32)
        running[name] = (np.zeros((c,), np.float32), np.ones((c,), np.float32))

    conv("stem", in_channels, base_width, 7)
    bn("stem_bn", base_width)
    for name, ci, co, stride in block_specs(base_width):
        conv(f"{name}.conv1", ci, co, 3)
        bn(f"{name}.bn1", co)
        conv(f"{name}.conv2", co, co, 3)
        bn(f"{name}.bn2", co)
        if stride != 1 or ci != co:
            conv(f"{name}.down", ci, co, 1)
            bn(f"{name}.down_bn", co)
    params["fc.W"] = _kaiming(rng, (base_width * 8, output_dim))
    params["fc.b"] = np.zeros((output_dim,), np.float32)
    return params, running


class _Tape:
    def __init__(self, dtype):
        self.ops = []
        self.grads = {}
        self.dtype = dtype

    def add_grad(self, name, value):
        if name in self.grads:
            self.grads[name] = self.grads[name] + value.astype(self.dtype, copy=False)
        else:
            self.grads[name] = np.array(value, dtype=self.dtype, copy=True)


def forward_backward(params, running, x, target, training=True, need_input_grad=False, backward=True,
                     decisions=None, record=None):
    """One forward + backward pass in the dtype of x (float32 is the reference path; float64 gives
    the high-precision comparison point). Returns (loss, grads by parameter name, output); with
    backward=False the pass stops after the loss (grads empty).

    The pass's discrete decisions are each ReLU's mask (input > 0, keyed by the ReLU's name:
    "stem_relu", "<block>.relu1", "<block>.out") and the stem max-pool's window choices ("pool",
    a one-hot mask over each window). ``record`` (a dict) receives them; ``decisions`` (the same
    form) imposes them instead of deciding from this pass's own values, so that two passes that
    took different branches at near-ties can be compared on their rounding alone. ``record`` also
    receives each decision's input ("<name>/input")."""
    dtype = x.dtype
    tape = _Tape(dtype)
    acts = {}

    def conv(src, name, stride, pad):
        w, b = params[f"{name}.weight"], params[f"{name}.bias"]
        y, cols = rp.conv2d_forward(acts[src], w, b, (stride, stride), (pad, pad))
        acts[name] = y
        tape.ops.append(("conv", name, src, stride, pad, cols))
        return name

    def bn(src, name):
        rm, rv = running[name]
        y, mean, inv_std = rp.batchnorm2d_forward(acts[src], params[f"{name}.gamma"], params[f"{name}.beta"], rm, rv,
                                                  training=training)
        acts[name] = y
        tape.ops.append(("bn", name, src, mean, inv_std))
        return name

    def relu(src, name):
        if record is not None:
            record[name] = acts[src] > 0
            record[name + "/input"] = acts[src]
        if decisions is None:
            acts[name] = np.maximum(0, acts[src])
            mask = None
        else:
            mask = decisions[name]
            acts[name] = np.where(mask, acts[src], dtype.type(0))
        tape.ops.append(("relu", name, src, mask))
        return name

    acts["x"] = x
    h = relu(bn(conv("x", "stem", 2, 3), "stem_bn"), "stem_relu")
    y, mask, padded = rp.maxpool2d_forward(acts[h], (3, 3), (2, 2))
    if record is not None:
        record["pool"] = mask
        record["pool/input"] = acts[h]
    if decisions is not None:
        mask = decisions["pool"]
        n, c = acts[h].shape[:2]
        patches = rp.im2col(acts[h], (3, 3), (2, 2), (0, 0)).reshape(n, -1, c, 9).transpose(0, 2, 1, 3)
        y = np.take_along_axis(patches, mask.argmax(axis=-1)[..., None], axis=-1)[..., 0].reshape(y.shape)
    acts["pool"] = y
    tape.ops.append(("pool", "pool", h, mask, padded))
    h = "pool"
    for name, ci, co, stride in block_specs(params["stem.weight"].shape[0]):
        a = relu(bn(conv(h, f"{name}.conv1", stride, 1), f"{name}.bn1"), f"{name}.relu1")
        b = bn(conv(a, f"{name}.conv2", 1, 1), f"{name}.bn2")
        shortcut = h
        if f"{name}.down.weight" in params:
            shortcut = bn(conv(h, f"{name}.down", stride, 0), f"{name}.down_bn")
        acts[f"{name}.add"] = acts[b] + acts[shortcut]
        tape.ops.append(("add", f"{name}.add", b, shortcut))
        h = relu(f"{name}.add", f"{name}.out")
    acts["gap"] = rp.gap_forward(acts[h])
    tape.ops.append(("gap", "gap", h))
    acts["fc"] = rp.linear_forward(acts["gap"], params["fc.W"], params["fc.b"])
    loss = rp.mse_forward(acts["fc"], target)
    if not backward:
        return loss, {}, acts["fc"]

    grad = {"fc": rp.mse_backward(acts["fc"], target, dtype.type(1.0)).astype(dtype)}

    def push(name, value):
        if name in grad:
            grad[name] = grad[name] + value.astype(dtype, copy=False)
        else:
            grad[name] = np.array(value, dtype=dtype, copy=True)

    dx, dw, db = rp.linear_backward(acts["gap"], params["fc.W"], params["fc.b"].shape, grad["fc"])
    tape.add_grad("fc.W", dw)
    tape.add_grad("fc.b", db)
    push("gap", dx)
    for op in reversed(tape.ops):
        kind, name, src = op[0], op[1], op[2]
        g = grad.pop(name, None)
        if g is None:
            continue
        if kind == "gap":
            push(src, rp.gap_backward(g, acts[src].shape))
        elif kind == "relu":
            mask = op[3]
            push(src, rp.relu_backward(acts[src], g) if mask is None else np.where(mask, g, dtype.type(0)))
        elif kind == "add":
            push(src, g)
            push(op[3], g)
        elif kind == "bn":
            _, _, _, mean, inv_std = op
            dx, dgamma, dbeta = rp.batchnorm2d_backward(acts[src], g, params[f"{name}.gamma"], mean, inv_std,
                                                       training=training)
            tape.add_grad(f"{name}.gamma", dgamma)
            tape.add_grad(f"{name}.beta", dbeta)
            push(src, dx)
        elif kind == "pool":
            _, _, _, mask, padded = op
            push(src, rp.maxpool2d_backward(g, mask, padded, (3, 3), (2, 2)))
        elif kind == "conv":
            _, _, _, stride, pad, cols = op
            need_x = src != "x" or need_input_grad
            dx, dw, db = rp.conv2d_backward(acts[src], params[f"{name}.weight"], g, cols, (stride, stride),
                                            (pad, pad), need_input_grad=need_x)
            tape.add_grad(f"{name}.weight", dw)
            tape.add_grad(f"{name}.bias", db)
            if need_x:
                push(src, dx)
    if need_input_grad:
        tape.grads["x"] = grad.get("x")
    return loss, tape.grads, acts["fc"]


def adam_step(params, grads, state, step, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8):
    """Adam update of every parameter in place (train/opt.py:254-281)."""
    for name, p in params.items():
        g = grads.get(name)
        if g is None:
            continue
        if name not in state:
            state[name] = (np.zeros_like(p), np.zeros_like(p))
        m, v = state[name]
        rp.adam_update(p, g, m, v, lr=lr, beta1=beta1, beta2=beta2, eps=eps, step=step)


def synthetic_batch(batch, height=120, width=160, in_channels=3, output_dim=2, seed=0):
    """x ~ N(0, 1) then targets ~ U(-1, 1) from one seeded stream, both float32."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((batch, in_channels, height, width)).astype(np.float32)
    target = rng.uniform(-1, 1, (batch, output_dim)).astype(np.float32)
    return x, target
