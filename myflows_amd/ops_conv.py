"""Convolution, max-pool and flatten operators on the ``hip_native`` backend.

The operator API of the reference's ``ops/convolution.py``: ``Conv2D_Op`` (:287-523; native
forward :347-360, native backward :426-457), ``Conv2D_ReLU_Op`` (:526-545), ``Conv2D_LeakyReLU_Op``
(:548-573), ``MaxPool2d_Op`` (:817-890) and ``Flatten_Op`` (:893-898), with the backend value
``hip_native`` (``auto`` means hip_native on the GPU; ``cuda_native_register`` is accepted as an
alias so code written for the reference's native backend runs unchanged). This package has no CPU
path: CPU tensors are rejected as the reference rejects a native backend on the CPU device.
"""

from __future__ import annotations

import os

import torch

from . import fused, native, streams
from .device import get_device
from .graph import GradientOp

NATIVE_BACKENDS = {"hip_native": "mfma", "cuda_native_register": "mfma"}
BACKENDS = ("auto", *NATIVE_BACKENDS)


def _backend_name(backend):
    if backend not in BACKENDS:
        raise ValueError(f"unknown convolution backend {backend!r}; this build offers {BACKENDS}")
    return backend


def _resolve_backend(backend, *arrays):
    """The backend that runs now (``auto`` -> hip_native), after checking that the active device is
    the GPU (``set_device``) and that every array is a GPU tensor on the current device."""
    chosen = "hip_native" if backend == "auto" else backend
    if get_device() != "cuda":
        raise ValueError(f"backend={chosen} is incompatible with device={get_device()}")
    current = native.current_device_index()
    for value in arrays:
        if value is None:
            continue
        if not isinstance(value, torch.Tensor):
            raise TypeError("operator arrays must be torch tensors on the active device")
        if not value.is_cuda:
            raise ValueError(f"backend={chosen} is incompatible with device=cpu")
        if value.get_device() != current:
            raise ValueError("operator arrays must be on the current GPU")
    return chosen


def _int_pair(value, name, minimum=1):
    if isinstance(value, int):
        value = (value, value)
    if not (isinstance(value, (tuple, list)) and len(value) == 2):
        raise TypeError(f"{name} must be an int or a pair of ints, got {value!r}")
    pair = (int(value[0]), int(value[1]))
    if min(pair) < minimum:
        raise ValueError(f"{name} must be {'non-negative' if minimum == 0 else 'positive'}, got {value!r}")
    return pair


class Conv2D_Op(GradientOp):
    """y = conv(x, kernel) (+ bias), NCHW / OIHW, through im2col and the MFMA GEMM engine.

    The im2col columns are kept for dW only when the kernel needs a gradient and
    ``recompute_im2col`` is off; the inputs are kept only when this node needs gradients.
    """

    fused_activation = None  # "relu" / "leaky_relu" in the fused subclasses
    _defer_bn = None  # set by a Graph: the training batch norm that is this node's only consumer
    _defer_dx = None  # set by a Graph: the batch-norm unit after this node in the backward order that
                      # consumes the gradient of this node's input alone

    def __init__(self, x, kernel, stride=1, padding=0, groups=1, dilation=1, bias=None, backend="auto",
                 recompute_im2col=None):
        super().__init__(*((x, kernel) if bias is None else (x, kernel, bias)))
        self.backend = _backend_name(backend)
        if int(groups) != 1 or _int_pair(dilation, "dilation") != (1, 1):
            raise ValueError(f"{backend} supports only groups=1 and dilation=1")
        self.bias = bias
        self.stride = _int_pair(stride, "stride")
        self.padding = _int_pair(padding, "padding", minimum=0)
        self.groups, self.dilation = 1, (1, 1)
        if recompute_im2col is None:
            recompute_im2col = os.environ.get("MYFLOWS_RECOMPUTE_IM2COL") == "1"
        self.recompute_im2col = bool(recompute_im2col)
        self._activation_fused = False
        self._saved = None
        self._orders = {}  # phase -> (kernel tensor, its reordered copy) handed over by the Graph

    def _activation_alpha(self):
        return 0.0

    def _implicit(self, geometry=None):
        """Whether this node's products take the implicit algorithm: the default one, for a
        convolution whose tensors it can read (native.implicit_fits; checked once the geometry is
        known, and the forward's choice holds for the backward)."""
        if native.default_conv_algorithm() != "implicit":
            return False
        if geometry is not None:
            return native.implicit_fits(geometry)
        return getattr(self, "_implicit_ran", True)

    def weight_orders(self, phase):
        """The kernel reorders this node's next forward ("forward") or backward ("backward") pass
        reads, as (kernel, flip) requests: a Graph batches them over every convolution of a pass
        into one launch (native.conv_weight_orders) and hands the results to take_weight_orders."""
        kernel = self.parents[1].value
        if not self._implicit() or not isinstance(kernel, torch.Tensor) or kernel.device.type != "cuda":
            return []  # the operator's own forward reports what is wrong with a non-GPU kernel
        if phase == "forward":
            if kernel.ndim != 4 or not native.implicit_chunked(kernel.shape[1]):
                return []
            return [(kernel, 0)]
        if self._saved is None or not self.parents[0].requires_grad:
            return []
        kernel = self._saved[1]
        if self.stride != (1, 1) and (kernel.ndim != 4 or not native.strided_dx_phases(
                kernel.shape[2], kernel.shape[3], kernel.shape[0], self.stride)):
            # That dX runs through the column gradient: its one implicit product reads the dX order
            # of the kernel seen as a 1x1 kernel of CI*KH*KW channels (when dy has chunked channels).
            if kernel.ndim == 4 and native.implicit_chunked(kernel.shape[0]):
                return [(kernel.reshape(kernel.shape[0], -1, 1, 1), 1)]
            return []
        return [(kernel, 1, self.stride, self.padding)]

    def take_weight_orders(self, phase, tensors):
        kernel = self.parents[1].value if phase == "forward" else self._saved[1]
        self._orders[phase] = (kernel, kernel._version, tensors[0])

    def drop_weight_orders(self, phase):
        self._orders.pop(phase, None)

    def _order_for(self, phase, kernel):
        """The reordered kernel handed over for this pass, if it was made from this kernel tensor
        as it is now (same object, no in-place change since); used once."""
        handed = self._orders.pop(phase, None)
        if handed is None or handed[0] is not kernel or handed[1] != kernel._version:
            return None
        return handed[2]

    @staticmethod
    def _grad_target(node, like):
        """node's gradient as an in-place dX target (contiguous float32 of x's shape), else None."""
        grad = node.grad
        if (isinstance(grad, torch.Tensor) and grad.dtype is torch.float32 and grad.shape == like.shape
                and grad.is_contiguous() and grad.get_device() == like.get_device()):
            return grad
        return None

    def forward(self, x_val, kernel_val, bias_val=None):
        self.actual_backend = _resolve_backend(self.backend, x_val, kernel_val, bias_val)
        if self.bias is not None and bias_val is None:
            raise ValueError("bias value is missing")
        self._orders.pop("backward", None)
        order = self._order_for("forward", kernel_val)
        extra = {"weight_order": order} if order is not None else {}
        geometry = native.ConvGeometry.of(x_val.shape, kernel_val.shape, self.stride, self.padding)
        self._implicit_ran = self._implicit(geometry)
        bn = self._defer_bn
        defer = bn is not None and bn.training and self.fused_activation is None and self._implicit_ran
        if defer:  # at most as many positions per channel as the batch norm can form in one launch
            n, _, oh, ow = geometry.out_shape
            defer = n * oh * ow <= fused.SPLIT_FORM_MAX_POSITIONS
        if defer:
            # The one consumer is a training batch norm, which can form this output from the
            # product's split-K slices (and the bias) itself: one launch less, the same bits.
            self.value, cols = native.conv2d_forward_deferred(
                x_val, kernel_val, bias_val, stride=self.stride, padding=self.padding,
                engine=NATIVE_BACKENDS[self.actual_backend], max_positions=fused.SPLIT_FORM_MAX_POSITIONS,
                **extra), None
        else:
            self.value, cols = native.conv2d_forward(
                x_val, kernel_val, bias_val, stride=self.stride, padding=self.padding,
                activation=self.fused_activation, alpha=self._activation_alpha(),
                engine=NATIVE_BACKENDS[self.actual_backend], **extra)
        self._activation_fused = self.fused_activation is not None
        keep_cols = self.parents[1].requires_grad and not self.recompute_im2col
        self._saved = (x_val, kernel_val, cols if keep_cols else None) if self.requires_grad else None

    def backward(self):
        if not hasattr(self, "actual_backend"):
            raise RuntimeError("forward must run before backward")
        _resolve_backend(self.actual_backend, self.grad, *(p.value for p in self.parents))
        x_node, kernel_node = self.parents[0], self.parents[1]
        need_x, need_w = x_node.requires_grad, kernel_node.requires_grad
        need_b = self.bias is not None and self.bias.requires_grad
        if not (need_x or need_w or need_b):
            return
        x_val, kernel_val, cols = self._saved
        extra = {}
        implicit = self._implicit() and (cols is None or self.recompute_im2col)
        if implicit:
            flip = self._order_for("backward", kernel_val)
            if flip is not None:
                extra["weight_flip"] = flip
            target = self._grad_target(x_node, x_val) if need_x else None
            if target is not None:  # dX is added to the gradient x already has, in the same pass
                extra["input_grad"] = target
            unit = self._defer_dx
            if need_x and target is None and x_node.grad is None and unit is not None and unit.forms_input_grad():
                # The batch norm that consumes dX next, and alone, can form it from the dX product's
                # split-K slices itself: one launch less, the same bits.
                extra["defer_dx_positions"] = fused.SPLIT_FORM_MAX_POSITIONS
        engine = NATIVE_BACKENDS[self.actual_backend]
        session = streams.active()
        # A product with no dX beside it (a frozen input, such as a network's first convolution)
        # stays on this stream: there it runs beside the dW products already queued on the side
        # stream instead of after them.
        if implicit and need_x and (need_w or need_b) and session is not None and session.usable():
            # dW and db on the weight-gradient stream, dX on this one (the same products and plans as
            # the one-stream call below)
            side, hold = session.fork()
            grads = native.conv2d_backward(
                x_val, kernel_val, self.grad, None, stride=self.stride, padding=self.padding,
                need_bias_grad=need_b, need_weight_grad=need_w, need_input_grad=need_x,
                activation=self.fused_activation if self._activation_fused else None,
                alpha=self._activation_alpha(), output=self.value, engine=engine, algorithm="implicit",
                dw_stream=side, hold=hold, **extra)
            if any(grad is not None and parent.grad is not None
                   for parent, grad in zip(self.parents[1:], grads[1:])):
                session.join()  # an existing gradient is added to on this stream
        else:
            grads = native.conv2d_backward(
                x_val, kernel_val, self.grad, cols, stride=self.stride, padding=self.padding,
                need_bias_grad=need_b, need_weight_grad=need_w, need_input_grad=need_x,
                activation=self.fused_activation if self._activation_fused else None,
                alpha=self._activation_alpha(), output=self.value, engine=engine,
                recompute_cols=self.recompute_im2col, **({"algorithm": "implicit"} if implicit else {}), **extra)
        for parent, grad in zip(self.parents, grads):
            if grad is None or ("input_grad" in extra and parent is x_node):
                continue
            parent.accumulate_grad(grad, owned=True)


class Conv2D_ReLU_Op(Conv2D_Op):
    """Conv2D(+bias) then ReLU: the activation runs in the GEMM epilogue and the backward gates dy
    by the output inside the transposed-gradient kernel."""

    fused_activation = "relu"


class Conv2D_AddReLU_Op(Conv2D_Op):
    """ReLU(Conv2D(+bias) + residual) with the residual add and the ReLU in the GEMM epilogue: the
    same float32 operations, in the same order, as the separate Conv2D, Add and ReLU nodes. Formed
    by the inference graph rewrite (``fusion.fuse_conv_add_relu``) for graphs that take no gradient,
    so it has no backward. Parents: x, kernel, [bias], residual. ``residual_first`` records that the
    replaced Add took the residual as its first operand.

    The epilogue reads a residual laid out as the output. Any other residual value (one that the Add
    would broadcast, such as a per-channel vector, or promote, such as float64, or one on another
    device) takes the separate operations instead: the convolution, the Add's broadcast sum in its
    operand order, then the ReLU operator, with the results and errors the unfused nodes give."""

    fused_activation = "relu"

    def __init__(self, x, kernel, residual, *, residual_first=False, **kwargs):
        super().__init__(x, kernel, **kwargs)
        self.residual_first = bool(residual_first)
        self.parents.append(residual)
        if self not in residual.children:
            residual.children.append(self)

    def _unfused(self, x_val, kernel_val, bias_val, residual_val):
        from . import fused
        from .ops_basic import _gpu_only

        self.actual_backend = _resolve_backend(self.backend, x_val, kernel_val, bias_val)
        self._orders.pop("backward", None)
        order = self._order_for("forward", kernel_val)
        extra = {"weight_order": order} if order is not None else {}
        conv, _ = native.conv2d_forward(x_val, kernel_val, bias_val, stride=self.stride, padding=self.padding,
                                        engine=NATIVE_BACKENDS[self.actual_backend], **extra)
        a, b = (residual_val, conv) if self.residual_first else (conv, residual_val)
        if a.ndim == 4 and b.ndim == 1:  # Add's per-channel bias form
            b = b.reshape(1, -1, 1, 1)
        total = a + b
        _gpu_only(total, "ReLU")
        self.value = fused.relu_forward(total)
        self._activation_fused = False
        self._saved = None

    def forward(self, x_val, kernel_val, *rest):
        bias_val, residual_val = (rest[0], rest[1]) if self.bias is not None else (None, rest[0])
        fits = (isinstance(residual_val, torch.Tensor) and isinstance(x_val, torch.Tensor)
                and residual_val.dtype == torch.float32 and residual_val.device == x_val.device
                and kernel_val.ndim == 4 and x_val.ndim == 4)
        if fits:  # the residual is read by the implicit product's epilogue
            geometry = native.ConvGeometry.of(tuple(x_val.shape), tuple(kernel_val.shape), self.stride, self.padding)
            fits = tuple(residual_val.shape) == geometry.out_shape and native.implicit_fits(geometry)
        if not fits:
            self._unfused(x_val, kernel_val, bias_val, residual_val)
            return
        self.actual_backend = _resolve_backend(self.backend, x_val, kernel_val, bias_val, residual_val)
        self._orders.pop("backward", None)
        order = self._order_for("forward", kernel_val)
        extra = {"weight_order": order} if order is not None else {}
        self.value, _ = native.conv2d_forward(
            x_val, kernel_val, bias_val, stride=self.stride, padding=self.padding, activation="relu",
            engine=NATIVE_BACKENDS[self.actual_backend], algorithm="implicit", residual=residual_val, **extra)
        self._activation_fused = True
        self._saved = None

    def weight_orders(self, phase):
        return super().weight_orders(phase) if phase == "forward" else []

    def backward(self):
        raise RuntimeError("Conv2D_AddReLU_Op is an inference fusion and has no backward; build the graph "
                           "without apply_graph_optimizations(mode='inference') to train it")


class Conv2D_LeakyReLU_Op(Conv2D_Op):
    """Conv2D(+bias) then LeakyReLU. Fused only for alpha > 0 (then y > 0 exactly where the
    pre-activation is > 0, so the output alone can gate the backward); otherwise applied after."""

    def __init__(self, *args, alpha=0.01, **kwargs):
        super().__init__(*args, **kwargs)
        self.alpha = float(alpha)
        self.fused_activation = "leaky_relu" if self.alpha > 0 else None
        self._positive = None

    def _activation_alpha(self):
        return self.alpha

    def forward(self, x_val, kernel_val, bias_val=None):
        super().forward(x_val, kernel_val, bias_val=bias_val)
        if self._activation_fused:
            return
        positive = self.value > 0
        self.value = torch.where(positive, self.value, self.alpha * self.value)
        self._positive = positive if self.requires_grad else None

    def backward(self):
        if not self._activation_fused:
            self.grad = torch.where(self._positive, self.grad, self.alpha * self.grad)
        super().backward()


class MaxPool2d_Op(GradientOp):
    """Max pooling. ``padding`` pads with -inf (as torch.nn.MaxPool2d); the native kernels then see an
    unpadded input and the input gradient is cropped back."""

    inference = False  # set by the inference rewrite: the window indices are not stored

    def __init__(self, x, kernel_size=2, stride=2, backend="auto", padding=0):
        super().__init__(x)
        self.backend = _backend_name(backend)
        self.kernel_size = _int_pair(kernel_size, "kernel_size")
        self.stride = _int_pair(stride, "stride")
        self.padding = _int_pair(padding, "padding", minimum=0)
        self._context = None

    def forward(self, x_val):
        self.actual_backend = _resolve_backend(self.backend, x_val)
        ph, pw = self.padding
        if ph or pw:
            x_val = torch.nn.functional.pad(x_val, (pw, pw, ph, ph), value=float("-inf"))
        # A pass no backward follows (no gradient needed, or an inference graph) does not store the
        # window indices.
        keep = self.requires_grad and not self.inference
        self.value, context = native.maxpool2d_forward(x_val, kernel_size=self.kernel_size, stride=self.stride,
                                                       with_argmax=keep)
        self._context = context if keep else None

    def backward(self):
        if not hasattr(self, "actual_backend"):
            raise RuntimeError("forward must run before backward")
        if self.inference:
            raise RuntimeError("MaxPool2d_Op of an inference graph (apply_graph_optimizations(mode='inference')) "
                               "keeps no window indices and has no backward")
        _resolve_backend(self.actual_backend, self.grad, self.parents[0].value)
        dx = native.maxpool2d_backward(self.grad, self._context)
        ph, pw = self.padding
        if ph or pw:
            dx = dx[:, :, ph:dx.shape[2] - ph, pw:dx.shape[3] - pw]
        self.parents[0].accumulate_grad(dx, owned=not (ph or pw))


class Flatten_Op(GradientOp):
    """(N, ...) -> (N, prod(...)), a view."""

    def forward(self, x):
        self.in_shape = tuple(x.shape)
        self.value = x.reshape(x.shape[0], -1)

    def backward(self):
        self.parents[0].accumulate_grad(self.grad.reshape(self.in_shape))
