"""Python boundary of libmfhip, the gfx950 library behind the ``hip_native`` backend.

PyTorch owns every device allocation and stream (the role CuPy plays in the reference). The library
never allocates: each call receives device addresses (``Tensor.data_ptr()``), int32 dimensions and
the current HIP stream, launches asynchronously and returns a status code that is turned into
``NativeHipError`` here. The public functions mirror ``ops/cuda_native/native.py`` of the reference
(``conv2d_forward`` :384-411, ``conv2d_backward`` :414-472, ``maxpool2d_forward/backward``
:491-522, ``matmul`` :525-562, ``gemm_plan`` :565-581, ``split_reduce`` :584-602, ``gemm`` :605-646)
with the same argument meaning and the same ``ValueError``/``TypeError`` checks before any call.

There is no fallback: if the library or a GPU is missing every entry point raises.
"""

from __future__ import annotations

import ctypes
import json
import os
from dataclasses import dataclass
from functools import lru_cache

import torch

from . import build as _build

LIBRARY_PATH = _build.LIBRARY
INT32_LIMIT = 2**31 - 1

_STATUS = {1: "initialization failed", 2: "invalid argument", 3: "HIP runtime error", 5: "wrong HIP device"}
_ACTIVATIONS = {None: 0, "relu": 1, "leaky_relu": 2}
MATMUL_VARIANTS = {"basic": 0, "tiled": 1, "shared": 2, "register": 4}
# The one GEMM engine: FP32 on the matrix cores (v_mfma_f32_32x32x2_f32). "register" names the same
# engine so that callers written against the reference's register engine keep working.
GEMM_ENGINES = {"mfma": 1, "register": 1}
MATMUL_ACCUMULATION = {"fp32": 0, "kahan": 1, "dot2": 2}
PLAN_BASE = 16
PLAN_SLICES = 128
CONV_GRAD_TILE = 64  # pixels per tile of the transposed-gradient kernel (grid_x counts these)


class NativeHipError(RuntimeError):
    pass


@dataclass
class NativePoolContext:
    input_shape: tuple
    output_shape: tuple
    kernel_size: tuple
    stride: tuple
    argmax: object
    device_id: int


def _u64(value):
    return ctypes.c_uint64(int(value))


def _i32(value):
    return ctypes.c_int(int(value))


def _configure(lib):
    u64, i64, i32, f32 = ctypes.c_uint64, ctypes.c_int64, ctypes.c_int, ctypes.c_float
    lib.mfh_init.argtypes = []
    lib.mfh_init.restype = i32
    lib.mfh_last_error.argtypes = []
    lib.mfh_last_error.restype = ctypes.c_char_p
    lib.mfh_info.argtypes = []
    lib.mfh_info.restype = ctypes.c_char_p
    lib.mfh_set_debug_sync.argtypes = [i32]
    lib.mfh_set_debug_sync.restype = None
    lib.mfh_conv_im2col.argtypes = [u64, u64] + [i32] * 13 + [u64]
    lib.mfh_conv_im2col.restype = i32
    lib.mfh_conv_forward.argtypes = [u64] * 6 + [i32] * 13 + [i32, f32, i32, u64, i64, u64]
    lib.mfh_conv_forward.restype = i32
    lib.mfh_conv_backward.argtypes = [u64] * 10 + [i32] * 13 + [i32, i32, f32, i32, i32, u64, i64, u64]
    lib.mfh_conv_backward.restype = i32
    lib.mfh_pool_forward.argtypes = [u64] * 3 + [i32] * 10 + [u64]
    lib.mfh_pool_forward.restype = i32
    lib.mfh_pool_backward.argtypes = [u64] * 3 + [i32] * 10 + [u64]
    lib.mfh_pool_backward.restype = i32
    lib.mfh_matmul.argtypes = [i32] * 3 + [u64] * 4 + [i32] * 3 + [u64]
    lib.mfh_matmul.restype = i32
    lib.mfh_gemm_tile_count.argtypes = []
    lib.mfh_gemm_tile_count.restype = i32
    lib.mfh_gemm_tile_info.argtypes = [i32, ctypes.POINTER(i32)]
    lib.mfh_gemm_tile_info.restype = i32
    lib.mfh_gemm_plan.argtypes = [i32] * 3 + [ctypes.POINTER(i32)] * 2
    lib.mfh_gemm_plan.restype = i32
    lib.mfh_gemm_workspace.argtypes = [i32] * 3
    lib.mfh_gemm_workspace.restype = i64
    lib.mfh_split_reduce.argtypes = [u64, u64] + [i32] * 5 + [u64]
    lib.mfh_split_reduce.restype = i32
    lib.mfh_gemm.argtypes = [i32] * 3 + [u64] * 4 + [i32] * 6 + [u64, i64, u64]
    lib.mfh_gemm.restype = i32
    return lib


# Every symbol include/mfhip.h declares; tests check that the built library exports all of them.
EXPORTS = ("mfh_init", "mfh_last_error", "mfh_info", "mfh_set_debug_sync", "mfh_conv_im2col", "mfh_conv_forward",
           "mfh_conv_backward", "mfh_pool_forward", "mfh_pool_backward", "mfh_matmul", "mfh_gemm_tile_count",
           "mfh_gemm_tile_info", "mfh_gemm_plan", "mfh_gemm_workspace", "mfh_split_reduce", "mfh_gemm")


def _error(status, lib):
    detail = lib.mfh_last_error().decode(errors="replace")
    return NativeHipError(f"native HIP {_STATUS.get(status, 'call failed')} ({status}): {detail}")


def load_library():
    """dlopen libmfhip.so and declare its signatures, without touching the GPU."""
    if not LIBRARY_PATH.exists():
        if os.environ.get("MFHIP_AUTOBUILD", "1") == "0":
            raise NativeHipError(f"libmfhip is missing: {LIBRARY_PATH} (MFHIP_AUTOBUILD=0); run myflows_amd/build.py")
        try:
            _build.build()
        except (_build.BuildError, OSError) as exc:
            raise NativeHipError(f"could not build {LIBRARY_PATH}: {exc}") from exc
    return _configure(ctypes.CDLL(str(LIBRARY_PATH)))


@lru_cache(maxsize=1)
def _library():
    if not torch.cuda.is_available():
        raise NativeHipError("the hip_native backend needs a HIP GPU; none is visible")
    lib = load_library()
    # mfh_init binds to the current device; make sure PyTorch's context for it exists first.
    torch.empty(1, device="cuda")
    status = lib.mfh_init()
    if status != 0:
        raise _error(status, lib)
    return lib


def is_available():
    return LIBRARY_PATH.exists() and torch.cuda.is_available()


def info():
    """Device and build facts of the loaded library: device_arch, cu_count, binary, load_ms."""
    return json.loads(_library().mfh_info().decode())


def set_debug_sync(enabled=True):
    """Synchronize after every native launch so asynchronous faults name the failing kernel."""
    _library().mfh_set_debug_sync(1 if enabled else 0)


def _check(status, lib):
    if status:
        raise _error(status, lib)


def _stream():
    return _u64(torch.cuda.current_stream().cuda_stream)


def _array(value, name):
    if not isinstance(value, torch.Tensor) or value.dtype != torch.float32 or value.device.type != "cuda":
        raise TypeError(f"{name} must be a float32 torch tensor on the GPU")
    return value.contiguous()


def _ptr(tensor):
    return _u64(tensor.data_ptr() if tensor is not None else 0)


def _guard_index(**sizes):
    for name, size in sizes.items():
        if int(size) > INT32_LIMIT:
            raise ValueError(f"{name} has {int(size)} elements; native kernels index with int32 "
                             f"(limit {INT32_LIMIT}), so use a smaller batch")


def _dims(x, weight, stride, padding):
    if x.ndim != 4 or weight.ndim != 4 or x.shape[1] != weight.shape[1]:
        raise ValueError("x and weight must be NCHW/OIHW arrays with matching channels")
    stride = tuple(int(v) for v in stride)
    padding = tuple(int(v) for v in padding)
    if len(stride) != 2 or len(padding) != 2 or min(stride) <= 0 or min(padding) < 0:
        raise ValueError("stride and padding must contain two valid integers")
    n, ci, h, w = map(int, x.shape)
    co, _, kh, kw = map(int, weight.shape)
    oh = (h + 2 * padding[0] - kh) // stride[0] + 1
    ow = (w + 2 * padding[1] - kw) // stride[1] + 1
    if oh <= 0 or ow <= 0:
        raise ValueError("convolution output shape is not positive")
    m, k = n * oh * ow, ci * kh * kw
    _guard_index(im2col_columns=m * k, output=m * co, input=n * ci * h * w)
    if n > 65535:
        raise ValueError("native convolution supports at most 65535 samples per call")
    return (n, ci, h, w, co, kh, kw, oh, ow, stride[0], stride[1], padding[0], padding[1])


def _activation(activation, alpha):
    if activation not in _ACTIVATIONS:
        raise ValueError(f"activation must be one of {sorted(a for a in _ACTIVATIONS if a)} or None")
    alpha = float(alpha)
    if activation == "leaky_relu" and not alpha > 0.0:
        raise ValueError("a fused leaky_relu needs alpha > 0")
    return _ACTIVATIONS[activation], ctypes.c_float(alpha)


def _engine(engine):
    if engine not in GEMM_ENGINES:
        raise ValueError(f"engine must be one of {sorted(GEMM_ENGINES)}")
    return GEMM_ENGINES[engine]


@lru_cache(maxsize=1)
def tile_catalog():
    """Tile name -> (index, BM, BN, WM, WN, BK) of the MFMA engine, in native order."""
    lib = load_library()
    result = {}
    for index in range(lib.mfh_gemm_tile_count()):
        values = (ctypes.c_int * 5)()
        status = lib.mfh_gemm_tile_info(_i32(index), values)
        if status:
            raise _error(status, lib)
        bm, bn, wm, wn, bk = values
        result[f"{bm}x{bn}"] = (index, bm, bn, wm, wn, bk)
    return result


@lru_cache(maxsize=2048)
def _plan_code(tile, requested):
    if type(requested) is not int or requested < 1:
        raise ValueError("expected a positive integer split count")
    if requested > PLAN_SLICES:
        raise ValueError(f"at most {PLAN_SLICES} K slices")
    entry = tile_catalog().get(tile)
    if entry is None:
        raise ValueError(f"unknown tile {tile}; known: {sorted(tile_catalog())}")
    return PLAN_BASE + entry[0] * PLAN_SLICES + requested - 1


def _slices(k, requested, bk=16):
    chunk = ((k + requested - 1) // requested + bk - 1) // bk * bk
    chunk = min(k, chunk)
    return (k + chunk - 1) // chunk


def _split_parameters(code):
    index, part = divmod(code - PLAN_BASE, PLAN_SLICES)
    return part + 1, tuple(tile_catalog().values())[index][-1]


def _choose_engine(engine, layout, m, n, k):
    if os.environ.get("MFHIP_GEMM_AUTOTUNE") == "1" and engine == GEMM_ENGINES["mfma"]:
        from .autotune import selected_plan
        return _plan_code(*selected_plan(layout, m, n, k))
    return engine


def _workspace(lib, *requests):
    """The GEMMs of one call share the largest workspace any of them requests."""
    floats = 0
    for engine, m, n, k in requests:
        if engine == GEMM_ENGINES["mfma"]:
            size = lib.mfh_gemm_workspace(m, n, k)
            if size < 0:
                raise _error(2, lib)
        else:
            requested, bk = _split_parameters(engine)
            splits = _slices(k, requested, bk)
            size = splits * m * n if splits > 1 else 0
        floats = max(floats, size)
    if not floats:
        return None, 0
    return torch.empty((floats,), dtype=torch.float32, device="cuda"), floats


@lru_cache(maxsize=8)
def _cu_count(device_id):
    return int(torch.cuda.get_device_properties(device_id).multi_processor_count)


def _spatial_blocks(n, ohw, co, device_id):
    # Enough blocks to fill the GPU (about 8 per CU) while each block still walks several pixel
    # tiles, which also bounds the FP64 bias partial buffer at roughly that many rows.
    tiles = (ohw + CONV_GRAD_TILE - 1) // CONV_GRAD_TILE
    per_sample = -(-8 * _cu_count(device_id) // max(1, n * ((co + CONV_GRAD_TILE - 1) // CONV_GRAD_TILE)))
    return max(1, min(tiles, per_sample))


def conv2d_im2col(x, kernel_shape, *, stride=(1, 1), padding=(0, 0)):
    """cols (N*OH*OW, CI*KH*KW) of x for a kernel of shape (CO, CI, KH, KW)."""
    x = _array(x, "x")
    weight = torch.empty(kernel_shape, dtype=torch.float32, device="meta")
    dims = _dims(x, weight, stride, padding)
    n, ci, h, w, co, kh, kw, oh, ow, *_ = dims
    cols = torch.empty((n * oh * ow, ci * kh * kw), dtype=torch.float32, device=x.device)
    lib = _library()
    _check(lib.mfh_conv_im2col(_ptr(x), _ptr(cols), *[_i32(v) for v in dims], _stream()), lib)
    return cols


def conv2d_forward(x, weight, bias=None, *, stride=(1, 1), padding=(0, 0), activation=None, alpha=0.0,
                   engine="mfma"):
    """Return the contiguous NCHW output (bias and activation fused) and the im2col columns."""
    engine = _engine(engine)
    x, weight = _array(x, "x"), _array(weight, "weight")
    if bias is not None:
        bias = _array(bias, "bias")
        if tuple(bias.shape) != (weight.shape[0],):
            raise ValueError("bias must have shape (out_channels,)")
    dims = _dims(x, weight, stride, padding)
    act, alpha = _activation(activation, alpha)
    n, ci, h, w, co, kh, kw, oh, ow, sh, sw, ph, pw = dims
    m, k = n * oh * ow, ci * kh * kw
    cols = torch.empty((m, k), dtype=torch.float32, device=x.device)
    rows = torch.empty((m, co), dtype=torch.float32, device=x.device)
    y = torch.empty((n, co, oh, ow), dtype=torch.float32, device=x.device)
    lib = _library()
    engine = _choose_engine(engine, "NT", m, co, k)
    workspace, floats = _workspace(lib, (engine, m, co, k))
    _check(lib.mfh_conv_forward(
        _ptr(x), _ptr(weight), _ptr(bias), _ptr(cols), _ptr(rows), _ptr(y), *[_i32(v) for v in dims], _i32(act),
        alpha, _i32(engine), _ptr(workspace), ctypes.c_int64(floats), _stream()), lib)
    return y, cols


def conv2d_backward(x, weight, grad_y, cols, *, stride=(1, 1), padding=(0, 0), need_bias_grad=True,
                    need_input_grad=True, need_weight_grad=True, activation=None, alpha=0.0, output=None,
                    engine="mfma", recompute_cols=False):
    """Return (dx, dw, db) with None for each unrequested gradient. Only dW needs forward cols."""
    engine = _engine(engine)
    x, weight, grad_y = _array(x, "x"), _array(weight, "weight"), _array(grad_y, "grad_y")
    dims = _dims(x, weight, stride, padding)
    act, alpha = _activation(activation, alpha)
    n, ci, h, w, co, kh, kw, oh, ow, sh, sw, ph, pw = dims
    if tuple(grad_y.shape) != (n, co, oh, ow):
        raise ValueError("grad_y shape does not match convolution output")
    m, k = n * oh * ow, ci * kh * kw
    if need_weight_grad and recompute_cols:
        cols = conv2d_im2col(x, tuple(weight.shape), stride=stride, padding=padding)
    else:
        cols = _array(cols, "cols") if need_weight_grad else None
    if cols is not None and tuple(cols.shape) != (m, k):
        raise ValueError("cols shape does not match convolution input")
    gate = None
    if act:
        if output is None:
            raise ValueError("a fused activation needs the forward output")
        gate = _array(output, "output")
        if gate.shape != grad_y.shape:
            raise ValueError("output shape does not match grad_y")
    if not (need_input_grad or need_weight_grad or need_bias_grad):
        return None, None, None
    direct_dx = need_input_grad and not (need_weight_grad or need_bias_grad)
    if direct_dx and act:
        inactive = alpha.value * grad_y if activation == "leaky_relu" else torch.zeros_like(grad_y)
        grad_y = torch.where(gate > 0, grad_y, inactive)
        act, gate = 0, None
    device = x.device
    blocks = _spatial_blocks(n, oh * ow, co, device.index or 0)
    dy_rows = (torch.empty((m, co), dtype=torch.float32, device=device)
               if need_weight_grad or (need_input_grad and need_bias_grad) else None)
    dw = torch.empty_like(weight) if need_weight_grad else None
    grad_cols = torch.empty((m, k), dtype=torch.float32, device=device) if need_input_grad else None
    dx = torch.empty_like(x) if need_input_grad else None
    partial = torch.empty((n * blocks * co,), dtype=torch.float64, device=device) if need_bias_grad else None
    db = torch.empty((co,), dtype=torch.float32, device=device) if need_bias_grad else None
    lib = _library()
    dw_engine = _choose_engine(engine, "TN", co, k, m) if need_weight_grad else engine
    dx_engine = engine
    requests = [(dw_engine, co, k, m)] if need_weight_grad else []
    if need_input_grad:
        dx_rows = oh * ow if direct_dx else m
        dx_engine = _choose_engine(engine, "TN" if direct_dx else "NN", dx_rows, k, co)
        requests.append((dx_engine, dx_rows, k, co))
    workspace, floats = _workspace(lib, *requests)
    _check(lib.mfh_conv_backward(
        _ptr(weight), _ptr(grad_y), _ptr(gate), _ptr(cols), _ptr(dy_rows), _ptr(dw), _ptr(grad_cols), _ptr(dx),
        _ptr(partial), _ptr(db), *[_i32(v) for v in dims], _i32(blocks), _i32(act), alpha, _i32(dw_engine),
        _i32(dx_engine), _ptr(workspace), ctypes.c_int64(floats), _stream()), lib)
    return dx, dw, db


def _pool_dims(x, kernel_size, stride):
    if x.ndim != 4:
        raise ValueError("x must be an NCHW array")
    kernel = tuple(int(v) for v in kernel_size)
    stride = tuple(int(v) for v in stride)
    if len(kernel) != 2 or len(stride) != 2 or min(kernel) <= 0 or min(stride) <= 0:
        raise ValueError("kernel_size and stride must contain positive pairs")
    n, c, h, w = map(int, x.shape)
    oh = (h - kernel[0]) // stride[0] + 1
    ow = (w - kernel[1]) // stride[1] + 1
    if oh <= 0 or ow <= 0:
        raise ValueError("pooling window is larger than the input")
    _guard_index(input=n * c * h * w)
    return n, c, h, w, oh, ow, kernel[0], kernel[1], stride[0], stride[1]


def maxpool2d_forward(x, *, kernel_size=(2, 2), stride=(2, 2)):
    x = _array(x, "x")
    dims = _pool_dims(x, kernel_size, stride)
    n, c, h, w, oh, ow, kh, kw, sh, sw = dims
    y = torch.empty((n, c, oh, ow), dtype=torch.float32, device=x.device)
    argmax = torch.empty((n, c, oh, ow), dtype=torch.int32, device=x.device)
    lib = _library()
    _check(lib.mfh_pool_forward(_ptr(x), _ptr(y), _ptr(argmax), *[_i32(v) for v in dims], _stream()), lib)
    return y, NativePoolContext(tuple(x.shape), tuple(y.shape), (kh, kw), (sh, sw), argmax, x.device.index)


def maxpool2d_backward(grad_y, context):
    if not isinstance(context, NativePoolContext) or context.device_id != torch.cuda.current_device():
        raise ValueError("context must come from maxpool2d_forward on the current device")
    grad_y = _array(grad_y, "grad_y")
    if tuple(grad_y.shape) != tuple(context.output_shape):
        raise ValueError("grad_y/context shape does not match pool output")
    n, c, h, w = map(int, context.input_shape)
    oh, ow = map(int, context.output_shape[2:])
    kh, kw = context.kernel_size
    sh, sw = context.stride
    dx = torch.empty(context.input_shape, dtype=torch.float32, device=grad_y.device)
    dims = (n, c, h, w, oh, ow, kh, kw, sh, sw)
    lib = _library()
    _check(lib.mfh_pool_backward(_ptr(grad_y), _ptr(context.argmax), _ptr(dx), *[_i32(v) for v in dims],
                                 _stream()), lib)
    return dx


def _out(out, m, n, like):
    if out is None:
        return torch.empty((m, n), dtype=torch.float32, device=like.device)
    if (not isinstance(out, torch.Tensor) or out.dtype != torch.float32 or tuple(out.shape) != (m, n)
            or not out.is_contiguous() or out.device != like.device):
        raise ValueError("out must be a contiguous float32 GPU tensor of the result shape")
    return out


def matmul(a, b, bias=None, *, variant="shared", tile=32, accumulate="kahan", out=None):
    """Row-major ``a @ b (+ bias)`` with one of the lecture kernels.

    ``variant``: basic (one thread per output), tiled (TILE x TILE blocks over global memory),
    shared (TILE x TILE LDS tiles) or register (64 x 64 block tiles with 4 x 4 outputs per thread;
    ``accumulate="fp32"`` runs the MFMA engine instead). ``accumulate``: fp32, kahan or dot2.
    """
    if variant not in MATMUL_VARIANTS:
        raise ValueError(f"variant must be one of {sorted(MATMUL_VARIANTS)}")
    if accumulate not in MATMUL_ACCUMULATION:
        raise ValueError(f"accumulate must be one of {sorted(MATMUL_ACCUMULATION)}")
    if int(tile) not in (16, 32):
        raise ValueError("tile must be 16 or 32")
    a, b = _array(a, "a"), _array(b, "b")
    if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[0]:
        raise ValueError("matmul needs 2-D operands with matching inner dimensions")
    m, k = map(int, a.shape)
    n = int(b.shape[1])
    if min(m, n, k) <= 0:
        raise ValueError("matmul dimensions must be positive")
    _guard_index(a=m * k, b=k * n, c=m * n)
    if bias is not None:
        bias = _array(bias, "bias").reshape(-1)
        if tuple(bias.shape) != (n,):
            raise ValueError("bias must have one value per output column")
    out = _out(out, m, n, a)
    lib = _library()
    _check(lib.mfh_matmul(
        _i32(MATMUL_VARIANTS[variant]), _i32(tile), _i32(MATMUL_ACCUMULATION[accumulate]), _ptr(a), _ptr(b),
        _ptr(bias), _ptr(out), _i32(m), _i32(n), _i32(k), _stream()), lib)
    return out


def gemm_plan(m, n, k, *, layout=None):
    """Tile name and split-K slices the MFMA engine uses for an (m, n) output over k."""
    if min(m, n, k) <= 0:
        raise ValueError("gemm dimensions must be positive")
    if layout is not None and os.environ.get("MFHIP_GEMM_AUTOTUNE") == "1":
        from .autotune import selected_plan
        tile, requested = selected_plan(layout, m, n, k)
        return tile, _slices(k, requested, tile_catalog()[tile][-1])
    lib = _library()
    shape, slices = ctypes.c_int(), ctypes.c_int()
    _check(lib.mfh_gemm_plan(_i32(m), _i32(n), _i32(k), ctypes.byref(shape), ctypes.byref(slices)), lib)
    return list(tile_catalog())[shape.value], slices.value


def split_reduce(partials, *, reference=False):
    """Sum split-K partials (slices x M x N float32) the way the engine finishes a split GEMM: in
    FP64, in slice order, rounded once."""
    partials = _array(partials, "partials")
    if partials.ndim != 3 or partials.shape[0] < 2:
        raise ValueError("partials must be a (slices >= 2, M, N) float32 array")
    slices, m, n = (int(v) for v in partials.shape)
    if min(m, n) <= 0:
        raise ValueError("partials must hold at least one output")
    _guard_index(partials=partials.numel())
    out = torch.empty((m, n), dtype=torch.float32, device=partials.device)
    lib = _library()
    _check(lib.mfh_split_reduce(_ptr(partials), _ptr(out), _i32(slices), _i32(m), _i32(n), _i32(n),
                                _i32(bool(reference)), _stream()), lib)
    return out


def gemm(a, b, bias=None, *, trans_a=False, trans_b=False, engine="mfma", out=None, plan=None):
    """Row-major ``op(a) @ op(b) (+ bias)`` on the MFMA engine.

    ``op(a)`` is ``a.T`` when ``trans_a`` (``a`` stored K x M), ``op(b)`` is ``b.T`` when
    ``trans_b`` (``b`` stored N x K); not both. ``plan=(tile, slices)`` forces a tile of
    ``tile_catalog()`` and a split-K slice count.
    """
    engine = _engine(engine)
    if trans_a and trans_b:
        raise ValueError("gemm supports a.T @ b and a @ b.T but not a.T @ b.T")
    a, b = _array(a, "a"), _array(b, "b")
    if a.ndim != 2 or b.ndim != 2:
        raise ValueError("gemm needs 2-D operands")
    m, k = (int(a.shape[1]), int(a.shape[0])) if trans_a else (int(a.shape[0]), int(a.shape[1]))
    n, k_b = (int(b.shape[0]), int(b.shape[1])) if trans_b else (int(b.shape[1]), int(b.shape[0]))
    if k != k_b:
        raise ValueError("gemm operands have different inner dimensions")
    if min(m, n, k) <= 0:
        raise ValueError("gemm dimensions must be positive")
    _guard_index(a=m * k, b=k * n, c=m * n)
    if bias is not None:
        bias = _array(bias, "bias").reshape(-1)
        if tuple(bias.shape) != (n,):
            raise ValueError("bias must have one value per output column")
    out = _out(out, m, n, a)
    lib = _library()
    if plan is not None:
        engine = _plan_code(*plan)
    else:
        engine = _choose_engine(engine, "TN" if trans_a else "NT" if trans_b else "NN", m, n, k)
    workspace, floats = _workspace(lib, (engine, m, n, k))
    _check(lib.mfh_gemm(
        _i32(engine), _i32(trans_a), _i32(trans_b), _ptr(a), _ptr(b), _ptr(bias), _ptr(out), _i32(m), _i32(n),
        _i32(k), _i32(a.shape[1]), _i32(b.shape[1]), _i32(n), _ptr(workspace), ctypes.c_int64(floats),
        _stream()), lib)
    return out
