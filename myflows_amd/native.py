"""Python side of libmfhip, the gfx950 library behind the ``hip_native`` backend.

PyTorch owns every device allocation and stream (the role CuPy plays in the reference). Each call
hands the library device addresses (``Tensor.data_ptr()``), int32 dimensions and the current HIP
stream; the library launches asynchronously and returns a status that becomes ``NativeHipError``.

The public functions keep the names, arguments and exceptions of the reference's
``ops/cuda_native/native.py``: ``conv2d_forward`` (:384-411), ``conv2d_backward`` (:414-472),
``maxpool2d_forward`` / ``maxpool2d_backward`` (:491-522), ``matmul`` (:525-562), ``gemm_plan``
(:565-581), ``split_reduce`` (:584-602), ``gemm`` (:605-646), ``tile_catalog``, ``info``,
``set_debug_sync``, ``is_available``. Shapes and dtypes are checked here first (``ValueError`` /
``TypeError``), as the reference does, so the C checks only see calls that passed them.

There is no fallback: without the library or a GPU every entry point raises.
"""

from __future__ import annotations

import contextlib
import ctypes
import json
import os
import threading
from dataclasses import dataclass
from functools import lru_cache

import torch

from . import build as _build

LIBRARY_PATH = _build.LIBRARY
INT32_LIMIT = 2**31 - 1
GRID_LIMIT = 65535

# The one GEMM engine is FP32 on the matrix cores; "register" is accepted as its name too, so code
# written against the reference's register engine runs unchanged.
GEMM_ENGINES = {"mfma": 1, "register": 1}
MATMUL_VARIANTS = {"basic": 0, "tiled": 1, "shared": 2, "register": 4}
MATMUL_ACCUMULATION = {"fp32": 0, "kahan": 1, "dot2": 2}
ACTIVATION_CODES = {None: 0, "relu": 1, "leaky_relu": 2}
# Explicit GEMM plan codes, with the reference's arithmetic (native.py:298-309 there): the reference's
# named tiles (its GEMM_TILES) take NAMED_PLAN_BASE + index * NAMED_PLAN_SLICES + slices - 1 (at most 32
# slices) and run on this library's tile of the same role; every tile of this library's catalogue
# takes EXTENDED_PLAN_BASE + index * EXTENDED_PLAN_SLICES + slices - 1 (at most 128).
NAMED_TILES = ("128x128", "128x64", "256x32", "64x128", "32x256")
NAMED_TILE_OF = {"128x128": "128x128", "128x64": "256x64", "256x32": "128x32", "64x128": "64x128", "32x256": "32x128"}
NAMED_PLAN_BASE, NAMED_PLAN_SLICES = 16, 32
EXTENDED_PLAN_BASE, EXTENDED_PLAN_SLICES = 1024, 128
# Plan codes of the implicit convolution products (their own 12 tiles): IMPLICIT_PLAN_BASE + tile *
# IMPLICIT_PLAN_SLICES + slices - 1.
IMPLICIT_PLAN_BASE, IMPLICIT_PLAN_SLICES = 16, 128
CONV_GRAD_TILE = 64                    # pixels per tile of the transposed-gradient kernel
ROWS_PATH_MAX_PIXELS = 0               # conv forward through a rows GEMM + epilogue below this OH*OW
# How convolutions form their GEMM operand: "implicit" gathers the im2col view inside the GEMM's
# loads (no cols buffer); "im2col" writes cols (N*OH*OW x CI*KH*KW) first and keeps it for dW.
CONV_ALGORITHMS = ("implicit", "im2col")
IMPLICIT_PASSES = {"forward": 0, "dw": 1, "dx": 2}
CHANNEL_CHUNK = 32        # implicit products take features in chunks of this many channels per tap
BIAS_PARTIAL_ROWS = 256   # rows of FP64 bias partials a dW product may write (its pixel slices)
CONV_WFLIP_READY, CONV_ACCUMULATE_DX, CONV_COLUMN_ORDER = 1, 2, 4  # flags of mfh_conv_backward_implicit
_STATUS_TEXT = {1: "initialization failed", 2: "invalid argument", 3: "HIP runtime error", 5: "wrong HIP device"}


class NativeHipError(RuntimeError):
    """A libmfhip call returned a non-zero status; the message carries the library's reason."""


class AdamTensor(ctypes.Structure):
    """One row of the mfh_adam_step table (include/mfhip.h)."""
    _fields_ = [("param", ctypes.c_uint64), ("grad", ctypes.c_uint64), ("m", ctypes.c_uint64),
                ("v", ctypes.c_uint64), ("size", ctypes.c_int64), ("lr", ctypes.c_float),
                ("weight_decay", ctypes.c_float), ("bias_correction1", ctypes.c_float),
                ("bias_correction2", ctypes.c_float)]


# Argument codes: p device pointer / stream (uint64), i int32, q int64, f float, d double,
# t pointer to an AdamTensor table, P pointer to int32 (host array), U pointer to uint64 (host array),
# L pointer to int64.
_CTYPE = {"p": ctypes.c_uint64, "i": ctypes.c_int, "q": ctypes.c_int64, "f": ctypes.c_float, "d": ctypes.c_double,
          "t": ctypes.POINTER(AdamTensor), "P": ctypes.POINTER(ctypes.c_int), "s": ctypes.c_char_p, "-": None,
          "U": ctypes.POINTER(ctypes.c_uint64), "L": ctypes.POINTER(ctypes.c_int64)}
_CONV = "i" * 13
# symbol: (result code, argument codes); mirrors include/mfhip.h.
_SIGNATURES = {
    "mfh_init": ("i", ""),
    "mfh_last_error": ("s", ""),
    "mfh_info": ("s", ""),
    "mfh_set_debug_sync": ("-", "i"),
    "mfh_stream_wait": ("i", "pp"),
    "mfh_program_begin": ("i", ""),
    "mfh_program_end": ("i", "UL"),
    "mfh_program_run": ("i", "p"),
    "mfh_program_free": ("-", "p"),
    "mfh_fill": ("i", "pqfp"),
    "mfh_conv_im2col": ("i", "pp" + _CONV + "p"),
    "mfh_conv_col2im": ("i", "pp" + _CONV + "iip"),
    "mfh_conv_forward": ("i", "pppppp" + _CONV + "ifipqp"),
    "mfh_conv_backward": ("i", "pppppppppp" + _CONV + "iifiipqp"),
    "mfh_conv_backward_single": ("i", "pppppppppp" + _CONV + "iifipqp"),
    "mfh_conv_forward_implicit": ("i", "pppippp" + _CONV + "ifipqp"),
    "mfh_conv_forward_implicit_deferred": ("i", "pppipp" + _CONV + "ipqPp"),
    "mfh_conv_weight_orders": ("i", "UUPip"),
    "mfh_conv_implicit_workspace": ("q", _CONV + "i"),
    "mfh_conv_backward_implicit": ("i", "ppppppppppp" + _CONV + "ifiiipqp"),
    "mfh_conv_backward_implicit_streams": ("i", "ppppppppppp" + _CONV + "ifiiipqqpp"),
    "mfh_conv_backward_implicit_deferred": ("i", "ppppppppppp" + _CONV + "ifiiipqqPpp"),
    "mfh_pool_forward": ("i", "ppp" + "i" * 10 + "p"),
    "mfh_pool_backward": ("i", "ppp" + "i" * 10 + "p"),
    "mfh_matmul": ("i", "iiipppp" + "iii" + "p"),
    "mfh_gemm_tile_count": ("i", ""),
    "mfh_gemm_tile_info": ("i", "iP"),
    "mfh_gemm_tile_stages": ("i", "i"),
    "mfh_gemm_tile_groups": ("i", "i"),
    "mfh_gemm_plan": ("i", "iiiPP"),
    "mfh_gemm_workspace": ("q", "iii"),
    "mfh_split_reduce": ("i", "pp" + "iiiii" + "p"),
    "mfh_gemm": ("i", "iiipppp" + "iiiiii" + "pqp"),
    "mfh_gemm_noalloc": ("i", "iiipppp" + "iiiiii" + "p"),
    "mfh_bn_workspace": ("q", "iii"),
    "mfh_bn_forward": ("i", "ppppppppppq" + "iiiii" + "ddd" + "p"),
    "mfh_bn_forward_split": ("i", "pip" + "p" * 9 + "iiii" + "ddd" + "p"),
    "mfh_bn_backward": ("i", "pppppppppppq" + "iii" + "iiiii" + "p"),
    "mfh_bn_backward_split": ("i", "pi" + "pppppppppppq" + "iii" + "iiiii" + "p"),
    "mfh_bn_relu_pool_supported": ("i", "iiiiiiii"),
    "mfh_bn_relu_pool_forward": ("i", "pppppppppp" + "q" + "iiiiiiii" + "i" + "ddd" + "p"),
    "mfh_bn_relu_pool_backward": ("i", "pppppppppp" + "pq" + "iiiiiiii" + "iiii" + "p"),
    "mfh_relu_forward": ("i", "ppqp"),
    "mfh_relu_backward": ("i", "pppqfip"),
    "mfh_adam_step": ("i", "ti" + "ffffff" + "p"),
    "mfh_plane_mean": ("i", "ppqip"),
    "mfh_plane_mean_backward": ("i", "ppqiip"),
    "mfh_mse_loss": ("i", "pppqp"),
    "mfh_mse_loss_backward": ("i", "ppppqip"),
    "mfh_column_sums": ("i", "ppqqp"),
}
EXPORTS = tuple(_SIGNATURES)


def _declare(lib):
    for name, (result, arguments) in _SIGNATURES.items():
        function = getattr(lib, name)
        function.restype = _CTYPE[result]
        function.argtypes = [_CTYPE[code] for code in arguments]
    return lib


def load_library():
    """dlopen libmfhip.so and declare its signatures, without touching the GPU (builds it first when
    it is missing, unless MFHIP_AUTOBUILD=0)."""
    if not LIBRARY_PATH.exists():
        if os.environ.get("MFHIP_AUTOBUILD", "1") == "0":
            raise NativeHipError(f"{LIBRARY_PATH} is missing and MFHIP_AUTOBUILD=0; run myflows_amd/build.py")
        try:
            _build.build()
        except (_build.BuildError, OSError) as exc:
            raise NativeHipError(f"could not build {LIBRARY_PATH}: {exc}") from exc
    return _declare(ctypes.CDLL(str(LIBRARY_PATH)))


@lru_cache(maxsize=1)
def _library():
    if not torch.cuda.is_available():
        raise NativeHipError("the hip_native backend needs a HIP GPU and none is visible")
    lib = load_library()
    torch.empty(1, device="cuda")  # make PyTorch create its context on the current device first
    _raise_for(lib.mfh_init(), lib)
    return lib


def _raise_for(status, lib):
    if status:
        reason = lib.mfh_last_error().decode(errors="replace")
        raise NativeHipError(f"native HIP {_STATUS_TEXT.get(status, 'call failed')} ({status}): {reason}")


def _call(symbol, *args):
    """Call a status-returning entry point on the current stream; raise on failure."""
    lib = _library()
    _raise_for(getattr(lib, symbol)(*args), lib)


def _addr(tensor):
    return 0 if tensor is None else tensor.data_ptr()


_launch = threading.local()


def _stream():
    """The raw handle (hipStream_t) the library's calls are issued on: the one set by launch_stream,
    else the current stream on the current device. torch's own accessor is taken directly:
    torch.cuda.current_stream() costs several microseconds of Python per call, paid for every
    launch."""
    override = getattr(_launch, "stream", None)
    return override if override is not None else _raw_stream(_current_device())


@contextlib.contextmanager
def launch_stream(handle):
    """Issue the library calls made in the block (on this thread) on raw stream `handle` instead of
    the current stream. Tensors are still allocated on the current stream: the caller orders
    `handle` after the current stream's work on them (stream_wait) and the current stream after
    `handle` before that memory is read or freed there."""
    previous = getattr(_launch, "stream", None)
    _launch.stream = handle
    try:
        yield
    finally:
        _launch.stream = previous


try:
    _raw_stream, _current_device = torch._C._cuda_getCurrentRawStream, torch._C._cuda_getDevice
except AttributeError:  # another torch build: the public accessors
    _raw_stream = lambda device: torch.cuda.current_stream(device).cuda_stream  # noqa: E731
    _current_device = torch.cuda.current_device


def current_device_index():
    return _current_device()


def stream_wait(waiting, signalling):
    """Raw stream `waiting` runs nothing issued after this call before the work issued so far on
    raw stream `signalling` has finished (mfh_stream_wait)."""
    _call("mfh_stream_wait", waiting, signalling)


def fill_(tensor, value):
    """tensor[...] = value (a contiguous float32 GPU tensor), as one library launch on the current
    stream (mfh_fill)."""
    tensor = _device_f32(tensor, "tensor")
    _call("mfh_fill", tensor.data_ptr(), tensor.numel(), float(value), _stream())
    return tensor


def program_begin():
    """Record every launch and stream ordering the library issues on this thread from now on into a
    program (mfh_program_begin); program_end returns it."""
    _call("mfh_program_begin")


def program_end():
    """(handle, kernel launches) of the program recorded since program_begin."""
    handle, launches = ctypes.c_uint64(0), ctypes.c_int64(0)
    _call("mfh_program_end", ctypes.byref(handle), ctypes.byref(launches))
    return handle.value, launches.value


def program_run(handle):
    """Issue a recorded program again (mfh_program_run)."""
    _call("mfh_program_run", handle)


def program_free(handle):
    _library().mfh_program_free(handle)


def is_available():
    return LIBRARY_PATH.exists() and torch.cuda.is_available()


def library_status():
    """Where the library is and whether it loads here, without initialising a device."""
    return {"path": str(LIBRARY_PATH), "built": LIBRARY_PATH.exists(), "stale": _build.stale_reason(),
            "gpu": torch.cuda.is_available()}


def info():
    """Device and build facts of the loaded library: device_arch, cu_count, binary, load_ms, ..."""
    return json.loads(_library().mfh_info().decode())


def set_debug_sync(enabled=True):
    """Synchronise after every native launch so that an asynchronous fault names its kernel."""
    _library().mfh_set_debug_sync(1 if enabled else 0)


# ---------------------------------------------------------------------------------------------
# argument checks shared by the entry points
# ---------------------------------------------------------------------------------------------
_F32 = torch.float32


def _device_f32(value, name):
    if not (isinstance(value, torch.Tensor) and value.dtype is _F32 and value.is_cuda):
        raise TypeError(f"{name} must be a float32 torch tensor on the GPU")
    return value if value.is_contiguous() else value.contiguous()


def _within_int32(**counts):
    for name, count in counts.items():
        if int(count) > INT32_LIMIT:
            raise ValueError(f"{name} would hold {int(count)} elements but native kernels use int32 offsets "
                             f"(at most {INT32_LIMIT}); split the batch")


def _pair(value, name, minimum):
    pair = tuple(int(v) for v in value)
    if len(pair) != 2 or min(pair) < minimum:
        raise ValueError(f"{name} must be two integers >= {minimum}")
    return pair


def _activation_code(activation, alpha):
    if activation not in ACTIVATION_CODES:
        raise ValueError(f"activation must be None, 'relu' or 'leaky_relu', not {activation!r}")
    alpha = float(alpha)
    if activation == "leaky_relu" and not alpha > 0.0:
        raise ValueError("a fused leaky_relu needs alpha > 0")
    return ACTIVATION_CODES[activation], alpha


def _engine_code(engine):
    try:
        return GEMM_ENGINES[engine]
    except (KeyError, TypeError):
        raise ValueError(f"engine must be one of {sorted(GEMM_ENGINES)}, not {engine!r}") from None


@dataclass(frozen=True)
class ConvGeometry:
    """Sizes of one convolution, in the order of the C ABI's 13 dimension arguments."""
    n: int
    ci: int
    h: int
    w: int
    co: int
    kh: int
    kw: int
    oh: int
    ow: int
    sh: int
    sw: int
    ph: int
    pw: int

    @classmethod
    def of(cls, x_shape, weight_shape, stride, padding):
        """The checked geometry; one shared instance per (shapes, stride, padding), since a network
        asks for the same few geometries at every step."""
        try:
            return _conv_geometry(x_shape, weight_shape, stride, padding)
        except TypeError:  # an unhashable stride or padding (a list): not cached
            return cls._checked(x_shape, weight_shape, stride, padding)

    @classmethod
    def _checked(cls, x_shape, weight_shape, stride, padding):
        if len(x_shape) != 4 or len(weight_shape) != 4 or x_shape[1] != weight_shape[1]:
            raise ValueError("x and weight must be NCHW and OIHW with the same input channels")
        (sh, sw), (ph, pw) = _pair(stride, "stride", 1), _pair(padding, "padding", 0)
        n, ci, h, w = (int(v) for v in x_shape)
        co, kh, kw = int(weight_shape[0]), int(weight_shape[2]), int(weight_shape[3])
        oh, ow = (h + 2 * ph - kh) // sh + 1, (w + 2 * pw - kw) // sw + 1
        if oh <= 0 or ow <= 0:
            raise ValueError("the convolution output would be empty")
        g = cls(n, ci, h, w, co, kh, kw, oh, ow, sh, sw, ph, pw)
        _within_int32(columns=g.m * g.k, output=g.m * co, input=n * ci * h * w)
        if n > GRID_LIMIT:
            raise ValueError(f"native convolution takes at most {GRID_LIMIT} samples per call")
        return g

    @property
    def ohw(self):
        return self.oh * self.ow

    @property
    def m(self):
        return self.n * self.oh * self.ow

    @property
    def k(self):
        return self.ci * self.kh * self.kw

    @property
    def out_shape(self):
        return (self.n, self.co, self.oh, self.ow)

    def c_args(self):
        return (self.n, self.ci, self.h, self.w, self.co, self.kh, self.kw, self.oh, self.ow, self.sh, self.sw,
                self.ph, self.pw)


@lru_cache(maxsize=1024)
def _conv_geometry(x_shape, weight_shape, stride, padding):
    return ConvGeometry._checked(x_shape, weight_shape, stride, padding)


# ---------------------------------------------------------------------------------------------
# GEMM plans and workspaces
# ---------------------------------------------------------------------------------------------
@lru_cache(maxsize=1)
def tile_catalog():
    """Tile name -> (index, BM, BN, WM, WN, BK) of the MFMA engine, in native order. A tile is named
    "BMxBN", or "BMxBNkG" when G groups of waves share its K range (mfh_gemm_tile_groups)."""
    lib = load_library()
    catalog = {}
    for index in range(lib.mfh_gemm_tile_count()):
        values = (ctypes.c_int * 5)()
        _raise_for(lib.mfh_gemm_tile_info(index, values), lib)
        groups = lib.mfh_gemm_tile_groups(index)
        if lib.mfh_gemm_tile_stages(index) < 0 or groups < 1:
            _raise_for(2, lib)
        bm, bn, wm, wn, bk = values
        catalog[f"{bm}x{bn}" + (f"k{groups}" if groups > 1 else "")] = (index, bm, bn, wm, wn, bk)
    return catalog


def tile_groups(tile):
    """K groups of a tile of tile_catalog(): 1, or the wave sets that share its K range (each sums
    its run of stages, the runs then added in group order: another order than the one-group tiles)."""
    return load_library().mfh_gemm_tile_groups(tile_catalog()[tile][0])


@lru_cache(maxsize=2048)
def _plan_code(tile, requested):
    """Engine code of an explicit plan: a tile and a requested split-K slice count. A name of the
    reference's named tiles with at most 32 slices takes its named code (run on this library's tile
    of the same role, NAMED_TILE_OF); a name of this library's catalogue takes its extended code."""
    if type(requested) is not int or not 1 <= requested <= EXTENDED_PLAN_SLICES:
        raise ValueError(f"the split count must be an integer in [1, {EXTENDED_PLAN_SLICES}]")
    if tile in NAMED_TILES and requested <= NAMED_PLAN_SLICES:
        return NAMED_PLAN_BASE + NAMED_TILES.index(tile) * NAMED_PLAN_SLICES + requested - 1
    if tile not in tile_catalog():
        raise ValueError(f"unknown tile {tile!r}; the catalogue has {sorted(tile_catalog())}"
                         + (f" (named tiles take at most {NAMED_PLAN_SLICES} slices)" if tile in NAMED_TILES else ""))
    return EXTENDED_PLAN_BASE + tile_catalog()[tile][0] * EXTENDED_PLAN_SLICES + requested - 1


def _slices(k, requested, bk=16):
    """Slices a requested split of k really makes (chunks are whole BK stages)."""
    per_slice = -(-k // requested)
    chunk = min(k, -(-per_slice // bk) * bk)
    return -(-k // chunk)


def _explicit_tile(code):
    """(catalogue tile name, requested slices) of an explicit GEMM plan code."""
    if NAMED_PLAN_BASE <= code < NAMED_PLAN_BASE + len(NAMED_TILES) * NAMED_PLAN_SLICES:
        named, part = divmod(code - NAMED_PLAN_BASE, NAMED_PLAN_SLICES)
        return NAMED_TILE_OF[NAMED_TILES[named]], part + 1
    index, part = divmod(code - EXTENDED_PLAN_BASE, EXTENDED_PLAN_SLICES)
    if code < EXTENDED_PLAN_BASE or index >= len(tile_catalog()):
        raise ValueError(f"unknown GEMM plan code {code}")
    return list(tile_catalog())[index], part + 1


def _explicit_split(code):
    """(requested slices, BK) of an explicit plan code."""
    tile, requested = _explicit_tile(code)
    return requested, tile_catalog()[tile][-1]


def _engine_for(engine, layout, m, n, k):
    """The automatic engine, or the autotuned plan when MFHIP_GEMM_AUTOTUNE=1."""
    if engine == GEMM_ENGINES["mfma"] and os.environ.get("MFHIP_GEMM_AUTOTUNE") == "1":
        from .autotune import selected_plan
        return _plan_code(*selected_plan(layout, m, n, k))
    return engine


def _workspace_floats(engine, m, n, k):
    if engine == GEMM_ENGINES["mfma"]:
        floats = _library().mfh_gemm_workspace(m, n, k)
        if floats < 0:
            _raise_for(2, _library())
        return floats
    requested, bk = _explicit_split(engine)
    slices = _slices(k, requested, bk)
    return slices * m * n if slices > 1 else 0


def _workspace(*problems):
    """One float32 buffer large enough for every (engine, m, n, k) GEMM of a call (they run in
    stream order, so they can share it); (None, 0) when none of them splits K."""
    floats = max((_workspace_floats(*p) for p in problems), default=0)
    if not floats:
        return None, 0
    return torch.empty(floats, dtype=torch.float32, device="cuda"), floats


@lru_cache(maxsize=8)
def _cu_count(device_index):
    return int(torch.cuda.get_device_properties(device_index).multi_processor_count)


def _grad_tiles(n, ohw, co, device_index):
    """Pixel tiles per image of the transposed-gradient kernel: enough workgroups to fill the GPU
    (about 8 per CU), at most one per 64-pixel tile."""
    tiles = -(-ohw // CONV_GRAD_TILE)
    wanted = -(-8 * _cu_count(device_index) // max(1, n * -(-co // CONV_GRAD_TILE)))
    return max(1, min(tiles, wanted))


# ---------------------------------------------------------------------------------------------
# convolution
# ---------------------------------------------------------------------------------------------
def conv2d_im2col(x, kernel_shape, *, stride=(1, 1), padding=(0, 0)):
    """The im2col matrix (N*OH*OW, CI*KH*KW) of x for a kernel of shape (CO, CI, KH, KW)."""
    x = _device_f32(x, "x")
    g = ConvGeometry.of(tuple(x.shape), tuple(kernel_shape), stride, padding)
    cols = torch.empty((g.m, g.k), dtype=torch.float32, device=x.device)
    _call("mfh_conv_im2col", x.data_ptr(), cols.data_ptr(), *g.c_args(), _stream())
    return cols


def conv2d_col2im(grad_cols, x_shape, kernel_shape, *, stride=(1, 1), padding=(0, 0), per_image=True, out=None,
                  accumulate=False):
    """dx of shape x_shape from a feature-major column gradient (mfh_conv_col2im): grad_cols holds
    [n][CI*KH*KW][OH*OW] when per_image, else [CI*KH*KW][N*OH*OW]. With out and accumulate, the sums
    are added to out."""
    grad_cols = _device_f32(grad_cols, "grad_cols")
    g = ConvGeometry.of(tuple(x_shape), tuple(kernel_shape), stride, padding)
    if grad_cols.numel() != g.m * g.k:
        raise ValueError("grad_cols must hold N*OH*OW*CI*KH*KW floats")
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs out")
        out = torch.empty(tuple(x_shape), dtype=torch.float32, device=grad_cols.device)
    elif not (isinstance(out, torch.Tensor) and out.dtype == torch.float32 and out.is_contiguous()
              and tuple(out.shape) == tuple(x_shape) and out.device == grad_cols.device):
        raise ValueError("out must be a contiguous float32 tensor of x's shape on grad_cols' device")
    _call("mfh_conv_col2im", grad_cols.data_ptr(), out.data_ptr(), *g.c_args(), int(bool(per_image)),
          int(bool(accumulate)), _stream())
    return out


def default_conv_algorithm():
    """The convolution algorithm of calls that do not name one: MFHIP_CONV_ALGO, else "implicit"."""
    return _conv_algorithm(os.environ.get("MFHIP_CONV_ALGO", "implicit"))


def _conv_algorithm(algorithm):
    if algorithm is None:
        return default_conv_algorithm()
    if algorithm not in CONV_ALGORITHMS:
        raise ValueError(f"algorithm must be one of {CONV_ALGORITHMS}, not {algorithm!r}")
    return algorithm


def _implicit_workspace_floats(g, pass_name):
    # Kept with the (shared) geometry instance: hashing a geometry costs more than the lookup.
    memo = g.__dict__.setdefault("_workspace_floats", {})
    floats = memo.get(pass_name)
    if floats is None:
        floats = _library().mfh_conv_implicit_workspace(*g.c_args(), IMPLICIT_PASSES[pass_name])
        if floats < 0:
            _raise_for(2, _library())
        memo[pass_name] = floats
    return floats


_STREAM_WORKSPACES = {}


def stream_workspace(count, dtype=torch.float32):
    """A scratch tensor of at least `count` elements for a call issued on the current stream, kept
    per (device, stream, dtype) and handed to every such call: calls on one stream run one after the
    other, so two of them never use it at the same time. A larger request replaces it (the old block
    goes back to torch's allocator on the same stream). The calls a training step makes would
    otherwise allocate and free one per launch."""
    key = (_current_device(), _stream(), dtype)
    held = _STREAM_WORKSPACES.get(key)
    if held is None or held.numel() < count or (_PENDING_SPLITS and _holds_pending_split(held)):
        # A block whose split-K slices still wait for their batch norm is never handed out again:
        # this call takes a fresh one (the pending entry keeps the old block until it is formed).
        held = torch.empty(count, dtype=dtype, device="cuda")
        _STREAM_WORKSPACES[key] = held
    return held


def _holds_pending_split(block):
    return any(entry[1] is block for entry in _PENDING_SPLITS.values())


def _implicit_workspace(g, *passes):
    floats = max((_implicit_workspace_floats(g, p) for p in passes), default=0)
    if not floats:
        return None, 0
    return stream_workspace(floats), floats


def implicit_chunked(channels):
    """Whether an implicit product over this many channels reads them in chunks of CHANNEL_CHUNK."""
    return int(channels) % CHANNEL_CHUNK == 0


# Floats of the largest tensor a chunked implicit product reads: its buffer loads take 32-bit byte
# offsets (2 GiB).
BUFFER_LIMIT_FLOATS = (2 ** 31 - 1) // 4


def implicit_fits(g):
    """Whether every implicit product of this convolution (forward, dW, dX) can read its tensors:
    a chunked product reads x, dy and the kernel orders with buffer loads of at most
    BUFFER_LIMIT_FLOATS floats. The geometry's own int32 limits leave only large 1x1-like
    convolutions outside; those take the im2col algorithm by default."""
    if not (implicit_chunked(g.ci) or implicit_chunked(g.co)):
        return True
    return max(g.n * g.ci * g.h * g.w, g.m * g.co, g.co * g.k) <= BUFFER_LIMIT_FLOATS


def _default_algorithm_for(g, algorithm):
    """The algorithm a call runs: the one asked for, else the default, which is im2col for a
    convolution whose tensors the implicit products cannot read (implicit_fits)."""
    if algorithm is not None:
        return _conv_algorithm(algorithm)
    algorithm = default_conv_algorithm()
    return algorithm if algorithm != "implicit" or implicit_fits(g) else "im2col"


def conv_weight_orders(requests):
    """The kernels of several convolutions in the orders the implicit products read them, from one
    launch: requests = [(weight (CO, CI, KH, KW), flip)] or [(weight, flip, stride, padding)], flip 0
    for the forward (pass the result to conv2d_forward as weight_order), 1 for the dX
    (conv2d_backward's weight_flip); a strided dX order (the phase sub-kernels) depends on the
    convolution's stride and padding, which default to (1, 1) and (0, 0).
    Returns one flat float32 tensor per request."""
    requests = list(requests)
    if not requests:
        return []
    weights, outs, dims = [], [], []
    for request in requests:
        weight, flip = request[0], request[1]
        stride = _pair(request[2], "stride", 1) if len(request) > 2 else (1, 1)
        padding = _pair(request[3], "padding", 0) if len(request) > 3 else (0, 0)
        weight = _device_f32(weight, "weight")
        if weight.ndim != 4:
            raise ValueError("weight must have shape (CO, CI, KH, KW)")
        if flip not in (0, 1):
            raise ValueError("flip must be 0 or 1")
        out = torch.empty(weight.numel(), dtype=torch.float32, device=weight.device)
        weights.append(weight)
        outs.append(out)
        dims.extend((*(int(v) for v in weight.shape), int(flip), *stride, *padding))
    count = len(requests)
    _call("mfh_conv_weight_orders", (ctypes.c_uint64 * count)(*(w.data_ptr() for w in weights)),
          (ctypes.c_uint64 * count)(*(o.data_ptr() for o in outs)), (ctypes.c_int * len(dims))(*dims), count,
          _stream())
    return outs


# Longest phase product (CO x its taps) that the automatic choice still runs as phases.
PHASE_MAX_K = 1024


def strided_dx_phases(kh, kw, co, stride):
    """Whether conv2d_backward's automatic choice runs a strided dX as phase products: a 1x1 kernel
    (one phase product), or phases of at most PHASE_MAX_K reduction depth, which all run in one
    launch. Measured on MI355X for ResNet18 at batch 64: the layer2 and layer3 3x3 stride-2 dX
    (K up to 512 and 1024) take 47 and 55 us as phases against 67 and 71 us through the column
    gradient; layer4's (K 2048, few pixels) 83 us against 67 us."""
    sh, sw = (int(v) for v in stride)
    longest = -(-int(kh) // sh) * -(-int(kw) // sw)
    return int(kh) * int(kw) == 1 or int(co) * longest <= PHASE_MAX_K


def _weight_order_buffer(order, weight, name):
    order = _device_f32(order, name)
    if order.numel() != weight.numel() or order.data_ptr() % 16:
        raise ValueError(f"{name} must be a 16-byte aligned float32 tensor of the kernel's size")
    return order


def conv2d_forward(x, weight, bias=None, *, stride=(1, 1), padding=(0, 0), activation=None, alpha=0.0,
                   engine="mfma", algorithm=None, weight_order=None, residual=None):
    """(y, cols): the contiguous NCHW output with bias and activation applied, and the im2col
    columns of x that conv2d_backward needs for dW. With algorithm "implicit" (the default) the GEMM
    gathers the columns from x itself and cols is None; "im2col" writes and returns them. Without an
    algorithm, a convolution whose tensors the implicit products cannot read (implicit_fits) takes
    "im2col".
    weight_order: this kernel from conv_weight_orders(flip 0), which the implicit product then reads
    instead of reordering the kernel itself. residual (implicit only): a tensor of y's shape added
    to conv + bias before the activation, act((conv + bias) + residual), each step one float32
    rounding as in separate Add and activation operators."""
    engine = _engine_code(engine)
    if algorithm is not None:
        algorithm = _conv_algorithm(algorithm)
    x, weight = _device_f32(x, "x"), _device_f32(weight, "weight")
    if bias is not None:
        bias = _device_f32(bias, "bias")
        if tuple(bias.shape) != (weight.shape[0],):
            raise ValueError("bias must have shape (out_channels,)")
    g = ConvGeometry.of(x.shape, weight.shape, stride, padding)
    algorithm = _default_algorithm_for(g, algorithm)
    act, alpha = _activation_code(activation, alpha)
    device = x.device
    y = torch.empty(g.out_shape, dtype=torch.float32, device=device)
    if residual is not None:
        if algorithm != "implicit":
            raise ValueError("a residual is added by the implicit algorithm's epilogue only")
        residual = _device_f32(residual, "residual")
        if tuple(residual.shape) != g.out_shape:
            raise ValueError("residual must have the convolution's output shape")
        if residual.device != device:
            raise ValueError("residual must be on x's device")
    if algorithm == "implicit":
        workspace, floats = _implicit_workspace(g, "forward")
        prepared = 0
        wt = None
        if implicit_chunked(g.ci):  # the kernel in chunked feature order
            if weight_order is not None:
                wt, prepared = _weight_order_buffer(weight_order, weight, "weight_order"), 1
            else:
                wt = torch.empty_like(weight)
        _call("mfh_conv_forward_implicit", x.data_ptr(), weight.data_ptr(), _addr(wt), prepared, _addr(bias),
              _addr(residual), y.data_ptr(), *g.c_args(), act, alpha, engine, _addr(workspace), floats, _stream())
        return y, None
    cols = torch.empty((g.m, g.k), dtype=torch.float32, device=device)
    rows = None
    if g.ohw < ROWS_PATH_MAX_PIXELS:  # rows = cols W^T, then the NCHW epilogue kernel
        rows = torch.empty((g.m, g.co), dtype=torch.float32, device=device)
        engine = _engine_for(engine, "NT", g.m, g.co, g.k)
        workspace, floats = _workspace((engine, g.m, g.co, g.k))
    else:  # one GEMM W cols^T over all images, stored into NCHW
        workspace, floats = _workspace((engine, g.co, g.m, g.k))
    _call("mfh_conv_forward", x.data_ptr(), weight.data_ptr(), _addr(bias), cols.data_ptr(), _addr(rows),
          y.data_ptr(), *g.c_args(), act, alpha, engine, _addr(workspace), floats, _stream())
    return y, cols


# Convolution outputs (and input gradients) whose split-K slices still wait in a workspace block
# (see conv2d_forward_deferred, conv2d_backward's defer_dx_positions):
# id(y) -> (y, block, slices, bias, offset of the slices in the block in floats).
_PENDING_SPLITS = {}


def conv2d_forward_deferred(x, weight, bias=None, *, stride=(1, 1), padding=(0, 0), engine="mfma", weight_order=None,
                            max_positions=0):
    """conv2d_forward (implicit, no residual or activation) for a caller that forms y itself:
    when the output has at most max_positions positions per channel (N * OH * OW) and the product's
    plan splits K, y is returned unwritten and its slices stay in this stream's convolution
    workspace, registered for take_pending_split(y); the next batch-norm forward of y
    (fused.batchnorm2d_forward) must form y before this stream runs another convolution. Otherwise
    y is complete, as from conv2d_forward."""
    x, weight = _device_f32(x, "x"), _device_f32(weight, "weight")
    g = ConvGeometry.of(x.shape, weight.shape, stride, padding)
    n, _, oh, ow = g.out_shape
    if n * oh * ow > max_positions:
        return conv2d_forward(x, weight, bias, stride=stride, padding=padding, engine=engine, algorithm="implicit",
                              weight_order=weight_order)[0]
    if bias is not None:
        bias = _device_f32(bias, "bias")
        if tuple(bias.shape) != (weight.shape[0],):
            raise ValueError("bias must have shape (out_channels,)")
    engine = _engine_code(engine)
    y = torch.empty(g.out_shape, dtype=torch.float32, device=x.device)
    workspace, floats = _implicit_workspace(g, "forward")
    prepared, wt = 0, None
    if implicit_chunked(g.ci):
        if weight_order is not None:
            wt, prepared = _weight_order_buffer(weight_order, weight, "weight_order"), 1
        else:
            wt = torch.empty_like(weight)
    slices = ctypes.c_int(1)
    _call("mfh_conv_forward_implicit_deferred", x.data_ptr(), weight.data_ptr(), _addr(wt), prepared, _addr(bias),
          y.data_ptr(),
          *g.c_args(), engine, _addr(workspace), floats, ctypes.byref(slices), _stream())
    if slices.value > 1:
        _PENDING_SPLITS[id(y)] = (y, workspace, slices.value, bias, 0)
    return y


def drop_pending_splits():
    """Forget every output left unformed by conv2d_forward_deferred (their batch norms never ran,
    e.g. an earlier forward raised between the product and the batch norm); the outputs stay
    unwritten and their workspace blocks go back to the allocator."""
    _PENDING_SPLITS.clear()


def take_pending_split(y):
    """(address of the slices, slices, bias, block) of a convolution output left unformed by
    conv2d_forward_deferred (or an input gradient left unformed by conv2d_backward with
    defer_dx_positions; bias None), else None; the caller then forms y, holding the block (the
    workspace tensor the slices lie in) until its launch is queued."""
    entry = _PENDING_SPLITS.pop(id(y), None)
    if entry is None:
        return None
    if entry[0] is not y:  # a stale entry of a freed tensor whose id was reused
        return None
    _, block, slices, bias, offset = entry
    return block.data_ptr() + 4 * offset, slices, bias, block


def conv2d_backward(x, weight, grad_y, cols, *, stride=(1, 1), padding=(0, 0), need_bias_grad=True,
                    need_input_grad=True, need_weight_grad=True, activation=None, alpha=0.0, output=None,
                    engine="mfma", recompute_cols=False, algorithm=None, weight_flip=None, input_grad=None,
                    strided_dx="auto", dw_stream=None, hold=None, defer_dx_positions=0):
    """(dx, dw, db), None for each gradient not requested; a fused activation gates grad_y through
    output. algorithm "im2col" computes dW from the forward's cols (recomputed from x when
    recompute_cols); "implicit" gathers them from x inside the GEMM. Without an algorithm, a call
    that passes cols (and does not recompute them) takes "im2col", any other the default (im2col,
    recomputing cols, where implicit_fits says the implicit products cannot read the tensors).
    Implicit only: weight_flip is this kernel from conv_weight_orders for the dX route taken (flip 1
    with this stride and padding for the dX orders; for the column route, the kernel seen as a
    (CO, CI*KH*KW, 1, 1) kernel with flip 1); input_grad is a gradient of x already there, to which
    dX is added in place (it is then the returned dx); strided_dx chooses how a strided
    convolution's dX runs: "phases" (one stride-1 implicit product per output phase, written to its
    lattice of dx), "columns" (the column gradient, then col2im: one implicit product over every
    image when CO is a multiple of 32, else a GEMM per image) or "auto" (strided_dx_phases decides).
    Implicit only: dw_stream (a raw stream handle of the current device) runs the dW and db
    products beside the dX product on the current stream (mfh_conv_backward_implicit_streams); dw
    and db are complete once the current stream has been ordered after dw_stream (stream_wait). The
    tensors are allocated on the current stream, so such a caller also passes a list as hold, which
    receives every tensor the call reads or writes, and keeps them until that ordering.
    Implicit only: with defer_dx_positions, a stride-1 convolution whose dx is fresh (no input_grad)
    and has at most that many positions per channel (N * H * W) may return dx unwritten, its dX
    product's split-K slices left in a workspace block registered for take_pending_split(dx)
    (mfh_conv_backward_implicit_deferred); the next batch-norm backward of dx
    (fused.batchnorm2d_backward with dy = dx) must form it. Otherwise dx is complete."""
    engine = _engine_code(engine)
    if algorithm is None and cols is not None and not recompute_cols:
        algorithm = "im2col"
    if algorithm is not None:
        algorithm = _conv_algorithm(algorithm)
    x, weight, grad_y = _device_f32(x, "x"), _device_f32(weight, "weight"), _device_f32(grad_y, "grad_y")
    g = ConvGeometry.of(x.shape, weight.shape, stride, padding)
    if algorithm is None:
        algorithm = _default_algorithm_for(g, None)
        recompute_cols = recompute_cols or (algorithm == "im2col" and cols is None)
    act, alpha = _activation_code(activation, alpha)
    if tuple(grad_y.shape) != g.out_shape:
        raise ValueError("grad_y does not have the convolution's output shape")
    if algorithm == "implicit":
        if strided_dx not in ("auto", "phases", "columns"):
            raise ValueError('strided_dx must be "auto", "phases" or "columns"')
        phases = strided_dx == "phases" or (strided_dx == "auto"
                                            and strided_dx_phases(g.kh, g.kw, g.co, (g.sh, g.sw)))
        return _conv2d_backward_implicit(x, weight, grad_y, g, need_bias_grad, need_input_grad, need_weight_grad,
                                         act, alpha, output, engine, weight_flip, input_grad, phases, dw_stream, hold,
                                         defer_dx_positions)
    if (weight_flip is not None or input_grad is not None or dw_stream is not None or hold is not None
            or defer_dx_positions):
        raise ValueError("weight_flip, input_grad, dw_stream, hold and defer_dx_positions apply to the implicit "
                         "algorithm only")
    if need_weight_grad:
        cols = (conv2d_im2col(x, tuple(weight.shape), stride=stride, padding=padding) if recompute_cols
                else _device_f32(cols, "cols"))
        if tuple(cols.shape) != (g.m, g.k):
            raise ValueError("cols does not match the convolution input")
    else:
        cols = None
    gate = None
    if act:
        if output is None:
            raise ValueError("a fused activation needs the forward output")
        gate = _device_f32(output, "output")
        if gate.shape != grad_y.shape:
            raise ValueError("output does not have grad_y's shape")
    if not (need_input_grad or need_weight_grad or need_bias_grad):
        return None, None, None
    device = x.device
    empty = lambda *shape, dtype=torch.float32: torch.empty(shape, dtype=dtype, device=device)
    tiles = _grad_tiles(g.n, g.ohw, g.co, device.index or 0)
    dy_rows = empty(g.m, g.co) if need_weight_grad or (need_input_grad and act) else None
    dw = torch.empty_like(weight) if need_weight_grad else None
    grad_cols = empty(g.m * g.k) if need_input_grad else None
    dx = torch.empty_like(x) if need_input_grad else None
    partial = empty(g.n * tiles * g.co, dtype=torch.float64) if need_bias_grad else None
    db = empty(g.co) if need_bias_grad else None
    dw_engine = _engine_for(engine, "TN", g.co, g.k, g.m) if need_weight_grad else engine
    workspace, floats = _workspace((dw_engine, g.co, g.k, g.m)) if need_weight_grad else (None, 0)
    _call("mfh_conv_backward", weight.data_ptr(), grad_y.data_ptr(), _addr(gate), _addr(cols), _addr(dy_rows),
          _addr(dw), _addr(grad_cols), _addr(dx), _addr(partial), _addr(db), *g.c_args(), tiles, act, alpha,
          dw_engine, engine, _addr(workspace), floats, _stream())
    return dx, dw, db


def _conv2d_backward_implicit(x, weight, grad_y, g, need_bias_grad, need_input_grad, need_weight_grad, act, alpha,
                              output, engine, weight_flip=None, input_grad=None, phases=True, dw_stream=None,
                              hold=None, defer_dx_positions=0):
    if dw_stream is not None and hold is None:
        raise ValueError("a dW product on another stream needs a hold list for the call's tensors")
    gate = None
    if act:
        if output is None:
            raise ValueError("a fused activation needs the forward output")
        gate = _device_f32(output, "output")
        if gate.shape != grad_y.shape:
            raise ValueError("output does not have grad_y's shape")
    if not (need_input_grad or need_weight_grad or need_bias_grad):
        return None, None, None
    device = x.device
    empty = lambda *shape, dtype=torch.float32: torch.empty(shape, dtype=dtype, device=device)
    unit_stride = g.sh == 1 and g.sw == 1
    flags = 0
    gated = torch.empty_like(grad_y) if act else None
    dw = torch.empty_like(weight) if need_weight_grad else None
    dx = None
    if need_input_grad:
        if input_grad is not None:
            if (not isinstance(input_grad, torch.Tensor) or input_grad.dtype != torch.float32
                    or tuple(input_grad.shape) != tuple(x.shape) or not input_grad.is_contiguous()
                    or input_grad.device != device):
                raise ValueError("input_grad must be a contiguous float32 tensor of x's shape on x's device")
            dx, flags = input_grad, flags | CONV_ACCUMULATE_DX
        else:
            dx = torch.empty_like(x)
    wflip = None
    through_orders = unit_stride or phases  # dX through the (phase) dX orders, else columns + col2im
    # The column gradient as one implicit product reads W through its column order (the dX order of
    # W seen as a 1x1 kernel of CI*KH*KW channels) when dy's channels come in chunks.
    column_order = need_input_grad and not through_orders and implicit_chunked(g.co)
    if need_input_grad and (through_orders or column_order):
        if weight_flip is not None:
            wflip, flags = _weight_order_buffer(weight_flip, weight, "weight_flip"), flags | CONV_WFLIP_READY
        else:
            wflip = empty(g.ci * g.co * g.kh * g.kw)
        if column_order:
            flags |= CONV_COLUMN_ORDER
    elif weight_flip is not None:
        raise ValueError("weight_flip applies to a dX through the dX orders or the column order")
    grad_cols = empty(g.m * g.k) if need_input_grad and not through_orders else None
    partial = empty(max(g.n, BIAS_PARTIAL_ROWS) * g.co, dtype=torch.float64) if need_bias_grad else None
    db = empty(g.co) if need_bias_grad else None
    passes = (("dw",) if need_weight_grad else ()) + (("dx",) if wflip is not None else ())
    pointers = (x.data_ptr(), weight.data_ptr(), grad_y.data_ptr(), _addr(gate), _addr(gated), _addr(dw), _addr(dx),
                _addr(wflip), _addr(grad_cols), _addr(partial), _addr(db), *g.c_args(), act, alpha, engine, engine,
                flags)
    defer = (need_input_grad and input_grad is None and unit_stride and 0 < defer_dx_positions
             and g.n * g.h * g.w <= defer_dx_positions)
    if dw_stream is None and not defer:
        workspace, floats = _implicit_workspace(g, *passes)
        _call("mfh_conv_backward_implicit", *pointers, _addr(workspace), floats, _stream())
    else:  # one workspace part each for the dW and dX products (which may run at the same time)
        dw_floats = _implicit_workspace_floats(g, "dw") if need_weight_grad else 0
        dx_floats = _implicit_workspace_floats(g, "dx") if "dx" in passes else 0
        floats = dw_floats + dx_floats
        if dw_stream is None:  # one stream: the block is this stream's workspace
            workspace = stream_workspace(floats) if floats else None
        else:
            workspace = torch.empty(floats, dtype=torch.float32, device="cuda") if floats else None
        if defer:
            slices = ctypes.c_int(1)
            _call("mfh_conv_backward_implicit_deferred", *pointers, _addr(workspace), dw_floats, floats,
                  ctypes.byref(slices), _stream(), _stream() if dw_stream is None else dw_stream)
            if slices.value > 1:
                _PENDING_SPLITS[id(dx)] = (dx, workspace, slices.value, None, dw_floats)
        else:
            _call("mfh_conv_backward_implicit_streams", *pointers, _addr(workspace), dw_floats, floats, _stream(),
                  dw_stream)
    if hold is not None:
        hold.extend(t for t in (x, weight, grad_y, gate, gated, dw, dx, wflip, grad_cols, partial, db, workspace)
                    if t is not None)
    return dx, dw, db


# ---------------------------------------------------------------------------------------------
# max pooling
# ---------------------------------------------------------------------------------------------
@dataclass
class NativePoolContext:
    """What maxpool2d_backward needs from the forward: shapes, window and the int32 argmax."""
    input_shape: tuple
    output_shape: tuple
    kernel_size: tuple
    stride: tuple
    argmax: object
    device_id: int

    def c_args(self):
        n, c, h, w = self.input_shape
        return (n, c, h, w, self.output_shape[2], self.output_shape[3], *self.kernel_size, *self.stride)


def maxpool2d_forward(x, *, kernel_size=(2, 2), stride=(2, 2), with_argmax=True):
    """(y, context) of a max-pool without padding: window maximum (first index wins ties, NaN wins)
    and its flat int32 index into x. Without with_argmax (a pass no backward follows) the index is
    not written and the context cannot take a backward."""
    x = _device_f32(x, "x")
    if x.ndim != 4:
        raise ValueError("x must be an NCHW tensor")
    kernel, step = _pair(kernel_size, "kernel_size", 1), _pair(stride, "stride", 1)
    n, c, h, w = (int(v) for v in x.shape)
    oh, ow = (h - kernel[0]) // step[0] + 1, (w - kernel[1]) // step[1] + 1
    if oh <= 0 or ow <= 0:
        raise ValueError("the pooling window does not fit in the input")
    _within_int32(input=n * c * h * w)
    y = torch.empty((n, c, oh, ow), dtype=torch.float32, device=x.device)
    argmax = torch.empty((n, c, oh, ow), dtype=torch.int32, device=x.device) if with_argmax else None
    context = NativePoolContext((n, c, h, w), (n, c, oh, ow), kernel, step, argmax, x.device.index)
    _call("mfh_pool_forward", x.data_ptr(), y.data_ptr(), _addr(argmax), *context.c_args(), _stream())
    return y, context


def maxpool2d_backward(grad_y, context):
    """dx: each dy goes to its window's argmax; overlapping windows add in (oh, ow) order."""
    if not isinstance(context, NativePoolContext) or context.device_id != torch.cuda.current_device():
        raise ValueError("context must come from maxpool2d_forward on the current device")
    if context.argmax is None:
        raise ValueError("the forward ran without its argmax (with_argmax=False): no backward")
    grad_y = _device_f32(grad_y, "grad_y")
    if tuple(grad_y.shape) != tuple(context.output_shape):
        raise ValueError("grad_y does not have the pooled output's shape")
    dx = torch.empty(context.input_shape, dtype=torch.float32, device=grad_y.device)
    _call("mfh_pool_backward", grad_y.data_ptr(), context.argmax.data_ptr(), dx.data_ptr(), *context.c_args(),
          _stream())
    return dx


# ---------------------------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------------------------
def _result(out, m, n, like):
    if out is None:
        return torch.empty((m, n), dtype=torch.float32, device=like.device)
    if (not isinstance(out, torch.Tensor) or out.dtype != torch.float32 or tuple(out.shape) != (m, n)
            or not out.is_contiguous() or out.device != like.device):
        raise ValueError("out must be a contiguous float32 GPU tensor of the result's shape")
    return out


def _bias_vector(bias, n):
    if bias is None:
        return None
    bias = _device_f32(bias, "bias").reshape(-1)
    if tuple(bias.shape) != (n,):
        raise ValueError("bias needs one value per output column")
    return bias


def matmul(a, b, bias=None, *, variant="shared", tile=32, accumulate="kahan", out=None):
    """Row-major ``a @ b (+ bias)`` on a teaching kernel.

    variant: basic (one thread per output), tiled (TILE x TILE workgroups over global memory), shared
    (TILE x TILE LDS tiles) or register (64 x 64 workgroup tiles, 4 x 4 outputs per thread; with
    accumulate="fp32" the MFMA engine). accumulate: fp32, kahan (grouped, compensated) or dot2.
    """
    if variant not in MATMUL_VARIANTS:
        raise ValueError(f"variant must be one of {sorted(MATMUL_VARIANTS)}")
    if accumulate not in MATMUL_ACCUMULATION:
        raise ValueError(f"accumulate must be one of {sorted(MATMUL_ACCUMULATION)}")
    if int(tile) not in (16, 32):
        raise ValueError("tile must be 16 or 32")
    a, b = _device_f32(a, "a"), _device_f32(b, "b")
    if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[0]:
        raise ValueError("matmul needs 2-D operands whose inner dimensions agree")
    m, k, n = int(a.shape[0]), int(a.shape[1]), int(b.shape[1])
    if min(m, n, k) <= 0:
        raise ValueError("matmul dimensions must be positive")
    _within_int32(a=m * k, b=k * n, c=m * n)
    bias = _bias_vector(bias, n)
    out = _result(out, m, n, a)
    _call("mfh_matmul", MATMUL_VARIANTS[variant], int(tile), MATMUL_ACCUMULATION[accumulate], a.data_ptr(),
          b.data_ptr(), _addr(bias), out.data_ptr(), m, n, k, _stream())
    return out


def gemm_plan(m, n, k, *, layout=None):
    """(tile name, split-K slices) the MFMA engine picks for an m x n output over k."""
    if min(m, n, k) <= 0:
        raise ValueError("gemm dimensions must be positive")
    if layout is not None and os.environ.get("MFHIP_GEMM_AUTOTUNE") == "1":
        from .autotune import selected_plan
        tile, requested = selected_plan(layout, m, n, k)
        return tile, _slices(k, requested, tile_catalog()[tile][-1])
    tile, slices = ctypes.c_int(), ctypes.c_int()
    _call("mfh_gemm_plan", m, n, k, ctypes.byref(tile), ctypes.byref(slices))
    return list(tile_catalog())[tile.value], slices.value


def split_reduce(partials, *, reference=False):
    """Sum split-K partials (slices x M x N, float32) the way the engine finishes a split GEMM: in
    FP64, in slice order, rounded once."""
    partials = _device_f32(partials, "partials")
    if partials.ndim != 3 or partials.shape[0] < 2:
        raise ValueError("partials must be a (slices >= 2, M, N) float32 tensor")
    slices, m, n = (int(v) for v in partials.shape)
    if min(m, n) <= 0:
        raise ValueError("partials must hold at least one output")
    _within_int32(partials=partials.numel())
    out = torch.empty((m, n), dtype=torch.float32, device=partials.device)
    _call("mfh_split_reduce", partials.data_ptr(), out.data_ptr(), slices, m, n, n, int(bool(reference)), _stream())
    return out


def gemm(a, b, bias=None, *, trans_a=False, trans_b=False, engine="mfma", out=None, plan=None):
    """Row-major ``op(a) @ op(b) (+ bias)`` on the MFMA engine (the automatic plan of a product with
    at most 8 output columns takes a one-wave-per-row kernel instead: lanes split K, a fixed
    butterfly adds them).

    op(a) = a.T when trans_a (a stored K x M), op(b) = b.T when trans_b (b stored N x K); not both.
    plan=(tile, slices) forces a tile of tile_catalog() and a split-K slice count.
    """
    engine = _engine_code(engine)
    if trans_a and trans_b:
        raise ValueError("gemm takes a.T @ b or a @ b.T, not a.T @ b.T")
    a, b = _device_f32(a, "a"), _device_f32(b, "b")
    if a.ndim != 2 or b.ndim != 2:
        raise ValueError("gemm needs 2-D operands")
    k, m = (int(a.shape[0]), int(a.shape[1])) if trans_a else (int(a.shape[1]), int(a.shape[0]))
    n, k_b = (int(b.shape[0]), int(b.shape[1])) if trans_b else (int(b.shape[1]), int(b.shape[0]))
    if k != k_b:
        raise ValueError("gemm operands disagree on the inner dimension")
    if min(m, n, k) <= 0:
        raise ValueError("gemm dimensions must be positive")
    _within_int32(a=m * k, b=k * n, c=m * n)
    bias = _bias_vector(bias, n)
    out = _result(out, m, n, a)
    if plan is not None:
        engine = _plan_code(*plan)
    else:
        engine = _engine_for(engine, "TN" if trans_a else "NT" if trans_b else "NN", m, n, k)
    workspace, floats = _workspace((engine, m, n, k))
    _call("mfh_gemm", engine, int(bool(trans_a)), int(bool(trans_b)), a.data_ptr(), b.data_ptr(), _addr(bias),
          out.data_ptr(), m, n, k, int(a.shape[1]), int(b.shape[1]), n, _addr(workspace), floats, _stream())
    return out
