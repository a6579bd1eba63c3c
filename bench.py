"""Benchmark of the hip_native hot path on one MI355X.

Workload: one ResNet18(output_dim=2) training step with Adam through the
Variable/Graph API, every convolution, the stem max-pool, the fc Linear, batch norm, ReLU and Adam
on libmfhip; batch 64, input 3x120x160 ~ N(0, 1), targets ~ U(-1, 1), MSE loss, Kaiming weights
from seed 0 (synthetic data, random-init weights of the reference architecture). The graph is built
with Graph(optimize=True), which runs BN+ReLU, BN+Add+ReLU and the stem's BN+ReLU+max-pool as single
units (--plain-graph keeps them as separate nodes, as the reference's own training task does); each
backward convolution runs its dW product on a second stream beside its dX (--single-stream keeps
one stream). ``value`` is images per second over the timed steps.

``roofline`` is the FP32 MFMA GEMM engine on the 4096^3 GEMM of BASELINE config 2 (the metric's
"GEMM TFLOP/s vs FP32 peak"): algorithmic 2*M*N*K flop per launch divided by the average launch
time measured with HIP events on the launch stream, against the 157.3 TFLOP/s FP32 matrix peak.
``cpu_baseline`` is the NumPy restatement of the reference CPU path (oracle/resnet.py) timed on this
host on a bounded sample: full forward + backward + Adam steps of ResNet18 at batch 2 (config 1);
``cpu_reference_ops`` puts the same NumPy path's config 2 GEMMs (GFLOP/s) and config 3 convolution
and max-pool operators (ms each) beside the GPU figures, with the cores and BLAS used.
The other configurations are reported beside the headline: ``c2_gemms`` (the standalone GEMMs of
config 2 against the FP32 matrix peak), ``c3_kernels`` (config 3's im2col and max-pool kernels
against the HBM peak, its convolution against the matrix peak) and ``c5_inference`` (config 5,
ResNet18 inference at batch 256, 224x224, with BN folded into the convolutions) and
``step_bandwidth_kernels`` (the step's batch-norm, max-pool, split-K reduction, kernel reorder and
Adam kernels at their step shapes against the HBM peak).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--plain-graph]
                       [--single-stream] [--step-only]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

# The CPU baseline uses as many BLAS threads as this process may run on (capped by OMP_NUM_THREADS
# when the host sets it); fix that before NumPy loads its BLAS.
_CORES = len(os.sched_getaffinity(0))
if os.environ.get("OMP_NUM_THREADS", "").isdigit():
    _CORES = min(_CORES, int(os.environ["OMP_NUM_THREADS"]))
os.environ.setdefault("OPENBLAS_NUM_THREADS", str(_CORES))

import numpy as np  # noqa: E402
import torch  # noqa: E402

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import myflows_amd as mf  # noqa: E402
from myflows_amd import native  # noqa: E402

FP32_MFMA_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0
METRIC = "ResNet18 FP32 train images/s (bs64, 3×120×160); GEMM TFLOP/s vs FP32 peak"
# Algorithmic work of one bs64 training step: 3x the forward conv + fc MACs minus the skipped stem
# dX, 4.138 GFLOP per image.
STEP_GFLOP = 264.85
# HBM bytes per launch of the roofline GEMM, from the FETCH_SIZE / WRITE_SIZE counter runs recorded
# in this summary (each counter scaled by what it reads for a copy kernel of known size).
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemm_mfma_4096_nn.md")


def profiled_traffic(path=TRAFFIC_PROFILE):
    """The "traffic_bytes_per_launch:" figure of a committed rocprofv3 summary, or None."""
    try:
        with open(path, encoding="utf-8") as handle:
            for line in handle:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def build_step(batch, height, width, seed=0, optimize=True):
    model = mf.ResNet18(output_dim=2, initializer=mf.make_initializer(seed=seed), conv_backend="hip_native")
    rng = np.random.default_rng(seed)
    x_np = rng.standard_normal((batch, 3, height, width)).astype(np.float32)
    t_np = rng.uniform(-1, 1, (batch, 2)).astype(np.float32)
    x = mf.Variable(torch.as_tensor(x_np, device="cuda"), requires_grad=False, name="images")
    t = mf.Variable(torch.as_tensor(t_np, device="cuda"), requires_grad=False, name="targets")
    loss = mf.MSELoss(model(x), t)
    graph = mf.Graph(loss, optimize=optimize)
    return mf.Adam(graph, learning_rate=1e-3), loss


def host_issue_ms(step, runs=5):
    """Median host time to issue one training step (replay or eager pass, then Adam) onto an idle
    GPU: the call returns before the GPU has finished, so this is what the host needs per step."""
    times = []
    for _ in range(runs):
        torch.cuda.synchronize()
        start = time.perf_counter()
        step.one_step()
        step.update()
        times.append((time.perf_counter() - start) * 1e3)
    torch.cuda.synchronize()
    return round(float(np.median(times)), 3)


def time_steps(opt, steps, warmup):
    for _ in range(warmup):
        opt.one_step()
        opt.update()
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(steps):
        opt.one_step()
        opt.update()
    torch.cuda.synchronize()
    return time.perf_counter() - start


def _settle(fn, warmup, settle_ms):
    """Untimed launches: `warmup` of them, then more until `settle_ms` of wall time has passed under
    the load. The GPU raises its shader clock over the first tens of milliseconds of sustained work
    after an idle spell (host-side set-up between the legs), so a kernel is timed at the clock it
    holds under load, not during the ramp."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = time.perf_counter()
    while (time.perf_counter() - start) * 1e3 < settle_ms:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()


def gemm_roofline(m=4096, n=4096, k=4096, reps=20, settle_ms=100.0):
    """Average launch time of the MFMA GEMM on C = A B (A, B ~ N(0, 1) seed 0), from HIP events on
    the stream the kernels are launched on, after the clock has settled under the load."""
    g = torch.Generator().manual_seed(0)
    a = torch.randn((m, k), generator=g).cuda()
    b = torch.randn((k, n), generator=g).cuda()
    out = torch.empty((m, n), device="cuda")
    stream = torch.cuda.current_stream()
    _settle(lambda: native.gemm(a, b, out=out), 3, settle_ms)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(reps):
        native.gemm(a, b, out=out)
    end.record(stream)
    end.synchronize()
    ms = start.elapsed_time(end) / reps
    achieved = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    tile, slices = native.gemm_plan(m, n, k)
    # A plain streaming kernel of known size (read 256 MiB, write 256 MiB): the calibration that
    # FETCH_SIZE / WRITE_SIZE counter runs divide by to turn counter units into HBM bytes.
    src = torch.empty((64 << 20,), device="cuda").fill_(1.0)
    torch.neg(src, out=torch.empty_like(src))
    torch.cuda.synchronize()
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4), "traffic": profiled_traffic(),
            "kernel": f"gemm_mfma_kernel NN {m}x{n}x{k} tile {tile} slices {slices}",
            "avg_launch_ms": round(ms, 4), "algorithmic_flop_per_launch": 2 * m * n * k}


_QUEUE_FILLER = []


def _event_time_us(fn, reps=20, warmup=3, settle_ms=30.0):
    """Average time of fn() in microseconds, from HIP events on the current stream (after _settle).
    A ~0.6 ms elementwise pass over 2 GiB runs ahead of the start event, so the host has queued all
    `reps` launches before the first one starts: a kernel of a few microseconds is then timed back
    to back, not at the rate the host issues launches."""
    stream = torch.cuda.current_stream()
    _settle(fn, warmup, settle_ms)
    if not _QUEUE_FILLER:
        _QUEUE_FILLER.append(torch.zeros(1 << 29, dtype=torch.float32, device="cuda"))
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    _QUEUE_FILLER[0].add_(1.0)
    start.record(stream)
    for _ in range(reps):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) * 1e3 / reps


def c3_kernels():
    """BASELINE config 3 on its own: Conv2D 64->64 3x3/1/1 at N=32, 30x40, then MaxPool 2x2/2. The
    bandwidth-bound kernels against the 8 TB/s HBM peak (algorithmic bytes: each required read or
    write once), the convolution products against the FP32 matrix peak."""
    lib = native._library()
    stream = torch.cuda.current_stream().cuda_stream
    n, ci, h, w, co = 32, 64, 30, 40, 64
    g = torch.Generator().manual_seed(0)
    x = torch.randn((n, ci, h, w), generator=g).cuda()
    weight = (torch.randn((co, ci, 3, 3), generator=g) * (2.0 / (ci * 9)) ** 0.5).cuda()
    dims = (n, ci, h, w, co, 3, 3, h, w, 1, 1, 1, 1)
    m, k = n * h * w, ci * 9
    cols = torch.empty((m, k), device="cuda")
    y = torch.empty((n, co, h, w), device="cuda")
    wt = torch.empty_like(weight)

    def im2col():
        native._raise_for(lib.mfh_conv_im2col(x.data_ptr(), cols.data_ptr(), *dims, stream), lib)

    def conv_forward():
        native._raise_for(lib.mfh_conv_forward_implicit(x.data_ptr(), weight.data_ptr(), wt.data_ptr(), 0, 0, 0,
                                                        y.data_ptr(), *dims, 0, 0.0, 1, 0, 0, stream), lib)

    pooled = torch.empty((n, co, h // 2, w // 2), device="cuda")
    argmax = torch.empty((n, co, h // 2, w // 2), dtype=torch.int32, device="cuda")
    dx = torch.empty_like(y)
    pool_dims = (n, co, h, w, h // 2, w // 2, 2, 2, 2, 2)

    def pool_forward():
        native._raise_for(lib.mfh_pool_forward(y.data_ptr(), pooled.data_ptr(), argmax.data_ptr(), *pool_dims,
                                               stream), lib)

    def pool_backward():
        native._raise_for(lib.mfh_pool_backward(pooled.data_ptr(), argmax.data_ptr(), dx.data_ptr(), *pool_dims,
                                                stream), lib)

    conv_forward()
    pool_forward()
    out = {"config": "Conv2D 64->64 3x3/1/1, N=32, 30x40; MaxPool 2x2/2", "peak_GB/s": HBM_PEAK_GBS,
           "peak_TFLOP/s": FP32_MFMA_PEAK_TFLOPS}
    grad_cols = torch.randn((n, k, h * w), generator=g).cuda()  # feature-major, per image
    dxc = torch.empty_like(x)

    def col2im():
        native._raise_for(lib.mfh_conv_col2im(grad_cols.data_ptr(), dxc.data_ptr(), *dims, 1, 0, stream), lib)

    bytes_im2col = 4 * (n * ci * h * w + m * k)  # read x, write cols; col2im: read grad_cols, write dx
    bytes_pool = 4 * n * co * h * w + 8 * n * co * (h // 2) * (w // 2)
    for name, fn, nbytes in (("im2col", im2col, bytes_im2col), ("col2im", col2im, bytes_im2col),
                             ("pool_forward", pool_forward, bytes_pool), ("pool_backward", pool_backward, bytes_pool)):
        us = _event_time_us(fn)
        gbs = nbytes / (us * 1e-6) / 1e9
        out[name] = {"us": round(us, 2), "bytes": nbytes, "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 3)}
    dy = torch.randn((n, co, h, w), generator=g).cuda()
    dxb = torch.empty_like(x)
    dw = torch.empty_like(weight)
    db = torch.empty(co, device="cuda")
    wflip = native.conv_weight_orders([(weight, 1)])[0]
    partial = torch.empty(max(n, native.BIAS_PARTIAL_ROWS) * co, dtype=torch.float64, device="cuda")
    workspace = torch.empty(max(lib.mfh_conv_implicit_workspace(*dims, p) for p in (1, 2)) + 4, device="cuda")

    def conv_dx():
        native._raise_for(lib.mfh_conv_backward_implicit(
            0, weight.data_ptr(), dy.data_ptr(), 0, 0, 0, dxb.data_ptr(), wflip.data_ptr(), 0, 0, 0, *dims, 0, 0.0,
            1, 1, native.CONV_WFLIP_READY, workspace.data_ptr(), workspace.numel(), stream), lib)

    def conv_dw():
        native._raise_for(lib.mfh_conv_backward_implicit(
            x.data_ptr(), weight.data_ptr(), dy.data_ptr(), 0, 0, dw.data_ptr(), 0, 0, 0, partial.data_ptr(),
            db.data_ptr(), *dims, 0, 0.0, 1, 1, 0, workspace.data_ptr(), workspace.numel(), stream), lib)

    for name, fn in (("conv_forward_implicit", conv_forward), ("conv_dx_implicit", conv_dx),
                     ("conv_dw_implicit", conv_dw)):
        us = _event_time_us(fn)
        tflops = 2.0 * m * co * k / (us * 1e-6) / 1e12
        out[name] = {"us": round(us, 2), "TFLOP/s": round(tflops, 2), "frac": round(tflops / FP32_MFMA_PEAK_TFLOPS, 3)}
    return out


def _bandwidth_entry(us, nbytes):
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"us": round(us, 2), "bytes": int(nbytes), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 3)}


def step_bandwidth_kernels():
    """The bandwidth-bound kernels of the bs64 training step at their step shapes, each against the
    8 TB/s HBM peak. Bytes are algorithmic (each required tensor read or write once), so a pass that
    reads a tensor twice shows it as a lower fraction. Batch norm: the two-launch path (partial sums,
    then the element pass) at layer1 and layer2, the one-launch channel kernels at layer3, the stem's
    BN+ReLU+max-pool unit; the stem-shaped max-pool kernels; a split-K reduction (layer4 forward,
    6 slices); the batched forward kernel reorders of all 20 convolutions; Adam over all 62
    parameter tensors."""
    lib = native._library()
    stream = torch.cuda.current_stream().cuda_stream
    g = torch.Generator().manual_seed(0)
    out = {"config": "ResNet18 bs64 3x120x160 step shapes", "peak_GB/s": HBM_PEAK_GBS}

    def bn_case(name, n, c, h, w, residual):
        x = (torch.randn((n, c, h, w), generator=g) * 2 + 0.5).cuda()
        r = torch.randn((n, c, h, w), generator=g).cuda() if residual else None
        gamma, beta = torch.ones(c, device="cuda"), torch.zeros(c, device="cuda")
        rm, rv = torch.zeros(c, device="cuda"), torch.ones(c, device="cuda")
        y, dx, dy = torch.empty_like(x), torch.empty_like(x), torch.randn((n, c, h, w), generator=g).cuda()
        rg = torch.empty_like(x) if residual else None
        mean, istd = torch.empty((2, c), device="cuda"), torch.empty(c, device="cuda")
        dg, db = torch.empty(c, device="cuda"), torch.empty(c, device="cuda")
        doubles = lib.mfh_bn_workspace(n, c, h * w)
        ws = torch.empty(doubles + 2, dtype=torch.float64, device="cuda")

        def forward():
            native._raise_for(lib.mfh_bn_forward(
                x.data_ptr(), gamma.data_ptr(), beta.data_ptr(), rm.data_ptr(), rv.data_ptr(), native._addr(r),
                y.data_ptr(), mean.data_ptr(), istd.data_ptr(), ws.data_ptr(), doubles, n, c, h * w, 1, 1, 0.1,
                1e-5, 1.0, stream), lib)

        def backward():
            native._raise_for(lib.mfh_bn_backward(
                x.data_ptr(), dy.data_ptr(), y.data_ptr(), gamma.data_ptr(), mean.data_ptr(), istd.data_ptr(),
                dx.data_ptr(), dg.data_ptr(), db.data_ptr(), native._addr(rg), ws.data_ptr(), doubles, n, c, h * w,
                1, 0, 0, 0, 0, stream), lib)

        forward()
        elems = 4 * n * c * h * w
        out[f"bn_forward_{name}"] = _bandwidth_entry(_event_time_us(forward), elems * (3 if residual else 2))
        out[f"bn_backward_{name}"] = _bandwidth_entry(_event_time_us(backward), elems * (5 if residual else 4))

    bn_case("layer1_two_launch", 64, 64, 29, 39, False)
    bn_case("layer2_two_launch_residual", 64, 128, 15, 20, True)
    bn_case("layer3_one_launch_residual", 64, 256, 8, 10, True)

    # The stem: BN + ReLU + 3x3/2 max-pool as one unit, and the plain max-pool kernels at its shape.
    n, c, h, w, oh, ow = 64, 64, 60, 80, 29, 39
    x = torch.randn((n, c, h, w), generator=g).cuda()
    gamma, beta = torch.ones(c, device="cuda"), torch.zeros(c, device="cuda")
    rm, rv = torch.zeros(c, device="cuda"), torch.ones(c, device="cuda")
    pooled, argmax = torch.empty((n, c, oh, ow), device="cuda"), torch.empty((n, c, oh, ow), dtype=torch.int32,
                                                                            device="cuda")
    mean, istd = torch.empty((2, c), device="cuda"), torch.empty(c, device="cuda")
    dg, db, dx = torch.empty(c, device="cuda"), torch.empty(c, device="cuda"), torch.empty_like(x)
    dp = torch.randn((n, c, oh, ow), generator=g).cuda()
    doubles = lib.mfh_bn_workspace(n, c, h * w)
    ws = torch.empty(doubles + 2, dtype=torch.float64, device="cuda")
    dims = (n, c, h, w, 3, 3, 2, 2)

    def unit_forward():
        native._raise_for(lib.mfh_bn_relu_pool_forward(
            x.data_ptr(), gamma.data_ptr(), beta.data_ptr(), rm.data_ptr(), rv.data_ptr(), pooled.data_ptr(),
            argmax.data_ptr(), mean.data_ptr(), istd.data_ptr(), ws.data_ptr(), doubles, *dims, 1, 0.1, 1e-5, 1.0,
            stream), lib)

    def unit_backward():
        native._raise_for(lib.mfh_bn_relu_pool_backward(
            x.data_ptr(), dp.data_ptr(), argmax.data_ptr(), gamma.data_ptr(), beta.data_ptr(), mean.data_ptr(),
            istd.data_ptr(), dx.data_ptr(), dg.data_ptr(), db.data_ptr(), ws.data_ptr(), doubles, *dims, 1, 0, 0, 0,
            stream), lib)

    unit_forward()
    big, small = 4 * n * c * h * w, 4 * n * c * oh * ow
    out["bn_relu_pool_forward_stem"] = _bandwidth_entry(_event_time_us(unit_forward), big + 2 * small)
    out["bn_relu_pool_backward_stem"] = _bandwidth_entry(_event_time_us(unit_backward), 2 * big + 2 * small)
    pool_dims = (n, c, h, w, oh, ow, 3, 3, 2, 2)
    out["pool_forward_stem"] = _bandwidth_entry(_event_time_us(lambda: native._raise_for(lib.mfh_pool_forward(
        x.data_ptr(), pooled.data_ptr(), argmax.data_ptr(), *pool_dims, stream), lib)), big + 2 * small)
    out["pool_backward_stem"] = _bandwidth_entry(_event_time_us(lambda: native._raise_for(lib.mfh_pool_backward(
        dp.data_ptr(), argmax.data_ptr(), dx.data_ptr(), *pool_dims, stream), lib)), big + 2 * small)

    # Split-K reduction of the layer4 3x3 forward product (512 x 1280 outputs, 6 slices).
    s, m, nn = 6, 512, 1280
    partial = torch.randn((s, m, nn), generator=g).cuda()
    cm = torch.empty((m, nn), device="cuda")
    out["split_reduce_layer4_forward"] = _bandwidth_entry(_event_time_us(lambda: native._raise_for(
        lib.mfh_split_reduce(partial.data_ptr(), cm.data_ptr(), s, m, nn, nn, 0, stream), lib)), 4 * (s + 1) * m * nn)

    # The forward kernel reorders of all of ResNet18's convolutions in one batched call.
    model = mf.ResNet18(output_dim=2, initializer=mf.make_initializer(seed=0), conv_backend="hip_native")
    kernels = [p.value for p in model.params if p.value.ndim == 4]
    outs = [torch.empty_like(k) for k in kernels]
    wdims = []
    for k in kernels:
        wdims += [*k.shape, 0, 1, 1, 0, 0]
    w_ptrs = (ctypes.c_uint64 * len(kernels))(*[k.data_ptr() for k in kernels])
    o_ptrs = (ctypes.c_uint64 * len(kernels))(*[o.data_ptr() for o in outs])
    d_arr = (ctypes.c_int * len(wdims))(*wdims)
    floats = sum(k.numel() for k in kernels)
    out["weight_order_all_convs"] = _bandwidth_entry(_event_time_us(lambda: native._raise_for(
        lib.mfh_conv_weight_orders(w_ptrs, o_ptrs, d_arr, len(kernels), stream), lib)), 8 * floats)

    # Adam over every parameter tensor (read p, g, m, v; write p, m, v).
    # The tensor table is built once, so the timed calls are the native launches alone.
    params = [p.value for p in model.params]
    held = [(p, torch.randn_like(p) * 1e-3, torch.zeros_like(p), torch.zeros_like(p)) for p in params]  # kept alive
    rows = [mf.fused._adam_row(p, grad, m, v, 1e-3, 0.0, 1, 0.9, 0.999) for p, grad, m, v in held]
    out["adam_all_params"] = _bandwidth_entry(_event_time_us(lambda: mf.fused._adam_launch(
        rows, 0.9, 0.999, 1e-8, 1.0)), 28 * sum(p.numel() for p in params))
    return out


def _median_seconds(fn, runs):
    fn()  # warm-up
    times = []
    for _ in range(runs):
        start = time.perf_counter()
        fn()
        times.append(time.perf_counter() - start)
    return float(np.median(times))


def _blas_name():
    try:
        info = np.show_config(mode="dicts")
        return info.get("Build Dependencies", {}).get("blas", {}).get("name", "unknown")
    except Exception:  # noqa: BLE001 - only a label
        return "unknown"


def cpu_reference_ops(runs=5):
    """The reference's NumPy path beside the GPU figures of configs 2 and 3, on this host's cores:
    float32 NumPy GEMMs (A, B ~ N(0, 1) seed 0) and config 3's convolution (im2col + GEMM forward,
    dX through col2im, dW, FP64 db) and max-pool (window max with first-index mask, masked
    scatter), each the median of `runs` runs after a warm-up."""
    from oracle import reference_path as rp

    out = {"cores": _CORES, "numpy": np.__version__, "blas": _blas_name(), "runs": runs, "c2_gemms": {}, "c3_ops_ms": {}}
    rng = np.random.default_rng(0)
    cases = [(f"{n}^3", n, n, n, False) for n in (512, 1024, 2048, 4096)]
    cases += [("im2col 38400x64x576", 38400, 64, 576, False), ("dW A^T B 576x64 over 38400", 576, 64, 38400, True)]
    for name, m, n, k, trans_a in cases:
        a = rng.standard_normal((k, m) if trans_a else (m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        seconds = _median_seconds(lambda: (a.T if trans_a else a) @ b, runs if m * n * k <= 2048 ** 3 else 3)
        out["c2_gemms"][name] = {"ms": round(seconds * 1e3, 3), "GFLOP/s": round(2.0 * m * n * k / seconds / 1e9, 1)}
    x = rng.standard_normal((32, 64, 30, 40)).astype(np.float32)
    w = (rng.standard_normal((64, 64, 3, 3)) * np.sqrt(2.0 / 576)).astype(np.float32)
    b = np.zeros(64, np.float32)
    y, cols = rp.conv2d_forward(x, w, b, (1, 1), (1, 1))
    dy = rng.standard_normal(y.shape).astype(np.float32)
    ops = out["c3_ops_ms"]
    ops["conv_forward"] = _median_seconds(lambda: rp.conv2d_forward(x, w, b, (1, 1), (1, 1)), runs) * 1e3
    ops["conv_dx"] = _median_seconds(lambda: rp.conv2d_backward(
        x, w, dy, cols, (1, 1), (1, 1), need_weight_grad=False, need_bias_grad=False), runs) * 1e3
    ops["conv_dw_db"] = _median_seconds(lambda: rp.conv2d_backward(
        x, w, dy, cols, (1, 1), (1, 1), need_input_grad=False), runs) * 1e3
    pooled, mask, padded = rp.maxpool2d_forward(y, (2, 2), (2, 2))
    dp = rng.standard_normal(pooled.shape).astype(np.float32)
    ops["pool_forward"] = _median_seconds(lambda: rp.maxpool2d_forward(y, (2, 2), (2, 2)), runs) * 1e3
    ops["pool_backward"] = _median_seconds(lambda: rp.maxpool2d_backward(dp, mask, padded, (2, 2), (2, 2)), runs) * 1e3
    for key in ops:
        ops[key] = round(ops[key], 3)
    return out


def c2_gemms(reps=20):
    """the standalone FP32 GEMMs C = A B (A, B ~ N(0, 1) seed 0) at M=N=K in
    {512, 1024, 2048, 4096}, the im2col-shaped 38400 x 64 x 576 product and its dW form A^T B
    (A stored 38400 x 576, B 38400 x 64, C 576 x 64), each under the automatic plan; TFLOP/s from
    HIP events over `reps` launches against the FP32 matrix peak."""
    out = {"peak_TFLOP/s": FP32_MFMA_PEAK_TFLOPS}
    g = torch.Generator().manual_seed(0)
    cases = [(f"{n}^3", n, n, n, False) for n in (512, 1024, 2048, 4096)]
    cases += [("im2col 38400x64x576", 38400, 64, 576, False), ("dW A^T B 576x64 over 38400", 576, 64, 38400, True)]
    for name, m, n, k, trans_a in cases:
        a = torch.randn((k, m) if trans_a else (m, k), generator=g).cuda()
        b = torch.randn((k, n), generator=g).cuda()
        c = torch.empty((m, n), device="cuda")
        us = _event_time_us(lambda: native.gemm(a, b, trans_a=trans_a, out=c), reps=reps)
        tflops = 2.0 * m * n * k / (us * 1e-6) / 1e12
        tile, slices = native.gemm_plan(m, n, k, layout="TN" if trans_a else "NN")
        out[name] = {"us": round(us, 2), "TFLOP/s": round(tflops, 2), "frac": round(tflops / FP32_MFMA_PEAK_TFLOPS, 3),
                     "plan": f"tile {tile} slices {slices}"}
        del a, b, c
    return out


# Algorithmic work of one bs256 224x224 ResNet18 forward (convolutions + fc), 3.594 GFLOP per image.
C5_STEP_GFLOP = 920.2


def c5_inference(batch=256, size=224, reps=10, warmup=3, seed=0):
    """ResNet18(output_dim=2) inference at batch 256, 3x224x224 ~ N(0, 1), eval-mode
    batch norm with running variance ~ U(0.5, 1.5) and mean ~ N(0, 0.1) (seeded), BN folded into the
    convolutions, ReLU and each block's residual add fused into their epilogues
    (apply_graph_optimizations(mode="inference"), then Graph(optimize=True)). Images per second over `reps` forward passes."""
    model = mf.ResNet18(output_dim=2, initializer=mf.make_initializer(seed=seed), conv_backend="hip_native")
    rng = np.random.default_rng(seed)
    x_np = rng.standard_normal((batch, 3, size, size)).astype(np.float32)
    bns = [model.stem_bn] + [bn for block in model.blocks()
                             for bn in (block.bn1, block.bn2, *((block.downsample_bn,) if block.downsample else ()))]
    for bn in bns:
        bn.running_mean.copy_(torch.as_tensor(rng.normal(0, 0.1, bn.num_features).astype(np.float32)))
        bn.running_var.copy_(torch.as_tensor(rng.uniform(0.5, 1.5, bn.num_features).astype(np.float32)))
    model.eval()
    out = model(mf.Variable(torch.as_tensor(x_np, device="cuda"), requires_grad=False, name="images"))
    root, stats = mf.apply_graph_optimizations(out, mode="inference", fold_constants=False)
    graph = mf.Graph(root, optimize=True)
    _settle(graph.forward, warmup, 100.0)
    start = time.perf_counter()
    for _ in range(reps):
        graph.forward()
    torch.cuda.synchronize()
    seconds = time.perf_counter() - start
    ms = seconds * 1e3 / reps
    return {"config": f"ResNet18 inference bs{batch} 3x{size}x{size}, BN folded, Conv+ReLU and Conv+Add+ReLU epilogues",
            "images/s": round(batch * reps / seconds, 1), "ms_per_batch": round(ms, 3),
            "TFLOP/s": round(C5_STEP_GFLOP * batch / 256 / (ms * 1e-3) / 1e3, 2), "bn_folds": stats["bn_folds"],
            "conv_act_fusions": graph._opt_stats["conv_act_fusions"], "conv_add_act_fusions": stats["conv_add_act_fusions"]}


def cpu_baseline(min_seconds=10.0, batch=2):
    """The NumPy reference-path ResNet18 step (forward + backward + Adam) on this host."""
    from oracle import resnet as oracle_resnet

    params, running = oracle_resnet.init_params(seed=0)
    x, target = oracle_resnet.synthetic_batch(batch, seed=0)
    state = {}
    _, grads, _ = oracle_resnet.forward_backward(params, running, x, target)  # warm-up
    oracle_resnet.adam_step(params, grads, state, 1)
    steps, start = 0, time.perf_counter()
    while True:
        _, grads, _ = oracle_resnet.forward_backward(params, running, x, target)
        oracle_resnet.adam_step(params, grads, state, steps + 2)
        steps += 1
        elapsed = time.perf_counter() - start
        if elapsed >= min_seconds and steps >= 2:
            break
    blas = _blas_name()
    return {"value": round(batch * steps / elapsed, 3), "unit": "images/s", "cores": _CORES, "kind": "port",
            "sample": f"{steps} ResNet18 train steps (fwd+bwd+Adam) at batch {batch}, 3x120x160, NumPy "
                      f"{np.__version__} ({blas}, {_CORES} threads), {elapsed:.1f} s"}


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--batch", type=int, default=64)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--step-only", action="store_true",
                        help="time the training step alone (no roofline, config 2/3/5 or bandwidth legs), for profiling")
    parser.add_argument("--single-stream", action="store_true",
                        help="run each backward's dW products on the current stream (no weight-gradient stream)")
    parser.add_argument("--plain-graph", action="store_true",
                        help="Graph(optimize=False): BN, Add and ReLU as separate nodes (the reference task's graph)")
    parser.add_argument("--eager", action="store_true",
                        help="issue every step from Python (Graph.forward/backward) instead of replaying the "
                             "library program recorded from one such step (RecordedStep)")
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build runs no multi-GPU path (use --gpus 1)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    torch.cuda.set_device(0)
    native._library()
    opt, _ = build_step(args.batch, 120, 160, optimize=not args.plain_graph)
    opt.graph.overlap_weight_grads = opt.graph.overlap_branches = not args.single_stream
    step = opt if args.eager else mf.RecordedStep(opt, warmup=2)
    seconds = time_steps(step, args.steps, args.warmup)
    ms_per_step = seconds * 1e3 / args.steps
    images_per_s = args.batch * args.steps / seconds
    issue_ms = host_issue_ms(step)
    issue = "eager" if args.eager else "recorded program"
    if args.step_only:
        print(json.dumps({"metric": METRIC, "value": round(images_per_s, 2), "unit": "images/s", "n_gpus": 1,
                          "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 3),
                          "single_stream": args.single_stream, "step_issue": issue,
                          "host_issue_ms_per_step": issue_ms, "step_only": True}), flush=True)
        return 0
    roofline = gemm_roofline()
    result = {
        "metric": METRIC, "value": round(images_per_s, 2), "unit": "images/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "ResNet18(output_dim=2) train step (fwd+bwd+Adam), hip_native backend",
                   "global_batch": args.batch, "input": [3, 120, 160], "loss": "MSE",
                   "graph": "optimize=False" if args.plain_graph else
                   "optimize=True (BN+ReLU, BN+Add+ReLU and stem BN+ReLU+max-pool units)",
                   "backward_streams": 1 if args.single_stream else 2, "step_issue": issue},
        "host_issue_ms_per_step": issue_ms,
        "step_tflops": round(STEP_GFLOP * args.batch / 64 / (ms_per_step * 1e-3) / 1e3, 2),
        "roofline": roofline,
        "c2_gemms": c2_gemms(),
        "c3_kernels": c3_kernels(),
        "c5_inference": c5_inference(),
        "step_bandwidth_kernels": step_bandwidth_kernels(),
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
        result["cpu_reference_ops"] = cpu_reference_ops()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
