"""Convolution parity on the GPU, through the operator API and the native.py boundary, for both
convolution algorithms: "implicit" (the GEMM gathers the im2col view from x; dX of stride-1
convolutions is a convolution of dy with the flipped kernel) and "im2col" (cols written first).

Bit-exact: the im2col matrix, and col2im (integer-valued dy and W make every GEMM product and
window sum exact in float32, so any index or window error shows as a bit difference) on each dX
path (from NCHW dy, from the transposed gated dy), and the implicit path on the same integer data.
Tolerance: outputs and gradients within 1e-5 of max|ref| of the FP64 loops of the reference's tests
(normwise, the reference's own criterion), db within one float32 ulp of the FP64 sum.
"""

import contextlib
import os

import numpy as np
import pytest
import torch

import myflows_amd as mf
from myflows_amd import native
from oracle import naive, reference_path as rp
from tests.fixtures import CONV_CASES, EPS32, PERFORMANCE_CASES, assert_near, conv_fixture

pytestmark = pytest.mark.gpu


def gpu(a):
    return torch.as_tensor(np.ascontiguousarray(a), device="cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


ALGORITHMS = native.CONV_ALGORITHMS
# ResNet18's convolution shapes at batch 2 (stem, layer1, a stride-2 3x3, a 1x1 downsample, layer4),
# plus a padding wider than the kernel, which makes the flipped dX convolution's padding negative.
RESNET_CASES = (
    ("stem", (2, 3, 48, 64), (64, 3, 7, 7), (2, 2), (3, 3)),
    ("l1", (2, 64, 29, 39), (64, 64, 3, 3), (1, 1), (1, 1)),
    ("l2down3x3", (2, 64, 29, 39), (128, 64, 3, 3), (2, 2), (1, 1)),
    ("l2ds1x1", (2, 64, 29, 39), (128, 64, 1, 1), (2, 2), (0, 0)),
    ("l4", (2, 512, 4, 5), (512, 512, 3, 3), (1, 1), (1, 1)),
    ("widepad", (1, 2, 5, 6), (3, 2, 1, 2), (1, 1), (1, 2)),
)
# Output channels that end inside a row tile: the last row tile of a chunked (co40) or padded
# natural-order (stem20) product reads dy's rows, and the forward the kernel's rows, with
# range-checked offsets, and its rows past CO read zero.
PARTIAL_ROW_CASES = (
    ("co40", (2, 64, 9, 11), (40, 64, 3, 3), (1, 1), (1, 1)),
    ("stem20", (2, 3, 20, 24), (20, 3, 7, 7), (2, 2), (3, 3)),
)


@contextlib.contextmanager
def conv_algorithm(name):
    """Make `name` the default convolution algorithm (MFHIP_CONV_ALGO) inside the block."""
    previous = os.environ.get("MFHIP_CONV_ALGO")
    os.environ["MFHIP_CONV_ALGO"] = name
    try:
        yield
    finally:
        if previous is None:
            os.environ.pop("MFHIP_CONV_ALGO", None)
        else:
            os.environ["MFHIP_CONV_ALGO"] = previous


def run_operator(case, op_class=mf.Conv2D_Op, input_grad=True, algorithm="implicit", **options):
    """Forward + backward of one convolution operator; returns (op, y, [dx, dw, db])."""
    with conv_algorithm(algorithm):
        return _run_operator(case, op_class, input_grad, **options)


def _run_operator(case, op_class, input_grad, **options):
    x, w, b, dy = (gpu(a) for a in conv_fixture(case))
    leaves = [mf.Variable(x, requires_grad=input_grad), mf.Variable(w, trainable=True), mf.Variable(b, trainable=True)]
    op = op_class(leaves[0], leaves[1], stride=case[3], padding=case[4], bias=leaves[2], backend="hip_native",
                  **options)
    op.forward(x, w, b)
    op.grad = dy
    op.backward()
    return op, host(op.value), [None if leaf.grad is None else host(leaf.grad) for leaf in leaves]


def fp64_case(case):
    x, w, b, dy = (a.astype(np.float64) for a in conv_fixture(case))
    return x, w, b, dy, naive.conv_forward(x, w, case[3], case[4]) + b[None, :, None, None]


@pytest.mark.parametrize("algorithm", ALGORITHMS)
@pytest.mark.parametrize("case", CONV_CASES + PERFORMANCE_CASES + RESNET_CASES, ids=lambda c: c[0])
def test_forward_and_gradients_match_fp64_loops(case, algorithm):
    """The forward is one GEMM over all images stored into NCHW (split over K when the planner asks);
    dW is a split-K GEMM; dX is the flipped-kernel convolution (implicit, stride 1) or a column
    gradient GEMM and col2im."""
    print("conv case", case[0], algorithm, flush=True)
    x, w, _, dy, pre = fp64_case(case)
    op, y, (dx, dw, db) = run_operator(case, algorithm=algorithm)
    assert op.value.is_contiguous()
    ref_dx, ref_dw = naive.conv_backward(x, w, dy, case[3], case[4])
    assert_near(y, pre, 1e-5, "y")
    assert_near(dx, ref_dx, 1e-5, "dx")
    assert_near(dw, ref_dw, 1e-5, "dw")
    ref_db = dy.sum(axis=(0, 2, 3))
    assert np.all(np.abs(db - ref_db) <= np.spacing(np.abs(ref_db).astype(np.float32))), "db beyond one ulp"


def test_known_answer_t0_is_exact():
    """arange(25) correlated with ones(3x3): every output is its 3x3 window sum, exactly."""
    _, y, _ = run_operator(CONV_CASES[0])
    grid = np.arange(25.0).reshape(5, 5)
    windows = np.array([[grid[i:i + 3, j:j + 3].sum() for j in range(3)] for i in range(3)], np.float32)
    np.testing.assert_array_equal(y[0, 0], windows)


@pytest.mark.parametrize("algorithm", ALGORITHMS)
@pytest.mark.parametrize("case", (CONV_CASES[1], CONV_CASES[3], PERFORMANCE_CASES[2]), ids=lambda c: c[0])
@pytest.mark.parametrize("variant", ("relu", "leaky"))
def test_fused_activation_forward_and_gated_backward(case, variant, algorithm):
    print("fused", variant, case[0], algorithm, flush=True)
    x, w, _, dy, pre = fp64_case(case)
    op_class, options, slope = ((mf.Conv2D_ReLU_Op, {}, 0.0) if variant == "relu"
                                else (mf.Conv2D_LeakyReLU_Op, {"alpha": 0.2}, 0.2))
    op, y, (dx, dw, db) = run_operator(case, op_class, algorithm=algorithm, **options)
    assert op._activation_fused
    gate = np.where(pre > 0, 1.0, slope)
    ref_dx, ref_dw = naive.conv_backward(x, w, dy * gate, case[3], case[4])
    assert_near(y, np.where(pre > 0, pre, slope * pre), 1e-5, "y")
    assert_near(dx, ref_dx, 1e-5, "dx")
    assert_near(dw, ref_dw, 1e-5, "dw")
    assert_near(db, (dy * gate).sum(axis=(0, 2, 3)), 4 * EPS32, "db")


@pytest.mark.parametrize("algorithm", ALGORITHMS)
def test_frozen_input_skips_dx_and_keeps_weight_gradients_bitwise(algorithm):
    case = PERFORMANCE_CASES[0]
    _, _, (_, dw_all, db_all) = run_operator(case, algorithm=algorithm)
    _, _, (dx, dw, db) = run_operator(case, input_grad=False, algorithm=algorithm)
    assert dx is None
    np.testing.assert_array_equal(dw, dw_all)
    np.testing.assert_array_equal(db, db_all)


@pytest.mark.parametrize("algorithm", ALGORITHMS)
@pytest.mark.parametrize("case", (PERFORMANCE_CASES[2], RESNET_CASES[1]), ids=lambda c: c[0])
def test_dx_only_through_fused_relu(case, algorithm):
    """Frozen weight and bias: only dX, gated by the fused ReLU's output."""
    x, w, b, dy = conv_fixture(case)
    xv = mf.Variable(gpu(x))
    wv, bv = mf.Variable(gpu(w), requires_grad=False), mf.Variable(gpu(b), requires_grad=False)
    with conv_algorithm(algorithm):
        op = mf.Conv2D_ReLU_Op(xv, wv, stride=case[3], padding=case[4], bias=bv, backend="hip_native")
        op.forward(xv.value, wv.value, bv.value)
        op.grad = gpu(dy)
        op.backward()
    pre = naive.conv_forward(x.astype(np.float64), w.astype(np.float64), case[3], case[4]) + b[None, :, None, None]
    ref_dx, _ = naive.conv_backward(x.astype(np.float64), w.astype(np.float64), dy * (pre > 0), case[3], case[4])
    assert wv.grad is None and bv.grad is None
    assert_near(host(xv.grad), ref_dx, 1e-5, "dx")


@pytest.mark.parametrize("algorithm", ALGORITHMS)
@pytest.mark.parametrize("case", (PERFORMANCE_CASES[0], PERFORMANCE_CASES[1], RESNET_CASES[1]),
                         ids=lambda c: c[0])
def test_gradients_are_bitwise_reproducible(case, algorithm):
    first = run_operator(case, algorithm=algorithm)[2]
    second = run_operator(case, algorithm=algorithm)[2]
    for a, b in zip(first, second):
        np.testing.assert_array_equal(a, b)


def test_recomputed_columns_give_identical_gradients():
    case = PERFORMANCE_CASES[0]
    saved = run_operator(case, algorithm="im2col")[2]
    recomputed = run_operator(case, algorithm="im2col", recompute_im2col=True)[2]
    for a, b in zip(saved, recomputed):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("case", CONV_CASES[1:] + RESNET_CASES + PARTIAL_ROW_CASES, ids=lambda c: c[0])
def test_implicit_path_is_exact_on_integer_data(case):
    """Small integers make every product and every partial sum exact in float32, whatever the
    summation order: the implicit forward, dW and dX must then equal the FP64 loops bit for bit,
    which pins the gather's indexing, padding and image boundaries (and the flipped dX kernel)."""
    print("integer", case[0], flush=True)
    _, x_shape, w_shape, stride, padding = case
    rng = np.random.default_rng(7)
    x = rng.integers(-2, 3, size=x_shape).astype(np.float32)
    w = rng.integers(-2, 3, size=w_shape).astype(np.float32)
    n, co, oh, ow = (x_shape[0], w_shape[0], *rp.out_size(x_shape[2], x_shape[3], w_shape[2:], stride, padding))
    dy = rng.integers(-2, 3, size=(n, co, oh, ow)).astype(np.float32)
    y, cols = native.conv2d_forward(gpu(x), gpu(w), stride=stride, padding=padding, algorithm="implicit")
    assert cols is None
    dx, dw, db = native.conv2d_backward(gpu(x), gpu(w), gpu(dy), None, stride=stride, padding=padding,
                                        algorithm="implicit")
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    ref_dx, ref_dw = naive.conv_backward(x64, w64, dy.astype(np.float64), stride, padding)
    np.testing.assert_array_equal(host(y), naive.conv_forward(x64, w64, stride, padding))
    np.testing.assert_array_equal(host(dx), ref_dx)
    np.testing.assert_array_equal(host(dw), ref_dw)
    np.testing.assert_array_equal(host(db), dy.astype(np.float64).sum(axis=(0, 2, 3)))


@pytest.mark.parametrize("shape,kernel,stride,padding", [
    ((2, 3, 7, 9), (3, 3), (1, 1), (1, 1)), ((1, 2, 8, 9), (3, 2), (2, 3), (1, 0)),
    ((2, 3, 16, 16), (7, 7), (2, 2), (3, 3)), ((3, 5, 6, 5), (1, 1), (2, 2), (0, 0)),
    ((2, 64, 30, 40), (3, 3), (1, 1), (1, 1)), ((2, 16, 29, 39), (3, 3), (2, 2), (1, 1)),
    # 4096 output rows take runs of a whole row (6 pixels): a 14-float input band, so the feature
    # offsets after it start at the next 16-byte boundary (the float4 path, K = 4).
    ((64, 2, 64, 7), (1, 2), (1, 1), (0, 0))])
def test_im2col_and_col2im_are_bit_exact(shape, kernel, stride, padding):
    print("im2col", shape, kernel, stride, padding, flush=True)
    rng = np.random.default_rng(3)
    x = rng.standard_normal(shape).astype(np.float32)
    co = 4
    w_shape = (co, shape[1], *kernel)
    cols = native.conv2d_im2col(gpu(x), w_shape, stride=stride, padding=padding)
    np.testing.assert_array_equal(host(cols), rp.im2col(x, kernel, stride, padding))
    np.testing.assert_array_equal(host(cols), naive.im2col(x, kernel, stride, padding))
    oh, ow = rp.out_size(shape[2], shape[3], kernel, stride, padding)
    w = rng.integers(-2, 3, size=w_shape).astype(np.float32)
    dy = rng.integers(-3, 4, size=(shape[0], co, oh, ow)).astype(np.float32)
    grad_cols = dy.transpose(0, 2, 3, 1).reshape(-1, co).astype(np.float64) @ w.reshape(co, -1)
    expected = rp.col2im_native(grad_cols.astype(np.float32), shape, kernel, stride, padding)
    np.testing.assert_array_equal(expected, naive.col2im(grad_cols, shape, kernel, stride, padding))
    ones = gpu(np.ones(dy.shape, np.float32))  # a ReLU gate that passes everything
    for need_w, activation in ((False, None), (True, None), (False, "relu"), (True, "relu")):
        dx, _, _ = native.conv2d_backward(gpu(x), gpu(w), gpu(dy), cols, stride=stride, padding=padding,
                                          need_bias_grad=need_w, need_weight_grad=need_w, activation=activation,
                                          output=ones)
        np.testing.assert_array_equal(host(dx), expected)
    # The col2im entry point alone, on both feature-major layouts, written fresh and added.
    n, k = shape[0], grad_cols.shape[1]
    pixel_major = grad_cols.astype(np.float32).reshape(n, oh * ow, k)
    layouts = {True: pixel_major.transpose(0, 2, 1), False: pixel_major.transpose(2, 0, 1)}
    for per_image, gct in layouts.items():
        dx = native.conv2d_col2im(gpu(gct), shape, w_shape, stride=stride, padding=padding, per_image=per_image)
        np.testing.assert_array_equal(host(dx), expected, err_msg=f"per_image={per_image}")
        base = rng.integers(-2, 3, size=shape).astype(np.float32)
        out = gpu(base)
        native.conv2d_col2im(gpu(gct), shape, w_shape, stride=stride, padding=padding, per_image=per_image, out=out,
                             accumulate=True)
        np.testing.assert_array_equal(host(out), base + expected, err_msg=f"per_image={per_image} accumulate")


@pytest.mark.parametrize("plan", ["mfma", ("64x64", 1)])
def test_single_engine_backward_is_the_two_engine_call(plan):
    """mfh_conv_backward_single (the reference's mf_conv_backward) gives the bits of mfh_conv_backward
    with its engine for both products, through a ReLU gate, with dW, db and dX requested."""
    print("single-engine backward", plan, flush=True)
    rng = np.random.default_rng(11)
    n, ci, h, w_, co = 2, 16, 12, 14, 8
    x = rng.standard_normal((n, ci, h, w_)).astype(np.float32)
    w = rng.standard_normal((co, ci, 3, 3)).astype(np.float32)
    dy = rng.standard_normal((n, co, h, w_)).astype(np.float32)
    gate = rng.standard_normal((n, co, h, w_)).astype(np.float32)
    code = native.GEMM_ENGINES["mfma"] if plan == "mfma" else native._plan_code(*plan)
    xg, wg, dyg, gateg = gpu(x), gpu(w), gpu(dy), gpu(gate)
    cols = native.conv2d_im2col(xg, w.shape, stride=(1, 1), padding=(1, 1))
    m, k = n * h * w_, ci * 9
    tiles = native._grad_tiles(n, h * w_, co, 0)
    workspace, floats = native._workspace((code, co, k, m))
    lib = native._library()

    def run(single):
        outs = [torch.empty((m, co), device="cuda"), torch.empty((co, k), device="cuda"),
                torch.empty(m * k, device="cuda"), torch.empty(x.shape, device="cuda"),
                torch.empty(n * tiles * co, dtype=torch.float64, device="cuda"), torch.empty(co, device="cuda")]
        head = (wg.data_ptr(), dyg.data_ptr(), gateg.data_ptr(), cols.data_ptr(), *(t.data_ptr() for t in outs),
                n, ci, h, w_, co, 3, 3, h, w_, 1, 1, 1, 1, tiles, 1, 0.0)
        tail = (workspace.data_ptr() if workspace is not None else 0, floats, native._stream())
        if single:
            status = lib.mfh_conv_backward_single(*head, code, *tail)
        else:
            status = lib.mfh_conv_backward(*head, code, code, *tail)
        native._raise_for(status, lib)
        return [host(t) for t in outs[1:]]

    single, pair = run(True), run(False)
    for name, a, b in zip(("dw", "grad_cols", "dx", "partial", "db"), single, pair):
        np.testing.assert_array_equal(a, b, err_msg=name)
    gated = np.where(gate > 0, dy, 0.0).astype(np.float64)
    np.testing.assert_allclose(single[4], gated.sum(axis=(0, 2, 3)), rtol=EPS32, atol=EPS32)
    dx_ref, dw_ref = naive.conv_backward(x.astype(np.float64), w.astype(np.float64), gated, (1, 1), (1, 1))
    assert_near(single[0].reshape(w.shape), dw_ref, 1e-5, "dw")
    assert_near(single[2], dx_ref, 1e-5, "dx")


def test_native_errors_name_the_reason():
    lib = native._library()
    x = torch.zeros((1, 1, 4, 4), device="cuda")
    p = x.data_ptr()
    status = lib.mfh_conv_forward(p, p, p, p, p, p, 1, 1, 4, 4, 1, 3, 3, 9, 9, 1, 1, 0, 0, 0, 0.0, 1, 0, 0, 0)
    with pytest.raises(native.NativeHipError, match=r"invalid argument.*api\.hip:\d+: .*output size"):
        native._raise_for(status, lib)
    status = lib.mfh_gemm(7, 0, 0, p, p, p, p, 2, 2, 2, 2, 2, 2, 0, 0, 0)
    with pytest.raises(native.NativeHipError, match="engine"):
        native._raise_for(status, lib)


def test_debug_sync_and_build_info():
    facts = native.info()
    assert facts["device_arch"].startswith("gfx950")
    assert facts["binary"] == "hsaco" and facts["cu_count"] > 0
    native.set_debug_sync(True)
    try:
        run_operator(CONV_CASES[1])
    finally:
        native.set_debug_sync(False)


@pytest.mark.parametrize("case", (CONV_CASES[1], PERFORMANCE_CASES[0]), ids=lambda c: c[0])
def test_rows_path_forward_matches_the_nchw_gemm(case, monkeypatch):
    """The reference's forward sequence (rows = cols W^T, then the NCHW epilogue kernel) and the
    single segmented GEMM agree within the FP64 tolerance and both keep the activation."""
    _, w_np, b_np, _ = conv_fixture(case)
    x, w, b = (gpu(a) for a in conv_fixture(case)[:3])
    direct, _ = native.conv2d_forward(x, w, b, stride=case[3], padding=case[4], activation="relu",
                                      algorithm="im2col")
    monkeypatch.setattr(native, "ROWS_PATH_MAX_PIXELS", 1 << 30)
    rows, _ = native.conv2d_forward(x, w, b, stride=case[3], padding=case[4], activation="relu",
                                    algorithm="im2col")
    _, _, _, _, pre = fp64_case(case)
    assert_near(host(direct), np.maximum(pre, 0), 1e-5, "direct")
    assert_near(host(rows), np.maximum(pre, 0), 1e-5, "rows")


def permuted_kernel(w, flip):
    """The kernel in the order an implicit product reads it, by plain tensor permutes: rows co over
    features (ci, tap) (flip 0), or rows ci over (co, KH*KW-1-tap) (flip 1); a multiple of 32
    channels takes the chunked order (channel chunk, tap, channel within the chunk)."""
    co, ci, kh, kw = w.shape
    t = w.reshape(co, ci, kh * kw)
    if flip:
        t = t.flip(2).transpose(0, 1)
    rows, channels, taps = t.shape
    if channels % 32 == 0:
        t = t.reshape(rows, channels // 32, 32, taps).permute(0, 1, 3, 2)
    return t.contiguous().reshape(-1)


def test_batched_weight_orders_match_the_permutation():
    """One conv_weight_orders call over more kernels than one launch takes (several launches), both
    orders, chunked and natural channel counts: each result equals the permuted kernel bit for bit."""
    g = torch.Generator().manual_seed(11)
    shapes = [case[2] for case in RESNET_CASES] + [(32, 96, 3, 3), (64, 32, 1, 1), (5, 7, 2, 3), (40, 64, 3, 3),
                                                    (64, 40, 3, 3), (32, 32, 5, 5)]
    requests = []
    for i in range(2 * len(shapes) + 7):
        w = torch.randn(shapes[(i // 2) % len(shapes)], generator=g).cuda()
        requests.append((w, i % 2))
    made = native.conv_weight_orders(requests)
    assert len(made) == len(requests)
    for (w, flip), out in zip(requests, made):
        np.testing.assert_array_equal(host(out), host(permuted_kernel(w, flip)), err_msg=f"{tuple(w.shape)} {flip}")


def phase_orders(w, stride, padding):
    """The strided dX order by plain tensor slicing: for each phase (a, b), a-major, the taps
    kh = (a + PH) % SH + SH * t, kw = (b + PW) % SW + SW * u of the kernel, flipped and transposed
    as the stride-1 dX order of that sub-kernel."""
    kh, kw = w.shape[2:]
    parts = []
    for a in range(stride[0]):
        for b in range(stride[1]):
            rows = list(range((a + padding[0]) % stride[0], kh, stride[0]))
            cols = list(range((b + padding[1]) % stride[1], kw, stride[1]))
            if rows and cols:
                parts.append(permuted_kernel(w[:, :, rows][:, :, :, cols].contiguous(), 1))
    return torch.cat(parts)


STRIDED = (("s2", (64, 32, 3, 3), (2, 2), (1, 1)), ("s2ds", (128, 64, 1, 1), (2, 2), (0, 0)),
           ("s3", (32, 5, 4, 5), (3, 2), (2, 1)), ("s2p0", (7, 3, 2, 3), (2, 2), (0, 0)),
           ("stem", (64, 3, 7, 7), (2, 2), (3, 3)))


def test_strided_dx_orders_are_the_phase_sub_kernels():
    """conv_weight_orders with flip 1 and a stride above 1 writes, back to back, the flipped and
    transposed sub-kernel of each dX phase (chunked when CO is a multiple of 32), bit for bit."""
    g = torch.Generator().manual_seed(13)
    weights = [torch.randn(shape, generator=g).cuda() for _, shape, _, _ in STRIDED]
    made = native.conv_weight_orders([(w, 1, s, p) for w, (_, _, s, p) in zip(weights, STRIDED)])
    for w, out, (name, _, s, p) in zip(weights, made, STRIDED):
        np.testing.assert_array_equal(host(out), host(phase_orders(w, s, p)), err_msg=name)


@pytest.mark.parametrize("case", CONV_CASES[1:] + (RESNET_CASES[2], RESNET_CASES[3], RESNET_CASES[0],
                                                   ("s3", (2, 32, 13, 11), (32, 32, 4, 5), (3, 2), (2, 1)),
                                                   ("ds_even", (2, 32, 8, 10), (64, 32, 1, 1), (2, 2), (0, 0)),
                                                   ("ds_pad", (1, 32, 7, 9), (32, 32, 1, 1), (2, 2), (1, 0)),
                                                   ("l4down3x3", (2, 256, 8, 10), (512, 256, 3, 3), (2, 2), (1, 1))),
                         ids=lambda c: c[0])
def test_strided_dx_phases_equal_the_column_path_on_integer_data(case):
    """The phase products and the column-gradient path give the same dX (and the FP64 loops') bit
    for bit on integer data, written fresh and added to an existing gradient; positions that no
    tap reaches (a 1x1 stride-2 kernel) are zero. The column path is one implicit product when the
    output channels come in chunks of 32 (its column order made by the call, or prepared by
    conv_weight_orders as the Graph does), a GEMM per image otherwise."""
    _, x_shape, w_shape, stride, padding = case
    print("phases", case[0], flush=True)
    rng = np.random.default_rng(19)
    x = rng.integers(-2, 3, size=x_shape).astype(np.float32)
    w = rng.integers(-2, 3, size=w_shape).astype(np.float32)
    n, co, oh, ow = (x_shape[0], w_shape[0], *rp.out_size(x_shape[2], x_shape[3], w_shape[2:], stride, padding))
    dy = rng.integers(-2, 3, size=(n, co, oh, ow)).astype(np.float32)
    ref_dx, _ = naive.conv_backward(x.astype(np.float64), w.astype(np.float64), dy.astype(np.float64), stride, padding)
    paths = [("phases", None), ("columns", None)]
    if w_shape[0] % 32 == 0:
        paths.append(("columns", native.conv_weight_orders([(gpu(w).reshape(w_shape[0], -1, 1, 1), 1)])[0]))
    for path, order in paths:
        label = path + (" prepared order" if order is not None else "")
        dx, _, _ = native.conv2d_backward(gpu(x), gpu(w), gpu(dy), None, stride=stride, padding=padding,
                                          algorithm="implicit", need_weight_grad=False, need_bias_grad=False,
                                          strided_dx=path, weight_flip=order)
        np.testing.assert_array_equal(host(dx), ref_dx, err_msg=label)
        existing = gpu(rng.integers(-2, 3, size=x_shape).astype(np.float32))
        expected = host(existing) + ref_dx
        native.conv2d_backward(gpu(x), gpu(w), gpu(dy), None, stride=stride, padding=padding, algorithm="implicit",
                               need_weight_grad=False, need_bias_grad=False, strided_dx=path, input_grad=existing,
                               weight_flip=order)
        np.testing.assert_array_equal(host(existing), expected, err_msg=f"{label} accumulate")


@pytest.mark.parametrize("shape,stride,padding", (((2, 64, 29, 39), (2, 2), (0, 0)), ((2, 64, 8, 10), (2, 2), (0, 0)),
                                                   ((1, 32, 7, 9), (2, 2), (1, 0)), ((1, 32, 10, 7), (3, 2), (0, 0))))
def test_strided_1x1_dx_writes_every_position(shape, stride, padding):
    """A strided 1x1 dX into a buffer full of NaN: the phase product (with the cell zeros of its
    epilogue, or after a fill when its phase is not the first) leaves no position unwritten."""
    print("1x1 strided", shape, stride, padding, flush=True)
    rng = np.random.default_rng(29)
    x = rng.integers(-2, 3, size=shape).astype(np.float32)
    w = rng.integers(-2, 3, size=(64, shape[1], 1, 1)).astype(np.float32)
    g = native.ConvGeometry.of(shape, w.shape, stride, padding)
    dy = rng.integers(-2, 3, size=g.out_shape).astype(np.float32)
    ref_dx, _ = naive.conv_backward(x.astype(np.float64), w.astype(np.float64), dy.astype(np.float64), stride, padding)
    lib, s = native._library(), torch.cuda.current_stream().cuda_stream
    wg, dyg = gpu(w), gpu(dy)
    (order,) = native.conv_weight_orders([(wg, 1, stride, padding)])
    dx = torch.full(shape, float("nan"), device="cuda")
    workspace = torch.empty(1 << 22, device="cuda")
    native._raise_for(lib.mfh_conv_backward_implicit(
        gpu(x).data_ptr(), wg.data_ptr(), dyg.data_ptr(), 0, 0, 0, dx.data_ptr(), order.data_ptr(), 0, 0, 0,
        *g.c_args(), 0, 0.0, 1, 1, native.CONV_WFLIP_READY, workspace.data_ptr(), workspace.numel(), s), lib)
    np.testing.assert_array_equal(host(dx), ref_dx)


@pytest.mark.parametrize("case", (RESNET_CASES[1], RESNET_CASES[2], RESNET_CASES[3], RESNET_CASES[4],
                                  RESNET_CASES[5], PERFORMANCE_CASES[0]), ids=lambda c: c[0])
def test_prepared_orders_and_in_place_dx_give_the_same_bits(case):
    """A forward that reads a prepared kernel order, a dX that reads a prepared dX order (the
    flipped kernel, or for a stride above 1 its phase sub-kernels) and a dX added in place to an
    existing gradient give exactly the results of the plain calls (the in-place add is the same
    float32 addition as a separate one)."""
    print("prepared", case[0], flush=True)
    x, w, b, dy = (gpu(a) for a in conv_fixture(case))
    stride, padding = case[3], case[4]
    plain_y, _ = native.conv2d_forward(x, w, b, stride=stride, padding=padding, algorithm="implicit")
    order, flip = native.conv_weight_orders([(w, 0), (w, 1, stride, padding)])
    prepared_y, _ = native.conv2d_forward(x, w, b, stride=stride, padding=padding, algorithm="implicit",
                                          weight_order=order)
    np.testing.assert_array_equal(host(prepared_y), host(plain_y))
    dx, dw, db = native.conv2d_backward(x, w, dy, None, stride=stride, padding=padding, algorithm="implicit",
                                        strided_dx="phases")
    existing = torch.randn(x.shape, generator=torch.Generator().manual_seed(5)).cuda()
    expected = host(existing) + host(dx)
    dx2, dw2, db2 = native.conv2d_backward(x, w, dy, None, stride=stride, padding=padding, algorithm="implicit",
                                           input_grad=existing, weight_flip=flip, strided_dx="phases")
    assert dx2 is existing
    np.testing.assert_array_equal(host(dx2), expected)
    np.testing.assert_array_equal(host(dw2), host(dw))
    np.testing.assert_array_equal(host(db2), host(db))


@pytest.mark.parametrize("case", (RESNET_CASES[0], RESNET_CASES[1], RESNET_CASES[4]), ids=lambda c: c[0])
def test_bias_gradient_with_and_without_the_weight_product(case):
    """db rides on the dW product when dW is requested (FP64 sums per pixel slice) and takes the
    per-image row sums otherwise: both within one float32 ulp of the FP64 sum."""
    x, w, _, dy = (gpu(a) for a in conv_fixture(case))
    ref = conv_fixture(case)[3].astype(np.float64).sum(axis=(0, 2, 3))
    for need_w in (True, False):
        _, dw, db = native.conv2d_backward(x, w, dy, None, stride=case[3], padding=case[4], algorithm="implicit",
                                           need_input_grad=False, need_weight_grad=need_w)
        assert (dw is not None) == need_w
        assert np.all(np.abs(host(db) - ref) <= np.spacing(np.abs(ref).astype(np.float32))), need_w


def test_stem_weight_gradient_at_batch_64_is_exact_on_integer_data():
    """The bs64 stem dW (64 x 147 over 307200 pixels: the measured plan splits it into 256 pixel
    slices, with the bias sums of every slice) on integer data, where every float32 partial sum is
    exact (|sum| <= 4 * 307200 < 2**24): dW and db equal the FP64 product bit for bit."""
    print("stem dW bs64", flush=True)
    rng = np.random.default_rng(23)
    x = rng.integers(-2, 3, size=(64, 3, 120, 160)).astype(np.float32)
    w = rng.integers(-2, 3, size=(64, 3, 7, 7)).astype(np.float32)
    dy = rng.integers(-2, 3, size=(64, 64, 60, 80)).astype(np.float32)
    _, dw, db = native.conv2d_backward(gpu(x), gpu(w), gpu(dy), None, stride=(2, 2), padding=(3, 3),
                                       algorithm="implicit", need_input_grad=False)
    padded = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (3, 3), (3, 3)))
    windows = np.lib.stride_tricks.sliding_window_view(padded, (7, 7), axis=(2, 3))[:, :, ::2, ::2]
    cols = windows.transpose(0, 2, 3, 1, 4, 5).reshape(64 * 60 * 80, 3 * 49)
    rows = dy.astype(np.float64).reshape(64, 64, 4800).transpose(1, 0, 2).reshape(64, -1)
    np.testing.assert_array_equal(host(dw).reshape(64, -1), rows @ cols)
    np.testing.assert_array_equal(host(db), rows.sum(axis=1))


def _stem_reference(x, w, stride, padding):
    """FP64 convolution through explicit windows (no im2col code of the library)."""
    kh, kw = w.shape[2:]
    padded = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (padding[0],) * 2, (padding[1],) * 2))
    windows = np.lib.stride_tricks.sliding_window_view(padded, (kh, kw), axis=(2, 3))
    windows = windows[:, :, ::stride[0], ::stride[1]]
    n, c, oh, ow = windows.shape[:4]
    cols = windows.transpose(0, 2, 3, 1, 4, 5).reshape(n * oh * ow, c * kh * kw)
    out = cols @ w.astype(np.float64).reshape(w.shape[0], -1).T
    return out.reshape(n, oh, ow, -1).transpose(0, 3, 1, 2)


@pytest.mark.parametrize("shape,kernel,stride,padding,co", [
    ((64, 3, 120, 160), (7, 7), (2, 2), (3, 3), 64),   # the ResNet18 stem at batch 64
    ((3, 3, 33, 47), (7, 5), (1, 1), (2, 2), 70),      # five taps per row, two channel tiles
    ((2, 3, 17, 29), (7, 8), (2, 3), (0, 4), 16),      # eight taps, uneven strides
])
def test_stem_forward_is_exact_on_integer_data(shape, kernel, stride, padding, co):
    """Stem-shaped forwards (3 input channels, a 7-row window of 5-8 taps, the natural feature
    order of the implicit product) on integer data, where every float32 sum is exact: y equals the
    FP64 convolution bit for bit, with bias and ReLU applied as the implicit epilogue does (bias
    after the sum, then the activation)."""
    print("stem forward", shape, kernel, stride, padding, co, flush=True)
    rng = np.random.default_rng(31)
    x = rng.integers(-2, 3, size=shape).astype(np.float32)
    w = rng.integers(-2, 3, size=(co, 3, *kernel)).astype(np.float32)
    bias = rng.integers(-3, 4, size=co).astype(np.float32)
    ref = _stem_reference(x, w, stride, padding)
    y, _ = native.conv2d_forward(gpu(x), gpu(w), stride=stride, padding=padding, algorithm="implicit")
    np.testing.assert_array_equal(host(y), ref)
    y, _ = native.conv2d_forward(gpu(x), gpu(w), gpu(bias), stride=stride, padding=padding, activation="relu",
                                 algorithm="implicit")
    np.testing.assert_array_equal(host(y), np.maximum(ref + bias.reshape(1, -1, 1, 1), 0.0))


def test_stem_forward_keeps_an_inf_out_of_windows_that_do_not_cover_it():
    """An Inf in the input reaches exactly the outputs whose windows cover it (as Inf, or NaN where
    the weight on it is zero): a gather that read a pixel beside a window, even under a zero weight,
    would turn that output into NaN."""
    print("stem inf", flush=True)
    rng = np.random.default_rng(5)
    x = rng.integers(-2, 3, size=(1, 3, 20, 24)).astype(np.float32)
    w = rng.integers(-2, 3, size=(8, 3, 7, 7)).astype(np.float32)
    x[0, 1, 9, 12] = np.inf
    y = host(native.conv2d_forward(gpu(x), gpu(w), stride=(2, 2), padding=(3, 3), algorithm="implicit")[0])
    covered = np.zeros(y.shape[2:], dtype=bool)
    for oh in range(y.shape[2]):
        for ow in range(y.shape[3]):
            covered[oh, ow] = 0 <= 9 - (2 * oh - 3) < 7 and 0 <= 12 - (2 * ow - 3) < 7
    assert covered.any() and (~covered).any()
    assert np.isfinite(y[:, :, ~covered]).all() and not np.isfinite(y[:, :, covered]).any()
    # Inf (nonzero weight) or NaN (zero weight) where the window covers the Inf, as in FP64.
    with np.errstate(invalid="ignore"):
        ref = _stem_reference(x, w, (2, 2), (3, 3))
    np.testing.assert_array_equal(y, ref)


IMPLICIT_TILES = 12  # tiles of the implicit products (plan code 16 + tile * 128 + slices - 1)


@pytest.mark.parametrize("case", (RESNET_CASES[1], ("l2s", (2, 128, 15, 20), (128, 128, 3, 3), (1, 1), (1, 1)),
                                  PARTIAL_ROW_CASES[0]), ids=lambda c: c[0])
def test_every_implicit_tile_is_exact_on_integer_data(case):
    """Each tile of the implicit catalogue (forced through its plan code, unsplit and split over K;
    the 24-way dW split takes the grouped reduction) gives the FP64 loops' forward, dX, dW and db
    bit for bit on integer data; a tile without a kernel for a product (the 96-pixel one: no dW,
    and no natural-order dX, which 40 output channels take) is refused with a reason instead of
    launched."""
    _, x_shape, w_shape, stride, padding = case
    print("tiles", case[0], flush=True)
    rng = np.random.default_rng(17)
    x = rng.integers(-2, 3, size=x_shape).astype(np.float32)
    w = rng.integers(-2, 3, size=w_shape).astype(np.float32)
    n, co = x_shape[0], w_shape[0]
    oh, ow = rp.out_size(x_shape[2], x_shape[3], w_shape[2:], stride, padding)
    dy = rng.integers(-2, 3, size=(n, co, oh, ow)).astype(np.float32)
    x64, w64, dy64 = x.astype(np.float64), w.astype(np.float64), dy.astype(np.float64)
    ref_y = naive.conv_forward(x64, w64, stride, padding)
    ref_dx, ref_dw = naive.conv_backward(x64, w64, dy64, stride, padding)
    ref_db = dy64.sum(axis=(0, 2, 3))
    g = native.ConvGeometry.of(x_shape, w_shape, stride, padding)
    lib, stream = native._library(), torch.cuda.current_stream().cuda_stream
    xg, wg, dyg = gpu(x), gpu(w), gpu(dy)
    order, flip = native.conv_weight_orders([(wg, 0), (wg, 1)])
    y, dx, dw = torch.empty(g.out_shape, device="cuda"), torch.empty_like(xg), torch.empty_like(wg)
    db = torch.empty(co, device="cuda")
    partial = torch.empty(max(n, native.BIAS_PARTIAL_ROWS) * co, dtype=torch.float64, device="cuda")
    workspace = torch.empty(1 << 24, device="cuda")
    for tile in range(IMPLICIT_TILES):
        for slices in (1, 3, 24):
            code = native.IMPLICIT_PLAN_BASE + tile * native.IMPLICIT_PLAN_SLICES + slices - 1
            native._raise_for(lib.mfh_conv_forward_implicit(
                xg.data_ptr(), wg.data_ptr(), order.data_ptr(), 1, 0, 0, y.data_ptr(), *g.c_args(), 0, 0.0, code,
                workspace.data_ptr(), workspace.numel(), stream), lib)
            status = lib.mfh_conv_backward_implicit(
                xg.data_ptr(), wg.data_ptr(), dyg.data_ptr(), 0, 0, 0, dx.data_ptr(), flip.data_ptr(), 0, 0, 0,
                *g.c_args(), 0, 0.0, 1, code, native.CONV_WFLIP_READY, workspace.data_ptr(), workspace.numel(),
                stream)
            np.testing.assert_array_equal(host(y), ref_y, err_msg=f"forward tile {tile} slices {slices}")
            if tile == 11 and co % 32 != 0:
                assert status == 2 and "no kernel" in lib.mfh_last_error().decode()
            else:
                native._raise_for(status, lib)
                np.testing.assert_array_equal(host(dx), ref_dx, err_msg=f"dX tile {tile} slices {slices}")
            status = lib.mfh_conv_backward_implicit(
                xg.data_ptr(), wg.data_ptr(), dyg.data_ptr(), 0, 0, dw.data_ptr(), 0, 0, 0, partial.data_ptr(),
                db.data_ptr(), *g.c_args(), 0, 0.0, code, 1, 0, workspace.data_ptr(), workspace.numel(), stream)
            if tile == 11:
                assert status == 2 and "no kernel" in lib.mfh_last_error().decode()
                continue
            native._raise_for(status, lib)
            np.testing.assert_array_equal(host(dw), ref_dw, err_msg=f"dW tile {tile} slices {slices}")
            np.testing.assert_array_equal(host(db), ref_db, err_msg=f"db tile {tile} slices {slices}")


@pytest.mark.parametrize("shape,kernel,stride,padding", [
    ((2, 64, 9, 11), (64, 64, 3, 3), 1, 1),     # chunked features, unsplit
    ((3, 3, 20, 18), (16, 3, 7, 7), 2, 3),      # natural-order stem-like gather
    ((4, 512, 4, 5), (512, 512, 3, 3), 1, 1),   # layer4-like: split K, residual in the slice reduction
])
def test_residual_epilogue_equals_separate_add_and_relu(shape, kernel, stride, padding):
    """act((conv + bias) + residual) from the epilogue against the same convolution without the
    residual, then a float32 add and ReLU: bit for bit, split and unsplit plans alike."""
    rng = np.random.default_rng(11)
    stride, padding = (stride, stride), (padding, padding)
    x = gpu(rng.standard_normal(shape).astype(np.float32))
    w = gpu((rng.standard_normal(kernel) * (2.0 / np.prod(kernel[1:])) ** 0.5).astype(np.float32))
    b = gpu(rng.standard_normal(kernel[0]).astype(np.float32))
    plain, _ = native.conv2d_forward(x, w, b, stride=stride, padding=padding, algorithm="implicit")
    residual = gpu(rng.standard_normal(tuple(plain.shape)).astype(np.float32))
    fused, _ = native.conv2d_forward(x, w, b, stride=stride, padding=padding, activation="relu",
                                     algorithm="implicit", residual=residual)
    torch.cuda.synchronize()
    assert torch.equal(fused, torch.relu(plain + residual))
    # The same through explicit plan codes (64 x 64 tile of four 32 x 32 waves), unsplit and split
    # three ways, so that the residual is read both by the product's epilogue and by the split-K
    # reduction that finishes the split plan.
    g = native.ConvGeometry.of(shape, kernel, stride, padding)
    lib, stream = native._library(), torch.cuda.current_stream().cuda_stream
    wt = torch.empty_like(w)
    workspace = torch.empty(3 * g.co * g.m, device="cuda")
    for slices in (1, 3):
        code = native.IMPLICIT_PLAN_BASE + 6 * native.IMPLICIT_PLAN_SLICES + slices - 1
        outputs = []
        for extra, act in ((0, 0), (residual.data_ptr(), 1)):
            out = torch.full(g.out_shape, float("nan"), device="cuda")
            native._raise_for(lib.mfh_conv_forward_implicit(
                x.data_ptr(), w.data_ptr(), wt.data_ptr(), 0, b.data_ptr(), extra, out.data_ptr(), *g.c_args(), act,
                0.0, code, workspace.data_ptr(), workspace.numel(), stream), lib)
            outputs.append(out)
        torch.cuda.synchronize()
        assert torch.equal(outputs[1], torch.relu(outputs[0] + residual)), f"slices {slices}"
    with pytest.raises(ValueError, match="output shape"):
        native.conv2d_forward(x, w, b, stride=stride, padding=padding, algorithm="implicit", residual=residual[:1])
    with pytest.raises(ValueError, match="implicit"):
        native.conv2d_forward(x, w, b, stride=stride, padding=padding, algorithm="im2col", residual=residual)


def test_residual_may_not_be_the_output():
    x = gpu(np.ones((1, 4, 6, 6), np.float32))
    w = gpu(np.ones((4, 4, 3, 3), np.float32))
    y = torch.zeros((1, 4, 6, 6), device="cuda")
    lib = native._library()
    dims = (1, 4, 6, 6, 4, 3, 3, 6, 6, 1, 1, 1, 1)
    status = lib.mfh_conv_forward_implicit(x.data_ptr(), w.data_ptr(), 0, 0, 0, y.data_ptr(), y.data_ptr(), *dims,
                                           1, 0.0, 1, 0, 0, torch.cuda.current_stream().cuda_stream)
    assert status != 0 and "residual" in lib.mfh_last_error().decode()


# Convolutions whose implicit products hit every entry of the measured-plan table of the implicit
# products (csrc/implicit.hip, MEASURED_PLANS: key orientation, M, N, K): ResNet18's batch-64
# convolutions at 3 x 120 x 160 (forward, dW, and the stride-1 dX, which shares its forward's key) and
# its batch-256 224 x 224 inference forwards. Passes that have no measured entry run their automatic
# plans and are checked too.
PLAN_GEOMETRIES = (
    ("bs64-stem", (64, 3, 120, 160), (64, 3, 7, 7), 2, 3, ("forward", "dw")),
    ("bs64-layer1", (64, 64, 29, 39), (64, 64, 3, 3), 1, 1, ("forward", "dx", "dw")),
    ("bs64-layer2.0-conv1", (64, 64, 29, 39), (128, 64, 3, 3), 2, 1, ("forward", "dx", "dw")),
    ("bs64-layer2-3x3", (64, 128, 15, 20), (128, 128, 3, 3), 1, 1, ("forward", "dx", "dw")),
    ("bs64-layer2-1x1", (64, 64, 29, 39), (128, 64, 1, 1), 2, 0, ("forward", "dx", "dw")),
    ("bs64-layer3.0-conv1", (64, 128, 15, 20), (256, 128, 3, 3), 2, 1, ("forward", "dx", "dw")),
    ("bs64-layer3-3x3", (64, 256, 8, 10), (256, 256, 3, 3), 1, 1, ("forward", "dx", "dw")),
    ("bs64-layer3-1x1", (64, 128, 15, 20), (256, 128, 1, 1), 2, 0, ("forward", "dx", "dw")),
    ("bs64-layer4.0-conv1", (64, 256, 8, 10), (512, 256, 3, 3), 2, 1, ("forward", "dx", "dw")),
    ("bs64-layer4-3x3", (64, 512, 4, 5), (512, 512, 3, 3), 1, 1, ("forward", "dx", "dw")),
    ("bs64-layer4-1x1", (64, 256, 8, 10), (512, 256, 1, 1), 2, 0, ("forward", "dx", "dw")),
    ("bs256-stem", (256, 3, 224, 224), (64, 3, 7, 7), 2, 3, ("forward",)),
    ("bs256-layer1", (256, 64, 55, 55), (64, 64, 3, 3), 1, 1, ("forward",)),
    ("bs256-layer2.0-conv1", (256, 64, 55, 55), (128, 64, 3, 3), 2, 1, ("forward",)),
    ("bs256-layer2-3x3", (256, 128, 28, 28), (128, 128, 3, 3), 1, 1, ("forward",)),
    ("bs256-layer2-1x1", (256, 64, 55, 55), (128, 64, 1, 1), 2, 0, ("forward",)),
    ("bs256-layer3.0-conv1", (256, 128, 28, 28), (256, 128, 3, 3), 2, 1, ("forward",)),
    ("bs256-layer3-3x3", (256, 256, 14, 14), (256, 256, 3, 3), 1, 1, ("forward",)),
    ("bs256-layer3-1x1", (256, 128, 28, 28), (256, 128, 1, 1), 2, 0, ("forward",)),
    ("bs256-layer4.0-conv1", (256, 256, 14, 14), (512, 256, 3, 3), 2, 1, ("forward",)),
    ("bs256-layer4-3x3", (256, 512, 7, 7), (512, 512, 3, 3), 1, 1, ("forward",)),
)


@pytest.mark.parametrize("geometry", PLAN_GEOMETRIES, ids=lambda g: g[0])
def test_measured_plans_are_exact_on_integer_data(geometry):
    """Each convolution at its full size under the automatic plan (so the measured plan of its
    shape, split-K and grouped reductions included) on integer data in [-2, 2], where every float32
    partial sum is exact: the forward and dX of the first, middle and last image (an output image
    depends on its own input image only) and dW and db over the whole batch equal the FP64
    convolution bit for bit."""
    name, x_shape, w_shape, stride, padding, passes = geometry
    print("measured plan", name, passes, flush=True)
    stride, padding = (stride, stride), (padding, padding)
    rng = np.random.default_rng(29)
    x = rng.integers(-2, 3, size=x_shape).astype(np.float32)
    w = rng.integers(-2, 3, size=w_shape).astype(np.float32)
    g = native.ConvGeometry.of(x_shape, w_shape, stride, padding)
    picks = sorted({0, x_shape[0] // 2, x_shape[0] - 1})
    x64, w64 = torch.from_numpy(x).double(), torch.from_numpy(w).double()
    xg, wg = gpu(x), gpu(w)
    y, _ = native.conv2d_forward(xg, wg, None, stride=stride, padding=padding, algorithm="implicit")
    ref_y = torch.nn.functional.conv2d(x64[picks], w64, stride=stride, padding=padding).numpy()
    np.testing.assert_array_equal(host(y[picks]), ref_y, err_msg=f"{name} forward")
    del y
    if "dx" not in passes and "dw" not in passes:
        return
    dy = rng.integers(-2, 3, size=g.out_shape).astype(np.float32)
    dx, dw, db = native.conv2d_backward(xg, wg, gpu(dy), None, stride=stride, padding=padding, algorithm="implicit",
                                        need_input_grad="dx" in passes, need_weight_grad="dw" in passes)
    dy64 = torch.from_numpy(dy).double()
    if "dx" in passes:
        ref_dx = torch.nn.grad.conv2d_input((len(picks),) + tuple(x_shape[1:]), w64, dy64[picks], stride=stride,
                                            padding=padding).numpy()
        np.testing.assert_array_equal(host(dx[picks]), ref_dx, err_msg=f"{name} dX")
    if "dw" in passes:
        ref_dw = torch.nn.grad.conv2d_weight(x64, tuple(w_shape), dy64, stride=stride, padding=padding).numpy()
        np.testing.assert_array_equal(host(dw), ref_dw, err_msg=f"{name} dW")
    np.testing.assert_array_equal(host(db), dy64.sum(dim=(0, 2, 3)).numpy(), err_msg=f"{name} db")


@pytest.mark.parametrize("shape,kernel,stride,padding,activation,in_place", [
    ((4, 64, 15, 20), (64, 64, 3, 3), 1, 1, "relu", False),   # gated dy, stride-1 dX
    ((4, 64, 15, 20), (128, 64, 3, 3), 2, 1, None, False),    # strided 3x3: column-gradient dX
    ((4, 64, 15, 20), (128, 64, 1, 1), 2, 0, None, True),     # strided 1x1: phase dX, added in place
    ((8, 512, 4, 5), (512, 512, 3, 3), 1, 1, None, True),     # split-K dW and dX at once
    ((3, 3, 20, 18), (16, 3, 7, 7), 2, 3, None, False),       # natural-order stem gather
])
def test_weight_gradient_stream_call_gives_the_one_stream_bits(shape, kernel, stride, padding, activation,
                                                               in_place):
    """mfh_conv_backward_implicit_streams (dW and db on a second stream, dX on the current one)
    against the one-stream call: dX, dW and db bit for bit once the current stream is ordered after
    the second one; every buffer of the call is handed to the hold list."""
    rng = np.random.default_rng(23)
    x = gpu(rng.standard_normal(shape).astype(np.float32))
    w = gpu((rng.standard_normal(kernel) * (2.0 / np.prod(kernel[1:])) ** 0.5).astype(np.float32))
    b = gpu(rng.standard_normal(kernel[0]).astype(np.float32))
    stride, padding = (stride, stride), (padding, padding)
    y, _ = native.conv2d_forward(x, w, b, stride=stride, padding=padding, activation=activation,
                                 algorithm="implicit")
    dy = gpu(rng.standard_normal(tuple(y.shape)).astype(np.float32))
    base = gpu(rng.standard_normal(shape).astype(np.float32))
    side = torch.cuda.Stream()
    results = []
    for two_streams in (False, True):
        extra = {"input_grad": base.clone()} if in_place else {}
        hold = [] if two_streams else None
        options = {"dw_stream": side.cuda_stream, "hold": hold} if two_streams else {}
        grads = native.conv2d_backward(x, w, dy, None, stride=stride, padding=padding, activation=activation,
                                       output=y, algorithm="implicit", **options, **extra)
        if two_streams:
            native.stream_wait(native._stream(), side.cuda_stream)
            assert len(hold) >= 5 and all(isinstance(t, torch.Tensor) for t in hold)
        results.append([host(g) for g in grads])
    for got, want, name in zip(results[1], results[0], ("dx", "dw", "db")):
        np.testing.assert_array_equal(got, want, err_msg=name)


def test_a_convolution_beyond_the_buffer_loads_takes_the_im2col_algorithm():
    """A 1x1 convolution over 32 channels whose input holds more floats than a chunked implicit
    product's buffer loads address (2 GiB) but whose columns fit the geometry's int32 limits: the
    default algorithm is then im2col (forward returns cols), the explicit implicit call is refused
    with status 2, and the forward, dX and dW are exact on integer data (FP64 on the GPU as the
    reference; a 1x1 convolution's rows are independent, so a crop run by the implicit product
    checks the forward too)."""
    shape, w_shape = (1, 32, 4100, 4100), (32, 32, 1, 1)
    g = native.ConvGeometry.of(shape, w_shape, (1, 1), (0, 0))
    assert not native.implicit_fits(g) and native.implicit_fits(native.ConvGeometry.of(
        (1, 32, 64, 4100), w_shape, (1, 1), (0, 0)))
    print("beyond buffer loads", shape, flush=True)
    gen = torch.Generator(device="cuda").manual_seed(37)
    x = torch.randint(-1, 2, shape, generator=gen, device="cuda").float()
    w = torch.randint(-2, 3, w_shape, generator=gen, device="cuda").float()
    dy = torch.randint(-1, 2, shape, generator=gen, device="cuda").float()
    with pytest.raises(native.NativeHipError):
        native.conv2d_forward(x, w, algorithm="implicit")
    y, cols = native.conv2d_forward(x, w)
    assert cols is not None
    crop, _ = native.conv2d_forward(x[:, :, :64].contiguous(), w, algorithm="implicit")
    assert torch.equal(y[:, :, :64], crop)
    w2 = w.reshape(32, 32).double()
    expected = (w2 @ x.reshape(32, -1).double()).reshape(shape)
    assert torch.equal(y.double(), expected)
    del expected, crop
    dx, dw, db = native.conv2d_backward(x, w, dy, None, need_bias_grad=True)
    dyf = dy.reshape(32, -1).double()
    assert torch.equal(dw.reshape(32, 32).double(), dyf @ x.reshape(32, -1).double().T)
    assert torch.equal(db.double(), dyf.sum(dim=1))
    assert torch.equal(dx.double(), (w2.T @ dyf).reshape(shape))
