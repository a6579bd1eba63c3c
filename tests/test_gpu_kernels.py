"""Parity of the libmfhip kernels with the CPU oracle, through the C ABI (the native.py boundary).

Bit-exact: im2col, col2im (native gather order), max-pool values, argmax and gradients (including
ties, -inf padding, overlapping windows and NaN), the split-K reduction. Tolerance (written in each
test): GEMM / convolution results against FP64 references, as the reference's own tests do
(tests/test_cuda_native_kernels.py:34-38, :214, :294-305 of the reference).
"""

import numpy as np
import pytest
import torch

import myflows_amd as mf
from myflows_amd import native
from oracle import naive, reference_path as rp
from tests.fixtures import CONV_CASES, EPS32, PERFORMANCE_CASES, POOL_CASES, assert_near, conv_fixture, gamma_k

pytestmark = pytest.mark.gpu


def gpu(a):
    return torch.as_tensor(np.ascontiguousarray(a), device="cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def _run_conv(case, op_class=mf.Conv2D_Op, needs_input_grad=True, **kwargs):
    x, w, b, dy = (gpu(a) for a in conv_fixture(case, 0))
    x_node = mf.Variable(x, requires_grad=needs_input_grad)
    w_node, b_node = mf.Variable(w, trainable=True), mf.Variable(b, trainable=True)
    op = op_class(x_node, w_node, stride=case[3], padding=case[4], bias=b_node, backend="hip_native", **kwargs)
    op.forward(x, w, b)
    op.grad = dy
    op.backward()
    grads = [None if n.grad is None else host(n.grad) for n in (x_node, w_node, b_node)]
    return op, host(op.value), grads


def _fp64_reference(case):
    x, w, b, dy = (a.astype(np.float64) for a in conv_fixture(case, 0))
    pre = naive.conv_forward(x, w, case[3], case[4]) + b[None, :, None, None]
    return x, w, b, dy, pre


@pytest.mark.parametrize("case", CONV_CASES + PERFORMANCE_CASES, ids=lambda c: c[0])
def test_conv_forward_backward_match_fp64(case):
    print("conv case", case[0], flush=True)
    x, w, _, dy, pre = _fp64_reference(case)
    op, y, (dx, dw, db) = _run_conv(case)
    assert op.value.is_contiguous()
    ref_dx, ref_dw = naive.conv_backward(x, w, dy, case[3], case[4])
    assert_near(y, pre, 1e-5, "y")
    assert_near(dx, ref_dx, 1e-5, "dx")
    assert_near(dw, ref_dw, 1e-5, "dw")
    ref_db = dy.sum(axis=(0, 2, 3))
    assert np.all(np.abs(db - ref_db) <= np.spacing(np.abs(ref_db).astype(np.float32))), "db beyond one ulp"


def test_conv_known_answer_t0_is_exact():
    _, y, _ = _run_conv(CONV_CASES[0])
    grid = np.arange(25).reshape(5, 5)
    expected = np.array([[grid[i:i + 3, j:j + 3].sum() for j in range(3)] for i in range(3)], dtype=np.float32)
    assert np.array_equal(y[0, 0], expected)


@pytest.mark.parametrize("case", (CONV_CASES[1], CONV_CASES[3], PERFORMANCE_CASES[2]), ids=lambda c: c[0])
@pytest.mark.parametrize("variant", ("relu", "leaky"))
def test_fused_relu_and_leaky_relu_match_fp64(case, variant):
    print("fused", variant, case[0], flush=True)
    x, w, _, dy, pre = _fp64_reference(case)
    op_class, kwargs, slope = ((mf.Conv2D_ReLU_Op, {}, 0.0) if variant == "relu"
                               else (mf.Conv2D_LeakyReLU_Op, {"alpha": 0.2}, 0.2))
    op, y, (dx, dw, db) = _run_conv(case, op_class, **kwargs)
    assert op._activation_fused
    gate = np.where(pre > 0, 1.0, slope)
    ref_dx, ref_dw = naive.conv_backward(x, w, dy * gate, case[3], case[4])
    assert_near(y, np.where(pre > 0, pre, slope * pre), 1e-5, "y")
    assert_near(dx, ref_dx, 1e-5, "dx")
    assert_near(dw, ref_dw, 1e-5, "dw")
    assert_near(db, (dy * gate).sum(axis=(0, 2, 3)), 4 * EPS32, "db")


def test_input_without_requires_grad_skips_dx():
    case = PERFORMANCE_CASES[0]
    _, _, (_, dw_full, db_full) = _run_conv(case)
    _, _, (dx, dw, db) = _run_conv(case, needs_input_grad=False)
    assert dx is None
    np.testing.assert_array_equal(dw, dw_full)
    np.testing.assert_array_equal(db, db_full)


def test_dx_only_direct_path_matches_fp64():
    """Frozen weights and bias: dX alone takes the per-image transposed-dy GEMM."""
    case = PERFORMANCE_CASES[2]
    x, w, b, dy = conv_fixture(case, 0)
    xv = mf.Variable(gpu(x))
    wv, bv = mf.Variable(gpu(w), requires_grad=False), mf.Variable(gpu(b), requires_grad=False)
    op = mf.Conv2D_ReLU_Op(xv, wv, stride=case[3], padding=case[4], bias=bv, backend="hip_native")
    op.forward(xv.value, wv.value, bv.value)
    op.grad = gpu(dy)
    op.backward()
    pre = naive.conv_forward(x.astype(np.float64), w.astype(np.float64), case[3], case[4]) + b[None, :, None, None]
    ref_dx, _ = naive.conv_backward(x.astype(np.float64), w.astype(np.float64), dy * (pre > 0), case[3], case[4])
    assert wv.grad is None and bv.grad is None
    assert_near(host(xv.grad), ref_dx, 1e-5, "dx")


@pytest.mark.parametrize("case", (PERFORMANCE_CASES[0], PERFORMANCE_CASES[1]), ids=lambda c: c[0])
def test_gradients_are_bitwise_reproducible(case):
    first = _run_conv(case)[2]
    second = _run_conv(case)[2]
    for a, b in zip(first, second):
        np.testing.assert_array_equal(a, b)


def test_native_errors_name_the_reason():
    lib = native._library()
    x = torch.zeros((1, 1, 4, 4), device="cuda")
    status = lib.mfh_conv_forward(*(native._u64(x.data_ptr()),) * 6,
                                  *(native._i32(v) for v in (1, 1, 4, 4, 1, 3, 3, 9, 9, 1, 1, 0, 0)),
                                  native._i32(0), native.ctypes.c_float(0.0), native._i32(1), native._u64(0),
                                  native.ctypes.c_int64(0), native._u64(0))
    with pytest.raises(native.NativeHipError, match=r"invalid argument.*api\.hip:\d+: .*output size"):
        native._check(status, lib)
    status = lib.mfh_gemm(native._i32(7), 0, 0, *(native._u64(x.data_ptr()),) * 4, *(native._i32(2),) * 6,
                          native._u64(0), native.ctypes.c_int64(0), native._u64(0))
    with pytest.raises(native.NativeHipError, match="engine"):
        native._check(status, lib)


def test_debug_sync_and_build_info():
    info = native.info()
    assert info["device_arch"].startswith("gfx950")
    assert info["binary"] == "hsaco" and info["cu_count"] > 0
    native.set_debug_sync(True)
    try:
        _run_conv(CONV_CASES[1])
    finally:
        native.set_debug_sync(False)


@pytest.mark.parametrize("shape,kernel,stride,padding", [
    ((2, 3, 7, 9), (3, 3), (1, 1), (1, 1)), ((1, 2, 8, 9), (3, 2), (2, 3), (1, 0)), ((2, 3, 16, 16), (7, 7), (2, 2), (3, 3)),
    ((3, 5, 6, 5), (1, 1), (2, 2), (0, 0)), ((2, 64, 30, 40), (3, 3), (1, 1), (1, 1))])
def test_im2col_and_col2im_are_bit_exact(shape, kernel, stride, padding):
    """im2col is a copy; col2im is checked with integer-valued dy and W, for which the dX GEMM and
    the gather sums are exact in float32, so any index or window error shows as a bit difference."""
    print("im2col", shape, kernel, stride, padding, flush=True)
    rng = np.random.default_rng(3)
    x = rng.standard_normal(shape).astype(np.float32)
    co = 4
    w_shape = (co, shape[1], *kernel)
    cols = native.conv2d_im2col(gpu(x), w_shape, stride=stride, padding=padding)
    np.testing.assert_array_equal(host(cols), rp.im2col(x, kernel, stride, padding))
    oh, ow = rp.out_size(shape[2], shape[3], kernel, stride, padding)
    w = rng.integers(-2, 3, size=w_shape).astype(np.float32)
    dy = rng.integers(-3, 4, size=(shape[0], co, oh, ow)).astype(np.float32)
    grad_cols = dy.transpose(0, 2, 3, 1).reshape(-1, co).astype(np.float64) @ w.reshape(co, -1)
    expected = rp.col2im_native(grad_cols.astype(np.float32), shape, kernel, stride, padding)
    np.testing.assert_array_equal(expected, naive.col2im(grad_cols, shape, kernel, stride, padding))
    for need_w in (False, True):  # dX-only (per-image TN GEMM) and the full path (NN GEMM)
        dx, _, _ = native.conv2d_backward(gpu(x), gpu(w), gpu(dy), cols, stride=stride, padding=padding,
                                          need_bias_grad=need_w, need_weight_grad=need_w)
        np.testing.assert_array_equal(host(dx), expected)


@pytest.mark.parametrize("shape,kernel,stride,padding", POOL_CASES + (((4, 8, 60, 80), (3, 3), (2, 2), (0, 0)),
                                                                       ((2, 4, 30, 40), (2, 2), (2, 2), (0, 0))))
def test_maxpool_bit_exact_with_ties_padding_and_overlap(shape, kernel, stride, padding):
    print("pool", shape, kernel, stride, padding, flush=True)
    rng = np.random.default_rng(7)
    x = rng.integers(-3, 4, size=shape).astype(np.float32)
    ph, pw = padding
    padded = np.pad(x, ((0, 0), (0, 0), (ph, ph), (pw, pw)), constant_values=-np.inf)
    y_ref, argmax_ref = rp.maxpool2d_native_forward(padded, kernel, stride)
    dy = rng.standard_normal(y_ref.shape).astype(np.float32)
    dx_ref = rp.maxpool2d_native_backward(dy, argmax_ref, padded.shape)[:, :, ph:ph + shape[2], pw:pw + shape[3]]
    node = mf.Variable(gpu(x))
    pool = mf.MaxPool2d_Op(node, kernel, stride, padding=padding, backend="hip_native")
    pool.forward(node.value)
    pool.grad = gpu(dy)
    pool.backward()
    np.testing.assert_array_equal(host(pool.value), y_ref)
    np.testing.assert_array_equal(host(pool._context.argmax), argmax_ref)
    np.testing.assert_array_equal(host(node.grad), dx_ref)
    # and the FP64 loops of the reference tests
    expected = naive.maxpool_forward(padded.astype(np.float64), kernel, stride)
    np.testing.assert_array_equal(host(pool.value), expected)


def test_maxpool_tie_nan_and_signed_zero():
    y, ctx = native.maxpool2d_forward(gpu(np.array([[[[1.0, 1.0], [0.0, 0.5]]]], np.float32)))
    dx = native.maxpool2d_backward(torch.ones_like(y), ctx)
    np.testing.assert_array_equal(host(dx), [[[[1.0, 0.0], [0.0, 0.0]]]])
    for position in range(4):
        z = np.arange(1, 5, dtype=np.float32).reshape(1, 1, 2, 2)
        z.reshape(-1)[position] = np.nan
        yz, _ = native.maxpool2d_forward(gpu(z))
        assert np.isnan(host(yz)).all()
    yz, cz = native.maxpool2d_forward(gpu(np.array([[[[-0.0, 0.0], [0.0, -0.0]]]], np.float32)))
    assert host(cz.argmax).item() == 0 and np.signbit(host(yz).item())


GEMM_SHAPES = ((67, 39, 45), (256, 132, 68), (300, 260, 1000), (36, 20, 3000), (16, 144, 19200), (4096, 16, 147),
               (64, 576, 2048), (1, 1, 1), (512, 512, 512), (38400, 64, 576))
LAYOUTS = ((False, False), (False, True), (True, False))


def _operands(rng, m, n, k, trans_a, trans_b):
    a = rng.standard_normal((k, m) if trans_a else (m, k)).astype(np.float32)
    b = rng.standard_normal((n, k) if trans_b else (k, n)).astype(np.float32)
    op_a = (a.T if trans_a else a).astype(np.float64)
    op_b = (b.T if trans_b else b).astype(np.float64)
    return a, b, op_a @ op_b, np.abs(op_a) @ np.abs(op_b)


@pytest.mark.parametrize("shape", GEMM_SHAPES, ids=str)
@pytest.mark.parametrize("layout", LAYOUTS, ids=("NN", "NT", "TN"))
def test_gemm_error_bound_and_determinism(shape, layout):
    """Every output within gamma_K |A||B| of the FP64 product (plus one rounding for the split-K
    reduction and the bias), and identical bits on a second run."""
    m, n, k = shape
    trans_a, trans_b = layout
    print("gemm", shape, layout, flush=True)
    rng = np.random.default_rng(2)
    a, b, exact, magnitude = _operands(rng, m, n, k, trans_a, trans_b)
    bias = rng.standard_normal(n).astype(np.float32)
    run = lambda: native.gemm(gpu(a), gpu(b), gpu(bias), trans_a=trans_a, trans_b=trans_b)
    got = run()
    assert torch.equal(got, run())
    error = np.abs(host(got).astype(np.float64) - (exact + bias))
    bound = gamma_k(k) * magnitude + EPS32 * (np.abs(exact) + np.abs(exact + bias)) + 1e-30
    assert np.all(error <= bound), f"max error {error.max():.3e}"
    # the normwise criterion of the north star: 1e-5 of max |C| (K up to 19200)
    assert_near(host(got), exact + bias, 1e-5 if k <= 4096 else 2e-5, "C")


def test_gemm_misaligned_operands_take_the_scalar_path():
    rng = np.random.default_rng(4)
    for (m, n, k), (trans_a, trans_b) in ((s, t) for s in ((300, 260, 100), (67, 39, 45)) for t in LAYOUTS):
        a, b, exact, magnitude = _operands(rng, m, n, k, trans_a, trans_b)
        da = torch.empty(a.size + 1, device="cuda")[1:].reshape(a.shape)
        db = torch.empty(b.size + 1, device="cuda")[1:].reshape(b.shape)
        da.copy_(gpu(a))
        db.copy_(gpu(b))
        got = host(native.gemm(da, db, trans_a=trans_a, trans_b=trans_b)).astype(np.float64)
        assert np.all(np.abs(got - exact) <= gamma_k(k) * magnitude + 1e-30)


def test_split_k_plan_workspace_and_accuracy():
    lib = native._library()
    assert lib.mfh_gemm_workspace(36, 20, 3000) > 0
    assert lib.mfh_gemm_workspace(4096, 4096, 1024) == 0
    tile, slices = native.gemm_plan(64, 576, 72384)
    assert slices > 1
    rng = np.random.default_rng(5)
    a, b, exact, _ = _operands(rng, 36, 20, 3000, False, False)
    split = host(native.gemm(gpu(a), gpu(b))).astype(np.float64)
    one_pass = host(native.gemm(gpu(a), gpu(b), plan=("128x128", 1))).astype(np.float64)
    assert np.abs(split - exact).max() <= np.abs(one_pass - exact).max() * 1.5 + 1e-6


def _fp64_loop(parts):
    with np.errstate(all="ignore"):
        expected = np.zeros(parts.shape[1:])
        for part in parts:
            expected = expected + part.astype(np.float64)
        return expected.astype(np.float32)


@pytest.mark.parametrize("slices", (2, 3, 8, 33, 128))
def test_split_reduce_is_the_fp64_loop_bit_for_bit(slices):
    rng = np.random.default_rng(31)
    for m, n in ((7, 13), (64, 128)):
        host_parts = rng.standard_normal((slices, m, n)).astype(np.float32) * np.exp2(
            rng.integers(-20, 20, size=(slices, m, n))).astype(np.float32)
        host_parts[0, 0, :3] = [np.inf, -0.0, np.float32(np.finfo(np.float32).tiny) / 8]
        got = host(native.split_reduce(gpu(host_parts)))
        expected = _fp64_loop(host_parts)
        nan = np.isnan(expected)
        np.testing.assert_array_equal(np.isnan(got), nan)
        np.testing.assert_array_equal(got.view(np.uint32)[~nan], expected.view(np.uint32)[~nan])


@pytest.mark.parametrize("plan", (("128x128", 5), ("64x128", 11), ("64x64", 2), ("256x64", 3)), ids=str)
def test_split_gemm_equals_fp64_reduction_of_its_chunks(plan):
    tile, requested = plan
    rng = np.random.default_rng(32)
    m, n, k = 96, 80, 2560
    a = gpu(rng.standard_normal((k, m)).astype(np.float32))
    b = gpu(rng.standard_normal((k, n)).astype(np.float32))
    bk = native.tile_catalog()[tile][-1]
    chunk = min(k, ((k + requested - 1) // requested + bk - 1) // bk * bk)
    parts = [native.gemm(a[lo:lo + chunk], b[lo:lo + chunk], trans_a=True, plan=(tile, 1)) for lo in range(0, k, chunk)]
    assert len(parts) == native._slices(k, requested, bk)
    expected = native.split_reduce(torch.stack(parts), reference=True) if len(parts) > 1 else parts[0]
    got = native.gemm(a, b, trans_a=True, plan=plan)
    assert host(got).tobytes() == host(expected).tobytes()


def _matmul_kernels():
    for variant in ("basic", "tiled", "shared", "register"):
        for tile in ((32,) if variant in ("basic", "register") else (16, 32)):
            for accumulate in native.MATMUL_ACCUMULATION:
                yield variant, tile, accumulate


def test_matmul_lecture_kernels_error_bounds():
    rng = np.random.default_rng(0)
    for m, n, k in ((8, 8, 8), (67, 39, 45), (33, 65, 300), (5, 129, 1000)):
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        exact = a.astype(np.float64) @ b.astype(np.float64)
        magnitude = np.abs(a).astype(np.float64) @ np.abs(b)
        for variant, tile, accumulate in _matmul_kernels():
            got = host(native.matmul(gpu(a), gpu(b), variant=variant, tile=tile, accumulate=accumulate)).astype(np.float64)
            error = np.abs(got - exact)
            assert np.all(error <= gamma_k(k) * magnitude + 1e-30), (variant, tile, accumulate, (m, n, k))
            if accumulate == "dot2":
                assert np.all(error <= np.spacing(np.abs(exact).astype(np.float32)) + gamma_k(k) ** 2 * magnitude)


def test_matmul_compensated_modes_beat_fp32_and_register_equals_basic():
    rng = np.random.default_rng(0)
    a = rng.standard_normal((64, 4096)).astype(np.float32)
    b = rng.standard_normal((4096, 64)).astype(np.float32)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    errors = {}
    for accumulate in native.MATMUL_ACCUMULATION:
        got = host(native.matmul(gpu(a), gpu(b), variant="shared", tile=32, accumulate=accumulate))
        errors[accumulate] = float(np.sqrt(np.mean((got - exact) ** 2)))
    assert errors["kahan"] < errors["fp32"] / 2
    assert errors["dot2"] < errors["kahan"]
    for m, n, k in ((256, 132, 68), (300, 260, 1000), (67, 39, 45)):
        a = gpu(rng.standard_normal((m, k)).astype(np.float32))
        b = gpu(rng.standard_normal((k, n)).astype(np.float32))
        for accumulate in ("kahan", "dot2"):
            got = native.matmul(a, b, variant="register", accumulate=accumulate)
            expected = native.matmul(a, b, variant="basic", accumulate=accumulate)
            assert torch.equal(got, expected), (m, n, k, accumulate)


def test_matmul_bias_epilogue():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((19, 31)).astype(np.float32)
    b = rng.standard_normal((31, 23)).astype(np.float32)
    bias = rng.standard_normal(23).astype(np.float32)
    exact = a.astype(np.float64) @ b + bias
    for variant, accumulate in (("shared", "kahan"), ("register", "fp32"), ("basic", "dot2")):
        got = host(native.matmul(gpu(a), gpu(b), gpu(bias), variant=variant, accumulate=accumulate))
        np.testing.assert_allclose(got, exact, rtol=0, atol=1e-5)
    with pytest.raises(ValueError):
        native.matmul(gpu(a), gpu(a))
    with pytest.raises(ValueError):
        native.matmul(gpu(a), gpu(b), tile=8)
    with pytest.raises(TypeError):
        native.matmul(gpu(a).double(), gpu(b))
