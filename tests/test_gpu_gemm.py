"""GEMM engine and teaching matmul parity on the GPU.

The MFMA engine's accumulation order differs from a sequential FMA loop (and so does the
one-wave-per-row kernel that the automatic plan takes for at most 8 output columns), so its results
are checked against the FP64 product: every output within the worst-case bound gamma_K |A||B| (plus one
rounding for the split-K reduction and the bias), the normwise criterion of 1e-5 of max|C|, and
identical bits run to run. The split-K reduction is bit-exact against the FP64 loop. The teaching
kernels keep the reference's properties (bounds, Dot2 within one ulp, the compensated modes more
accurate than FP32, register-blocked == one-thread-per-output bit for bit).
"""

import numpy as np
import pytest
import torch

from myflows_amd import native
from tests.fixtures import EPS32, assert_near, gamma_k

pytestmark = pytest.mark.gpu

SHAPES = ((67, 39, 45), (256, 132, 68), (300, 260, 1000), (36, 20, 3000), (16, 144, 19200), (4096, 16, 147),
          (64, 576, 2048), (1, 1, 1), (512, 512, 512), (38400, 64, 576), (576, 64, 38400),
          # up to 8 output columns: the one-wave-per-row kernel of the automatic plan
          (64, 2, 512), (512, 2, 64), (4096, 8, 147), (7, 5, 3000), (300, 1, 1000))
LAYOUTS = {"NN": (False, False), "NT": (False, True), "TN": (True, False)}


def gpu(a):
    return torch.as_tensor(np.ascontiguousarray(a), device="cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def operands(rng, m, n, k, trans_a, trans_b):
    """A, B as stored, and the FP64 product op(A) op(B) with its magnitude |op(A)| |op(B)|."""
    a = rng.standard_normal((k, m) if trans_a else (m, k)).astype(np.float32)
    b = rng.standard_normal((n, k) if trans_b else (k, n)).astype(np.float32)
    left = (a.T if trans_a else a).astype(np.float64)
    right = (b.T if trans_b else b).astype(np.float64)
    return a, b, left @ right, np.abs(left) @ np.abs(right)


@pytest.mark.parametrize("shape", SHAPES, ids=str)
@pytest.mark.parametrize("layout", LAYOUTS)
def test_engine_error_bound_and_determinism(shape, layout):
    m, n, k = shape
    trans_a, trans_b = LAYOUTS[layout]
    print("gemm", shape, layout, flush=True)
    rng = np.random.default_rng(2)
    a, b, exact, magnitude = operands(rng, m, n, k, trans_a, trans_b)
    bias = rng.standard_normal(n).astype(np.float32)
    launch = lambda: native.gemm(gpu(a), gpu(b), gpu(bias), trans_a=trans_a, trans_b=trans_b)
    got = launch()
    assert torch.equal(got, launch())
    error = np.abs(host(got).astype(np.float64) - (exact + bias))
    bound = gamma_k(k) * magnitude + EPS32 * (np.abs(exact) + np.abs(exact + bias)) + 1e-30
    assert np.all(error <= bound), f"max error {error.max():.3e}"
    assert_near(host(got), exact + bias, 1e-5 if k <= 4096 else 2e-5, "C")


@pytest.mark.parametrize("size,layout", [(1024, "NN"), (2048, "NN"), (4096, "NN"), (4096, "NT"), (4096, "TN")],
                         ids=lambda v: str(v))
def test_config2_square_products_at_their_stated_sizes(size, layout):
    """Config 2's square GEMMs at full size (the 4096^3 NN product is the roofline figure's, on the
    256 x 128 tile), with config 2's inputs (A then B, N(0, 1), seed 0): every output within
    gamma_K |A||B| of the FP64 product, 1e-5 of max|C| normwise, the same bits on a second launch."""
    trans_a, trans_b = LAYOUTS[layout]
    print("config 2 gemm", size, layout, native.gemm_plan(size, size, size), flush=True)
    rng = np.random.default_rng(0)
    a, b, exact, magnitude = operands(rng, size, size, size, trans_a, trans_b)
    da, db = gpu(a), gpu(b)
    got = native.gemm(da, db, trans_a=trans_a, trans_b=trans_b)
    assert torch.equal(got, native.gemm(da, db, trans_a=trans_a, trans_b=trans_b))
    result = host(got).astype(np.float64)
    error = np.abs(result - exact)
    assert np.all(error <= gamma_k(size) * magnitude + EPS32 * np.abs(exact) + 1e-30), f"max error {error.max():.3e}"
    assert_near(result, exact, 1e-5, "C")


@pytest.mark.parametrize("shape", ((1024, 1024, 1024), (256, 256, 4096), (38400, 64, 576)), ids=str)
def test_engine_is_no_less_accurate_than_one_fma_chain_per_output(shape):
    """The reference's FP32 GEMM (its register engine) adds each output's K products in one FMA
    chain; the teaching kernel "basic" with fp32 accumulation does exactly that. The MFMA engine's
    normwise error against the FP64 product stays within 1.25x that chain's on the same inputs
    (config 2's inputs, A then B ~ N(0, 1), seed 0)."""
    m, n, k = shape
    rng = np.random.default_rng(0)
    a, b, exact, _ = operands(rng, m, n, k, False, False)
    da, db = gpu(a), gpu(b)
    engine = host(native.gemm(da, db)).astype(np.float64)
    chain = host(native.matmul(da, db, variant="basic", accumulate="fp32")).astype(np.float64)
    scale = np.abs(exact).max()
    err_engine, err_chain = np.abs(engine - exact).max() / scale, np.abs(chain - exact).max() / scale
    print("engine / one chain", shape, err_engine, err_chain, err_engine / err_chain, flush=True)
    assert err_engine <= 1.25 * err_chain


def test_misaligned_operands_take_the_scalar_loads():
    rng = np.random.default_rng(4)
    for (m, n, k) in ((300, 260, 100), (67, 39, 45)):
        for trans_a, trans_b in LAYOUTS.values():
            a, b, exact, magnitude = operands(rng, m, n, k, trans_a, trans_b)
            da = torch.empty(a.size + 1, device="cuda")[1:].view(a.shape)  # 4-byte, not 16-byte, aligned
            db = torch.empty(b.size + 1, device="cuda")[1:].view(b.shape)
            da.copy_(gpu(a))
            db.copy_(gpu(b))
            got = host(native.gemm(da, db, trans_a=trans_a, trans_b=trans_b)).astype(np.float64)
            assert np.all(np.abs(got - exact) <= gamma_k(k) * magnitude + 1e-30)


def test_split_k_plan_workspace_and_accuracy():
    lib = native._library()
    assert lib.mfh_gemm_workspace(36, 20, 3000) > 0
    assert lib.mfh_gemm_workspace(4096, 4096, 1024) == 0
    _, slices = native.gemm_plan(64, 576, 72384)
    assert slices > 1
    rng = np.random.default_rng(5)
    a, b, exact, _ = operands(rng, 36, 20, 3000, False, False)
    split = host(native.gemm(gpu(a), gpu(b))).astype(np.float64)
    single = host(native.gemm(gpu(a), gpu(b), plan=("128x128", 1))).astype(np.float64)
    assert np.abs(split - exact).max() <= np.abs(single - exact).max() * 1.5 + 1e-6


def fp64_slice_sum(parts):
    with np.errstate(all="ignore"):
        total = np.zeros(parts.shape[1:])
        for part in parts:
            total = total + part.astype(np.float64)
        return total.astype(np.float32)


@pytest.mark.parametrize("slices", (2, 3, 8, 33, 128))
def test_split_reduce_is_the_fp64_loop_bit_for_bit(slices):
    rng = np.random.default_rng(31)
    for m, n in ((7, 13), (64, 128)):
        parts = rng.standard_normal((slices, m, n)).astype(np.float32)
        parts *= np.exp2(rng.integers(-20, 20, size=parts.shape)).astype(np.float32)  # wide exponent range
        parts[0, 0, :3] = [np.inf, -0.0, np.float32(np.finfo(np.float32).tiny) / 8]
        got = host(native.split_reduce(gpu(parts)))
        expected = fp64_slice_sum(parts)
        nan = np.isnan(expected)
        np.testing.assert_array_equal(np.isnan(got), nan)
        np.testing.assert_array_equal(got.view(np.uint32)[~nan], expected.view(np.uint32)[~nan])


@pytest.mark.parametrize("plan", (("128x128", 5), ("64x128", 11), ("64x64", 2), ("256x64", 3), ("64x64k2", 4),
                                  ("256x256", 3)), ids=str)
def test_split_gemm_is_the_fp64_reduction_of_its_chunks(plan):
    tile, requested = plan
    rng = np.random.default_rng(32)
    m, n, k = 96, 80, 2560
    a = gpu(rng.standard_normal((k, m)).astype(np.float32))
    b = gpu(rng.standard_normal((k, n)).astype(np.float32))
    bk = native.tile_catalog()[tile][-1]
    per_slice = -(-k // requested)
    chunk = min(k, -(-per_slice // bk) * bk)
    chunks = [native.gemm(a[lo:lo + chunk], b[lo:lo + chunk], trans_a=True, plan=(tile, 1)) for lo in range(0, k, chunk)]
    assert len(chunks) == native._slices(k, requested, bk)
    expected = native.split_reduce(torch.stack(chunks), reference=True) if len(chunks) > 1 else chunks[0]
    got = native.gemm(a, b, trans_a=True, plan=plan)
    assert host(got).tobytes() == host(expected).tobytes()


def test_reference_plan_codes_run_on_the_tile_of_the_same_role():
    """A named plan of the reference (its 128x64 tile, 4 slices) runs on this library's 256x64 tile with
    the same split, bit for bit the extended code of that tile; the raw codes give the same bits."""
    rng = np.random.default_rng(41)
    a, b = gpu(rng.standard_normal((300, 700)).astype(np.float32)), gpu(rng.standard_normal((700, 60)).astype(np.float32))
    named = native.gemm(a, b, plan=("128x64", 4))
    assert torch.equal(named, native.gemm(a, b, plan=("256x64", 4)))
    lib, out = native._library(), torch.empty_like(named)
    workspace = torch.empty(4 * 300 * 60, device="cuda")
    for code in (16 + 32 + 3, 1024 + 128 + 3):
        native._raise_for(lib.mfh_gemm(code, 0, 0, a.data_ptr(), b.data_ptr(), 0, out.data_ptr(), 300, 60, 700, 700, 60,
                                       60, workspace.data_ptr(), workspace.numel(), torch.cuda.current_stream().cuda_stream), lib)
        assert torch.equal(out, named)
    assert [lib.mfh_gemm_tile_stages(i) for i in range(lib.mfh_gemm_tile_count())] == [2] * lib.mfh_gemm_tile_count()
    assert lib.mfh_gemm_tile_stages(lib.mfh_gemm_tile_count()) == -1


def teaching_kernels():
    for variant in ("basic", "tiled", "shared", "register"):
        for tile in ((32,) if variant in ("basic", "register") else (16, 32)):
            for accumulate in native.MATMUL_ACCUMULATION:
                yield variant, tile, accumulate


def test_teaching_kernels_error_bounds():
    rng = np.random.default_rng(0)
    for m, n, k in ((8, 8, 8), (67, 39, 45), (33, 65, 300), (5, 129, 1000)):
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        exact = a.astype(np.float64) @ b.astype(np.float64)
        magnitude = np.abs(a).astype(np.float64) @ np.abs(b)
        for variant, tile, accumulate in teaching_kernels():
            got = host(native.matmul(gpu(a), gpu(b), variant=variant, tile=tile, accumulate=accumulate))
            error = np.abs(got.astype(np.float64) - exact)
            assert np.all(error <= gamma_k(k) * magnitude + 1e-30), (variant, tile, accumulate, (m, n, k))
            if accumulate == "dot2":  # as if computed in twice the precision and rounded once
                assert np.all(error <= np.spacing(np.abs(exact).astype(np.float32)) + gamma_k(k) ** 2 * magnitude)


def test_compensated_modes_beat_fp32_and_register_blocking_repeats_the_basic_kernel():
    rng = np.random.default_rng(0)
    a = rng.standard_normal((64, 4096)).astype(np.float32)
    b = rng.standard_normal((4096, 64)).astype(np.float32)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    rms = {}
    for accumulate in native.MATMUL_ACCUMULATION:
        got = host(native.matmul(gpu(a), gpu(b), variant="shared", tile=32, accumulate=accumulate))
        rms[accumulate] = float(np.sqrt(np.mean((got - exact) ** 2)))
    assert rms["kahan"] < rms["fp32"] / 2 and rms["dot2"] < rms["kahan"]
    for m, n, k in ((256, 132, 68), (300, 260, 1000), (67, 39, 45)):
        a = gpu(rng.standard_normal((m, k)).astype(np.float32))
        b = gpu(rng.standard_normal((k, n)).astype(np.float32))
        for accumulate in ("kahan", "dot2"):
            register = native.matmul(a, b, variant="register", accumulate=accumulate)
            basic = native.matmul(a, b, variant="basic", accumulate=accumulate)
            assert torch.equal(register, basic), (m, n, k, accumulate)


def test_teaching_kernel_bias_and_argument_checks():
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


def test_large_products_take_the_256x256_tile():
    """The automatic plan of a 4096^3 product is the 256x256 tile (one workgroup per CU), whose
    32-deep stages give the 16-deep tiles' bits in every layout."""
    assert native.gemm_plan(4096, 4096, 4096) == ("256x256", 1)
    rng = np.random.default_rng(12)
    for layout, (trans_a, trans_b) in LAYOUTS.items():
        a, b, _, _ = operands(rng, 520, 300, 1000, trans_a, trans_b)
        a, b = gpu(a), gpu(b)
        wide = native.gemm(a, b, trans_a=trans_a, trans_b=trans_b, plan=("256x256", 1))
        assert torch.equal(wide, native.gemm(a, b, trans_a=trans_a, trans_b=trans_b, plan=("256x128", 1))), layout


@pytest.mark.parametrize("layout", LAYOUTS)
def test_every_unsplit_tile_adds_in_the_same_order(layout):
    """All one-group tiles use the same k mapping (the two terms of an MFMA 8 apart in sub-stages of
    16 k, the 256x256 tile's 32-deep stages included), so one-pass products are bit-identical
    whatever the tile (and the XCD tile order); K = 1000 ends inside a stage of every tile."""
    trans_a, trans_b = LAYOUTS[layout]
    rng = np.random.default_rng(6)
    a, b, _, _ = operands(rng, 300, 260, 1000, trans_a, trans_b)
    tiles = [tile for tile in native.tile_catalog() if native.tile_groups(tile) == 1]
    assert len(tiles) == 9 and "256x256" in tiles
    results = [native.gemm(gpu(a), gpu(b), trans_a=trans_a, trans_b=trans_b, plan=(tile, 1)) for tile in tiles]
    for other in results[1:]:
        assert torch.equal(results[0], other)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("m,n,k", ((300, 260, 1000), (64, 64, 16), (130, 70, 37), (1024, 1024, 1024)), ids=str)
def test_k_grouped_tile_is_the_group_order_sum_of_one_group_products(layout, m, n, k):
    """The 64x64k2 tile splits each workgroup's stages into two runs (the first ceil(stages / 2)
    stages, then the rest) and adds the runs' FP32 sums in order: bit for bit the one-group tile's
    products over the two K ranges added in float32 (with a bias, added after the sum)."""
    trans_a, trans_b = LAYOUTS[layout]
    rng = np.random.default_rng(8)
    a, b, _, _ = operands(rng, m, n, k, trans_a, trans_b)
    a, b = gpu(a), gpu(b)
    bias = gpu(rng.standard_normal(n).astype(np.float32))
    bk = native.tile_catalog()["64x64k2"][-1]
    assert native.tile_groups("64x64k2") == 2
    split = -(-(-(-k // bk)) // 2) * bk  # the first run: ceil(stages / 2) stages
    cut = lambda x, lo, hi, k_first: x[lo:hi] if k_first else x[:, lo:hi]
    parts = [native.gemm(cut(a, lo, hi, trans_a).contiguous(), cut(b, lo, hi, not trans_b).contiguous(),
                         trans_a=trans_a, trans_b=trans_b, plan=("64x64", 1)) for lo, hi in ((0, split), (split, k))
             if lo < hi]
    expected = parts[0] + parts[1] if len(parts) == 2 else parts[0]
    got = native.gemm(a, b, trans_a=trans_a, trans_b=trans_b, plan=("64x64k2", 1))
    assert torch.equal(got, expected)
    got = native.gemm(a, b, bias, trans_a=trans_a, trans_b=trans_b, plan=("64x64k2", 1))
    assert torch.equal(got, expected + bias)
