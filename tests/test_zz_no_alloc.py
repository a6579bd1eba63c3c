"""mfh_gemm_noalloc: the GEMM entry point whose split-K partials live in the library's fixed device
scratch instead of a caller's workspace. Called through the C ABI, its results must be bitwise
those of mfh_gemm with the same engine code and a workspace of the plan's size, on consecutive calls
(the second smaller than the first, so stale scratch contents would show), and a plan whose
partials exceed the scratch must be refused before anything runs.
"""


import numpy as np
import pytest
import torch

from myflows_amd import native
from tests.fixtures import EPS32, gamma_k

pytestmark = pytest.mark.gpu

SCRATCH_FLOATS = 8388608  # MFH_GEMM_NOALLOC_SCRATCH_FLOATS of include/mfhip.h


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _operands(rng, m, n, k, trans_a, trans_b):
    a = rng.standard_normal((k, m) if trans_a else (m, k)).astype(np.float32)
    b = rng.standard_normal((n, k) if trans_b else (k, n)).astype(np.float32)
    return a, b


def _run(lib, symbol, engine, trans_a, trans_b, a, b, bias, m, n, k, workspace=None):
    """C = op(a) op(b) [+ bias] through `symbol`; returns (status, C on the device)."""
    c = torch.full((m, n), float("nan"), device="cuda")
    lda, ldb = int(a.shape[1]), int(b.shape[1])
    common = (engine, int(trans_a), int(trans_b), a.data_ptr(), b.data_ptr(), 0 if bias is None else bias.data_ptr(),
              c.data_ptr(), m, n, k, lda, ldb, n)
    if symbol == "mfh_gemm":
        floats = 0 if workspace is None else workspace.numel()
        status = lib.mfh_gemm(*common, 0 if workspace is None else workspace.data_ptr(), floats, _stream())
    else:
        status = lib.mfh_gemm_noalloc(*common, _stream())
    torch.cuda.synchronize()
    return status, c


def _workspace_floats(lib, engine, m, n, k):
    if engine == 1:
        return lib.mfh_gemm_workspace(m, n, k)
    requested, bk = native._explicit_split(engine)
    slices = native._slices(k, requested, bk)
    return slices * m * n if slices > 1 else 0


# (m, n, k, layout, engine): the dW form of config 2 under the automatic plan (127 K slices), then a
# smaller NN product with an explicit 4-way split, then a split product with a bias.
CALLS = ((576, 64, 38400, "TN", None), (300, 260, 1000, "NN", ("64x64", 4)), (36, 20, 3000, "NT", None))
LAYOUTS = {"NN": (False, False), "NT": (False, True), "TN": (True, False)}


def test_noalloc_gemm_repeats_mfh_gemm_bit_for_bit_on_consecutive_calls():
    lib = native._library()
    rng = np.random.default_rng(71)
    for index, (m, n, k, layout, plan) in enumerate(CALLS):
        print("mfh_gemm_noalloc", (m, n, k), layout, plan, flush=True)
        trans_a, trans_b = LAYOUTS[layout]
        engine = 1 if plan is None else native._plan_code(*plan)
        floats = _workspace_floats(lib, engine, m, n, k)
        assert 0 < floats <= SCRATCH_FLOATS, "each call must split K through the scratch"
        a_host, b_host = _operands(rng, m, n, k, trans_a, trans_b)
        a, b = torch.as_tensor(a_host, device="cuda"), torch.as_tensor(b_host, device="cuda")
        bias = torch.as_tensor(rng.standard_normal(n).astype(np.float32), device="cuda") if index == 2 else None
        workspace = torch.empty(floats, device="cuda")
        status, expected = _run(lib, "mfh_gemm", engine, trans_a, trans_b, a, b, bias, m, n, k, workspace)
        assert status == 0, lib.mfh_last_error()
        status, got = _run(lib, "mfh_gemm_noalloc", engine, trans_a, trans_b, a, b, bias, m, n, k)
        assert status == 0, lib.mfh_last_error()
        assert got.cpu().numpy().tobytes() == expected.cpu().numpy().tobytes()
        # and both are the product: within gamma_K |A||B| (plus the bias rounding) of the FP64 product
        left = (a_host.T if trans_a else a_host).astype(np.float64)
        right = (b_host.T if trans_b else b_host).astype(np.float64)
        exact = left @ right + (0.0 if bias is None else bias.cpu().numpy().astype(np.float64))
        bound = gamma_k(k) * (np.abs(left) @ np.abs(right)) + 2 * EPS32 * np.abs(exact) + 1e-30
        assert np.all(np.abs(got.cpu().numpy().astype(np.float64) - exact) <= bound)


def test_noalloc_gemm_without_a_split_needs_no_scratch():
    lib = native._library()
    rng = np.random.default_rng(72)
    m, n, k = 256, 132, 68
    a_host, b_host = _operands(rng, m, n, k, False, False)
    a, b = torch.as_tensor(a_host, device="cuda"), torch.as_tensor(b_host, device="cuda")
    engine = native._plan_code("64x64", 1)
    status, expected = _run(lib, "mfh_gemm", engine, False, False, a, b, None, m, n, k)
    assert status == 0, lib.mfh_last_error()
    status, got = _run(lib, "mfh_gemm_noalloc", engine, False, False, a, b, None, m, n, k)
    assert status == 0, lib.mfh_last_error()
    assert torch.equal(got, expected)


def test_noalloc_gemm_refuses_a_plan_beyond_the_scratch():
    lib = native._library()
    m = n = k = 4096
    engine = native._plan_code("128x128", 2)  # 2 x 4096 x 4096 floats of partials: 4x the scratch
    assert _workspace_floats(lib, engine, m, n, k) > SCRATCH_FLOATS
    a = torch.zeros((m, k), device="cuda")
    b = torch.zeros((k, n), device="cuda")
    status, c = _run(lib, "mfh_gemm_noalloc", engine, False, False, a, b, None, m, n, k)
    assert status == 2
    reason = lib.mfh_last_error().decode()
    assert "static scratch" in reason and str(SCRATCH_FLOATS) in reason
    assert torch.isnan(c).all(), "a refused call must not launch anything"
