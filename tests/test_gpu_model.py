"""End-to-end parity on the GPU through the Variable/Graph API on the hip_native backend: Linear,
the C3 convolution + pooling configuration, the ResNet18 training step (C1 shape, both graph modes,
and C4 at batch 64), and ResNet18 inference with BN folding and the Conv+ReLU and Conv+Add+ReLU
epilogues (a small C5, and C5 at batch 256, 224 x 224).

Model-level tolerance, "no worse than the reference FP32 path": against the same pass computed in
float64 by the oracle, the GPU's error is at most the NumPy float32 path's own error plus a floor
of about one float32 ulp; a training step is compared with the GPU's ReLU and max-pool decisions
imposed on both oracle passes, after checking that the decisions that differ from FP64 are
near-ties (see test_resnet18_training_step_matches_numpy_reference).
"""

import json

import numpy as np
import pytest
import torch

import myflows_amd as mf
from myflows_amd import native
from oracle import naive, reference_path as rp
from oracle import resnet as oracle_resnet
from tests.fixtures import EPS32, assert_near, gamma_k

pytestmark = pytest.mark.gpu


def gpu(a):
    return torch.as_tensor(np.ascontiguousarray(a), device="cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def normwise(a, ref):
    return float(np.abs(np.asarray(a, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def test_linear_backends_match_fp64():
    rng = np.random.default_rng(1)
    x, w = rng.standard_normal((37, 300), dtype=np.float32), rng.standard_normal((300, 23), dtype=np.float32)
    b, g = rng.standard_normal((1, 23), dtype=np.float32), rng.standard_normal((37, 23), dtype=np.float32)
    x64, w64, b64, g64 = (a.astype(np.float64) for a in (x, w, b, g))
    exact = (x64 @ w64 + b64, g64 @ w64.T, x64.T @ g64)
    magnitude = (np.abs(x64) @ np.abs(w64) + np.abs(b64), np.abs(g64) @ np.abs(w64.T), np.abs(x64.T) @ np.abs(g64))
    db_exact = g64.sum(axis=0, keepdims=True)
    for backend in ("hip_native", "hip_native_kahan", "hip_native_dot2"):
        leaves = [mf.Variable(gpu(x)), mf.Variable(gpu(w), trainable=True), mf.Variable(gpu(b), trainable=True)]
        op = mf.Linear(*leaves, backend=backend)
        op.forward(*(leaf.value for leaf in leaves))
        op.grad = gpu(g)
        op.backward()
        got = [host(op.value)] + [host(leaf.grad) for leaf in leaves]
        for actual, ref, bound in zip(got[:3], exact, magnitude):
            assert np.all(np.abs(actual - ref) <= gamma_k(300) * bound + EPS32 * np.abs(ref) + 1e-30), backend
        assert np.all(np.abs(got[3] - db_exact) <= np.spacing(np.abs(db_exact).astype(np.float32))), backend
    leaves = [mf.Variable(gpu(x), requires_grad=False), mf.Variable(gpu(w), trainable=True),
              mf.Variable(gpu(b), trainable=True)]
    op = mf.Linear(*leaves, backend="hip_native")
    op.forward(*(leaf.value for leaf in leaves))
    op.grad = gpu(g)
    op.backward()
    assert leaves[0].grad is None  # an input without requires_grad skips the dX GEMM


@pytest.mark.parametrize("algorithm", native.CONV_ALGORITHMS)
def test_c3_convolution_and_pool_configuration(algorithm):
    """Conv 64->64 3x3/1/1 at N=32, 30x40 (forward, dX, dW, db), then MaxPool 2x2/2 forward/backward;
    the im2col matrix bit-exact (written by the forward, or by conv2d_im2col for the implicit path)."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((32, 64, 30, 40)).astype(np.float32)
    w = (rng.standard_normal((64, 64, 3, 3)) * np.sqrt(2.0 / 576)).astype(np.float32)
    b = np.zeros(64, np.float32)
    y, cols = native.conv2d_forward(gpu(x), gpu(w), gpu(b), stride=(1, 1), padding=(1, 1), algorithm=algorithm)
    y64, cols_ref = rp.conv2d_forward(x.astype(np.float64), w.astype(np.float64), b, (1, 1), (1, 1))
    if algorithm == "implicit":
        assert cols is None
        cols_check = native.conv2d_im2col(gpu(x), w.shape, stride=(1, 1), padding=(1, 1))
    else:
        cols_check = cols
    np.testing.assert_array_equal(host(cols_check), cols_ref.astype(np.float32))
    assert_near(host(y), y64, 1e-5, "y")
    pooled, ctx = native.maxpool2d_forward(y, kernel_size=(2, 2), stride=(2, 2))
    y_host = host(y)
    pooled_ref, argmax_ref = rp.maxpool2d_native_forward(y_host, (2, 2), (2, 2))
    np.testing.assert_array_equal(host(pooled), pooled_ref)
    np.testing.assert_array_equal(host(ctx.argmax), argmax_ref)
    dp = rng.standard_normal(pooled_ref.shape).astype(np.float32)
    dy = native.maxpool2d_backward(gpu(dp), ctx)
    dy_ref = rp.maxpool2d_native_backward(dp, argmax_ref, y_host.shape)
    np.testing.assert_array_equal(host(dy), dy_ref)
    dx, dw, db = native.conv2d_backward(gpu(x), gpu(w), dy, cols, stride=(1, 1), padding=(1, 1),
                                        algorithm=algorithm)
    dx64, dw64, db64 = rp.conv2d_backward(x.astype(np.float64), w.astype(np.float64), dy_ref.astype(np.float64),
                                          cols_ref, (1, 1), (1, 1))
    assert_near(host(dx), dx64, 1e-5, "dx")
    assert_near(host(dw), dw64, 1e-5, "dw")
    assert np.all(np.abs(host(db) - db64) <= np.spacing(np.abs(db64).astype(np.float32)))


def build_resnet(batch, height, width, base_width=64, seed=0, optimize=False):
    model = mf.ResNet18(output_dim=2, base_width=base_width, initializer=mf.make_initializer(seed=seed),
                        conv_backend="hip_native")
    x_np, t_np = oracle_resnet.synthetic_batch(batch, height, width, seed=seed)
    x = mf.Variable(gpu(x_np), requires_grad=False, name="images")
    t = mf.Variable(gpu(t_np), requires_grad=False, name="targets")
    out = model(x)
    loss = mf.MSELoss(out, t)
    return model, mf.Graph(loss, optimize=optimize), out, loss, x_np, t_np


def relu_output(relu):
    """A ReLU node's output; for the stem's ReLU inside a BatchNormReLUPool unit (never stored), the
    separate BN+ReLU pass over the same input, which gives the unit's bits (running statistics left
    untouched)."""
    if relu.value is not None:
        return relu.value
    bn = relu.parents[0]
    x, gamma, beta = (p.value for p in bn.parents)
    y, _, _ = mf.fused.batchnorm2d_forward(x, gamma, beta, bn.running_mean.clone(), bn.running_var.clone(),
                                           momentum=bn.momentum, eps=bn.eps, training=bn.training, relu=True)
    return y


def gpu_decisions(graph, base_width):
    """The discrete decisions of the GPU's forward in the oracle's form: each ReLU's mask (output > 0,
    the same as input > 0) by the oracle's ReLU names, and the stem max-pool's choice in each window
    (from its int32 argmax) as a one-hot mask."""
    relus = [node for node in graph.nodes if type(node) is mf.ReLU]
    names = ["stem_relu"] + [f"{spec[0]}.{part}" for spec in oracle_resnet.block_specs(base_width)
                             for part in ("relu1", "out")]
    assert len(relus) == len(names)
    decisions = {name: host(relu_output(node)) > 0 for name, node in zip(names, relus)}
    context = next(node for node in graph.nodes if isinstance(node, mf.MaxPool2d_Op))._context
    n, c, h, w = context.input_shape
    oh, ow = context.output_shape[2:]
    argmax = host(context.argmax).astype(np.int64)
    kh = (argmax // w) % h - 2 * np.arange(oh)[:, None]
    kw = argmax % w - 2 * np.arange(ow)[None, :]
    mask = np.zeros((n, c, oh * ow, 9), bool)
    np.put_along_axis(mask, (kh * 3 + kw).reshape(n, c, oh * ow)[..., None], True, axis=-1)
    decisions["pool"] = mask
    return decisions


def decision_flips(decisions, record, tie=1e-5):
    """Where the GPU's decisions differ from the FP64 pass's: (count, worst distance of a flipped
    decision from a tie, relative to the largest input of its ReLU / pool)."""
    count, worst = 0, 0.0
    for name, mask in decisions.items():
        flipped = mask != record[name]
        if not flipped.any():
            continue
        values = record[name + "/input"]
        scale = np.abs(values).max()
        if name == "pool":
            n, c = values.shape[:2]
            patches = rp.im2col(values, (3, 3), (2, 2), (0, 0)).reshape(n, -1, c, 9).transpose(0, 2, 1, 3)
            chosen_gpu = np.take_along_axis(patches, mask.argmax(-1)[..., None], -1)[..., 0]
            chosen_64 = np.take_along_axis(patches, record[name].argmax(-1)[..., None], -1)[..., 0]
            windows = flipped.any(-1)
            count += int(windows.sum())
            worst = max(worst, float(np.abs(chosen_64 - chosen_gpu)[windows].max() / scale))
        else:
            count += int(flipped.sum())
            worst = max(worst, float(np.abs(values[flipped]).max() / scale))
    return count, worst


@pytest.mark.parametrize("batch,height,width,base_width,optimize",
                         [(2, 120, 160, 64, False), (2, 120, 160, 64, True), (4, 64, 64, 16, True),
                          (64, 120, 160, 64, True)],
                         ids=("C1-bs2-120x160", "C1-bs2-120x160-fused-units", "small-fused-units",
                              "C4-bs64-120x160-fused-units"))
def test_resnet18_training_step_matches_numpy_reference(batch, height, width, base_width, optimize):
    """One training step against the oracle, "no worse than the reference FP32 path". A ReLU mask or
    max-pool choice is a discontinuity: where a pre-activation lies within rounding of zero (or two
    window values within rounding of each other), the GPU, the NumPy float32 path and FP64 may
    branch differently, and one such flip moves a gradient by a whole term rather than by rounding
    (at batch 64 the GPU and FP64 differ in 14 of ~10^8 decisions, all within 6e-7 of a tie). So
    the step is compared in two parts:
      * every decision the GPU took that differs from the FP64 pass's is a near-tie (its input within
        1e-5 of its ReLU's / pool's largest input), and the loss agrees;
      * with the GPU's decisions imposed on the FP64 and the NumPy float32 passes, the GPU's error of
        the output and of every gradient is at most the NumPy path's, plus a floor of about one
        float32 ulp (written below)."""
    print("resnet step", batch, height, width, base_width, optimize, flush=True)
    model, graph, out, loss, x_np, t_np = build_resnet(batch, height, width, base_width, optimize=optimize)
    if optimize:
        assert len(graph._bn_groups) == 17  # stem + 8 blocks x (BN+ReLU, BN+Add+ReLU)
    opt = mf.Adam(graph, learning_rate=1e-3)
    opt.one_step()
    grads = [host(p.grad) for p in model.params]
    gpu_out, gpu_loss = host(out.value), float(host(loss.value))
    decisions = gpu_decisions(graph, base_width)
    opt.update()
    updated = [host(p.value) for p in model.params]

    params32, running32 = oracle_resnet.init_params(base_width=base_width, seed=0)
    params64, running64 = oracle_resnet.as_dtype(params32, running32, np.float64)
    x64, t64 = x_np.astype(np.float64), t_np.astype(np.float64)
    record = {}
    loss64, _, out64 = oracle_resnet.forward_backward(params64, oracle_resnet.as_dtype(params32, running32,
                                                      np.float64)[1], x64, t64, record=record, backward=False)
    flips, tie = decision_flips(decisions, record)
    del record
    assert tie <= 1e-5, f"a decision differs from FP64 away from a tie ({flips} flips, worst {tie:.2e})"
    assert abs(gpu_loss - loss64) <= 1e-4 * abs(loss64)
    _, grads64, out64 = oracle_resnet.forward_backward(params64, running64, x64, t64, decisions=decisions)
    _, grads32, out32 = oracle_resnet.forward_backward(params32, running32, x_np, t_np, decisions=decisions)
    ratios = {"output": (normwise(gpu_out, out64) / max(normwise(out32, out64), 1e-30), 0, 0, 0)}
    largest = max(np.abs(g).max() for g in grads64.values())
    for name, g in zip(params32, grads):
        ref = grads64[name]
        eg, en = float(np.abs(g - ref).max()), float(np.abs(grads32[name] - ref).max())
        ratios[name] = (eg / max(en, 1e-30), eg, en, float(np.abs(ref).max()))
    print("ERROR_RATIOS", json.dumps({"case": [batch, height, width, base_width, optimize], "flips": flips,
                                      "worst_tie": tie, "largest": float(largest),
                                      "worst": sorted(ratios.items(), key=lambda kv: -kv[1][0])[:10],
                                      "median": float(np.median([v[0] for v in ratios.values()]))}), flush=True)
    assert normwise(gpu_out, out64) <= normwise(out32, out64) + 1e-7
    for name, g in zip(params32, grads):
        ref = grads64[name]
        err_gpu, err_numpy = np.abs(g - ref).max(), np.abs(grads32[name] - ref).max()
        # The floor: 1e-6 of the tensor's scale (a few float32 ulps), and 1e-7 of the largest gradient,
        # the rounding noise of a convolution bias ahead of a train-mode batch norm, whose exact
        # gradient is zero (the norm removes the channel mean), so that any float32 path computes it
        # as cancellation noise of its dy terms.
        assert err_gpu <= err_numpy + 1e-6 * np.abs(ref).max() + 1e-7 * largest, (name, err_gpu, err_numpy)
    # The reference's Adam step applied to the GPU's gradients reproduces the GPU update bit for bit.
    for name, p_new, g in zip(params32, updated, grads):
        p = params32[name].copy()
        rp.adam_update(p, g, np.zeros_like(p), np.zeros_like(p), lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, step=1)
        np.testing.assert_array_equal(p_new, p, err_msg=name)


def test_fused_units_reproduce_the_unfused_graph_bit_for_bit():
    """Graph(optimize=True) runs BN+ReLU and BN+Add+ReLU as single units with the same float32
    operations as the separate BN, Add and ReLU nodes, so both graphs give the same bits."""
    runs = []
    for optimize in (False, True):
        model, graph, out, loss, _, _ = build_resnet(2, 64, 64, base_width=16, optimize=optimize)
        graph.forward()
        graph.backward()
        runs.append([host(out.value)] + [host(p.grad) for p in model.params])
    for a, b in zip(*runs):
        np.testing.assert_array_equal(a, b)


def test_resnet18_two_steps_are_deterministic():
    runs = []
    for _ in range(2):
        model, graph, _, _, _, _ = build_resnet(2, 64, 64, base_width=16)
        opt = mf.Adam(graph, learning_rate=1e-3)
        for _ in range(2):
            opt.one_step()
            opt.update()
        runs.append([host(p.value) for p in model.params])
    for a, b in zip(*runs):
        np.testing.assert_array_equal(a, b)


def test_weight_gradient_stream_gives_the_single_stream_gradients_bit_for_bit(monkeypatch):
    """Graph.backward with the convolutions' dW products on the weight-gradient stream and
    Graph.forward with the downsample shortcuts on the side stream (the defaults) against the same
    passes on one stream: the same bits for every output, gradient and updated parameter over two
    Adam steps at batch 8, and the stream is left joined and idle."""
    from myflows_amd import native, streams

    forks, side_launches = [], []
    original = streams.WeightGradSession.fork
    original_launch = native.launch_stream

    def counting(self):
        forks.append(1)
        return original(self)

    def counting_launch(handle):
        side_launches.append(handle)
        return original_launch(handle)

    monkeypatch.setattr(streams.WeightGradSession, "fork", counting)
    monkeypatch.setattr(native, "launch_stream", counting_launch)
    runs = []
    for overlap in (False, True):
        forks.clear()
        side_launches.clear()
        model, graph, _, _, _, _ = build_resnet(8, 64, 80, base_width=16, optimize=True)
        graph.overlap_weight_grads = graph.overlap_branches = overlap
        opt = mf.Adam(graph, learning_rate=1e-3)
        grads, outputs = [], []
        for _ in range(2):
            opt.one_step()
            outputs.append(host(graph.target_node.value))
            grads.append([host(p.grad) for p in model.params])
            opt.update()
        runs.append((grads, [host(p.value) for p in model.params], len(forks), len(side_launches), outputs))
        assert streams.active() is None
    # ResNet18's 20 convolutions but the stem (no dX: its dW stays on the current stream), two passes
    assert runs[0][2] == 0 and runs[1][2] == 2 * 19
    assert runs[0][3] == 0 and runs[1][3] == 2 * 3 * 2  # three downsample conv + BN shortcuts, two passes
    for a, b in zip(runs[0][4], runs[1][4]):
        np.testing.assert_array_equal(a, b)
    for step_a, step_b in zip(runs[0][0], runs[1][0]):
        for a, b in zip(step_a, step_b):
            np.testing.assert_array_equal(a, b)
    for a, b in zip(runs[0][1], runs[1][1]):
        np.testing.assert_array_equal(a, b)


def test_shared_weight_on_two_branches_accumulates():
    rng = np.random.default_rng(9)
    x_np = rng.standard_normal((2, 3, 10, 12)).astype(np.float32)
    w_np = rng.standard_normal((4, 3, 3, 3)).astype(np.float32)
    x = mf.Variable(gpu(x_np), requires_grad=False)
    w = mf.Variable(gpu(w_np), trainable=True)
    a = mf.Conv2D_Op(x, w, stride=1, padding=1, backend="hip_native")
    b = mf.Conv2D_Op(x, w, stride=2, padding=0, backend="hip_native")
    t1 = mf.Variable(torch.zeros((2, 4, 10, 12), device="cuda"), requires_grad=False)
    t2 = mf.Variable(torch.zeros((2, 4, 4, 5), device="cuda"), requires_grad=False)
    graph = mf.Graph(mf.Add(mf.MSELoss(a, t1), mf.MSELoss(b, t2)))
    graph.forward()
    graph.backward()
    x64, w64 = x_np.astype(np.float64), w_np.astype(np.float64)
    ya, yb = naive.conv_forward(x64, w64, (1, 1), (1, 1)), naive.conv_forward(x64, w64, (2, 2), (0, 0))
    _, gwa = naive.conv_backward(x64, w64, 2 * ya / ya.size, (1, 1), (1, 1))
    _, gwb = naive.conv_backward(x64, w64, 2 * yb / yb.size, (2, 2), (0, 0))
    assert_near(host(w.grad), gwa + gwb, 1e-5, "shared dW")


def test_resnet18_inference_with_bn_folding_and_conv_relu_epilogue():
    """A small C5: eval-mode BN with random running statistics, folded into the convolutions, the
    stem and conv1 ReLUs fused into their epilogues by a second pass; the output against the
    oracle's eval-mode forward in float64."""
    batch, size, width = 4, 64, 16
    model = mf.ResNet18(output_dim=2, base_width=width, initializer=mf.make_initializer(seed=0),
                        conv_backend="hip_native")
    params32, running32 = oracle_resnet.init_params(base_width=width, seed=0)
    rng = np.random.default_rng(5)
    bns = [model.stem_bn] + [bn for block in model.blocks()
                             for bn in (block.bn1, block.bn2, *((block.downsample_bn,) if block.downsample else ()))]
    assert len(bns) == len(running32)
    for bn, name in zip(bns, running32):
        mean = rng.normal(0, 0.1, bn.num_features).astype(np.float32)
        var = rng.uniform(0.5, 1.5, bn.num_features).astype(np.float32)
        bn.running_mean.copy_(gpu(mean))
        bn.running_var.copy_(gpu(var))
        running32[name] = (mean, var)
    model.eval()
    x_np, t_np = oracle_resnet.synthetic_batch(batch, size, size, seed=0)
    out = model(mf.Variable(gpu(x_np), requires_grad=False))
    root, stats = mf.apply_graph_optimizations(out, mode="inference", fold_constants=False)
    assert stats["bn_folds"] == 20 and stats["conv_add_act_fusions"] == 8  # conv2 + shortcut + ReLU
    graph = mf.Graph(root, optimize=True)
    assert graph._opt_stats["conv_act_fusions"] == 9  # stem + conv1 of each block
    graph.forward()
    got = host(graph.target_node.value)
    params64, running64 = oracle_resnet.as_dtype(params32, running32, np.float64)
    _, _, out64 = oracle_resnet.forward_backward(params64, running64, x_np.astype(np.float64),
                                                 t_np.astype(np.float64), training=False)
    _, _, out32 = oracle_resnet.forward_backward(params32, {k: (m.copy(), v.copy()) for k, (m, v) in running32.items()},
                                                 x_np, t_np, training=False)
    print("ERROR_RATIOS", json.dumps({"case": "small C5", "output": normwise(got, out64) / normwise(out32, out64)}))
    assert normwise(got, out64) <= normwise(out32, out64) + 1e-7


def _c5_model(seed=0):
    """ResNet18 in eval mode with config 5's running statistics (var ~ U(0.5, 1.5), mean ~ N(0, 0.1),
    drawn after the input from the same seeded stream, as bench.py does) and the oracle's copy."""
    model = mf.ResNet18(output_dim=2, initializer=mf.make_initializer(seed=seed), conv_backend="hip_native")
    params32, running32 = oracle_resnet.init_params(seed=seed)
    rng = np.random.default_rng(seed)
    x_np = rng.standard_normal((256, 3, 224, 224)).astype(np.float32)
    bns = [model.stem_bn] + [bn for block in model.blocks()
                             for bn in (block.bn1, block.bn2, *((block.downsample_bn,) if block.downsample else ()))]
    for bn, name in zip(bns, running32):
        mean = rng.normal(0, 0.1, bn.num_features).astype(np.float32)
        var = rng.uniform(0.5, 1.5, bn.num_features).astype(np.float32)
        bn.running_mean.copy_(gpu(mean))
        bn.running_var.copy_(gpu(var))
        running32[name] = (mean, var)
    model.eval()
    return model, params32, running32, x_np


def test_config5_inference_at_batch_256_and_224x224():
    """Config 5 at its stated size: the folded, fused bs256 224 x 224 pass (the measured bs256 plans,
    the Conv+ReLU and Conv+Add+ReLU epilogues). Eval-mode outputs are per image, so images 0, 85,
    170 and 255 are checked against the oracle's eval forward of those images alone (FP64), within
    the NumPy float32 path's own error (a forward pass: a ReLU that flips at a near-tie moves the
    output only by the near-zero value it gates)."""
    print("config 5 full size", flush=True)
    model, params32, running32, x_np = _c5_model()
    out = model(mf.Variable(gpu(x_np), requires_grad=False))
    root, stats = mf.apply_graph_optimizations(out, mode="inference", fold_constants=False)
    assert stats["bn_folds"] == 20 and stats["conv_add_act_fusions"] == 8
    graph = mf.Graph(root, optimize=True)
    graph.forward()
    got = host(graph.target_node.value)
    assert got.shape == (256, 2) and np.isfinite(got).all()
    picks = [0, 85, 170, 255]
    sample, target = x_np[picks], np.zeros((len(picks), 2), np.float32)
    params64, running64 = oracle_resnet.as_dtype(params32, running32, np.float64)
    _, _, out64 = oracle_resnet.forward_backward(params64, running64, sample.astype(np.float64),
                                                 target.astype(np.float64), training=False, backward=False)
    _, _, out32 = oracle_resnet.forward_backward(params32, running32, sample, target, training=False, backward=False)
    print("ERROR_RATIOS", json.dumps({"case": "C5 bs256 224", "output": normwise(got[picks], out64) /
                                      normwise(out32, out64)}), flush=True)
    assert normwise(got[picks], out64) <= normwise(out32, out64) + 1e-7


def test_conv_add_relu_epilogue_equals_separate_add_and_relu_bit_for_bit():
    """The inference graph with ReLU(conv2 + shortcut) in the GEMM epilogue against the same folded
    graph with Add and ReLU as separate nodes: one float32 addition and one ReLU per element in both,
    so the outputs agree bit for bit (ResNet18 at base width 16, all four stages)."""
    outputs = []
    for fuse in (True, False):
        model = mf.ResNet18(output_dim=2, base_width=16, initializer=mf.make_initializer(seed=3),
                            conv_backend="hip_native")
        rng = np.random.default_rng(9)
        for bn in [model.stem_bn] + [bn for block in model.blocks() for bn in
                                     (block.bn1, block.bn2, *((block.downsample_bn,) if block.downsample else ()))]:
            bn.running_mean.copy_(gpu(rng.normal(0, 0.1, bn.num_features).astype(np.float32)))
            bn.running_var.copy_(gpu(rng.uniform(0.5, 1.5, bn.num_features).astype(np.float32)))
        model.eval()
        x = mf.Variable(gpu(np.random.default_rng(1).standard_normal((3, 3, 48, 40)).astype(np.float32)),
                        requires_grad=False)
        root, stats = mf.apply_graph_optimizations(model(x), mode="inference", fold_constants=False,
                                                   fuse_activations=fuse)
        assert stats["conv_add_act_fusions"] == (8 if fuse else 0)
        graph = mf.Graph(root, optimize=True)
        adds = [n for n in graph.nodes if isinstance(n, mf.Conv2D_AddReLU_Op)]
        assert len(adds) == (8 if fuse else 0)
        graph.forward()
        graph.forward()  # a second pass reads the kernel orders batched by the Graph
        outputs.append(host(graph.target_node.value))
    assert np.array_equal(outputs[0], outputs[1])


@pytest.mark.parametrize("kind", ("channel_vector", "broadcast_plane", "residual_first", "float64"))
def test_conv_add_relu_node_falls_back_to_separate_operations_for_other_residuals(kind):
    """ReLU(Add(conv, r)) rewritten into one node must give what the separate Conv2D, Add and ReLU
    nodes give whatever r is: a per-channel vector (Add's 1-D bias form), a (1, C, H, W) tensor that
    broadcasts over the batch, the residual as the Add's first operand, and a float64 residual
    (the Add promotes, then the ReLU operator refuses the float64 sum: both graphs raise the same
    TypeError)."""
    rng = np.random.default_rng(13)
    x_np = rng.standard_normal((2, 8, 10, 12)).astype(np.float32)
    residual_np = {"channel_vector": rng.standard_normal(16), "broadcast_plane": rng.standard_normal((1, 16, 10, 12)),
                   "residual_first": rng.standard_normal((2, 16, 10, 12)),
                   "float64": rng.standard_normal((2, 16, 10, 12))}[kind]
    residual_np = residual_np.astype(np.float64 if kind == "float64" else np.float32)
    results = []
    for fuse in (True, False):
        x = mf.Variable(gpu(x_np), requires_grad=False)
        r = mf.Variable(gpu(residual_np), requires_grad=False)
        conv = mf.Conv2D(8, 16, 3, padding=1, fuse_activation=False, initializer=mf.make_initializer(seed=4),
                         backend="hip_native")
        c = conv(x)
        root = mf.ReLU(mf.Add(r, c) if kind == "residual_first" else mf.Add(c, r))
        if fuse:
            root, count = mf.fusion.fuse_conv_add_relu(root)
            assert count == 1 and type(root) is mf.Conv2D_AddReLU_Op
            assert root.residual_first == (kind == "residual_first")
        graph = mf.Graph(root)
        if kind == "float64":
            with pytest.raises(TypeError, match="float32"):
                graph.forward()
            continue
        graph.forward()
        results.append(host(graph.target_node.value))
    if kind != "float64":
        np.testing.assert_array_equal(results[0], results[1])


def test_batched_kernel_orders_and_in_place_dx_reproduce_the_per_call_path(monkeypatch):
    """The Graph reorders every convolution kernel of a pass in one launch and adds dX into an
    existing input gradient in place; turning both off (each convolution reorders its own kernel,
    dX goes through a separate add) gives the same bits."""
    from myflows_amd import graph as graph_module, ops_conv

    runs = []
    for batched in (True, False):
        if not batched:
            monkeypatch.setattr(graph_module, "_prepare_weight_orders", lambda units, phase: ())
            monkeypatch.setattr(ops_conv.Conv2D_Op, "_grad_target", staticmethod(lambda node, like: None))
        model, graph, out, _, _, _ = build_resnet(2, 64, 64, base_width=32, optimize=True)
        graph.forward()
        graph.backward()
        runs.append([host(out.value)] + [host(p.grad) for p in model.params])
    for a, b in zip(*runs):
        np.testing.assert_array_equal(a, b)


def _torch_resnet18_tv(model, P, x, dropout_mask):
    """torchvision's resnet18 structure in float64 on the host (torch.nn.functional), with P(variable)
    giving each model parameter's float64 leaf: ImageNet input normalisation, bias-free
    convolutions, training-mode batch norm, the padded stem pool, dropout by the given mask, then
    the Linear head."""
    import torch.nn.functional as F
    mean = torch.tensor([0.485, 0.456, 0.406], dtype=torch.float64).reshape(1, 3, 1, 1)
    std = torch.tensor([0.229, 0.224, 0.225], dtype=torch.float64).reshape(1, 3, 1, 1)

    def conv(layer, v, stride, padding):
        return F.conv2d(v, P(layer.kernel), stride=stride, padding=padding)

    def bn(layer, v):
        return F.batch_norm(v, None, None, P(layer.gamma), P(layer.beta), training=True, eps=layer.eps)

    v = (x - mean) / std
    v = F.relu(bn(model.stem_bn, conv(model.stem_conv, v, 2, 3)))
    v = F.max_pool2d(v, 3, 2, padding=1)
    for block in model.blocks():
        stride = block.conv1.stride
        out = F.relu(bn(block.bn1, conv(block.conv1, v, stride, 1)))
        out = bn(block.bn2, conv(block.conv2, out, 1, 1))
        short = v if block.downsample is None else bn(block.downsample_bn, conv(block.downsample_conv, v, stride, 0))
        v = F.relu(out + short)
    features = v.mean(dim=(2, 3)) * dropout_mask
    return features @ P(model.fc_W) + P(model.fc_b)


def test_torchvision_compat_resnet18_step_against_torch_fp64():
    """ResNet18(compat="torchvision", input_norm="imagenet", dropout=0.5) at batch 4, 3x64x64: the
    loss, the output and every parameter gradient of one forward + backward on the GPU against the
    same network in float64 (torch.nn.functional on the host, the dropout mask the seed draws),
    normwise within 1e-4 (float32 arithmetic through 18 layers)."""
    print("torchvision-compat resnet18 step", flush=True)
    model = mf.ResNet18(output_dim=2, compat="torchvision", input_norm="imagenet", dropout=0.5, dropout_seed=5,
                        initializer=mf.make_initializer(seed=3), conv_backend="hip_native")
    rng = np.random.default_rng(4)
    x_np = rng.random((4, 3, 64, 64)).astype(np.float32)
    t_np = rng.uniform(-1, 1, (4, 2)).astype(np.float32)
    x = mf.Variable(gpu(x_np), requires_grad=False, name="images")
    out = model(x)
    loss = mf.MSELoss(out, mf.Variable(gpu(t_np), requires_grad=False))
    graph = mf.Graph(loss, optimize=True)
    graph.forward()
    graph.backward()
    mask = torch.as_tensor((np.random.default_rng(5).random((4, 512)) < 0.5).astype(np.float64) / 0.5)
    params = list(model.params)
    leaves = {id(p): p.value.detach().double().cpu().requires_grad_(True) for p in params}
    ref_out = _torch_resnet18_tv(model, lambda v: leaves[id(v)], torch.as_tensor(x_np, dtype=torch.float64), mask)
    ref_loss = ((ref_out - torch.as_tensor(t_np, dtype=torch.float64)) ** 2).mean()
    ref_loss.backward()
    assert normwise(host(out.value), ref_out.detach().numpy()) < 1e-4
    assert normwise(host(loss.value), ref_loss.detach().numpy()) < 1e-4
    for p in params:
        assert normwise(host(p.grad), leaves[id(p)].grad.numpy()) < 1e-3, p.name
