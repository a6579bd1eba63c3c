"""The C ABI and the Python boundary without a GPU.

* the built library exports every symbol include/mfhip.h declares, and native.py declares each with
  the header's number of parameters;
* the one struct of the ABI (mfh_adam_tensor) has the same layout in C (gcc on the header) and in
  ctypes;
* host-side argument checks raise before any device call; operators reject CPU tensors;
* seeded model weights, the graph executor and the graph rewrites, on CPU tensors.
"""

import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

import myflows_amd as mf
from myflows_amd import native
from myflows_amd.graph import GradientOp

HEADER = Path(__file__).resolve().parents[1] / "include" / "mfhip.h"


def header_prototypes():
    """{symbol: parameter count} of every MFH_API function in the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    found = {}
    for name, params in re.findall(r"MFH_API\s+[\w\s\*]+?\b(mfh_\w+)\s*\(([^)]*)\)", text):
        params = params.strip()
        found[name] = 0 if params in ("", "void") else params.count(",") + 1
    return found


def test_library_exports_every_declared_symbol_with_its_arity():
    lib = native.load_library()
    prototypes = header_prototypes()
    assert sorted(prototypes) == sorted(native.EXPORTS)
    for name, count in prototypes.items():
        assert hasattr(lib, name), name
        assert len(native._SIGNATURES[name][1]) == count, name


def test_adam_table_layout_matches_the_header(tmp_path):
    probe = tmp_path / "probe.c"
    probe.write_text(
        '#include <stddef.h>\n#include <stdio.h>\n#include "mfhip.h"\n'
        "int main(void) { printf(\"%zu %zu %zu %zu\\n\", sizeof(mfh_adam_tensor), offsetof(mfh_adam_tensor, size),"
        " offsetof(mfh_adam_tensor, lr), offsetof(mfh_adam_tensor, bias_correction2)); return 0; }\n")
    subprocess.run(["gcc", "-I", str(HEADER.parent), str(probe), "-o", str(tmp_path / "probe")], check=True)
    c_layout = [int(v) for v in subprocess.run([str(tmp_path / "probe")], capture_output=True, text=True,
                                               check=True).stdout.split()]
    t = native.AdamTensor
    assert c_layout == [ctypes.sizeof(t), t.size.offset, t.lr.offset, t.bias_correction2.offset]


def test_tile_catalogue_and_plan_codes():
    catalogue = native.tile_catalog()
    assert catalogue["128x128"][0] == 0
    assert all(entry[-1] == (32 if name == "256x256" else 16) for name, entry in catalogue.items())
    # The reference's code arithmetic (native.py:298-309 there): its named tiles take
    # 16 + index * 32 + slices - 1 (run here on the tile of the same role), catalogue tiles
    # 1024 + index * 128 + slices - 1.
    assert native._plan_code("128x128", 1) == 16 and native._plan_code("128x64", 4) == 16 + 32 + 3
    assert native._plan_code("32x256", 32) == 16 + 4 * 32 + 31
    assert native._plan_code("256x64", 3) == 1024 + 128 + 2
    assert native._plan_code("128x128", 33) == 1024 + 32
    assert native._explicit_tile(16 + 32 + 3) == ("256x64", 4)    # the reference's 128x64, N <= 64
    assert native._explicit_tile(16 + 2 * 32) == ("128x32", 1)    # 256x32, N <= 32
    assert native._explicit_tile(16 + 3 * 32 + 7) == ("64x128", 8)
    assert native._explicit_tile(16 + 4 * 32) == ("32x128", 1)    # 32x256, M <= 32
    assert native._explicit_tile(1024 + 6 * 128 + 1) == ("256x128", 2)
    assert all(native.NAMED_TILE_OF[name] in catalogue for name in native.NAMED_TILES)
    for bad in (("7x7", 1), ("128x128", 0), ("128x128", native.EXTENDED_PLAN_SLICES + 1), ("128x128", 2.0),
                ("128x64", 33)):
        with pytest.raises(ValueError):
            native._plan_code(*bad)
    with pytest.raises(ValueError):
        native._explicit_tile(1024 + len(catalogue) * 128)
    # requested slices -> slices made, with BK-aligned chunks
    assert [native._slices(k, r, 16) for k, r in ((3000, 5), (100, 7), (10, 4), (4096, 1))] == [5, 7, 1, 1]


def test_argument_checks_raise_before_any_device_call():
    cpu = torch.zeros((1, 1, 4, 4))
    with pytest.raises(TypeError):
        native.conv2d_forward(cpu, torch.zeros((1, 1, 3, 3)))
    with pytest.raises(ValueError, match="engine"):
        native.conv2d_forward(cpu, torch.zeros((1, 1, 3, 3)), engine="tf32")
    with pytest.raises(ValueError, match="int32"):
        native._within_int32(columns=2**31)
    with pytest.raises(ValueError, match="alpha > 0"):
        native._activation_code("leaky_relu", 0.0)
    with pytest.raises(ValueError):
        native._activation_code("gelu", 0.0)
    with pytest.raises(ValueError, match="input channels"):
        native.ConvGeometry.of((1, 2, 4, 4), (1, 3, 3, 3), (1, 1), (0, 0))
    with pytest.raises(ValueError, match="empty"):
        native.ConvGeometry.of((1, 1, 2, 2), (1, 1, 3, 3), (1, 1), (0, 0))
    with pytest.raises(ValueError):
        native.ConvGeometry.of((1, 1, 8, 8), (1, 1, 3, 3), (0, 1), (0, 0))
    g = native.ConvGeometry.of((2, 3, 7, 9), (4, 3, 3, 3), (2, 2), (1, 1))
    assert (g.oh, g.ow, g.m, g.k) == (4, 5, 40, 27) and len(g.c_args()) == 13
    with pytest.raises(ValueError):
        native.matmul(cpu.reshape(4, 4), cpu.reshape(4, 4), variant="cublas")
    with pytest.raises(ValueError):
        native.gemm(cpu.reshape(4, 4), cpu.reshape(4, 4), trans_a=True, trans_b=True)
    with pytest.raises(TypeError):
        mf.fused.relu_forward(cpu)


def test_operators_reject_cpu_arrays_and_unsupported_options():
    mf.set_device("cpu")
    try:
        x = mf.Variable(torch.zeros((1, 1, 5, 5)), requires_grad=False)
        conv = mf.Conv2D(1, 2, kernel_size=3, backend="hip_native")(x)
        with pytest.raises(ValueError, match="incompatible with device=cpu"):
            conv.forward(*(p.value for p in conv.parents))
        pool = mf.MaxPool2d(2, 2, backend="hip_native")(x)
        with pytest.raises(ValueError, match="incompatible with device=cpu"):
            pool.forward(x.value)
        with pytest.raises(ValueError, match="GPU tensor"):
            mf.ReLU(x).forward(x.value)
        for options in ({"groups": 2}, {"dilation": 2}):
            with pytest.raises(ValueError):
                mf.Conv2D_Op(x, mf.Variable(torch.zeros((2, 1, 3, 3))), backend="hip_native", **options)
        with pytest.raises(ValueError):
            mf.Conv2D(1, 2, backend="cudnn")
        with pytest.raises(ValueError):
            mf.Dense(3, 2, backend="tf32")
    finally:
        if torch.cuda.is_available():
            mf.set_device("cuda")


def test_seeded_resnet_weights_match_the_oracle_draw_order():
    """ResNet18(initializer=make_initializer(seed=0)) holds exactly the oracle model's weights, in the
    reference's parameter order."""
    from oracle import resnet as oracle_resnet

    mf.set_device("cpu")
    try:
        model = mf.ResNet18(output_dim=2, initializer=mf.make_initializer(seed=0), conv_backend="hip_native")
    finally:
        if torch.cuda.is_available():
            mf.set_device("cuda")
    params, _ = oracle_resnet.init_params(seed=0)
    assert len(model.params) == len(params) == 82  # stem 4, eight blocks 8 each, three shortcuts 4 each, fc 2
    assert sum(p.value.numel() for p in model.params) == 11_182_338
    for ours, expected in zip(model.params, params.values()):
        assert np.array_equal(ours.value.numpy(), expected)


class _Square(GradientOp):
    """x * x: a test-local operator, so the executor is exercised without libmfhip."""

    def forward(self, x):
        self.value = x * x

    def backward(self):
        self.parents[0].accumulate_grad(2 * self.parents[0].value * self.grad, owned=True)


def test_graph_executor_on_cpu_tensors():
    """Gradient accumulation over a leaf used three times, a requires_grad=False leaf, gradient
    release of intermediates, retain_grad, and the plan rebuilt when a leaf flag changes."""
    a = mf.Variable(torch.tensor([1.0, -2.0, 3.0]), trainable=True, name="a")
    c = mf.Variable(torch.tensor([0.5, 0.5, 0.5]), requires_grad=False, name="c")
    t = mf.Variable(torch.zeros(3), requires_grad=False, name="t")
    square = _Square(a)
    pred = mf.Add(square, mf.Add(a, mf.Add(a, c)))
    loss = mf.MSELoss(pred, t)
    graph = mf.Graph(loss)
    graph.forward()
    graph.backward()
    p = a.value ** 2 + 2 * a.value + c.value
    dpred = 2.0 * p / 3
    torch.testing.assert_close(a.grad, dpred * (2 * a.value + 2))
    assert c.grad is None and square.grad is None
    assert abs(loss.value.item() - float((p * p).mean())) < 1e-6
    graph.retain_grad(square)
    graph.forward()
    graph.backward()
    torch.testing.assert_close(square.grad, dpred)
    c.requires_grad = True  # needs a new plan; asking for it without a new forward is an error
    with pytest.raises(RuntimeError, match="run forward again"):
        graph.backward()
    graph.forward()
    graph.backward()
    torch.testing.assert_close(c.grad, dpred)


def test_graph_rewrites_on_cpu():
    """Conv+ReLU fusion, eval-mode BN folding (FP64 folded parameters, model parameters untouched),
    constant folding, and the BN(+Add)+ReLU groups of a ResNet block."""
    mf.set_device("cpu")
    try:
        x = mf.Variable(torch.zeros((1, 3, 8, 8)), requires_grad=False)
        conv = mf.Conv2D(3, 4, 3, padding=1, fuse_activation=False, initializer=mf.make_initializer(seed=1),
                         backend="hip_native")
        root, stats = mf.apply_graph_optimizations(mf.ReLU(conv(x)), fold_constants=False)
        assert type(root) is mf.Conv2D_ReLU_Op and stats["conv_act_fusions"] == 1

        bn = mf.BatchNorm2d(4)
        bn.running_mean.copy_(torch.tensor([0.1, -0.2, 0.3, 0.0]))
        bn.running_var.copy_(torch.tensor([0.5, 1.5, 1.0, 2.0]))
        bn.gamma.value.copy_(torch.tensor([1.0, 2.0, 0.5, -1.0]))
        bn.beta.value.copy_(torch.tensor([0.0, 0.1, -0.1, 0.2]))
        bn.eval()
        kernel_before = conv.kernel.value.clone()
        root, stats = mf.apply_graph_optimizations(bn(conv(x)), mode="inference", fold_constants=False)
        assert type(root) is mf.Conv2D_Op and stats["bn_folds"] == 1
        scale = bn.gamma.value.double() / torch.sqrt(bn.running_var.double() + bn.eps)
        torch.testing.assert_close(root.parents[1].value, (kernel_before.double() * scale[:, None, None, None]).float())
        torch.testing.assert_close(root.parents[2].value,
                                   ((0 - bn.running_mean.double()) * scale + bn.beta.value.double()).float())
        assert torch.equal(conv.kernel.value, kernel_before)

        k1 = mf.Variable(torch.ones(3), constant=True)
        k2 = mf.Variable(torch.full((3,), 2.0), constant=True)
        root, stats = mf.apply_graph_optimizations(mf.Add(k1, k2))
        assert stats["constant_folds"] == 1 and torch.equal(root.value, torch.full((3,), 3.0))

        block = mf.BasicBlock(4, 8, stride=2, conv_backend="hip_native")
        out = block(mf.Variable(torch.zeros((1, 4, 8, 8)), requires_grad=False))
        graph = mf.Graph(out, optimize=True)
        names = sorted(g.name for g in graph._bn_groups.values())
        assert names == ["BatchNormAddReLU", "BatchNormReLU"]

        # Inference: both BNs and the shortcut's fold, then ReLU(conv2 + shortcut) becomes one node
        # whose last parent is the shortcut; a second optimising Graph fuses conv1's ReLU.
        block = mf.BasicBlock(4, 8, stride=2, conv_backend="hip_native")
        for bn in (block.bn1, block.bn2, block.downsample_bn):
            bn.eval()
        out = block(mf.Variable(torch.zeros((1, 4, 8, 8)), requires_grad=False))
        root, stats = mf.apply_graph_optimizations(out, mode="inference", fold_constants=False)
        assert stats["bn_folds"] == 3 and stats["conv_add_act_fusions"] == 1
        assert type(root) is mf.Conv2D_AddReLU_Op and len(root.parents) == 4
        residual = root.parents[3]
        assert type(residual) is mf.Conv2D_Op and residual.children == [root] and residual.stride == (2, 2)
        graph = mf.Graph(root, optimize=True)
        assert graph._opt_stats["conv_act_fusions"] == 1
        assert sorted(type(n).__name__ for n in graph.nodes if isinstance(n, mf.Conv2D_Op)) == [
            "Conv2D_AddReLU_Op", "Conv2D_Op", "Conv2D_ReLU_Op"]
        with pytest.raises(RuntimeError, match="no backward"):
            root.backward()

        # No rewrite when the convolution or the sum has another reader, or the activation is not ReLU.
        x = mf.Variable(torch.zeros((1, 3, 8, 8)), requires_grad=False)
        shortcut = mf.Variable(torch.zeros((1, 4, 8, 8)), requires_grad=False)
        conv = mf.Conv2D(3, 4, 3, padding=1, fuse_activation=False, initializer=mf.make_initializer(seed=2),
                         backend="hip_native")
        c = conv(x)
        total = mf.Add(mf.ReLU(mf.Add(c, shortcut)), c)  # c read twice
        _, stats = mf.fusion.fuse_conv_add_relu(total)
        assert stats == 0
        s = mf.Add(conv(x), shortcut)
        root, stats = mf.fusion.fuse_conv_add_relu(mf.Add(mf.ReLU(s), s))  # the sum read twice
        assert stats == 0
        root, stats = mf.fusion.fuse_conv_add_relu(mf.LeakyReLU(mf.Add(conv(x), shortcut), alpha=0.1))
        assert stats == 0 and type(root) is mf.LeakyReLU
        root, stats = mf.fusion.fuse_conv_add_relu(mf.ReLU(mf.Add(shortcut, conv(x))))  # either operand order
        assert stats == 1 and type(root) is mf.Conv2D_AddReLU_Op and root.parents[-1] is shortcut
        assert root.residual_first  # the node keeps the Add's operand order for its unfused fallback
        root, stats = mf.fusion.fuse_conv_add_relu(mf.ReLU(mf.Add(conv(x), shortcut)))
        assert stats == 1 and not root.residual_first
    finally:
        if torch.cuda.is_available():
            mf.set_device("cuda")


def test_forward_steps_put_downsample_shortcuts_beside_the_main_path():
    """Graph._forward_steps (no device work): a BasicBlock with a downsample takes its 1x1 conv and
    BN onto the side stream right after the block input is made and joins before the fused
    BN+Add+ReLU; every unit still runs after its parents; a block without a downsample, or a
    shortcut BN with a second consumer, keeps one stream."""
    from myflows_amd import graph as G

    def steps_of(root):
        graph = mf.Graph(root, optimize=True)
        return [(u, k) for u, k in graph._plan().forward_steps if u is None or u.parents]

    def check_order(steps):
        done = set()
        for unit, _ in steps:
            if unit is None:
                continue
            for parent in unit.parents:
                producer_known = not parent.parents or parent in done
                assert producer_known, f"{unit.name} runs before its parent {parent.name}"
            done.add(getattr(unit, "output", unit))
            done.update(getattr(unit, "hidden", ()))

    mf.set_device("cpu")
    try:
        x = mf.Variable(torch.zeros((1, 4, 8, 8)), requires_grad=False)
        stem = mf.ReLU(mf.BatchNorm2d(4)(mf.Conv2D(4, 4, 3, padding=1, fuse_activation=False,
                                                   backend="hip_native")(x)))
        block = mf.BasicBlock(4, 8, stride=2, conv_backend="hip_native")
        steps = steps_of(block(stem))
        kinds = [k for _, k in steps]
        assert kinds.count(G.FORK) == 1 and kinds.count(G.JOIN) == 1 and kinds.count(G.SIDE) == 2
        fork, join = kinds.index(G.FORK), kinds.index(G.JOIN)
        side = [u for u, k in steps if k == G.SIDE]
        assert [type(u).__name__ for u in side] == ["Conv2D_Op", "BatchNorm2d_Op"]
        assert steps[fork - 1][0].name == "BatchNormReLU"  # right after the block input is made
        assert steps[join + 1][0].name == "BatchNormAddReLU"  # the fused unit that reads the shortcut
        assert all(k == G.MAIN for _, k in steps[fork + 3:join])  # the main path between them
        check_order(steps)

        plain = mf.BasicBlock(8, 8, stride=1, conv_backend="hip_native")
        steps = steps_of(plain(mf.Variable(torch.zeros((1, 8, 4, 4)), requires_grad=False)))
        assert all(k == G.MAIN for _, k in steps)

        conv = mf.Conv2D(4, 8, 1, stride=2, fuse_activation=False, backend="hip_native")
        bn = mf.BatchNorm2d(8)
        shortcut = bn(conv(stem))
        main = mf.BatchNorm2d(8)(mf.Conv2D(4, 8, 3, stride=2, padding=1, fuse_activation=False,
                                            backend="hip_native")(stem))
        out = mf.Add(mf.ReLU(mf.Add(main, shortcut)), shortcut)  # the shortcut BN has two consumers
        steps = steps_of(out)
        assert all(k == G.MAIN for _, k in steps)
    finally:
        if torch.cuda.is_available():
            mf.set_device("cuda")


def test_deferred_input_gradients_pair_a_convolution_with_the_next_batch_norm_unit_only():
    """Graph._deferred_input_grads (no device work): in a BasicBlock the second convolution's dX
    may be formed by the first BN+ReLU unit, the next backward unit and the only consumer of the
    convolution's input; the first convolution (its input also feeds the residual Add) and a
    convolution whose input is retained are not paired."""
    mf.set_device("cpu")
    try:
        x = mf.Variable(torch.zeros((1, 8, 4, 4)), requires_grad=False)
        stem = mf.ReLU(mf.BatchNorm2d(8)(mf.Conv2D(8, 8, 3, padding=1, fuse_activation=False,
                                                   backend="hip_native")(x)))
        block = mf.BasicBlock(8, 8, stride=1, conv_backend="hip_native")
        out = block(stem)
        graph = mf.Graph(out, optimize=True)
        plan = graph._plan()
        pairs = plan.deferred_dx
        assert len(pairs) == 1
        (conv, unit), = pairs.items()
        assert unit.name == "BatchNormReLU" and conv.parents[0] is unit.output
        position = [u for u, _ in plan.backward_units]
        assert position.index(unit) == position.index(conv) + 1
        assert unit.output is not stem  # the block's first unit, not the stem's (which feeds the Add too)
        graph.retain_grad(unit.output)
        assert not graph._plan().deferred_dx
    finally:
        if torch.cuda.is_available():
            mf.set_device("cuda")
