"""Graph optimisations used by ``Graph(optimize=True)``.

Restates the two passes of ``core/graph_opt.py`` that the ResNet18 inference configuration needs:
``fuse_conv_activation_ops`` (ReLU(Conv2D_Op) -> Conv2D_ReLU_Op, :295-349) and
``fold_bn_into_conv`` (eval-mode BN folded into the preceding convolution, :114-190), plus the
``batchnorm_activation_groups`` hook (:231-257), which this package leaves empty.
"""

from __future__ import annotations

import torch

from .activation import ReLU
from .batchnorm import BatchNorm2d_Op
from .convolution import Conv2D_Op, Conv2D_ReLU_Op
from .core import Graph, Variable


def _replace(old, new):
    """Point every child of ``old`` at ``new``."""
    for child in list(old.children):
        child.parents = [new if p is old else p for p in child.parents]
        new.children.append(child)
    old.children = []


def _detach(node):
    for p in node.parents:
        if node in p.children:
            p.children.remove(node)


def fuse_conv_activation_ops(root):
    """ReLU whose only parent is a plain Conv2D_Op used only by that ReLU -> Conv2D_ReLU_Op."""
    fused = 0
    for node in Graph._build_topo_sort(root):
        if type(node) is not ReLU:
            continue
        conv = node.parents[0]
        if type(conv) is not Conv2D_Op or len(conv.children) != 1:
            continue
        parents = conv.parents
        _detach(conv)
        new = Conv2D_ReLU_Op(parents[0], parents[1], stride=conv.stride, padding=conv.padding,
                             bias=parents[2] if len(parents) > 2 else None, backend=conv.backend,
                             recompute_im2col=conv.recompute_im2col)
        _detach(node)
        _replace(node, new)
        if node is root:
            root = new
        fused += 1
    return root, fused


def fold_bn_into_conv(root):
    """Eval-mode BN(Conv2D_Op(x, W, b)) -> Conv2D_Op(x, W * s, (b - mean) * s + beta) with
    s = gamma / sqrt(var + eps), computed in FP64 and rounded once."""
    folded = 0
    for node in Graph._build_topo_sort(root):
        if not isinstance(node, BatchNorm2d_Op) or node.training:
            continue
        conv = node.parents[0]
        if type(conv) is not Conv2D_Op or len(conv.children) != 1:
            continue
        w = conv.parents[1].value.double()
        b = conv.parents[2].value.double() if len(conv.parents) > 2 else torch.zeros(w.shape[0], dtype=torch.float64,
                                                                                      device=w.device)
        gamma, beta = node.parents[1].value.double(), node.parents[2].value.double()
        scale = gamma / torch.sqrt(node.running_var.double() + node.eps)
        kernel = Variable((w * scale.reshape(-1, 1, 1, 1)).float(), name=f"{conv.parents[1].name}_folded")
        bias = Variable(((b - node.running_mean.double()) * scale + beta).float(), name="folded_bias")
        kernel.requires_grad = bias.requires_grad = False
        x = conv.parents[0]
        _detach(conv)
        new = Conv2D_Op(x, kernel, stride=conv.stride, padding=conv.padding, bias=bias, backend=conv.backend)
        _detach(node)
        _replace(node, new)
        if node is root:
            root = new
        folded += 1
    return root, folded


def apply_graph_optimizations(root, *, mode="train", fold_constants=False, fuse_linear=True, fuse_activations=True):
    stats = {"conv_activation_fusions": 0, "bn_folds": 0}
    if fuse_activations:
        root, stats["conv_activation_fusions"] = fuse_conv_activation_ops(root)
    if mode == "inference":
        root, stats["bn_folds"] = fold_bn_into_conv(root)
    return root, stats


def batchnorm_activation_groups(nodes):
    return {}
