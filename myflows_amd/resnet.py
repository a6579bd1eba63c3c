"""ResNet18 on the hip_native backend (``layers/resnet.py:32-360`` of the reference). Two structures,
as there: ``compat="myflows"`` (the default: convolutions with bias, biased running variance, stem
max-pool 3x3/2 without padding) and ``compat="torchvision"`` (torchvision's resnet18 layer for
layer: convolutions without bias, running variance from the unbiased batch variance, stem max-pool
with padding 1), with an optional in-graph ImageNet input normalisation and dropout before the
head.

``ResNet18(conv_backend="hip_native")`` runs every convolution and the stem max-pool on libmfhip, and
its fc ``Linear`` on the MFMA engine too (``auto`` is that engine on the GPU; the reference's fc used
its CuPy path, ``layers/resnet.py:228,328``). BatchNorm, ReLU and Adam run on libmfhip as well.
Parameters are drawn in the reference's order: stem conv, then per block conv1, conv2, downsample
conv, then fc.
"""

from __future__ import annotations

import weakref

import torch

from .device import torch_device
from .graph import Variable
from .init import make_initializer
from .layers import Conv2D, Dropout, Layer
from .ops_basic import Add, ChannelNormalize_Op, Linear, ReLU
from .ops_conv import MaxPool2d_Op, _backend_name
from .ops_norm import BatchNorm2d_Op, GlobalAvgPool2d_Op


class BatchNorm2d(Layer):
    """Batch norm over channels with gamma = 1, beta = 0, running mean 0 and running variance 1.
    ``train()`` / ``eval()`` switch the mode of every operator this layer has built; a frozen layer
    stays in eval mode and stops training gamma and beta."""

    def __init__(self, num_features, momentum=0.1, eps=1e-5, name=None, dtype=None, unbiased_running_var=False):
        super().__init__(name=name)
        self.num_features = int(num_features)
        self.momentum, self.eps = float(momentum), float(eps)
        self.unbiased_running_var = bool(unbiased_running_var)
        self.training, self.frozen = True, False
        device = torch_device()
        prefix = f"{name}_" if name else ""
        self.gamma = Variable(torch.ones(self.num_features, device=device), trainable=True, name=prefix + "gamma")
        self.beta = Variable(torch.zeros(self.num_features, device=device), trainable=True, name=prefix + "beta")
        self.params = [self.gamma, self.beta]
        self.running_mean = torch.zeros(self.num_features, device=device)
        self.running_var = torch.ones(self.num_features, device=device)
        self._built = weakref.WeakSet()

    def forward(self, input_node):
        op = BatchNorm2d_Op(input_node, self.gamma, self.beta, self.running_mean, self.running_var,
                            momentum=self.momentum, eps=self.eps, training=self.training,
                            unbiased_running_var=self.unbiased_running_var)
        self._built.add(op)
        return op

    def train(self, mode=True):
        self.training = bool(mode) and not self.frozen
        for op in self._built:
            op.training = self.training

    def eval(self):
        self.train(False)

    def freeze(self, frozen=True):
        self.frozen = bool(frozen)
        for param in self.params:
            param.trainable = not self.frozen
        if self.frozen:
            self.train(False)


class GlobalAvgPool2d(Layer):
    def forward(self, input_node):
        return GlobalAvgPool2d_Op(input_node)


COMPAT_MODES = ("myflows", "torchvision")


def _conv(in_c, out_c, size, stride, initializer, backend, bias=True):
    return Conv2D(in_c, out_c, kernel_size=size, stride=stride, padding=size // 2, fuse_activation=False,
                  initializer=initializer, backend=backend, bias=bias)


class BasicBlock(Layer):
    """ReLU(BN(conv3x3(ReLU(BN(conv3x3(x))))) + shortcut(x)); the shortcut is a 1x1 convolution +
    BN when the stride or the width changes, the identity otherwise."""

    expansion = 1

    def __init__(self, in_channels, out_channels, stride=1, name=None, initializer=None, conv_backend="auto",
                 compat="myflows"):
        super().__init__(name=name)
        if compat not in COMPAT_MODES:
            raise ValueError(f"compat must be one of {COMPAT_MODES}")
        bias, unbiased = compat != "torchvision", compat == "torchvision"
        self.conv1 = _conv(in_channels, out_channels, 3, stride, initializer, conv_backend, bias)
        self.bn1 = BatchNorm2d(out_channels, unbiased_running_var=unbiased)
        self.conv2 = _conv(out_channels, out_channels, 3, 1, initializer, conv_backend, bias)
        self.bn2 = BatchNorm2d(out_channels, unbiased_running_var=unbiased)
        self.sub_layers = [self.conv1, self.bn1, self.conv2, self.bn2]
        self.downsample = None
        if stride != 1 or in_channels != out_channels:
            self.downsample_conv = _conv(in_channels, out_channels, 1, stride, initializer, conv_backend, bias)
            self.downsample_bn = BatchNorm2d(out_channels, unbiased_running_var=unbiased)
            self.downsample = (self.downsample_conv, self.downsample_bn)
            self.sub_layers += [self.downsample_conv, self.downsample_bn]
        self.params = [p for layer in self.sub_layers for p in layer.params]

    def forward(self, input_node):
        main = self.bn2(self.conv2(ReLU(self.bn1(self.conv1(input_node)))))
        shortcut = input_node if self.downsample is None else self.downsample_bn(self.downsample_conv(input_node))
        return ReLU(Add(main, shortcut))


class ResNet18(Layer):
    """Stem (7x7/2 conv + BN + ReLU + 3x3/2 max-pool for ``stem="imagenet"``, 3x3/1 conv + BN + ReLU
    for ``"cifar"``), four stages of two BasicBlocks (widths base_width x 1, 2, 4, 8; strides 1, 2,
    2, 2), global average pooling, dropout (when ``dropout`` > 0) and a Linear head.
    ``compat="torchvision"`` (imagenet stem, base width 64, 3 input channels) builds torchvision's
    structure; ``input_norm="imagenet"`` normalises [0, 1] RGB inputs by ImageNet's channel mean and
    std in the graph (ChannelNormalize_Op)."""

    def __init__(self, in_channels=3, output_dim=2, stem="imagenet", base_width=64, name=None, dropout=0.0,
                 initializer=None, conv_backend="auto", dropout_seed=None, compat="myflows", input_norm=None,
                 linear_backend="auto"):
        super().__init__(name=name)
        if stem not in ("imagenet", "cifar"):
            raise ValueError("stem must be 'imagenet' or 'cifar'")
        if compat not in COMPAT_MODES:
            raise ValueError(f"compat must be one of {COMPAT_MODES}")
        if compat == "torchvision" and (stem != "imagenet" or int(base_width) != 64 or in_channels != 3):
            raise ValueError("compat='torchvision' requires stem='imagenet', base_width=64 and 3 input channels")
        if input_norm not in (None, "imagenet"):
            raise ValueError("input_norm must be None or 'imagenet'")
        self.conv_backend = _backend_name(conv_backend)
        self.linear_backend = linear_backend
        self.stem_type = stem
        self.compat = compat
        self.input_norm = input_norm
        self.output_dim = int(output_dim)
        bias, unbiased = compat != "torchvision", compat == "torchvision"
        self.widths = [base_width * f for f in (1, 2, 4, 8)]
        if stem == "imagenet":
            self.stem_conv = _conv(in_channels, self.widths[0], 7, 2, initializer, self.conv_backend, bias)
        else:
            self.stem_conv = _conv(in_channels, self.widths[0], 3, 1, initializer, self.conv_backend)
        self.stem_bn = BatchNorm2d(self.widths[0], unbiased_running_var=unbiased)
        in_c = self.widths[0]
        stages = []
        for width, stride in zip(self.widths, (1, 2, 2, 2)):
            stages.append([BasicBlock(in_c, width, stride, initializer=initializer, conv_backend=self.conv_backend,
                                      compat=compat),
                           BasicBlock(width, width, 1, initializer=initializer, conv_backend=self.conv_backend,
                                      compat=compat)])
            in_c = width
        self.layer1, self.layer2, self.layer3, self.layer4 = stages
        self.avgpool = GlobalAvgPool2d()
        self.dropout = (Dropout(float(dropout), seed=dropout_seed, name="resnet_dropout")
                        if float(dropout or 0.0) > 0.0 else None)
        device = torch_device()
        draw = make_initializer(initializer)
        self.fc_W = Variable(torch.as_tensor(draw((self.widths[3], self.output_dim)), dtype=torch.float32,
                                             device=device), trainable=True, name="fc_W")
        self.fc_b = Variable(torch.zeros(self.output_dim, device=device), trainable=True, name="fc_b")
        self.sub_layers = [self.stem_conv, self.stem_bn]
        for block in self.blocks():
            self.sub_layers += [block, *block.sub_layers]
        self.params = [*self.stem_conv.params, *self.stem_bn.params]
        for block in self.blocks():
            self.params += block.params
        self.params += [self.fc_W, self.fc_b]
        if self.dropout is not None:
            self.sub_layers.append(self.dropout)

    def blocks(self):
        return [*self.layer1, *self.layer2, *self.layer3, *self.layer4]

    def spatial_features(self, input_node):
        if self.input_norm == "imagenet":
            input_node = ChannelNormalize_Op(input_node)
        x = ReLU(self.stem_bn(self.stem_conv(input_node)))
        if self.stem_type == "imagenet":
            # torchvision's stem pool pads by 1 (56 x 56 from a 224 x 224 input); the default does not.
            x = MaxPool2d_Op(x, kernel_size=3, stride=2, backend=self.conv_backend,
                             padding=1 if self.compat == "torchvision" else 0)
        for block in self.blocks():
            x = block(x)
        return x

    def forward(self, input_node):
        features = self.avgpool(self.spatial_features(input_node))
        if self.dropout is not None:
            features = self.dropout(features)
        return Linear(features, self.fc_W, self.fc_b, backend=self.linear_backend)

    def train(self, mode=True):
        for layer in self.sub_layers:
            if hasattr(layer, "train"):
                layer.train(mode)

    def eval(self):
        self.train(False)
