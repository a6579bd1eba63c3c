"""ResNet18 on the hip_native backend, restating ``layers/resnet.py:32-360`` (``compat="myflows"``).

``ResNet18(conv_backend="hip_native")`` routes every convolution, the stem max-pool and (unlike the
reference, whose fc uses the auto backend, ``layers/resnet.py:228,328``) the fc Linear through
libmfhip. Parameters are drawn in the reference's order: stem conv, then per block conv1, conv2,
downsample conv, then fc.
"""

from __future__ import annotations

import weakref

import torch

from .activation import ReLU
from .basic import Add, Linear
from .batchnorm import BatchNorm2d_Op, GlobalAvgPool2d_Op
from .convolution import MaxPool2d_Op, _backend_name
from .core import Variable
from .device import torch_device
from .initializers import make_initializer
from .layers import Conv2D, Layer


class BatchNorm2d(Layer):
    def __init__(self, num_features, momentum=0.1, eps=1e-5, name=None, dtype=None, unbiased_running_var=False):
        super().__init__(name=name)
        self.num_features = int(num_features)
        self.momentum, self.eps = float(momentum), float(eps)
        self.unbiased_running_var = bool(unbiased_running_var)
        self.training, self.frozen = True, False
        device = torch_device()
        self.gamma = Variable(torch.ones(self.num_features, device=device), trainable=True,
                              name=f"{name}_gamma" if name else "gamma")
        self.beta = Variable(torch.zeros(self.num_features, device=device), trainable=True,
                             name=f"{name}_beta" if name else "beta")
        self.params = [self.gamma, self.beta]
        self.running_mean = torch.zeros(self.num_features, device=device)
        self.running_var = torch.ones(self.num_features, device=device)
        self._ops = weakref.WeakSet()

    def forward(self, input_node):
        op = BatchNorm2d_Op(input_node, self.gamma, self.beta, self.running_mean, self.running_var,
                            momentum=self.momentum, eps=self.eps, training=self.training,
                            unbiased_running_var=self.unbiased_running_var)
        self._ops.add(op)
        return op

    def train(self, mode=True):
        self.training = bool(mode) and not self.frozen
        for op in self._ops:
            op.training = self.training

    def eval(self):
        self.train(False)


class GlobalAvgPool2d(Layer):
    def forward(self, input_node):
        return GlobalAvgPool2d_Op(input_node)


def _conv3x3(in_c, out_c, stride=1, initializer=None, backend="auto", bias=True):
    return Conv2D(in_c, out_c, kernel_size=3, stride=stride, padding=1, fuse_activation=False,
                  initializer=initializer, backend=backend, bias=bias)


def _conv1x1(in_c, out_c, stride=1, initializer=None, backend="auto", bias=True):
    return Conv2D(in_c, out_c, kernel_size=1, stride=stride, padding=0, fuse_activation=False,
                  initializer=initializer, backend=backend, bias=bias)


class BasicBlock(Layer):
    """out = ReLU(BN(conv3x3(ReLU(BN(conv3x3(x))))) + shortcut(x)); 1x1 conv + BN projection when the
    stride or the width changes (layers/resnet.py:135-188)."""

    expansion = 1

    def __init__(self, in_channels, out_channels, stride=1, name=None, initializer=None, conv_backend="auto"):
        super().__init__(name=name)
        self.conv1 = _conv3x3(in_channels, out_channels, stride, initializer, conv_backend)
        self.bn1 = BatchNorm2d(out_channels)
        self.conv2 = _conv3x3(out_channels, out_channels, 1, initializer, conv_backend)
        self.bn2 = BatchNorm2d(out_channels)
        self.downsample = None
        if stride != 1 or in_channels != out_channels:
            self.downsample_conv = _conv1x1(in_channels, out_channels, stride, initializer, conv_backend)
            self.downsample_bn = BatchNorm2d(out_channels)
            self.downsample = (self.downsample_conv, self.downsample_bn)
        self.params = self.conv1.params + self.bn1.params + self.conv2.params + self.bn2.params
        self.sub_layers = [self.conv1, self.bn1, self.conv2, self.bn2]
        if self.downsample is not None:
            self.params += self.downsample_conv.params + self.downsample_bn.params
            self.sub_layers += [self.downsample_conv, self.downsample_bn]

    def forward(self, input_node):
        out = ReLU(self.bn1(self.conv1(input_node)))
        out = self.bn2(self.conv2(out))
        identity = input_node
        if self.downsample is not None:
            identity = self.downsample_bn(self.downsample_conv(input_node))
        return ReLU(Add(out, identity))


class ResNet18(Layer):
    def __init__(self, in_channels=3, output_dim=2, stem="imagenet", base_width=64, name=None, initializer=None,
                 conv_backend="auto", linear_backend=None):
        super().__init__(name=name)
        if stem not in ("imagenet", "cifar"):
            raise ValueError("stem must be 'imagenet' or 'cifar'")
        self.conv_backend = _backend_name(conv_backend)
        self.linear_backend = linear_backend or ("hip_native" if self.conv_backend == "hip_native" else "auto")
        self.stem_type = stem
        self.output_dim = int(output_dim)
        widths = [base_width, base_width * 2, base_width * 4, base_width * 8]
        if stem == "imagenet":
            self.stem_conv = Conv2D(in_channels, widths[0], kernel_size=7, stride=2, padding=3, fuse_activation=False,
                                    initializer=initializer, backend=self.conv_backend)
        else:
            self.stem_conv = Conv2D(in_channels, widths[0], kernel_size=3, stride=1, padding=1, fuse_activation=False,
                                    initializer=initializer, backend=self.conv_backend)
        self.stem_bn = BatchNorm2d(widths[0])
        self.layer1 = self._make_stage(widths[0], widths[0], 1, initializer)
        self.layer2 = self._make_stage(widths[0], widths[1], 2, initializer)
        self.layer3 = self._make_stage(widths[1], widths[2], 2, initializer)
        self.layer4 = self._make_stage(widths[2], widths[3], 2, initializer)
        self.avgpool = GlobalAvgPool2d()
        init = make_initializer(initializer)
        device = torch_device()
        self.fc_W = Variable(torch.as_tensor(init((widths[3], self.output_dim)), dtype=torch.float32, device=device),
                             trainable=True, name="fc_W")
        self.fc_b = Variable(torch.zeros(self.output_dim, device=device), trainable=True, name="fc_b")
        self.params = list(self.stem_conv.params) + list(self.stem_bn.params)
        self.sub_layers = [self.stem_conv, self.stem_bn]
        for stage in (self.layer1, self.layer2, self.layer3, self.layer4):
            for block in stage:
                self.params += block.params
                self.sub_layers.append(block)
                self.sub_layers.extend(block.sub_layers)
        self.params += [self.fc_W, self.fc_b]
        self.widths = widths

    def _make_stage(self, in_c, out_c, stride, initializer):
        return [BasicBlock(in_c, out_c, stride, initializer=initializer, conv_backend=self.conv_backend),
                BasicBlock(out_c, out_c, 1, initializer=initializer, conv_backend=self.conv_backend)]

    def spatial_features(self, input_node):
        x = ReLU(self.stem_bn(self.stem_conv(input_node)))
        if self.stem_type == "imagenet":
            x = MaxPool2d_Op(x, kernel_size=3, stride=2, backend=self.conv_backend, padding=0)
        for stage in (self.layer1, self.layer2, self.layer3, self.layer4):
            for block in stage:
                x = block(x)
        return x

    def forward(self, input_node):
        features = self.avgpool(self.spatial_features(input_node))
        return Linear(features, self.fc_W, self.fc_b, backend=self.linear_backend)

    def train(self, mode=True):
        for layer in self.sub_layers:
            if hasattr(layer, "train"):
                layer.train(mode)

    def eval(self):
        self.train(False)
