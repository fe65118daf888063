"""Modules over the lazy tensor graph (tensor.py), as crates/oxide-torch/src/nn.rs and the
MobileNetV4-Conv-S model (crates/oxide-torch-models/src/models/mobilenet_v4.rs:84-195) define
them: parameters live on the device (torch tensors), ``forward`` builds the lazy graph, and a
``tensor.training_program`` of the loss trains them (forward, reverse mode, AdamW).

This is the general path: any model built from these ops compiles to one training program.
``MobileNetV4ConvSmall`` here is assembled from the generic modules; liboxide_hip's native
``oxh_mnv4_create`` / ``oxh_trainer_create`` trace the same network through the same graph
builders.
"""

from __future__ import annotations

import numpy as np

import oxide_hip as ox
import tensor as tn

BN_MOMENTUM, BN_EPSILON = 0.1, 1e-5


def _device():
    import torch

    return torch.device("cuda:0")


class Parameter:
    """nn.rs:35-80: a trainable device tensor with a stable identity."""

    def __init__(self, values):
        import torch

        self.data = torch.as_tensor(np.ascontiguousarray(values, np.float32)).to(_device())
        self.shape = tuple(self.data.shape)

    def data_ptr(self) -> int:
        return self.data.data_ptr()

    def tensor(self) -> tn.Tensor:
        return tn.parameter_tensor(self)

    def host(self) -> np.ndarray:
        return self.data.detach().cpu().numpy()


class Module:
    """Module + Trainable + ModuleMode (nn.rs:10-32,83-104)."""

    def __call__(self, x: tn.Tensor) -> tn.Tensor:
        return self.forward(x)

    def children(self) -> list:
        return []

    def own_parameters(self) -> list:
        return []

    def parameters(self) -> list:
        """visit_parameters order: a module's own, then its children in order."""
        out = list(self.own_parameters())
        for c in self.children():
            out.extend(c.parameters())
        return out

    def batch_norms(self) -> list:
        out = [self] if isinstance(self, BatchNorm2d) else []
        for c in self.children():
            out.extend(c.batch_norms())
        return out

    def set_training(self, training: bool) -> None:
        for c in self.children():
            c.set_training(training)


class Conv2d(Module):
    """nn.rs:236-297: deterministic variance-scaled weight (nn.rs:657-674), zero bias,
    padding kernel / 2."""

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, groups=1):
        if kernel_size == 0 or groups == 0 or in_channels % groups or out_channels % groups:
            raise ox.OxideError(ox.INVALID_SHAPE,
                                "invalid Conv2d channel, group, or kernel configuration")
        shape = [out_channels, in_channels // groups, kernel_size, kernel_size]
        self.weight = Parameter(ox.initialized_weights(shape, in_channels // groups)
                                .reshape(shape))
        self.bias = Parameter(np.zeros(out_channels, np.float32))
        self.stride, self.padding, self.groups = stride, kernel_size // 2, groups

    def own_parameters(self):
        return [self.weight, self.bias]

    def forward(self, x):
        return x.conv2d(self.weight.tensor(), self.bias.tensor(), self.stride, self.padding,
                        self.groups)


class BatchNorm2d(Module):
    """nn.rs:107-233: gamma 1, beta 0, running mean 0 / variance 1, momentum 0.1, eps 1e-5."""

    def __init__(self, channels):
        if channels == 0:
            raise ox.OxideError(ox.INVALID_SHAPE, "BatchNorm2d channels must be non-zero")
        self.weight = Parameter(np.ones(channels, np.float32))
        self.bias = Parameter(np.zeros(channels, np.float32))
        self.state = tn.BatchNormState(channels)
        self.training, self.momentum, self.epsilon = True, BN_MOMENTUM, BN_EPSILON

    def own_parameters(self):
        return [self.weight, self.bias]

    def set_training(self, training):
        self.training = bool(training)

    def forward(self, x):
        return x.batch_norm2d(self.weight.tensor(), self.bias.tensor(), self.state,
                              self.training, self.momentum, self.epsilon)


class ConvNormAct(Module):
    """nn.rs:349-397: conv, BatchNorm2d, optional ReLU."""

    def __init__(self, in_channels, out_channels, kernel_size, stride, groups, activation):
        self.conv = Conv2d(in_channels, out_channels, kernel_size, stride, groups)
        self.norm = BatchNorm2d(out_channels)
        self.activation = activation

    def children(self):
        return [self.conv, self.norm]

    def forward(self, x):
        y = self.norm(self.conv(x))
        return y.relu() if self.activation else y


class UniversalInvertedBottleneck(Module):
    """nn.rs:425-515: optional start depthwise, 1x1 expand, optional middle depthwise carrying
    the stride, 1x1 project (no ReLU), residual when stride 1 and channels match."""

    def __init__(self, in_c, out_c, expanded, start_dw, middle_dw, stride):
        if stride > 1 and not middle_dw:
            raise ox.OxideError(ox.INVALID_SHAPE,
                                "a strided UIB requires a middle depthwise convolution")
        self.layers = []
        if start_dw:
            self.layers.append(ConvNormAct(in_c, in_c, start_dw, 1, in_c, True))
        self.layers.append(ConvNormAct(in_c, expanded, 1, 1, 1, True))
        if middle_dw:
            self.layers.append(ConvNormAct(expanded, expanded, middle_dw, stride, expanded, True))
        self.layers.append(ConvNormAct(expanded, out_c, 1, 1, 1, False))
        self.residual = stride == 1 and in_c == out_c

    def children(self):
        return list(self.layers)

    def forward(self, x):
        y = x
        for layer in self.layers:
            y = layer(y)
        return y.add(x) if self.residual else y


class FusedInvertedBottleneck(Module):
    """nn.rs:565-655: full k x k expand with ReLU, 1x1 project."""

    def __init__(self, in_c, out_c, expanded, kernel, stride):
        self.expand = ConvNormAct(in_c, expanded, kernel, stride, 1, True)
        self.project = ConvNormAct(expanded, out_c, 1, 1, 1, False)
        self.residual = stride == 1 and in_c == out_c

    def children(self):
        return [self.expand, self.project]

    def forward(self, x):
        y = self.project(self.expand(x))
        return y.add(x) if self.residual else y


class GlobalAveragePool(Module):
    def forward(self, x):
        return x.global_avg_pool2d()


class MobileNetV4ConvSmall(Module):
    """mobilenet_v4.rs:111-195 (supplement table 11): conv stem, two fused IBs, twelve UIBs, a
    1x1 conv to 960, global average pool, 1x1 conv to 1280, classifier conv, reshape to
    [N, classes]."""

    # mobilenet_v4.rs:140-153: in, out, expanded, start DW, middle DW (0 = none), stride
    UIB = [(64, 96, 192, 5, 5, 2), (96, 96, 192, 0, 3, 1), (96, 96, 192, 0, 3, 1),
           (96, 96, 192, 0, 3, 1), (96, 96, 192, 0, 3, 1), (96, 96, 384, 3, 0, 1),
           (96, 128, 576, 3, 3, 2), (128, 128, 512, 5, 5, 1), (128, 128, 512, 0, 5, 1),
           (128, 128, 384, 0, 5, 1), (128, 128, 512, 0, 3, 1), (128, 128, 512, 0, 3, 1)]

    def __init__(self, num_classes=10, input_channels=1):
        if num_classes == 0:
            raise ox.OxideError(ox.INVALID_SHAPE, "num_classes must be non-zero")
        self.num_classes = num_classes
        self.blocks = [ConvNormAct(input_channels, 32, 3, 2, 1, True),
                       FusedInvertedBottleneck(32, 32, 32, 3, 2),
                       FusedInvertedBottleneck(32, 64, 96, 3, 2)]
        self.blocks += [UniversalInvertedBottleneck(*spec) for spec in self.UIB]
        self.blocks += [ConvNormAct(128, 960, 1, 1, 1, True), GlobalAveragePool(),
                        ConvNormAct(960, 1280, 1, 1, 1, True)]
        self.classifier = Conv2d(1280, num_classes, 1)

    @classmethod
    def mnist(cls):
        return cls(10, 1)

    def children(self):
        return self.blocks + [self.classifier]

    def forward(self, x):
        for b in self.blocks:
            x = b(x)
        x = self.classifier(x)
        return x.reshape((x.shape[0], self.num_classes))


class AdamW:
    """optim.rs:35-76: bias-corrected, decoupled weight decay; betas (0.9, 0.999), eps 1e-8."""

    def __init__(self, learning_rate: float, weight_decay: float):
        lr, wd = np.float32(learning_rate), np.float32(weight_decay)
        if not np.isfinite(lr) or lr <= 0:
            raise ox.OxideError(ox.EXECUTION, "AdamW learning rate must be positive and finite")
        if not np.isfinite(wd) or wd < 0:
            raise ox.OxideError(ox.EXECUTION,
                                "AdamW weight decay must be non-negative and finite")
        self.learning_rate, self.weight_decay = float(lr), float(wd)
        self.betas, self.epsilon = (0.9, 0.999), 1e-8
