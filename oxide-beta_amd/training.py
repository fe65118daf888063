"""Fixed-schedule training step for MobileNetV4-Conv-S (MNIST variant) on liboxide_hip.so.

Mirrors the reference's model and training driver on the device path:

* modules: ``Conv2d``, ``BatchNorm2d``, ``ConvNormAct``, ``UniversalInvertedBottleneck``,
  ``FusedInvertedBottleneck`` (crates/oxide-torch/src/nn.rs:107-655) and
  ``MobileNetV4ConvSmall.mnist`` (crates/oxide-torch-models/src/models/mobilenet_v4.rs:84-195);
* lazy ops traced from the modules' ``forward`` (``conv2d``, ``batch_norm2d``, ``relu``, ``add``,
  ``global_avg_pool2d``, ``reshape``, ``cross_entropy``; crates/oxide-torch/src/tensor/mod.rs);
* the step of examples/mnist_training.rs:75-92: forward, cross entropy, backward, AdamW
  (lr 1e-3, weight decay 1e-4, betas 0.9 / 0.999, eps 1e-8; optim.rs:48-127) over every
  parameter.

The reference's eager executor (crates/oxide-torch/src/cuda/runtime.rs) walks the lazy graph on
every step. Here the graph is traced once into a fixed list of C-ABI launches over preallocated
device buffers -- forward in topological order, the fused loss + logit gradient (the loss is the
backward root, outer gradient 1), the backward in reverse topological order with
first-write-then-accumulate gradients (runtime.rs:671-692), and one multi-tensor AdamW that
advances a device step counter -- and that list is captured into one hipGraph, so a step is one
graph launch. Each scheduled ``Op`` records the tensors it reads and writes so a checker can
recompute it independently.

Two rewrites keep the launch count down without changing any value: a BatchNorm whose only
consumer is a ReLU (ConvNormAct with activation) runs as one fused BN + ReLU launch group each
way (the ReLU backward's mask is read from the ReLU output, which is positive exactly where its
input is), and the gradient of a residual add's first operand, when the add is that operand's
only consumer, is the add's own gradient buffer (the add's backward is the identity).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable

import numpy as np

import oxide_hip as ox

BN_MOMENTUM, BN_EPSILON = 0.1, 1e-5


# ----------------------------------------------------------------------------- lazy graph

class Node:
    """A traced value: one of the graph ops (graph.rs) the model uses."""

    _ids = 0

    def __init__(self, op: str, inputs: tuple, shape: tuple, **attrs):
        Node._ids += 1
        self.id = Node._ids
        self.op, self.inputs, self.shape, self.attrs = op, inputs, tuple(shape), attrs

    def numel(self) -> int:
        return int(np.prod(self.shape))

    def conv2d(self, weight: "Parameter", bias: "Parameter", stride: int, padding: int,
               groups: int) -> "Node":
        n, cin, h, w = self.shape
        cout, cin_g, kh, kw = weight.shape
        if cin != cin_g * groups:
            raise ox.OxideError(ox.INVALID_SHAPE, "conv2d input channels do not match weight")
        oh, ow = (h + 2 * padding - kh) // stride + 1, (w + 2 * padding - kw) // stride + 1
        return Node("conv2d", (self, weight.node, bias.node), (n, cout, oh, ow), stride=stride,
                    padding=padding, groups=groups)

    def batch_norm2d(self, bn: "BatchNorm2d") -> "Node":
        return Node("batch_norm2d", (self, bn.weight.node, bn.bias.node), self.shape, bn=bn)

    def relu(self) -> "Node":
        return Node("relu", (self,), self.shape)

    def add(self, other: "Node") -> "Node":
        if other.shape != self.shape:
            raise ox.OxideError(ox.INVALID_SHAPE, "add needs equal shapes")
        return Node("add", (self, other), self.shape)

    def global_avg_pool2d(self) -> "Node":
        """tensor/mod.rs:273-283: average pooling with the whole plane as the window."""
        n, c, h, w = self.shape
        return Node("avg_pool2d", (self,), (n, c, 1, 1), kernel=(h, w), stride=(h, w))

    def reshape(self, shape) -> "Node":
        if int(np.prod(shape)) != self.numel():
            raise ox.OxideError(ox.INVALID_SHAPE, "reshape must preserve the element count")
        return Node("reshape", (self,), tuple(shape))

    def cross_entropy(self, targets: "Node") -> "Node":
        return Node("cross_entropy", (self, targets), (1,))


class Parameter:
    """nn.rs Parameter: a trainable tensor with a stable identity."""

    def __init__(self, values: np.ndarray):
        self.values = np.ascontiguousarray(values, dtype=np.float32)
        self.shape = self.values.shape
        self.node = Node("param", (), self.shape, param=self)
        self.value = self.grad = self.first_moment = self.second_moment = None


# ----------------------------------------------------------------------------- modules

class Conv2d:
    """nn.rs:236-274: OIHW weight from the deterministic initialisation, zero bias,
    padding kernel // 2."""

    def __init__(self, in_channels, out_channels, kernel, stride, groups):
        if kernel == 0 or groups == 0 or in_channels % groups or out_channels % groups:
            raise ox.OxideError(ox.INVALID_SHAPE,
                                "invalid Conv2d channel, group, or kernel configuration")
        shape = [out_channels, in_channels // groups, kernel, kernel]
        self.weight = Parameter(ox.initialized_weights(shape, in_channels // groups))
        self.bias = Parameter(np.zeros(out_channels, np.float32))
        self.stride, self.padding, self.groups = stride, kernel // 2, groups

    def forward(self, x: Node) -> Node:
        return x.conv2d(self.weight, self.bias, self.stride, self.padding, self.groups)

    def parameters(self):
        return [self.weight, self.bias]

    def batch_norms(self):
        return []


class BatchNorm2d:
    """nn.rs:107-233: gamma 1, beta 0, running mean 0 / variance 1, momentum 0.1, eps 1e-5,
    training mode."""

    def __init__(self, channels):
        self.weight = Parameter(np.ones(channels, np.float32))
        self.bias = Parameter(np.zeros(channels, np.float32))
        self.running_mean = np.zeros(channels, np.float32)
        self.running_variance = np.ones(channels, np.float32)
        self.channels = channels
        self.device_running_mean = self.device_running_variance = None

    def forward(self, x: Node) -> Node:
        return x.batch_norm2d(self)

    def parameters(self):
        return [self.weight, self.bias]


class ConvNormAct:
    """nn.rs:349-385: convolution, BatchNorm, optional ReLU."""

    def __init__(self, in_channels, out_channels, kernel, stride, groups, activation):
        self.conv = Conv2d(in_channels, out_channels, kernel, stride, groups)
        self.norm = BatchNorm2d(out_channels)
        self.activation = activation

    def forward(self, x: Node) -> Node:
        y = self.norm.forward(self.conv.forward(x))
        return y.relu() if self.activation else y

    def parameters(self):
        return self.conv.parameters() + self.norm.parameters()

    def batch_norms(self):
        return [self.norm]


class UniversalInvertedBottleneck:
    """nn.rs:425-515: optional start depthwise (with ReLU), expand 1x1, optional (strided)
    middle depthwise, project 1x1 without activation; residual when stride 1 and the channel
    counts match."""

    def __init__(self, cin, cout, expanded, start_dw, middle_dw, stride):
        if stride > 1 and middle_dw is None:
            raise ox.OxideError(ox.INVALID_SHAPE,
                                "a strided UIB requires a middle depthwise convolution")
        self.start = ConvNormAct(cin, cin, start_dw, 1, cin, True) if start_dw else None
        self.expand = ConvNormAct(cin, expanded, 1, 1, 1, True)
        self.middle = (ConvNormAct(expanded, expanded, middle_dw, stride, expanded, True)
                       if middle_dw else None)
        self.project = ConvNormAct(expanded, cout, 1, 1, 1, False)
        self.residual = stride == 1 and cin == cout

    def layers(self):
        return [l for l in (self.start, self.expand, self.middle, self.project) if l is not None]

    def forward(self, x: Node) -> Node:
        y = x
        for layer in self.layers():
            y = layer.forward(y)
        return y.add(x) if self.residual else y

    def parameters(self):
        return [p for l in self.layers() for p in l.parameters()]

    def batch_norms(self):
        return [l.norm for l in self.layers()]


class FusedInvertedBottleneck:
    """nn.rs:565-655: full k x k expand convolution with ReLU, 1x1 project; residual when
    stride 1 and the channel counts match."""

    def __init__(self, cin, cout, expanded, kernel, stride):
        self.expand = ConvNormAct(cin, expanded, kernel, stride, 1, True)
        self.project = ConvNormAct(expanded, cout, 1, 1, 1, False)
        self.residual = stride == 1 and cin == cout

    def forward(self, x: Node) -> Node:
        y = self.project.forward(self.expand.forward(x))
        return y.add(x) if self.residual else y

    def parameters(self):
        return self.expand.parameters() + self.project.parameters()

    def batch_norms(self):
        return [self.expand.norm, self.project.norm]


class GlobalAverage:
    def forward(self, x: Node) -> Node:
        return x.global_avg_pool2d()

    def parameters(self):
        return []

    def batch_norms(self):
        return []


class MobileNetV4ConvSmall:
    """mobilenet_v4.rs:84-195; ``mnist()`` maps [N, 1, 28, 28] to 10 logits."""

    # in, out, expanded, start depthwise, middle depthwise, stride (mobilenet_v4.rs:140-153)
    UIB_SPECS = [
        (64, 96, 192, 5, 5, 2), (96, 96, 192, None, 3, 1), (96, 96, 192, None, 3, 1),
        (96, 96, 192, None, 3, 1), (96, 96, 192, None, 3, 1), (96, 96, 384, 3, None, 1),
        (96, 128, 576, 3, 3, 2), (128, 128, 512, 5, 5, 1), (128, 128, 512, None, 5, 1),
        (128, 128, 384, None, 5, 1), (128, 128, 512, None, 3, 1), (128, 128, 512, None, 3, 1),
    ]

    def __init__(self, num_classes=10, input_channels=1, input_resolution=28):
        if num_classes == 0:
            raise ox.OxideError(ox.INVALID_SHAPE, "num_classes must be non-zero")
        self.num_classes = num_classes
        self.input_channels, self.input_resolution = input_channels, input_resolution
        self.blocks = [ConvNormAct(input_channels, 32, 3, 2, 1, True),
                       FusedInvertedBottleneck(32, 32, 32, 3, 2),
                       FusedInvertedBottleneck(32, 64, 96, 3, 2)]
        self.blocks += [UniversalInvertedBottleneck(*spec) for spec in self.UIB_SPECS]
        self.blocks += [ConvNormAct(128, 960, 1, 1, 1, True), GlobalAverage(),
                        ConvNormAct(960, 1280, 1, 1, 1, True),
                        Conv2d(1280, num_classes, 1, 1, 1)]

    @classmethod
    def new(cls, num_classes):
        """The 224 x 224 RGB table-11 network."""
        return cls(num_classes, 3, 224)

    @classmethod
    def mnist(cls):
        return cls(10, 1, 28)

    def forward_with_shapes(self, x: Node):
        """mobilenet_v4.rs:182-195: the output and every block's output shape, the last one
        replaced by the reshaped [N, classes]."""
        if x.shape[1:] != (self.input_channels, self.input_resolution, self.input_resolution):
            raise ox.OxideError(ox.INVALID_SHAPE, f"expected [N, {self.input_channels}, "
                                f"{self.input_resolution}, {self.input_resolution}] input")
        shapes = []
        for block in self.blocks:
            x = block.forward(x)
            shapes.append(x.shape)
        x = x.reshape((x.shape[0], self.num_classes))
        shapes[-1] = x.shape
        return x, shapes

    def forward(self, x: Node) -> Node:
        return self.forward_with_shapes(x)[0]

    def parameters(self):
        """visit_parameters order, block by block."""
        return [p for b in self.blocks for p in b.parameters()]

    def batch_norms(self):
        return [bn for b in self.blocks for bn in b.batch_norms()]

    def parameter_count(self) -> int:
        return sum(p.values.size for p in self.parameters())

    def train(self):
        self.training = True

    def eval(self):
        self.training = False

    training = True

    def save(self, path) -> None:
        """OXTR checkpoint (mobilenet_v4.rs:217-264): every parameter in visit order, then each
        BatchNorm's running mean and running variance.  Values come from the host copies; a
        TrainingStep's device state is brought back first with ``TrainingStep.sync_to_model``."""
        tensors = [(p.shape, p.values) for p in self.parameters()]
        for bn in self.batch_norms():
            tensors += [((bn.channels,), bn.running_mean), ((bn.channels,), bn.running_variance)]
        ox.checkpoint_save(path, tensors)

    @classmethod
    def load_mnist(cls, path) -> "MobileNetV4ConvSmall":
        """load_mnist (mobilenet_v4.rs:266-321): the MNIST model with the checkpoint's
        parameters and running statistics, in inference mode.  Too few or extra tensors ->
        Execution; a parameter or buffer of another shape -> InvalidShape."""
        tensors = ox.checkpoint_load(path)
        model = cls.mnist()
        nxt = 0
        for p in model.parameters():
            if nxt >= len(tensors):
                raise ox.OxideError(ox.EXECUTION, "checkpoint has too few tensors")
            shape, values = tensors[nxt]
            if tuple(shape) != tuple(p.shape):
                raise ox.OxideError(ox.INVALID_SHAPE, f"checkpoint tensor {nxt} has shape "
                                    f"{list(shape)}, expected {list(p.shape)}")
            if values.size != p.values.size:  # Tensor::from_vec in replace_data
                raise ox.OxideError(ox.INVALID_SHAPE, "data length does not match the shape")
            p.values = values.reshape(p.shape).astype(np.float32)
            nxt += 1
        for bn in model.batch_norms():
            for name in ("running_mean", "running_variance"):
                if nxt >= len(tensors):
                    raise ox.OxideError(ox.EXECUTION, "checkpoint has too few buffers")
                shape, values = tensors[nxt]
                if tuple(shape) != (bn.channels,) or values.size != bn.channels:
                    raise ox.OxideError(ox.INVALID_SHAPE, f"checkpoint buffer {nxt} shape mismatch")
                setattr(bn, name, values.astype(np.float32))
                nxt += 1
        if nxt != len(tensors):
            raise ox.OxideError(ox.EXECUTION, "checkpoint has extra tensors")
        model.eval()
        return model


# ----------------------------------------------------------------------------- schedule

@dataclass
class Op:
    """One scheduled launch group.

    ``kind`` names what it computes; ``reads`` / ``writes`` map argument names to the device
    tensors it reads and writes; ``inplace`` lists tensors it updates in place (their values
    before the launch are part of its input); ``attrs`` holds its static arguments. A gradient
    contribution to a value that already holds one is written to ``writes["contribution"]``
    and then added into ``accumulate_into`` by the same op."""

    name: str
    kind: str
    reads: dict = field(default_factory=dict)
    writes: dict = field(default_factory=dict)
    inplace: tuple = ()
    attrs: dict = field(default_factory=dict)
    accumulate_into: object = None
    launch: Callable[[], None] | None = None


def _topological(root: Node) -> list[Node]:
    """Inputs before consumers (iterative depth-first post-order)."""
    order, seen, stack = [], set(), [(root, False)]
    while stack:
        node, expanded = stack.pop()
        if expanded:
            order.append(node)
            continue
        if node.id in seen:
            continue
        seen.add(node.id)
        stack.append((node, True))
        for i in reversed(node.inputs):
            if i.id not in seen:
                stack.append((i, False))
    return order


class TrainingStep:
    """examples/mnist_training.rs:75-92 as a fixed launch list over preallocated device
    buffers, replayable from one hipGraph.

    Parameters, Adam moments, BatchNorm running statistics, activations and gradients live on
    the device for the object's lifetime; ``set_batch`` uploads one batch; ``run_eager`` issues
    the launch list; ``capture`` records it into a graph that ``replay`` launches."""

    def __init__(self, model: MobileNetV4ConvSmall, batch: int, learning_rate=1e-3,
                 weight_decay=1e-4, beta1=0.9, beta2=0.999, epsilon=1e-8, device: int = 0):
        import torch

        if batch <= 0:
            raise ox.OxideError(ox.INVALID_SHAPE, "batch must be positive")
        if not (np.isfinite(learning_rate) and learning_rate > 0):
            raise ox.OxideError(ox.INVALID_SHAPE,
                                "AdamW learning rate must be positive and finite")
        if not (np.isfinite(weight_decay) and weight_decay >= 0):
            raise ox.OxideError(ox.INVALID_SHAPE,
                                "AdamW weight decay must be non-negative and finite")
        self.torch = torch
        self.model, self.batch = model, batch
        self.hyper = dict(learning_rate=learning_rate, weight_decay=weight_decay, beta1=beta1,
                          beta2=beta2, epsilon=epsilon)
        self.dev = torch.device(f"cuda:{device}")
        # a private module: its workspaces are sized once below and never move, so the
        # addresses a captured graph holds stay valid
        self.m = ox.LoadedModule(device)
        self.stream = torch.cuda.Stream(device=self.dev)
        r = model.input_resolution
        self.input_node = Node("input", (), (batch, model.input_channels, r, r))
        self.target_node = Node("targets", (), (batch,))
        self.logits_node = model.forward(self.input_node)
        self.loss_node = self.logits_node.cross_entropy(self.target_node)
        self.order = _topological(self.loss_node)
        self.consumers: dict[int, list[Node]] = {}
        for n in self.order:
            for i in n.inputs:
                self.consumers.setdefault(i.id, []).append(n)
        # relu node id -> the batch norm it absorbs
        self.fused_relu: dict[int, Node] = {}
        for n in self.order:
            if n.op == "relu" and n.inputs[0].op == "batch_norm2d" and \
                    len(self.consumers[n.inputs[0].id]) == 1:
                self.fused_relu[n.id] = n.inputs[0]
        self.fused_bn = {bn.id for bn in self.fused_relu.values()}
        self.params = model.parameters()
        self.value: dict[int, object] = {}
        self.grad: dict[int, object] = {}
        self._written: set[int] = set()
        self._allocate()
        self.ops: list[Op] = []
        self._schedule_forward()
        self._schedule_backward()
        self._schedule_optimizer()
        self._size_workspaces()
        self.graph = None

    # -- buffers
    def _empty(self, shape):
        return self.torch.empty(tuple(shape), device=self.dev)

    def _allocate(self):
        torch = self.torch
        for n in self.order:
            if n.op == "param":
                p = n.attrs["param"]
                p.value = torch.from_numpy(p.values.copy()).to(self.dev)
                p.grad = self._empty(p.shape)
                p.first_moment = torch.zeros(p.shape, device=self.dev)
                p.second_moment = torch.zeros(p.shape, device=self.dev)
                self.value[n.id], self.grad[n.id] = p.value, p.grad
                continue
            if n.op == "reshape":
                self.value[n.id] = self.value[n.inputs[0].id].view(n.shape)
                continue
            if n.id not in self.fused_bn:  # a fused BN's output is never stored
                self.value[n.id] = self._empty(n.shape)
            if n.op == "batch_norm2d":
                bn = n.attrs["bn"]
                bn.device_running_mean = torch.from_numpy(bn.running_mean.copy()).to(self.dev)
                bn.device_running_variance = torch.from_numpy(
                    bn.running_variance.copy()).to(self.dev)
                n.attrs["saved_mean"] = self._empty((bn.channels,))
                n.attrs["saved_inverse_std"] = self._empty((bn.channels,))
        # activation gradients, consumers before producers: a reshape shares its input's
        # buffer; an add's first operand, consumed only by the add, shares the add's
        self.aliased: set[int] = set()
        for n in reversed(self.order):
            if n.op in ("param", "input", "targets", "cross_entropy") or n.id in self.fused_bn:
                continue
            if n.id not in self.grad:
                self.grad[n.id] = self._empty(n.shape)
            if n.op == "reshape":
                self.grad[n.inputs[0].id] = self.grad[n.id].view(n.inputs[0].shape)
            elif n.op == "add":
                first = n.inputs[0]
                if len(self.consumers[first.id]) == 1 and first.id not in self.grad and \
                        first.op not in ("param", "input"):
                    self.grad[first.id] = self.grad[n.id]
                    self.aliased.add(first.id)
        self.outer_gradient = torch.ones(1, device=self.dev)
        self.error_flag = torch.zeros(1, dtype=torch.int32, device=self.dev)
        self.step_counter = torch.zeros(1, dtype=torch.int32, device=self.dev)
        largest = max(n.numel() for n in self.order if n.op not in ("param", "cross_entropy"))
        self.scratch = self._empty((largest,))
        self.class_indices = torch.zeros(self.batch, dtype=torch.int32, device=self.dev)
        self.input = self.value[self.input_node.id]
        self.targets = self.value[self.target_node.id]
        self.loss = self.value[self.loss_node.id]
        self.logits = self.value[self.logits_node.id]
        torch.cuda.synchronize()

    def _size_workspaces(self):
        bn, conv = 0, 0
        for n in self.order:
            if n.op == "batch_norm2d":
                b, c, h, w = n.shape
                bn = max(bn, ox.batch_norm_workspace_size(b, c, h * w))
            elif n.op == "conv2d":
                conv = max(conv, ox.conv2d_workspace_size(n.attrs["cshape"]))
        rows, classes = self.logits_node.shape
        self.m._bn_ws.get(bn)
        self.m._conv_ws.get(conv)
        self.m._ce_ws.get(ox.cross_entropy_workspace_size(rows, classes))

    # -- gradient contributions (runtime.rs:671-692: the first writes, later ones accumulate)
    def _contribution(self, node: Node):
        """(destination, accumulate_into) for a new contribution to node's gradient."""
        g = self.grad[node.id]
        if node.id not in self._written:
            self._written.add(node.id)
            return g, None
        return self.scratch[: g.numel()].view(g.shape), g

    def _emit(self, op: Op, body: Callable[[], None]):
        s, acc = self.stream, op.accumulate_into
        if acc is None:
            op.launch = body
        else:
            part = op.writes["contribution"]

            def launch():
                body()
                self.m.accumulate(acc, part, acc, stream=s)

            op.launch = launch
            op.inplace = op.inplace + (acc,)
        self.ops.append(op)

    # -- forward, topological order
    def _schedule_forward(self):
        m, s, V = self.m, self.stream, self.value
        for n in self.order:
            if n.op in ("param", "input", "targets", "reshape"):
                continue
            if n.id in self.fused_bn:
                continue  # scheduled with its ReLU
            out = V[n.id]
            if n.op == "relu" and n.id in self.fused_relu:
                bn_node = self.fused_relu[n.id]
                x, gamma, beta = (V[i.id] for i in bn_node.inputs)
                bn = bn_node.attrs["bn"]
                sm, si = bn_node.attrs["saved_mean"], bn_node.attrs["saved_inverse_std"]
                rm, rv = bn.device_running_mean, bn.device_running_variance
                self._emit(Op(f"bn{bn_node.id}+relu{n.id}", "batch_norm2d_relu_forward",
                              dict(x=x, weight=gamma, bias=beta),
                              dict(y=out, saved_mean=sm, saved_inverse_std=si),
                              inplace=(rm, rv),
                              attrs=dict(momentum=BN_MOMENTUM, epsilon=BN_EPSILON,
                                         running_mean=rm, running_variance=rv)),
                           lambda x=x, gamma=gamma, beta=beta, rm=rm, rv=rv, sm=sm, si=si,
                           out=out: m.batch_norm_relu_forward_train(
                               x, gamma, beta, rm, rv, sm, si, out, BN_MOMENTUM, BN_EPSILON,
                               stream=s))
            elif n.op == "conv2d":
                x, w, b = (V[i.id] for i in n.inputs)
                shape = ox.conv2d_shape(*n.inputs[0].shape, n.shape[1], n.inputs[1].shape[2],
                                        n.attrs["stride"], n.attrs["padding"], n.attrs["groups"])
                n.attrs["cshape"] = shape
                self._emit(Op(f"conv{n.id}", "conv2d_forward", dict(x=x, weight=w, bias=b),
                              dict(y=out), attrs=_conv_attrs(n)),
                           lambda shape=shape, x=x, w=w, b=b, out=out:
                           m.conv2d_forward(shape, x, w, b, out, stream=s))
            elif n.op == "batch_norm2d":
                x, gamma, beta = (V[i.id] for i in n.inputs)
                bn = n.attrs["bn"]
                sm, si = n.attrs["saved_mean"], n.attrs["saved_inverse_std"]
                rm, rv = bn.device_running_mean, bn.device_running_variance
                self._emit(Op(f"bn{n.id}", "batch_norm2d_forward",
                              dict(x=x, weight=gamma, bias=beta),
                              dict(y=out, saved_mean=sm, saved_inverse_std=si),
                              inplace=(rm, rv),
                              attrs=dict(momentum=BN_MOMENTUM, epsilon=BN_EPSILON,
                                         running_mean=rm, running_variance=rv)),
                           lambda x=x, gamma=gamma, beta=beta, rm=rm, rv=rv, sm=sm, si=si,
                           out=out: m.batch_norm_forward_train(x, gamma, beta, rm, rv, sm, si,
                                                               out, BN_MOMENTUM, BN_EPSILON,
                                                               stream=s))
            elif n.op == "relu":
                x = V[n.inputs[0].id]
                self._emit(Op(f"relu{n.id}", "relu_forward", dict(x=x), dict(y=out)),
                           lambda x=x, out=out: m.relu(x, out, stream=s))
            elif n.op == "add":
                a, b = V[n.inputs[0].id], V[n.inputs[1].id]
                self._emit(Op(f"add{n.id}", "add_forward", dict(a=a, b=b), dict(y=out)),
                           lambda a=a, b=b, out=out: m.add(a, b, out, stream=s))
            elif n.op == "avg_pool2d":
                x = V[n.inputs[0].id]
                ps = ox.Pool2dShape(*n.inputs[0].shape, *n.attrs["kernel"], *n.attrs["stride"])
                n.attrs["pshape"] = ps
                self._emit(Op(f"pool{n.id}", "avg_pool2d_forward", dict(x=x), dict(y=out),
                              attrs=dict(kernel=n.attrs["kernel"], stride=n.attrs["stride"])),
                           lambda ps=ps, x=x, out=out: m.avg_pool2d_forward(ps, x, out,
                                                                            stream=s))
            elif n.op == "cross_entropy":
                logits_node = n.inputs[0]
                logits, targets = V[logits_node.id], V[n.inputs[1].id]
                rows, classes = logits_node.shape
                dlogits, _ = self._contribution(logits_node)
                self._emit(Op(f"ce{n.id}", "cross_entropy",
                              dict(logits=logits, targets=targets,
                                   outer_gradient=self.outer_gradient),
                              dict(loss=out, gradient=dlogits), inplace=(self.error_flag,)),
                           lambda logits=logits, targets=targets, out=out, dl=dlogits:
                           m.cross_entropy_forward_backward(rows, classes, logits, targets,
                                                            self.outer_gradient, out, dl,
                                                            self.error_flag, stream=s))
            else:
                raise ox.OxideError(ox.TRACE, f"no forward for {n.op}")

    # -- backward, reverse topological order: every consumer of a value runs before it
    def _schedule_backward(self):
        m, s, V, G = self.m, self.stream, self.value, self.grad
        for n in reversed(self.order):
            if n.op in ("param", "input", "targets", "cross_entropy"):
                continue
            if n.id in self.fused_bn:
                continue  # its backward ran with its ReLU's
            if n.id not in self._written:
                raise ox.OxideError(ox.TRACE, f"{n.op} value {n.id} receives no gradient")
            g = G[n.id]
            if n.op == "relu" and n.id in self.fused_relu:
                bn_node = self.fused_relu[n.id]
                x_node, w_node, b_node = bn_node.inputs
                x, gamma, y = V[x_node.id], V[w_node.id], V[n.id]
                sm, si = bn_node.attrs["saved_mean"], bn_node.attrs["saved_inverse_std"]
                dgamma, _ = self._contribution(w_node)
                dbeta, _ = self._contribution(b_node)
                dst, acc = self._contribution(x_node)
                self._emit(Op(f"bn{bn_node.id}+relu{n.id}.backward",
                              "batch_norm2d_relu_backward",
                              dict(gradient=g, y=y, x=x, weight=gamma, saved_mean=sm,
                                   saved_inverse_std=si),
                              dict(contribution=dst, weight_gradient=dgamma,
                                   bias_gradient=dbeta),
                              accumulate_into=acc),
                           lambda g=g, y=y, x=x, gamma=gamma, sm=sm, si=si, dst=dst,
                           dgamma=dgamma, dbeta=dbeta: m.batch_norm_relu_backward_train(
                               g, y, x, gamma, sm, si, dst, dgamma, dbeta, stream=s))
            elif n.op == "reshape":
                # the gradient buffer is the input's; its one consumer has written it
                if n.inputs[0].id in self._written:
                    raise ox.OxideError(ox.TRACE, "a reshaped value must have one consumer")
                self._written.add(n.inputs[0].id)
            elif n.op == "relu":
                x_node = n.inputs[0]
                x = V[x_node.id]
                dst, acc = self._contribution(x_node)
                self._emit(Op(f"relu{n.id}.backward", "relu_backward", dict(gradient=g, x=x),
                              dict(contribution=dst), accumulate_into=acc),
                           lambda g=g, x=x, dst=dst: m.relu_backward(g, x, dst, stream=s))
            elif n.op == "add":
                for i, inp in enumerate(n.inputs):
                    if i == 0 and inp.id in self.aliased:
                        self._written.add(inp.id)  # the add's gradient buffer is its own
                        continue
                    dst, acc = self._contribution(inp)
                    self._emit(Op(f"add{n.id}.backward{i}", "add_backward", dict(gradient=g),
                                  dict(contribution=dst), accumulate_into=acc),
                               lambda g=g, dst=dst: ox.check(ox.lib().oxh_memcpy_d2d_async(
                                   dst.data_ptr(), g.data_ptr(), g.numel() * 4,
                                   ox._stream(s))))
            elif n.op == "avg_pool2d":
                x_node = n.inputs[0]
                ps = n.attrs["pshape"]
                dst, acc = self._contribution(x_node)
                self._emit(Op(f"pool{n.id}.backward", "avg_pool2d_backward", dict(gradient=g),
                              dict(contribution=dst),
                              attrs=dict(input_shape=x_node.shape, kernel=n.attrs["kernel"],
                                         stride=n.attrs["stride"]),
                              accumulate_into=acc),
                           lambda ps=ps, g=g, dst=dst: m.avg_pool2d_backward(ps, g, dst,
                                                                             stream=s))
            elif n.op == "batch_norm2d":
                x_node, w_node, b_node = n.inputs
                x, gamma = V[x_node.id], V[w_node.id]
                sm, si = n.attrs["saved_mean"], n.attrs["saved_inverse_std"]
                dgamma, _ = self._contribution(w_node)
                dbeta, _ = self._contribution(b_node)
                dst, acc = self._contribution(x_node)
                self._emit(Op(f"bn{n.id}.backward", "batch_norm2d_backward",
                              dict(gradient=g, x=x, weight=gamma, saved_mean=sm,
                                   saved_inverse_std=si),
                              dict(contribution=dst, weight_gradient=dgamma,
                                   bias_gradient=dbeta),
                              accumulate_into=acc),
                           lambda g=g, x=x, gamma=gamma, sm=sm, si=si, dst=dst, dgamma=dgamma,
                           dbeta=dbeta: m.batch_norm_backward_train(g, x, gamma, sm, si, dst,
                                                                    dgamma, dbeta, stream=s))
            elif n.op == "conv2d":
                x_node, w_node, b_node = n.inputs
                x, w = V[x_node.id], V[w_node.id]
                shape = n.attrs["cshape"]
                dw, _ = self._contribution(w_node)
                db, _ = self._contribution(b_node)
                self._emit(Op(f"conv{n.id}.backward_parameters", "conv2d_parameter_backward",
                              dict(gradient=g, x=x, weight=w),
                              dict(weight_gradient=dw, bias_gradient=db), attrs=_conv_attrs(n)),
                           lambda shape=shape, g=g, x=x, dw=dw, db=db:
                           (m.conv2d_weight_backward(shape, g, x, dw, stream=s),
                            m.conv2d_bias_backward(shape, g, db, stream=s)))
                if x_node.op == "input":  # the network input needs no gradient
                    continue
                dst, acc = self._contribution(x_node)
                self._emit(Op(f"conv{n.id}.backward_input", "conv2d_input_backward",
                              dict(gradient=g, x=x, weight=w), dict(contribution=dst),
                              attrs=_conv_attrs(n), accumulate_into=acc),
                           lambda shape=shape, g=g, w=w, dst=dst:
                           m.conv2d_input_backward(shape, g, w, dst, stream=s))
            else:
                raise ox.OxideError(ox.TRACE, f"no backward for {n.op}")

    def _schedule_optimizer(self):
        h = self.hyper
        tensors = [(p.value, p.grad, p.first_moment, p.second_moment) for p in self.params]
        inplace = tuple(t for p in self.params
                        for t in (p.value, p.first_moment, p.second_moment))
        s = self.stream

        def launch():
            self.m.adamw_multi_tensor_step(h["learning_rate"], h["weight_decay"], h["beta1"],
                                           h["beta2"], h["epsilon"], self.step_counter, tensors,
                                           stream=s)

        self.ops.append(Op("adamw", "adamw", dict(gradients=[p.grad for p in self.params]), {},
                           inplace=inplace + (self.step_counter,),
                           attrs=dict(self.hyper, tensors=tensors,
                                      step_counter=self.step_counter),
                           launch=launch))

    # -- running
    def set_batch(self, images: np.ndarray, labels: np.ndarray):
        """Uploads one batch: images [N, C, H, W] float32, labels [N] class indices."""
        torch = self.torch
        images = np.ascontiguousarray(images, np.float32).reshape(self.input.shape)
        labels = np.ascontiguousarray(labels, np.float32).reshape(self.targets.shape)
        self.stream.synchronize()
        self.input.copy_(torch.from_numpy(images))
        self.targets.copy_(torch.from_numpy(labels))
        torch.cuda.synchronize()

    def run_eager(self, before: Callable[[Op], None] | None = None,
                  after: Callable[[Op], None] | None = None):
        """Issues the launch list on the step's stream; ``before`` / ``after`` run around each
        op (checkers synchronise for themselves)."""
        for op in self.ops:
            if before is not None:
                before(op)
            op.launch()
            if after is not None:
                after(op)

    def capture(self) -> ox.HipGraphExec:
        """Records the launch list into one graph. Every launch's arguments are validated by
        the library while recording; a failure aborts the capture and raises."""
        self.graph = ox.HipGraphExec.capture(self.stream, self.run_eager)
        return self.graph

    def replay(self):
        if self.graph is None:
            raise ox.OxideError(ox.EXECUTION, "no captured step; call capture() first")
        self.graph.launch(self.stream)

    def synchronize(self):
        self.stream.synchronize()

    def loss_value(self) -> float:
        """The last step's loss; raises InvalidShape if a target was not a class index
        (evaluation.rs:622-636)."""
        self.synchronize()
        if int(self.error_flag.item()) != 0:
            self.error_flag.zero_()
            self.torch.cuda.synchronize()
            raise ox.OxideError(ox.INVALID_SHAPE, "cross entropy target is not a class index")
        return float(self.loss.item())

    def predicted_classes(self) -> np.ndarray:
        """argmax over the last forward's logits (ties go to the last index)."""
        self.m.argmax_rows(self.logits, self.class_indices, stream=self.stream)
        self.synchronize()
        return self.class_indices.cpu().numpy().astype(np.int64)

    def steps_taken(self) -> int:
        self.synchronize()
        return int(self.step_counter.item())

    def sync_to_model(self) -> None:
        """Copies the device parameters and BatchNorm running statistics back into the model's
        host arrays (sync_batch_norm_state, runtime.rs:1268-1304), e.g. before ``save``."""
        self.synchronize()
        for p in self.params:
            p.values = p.value.detach().cpu().numpy().copy()
        for bn in self.model.batch_norms():
            bn.running_mean = bn.device_running_mean.detach().cpu().numpy().copy()
            bn.running_variance = bn.device_running_variance.detach().cpu().numpy().copy()

class EvalForward:
    """The inference-mode forward (``model.eval()``: BatchNorm normalizes with the running
    statistics, evaluation.rs:448-488,560-575) of ``batch`` images, as mnist_training.rs
    evaluates the test set, with argmax predictions.  Parameters and running statistics are the
    device tensors of ``source`` (a TrainingStep over the same model) when given, else uploaded
    from the model's host arrays (e.g. after ``MobileNetV4ConvSmall.load_mnist``)."""

    def __init__(self, model: MobileNetV4ConvSmall, batch: int,
                 source: TrainingStep | None = None, device: int = 0):
        import torch

        if source is not None and source.model is not model:
            raise ox.OxideError(ox.INVALID_SHAPE, "source trains another model")
        self.torch, self.model, self.batch = torch, model, batch
        self.dev = torch.device(f"cuda:{device}")
        self.m = source.m if source is not None else ox.LoadedModule(device)
        self.stream = source.stream if source is not None else torch.cuda.Stream(device=self.dev)
        r = model.input_resolution
        self.input_node = Node("input", (), (batch, model.input_channels, r, r))
        self.logits_node = model.forward(self.input_node)
        order = _topological(self.logits_node)
        V: dict[int, object] = {}
        for n in order:
            if n.op == "param":
                p = n.attrs["param"]
                V[n.id] = (p.value if source is not None
                           else torch.from_numpy(p.values.copy()).to(self.dev))
            elif n.op == "reshape":
                V[n.id] = V[n.inputs[0].id].view(n.shape)
            else:
                V[n.id] = torch.empty(n.shape, device=self.dev)
        self.input, self.logits = V[self.input_node.id], V[self.logits_node.id]
        self.class_indices = torch.zeros(batch, dtype=torch.int32, device=self.dev)
        self.ops: list[Op] = []
        m, s = self.m, self.stream
        for n in order:
            if n.op in ("param", "input", "reshape"):
                continue
            out = V[n.id]
            if n.op == "conv2d":
                x, w, b = (V[i.id] for i in n.inputs)
                shape = ox.conv2d_shape(*n.inputs[0].shape, n.shape[1], n.inputs[1].shape[2],
                                        n.attrs["stride"], n.attrs["padding"], n.attrs["groups"])
                self.ops.append(Op(f"conv{n.id}", "conv2d_forward", dict(x=x, weight=w, bias=b),
                                   dict(y=out), attrs=_conv_attrs(n),
                                   launch=lambda shape=shape, x=x, w=w, b=b, out=out:
                                   m.conv2d_forward(shape, x, w, b, out, stream=s)))
            elif n.op == "batch_norm2d":
                x, gamma, beta = (V[i.id] for i in n.inputs)
                bn = n.attrs["bn"]
                if source is not None:
                    rm, rv = bn.device_running_mean, bn.device_running_variance
                else:
                    rm = torch.from_numpy(bn.running_mean.copy()).to(self.dev)
                    rv = torch.from_numpy(bn.running_variance.copy()).to(self.dev)
                inv = torch.empty(bn.channels, device=self.dev)
                _, c, h, w_ = n.shape

                def launch(x=x, gamma=gamma, beta=beta, rm=rm, rv=rv, inv=inv, out=out, c=c,
                           hw=h * w_):
                    # evaluation.rs:560-575 then 577-597
                    m.batch_norm_running_inverse_std(BN_EPSILON, rv, inv, stream=s)
                    m.batch_norm_apply(c, hw, x, gamma, beta, rm, inv, out, stream=s)

                self.ops.append(Op(f"bn{n.id}", "batch_norm2d_eval_forward",
                                   dict(x=x, weight=gamma, bias=beta, running_mean=rm,
                                        running_variance=rv),
                                   dict(y=out, inverse_std=inv),
                                   attrs=dict(epsilon=BN_EPSILON), launch=launch))
            elif n.op == "relu":
                x = V[n.inputs[0].id]
                self.ops.append(Op(f"relu{n.id}", "relu_forward", dict(x=x), dict(y=out),
                                   launch=lambda x=x, out=out: m.relu(x, out, stream=s)))
            elif n.op == "add":
                a, b = V[n.inputs[0].id], V[n.inputs[1].id]
                self.ops.append(Op(f"add{n.id}", "add_forward", dict(a=a, b=b), dict(y=out),
                                   launch=lambda a=a, b=b, out=out: m.add(a, b, out, stream=s)))
            elif n.op == "avg_pool2d":
                x = V[n.inputs[0].id]
                ps = ox.Pool2dShape(*n.inputs[0].shape, *n.attrs["kernel"], *n.attrs["stride"])
                self.ops.append(Op(f"pool{n.id}", "avg_pool2d_forward", dict(x=x), dict(y=out),
                                   attrs=dict(kernel=n.attrs["kernel"],
                                              stride=n.attrs["stride"]),
                                   launch=lambda ps=ps, x=x, out=out:
                                   m.avg_pool2d_forward(ps, x, out, stream=s)))
            else:
                raise ox.OxideError(ox.TRACE, f"no inference forward for {n.op}")
        torch.cuda.synchronize()

    def set_images(self, images: np.ndarray) -> None:
        images = np.ascontiguousarray(images, np.float32).reshape(self.input.shape)
        self.stream.synchronize()
        self.input.copy_(self.torch.from_numpy(images))
        self.torch.cuda.synchronize()

    def run(self, before=None, after=None) -> None:
        for op in self.ops:
            if before is not None:
                before(op)
            op.launch()
            if after is not None:
                after(op)

    def predicted_classes(self) -> np.ndarray:
        """argmax of each row of the logits (count_correct, mnist_training.rs:201-218: ties go
        to the last index)."""
        self.m.argmax_rows(self.logits, self.class_indices, stream=self.stream)
        self.stream.synchronize()
        return self.class_indices.cpu().numpy().astype(np.int64)


def op_bytes(op: Op) -> tuple[str, int]:
    """(category, algorithmic HBM bytes) of one launch group: every tensor it must read or
    write, once (fp32).  Categories: the hot-path kernel families (batch_norm2d, elementwise,
    cross_entropy, adamw) and the layers around them (conv2d, avg_pool2d)."""
    nb = lambda t: t.numel() * 4  # noqa: E731
    acc = 3 * nb(op.accumulate_into) if op.accumulate_into is not None else 0
    k = op.kind
    if k in ("batch_norm2d_forward", "batch_norm2d_relu_forward"):
        return "batch_norm2d", 2 * nb(op.reads["x"])                       # x in, y out
    if k == "batch_norm2d_backward":
        return "batch_norm2d", 3 * nb(op.reads["x"]) + acc                 # g, x in; dx out
    if k == "batch_norm2d_relu_backward":
        return "batch_norm2d", 4 * nb(op.reads["x"]) + acc                 # g, y, x in; dx out
    if k == "add_forward":
        return "elementwise", 3 * nb(op.reads["a"])
    if k == "relu_forward":
        return "elementwise", 2 * nb(op.reads["x"])
    if k == "relu_backward":
        return "elementwise", 3 * nb(op.reads["gradient"]) + acc           # g, x in; out
    if k == "add_backward":
        return "elementwise", 2 * nb(op.reads["gradient"]) + acc           # copy of g
    if k == "cross_entropy":
        return "cross_entropy", 2 * nb(op.reads["logits"])
    if k == "adamw":
        return "adamw", sum(7 * nb(t[0]) for t in op.attrs["tensors"])
    if k.startswith("avg_pool2d"):
        return "avg_pool2d", 0
    return "conv2d", 0


def _conv_attrs(n: Node) -> dict:
    return {k: n.attrs[k] for k in ("stride", "padding", "groups")}
