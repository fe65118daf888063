"""The per-launch oracle checker of the device programs: ``before`` snapshots what a launch
group updates in place, ``after`` recomputes the group with the oracle from the device tensors
it actually read and compares what it wrote.

Bars per kind: conv input gradients and forwards summed in the CPU path's order
(oxh_conv2d_input_backward_serial, oxh_conv2d_forward_serial), pooling, ReLU, add, mul,
copies, accumulate and AdamW bit-exact; BatchNorm and cross entropy within the north star's
1e-5 relative (1e-6 absolute, or the conditioning bound of a cancelling sum); the other conv
input gradients and forwards, conv weight / bias and BatchNorm affine gradients within
1e-5 * sum|terms| (fixed-order sums)."""

from collections import Counter

import numpy as np
import torch

import oracle
from helpers import (assert_bitexact, assert_close, assert_conv_forward,
                     assert_conv_input_gradient, assert_within,
                     check_batch_norm_backward, check_batch_norm_forward, host)


class OracleChecker:
    """``before`` snapshots what an op updates in place; ``after`` recomputes the op with the
    oracle from the device tensors it read and compares what it wrote."""

    def __init__(self):
        self.prior = {}
        self.counts = Counter()

    def before(self, op):
        torch.cuda.synchronize()
        self.prior = {id(t): host(t).copy() for t in op.inplace}

    def after(self, op):
        torch.cuda.synchronize()
        getattr(self, op.kind)(op, {k: host(v) for k, v in op.reads.items()})
        if op.accumulate_into is not None:
            prev = self.prior[id(op.accumulate_into)]
            assert_bitexact(host(op.accumulate_into),
                            oracle.accumulate(prev, host(op.writes["contribution"])),
                            f"{op.name} accumulate")
        for role, into in op.side_accumulate.items():
            assert_bitexact(host(into),
                            oracle.accumulate(self.prior[id(into)], host(op.writes[role])),
                            f"{op.name} accumulate {role}")
            self.counts["side accumulate"] += 1
        self.counts[op.kind] += 1

    # -- per kind
    def conv2d_forward(self, op, r):
        a = op.attrs
        assert_conv_forward(host(op.writes["y"]), r["x"], r["weight"], r["bias"], a["stride"],
                            a["padding"], a["groups"], op.name)

    def conv2d_input_backward(self, op, r):
        a = op.attrs
        addend = r.get("addend")  # a residual add's gradient accumulated in the same pass
        if addend is not None:
            self.counts["conv input backward with addend"] += 1
        assert_conv_input_gradient(host(op.writes["contribution"]), r["gradient"], r["weight"],
                                   a["stride"], a["padding"], a["groups"], r["x"].shape, addend,
                                   op.name)

    def conv2d_parameter_backward(self, op, r):
        a = op.attrs
        g, x, w = r["gradient"], r["x"], r["weight"]
        _, rdw, rdb = oracle.conv2d_backward(g, x, w, a["stride"], a["padding"], a["groups"])
        abs_dw = oracle.conv2d_backward(np.abs(g), np.abs(x), np.abs(w), a["stride"],
                                        a["padding"], a["groups"])[1]
        assert_within(host(op.writes["weight_gradient"]), rdw,
                      1e-5 * abs_dw.astype(np.float64) + 1e-7, f"{op.name} weight")
        if "bias_gradient" in op.writes:  # else the following BatchNorm's backward formed it
            assert_within(host(op.writes["bias_gradient"]), rdb,
                          1e-5 * np.abs(g).astype(np.float64).sum(axis=(0, 2, 3)) + 1e-7,
                          f"{op.name} bias")
            self.counts["conv bias in parameter backward"] += 1

    def conv2d_backward(self, op, r):
        """The whole conv VJP in one group: parameter gradients within their bound, the input
        gradient (plus a residual add's gradient) as the input backward's."""
        self.conv2d_parameter_backward(op, r)
        self.conv2d_input_backward(op, r)

    def _conv_bias(self, op):
        """The bias gradient of the convolution feeding a BatchNorm, formed by the BN backward
        from the input gradient it wrote."""
        if "conv_bias_gradient" not in op.writes:
            return
        dx = host(op.writes["contribution"])
        assert_within(host(op.writes["conv_bias_gradient"]), oracle.conv2d_bias_backward(dx),
                      1e-5 * np.abs(dx).astype(np.float64).sum(axis=(0, 2, 3)) + 1e-7,
                      f"{op.name} conv bias")
        self.counts["conv bias in batch norm backward"] += 1

    def batch_norm2d_forward(self, op, r):
        a, w = op.attrs, op.writes
        out = dict(y=host(w["y"]), mean=host(w["saved_mean"]), inv=host(w["saved_inverse_std"]),
                   rm=host(a["running_mean"]), rv=host(a["running_variance"]))
        check_batch_norm_forward(out, r["x"], r["weight"], r["bias"],
                                 self.prior[id(a["running_mean"])],
                                 self.prior[id(a["running_variance"])], a["momentum"],
                                 a["epsilon"])

    def batch_norm2d_add_forward(self, op, r):
        """BN forward writing BN(x) + shortcut: the statistics against the oracle, the output
        equal to the fp32 normalization with those statistics followed by the add."""
        a, w = op.attrs, op.writes
        x, gamma, beta = r["x"], r["weight"], r["bias"]
        mean, inv = host(w["saved_mean"]), host(w["saved_inverse_std"])
        sh = (1, x.shape[1], 1, 1)
        y_bn = ((x - mean.reshape(sh)) * inv.reshape(sh)) * gamma.reshape(sh) + beta.reshape(sh)
        out = dict(y=y_bn, mean=mean, inv=inv, rm=host(a["running_mean"]),
                   rv=host(a["running_variance"]))
        check_batch_norm_forward(out, x, gamma, beta, self.prior[id(a["running_mean"])],
                                 self.prior[id(a["running_variance"])], a["momentum"],
                                 a["epsilon"])
        assert_bitexact(host(w["y"]), oracle.add(y_bn, r["addend"]), op.name)

    def batch_norm2d_backward(self, op, r):
        w = op.writes
        out = dict(dx=host(w["contribution"]), dw=host(w["weight_gradient"]),
                   db=host(w["bias_gradient"]))
        check_batch_norm_backward(out, r["gradient"], r["x"], r["weight"], r["saved_mean"],
                                  r["saved_inverse_std"])
        self._conv_bias(op)

    def batch_norm2d_relu_forward(self, op, r):
        a, w = op.attrs, op.writes
        out = dict(y=host(w["y"]), mean=host(w["saved_mean"]), inv=host(w["saved_inverse_std"]),
                   rm=host(a["running_mean"]), rv=host(a["running_variance"]))
        assert (out["y"] >= 0).all()
        check_batch_norm_forward(out, r["x"], r["weight"], r["bias"],
                                 self.prior[id(a["running_mean"])],
                                 self.prior[id(a["running_variance"])], a["momentum"],
                                 a["epsilon"], relu=True)

    def batch_norm2d_relu_backward(self, op, r):
        w = op.writes
        out = dict(dx=host(w["contribution"]), dw=host(w["weight_gradient"]),
                   db=host(w["bias_gradient"]))
        masked = oracle.relu_backward(r["gradient"], r["y"])
        check_batch_norm_backward(out, masked, r["x"], r["weight"], r["saved_mean"],
                                  r["saved_inverse_std"])
        self._conv_bias(op)

    def _depthwise_forward(self, op, r, relu):
        """Depthwise conv + BN (+ ReLU) in one launch: the convolution output bit-exact, the
        BatchNorm on it as a separate BatchNorm forward is checked."""
        a, w = op.attrs, op.writes
        conv_y = host(w["conv_y"])
        assert_bitexact(conv_y, oracle.conv2d_forward(r["x"], r["conv_weight"], r["conv_bias"],
                                                      a["stride"], a["padding"], a["groups"]),
                        f"{op.name} conv")
        out = dict(y=host(w["y"]), mean=host(w["saved_mean"]), inv=host(w["saved_inverse_std"]),
                   rm=host(a["running_mean"]), rv=host(a["running_variance"]))
        check_batch_norm_forward(out, conv_y, r["weight"], r["bias"],
                                 self.prior[id(a["running_mean"])],
                                 self.prior[id(a["running_variance"])], a["momentum"],
                                 a["epsilon"], relu=relu)

    def depthwise_conv2d_batch_norm_forward(self, op, r):
        self._depthwise_forward(op, r, False)

    def depthwise_conv2d_batch_norm_relu_forward(self, op, r):
        self._depthwise_forward(op, r, True)

    def _depthwise_backward(self, op, r, relu, input_gradient=True):
        """Its backward: the BatchNorm gradients as a BatchNorm backward's, then the
        convolution's bias / weight gradients (fixed-order sums) and input gradient (bit-exact,
        + the residual addend where one is folded in) from the output gradient it wrote.
        Returns the oracle's input gradient of the convolution (before any addend)."""
        a, w = op.attrs, op.writes
        gc = host(w["conv_output_gradient"])
        g = oracle.relu_backward(r["gradient"], r["y"]) if relu else r["gradient"]
        check_batch_norm_backward(dict(dx=gc, dw=host(w["weight_gradient"]),
                                       db=host(w["bias_gradient"])), g, r["conv_y"],
                                  r["weight"], r["saved_mean"], r["saved_inverse_std"])
        x, cw = r["x"], r["conv_weight"]
        s, p, grp = a["stride"], a["padding"], a["groups"]
        rdx, rdw, rdb = oracle.conv2d_backward(gc, x, cw, s, p, grp)
        abs_dw = oracle.conv2d_backward(np.abs(gc), np.abs(x), np.abs(cw), s, p, grp)[1]
        assert_within(host(w["conv_weight_gradient"]), rdw,
                      1e-5 * abs_dw.astype(np.float64) + 1e-7, f"{op.name} conv weight")
        assert_within(host(w["conv_bias_gradient"]), rdb,
                      1e-5 * np.abs(gc).astype(np.float64).sum(axis=(0, 2, 3)) + 1e-7,
                      f"{op.name} conv bias")
        self.counts["conv bias in batch norm backward"] += 1
        if input_gradient and "contribution" in w:
            ref = rdx
            if "addend" in r:
                ref = oracle.accumulate(r["addend"], rdx)
                self.counts["conv input backward with addend"] += 1
            assert_bitexact(host(w["contribution"]), ref, f"{op.name} input gradient")
        return rdx

    def _pre_forward(self, op, r, pre_relu, relu):
        """A BatchNorm (+ ReLU) in front of a depthwise layer, run in the layer's launch: the
        BatchNorm checked as its own forward (statistics, output, running update), then the
        layer from the output it wrote."""
        a, w = op.attrs, op.writes
        pre_y = host(w["pre_y"])
        out = dict(y=pre_y, mean=host(w["pre_saved_mean"]),
                   inv=host(w["pre_saved_inverse_std"]), rm=host(a["pre_running_mean"]),
                   rv=host(a["pre_running_variance"]))
        if "pre_residual" in r:  # BN + residual add: the normalized values, then the add
            x, gamma, beta = r["pre_x"], r["pre_weight"], r["pre_bias"]
            sh = (1, x.shape[1], 1, 1)
            out["y"] = ((x - out["mean"].reshape(sh)) * out["inv"].reshape(sh)) * \
                gamma.reshape(sh) + beta.reshape(sh)
            assert_bitexact(pre_y, oracle.add(out["y"], r["pre_residual"]), f"{op.name} add")
        check_batch_norm_forward(out, r["pre_x"], r["pre_weight"], r["pre_bias"],
                                 self.prior[id(a["pre_running_mean"])],
                                 self.prior[id(a["pre_running_variance"])], a["pre_momentum"],
                                 a["pre_epsilon"], relu=pre_relu)
        self._depthwise_forward(op, dict(r, x=pre_y), relu)
        self.counts["batch norm before depthwise"] += 1

    def _pre_backward(self, op, r, pre_relu, relu):
        """Its backward: the layer's gradients as its own backward's; the BatchNorm in front
        from the layer's input gradient (the oracle's, bit-exact from the output gradient the
        launch wrote) through its ReLU, as a BatchNorm backward's; the bias gradient of a
        convolution feeding it as that BatchNorm backward's dx sum."""
        w = op.writes
        da = self._depthwise_backward(op, r, relu, input_gradient=False)
        whole = da
        inplace = op.by_role.get("conv_input_gradient", [None])[0]
        if "addend" in r:  # the layer input's other contributions (before an in-place update)
            addend = r["addend"]
            if inplace is not None and id(inplace) in self.prior and \
                    op.by_role["addend"][0].ptr == inplace.ptr:
                addend = self.prior[id(inplace)]
            whole = oracle.accumulate(addend, da)
            self.counts["conv input backward with addend"] += 1
        if inplace is not None:
            assert_bitexact(host(inplace), whole, f"{op.name} layer input gradient")
        g = oracle.relu_backward(whole, r["x"]) if pre_relu else whole
        dx = host(w["contribution"])
        check_batch_norm_backward(dict(dx=dx, dw=host(w["pre_weight_gradient"]),
                                       db=host(w["pre_bias_gradient"])), g, r["pre_x"],
                                  r["pre_weight"], r["pre_saved_mean"],
                                  r["pre_saved_inverse_std"])
        if "pre_conv_bias_gradient" in w:
            assert_within(host(w["pre_conv_bias_gradient"]), oracle.conv2d_bias_backward(dx),
                          1e-5 * np.abs(dx).astype(np.float64).sum(axis=(0, 2, 3)) + 1e-7,
                          f"{op.name} conv bias in front")
            self.counts["conv bias in batch norm backward"] += 1
        self.counts["batch norm before depthwise"] += 1

    def batch_norm2d_add_depthwise_conv2d_batch_norm_relu_forward(self, op, r):
        self._pre_forward(op, r, False, True)

    def batch_norm2d_add_depthwise_conv2d_batch_norm_forward(self, op, r):
        self._pre_forward(op, r, False, False)

    def batch_norm2d_add_depthwise_conv2d_batch_norm_relu_backward(self, op, r):
        self._pre_backward(op, r, False, True)

    def batch_norm2d_add_depthwise_conv2d_batch_norm_backward(self, op, r):
        self._pre_backward(op, r, False, False)

    def batch_norm2d_relu_depthwise_conv2d_batch_norm_relu_forward(self, op, r):
        self._pre_forward(op, r, True, True)

    def batch_norm2d_relu_depthwise_conv2d_batch_norm_forward(self, op, r):
        self._pre_forward(op, r, True, False)

    def batch_norm2d_depthwise_conv2d_batch_norm_relu_forward(self, op, r):
        self._pre_forward(op, r, False, True)

    def batch_norm2d_depthwise_conv2d_batch_norm_forward(self, op, r):
        self._pre_forward(op, r, False, False)

    def batch_norm2d_relu_depthwise_conv2d_batch_norm_relu_backward(self, op, r):
        self._pre_backward(op, r, True, True)

    def batch_norm2d_relu_depthwise_conv2d_batch_norm_backward(self, op, r):
        self._pre_backward(op, r, True, False)

    def batch_norm2d_depthwise_conv2d_batch_norm_relu_backward(self, op, r):
        self._pre_backward(op, r, False, True)

    def batch_norm2d_depthwise_conv2d_batch_norm_backward(self, op, r):
        self._pre_backward(op, r, False, False)

    def depthwise_conv2d_batch_norm_backward(self, op, r):
        self._depthwise_backward(op, r, False)

    def depthwise_conv2d_batch_norm_relu_backward(self, op, r):
        self._depthwise_backward(op, r, True)

    def relu_forward(self, op, r):
        assert_bitexact(host(op.writes["y"]), oracle.relu(r["x"]), op.name)

    def relu_backward(self, op, r):
        assert_bitexact(host(op.writes["contribution"]),
                        oracle.relu_backward(r["gradient"], r["x"]), op.name)

    def add_forward(self, op, r):
        assert_bitexact(host(op.writes["y"]), oracle.add(r["a"], r["b"]), op.name)

    def add_backward(self, op, r):
        assert_bitexact(host(op.writes["contribution"]), r["gradient"], op.name)

    def avg_pool2d_forward(self, op, r):
        a = op.attrs
        assert_bitexact(host(op.writes["y"]),
                        oracle.avg_pool2d_forward(r["x"], a["kernel"], a["stride"]), op.name)

    def avg_pool2d_backward(self, op, r):
        a = op.attrs
        assert_bitexact(host(op.writes["contribution"]),
                        oracle.avg_pool2d_backward(r["gradient"], op.writes["contribution"].shape,
                                                   a["kernel"], a["stride"]), op.name)

    def cross_entropy(self, op, r):
        logits, targets = r["logits"], r["targets"]
        outer = float(r["outer_gradient"][0])
        assert_close(host(op.writes["loss"]).astype(np.float32),
                     np.float32([oracle.ce_forward(logits, targets)]), what="loss")
        assert_close(host(op.writes["gradient"]), oracle.ce_backward(logits, targets, outer),
                     atol=1e-6 * abs(outer) / logits.shape[0], what="logit gradient")
        assert int(host(op.inplace[0])[0]) == 0

    def adamw(self, op, r):
        a = op.attrs
        step = int(host(a["step_counter"])[0])
        assert step == int(self.prior[id(a["step_counter"])][0]) + 1
        for i, (p, g, m, v) in enumerate(a["tensors"]):
            rp, rm, rv = oracle.adamw_update(self.prior[id(p)], host(g), self.prior[id(m)],
                                             self.prior[id(v)], step, a["learning_rate"],
                                             a["weight_decay"], a["beta1"], a["beta2"],
                                             a["epsilon"])
            assert_bitexact(host(p), rp, f"adamw parameter {i}")
            assert_bitexact(host(m), rm, f"adamw first moment {i}")
            assert_bitexact(host(v), rv, f"adamw second moment {i}")

    # -- kinds of general graphs (mul, reshape, non-root cross entropy, eval BatchNorm)
    def mul_forward(self, op, r):
        assert_bitexact(host(op.writes["y"]), oracle.mul(r["a"], r["b"]), op.name)

    def mul_backward(self, op, r):
        assert_bitexact(host(op.writes["contribution"]),
                        oracle.mul_backward(r["gradient"], r["other"]), op.name)

    def reshape_backward(self, op, r):
        assert_bitexact(host(op.writes["contribution"]).ravel(), r["gradient"].ravel(), op.name)

    def avg_pool2d_view_backward(self, op, r):  # a 1 x 1 window: the gradient passes unchanged
        assert_bitexact(host(op.writes["contribution"]), oracle.avg_pool2d_backward(
            r["gradient"], op.writes["contribution"].shape, (1, 1), (1, 1)), op.name)

    def seed(self, op, r):
        assert host(op.writes["gradient"]).ravel().tolist() == [1.0]

    def cross_entropy_forward(self, op, r):
        assert_close(host(op.writes["loss"]).astype(np.float32),
                     np.float32([oracle.ce_forward(r["logits"], r["targets"])]), what="loss")
        assert int(host(op.inplace[0])[0]) == 0

    def cross_entropy_backward(self, op, r):
        logits, outer = r["logits"], float(r["outer_gradient"].ravel()[0])
        assert_close(host(op.writes["contribution"]),
                     oracle.ce_backward(logits, r["targets"], outer),
                     atol=1e-6 * abs(outer) / logits.shape[0], what=op.name)

    def batch_norm2d_eval_forward(self, op, r):
        y, _, inv, _, _ = oracle.bn_forward(r["x"], r["weight"], r["bias"], r["running_mean"],
                                            r["running_variance"], False, 0.1,
                                            op.attrs["epsilon"])
        assert_bitexact(host(op.writes["inverse_std"]), inv, f"{op.name} inverse std")
        assert_bitexact(host(op.writes["y"]), y, f"{op.name} y")

    def batch_norm2d_eval_backward(self, op, r):
        """autograd.rs:340-381 in eval mode: dx = (g * w) * inv elementwise (bit-exact), the
        affine sums within 1e-5 * sum|terms| of the oracle's."""
        g, x, w = r["gradient"], r["x"], r["weight"]
        mean, inv = r["running_mean"], r["inverse_std"]
        dx, dw, db = oracle.bn_backward(g, x, w, mean, inv, False)
        if "contribution" in op.writes:
            assert_bitexact(host(op.writes["contribution"]), dx, f"{op.name} dx")
        c = x.shape[1]
        xhat = (x - mean.reshape(1, c, 1, 1)) * inv.reshape(1, c, 1, 1)
        assert_within(host(op.writes["weight_gradient"]), dw,
                      1e-5 * np.abs(g * xhat).astype(np.float64).sum(axis=(0, 2, 3)) + 1e-7,
                      f"{op.name} dweight")
        assert_within(host(op.writes["bias_gradient"]), db,
                      1e-5 * np.abs(g).astype(np.float64).sum(axis=(0, 2, 3)) + 1e-7,
                      f"{op.name} dbias")
