// net.hip -- the traced graph's builders, its forward and training programs, and their C ABI
// (oxh_net_*, oxh_program_*).  Host C++ over this library's own launchers.
//
// Reference: the lazy graph and its builders (crates/oxide-torch/src/tensor/graph.rs:70-139,
// tensor/mod.rs:103-389), the CUDA executor's eager evaluation (cuda/runtime.rs:125-379,
// 526-669) and reverse mode (1198-1217: collect_topological 1388-1476, propagate_node 694-860,
// accumulate_gradient 671-692, backward_batch_norm 1092-1156), and the optimizer step
// (optim.rs:78-152 with runtime.rs:1306-1386).
//
// Schedule of a training program.  Nodes are created in dependency order, so index order is
// topological.  Only the root's ancestors take part (the reference evaluates and walks only
// what the root reaches); a node needs a gradient when a trainable parameter or an input that
// requires one lies below it.  The forward runs in index order, the backward in reverse, so
// every consumer of a value has contributed to its gradient before the value's own backward
// runs.  A value's first contribution is written in place, later ones go to a scratch buffer
// and are added with oxh_accumulate.  Rewrites that cut launches without changing any value:
// a training BatchNorm whose only consumer is a ReLU runs as the fused BN + ReLU entry points
// (the ReLU mask is read from the ReLU output, positive exactly where its input is); a
// training BatchNorm that is a residual add's first operand and only feeds it writes BN(x) +
// addend in one pass; a depthwise convolution whose only consumer is the training BatchNorm
// created right after it runs with it (and its ReLU) as one launch per direction; a
// convolution whose only consumer is a training BatchNorm gets its bias gradient from that
// BatchNorm's backward (the per-channel sum of the dx it writes); an add's first operand with
// no other consumer shares the add's gradient buffer (the add's backward is the identity), and
// the gradient it hands its second operand is added by that operand's next contribution when
// that is a convolution's input backward, instead of being copied first.  A cross entropy that
// is the root gives loss and logit gradient in one fused launch (outer gradient 1).
#include <hip/hip_runtime.h>

#include <cmath>
#include <memory>

#include "net.h"

namespace oxh {
namespace net {

oxh_status Arena::allocate() {
  if (size == 0) return oxh::ok();
  OXH_HIP_CHECK(hipMalloc(reinterpret_cast<void **>(&base), size));
  OXH_HIP_CHECK(hipMemset(base, 0, size));
  return oxh::ok();
}

Arena::~Arena() {
  if (base) (void)hipFree(base);
}

oxh_status make_stream(hipStream_t &s) {
  OXH_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  return oxh::ok();
}

// ---------------------------------------------------------------- builders

namespace {

oxh_status node_index(const Graph &g, int i, const char *what) {
  OXH_REQUIRE(i >= 0 && static_cast<size_t>(i) < g.nodes.size(), OXH_INVALID_SHAPE,
              std::string(what) + ": node index out of range");
  return oxh::ok();
}

// checked_numel (tensor/shape.rs:13-24): no scalar shapes; ranks above 4 are not served here.
oxh_status set_shape(Node &n, uint32_t rank, const uint64_t *shape, const char *what) {
  OXH_REQUIRE(rank >= 1, OXH_INVALID_SHAPE, "scalar shapes are not implemented");
  OXH_REQUIRE(rank <= 4, OXH_INVALID_SHAPE, std::string(what) + ": rank above 4");
  OXH_REQUIRE(shape != nullptr, OXH_INVALID_SHAPE, std::string(what) + ": shape is null");
  uint64_t total = 1;
  for (uint32_t i = 0; i < rank; ++i) {
    OXH_REQUIRE(shape[i] == 0 || total <= (1ull << 62) / shape[i], OXH_INVALID_SHAPE,
                "element count overflow");
    total *= shape[i];
  }
  n.rank = rank;
  n.shape = {1, 1, 1, 1};
  for (uint32_t i = 0; i < rank; ++i) n.shape[i] = shape[i];
  return oxh::ok();
}

bool same_shape(const Node &a, const Node &b) {
  if (a.rank != b.rank) return false;
  for (uint32_t i = 0; i < a.rank; ++i)
    if (a.shape[i] != b.shape[i]) return false;
  return true;
}

}  // namespace

oxh_status input(Graph &g, uint32_t rank, const uint64_t *shape, bool requires_grad, int *node) {
  Node n{Op::Input, {}};
  oxh_status st = set_shape(n, rank, shape, "input");
  if (st != OXH_OK) return st;
  n.requires_grad = requires_grad;
  *node = g.add(n);
  return oxh::ok();
}

oxh_status leaf_values(Graph &g, uint32_t rank, const uint64_t *shape, float *values,
                       bool trainable, int *node) {
  Node n{trainable ? Op::Param : Op::Constant, {}};
  oxh_status st = set_shape(n, rank, shape, trainable ? "parameter" : "constant");
  if (st != OXH_OK) return st;
  OXH_REQUIRE(values != nullptr || n.numel() == 0, OXH_INVALID_SHAPE,
              "parameter / constant values are null");
  n.data = values;
  *node = g.add(n);
  if (trainable) g.params.push_back(*node);
  return oxh::ok();
}

// tensor/mod.rs:536-552: equal shapes, no broadcasting.
oxh_status binary(Graph &g, Op op, int a, int b, int *node) {
  oxh_status st = node_index(g, a, "binary op");
  if (st == OXH_OK) st = node_index(g, b, "binary op");
  if (st != OXH_OK) return st;
  const Node &x = g.nodes[a], &y = g.nodes[b];
  OXH_REQUIRE(same_shape(x, y), OXH_INVALID_SHAPE, "elementwise operands differ in shape");
  Node n{op, {a, b}};
  n.rank = x.rank;
  n.shape = x.shape;
  *node = g.add(n);
  return oxh::ok();
}

oxh_status relu(Graph &g, int x, int *node) {
  oxh_status st = node_index(g, x, "relu");
  if (st != OXH_OK) return st;
  Node n{Op::Relu, {x}};
  n.rank = g.nodes[x].rank;
  n.shape = g.nodes[x].shape;
  *node = g.add(n);
  return oxh::ok();
}

// tensor/mod.rs:293-301
oxh_status reshape(Graph &g, int x, uint32_t rank, const uint64_t *shape, int *node) {
  oxh_status st = node_index(g, x, "reshape");
  if (st != OXH_OK) return st;
  Node n{Op::Reshape, {x}};
  st = set_shape(n, rank, shape, "reshape");
  if (st != OXH_OK) return st;
  OXH_REQUIRE(n.numel() == g.nodes[x].numel(), OXH_INVALID_SHAPE,
              "reshape must preserve the element count");
  *node = g.add(n);
  return oxh::ok();
}

// tensor/mod.rs:158-237
oxh_status conv2d(Graph &g, int x, int weight, int bias, uint64_t stride, uint64_t padding,
                  uint64_t groups, int *node) {
  oxh_status st = node_index(g, x, "conv2d");
  if (st == OXH_OK) st = node_index(g, weight, "conv2d");
  if (st == OXH_OK) st = node_index(g, bias, "conv2d");
  if (st != OXH_OK) return st;
  const Node &in = g.nodes[x], &w = g.nodes[weight], &b = g.nodes[bias];
  OXH_REQUIRE(in.rank == 4 && w.rank == 4 && b.rank == 1, OXH_INVALID_SHAPE,
              "conv2d expects NCHW input, OIHW weight, and rank-1 bias");
  OXH_REQUIRE(stride != 0 && groups != 0, OXH_INVALID_SHAPE,
              "conv2d stride and groups must be non-zero");
  const uint64_t kh = w.shape[2], kw = w.shape[3];
  OXH_REQUIRE(kh != 0 && kw != 0 && kh == kw, OXH_INVALID_SHAPE,
              "conv2d currently requires a non-zero square kernel");
  OXH_REQUIRE(in.shape[1] % groups == 0 && w.shape[0] % groups == 0 &&
                  w.shape[1] == in.shape[1] / groups && b.shape[0] == w.shape[0],
              OXH_INVALID_SHAPE, "conv2d group/channel dimensions are inconsistent");
  OXH_REQUIRE(padding < (1ull << 31) && stride < (1ull << 31) && groups < (1ull << 31),
              OXH_INVALID_SHAPE, "conv2d argument too large");
  const uint64_t ph = in.shape[2] + 2 * padding, pw = in.shape[3] + 2 * padding;
  OXH_REQUIRE(ph >= kh && pw >= kw, OXH_INVALID_SHAPE, "conv2d kernel exceeds input");
  Node n{Op::Conv, {x, weight, bias}};
  n.stride = static_cast<uint32_t>(stride);
  n.pad = static_cast<uint32_t>(padding);
  n.groups = static_cast<uint32_t>(groups);
  n.shape = {in.shape[0], w.shape[0], (ph - kh) / stride + 1, (pw - kw) / stride + 1};
  *node = g.add(n);
  return oxh::ok();
}

// tensor/mod.rs:239-272
oxh_status avg_pool2d(Graph &g, int x, uint64_t kernel_h, uint64_t kernel_w, uint64_t stride_h,
                      uint64_t stride_w, int *node) {
  oxh_status st = node_index(g, x, "avg_pool2d");
  if (st != OXH_OK) return st;
  const Node &in = g.nodes[x];
  OXH_REQUIRE(in.rank == 4, OXH_INVALID_SHAPE, "avg_pool2d expects NCHW input");
  OXH_REQUIRE(kernel_h != 0 && kernel_w != 0 && stride_h != 0 && stride_w != 0,
              OXH_INVALID_SHAPE, "avg_pool2d kernel and stride must be non-zero");
  OXH_REQUIRE(kernel_h <= in.shape[2] && kernel_w <= in.shape[3], OXH_INVALID_SHAPE,
              "avg_pool2d kernel exceeds input");
  OXH_REQUIRE(stride_h < (1ull << 31) && stride_w < (1ull << 31), OXH_INVALID_SHAPE,
              "avg_pool2d stride too large");
  Node n{Op::Pool, {x}};
  n.kernel_h = static_cast<uint32_t>(kernel_h);
  n.kernel_w = static_cast<uint32_t>(kernel_w);
  n.stride_h = static_cast<uint32_t>(stride_h);
  n.stride_w = static_cast<uint32_t>(stride_w);
  n.shape = {in.shape[0], in.shape[1], (in.shape[2] - kernel_h) / stride_h + 1,
             (in.shape[3] - kernel_w) / stride_w + 1};
  *node = g.add(n);
  return oxh::ok();
}

// tensor/mod.rs:331-389
oxh_status batch_norm2d(Graph &g, int x, int weight, int bias, float *running_mean,
                        float *running_variance, bool training, float momentum, float epsilon,
                        int *node) {
  oxh_status st = node_index(g, x, "batch_norm2d");
  if (st == OXH_OK) st = node_index(g, weight, "batch_norm2d");
  if (st == OXH_OK) st = node_index(g, bias, "batch_norm2d");
  if (st != OXH_OK) return st;
  const Node &in = g.nodes[x], &w = g.nodes[weight], &b = g.nodes[bias];
  OXH_REQUIRE(in.rank == 4 && w.rank == 1 && b.rank == 1, OXH_INVALID_SHAPE,
              "batch_norm2d expects NCHW input and rank-1 weight/bias");
  OXH_REQUIRE(w.shape[0] == in.shape[1] && b.shape[0] == in.shape[1], OXH_INVALID_SHAPE,
              "batch_norm2d weight/bias must match the channel count");
  OXH_REQUIRE(std::isfinite(momentum) && momentum >= 0.0f && momentum <= 1.0f, OXH_EXECUTION,
              "batch_norm2d momentum must be finite and in 0..=1");
  OXH_REQUIRE(std::isfinite(epsilon) && epsilon > 0.0f, OXH_EXECUTION,
              "batch_norm2d epsilon must be positive and finite");
  OXH_REQUIRE(running_mean != nullptr && running_variance != nullptr, OXH_INVALID_SHAPE,
              "batch_norm2d running statistics are null");
  Node n{Op::Bn, {x, weight, bias}};
  n.shape = in.shape;
  n.running_mean = running_mean;
  n.running_variance = running_variance;
  n.training = training;
  n.momentum = momentum;
  n.epsilon = epsilon;
  *node = g.add(n);
  return oxh::ok();
}

// tensor/mod.rs:303-329
oxh_status cross_entropy(Graph &g, int logits, int targets, int *node) {
  oxh_status st = node_index(g, logits, "cross_entropy");
  if (st == OXH_OK) st = node_index(g, targets, "cross_entropy");
  if (st != OXH_OK) return st;
  const Node &l = g.nodes[logits], &t = g.nodes[targets];
  OXH_REQUIRE(l.rank == 2 && t.rank == 1 && l.shape[0] == t.shape[0], OXH_INVALID_SHAPE,
              "cross_entropy expects [batch, classes] logits and [batch] targets");
  Node n{Op::CrossEntropy, {logits, targets}};
  n.rank = 1;
  n.shape = {1, 1, 1, 1};
  *node = g.add(n);
  return oxh::ok();
}

// ---------------------------------------------------------------- program helpers

namespace {

TensorRef ref(const char *role, void *data, const Node &n, int access) {
  TensorRef t;
  t.role = role;
  t.data = data;
  t.shape = n.shape;
  t.rank = n.rank;
  t.access = access;
  return t;
}

TensorRef ref_flat(const char *role, void *data, uint64_t count, int access, int dtype = 0) {
  TensorRef t;
  t.role = role;
  t.data = data;
  t.shape = {count, 1, 1, 1};
  t.rank = 1;
  t.access = access;
  t.dtype = dtype;
  return t;
}

uint64_t node_bytes(const Node &n) { return n.numel() * 4; }

oxh_conv2d_shape conv_shape(const Graph &g, const Node &n) {
  const Node &x = g.nodes[n.in[0]], &w = g.nodes[n.in[1]];
  return oxh_conv2d_shape{x.shape[0], x.shape[1], x.shape[2], x.shape[3], n.shape[1],
                          w.shape[2], w.shape[3], n.stride, n.pad, n.groups};
}

oxh_pool2d_shape pool_shape(const Graph &g, const Node &n) {
  const Node &x = g.nodes[n.in[0]];
  return oxh_pool2d_shape{x.shape[0], x.shape[1], x.shape[2], x.shape[3],
                          n.kernel_h, n.kernel_w, n.stride_h, n.stride_w};
}

std::vector<std::pair<std::string, double>> conv_attrs(const Node &x) {
  return {{"stride", x.stride}, {"padding", x.pad}, {"groups", x.groups}};
}

std::vector<std::pair<std::string, double>> pool_attrs(const Node &x) {
  return {{"kernel_h", static_cast<double>(x.kernel_h)},
          {"kernel_w", static_cast<double>(x.kernel_w)},
          {"stride_h", static_cast<double>(x.stride_h)},
          {"stride_w", static_cast<double>(x.stride_w)}};
}

// A node whose values are its input's, so it shares the input's storage and launches nothing:
// a reshape (an alias, jit.rs:345) or an average pool with a 1 x 1 window that keeps every
// position (each output is one input value divided by 1, evaluation.rs:405-445; the CPU sum
// 0 + v turns -0 into +0, a difference the fp32 comparisons treat as none).  MobileNetV4's
// global pool of a 1 x 1 plane is one.
bool is_view(const Graph &g, const Node &x) {
  if (x.op == Op::Reshape) return true;
  if (x.op != Op::Pool || x.kernel_h != 1 || x.kernel_w != 1) return false;
  const Node &in = g.nodes[x.in[0]];
  return x.shape[2] == in.shape[2] && x.shape[3] == in.shape[3];
}

// The root's ancestors (collect_topological's reach, runtime.rs:1388-1476).
std::vector<char> ancestors(const Graph &g, int root) {
  std::vector<char> active(g.nodes.size(), 0);
  active[root] = 1;
  for (size_t r = static_cast<size_t>(root) + 1; r-- > 0;)
    if (active[r])
      for (int i : g.nodes[r].in) active[i] = 1;
  return active;
}

oxh_status plan_workspace(const Graph &g, const std::vector<char> &active, uint64_t &bytes) {
  bytes = 256;
  for (size_t i = 0; i < g.nodes.size(); ++i) {
    if (!active[i]) continue;
    const Node &n = g.nodes[i];
    uint64_t b = 0;
    oxh_status st = oxh::ok();
    if (n.op == Op::Bn) {
      st = oxh_batch_norm_workspace_size(n.shape[0], n.shape[1], n.shape[2] * n.shape[3], &b);
    } else if (n.op == Op::Conv) {
      const oxh_conv2d_shape s = conv_shape(g, n);
      st = oxh_conv2d_weight_backward_workspace_size(&s, &b);
    } else if (n.op == Op::CrossEntropy) {
      const Node &l = g.nodes[n.in[0]];
      st = oxh_cross_entropy_workspace_size(l.shape[0], l.shape[1], &b);
    }
    if (st != OXH_OK) return st;
    if (b > bytes) bytes = b;
  }
  return oxh::ok();
}

// Launch records of the forward ops both program kinds share.
OpRec conv_forward_op(const Graph &g, const std::vector<float *> &value, size_t i) {
  const Node &x = g.nodes[i];
  const oxh_conv2d_shape s = conv_shape(g, x);
  const float *xi = value[x.in[0]], *w = value[x.in[1]], *b = value[x.in[2]];
  float *out = value[i];
  OpRec op;
  op.kind = "conv2d_forward";
  op.name = "conv" + std::to_string(i);
  op.tensors = {ref("x", const_cast<float *>(xi), g.nodes[x.in[0]], 0),
                ref("weight", const_cast<float *>(w), g.nodes[x.in[1]], 0),
                ref("bias", const_cast<float *>(b), g.nodes[x.in[2]], 0), ref("y", out, x, 1)};
  op.attrs = conv_attrs(x);
  op.launch = [s, xi, w, b, out](hipStream_t st) {
    return oxh_conv2d_forward(st, &s, xi, w, b, out);
  };
  return op;
}

OpRec elementwise_forward_op(const Graph &g, const std::vector<float *> &value, size_t i) {
  const Node &x = g.nodes[i];
  float *out = value[i];
  const uint64_t cnt = x.numel();
  OpRec op;
  if (x.op == Op::Relu) {
    const float *xi = value[x.in[0]];
    op.kind = "relu_forward";
    op.name = "relu" + std::to_string(i);
    op.tensors = {ref("x", const_cast<float *>(xi), g.nodes[x.in[0]], 0), ref("y", out, x, 1)};
    op.launch = [xi, out, cnt](hipStream_t st) { return oxh_relu(st, xi, out, cnt); };
    return op;
  }
  const float *p = value[x.in[0]], *q = value[x.in[1]];
  const bool add = x.op == Op::Add;
  op.kind = add ? "add_forward" : "mul_forward";
  op.name = (add ? "add" : "mul") + std::to_string(i);
  op.tensors = {ref("a", const_cast<float *>(p), g.nodes[x.in[0]], 0),
                ref("b", const_cast<float *>(q), g.nodes[x.in[1]], 0), ref("y", out, x, 1)};
  op.launch = [p, q, out, cnt, add](hipStream_t st) {
    return add ? oxh_add(st, p, q, out, cnt) : oxh_mul(st, p, q, out, cnt);
  };
  return op;
}

OpRec pool_forward_op(const Graph &g, const std::vector<float *> &value, size_t i) {
  const Node &x = g.nodes[i];
  const oxh_pool2d_shape ps = pool_shape(g, x);
  const float *xi = value[x.in[0]];
  float *out = value[i];
  OpRec op;
  op.kind = "avg_pool2d_forward";
  op.name = "pool" + std::to_string(i);
  op.tensors = {ref("x", const_cast<float *>(xi), g.nodes[x.in[0]], 0), ref("y", out, x, 1)};
  op.attrs = pool_attrs(x);
  op.launch = [ps, xi, out](hipStream_t st) { return oxh_avg_pool2d_forward(st, &ps, xi, out); };
  return op;
}

// evaluation.rs:560-575, then the apply of 577-597: BatchNorm from the running statistics.
OpRec bn_eval_forward_op(const Graph &g, const std::vector<float *> &value, float *inv,
                         size_t i) {
  const Node &x = g.nodes[i];
  const float *xi = value[x.in[0]], *w = value[x.in[1]], *b = value[x.in[2]];
  float *out = value[i], *rm = x.running_mean, *rv = x.running_variance;
  const uint64_t N = x.shape[0], C = x.shape[1], HW = x.shape[2] * x.shape[3];
  const float eps = x.epsilon;
  OpRec op;
  op.kind = "batch_norm2d_eval_forward";
  op.name = "bn" + std::to_string(i);
  op.tensors = {ref("x", const_cast<float *>(xi), g.nodes[x.in[0]], 0),
                ref("weight", const_cast<float *>(w), g.nodes[x.in[1]], 0),
                ref("bias", const_cast<float *>(b), g.nodes[x.in[2]], 0),
                ref_flat("running_mean", rm, C, 0), ref_flat("running_variance", rv, C, 0),
                ref("y", out, x, 1), ref_flat("inverse_std", inv, C, 1)};
  op.attrs = {{"epsilon", eps}};
  op.launch = [=](hipStream_t st) {
    oxh_status r = oxh_batch_norm_running_inverse_std(st, C, eps, rv, inv);
    if (r != OXH_OK) return r;
    return oxh_batch_norm_apply(st, N, C, HW, xi, w, b, rm, inv, out);
  };
  return op;
}

}  // namespace

// ---------------------------------------------------------------- forward program

oxh_status build_forward(const Graph &g, int output, oxh_program &p) {
  const size_t n = g.nodes.size();
  OXH_REQUIRE(output >= 0 && static_cast<size_t>(output) < n, OXH_INVALID_SHAPE,
              "output node out of range");
  const std::vector<char> active = ancestors(g, output);
  Arena &a = p.arena;
  std::vector<int64_t> voff(n, -1), soff(n, -1), ioff(n, -1);
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (x.op == Op::Input) voff[i] = a.reserve(node_bytes(x));  // fed per run, even if unused
    if (!active[i] || x.leaf() || is_view(g, x)) continue;
    voff[i] = a.reserve(node_bytes(x));
    if (x.op == Op::Bn) {
      soff[i] = a.reserve(x.shape[1] * 4);
      ioff[i] = a.reserve(x.shape[1] * 4);
    }
  }
  const uint64_t flag_off = a.reserve(4);
  uint64_t ws_bytes = 0;
  oxh_status st = plan_workspace(g, active, ws_bytes);
  if (st != OXH_OK) return st;
  const uint64_t ws_off = a.reserve(ws_bytes);
  st = a.allocate();
  if (st != OXH_OK) return st;
  p.value.assign(n, nullptr);
  p.grad.assign(n, nullptr);
  p.saved_mean.assign(n, nullptr);
  p.saved_inv.assign(n, nullptr);
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (x.op == Op::Param || x.op == Op::Constant) p.value[i] = x.data;
    if (voff[i] >= 0) p.value[i] = a.at<float>(voff[i]);
    if (soff[i] >= 0) p.saved_mean[i] = a.at<float>(soff[i]);
    if (ioff[i] >= 0) p.saved_inv[i] = a.at<float>(ioff[i]);
    if (is_view(g, x)) p.value[i] = p.value[x.in[0]];
  }
  p.error_flag = a.at<uint32_t>(flag_off);
  p.root = output;
  void *ws = a.at<void>(ws_off);
  const uint64_t wsb = ws_bytes;
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (!active[i] || x.leaf() || is_view(g, x)) continue;
    switch (x.op) {
      case Op::Conv:
        p.ops.push_back(conv_forward_op(g, p.value, i));
        break;
      case Op::Relu:
      case Op::Add:
      case Op::Mul:
        p.ops.push_back(elementwise_forward_op(g, p.value, i));
        break;
      case Op::Pool:
        p.ops.push_back(pool_forward_op(g, p.value, i));
        break;
      case Op::Bn: {
        if (!x.training) {
          p.ops.push_back(bn_eval_forward_op(g, p.value, p.saved_inv[i], i));
          break;
        }
        // evaluation.rs:448-558: batch statistics, running update, apply
        const float *xi = p.value[x.in[0]], *w = p.value[x.in[1]], *b = p.value[x.in[2]];
        float *out = p.value[i], *sm = p.saved_mean[i], *si = p.saved_inv[i];
        float *rm = x.running_mean, *rv = x.running_variance;
        const uint64_t N = x.shape[0], C = x.shape[1], HW = x.shape[2] * x.shape[3];
        const float mom = x.momentum, eps = x.epsilon;
        OpRec op;
        op.kind = "batch_norm2d_forward";
        op.name = "bn" + std::to_string(i);
        op.tensors = {ref("x", const_cast<float *>(xi), g.nodes[x.in[0]], 0),
                      ref("weight", const_cast<float *>(w), g.nodes[x.in[1]], 0),
                      ref("bias", const_cast<float *>(b), g.nodes[x.in[2]], 0),
                      ref("y", out, x, 1), ref_flat("saved_mean", sm, C, 1),
                      ref_flat("saved_inverse_std", si, C, 1),
                      ref_flat("running_mean", rm, C, 2), ref_flat("running_variance", rv, C, 2)};
        op.attrs = {{"momentum", mom}, {"epsilon", eps}};
        op.launch = [=](hipStream_t st) {
          return oxh_batch_norm_forward_train(st, N, C, HW, mom, eps, xi, w, b, rm, rv, sm, si,
                                              out, ws, wsb);
        };
        p.ops.push_back(std::move(op));
        break;
      }
      case Op::CrossEntropy: {
        const Node &ln = g.nodes[x.in[0]];
        const float *lg = p.value[x.in[0]], *tg = p.value[x.in[1]];
        float *loss = p.value[i];
        uint32_t *flag = p.error_flag;
        const uint64_t rows = ln.shape[0], classes = ln.shape[1];
        OpRec op;
        op.kind = "cross_entropy_forward";
        op.name = "ce" + std::to_string(i);
        op.tensors = {ref("logits", const_cast<float *>(lg), ln, 0),
                      ref("targets", const_cast<float *>(tg), g.nodes[x.in[1]], 0),
                      ref("loss", loss, x, 1), ref_flat("error_flag", flag, 1, 2, 1)};
        op.launch = [=](hipStream_t st) {
          return oxh_cross_entropy_forward(st, rows, classes, lg, tg, loss, flag, ws, wsb);
        };
        p.ops.push_back(std::move(op));
        break;
      }
      default:
        return oxh::fail(OXH_TRACE, "no forward for a traced node");
    }
  }
  return p.finalize();
}

// ---------------------------------------------------------------- training program

oxh_status build_training(const Graph &g, int root, const AdamConfig *adam, oxh_program &p) {
  const size_t n = g.nodes.size();
  OXH_REQUIRE(root >= 0 && static_cast<size_t>(root) < n, OXH_INVALID_SHAPE,
              "root node out of range");
  // tensor/mod.rs:399-404
  OXH_REQUIRE(g.nodes[root].numel() == 1, OXH_EXECUTION,
              "backward requires a scalar loss tensor");
  if (adam != nullptr) {  // optim.rs:54-65
    OXH_REQUIRE(std::isfinite(adam->learning_rate) && adam->learning_rate > 0.0f,
                OXH_EXECUTION, "AdamW learning rate must be positive and finite");
    OXH_REQUIRE(std::isfinite(adam->weight_decay) && adam->weight_decay >= 0.0f,
                OXH_EXECUTION, "AdamW weight decay must be non-negative and finite");
    OXH_REQUIRE(std::isfinite(adam->beta1) && std::isfinite(adam->beta2) &&
                    std::isfinite(adam->epsilon),
                OXH_INVALID_SHAPE, "AdamW betas and epsilon must be finite");
  }
  const std::vector<char> active = ancestors(g, root);

  // which values need a gradient: a trainable parameter or an input requiring one below them
  std::vector<char> needs(n, 0);
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (x.op == Op::Param) needs[i] = 1;
    else if (x.op == Op::Input) needs[i] = x.requires_grad ? 1 : 0;
    else if (x.op == Op::CrossEntropy) needs[i] = needs[x.in[0]];  // targets take none
    else
      for (int k : x.in) needs[i] = needs[i] || needs[k];
  }
  auto want = [&](int i) { return active[i] && needs[i]; };

  // consumers among the participating nodes
  std::vector<int> consumers(n, 0);
  for (size_t i = 0; i < n; ++i)
    if (active[i])
      for (int k : g.nodes[i].in) ++consumers[k];
  auto train_bn = [&](int i) { return g.nodes[i].op == Op::Bn && g.nodes[i].training; };

  // fused BN + ReLU pairs
  std::vector<char> fused_bn(n, 0), fused_relu(n, 0);
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (active[i] && x.op == Op::Relu && train_bn(x.in[0]) && consumers[x.in[0]] == 1) {
      fused_relu[i] = 1;
      fused_bn[x.in[0]] = 1;
    }
  }
  // a training BN (without ReLU) whose only consumer is a residual add, as the add's first
  // operand: one launch at the add's place writes the add's output (BN + addend), and the BN
  // launches nothing of its own
  std::vector<int64_t> bn_into_add(n, -1);
  std::vector<char> add_absorbed(n, 0);
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (!active[i] || x.op != Op::Add) continue;
    const int first = x.in[0];
    if (train_bn(first) && !fused_bn[first] && consumers[first] == 1 && x.in[1] != first) {
      bn_into_add[first] = static_cast<int64_t>(i);
      add_absorbed[i] = 1;
    }
  }
  // a depthwise convolution whose only consumer is the training BatchNorm created next
  // (leaves aside), on planes the one-launch depthwise ConvNormAct kernels take: the pair runs
  // as one launch per direction, at the BN's place in each pass (no launch lies between the
  // two in either order, so every gradient contribution keeps its order)
  std::vector<char> dw_conv(n, 0);
  std::vector<int64_t> dw_conv_of(n, -1);  // BN node -> its fused depthwise convolution
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (!active[i] || x.op != Op::Conv || consumers[i] != 1) continue;
    size_t j = i + 1;
    while (j < n && g.nodes[j].leaf()) ++j;
    if (j == n || !active[j] || !train_bn(static_cast<int>(j)) ||
        g.nodes[j].in[0] != static_cast<int>(i) || bn_into_add[j] >= 0)
      continue;
    if (x.groups != g.nodes[x.in[0]].shape[1] || x.groups != x.shape[1]) continue;
    const oxh_conv2d_shape s = conv_shape(g, x);
    if (!oxh_depthwise_conv_batch_norm_supported(&s)) continue;
    dw_conv[i] = 1;
    dw_conv_of[j] = static_cast<int64_t>(i);
  }
  // a training BatchNorm (+ ReLU) whose only consumer is such a fused depthwise convolution,
  // on planes of at most 2048 values per channel: it runs inside that layer's launches (its
  // statistics, output and backward per channel, in the same workgroup as the layer's channel);
  // in either pass nothing reads its output or writes its inputs in between
  // The layer's input may be the BN's output, its ReLU's, or a residual add's whose first
  // operand is the BN (BN + add as one pass); other consumers of that input must come after the
  // layer, so that in the backward their gradient contributions are in place (written, or
  // waiting as an add's) when the fused launch adds them to the layer's input gradient.
  std::vector<int64_t> first_consumer(n, -1);
  for (size_t i = 0; i < n; ++i)
    if (active[i])
      for (int k : g.nodes[i].in)
        if (first_consumer[k] < 0) first_consumer[k] = static_cast<int64_t>(i);
  std::vector<int64_t> pre_bn_of(n, -1);  // fused depthwise convolution -> BN in front
  std::vector<char> pre_fused(n, 0);      // that BN and its ReLU: no launch of their own
  for (size_t i = 0; i < n; ++i) {
    if (!dw_conv[i]) continue;
    const int cin = g.nodes[i].in[0];
    if (first_consumer[cin] != static_cast<int64_t>(i)) continue;
    int b1 = -1;
    if (fused_relu[cin])
      b1 = g.nodes[cin].in[0];
    else if (train_bn(cin) && !fused_bn[cin] && bn_into_add[cin] < 0 && dw_conv_of[cin] < 0)
      b1 = cin;
    else if (g.nodes[cin].op == Op::Add && add_absorbed[cin])
      b1 = g.nodes[cin].in[0];
    if (b1 < 0 || dw_conv_of[b1] >= 0) continue;
    const oxh_conv2d_shape s = conv_shape(g, g.nodes[i]);
    if (!oxh_batch_norm_depthwise_conv_batch_norm_supported(&s)) continue;
    pre_bn_of[i] = b1;
    pre_fused[b1] = 1;
    if (g.nodes[cin].op != Op::Add) pre_fused[cin] = 1;  // an add keeps its backward
  }
  // gradient buffers, consumers before producers
  std::vector<int64_t> grad_of(n, -1);  // node whose grad buffer this node uses (-1: own)
  std::vector<char> has_grad(n, 0);
  std::vector<char> aliased(n, 0);      // an add's first operand using the add's buffer
  std::vector<char> view_alias(n, 0);  // a view (is_view) whose input uses its buffer
  const bool root_fused_ce =
      g.nodes[root].op == Op::CrossEntropy && want(g.nodes[root].in[0]);
  for (size_t r = n; r-- > 0;) {
    const Node &x = g.nodes[r];
    if (!want(static_cast<int>(r)) || fused_bn[r] || pre_fused[r]) continue;
    if (static_cast<int>(r) == root && root_fused_ce) continue;  // its outer gradient is 1
    if (x.op == Op::Param) continue;  // its gradient buffer is the optimizer's
    has_grad[r] = 1;
    if (is_view(g, x)) {
      const int in = x.in[0];
      if (!g.nodes[in].leaf() && consumers[in] == 1 && want(in)) {
        grad_of[in] = grad_of[r] >= 0 ? grad_of[r] : static_cast<int64_t>(r);
        view_alias[r] = 1;
      }
    } else if (x.op == Op::Add) {
      const int first = x.in[0];
      if (!g.nodes[first].leaf() && consumers[first] == 1 && grad_of[first] < 0 && want(first)) {
        grad_of[first] = grad_of[r] >= 0 ? grad_of[r] : static_cast<int64_t>(r);
        aliased[first] = 1;
      }
    }
  }

  // ---- plan the arena
  Arena &a = p.arena;
  std::vector<int64_t> voff(n, -1), goff(n, -1), smoff(n, -1), sioff(n, -1);
  uint64_t largest = 1;
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (active[i] && x.leaf()) largest = std::max(largest, x.numel());  // scratch accumulates
    if (x.op == Op::Input) {
      voff[i] = a.reserve(node_bytes(x));  // fed per run, even if unused
      continue;
    }
    if (!active[i]) continue;
    if (x.op == Op::Bn) {  // saved statistics, also for a BN fused with its ReLU
      smoff[i] = a.reserve(x.shape[1] * 4);
      sioff[i] = a.reserve(x.shape[1] * 4);
    }
    if (x.leaf() || is_view(g, x) || fused_bn[i]) continue;
    voff[i] = a.reserve(node_bytes(x));
    if (x.op != Op::CrossEntropy) largest = std::max(largest, x.numel());
  }
  for (size_t i = 0; i < n; ++i)
    if (has_grad[i] && grad_of[i] < 0) goff[i] = a.reserve(node_bytes(g.nodes[i]));
  // trainable parameters that receive a gradient (the optimizer skips the others,
  // runtime.rs:1330-1332)
  std::vector<int> trained;
  for (int pn : g.params)
    if (active[pn]) trained.push_back(pn);
  std::vector<std::array<int64_t, 3>> poff(trained.size());
  for (size_t k = 0; k < trained.size(); ++k) {
    const uint64_t bytes = node_bytes(g.nodes[trained[k]]);
    poff[k] = {static_cast<int64_t>(a.reserve(bytes)),
               adam ? static_cast<int64_t>(a.reserve(bytes)) : -1,
               adam ? static_cast<int64_t>(a.reserve(bytes)) : -1};
  }
  const uint64_t scratch_off = a.reserve(largest * 4), one_off = a.reserve(4),
                 step_off = a.reserve(4), flag_off = a.reserve(4);
  const uint64_t table_off = a.reserve(std::max<size_t>(trained.size(), 1) *
                                       sizeof(oxh_adamw_tensor));
  const uint64_t starts_off = a.reserve((trained.size() + 1) * 4);
  // A BatchNorm backward forms dx, dweight and dbias together (and a fused depthwise layer
  // its convolution's gradients too): those a value without a gradient does not take go to
  // one of kDiscardSlots discard buffers, handed out in turn (distinct within one launch).
  constexpr int kDiscardSlots = 6;
  bool discards = false;
  for (size_t i = 0; i < n; ++i)
    if (want(static_cast<int>(i)) && (g.nodes[i].op == Op::Bn || dw_conv[i]))
      for (int k : g.nodes[i].in) discards = discards || !want(k);
  const uint64_t discard_off = a.reserve(discards ? kDiscardSlots * largest * 4 : 4);
  // A gradient a launch forms beside its main contribution (a convolution's or BatchNorm's
  // parameters) whose node already holds a contribution (a value feeding several layers) goes
  // to one of kSideSlots side buffers and is added into the node's gradient after the launch.
  constexpr size_t kSideSlots = 8;
  bool sides = false;
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (!active[i] || (x.op != Op::Conv && x.op != Op::Bn)) continue;
    for (size_t k = 1; k < x.in.size(); ++k)
      sides = sides || (want(x.in[k]) && consumers[x.in[k]] > 1);
  }
  const uint64_t side_off = a.reserve(sides ? kSideSlots * largest * 4 : 4);
  uint64_t ws_bytes = 0;
  oxh_status st = plan_workspace(g, active, ws_bytes);
  if (st != OXH_OK) return st;
  const uint64_t ws_off = a.reserve(ws_bytes);
  // A convolution whose parameters feed it alone takes a workspace of its own when the program
  // ends with AdamW: its weight-gradient chunk partials then stay put until the optimizer
  // group, which sums every such convolution's in one launch (with the step counter advance).
  std::vector<int64_t> defer_off(n, -1);
  std::vector<uint64_t> defer_bytes(n, 0);
  if (adam != nullptr) {
    for (size_t i = 0; i < n; ++i) {
      const Node &x = g.nodes[i];
      if (!active[i] || x.op != Op::Conv || !want(x.in[1])) continue;
      bool alone = true;  // trainable parameters read by this convolution only
      for (size_t k = 1; k < x.in.size(); ++k)
        alone = alone && g.nodes[x.in[k]].op == Op::Param && consumers[x.in[k]] == 1;
      const oxh_conv2d_shape cs = conv_shape(g, x);
      uint64_t b = 0;
      st = oxh_conv2d_weight_backward_workspace_size(&cs, &b);
      if (st != OXH_OK) return st;
      if (!alone || b == 0) continue;
      defer_off[i] = static_cast<int64_t>(a.reserve(b));
      defer_bytes[i] = b;
    }
  }
  st = a.allocate();  // zero-filled: moments, step counter, error flag start at 0
  if (st != OXH_OK) return st;

  p.value.assign(n, nullptr);
  p.grad.assign(n, nullptr);
  p.saved_mean.assign(n, nullptr);
  p.saved_inv.assign(n, nullptr);
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (x.op == Op::Param || x.op == Op::Constant) p.value[i] = x.data;
    if (voff[i] >= 0) p.value[i] = a.at<float>(voff[i]);
    if (smoff[i] >= 0) p.saved_mean[i] = a.at<float>(smoff[i]);
    if (sioff[i] >= 0) p.saved_inv[i] = a.at<float>(sioff[i]);
    if (goff[i] >= 0) p.grad[i] = a.at<float>(goff[i]);
  }
  for (size_t i = 0; i < n; ++i)
    if (is_view(g, g.nodes[i])) p.value[i] = p.value[g.nodes[i].in[0]];
  for (size_t i = 0; i < n; ++i)
    if (grad_of[i] >= 0) p.grad[i] = p.grad[grad_of[i]];
  std::vector<float *> pm(n, nullptr), pv(n, nullptr);
  for (size_t k = 0; k < trained.size(); ++k) {
    p.grad[trained[k]] = a.at<float>(poff[k][0]);
    if (adam) {
      pm[trained[k]] = a.at<float>(poff[k][1]);
      pv[trained[k]] = a.at<float>(poff[k][2]);
    }
  }
  float *scratch = a.at<float>(scratch_off), *discard = a.at<float>(discard_off);
  float *side_base = a.at<float>(side_off);
  int discard_next = 0;
  bool discard_unplanned = false;  // a discard the arena did not plan for (a scheduling bug)
  bool side_unplanned = false;     // likewise for a side buffer
  float *one = a.at<float>(one_off);
  p.step = a.at<int32_t>(step_off);
  p.error_flag = a.at<uint32_t>(flag_off);
  p.adam_table = a.at<oxh_adamw_tensor>(table_off);
  p.adam_starts = a.at<uint32_t>(starts_off);
  p.root = root;
  oxh_program *self = &p;
  void *ws = a.at<void>(ws_off);
  const uint64_t wsb = ws_bytes;
  const float one_value = 1.0f;
  OXH_HIP_CHECK(hipMemcpy(one, &one_value, 4, hipMemcpyHostToDevice));

  // ---- schedule
  auto &ops = p.ops;
  auto name = [](const char *prefix, size_t i) { return std::string(prefix) + std::to_string(i); };
  std::vector<char> written(n, 0);
  std::vector<char> conv_bias_done(n, 0);  // conv nodes whose bias gradient a BN backward forms
  // A residual add's gradient handed to its non-aliased operand waits here and is added by
  // that operand's next contribution in the same pass (a convolution's input backward) rather
  // than copied into its buffer first; anything else flushes it as the copy.
  struct Pending {
    const float *gradient = nullptr;
    std::string name;
    int add = -1;
  };
  std::vector<Pending> pending(n);
  auto flush = [&](int x) {
    if (pending[x].gradient == nullptr) return;
    const Pending pe = pending[x];
    pending[x] = Pending{};
    written[x] = 1;
    float *dst = p.grad[x];
    const uint64_t bytes = node_bytes(g.nodes[x]);
    OpRec c;
    c.kind = "add_backward";
    c.name = pe.name;
    c.tensors = {ref("gradient", const_cast<float *>(pe.gradient), g.nodes[pe.add], 0),
                 ref("contribution", dst, g.nodes[x], 1)};
    const float *gr = pe.gradient;
    c.launch = [dst, gr, bytes](hipStream_t st) {
      return oxh_memcpy_d2d_async(dst, gr, bytes, st);
    };
    ops.push_back(std::move(c));
  };
  // Where a contribution to node x's gradient goes: its buffer (first) or the scratch buffer
  // added into it afterwards; a value that needs no gradient takes it into the discard buffer.
  auto contribution = [&](int x, float *&dst, float *&acc) {
    if (!want(x)) {
      discard_unplanned = discard_unplanned || !discards;
      dst = discard + static_cast<uint64_t>(discard_next) * largest;
      discard_next = (discard_next + 1) % kDiscardSlots;
      acc = nullptr;
      return;
    }
    flush(x);
    if (!written[x]) {
      written[x] = 1;
      dst = p.grad[x];
      acc = nullptr;
    } else {
      dst = scratch;
      acc = p.grad[x];
    }
  };
  // A side contribution to node x (role: the launch's output it is): in place when it is the
  // node's first, else into the next side buffer, added after the launch by attach_sides.
  struct SideAdd {
    float *into, *part;
    uint64_t count;
    std::string role;
    int node;
  };
  std::vector<SideAdd> side_adds;
  auto side = [&](int x, float *&dst, const char *role) {
    float *acc;
    contribution(x, dst, acc);
    if (acc == nullptr) return;
    if (!sides || side_adds.size() >= kSideSlots) {
      side_unplanned = true;
      return;
    }
    dst = side_base + side_adds.size() * largest;
    side_adds.push_back(SideAdd{acc, dst, g.nodes[x].numel(), role, x});
  };
  auto attach_sides = [&](OpRec &op) {
    if (side_adds.empty()) return;
    op.program_launch = nullptr;  // a side add reads its part right after the launch
    std::vector<SideAdd> adds;
    adds.swap(side_adds);
    for (const SideAdd &sa : adds)
      op.tensors.push_back(ref(("accumulate_into:" + sa.role).c_str(), sa.into,
                               g.nodes[sa.node], 2));
    auto body = std::move(op.launch);
    op.launch = [body, adds](hipStream_t st) {
      oxh_status e = body(st);
      for (const SideAdd &sa : adds) {
        if (e != OXH_OK) return e;
        e = oxh_accumulate(st, sa.into, sa.part, sa.into, sa.count);
      }
      return e;
    };
  };
  // program_body: set for a group the whole program runs another way (OpRec::program_launch)
  auto emit = [&](OpRec op, float *acc, const Node &target,
                  std::function<oxh_status(hipStream_t)> body,
                  std::function<oxh_status(hipStream_t)> program_body = nullptr) {
    using Body = std::function<oxh_status(hipStream_t)>;
    auto then_accumulate = [&](Body b) -> Body {
      if (acc == nullptr || !b) return b;
      float *part = scratch;
      const uint64_t cnt = target.numel();
      return [b, acc, part, cnt](hipStream_t s) {
        oxh_status e = b(s);
        if (e != OXH_OK) return e;
        return oxh_accumulate(s, acc, part, acc, cnt);
      };
    };
    if (acc != nullptr) op.tensors.push_back(ref("accumulate_into", acc, target, 2));
    op.launch = then_accumulate(std::move(body));
    op.program_launch = then_accumulate(std::move(program_body));
    attach_sides(op);
    ops.push_back(std::move(op));
  };
  // a copy contribution: d2d copy of `gradient` (the backward of an identity)
  auto copy_contribution = [&](const char *kind, const std::string &cname, const float *gr,
                               const Node &from, int target) {
    float *dst, *acc;
    contribution(target, dst, acc);
    const uint64_t bytes = node_bytes(g.nodes[target]);
    OpRec c;
    c.kind = kind;
    c.name = cname;
    c.tensors = {ref("gradient", const_cast<float *>(gr), from, 0),
                 ref("contribution", dst, g.nodes[target], 1)};
    emit(std::move(c), acc, g.nodes[target], [dst, gr, bytes](hipStream_t st) {
      return oxh_memcpy_d2d_async(dst, gr, bytes, st);
    });
  };

  // forward
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (!active[i] || x.leaf() || is_view(g, x) || fused_bn[i] || dw_conv[i] || pre_fused[i])
      continue;
    // a BatchNorm absorbed by its residual add launches at the add's place, where the addend
    // (possibly created after the BatchNorm) has been written; one whose add feeds a fused
    // depthwise layer launches inside that layer
    if (x.op == Op::Bn && bn_into_add[i] >= 0) continue;
    if (add_absorbed[i] && pre_fused[x.in[0]]) continue;
    float *out = p.value[i];
    OpRec op;
    switch (x.op) {
      case Op::Conv:
        ops.push_back(conv_forward_op(g, p.value, i));
        break;
      case Op::Add:
        if (add_absorbed[i]) {  // BN + residual add in one launch
          const int bi = x.in[0];
          const Node &bn = g.nodes[bi];
          const float *xi = p.value[bn.in[0]], *w = p.value[bn.in[1]], *b = p.value[bn.in[2]];
          const float *skip = p.value[x.in[1]];
          float *sm = p.saved_mean[bi], *si = p.saved_inv[bi];
          float *rm = bn.running_mean, *rv = bn.running_variance;
          const uint64_t N = bn.shape[0], C = bn.shape[1], HW = bn.shape[2] * bn.shape[3];
          const float mom = bn.momentum, eps = bn.epsilon;
          op.kind = "batch_norm2d_add_forward";
          op.name = name("bn", bi) + "+" + name("add", i);
          op.tensors = {ref("x", const_cast<float *>(xi), g.nodes[bn.in[0]], 0),
                        ref("weight", const_cast<float *>(w), g.nodes[bn.in[1]], 0),
                        ref("bias", const_cast<float *>(b), g.nodes[bn.in[2]], 0),
                        ref("addend", const_cast<float *>(skip), g.nodes[x.in[1]], 0),
                        ref("y", out, x, 1), ref_flat("saved_mean", sm, C, 1),
                        ref_flat("saved_inverse_std", si, C, 1),
                        ref_flat("running_mean", rm, C, 2), ref_flat("running_variance", rv, C, 2)};
          op.attrs = {{"momentum", mom}, {"epsilon", eps}};
          op.launch = [=](hipStream_t st) {
            return oxh_batch_norm_add_forward_train(st, N, C, HW, mom, eps, xi, w, b, rm, rv, sm,
                                                    si, skip, out, ws, wsb);
          };
          ops.push_back(std::move(op));
          break;
        }
        [[fallthrough]];
      case Op::Mul:
        ops.push_back(elementwise_forward_op(g, p.value, i));
        break;
      case Op::Relu:
        if (!fused_relu[i]) {
          ops.push_back(elementwise_forward_op(g, p.value, i));
          break;
        }
        [[fallthrough]];
      case Op::Bn: {
        const bool fused = x.op == Op::Relu;
        const int bi = fused ? x.in[0] : static_cast<int>(i);
        const Node &bn = g.nodes[bi];
        if (!bn.training) {
          ops.push_back(bn_eval_forward_op(g, p.value, p.saved_inv[bi], bi));
          break;
        }
        const float *xi = p.value[bn.in[0]], *w = p.value[bn.in[1]], *b = p.value[bn.in[2]];
        float *sm = p.saved_mean[bi], *si = p.saved_inv[bi];
        float *rm = bn.running_mean, *rv = bn.running_variance;
        const uint64_t N = bn.shape[0], C = bn.shape[1], HW = bn.shape[2] * bn.shape[3];
        const float mom = bn.momentum, eps = bn.epsilon;
        if (dw_conv_of[bi] >= 0) {  // depthwise conv + BN (+ ReLU) in one launch
          const int ci = static_cast<int>(dw_conv_of[bi]);
          const Node &cv = g.nodes[ci];
          const oxh_conv2d_shape s = conv_shape(g, cv);
          const float *cx = p.value[cv.in[0]], *cw = p.value[cv.in[1]], *cb = p.value[cv.in[2]];
          float *cy = p.value[ci];
          op.kind = fused ? "depthwise_conv2d_batch_norm_relu_forward"
                          : "depthwise_conv2d_batch_norm_forward";
          op.name = name("conv", ci) + "+" + name("bn", bi) + (fused ? "+" + name("relu", i) : "");
          op.tensors = {ref("x", const_cast<float *>(cx), g.nodes[cv.in[0]], 0),
                        ref("conv_weight", const_cast<float *>(cw), g.nodes[cv.in[1]], 0),
                        ref("conv_bias", const_cast<float *>(cb), g.nodes[cv.in[2]], 0),
                        ref("weight", const_cast<float *>(w), g.nodes[bn.in[1]], 0),
                        ref("bias", const_cast<float *>(b), g.nodes[bn.in[2]], 0),
                        ref("conv_y", cy, cv, 1), ref("y", out, x, 1),
                        ref_flat("saved_mean", sm, C, 1), ref_flat("saved_inverse_std", si, C, 1),
                        ref_flat("running_mean", rm, C, 2), ref_flat("running_variance", rv, C, 2)};
          op.attrs = conv_attrs(cv);
          op.attrs.push_back({"momentum", mom});
          op.attrs.push_back({"epsilon", eps});
          if (pre_bn_of[ci] >= 0) {  // the BN (+ ReLU) in front, inside the same launch
            const int b1 = static_cast<int>(pre_bn_of[ci]);
            const Node &pb = g.nodes[b1];
            const Node &pin = g.nodes[cv.in[0]];
            const bool padd = pin.op == Op::Add;  // BN + residual add in front
            const bool prelu = cv.in[0] != b1 && !padd;
            const float *px = p.value[pb.in[0]], *pw = p.value[pb.in[1]],
                        *pbb = p.value[pb.in[2]];
            const float *pres = padd ? p.value[pin.in[1]] : nullptr;
            float *psm = p.saved_mean[b1], *psi = p.saved_inv[b1];
            float *prm = pb.running_mean, *prv = pb.running_variance;
            float *py = const_cast<float *>(cx);
            const float pmom = pb.momentum, peps = pb.epsilon;
            const uint64_t PC = pb.shape[1];
            op.kind = std::string(prelu ? "batch_norm2d_relu_" : padd ? "batch_norm2d_add_"
                                                                       : "batch_norm2d_") +
                      (fused ? "depthwise_conv2d_batch_norm_relu_forward"
                             : "depthwise_conv2d_batch_norm_forward");
            op.name = (prelu  ? name("bn", b1) + "+" + name("relu", cv.in[0])
                       : padd ? name("bn", b1) + "+" + name("add", cv.in[0])
                              : name("bn", b1)) +
                      "+" + op.name;
            op.tensors.erase(op.tensors.begin());  // the layer's input is pre_y, written here
            op.tensors.push_back(ref("pre_x", const_cast<float *>(px), g.nodes[pb.in[0]], 0));
            op.tensors.push_back(ref("pre_weight", const_cast<float *>(pw), g.nodes[pb.in[1]], 0));
            op.tensors.push_back(ref("pre_bias", const_cast<float *>(pbb), g.nodes[pb.in[2]], 0));
            if (padd)
              op.tensors.push_back(ref("pre_residual", const_cast<float *>(pres),
                                       g.nodes[pin.in[1]], 0));
            op.tensors.push_back(ref("pre_y", py, g.nodes[cv.in[0]], 1));
            op.tensors.push_back(ref_flat("pre_saved_mean", psm, PC, 1));
            op.tensors.push_back(ref_flat("pre_saved_inverse_std", psi, PC, 1));
            op.tensors.push_back(ref_flat("pre_running_mean", prm, PC, 2));
            op.tensors.push_back(ref_flat("pre_running_variance", prv, PC, 2));
            op.attrs.push_back({"pre_momentum", pmom});
            op.attrs.push_back({"pre_epsilon", peps});
            op.launch = [=](hipStream_t st) {
              return oxh_batch_norm_depthwise_conv_batch_norm_forward_train(
                  st, &s, prelu ? 1 : 0, pmom, peps, px, pw, pbb, pres, prm, prv, psm, psi, py,
                  fused ? 1 : 0, mom, eps, cw, cb, cy, w, b, rm, rv, sm, si, out);
            };
            ops.push_back(std::move(op));
            break;
          }
          op.launch = [=](hipStream_t st) {
            return oxh_depthwise_conv_batch_norm_forward_train(st, &s, fused ? 1 : 0, mom, eps,
                                                               cx, cw, cb, cy, w, b, rm, rv, sm,
                                                               si, out);
          };
          ops.push_back(std::move(op));
          break;
        }
        op.kind = fused ? "batch_norm2d_relu_forward" : "batch_norm2d_forward";
        op.name = fused ? name("bn", bi) + "+" + name("relu", i) : name("bn", bi);
        op.tensors = {ref("x", const_cast<float *>(xi), g.nodes[bn.in[0]], 0),
                      ref("weight", const_cast<float *>(w), g.nodes[bn.in[1]], 0),
                      ref("bias", const_cast<float *>(b), g.nodes[bn.in[2]], 0),
                      ref("y", out, x, 1), ref_flat("saved_mean", sm, C, 1),
                      ref_flat("saved_inverse_std", si, C, 1), ref_flat("running_mean", rm, C, 2),
                      ref_flat("running_variance", rv, C, 2)};
        op.attrs = {{"momentum", mom}, {"epsilon", eps}};
        op.launch = [=](hipStream_t st) {
          return fused ? oxh_batch_norm_relu_forward_train(st, N, C, HW, mom, eps, xi, w, b, rm,
                                                           rv, sm, si, out, ws, wsb)
                       : oxh_batch_norm_forward_train(st, N, C, HW, mom, eps, xi, w, b, rm, rv,
                                                      sm, si, out, ws, wsb);
        };
        ops.push_back(std::move(op));
        break;
      }
      case Op::Pool:
        ops.push_back(pool_forward_op(g, p.value, i));
        break;
      case Op::CrossEntropy: {
        const Node &ln = g.nodes[x.in[0]];
        const float *lg = p.value[x.in[0]], *tg = p.value[x.in[1]];
        const uint64_t rows = ln.shape[0], classes = ln.shape[1];
        uint32_t *flag = p.error_flag;
        if (static_cast<int>(i) == root && root_fused_ce) {
          // the root: loss and logit gradient in one pass, outer gradient 1
          float *dl = nullptr, *acc = nullptr;
          contribution(x.in[0], dl, acc);
          op.kind = "cross_entropy";
          op.name = name("ce", i);
          op.tensors = {ref("logits", const_cast<float *>(lg), ln, 0),
                        ref("targets", const_cast<float *>(tg), g.nodes[x.in[1]], 0),
                        ref_flat("outer_gradient", one, 1, 0), ref("loss", out, x, 1),
                        ref("gradient", dl, ln, 1), ref_flat("error_flag", flag, 1, 2, 1)};
          op.launch = [=](hipStream_t st) {
            return oxh_cross_entropy_forward_backward(st, rows, classes, lg, tg, one, out, dl,
                                                      flag, ws, wsb);
          };
        } else {
          op.kind = "cross_entropy_forward";
          op.name = name("ce", i);
          op.tensors = {ref("logits", const_cast<float *>(lg), ln, 0),
                        ref("targets", const_cast<float *>(tg), g.nodes[x.in[1]], 0),
                        ref("loss", out, x, 1), ref_flat("error_flag", flag, 1, 2, 1)};
          op.launch = [=](hipStream_t st) {
            return oxh_cross_entropy_forward(st, rows, classes, lg, tg, out, flag, ws, wsb);
          };
        }
        ops.push_back(std::move(op));
        break;
      }
      default:
        return oxh::fail(OXH_TRACE, "no forward for a traced node");
    }
  }

  // the root's own gradient: 1 (runtime.rs:1207-1209), unless the fused cross entropy used it
  if (want(root) && !root_fused_ce) {
    float *dst, *acc;
    contribution(root, dst, acc);
    OpRec c;
    c.kind = "seed";
    c.name = "seed" + std::to_string(root);
    c.tensors = {ref_flat("one", one, 1, 0), ref("gradient", dst, g.nodes[root], 1)};
    c.launch = [dst, one](hipStream_t st) { return oxh_memcpy_d2d_async(dst, one, 4, st); };
    ops.push_back(std::move(c));
  }

  // backward, reverse topological order
  for (size_t r = n; r-- > 0;) {
    const Node &x = g.nodes[r];
    if (!want(static_cast<int>(r)) || x.leaf() || fused_bn[r] || pre_fused[r]) continue;
    if (x.op == Op::CrossEntropy && static_cast<int>(r) == root && root_fused_ce) continue;
    flush(static_cast<int>(r));  // a gradient still waiting for a second contribution
    OXH_REQUIRE(written[r], OXH_TRACE, "a traced value receives no gradient");
    const float *gr = p.grad[r];
    OpRec op;
    if (is_view(g, x)) {
      if (view_alias[r]) {
        written[x.in[0]] = 1;  // shares this gradient buffer
      } else {
        const bool reshape = x.op == Op::Reshape;
        copy_contribution(reshape ? "reshape_backward" : "avg_pool2d_view_backward",
                          name(reshape ? "reshape" : "pool", r) + ".backward", gr, x, x.in[0]);
      }
      continue;
    }
    switch (x.op) {
      case Op::CrossEntropy: {  // autograd.rs:529-554 with the node's gradient as outer
        const Node &ln = g.nodes[x.in[0]];
        const float *lg = p.value[x.in[0]], *tg = p.value[x.in[1]];
        const uint64_t rows = ln.shape[0], classes = ln.shape[1];
        uint32_t *flag = p.error_flag;
        float *dst, *acc;
        contribution(x.in[0], dst, acc);
        op.kind = "cross_entropy_backward";
        op.name = name("ce", r) + ".backward";
        op.tensors = {ref("logits", const_cast<float *>(lg), ln, 0),
                      ref("targets", const_cast<float *>(tg), g.nodes[x.in[1]], 0),
                      ref("outer_gradient", const_cast<float *>(gr), x, 0),
                      ref("contribution", dst, ln, 1), ref_flat("error_flag", flag, 1, 2, 1)};
        emit(std::move(op), acc, ln, [=](hipStream_t st) {
          return oxh_cross_entropy_backward(st, rows, classes, lg, tg, gr, dst, flag);
        });
        break;
      }
      case Op::Mul: {  // autograd.rs:123-138: d left = g * right, d right = g * left
        for (int k = 0; k < 2; ++k) {
          const int inp = x.in[k];
          if (!want(inp)) continue;
          const float *other = p.value[x.in[1 - k]];
          float *dst, *acc;
          contribution(inp, dst, acc);
          const uint64_t cnt = x.numel();
          OpRec c;
          c.kind = "mul_backward";
          c.name = name("mul", r) + ".backward" + std::to_string(k);
          c.tensors = {ref("gradient", const_cast<float *>(gr), x, 0),
                       ref("other", const_cast<float *>(other), g.nodes[x.in[1 - k]], 0),
                       ref("contribution", dst, g.nodes[inp], 1)};
          emit(std::move(c), acc, g.nodes[inp], [gr, other, dst, cnt](hipStream_t st) {
            return oxh_mul_backward(st, gr, other, dst, cnt);
          });
        }
        break;
      }
      case Op::Relu:
        if (!fused_relu[r]) {
          const int xin = x.in[0];
          const float *xi = p.value[xin];
          float *dst, *acc;
          contribution(xin, dst, acc);
          const uint64_t cnt = x.numel();
          op.kind = "relu_backward";
          op.name = name("relu", r) + ".backward";
          op.tensors = {ref("gradient", const_cast<float *>(gr), x, 0),
                        ref("x", const_cast<float *>(xi), g.nodes[xin], 0),
                        ref("contribution", dst, g.nodes[xin], 1)};
          emit(std::move(op), acc, g.nodes[xin], [gr, xi, dst, cnt](hipStream_t st) {
            return oxh_relu_backward(st, gr, xi, dst, cnt);
          });
          break;
        }
        [[fallthrough]];
      case Op::Bn: {
        const bool fused = x.op == Op::Relu;
        const int bi = fused ? x.in[0] : static_cast<int>(r);
        const Node &bn = g.nodes[bi];
        const int xin = bn.in[0];
        const float *xi = p.value[xin], *w = p.value[bn.in[1]];
        const float *y = fused ? p.value[r] : nullptr;
        const float *sm = p.saved_mean[bi], *si = p.saved_inv[bi];
        const uint64_t N = bn.shape[0], C = bn.shape[1], HW = bn.shape[2] * bn.shape[3];
        float *dg, *db, *dst, *acc;
        if (!bn.training) {  // autograd.rs:340-381 with running statistics
          const float *rm = bn.running_mean;
          side(bn.in[1], dg, "weight_gradient");
          side(bn.in[2], db, "bias_gradient");
          op.kind = "batch_norm2d_eval_backward";
          op.name = name("bn", bi) + ".backward";
          op.tensors = {ref("gradient", const_cast<float *>(gr), x, 0),
                        ref("x", const_cast<float *>(xi), g.nodes[xin], 0),
                        ref("weight", const_cast<float *>(w), g.nodes[bn.in[1]], 0),
                        ref_flat("running_mean", const_cast<float *>(rm), C, 0),
                        ref_flat("inverse_std", const_cast<float *>(si), C, 0),
                        ref_flat("weight_gradient", dg, C, 1), ref_flat("bias_gradient", db, C, 1)};
          const bool input_grad = want(xin);
          acc = nullptr;
          dst = nullptr;
          if (input_grad) {
            contribution(xin, dst, acc);
            op.tensors.push_back(ref("contribution", dst, g.nodes[xin], 1));
          }
          emit(std::move(op), acc, g.nodes[xin], [=](hipStream_t st) {
            oxh_status e = oxh_batch_norm_affine_backward(st, N, C, HW, gr, xi, rm, si, dg, db,
                                                          ws, wsb);
            if (e != OXH_OK || !input_grad) return e;
            return oxh_batch_norm_input_backward(st, N, C, HW, 0, gr, xi, w, rm, si, dg, db,
                                                 dst);
          });
          break;
        }
        if (dw_conv_of[bi] >= 0) {  // depthwise conv + BN (+ ReLU) backward in one launch
          const Node &cv = g.nodes[xin];
          const int cin = cv.in[0];
          float *cgr, *cdw, *cdb;
          side(bn.in[1], dg, "weight_gradient");
          side(bn.in[2], db, "bias_gradient");
          side(xin, cgr, "conv_output_gradient");  // the BN is its only consumer
          side(cv.in[2], cdb, "conv_bias_gradient");
          side(cv.in[1], cdw, "conv_weight_gradient");
          const oxh_conv2d_shape s = conv_shape(g, cv);
          const float *cx = p.value[cin], *cw = p.value[cv.in[1]];
          if (pre_bn_of[xin] >= 0) {  // with the BN (+ ReLU) in front, in the same launch
            const int b1 = static_cast<int>(pre_bn_of[xin]);
            const Node &pb = g.nodes[b1];
            const bool padd = g.nodes[cin].op == Op::Add;
            const bool prelu = cin != b1 && !padd;
            const int px_node = pb.in[0];
            // the layer input's other gradient contributions (its later consumers', already
            // made) are added to the layer's input gradient; an add in front keeps its node's
            // gradient (its second operand takes it)
            const float *addend = nullptr;
            if (pending[cin].gradient != nullptr && !written[cin]) {
              addend = pending[cin].gradient;
              op.tensors.push_back(ref("addend", const_cast<float *>(addend),
                                       g.nodes[pending[cin].add], 0));
              pending[cin] = Pending{};
            } else if (written[cin]) {
              addend = p.grad[cin];
              op.tensors.push_back(ref("addend", const_cast<float *>(addend), g.nodes[cin], 0));
            }
            float *cdx = nullptr;
            if (padd) {
              cdx = p.grad[cin];
              written[cin] = 1;
            }
            const float *px = p.value[px_node], *pw = p.value[pb.in[1]];
            const float *psm = p.saved_mean[b1], *psi = p.saved_inv[b1];
            const uint64_t PC = pb.shape[1];
            float *pdg, *pdb;
            side(pb.in[1], pdg, "pre_weight_gradient");
            side(pb.in[2], pdb, "pre_bias_gradient");
            contribution(px_node, dst, acc);
            // a convolution feeding only this BN: its bias gradient is the sum of this dx
            float *pconv_db = nullptr;
            const Node &src = g.nodes[px_node];
            if (src.op == Op::Conv && consumers[px_node] == 1 && acc == nullptr &&
                want(px_node) && want(src.in[2])) {
              side(src.in[2], pconv_db, "pre_conv_bias_gradient");
              conv_bias_done[px_node] = 1;
            }
            op.kind = std::string(prelu ? "batch_norm2d_relu_" : padd ? "batch_norm2d_add_"
                                                                       : "batch_norm2d_") +
                      (fused ? "depthwise_conv2d_batch_norm_relu_backward"
                             : "depthwise_conv2d_batch_norm_backward");
            op.name = (prelu  ? name("bn", b1) + "+" + name("relu", cin)
                       : padd ? name("bn", b1) + "+" + name("add", cin)
                              : name("bn", b1)) +
                      "+" + name("conv", xin) + "+" + name("bn", bi) +
                      (fused ? "+" + name("relu", r) : "") + ".backward";
            op.tensors.push_back(ref("gradient", const_cast<float *>(gr), x, 0));
            if (fused) op.tensors.push_back(ref("y", const_cast<float *>(y), x, 0));
            op.tensors.push_back(ref("conv_y", const_cast<float *>(xi), cv, 0));
            op.tensors.push_back(ref("weight", const_cast<float *>(w), g.nodes[bn.in[1]], 0));
            op.tensors.push_back(ref_flat("saved_mean", const_cast<float *>(sm), C, 0));
            op.tensors.push_back(ref_flat("saved_inverse_std", const_cast<float *>(si), C, 0));
            op.tensors.push_back(ref("x", const_cast<float *>(cx), g.nodes[cin], 0));
            op.tensors.push_back(ref("conv_weight", const_cast<float *>(cw), g.nodes[cv.in[1]], 0));
            op.tensors.push_back(ref("pre_x", const_cast<float *>(px), g.nodes[px_node], 0));
            op.tensors.push_back(ref("pre_weight", const_cast<float *>(pw), g.nodes[pb.in[1]], 0));
            op.tensors.push_back(ref_flat("pre_saved_mean", const_cast<float *>(psm), PC, 0));
            op.tensors.push_back(ref_flat("pre_saved_inverse_std", const_cast<float *>(psi), PC, 0));
            op.tensors.push_back(ref("conv_output_gradient", cgr, cv, 1));
            op.tensors.push_back(ref_flat("weight_gradient", dg, C, 1));
            op.tensors.push_back(ref_flat("bias_gradient", db, C, 1));
            op.tensors.push_back(ref("conv_bias_gradient", cdb, g.nodes[cv.in[2]], 1));
            op.tensors.push_back(ref("conv_weight_gradient", cdw, g.nodes[cv.in[1]], 1));
            op.tensors.push_back(ref_flat("pre_weight_gradient", pdg, PC, 1));
            op.tensors.push_back(ref_flat("pre_bias_gradient", pdb, PC, 1));
            if (pconv_db)
              op.tensors.push_back(ref_flat("pre_conv_bias_gradient", pconv_db, PC, 1));
            if (cdx)
              op.tensors.push_back(ref("conv_input_gradient", cdx, g.nodes[cin],
                                       addend == cdx ? 2 : 1));
            op.tensors.push_back(ref("contribution", dst, g.nodes[px_node], 1));
            op.attrs = conv_attrs(cv);
            emit(std::move(op), acc, g.nodes[px_node], [=](hipStream_t st) {
              return oxh_batch_norm_depthwise_conv_batch_norm_backward_train(
                  st, &s, gr, y, xi, w, sm, si, cx, cw, addend, prelu ? 1 : 0, px, pw, psm, psi,
                  cgr, dg, db, cdb, cdw, cdx, pdg, pdb, dst, pconv_db);
            });
            break;
          }
          const float *addend = nullptr;
          dst = nullptr;
          acc = nullptr;
          if (want(cin)) {  // e.g. the network input needs no gradient
            if (pending[cin].gradient != nullptr && !written[cin]) {
              addend = pending[cin].gradient;
              op.tensors.push_back(ref("addend", const_cast<float *>(addend),
                                       g.nodes[pending[cin].add], 0));
              pending[cin] = Pending{};
              written[cin] = 1;
              dst = p.grad[cin];
            } else {
              contribution(cin, dst, acc);
            }
          }
          op.kind = fused ? "depthwise_conv2d_batch_norm_relu_backward"
                          : "depthwise_conv2d_batch_norm_backward";
          op.name = name("conv", xin) + "+" + name("bn", bi) + (fused ? "+" + name("relu", r) : "") +
                    ".backward";
          op.tensors.push_back(ref("gradient", const_cast<float *>(gr), x, 0));
          if (fused) op.tensors.push_back(ref("y", const_cast<float *>(y), x, 0));
          op.tensors.push_back(ref("conv_y", const_cast<float *>(xi), cv, 0));
          op.tensors.push_back(ref("weight", const_cast<float *>(w), g.nodes[bn.in[1]], 0));
          op.tensors.push_back(ref_flat("saved_mean", const_cast<float *>(sm), C, 0));
          op.tensors.push_back(ref_flat("saved_inverse_std", const_cast<float *>(si), C, 0));
          op.tensors.push_back(ref("x", const_cast<float *>(cx), g.nodes[cin], 0));
          op.tensors.push_back(ref("conv_weight", const_cast<float *>(cw), g.nodes[cv.in[1]], 0));
          op.tensors.push_back(ref("conv_output_gradient", cgr, cv, 1));
          op.tensors.push_back(ref_flat("weight_gradient", dg, C, 1));
          op.tensors.push_back(ref_flat("bias_gradient", db, C, 1));
          op.tensors.push_back(ref("conv_bias_gradient", cdb, g.nodes[cv.in[2]], 1));
          op.tensors.push_back(ref("conv_weight_gradient", cdw, g.nodes[cv.in[1]], 1));
          if (dst != nullptr) op.tensors.push_back(ref("contribution", dst, g.nodes[cin], 1));
          op.attrs = conv_attrs(cv);
          emit(std::move(op), acc, g.nodes[cin], [=](hipStream_t st) {
            return oxh_depthwise_conv_batch_norm_backward_train(st, &s, gr, y, xi, w, sm, si, cx,
                                                                cw, addend, cgr, dg, db, cdb, cdw,
                                                                dst);
          });
          break;
        }
        side(bn.in[1], dg, "weight_gradient");
        side(bn.in[2], db, "bias_gradient");
        contribution(xin, dst, acc);
        // a convolution whose only consumer is this BN: its output gradient is this dx, whose
        // per-channel sum (the convolution's bias gradient) the BN backward forms in passing
        // when it runs one block per channel (else in two launches of its own: the
        // convolution's parameter backward forms it instead)
        float *conv_db = nullptr;
        const Node &src = g.nodes[xin];
        if (src.op == Op::Conv && consumers[xin] == 1 && acc == nullptr && want(xin) &&
            want(src.in[2]) && oxh::batch_norm_single_launch(N, C, HW)) {
          side(src.in[2], conv_db, "conv_bias_gradient");
          conv_bias_done[xin] = 1;
        }
        op.kind = fused ? "batch_norm2d_relu_backward" : "batch_norm2d_backward";
        op.name = (fused ? name("bn", bi) + "+" + name("relu", r) : name("bn", bi)) + ".backward";
        op.tensors = {ref("gradient", const_cast<float *>(gr), x, 0)};
        if (fused) op.tensors.push_back(ref("y", const_cast<float *>(y), x, 0));
        op.tensors.push_back(ref("x", const_cast<float *>(xi), g.nodes[xin], 0));
        op.tensors.push_back(ref("weight", const_cast<float *>(w), g.nodes[bn.in[1]], 0));
        op.tensors.push_back(ref_flat("saved_mean", const_cast<float *>(sm), C, 0));
        op.tensors.push_back(ref_flat("saved_inverse_std", const_cast<float *>(si), C, 0));
        op.tensors.push_back(ref("contribution", dst, g.nodes[xin], 1));
        op.tensors.push_back(ref_flat("weight_gradient", dg, C, 1));
        op.tensors.push_back(ref_flat("bias_gradient", db, C, 1));
        if (conv_db) op.tensors.push_back(ref_flat("conv_bias_gradient", conv_db, C, 1));
        emit(std::move(op), acc, g.nodes[xin], [=](hipStream_t st) {
          if (conv_db)
            return oxh_conv_batch_norm_backward_train(st, N, C, HW, gr, y, xi, w, sm, si, dst,
                                                      dg, db, conv_db, ws, wsb);
          return fused ? oxh_batch_norm_relu_backward_train(st, N, C, HW, gr, y, xi, w, sm, si,
                                                            dst, dg, db, ws, wsb)
                       : oxh_batch_norm_backward_train(st, N, C, HW, gr, xi, w, sm, si, dst, dg,
                                                       db, ws, wsb);
        });
        break;
      }
      case Op::Add: {  // autograd.rs:119-122: both operands take the gradient unchanged
        for (int k = 0; k < 2; ++k) {
          const int inp = x.in[k];
          if (!want(inp)) continue;
          if (k == 0 && aliased[inp]) {
            written[inp] = 1;  // the add's gradient buffer is its own
            continue;
          }
          const std::string cname = name("add", r) + ".backward" + std::to_string(k);
          if (!written[inp] && pending[inp].gradient == nullptr) {
            pending[inp] = Pending{gr, cname, static_cast<int>(r)};
            continue;
          }
          copy_contribution("add_backward", cname, gr, x, inp);
        }
        break;
      }
      case Op::Pool: {
        const Node &xin = g.nodes[x.in[0]];
        const oxh_pool2d_shape ps = pool_shape(g, x);
        float *dst, *acc;
        contribution(x.in[0], dst, acc);
        op.kind = "avg_pool2d_backward";
        op.name = name("pool", r) + ".backward";
        op.tensors = {ref("gradient", const_cast<float *>(gr), x, 0),
                      ref("contribution", dst, xin, 1)};
        op.attrs = pool_attrs(x);
        emit(std::move(op), acc, xin, [ps, gr, dst](hipStream_t st) {
          return oxh_avg_pool2d_backward(st, &ps, gr, dst);
        });
        break;
      }
      case Op::Conv: {
        if (dw_conv[r]) break;  // its backward ran with its BatchNorm's
        const oxh_conv2d_shape s = conv_shape(g, x);
        const int xin = x.in[0];
        const float *xi = p.value[xin], *w = p.value[x.in[1]];
        float *dw = nullptr, *db = nullptr;
        const bool weight_here = want(x.in[1]);
        if (weight_here) side(x.in[1], dw, "weight_gradient");
        const bool bias_here = !conv_bias_done[r] && want(x.in[2]);  // else the BN formed it
        if (bias_here) side(x.in[2], db, "bias_gradient");
        if (weight_here && want(xin)) {  // the whole VJP in one launch group
          float *dst, *acc;
          const float *addend = nullptr;
          if (pending[xin].gradient != nullptr && !written[xin]) {
            addend = pending[xin].gradient;
            op.tensors.push_back(ref("addend", const_cast<float *>(addend),
                                     g.nodes[pending[xin].add], 0));
            pending[xin] = Pending{};
            written[xin] = 1;
            dst = p.grad[xin];
            acc = nullptr;
          } else {
            contribution(xin, dst, acc);
          }
          op.kind = "conv2d_backward";
          op.name = name("conv", r) + ".backward";
          op.tensors.push_back(ref("gradient", const_cast<float *>(gr), x, 0));
          op.tensors.push_back(ref("x", const_cast<float *>(xi), g.nodes[xin], 0));
          op.tensors.push_back(ref("weight", const_cast<float *>(w), g.nodes[x.in[1]], 0));
          op.tensors.push_back(ref("weight_gradient", dw, g.nodes[x.in[1]], 1));
          if (bias_here) op.tensors.push_back(ref("bias_gradient", db, g.nodes[x.in[2]], 1));
          op.tensors.push_back(ref("contribution", dst, g.nodes[xin], 1));
          op.attrs = conv_attrs(x);
          std::function<oxh_status(hipStream_t)> deferred;
          if (defer_off[r] >= 0) {
            void *own = a.at<void>(static_cast<uint64_t>(defer_off[r]));
            const uint64_t own_bytes = defer_bytes[r];
            deferred = [s, gr, xi, w, addend, dst, dw, db, own, own_bytes, self](hipStream_t st) {
              return oxh::conv2d_backward_deferred(st, &s, gr, xi, w, addend, dst, dw, db, own,
                                                   own_bytes, self->deferred_sums);
            };
          }
          emit(std::move(op), acc, g.nodes[xin],
               [s, gr, xi, w, addend, dst, dw, db, ws, wsb](hipStream_t st) {
                 return oxh_conv2d_backward(st, &s, gr, xi, w, addend, dst, dw, db, ws, wsb);
               },
               std::move(deferred));
          break;
        }
        if (weight_here || bias_here) {
          OpRec pr;
          pr.kind = "conv2d_parameter_backward";
          pr.name = name("conv", r) + ".backward_parameters";
          pr.tensors = {ref("gradient", const_cast<float *>(gr), x, 0),
                        ref("x", const_cast<float *>(xi), g.nodes[xin], 0),
                        ref("weight", const_cast<float *>(w), g.nodes[x.in[1]], 0)};
          if (weight_here) pr.tensors.push_back(ref("weight_gradient", dw, g.nodes[x.in[1]], 1));
          if (bias_here) pr.tensors.push_back(ref("bias_gradient", db, g.nodes[x.in[2]], 1));
          pr.attrs = conv_attrs(x);
          pr.launch = [s, gr, xi, w, dw, db, ws, wsb](hipStream_t st) {
            // both: one parameter-only VJP (the bias summed with the weights where it can be)
            if (dw != nullptr && db != nullptr)
              return oxh_conv2d_backward(st, &s, gr, xi, w, nullptr, nullptr, dw, db, ws, wsb);
            if (dw != nullptr) return oxh_conv2d_weight_backward(st, &s, gr, xi, dw, ws, wsb);
            return oxh_conv2d_bias_backward(st, &s, gr, db, ws, wsb);
          };
          if (defer_off[r] >= 0 && dw != nullptr) {  // the same launches, sums left to AdamW
            void *own = a.at<void>(static_cast<uint64_t>(defer_off[r]));
            const uint64_t own_bytes = defer_bytes[r];
            pr.program_launch = [s, gr, xi, w, dw, db, own, own_bytes, self](hipStream_t st) {
              return oxh::conv2d_backward_deferred(st, &s, gr, xi, w, nullptr, nullptr, dw, db,
                                                   own, own_bytes, self->deferred_sums);
            };
          }
          attach_sides(pr);
          ops.push_back(std::move(pr));
        }
        if (!want(xin)) break;  // e.g. the network input needs no gradient
        float *dst, *acc;
        const float *addend = nullptr;
        if (pending[xin].gradient != nullptr && !written[xin]) {
          addend = pending[xin].gradient;
          op.tensors.push_back(ref("addend", const_cast<float *>(addend),
                                   g.nodes[pending[xin].add], 0));
          pending[xin] = Pending{};
          written[xin] = 1;
          dst = p.grad[xin];
          acc = nullptr;
        } else {
          contribution(xin, dst, acc);
        }
        op.kind = "conv2d_input_backward";
        op.name = name("conv", r) + ".backward_input";
        op.tensors.push_back(ref("gradient", const_cast<float *>(gr), x, 0));
        op.tensors.push_back(ref("x", const_cast<float *>(xi), g.nodes[xin], 0));
        op.tensors.push_back(ref("weight", const_cast<float *>(w), g.nodes[x.in[1]], 0));
        op.tensors.push_back(ref("contribution", dst, g.nodes[xin], 1));
        op.attrs = conv_attrs(x);
        emit(std::move(op), acc, g.nodes[xin], [s, gr, w, addend, dst](hipStream_t st) {
          return addend ? oxh_conv2d_input_backward_accumulate(st, &s, gr, w, addend, dst)
                        : oxh_conv2d_input_backward(st, &s, gr, w, dst);
        });
        break;
      }
      default:
        return oxh::fail(OXH_TRACE, "no backward for a traced node");
    }
  }
  for (size_t i = 0; i < n; ++i) flush(static_cast<int>(i));
  OXH_REQUIRE(!discard_unplanned, OXH_EXECUTION, "internal: unplanned gradient discard");
  OXH_REQUIRE(!side_unplanned && side_adds.empty(), OXH_EXECUTION,
              "internal: unplanned side contribution");

  // AdamW over every parameter that received a gradient (creation order)
  if (adam != nullptr && !trained.empty()) {
    p.has_adam = true;
    p.adam_config = *adam;
    p.adam.clear();
    OpRec op;
    op.kind = "adamw";
    op.name = "adamw";
    for (int pn : trained) {
      const Node &pr = g.nodes[pn];
      p.adam.push_back(oxh_adamw_tensor{pr.data, p.grad[pn], pm[pn], pv[pn], pr.numel()});
      op.tensors.push_back(ref_flat("parameter", pr.data, pr.numel(), 2));
      op.tensors.push_back(ref_flat("gradient", p.grad[pn], pr.numel(), 0));
      op.tensors.push_back(ref_flat("first_moment", pm[pn], pr.numel(), 2));
      op.tensors.push_back(ref_flat("second_moment", pv[pn], pr.numel(), 2));
    }
    op.tensors.push_back(ref_flat("step", p.step, 1, 2, 1));
    op.attrs = {{"learning_rate", adam->learning_rate}, {"weight_decay", adam->weight_decay},
                {"beta1", adam->beta1}, {"beta2", adam->beta2}, {"epsilon", adam->epsilon}};
    const uint32_t count = static_cast<uint32_t>(p.adam.size());
    std::vector<uint32_t> starts(count + 1);
    st = oxh_adamw_table_layout(p.adam.data(), count, starts.data(), &p.adam_chunks);
    if (st != OXH_OK) return st;
    OXH_HIP_CHECK(hipMemcpy(p.adam_table, p.adam.data(), count * sizeof(oxh_adamw_tensor),
                            hipMemcpyHostToDevice));
    OXH_HIP_CHECK(hipMemcpy(p.adam_starts, starts.data(), (count + 1) * 4,
                            hipMemcpyHostToDevice));
    op.launch = [self](hipStream_t s) {
      const AdamConfig &c = self->adam_config;
      return oxh_adamw_multi_tensor_table_step(
          s, c.learning_rate, c.weight_decay, c.beta1, c.beta2, c.epsilon, self->step,
          self->adam_table, self->adam_starts,
          static_cast<uint32_t>(self->adam.size()), self->adam_chunks);
    };
    bool deferring = false;
    for (const OpRec &o : ops) deferring = deferring || static_cast<bool>(o.program_launch);
    if (deferring)  // the convolutions' chunk sums and the step advance in one launch first
      op.program_launch = [self](hipStream_t s) {
        oxh_status e = oxh::launch_chunk_sums(s, self->deferred_sums, self->step);
        if (e != OXH_OK) return e;
        const AdamConfig &c = self->adam_config;
        return oxh::adamw_table_step_advanced(
            s, c.learning_rate, c.weight_decay, c.beta1, c.beta2, c.epsilon, self->step,
            self->adam_table, self->adam_starts, static_cast<uint32_t>(self->adam.size()),
            self->adam_chunks);
      };
    ops.push_back(std::move(op));
  }
  return p.finalize();
}

}  // namespace net
}  // namespace oxh

// ---------------------------------------------------------------- oxh_program

oxh_status oxh_program::finalize() {
  for (const oxh::net::OpRec &op : ops)
    for (const oxh::net::TensorRef &t : op.tensors)
      OXH_REQUIRE(t.data != nullptr, OXH_EXECUTION,
                  "internal: " + op.name + " has no buffer for " + t.role);
  for (oxh::net::OpRec &op : ops) {
    op.c_tensors.clear();
    for (const oxh::net::TensorRef &t : op.tensors) {
      oxh_op_tensor c{};
      c.role = t.role.c_str();
      c.data = t.data;
      c.rank = t.rank;
      for (int i = 0; i < 4; ++i) c.shape[i] = t.shape[i];
      c.access = t.access;
      c.dtype = t.dtype;
      op.c_tensors.push_back(c);
    }
    op.c_attrs.clear();
    for (const auto &a : op.attrs) op.c_attrs.push_back(oxh_op_attr{a.first.c_str(), a.second});
  }
  return oxh::ok();
}

oxh_status oxh_program::run() {
  deferred_sums.clear();
  for (oxh::net::OpRec &op : ops) {
    oxh_status st = op.program_launch ? op.program_launch(stream) : op.launch(stream);
    if (st != OXH_OK) return st;
  }
  return oxh::ok();
}

oxh_status oxh_program::capture() {
  if (graph) {
    (void)oxh_graph_destroy(graph);
    graph = nullptr;
  }
  oxh_status st = oxh_graph_begin(stream);
  if (st != OXH_OK) return st;
  st = run();
  if (st != OXH_OK) {
    const std::string msg = oxh_last_error();
    (void)oxh_graph_abort(stream);
    return oxh::fail(OXH_EXECUTION, "graph recording failed: " + msg);
  }
  return oxh_graph_end(stream, &graph);
}

oxh_program::~oxh_program() {
  if (stream) (void)hipStreamSynchronize(stream);
  if (graph) (void)oxh_graph_destroy(graph);
  if (stream) (void)hipStreamDestroy(stream);
}

// ---------------------------------------------------------------- C ABI

struct oxh_net {
  oxh::net::Graph graph;
};

namespace {

oxh_status out_node(int index, uint32_t *node) {
  *node = static_cast<uint32_t>(index);
  return oxh::ok();
}

int as_index(uint32_t node) {
  return node > 0x7FFFFFFFu ? -1 : static_cast<int>(node);
}

oxh_status make_program(const oxh_net *net, uint32_t node, bool training,
                        const oxh_adamw_config *adamw, oxh_program **program) {
  OXH_REQUIRE(net != nullptr && program != nullptr, OXH_INVALID_SHAPE, "null argument");
  *program = nullptr;
  std::unique_ptr<oxh_program> p(new oxh_program());
  p->owned = true;
  oxh::net::AdamConfig cfg;
  if (adamw != nullptr)
    cfg = oxh::net::AdamConfig{adamw->learning_rate, adamw->weight_decay, adamw->beta1,
                               adamw->beta2, adamw->epsilon};
  oxh_status st = training ? oxh::net::build_training(net->graph, as_index(node),
                                                      adamw != nullptr ? &cfg : nullptr, *p)
                           : oxh::net::build_forward(net->graph, as_index(node), *p);
  if (st == OXH_OK) st = oxh::net::make_stream(p->stream);
  if (st != OXH_OK) return st;
  *program = p.release();
  return oxh::ok();
}

}  // namespace

extern "C" {

oxh_status oxh_net_create(oxh_net **net) {
  OXH_REQUIRE(net != nullptr, OXH_INVALID_SHAPE, "net out-pointer is null");
  *net = new oxh_net();
  return oxh::ok();
}

oxh_status oxh_net_destroy(oxh_net *net) {
  delete net;
  return OXH_OK;
}

oxh_status oxh_net_node_count(const oxh_net *net, uint32_t *count) {
  OXH_REQUIRE(net != nullptr && count != nullptr, OXH_INVALID_SHAPE, "null argument");
  *count = static_cast<uint32_t>(net->graph.nodes.size());
  return oxh::ok();
}

oxh_status oxh_net_node_shape(const oxh_net *net, uint32_t node, uint32_t *rank,
                              uint64_t shape[4]) {
  OXH_REQUIRE(net != nullptr && rank != nullptr && shape != nullptr, OXH_INVALID_SHAPE,
              "null argument");
  OXH_REQUIRE(node < net->graph.nodes.size(), OXH_INVALID_SHAPE, "node index out of range");
  const oxh::net::Node &x = net->graph.nodes[node];
  *rank = x.rank;
  for (int i = 0; i < 4; ++i) shape[i] = x.shape[i];
  return oxh::ok();
}

#define OXH_NET_BUILD(call)                                                    \
  do {                                                                         \
    OXH_REQUIRE(net != nullptr && node != nullptr, OXH_INVALID_SHAPE, "null argument"); \
    int index = -1;                                                            \
    oxh_status st_ = (call);                                                   \
    if (st_ != OXH_OK) return st_;                                             \
    return out_node(index, node);                                              \
  } while (0)

oxh_status oxh_net_input(oxh_net *net, uint32_t rank, const uint64_t *shape, int requires_grad,
                         uint32_t *node) {
  OXH_NET_BUILD(oxh::net::input(net->graph, rank, shape, requires_grad != 0, &index));
}

oxh_status oxh_net_parameter(oxh_net *net, uint32_t rank, const uint64_t *shape, float *values,
                             uint32_t *node) {
  OXH_NET_BUILD(oxh::net::leaf_values(net->graph, rank, shape, values, true, &index));
}

oxh_status oxh_net_constant(oxh_net *net, uint32_t rank, const uint64_t *shape,
                            const float *values, uint32_t *node) {
  OXH_NET_BUILD(oxh::net::leaf_values(net->graph, rank, shape, const_cast<float *>(values),
                                      false, &index));
}

oxh_status oxh_net_add(oxh_net *net, uint32_t a, uint32_t b, uint32_t *node) {
  OXH_NET_BUILD(oxh::net::binary(net->graph, oxh::net::Op::Add, as_index(a), as_index(b), &index));
}

oxh_status oxh_net_mul(oxh_net *net, uint32_t a, uint32_t b, uint32_t *node) {
  OXH_NET_BUILD(oxh::net::binary(net->graph, oxh::net::Op::Mul, as_index(a), as_index(b), &index));
}

oxh_status oxh_net_relu(oxh_net *net, uint32_t x, uint32_t *node) {
  OXH_NET_BUILD(oxh::net::relu(net->graph, as_index(x), &index));
}

oxh_status oxh_net_reshape(oxh_net *net, uint32_t x, uint32_t rank, const uint64_t *shape,
                           uint32_t *node) {
  OXH_NET_BUILD(oxh::net::reshape(net->graph, as_index(x), rank, shape, &index));
}

oxh_status oxh_net_conv2d(oxh_net *net, uint32_t x, uint32_t weight, uint32_t bias,
                          uint64_t stride, uint64_t padding, uint64_t groups, uint32_t *node) {
  OXH_NET_BUILD(oxh::net::conv2d(net->graph, as_index(x), as_index(weight), as_index(bias),
                                 stride, padding, groups, &index));
}

oxh_status oxh_net_avg_pool2d(oxh_net *net, uint32_t x, uint64_t kernel_h, uint64_t kernel_w,
                              uint64_t stride_h, uint64_t stride_w, uint32_t *node) {
  OXH_NET_BUILD(oxh::net::avg_pool2d(net->graph, as_index(x), kernel_h, kernel_w, stride_h,
                                     stride_w, &index));
}

oxh_status oxh_net_batch_norm2d(oxh_net *net, uint32_t x, uint32_t weight, uint32_t bias,
                                float *running_mean, float *running_variance, int training,
                                float momentum, float epsilon, uint32_t *node) {
  OXH_NET_BUILD(oxh::net::batch_norm2d(net->graph, as_index(x), as_index(weight),
                                       as_index(bias), running_mean, running_variance,
                                       training != 0, momentum, epsilon, &index));
}

oxh_status oxh_net_cross_entropy(oxh_net *net, uint32_t logits, uint32_t targets,
                                 uint32_t *node) {
  OXH_NET_BUILD(oxh::net::cross_entropy(net->graph, as_index(logits), as_index(targets), &index));
}

#undef OXH_NET_BUILD

oxh_status oxh_net_forward_program(const oxh_net *net, uint32_t output, oxh_program **program) {
  return make_program(net, output, false, nullptr, program);
}

oxh_status oxh_net_training_program(const oxh_net *net, uint32_t root,
                                    const oxh_adamw_config *adamw, oxh_program **program) {
  return make_program(net, root, true, adamw, program);
}

oxh_status oxh_program_destroy(oxh_program *program) {
  if (program == nullptr) return oxh::ok();
  OXH_REQUIRE(program->owned, OXH_INVALID_SHAPE,
              "the program belongs to its trainer or evaluator");
  delete program;
  return oxh::ok();
}

oxh_status oxh_program_value(const oxh_program *p, uint32_t node, float **device) {
  OXH_REQUIRE(p != nullptr && device != nullptr, OXH_INVALID_SHAPE, "null argument");
  OXH_REQUIRE(node < p->value.size(), OXH_INVALID_SHAPE, "node index out of range");
  OXH_REQUIRE(p->value[node] != nullptr, OXH_TRACE, "the program holds no value for the node");
  *device = p->value[node];
  return oxh::ok();
}

oxh_status oxh_program_gradient(const oxh_program *p, uint32_t node, float **device) {
  OXH_REQUIRE(p != nullptr && device != nullptr, OXH_INVALID_SHAPE, "null argument");
  OXH_REQUIRE(node < p->grad.size(), OXH_INVALID_SHAPE, "node index out of range");
  *device = p->grad[node];  // null: the node receives no gradient
  return oxh::ok();
}

oxh_status oxh_program_check(oxh_program *p) {
  OXH_REQUIRE(p != nullptr, OXH_INVALID_SHAPE, "program is null");
  OXH_HIP_CHECK(hipStreamSynchronize(p->stream));
  if (p->error_flag == nullptr) return oxh::ok();
  uint32_t flag = 0;
  OXH_HIP_CHECK(hipMemcpy(&flag, p->error_flag, 4, hipMemcpyDeviceToHost));
  if (flag != 0) {
    OXH_HIP_CHECK(hipMemset(p->error_flag, 0, 4));
    return oxh::fail(OXH_INVALID_SHAPE, "cross entropy target is not a class index");
  }
  return oxh::ok();
}

oxh_status oxh_program_steps(oxh_program *p, int32_t *steps) {
  OXH_REQUIRE(p != nullptr && steps != nullptr, OXH_INVALID_SHAPE, "null argument");
  OXH_HIP_CHECK(hipStreamSynchronize(p->stream));
  *steps = 0;
  if (p->step != nullptr) OXH_HIP_CHECK(hipMemcpy(steps, p->step, 4, hipMemcpyDeviceToHost));
  return oxh::ok();
}

oxh_status oxh_program_stream(const oxh_program *p, oxh_stream *stream) {
  OXH_REQUIRE(p != nullptr && stream != nullptr, OXH_INVALID_SHAPE, "null argument");
  *stream = p->stream;
  return oxh::ok();
}

oxh_status oxh_program_run(oxh_program *p) {
  OXH_REQUIRE(p != nullptr, OXH_INVALID_SHAPE, "program is null");
  return p->run();
}

oxh_status oxh_program_capture(oxh_program *p) {
  OXH_REQUIRE(p != nullptr, OXH_INVALID_SHAPE, "program is null");
  return p->capture();
}

oxh_status oxh_program_replay(oxh_program *p) {
  OXH_REQUIRE(p != nullptr, OXH_INVALID_SHAPE, "program is null");
  OXH_REQUIRE(p->graph != nullptr, OXH_EXECUTION, "no captured program; capture first");
  return oxh_graph_launch(p->graph, p->stream);
}

oxh_status oxh_program_op_count(const oxh_program *p, uint64_t *count) {
  OXH_REQUIRE(p != nullptr && count != nullptr, OXH_INVALID_SHAPE, "null argument");
  *count = p->ops.size();
  return oxh::ok();
}

oxh_status oxh_program_op(const oxh_program *p, uint64_t index, oxh_op_info *info) {
  OXH_REQUIRE(p != nullptr && info != nullptr, OXH_INVALID_SHAPE, "null argument");
  OXH_REQUIRE(index < p->ops.size(), OXH_INVALID_SHAPE, "op index out of range");
  const oxh::net::OpRec &op = p->ops[index];
  info->kind = op.kind.c_str();
  info->name = op.name.c_str();
  info->tensor_count = static_cast<uint32_t>(op.c_tensors.size());
  info->tensors = op.c_tensors.data();
  info->attr_count = static_cast<uint32_t>(op.c_attrs.size());
  info->attrs = op.c_attrs.data();
  return oxh::ok();
}

oxh_status oxh_program_run_op(oxh_program *p, uint64_t index) {
  OXH_REQUIRE(p != nullptr, OXH_INVALID_SHAPE, "program is null");
  OXH_REQUIRE(index < p->ops.size(), OXH_INVALID_SHAPE, "op index out of range");
  return p->ops[index].launch(p->stream);
}

}  // extern "C"
