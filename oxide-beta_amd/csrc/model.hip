// model.hip -- MobileNetV4-Conv-S and its MNIST training step as a native executor: the model
// (parameters and BatchNorm state resident on the device), a trainer that traces one training
// step into a fixed list of launches over preallocated buffers and replays it from one
// hipGraph, an inference-mode evaluator, and OXTR save / load at model level.  Host C++ that
// calls this library's own kernels through the C ABI.
//
// Reference: MobileNetV4ConvSmall (crates/oxide-torch-models/src/models/mobilenet_v4.rs:84-321)
// built from Conv2d / BatchNorm2d / ConvNormAct / UniversalInvertedBottleneck /
// FusedInvertedBottleneck (crates/oxide-torch/src/nn.rs:107-655); the training step of
// examples/mnist_training.rs:75-92 (zero_grad, forward, cross_entropy, backward, AdamW with
// lr 1e-3, weight decay 1e-4, betas 0.9 / 0.999, eps 1e-8, optim.rs:48-127); the device
// executor it replaces is crates/oxide-torch/src/cuda/runtime.rs (eager evaluation of the lazy
// graph, reverse-topological backward with first-write-then-accumulate gradients, 671-692).
//
// Schedule.  The forward is traced once (nodes are created in dependency order, so creation
// order is topological); the backward visits nodes in reverse, so every consumer of a value
// has contributed to its gradient before the value's own backward runs.  A value's first
// gradient contribution is written in place; later ones go to a scratch buffer and are added
// with oxh_accumulate.  Two rewrites cut launches without changing any value: a BatchNorm
// whose only consumer is a ReLU runs as the fused BN + ReLU entry points (the ReLU mask is
// read from the ReLU output, positive exactly where its input is), and a residual add's
// first operand, when the add is its only consumer, takes the add's gradient buffer (the
// add's backward is the identity).  The loss is the backward root (outer gradient 1): one
// fused cross-entropy launch gives loss and logit gradient.  One multi-tensor AdamW launch
// group with a device step counter ends the step, so the captured graph replays correctly.
//
// Every device buffer of a trainer or evaluator is carved from one allocation made at
// creation; nothing is allocated per step.
#include <hip/hip_runtime.h>

#include <array>
#include <cmath>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "common.h"

namespace {

constexpr float kBnMomentum = 0.1f, kBnEpsilon = 1e-5f;

// ---------------------------------------------------------------- device arena

// Offsets are planned first, then one hipMalloc serves them all.
struct Arena {
  uint64_t size = 0;
  char *base = nullptr;
  uint64_t reserve(uint64_t bytes) {
    const uint64_t at = size;
    size += (bytes + 255) / 256 * 256;
    return at;
  }
  oxh_status allocate() {
    if (size == 0) return oxh::ok();
    OXH_HIP_CHECK(hipMalloc(reinterpret_cast<void **>(&base), size));
    OXH_HIP_CHECK(hipMemset(base, 0, size));
    return oxh::ok();
  }
  template <typename T>
  T *at(uint64_t offset) const {
    return reinterpret_cast<T *>(base + offset);
  }
  ~Arena() {
    if (base) (void)hipFree(base);
  }
};

// ---------------------------------------------------------------- model

struct Param {
  std::vector<uint64_t> shape;
  uint64_t n = 0;
  std::vector<float> host;  // initial / loaded values
  float *value = nullptr;   // device
};

struct BnState {
  uint64_t channels = 0;
  int weight = -1, bias = -1;
  std::vector<float> running_mean, running_variance;  // host copies
  float *rm = nullptr, *rv = nullptr;                 // device
};

struct ConvLayer {
  int weight = -1, bias = -1;
  uint32_t in_c = 0, out_c = 0, kernel = 0, stride = 1, pad = 0, groups = 1;
};

struct ConvNormAct {
  ConvLayer conv;
  int bn = -1;
  bool relu = false;
};

enum class BlockKind { Conv, Fused, Uib, GlobalAverage, Classifier };

struct Block {
  BlockKind kind;
  std::vector<ConvNormAct> layers;  // Conv: 1; Fused: expand, project; Uib: 2..4
  bool residual = false;
  ConvLayer classifier;
};

}  // namespace

struct oxh_model {
  std::vector<Param> params;
  std::vector<BnState> bns;
  std::vector<Block> blocks;
  uint64_t classes = 0, in_channels = 0, resolution = 0;
  bool training = true;
  Arena arena;
};

namespace {

int add_param(oxh_model &m, std::vector<uint64_t> shape, std::vector<float> values) {
  Param p;
  p.n = 1;
  for (uint64_t d : shape) p.n *= d;
  p.shape = std::move(shape);
  p.host = std::move(values);
  m.params.push_back(std::move(p));
  return static_cast<int>(m.params.size()) - 1;
}

// nn.rs:236-274: OIHW weight from the deterministic init, zero bias, padding kernel / 2.
oxh_status make_conv(oxh_model &m, uint64_t in_c, uint64_t out_c, uint64_t kernel, uint64_t stride,
                     uint64_t groups, ConvLayer &out) {
  OXH_REQUIRE(kernel != 0 && groups != 0 && in_c % groups == 0 && out_c % groups == 0,
              OXH_INVALID_SHAPE, "invalid Conv2d channel, group, or kernel configuration");
  const uint64_t shape[4] = {out_c, in_c / groups, kernel, kernel};
  std::vector<float> w(out_c * (in_c / groups) * kernel * kernel);
  oxh_status st = oxh_initialized_weights(shape, in_c / groups, w.data());
  if (st != OXH_OK) return st;
  out.weight = add_param(m, {shape[0], shape[1], shape[2], shape[3]}, std::move(w));
  out.bias = add_param(m, {out_c}, std::vector<float>(out_c, 0.0f));
  out.in_c = static_cast<uint32_t>(in_c);
  out.out_c = static_cast<uint32_t>(out_c);
  out.kernel = static_cast<uint32_t>(kernel);
  out.stride = static_cast<uint32_t>(stride);
  out.pad = static_cast<uint32_t>(kernel / 2);
  out.groups = static_cast<uint32_t>(groups);
  return oxh::ok();
}

// nn.rs:107-233: gamma 1, beta 0, running mean 0 / variance 1.
int make_bn(oxh_model &m, uint64_t channels) {
  BnState b;
  b.channels = channels;
  b.weight = add_param(m, {channels}, std::vector<float>(channels, 1.0f));
  b.bias = add_param(m, {channels}, std::vector<float>(channels, 0.0f));
  b.running_mean.assign(channels, 0.0f);
  b.running_variance.assign(channels, 1.0f);
  m.bns.push_back(std::move(b));
  return static_cast<int>(m.bns.size()) - 1;
}

// nn.rs:349-385
oxh_status make_cna(oxh_model &m, uint64_t in_c, uint64_t out_c, uint64_t kernel,
                    uint64_t stride, uint64_t groups, bool relu, ConvNormAct &out) {
  oxh_status st = make_conv(m, in_c, out_c, kernel, stride, groups, out.conv);
  if (st != OXH_OK) return st;
  out.bn = make_bn(m, out_c);
  out.relu = relu;
  return oxh::ok();
}

// mobilenet_v4.rs:111-175 (table 11, MNIST variant: input_channels 1, resolution 28)
oxh_status build_model(oxh_model &m, uint64_t classes, uint64_t in_c, uint64_t resolution) {
  OXH_REQUIRE(classes != 0, OXH_INVALID_SHAPE, "num_classes must be non-zero");
  OXH_REQUIRE(in_c > 0 && resolution > 0 && in_c < 65536 && resolution < 65536,
              OXH_INVALID_SHAPE, "invalid input channels or resolution");
  m.classes = classes;
  m.in_channels = in_c;
  m.resolution = resolution;
  oxh_status st = oxh::ok();
  auto conv_block = [&](uint64_t i, uint64_t o, uint64_t k, uint64_t s, bool relu) {
    Block b{BlockKind::Conv, {}, false, {}};
    b.layers.resize(1);
    st = make_cna(m, i, o, k, s, 1, relu, b.layers[0]);
    m.blocks.push_back(std::move(b));
  };
  // nn.rs:565-655: full k x k expand with ReLU, 1x1 project
  auto fused = [&](uint64_t i, uint64_t o, uint64_t e, uint64_t k, uint64_t s) {
    Block b{BlockKind::Fused, {}, s == 1 && i == o, {}};
    b.layers.resize(2);
    if (st == OXH_OK) st = make_cna(m, i, e, k, s, 1, true, b.layers[0]);
    if (st == OXH_OK) st = make_cna(m, e, o, 1, 1, 1, false, b.layers[1]);
    m.blocks.push_back(std::move(b));
  };
  // nn.rs:425-515: optional start depthwise (ReLU), expand 1x1 (ReLU), optional middle
  // depthwise carrying the stride (ReLU), project 1x1
  auto uib = [&](uint64_t i, uint64_t o, uint64_t e, uint64_t start, uint64_t middle,
                 uint64_t s) {
    if (st != OXH_OK) return;
    if (s > 1 && middle == 0) {
      st = oxh::fail(OXH_INVALID_SHAPE, "a strided UIB requires a middle depthwise convolution");
      return;
    }
    Block b{BlockKind::Uib, {}, s == 1 && i == o, {}};
    ConvNormAct l;
    if (start) {
      if (st == OXH_OK) st = make_cna(m, i, i, start, 1, i, true, l);
      b.layers.push_back(l);
    }
    if (st == OXH_OK) st = make_cna(m, i, e, 1, 1, 1, true, l);
    b.layers.push_back(l);
    if (middle) {
      if (st == OXH_OK) st = make_cna(m, e, e, middle, s, e, true, l);
      b.layers.push_back(l);
    }
    if (st == OXH_OK) st = make_cna(m, e, o, 1, 1, 1, false, l);
    b.layers.push_back(l);
    m.blocks.push_back(std::move(b));
  };
  conv_block(in_c, 32, 3, 2, true);
  if (st == OXH_OK) fused(32, 32, 32, 3, 2);
  if (st == OXH_OK) fused(32, 64, 96, 3, 2);
  // mobilenet_v4.rs:140-153: in, out, expanded, start DW, middle DW (0 = none), stride
  const uint64_t specs[12][6] = {{64, 96, 192, 5, 5, 2},    {96, 96, 192, 0, 3, 1},
                                 {96, 96, 192, 0, 3, 1},    {96, 96, 192, 0, 3, 1},
                                 {96, 96, 192, 0, 3, 1},    {96, 96, 384, 3, 0, 1},
                                 {96, 128, 576, 3, 3, 2},   {128, 128, 512, 5, 5, 1},
                                 {128, 128, 512, 0, 5, 1},  {128, 128, 384, 0, 5, 1},
                                 {128, 128, 512, 0, 3, 1},  {128, 128, 512, 0, 3, 1}};
  for (const auto &sp : specs)
    if (st == OXH_OK) uib(sp[0], sp[1], sp[2], sp[3], sp[4], sp[5]);
  if (st == OXH_OK) conv_block(128, 960, 1, 1, true);
  m.blocks.push_back(Block{BlockKind::GlobalAverage, {}, false, {}});
  if (st == OXH_OK) conv_block(960, 1280, 1, 1, true);
  if (st == OXH_OK) {
    Block b{BlockKind::Classifier, {}, false, {}};
    st = make_conv(m, 1280, classes, 1, 1, 1, b.classifier);
    m.blocks.push_back(std::move(b));
  }
  return st;
}

oxh_status upload_model(oxh_model &m) {
  std::vector<uint64_t> poff(m.params.size());
  std::vector<std::array<uint64_t, 2>> boff(m.bns.size());
  for (size_t i = 0; i < m.params.size(); ++i) poff[i] = m.arena.reserve(m.params[i].n * 4);
  for (size_t i = 0; i < m.bns.size(); ++i)
    boff[i] = {m.arena.reserve(m.bns[i].channels * 4), m.arena.reserve(m.bns[i].channels * 4)};
  oxh_status st = m.arena.allocate();
  if (st != OXH_OK) return st;
  for (size_t i = 0; i < m.params.size(); ++i) {
    Param &p = m.params[i];
    p.value = m.arena.at<float>(poff[i]);
    OXH_HIP_CHECK(hipMemcpy(p.value, p.host.data(), p.n * 4, hipMemcpyHostToDevice));
  }
  for (size_t i = 0; i < m.bns.size(); ++i) {
    BnState &b = m.bns[i];
    b.rm = m.arena.at<float>(boff[i][0]);
    b.rv = m.arena.at<float>(boff[i][1]);
    OXH_HIP_CHECK(hipMemcpy(b.rm, b.running_mean.data(), b.channels * 4, hipMemcpyHostToDevice));
    OXH_HIP_CHECK(
        hipMemcpy(b.rv, b.running_variance.data(), b.channels * 4, hipMemcpyHostToDevice));
  }
  return oxh::ok();
}

// sync_batch_norm_state (runtime.rs:1268-1304) and the parameters: device -> host copies.
oxh_status sync_model(oxh_model &m) {
  OXH_HIP_CHECK(hipDeviceSynchronize());
  for (Param &p : m.params)
    OXH_HIP_CHECK(hipMemcpy(p.host.data(), p.value, p.n * 4, hipMemcpyDeviceToHost));
  for (BnState &b : m.bns) {
    OXH_HIP_CHECK(
        hipMemcpy(b.running_mean.data(), b.rm, b.channels * 4, hipMemcpyDeviceToHost));
    OXH_HIP_CHECK(
        hipMemcpy(b.running_variance.data(), b.rv, b.channels * 4, hipMemcpyDeviceToHost));
  }
  return oxh::ok();
}

// ---------------------------------------------------------------- traced graph

enum class Op { Input, Targets, Param, Conv, Bn, Relu, Add, Pool, Reshape, CrossEntropy };

struct Node {
  Node(Op o, std::vector<int> i) : op(o), in(std::move(i)) {}
  Op op;
  std::vector<int> in;
  std::array<uint64_t, 4> shape{1, 1, 1, 1};
  uint32_t rank = 4;
  int param = -1, bn = -1;
  ConvLayer conv;
  uint64_t numel() const {
    uint64_t n = 1;
    for (uint32_t i = 0; i < rank; ++i) n *= shape[i];
    return n;
  }
};

struct Graph {
  std::vector<Node> nodes;
  std::vector<int> param_node;  // parameter index -> node (lazily created)
  int add(Node n) {
    nodes.push_back(std::move(n));
    return static_cast<int>(nodes.size()) - 1;
  }
  int param(const oxh_model &m, int p) {
    if (param_node.empty()) param_node.assign(m.params.size(), -1);
    if (param_node[p] < 0) {
      Node n{Op::Param, {}};
      n.param = p;
      n.rank = static_cast<uint32_t>(m.params[p].shape.size());
      for (uint32_t i = 0; i < n.rank; ++i) n.shape[i] = m.params[p].shape[i];
      param_node[p] = add(n);
    }
    return param_node[p];
  }
};

// tensor/mod.rs conv2d shape rule
int trace_conv(Graph &g, const oxh_model &m, int x, const ConvLayer &c) {
  const int w = g.param(m, c.weight), b = g.param(m, c.bias);
  const Node &in = g.nodes[x];
  Node n{Op::Conv, {x, w, b}};
  n.conv = c;
  n.shape = {in.shape[0], c.out_c, (in.shape[2] + 2 * c.pad - c.kernel) / c.stride + 1,
             (in.shape[3] + 2 * c.pad - c.kernel) / c.stride + 1};
  return g.add(n);
}

int trace_cna(Graph &g, const oxh_model &m, int x, const ConvNormAct &l) {
  const int c = trace_conv(g, m, x, l.conv);
  const BnState &bs = m.bns[l.bn];
  Node bn{Op::Bn, {c, g.param(m, bs.weight), g.param(m, bs.bias)}};
  bn.bn = l.bn;
  bn.shape = g.nodes[c].shape;
  int y = g.add(bn);
  if (l.relu) {
    Node r{Op::Relu, {y}};
    r.shape = g.nodes[y].shape;
    y = g.add(r);
  }
  return y;
}

// mobilenet_v4.rs:182-195: the logits, every block's output shape recorded.
int trace_forward(Graph &g, const oxh_model &m, int x, std::vector<std::array<uint64_t, 4>> *shapes) {
  for (const Block &b : m.blocks) {
    const int input = x;
    switch (b.kind) {
      case BlockKind::Conv:
      case BlockKind::Fused:
      case BlockKind::Uib:
        for (const ConvNormAct &l : b.layers) x = trace_cna(g, m, x, l);
        if (b.residual) {
          Node a{Op::Add, {x, input}};
          a.shape = g.nodes[x].shape;
          x = g.add(a);
        }
        break;
      case BlockKind::GlobalAverage: {  // tensor/mod.rs:273-283
        Node p{Op::Pool, {x}};
        const auto &s = g.nodes[x].shape;
        p.shape = {s[0], s[1], 1, 1};
        x = g.add(p);
        break;
      }
      case BlockKind::Classifier:
        x = trace_conv(g, m, x, b.classifier);
        break;
    }
    if (shapes) shapes->push_back(g.nodes[x].shape);
  }
  Node r{Op::Reshape, {x}};
  r.rank = 2;
  r.shape = {g.nodes[x].shape[0], m.classes, 1, 1};
  if (shapes) shapes->back() = r.shape;
  return g.add(r);
}

// ---------------------------------------------------------------- launch programs

struct TensorRef {
  std::string role;
  void *data = nullptr;
  std::array<uint64_t, 4> shape{1, 1, 1, 1};
  uint32_t rank = 1;
  int access = 0;  // 0 read, 1 write, 2 updated in place
  int dtype = 0;   // 0 f32, 1 i32
};

struct OpRec {
  std::string kind, name;
  std::vector<TensorRef> tensors;
  std::vector<std::pair<std::string, double>> attrs;
  std::function<oxh_status(hipStream_t)> launch;
  // C views of the above, built once
  std::vector<oxh_op_tensor> c_tensors;
  std::vector<oxh_op_attr> c_attrs;
};

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

}  // namespace

struct oxh_program {
  std::vector<OpRec> ops;
  hipStream_t stream = nullptr;
  oxh_graph *graph = nullptr;

  oxh_status finalize() {
    for (const OpRec &op : ops)
      for (const TensorRef &t : op.tensors)
        OXH_REQUIRE(t.data != nullptr, OXH_EXECUTION,
                    "internal: " + op.name + " has no buffer for " + t.role);
    for (OpRec &op : ops) {
      op.c_tensors.clear();
      for (const TensorRef &t : op.tensors) {
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
  oxh_status run() {
    for (OpRec &op : ops) {
      oxh_status st = op.launch(stream);
      if (st != OXH_OK) return st;
    }
    return oxh::ok();
  }
  oxh_status capture() {
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
  ~oxh_program() {
    if (graph) (void)oxh_graph_destroy(graph);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

struct oxh_trainer {
  oxh_model *model = nullptr;
  uint64_t batch = 0;
  float lr = 1e-3f, wd = 1e-4f, beta1 = 0.9f, beta2 = 0.999f, eps = 1e-8f;
  Graph g;
  Arena arena;
  oxh_program program;
  std::vector<float *> value, grad;
  std::vector<float *> saved_mean, saved_inv;  // per node (BN)
  std::vector<float *> pgrad, pm, pv;           // per parameter
  std::vector<oxh_adamw_tensor> adam;
  oxh_adamw_tensor *adam_table = nullptr;  // device copy of `adam`
  uint32_t *adam_starts = nullptr, *adam_ticket = nullptr;
  uint64_t adam_chunks = 0;
  float *scratch = nullptr, *outer = nullptr, *loss = nullptr;
  int32_t *step = nullptr;
  uint32_t *error_flag = nullptr;
  void *workspace = nullptr;
  uint64_t workspace_bytes = 0;
  int input = -1, targets = -1, logits = -1, loss_node = -1;
};

struct oxh_evaluator {
  oxh_model *model = nullptr;
  uint64_t batch = 0;
  Graph g;
  Arena arena;
  oxh_program program;
  std::vector<float *> value;
  uint32_t *classes = nullptr;
  int input = -1, logits = -1;
};

namespace {

uint64_t node_bytes(const Node &n) { return n.numel() * 4; }

oxh_conv2d_shape conv_shape(const Graph &g, const Node &n) {
  const Node &x = g.nodes[n.in[0]];
  return oxh_conv2d_shape{x.shape[0], x.shape[1], x.shape[2], x.shape[3], n.conv.out_c,
                          n.conv.kernel, n.conv.kernel, n.conv.stride, n.conv.pad, n.conv.groups};
}

oxh_status plan_workspace(const Graph &g, uint64_t &bytes) {
  bytes = 256;
  for (const Node &n : g.nodes) {
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

// ---- trainer construction

oxh_status build_trainer(oxh_trainer &t) {
  oxh_model &m = *t.model;
  Graph &g = t.g;
  Node in{Op::Input, {}};
  in.shape = {t.batch, m.in_channels, m.resolution, m.resolution};
  t.input = g.add(in);
  t.logits = trace_forward(g, m, t.input, nullptr);
  Node tg{Op::Targets, {}};
  tg.rank = 1;
  tg.shape = {t.batch, 1, 1, 1};
  t.targets = g.add(tg);
  Node ce{Op::CrossEntropy, {t.logits, t.targets}};
  ce.rank = 1;
  ce.shape = {1, 1, 1, 1};
  t.loss_node = g.add(ce);
  const size_t n = g.nodes.size();

  // consumers, fused BN + ReLU pairs, aliased add operands
  std::vector<int> consumers(n, 0);
  for (const Node &x : g.nodes)
    for (int i : x.in) ++consumers[i];
  std::vector<char> fused_bn(n, 0), fused_relu(n, 0);
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (x.op == Op::Relu && g.nodes[x.in[0]].op == Op::Bn && consumers[x.in[0]] == 1) {
      fused_relu[i] = 1;
      fused_bn[x.in[0]] = 1;
    }
  }
  // a BN (without ReLU) whose only consumer is a residual add, as the add's first operand:
  // its forward writes the add's output (BN + shortcut) and the add launches nothing
  std::vector<int64_t> bn_into_add(n, -1);
  std::vector<char> add_absorbed(n, 0);
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (x.op != Op::Add) continue;
    const int first = x.in[0];
    if (g.nodes[first].op == Op::Bn && !fused_bn[first] && consumers[first] == 1 &&
        x.in[1] != first) {
      bn_into_add[first] = static_cast<int64_t>(i);
      add_absorbed[i] = 1;
    }
  }
  // a depthwise convolution whose only consumer is the BatchNorm traced next (parameter nodes
  // aside), on planes the one-launch depthwise ConvNormAct kernels take: the pair runs as one
  // launch per direction, at the BN's place in each pass (no launch lies between the two in
  // either order, so every gradient contribution keeps its order)
  std::vector<char> dw_conv(n, 0);
  std::vector<int64_t> dw_conv_of(n, -1);  // BN node -> its fused depthwise convolution
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (x.op != Op::Conv || consumers[i] != 1) continue;
    size_t j = i + 1;
    while (j < n && g.nodes[j].op == Op::Param) ++j;
    if (j == n || g.nodes[j].op != Op::Bn || g.nodes[j].in[0] != static_cast<int>(i) ||
        bn_into_add[j] >= 0)
      continue;
    if (x.conv.groups != g.nodes[x.in[0]].shape[1] || x.conv.groups != x.shape[1]) continue;
    const oxh_conv2d_shape s = conv_shape(g, x);
    if (!oxh_depthwise_conv_batch_norm_supported(&s)) continue;
    dw_conv[i] = 1;
    dw_conv_of[j] = static_cast<int64_t>(i);
  }
  // gradient buffers, consumers before producers
  std::vector<int64_t> grad_of(n, -1);  // node whose grad buffer this node uses (-1: own)
  std::vector<char> has_grad(n, 0), aliased(n, 0);
  for (size_t r = n; r-- > 0;) {
    const Node &x = g.nodes[r];
    if (x.op == Op::Param || x.op == Op::Input || x.op == Op::Targets ||
        x.op == Op::CrossEntropy || fused_bn[r])
      continue;
    has_grad[r] = 1;
    if (x.op == Op::Reshape) {
      grad_of[x.in[0]] = grad_of[r] >= 0 ? grad_of[r] : static_cast<int64_t>(r);
    } else if (x.op == Op::Add) {
      const int first = x.in[0];
      const Op fo = g.nodes[first].op;
      if (consumers[first] == 1 && grad_of[first] < 0 && fo != Op::Param && fo != Op::Input) {
        grad_of[first] = grad_of[r] >= 0 ? grad_of[r] : static_cast<int64_t>(r);
        aliased[first] = 1;
      }
    }
  }

  // ---- plan the arena
  Arena &a = t.arena;
  std::vector<int64_t> voff(n, -1), goff(n, -1), smoff(n, -1), sioff(n, -1);
  uint64_t largest = 1;
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (x.op == Op::Bn) {  // saved statistics, also for a BN fused with its ReLU
      smoff[i] = a.reserve(x.shape[1] * 4);
      sioff[i] = a.reserve(x.shape[1] * 4);
    }
    if (x.op == Op::Param || x.op == Op::Reshape || fused_bn[i]) continue;
    voff[i] = a.reserve(node_bytes(x));
    if (x.op != Op::CrossEntropy && x.op != Op::Targets) largest = std::max(largest, x.numel());
  }
  for (size_t i = 0; i < n; ++i)
    if (has_grad[i] && grad_of[i] < 0) goff[i] = a.reserve(node_bytes(g.nodes[i]));
  std::vector<std::array<uint64_t, 3>> poff(m.params.size());
  for (size_t p = 0; p < m.params.size(); ++p)
    poff[p] = {a.reserve(m.params[p].n * 4), a.reserve(m.params[p].n * 4),
               a.reserve(m.params[p].n * 4)};
  const uint64_t scratch_off = a.reserve(largest * 4), outer_off = a.reserve(4),
                 step_off = a.reserve(4), flag_off = a.reserve(4), ticket_off = a.reserve(4);
  // the optimizer's device tensor table and chunk starts (one launch over every parameter)
  const uint64_t table_off = a.reserve(m.params.size() * sizeof(oxh_adamw_tensor));
  const uint64_t starts_off = a.reserve((m.params.size() + 1) * 4);
  oxh_status st = plan_workspace(g, t.workspace_bytes);
  if (st != OXH_OK) return st;
  const uint64_t ws_off = a.reserve(t.workspace_bytes);
  st = a.allocate();  // zero-filled: moments, step counter, error flag start at 0
  if (st != OXH_OK) return st;

  t.value.assign(n, nullptr);
  t.grad.assign(n, nullptr);
  t.saved_mean.assign(n, nullptr);
  t.saved_inv.assign(n, nullptr);
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (x.op == Op::Param) t.value[i] = m.params[x.param].value;
    if (voff[i] >= 0) t.value[i] = a.at<float>(voff[i]);
    if (smoff[i] >= 0) t.saved_mean[i] = a.at<float>(smoff[i]);
    if (sioff[i] >= 0) t.saved_inv[i] = a.at<float>(sioff[i]);
    if (goff[i] >= 0) t.grad[i] = a.at<float>(goff[i]);
  }
  for (size_t i = 0; i < n; ++i)
    if (g.nodes[i].op == Op::Reshape) t.value[i] = t.value[g.nodes[i].in[0]];
  for (size_t i = 0; i < n; ++i)
    if (grad_of[i] >= 0) t.grad[i] = t.grad[grad_of[i]];
  t.pgrad.resize(m.params.size());
  t.pm.resize(m.params.size());
  t.pv.resize(m.params.size());
  for (size_t p = 0; p < m.params.size(); ++p) {
    t.pgrad[p] = a.at<float>(poff[p][0]);
    t.pm[p] = a.at<float>(poff[p][1]);
    t.pv[p] = a.at<float>(poff[p][2]);
  }
  for (size_t i = 0; i < n; ++i)
    if (g.nodes[i].op == Op::Param) t.grad[i] = t.pgrad[g.nodes[i].param];
  t.scratch = a.at<float>(scratch_off);
  t.outer = a.at<float>(outer_off);
  t.step = a.at<int32_t>(step_off);
  t.error_flag = a.at<uint32_t>(flag_off);
  t.adam_ticket = a.at<uint32_t>(ticket_off);
  t.adam_table = a.at<oxh_adamw_tensor>(table_off);
  t.adam_starts = a.at<uint32_t>(starts_off);
  t.workspace = a.at<void>(ws_off);
  t.loss = t.value[t.loss_node];
  const float one = 1.0f;
  OXH_HIP_CHECK(hipMemcpy(t.outer, &one, 4, hipMemcpyHostToDevice));

  // ---- schedule
  auto &ops = t.program.ops;
  void *ws = t.workspace;
  const uint64_t wsb = t.workspace_bytes;
  auto name = [](const char *p, size_t i) { return std::string(p) + std::to_string(i); };
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
    const Pending p = pending[x];
    pending[x] = Pending{};
    written[x] = 1;
    float *dst = t.grad[x];
    const uint64_t bytes = node_bytes(g.nodes[x]);
    OpRec c;
    c.kind = "add_backward";
    c.name = p.name;
    c.tensors = {ref("gradient", const_cast<float *>(p.gradient), g.nodes[p.add], 0),
                 ref("contribution", dst, g.nodes[x], 1)};
    const float *gr = p.gradient;
    c.launch = [dst, gr, bytes](hipStream_t st) {
      return oxh_memcpy_d2d_async(dst, gr, bytes, st);
    };
    ops.push_back(std::move(c));
  };
  // Where a contribution to node x's gradient goes: its buffer (first) or the scratch buffer
  // added into it afterwards.
  auto contribution = [&](int x, float *&dst, float *&acc) {
    flush(x);
    if (!written[x]) {
      written[x] = 1;
      dst = t.grad[x];
      acc = nullptr;
    } else {
      dst = t.scratch;
      acc = t.grad[x];
    }
  };
  auto emit = [&](OpRec op, float *acc, const Node &target,
                  std::function<oxh_status(hipStream_t)> body) {
    if (acc == nullptr) {
      op.launch = std::move(body);
    } else {
      float *part = t.scratch;
      const uint64_t cnt = target.numel();
      op.tensors.push_back(ref("accumulate_into", acc, target, 2));
      op.launch = [body, acc, part, cnt](hipStream_t s) {
        oxh_status st = body(s);
        if (st != OXH_OK) return st;
        return oxh_accumulate(s, acc, part, acc, cnt);
      };
    }
    ops.push_back(std::move(op));
  };
  auto conv_attrs = [](const Node &x) {
    return std::vector<std::pair<std::string, double>>{
        {"stride", x.conv.stride}, {"padding", x.conv.pad}, {"groups", x.conv.groups}};
  };

  // forward
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (x.op == Op::Param || x.op == Op::Input || x.op == Op::Targets || x.op == Op::Reshape ||
        fused_bn[i] || add_absorbed[i] || dw_conv[i])
      continue;
    float *out = t.value[i];
    OpRec op;
    switch (x.op) {
      case Op::Conv: {
        const oxh_conv2d_shape s = conv_shape(g, x);
        const float *xi = t.value[x.in[0]], *w = t.value[x.in[1]], *b = t.value[x.in[2]];
        op.kind = "conv2d_forward";
        op.name = name("conv", i);
        op.tensors = {ref("x", const_cast<float *>(xi), g.nodes[x.in[0]], 0),
                      ref("weight", const_cast<float *>(w), g.nodes[x.in[1]], 0),
                      ref("bias", const_cast<float *>(b), g.nodes[x.in[2]], 0),
                      ref("y", out, x, 1)};
        op.attrs = conv_attrs(x);
        op.launch = [s, xi, w, b, out](hipStream_t st) {
          return oxh_conv2d_forward(st, &s, xi, w, b, out);
        };
        ops.push_back(std::move(op));
        break;
      }
      case Op::Relu:
      case Op::Bn: {
        const bool fused = x.op == Op::Relu && fused_relu[i];
        if (x.op == Op::Relu && !fused) {
          const float *xi = t.value[x.in[0]];
          const uint64_t cnt = x.numel();
          op.kind = "relu_forward";
          op.name = name("relu", i);
          op.tensors = {ref("x", const_cast<float *>(xi), g.nodes[x.in[0]], 0), ref("y", out, x, 1)};
          op.launch = [xi, out, cnt](hipStream_t st) { return oxh_relu(st, xi, out, cnt); };
          ops.push_back(std::move(op));
          break;
        }
        const int bi = fused ? x.in[0] : static_cast<int>(i);
        const Node &bn = g.nodes[bi];
        const BnState &bs = m.bns[bn.bn];
        const float *xi = t.value[bn.in[0]], *w = t.value[bn.in[1]], *b = t.value[bn.in[2]];
        float *sm = t.saved_mean[bi], *si = t.saved_inv[bi], *rm = bs.rm, *rv = bs.rv;
        const uint64_t N = bn.shape[0], C = bn.shape[1], HW = bn.shape[2] * bn.shape[3];
        if (!fused && bn_into_add[i] >= 0) {  // BN + residual add in one launch
          const Node &ad = g.nodes[bn_into_add[i]];
          const float *skip = t.value[ad.in[1]];
          float *sum = t.value[bn_into_add[i]];
          op.kind = "batch_norm2d_add_forward";
          op.name = name("bn", bi) + "+" + name("add", bn_into_add[i]);
          op.tensors = {ref("x", const_cast<float *>(xi), g.nodes[bn.in[0]], 0),
                        ref("weight", const_cast<float *>(w), g.nodes[bn.in[1]], 0),
                        ref("bias", const_cast<float *>(b), g.nodes[bn.in[2]], 0),
                        ref("addend", const_cast<float *>(skip), g.nodes[ad.in[1]], 0),
                        ref("y", sum, ad, 1), ref_flat("saved_mean", sm, C, 1),
                        ref_flat("saved_inverse_std", si, C, 1),
                        ref_flat("running_mean", rm, C, 2), ref_flat("running_variance", rv, C, 2)};
          op.attrs = {{"momentum", kBnMomentum}, {"epsilon", kBnEpsilon}};
          op.launch = [=](hipStream_t st) {
            return oxh_batch_norm_add_forward_train(st, N, C, HW, kBnMomentum, kBnEpsilon, xi, w,
                                                    b, rm, rv, sm, si, skip, sum, ws, wsb);
          };
          ops.push_back(std::move(op));
          break;
        }
        if (dw_conv_of[bi] >= 0) {  // depthwise conv + BN (+ ReLU) in one launch
          const int ci = static_cast<int>(dw_conv_of[bi]);
          const Node &cv = g.nodes[ci];
          const oxh_conv2d_shape s = conv_shape(g, cv);
          const float *cx = t.value[cv.in[0]], *cw = t.value[cv.in[1]], *cb = t.value[cv.in[2]];
          float *cy = t.value[ci];
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
          op.attrs.push_back({"momentum", kBnMomentum});
          op.attrs.push_back({"epsilon", kBnEpsilon});
          op.launch = [=](hipStream_t st) {
            return oxh_depthwise_conv_batch_norm_forward_train(st, &s, fused ? 1 : 0, kBnMomentum,
                                                               kBnEpsilon, cx, cw, cb, cy, w, b,
                                                               rm, rv, sm, si, out);
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
        op.attrs = {{"momentum", kBnMomentum}, {"epsilon", kBnEpsilon}};
        op.launch = [=](hipStream_t st) {
          return fused ? oxh_batch_norm_relu_forward_train(st, N, C, HW, kBnMomentum, kBnEpsilon,
                                                           xi, w, b, rm, rv, sm, si, out, ws, wsb)
                       : oxh_batch_norm_forward_train(st, N, C, HW, kBnMomentum, kBnEpsilon, xi,
                                                      w, b, rm, rv, sm, si, out, ws, wsb);
        };
        ops.push_back(std::move(op));
        break;
      }
      case Op::Add: {
        const float *p = t.value[x.in[0]], *q = t.value[x.in[1]];
        const uint64_t cnt = x.numel();
        op.kind = "add_forward";
        op.name = name("add", i);
        op.tensors = {ref("a", const_cast<float *>(p), g.nodes[x.in[0]], 0),
                      ref("b", const_cast<float *>(q), g.nodes[x.in[1]], 0), ref("y", out, x, 1)};
        op.launch = [p, q, out, cnt](hipStream_t st) { return oxh_add(st, p, q, out, cnt); };
        ops.push_back(std::move(op));
        break;
      }
      case Op::Pool: {
        const Node &xin = g.nodes[x.in[0]];
        const oxh_pool2d_shape ps{xin.shape[0], xin.shape[1], xin.shape[2], xin.shape[3],
                                  xin.shape[2], xin.shape[3], xin.shape[2], xin.shape[3]};
        const float *xi = t.value[x.in[0]];
        op.kind = "avg_pool2d_forward";
        op.name = name("pool", i);
        op.tensors = {ref("x", const_cast<float *>(xi), xin, 0), ref("y", out, x, 1)};
        op.attrs = {{"kernel_h", static_cast<double>(xin.shape[2])},
                    {"kernel_w", static_cast<double>(xin.shape[3])},
                    {"stride_h", static_cast<double>(xin.shape[2])},
                    {"stride_w", static_cast<double>(xin.shape[3])}};
        op.launch = [ps, xi, out](hipStream_t st) {
          return oxh_avg_pool2d_forward(st, &ps, xi, out);
        };
        ops.push_back(std::move(op));
        break;
      }
      case Op::CrossEntropy: {
        const Node &ln = g.nodes[x.in[0]];
        const float *lg = t.value[x.in[0]], *tg = t.value[x.in[1]];
        float *dl = nullptr, *acc = nullptr;
        contribution(x.in[0], dl, acc);
        const uint64_t rows = ln.shape[0], classes = ln.shape[1];
        float *outer = t.outer;
        uint32_t *flag = t.error_flag;
        op.kind = "cross_entropy";
        op.name = name("ce", i);
        op.tensors = {ref("logits", const_cast<float *>(lg), ln, 0),
                      ref("targets", const_cast<float *>(tg), g.nodes[x.in[1]], 0),
                      ref_flat("outer_gradient", outer, 1, 0), ref("loss", out, x, 1),
                      ref("gradient", dl, ln, 1), ref_flat("error_flag", flag, 1, 2, 1)};
        op.launch = [=](hipStream_t st) {
          return oxh_cross_entropy_forward_backward(st, rows, classes, lg, tg, outer, out, dl,
                                                    flag, ws, wsb);
        };
        ops.push_back(std::move(op));
        break;
      }
      default:
        return oxh::fail(OXH_TRACE, "no forward for a traced node");
    }
  }

  // backward, reverse topological order
  for (size_t r = n; r-- > 0;) {
    const Node &x = g.nodes[r];
    if (x.op == Op::Param || x.op == Op::Input || x.op == Op::Targets ||
        x.op == Op::CrossEntropy || fused_bn[r])
      continue;
    flush(static_cast<int>(r));  // a gradient still waiting for a second contribution
    OXH_REQUIRE(written[r], OXH_TRACE, "a traced value receives no gradient");
    const float *gr = t.grad[r];
    OpRec op;
    switch (x.op) {
      case Op::Reshape:
        OXH_REQUIRE(!written[x.in[0]], OXH_TRACE, "a reshaped value must have one consumer");
        written[x.in[0]] = 1;  // shares this gradient buffer
        break;
      case Op::Relu:
        if (!fused_relu[r]) {
          const int xin = x.in[0];
          const float *xi = t.value[xin];
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
        const float *xi = t.value[xin], *w = t.value[bn.in[1]];
        const float *y = fused ? t.value[r] : nullptr;
        const float *sm = t.saved_mean[bi], *si = t.saved_inv[bi];
        float *dg, *db, *dst, *acc, *unused;
        if (dw_conv_of[bi] >= 0) {  // depthwise conv + BN (+ ReLU) backward in one launch
          const Node &cv = g.nodes[xin];
          const int cin = cv.in[0];
          OXH_REQUIRE(!written[bn.in[1]] && !written[bn.in[2]] && !written[xin] &&
                          !written[cv.in[1]] && !written[cv.in[2]],
                      OXH_TRACE, "a fused depthwise layer's gradients have other contributions");
          float *cgr, *cdw, *cdb;
          contribution(bn.in[1], dg, unused);
          contribution(bn.in[2], db, unused);
          contribution(xin, cgr, unused);
          contribution(cv.in[2], cdb, unused);
          contribution(cv.in[1], cdw, unused);
          const oxh_conv2d_shape s = conv_shape(g, cv);
          const float *cx = t.value[cin], *cw = t.value[cv.in[1]];
          const uint64_t C = bn.shape[1];
          const float *addend = nullptr;
          dst = nullptr;
          acc = nullptr;
          if (g.nodes[cin].op != Op::Input) {  // the network input needs no gradient
            if (pending[cin].gradient != nullptr && !written[cin]) {
              addend = pending[cin].gradient;
              op.tensors.push_back(ref("addend", const_cast<float *>(addend),
                                       g.nodes[pending[cin].add], 0));
              pending[cin] = Pending{};
              written[cin] = 1;
              dst = t.grad[cin];
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
        contribution(bn.in[1], dg, unused);
        contribution(bn.in[2], db, unused);
        contribution(xin, dst, acc);
        // a convolution whose only consumer is this BN: its output gradient is this dx, whose
        // per-channel sum (the convolution's bias gradient) the BN backward forms in passing
        float *conv_db = nullptr;
        const Node &src = g.nodes[xin];
        if (src.op == Op::Conv && consumers[xin] == 1 && acc == nullptr &&
            !written[src.in[2]]) {
          contribution(src.in[2], conv_db, unused);
          conv_bias_done[xin] = 1;
        }
        const uint64_t N = bn.shape[0], C = bn.shape[1], HW = bn.shape[2] * bn.shape[3];
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
      case Op::Add: {
        for (int k = 0; k < 2; ++k) {
          const int inp = x.in[k];
          if (k == 0 && aliased[inp]) {
            written[inp] = 1;  // the add's gradient buffer is its own
            continue;
          }
          const std::string cname = name("add", r) + ".backward" + std::to_string(k);
          if (!written[inp] && pending[inp].gradient == nullptr) {
            pending[inp] = Pending{gr, cname, static_cast<int>(r)};
            continue;
          }
          float *dst, *acc;
          contribution(inp, dst, acc);
          const uint64_t bytes = node_bytes(x);
          OpRec c;
          c.kind = "add_backward";
          c.name = cname;
          c.tensors = {ref("gradient", const_cast<float *>(gr), x, 0),
                       ref("contribution", dst, g.nodes[inp], 1)};
          emit(std::move(c), acc, g.nodes[inp], [dst, gr, bytes](hipStream_t st) {
            return oxh_memcpy_d2d_async(dst, gr, bytes, st);
          });
        }
        break;
      }
      case Op::Pool: {
        const Node &xin = g.nodes[x.in[0]];
        const oxh_pool2d_shape ps{xin.shape[0], xin.shape[1], xin.shape[2], xin.shape[3],
                                  xin.shape[2], xin.shape[3], xin.shape[2], xin.shape[3]};
        float *dst, *acc;
        contribution(x.in[0], dst, acc);
        op.kind = "avg_pool2d_backward";
        op.name = name("pool", r) + ".backward";
        op.tensors = {ref("gradient", const_cast<float *>(gr), x, 0),
                      ref("contribution", dst, xin, 1)};
        op.attrs = {{"kernel_h", static_cast<double>(xin.shape[2])},
                    {"kernel_w", static_cast<double>(xin.shape[3])},
                    {"stride_h", static_cast<double>(xin.shape[2])},
                    {"stride_w", static_cast<double>(xin.shape[3])}};
        emit(std::move(op), acc, xin, [ps, gr, dst](hipStream_t st) {
          return oxh_avg_pool2d_backward(st, &ps, gr, dst);
        });
        break;
      }
      case Op::Conv: {
        if (dw_conv[r]) break;  // its backward ran with its BatchNorm's
        const oxh_conv2d_shape s = conv_shape(g, x);
        const int xin = x.in[0];
        const float *xi = t.value[xin], *w = t.value[x.in[1]];
        float *dw, *db = nullptr, *unused;
        contribution(x.in[1], dw, unused);
        const bool bias_here = !conv_bias_done[r];  // else the following BN formed it
        if (bias_here) contribution(x.in[2], db, unused);
        OpRec p;
        p.kind = "conv2d_parameter_backward";
        p.name = name("conv", r) + ".backward_parameters";
        p.tensors = {ref("gradient", const_cast<float *>(gr), x, 0),
                     ref("x", const_cast<float *>(xi), g.nodes[xin], 0),
                     ref("weight", const_cast<float *>(w), g.nodes[x.in[1]], 0),
                     ref("weight_gradient", dw, g.nodes[x.in[1]], 1)};
        if (bias_here) p.tensors.push_back(ref("bias_gradient", db, g.nodes[x.in[2]], 1));
        p.attrs = conv_attrs(x);
        p.launch = [s, gr, xi, dw, db, ws, wsb](hipStream_t st) {
          oxh_status e = oxh_conv2d_weight_backward(st, &s, gr, xi, dw, ws, wsb);
          if (e != OXH_OK || db == nullptr) return e;
          return oxh_conv2d_bias_backward(st, &s, gr, db, ws, wsb);
        };
        ops.push_back(std::move(p));
        if (g.nodes[xin].op == Op::Input) break;  // the network input needs no gradient
        float *dst, *acc;
        const float *addend = nullptr;
        if (pending[xin].gradient != nullptr && !written[xin]) {
          addend = pending[xin].gradient;
          op.tensors.push_back(ref("addend", const_cast<float *>(addend),
                                   g.nodes[pending[xin].add], 0));
          pending[xin] = Pending{};
          written[xin] = 1;
          dst = t.grad[xin];
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

  // AdamW over every parameter (visit order)
  t.adam.clear();
  OpRec op;
  op.kind = "adamw";
  op.name = "adamw";
  for (size_t p = 0; p < m.params.size(); ++p) {
    const Param &pr = m.params[p];
    t.adam.push_back(oxh_adamw_tensor{pr.value, t.pgrad[p], t.pm[p], t.pv[p], pr.n});
    op.tensors.push_back(ref_flat("parameter", pr.value, pr.n, 2));
    op.tensors.push_back(ref_flat("gradient", t.pgrad[p], pr.n, 0));
    op.tensors.push_back(ref_flat("first_moment", t.pm[p], pr.n, 2));
    op.tensors.push_back(ref_flat("second_moment", t.pv[p], pr.n, 2));
  }
  op.tensors.push_back(ref_flat("step", t.step, 1, 2, 1));
  op.attrs = {{"learning_rate", t.lr}, {"weight_decay", t.wd}, {"beta1", t.beta1},
              {"beta2", t.beta2}, {"epsilon", t.eps}};
  {
    const uint32_t count = static_cast<uint32_t>(t.adam.size());
    std::vector<uint32_t> starts(count + 1);
    st = oxh_adamw_table_layout(t.adam.data(), count, starts.data(), &t.adam_chunks);
    if (st != OXH_OK) return st;
    OXH_HIP_CHECK(hipMemcpy(t.adam_table, t.adam.data(), count * sizeof(oxh_adamw_tensor),
                            hipMemcpyHostToDevice));
    OXH_HIP_CHECK(hipMemcpy(t.adam_starts, starts.data(), (count + 1) * 4,
                            hipMemcpyHostToDevice));
  }
  oxh_trainer *self = &t;
  op.launch = [self](hipStream_t st) {
    return oxh_adamw_multi_tensor_table_step(
        st, self->lr, self->wd, self->beta1, self->beta2, self->eps, self->step,
        self->adam_ticket, self->adam_table, self->adam_starts,
        static_cast<uint32_t>(self->adam.size()), self->adam_chunks);
  };
  ops.push_back(std::move(op));
  return t.program.finalize();
}

// ---- evaluator construction (inference mode: BN from running statistics)

oxh_status build_evaluator(oxh_evaluator &e) {
  oxh_model &m = *e.model;
  Graph &g = e.g;
  Node in{Op::Input, {}};
  in.shape = {e.batch, m.in_channels, m.resolution, m.resolution};
  e.input = g.add(in);
  e.logits = trace_forward(g, m, e.input, nullptr);
  const size_t n = g.nodes.size();
  Arena &a = e.arena;
  std::vector<int64_t> voff(n, -1), ioff(n, -1);
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (x.op == Op::Param || x.op == Op::Reshape) continue;
    voff[i] = a.reserve(node_bytes(x));
    if (x.op == Op::Bn) ioff[i] = a.reserve(x.shape[1] * 4);
  }
  const uint64_t cls_off = a.reserve(e.batch * 4);
  oxh_status st = a.allocate();
  if (st != OXH_OK) return st;
  e.value.assign(n, nullptr);
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    if (x.op == Op::Param) e.value[i] = m.params[x.param].value;
    if (voff[i] >= 0) e.value[i] = a.at<float>(voff[i]);
    if (x.op == Op::Reshape) e.value[i] = e.value[x.in[0]];
  }
  e.classes = a.at<uint32_t>(cls_off);
  auto &ops = e.program.ops;
  for (size_t i = 0; i < n; ++i) {
    const Node &x = g.nodes[i];
    float *out = e.value[i];
    OpRec op;
    switch (x.op) {
      case Op::Param:
      case Op::Input:
      case Op::Reshape:
        continue;
      case Op::Conv: {
        const oxh_conv2d_shape s = conv_shape(g, x);
        const float *xi = e.value[x.in[0]], *w = e.value[x.in[1]], *b = e.value[x.in[2]];
        op.kind = "conv2d_forward";
        op.name = "conv" + std::to_string(i);
        op.tensors = {ref("x", const_cast<float *>(xi), g.nodes[x.in[0]], 0),
                      ref("weight", const_cast<float *>(w), g.nodes[x.in[1]], 0),
                      ref("bias", const_cast<float *>(b), g.nodes[x.in[2]], 0),
                      ref("y", out, x, 1)};
        op.attrs = {{"stride", x.conv.stride}, {"padding", x.conv.pad}, {"groups", x.conv.groups}};
        op.launch = [s, xi, w, b, out](hipStream_t st) {
          return oxh_conv2d_forward(st, &s, xi, w, b, out);
        };
        break;
      }
      case Op::Bn: {  // evaluation.rs:560-575, then the apply of 577-597
        const BnState &bs = m.bns[x.bn];
        const float *xi = e.value[x.in[0]], *w = e.value[x.in[1]], *b = e.value[x.in[2]];
        float *inv = a.at<float>(ioff[i]), *rm = bs.rm, *rv = bs.rv;
        const uint64_t N = x.shape[0], C = x.shape[1], HW = x.shape[2] * x.shape[3];
        op.kind = "batch_norm2d_eval_forward";
        op.name = "bn" + std::to_string(i);
        op.tensors = {ref("x", const_cast<float *>(xi), g.nodes[x.in[0]], 0),
                      ref("weight", const_cast<float *>(w), g.nodes[x.in[1]], 0),
                      ref("bias", const_cast<float *>(b), g.nodes[x.in[2]], 0),
                      ref_flat("running_mean", rm, C, 0), ref_flat("running_variance", rv, C, 0),
                      ref("y", out, x, 1), ref_flat("inverse_std", inv, C, 1)};
        op.attrs = {{"epsilon", kBnEpsilon}};
        op.launch = [=](hipStream_t st) {
          oxh_status r = oxh_batch_norm_running_inverse_std(st, C, kBnEpsilon, rv, inv);
          if (r != OXH_OK) return r;
          return oxh_batch_norm_apply(st, N, C, HW, xi, w, b, rm, inv, out);
        };
        break;
      }
      case Op::Relu: {
        const float *xi = e.value[x.in[0]];
        const uint64_t cnt = x.numel();
        op.kind = "relu_forward";
        op.name = "relu" + std::to_string(i);
        op.tensors = {ref("x", const_cast<float *>(xi), g.nodes[x.in[0]], 0), ref("y", out, x, 1)};
        op.launch = [xi, out, cnt](hipStream_t st) { return oxh_relu(st, xi, out, cnt); };
        break;
      }
      case Op::Add: {
        const float *p = e.value[x.in[0]], *q = e.value[x.in[1]];
        const uint64_t cnt = x.numel();
        op.kind = "add_forward";
        op.name = "add" + std::to_string(i);
        op.tensors = {ref("a", const_cast<float *>(p), g.nodes[x.in[0]], 0),
                      ref("b", const_cast<float *>(q), g.nodes[x.in[1]], 0), ref("y", out, x, 1)};
        op.launch = [p, q, out, cnt](hipStream_t st) { return oxh_add(st, p, q, out, cnt); };
        break;
      }
      case Op::Pool: {
        const Node &xin = g.nodes[x.in[0]];
        const oxh_pool2d_shape ps{xin.shape[0], xin.shape[1], xin.shape[2], xin.shape[3],
                                  xin.shape[2], xin.shape[3], xin.shape[2], xin.shape[3]};
        const float *xi = e.value[x.in[0]];
        op.kind = "avg_pool2d_forward";
        op.name = "pool" + std::to_string(i);
        op.tensors = {ref("x", const_cast<float *>(xi), xin, 0), ref("y", out, x, 1)};
        op.attrs = {{"kernel_h", static_cast<double>(xin.shape[2])},
                    {"kernel_w", static_cast<double>(xin.shape[3])},
                    {"stride_h", static_cast<double>(xin.shape[2])},
                    {"stride_w", static_cast<double>(xin.shape[3])}};
        op.launch = [ps, xi, out](hipStream_t st) {
          return oxh_avg_pool2d_forward(st, &ps, xi, out);
        };
        break;
      }
      default:
        return oxh::fail(OXH_TRACE, "no inference forward for a traced node");
    }
    ops.push_back(std::move(op));
  }
  return e.program.finalize();
}

oxh_status make_stream(hipStream_t &s) {
  OXH_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  return oxh::ok();
}

}  // namespace

extern "C" {

oxh_status oxh_mnv4_create(uint64_t num_classes, uint64_t input_channels,
                           uint64_t input_resolution, oxh_model **model) {
  OXH_REQUIRE(model != nullptr, OXH_INVALID_SHAPE, "model out-pointer is null");
  *model = nullptr;
  std::unique_ptr<oxh_model> m(new oxh_model());
  oxh_status st = build_model(*m, num_classes, input_channels, input_resolution);
  if (st != OXH_OK) return st;
  st = upload_model(*m);
  if (st != OXH_OK) return st;
  *model = m.release();
  return oxh::ok();
}

oxh_status oxh_mnv4_describe(uint64_t num_classes, uint64_t input_channels,
                             uint64_t input_resolution, uint64_t batch, uint64_t *parameters,
                             uint64_t *values, uint64_t *batch_norms, uint64_t *block_shapes,
                             uint64_t capacity, uint64_t *blocks) {
  OXH_REQUIRE(batch > 0, OXH_INVALID_SHAPE, "batch must be positive");
  oxh_model m;
  oxh_status st = build_model(m, num_classes, input_channels, input_resolution);
  if (st != OXH_OK) return st;
  uint64_t total = 0;
  for (const Param &p : m.params) total += p.n;
  if (parameters) *parameters = m.params.size();
  if (values) *values = total;
  if (batch_norms) *batch_norms = m.bns.size();
  Graph g;
  Node in{Op::Input, {}};
  in.shape = {batch, input_channels, input_resolution, input_resolution};
  const int x = g.add(in);
  std::vector<std::array<uint64_t, 4>> shapes;
  trace_forward(g, m, x, &shapes);
  if (blocks) *blocks = shapes.size();
  OXH_REQUIRE(block_shapes != nullptr || capacity == 0, OXH_INVALID_SHAPE, "shapes is null");
  for (size_t i = 0; i < shapes.size() && i < capacity; ++i)
    for (int d = 0; d < 4; ++d) block_shapes[i * 4 + d] = shapes[i][d];
  return oxh::ok();
}

oxh_status oxh_model_destroy(oxh_model *model) {
  delete model;  // the last error stays untouched
  return OXH_OK;
}

oxh_status oxh_model_info(const oxh_model *model, uint64_t *parameters, uint64_t *batch_norms,
                          uint64_t *values, int *training) {
  OXH_REQUIRE(model != nullptr, OXH_INVALID_SHAPE, "model is null");
  uint64_t total = 0;
  for (const Param &p : model->params) total += p.n;
  if (parameters) *parameters = model->params.size();
  if (batch_norms) *batch_norms = model->bns.size();
  if (values) *values = total;
  if (training) *training = model->training ? 1 : 0;
  return oxh::ok();
}

oxh_status oxh_model_parameter(const oxh_model *model, uint64_t index, uint64_t *rank,
                               uint64_t shape[4], float **device_values) {
  OXH_REQUIRE(model != nullptr && index < model->params.size(), OXH_INVALID_SHAPE,
              "parameter index out of range");
  const Param &p = model->params[index];
  if (rank) *rank = p.shape.size();
  if (shape)
    for (size_t i = 0; i < 4; ++i) shape[i] = i < p.shape.size() ? p.shape[i] : 1;
  if (device_values) *device_values = p.value;
  return oxh::ok();
}

oxh_status oxh_model_batch_norm(const oxh_model *model, uint64_t index, uint64_t *channels,
                                float **running_mean, float **running_variance) {
  OXH_REQUIRE(model != nullptr && index < model->bns.size(), OXH_INVALID_SHAPE,
              "batch norm index out of range");
  const BnState &b = model->bns[index];
  if (channels) *channels = b.channels;
  if (running_mean) *running_mean = b.rm;
  if (running_variance) *running_variance = b.rv;
  return oxh::ok();
}

oxh_status oxh_model_set_training(oxh_model *model, int training) {
  OXH_REQUIRE(model != nullptr, OXH_INVALID_SHAPE, "model is null");
  model->training = training != 0;
  return oxh::ok();
}

oxh_status oxh_model_save(oxh_model *model, const char *path) {
  OXH_REQUIRE(model != nullptr && path != nullptr, OXH_INVALID_SHAPE, "null argument");
  oxh_status st = sync_model(*model);
  if (st != OXH_OK) return st;
  std::vector<oxh_checkpoint_tensor> table;
  std::vector<std::array<uint64_t, 1>> channel_shapes(model->bns.size());
  for (const Param &p : model->params)
    table.push_back(oxh_checkpoint_tensor{p.shape.size(), p.shape.data(), p.n, p.host.data()});
  for (size_t i = 0; i < model->bns.size(); ++i) {
    const BnState &b = model->bns[i];
    channel_shapes[i][0] = b.channels;
    table.push_back(oxh_checkpoint_tensor{1, channel_shapes[i].data(), b.channels,
                                          b.running_mean.data()});
    table.push_back(oxh_checkpoint_tensor{1, channel_shapes[i].data(), b.channels,
                                          b.running_variance.data()});
  }
  return oxh_checkpoint_save(path, table.data(), table.size());
}

oxh_status oxh_model_load_mnist(const char *path, oxh_model **model) {
  OXH_REQUIRE(path != nullptr && model != nullptr, OXH_INVALID_SHAPE, "null argument");
  *model = nullptr;
  oxh_checkpoint *ck = nullptr;
  oxh_status st = oxh_checkpoint_load(path, &ck);
  if (st != OXH_OK) return st;
  std::unique_ptr<oxh_checkpoint, oxh_status (*)(oxh_checkpoint *)> guard(ck, oxh_checkpoint_free);
  std::unique_ptr<oxh_model> m(new oxh_model());
  st = build_model(*m, 10, 1, 28);
  if (st != OXH_OK) return st;
  uint64_t count = 0;
  oxh_checkpoint_count(ck, &count);
  uint64_t next = 0;
  auto entry = [&](uint64_t i, std::vector<uint64_t> &shape, const float *&data, uint64_t &len) {
    uint64_t rank = 0;
    const uint64_t *dims = nullptr;
    oxh_checkpoint_entry(ck, i, &rank, &dims, &len, &data);
    shape.assign(dims, dims + rank);
  };
  // mobilenet_v4.rs:271-321
  for (Param &p : m->params) {
    OXH_REQUIRE(next < count, OXH_EXECUTION, "checkpoint has too few tensors");
    std::vector<uint64_t> shape;
    const float *data = nullptr;
    uint64_t len = 0;
    entry(next, shape, data, len);
    OXH_REQUIRE(shape == p.shape, OXH_INVALID_SHAPE,
                "checkpoint tensor " + std::to_string(next) + " has a different shape");
    OXH_REQUIRE(len == p.n, OXH_INVALID_SHAPE, "data length does not match the shape");
    p.host.assign(data, data + len);
    ++next;
  }
  for (BnState &b : m->bns) {
    for (std::vector<float> *buffer : {&b.running_mean, &b.running_variance}) {
      OXH_REQUIRE(next < count, OXH_EXECUTION, "checkpoint has too few buffers");
      std::vector<uint64_t> shape;
      const float *data = nullptr;
      uint64_t len = 0;
      entry(next, shape, data, len);
      OXH_REQUIRE(shape == std::vector<uint64_t>{b.channels} && len == b.channels,
                  OXH_INVALID_SHAPE,
                  "checkpoint buffer " + std::to_string(next) + " shape mismatch");
      buffer->assign(data, data + len);
      ++next;
    }
  }
  OXH_REQUIRE(next == count, OXH_EXECUTION, "checkpoint has extra tensors");
  st = upload_model(*m);
  if (st != OXH_OK) return st;
  m->training = false;  // model.eval()
  *model = m.release();
  return oxh::ok();
}

// ---- trainer

oxh_status oxh_trainer_create(oxh_model *model, uint64_t batch, float learning_rate,
                              float weight_decay, oxh_trainer **trainer) {
  OXH_REQUIRE(model != nullptr && trainer != nullptr, OXH_INVALID_SHAPE, "null argument");
  *trainer = nullptr;
  OXH_REQUIRE(batch > 0 && batch < (1u << 20), OXH_INVALID_SHAPE, "batch must be in 1..2^20");
  // optim.rs:54-65
  OXH_REQUIRE(std::isfinite(learning_rate) && learning_rate > 0.0f, OXH_INVALID_SHAPE,
              "AdamW learning rate must be positive and finite");
  OXH_REQUIRE(std::isfinite(weight_decay) && weight_decay >= 0.0f, OXH_INVALID_SHAPE,
              "AdamW weight decay must be non-negative and finite");
  OXH_REQUIRE(model->training, OXH_EXECUTION, "the model is in inference mode");
  std::unique_ptr<oxh_trainer> t(new oxh_trainer());
  t->model = model;
  t->batch = batch;
  t->lr = learning_rate;
  t->wd = weight_decay;
  oxh_status st = make_stream(t->program.stream);
  if (st != OXH_OK) return st;
  st = build_trainer(*t);
  if (st != OXH_OK) return st;
  *trainer = t.release();
  return oxh::ok();
}

oxh_status oxh_trainer_destroy(oxh_trainer *trainer) {
  if (trainer) (void)hipStreamSynchronize(trainer->program.stream);
  delete trainer;  // the last error stays untouched
  return OXH_OK;
}

oxh_status oxh_trainer_buffers(const oxh_trainer *t, float **images, float **labels,
                               float **logits, float **loss) {
  OXH_REQUIRE(t != nullptr, OXH_INVALID_SHAPE, "trainer is null");
  if (images) *images = t->value[t->input];
  if (labels) *labels = t->value[t->targets];
  if (logits) *logits = t->value[t->logits];
  if (loss) *loss = t->loss;
  return oxh::ok();
}

oxh_status oxh_trainer_program(oxh_trainer *t, oxh_program **program) {
  OXH_REQUIRE(t != nullptr && program != nullptr, OXH_INVALID_SHAPE, "null argument");
  *program = &t->program;
  return oxh::ok();
}

oxh_status oxh_trainer_loss(oxh_trainer *t, float *loss) {
  OXH_REQUIRE(t != nullptr && loss != nullptr, OXH_INVALID_SHAPE, "null argument");
  OXH_HIP_CHECK(hipStreamSynchronize(t->program.stream));
  uint32_t flag = 0;
  OXH_HIP_CHECK(hipMemcpy(&flag, t->error_flag, 4, hipMemcpyDeviceToHost));
  if (flag != 0) {
    OXH_HIP_CHECK(hipMemset(t->error_flag, 0, 4));
    return oxh::fail(OXH_INVALID_SHAPE, "cross entropy target is not a class index");
  }
  OXH_HIP_CHECK(hipMemcpy(loss, t->loss, 4, hipMemcpyDeviceToHost));
  return oxh::ok();
}

oxh_status oxh_trainer_steps(oxh_trainer *t, int32_t *steps) {
  OXH_REQUIRE(t != nullptr && steps != nullptr, OXH_INVALID_SHAPE, "null argument");
  OXH_HIP_CHECK(hipStreamSynchronize(t->program.stream));
  OXH_HIP_CHECK(hipMemcpy(steps, t->step, 4, hipMemcpyDeviceToHost));
  return oxh::ok();
}

// ---- evaluator

oxh_status oxh_evaluator_create(oxh_model *model, uint64_t batch, oxh_evaluator **evaluator) {
  OXH_REQUIRE(model != nullptr && evaluator != nullptr, OXH_INVALID_SHAPE, "null argument");
  *evaluator = nullptr;
  OXH_REQUIRE(batch > 0 && batch < (1u << 20), OXH_INVALID_SHAPE, "batch must be in 1..2^20");
  std::unique_ptr<oxh_evaluator> e(new oxh_evaluator());
  e->model = model;
  e->batch = batch;
  oxh_status st = make_stream(e->program.stream);
  if (st != OXH_OK) return st;
  st = build_evaluator(*e);
  if (st != OXH_OK) return st;
  *evaluator = e.release();
  return oxh::ok();
}

oxh_status oxh_evaluator_destroy(oxh_evaluator *e) {
  if (e) (void)hipStreamSynchronize(e->program.stream);
  delete e;  // the last error stays untouched
  return OXH_OK;
}

oxh_status oxh_evaluator_buffers(const oxh_evaluator *e, float **images, float **logits,
                                 uint32_t **predictions) {
  OXH_REQUIRE(e != nullptr, OXH_INVALID_SHAPE, "evaluator is null");
  if (images) *images = e->value[e->input];
  if (logits) *logits = e->value[e->logits];
  if (predictions) *predictions = e->classes;
  return oxh::ok();
}

oxh_status oxh_evaluator_program(oxh_evaluator *e, oxh_program **program) {
  OXH_REQUIRE(e != nullptr && program != nullptr, OXH_INVALID_SHAPE, "null argument");
  *program = &e->program;
  return oxh::ok();
}

// count_correct's argmax (mnist_training.rs:201-218) of the last logits, on the device.
oxh_status oxh_evaluator_predict(oxh_evaluator *e) {
  OXH_REQUIRE(e != nullptr, OXH_INVALID_SHAPE, "evaluator is null");
  return oxh_argmax_rows(e->program.stream, e->batch, e->model->classes, e->value[e->logits],
                         e->classes);
}

// ---- programs

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
  const OpRec &op = p->ops[index];
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
