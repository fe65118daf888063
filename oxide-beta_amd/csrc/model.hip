// model.hip -- MobileNetV4-Conv-S and its MNIST training step: the model (parameters and
// BatchNorm state resident on the device), its forward traced through the graph builders of
// net.h, a trainer (the traced training step as a training program: forward, cross entropy,
// reverse-mode backward, one AdamW launch, replayed from one hipGraph), an inference-mode
// evaluator (a forward program with BatchNorm from the running statistics), and OXTR save /
// load at model level.  Host C++ over this library's own C ABI.
//
// Reference: MobileNetV4ConvSmall (crates/oxide-torch-models/src/models/mobilenet_v4.rs:84-321)
// built from Conv2d / BatchNorm2d / ConvNormAct / UniversalInvertedBottleneck /
// FusedInvertedBottleneck (crates/oxide-torch/src/nn.rs:107-655); the training step of
// examples/mnist_training.rs:75-92 (zero_grad, forward, cross_entropy, backward, AdamW with
// lr 1e-3, weight decay 1e-4, betas 0.9 / 0.999, eps 1e-8, optim.rs:48-127).  The schedule and
// its launch-saving rewrites are net.hip's; every device buffer of a trainer or evaluator is
// carved from one allocation made at creation, nothing is allocated per step.
#include <hip/hip_runtime.h>

#include <array>
#include <cmath>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "common.h"
#include "net.h"

namespace {

constexpr float kBnMomentum = 0.1f, kBnEpsilon = 1e-5f;

using oxh::net::Arena;
namespace net = oxh::net;

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

// ---------------------------------------------------------------- traced forward

// Traces the model through the graph builders.  Parameters become graph leaves at their first
// use (the lazy graph's order); `shapes_only` traces with stand-in device pointers (no program
// is built from such a graph).
struct Tracer {
  net::Graph &g;
  const oxh_model &m;
  bool training;
  bool shapes_only = false;
  std::vector<int> param_node;
  float *stand_in() {
    static float unused;
    return &unused;
  }
  oxh_status param(int p, int *node) {
    if (param_node.empty()) param_node.assign(m.params.size(), -1);
    if (param_node[p] < 0) {
      const Param &pr = m.params[p];
      oxh_status st = net::leaf_values(g, static_cast<uint32_t>(pr.shape.size()),
                                       pr.shape.data(), shapes_only ? stand_in() : pr.value,
                                       true, &param_node[p]);
      if (st != OXH_OK) return st;
    }
    *node = param_node[p];
    return oxh::ok();
  }
};

// nn.rs:288-297 (Conv2d::forward)
oxh_status trace_conv(Tracer &t, int x, const ConvLayer &c, int *out) {
  int w = -1, b = -1;
  oxh_status st = t.param(c.weight, &w);
  if (st == OXH_OK) st = t.param(c.bias, &b);
  if (st != OXH_OK) return st;
  return net::conv2d(t.g, x, w, b, c.stride, c.pad, c.groups, out);
}

// nn.rs:386-397 (ConvNormAct::forward): conv, BatchNorm2d, optional ReLU
oxh_status trace_cna(Tracer &t, int x, const ConvNormAct &l, int *out) {
  int c = -1, w = -1, b = -1, y = -1;
  oxh_status st = trace_conv(t, x, l.conv, &c);
  const BnState &bs = t.m.bns[l.bn];
  if (st == OXH_OK) st = t.param(bs.weight, &w);
  if (st == OXH_OK) st = t.param(bs.bias, &b);
  if (st == OXH_OK)
    st = net::batch_norm2d(t.g, c, w, b, t.shapes_only ? t.stand_in() : bs.rm,
                           t.shapes_only ? t.stand_in() : bs.rv, t.training, kBnMomentum,
                           kBnEpsilon, &y);
  if (st == OXH_OK && l.relu) st = net::relu(t.g, y, &y);
  *out = y;
  return st;
}

// mobilenet_v4.rs:182-195: the logits [N, classes], every block's output shape recorded.
oxh_status trace_forward(Tracer &t, int x, int *logits,
                         std::vector<std::array<uint64_t, 4>> *shapes) {
  oxh_status st = oxh::ok();
  for (const Block &b : t.m.blocks) {
    const int input = x;
    switch (b.kind) {
      case BlockKind::Conv:
      case BlockKind::Fused:
      case BlockKind::Uib:
        for (const ConvNormAct &l : b.layers)
          if (st == OXH_OK) st = trace_cna(t, x, l, &x);
        if (st == OXH_OK && b.residual) st = net::binary(t.g, net::Op::Add, x, input, &x);
        break;
      case BlockKind::GlobalAverage: {  // tensor/mod.rs:273-283
        const auto &s = t.g.nodes[x].shape;
        st = net::avg_pool2d(t.g, x, s[2], s[3], s[2], s[3], &x);
        break;
      }
      case BlockKind::Classifier:
        st = trace_conv(t, x, b.classifier, &x);
        break;
    }
    if (st != OXH_OK) return st;
    if (shapes) shapes->push_back(t.g.nodes[x].shape);
  }
  const uint64_t logit_shape[2] = {t.g.nodes[x].shape[0], t.m.classes};
  st = net::reshape(t.g, x, 2, logit_shape, logits);
  if (st == OXH_OK && shapes) shapes->back() = t.g.nodes[*logits].shape;
  return st;
}

}  // namespace

struct oxh_trainer {
  oxh_model *model = nullptr;
  uint64_t batch = 0;
  net::Graph g;
  oxh_program program;
  int input = -1, targets = -1, logits = -1, loss_node = -1;
};

struct oxh_evaluator {
  oxh_model *model = nullptr;
  uint64_t batch = 0;
  net::Graph g;
  oxh_program program;
  Arena arena;  // the predictions
  uint32_t *classes = nullptr;
  int input = -1, logits = -1;
};

namespace {

// examples/mnist_training.rs:75-92: images -> logits -> cross entropy (the backward root) ->
// AdamW over every parameter.
oxh_status build_trainer(oxh_trainer &t, float learning_rate, float weight_decay) {
  oxh_model &m = *t.model;
  const uint64_t image[4] = {t.batch, m.in_channels, m.resolution, m.resolution};
  oxh_status st = net::input(t.g, 4, image, false, &t.input);
  Tracer tr{t.g, m, true, false, {}};
  if (st == OXH_OK) st = trace_forward(tr, t.input, &t.logits, nullptr);
  const uint64_t labels[1] = {t.batch};
  if (st == OXH_OK) st = net::input(t.g, 1, labels, false, &t.targets);
  if (st == OXH_OK) st = net::cross_entropy(t.g, t.logits, t.targets, &t.loss_node);
  if (st != OXH_OK) return st;
  const net::AdamConfig adam{learning_rate, weight_decay, 0.9f, 0.999f, 1e-8f};
  return net::build_training(t.g, t.loss_node, &adam, t.program);
}

oxh_status build_evaluator(oxh_evaluator &e) {
  oxh_model &m = *e.model;
  const uint64_t image[4] = {e.batch, m.in_channels, m.resolution, m.resolution};
  oxh_status st = net::input(e.g, 4, image, false, &e.input);
  Tracer tr{e.g, m, false, false, {}};
  if (st == OXH_OK) st = trace_forward(tr, e.input, &e.logits, nullptr);
  if (st == OXH_OK) st = net::build_forward(e.g, e.logits, e.program);
  if (st != OXH_OK) return st;
  const uint64_t off = e.arena.reserve(e.batch * 4);
  st = e.arena.allocate();
  if (st != OXH_OK) return st;
  e.classes = e.arena.at<uint32_t>(off);
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
  net::Graph g;
  const uint64_t image[4] = {batch, input_channels, input_resolution, input_resolution};
  int x = -1, logits = -1;
  st = net::input(g, 4, image, false, &x);
  if (st != OXH_OK) return st;
  std::vector<std::array<uint64_t, 4>> shapes;
  Tracer tr{g, m, true, true, {}};
  st = trace_forward(tr, x, &logits, &shapes);
  if (st != OXH_OK) return st;
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
  OXH_REQUIRE(std::isfinite(learning_rate) && learning_rate > 0.0f, OXH_EXECUTION,
              "AdamW learning rate must be positive and finite");
  OXH_REQUIRE(std::isfinite(weight_decay) && weight_decay >= 0.0f, OXH_EXECUTION,
              "AdamW weight decay must be non-negative and finite");
  OXH_REQUIRE(model->training, OXH_EXECUTION, "the model is in inference mode");
  std::unique_ptr<oxh_trainer> t(new oxh_trainer());
  t->model = model;
  t->batch = batch;
  oxh_status st = net::make_stream(t->program.stream);
  if (st != OXH_OK) return st;
  st = build_trainer(*t, learning_rate, weight_decay);
  if (st != OXH_OK) return st;
  *trainer = t.release();
  return oxh::ok();
}

oxh_status oxh_trainer_destroy(oxh_trainer *trainer) {
  delete trainer;  // the program waits for its stream; the last error stays untouched
  return OXH_OK;
}

oxh_status oxh_trainer_buffers(const oxh_trainer *t, float **images, float **labels,
                               float **logits, float **loss) {
  OXH_REQUIRE(t != nullptr, OXH_INVALID_SHAPE, "trainer is null");
  if (images) *images = t->program.value[t->input];
  if (labels) *labels = t->program.value[t->targets];
  if (logits) *logits = t->program.value[t->logits];
  if (loss) *loss = t->program.value[t->loss_node];
  return oxh::ok();
}

oxh_status oxh_trainer_program(oxh_trainer *t, oxh_program **program) {
  OXH_REQUIRE(t != nullptr && program != nullptr, OXH_INVALID_SHAPE, "null argument");
  *program = &t->program;
  return oxh::ok();
}

oxh_status oxh_trainer_loss(oxh_trainer *t, float *loss) {
  OXH_REQUIRE(t != nullptr && loss != nullptr, OXH_INVALID_SHAPE, "null argument");
  oxh_status st = oxh_program_check(&t->program);
  if (st != OXH_OK) return st;
  OXH_HIP_CHECK(hipMemcpy(loss, t->program.value[t->loss_node], 4, hipMemcpyDeviceToHost));
  return oxh::ok();
}

oxh_status oxh_trainer_steps(oxh_trainer *t, int32_t *steps) {
  OXH_REQUIRE(t != nullptr && steps != nullptr, OXH_INVALID_SHAPE, "null argument");
  return oxh_program_steps(&t->program, steps);
}

// ---- evaluator

oxh_status oxh_evaluator_create(oxh_model *model, uint64_t batch, oxh_evaluator **evaluator) {
  OXH_REQUIRE(model != nullptr && evaluator != nullptr, OXH_INVALID_SHAPE, "null argument");
  *evaluator = nullptr;
  OXH_REQUIRE(batch > 0 && batch < (1u << 20), OXH_INVALID_SHAPE, "batch must be in 1..2^20");
  std::unique_ptr<oxh_evaluator> e(new oxh_evaluator());
  e->model = model;
  e->batch = batch;
  oxh_status st = net::make_stream(e->program.stream);
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
  if (images) *images = e->program.value[e->input];
  if (logits) *logits = e->program.value[e->logits];
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
  return oxh_argmax_rows(e->program.stream, e->batch, e->model->classes,
                         e->program.value[e->logits], e->classes);
}

}  // extern "C"
