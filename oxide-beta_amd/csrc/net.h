// net.h -- the traced graph and the device programs built from it (internal to the library).
//
// A Graph is the reference's lazy Tensor graph (crates/oxide-torch/src/tensor/graph.rs:70-139,
// the ops the hot path and the convolutional models use) recorded node by node in creation
// order, which is a topological order: leaves (inputs fed per run, trainable parameters,
// constants; caller-owned device values) and Conv2d / BatchNorm2d / ReLU / Add / Mul /
// AvgPool2d / Reshape / CrossEntropy nodes with the builders' shape rules
// (tensor/mod.rs:103-389).  A program is a fixed list of launch groups over buffers carved
// from one device allocation:
//   * forward program: the eager device evaluation of a node (runtime.rs:125-379), used for
//     inference and for JIT plans the fused-plan compiler cannot take (jit.rs:205-207,226-243);
//   * training program: forward, then reverse-mode from a one-element root in reverse
//     topological order (runtime.rs:1198-1217,1388-1476,694-860) with a value's first
//     gradient contribution written in place and later ones accumulated (671-692), and
//     optionally one AdamW launch over every parameter that received a gradient
//     (optim.rs:78-152, runtime.rs:1306-1386).
#pragma once

#include <hip/hip_runtime.h>

#include <array>
#include <functional>
#include <string>
#include <utility>
#include <vector>

#include "common.h"

namespace oxh {
namespace net {

// ---------------------------------------------------------------- device arena

// Offsets are planned first, then one hipMalloc serves them all (zero-filled).
struct Arena {
  uint64_t size = 0;
  char *base = nullptr;
  uint64_t reserve(uint64_t bytes) {
    const uint64_t at = size;
    size += (bytes + 255) / 256 * 256;
    return at;
  }
  oxh_status allocate();
  template <typename T>
  T *at(uint64_t offset) const {
    return reinterpret_cast<T *>(base + offset);
  }
  Arena() = default;
  Arena(const Arena &) = delete;
  Arena &operator=(const Arena &) = delete;
  ~Arena();
};

// ---------------------------------------------------------------- graph

enum class Op { Input, Param, Constant, Conv, Bn, Relu, Add, Mul, Pool, Reshape, CrossEntropy };

struct Node {
  Node(Op o, std::vector<int> i) : op(o), in(std::move(i)) {}
  Op op;
  std::vector<int> in;
  std::array<uint64_t, 4> shape{1, 1, 1, 1};
  uint32_t rank = 4;
  float *data = nullptr;       // Param / Constant: caller-owned device values
  bool requires_grad = false;  // Input: the program forms its gradient
  uint32_t stride = 1, pad = 0, groups = 1;                            // Conv
  uint32_t kernel_h = 1, kernel_w = 1, stride_h = 1, stride_w = 1;     // Pool
  float *running_mean = nullptr, *running_variance = nullptr;          // Bn (device, in place)
  bool training = true;
  float momentum = 0.1f, epsilon = 1e-5f;
  uint64_t numel() const {
    uint64_t n = 1;
    for (uint32_t i = 0; i < rank; ++i) n *= shape[i];
    return n;
  }
  bool leaf() const { return op == Op::Input || op == Op::Param || op == Op::Constant; }
};

struct Graph {
  std::vector<Node> nodes;
  std::vector<int> params;  // trainable parameter nodes, creation order (the optimizer's)
  int add(Node n) {
    nodes.push_back(std::move(n));
    return static_cast<int>(nodes.size()) - 1;
  }
};

// Builders (the reference's shape and argument rules); the new node's index goes to *node.
oxh_status input(Graph &g, uint32_t rank, const uint64_t *shape, bool requires_grad, int *node);
oxh_status leaf_values(Graph &g, uint32_t rank, const uint64_t *shape, float *values,
                       bool trainable, int *node);
oxh_status binary(Graph &g, Op op, int a, int b, int *node);
oxh_status relu(Graph &g, int x, int *node);
oxh_status reshape(Graph &g, int x, uint32_t rank, const uint64_t *shape, int *node);
oxh_status conv2d(Graph &g, int x, int weight, int bias, uint64_t stride, uint64_t padding,
                  uint64_t groups, int *node);
oxh_status avg_pool2d(Graph &g, int x, uint64_t kernel_h, uint64_t kernel_w, uint64_t stride_h,
                      uint64_t stride_w, int *node);
oxh_status batch_norm2d(Graph &g, int x, int weight, int bias, float *running_mean,
                        float *running_variance, bool training, float momentum, float epsilon,
                        int *node);
oxh_status cross_entropy(Graph &g, int logits, int targets, int *node);

struct AdamConfig {
  float learning_rate = 1e-3f, weight_decay = 0.01f, beta1 = 0.9f, beta2 = 0.999f,
        epsilon = 1e-8f;
};

// ---------------------------------------------------------------- launch records

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
  // Where set, what the whole program runs (run, capture) in place of `launch`: the same
  // values, with work moved to a later group of the program (a convolution's weight-gradient
  // chunk sums, run with every other convolution's before the optimizer step).  `launch` alone
  // (oxh_program_run_op) always leaves every output of the group formed.
  std::function<oxh_status(hipStream_t)> program_launch;
  // C views of the above, built once
  std::vector<oxh_op_tensor> c_tensors;
  std::vector<oxh_op_attr> c_attrs;
};

oxh_status make_stream(hipStream_t &s);

}  // namespace net
}  // namespace oxh

// A fixed launch list with the buffers it runs over (one arena), its stream and, once
// captured, its graph.
struct oxh_program {
  std::vector<oxh::net::OpRec> ops;
  hipStream_t stream = nullptr;
  oxh_graph *graph = nullptr;
  bool owned = false;  // created by oxh_net_*_program: released by oxh_program_destroy
  oxh::net::Arena arena;
  // per node of the graph the program was built from (null: none)
  std::vector<float *> value, grad, saved_mean, saved_inv;
  int root = -1;
  // optimizer (training programs with AdamW)
  bool has_adam = false;
  oxh::net::AdamConfig adam_config;
  std::vector<oxh_adamw_tensor> adam;
  oxh_adamw_tensor *adam_table = nullptr;  // device copy of `adam`
  uint32_t *adam_starts = nullptr;
  uint64_t adam_chunks = 0;
  int32_t *step = nullptr;
  uint32_t *error_flag = nullptr;  // raised by a cross entropy with an invalid target
  // chunk sums the program's convolutions leave to the optimizer group, recorded by each run
  std::vector<oxh::ChunkSum> deferred_sums;

  oxh_status finalize();
  oxh_status run();
  oxh_status capture();
  ~oxh_program();
};

namespace oxh {
namespace net {

// Programs over `g` (which must outlive nothing: the program copies what it needs).  The
// program's stream must be set before building.
oxh_status build_forward(const Graph &g, int output, oxh_program &p);
oxh_status build_training(const Graph &g, int root, const AdamConfig *adam, oxh_program &p);

}  // namespace net
}  // namespace oxh
