// plan.hip -- fixed-buffer execution plans captured into a HIP graph.
//
// Host-side counterpart of the reference's CudaJitPlan (crates/oxide-torch/src/cuda/jit.rs:
// 10-99) over its GraphPlan (crates/oxide-torch/src/jit.rs:24-56):
//   compile: one dedicated non-default stream (cuda/jit.rs:27-30), every Input / Workspace
//            buffer allocated zeroed and every Constant uploaded (34-45), the operation list
//            recorded once into a graph and instantiated (47-55);
//   run:     inputs copied host-to-device into their fixed buffers, one graph replay, the
//            output copied back synchronously (70-99);
//   replay:  one launch of the graph alone, for callers whose inputs are already resident;
//   launch:  the graph's launches issued directly on the plan's stream (no graph launch).
// Plan operations are the reference's Add / Mul / Relu plus the backward elementwise kernels.
// compile fuses each run of operations in which every operation consumes the previous one's
// result (and reads no buffer an earlier operation of the run wrote) into one streaming kernel
// (chain.h): the same fp32 operation per element and step, so the output is bit-identical to
// the separate launches; a workspace read only inside its run is never written (it lives in
// registers).  Single operations go through this library's C ABI launchers.
#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "chain.h"
#include "common.h"

namespace {

enum class BufferKind { Input, Constant, Workspace };

struct Buffer {
  BufferKind kind;
  uint64_t elements;
  std::vector<float> constant;
  float *device = nullptr;
};

struct Operation {
  uint32_t op;
  std::vector<uint32_t> inputs;
  uint32_t output;
};

int arity(uint32_t op) {
  switch (op) {
    case OXH_PLAN_ADD:
    case OXH_PLAN_MUL:
    case OXH_PLAN_RELU_BACKWARD:
    case OXH_PLAN_MUL_BACKWARD:
    case OXH_PLAN_ACCUMULATE:
      return 2;
    case OXH_PLAN_RELU:
      return 1;
    default:
      return -1;
  }
}

}  // namespace

struct oxh_plan {
  int device = 0;
  std::vector<Buffer> buffers;
  std::vector<Operation> operations;
  std::vector<uint32_t> inputs;  // input slots in creation order
  int64_t output = -1;
  hipStream_t stream = nullptr;
  oxh_graph *graph = nullptr;
  std::vector<std::pair<size_t, size_t>> launches;  // compiled launch groups [begin, end)
  bool compiled = false;
};

namespace {

oxh_status launch_operation(const oxh_plan &p, const Operation &o) {
  const float *in0 = p.buffers[o.inputs[0]].device;
  const float *in1 = o.inputs.size() > 1 ? p.buffers[o.inputs[1]].device : nullptr;
  float *out = p.buffers[o.output].device;
  const uint64_t n = p.buffers[o.output].elements;
  oxh_stream s = p.stream;
  switch (o.op) {
    case OXH_PLAN_ADD: return oxh_add(s, in0, in1, out, n);
    case OXH_PLAN_MUL: return oxh_mul(s, in0, in1, out, n);
    case OXH_PLAN_RELU: return oxh_relu(s, in0, out, n);
    case OXH_PLAN_RELU_BACKWARD: return oxh_relu_backward(s, in0, in1, out, n);
    case OXH_PLAN_MUL_BACKWARD: return oxh_mul_backward(s, in0, in1, out, n);
    case OXH_PLAN_ACCUMULATE: return oxh_accumulate(s, in0, in1, out, n);
    default: return oxh::fail(OXH_TRACE, "unknown plan operation");
  }
}

// Runs of fusable operations, [begin, end) in plan order.
struct Run {
  size_t begin, end;
};

std::vector<Run> form_runs(const oxh_plan &p) {
  std::vector<Run> runs;
  const auto &ops = p.operations;
  size_t i = 0;
  while (i < ops.size()) {
    size_t j = i + 1;
    std::vector<uint32_t> written = {ops[i].output};
    while (j < ops.size() && j - i < static_cast<size_t>(oxh::kChainMax)) {
      const Operation &o = ops[j];
      const uint32_t prev = ops[j - 1].output;
      int pos = -1;
      for (size_t q = 0; q < o.inputs.size(); ++q)
        if (o.inputs[q] == prev) {
          pos = static_cast<int>(q);
          break;
        }
      if (pos < 0) break;
      bool ok = true;
      for (size_t q = 0; q < o.inputs.size(); ++q) {
        const uint32_t in = o.inputs[q];
        if (in == prev) continue;
        for (uint32_t w : written) ok = ok && in != w;
      }
      if (!ok) break;
      written.push_back(o.output);
      ++j;
    }
    runs.push_back(Run{i, j});
    i = j;
  }
  return runs;
}

// The chain of a run: step k stores its result when no later step of the run writes the
// buffer again and the buffer is the plan output or is read from memory by any operation --
// after the run, or before it (that read sees this replay's value in the next replay) --
// rather than taken as the running value by step k + 1.
oxh_status launch_run(const oxh_plan &p, const Run &r) {
  oxh::Chain c{};
  const auto &ops = p.operations;
  c.first = p.buffers[ops[r.begin].inputs[0]].device;
  c.count = static_cast<uint32_t>(r.end - r.begin);
  uint32_t n_other = 0, n_store = 0;
  for (size_t k = r.begin; k < r.end; ++k) {
    const Operation &o = ops[k];
    oxh::ChainStep &st = c.steps[k - r.begin];
    st.op = o.op;
    st.other = -1;
    st.acc_second = 0;
    st.store = -1;
    if (k == r.begin) {
      if (o.inputs.size() > 1) {
        st.other = static_cast<int32_t>(n_other);
        c.other[n_other++] = p.buffers[o.inputs[1]].device;
      }
    } else {
      const uint32_t prev = ops[k - 1].output;
      if (o.inputs.size() > 1) {
        const bool first_is_acc = o.inputs[0] == prev;
        const uint32_t b = first_is_acc ? o.inputs[1] : o.inputs[0];
        st.acc_second = first_is_acc ? 0u : 1u;
        if (b != prev) {
          st.other = static_cast<int32_t>(n_other);
          c.other[n_other++] = p.buffers[b].device;
        }
      }
    }
    bool needed = static_cast<int64_t>(o.output) == p.output;
    for (size_t q = 0; q < ops.size() && !needed; ++q) {
      if (q == k + 1 && q < r.end) continue;  // the running value, in registers
      for (uint32_t in : ops[q].inputs) needed = needed || in == o.output;
    }
    for (size_t q = k + 1; q < r.end && needed; ++q) needed = ops[q].output != o.output;
    if (needed) {
      st.store = static_cast<int32_t>(n_store);
      c.store[n_store++] = p.buffers[o.output].device;
    }
  }
  // relu((a + b) * c) with only its result stored -- config 1's plan, the reference's own
  // chain -- runs on the dedicated fused kernel: the same three fp32 operations per element in
  // the same order, two float4 per lane per stream (a generic chain keeps one: its step
  // registers would otherwise cost occupancy)
  if (c.count == 3 && c.steps[0].op == OXH_PLAN_ADD && c.steps[0].other == 0 &&
      c.steps[1].op == OXH_PLAN_MUL && c.steps[1].other == 1 && c.steps[2].op == OXH_PLAN_RELU &&
      c.steps[0].store < 0 && c.steps[1].store < 0 && c.steps[2].store == 0 && n_store == 1)
    return oxh_elementwise_chain_forward(p.stream, c.first, c.other[0], c.other[1], c.store[0],
                                         p.buffers[ops[r.begin].output].elements);
  return oxh::launch_chain(p.stream, c, p.buffers[ops[r.begin].output].elements);
}

void release(oxh_plan *p) {
  if (p->graph) (void)oxh_graph_destroy(p->graph);
  p->graph = nullptr;
  for (Buffer &b : p->buffers) {
    if (b.device) (void)hipFree(b.device);
    b.device = nullptr;
  }
  if (p->stream) (void)hipStreamDestroy(p->stream);
  p->stream = nullptr;
  p->compiled = false;
}

oxh_status add_buffer(oxh_plan *plan, Buffer b, uint32_t *slot) {
  OXH_REQUIRE(plan != nullptr && slot != nullptr, OXH_INVALID_SHAPE, "null plan or slot");
  OXH_REQUIRE(!plan->compiled, OXH_TRACE, "plan is already compiled");
  OXH_REQUIRE(b.elements > 0, OXH_INVALID_SHAPE, "plan buffers must be non-empty");
  OXH_REQUIRE(plan->buffers.size() < UINT32_MAX, OXH_INVALID_SHAPE, "too many buffers");
  *slot = static_cast<uint32_t>(plan->buffers.size());
  if (b.kind == BufferKind::Input) plan->inputs.push_back(*slot);
  plan->buffers.push_back(std::move(b));
  return oxh::ok();
}

}  // namespace

extern "C" {

oxh_status oxh_plan_create(int device, oxh_plan **plan) {
  OXH_REQUIRE(plan != nullptr, OXH_INVALID_SHAPE, "plan out-pointer is null");
  OXH_REQUIRE(device >= 0, OXH_INVALID_SHAPE, "negative device");
  *plan = new oxh_plan();
  (*plan)->device = device;
  return oxh::ok();
}

oxh_status oxh_plan_add_input(oxh_plan *plan, uint64_t elements, uint32_t *slot) {
  return add_buffer(plan, Buffer{BufferKind::Input, elements, {}, nullptr}, slot);
}

oxh_status oxh_plan_add_constant(oxh_plan *plan, const float *values, uint64_t elements,
                                 uint32_t *slot) {
  OXH_REQUIRE(values != nullptr || elements == 0, OXH_INVALID_SHAPE, "null constant values");
  return add_buffer(plan,
                    Buffer{BufferKind::Constant, elements,
                           std::vector<float>(values, values + elements), nullptr},
                    slot);
}

oxh_status oxh_plan_add_workspace(oxh_plan *plan, uint64_t elements, uint32_t *slot) {
  return add_buffer(plan, Buffer{BufferKind::Workspace, elements, {}, nullptr}, slot);
}

oxh_status oxh_plan_add_operation(oxh_plan *plan, uint32_t op, const uint32_t *inputs,
                                  uint32_t input_count, uint32_t output) {
  OXH_REQUIRE(plan != nullptr, OXH_INVALID_SHAPE, "null plan");
  OXH_REQUIRE(!plan->compiled, OXH_TRACE, "plan is already compiled");
  const int want = arity(op);
  OXH_REQUIRE(want >= 0, OXH_TRACE, "unknown plan operation " + std::to_string(op));
  OXH_REQUIRE(static_cast<int>(input_count) == want && inputs != nullptr, OXH_TRACE,
              "operation " + std::to_string(op) + " takes " + std::to_string(want) + " inputs");
  const uint64_t nb = plan->buffers.size();
  OXH_REQUIRE(output < nb, OXH_TRACE, "output slot out of range");
  OXH_REQUIRE(plan->buffers[output].kind == BufferKind::Workspace, OXH_TRACE,
              "an operation must write a workspace buffer");
  Operation o{op, {}, output};
  for (uint32_t i = 0; i < input_count; ++i) {
    OXH_REQUIRE(inputs[i] < nb, OXH_TRACE, "input slot out of range");
    OXH_REQUIRE(inputs[i] != output, OXH_TRACE,
                "an operation may not read its own output buffer");
    OXH_REQUIRE(plan->buffers[inputs[i]].elements == plan->buffers[output].elements,
                OXH_INVALID_SHAPE, "elementwise plan operations need equal sizes");
    o.inputs.push_back(inputs[i]);
  }
  plan->operations.push_back(std::move(o));
  return oxh::ok();
}

oxh_status oxh_plan_set_output(oxh_plan *plan, uint32_t slot) {
  OXH_REQUIRE(plan != nullptr, OXH_INVALID_SHAPE, "null plan");
  OXH_REQUIRE(!plan->compiled, OXH_TRACE, "plan is already compiled");
  OXH_REQUIRE(slot < plan->buffers.size(), OXH_TRACE, "output slot out of range");
  plan->output = slot;
  return oxh::ok();
}

oxh_status oxh_plan_compile(oxh_plan *plan) {
  OXH_REQUIRE(plan != nullptr, OXH_INVALID_SHAPE, "null plan");
  OXH_REQUIRE(!plan->compiled, OXH_TRACE, "plan is already compiled");
  OXH_REQUIRE(plan->output >= 0, OXH_TRACE, "plan has no output");
  oxh_status st = oxh_init(plan->device);
  if (st != OXH_OK) return st;
  hipError_t err = hipStreamCreateWithFlags(&plan->stream, hipStreamNonBlocking);
  if (err != hipSuccess) {
    release(plan);
    return oxh::hip_status(err, "hipStreamCreateWithFlags");
  }
  for (Buffer &b : plan->buffers) {
    err = hipMalloc(&b.device, b.elements * sizeof(float));
    if (err == hipSuccess) {
      if (b.kind == BufferKind::Constant)
        err = hipMemcpyAsync(b.device, b.constant.data(), b.elements * sizeof(float),
                             hipMemcpyHostToDevice, plan->stream);
      else
        err = hipMemsetAsync(b.device, 0, b.elements * sizeof(float), plan->stream);
    }
    if (err != hipSuccess) {
      release(plan);
      return oxh::hip_status(err, "plan buffer allocation");
    }
  }
  st = oxh_graph_begin(plan->stream);
  if (st != OXH_OK) {
    release(plan);
    return st;
  }
  plan->launches.clear();
  for (const Run &r : form_runs(*plan)) {
    plan->launches.emplace_back(r.begin, r.end);
    st = r.end - r.begin == 1 ? launch_operation(*plan, plan->operations[r.begin])
                              : launch_run(*plan, r);
    if (st != OXH_OK) {
      const std::string message = oxh_last_error();
      (void)oxh_graph_abort(plan->stream);
      release(plan);
      return oxh::fail(st, "plan recording failed: " + message);
    }
  }
  st = oxh_graph_end(plan->stream, &plan->graph);
  if (st != OXH_OK) {
    release(plan);
    return st;
  }
  plan->compiled = true;
  return oxh::ok();
}

oxh_status oxh_plan_run(oxh_plan *plan, const float *const *host_inputs, uint32_t input_count,
                        float *host_output, uint64_t output_elements) {
  OXH_REQUIRE(plan != nullptr && plan->compiled, OXH_TRACE, "plan is not compiled");
  // jit.rs:183-203 validate_inputs: count and extents must match the compiled signature.
  OXH_REQUIRE(input_count == plan->inputs.size(), OXH_TRACE,
              "expected " + std::to_string(plan->inputs.size()) + " inputs, got " +
                  std::to_string(input_count));
  const Buffer &out = plan->buffers[static_cast<size_t>(plan->output)];
  OXH_REQUIRE(output_elements == out.elements && host_output != nullptr, OXH_TRACE,
              "output buffer must hold " + std::to_string(out.elements) + " elements");
  for (uint32_t i = 0; i < input_count; ++i) {
    const Buffer &b = plan->buffers[plan->inputs[i]];
    OXH_REQUIRE(host_inputs != nullptr && host_inputs[i] != nullptr, OXH_TRACE, "null input");
    OXH_HIP_CHECK(hipMemcpyAsync(b.device, host_inputs[i], b.elements * sizeof(float),
                                 hipMemcpyHostToDevice, plan->stream));
  }
  oxh_status st = oxh_graph_launch(plan->graph, plan->stream);
  if (st != OXH_OK) return st;
  return oxh_memcpy_d2h(host_output, out.device, out.elements * sizeof(float), plan->stream);
}

// cuda/jit.rs:86-97 / cuda_graph.rs:157-164: one launch of the plan's hipGraph.
oxh_status oxh_plan_replay(oxh_plan *plan) {
  OXH_REQUIRE(plan != nullptr && plan->compiled, OXH_TRACE, "plan is not compiled");
  return oxh_graph_launch(plan->graph, plan->stream);
}

// The same launches the graph holds, issued directly on the plan's stream.
oxh_status oxh_plan_launch(oxh_plan *plan) {
  OXH_REQUIRE(plan != nullptr && plan->compiled, OXH_TRACE, "plan is not compiled");
  for (const auto &l : plan->launches) {
    const Run r{l.first, l.second};
    oxh_status st = r.end - r.begin == 1 ? launch_operation(*plan, plan->operations[r.begin])
                                         : launch_run(*plan, r);
    if (st != OXH_OK) return st;
  }
  return oxh::ok();
}

oxh_status oxh_plan_stream(const oxh_plan *plan, oxh_stream *stream) {
  OXH_REQUIRE(plan != nullptr && stream != nullptr, OXH_INVALID_SHAPE, "null argument");
  OXH_REQUIRE(plan->compiled, OXH_TRACE, "plan is not compiled");
  *stream = plan->stream;
  return oxh::ok();
}

oxh_status oxh_plan_buffer(const oxh_plan *plan, uint32_t slot, float **device_pointer,
                           uint64_t *elements) {
  OXH_REQUIRE(plan != nullptr && device_pointer != nullptr && elements != nullptr,
              OXH_INVALID_SHAPE, "null argument");
  OXH_REQUIRE(plan->compiled, OXH_TRACE, "plan is not compiled");
  OXH_REQUIRE(slot < plan->buffers.size(), OXH_TRACE, "slot out of range");
  *device_pointer = plan->buffers[slot].device;
  *elements = plan->buffers[slot].elements;
  return oxh::ok();
}

oxh_status oxh_plan_destroy(oxh_plan *plan) {
  if (plan == nullptr) return oxh::ok();
  if (plan->compiled || plan->stream) {
    if (plan->stream) (void)hipStreamSynchronize(plan->stream);
  }
  release(plan);
  delete plan;
  return oxh::ok();
}

}  // extern "C"
