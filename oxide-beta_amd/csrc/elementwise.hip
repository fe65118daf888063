// elementwise.hip -- add / mul / relu, their backward, gradient accumulation and the fused
// relu((a + b) * c) chain, as one streaming map kernel instantiated per operation.
//
// Reference kernels: kernel_module.rs:8-34 (add, mul, relu), 492-508 (mul_backward,
// relu_backward), 1052-1059 (accumulate).  The reference launches one thread per element with
// scalar 4-byte loads; here every thread moves kUnroll 128-bit vectors per stream, so each wave
// issues 1 KiB-wide fully coalesced loads.  On MI355X many short blocks (one float4 per lane)
// stream faster than fewer blocks with long per-lane loops (measured best: 2).  Every
// operation is a single IEEE fp32 add, multiply or compare per element (no contraction), so the
// results are bit-identical to the reference's CPU path (evaluation.rs:21-34,
// autograd.rs:94-147).
#include <hip/hip_runtime.h>

#include "chain.h"
#include "common.h"

namespace {

#ifndef OXH_EW_UNROLL
#define OXH_EW_UNROLL 2  // float4 per thread per stream (overridable for tuning sweeps)
#endif
// Non-temporal hints (bit 1: loads, bit 2: stores), measured per kind of operation: the single
// reference ops stream faster with non-temporal loads, the fused chain (three outputs in the
// backward) with both.
#ifndef OXH_EW_NT_OP
#define OXH_EW_NT_OP 1
#endif
#ifndef OXH_EW_NT_CHAIN
#define OXH_EW_NT_CHAIN 3
#endif
constexpr int kUnroll = OXH_EW_UNROLL;
// The compiled-plan chain kernel streams fastest with one float4 per thread per stream
// (config 1's plan: 42.3 us at 1, 44.9 at 2, 46.4 at 4), the map kernels with two.
#ifndef OXH_EW_CHAIN_UNROLL
#define OXH_EW_CHAIN_UNROLL 1
#endif
constexpr int kChainUnroll = OXH_EW_CHAIN_UNROLL;

template <int NT>
__device__ __forceinline__ float4 ld(const float4 *p) {
  if constexpr ((NT & 1) != 0) return oxh::load_nt(p);
  else return *p;
}
template <int NT>
__device__ __forceinline__ void st(float4 *p, const float4 &v) {
  if constexpr ((NT & 2) != 0) oxh::store_nt(p, v);
  else *p = v;
}

template <int NI, int NO>
struct MapArgs {
  const float *in[NI];
  float *out[NO];
};

// Operations: scalar functors applied lane-wise.
struct AddOp {
  static constexpr int NT = OXH_EW_NT_OP;
  static constexpr int NI = 2, NO = 1;
  __device__ static void apply(const float (&x)[NI], float (&y)[NO]) { y[0] = x[0] + x[1]; }
};
struct MulOp {
  static constexpr int NT = OXH_EW_NT_OP;
  static constexpr int NI = 2, NO = 1;
  __device__ static void apply(const float (&x)[NI], float (&y)[NO]) { y[0] = x[0] * x[1]; }
};
struct ReluOp {  // kernel_module.rs:26-34: x > 0 ? x : 0 (NaN and -0 give +0)
  static constexpr int NT = OXH_EW_NT_OP;
  static constexpr int NI = 1, NO = 1;
  __device__ static void apply(const float (&x)[NI], float (&y)[NO]) {
    y[0] = x[0] > 0.0f ? x[0] : 0.0f;
  }
};
struct ReluBackwardOp {  // in0 = gradient, in1 = forward input
  static constexpr int NT = OXH_EW_NT_OP;
  static constexpr int NI = 2, NO = 1;
  __device__ static void apply(const float (&x)[NI], float (&y)[NO]) {
    y[0] = x[1] > 0.0f ? x[0] : 0.0f;
  }
};
struct ChainForwardOp {  // relu((a + b) * c)
  static constexpr int NT = OXH_EW_NT_CHAIN;
  static constexpr int NI = 3, NO = 1;
  __device__ static void apply(const float (&x)[NI], float (&y)[NO]) {
    float s = x[0] + x[1];
    float m = s * x[2];
    y[0] = m > 0.0f ? m : 0.0f;
  }
};
// Backward of relu((a + b) * c) through the reference VJPs: relu (autograd.rs:139-147), mul
// (123-138: left grad = g * right, right grad = g * left), add (119-122: both get g).
struct ChainBackwardOnesOp {
  static constexpr int NT = OXH_EW_NT_CHAIN;
  static constexpr int NI = 3, NO = 3;
  __device__ static void apply(const float (&x)[NI], float (&y)[NO]) {
    float s = x[0] + x[1];
    float m = s * x[2];
    float g = m > 0.0f ? 1.0f : 0.0f;
    float left = g * x[2];
    y[0] = left;
    y[1] = left;
    y[2] = g * s;
  }
};
struct ChainBackwardOp {  // in3 = upstream gradient
  static constexpr int NT = OXH_EW_NT_CHAIN;
  static constexpr int NI = 4, NO = 3;
  __device__ static void apply(const float (&x)[NI], float (&y)[NO]) {
    float s = x[0] + x[1];
    float m = s * x[2];
    float g = m > 0.0f ? x[3] : 0.0f;
    float left = g * x[2];
    y[0] = left;
    y[1] = left;
    y[2] = g * s;
  }
};

__device__ inline float lane(const float4 &v, int k) {
  return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}
__device__ inline void set_lane(float4 &v, int k, float f) {
  if (k == 0) v.x = f;
  else if (k == 1) v.y = f;
  else if (k == 2) v.z = f;
  else v.w = f;
}

// Vector path: all pointers 16-byte aligned.  Tiles of kBlock * kUnroll float4; a grid-stride
// loop over tiles; the n % 4 tail is done by block 0.
template <class Op>
__global__ __launch_bounds__(oxh::kBlock) void map_vec4_kernel(
    MapArgs<Op::NI, Op::NO> args, uint64_t n4, uint64_t n) {
  constexpr int NI = Op::NI, NO = Op::NO;
  const uint64_t tile = static_cast<uint64_t>(oxh::kBlock) * kUnroll;
  const uint64_t tiles = (n4 + tile - 1) / tile;
  for (uint64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
    const uint64_t base = t * tile + threadIdx.x;
    float4 in[kUnroll][NI];
    if (base + (kUnroll - 1) * oxh::kBlock < n4) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
#pragma unroll
        for (int i = 0; i < NI; ++i)
          in[u][i] = ld<Op::NT>(reinterpret_cast<const float4 *>(args.in[i]) + base + u * oxh::kBlock);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        float4 out[NO];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          float x[NI], y[NO];
#pragma unroll
          for (int i = 0; i < NI; ++i) x[i] = lane(in[u][i], k);
          Op::apply(x, y);
#pragma unroll
          for (int o = 0; o < NO; ++o) set_lane(out[o], k, y[o]);
        }
#pragma unroll
        for (int o = 0; o < NO; ++o)
          st<Op::NT>(reinterpret_cast<float4 *>(args.out[o]) + base + u * oxh::kBlock, out[o]);
      }
    } else {
      for (int u = 0; u < kUnroll; ++u) {
        const uint64_t idx = base + u * oxh::kBlock;
        if (idx >= n4) break;
        float4 v[NI], out[NO];
#pragma unroll
        for (int i = 0; i < NI; ++i) v[i] = ld<Op::NT>(reinterpret_cast<const float4 *>(args.in[i]) + idx);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          float x[NI], y[NO];
#pragma unroll
          for (int i = 0; i < NI; ++i) x[i] = lane(v[i], k);
          Op::apply(x, y);
#pragma unroll
          for (int o = 0; o < NO; ++o) set_lane(out[o], k, y[o]);
        }
#pragma unroll
        for (int o = 0; o < NO; ++o) st<Op::NT>(reinterpret_cast<float4 *>(args.out[o]) + idx, out[o]);
      }
    }
  }
  if (blockIdx.x == 0) {
    const uint64_t idx = n4 * 4 + threadIdx.x;
    if (idx < n) {
      float x[NI], y[NO];
#pragma unroll
      for (int i = 0; i < NI; ++i) x[i] = args.in[i][idx];
      Op::apply(x, y);
#pragma unroll
      for (int o = 0; o < NO; ++o) args.out[o][idx] = y[o];
    }
  }
}

// Scalar path for unaligned pointers.
template <class Op>
__global__ __launch_bounds__(oxh::kBlock) void map_scalar_kernel(
    MapArgs<Op::NI, Op::NO> args, uint64_t n) {
  constexpr int NI = Op::NI, NO = Op::NO;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < n;
       idx += stride) {
    float x[NI], y[NO];
#pragma unroll
    for (int i = 0; i < NI; ++i) x[i] = args.in[i][idx];
    Op::apply(x, y);
#pragma unroll
    for (int o = 0; o < NO; ++o) args.out[o][idx] = y[o];
  }
}

constexpr uint64_t kMaxGrid = 1u << 24;

template <class Op>
oxh_status launch_map(const char *name, oxh_stream stream, const MapArgs<Op::NI, Op::NO> &args,
                      uint64_t n) {
  if (n == 0) return oxh::ok();
  for (int i = 0; i < Op::NI; ++i)
    OXH_REQUIRE(args.in[i] != nullptr, OXH_INVALID_SHAPE, std::string(name) + ": null input");
  for (int o = 0; o < Op::NO; ++o) {
    OXH_REQUIRE(args.out[o] != nullptr, OXH_INVALID_SHAPE, std::string(name) + ": null output");
    // An output may be exactly an input (in place) but must not partially overlap one, and
    // outputs must be distinct from each other.
    for (int i = 0; i < Op::NI; ++i)
      OXH_REQUIRE(!oxh::partial_overlap(args.out[o], args.in[i], n * sizeof(float)),
                  OXH_INVALID_SHAPE, std::string(name) + ": output partially overlaps an input");
    for (int p = 0; p < o; ++p)
      OXH_REQUIRE(!oxh::any_overlap(args.out[o], n * 4, args.out[p], n * 4), OXH_INVALID_SHAPE,
                  std::string(name) + ": outputs overlap");
  }
  bool vec = true;
  for (int i = 0; i < Op::NI; ++i) vec = vec && oxh::aligned16(args.in[i]);
  for (int o = 0; o < Op::NO; ++o) vec = vec && oxh::aligned16(args.out[o]);
  hipStream_t s = oxh::as_stream(stream);
  if (vec) {
    const uint64_t n4 = n / 4;
    const uint64_t tile = static_cast<uint64_t>(oxh::kBlock) * kUnroll;
    uint64_t grid = (n4 + tile - 1) / tile;
    if (grid == 0) grid = 1;
    if (grid > kMaxGrid) grid = kMaxGrid;
    oxh::launch(map_vec4_kernel<Op>, dim3(static_cast<uint32_t>(grid)), dim3(oxh::kBlock),
                       0, s, args, n4, n);
  } else {
    uint64_t grid = (n + oxh::kBlock - 1) / oxh::kBlock;
    if (grid > kMaxGrid) grid = kMaxGrid;
    oxh::launch(map_scalar_kernel<Op>, dim3(static_cast<uint32_t>(grid)),
                       dim3(oxh::kBlock), 0, s, args, n);
  }
  return oxh::launched(name);
}

// One step of a fused chain on one value (the plan operations' formulas above).
__device__ __forceinline__ float chain_step(uint32_t op, float x0, float x1) {
  switch (op) {
    case OXH_PLAN_ADD:
    case OXH_PLAN_ACCUMULATE: return x0 + x1;
    case OXH_PLAN_MUL:
    case OXH_PLAN_MUL_BACKWARD: return x0 * x1;
    case OXH_PLAN_RELU: return x0 > 0.0f ? x0 : 0.0f;
    default: return x1 > 0.0f ? x0 : 0.0f;  // OXH_PLAN_RELU_BACKWARD
  }
}

__device__ __forceinline__ float4 chain_step4(const oxh::ChainStep &s, const float4 &acc,
                                              const float4 &b) {
  const float4 x0 = s.acc_second ? b : acc, x1 = s.acc_second ? acc : b;
  return make_float4(chain_step(s.op, x0.x, x1.x), chain_step(s.op, x0.y, x1.y),
                     chain_step(s.op, x0.z, x1.z), chain_step(s.op, x0.w, x1.w));
}

// A fused chain: per float4 of elements the steps run in order on registers, each combining
// the running value with its other operand and storing its result where the plan needs it.
// Every step's other operand is loaded before the first step runs (non-temporal; no step
// writes a buffer a later step reads), so all of a tile's loads are in flight together.  The
// steps are kernel arguments: the loops over them are unrolled to MaxSteps with
// block-uniform exits, keeping the operand registers statically indexed.  Chains of up to four
// steps (config 1's plan has three) take the 4-step instance: half the operand registers, so
// more waves stay in flight.
template <int MaxSteps>
__global__ __launch_bounds__(oxh::kBlock) void chain_vec4_kernel(oxh::Chain c, uint64_t n4,
                                                                 uint64_t n) {
  constexpr int U = kChainUnroll;  // float4 per thread per stream
  const uint64_t tile = static_cast<uint64_t>(oxh::kBlock) * U;
  for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * tile + threadIdx.x; base < n4;
       base += static_cast<uint64_t>(gridDim.x) * tile) {
    uint64_t idx[U];
    bool live[U];
    float4 acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      idx[u] = base + static_cast<uint64_t>(u) * oxh::kBlock;
      live[u] = idx[u] < n4;
      if (!live[u]) idx[u] = base;  // a repeat of element base: loaded, never stored
      acc[u] = oxh::load_nt(reinterpret_cast<const float4 *>(c.first) + idx[u]);
    }
    float4 operand[MaxSteps][U];
#pragma unroll
    for (int k = 0; k < MaxSteps; ++k) {
      if (k >= static_cast<int>(c.count)) break;
      if (c.steps[k].other < 0) continue;
      const float4 *src = reinterpret_cast<const float4 *>(c.other[c.steps[k].other]);
#pragma unroll
      for (int u = 0; u < U; ++u) operand[k][u] = oxh::load_nt(src + idx[u]);
    }
#pragma unroll
    for (int k = 0; k < MaxSteps; ++k) {
      if (k >= static_cast<int>(c.count)) break;
      const oxh::ChainStep s = c.steps[k];
#pragma unroll
      for (int u = 0; u < U; ++u)
        acc[u] = chain_step4(s, acc[u], s.other >= 0 ? operand[k][u] : acc[u]);
      if (s.store >= 0) {
        float4 *dst = reinterpret_cast<float4 *>(c.store[s.store]);
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (live[u]) oxh::store_nt(dst + idx[u], acc[u]);
      }
    }
  }
  if (blockIdx.x == 0) {
    const uint64_t i = n4 * 4 + threadIdx.x;
    if (i < n) {
      float acc = c.first[i];
      for (uint32_t k = 0; k < c.count; ++k) {
        const oxh::ChainStep s = c.steps[k];
        const float b = s.other >= 0 ? c.other[s.other][i] : acc;
        acc = s.acc_second ? chain_step(s.op, b, acc) : chain_step(s.op, acc, b);
        if (s.store >= 0) c.store[s.store][i] = acc;
      }
    }
  }
}

}  // namespace

namespace oxh {

// Plan buffers are separate hipMalloc allocations (256-byte aligned): the vector path only.
oxh_status launch_chain(hipStream_t stream, const Chain &c, uint64_t n) {
  if (n == 0) return ok();
  OXH_REQUIRE(c.count >= 1 && c.count <= static_cast<uint32_t>(kChainMax) && c.first != nullptr,
              OXH_TRACE, "malformed elementwise chain");
  OXH_REQUIRE(aligned16(c.first), OXH_TRACE, "chain buffers must be 16-byte aligned");
  const uint64_t n4 = n / 4;
  const uint64_t tile = static_cast<uint64_t>(kBlock) * kChainUnroll;
  uint64_t grid = (n4 + tile - 1) / tile;
  if (grid == 0) grid = 1;
  if (grid > kMaxGrid) grid = kMaxGrid;
  if (c.count <= 4)
    launch(chain_vec4_kernel<4>, dim3(static_cast<uint32_t>(grid)), dim3(kBlock), 0, stream, c,
           n4, n);
  else
    launch(chain_vec4_kernel<kChainMax>, dim3(static_cast<uint32_t>(grid)), dim3(kBlock), 0,
           stream, c, n4, n);
  return launched("elementwise chain");
}

}  // namespace oxh

extern "C" {

oxh_status oxh_add(oxh_stream stream, const float *a, const float *b, float *output, uint64_t n) {
  return launch_map<AddOp>("oxh_add", stream, {{a, b}, {output}}, n);
}

oxh_status oxh_mul(oxh_stream stream, const float *a, const float *b, float *output, uint64_t n) {
  return launch_map<MulOp>("oxh_mul", stream, {{a, b}, {output}}, n);
}

oxh_status oxh_relu(oxh_stream stream, const float *input, float *output, uint64_t n) {
  return launch_map<ReluOp>("oxh_relu", stream, {{input}, {output}}, n);
}

oxh_status oxh_mul_backward(oxh_stream stream, const float *gradient, const float *other,
                            float *output, uint64_t n) {
  return launch_map<MulOp>("oxh_mul_backward", stream, {{gradient, other}, {output}}, n);
}

oxh_status oxh_relu_backward(oxh_stream stream, const float *gradient, const float *input,
                             float *output, uint64_t n) {
  return launch_map<ReluBackwardOp>("oxh_relu_backward", stream, {{gradient, input}, {output}},
                                    n);
}

oxh_status oxh_accumulate(oxh_stream stream, const float *a, const float *b, float *output,
                          uint64_t n) {
  return launch_map<AddOp>("oxh_accumulate", stream, {{a, b}, {output}}, n);
}

oxh_status oxh_elementwise_chain_forward(oxh_stream stream, const float *a, const float *b,
                                         const float *c, float *y, uint64_t n) {
  return launch_map<ChainForwardOp>("oxh_elementwise_chain_forward", stream, {{a, b, c}, {y}},
                                    n);
}

oxh_status oxh_elementwise_chain_backward(oxh_stream stream, const float *a, const float *b,
                                          const float *c, const float *gradient, float *da,
                                          float *db, float *dc, uint64_t n) {
  if (gradient == nullptr)
    return launch_map<ChainBackwardOnesOp>("oxh_elementwise_chain_backward", stream,
                                           {{a, b, c}, {da, db, dc}}, n);
  return launch_map<ChainBackwardOp>("oxh_elementwise_chain_backward", stream,
                                     {{a, b, c, gradient}, {da, db, dc}}, n);
}

}  // extern "C"
