// chain.h -- fused elementwise chains for compiled plans (library-internal).
//
// A chain is a run of plan operations in which each operation consumes the previous one's
// result: per element, the running value ("acc") starts as the first operation's first input
// and each step combines it with at most one other buffer, in plan order.  The plan compiler
// (plan.hip) forms chains; elementwise.hip runs one as a single streaming kernel whose
// per-element results are those of the separate launches bit for bit (the same fp32 operation
// per step, no contraction).
#pragma once

#include <cstdint>

#include "common.h"

namespace oxh {

constexpr int kChainMax = 8;

struct ChainStep {
  uint32_t op;          // OXH_PLAN_* code
  int32_t other;        // index into Chain::other, or -1: the step's other operand is acc
  uint32_t acc_second;  // 1: acc is the operation's second input (in1), else its first
  int32_t store;        // index into Chain::store, or -1: the step's result is not stored
};

struct Chain {
  const float *first;             // acc before step 0 (step 0's first input)
  const float *other[kChainMax];  // buffers read by the steps (never written earlier in the chain)
  float *store[kChainMax];        // buffers written
  ChainStep steps[kChainMax];
  uint32_t count;
};

oxh_status launch_chain(hipStream_t stream, const Chain &chain, uint64_t n);

}  // namespace oxh
