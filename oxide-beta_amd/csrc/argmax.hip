// argmax.hip -- per-row argmax under IEEE total order, the last index winning ties.
//
// Reference: count_correct (crates/oxide-torch-models/examples/mnist_training.rs:201-218) takes
// `max_by(|a, b| a.1.total_cmp(b.1))` over each row of logits on the host; Iterator::max_by
// returns the last of several equal maxima.  Here one wave per row scans the row with strided
// loads and reduces (key, index) pairs with wave64 shuffles.  Integer-exact.
#include <hip/hip_runtime.h>

#include <string>

#include "common.h"

namespace {

// f32::total_cmp key: the bit pattern with the magnitude bits flipped for negative values,
// compared as a signed integer.
__device__ __forceinline__ int32_t total_key(float v) {
  int32_t bits = __float_as_int(v);
  return bits ^ static_cast<int32_t>(static_cast<uint32_t>(bits >> 31) >> 1);
}

__device__ __forceinline__ bool better(int32_t k, uint32_t i, int32_t bk, uint32_t bi) {
  return k > bk || (k == bk && i > bi);
}

constexpr int kRowsPerBlock = 4;  // one wave per row

__global__ __launch_bounds__(64 * kRowsPerBlock) void argmax_kernel(uint64_t rows,
                                                                    uint64_t classes,
                                                                    const float *logits,
                                                                    uint32_t *indices) {
  const uint64_t row = static_cast<uint64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / 64;
  if (row >= rows) return;
  const uint32_t lane = threadIdx.x % 64;
  const float *x = logits + row * classes;
  int32_t best_key = INT32_MIN;
  uint32_t best_idx = 0;
  bool have = false;
  for (uint64_t i = lane; i < classes; i += 64) {
    const int32_t k = total_key(x[i]);
    if (!have || better(k, static_cast<uint32_t>(i), best_key, best_idx)) {
      best_key = k;
      best_idx = static_cast<uint32_t>(i);
      have = true;
    }
  }
  // Lanes with no element keep (INT32_MIN, 0): every real key beats or ties it only with a
  // larger index, and index 0 is held by lane 0 itself.
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int32_t k = __shfl_xor(best_key, off, 64);
    const uint32_t i = __shfl_xor(best_idx, off, 64);
    const bool h = __shfl_xor(static_cast<int>(have), off, 64) != 0;
    if (h && (!have || better(k, i, best_key, best_idx))) {
      best_key = k;
      best_idx = i;
      have = true;
    }
  }
  if (lane == 0) indices[row] = best_idx;
}

}  // namespace

extern "C" oxh_status oxh_argmax_rows(oxh_stream stream, uint64_t rows, uint64_t classes,
                                      const float *logits, uint32_t *indices) {
  if (rows == 0) return oxh::ok();
  OXH_REQUIRE(classes > 0 && classes < (1ull << 32), OXH_INVALID_SHAPE,
              "oxh_argmax_rows: classes must be in 1..2^32");
  OXH_REQUIRE(logits && indices, OXH_INVALID_SHAPE, "oxh_argmax_rows: null pointer");
  OXH_REQUIRE(rows < (1ull << 33), OXH_INVALID_SHAPE, "oxh_argmax_rows: too many rows");
  const uint64_t grid = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  oxh::launch(argmax_kernel, dim3(static_cast<uint32_t>(grid)), dim3(64 * kRowsPerBlock),
                     0, oxh::as_stream(stream), rows, classes, logits, indices);
  return oxh::launched("oxh_argmax_rows");
}
