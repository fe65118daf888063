// chunk_sum.h -- the fixed-order sum of weight-gradient chunk partials, shared by the
// convolution's own sum launch (conv.hip) and a training program's one launch of every
// convolution's sums before its optimizer step (adamw.hip): each element is the same sum, in
// the same order, in both.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace oxh {

// Lanes per element: a power of two up to 16 leaving at most 8 chunks per lane.
inline uint32_t chunk_sum_lanes(uint32_t chunks) {
  uint32_t lanes = 1;
  while (lanes < 16 && chunks > 8 * lanes) lanes *= 2;
  return lanes;
}

// Block `block` (of 256 threads) of out[e] = sum over chunks of partial[chunk][e]: `lanes`
// threads share an element (a block serves 256 / lanes elements; thread t takes lane
// t / (256 / lanes) of element t % (256 / lanes), so each lane's loads are contiguous across
// elements); lane l sums the l-th contiguous part of the chunks serially (loads issued in
// groups of 8 ahead of the adds), and the lane sums are then added in lane order.  Elements
// e >= split go to out2[e - split] (a second output sharing the chunks' layout).  `part`: 256
// floats of LDS.
__device__ inline void sum_chunks_block(uint32_t block, uint32_t count, uint32_t chunks,
                                        uint32_t lanes, const float *__restrict__ partial,
                                        float *__restrict__ out, uint32_t split,
                                        float *__restrict__ out2, float *part) {
  const uint32_t per_block = 256 / lanes;
  const uint32_t l = threadIdx.x / per_block, j = threadIdx.x - l * per_block;
  const uint32_t e = block * per_block + j;
  float acc = 0.0f;
  if (e < count) {
    const uint32_t c1 = (l + 1) * chunks / lanes;
    uint32_t c = l * chunks / lanes;
    for (; c + 8 <= c1; c += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = partial[static_cast<uint64_t>(c + u) * count + e];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += v[u];
    }
    for (; c < c1; ++c) acc += partial[static_cast<uint64_t>(c) * count + e];
  }
  if (lanes == 1) {
    if (e < count) (e < split ? out[e] : out2[e - split]) = acc;
    return;
  }
  part[threadIdx.x] = acc;
  __syncthreads();
  if (l != 0 || e >= count) return;
  for (uint32_t r = 1; r < lanes; ++r) acc += part[r * per_block + j];
  (e < split ? out[e] : out2[e - split]) = acc;
}

}  // namespace oxh
