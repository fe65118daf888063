// adamw.hip -- fused AdamW update (moments + decoupled weight decay + parameter), in place or
// into separate outputs, for one tensor or many tensors in one launch.
//
// Reference: kernel adamw (kernel_module.rs:1094-1127), driver runtime.rs:1306-1386 (which
// writes three freshly allocated buffers per parameter per step), CPU loop optim.rs:98-125.
// Per element the arithmetic is the reference's exact sequence of fp32 operations:
//   first  = b1*m + (1-b1)*g
//   second = b2*v + ((1-b2)*g)*g
//   p'     = p - lr*((first/c1) / (sqrt(second/c2) + eps) + wd*p)
// built with -ffp-contract=off and IEEE (correctly rounded) division and square root, so the
// result is bit-identical to the CPU path.  Traffic: 4 reads + 3 writes of 4 bytes per element,
// all as 128-bit accesses.  The one-tensor kernel streams them with the non-temporal hint (every
// byte is touched once per step; measured on MI355X: 5.93 TB/s with the hint on loads and
// stores, 5.40 TB/s without).  The multi-tensor and table kernels update a model's parameters,
// which the next step's layers read again: they keep the default cache policy, so the updated
// parameters (and the moments) stay in the caches (config 5: 846 -> 824 us per step against
// the non-temporal hint on both, 841 us with it on the loads only).
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>

#include "chunk_sum.h"
#include "common.h"

namespace {

#ifndef OXH_ADAMW_UNROLL
#define OXH_ADAMW_UNROLL 2  // float4 per thread per stream (overridable for tuning sweeps)
#endif
#ifndef OXH_ADAMW_NT
#define OXH_ADAMW_NT 3  // 1: non-temporal loads, 2: non-temporal stores, 3: both
#endif
constexpr int kUnroll = OXH_ADAMW_UNROLL;

// Stream: the one-tensor kernel's accesses (non-temporal per OXH_ADAMW_NT); else the default
// cache policy.
template <bool Stream>
__device__ __forceinline__ float4 ld(const float4 *p) {
  if constexpr (Stream && (OXH_ADAMW_NT & 1) != 0) return oxh::load_nt(p);
  else return *p;
}
template <bool Stream>
__device__ __forceinline__ void st(float4 *p, const float4 &v) {
  if constexpr (Stream && (OXH_ADAMW_NT & 2) != 0) oxh::store_nt(p, v);
  else *p = v;
}

struct Hyper {
  float lr, wd, b1, b2, c1, c2, eps;
};

__device__ __forceinline__ void adamw_scalar(const Hyper &h, float p, float g, float m, float v,
                                             float &p_out, float &m_out, float &v_out) {
  const float first = h.b1 * m + (1.0f - h.b1) * g;
  const float second = h.b2 * v + (1.0f - h.b2) * g * g;
  const float normalized = (first / h.c1) / (sqrtf(second / h.c2) + h.eps);
  p_out = p - h.lr * (normalized + h.wd * p);
  m_out = first;
  v_out = second;
}

__device__ __forceinline__ void adamw_vec(const Hyper &h, const float4 &p, const float4 &g,
                                          const float4 &m, const float4 &v, float4 &po,
                                          float4 &mo, float4 &vo) {
  adamw_scalar(h, p.x, g.x, m.x, v.x, po.x, mo.x, vo.x);
  adamw_scalar(h, p.y, g.y, m.y, v.y, po.y, mo.y, vo.y);
  adamw_scalar(h, p.z, g.z, m.z, v.z, po.z, mo.z, vo.z);
  adamw_scalar(h, p.w, g.w, m.w, v.w, po.w, mo.w, vo.w);
}

struct Streams {
  const float *p, *g, *m, *v;
  float *po, *mo, *vo;
};

// Elements [begin, end) of one tensor, processed by one block.  Vector accesses when all seven
// pointers are 16-byte aligned and begin is a multiple of 4.
template <bool Stream>
__device__ __forceinline__ void adamw_range(const Hyper &h, const Streams &s, uint64_t begin,
                                            uint64_t end, bool vec) {
  if (vec) {
    const uint64_t b4 = begin / 4, e4 = end / 4;
    const float4 *p4 = reinterpret_cast<const float4 *>(s.p);
    const float4 *g4 = reinterpret_cast<const float4 *>(s.g);
    const float4 *m4 = reinterpret_cast<const float4 *>(s.m);
    const float4 *v4 = reinterpret_cast<const float4 *>(s.v);
    float4 *po4 = reinterpret_cast<float4 *>(s.po);
    float4 *mo4 = reinterpret_cast<float4 *>(s.mo);
    float4 *vo4 = reinterpret_cast<float4 *>(s.vo);
    uint64_t i = b4 + threadIdx.x;
    for (; i + (kUnroll - 1) * oxh::kBlock < e4; i += kUnroll * oxh::kBlock) {
      float4 p[kUnroll], g[kUnroll], m[kUnroll], v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        p[u] = ld<Stream>(&p4[i + u * oxh::kBlock]);
        g[u] = ld<Stream>(&g4[i + u * oxh::kBlock]);
        m[u] = ld<Stream>(&m4[i + u * oxh::kBlock]);
        v[u] = ld<Stream>(&v4[i + u * oxh::kBlock]);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        float4 po, mo, vo;
        adamw_vec(h, p[u], g[u], m[u], v[u], po, mo, vo);
        st<Stream>(&po4[i + u * oxh::kBlock], po);
        st<Stream>(&mo4[i + u * oxh::kBlock], mo);
        st<Stream>(&vo4[i + u * oxh::kBlock], vo);
      }
    }
    for (; i < e4; i += oxh::kBlock) {
      float4 po, mo, vo;
      adamw_vec(h, ld<Stream>(&p4[i]), ld<Stream>(&g4[i]), ld<Stream>(&m4[i]),
                ld<Stream>(&v4[i]), po, mo, vo);
      st<Stream>(&po4[i], po);
      st<Stream>(&mo4[i], mo);
      st<Stream>(&vo4[i], vo);
    }
    begin = e4 * 4;
  }
  for (uint64_t i = begin + threadIdx.x; i < end; i += oxh::kBlock) {
    float po, mo, vo;
    adamw_scalar(h, s.p[i], s.g[i], s.m[i], s.v[i], po, mo, vo);
    s.po[i] = po;
    s.mo[i] = mo;
    s.vo[i] = vo;
  }
}

// Elements per block: kBlock threads x kUnroll float4 (one pass; many short blocks stream
// faster on MI355X than long per-lane loops).
constexpr uint64_t kChunk = static_cast<uint64_t>(oxh::kBlock) * kUnroll * 4;

__global__ __launch_bounds__(oxh::kBlock) void adamw_kernel(Hyper h, Streams s, uint64_t n,
                                                            bool vec) {
  const uint64_t chunks = (n + kChunk - 1) / kChunk;
  for (uint64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
    const uint64_t begin = c * kChunk;
    const uint64_t end = begin + kChunk < n ? begin + kChunk : n;
    adamw_range<true>(h, s, begin, end, vec);
  }
}

// Multi-tensor: up to kMaxTensors descriptors in the kernel argument block; block b works on
// chunk (b - first_chunk[t]) of the tensor t whose chunk range holds b.
constexpr int kMaxTensors = 48;

struct TensorTable {
  Streams s[kMaxTensors];
  uint64_t n[kMaxTensors];
  uint32_t first_chunk[kMaxTensors + 1];
  uint32_t count;
  uint32_t vec_mask_lo, vec_mask_hi;
};

// Rust's f32::powi(i32) as compiler-rt's __powisf2: square-and-multiply over |b|, then one
// reciprocal when b < 0 (host and device use this same sequence of fp32 operations).
__host__ __device__ inline float powi_f32(float a, int32_t b) {
  const bool recip = b < 0;
  float r = 1.0f;
  for (;;) {
    if (b & 1) r *= a;
    b /= 2;
    if (b == 0) break;
    a *= a;
  }
  return recip ? 1.0f / r : r;
}

__global__ void increment_step_kernel(int32_t *step) { *step += 1; }

// Up to kChunkSumsPerLaunch weight-gradient chunk sums in one launch: block b serves the last
// sum whose first block is <= b, as block b - first of that sum's own launch would
// (oxh::sum_chunks_block); with `step` not null, thread 0 of block 0 also advances the
// optimizer step counter (the AdamW table launch after it reads the new value).
struct ChunkSumJob {
  const float *partial;
  float *out, *out2;
  uint32_t count, chunks, lanes, split, first_block;
};
struct ChunkSumTable {
  ChunkSumJob job[oxh::kChunkSumsPerLaunch];
  uint32_t jobs;
  int32_t *step;
};

__global__ __launch_bounds__(256) void sum_chunks_table_kernel(ChunkSumTable t) {
  __shared__ float part[256];
  const uint32_t b = blockIdx.x;
  if (t.step != nullptr && b == 0 && threadIdx.x == 0) *t.step += 1;
  if (t.jobs == 0) return;
  uint32_t j = 0;
  while (j + 1 < t.jobs && t.job[j + 1].first_block <= b) ++j;  // block-uniform
  const ChunkSumJob &c = t.job[j];
  oxh::sum_chunks_block(b - c.first_block, c.count, c.chunks, c.lanes, c.partial, c.out,
                        c.split, c.out2, part);
}

// step != null: the bias corrections come from the device step counter (optim.rs:113-114).
__global__ __launch_bounds__(oxh::kBlock) void adamw_multi_kernel(Hyper h, TensorTable table,
                                                                  const int32_t *step) {
  if (step != nullptr) {
    const int32_t t = *step;
    h.c1 = 1.0f - powi_f32(h.b1, t);
    h.c2 = 1.0f - powi_f32(h.b2, t);
  }
  const uint32_t b = blockIdx.x;
  uint32_t t = 0;
  while (t + 1 < table.count && table.first_chunk[t + 1] <= b) ++t;
  const uint64_t begin = static_cast<uint64_t>(b - table.first_chunk[t]) * kChunk;
  const uint64_t n = table.n[t];
  const uint64_t end = begin + kChunk < n ? begin + kChunk : n;
  const bool vec = t < 32 ? ((table.vec_mask_lo >> t) & 1u) : ((table.vec_mask_hi >> (t - 32)) & 1u);
  adamw_range<false>(h, table.s[t], begin, end, vec);
}

// Device-table variant: the tensor descriptors and each tensor's first chunk live in device
// memory (any number of tensors, one launch).  Up to kBlock tensors: thread i loads tensor i's
// chunk range [starts[i], starts[i + 1]) and descriptor together, and the one thread whose
// range holds b hands its descriptor to the block through LDS (one memory round trip and one
// barrier before the data loads).  More tensors: a block-parallel search -- each round the
// block's threads probe kBlock evenly spaced starts at once, the probes at or below b form a
// prefix (starts never decrease) whose length a barrier count gives -- then the descriptor's
// load.  Every block reads the step count t = *step, which the launch before it has advanced
// (a "last block stores t" ticket would serialise one atomic per block on a single address:
// about 7 us over config 5's 1360 blocks, against about 2 us for the extra launch).
__global__ __launch_bounds__(oxh::kBlock) void adamw_table_kernel(
    Hyper h, const oxh_adamw_tensor *__restrict__ table, const uint32_t *__restrict__ starts,
    uint32_t count, const int32_t *step) {
  __shared__ oxh_adamw_tensor mine;
  __shared__ uint32_t mine_start;
  const int32_t t = *step;
  h.c1 = 1.0f - powi_f32(h.b1, t);
  h.c2 = 1.0f - powi_f32(h.b2, t);
  const uint32_t b = blockIdx.x;
  oxh_adamw_tensor d;
  uint32_t first;
  if (count <= oxh::kBlock) {
    const uint32_t i = threadIdx.x;
    if (i < count) {
      const uint32_t lo = starts[i], hi = starts[i + 1];
      const oxh_adamw_tensor own = table[i];
      // exactly one thread: the ranges tile [0, starts[count]) (the first and last tensors
      // also take blocks outside it, which then find no elements of theirs)
      if ((lo <= b || i == 0) && (b < hi || i + 1 == count)) {
        mine = own;
        mine_start = lo;
      }
    }
    __syncthreads();
    d = mine;
    first = mine_start;
  } else {
    uint32_t lo = 0, hi = count;  // the last tensor index with starts[i] <= b is in [lo, hi)
    while (hi - lo > 1) {          // block-uniform
      const uint32_t spacing = (hi - lo + oxh::kBlock - 1) / oxh::kBlock;
      const uint32_t probe = lo + threadIdx.x * spacing;
      const int at_or_below = __syncthreads_count(probe < hi && starts[probe] <= b);
      const uint32_t f = lo + static_cast<uint32_t>(at_or_below - 1) * spacing;  // >= lo
      hi = f + spacing < hi ? f + spacing : hi;
      lo = f;
    }
    d = table[lo];
    first = starts[lo];
  }
  const uint64_t begin = static_cast<uint64_t>(b - first) * kChunk;
  const uint64_t end = begin + kChunk < d.n ? begin + kChunk : d.n;
  const bool vec = ((reinterpret_cast<uintptr_t>(d.parameter) |
                     reinterpret_cast<uintptr_t>(d.gradient) |
                     reinterpret_cast<uintptr_t>(d.first_moment) |
                     reinterpret_cast<uintptr_t>(d.second_moment)) & 15u) == 0;
  adamw_range<false>(h,
              Streams{d.parameter, d.gradient, d.first_moment, d.second_moment, d.parameter,
                      d.first_moment, d.second_moment},
              begin, end, vec);
}

bool finite_hyper(const Hyper &h) {
  return std::isfinite(h.lr) && std::isfinite(h.wd) && std::isfinite(h.b1) &&
         std::isfinite(h.b2) && std::isfinite(h.c1) && std::isfinite(h.c2) &&
         std::isfinite(h.eps);
}

}  // namespace

extern "C" {

oxh_status oxh_adamw_corrections(float beta1, float beta2, int32_t step, float *first_correction,
                                 float *second_correction) {
  OXH_REQUIRE(first_correction != nullptr && second_correction != nullptr, OXH_INVALID_SHAPE,
              "oxh_adamw_corrections: null output");
  *first_correction = 1.0f - powi_f32(beta1, step);
  *second_correction = 1.0f - powi_f32(beta2, step);
  return oxh::ok();
}

oxh_status oxh_adamw(oxh_stream stream, float learning_rate, float weight_decay, float beta1,
                     float beta2, float first_correction, float second_correction, float epsilon,
                     const float *parameter, const float *gradient, const float *first_moment,
                     const float *second_moment, float *new_parameter, float *new_first_moment,
                     float *new_second_moment, uint64_t n) {
  if (n == 0) return oxh::ok();
  const Hyper h{learning_rate, weight_decay, beta1, beta2, first_correction, second_correction,
                epsilon};
  OXH_REQUIRE(finite_hyper(h), OXH_INVALID_SHAPE, "oxh_adamw: non-finite hyper-parameter");
  const float *ins[4] = {parameter, gradient, first_moment, second_moment};
  float *outs[3] = {new_parameter, new_first_moment, new_second_moment};
  for (const float *p : ins) OXH_REQUIRE(p != nullptr, OXH_INVALID_SHAPE, "oxh_adamw: null input");
  for (float *p : outs) OXH_REQUIRE(p != nullptr, OXH_INVALID_SHAPE, "oxh_adamw: null output");
  const uint64_t bytes = n * sizeof(float);
  for (float *o : outs)
    for (const float *i : ins)
      OXH_REQUIRE(!oxh::partial_overlap(o, i, bytes), OXH_INVALID_SHAPE,
                  "oxh_adamw: an output partially overlaps an input");
  OXH_REQUIRE(!oxh::any_overlap(outs[0], bytes, outs[1], bytes) &&
                  !oxh::any_overlap(outs[0], bytes, outs[2], bytes) &&
                  !oxh::any_overlap(outs[1], bytes, outs[2], bytes),
              OXH_INVALID_SHAPE, "oxh_adamw: outputs overlap");
  bool vec = true;
  for (const float *p : ins) vec = vec && oxh::aligned16(p);
  for (float *p : outs) vec = vec && oxh::aligned16(p);
  const Streams s{parameter, gradient, first_moment, second_moment,
                  new_parameter, new_first_moment, new_second_moment};
  uint64_t grid = (n + kChunk - 1) / kChunk;
  if (grid > 0x7FFFFFFFull) grid = 0x7FFFFFFFull;
  oxh::launch(adamw_kernel, dim3(static_cast<uint32_t>(grid)), dim3(oxh::kBlock), 0,
                     oxh::as_stream(stream), h, s, n, vec);
  return oxh::launched("oxh_adamw");
}

namespace {
oxh_status adamw_multi(const char *name, oxh_stream stream, const Hyper &h, const int32_t *step,
                       const oxh_adamw_tensor *tensors, uint32_t count);
}

oxh_status oxh_adamw_multi_tensor(oxh_stream stream, float learning_rate, float weight_decay,
                                  float beta1, float beta2, float first_correction,
                                  float second_correction, float epsilon,
                                  const oxh_adamw_tensor *tensors, uint32_t count) {
  const Hyper h{learning_rate, weight_decay, beta1, beta2, first_correction, second_correction,
                epsilon};
  return adamw_multi("oxh_adamw_multi_tensor", stream, h, nullptr, tensors, count);
}

oxh_status oxh_adamw_multi_tensor_step(oxh_stream stream, float learning_rate,
                                       float weight_decay, float beta1, float beta2,
                                       float epsilon, int32_t *step,
                                       const oxh_adamw_tensor *tensors, uint32_t count) {
  OXH_REQUIRE(step != nullptr, OXH_INVALID_SHAPE,
              "oxh_adamw_multi_tensor_step: null step counter");
  const Hyper h{learning_rate, weight_decay, beta1, beta2, 1.0f, 1.0f, epsilon};
  oxh::launch(increment_step_kernel, dim3(1), dim3(1), 0, oxh::as_stream(stream), step);
  oxh_status st = oxh::launched("oxh_adamw_multi_tensor_step");
  if (st != OXH_OK) return st;
  return adamw_multi("oxh_adamw_multi_tensor_step", stream, h, step, tensors, count);
}

oxh_status oxh_adamw_table_layout(const oxh_adamw_tensor *tensors, uint32_t count,
                                  uint32_t *chunk_starts, uint64_t *total_chunks) {
  OXH_REQUIRE(tensors != nullptr && chunk_starts != nullptr && total_chunks != nullptr,
              OXH_INVALID_SHAPE, "oxh_adamw_table_layout: null argument");
  uint64_t chunks = 0;
  for (uint32_t i = 0; i < count; ++i) {
    OXH_REQUIRE(tensors[i].n > 0 && tensors[i].n <= (1ull << 44), OXH_INVALID_SHAPE,
                "oxh_adamw_table_layout: tensor " + std::to_string(i) +
                    " is empty or too large");
    chunk_starts[i] = static_cast<uint32_t>(chunks);
    chunks += (tensors[i].n + kChunk - 1) / kChunk;
    OXH_REQUIRE(chunks < (1ull << 31), OXH_INVALID_SHAPE,
                "oxh_adamw_table_layout: more than 2^31 chunks");
  }
  chunk_starts[count] = static_cast<uint32_t>(chunks);
  *total_chunks = chunks;
  return oxh::ok();
}

oxh_status oxh_adamw_multi_tensor_table_step(oxh_stream stream, float learning_rate,
                                             float weight_decay, float beta1, float beta2,
                                             float epsilon, int32_t *step,
                                             const oxh_adamw_tensor *device_tensors,
                                             const uint32_t *device_chunk_starts,
                                             uint32_t count, uint64_t total_chunks) {
  const char *name = "oxh_adamw_multi_tensor_table_step";
  OXH_REQUIRE(step != nullptr && device_tensors != nullptr && device_chunk_starts != nullptr,
              OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  OXH_REQUIRE(count > 0 && total_chunks > 0 && total_chunks < (1ull << 31), OXH_INVALID_SHAPE,
              std::string(name) + ": empty table or more than 2^31 chunks");
  const Hyper h{learning_rate, weight_decay, beta1, beta2, 1.0f, 1.0f, epsilon};
  OXH_REQUIRE(finite_hyper(h), OXH_INVALID_SHAPE,
              std::string(name) + ": non-finite hyper-parameter");
  hipStream_t s = oxh::as_stream(stream);
  oxh::launch(increment_step_kernel, dim3(1), dim3(1), 0, s, step);
  oxh_status st = oxh::launched(name);
  if (st != OXH_OK) return st;
  oxh::launch(adamw_table_kernel, dim3(static_cast<uint32_t>(total_chunks)), dim3(oxh::kBlock),
              0, s, h, device_tensors, device_chunk_starts, count, step);
  return oxh::launched(name);
}

}  // extern "C"

oxh_status oxh::adamw_table_step_advanced(hipStream_t s, float learning_rate, float weight_decay,
                                          float beta1, float beta2, float epsilon,
                                          const int32_t *step,
                                          const oxh_adamw_tensor *device_tensors,
                                          const uint32_t *device_chunk_starts, uint32_t count,
                                          uint64_t total_chunks) {
  const char *name = "adamw_table_step_advanced";
  OXH_REQUIRE(step != nullptr && device_tensors != nullptr && device_chunk_starts != nullptr,
              OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  OXH_REQUIRE(count > 0 && total_chunks > 0 && total_chunks < (1ull << 31), OXH_INVALID_SHAPE,
              std::string(name) + ": empty table or more than 2^31 chunks");
  const Hyper h{learning_rate, weight_decay, beta1, beta2, 1.0f, 1.0f, epsilon};
  OXH_REQUIRE(finite_hyper(h), OXH_INVALID_SHAPE,
              std::string(name) + ": non-finite hyper-parameter");
  oxh::launch(adamw_table_kernel, dim3(static_cast<uint32_t>(total_chunks)), dim3(oxh::kBlock),
              0, s, h, device_tensors, device_chunk_starts, count, step);
  return oxh::launched(name);
}

oxh_status oxh::launch_chunk_sums(hipStream_t s, const std::vector<ChunkSum> &sums,
                                  int32_t *step) {
  size_t k = 0;
  do {
    ChunkSumTable t{};
    t.step = k == 0 ? step : nullptr;
    uint32_t blocks = 0;
    for (; k < sums.size() && t.jobs < kChunkSumsPerLaunch; ++k, ++t.jobs) {
      const ChunkSum &c = sums[k];
      OXH_REQUIRE(c.partial != nullptr && c.out != nullptr && c.count > 0 && c.chunks > 0 &&
                      c.split <= c.count && (c.split == c.count || c.out2 != nullptr),
                  OXH_INVALID_SHAPE, "launch_chunk_sums: malformed sum");
      const uint32_t lanes = chunk_sum_lanes(c.chunks), per_block = 256 / lanes;
      t.job[t.jobs] = ChunkSumJob{c.partial, c.out,   c.out2, c.count,
                                  c.chunks,  lanes,   c.split, blocks};
      blocks += (c.count + per_block - 1) / per_block;
    }
    oxh::launch(sum_chunks_table_kernel, dim3(blocks > 0 ? blocks : 1), dim3(256), 0, s, t);
    oxh_status st = oxh::launched("launch_chunk_sums");
    if (st != OXH_OK) return st;
  } while (k < sums.size());
  return oxh::ok();
}

namespace {
oxh_status adamw_multi(const char *name, oxh_stream stream, const Hyper &h, const int32_t *step,
                       const oxh_adamw_tensor *tensors, uint32_t count) {
  if (count == 0) return oxh::ok();
  OXH_REQUIRE(tensors != nullptr, OXH_INVALID_SHAPE, std::string(name) + ": null table");
  OXH_REQUIRE(finite_hyper(h), OXH_INVALID_SHAPE,
              std::string(name) + ": non-finite hyper-parameter");
  for (uint32_t i = 0; i < count; ++i) {
    const oxh_adamw_tensor &t = tensors[i];
    if (t.n == 0) continue;
    OXH_REQUIRE(t.parameter && t.gradient && t.first_moment && t.second_moment,
                OXH_INVALID_SHAPE,
                "oxh_adamw_multi_tensor: tensor " + std::to_string(i) + " has a null pointer");
    OXH_REQUIRE(t.n <= (1ull << 44), OXH_INVALID_SHAPE,
                "oxh_adamw_multi_tensor: tensor too large");
  }
  // Tensors are packed into launches of at most kMaxTensors descriptors and at most 2^31
  // chunks each.
  uint32_t i = 0;
  while (i < count) {
    TensorTable table;
    std::memset(&table, 0, sizeof(table));
    uint64_t chunks = 0;
    uint32_t k = 0;
    while (i < count && k < static_cast<uint32_t>(kMaxTensors)) {
      const oxh_adamw_tensor &t = tensors[i];
      const uint64_t c = (t.n + kChunk - 1) / kChunk;
      if (c == 0) {
        ++i;
        continue;
      }
      if (k > 0 && chunks + c >= (1ull << 31)) break;
      table.s[k] = Streams{t.parameter, t.gradient, t.first_moment, t.second_moment,
                           t.parameter, t.first_moment, t.second_moment};
      table.n[k] = t.n;
      table.first_chunk[k] = static_cast<uint32_t>(chunks);
      const bool vec = oxh::aligned16(t.parameter) && oxh::aligned16(t.gradient) &&
                       oxh::aligned16(t.first_moment) && oxh::aligned16(t.second_moment);
      if (vec) {
        if (k < 32) table.vec_mask_lo |= 1u << k;
        else table.vec_mask_hi |= 1u << (k - 32);
      }
      chunks += c;
      ++k;
      ++i;
    }
    if (k == 0) continue;
    table.count = k;
    table.first_chunk[k] = static_cast<uint32_t>(chunks);
    oxh::launch(adamw_multi_kernel, dim3(static_cast<uint32_t>(chunks)), dim3(oxh::kBlock), 0,
                oxh::as_stream(stream), h, table, step);
    oxh_status st = oxh::launched(name);
    if (st != OXH_OK) return st;
  }
  return oxh::ok();
}

}  // namespace
