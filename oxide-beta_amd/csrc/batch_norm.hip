// batch_norm.hip -- BatchNorm2d (NCHW, fp32) training statistics with the running-stat update,
// apply, and the input / weight / bias backward with each channel reduction done once.
//
// Reference kernels (kernel_module.rs): batch_norm_statistics 827-875 and
// batch_norm_affine_backward 929-964 run one thread per channel over all N*H*W values (128
// threads busy at the named shape); batch_norm_apply 877-895 and batch_norm_input_backward
// 897-927 are one thread per element.  CPU semantics: evaluation.rs:490-597,
// autograd.rs:315-383.
//
// Design (gfx950):
//   * Reductions: grid (S slices, C channels).  Block (s, c) walks a contiguous slice of channel
//     c's N*H*W values as 128-bit loads (the N planes of a channel lie C*H*W floats apart; the
//     float4 index within the channel is split into plane / offset with a multiply-high
//     division), accumulates in fp64, reduces the block with wave64 shuffles and LDS, and writes
//     one fp64 partial pair.  The last block of a channel to finish (device-scope counter) sums
//     the S partials in fixed order and writes the per-channel results -- for the forward also
//     the running-stat update -- then resets the counter, so the workspace stays zeroed.
//   * Apply / input-backward: one streaming pass with 128-bit loads; per-channel values are
//     gathered from L1-resident [C] vectors.
//   * Per-element arithmetic follows the CPU path's fp32 operation order exactly
//     (-ffp-contract=off): y = ((x - mean) * inv) * w + b, x_hat = (x - mean) * inv,
//     dx = ((w * inv) / M) * ((M * g - sum_g) - x_hat * sum_g_xhat).
#include <hip/hip_runtime.h>

#include <cmath>
#include <string>

#include "common.h"

namespace {

constexpr int kRedBlock = 256;  // 4 waves
constexpr int kRedWaves = kRedBlock / 64;

struct Geometry {
  uint32_t batch, channels, spatial;
  uint64_t samples;      // batch * spatial (values per channel)
  uint32_t slices;       // S
  uint64_t slice_len;    // values per slice (multiple of 4 on the vector path)
  bool vec;              // spatial % 4 == 0 and pointers aligned
  oxh::FastDiv spatial_div;   // divides a channel-relative index by spatial (or spatial / 4)
};

// Workspace layout: double2 partial[C][S], then uint32 counter[C].
inline uint64_t partial_bytes(uint64_t c, uint64_t s) { return c * s * 16; }
inline uint64_t workspace_bytes_for(uint64_t c, uint64_t s) {
  return ((partial_bytes(c, s) + c * 4) + 255) / 256 * 256;
}

uint32_t choose_slices(uint64_t channels, uint64_t samples) {
  // Aim for ~8 blocks per CU in total, but keep >= 4096 values per block.
  uint64_t target = (8ull * oxh::kComputeUnits + channels - 1) / channels;
  uint64_t max_by_work = samples / 4096;
  if (max_by_work < 1) max_by_work = 1;
  uint64_t s = target < max_by_work ? target : max_by_work;
  if (s > 1024) s = 1024;
  if (s < 1) s = 1;
  return static_cast<uint32_t>(s);
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Block-wide sum of two doubles; the result is valid in thread 0.
__device__ __forceinline__ void block_sum2(double &a, double &b, double (*lds)[kRedWaves]) {
  a = wave_sum(a);
  b = wave_sum(b);
  const int wave = threadIdx.x / 64, lane_id = threadIdx.x % 64;
  if (lane_id == 0) {
    lds[0][wave] = a;
    lds[1][wave] = b;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    a = 0.0;
    b = 0.0;
#pragma unroll
    for (int w = 0; w < kRedWaves; ++w) {
      a += lds[0][w];
      b += lds[1][w];
    }
  }
}

// Called by thread 0 of every block after its partial is stored: returns true in exactly one
// block per channel (the last to arrive), after which that block may read all partials.
__device__ __forceinline__ bool arrive_last(uint32_t *counter, uint32_t expected) {
  __threadfence();
  const uint32_t prev =
      __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
  const bool last = prev + 1 == expected;
  if (last) {
    __threadfence();
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return last;
}

// Address (in floats) of channel-relative value j of channel c.
__device__ __forceinline__ uint64_t nchw_index(const Geometry &g, uint32_t c, uint32_t j) {
  const uint32_t n = oxh::fast_div(j, g.spatial_div);
  const uint32_t i = j - n * g.spatial_div.d;
  return (static_cast<uint64_t>(n) * g.channels + c) * g.spatial_div.d + i;
}

// ---------------------------------------------------------------- forward statistics

struct StatsOut {
  float *mean, *inverse_std, *unbiased_variance;  // unbiased_variance may be null
  float *running_mean, *running_variance;         // null: no running update
  float momentum, epsilon;
};

__global__ __launch_bounds__(kRedBlock) void bn_stats_kernel(Geometry g, const float *__restrict__ x,
                                                           StatsOut out, double2 *partial,
                                                           uint32_t *counter) {
  __shared__ double lds[2][kRedWaves];
  __shared__ bool is_last;
  const uint32_t s = blockIdx.x, c = blockIdx.y;
  // Shift by the channel's first value: sums of (x - K) and (x - K)^2 in fp64 keep the
  // variance free of cancellation even when |mean| >> std.
  const float shift = x[static_cast<uint64_t>(c) * g.spatial];
  const double k = shift;
  double sum = 0.0, sq = 0.0;
  const uint64_t begin = static_cast<uint64_t>(s) * g.slice_len;
  uint64_t end = begin + g.slice_len;
  if (end > g.samples) end = g.samples;
  if (g.vec) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const uint32_t b4 = static_cast<uint32_t>(begin / 4), e4 = static_cast<uint32_t>(end / 4);
    uint32_t j = b4 + threadIdx.x;
    for (; j + 3 * kRedBlock < e4; j += 4 * kRedBlock) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = x4[nchw_index(g, c, j + u * kRedBlock)];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const double d0 = static_cast<double>(v[u].x) - k, d1 = static_cast<double>(v[u].y) - k;
        const double d2 = static_cast<double>(v[u].z) - k, d3 = static_cast<double>(v[u].w) - k;
        sum += (d0 + d1) + (d2 + d3);
        sq += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
      }
    }
    for (; j < e4; j += kRedBlock) {
      const float4 v = x4[nchw_index(g, c, j)];
      const double d0 = static_cast<double>(v.x) - k, d1 = static_cast<double>(v.y) - k;
      const double d2 = static_cast<double>(v.z) - k, d3 = static_cast<double>(v.w) - k;
      sum += (d0 + d1) + (d2 + d3);
      sq += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
    }
  } else {
    for (uint64_t j = begin + threadIdx.x; j < end; j += kRedBlock) {
      const double d = static_cast<double>(x[nchw_index(g, c, static_cast<uint32_t>(j))]) - k;
      sum += d;
      sq += d * d;
    }
  }
  block_sum2(sum, sq, lds);
  if (threadIdx.x == 0) {
    partial[static_cast<uint64_t>(c) * g.slices + s] = make_double2(sum, sq);
    is_last = arrive_last(&counter[c], g.slices);
  }
  __syncthreads();
  if (!is_last || threadIdx.x != 0) return;
  // Last block of channel c: combine the slices in fixed order.
  double total = 0.0, total_sq = 0.0;
  for (uint32_t t = 0; t < g.slices; ++t) {
    const double2 p = partial[static_cast<uint64_t>(c) * g.slices + t];
    total += p.x;
    total_sq += p.y;
  }
  const double m = static_cast<double>(g.samples);
  const double mean_shifted = total / m;
  double var = total_sq / m - mean_shifted * mean_shifted;
  if (var < 0.0) var = 0.0;
  const float mean_f = static_cast<float>(k + mean_shifted);
  const float var_f = static_cast<float>(var);
  // evaluation.rs:531-534: (variance + epsilon).sqrt().recip()
  out.mean[c] = mean_f;
  out.inverse_std[c] = 1.0f / sqrtf(var_f + out.epsilon);
  // evaluation.rs:537-558: the running update recomputes the statistics with epsilon 0 and
  // recovers the biased variance as inv_std.powi(-2) (== 1 / (inv * inv)), then applies the
  // unbiased correction M / (M - 1) in fp32.
  const float inv0 = 1.0f / sqrtf(var_f);
  const float biased = 1.0f / (inv0 * inv0);
  const float correction =
      static_cast<float>(g.samples) / static_cast<float>(g.samples - 1);
  if (out.unbiased_variance) out.unbiased_variance[c] = biased * correction;
  if (out.running_mean) {
    const float mom = out.momentum;
    out.running_mean[c] = (1.0f - mom) * out.running_mean[c] + mom * mean_f;
    out.running_variance[c] =
        (1.0f - mom) * out.running_variance[c] + mom * biased * correction;
  }
}

// ---------------------------------------------------------------- backward affine reduction

struct AffineOut {
  float *weight_gradient, *bias_gradient;
};

__global__ __launch_bounds__(kRedBlock) void bn_affine_kernel(
    Geometry g, const float *__restrict__ grad, const float *__restrict__ x,
    const float *__restrict__ mean, const float *__restrict__ inverse_std, AffineOut out,
    double2 *partial, uint32_t *counter) {
  __shared__ double lds[2][kRedWaves];
  __shared__ bool is_last;
  const uint32_t s = blockIdx.x, c = blockIdx.y;
  const float mu = mean[c], inv = inverse_std[c];
  double sg = 0.0, sgx = 0.0;
  const uint64_t begin = static_cast<uint64_t>(s) * g.slice_len;
  uint64_t end = begin + g.slice_len;
  if (end > g.samples) end = g.samples;
  // autograd.rs:353-362: normalized = (x - mean) * inv (fp32); terms g and g * normalized.
  if (g.vec) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const float4 *g4 = reinterpret_cast<const float4 *>(grad);
    const uint32_t b4 = static_cast<uint32_t>(begin / 4), e4 = static_cast<uint32_t>(end / 4);
    uint32_t j = b4 + threadIdx.x;
    auto accumulate = [&](const float4 &xv, const float4 &gv) {
      const float n0 = (xv.x - mu) * inv, n1 = (xv.y - mu) * inv;
      const float n2 = (xv.z - mu) * inv, n3 = (xv.w - mu) * inv;
      sg += (static_cast<double>(gv.x) + static_cast<double>(gv.y)) +
            (static_cast<double>(gv.z) + static_cast<double>(gv.w));
      sgx += (static_cast<double>(gv.x * n0) + static_cast<double>(gv.y * n1)) +
             (static_cast<double>(gv.z * n2) + static_cast<double>(gv.w * n3));
    };
    for (; j + 3 * kRedBlock < e4; j += 4 * kRedBlock) {
      float4 xv[4], gv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint64_t idx = nchw_index(g, c, j + u * kRedBlock);
        xv[u] = x4[idx];
        gv[u] = g4[idx];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) accumulate(xv[u], gv[u]);
    }
    for (; j < e4; j += kRedBlock) {
      const uint64_t idx = nchw_index(g, c, j);
      accumulate(x4[idx], g4[idx]);
    }
  } else {
    for (uint64_t j = begin + threadIdx.x; j < end; j += kRedBlock) {
      const uint64_t idx = nchw_index(g, c, static_cast<uint32_t>(j));
      const float gv = grad[idx];
      const float nv = (x[idx] - mu) * inv;
      sg += static_cast<double>(gv);
      sgx += static_cast<double>(gv * nv);
    }
  }
  block_sum2(sg, sgx, lds);
  if (threadIdx.x == 0) {
    partial[static_cast<uint64_t>(c) * g.slices + s] = make_double2(sg, sgx);
    is_last = arrive_last(&counter[c], g.slices);
  }
  __syncthreads();
  if (!is_last || threadIdx.x != 0) return;
  double total_g = 0.0, total_gx = 0.0;
  for (uint32_t t = 0; t < g.slices; ++t) {
    const double2 p = partial[static_cast<uint64_t>(c) * g.slices + t];
    total_g += p.x;
    total_gx += p.y;
  }
  out.weight_gradient[c] = static_cast<float>(total_gx);
  out.bias_gradient[c] = static_cast<float>(total_g);
}

// ---------------------------------------------------------------- elementwise passes

struct ChannelMap {
  uint64_t total;        // batch * channels * spatial
  oxh::FastDiv plane;    // divides an element (or float4) index by spatial (or spatial / 4)
  oxh::FastDiv channel;  // divides a plane index by channels
  bool vec;
};

__device__ __forceinline__ uint32_t channel_of(const ChannelMap &m, uint32_t idx) {
  const uint32_t p = oxh::fast_div(idx, m.plane);
  return p - oxh::fast_div(p, m.channel) * m.channel.d;
}

// 64-bit element indices: the plane index of element e is e / spatial; only the plane index is
// taken through the 32-bit divider, so totals up to 2^31 planes are supported.
__device__ __forceinline__ uint32_t channel_of64(const ChannelMap &m, uint64_t idx) {
  const uint64_t p = idx / m.plane.d;
  return static_cast<uint32_t>(p % m.channel.d);
}

struct ApplyArgs {
  const float *x, *weight, *bias, *mean, *inverse_std;
  float *y;
};

__device__ __forceinline__ float bn_apply1(float v, float mu, float inv, float w, float b) {
  return (v - mu) * inv * w + b;
}

constexpr int kMapUnroll = 4;

__global__ __launch_bounds__(oxh::kBlock) void bn_apply_kernel(ChannelMap m, ApplyArgs a) {
  const uint64_t tile = static_cast<uint64_t>(oxh::kBlock) * kMapUnroll;
  if (m.vec) {
    const uint64_t n4 = m.total / 4;
    const float4 *x4 = reinterpret_cast<const float4 *>(a.x);
    float4 *y4 = reinterpret_cast<float4 *>(a.y);
    for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * tile; base < n4;
         base += static_cast<uint64_t>(gridDim.x) * tile) {
      float4 v[kMapUnroll];
      uint32_t ch[kMapUnroll];
#pragma unroll
      for (int u = 0; u < kMapUnroll; ++u) {
        const uint64_t q = base + threadIdx.x + u * oxh::kBlock;
        if (q < n4) {
          v[u] = x4[q];
          ch[u] = channel_of(m, static_cast<uint32_t>(q));
        }
      }
#pragma unroll
      for (int u = 0; u < kMapUnroll; ++u) {
        const uint64_t q = base + threadIdx.x + u * oxh::kBlock;
        if (q < n4) {
          const uint32_t c = ch[u];
          const float mu = a.mean[c], inv = a.inverse_std[c], w = a.weight[c], b = a.bias[c];
          float4 r;
          r.x = bn_apply1(v[u].x, mu, inv, w, b);
          r.y = bn_apply1(v[u].y, mu, inv, w, b);
          r.z = bn_apply1(v[u].z, mu, inv, w, b);
          r.w = bn_apply1(v[u].w, mu, inv, w, b);
          y4[q] = r;
        }
      }
    }
  } else {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < m.total;
         e += stride) {
      const uint32_t c = channel_of64(m, e);
      a.y[e] = bn_apply1(a.x[e], a.mean[c], a.inverse_std[c], a.weight[c], a.bias[c]);
    }
  }
}

struct InputBackwardArgs {
  const float *grad, *x, *weight, *mean, *inverse_std, *weight_gradient, *bias_gradient;
  float *dx;
  float samples;  // M as fp32 (autograd.rs:344-345)
  bool training;
};

__device__ __forceinline__ float bn_dx1(const InputBackwardArgs &a, uint32_t c, float g,
                                        float v) {
  const float w = a.weight[c], inv = a.inverse_std[c];
  if (!a.training) return g * w * inv;  // autograd.rs:374-378
  const float normalized = (v - a.mean[c]) * inv;
  // autograd.rs:367-373
  return w * inv / a.samples *
         (a.samples * g - a.bias_gradient[c] - normalized * a.weight_gradient[c]);
}

__global__ __launch_bounds__(oxh::kBlock) void bn_input_backward_kernel(ChannelMap m,
                                                                        InputBackwardArgs a) {
  const uint64_t tile = static_cast<uint64_t>(oxh::kBlock) * kMapUnroll;
  if (m.vec) {
    const uint64_t n4 = m.total / 4;
    const float4 *x4 = reinterpret_cast<const float4 *>(a.x);
    const float4 *g4 = reinterpret_cast<const float4 *>(a.grad);
    float4 *d4 = reinterpret_cast<float4 *>(a.dx);
    for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * tile; base < n4;
         base += static_cast<uint64_t>(gridDim.x) * tile) {
      float4 xv[kMapUnroll], gv[kMapUnroll];
      uint32_t ch[kMapUnroll];
#pragma unroll
      for (int u = 0; u < kMapUnroll; ++u) {
        const uint64_t q = base + threadIdx.x + u * oxh::kBlock;
        if (q < n4) {
          gv[u] = g4[q];
          if (a.training) xv[u] = x4[q];
          ch[u] = channel_of(m, static_cast<uint32_t>(q));
        }
      }
#pragma unroll
      for (int u = 0; u < kMapUnroll; ++u) {
        const uint64_t q = base + threadIdx.x + u * oxh::kBlock;
        if (q < n4) {
          const uint32_t c = ch[u];
          float4 r;
          r.x = bn_dx1(a, c, gv[u].x, xv[u].x);
          r.y = bn_dx1(a, c, gv[u].y, xv[u].y);
          r.z = bn_dx1(a, c, gv[u].z, xv[u].z);
          r.w = bn_dx1(a, c, gv[u].w, xv[u].w);
          d4[q] = r;
        }
      }
    }
  } else {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < m.total;
         e += stride) {
      const uint32_t c = channel_of64(m, e);
      a.dx[e] = bn_dx1(a, c, a.grad[e], a.training ? a.x[e] : 0.0f);
    }
  }
}

__global__ void bn_update_running_kernel(uint32_t channels, float momentum,
                                         const float *batch_mean, const float *batch_variance,
                                         const float *old_mean, const float *old_variance,
                                         float *new_mean, float *new_variance) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= channels) return;
  const float m = old_mean[c], v = old_variance[c];
  new_mean[c] = (1.0f - momentum) * m + momentum * batch_mean[c];
  new_variance[c] = (1.0f - momentum) * v + momentum * batch_variance[c];
}

__global__ void bn_running_inverse_std_kernel(uint32_t channels, float epsilon,
                                              const float *variance, float *inverse_std) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= channels) return;
  inverse_std[c] = 1.0f / sqrtf(variance[c] + epsilon);
}

// ---------------------------------------------------------------- host side

oxh_status check_shape(const char *name, uint64_t batch, uint64_t channels, uint64_t spatial) {
  OXH_REQUIRE(batch > 0 && channels > 0 && spatial > 0, OXH_INVALID_SHAPE,
              std::string(name) + ": empty NCHW shape");
  OXH_REQUIRE(batch < (1ull << 31) && channels <= 65535 && spatial < (1ull << 31),
              OXH_INVALID_SHAPE, std::string(name) + ": dimension too large (channels <= 65535)");
  OXH_REQUIRE(batch * spatial < (1ull << 31), OXH_INVALID_SHAPE,
              std::string(name) + ": more than 2^31 values per channel");
  OXH_REQUIRE(batch * channels * spatial < (1ull << 40), OXH_INVALID_SHAPE,
              std::string(name) + ": tensor too large");
  return oxh::ok();
}

Geometry make_geometry(uint64_t batch, uint64_t channels, uint64_t spatial, bool aligned) {
  Geometry g{};
  g.batch = static_cast<uint32_t>(batch);
  g.channels = static_cast<uint32_t>(channels);
  g.spatial = static_cast<uint32_t>(spatial);
  g.samples = batch * spatial;
  g.vec = aligned && spatial % 4 == 0;
  g.slices = choose_slices(channels, g.samples);
  uint64_t len = (g.samples + g.slices - 1) / g.slices;
  if (g.vec) len = (len + 3) / 4 * 4;
  g.slice_len = len;
  // Slices that would start past the end are dropped.
  g.slices = static_cast<uint32_t>((g.samples + len - 1) / len);
  g.spatial_div = oxh::make_fastdiv(static_cast<uint32_t>(g.vec ? spatial / 4 : spatial));
  return g;
}

ChannelMap make_channel_map(uint64_t batch, uint64_t channels, uint64_t spatial, bool aligned) {
  ChannelMap m{};
  m.total = batch * channels * spatial;
  m.vec = aligned && spatial % 4 == 0 && m.total / 4 < (1ull << 31);
  m.plane = oxh::make_fastdiv(static_cast<uint32_t>(m.vec ? spatial / 4 : spatial));
  m.channel = oxh::make_fastdiv(static_cast<uint32_t>(channels));
  return m;
}

uint32_t map_grid(const ChannelMap &m) {
  const uint64_t units = m.vec ? m.total / 4 : m.total;
  const uint64_t per_block = static_cast<uint64_t>(oxh::kBlock) * (m.vec ? kMapUnroll : 1);
  uint64_t grid = (units + per_block - 1) / per_block;
  if (grid < 1) grid = 1;
  if (grid > (1u << 20)) grid = 1u << 20;
  return static_cast<uint32_t>(grid);
}

oxh_status check_workspace(const char *name, const Geometry &g, void *workspace,
                           uint64_t bytes) {
  const uint64_t need = workspace_bytes_for(g.channels, g.slices);
  OXH_REQUIRE(workspace != nullptr && bytes >= need, OXH_INVALID_SHAPE,
              std::string(name) + ": workspace of " + std::to_string(need) +
                  " bytes required (oxh_batch_norm_workspace_size)");
  OXH_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15u) == 0, OXH_INVALID_SHAPE,
              std::string(name) + ": workspace must be 16-byte aligned");
  return oxh::ok();
}

oxh_status launch_stats(const char *name, oxh_stream stream, uint64_t batch, uint64_t channels,
                        uint64_t spatial, const float *input, const StatsOut &out,
                        void *workspace, uint64_t workspace_bytes) {
  oxh_status st = check_shape(name, batch, channels, spatial);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(batch * spatial > 1, OXH_EXECUTION,
              "BatchNorm training requires more than one value per channel");
  OXH_REQUIRE(input && out.mean && out.inverse_std, OXH_INVALID_SHAPE,
              std::string(name) + ": null pointer");
  const Geometry g = make_geometry(batch, channels, spatial, oxh::aligned16(input));
  st = check_workspace(name, g, workspace, workspace_bytes);
  if (st != OXH_OK) return st;
  auto *partial = static_cast<double2 *>(workspace);
  auto *counter = reinterpret_cast<uint32_t *>(static_cast<char *>(workspace) +
                                               partial_bytes(g.channels, g.slices));
  hipLaunchKernelGGL(bn_stats_kernel, dim3(g.slices, g.channels), dim3(kRedBlock), 0,
                     oxh::as_stream(stream), g, input, out, partial, counter);
  return oxh::launched(name);
}

oxh_status launch_affine(const char *name, oxh_stream stream, uint64_t batch, uint64_t channels,
                         uint64_t spatial, const float *gradient, const float *input,
                         const float *mean, const float *inverse_std, float *weight_gradient,
                         float *bias_gradient, void *workspace, uint64_t workspace_bytes) {
  oxh_status st = check_shape(name, batch, channels, spatial);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(gradient && input && mean && inverse_std && weight_gradient && bias_gradient,
              OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  const Geometry g = make_geometry(batch, channels, spatial,
                                   oxh::aligned16(input) && oxh::aligned16(gradient));
  st = check_workspace(name, g, workspace, workspace_bytes);
  if (st != OXH_OK) return st;
  auto *partial = static_cast<double2 *>(workspace);
  auto *counter = reinterpret_cast<uint32_t *>(static_cast<char *>(workspace) +
                                               partial_bytes(g.channels, g.slices));
  hipLaunchKernelGGL(bn_affine_kernel, dim3(g.slices, g.channels), dim3(kRedBlock), 0,
                     oxh::as_stream(stream), g, gradient, input, mean, inverse_std,
                     AffineOut{weight_gradient, bias_gradient}, partial, counter);
  return oxh::launched(name);
}

oxh_status launch_apply(const char *name, oxh_stream stream, uint64_t batch, uint64_t channels,
                        uint64_t spatial, const ApplyArgs &a) {
  oxh_status st = check_shape(name, batch, channels, spatial);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(a.x && a.weight && a.bias && a.mean && a.inverse_std && a.y, OXH_INVALID_SHAPE,
              std::string(name) + ": null pointer");
  const uint64_t bytes = batch * channels * spatial * 4;
  OXH_REQUIRE(!oxh::any_overlap(a.x, bytes, a.y, bytes) || a.x == a.y, OXH_INVALID_SHAPE,
              std::string(name) + ": output partially overlaps the input");
  const ChannelMap m = make_channel_map(batch, channels, spatial,
                                        oxh::aligned16(a.x) && oxh::aligned16(a.y));
  hipLaunchKernelGGL(bn_apply_kernel, dim3(map_grid(m)), dim3(oxh::kBlock), 0,
                     oxh::as_stream(stream), m, a);
  return oxh::launched(name);
}

oxh_status launch_input_backward(const char *name, oxh_stream stream, uint64_t batch,
                                 uint64_t channels, uint64_t spatial, const InputBackwardArgs &a) {
  oxh_status st = check_shape(name, batch, channels, spatial);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(a.grad && a.weight && a.inverse_std && a.dx, OXH_INVALID_SHAPE,
              std::string(name) + ": null pointer");
  OXH_REQUIRE(!a.training || (a.x && a.mean && a.weight_gradient && a.bias_gradient),
              OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  const bool aligned = oxh::aligned16(a.grad) && oxh::aligned16(a.dx) &&
                       (!a.training || oxh::aligned16(a.x));
  const ChannelMap m = make_channel_map(batch, channels, spatial, aligned);
  hipLaunchKernelGGL(bn_input_backward_kernel, dim3(map_grid(m)), dim3(oxh::kBlock), 0,
                     oxh::as_stream(stream), m, a);
  return oxh::launched(name);
}

}  // namespace

extern "C" {

oxh_status oxh_batch_norm_workspace_size(uint64_t batch, uint64_t channels, uint64_t spatial,
                                         uint64_t *bytes) {
  OXH_REQUIRE(bytes != nullptr, OXH_INVALID_SHAPE, "bytes is null");
  oxh_status st = check_shape("oxh_batch_norm_workspace_size", batch, channels, spatial);
  if (st != OXH_OK) return st;
  // The slice count does not depend on alignment, so either geometry gives the same size.
  const Geometry g = make_geometry(batch, channels, spatial, true);
  const Geometry h = make_geometry(batch, channels, spatial, false);
  const uint64_t a = workspace_bytes_for(g.channels, g.slices);
  const uint64_t b = workspace_bytes_for(h.channels, h.slices);
  *bytes = a > b ? a : b;
  return oxh::ok();
}

oxh_status oxh_batch_norm_statistics(oxh_stream stream, uint64_t batch, uint64_t channels,
                                     uint64_t spatial, float epsilon, const float *input,
                                     float *mean, float *inverse_std, float *unbiased_variance,
                                     void *workspace, uint64_t workspace_bytes) {
  StatsOut out{mean, inverse_std, unbiased_variance, nullptr, nullptr, 0.0f, epsilon};
  return launch_stats("oxh_batch_norm_statistics", stream, batch, channels, spatial, input, out,
                      workspace, workspace_bytes);
}

oxh_status oxh_batch_norm_update_running(oxh_stream stream, uint64_t channels, float momentum,
                                         const float *batch_mean, const float *batch_variance,
                                         const float *old_mean, const float *old_variance,
                                         float *new_mean, float *new_variance) {
  if (channels == 0) return oxh::ok();
  OXH_REQUIRE(channels < (1ull << 31), OXH_INVALID_SHAPE, "too many channels");
  OXH_REQUIRE(batch_mean && batch_variance && old_mean && old_variance && new_mean &&
                  new_variance,
              OXH_INVALID_SHAPE, "oxh_batch_norm_update_running: null pointer");
  const uint32_t grid = static_cast<uint32_t>((channels + 255) / 256);
  hipLaunchKernelGGL(bn_update_running_kernel, dim3(grid), dim3(256), 0, oxh::as_stream(stream),
                     static_cast<uint32_t>(channels), momentum, batch_mean, batch_variance,
                     old_mean, old_variance, new_mean, new_variance);
  return oxh::launched("oxh_batch_norm_update_running");
}

oxh_status oxh_batch_norm_running_inverse_std(oxh_stream stream, uint64_t channels,
                                              float epsilon, const float *variance,
                                              float *inverse_std) {
  if (channels == 0) return oxh::ok();
  OXH_REQUIRE(channels < (1ull << 31), OXH_INVALID_SHAPE, "too many channels");
  OXH_REQUIRE(variance && inverse_std, OXH_INVALID_SHAPE,
              "oxh_batch_norm_running_inverse_std: null pointer");
  const uint32_t grid = static_cast<uint32_t>((channels + 255) / 256);
  hipLaunchKernelGGL(bn_running_inverse_std_kernel, dim3(grid), dim3(256), 0,
                     oxh::as_stream(stream), static_cast<uint32_t>(channels), epsilon, variance,
                     inverse_std);
  return oxh::launched("oxh_batch_norm_running_inverse_std");
}

oxh_status oxh_batch_norm_apply(oxh_stream stream, uint64_t batch, uint64_t channels,
                                uint64_t spatial, const float *input, const float *weight,
                                const float *bias, const float *mean, const float *inverse_std,
                                float *output) {
  return launch_apply("oxh_batch_norm_apply", stream, batch, channels, spatial,
                      ApplyArgs{input, weight, bias, mean, inverse_std, output});
}

oxh_status oxh_batch_norm_affine_backward(oxh_stream stream, uint64_t batch, uint64_t channels,
                                          uint64_t spatial, const float *gradient,
                                          const float *input, const float *mean,
                                          const float *inverse_std, float *weight_gradient,
                                          float *bias_gradient, void *workspace,
                                          uint64_t workspace_bytes) {
  return launch_affine("oxh_batch_norm_affine_backward", stream, batch, channels, spatial,
                       gradient, input, mean, inverse_std, weight_gradient, bias_gradient,
                       workspace, workspace_bytes);
}

oxh_status oxh_batch_norm_input_backward(oxh_stream stream, uint64_t batch, uint64_t channels,
                                         uint64_t spatial, int training, const float *gradient,
                                         const float *input, const float *weight,
                                         const float *mean, const float *inverse_std,
                                         const float *weight_gradient,
                                         const float *bias_gradient, float *output) {
  InputBackwardArgs a{gradient, input, weight, mean, inverse_std, weight_gradient,
                      bias_gradient, output, static_cast<float>(batch * spatial),
                      training != 0};
  return launch_input_backward("oxh_batch_norm_input_backward", stream, batch, channels,
                               spatial, a);
}

oxh_status oxh_batch_norm_statistics_running(oxh_stream stream, uint64_t batch,
                                             uint64_t channels, uint64_t spatial, float momentum,
                                             float epsilon, const float *input,
                                             float *running_mean, float *running_variance,
                                             float *saved_mean, float *saved_inverse_std,
                                             void *workspace, uint64_t workspace_bytes) {
  OXH_REQUIRE(std::isfinite(momentum) && std::isfinite(epsilon) && epsilon >= 0.0f,
              OXH_INVALID_SHAPE, "oxh_batch_norm_statistics_running: bad momentum or epsilon");
  OXH_REQUIRE(running_mean && running_variance, OXH_INVALID_SHAPE,
              "oxh_batch_norm_statistics_running: null running statistics");
  StatsOut out{saved_mean, saved_inverse_std, nullptr, running_mean, running_variance, momentum,
               epsilon};
  return launch_stats("oxh_batch_norm_statistics_running", stream, batch, channels, spatial,
                      input, out, workspace, workspace_bytes);
}

oxh_status oxh_batch_norm_forward_train(oxh_stream stream, uint64_t batch, uint64_t channels,
                                        uint64_t spatial, float momentum, float epsilon,
                                        const float *input, const float *weight,
                                        const float *bias, float *running_mean,
                                        float *running_variance, float *saved_mean,
                                        float *saved_inverse_std, float *output, void *workspace,
                                        uint64_t workspace_bytes) {
  oxh_status st = oxh_batch_norm_statistics_running(stream, batch, channels, spatial, momentum,
                                                    epsilon, input, running_mean,
                                                    running_variance, saved_mean,
                                                    saved_inverse_std, workspace,
                                                    workspace_bytes);
  if (st != OXH_OK) return st;
  return launch_apply("oxh_batch_norm_forward_train", stream, batch, channels, spatial,
                      ApplyArgs{input, weight, bias, saved_mean, saved_inverse_std, output});
}

oxh_status oxh_batch_norm_backward_train(oxh_stream stream, uint64_t batch, uint64_t channels,
                                         uint64_t spatial, const float *gradient,
                                         const float *input, const float *weight,
                                         const float *saved_mean,
                                         const float *saved_inverse_std, float *input_gradient,
                                         float *weight_gradient, float *bias_gradient,
                                         void *workspace, uint64_t workspace_bytes) {
  oxh_status st = launch_affine("oxh_batch_norm_backward_train", stream, batch, channels,
                                spatial, gradient, input, saved_mean, saved_inverse_std,
                                weight_gradient, bias_gradient, workspace, workspace_bytes);
  if (st != OXH_OK) return st;
  InputBackwardArgs a{gradient, input, weight, saved_mean, saved_inverse_std, weight_gradient,
                      bias_gradient, input_gradient, static_cast<float>(batch * spatial), true};
  return launch_input_backward("oxh_batch_norm_backward_train", stream, batch, channels, spatial,
                               a);
}

}  // extern "C"
