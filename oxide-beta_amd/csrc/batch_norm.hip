// batch_norm.hip -- BatchNorm2d (NCHW, fp32) training statistics with the running-stat update,
// apply, and the input / weight / bias backward with each channel reduction done once.
//
// Reference kernels (kernel_module.rs): batch_norm_statistics 827-875 and
// batch_norm_affine_backward 929-964 run one thread per channel over all N*H*W values (128
// threads busy at the named shape); batch_norm_apply 877-895 and batch_norm_input_backward
// 897-927 are one thread per element.  CPU semantics: evaluation.rs:490-597,
// autograd.rs:315-383.
//
// Design (gfx950), two launches per direction, no inter-block synchronization:
//   * Reduce: grid (S slices, C channels).  Block (s, c) walks a contiguous slice of channel
//     c's N*H*W values with 128-bit loads (the N planes of a channel lie C*H*W floats apart; the
//     float4 index within the channel is split into plane / offset with a multiply-high
//     division), accumulates in fp64, reduces the block with wave64 shuffles and LDS, and stores
//     one fp64 partial pair to the workspace.  Forward partials are sums of (x - K) and
//     (x - K)^2 with K = x[0, c, 0]; backward partials are sums of g and g * x_hat.
//   * Map: each block of the streaming pass (apply or dx) covers a flat range of 1024 elements
//     (one float4 per lane per stream: on MI355X short blocks stream faster than long per-lane
//     loops, and they re-read what the reduce just read while it is still in the 256 MB MALL).
//     It issues its loads, then finalizes the statistics of the <= kMaxPlanes channels its
//     planes belong to, summing that channel's S partials in a fixed order, so all blocks
//     derive bit-identical values; the block holding the first element of plane (n = 0, c)
//     also writes the per-channel outputs (saved mean / inverse std and the running update, or
//     dweight / dbias).  Channel values are read back from LDS.
//     A kernel boundary separates reduce and map, so no fence or atomic is needed (on gfx950 an
//     agent-scope release writes back the XCD's L2, far too costly per block).
//   * Small planes (H*W < OXH_BN_FLAT_SPATIAL, e.g. the 7x7 ... 1x1 layers of a MobileNet at
//     MNIST resolution): a map block would span hundreds of planes and finalize each, so one
//     wave per channel finalizes into the per-channel outputs (saved mean / inverse std and the
//     running update, or dweight / dbias) and a flat pass reads them per element: three
//     launches per direction, each channel finalized once, same arithmetic.
//   * Per-element arithmetic follows the CPU path's fp32 operation order exactly
//     (-ffp-contract=off): y = ((x - mean) * inv) * w + b, x_hat = (x - mean) * inv,
//     dx = ((w * inv) / M) * ((M * g - sum_g) - x_hat * sum_g_xhat), eval dx = (g * w) * inv.
#include <hip/hip_runtime.h>

#include <cmath>
#include <mutex>
#include <string>

#include "bn_channel.h"
#include "common.h"

namespace {

using oxh::block_sum2_all;
using oxh::channel_backward_kept;
using oxh::channel_forward_kept;
using oxh::channel_index;
using oxh::ChannelGeom;
using oxh::forward_moments;
using oxh::kChannelKeep;
using oxh::Moments;
using oxh::relu_masked;
using oxh::StatsOut;
using oxh::wave_sum;
using oxh::load_running;
using oxh::RunningPrev;
using oxh::write_forward_outputs;

// Launch-shape constants (overridable at build time for tuning sweeps).
#ifndef OXH_BN_RED_BLOCKS_PER_CU
#define OXH_BN_RED_BLOCKS_PER_CU 32  // reduce grid: target blocks per CU over all channels
#endif
#ifndef OXH_BN_RED_UNROLL
#define OXH_BN_RED_UNROLL 4  // float4 loads in flight per thread per stream in a reduce pass
#endif
#ifndef OXH_BN_NT_STORE
#define OXH_BN_NT_STORE 3  // non-temporal stores: 1 = apply's y, 2 = input backward's dx
#endif
constexpr int kStorePolicy = 2 | 16;  // buffer store cache policy of the map outputs: nt | sc1
#ifndef OXH_BN_MAP_VEC
#define OXH_BN_MAP_VEC 2  // float4 per thread per stream in a map block
#endif
#ifndef OXH_BN_FLAT_SPATIAL
#define OXH_BN_FLAT_SPATIAL 64  // planes smaller than this use finalize + flat map
#endif

constexpr int kRedBlock = 256;  // 4 waves
constexpr int kRedWaves = kRedBlock / 64;
constexpr int kRedUnroll = OXH_BN_RED_UNROLL;
constexpr uint32_t kMaxSlices = 64;  // partials per channel (summed by every map block)
constexpr int kMapBlock = 256;
constexpr int kMapVec = OXH_BN_MAP_VEC;
constexpr uint32_t kMapElems = kMapBlock * 4 * kMapVec;  // elements per map block
constexpr uint32_t kMaxPlanes = 256;  // planes one map block may touch
constexpr uint64_t kFlatSpatial = OXH_BN_FLAT_SPATIAL;

// ---------------------------------------------------------------- geometry

struct Geometry {
  uint32_t batch, channels, spatial;
  uint64_t samples;          // batch * spatial (values per channel)
  uint32_t slices;           // S
  uint64_t slice_len;        // values per slice (always a multiple of 4)
  bool vec;                  // spatial % 4 == 0 and pointers aligned
  oxh::FastDiv spatial_div;  // divides a channel-relative index by spatial (or spatial / 4)
};

uint32_t choose_slices(uint64_t channels, uint64_t samples) {
  // Aim for OXH_BN_RED_BLOCKS_PER_CU blocks per CU in total, but keep >= 4096 values per
  // block and at most kMaxSlices partials per channel.
  uint64_t target =
      (static_cast<uint64_t>(OXH_BN_RED_BLOCKS_PER_CU) * oxh::kComputeUnits + channels - 1) /
      channels;
  uint64_t max_by_work = samples / 4096;
  if (max_by_work < 1) max_by_work = 1;
  uint64_t s = target < max_by_work ? target : max_by_work;
  if (s > kMaxSlices) s = kMaxSlices;
  if (s < 1) s = 1;
  return static_cast<uint32_t>(s);
}

// The slicing depends only on the shape (never on alignment), so the reduce and map kernels of
// one operation always agree on S.
Geometry make_geometry(uint64_t batch, uint64_t channels, uint64_t spatial, bool aligned) {
  Geometry g{};
  g.batch = static_cast<uint32_t>(batch);
  g.channels = static_cast<uint32_t>(channels);
  g.spatial = static_cast<uint32_t>(spatial);
  g.samples = batch * spatial;
  g.vec = aligned && spatial % 4 == 0;
  const uint32_t s = choose_slices(channels, g.samples);
  uint64_t len = (g.samples + s - 1) / s;
  len = (len + 3) / 4 * 4;
  g.slice_len = len;
  g.slices = static_cast<uint32_t>((g.samples + len - 1) / len);  // drop empty slices
  g.spatial_div = oxh::make_fastdiv(static_cast<uint32_t>(g.vec ? spatial / 4 : spatial));
  return g;
}

uint64_t workspace_bytes_for(const Geometry &g) {
  return (static_cast<uint64_t>(g.channels) * g.slices * 16 + 255) / 256 * 256;
}

// Map blocks: block b covers the flattened elements [b * E, (b + 1) * E) of the NCHW tensor,
// which touch at most kMaxPlanes (n, c) planes.  E = kMapElems, reduced for tiny planes.
struct PlaneMap {
  uint32_t channels, spatial;
  uint64_t total;        // batch * channels * spatial
  uint32_t block_elems;  // E (a multiple of 4 on the vector path)
  bool vec;
  oxh::FastDiv spatial_div;
  uint64_t blocks;
};

PlaneMap make_plane_map(uint64_t batch, uint64_t channels, uint64_t spatial, bool aligned) {
  PlaneMap m{};
  m.channels = static_cast<uint32_t>(channels);
  m.spatial = static_cast<uint32_t>(spatial);
  m.total = batch * channels * spatial;
  m.vec = aligned && spatial % 4 == 0;
  uint64_t e = kMapElems;
  const uint64_t cap = static_cast<uint64_t>(kMaxPlanes - 1) * spatial;  // <= kMaxPlanes planes
  if (e > cap) e = cap;
  if (m.vec) e = e / 4 * 4;  // spatial % 4 == 0 keeps cap >= 4
  m.block_elems = static_cast<uint32_t>(e);
  m.blocks = (m.total + e - 1) / e;
  m.spatial_div = oxh::make_fastdiv(m.spatial);
  return m;
}

// Block-wide sum of two doubles; the result is valid in thread 0.
__device__ __forceinline__ void block_sum2(double &a, double &b, double (*lds)[kRedWaves]) {
  oxh::wave_sum2(a, b);
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

// Address (in floats or float4) of channel-relative value j of channel c.
__device__ __forceinline__ uint64_t nchw_index(const Geometry &g, uint32_t c, uint32_t j) {
  const uint32_t n = oxh::fast_div(j, g.spatial_div);
  const uint32_t i = j - n * g.spatial_div.d;
  return (static_cast<uint64_t>(n) * g.channels + c) * g.spatial_div.d + i;
}

// ---------------------------------------------------------------- reductions

// Forward partials: (sum (x - K), sum (x - K)^2), K = x[0, c, 0].
__global__ __launch_bounds__(kRedBlock) void bn_reduce_x_kernel(Geometry g,
                                                                const float *__restrict__ x,
                                                                double2 *__restrict__ partial) {
  __shared__ double lds[2][kRedWaves];
  const uint32_t s = blockIdx.x, c = blockIdx.y;
  const double k = static_cast<double>(x[static_cast<uint64_t>(c) * g.spatial]);
  double sum = 0.0, sq = 0.0;
  const uint64_t begin = static_cast<uint64_t>(s) * g.slice_len;
  const uint64_t end = begin + g.slice_len < g.samples ? begin + g.slice_len : g.samples;
  if (g.vec) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const uint32_t e4 = static_cast<uint32_t>(end / 4);
    uint32_t j = static_cast<uint32_t>(begin / 4) + threadIdx.x;
    auto add4 = [&](const float4 &v) {
      const double d0 = static_cast<double>(v.x) - k, d1 = static_cast<double>(v.y) - k;
      const double d2 = static_cast<double>(v.z) - k, d3 = static_cast<double>(v.w) - k;
      sum += (d0 + d1) + (d2 + d3);
      sq += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
    };
    for (; j + (kRedUnroll - 1) * kRedBlock < e4; j += kRedUnroll * kRedBlock) {
      float4 v[kRedUnroll];
#pragma unroll
      for (int u = 0; u < kRedUnroll; ++u) v[u] = x4[nchw_index(g, c, j + u * kRedBlock)];
#pragma unroll
      for (int u = 0; u < kRedUnroll; ++u) add4(v[u]);
    }
    for (; j < e4; j += kRedBlock) add4(x4[nchw_index(g, c, j)]);
  } else {
    for (uint64_t j = begin + threadIdx.x; j < end; j += kRedBlock) {
      const double d = static_cast<double>(x[nchw_index(g, c, static_cast<uint32_t>(j))]) - k;
      sum += d;
      sq += d * d;
    }
  }
  block_sum2(sum, sq, lds);
  if (threadIdx.x == 0) partial[static_cast<uint64_t>(c) * g.slices + s] = make_double2(sum, sq);
}

// Backward partials: (sum g, sum g * x_hat) with x_hat = (x - mean) * inv in fp32 and the
// product g * x_hat rounded to fp32 as the CPU path forms it (autograd.rs:353-362).  With
// Relu, g is first masked by the following ReLU's output (relu_out).
template <bool Relu>
__global__ __launch_bounds__(kRedBlock) void bn_reduce_gx_kernel(
    Geometry g, const float *__restrict__ grad, const float *__restrict__ relu_out,
    const float *__restrict__ x, const float *__restrict__ mean,
    const float *__restrict__ inverse_std, double2 *__restrict__ partial) {
  __shared__ double lds[2][kRedWaves];
  const uint32_t s = blockIdx.x, c = blockIdx.y;
  const float mu = mean[c], inv = inverse_std[c];
  double sg = 0.0, sgx = 0.0;
  const uint64_t begin = static_cast<uint64_t>(s) * g.slice_len;
  const uint64_t end = begin + g.slice_len < g.samples ? begin + g.slice_len : g.samples;
  if (g.vec) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const float4 *g4 = reinterpret_cast<const float4 *>(grad);
    const float4 *r4 = reinterpret_cast<const float4 *>(relu_out);
    const uint32_t e4 = static_cast<uint32_t>(end / 4);
    uint32_t j = static_cast<uint32_t>(begin / 4) + threadIdx.x;
    auto load_g = [&](uint64_t idx) {
      float4 v = g4[idx];
      if constexpr (Relu) {
        const float4 r = r4[idx];
        v = make_float4(relu_masked(v.x, r.x), relu_masked(v.y, r.y), relu_masked(v.z, r.z),
                        relu_masked(v.w, r.w));
      }
      return v;
    };
    auto add4 = [&](const float4 &xv, const float4 &gv) {
      const float n0 = (xv.x - mu) * inv, n1 = (xv.y - mu) * inv;
      const float n2 = (xv.z - mu) * inv, n3 = (xv.w - mu) * inv;
      sg += (static_cast<double>(gv.x) + static_cast<double>(gv.y)) +
            (static_cast<double>(gv.z) + static_cast<double>(gv.w));
      sgx += (static_cast<double>(gv.x * n0) + static_cast<double>(gv.y * n1)) +
             (static_cast<double>(gv.z * n2) + static_cast<double>(gv.w * n3));
    };
    for (; j + (kRedUnroll - 1) * kRedBlock < e4; j += kRedUnroll * kRedBlock) {
      float4 xv[kRedUnroll], gv[kRedUnroll];
#pragma unroll
      for (int u = 0; u < kRedUnroll; ++u) {
        const uint64_t idx = nchw_index(g, c, j + u * kRedBlock);
        xv[u] = x4[idx];
        gv[u] = load_g(idx);
      }
#pragma unroll
      for (int u = 0; u < kRedUnroll; ++u) add4(xv[u], gv[u]);
    }
    for (; j < e4; j += kRedBlock) {
      const uint64_t idx = nchw_index(g, c, j);
      add4(x4[idx], load_g(idx));
    }
  } else {
    for (uint64_t j = begin + threadIdx.x; j < end; j += kRedBlock) {
      const uint64_t idx = nchw_index(g, c, static_cast<uint32_t>(j));
      float gv = grad[idx];
      if constexpr (Relu) gv = relu_masked(gv, relu_out[idx]);
      const float nv = (x[idx] - mu) * inv;
      sg += static_cast<double>(gv);
      sgx += static_cast<double>(gv * nv);
    }
  }
  block_sum2(sg, sgx, lds);
  if (threadIdx.x == 0) partial[static_cast<uint64_t>(c) * g.slices + s] = make_double2(sg, sgx);
}

// ---------------------------------------------------------------- finalization

__device__ __forceinline__ bool lane0() { return threadIdx.x % 64 == 0; }

// Per-lane share of a channel's partials: lane l holds partial l (S <= kMaxSlices = 64, so one
// load per lane); loading only -- the sums are formed later, after the block's data loads have
// been issued, so the two load latencies overlap.
__device__ __forceinline__ double2 load_lane_partial(const double2 *partial, uint32_t slices,
                                                     uint32_t c) {
  const uint32_t lane = threadIdx.x % 64;
  return lane < slices ? partial[static_cast<uint64_t>(c) * slices + lane]
                       : make_double2(0.0, 0.0);
}

// Fixed-order sums over the wave, the same in every lane (bit-identical in all blocks and in
// the finalize kernels, which use the same reduction).
__device__ __forceinline__ double2 wave_sums_lane0(double2 v) {
  double a = v.x, b = v.y;
  oxh::wave_sum2(a, b);
  return make_double2(a, b);
}

// One wave per channel: the reference's separate statistics output (no consumer kernel).
__global__ __launch_bounds__(256) void bn_finalize_forward_kernel(
    Geometry g, const float *__restrict__ x, const double2 *__restrict__ partial, StatsOut out) {
  const uint32_t c = blockIdx.x * 4 + threadIdx.x / 64;
  if (c >= g.channels) return;
  const float shift = x[static_cast<uint64_t>(c) * g.spatial];
  const Moments r = forward_moments(wave_sums_lane0(load_lane_partial(partial, g.slices, c)),
                                    shift, g.samples, out.epsilon);
  if (lane0()) write_forward_outputs(out, c, r);
}

__global__ __launch_bounds__(256) void bn_finalize_affine_kernel(
    Geometry g, const double2 *__restrict__ partial, float *weight_gradient,
    float *bias_gradient) {
  const uint32_t c = blockIdx.x * 4 + threadIdx.x / 64;
  if (c >= g.channels) return;
  const double2 sums = wave_sums_lane0(load_lane_partial(partial, g.slices, c));
  if (lane0()) {
    weight_gradient[c] = static_cast<float>(sums.y);
    bias_gradient[c] = static_cast<float>(sums.x);
  }
}

// ---------------------------------------------------------------- map passes

// Per-plane channel values cached in LDS (V floats per plane).
template <int V>
struct Cache {
  float v[V][kMaxPlanes];
};

// Map phases.  load() (all lanes of a wave, for channel c) only issues the channel's loads;
// finish() forms the channel values and lane 0 stores them in the LDS cache and, in the block
// holding the first element of plane (0, c), the per-channel outputs.

// Forward apply.  Channel values: mean, inv, w, b.  Statistics come from the partials
// (finalize + apply) or from mean / inverse_std arrays (the reference's separate apply).
struct ApplyPhase {
  static constexpr int V = 4, NI = 1, kNtStoreBit = 1;
  struct Args {
    const float *x, *weight, *bias;
    const float *mean, *inverse_std;  // used when partial == null
    const double2 *partial;
    uint32_t slices;
    uint64_t samples;
    StatsOut out;  // written by the designated block when partial != null
    float *y;
    bool relu;     // y = relu(batch norm) (ConvNormAct, nn.rs:376-385)
  };
  struct Pre {
    double2 part;
    float shift, mu, inv, w, b;
  };
  __device__ static Pre load(const Args &a, const PlaneMap &m, uint32_t c) {
    Pre p;
    if (a.partial) {
      p.part = load_lane_partial(a.partial, a.slices, c);
      p.shift = a.x[static_cast<uint64_t>(c) * m.spatial];
    } else {
      p.mu = a.mean[c];
      p.inv = a.inverse_std[c];
    }
    p.w = a.weight[c];
    p.b = a.bias[c];
    return p;
  }
  __device__ static void finish(const Args &a, uint32_t c, const Pre &p, bool designated,
                                Cache<V> &cache, uint32_t k) {
    float mu = p.mu, inv = p.inv;
    if (a.partial) {
      const Moments r = forward_moments(wave_sums_lane0(p.part), p.shift, a.samples,
                                        a.out.epsilon);
      if (designated && lane0()) write_forward_outputs(a.out, c, r);
      mu = r.mean;
      inv = r.inv;
    }
    if (lane0()) {
      cache.v[0][k] = mu;
      cache.v[1][k] = inv;
      cache.v[2][k] = p.w;
      cache.v[3][k] = p.b;
    }
  }
  // Channel values read from the per-channel arrays (partial == null).
  __device__ static void direct(const Args &a, uint32_t c, float (&cv)[V]) {
    cv[0] = a.mean[c];
    cv[1] = a.inverse_std[c];
    cv[2] = a.weight[c];
    cv[3] = a.bias[c];
  }
  __device__ static const float *input(const Args &a, int) { return a.x; }
  __device__ static float *output(const Args &a) { return a.y; }
  __device__ static float element(const Args &a, const float (&cv)[V], const float (&in)[NI]) {
    // evaluation.rs:590-595, then kernel_module.rs:26-34 (x > 0 ? x : 0)
    const float y = (in[0] - cv[0]) * cv[1] * cv[2] + cv[3];
    return a.relu ? (y > 0.0f ? y : 0.0f) : y;
  }
};

// Training input backward.  Channel values: mean, inv, (w * inv) / M, sum g, sum g * x_hat.
// With Relu the incoming gradient is masked by the following ReLU's output (in[2]).
template <bool Relu>
struct DxTrainPhaseT {
  static constexpr int V = 5, NI = Relu ? 3 : 2, kNtStoreBit = 2;  // in: g, x, relu output
  struct Args {
    const float *grad, *x, *weight, *mean, *inverse_std;
    const float *weight_gradient, *bias_gradient;  // used when partial == null
    const double2 *partial;
    uint32_t slices;
    float samples;                                   // M in fp32 (autograd.rs:344-345)
    float *out_weight_gradient, *out_bias_gradient;  // written when partial != null
    float *dx;
    const float *relu_out;                           // read when Relu
  };
  struct Pre {
    double2 part;
    float sg, sgx, mu, inv, w;
  };
  __device__ static Pre load(const Args &a, const PlaneMap &, uint32_t c) {
    Pre p;
    if (a.partial) {
      p.part = load_lane_partial(a.partial, a.slices, c);
    } else {
      p.sg = a.bias_gradient[c];
      p.sgx = a.weight_gradient[c];
    }
    p.mu = a.mean[c];
    p.inv = a.inverse_std[c];
    p.w = a.weight[c];
    return p;
  }
  __device__ static void finish(const Args &a, uint32_t c, const Pre &p, bool designated,
                                Cache<V> &cache, uint32_t k) {
    float sg = p.sg, sgx = p.sgx;
    if (a.partial) {
      const double2 sums = wave_sums_lane0(p.part);
      sg = static_cast<float>(sums.x);
      sgx = static_cast<float>(sums.y);
      if (designated && lane0()) {
        a.out_weight_gradient[c] = sgx;
        a.out_bias_gradient[c] = sg;
      }
    }
    if (lane0()) {
      cache.v[0][k] = p.mu;
      cache.v[1][k] = p.inv;
      cache.v[2][k] = p.w * p.inv / a.samples;
      cache.v[3][k] = sg;
      cache.v[4][k] = sgx;
    }
  }
  __device__ static void direct(const Args &a, uint32_t c, float (&cv)[V]) {
    cv[0] = a.mean[c];
    cv[1] = a.inverse_std[c];
    cv[2] = a.weight[c] * cv[1] / a.samples;
    cv[3] = a.bias_gradient[c];
    cv[4] = a.weight_gradient[c];
  }
  __device__ static const float *input(const Args &a, int i) {
    return i == 0 ? a.grad : (i == 1 ? a.x : a.relu_out);
  }
  __device__ static float *output(const Args &a) { return a.dx; }
  __device__ static float element(const Args &a, const float (&cv)[V], const float (&in)[NI]) {
    // autograd.rs:367-373
    float g = in[0];
    if constexpr (Relu) g = relu_masked(g, in[NI - 1]);
    const float normalized = (in[1] - cv[0]) * cv[1];
    return cv[2] * (a.samples * g - cv[3] - normalized * cv[4]);
  }
};
using DxTrainPhase = DxTrainPhaseT<false>;

// Eval input backward: dx = (g * w) * inv (autograd.rs:374-378).
struct DxEvalPhase {
  static constexpr int V = 2, NI = 1, kNtStoreBit = 2;
  struct Args {
    const float *grad, *weight, *inverse_std;
    float *dx;
  };
  struct Pre {
    float w, inv;
  };
  __device__ static Pre load(const Args &a, const PlaneMap &, uint32_t c) {
    return Pre{a.weight[c], a.inverse_std[c]};
  }
  __device__ static void finish(const Args &, uint32_t, const Pre &p, bool, Cache<V> &cache,
                                uint32_t k) {
    if (lane0()) {
      cache.v[0][k] = p.w;
      cache.v[1][k] = p.inv;
    }
  }
  __device__ static void direct(const Args &a, uint32_t c, float (&cv)[V]) {
    cv[0] = a.weight[c];
    cv[1] = a.inverse_std[c];
  }
  __device__ static const float *input(const Args &a, int) { return a.grad; }
  __device__ static float *output(const Args &a) { return a.dx; }
  __device__ static float element(const Args &, const float (&cv)[V], const float (&in)[NI]) {
    return in[0] * cv[0] * cv[1];
  }
};

// Channel finalize for planes k = wave, wave + 4, ... of the block (wave-uniform loop).  The
// first plane's loads may already be in flight (pre / have_pre).
template <class P>
__device__ __forceinline__ void finish_planes(const PlaneMap &m, const typename P::Args &a,
                                              uint64_t plane0, uint32_t r0, uint32_t nplanes,
                                              const typename P::Pre &pre, bool have_pre,
                                              Cache<P::V> &cache) {
  for (uint32_t k = threadIdx.x / 64; k < nplanes; k += kMapBlock / 64) {
    const uint64_t plane = plane0 + k;
    const uint32_t c = static_cast<uint32_t>(plane % m.channels);
    const bool designated = plane < m.channels && (k > 0 || r0 == 0);
    const bool first = k == threadIdx.x / 64;
    P::finish(a, c, first && have_pre ? pre : P::load(a, m, c), designated, cache, k);
  }
}

template <class P>
__global__ __launch_bounds__(kMapBlock) void bn_map_kernel(PlaneMap m, typename P::Args a) {
  __shared__ Cache<P::V> cache;
  const uint64_t e0 = static_cast<uint64_t>(blockIdx.x) * m.block_elems;
  const uint64_t e1 = e0 + m.block_elems < m.total ? e0 + m.block_elems : m.total;
  const uint64_t plane0 = e0 / m.spatial;
  const uint32_t r0 = static_cast<uint32_t>(e0 - plane0 * m.spatial);  // offset in plane0
  const uint32_t nplanes = static_cast<uint32_t>((e1 - 1) / m.spatial - plane0 + 1);
  const uint32_t n = static_cast<uint32_t>(e1 - e0);
  float *out = P::output(a);
  // 1) the channel loads of this wave's first plane, 2) the block's data loads, 3) the channel
  // finalize (its loads return first), 4) the elementwise pass.
  const uint32_t wave = threadIdx.x / 64;
  typename P::Pre pre{};
  const bool have_pre = wave < nplanes;
  if (have_pre) pre = P::load(a, m, static_cast<uint32_t>((plane0 + wave) % m.channels));
  if (m.vec) {
    // e0 and r0 are multiples of 4 (spatial % 4 == 0, block_elems % 4 == 0).
    const uint32_t n4 = n / 4;
    float4 v[kMapVec][P::NI];
#pragma unroll
    for (int u = 0; u < kMapVec; ++u) {
      const uint32_t q = threadIdx.x + u * kMapBlock;
      if (q < n4) {
#pragma unroll
        for (int i = 0; i < P::NI; ++i)
          v[u][i] = reinterpret_cast<const float4 *>(P::input(a, i) + e0)[q];
      }
    }
    finish_planes<P>(m, a, plane0, r0, nplanes, pre, have_pre, cache);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kMapVec; ++u) {
      const uint32_t q = threadIdx.x + u * kMapBlock;
      if (q < n4) {
        const uint32_t k = oxh::fast_div(r0 + q * 4, m.spatial_div);
        float cv[P::V];
#pragma unroll
        for (int j = 0; j < P::V; ++j) cv[j] = cache.v[j][k];
        float x0[P::NI], x1[P::NI], x2[P::NI], x3[P::NI];
#pragma unroll
        for (int i = 0; i < P::NI; ++i) {
          x0[i] = v[u][i].x;
          x1[i] = v[u][i].y;
          x2[i] = v[u][i].z;
          x3[i] = v[u][i].w;
        }
        float4 r;
        r.x = P::element(a, cv, x0);
        r.y = P::element(a, cv, x1);
        r.z = P::element(a, cv, x2);
        r.w = P::element(a, cv, x3);
        if constexpr ((OXH_BN_NT_STORE & P::kNtStoreBit) != 0) {
          // non-temporal, system scope (buffer cache policy nt | sc1): the apply's y and the
          // input backward's dx are not read again in the step; 0.1290 -> 0.1279 ms per
          // headline step against nt alone (sc0 | sc1 without nt: 0.137 ms)
          const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
              out + e0, 0, static_cast<int>(n4 * 16), 0x00020000);
          typedef unsigned u32x4_t __attribute__((vector_size(16)));
          const u32x4_t bits = {__float_as_uint(r.x), __float_as_uint(r.y), __float_as_uint(r.z),
                                __float_as_uint(r.w)};
          __builtin_amdgcn_raw_buffer_store_b128(bits, rs, q * 16, 0, kStorePolicy);
        } else {
          reinterpret_cast<float4 *>(out + e0)[q] = r;
        }
      }
    }
  } else {
    finish_planes<P>(m, a, plane0, r0, nplanes, pre, have_pre, cache);
    __syncthreads();
    for (uint32_t q = threadIdx.x; q < n; q += kMapBlock) {
      const uint32_t k = oxh::fast_div(r0 + q, m.spatial_div);
      float cv[P::V];
#pragma unroll
      for (int j = 0; j < P::V; ++j) cv[j] = cache.v[j][k];
      float x[P::NI];
#pragma unroll
      for (int i = 0; i < P::NI; ++i) x[i] = P::input(a, i)[e0 + q];
      out[e0 + q] = P::element(a, cv, x);
    }
  }
}

// Small planes: a map block of kMapElems elements would span hundreds of (n, c) planes and
// finalize each of them, so for spatial < kFlatSpatial the statistics are finalized once per
// channel by the finalize kernels above (into the per-channel output arrays), and this flat pass
// reads each element's channel values from those arrays (cached: C * V floats).
struct FlatMap {
  uint32_t channels;
  uint32_t units;  // float4 units (vec) or elements
  bool vec;        // spatial % 4 == 0 and pointers aligned: a float4 lies in one plane
  oxh::FastDiv spatial_div, channel_div;
};

template <class P>
__global__ __launch_bounds__(kMapBlock) void bn_flat_map_kernel(FlatMap m, typename P::Args a) {
  float *out = P::output(a);
  const uint32_t stride = gridDim.x * kMapBlock;
  for (uint32_t q = blockIdx.x * kMapBlock + threadIdx.x; q < m.units; q += stride) {
    const uint32_t e = m.vec ? q * 4 : q;  // < 2^31 (checked on the host)
    const uint32_t plane = oxh::fast_div(e, m.spatial_div);
    const uint32_t c = plane - oxh::fast_div(plane, m.channel_div) * m.channels;
    float cv[P::V];
    P::direct(a, c, cv);
    if (m.vec) {
      float4 v[P::NI];
#pragma unroll
      for (int i = 0; i < P::NI; ++i) v[i] = reinterpret_cast<const float4 *>(P::input(a, i))[q];
      float x0[P::NI], x1[P::NI], x2[P::NI], x3[P::NI];
#pragma unroll
      for (int i = 0; i < P::NI; ++i) {
        x0[i] = v[i].x;
        x1[i] = v[i].y;
        x2[i] = v[i].z;
        x3[i] = v[i].w;
      }
      float4 r;
      r.x = P::element(a, cv, x0);
      r.y = P::element(a, cv, x1);
      r.z = P::element(a, cv, x2);
      r.w = P::element(a, cv, x3);
      reinterpret_cast<float4 *>(out)[q] = r;
    } else {
      float x[P::NI];
#pragma unroll
      for (int i = 0; i < P::NI; ++i) x[i] = P::input(a, i)[q];
      out[q] = P::element(a, cv, x);
    }
  }
}

// Small planes with few values per channel: one block per channel performs the whole
// operation -- the channel sums, their finalization, and the elementwise pass (whose second
// read of the channel is served by L2) -- in a single launch.
constexpr uint64_t kChannelMaxSamples = 65536;

// Blocks have 256 threads, or 1024 when there are few channels (a block per channel would
// leave most CUs idle) and more values than 256 threads keep.
int channel_threads(const ChannelGeom &g) {
  return g.channels <= 128 && g.samples > 256 * kChannelKeep ? 1024 : 256;
}

// addend (may be null; never with Relu): y = BN(x) + addend, the residual add that follows a
// block's last BatchNorm, in the same pass.
template <bool Relu, bool Keep, int Threads>
__global__ __launch_bounds__(Threads) void bn_channel_forward_kernel(
    ChannelGeom g, const float *__restrict__ x, const float *__restrict__ weight,
    const float *__restrict__ bias, StatsOut out, const float *__restrict__ addend,
    float *__restrict__ y) {
  __shared__ double lds[2][Threads / 64];
  const uint32_t c = blockIdx.x;
  const float shift = x[static_cast<uint64_t>(c) * g.spatial];  // x[0, c, 0]
  const RunningPrev prev = load_running(out, c);
  if constexpr (Keep) {
    float kept[kChannelKeep], added[kChannelKeep];
    uint32_t at[kChannelKeep];
#pragma unroll
    for (int u = 0; u < kChannelKeep; ++u) {
      const uint32_t j = threadIdx.x + u * Threads;
      at[u] = j < g.samples ? channel_index(g, c, j) : 0;
      kept[u] = x[at[u]];
    }
    if (addend != nullptr) {
#pragma unroll
      for (int u = 0; u < kChannelKeep; ++u) added[u] = addend[at[u]];
    }
    channel_forward_kept<Relu, Threads>(g.samples, c, shift, kept, at, weight[c], bias[c], out,
                                        prev, addend != nullptr, added, y, lds);
  } else {
    const double k = static_cast<double>(shift);
    double sum = 0.0, sq = 0.0;
    for (uint32_t j = threadIdx.x; j < g.samples; j += Threads) {
      const double d = static_cast<double>(x[channel_index(g, c, j)]) - k;
      sum += d;
      sq += d * d;
    }
    block_sum2_all<Threads / 64>(sum, sq, lds);
    const Moments r = forward_moments(make_double2(sum, sq), shift, g.samples, out.epsilon);
    if (threadIdx.x == 0) write_forward_outputs(out, c, r, prev);
    const float mu = r.mean, inv = r.inv, w = weight[c], b = bias[c];
    for (uint32_t j = threadIdx.x; j < g.samples; j += Threads) {
      const uint32_t idx = channel_index(g, c, j);
      float v = (x[idx] - mu) * inv * w + b;  // evaluation.rs:590-595
      if constexpr (Relu) v = v > 0.0f ? v : 0.0f;
      y[idx] = addend != nullptr ? v + addend[idx] : v;
    }
  }
}

// With DxSum, the block also sums the dx it writes (fp64, fixed order) into dx_sum[c]: the
// bias gradient of a convolution whose output is this BatchNorm's input (autograd.rs:412-527
// reduces the same values over (n, y, x) in a pass of its own).
template <bool Relu, bool DxSum, bool Keep, int Threads>
__global__ __launch_bounds__(Threads) void bn_channel_backward_kernel(
    ChannelGeom g, const float *__restrict__ grad, const float *__restrict__ relu_out,
    const float *__restrict__ x, const float *__restrict__ weight, const float *__restrict__ mean,
    const float *__restrict__ inverse_std, float *__restrict__ dx, float *__restrict__ dweight,
    float *__restrict__ dbias, float *__restrict__ dx_sum) {
  __shared__ double lds[2][2][Threads / 64];  // one region per block sum
  const uint32_t c = blockIdx.x;
  const float mu = mean[c], inv = inverse_std[c];
  double total = 0.0, unused = 0.0;
  if constexpr (Keep) {
    float kg[kChannelKeep], kn[kChannelKeep], d[kChannelKeep];
    uint32_t at[kChannelKeep];
#pragma unroll
    for (int u = 0; u < kChannelKeep; ++u) {
      const uint32_t j = threadIdx.x + u * Threads;
      at[u] = j < g.samples ? channel_index(g, c, j) : 0;
      float gv = grad[at[u]];
      if constexpr (Relu) gv = relu_masked(gv, relu_out[at[u]]);
      kg[u] = gv;
      kn[u] = (x[at[u]] - mu) * inv;
    }
    channel_backward_kept<Threads>(g.samples, kg, kn, weight[c], inv, dweight + c, dbias + c, d,
                                   lds[0]);
#pragma unroll
    for (int u = 0; u < kChannelKeep; ++u) {
      if (threadIdx.x + u * Threads >= g.samples) break;
      dx[at[u]] = d[u];
      if constexpr (DxSum) total += static_cast<double>(d[u]);
    }
  } else {
    double sg = 0.0, sgx = 0.0;
    for (uint32_t j = threadIdx.x; j < g.samples; j += Threads) {
      const uint32_t idx = channel_index(g, c, j);
      float gv = grad[idx];
      if constexpr (Relu) gv = relu_masked(gv, relu_out[idx]);
      const float nv = (x[idx] - mu) * inv;
      sg += static_cast<double>(gv);
      sgx += static_cast<double>(gv * nv);
    }
    block_sum2_all<Threads / 64>(sg, sgx, lds[0]);
    const float sgf = static_cast<float>(sg), sgxf = static_cast<float>(sgx);
    if (threadIdx.x == 0) {
      dbias[c] = sgf;
      dweight[c] = sgxf;
    }
    // autograd.rs:344-373: ((w * inv) / M) * ((M * g - sum_g) - x_hat * sum_g_xhat)
    const float samples = static_cast<float>(g.samples);
    const float coef = weight[c] * inv / samples;
    for (uint32_t j = threadIdx.x; j < g.samples; j += Threads) {
      const uint32_t idx = channel_index(g, c, j);
      float gv = grad[idx];
      if constexpr (Relu) gv = relu_masked(gv, relu_out[idx]);
      const float normalized = (x[idx] - mu) * inv;
      const float d = coef * (samples * gv - sgf - normalized * sgxf);
      dx[idx] = d;
      if constexpr (DxSum) total += static_cast<double>(d);
    }
  }
  if constexpr (DxSum) {
    block_sum2_all<Threads / 64>(total, unused, lds[1]);
    if (threadIdx.x == 0) dx_sum[c] = static_cast<float>(total);
  }
}

// Per-channel sum of an NCHW tensor (fp64, fixed order) for the planes the
// one-block-per-channel backward does not take: partial sums over the reduce slices, then one
// thread per channel adds them in slice order.
__global__ __launch_bounds__(kRedBlock) void bn_sum_partial_kernel(Geometry g,
                                                                   const float *__restrict__ v,
                                                                   double *__restrict__ partial) {
  __shared__ double lds[2][kRedWaves];
  const uint32_t s = blockIdx.x, c = blockIdx.y;
  double total = 0.0, unused = 0.0;
  const uint64_t begin = static_cast<uint64_t>(s) * g.slice_len;
  const uint64_t end = begin + g.slice_len < g.samples ? begin + g.slice_len : g.samples;
  if (g.vec) {
    const float4 *v4 = reinterpret_cast<const float4 *>(v);
    const uint32_t e4 = static_cast<uint32_t>(end / 4);
    for (uint32_t j = static_cast<uint32_t>(begin / 4) + threadIdx.x; j < e4; j += kRedBlock) {
      const float4 q = v4[nchw_index(g, c, j)];
      total += (static_cast<double>(q.x) + static_cast<double>(q.y)) +
               (static_cast<double>(q.z) + static_cast<double>(q.w));
    }
  } else {
    for (uint64_t j = begin + threadIdx.x; j < end; j += kRedBlock)
      total += static_cast<double>(v[nchw_index(g, c, static_cast<uint32_t>(j))]);
  }
  block_sum2(total, unused, lds);
  if (threadIdx.x == 0) partial[static_cast<uint64_t>(c) * g.slices + s] = total;
}

__global__ void bn_sum_finalize_kernel(uint32_t channels, uint32_t slices,
                                       const double *__restrict__ partial,
                                       float *__restrict__ out) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= channels) return;
  double total = 0.0;
  for (uint32_t s = 0; s < slices; ++s) total += partial[static_cast<uint64_t>(c) * slices + s];
  out[c] = static_cast<float>(total);
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
              OXH_INVALID_SHAPE,
              std::string(name) + ": dimension too large (channels <= 65535)");
  OXH_REQUIRE(batch * spatial < (1ull << 31), OXH_INVALID_SHAPE,
              std::string(name) + ": more than 2^31 values per channel");
  OXH_REQUIRE(batch * channels * spatial < (1ull << 40), OXH_INVALID_SHAPE,
              std::string(name) + ": tensor too large");
  const PlaneMap m = make_plane_map(batch, channels, spatial, false);
  OXH_REQUIRE(m.blocks < (1ull << 31), OXH_INVALID_SHAPE,
              std::string(name) + ": too many planes");
  return oxh::ok();
}

oxh_status check_workspace(const char *name, const Geometry &g, const void *workspace,
                           uint64_t bytes) {
  const uint64_t need = workspace_bytes_for(g);
  OXH_REQUIRE(workspace != nullptr && bytes >= need, OXH_INVALID_SHAPE,
              std::string(name) + ": workspace of " + std::to_string(need) +
                  " bytes required (oxh_batch_norm_workspace_size)");
  OXH_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15u) == 0, OXH_INVALID_SHAPE,
              std::string(name) + ": workspace must be 16-byte aligned");
  return oxh::ok();
}

oxh_status no_overlap(const char *name, const void *out, uint64_t out_bytes,
                      std::initializer_list<const void *> ins, uint64_t in_bytes) {
  for (const void *in : ins)
    if (in) OXH_REQUIRE(!oxh::any_overlap(out, out_bytes, in, in_bytes), OXH_INVALID_SHAPE,
                        std::string(name) + ": output overlaps an input");
  return oxh::ok();
}

oxh_status launch_reduce_x(const char *name, oxh_stream stream, uint64_t batch,
                           uint64_t channels, uint64_t spatial, const float *input,
                           void *workspace, uint64_t workspace_bytes, Geometry *geometry) {
  oxh_status st = check_shape(name, batch, channels, spatial);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(batch * spatial > 1, OXH_EXECUTION,
              "BatchNorm training requires more than one value per channel");
  OXH_REQUIRE(input != nullptr, OXH_INVALID_SHAPE, std::string(name) + ": null input");
  const Geometry g = make_geometry(batch, channels, spatial, oxh::aligned16(input));
  st = check_workspace(name, g, workspace, workspace_bytes);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(!oxh::any_overlap(workspace, workspace_bytes_for(g), input,
                                batch * channels * spatial * 4),
              OXH_INVALID_SHAPE, std::string(name) + ": workspace overlaps the input");
  oxh::launch(bn_reduce_x_kernel, dim3(g.slices, g.channels), dim3(kRedBlock), 0,
                     oxh::as_stream(stream), g, input, static_cast<double2 *>(workspace));
  if (geometry) *geometry = g;
  return oxh::launched(name);
}

oxh_status launch_reduce_gx(const char *name, oxh_stream stream, uint64_t batch,
                            uint64_t channels, uint64_t spatial, const float *gradient,
                            const float *relu_out, const float *input, const float *mean,
                            const float *inverse_std, void *workspace, uint64_t workspace_bytes,
                            Geometry *geometry) {
  oxh_status st = check_shape(name, batch, channels, spatial);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(gradient && input && mean && inverse_std, OXH_INVALID_SHAPE,
              std::string(name) + ": null pointer");
  const Geometry g = make_geometry(
      batch, channels, spatial,
      oxh::aligned16(input) && oxh::aligned16(gradient) && oxh::aligned16(relu_out));
  st = check_workspace(name, g, workspace, workspace_bytes);
  if (st != OXH_OK) return st;
  const dim3 grid(g.slices, g.channels);
  auto *partial = static_cast<double2 *>(workspace);
  if (relu_out)
    oxh::launch(bn_reduce_gx_kernel<true>, grid, dim3(kRedBlock), 0, oxh::as_stream(stream), g,
                gradient, relu_out, input, mean, inverse_std, partial);
  else
    oxh::launch(bn_reduce_gx_kernel<false>, grid, dim3(kRedBlock), 0, oxh::as_stream(stream), g,
                gradient, relu_out, input, mean, inverse_std, partial);
  if (geometry) *geometry = g;
  return oxh::launched(name);
}

bool a_is_direct(const ApplyPhase::Args &a) { return a.partial == nullptr; }
bool a_is_direct(const DxTrainPhaseT<false>::Args &a) { return a.partial == nullptr; }
bool a_is_direct(const DxTrainPhaseT<true>::Args &a) { return a.partial == nullptr; }
bool a_is_direct(const DxEvalPhase::Args &) { return true; }

// The flat pass serves planes smaller than kFlatSpatial values (tensors under 2^31 elements).
bool use_flat(uint64_t batch, uint64_t channels, uint64_t spatial) {
  return spatial < kFlatSpatial && batch * channels * spatial < (1ull << 31);
}

// Per-element pass.  With a.partial set, the block-finalizing map kernel is the only option
// (the flat pass reads finalized per-channel arrays; the entry points finalize first).
template <class P>
oxh_status launch_map(const char *name, oxh_stream stream, uint64_t batch, uint64_t channels,
                      uint64_t spatial, bool aligned, const typename P::Args &a) {
  if (a_is_direct(a) && use_flat(batch, channels, spatial)) {
    FlatMap f{};
    const uint64_t total = batch * channels * spatial;
    f.channels = static_cast<uint32_t>(channels);
    f.vec = aligned && spatial % 4 == 0;
    f.units = static_cast<uint32_t>(f.vec ? total / 4 : total);
    f.spatial_div = oxh::make_fastdiv(static_cast<uint32_t>(spatial));
    f.channel_div = oxh::make_fastdiv(static_cast<uint32_t>(channels));
    uint64_t blocks = (f.units + kMapBlock - 1) / kMapBlock;
    const uint64_t cap = 8ull * oxh::kComputeUnits;
    if (blocks > cap) blocks = cap;
    oxh::launch(bn_flat_map_kernel<P>, dim3(static_cast<uint32_t>(blocks)), dim3(kMapBlock), 0,
                oxh::as_stream(stream), f, a);
    return oxh::launched(name);
  }
  const PlaneMap m = make_plane_map(batch, channels, spatial, aligned);
  oxh::launch(bn_map_kernel<P>, dim3(static_cast<uint32_t>(m.blocks)), dim3(kMapBlock),
                     0, oxh::as_stream(stream), m, a);
  return oxh::launched(name);
}

uint32_t channel_grid(uint64_t channels) { return static_cast<uint32_t>((channels + 255) / 256); }

bool use_channel(uint64_t batch, uint64_t channels, uint64_t spatial) {
  return spatial < kFlatSpatial && batch * spatial <= kChannelMaxSamples &&
         batch * channels * spatial < (1ull << 31);
}

ChannelGeom make_channel_geom(uint64_t batch, uint64_t channels, uint64_t spatial) {
  ChannelGeom g{};
  g.channels = static_cast<uint32_t>(channels);
  g.spatial = static_cast<uint32_t>(spatial);
  g.samples = static_cast<uint32_t>(batch * spatial);
  g.spatial_div = oxh::make_fastdiv(g.spatial);
  return g;
}

// forward_apply after forward_reduce; relu: y = relu(batch norm).
oxh_status forward_apply_impl(const char *name, oxh_stream stream, uint64_t batch,
                              uint64_t channels, uint64_t spatial, float momentum,
                              float epsilon, const float *input, const float *weight,
                              const float *bias, float *running_mean, float *running_variance,
                              float *saved_mean, float *saved_inverse_std, float *output,
                              const void *workspace, uint64_t workspace_bytes, bool relu) {
  OXH_REQUIRE(std::isfinite(momentum) && std::isfinite(epsilon) && epsilon >= 0.0f,
              OXH_INVALID_SHAPE, std::string(name) + ": bad momentum or epsilon");
  oxh_status st = check_shape(name, batch, channels, spatial);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(batch * spatial > 1, OXH_EXECUTION,
              "BatchNorm training requires more than one value per channel");
  OXH_REQUIRE(input && weight && bias && running_mean && running_variance && saved_mean &&
                  saved_inverse_std && output,
              OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  const Geometry g = make_geometry(batch, channels, spatial, false);
  st = check_workspace(name, g, workspace, workspace_bytes);
  if (st != OXH_OK) return st;
  const uint64_t bytes = batch * channels * spatial * 4;
  st = no_overlap(name, output, bytes, {input}, bytes);
  if (st != OXH_OK) return st;
  const StatsOut stats{saved_mean, saved_inverse_std, nullptr, running_mean, running_variance,
                       momentum, epsilon};
  const bool aligned = oxh::aligned16(input) && oxh::aligned16(output);
  if (use_flat(batch, channels, spatial)) {
    oxh::launch(bn_finalize_forward_kernel, dim3((channels + 3) / 4), dim3(256), 0,
                oxh::as_stream(stream), g, input, static_cast<const double2 *>(workspace),
                stats);
    st = oxh::launched(name);
    if (st != OXH_OK) return st;
    ApplyPhase::Args a{input, weight, bias, saved_mean, saved_inverse_std, nullptr, 0, 0,
                       StatsOut{}, output, relu};
    return launch_map<ApplyPhase>(name, stream, batch, channels, spatial, aligned, a);
  }
  ApplyPhase::Args a{input,    weight,    bias,  nullptr, nullptr,
                     static_cast<const double2 *>(workspace), g.slices, g.samples, stats, output,
                     relu};
  return launch_map<ApplyPhase>(name, stream, batch, channels, spatial, aligned, a);
}

// backward_input after backward_reduce; relu_out (nullable): the following ReLU's output,
// whose sign masks the incoming gradient.
oxh_status backward_input_impl(const char *name, oxh_stream stream, uint64_t batch,
                               uint64_t channels, uint64_t spatial, const float *gradient,
                               const float *relu_out, const float *input, const float *weight,
                               const float *saved_mean, const float *saved_inverse_std,
                               float *input_gradient, float *weight_gradient,
                               float *bias_gradient, const void *workspace,
                               uint64_t workspace_bytes) {
  oxh_status st = check_shape(name, batch, channels, spatial);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(gradient && input && weight && saved_mean && saved_inverse_std &&
                  input_gradient && weight_gradient && bias_gradient,
              OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  const Geometry g = make_geometry(batch, channels, spatial, false);
  st = check_workspace(name, g, workspace, workspace_bytes);
  if (st != OXH_OK) return st;
  const uint64_t bytes = batch * channels * spatial * 4;
  st = no_overlap(name, input_gradient, bytes, {input, gradient, relu_out}, bytes);
  if (st != OXH_OK) return st;
  const bool aligned = oxh::aligned16(gradient) && oxh::aligned16(input) &&
                       oxh::aligned16(input_gradient) && oxh::aligned16(relu_out);
  const float samples = static_cast<float>(batch * spatial);
  const double2 *partial = static_cast<const double2 *>(workspace);
  const bool flat = use_flat(batch, channels, spatial);
  if (flat) {
    oxh::launch(bn_finalize_affine_kernel, dim3((channels + 3) / 4), dim3(256), 0,
                oxh::as_stream(stream), g, partial, weight_gradient, bias_gradient);
    st = oxh::launched(name);
    if (st != OXH_OK) return st;
  }
  const float *wg_in = flat ? weight_gradient : nullptr;
  const float *bg_in = flat ? bias_gradient : nullptr;
  const double2 *part = flat ? nullptr : partial;
  float *wg_out = flat ? nullptr : weight_gradient;
  float *bg_out = flat ? nullptr : bias_gradient;
  if (relu_out) {
    DxTrainPhaseT<true>::Args a{gradient, input,  weight, saved_mean, saved_inverse_std,
                                wg_in,    bg_in,  part,   g.slices,   samples,
                                wg_out,   bg_out, input_gradient, relu_out};
    return launch_map<DxTrainPhaseT<true>>(name, stream, batch, channels, spatial, aligned, a);
  }
  DxTrainPhase::Args a{gradient, input,  weight, saved_mean, saved_inverse_std,
                       wg_in,    bg_in,  part,   g.slices,   samples,
                       wg_out,   bg_out, input_gradient, nullptr};
  return launch_map<DxTrainPhase>(name, stream, batch, channels, spatial, aligned, a);
}

oxh_status forward_train_impl(const char *name, oxh_stream stream, uint64_t batch,
                              uint64_t channels, uint64_t spatial, float momentum,
                              float epsilon, const float *input, const float *weight,
                              const float *bias, float *running_mean, float *running_variance,
                              float *saved_mean, float *saved_inverse_std, float *output,
                              void *workspace, uint64_t workspace_bytes, bool relu,
                              const float *addend = nullptr) {
  if (!use_channel(batch, channels, spatial)) {
    oxh_status st = launch_reduce_x(name, stream, batch, channels, spatial, input, workspace,
                                    workspace_bytes, nullptr);
    if (st != OXH_OK) return st;
    st = forward_apply_impl(name, stream, batch, channels, spatial, momentum, epsilon, input,
                            weight, bias, running_mean, running_variance, saved_mean,
                            saved_inverse_std, output, workspace, workspace_bytes, relu);
    if (st != OXH_OK || addend == nullptr) return st;
    return oxh_add(stream, output, addend, output, batch * channels * spatial);
  }
  OXH_REQUIRE(std::isfinite(momentum) && std::isfinite(epsilon) && epsilon >= 0.0f,
              OXH_INVALID_SHAPE, std::string(name) + ": bad momentum or epsilon");
  oxh_status st = check_shape(name, batch, channels, spatial);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(batch * spatial > 1, OXH_EXECUTION,
              "BatchNorm training requires more than one value per channel");
  OXH_REQUIRE(input && weight && bias && running_mean && running_variance && saved_mean &&
                  saved_inverse_std && output,
              OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  st = check_workspace(name, make_geometry(batch, channels, spatial, false), workspace,
                       workspace_bytes);
  if (st != OXH_OK) return st;
  const uint64_t bytes = batch * channels * spatial * 4;
  st = no_overlap(name, output, bytes, {input}, bytes);
  if (st != OXH_OK) return st;
  const StatsOut stats{saved_mean, saved_inverse_std, nullptr, running_mean, running_variance,
                       momentum, epsilon};
  const ChannelGeom cg = make_channel_geom(batch, channels, spatial);
  const int threads = channel_threads(cg);
  const bool keep = cg.samples <= static_cast<uint32_t>(threads * kChannelKeep);
  using K = decltype(&bn_channel_forward_kernel<true, true, 256>);
  const K kernels[2][2][2] = {
      {{bn_channel_forward_kernel<false, false, 256>, bn_channel_forward_kernel<false, true, 256>},
       {bn_channel_forward_kernel<true, false, 256>, bn_channel_forward_kernel<true, true, 256>}},
      {{bn_channel_forward_kernel<false, false, 1024>,
        bn_channel_forward_kernel<false, true, 1024>},
       {bn_channel_forward_kernel<true, false, 1024>,
        bn_channel_forward_kernel<true, true, 1024>}}};
  oxh::launch(kernels[threads == 1024][relu][keep], dim3(cg.channels), dim3(threads), 0,
              oxh::as_stream(stream), cg, input, weight, bias, stats, addend, output);
  return oxh::launched(name);
}

oxh_status backward_train_impl(const char *name, oxh_stream stream, uint64_t batch,
                               uint64_t channels, uint64_t spatial, const float *gradient,
                               const float *relu_out, const float *input, const float *weight,
                               const float *saved_mean, const float *saved_inverse_std,
                               float *input_gradient, float *weight_gradient,
                               float *bias_gradient, float *input_gradient_sum, void *workspace,
                               uint64_t workspace_bytes) {
  if (!use_channel(batch, channels, spatial)) {
    oxh_status st = launch_reduce_gx(name, stream, batch, channels, spatial, gradient, relu_out,
                                     input, saved_mean, saved_inverse_std, workspace,
                                     workspace_bytes, nullptr);
    if (st != OXH_OK) return st;
    st = backward_input_impl(name, stream, batch, channels, spatial, gradient, relu_out, input,
                             weight, saved_mean, saved_inverse_std, input_gradient,
                             weight_gradient, bias_gradient, workspace, workspace_bytes);
    if (st != OXH_OK || input_gradient_sum == nullptr) return st;
    // the backward's partials are consumed (stream order): the workspace holds the dx sums'
    const Geometry g =
        make_geometry(batch, channels, spatial, oxh::aligned16(input_gradient));
    auto *partial = static_cast<double *>(workspace);
    oxh::launch(bn_sum_partial_kernel, dim3(g.slices, g.channels), dim3(kRedBlock), 0,
                oxh::as_stream(stream), g, static_cast<const float *>(input_gradient), partial);
    st = oxh::launched(name);
    if (st != OXH_OK) return st;
    oxh::launch(bn_sum_finalize_kernel, dim3((g.channels + 255) / 256), dim3(256), 0,
                oxh::as_stream(stream), g.channels, g.slices,
                static_cast<const double *>(partial), input_gradient_sum);
    return oxh::launched(name);
  }
  oxh_status st = check_shape(name, batch, channels, spatial);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(gradient && input && weight && saved_mean && saved_inverse_std &&
                  input_gradient && weight_gradient && bias_gradient,
              OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  st = check_workspace(name, make_geometry(batch, channels, spatial, false), workspace,
                       workspace_bytes);
  if (st != OXH_OK) return st;
  const uint64_t bytes = batch * channels * spatial * 4;
  st = no_overlap(name, input_gradient, bytes, {input, gradient, relu_out}, bytes);
  if (st != OXH_OK) return st;
  const ChannelGeom cg = make_channel_geom(batch, channels, spatial);
  const int threads = channel_threads(cg);
  const bool keep = cg.samples <= static_cast<uint32_t>(threads * kChannelKeep);
  using K = decltype(&bn_channel_backward_kernel<true, true, true, 256>);
#define OXH_BN_BWD(T)                                                                      \
  {{{bn_channel_backward_kernel<false, false, false, T>,                                   \
     bn_channel_backward_kernel<false, false, true, T>},                                   \
    {bn_channel_backward_kernel<false, true, false, T>,                                    \
     bn_channel_backward_kernel<false, true, true, T>}},                                   \
   {{bn_channel_backward_kernel<true, false, false, T>,                                    \
     bn_channel_backward_kernel<true, false, true, T>},                                    \
    {bn_channel_backward_kernel<true, true, false, T>,                                     \
     bn_channel_backward_kernel<true, true, true, T>}}}
  const K kernels[2][2][2][2] = {OXH_BN_BWD(256), OXH_BN_BWD(1024)};
#undef OXH_BN_BWD
  const K kernel =
      kernels[threads == 1024][relu_out != nullptr][input_gradient_sum != nullptr][keep];
  oxh::launch(kernel, dim3(cg.channels), dim3(threads), 0, oxh::as_stream(stream), cg,
              gradient, relu_out, input, weight, saved_mean, saved_inverse_std, input_gradient,
              weight_gradient, bias_gradient, input_gradient_sum);
  return oxh::launched(name);
}

}  // namespace

bool oxh::batch_norm_single_launch(uint64_t batch, uint64_t channels, uint64_t spatial) {
  return use_channel(batch, channels, spatial);
}

namespace {

// ---------------------------------------------------------------- allocation-free forward

// The reduce partials of oxh_batch_norm_forward_train_no_alloc live in this array: one copy per
// GPU (each device loads its own copy of the code object), held until the process ends.  Host
// code never passes the array's name to a kernel (on the host it is only a stand-in symbol):
// the device address of each GPU's copy is looked up once per device and used instead.
}  // namespace

static __device__ __align__(256) unsigned char scratch[OXH_BN_NO_ALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex scratch_mutex;
void *scratch_address[kMaxScratchDevices] = {};

// Resolves (once) the device address of `device`'s copy of `scratch`; `device` is current.
oxh_status resolve_scratch(int device, void **address) {
  OXH_REQUIRE(device >= 0 && device < kMaxScratchDevices, OXH_INVALID_SHAPE,
              "device " + std::to_string(device) + " is beyond the scratch table");
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_address[device] == nullptr) {
    void *p = nullptr;
    OXH_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    OXH_REQUIRE(p != nullptr, OXH_HIP_ERROR, "hipGetSymbolAddress returned no address");
    scratch_address[device] = p;
  }
  *address = scratch_address[device];
  return oxh::ok();
}

}  // namespace

namespace oxh {
// Called by oxh_init with `device` current.
oxh_status bn_scratch_init(int device) {
  void *unused = nullptr;
  return resolve_scratch(device, &unused);
}
}  // namespace oxh

extern "C" {

oxh_status oxh_batch_norm_workspace_size(uint64_t batch, uint64_t channels, uint64_t spatial,
                                         uint64_t *bytes) {
  OXH_REQUIRE(bytes != nullptr, OXH_INVALID_SHAPE, "bytes is null");
  oxh_status st = check_shape("oxh_batch_norm_workspace_size", batch, channels, spatial);
  if (st != OXH_OK) return st;
  *bytes = workspace_bytes_for(make_geometry(batch, channels, spatial, true));
  return oxh::ok();
}

oxh_status oxh_batch_norm_statistics(oxh_stream stream, uint64_t batch, uint64_t channels,
                                     uint64_t spatial, float epsilon, const float *input,
                                     float *mean, float *inverse_std, float *unbiased_variance,
                                     void *workspace, uint64_t workspace_bytes) {
  const char *name = "oxh_batch_norm_statistics";
  OXH_REQUIRE(mean && inverse_std, OXH_INVALID_SHAPE, std::string(name) + ": null output");
  Geometry g;
  oxh_status st = launch_reduce_x(name, stream, batch, channels, spatial, input, workspace,
                                  workspace_bytes, &g);
  if (st != OXH_OK) return st;
  StatsOut out{mean, inverse_std, unbiased_variance, nullptr, nullptr, 0.0f, epsilon};
  oxh::launch(bn_finalize_forward_kernel, dim3((channels + 3) / 4), dim3(256), 0,
                     oxh::as_stream(stream), g, input,
                     static_cast<const double2 *>(workspace), out);
  return oxh::launched(name);
}

oxh_status oxh_batch_norm_update_running(oxh_stream stream, uint64_t channels, float momentum,
                                         const float *batch_mean, const float *batch_variance,
                                         const float *old_mean, const float *old_variance,
                                         float *new_mean, float *new_variance) {
  if (channels == 0) return oxh::ok();
  OXH_REQUIRE(channels <= 65535, OXH_INVALID_SHAPE, "too many channels");
  OXH_REQUIRE(batch_mean && batch_variance && old_mean && old_variance && new_mean &&
                  new_variance,
              OXH_INVALID_SHAPE, "oxh_batch_norm_update_running: null pointer");
  oxh::launch(bn_update_running_kernel, dim3(channel_grid(channels)), dim3(256), 0,
                     oxh::as_stream(stream), static_cast<uint32_t>(channels), momentum,
                     batch_mean, batch_variance, old_mean, old_variance, new_mean,
                     new_variance);
  return oxh::launched("oxh_batch_norm_update_running");
}

oxh_status oxh_batch_norm_running_inverse_std(oxh_stream stream, uint64_t channels,
                                              float epsilon, const float *variance,
                                              float *inverse_std) {
  if (channels == 0) return oxh::ok();
  OXH_REQUIRE(channels <= 65535, OXH_INVALID_SHAPE, "too many channels");
  OXH_REQUIRE(variance && inverse_std, OXH_INVALID_SHAPE,
              "oxh_batch_norm_running_inverse_std: null pointer");
  oxh::launch(bn_running_inverse_std_kernel, dim3(channel_grid(channels)), dim3(256), 0,
                     oxh::as_stream(stream), static_cast<uint32_t>(channels), epsilon, variance,
                     inverse_std);
  return oxh::launched("oxh_batch_norm_running_inverse_std");
}

oxh_status oxh_batch_norm_apply(oxh_stream stream, uint64_t batch, uint64_t channels,
                                uint64_t spatial, const float *input, const float *weight,
                                const float *bias, const float *mean, const float *inverse_std,
                                float *output) {
  const char *name = "oxh_batch_norm_apply";
  oxh_status st = check_shape(name, batch, channels, spatial);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(input && weight && bias && mean && inverse_std && output, OXH_INVALID_SHAPE,
              std::string(name) + ": null pointer");
  const uint64_t bytes = batch * channels * spatial * 4;
  OXH_REQUIRE(input == output || !oxh::any_overlap(input, bytes, output, bytes),
              OXH_INVALID_SHAPE, std::string(name) + ": output partially overlaps the input");
  ApplyPhase::Args a{input,  weight, bias, mean, inverse_std, nullptr, 0, 0, StatsOut{}, output,
                     false};
  return launch_map<ApplyPhase>(name, stream, batch, channels, spatial,
                                oxh::aligned16(input) && oxh::aligned16(output), a);
}

oxh_status oxh_batch_norm_affine_backward(oxh_stream stream, uint64_t batch, uint64_t channels,
                                          uint64_t spatial, const float *gradient,
                                          const float *input, const float *mean,
                                          const float *inverse_std, float *weight_gradient,
                                          float *bias_gradient, void *workspace,
                                          uint64_t workspace_bytes) {
  const char *name = "oxh_batch_norm_affine_backward";
  OXH_REQUIRE(weight_gradient && bias_gradient, OXH_INVALID_SHAPE,
              std::string(name) + ": null output");
  Geometry g;
  oxh_status st = launch_reduce_gx(name, stream, batch, channels, spatial, gradient, nullptr,
                                   input, mean, inverse_std, workspace, workspace_bytes, &g);
  if (st != OXH_OK) return st;
  oxh::launch(bn_finalize_affine_kernel, dim3((channels + 3) / 4), dim3(256), 0,
                     oxh::as_stream(stream), g, static_cast<const double2 *>(workspace),
                     weight_gradient, bias_gradient);
  return oxh::launched(name);
}

oxh_status oxh_batch_norm_input_backward(oxh_stream stream, uint64_t batch, uint64_t channels,
                                         uint64_t spatial, int training, const float *gradient,
                                         const float *input, const float *weight,
                                         const float *mean, const float *inverse_std,
                                         const float *weight_gradient,
                                         const float *bias_gradient, float *output) {
  const char *name = "oxh_batch_norm_input_backward";
  oxh_status st = check_shape(name, batch, channels, spatial);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(gradient && weight && inverse_std && output, OXH_INVALID_SHAPE,
              std::string(name) + ": null pointer");
  const uint64_t bytes = batch * channels * spatial * 4;
  if (!training) {
    OXH_REQUIRE(gradient == output || !oxh::any_overlap(gradient, bytes, output, bytes),
                OXH_INVALID_SHAPE, std::string(name) + ": output partially overlaps gradient");
    DxEvalPhase::Args a{gradient, weight, inverse_std, output};
    return launch_map<DxEvalPhase>(name, stream, batch, channels, spatial,
                                   oxh::aligned16(gradient) && oxh::aligned16(output), a);
  }
  OXH_REQUIRE(input && mean && weight_gradient && bias_gradient, OXH_INVALID_SHAPE,
              std::string(name) + ": null pointer");
  st = no_overlap(name, output, bytes, {input, gradient}, bytes);
  if (st != OXH_OK) return st;
  DxTrainPhase::Args a{gradient, input, weight, mean, inverse_std, weight_gradient,
                       bias_gradient, nullptr, 0, static_cast<float>(batch * spatial),
                       nullptr, nullptr, output, nullptr};
  return launch_map<DxTrainPhase>(
      name, stream, batch, channels, spatial,
      oxh::aligned16(gradient) && oxh::aligned16(input) && oxh::aligned16(output), a);
}

oxh_status oxh_batch_norm_forward_reduce(oxh_stream stream, uint64_t batch, uint64_t channels,
                                         uint64_t spatial, const float *input, void *workspace,
                                         uint64_t workspace_bytes) {
  return launch_reduce_x("oxh_batch_norm_forward_reduce", stream, batch, channels, spatial,
                         input, workspace, workspace_bytes, nullptr);
}

oxh_status oxh_batch_norm_forward_apply(oxh_stream stream, uint64_t batch, uint64_t channels,
                                        uint64_t spatial, float momentum, float epsilon,
                                        const float *input, const float *weight,
                                        const float *bias, float *running_mean,
                                        float *running_variance, float *saved_mean,
                                        float *saved_inverse_std, float *output,
                                        const void *workspace, uint64_t workspace_bytes) {
  return forward_apply_impl("oxh_batch_norm_forward_apply", stream, batch, channels, spatial,
                            momentum, epsilon, input, weight, bias, running_mean,
                            running_variance, saved_mean, saved_inverse_std, output, workspace,
                            workspace_bytes, false);
}

oxh_status oxh_batch_norm_backward_reduce(oxh_stream stream, uint64_t batch, uint64_t channels,
                                          uint64_t spatial, const float *gradient,
                                          const float *input, const float *saved_mean,
                                          const float *saved_inverse_std, void *workspace,
                                          uint64_t workspace_bytes) {
  return launch_reduce_gx("oxh_batch_norm_backward_reduce", stream, batch, channels, spatial,
                          gradient, nullptr, input, saved_mean, saved_inverse_std, workspace,
                          workspace_bytes, nullptr);
}

oxh_status oxh_batch_norm_backward_input(oxh_stream stream, uint64_t batch, uint64_t channels,
                                         uint64_t spatial, const float *gradient,
                                         const float *input, const float *weight,
                                         const float *saved_mean,
                                         const float *saved_inverse_std, float *input_gradient,
                                         float *weight_gradient, float *bias_gradient,
                                         const void *workspace, uint64_t workspace_bytes) {
  return backward_input_impl("oxh_batch_norm_backward_input", stream, batch, channels, spatial,
                             gradient, nullptr, input, weight, saved_mean, saved_inverse_std,
                             input_gradient, weight_gradient, bias_gradient, workspace,
                             workspace_bytes);
}

oxh_status oxh_batch_norm_forward_train(oxh_stream stream, uint64_t batch, uint64_t channels,
                                        uint64_t spatial, float momentum, float epsilon,
                                        const float *input, const float *weight,
                                        const float *bias, float *running_mean,
                                        float *running_variance, float *saved_mean,
                                        float *saved_inverse_std, float *output, void *workspace,
                                        uint64_t workspace_bytes) {
  return forward_train_impl("oxh_batch_norm_forward_train", stream, batch, channels, spatial,
                            momentum, epsilon, input, weight, bias, running_mean,
                            running_variance, saved_mean, saved_inverse_std, output, workspace,
                            workspace_bytes, false);
}

// The training forward with its partials in the static per-GPU array: no allocation, no
// workspace argument.  The partials need no initialisation (every reduce block writes its own
// before the apply reads them), so nothing is cleared between calls.
oxh_status oxh_batch_norm_forward_train_no_alloc(oxh_stream stream, uint64_t batch,
                                                 uint64_t channels, uint64_t spatial,
                                                 float momentum, float epsilon,
                                                 const float *input, const float *weight,
                                                 const float *bias, float *running_mean,
                                                 float *running_variance, float *saved_mean,
                                                 float *saved_inverse_std, float *output) {
  const char *name = "oxh_batch_norm_forward_train_no_alloc";
  oxh_status st = check_shape(name, batch, channels, spatial);
  if (st != OXH_OK) return st;
  const uint64_t need = workspace_bytes_for(make_geometry(batch, channels, spatial, false));
  OXH_REQUIRE(need <= OXH_BN_NO_ALLOC_SCRATCH_BYTES, OXH_INVALID_SHAPE,
              std::string(name) + ": " + std::to_string(channels) + " channels need " +
                  std::to_string(need) + " bytes of partials, above the static " +
                  std::to_string(OXH_BN_NO_ALLOC_SCRATCH_BYTES) + "-byte array");
  int device = -1;
  OXH_HIP_CHECK(hipGetDevice(&device));
  if (stream != nullptr) {
    int stream_device = -1;
    OXH_HIP_CHECK(hipStreamGetDevice(oxh::as_stream(stream), &stream_device));
    OXH_REQUIRE(stream_device == device, OXH_INVALID_SHAPE,
                std::string(name) + ": the stream belongs to device " +
                    std::to_string(stream_device) + " but device " + std::to_string(device) +
                    " is current");
  }
  void *partials = nullptr;
  st = resolve_scratch(device, &partials);
  if (st != OXH_OK) return st;
  return forward_train_impl(name, stream, batch, channels, spatial, momentum, epsilon, input,
                            weight, bias, running_mean, running_variance, saved_mean,
                            saved_inverse_std, output, partials, OXH_BN_NO_ALLOC_SCRATCH_BYTES,
                            false);
}

oxh_status oxh_batch_norm_backward_train(oxh_stream stream, uint64_t batch, uint64_t channels,
                                         uint64_t spatial, const float *gradient,
                                         const float *input, const float *weight,
                                         const float *saved_mean,
                                         const float *saved_inverse_std, float *input_gradient,
                                         float *weight_gradient, float *bias_gradient,
                                         void *workspace, uint64_t workspace_bytes) {
  return backward_train_impl("oxh_batch_norm_backward_train", stream, batch, channels, spatial,
                             gradient, nullptr, input, weight, saved_mean, saved_inverse_std,
                             input_gradient, weight_gradient, bias_gradient, nullptr, workspace,
                             workspace_bytes);
}

oxh_status oxh_batch_norm_relu_forward_train(oxh_stream stream, uint64_t batch,
                                             uint64_t channels, uint64_t spatial, float momentum,
                                             float epsilon, const float *input,
                                             const float *weight, const float *bias,
                                             float *running_mean, float *running_variance,
                                             float *saved_mean, float *saved_inverse_std,
                                             float *output, void *workspace,
                                             uint64_t workspace_bytes) {
  return forward_train_impl("oxh_batch_norm_relu_forward_train", stream, batch, channels,
                            spatial, momentum, epsilon, input, weight, bias, running_mean,
                            running_variance, saved_mean, saved_inverse_std, output, workspace,
                            workspace_bytes, true);
}

oxh_status oxh_batch_norm_add_forward_train(oxh_stream stream, uint64_t batch, uint64_t channels,
                                            uint64_t spatial, float momentum, float epsilon,
                                            const float *input, const float *weight,
                                            const float *bias, float *running_mean,
                                            float *running_variance, float *saved_mean,
                                            float *saved_inverse_std, const float *addend,
                                            float *output, void *workspace,
                                            uint64_t workspace_bytes) {
  const char *name = "oxh_batch_norm_add_forward_train";
  OXH_REQUIRE(addend != nullptr, OXH_INVALID_SHAPE, std::string(name) + ": null addend");
  const uint64_t bytes = batch * channels * spatial * 4;
  OXH_REQUIRE(!oxh::any_overlap(output, bytes, addend, bytes), OXH_INVALID_SHAPE,
              std::string(name) + ": output overlaps the addend");
  return forward_train_impl(name, stream, batch, channels, spatial, momentum, epsilon, input,
                            weight, bias, running_mean, running_variance, saved_mean,
                            saved_inverse_std, output, workspace, workspace_bytes, false, addend);
}

oxh_status oxh_batch_norm_relu_backward_train(oxh_stream stream, uint64_t batch,
                                              uint64_t channels, uint64_t spatial,
                                              const float *gradient, const float *output,
                                              const float *input, const float *weight,
                                              const float *saved_mean,
                                              const float *saved_inverse_std,
                                              float *input_gradient, float *weight_gradient,
                                              float *bias_gradient, void *workspace,
                                              uint64_t workspace_bytes) {
  OXH_REQUIRE(output != nullptr, OXH_INVALID_SHAPE,
              "oxh_batch_norm_relu_backward_train: null output");
  return backward_train_impl("oxh_batch_norm_relu_backward_train", stream, batch, channels,
                             spatial, gradient, output, input, weight, saved_mean,
                             saved_inverse_std, input_gradient, weight_gradient, bias_gradient,
                             nullptr, workspace, workspace_bytes);
}

oxh_status oxh_conv_batch_norm_backward_train(
    oxh_stream stream, uint64_t batch, uint64_t channels, uint64_t spatial,
    const float *gradient, const float *relu_output, const float *input, const float *weight,
    const float *saved_mean, const float *saved_inverse_std, float *input_gradient,
    float *weight_gradient, float *bias_gradient, float *conv_bias_gradient, void *workspace,
    uint64_t workspace_bytes) {
  const char *name = "oxh_conv_batch_norm_backward_train";
  OXH_REQUIRE(conv_bias_gradient != nullptr, OXH_INVALID_SHAPE,
              std::string(name) + ": null conv_bias_gradient");
  return backward_train_impl(name, stream, batch, channels, spatial, gradient, relu_output,
                             input, weight, saved_mean, saved_inverse_std, input_gradient,
                             weight_gradient, bias_gradient, conv_bias_gradient, workspace,
                             workspace_bytes);
}

}  // extern "C"
