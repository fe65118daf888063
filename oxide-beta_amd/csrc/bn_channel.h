// bn_channel.h -- BatchNorm2d building blocks shared by the BatchNorm kernels and the kernels
// that fuse a BatchNorm with the convolution feeding it: fixed-order fp64 sums, the channel
// statistics (evaluation.rs:490-558), the saved / running statistics outputs, and the
// one-workgroup-per-channel forward and backward passes over values held in registers.
//
// Per-element arithmetic follows the CPU path's fp32 operation order exactly
// (-ffp-contract=off): y = ((x - mean) * inv) * w + b, x_hat = (x - mean) * inv,
// dx = ((w * inv) / M) * ((M * g - sum_g) - x_hat * sum_g_xhat).
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "common.h"

namespace oxh {

// Wave sums of doubles in wave_sums_rows' fixed order (the total in every lane).
__device__ __forceinline__ double wave_sum(double v) {
  double a[1] = {v};
  wave_sums_rows(a);
  return a[0];
}

__device__ __forceinline__ void wave_sum2(double &a, double &b) {
  double v[2] = {a, b};
  wave_sums_rows(v);
  a = v[0];
  b = v[1];
}

// ReLU backward applied to the incoming gradient (kernel_module.rs:501-508): g where the ReLU's
// output r (hence its input) is positive, else 0.
__device__ __forceinline__ float relu_masked(float g, float r) { return r > 0.0f ? g : 0.0f; }

struct Moments {
  float mean, inv, biased, correction;
};

// Channel statistics from the sums of (x - shift) and (x - shift)^2 over its M values.
__device__ __forceinline__ Moments forward_moments(double2 sums, float shift, uint64_t samples,
                                                   float epsilon) {
  const double m = static_cast<double>(samples);
  const double mean_shifted = sums.x / m;
  double var = sums.y / m - mean_shifted * mean_shifted;
  if (var < 0.0) var = 0.0;
  Moments r;
  r.mean = static_cast<float>(static_cast<double>(shift) + mean_shifted);
  const float var_f = static_cast<float>(var);
  // evaluation.rs:531-534: (variance + epsilon).sqrt().recip()
  r.inv = 1.0f / sqrtf(var_f + epsilon);
  // evaluation.rs:537-558: the running update recomputes the statistics with epsilon 0 and
  // recovers the biased variance as inv_std.powi(-2) (== 1 / (inv * inv)); the unbiased
  // correction M / (M - 1) is formed in fp32.
  const float inv0 = 1.0f / sqrtf(var_f);
  r.biased = 1.0f / (inv0 * inv0);
  r.correction = static_cast<float>(samples) / static_cast<float>(samples - 1);
  return r;
}

struct StatsOut {
  float *mean, *inverse_std, *unbiased_variance;  // unbiased_variance may be null
  float *running_mean, *running_variance;         // null: no running update
  float momentum, epsilon;
};

// The running statistics before their update, loaded at a kernel's start with the channel's
// values: read by the update itself, after the statistics, they put a memory round trip on the
// block's last thread to finish (measured ~0.8 us of a ~4 us small-plane kernel).  Zero
// without a running update.
struct RunningPrev {
  float mean, variance;
};
__device__ __forceinline__ RunningPrev load_running(const StatsOut &o, uint32_t c) {
  if (o.running_mean == nullptr) return RunningPrev{0.0f, 0.0f};
  return RunningPrev{o.running_mean[c], o.running_variance[c]};
}

__device__ __forceinline__ void write_forward_outputs(const StatsOut &o, uint32_t c,
                                                      const Moments &r, const RunningPrev &p) {
  o.mean[c] = r.mean;
  o.inverse_std[c] = r.inv;
  if (o.unbiased_variance) o.unbiased_variance[c] = r.biased * r.correction;
  if (o.running_mean) {
    const float mom = o.momentum;
    o.running_mean[c] = (1.0f - mom) * p.mean + mom * r.mean;
    o.running_variance[c] = (1.0f - mom) * p.variance + mom * r.biased * r.correction;
  }
}
__device__ __forceinline__ void write_forward_outputs(const StatsOut &o, uint32_t c,
                                                      const Moments &r) {
  write_forward_outputs(o, c, r, load_running(o, c));
}

// Small planes with few values per channel: one block per channel performs the whole
// operation -- the channel sums, their finalization, and the elementwise pass -- in a single
// launch.  Channel-relative value j of channel c is (n, p) = (j / spatial, j % spatial).
struct ChannelGeom {
  uint32_t channels, spatial, samples;  // samples = batch * spatial
  FastDiv spatial_div;
};

__device__ __forceinline__ uint32_t channel_index(const ChannelGeom &g, uint32_t c, uint32_t j) {
  const uint32_t n = fast_div(j, g.spatial_div);
  return (n * g.channels + c) * g.spatial + (j - n * g.spatial);
}

// Block-wide sums of two doubles, the total in every thread: each wave's butterfly total goes
// to LDS and every thread adds the Waves wave totals in the same order (one barrier, no
// broadcast step).  `lds` must not be in use by another sum of the same block.
template <int Waves>
__device__ __forceinline__ void block_sum2_all(double &a, double &b, double (*lds)[Waves]) {
  wave_sum2(a, b);
  const int wave = threadIdx.x / 64;
  if (threadIdx.x % 64 == 0) {
    lds[0][wave] = a;
    lds[1][wave] = b;
  }
  __syncthreads();
  a = 0.0;
  b = 0.0;
#pragma unroll
  for (int w = 0; w < Waves; ++w) {
    a += lds[0][w];
    b += lds[1][w];
  }
}

// Up to kChannelKeep values per thread stay in registers between a channel kernel's sum pass
// and its elementwise pass; larger channels read their values again (L2).  Thread t holds the
// channel's values j = t + u * Threads, u < kChannelKeep.
constexpr int kChannelKeep = 8;

// Training forward of channel c from the values in registers: fp64 sums of (v - shift) and
// (v - shift)^2 with shift = the channel's first value (x[0, c, 0]), the statistics (thread 0
// writes the saved / running outputs, the running update from prev), then y = relu?(BN(v))
// (+ added[u] when `add`) at the positions `at`, and to copy[j] (channel-relative j) when copy
// is not null.  The BatchNorm weight w, bias b, the addend values and prev are passed in,
// loaded by the caller together with the channel's values (a load issued after the sums'
// barrier would put a second memory round trip on the block).
template <bool Relu, int Threads>
__device__ __forceinline__ void channel_forward_kept(uint32_t samples, uint32_t c, float shift,
                                                     const float (&kept)[kChannelKeep],
                                                     const uint32_t (&at)[kChannelKeep], float w,
                                                     float b, const StatsOut &out,
                                                     const RunningPrev &prev, bool add,
                                                     const float (&added)[kChannelKeep], float *y,
                                                     double (*lds)[Threads / 64],
                                                     float *copy = nullptr) {
  const double k = static_cast<double>(shift);
  double sum = 0.0, sq = 0.0;
#pragma unroll
  for (int u = 0; u < kChannelKeep; ++u) {
    if (threadIdx.x + u * Threads >= samples) break;
    const double d = static_cast<double>(kept[u]) - k;
    sum += d;
    sq += d * d;
  }
  block_sum2_all<Threads / 64>(sum, sq, lds);
  const Moments r = forward_moments(make_double2(sum, sq), shift, samples, out.epsilon);
  if (threadIdx.x == 0) write_forward_outputs(out, c, r, prev);
  const float mu = r.mean, inv = r.inv;
#pragma unroll
  for (int u = 0; u < kChannelKeep; ++u)
    if (threadIdx.x + u * Threads < samples) {
      float v = (kept[u] - mu) * inv * w + b;  // evaluation.rs:590-595
      if constexpr (Relu) v = v > 0.0f ? v : 0.0f;
      if (add) v = v + added[u];
      y[at[u]] = v;
      if (copy != nullptr) copy[threadIdx.x + u * Threads] = v;
    }
}

// Training backward of a channel from registers: kg = the incoming gradient (already masked by
// a following ReLU), kn = x_hat in fp32.  Sums (sum g, sum g * x_hat) in fp64, rounded to fp32
// and stored by thread 0 to *dbias_c / *dweight_c when those are not null, and d[u] = dx for
// the thread's valid positions (autograd.rs:344-373).
template <int Threads>
__device__ __forceinline__ void channel_backward_kept(uint32_t samples,
                                                      const float (&kg)[kChannelKeep],
                                                      const float (&kn)[kChannelKeep],
                                                      float weight_c, float inv, float *dweight_c,
                                                      float *dbias_c, float (&d)[kChannelKeep],
                                                      double (*lds)[Threads / 64]) {
  double sg = 0.0, sgx = 0.0;
#pragma unroll
  for (int u = 0; u < kChannelKeep; ++u) {
    if (threadIdx.x + u * Threads >= samples) break;
    sg += static_cast<double>(kg[u]);
    sgx += static_cast<double>(kg[u] * kn[u]);
  }
  block_sum2_all<Threads / 64>(sg, sgx, lds);
  const float sgf = static_cast<float>(sg), sgxf = static_cast<float>(sgx);
  if (threadIdx.x == 0 && dbias_c != nullptr) {
    *dbias_c = sgf;
    *dweight_c = sgxf;
  }
  const float m = static_cast<float>(samples);
  const float coef = weight_c * inv / m;
#pragma unroll
  for (int u = 0; u < kChannelKeep; ++u) {
    if (threadIdx.x + u * Threads >= samples) break;
    d[u] = coef * (m * kg[u] - sgf - kn[u] * sgxf);
  }
}

}  // namespace oxh
