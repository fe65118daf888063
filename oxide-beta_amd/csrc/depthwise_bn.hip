// depthwise_bn.hip -- a depthwise ConvNormAct (nn.rs:362-395 with groups == channels: conv2d,
// BatchNorm2d in training mode, optional ReLU) in one launch per direction.
//
// Output channel c of a depthwise convolution reads input channel c only, and the BatchNorm
// that follows reduces over channel c only, so one workgroup per channel can run the whole
// layer: on small planes (the MNIST MobileNetV4's depthwise layers have at most 2048 values
// per channel) that saves the launches in between, each of which costs more than the
// layer's arithmetic.  Every value is formed by the same arithmetic, in the same order, as
// the separate kernels:
//   forward   conv sum = bias, then + x * w per tap in (ky, kx) order, taps outside the input
//             adding -0.0f (conv.hip's tap kernels); the BatchNorm (relu) channel pass
//             (bn_channel.h) over the sums, kept in registers;
//   backward  the BatchNorm (relu) channel backward in registers; its dx (the convolution's
//             output gradient) staged in LDS; the bias gradient as the BatchNorm backward's dx
//             sum; the weight gradient as conv.hip's depthwise weight kernel at the block's
//             thread count (per-tap register sums, fixed-order wave sums); the input gradient as conv.hip's
//             input-backward tap kernel (ascending output taps, -0.0f outside, then + addend).
// The channel's convolution input is staged in LDS once (coalesced plane rows) and read by
// every tap from there.
#include <hip/hip_runtime.h>

#include <string>

#include "bn_channel.h"
#include "common.h"

namespace {

using oxh::ChannelGeom;
using oxh::kChannelKeep;
using oxh::StatsOut;
using oxh::tap_mask;
using oxh::tap_term;

constexpr int kDwThreads = 256;
constexpr uint32_t kDwMaxOut = kDwThreads * kChannelKeep;  // output values per channel
constexpr uint32_t kDwMaxIn = 8192;                        // input values per channel (32 KB)
constexpr int kStageUnroll = 8;

struct DwGeom {
  uint32_t h, w, oh, ow, pad;
  uint32_t in_samples;  // batch * h * w
  ChannelGeom out;      // channels, oh * ow, batch * oh * ow
  oxh::FastDiv plane_div, w_div, ow_div;
};

// The BatchNorm (ReLU when Pre == kPreBnRelu) in front of the depthwise convolution, fused into
// its kernels when the convolution is its only consumer: a channel of the convolution's input
// is a channel of that BatchNorm, so the same block owns both.
constexpr int kPreNone = 0, kPreBn = 1, kPreBnRelu = 2;
struct PreBnForward {
  const float *input;          // the BatchNorm's input [N, C, H, W]
  const float *weight, *bias;  // its affine parameters
  const float *residual;       // added to the BatchNorm's output (a residual add), or null
  StatsOut stats;              // its saved and running statistics
  float *output;               // its output (+ residual): the convolution's input, stored
};
struct PreBnBackward {
  const float *input;             // the BatchNorm's input, for x_hat
  const float *weight;            // gamma
  const float *mean, *inverse_std;  // saved statistics
  float *dweight, *dbias;         // its affine gradients
  float *input_gradient;          // its dx: the gradient of the layer feeding it
  float *input_sum;               // per-channel sum of input_gradient (the feeding
                                  // convolution's bias gradient), or null
};

// Channel-relative value j of the convolution's input channel c: (n, p) = (j / plane, j % plane).
__device__ __forceinline__ uint32_t input_index(const DwGeom &g, uint32_t c, uint32_t j) {
  const uint32_t plane = g.h * g.w, n = oxh::fast_div(j, g.plane_div);
  return (n * g.out.channels + c) * plane + (j - n * plane);
}

// LDS copy of input channel c: xs[n * h * w + p] = x[n, c, p], kStageUnroll loads in flight
// per thread (addresses clamped into the channel, stores guarded).
template <int T>
__device__ __forceinline__ void stage_channel(const DwGeom &g, uint32_t c,
                                              const float *__restrict__ x, float *xs) {
  const uint32_t plane = g.h * g.w, last = g.in_samples - 1;
  for (uint32_t base = 0; base < g.in_samples; base += T * kStageUnroll) {
    float v[kStageUnroll];
#pragma unroll
    for (int u = 0; u < kStageUnroll; ++u) {
      uint32_t i = base + u * T + threadIdx.x;
      i = i < last ? i : last;
      const uint32_t n = oxh::fast_div(i, g.plane_div);
      v[u] = x[(n * g.out.channels + c) * plane + (i - n * plane)];
    }
#pragma unroll
    for (int u = 0; u < kStageUnroll; ++u) {
      const uint32_t i = base + u * T + threadIdx.x;
      if (i < g.in_samples) xs[i] = v[u];
    }
  }
}

// C: the input plane is 1 x 1 (one output per image), where the only tap inside the input is
// the centre (ky, kx) = (pad, pad): the other taps' -0.0f terms leave every sum unchanged and
// are skipped (bit-identical to the general path).
__host__ __device__ inline bool centre_only(uint32_t h, uint32_t w, uint32_t oh, uint32_t ow) {
  return h == 1 && w == 1 && oh == 1 && ow == 1;
}

// Input planes of 4 x 4 with pad K / 2 (config 5's first UIB layers, where the backward's
// per-value input-gradient loop spends most of its instructions on indices and on taps outside
// the plane): one thread per image forms all of the image's input-gradient sums from registers,
// with every index known at compile time.  Each sum adds exactly the terms the per-value loop
// adds, in its order; the candidates outside the plane, which that loop adds as -0.0f, change
// no sum and are skipped.  (The same form for the forward's outputs was slower.)
template <int K, int S>
struct Plane4 {
  static constexpr int H = 4, P = K / 2, OH = (H + 2 * P - K) / S + 1, M = (K + S - 1) / S;
  __device__ __forceinline__ static bool takes(const DwGeom &g) {
    return g.h == H && g.w == H && g.pad == static_cast<uint32_t>(P) &&
           g.oh == static_cast<uint32_t>(OH) && g.ow == static_cast<uint32_t>(OH) &&
           g.in_samples <= kDwMaxOut;
  }
  // image n's input-gradient sums (the candidate outputs in input_sum's order) from its output
  // gradient gp[OH * OH] and the weights wp[K * K]; out(p, value) for input position p
  template <typename Out>
  __device__ __forceinline__ static void input(const float *gp, const float *wp, Out out) {
    float gv[OH * OH], wv[K * K];
#pragma unroll
    for (int i = 0; i < OH * OH; ++i) gv[i] = gp[i];
#pragma unroll
    for (int t = 0; t < K * K; ++t) wv[t] = wp[t];
#pragma unroll
    for (int iy = 0; iy < H; ++iy)
#pragma unroll
      for (int ix = 0; ix < H; ++ix) {
        const int ty = iy + P, tx = ix + P;
        float a = 0.0f;
#pragma unroll
        for (int t = 0; t < M * M; ++t) {
          const int oy = ty / S - (M - 1) + t / M, ox = tx / S - (M - 1) + t % M;
          const int ky = ty - oy * S, kx = tx - ox * S;
          if (oy >= 0 && oy < OH && ky < K && ox >= 0 && ox < OH && kx < K)
            a += gv[oy * OH + ox] * wv[ky * K + kx];
        }
        out(iy * H + ix, a);
      }
  }
};

template <int K, int S, bool Relu, int Pre, bool C = false, int T = 256>
__global__ __launch_bounds__(T) void dw_bn_forward_kernel(
    DwGeom g, const float *__restrict__ x, const float *__restrict__ conv_weight,
    const float *__restrict__ conv_bias, float *__restrict__ conv_out,
    const float *__restrict__ bn_weight, const float *__restrict__ bn_bias, StatsOut stats,
    float *__restrict__ y, PreBnForward pre) {
  __shared__ float xs[kDwMaxIn];
  __shared__ double lds[2][T / 64];
  __shared__ float shift;
  const uint32_t c = blockIdx.x;
  // the layer's parameters, loaded before the first reduction (after it they would add a
  // memory round trip to the block)
  float wv[K * K];
#pragma unroll
  for (int t = 0; t < K * K; ++t) wv[t] = conv_weight[c * (K * K) + t];
  const float bias = conv_bias[c], w = bn_weight[c], b = bn_bias[c];
  // both BatchNorms' running statistics before their update, loaded now for the same reason
  const oxh::RunningPrev prev = oxh::load_running(stats, c);
  oxh::RunningPrev pre_prev{0.0f, 0.0f};
  if constexpr (Pre != kPreNone) pre_prev = oxh::load_running(pre.stats, c);
  if constexpr (Pre != kPreNone) {
    // the BatchNorm (relu) in front over input channel c (at most T * kChannelKeep
    // values), exactly as its channel kernel forms it; its output goes to LDS for the taps
    float kin[kChannelKeep], kadd[kChannelKeep];
    uint32_t ain[kChannelKeep];
    const bool add = pre.residual != nullptr;
#pragma unroll
    for (int u = 0; u < kChannelKeep; ++u) {
      const uint32_t j = threadIdx.x + u * T;
      ain[u] = j < g.in_samples ? input_index(g, c, j) : 0;
      kin[u] = pre.input[ain[u]];
      kadd[u] = add ? pre.residual[ain[u]] : 0.0f;
    }
    const float pshift = pre.input[input_index(g, c, 0)];
    oxh::channel_forward_kept<Pre == kPreBnRelu, T>(g.in_samples, c, pshift, kin, ain,
                                                             pre.weight[c], pre.bias[c],
                                                             pre.stats, pre_prev, add, kadd,
                                                             pre.output, lds, xs);
  } else {
    stage_channel<T>(g, c, x, xs);
  }
  __syncthreads();
  const uint32_t oplane = g.oh * g.ow, plane = g.h * g.w, samples = g.out.samples;
  float kept[kChannelKeep];
  uint32_t at[kChannelKeep];
#pragma unroll
  for (int u = 0; u < kChannelKeep; ++u) {
    const uint32_t j = threadIdx.x + u * T;
    if (j >= samples) break;  // kept / at beyond are never read
    const uint32_t n = oxh::fast_div(j, g.out.spatial_div), r = j - n * oplane;
    const uint32_t oy = oxh::fast_div(r, g.ow_div), ox = r - oy * g.ow;
    const int by = static_cast<int>(oy) * S - static_cast<int>(g.pad);
    const int bx = static_cast<int>(ox) * S - static_cast<int>(g.pad);
    const float *xp = xs + n * plane;
    float sum = bias;
    if constexpr (C) {
      sum += xs[n] * wv[g.pad * K + g.pad];
    } else {
      int row[K], col[K];
      uint32_t my[K], mx[K];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const bool vy = static_cast<uint32_t>(by + k) < g.h;
        const bool vx = static_cast<uint32_t>(bx + k) < g.w;
        row[k] = vy ? (by + k) * static_cast<int>(g.w) : 0;
        col[k] = vx ? bx + k : 0;
        my[k] = tap_mask(vy);
        mx[k] = tap_mask(vx);
      }
      float xv[K * K];
#pragma unroll
      for (int t = 0; t < K * K; ++t) xv[t] = xp[row[t / K] + col[t % K]];
#pragma unroll
      for (int t = 0; t < K * K; ++t) sum += tap_term(xv[t] * wv[t], my[t / K] & mx[t % K]);
    }
    kept[u] = sum;
    at[u] = (n * g.out.channels + c) * oplane + r;
    conv_out[at[u]] = sum;
  }
  if (threadIdx.x == 0) shift = kept[0];  // conv_out[0, c, 0] (samples >= 2)
  __syncthreads();
  const float none[kChannelKeep] = {};
  oxh::channel_forward_kept<Relu, T>(samples, c, shift, kept, at, w, b, stats, prev, false,
                                              none, y, lds);
}

template <int K, int S, bool Relu, int Pre, bool C = false, int T = 256>
__global__ __launch_bounds__(T) void dw_bn_backward_kernel(
    DwGeom g, const float *__restrict__ grad, const float *__restrict__ relu_out,
    const float *__restrict__ conv_out, const float *__restrict__ bn_weight,
    const float *__restrict__ mean, const float *__restrict__ inverse_std,
    const float *__restrict__ x, const float *__restrict__ conv_weight, const float *addend,
    float *__restrict__ conv_grad, float *__restrict__ bn_dweight, float *__restrict__ bn_dbias,
    float *__restrict__ conv_dbias, float *__restrict__ conv_dweight, float *dx,
    PreBnBackward pre) {
  constexpr int kTaps = K * K, kWaves = T / 64;
  __shared__ float xs[kDwMaxIn];
  __shared__ float gs[kDwMaxOut];
  __shared__ float wts[kTaps];
  __shared__ double lds[2][2][kWaves];
  __shared__ double lds_pre[2][2][kWaves];
  __shared__ float wave_sums[kWaves][kTaps];
  const uint32_t c = blockIdx.x;
  const uint32_t oplane = g.oh * g.ow, plane = g.h * g.w, samples = g.out.samples;
  const float mu = mean[c], inv = inverse_std[c];
  // every load the block needs is issued here, before the first reduction: the convolution's
  // input channel (kept in registers when it fits, for the LDS copy), the addend, the
  // convolution weights, and the BatchNorm in front's input values and statistics
  // These loads are unconditional (indices clamped into the channel, the addend read from x
  // when there is none, unused then): a branch around them makes its merge wait for every
  // load in flight (the merged registers are their destinations), a memory round trip before
  // the next loads issue.
  const bool kept_in = g.in_samples <= static_cast<uint32_t>(T * kChannelKeep);
  const float *add_src = addend != nullptr ? addend : x;
  float xin[kChannelKeep], addv[kChannelKeep], pin[kChannelKeep];
  uint32_t pat[kChannelKeep];
#pragma unroll
  for (int u = 0; u < kChannelKeep; ++u) {
    pat[u] = input_index(g, c, min(threadIdx.x + u * T, g.in_samples - 1));
    xin[u] = x[pat[u]];
    addv[u] = add_src[pat[u]];
  }
  const float wt_reg = threadIdx.x < static_cast<uint32_t>(kTaps)
                           ? conv_weight[c * kTaps + threadIdx.x] : 0.0f;
  float pmu = 0.0f, pinv = 0.0f, pw = 0.0f;
  if constexpr (Pre != kPreNone) {  // pre_eligible: the input channel is kept
#pragma unroll
    for (int u = 0; u < kChannelKeep; ++u) pin[u] = pre.input[pat[u]];
    pmu = pre.mean[c];
    pinv = pre.inverse_std[c];
    pw = pre.weight[c];
  }
  // BatchNorm (relu) backward from registers
  float kg[kChannelKeep], kn[kChannelKeep], d[kChannelKeep];
  uint32_t at[kChannelKeep];
#pragma unroll
  for (int u = 0; u < kChannelKeep; ++u) {
    const uint32_t j = threadIdx.x + u * T;
    at[u] = j < samples ? oxh::channel_index(g.out, c, j) : 0;
    float gv = grad[at[u]];
    if constexpr (Relu) gv = oxh::relu_masked(gv, relu_out[at[u]]);
    kg[u] = gv;
    kn[u] = (conv_out[at[u]] - mu) * inv;
  }
  if (kept_in) {
#pragma unroll
    for (int u = 0; u < kChannelKeep; ++u) {
      const uint32_t j = threadIdx.x + u * T;
      if (j < g.in_samples) xs[j] = xin[u];
    }
  } else {
    stage_channel<T>(g, c, x, xs);
  }
  if (threadIdx.x < kTaps) wts[threadIdx.x] = wt_reg;
  oxh::channel_backward_kept<T>(samples, kg, kn, bn_weight[c], inv, bn_dweight + c,
                                         bn_dbias + c, d, lds[0]);
  double total = 0.0, unused = 0.0;
#pragma unroll
  for (int u = 0; u < kChannelKeep; ++u) {
    const uint32_t j = threadIdx.x + u * T;
    if (j >= samples) break;
    if (conv_grad != nullptr) conv_grad[at[u]] = d[u];
    gs[j] = d[u];
    total += static_cast<double>(d[u]);
  }
  // the sum's barrier also publishes gs, xs and wts to the block
  oxh::block_sum2_all<kWaves>(total, unused, lds[1]);
  if (threadIdx.x == 0) conv_dbias[c] = static_cast<float>(total);

  // weight gradient: per-tap sums over the channel's output positions j, j + 256, ...
  constexpr int kSums = C ? 1 : kTaps;  // with C only the centre tap's (the others are +0)
  float acc[kSums];
#pragma unroll
  for (int t = 0; t < kSums; ++t) acc[t] = 0.0f;
  if constexpr (C) {
    for (uint32_t j = threadIdx.x; j < samples; j += T) acc[0] += gs[j] * xs[j];
  } else for (uint32_t j = threadIdx.x; j < samples; j += T) {
    const uint32_t n = oxh::fast_div(j, g.out.spatial_div), r = j - n * oplane;
    const uint32_t oy = oxh::fast_div(r, g.ow_div), ox = r - oy * g.ow;
    const float gv = gs[j];
    const float *xp = xs + n * plane;
    const int by = static_cast<int>(oy * S) - static_cast<int>(g.pad);
    const int bx = static_cast<int>(ox * S) - static_cast<int>(g.pad);
    float xv[kTaps];
    uint32_t mask[kTaps];
#pragma unroll
    for (int t = 0; t < kTaps; ++t) {
      const int iy = by + t / K, ix = bx + t % K;
      const bool v = static_cast<uint32_t>(iy) < g.h && static_cast<uint32_t>(ix) < g.w;
      xv[t] = xp[v ? iy * static_cast<int>(g.w) + ix : 0];
      mask[t] = tap_mask(v);
    }
#pragma unroll
    for (int t = 0; t < kTaps; ++t) acc[t] += tap_term(gv * xv[t], mask[t]);
  }
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  oxh::wave_sums_rows(acc);  // per-tap wave sums, fixed order
  if (lane == 0) {
#pragma unroll
    for (int t = 0; t < kSums; ++t) wave_sums[wave][t] = acc[t];
  }

  // input gradient: input (iy, ix) feeds outputs oy = floor(ty / S) - (M - 1) + j, j < M
  auto input_sum = [&](uint32_t i) {
    if constexpr (C) {  // image i's one output, through the centre tap
      float a = 0.0f;
      a += gs[i] * wts[g.pad * K + g.pad];
      return a;
    }
    constexpr int M = (K + S - 1) / S;
    const uint32_t n = oxh::fast_div(i, g.plane_div), r = i - n * plane;
    const uint32_t iy = oxh::fast_div(r, g.w_div), ix = r - iy * g.w;
    const int ty = static_cast<int>(iy + g.pad), tx = static_cast<int>(ix + g.pad);
    int grow[M], gcol[M], wrow[M], wcol[M];
    bool vy[M], vx[M];
#pragma unroll
    for (int j = 0; j < M; ++j) {
      const int oy = ty / S - (M - 1) + j, ox = tx / S - (M - 1) + j;
      const int ky = ty - oy * S, kx = tx - ox * S;
      vy[j] = oy >= 0 && oy < static_cast<int>(g.oh) && ky < K;
      vx[j] = ox >= 0 && ox < static_cast<int>(g.ow) && kx < K;
      grow[j] = vy[j] ? oy * static_cast<int>(g.ow) : 0;
      gcol[j] = vx[j] ? ox : 0;
      wrow[j] = vy[j] ? ky * K : 0;
      wcol[j] = vx[j] ? kx : 0;
    }
    const float *gp = gs + n * oplane;
    float a = 0.0f;
#pragma unroll
    for (int t = 0; t < M * M; ++t) {
      const float p = gp[grow[t / M] + gcol[t % M]] * wts[wrow[t / M] + wcol[t % M]];
      a += tap_term(p, tap_mask(vy[t / M] && vx[t % M]));
    }
    return a;
  };
  if constexpr (Pre != kPreNone) {
    // the BatchNorm (relu) in front, backward over its channel from the input gradient just
    // formed plus the addend (the convolution input's other gradient contributions: its whole
    // gradient, stored to dx when given; its relu output is the staged convolution input),
    // exactly as its channel backward forms it; its dx sum is the feeding convolution's bias
    // gradient
    const bool p4 = !C && Plane4<K, S>::takes(g);
    float *isum = xs + kDwMaxOut;  // past the staged input (at most kDwMaxOut values then)
    if (p4) {  // the image sums through LDS (read by the value's thread below)
      for (uint32_t n = threadIdx.x; n * 16 < g.in_samples; n += T)
        Plane4<K, S>::input(gs + n * oplane, wts, [&](int p, float a) { isum[n * 16 + p] = a; });
      __syncthreads();
    }
    float kg[kChannelKeep], kn[kChannelKeep], d[kChannelKeep];
#pragma unroll
    for (int u = 0; u < kChannelKeep; ++u) {
      const uint32_t i = threadIdx.x + u * T;
      if (i >= g.in_samples) break;
      float a = p4 ? isum[i] : input_sum(i);
      if (addend != nullptr) a = a + addv[u];
      if (dx != nullptr) dx[pat[u]] = a;
      kg[u] = Pre == kPreBnRelu ? oxh::relu_masked(a, xs[i]) : a;
      kn[u] = (pin[u] - pmu) * pinv;
    }
    oxh::channel_backward_kept<T>(g.in_samples, kg, kn, pw, pinv, pre.dweight + c,
                                           pre.dbias + c, d, lds_pre[0]);
    double ptotal = 0.0, punused = 0.0;
#pragma unroll
    for (int u = 0; u < kChannelKeep; ++u) {
      const uint32_t i = threadIdx.x + u * T;
      if (i >= g.in_samples) break;
      pre.input_gradient[pat[u]] = d[u];
      ptotal += static_cast<double>(d[u]);
    }
    oxh::block_sum2_all<kWaves>(ptotal, punused, lds_pre[1]);
    if (threadIdx.x == 0 && pre.input_sum != nullptr) pre.input_sum[c] = static_cast<float>(ptotal);
  } else if (dx != nullptr && kept_in) {
#pragma unroll
    for (int u = 0; u < kChannelKeep; ++u) {
      const uint32_t i = threadIdx.x + u * T;
      if (i >= g.in_samples) break;
      const float a = input_sum(i);
      dx[pat[u]] = addend != nullptr ? a + addv[u] : a;
    }
  } else if (dx != nullptr) {
    for (uint32_t i = threadIdx.x; i < g.in_samples; i += T) {
      const float a = input_sum(i);
      const uint32_t idx = input_index(g, c, i);
      dx[idx] = addend != nullptr ? a + addend[idx] : a;
    }
  }
  __syncthreads();
  if (threadIdx.x < kTaps) {
    const int t = threadIdx.x;
    const int r = C ? 0 : t;
    float v = wave_sums[0][r];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) v += wave_sums[w][r];
    if (C && t != static_cast<int>(g.pad * K + g.pad)) v = 0.0f;
    conv_dweight[c * kTaps + t] = v;
  }
}

// Shape check; fills g for an eligible shape.
bool make_dw_geom(const oxh_conv2d_shape *s, DwGeom &g) {
  if (s == nullptr) return false;
  const uint64_t c = s->in_channels;
  if (s->batch == 0 || c == 0 || s->height == 0 || s->width == 0) return false;
  if (s->groups != c || s->out_channels != c) return false;
  if (s->kernel_h != s->kernel_w || (s->kernel_h != 3 && s->kernel_h != 5)) return false;
  if (s->stride != 1 && s->stride != 2) return false;
  if (s->padding >= (1ull << 20)) return false;
  if (s->height + 2 * s->padding < s->kernel_h || s->width + 2 * s->padding < s->kernel_w)
    return false;
  const uint64_t oh = (s->height + 2 * s->padding - s->kernel_h) / s->stride + 1;
  const uint64_t ow = (s->width + 2 * s->padding - s->kernel_w) / s->stride + 1;
  const uint64_t out_samples = s->batch * oh * ow, in_samples = s->batch * s->height * s->width;
  if (out_samples < 2 || out_samples > kDwMaxOut || in_samples > kDwMaxIn) return false;
  if (c * in_samples >= (1ull << 31) || c * out_samples >= (1ull << 31)) return false;
  g.h = static_cast<uint32_t>(s->height);
  g.w = static_cast<uint32_t>(s->width);
  g.oh = static_cast<uint32_t>(oh);
  g.ow = static_cast<uint32_t>(ow);
  g.pad = static_cast<uint32_t>(s->padding);
  g.in_samples = static_cast<uint32_t>(in_samples);
  g.out.channels = static_cast<uint32_t>(c);
  g.out.spatial = static_cast<uint32_t>(oh * ow);
  g.out.samples = static_cast<uint32_t>(out_samples);
  g.out.spatial_div = oxh::make_fastdiv(g.out.spatial);
  g.plane_div = oxh::make_fastdiv(g.h * g.w);
  g.w_div = oxh::make_fastdiv(g.w);
  g.ow_div = oxh::make_fastdiv(g.ow);
  return true;
}

int variant(const oxh_conv2d_shape *s) { return static_cast<int>(10 * s->kernel_h + s->stride); }

// The fused BatchNorm in front keeps its channel in registers: at most kDwThreads *
// kChannelKeep values, at least 2 (the unbiased running variance).
bool pre_eligible(const DwGeom &g) {
  return g.in_samples >= 2 && g.in_samples <= static_cast<uint32_t>(kDwThreads * kChannelKeep);
}

// Threads per channel block: 1024 for few channels (at most 128, as the separate depthwise
// weight kernel) with at least 1024 output values, where 256 threads would leave most CUs
// idle and each thread several values; else 256.  C: the centre-only kernels (1 x 1 planes).
enum class DwBlock { k256, k1024, kCentre };
DwBlock dw_block(const DwGeom &g) {
  if (centre_only(g.h, g.w, g.oh, g.ow)) return DwBlock::kCentre;
  return g.out.channels <= 128 && g.out.samples >= 1024 ? DwBlock::k1024 : DwBlock::k256;
}

template <int K, int S, bool Relu, int Pre>
void launch_forward_kind(DwBlock kind, hipStream_t st, const dim3 grid, const DwGeom &g,
                         const float *x, const float *cw, const float *cb, float *co,
                         const float *bw, const float *bb, const StatsOut &so, float *y,
                         const PreBnForward &pre) {
  if (kind == DwBlock::kCentre)
    oxh::launch(dw_bn_forward_kernel<K, S, Relu, Pre, true>, grid, dim3(256), 0, st, g, x, cw, cb, co, bw, bb, so, y, pre);
  else if (kind == DwBlock::k1024)
    oxh::launch(dw_bn_forward_kernel<K, S, Relu, Pre, false, 1024>, grid, dim3(1024), 0, st, g, x, cw, cb, co, bw, bb, so, y, pre);
  else
    oxh::launch(dw_bn_forward_kernel<K, S, Relu, Pre>, grid, dim3(256), 0, st, g, x, cw, cb, co, bw, bb, so, y, pre);
}

template <int K, int S, bool Relu>
void launch_forward_pre(int pre_kind, hipStream_t st, const dim3 grid, const DwGeom &g,
                        const float *x, const float *cw, const float *cb, float *co,
                        const float *bw, const float *bb, const StatsOut &so, float *y,
                        const PreBnForward &pre) {
  const DwBlock kind = dw_block(g);
  if (pre_kind == kPreBnRelu)
    launch_forward_kind<K, S, Relu, kPreBnRelu>(kind, st, grid, g, x, cw, cb, co, bw, bb, so, y, pre);
  else if (pre_kind == kPreBn)
    launch_forward_kind<K, S, Relu, kPreBn>(kind, st, grid, g, x, cw, cb, co, bw, bb, so, y, pre);
  else
    launch_forward_kind<K, S, Relu, kPreNone>(kind, st, grid, g, x, cw, cb, co, bw, bb, so, y, pre);
}

template <bool Relu>
void launch_forward(int v, int pre_kind, hipStream_t st, uint32_t channels, const DwGeom &g,
                    const float *x, const float *cw, const float *cb, float *co, const float *bw,
                    const float *bb, const StatsOut &so, float *y, const PreBnForward &pre) {
  const dim3 grid(channels);
  switch (v) {
    case 31: launch_forward_pre<3, 1, Relu>(pre_kind, st, grid, g, x, cw, cb, co, bw, bb, so, y, pre); break;
    case 32: launch_forward_pre<3, 2, Relu>(pre_kind, st, grid, g, x, cw, cb, co, bw, bb, so, y, pre); break;
    case 51: launch_forward_pre<5, 1, Relu>(pre_kind, st, grid, g, x, cw, cb, co, bw, bb, so, y, pre); break;
    default: launch_forward_pre<5, 2, Relu>(pre_kind, st, grid, g, x, cw, cb, co, bw, bb, so, y, pre);
  }
}

struct BackwardArgs {
  const float *gr, *ro, *co, *bw, *sm, *si, *x, *cw, *ad;
  float *cg, *dbw, *dbb, *dcb, *dcw, *dx;
};

template <int K, int S, bool Relu, int Pre>
void launch_backward_kind(DwBlock kind, hipStream_t st, const dim3 grid, const DwGeom &g,
                          const BackwardArgs &a, const PreBnBackward &pre) {
  if (kind == DwBlock::kCentre)
    oxh::launch(dw_bn_backward_kernel<K, S, Relu, Pre, true>, grid, dim3(256), 0, st, g, a.gr, a.ro, a.co, a.bw, a.sm, a.si, a.x, a.cw, a.ad, a.cg, a.dbw, a.dbb, a.dcb, a.dcw, a.dx, pre);
  else if (kind == DwBlock::k1024)
    oxh::launch(dw_bn_backward_kernel<K, S, Relu, Pre, false, 1024>, grid, dim3(1024), 0, st, g, a.gr, a.ro, a.co, a.bw, a.sm, a.si, a.x, a.cw, a.ad, a.cg, a.dbw, a.dbb, a.dcb, a.dcw, a.dx, pre);
  else
    oxh::launch(dw_bn_backward_kernel<K, S, Relu, Pre>, grid, dim3(256), 0, st, g, a.gr, a.ro, a.co, a.bw, a.sm, a.si, a.x, a.cw, a.ad, a.cg, a.dbw, a.dbb, a.dcb, a.dcw, a.dx, pre);
}

template <int K, int S, bool Relu>
void launch_backward_pre(int pre_kind, hipStream_t st, const dim3 grid, const DwGeom &g,
                         const BackwardArgs &a, const PreBnBackward &pre) {
  const DwBlock kind = dw_block(g);
  if (pre_kind == kPreBnRelu)
    launch_backward_kind<K, S, Relu, kPreBnRelu>(kind, st, grid, g, a, pre);
  else if (pre_kind == kPreBn)
    launch_backward_kind<K, S, Relu, kPreBn>(kind, st, grid, g, a, pre);
  else
    launch_backward_kind<K, S, Relu, kPreNone>(kind, st, grid, g, a, pre);
}

template <bool Relu>
void launch_backward(int v, int pre_kind, hipStream_t st, uint32_t channels, const DwGeom &g,
                     const BackwardArgs &a, const PreBnBackward &pre) {
  const dim3 grid(channels);
  switch (v) {
    case 31: launch_backward_pre<3, 1, Relu>(pre_kind, st, grid, g, a, pre); break;
    case 32: launch_backward_pre<3, 2, Relu>(pre_kind, st, grid, g, a, pre); break;
    case 51: launch_backward_pre<5, 1, Relu>(pre_kind, st, grid, g, a, pre); break;
    default: launch_backward_pre<5, 2, Relu>(pre_kind, st, grid, g, a, pre);
  }
}

}  // namespace

extern "C" {

int oxh_depthwise_conv_batch_norm_supported(const oxh_conv2d_shape *shape) {
  DwGeom g;
  return make_dw_geom(shape, g) ? 1 : 0;
}

oxh_status oxh_depthwise_conv_batch_norm_forward_train(
    oxh_stream stream, const oxh_conv2d_shape *shape, int relu, float momentum, float epsilon,
    const float *input, const float *conv_weight, const float *conv_bias, float *conv_output,
    const float *bn_weight, const float *bn_bias, float *running_mean, float *running_variance,
    float *saved_mean, float *saved_inverse_std, float *output) {
  const char *name = "oxh_depthwise_conv_batch_norm_forward_train";
  DwGeom g;
  OXH_REQUIRE(make_dw_geom(shape, g), OXH_INVALID_SHAPE,
              std::string(name) + ": not a supported depthwise shape "
                                  "(oxh_depthwise_conv_batch_norm_supported)");
  OXH_REQUIRE(input && conv_weight && conv_bias && conv_output && bn_weight && bn_bias &&
                  running_mean && running_variance && saved_mean && saved_inverse_std && output,
              OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  const uint64_t c = g.out.channels;
  const uint64_t in_bytes = c * g.in_samples * 4, out_bytes = c * g.out.samples * 4;
  OXH_REQUIRE(!oxh::any_overlap(conv_output, out_bytes, input, in_bytes) &&
                  !oxh::any_overlap(output, out_bytes, input, in_bytes) &&
                  !oxh::any_overlap(output, out_bytes, conv_output, out_bytes),
              OXH_INVALID_SHAPE, std::string(name) + ": outputs overlap an input or each other");
  const StatsOut so{saved_mean, saved_inverse_std, nullptr, running_mean, running_variance,
                    momentum, epsilon};
  hipStream_t st = oxh::as_stream(stream);
  const PreBnForward none{};
  if (relu)
    launch_forward<true>(variant(shape), kPreNone, st, g.out.channels, g, input, conv_weight,
                         conv_bias, conv_output, bn_weight, bn_bias, so, output, none);
  else
    launch_forward<false>(variant(shape), kPreNone, st, g.out.channels, g, input, conv_weight,
                          conv_bias, conv_output, bn_weight, bn_bias, so, output, none);
  return oxh::launched(name);
}

oxh_status oxh_depthwise_conv_batch_norm_backward_train(
    oxh_stream stream, const oxh_conv2d_shape *shape, const float *gradient,
    const float *relu_output, const float *conv_output, const float *bn_weight,
    const float *saved_mean, const float *saved_inverse_std, const float *input,
    const float *conv_weight, const float *addend, float *conv_output_gradient,
    float *bn_weight_gradient, float *bn_bias_gradient, float *conv_bias_gradient,
    float *conv_weight_gradient, float *input_gradient) {
  const char *name = "oxh_depthwise_conv_batch_norm_backward_train";
  DwGeom g;
  OXH_REQUIRE(make_dw_geom(shape, g), OXH_INVALID_SHAPE,
              std::string(name) + ": not a supported depthwise shape "
                                  "(oxh_depthwise_conv_batch_norm_supported)");
  OXH_REQUIRE(gradient && conv_output && bn_weight && saved_mean && saved_inverse_std && input &&
                  conv_weight && bn_weight_gradient && bn_bias_gradient && conv_bias_gradient &&
                  conv_weight_gradient,
              OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  OXH_REQUIRE(addend == nullptr || input_gradient != nullptr, OXH_INVALID_SHAPE,
              std::string(name) + ": addend without input_gradient");
  const uint64_t c = g.out.channels;
  const uint64_t in_bytes = c * g.in_samples * 4, out_bytes = c * g.out.samples * 4;
  if (input_gradient != nullptr) {
    // every block reads its own channel of these while others write theirs: no overlap at
    // all (addend may equal input_gradient exactly: each element is read, then written, by
    // the same thread)
    for (const void *p : {static_cast<const void *>(gradient), static_cast<const void *>(input),
                          static_cast<const void *>(conv_output),
                          static_cast<const void *>(relu_output)})
      OXH_REQUIRE(p == nullptr || !oxh::any_overlap(input_gradient, in_bytes, p,
                                                    p == input ? in_bytes : out_bytes),
                  OXH_INVALID_SHAPE, std::string(name) + ": input_gradient overlaps an input");
    OXH_REQUIRE(addend == nullptr || addend == input_gradient ||
                    !oxh::any_overlap(input_gradient, in_bytes, addend, in_bytes),
                OXH_INVALID_SHAPE, std::string(name) + ": addend partially overlaps");
  }
  if (conv_output_gradient != nullptr)
    for (const void *p : {static_cast<const void *>(gradient), static_cast<const void *>(input),
                          static_cast<const void *>(conv_output),
                          static_cast<const void *>(relu_output),
                          static_cast<const void *>(addend),
                          static_cast<const void *>(input_gradient)})
      OXH_REQUIRE(p == nullptr || !oxh::any_overlap(conv_output_gradient, out_bytes, p,
                                                    (p == input || p == addend ||
                                                     p == input_gradient)
                                                        ? in_bytes
                                                        : out_bytes),
                  OXH_INVALID_SHAPE,
                  std::string(name) + ": conv_output_gradient overlaps another tensor");
  hipStream_t st = oxh::as_stream(stream);
  const BackwardArgs a{gradient, relu_output, conv_output, bn_weight, saved_mean,
                       saved_inverse_std, input, conv_weight, addend, conv_output_gradient,
                       bn_weight_gradient, bn_bias_gradient, conv_bias_gradient,
                       conv_weight_gradient, input_gradient};
  const PreBnBackward none{};
  if (relu_output)
    launch_backward<true>(variant(shape), kPreNone, st, g.out.channels, g, a, none);
  else
    launch_backward<false>(variant(shape), kPreNone, st, g.out.channels, g, a, none);
  return oxh::launched(name);
}

int oxh_batch_norm_depthwise_conv_batch_norm_supported(const oxh_conv2d_shape *shape) {
  DwGeom g;
  return make_dw_geom(shape, g) && pre_eligible(g) ? 1 : 0;
}

oxh_status oxh_batch_norm_depthwise_conv_batch_norm_forward_train(
    oxh_stream stream, const oxh_conv2d_shape *shape, int pre_relu, float pre_momentum,
    float pre_epsilon, const float *pre_input, const float *pre_weight, const float *pre_bias,
    const float *pre_residual, float *pre_running_mean, float *pre_running_variance,
    float *pre_saved_mean, float *pre_saved_inverse_std, float *pre_output, int relu,
    float momentum, float epsilon,
    const float *conv_weight, const float *conv_bias, float *conv_output,
    const float *bn_weight, const float *bn_bias, float *running_mean, float *running_variance,
    float *saved_mean, float *saved_inverse_std, float *output) {
  const char *name = "oxh_batch_norm_depthwise_conv_batch_norm_forward_train";
  DwGeom g;
  OXH_REQUIRE(make_dw_geom(shape, g) && pre_eligible(g), OXH_INVALID_SHAPE,
              std::string(name) + ": not a supported shape "
                                  "(oxh_batch_norm_depthwise_conv_batch_norm_supported)");
  OXH_REQUIRE(pre_input && pre_weight && pre_bias && pre_running_mean && pre_running_variance &&
                  pre_saved_mean && pre_saved_inverse_std && pre_output && conv_weight &&
                  conv_bias && conv_output && bn_weight && bn_bias && running_mean &&
                  running_variance && saved_mean && saved_inverse_std && output,
              OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  OXH_REQUIRE(pre_residual == nullptr || !pre_relu, OXH_INVALID_SHAPE,
              std::string(name) + ": a residual after a ReLU");
  const uint64_t c = g.out.channels;
  const uint64_t in_bytes = c * g.in_samples * 4, out_bytes = c * g.out.samples * 4;
  OXH_REQUIRE(pre_residual == nullptr ||
                  !oxh::any_overlap(pre_output, in_bytes, pre_residual, in_bytes),
              OXH_INVALID_SHAPE, std::string(name) + ": pre_output overlaps the residual");
  OXH_REQUIRE(!oxh::any_overlap(pre_output, in_bytes, pre_input, in_bytes) &&
                  !oxh::any_overlap(conv_output, out_bytes, pre_input, in_bytes) &&
                  !oxh::any_overlap(conv_output, out_bytes, pre_output, in_bytes) &&
                  !oxh::any_overlap(output, out_bytes, pre_input, in_bytes) &&
                  !oxh::any_overlap(output, out_bytes, pre_output, in_bytes) &&
                  !oxh::any_overlap(output, out_bytes, conv_output, out_bytes),
              OXH_INVALID_SHAPE, std::string(name) + ": outputs overlap an input or each other");
  const StatsOut so{saved_mean, saved_inverse_std, nullptr, running_mean, running_variance,
                    momentum, epsilon};
  const PreBnForward pre{pre_input, pre_weight, pre_bias, pre_residual,
                         StatsOut{pre_saved_mean, pre_saved_inverse_std, nullptr,
                                  pre_running_mean, pre_running_variance, pre_momentum,
                                  pre_epsilon},
                         pre_output};
  const int kind = pre_relu ? kPreBnRelu : kPreBn;
  hipStream_t st = oxh::as_stream(stream);
  if (relu)
    launch_forward<true>(variant(shape), kind, st, g.out.channels, g, pre_output, conv_weight,
                         conv_bias, conv_output, bn_weight, bn_bias, so, output, pre);
  else
    launch_forward<false>(variant(shape), kind, st, g.out.channels, g, pre_output, conv_weight,
                          conv_bias, conv_output, bn_weight, bn_bias, so, output, pre);
  return oxh::launched(name);
}

oxh_status oxh_batch_norm_depthwise_conv_batch_norm_backward_train(
    oxh_stream stream, const oxh_conv2d_shape *shape, const float *gradient,
    const float *relu_output, const float *conv_output, const float *bn_weight,
    const float *saved_mean, const float *saved_inverse_std, const float *conv_input,
    const float *conv_weight, const float *addend, int pre_relu, const float *pre_input,
    const float *pre_weight, const float *pre_saved_mean, const float *pre_saved_inverse_std,
    float *conv_output_gradient, float *bn_weight_gradient, float *bn_bias_gradient,
    float *conv_bias_gradient, float *conv_weight_gradient, float *conv_input_gradient,
    float *pre_weight_gradient, float *pre_bias_gradient, float *pre_input_gradient,
    float *pre_input_gradient_sum) {
  const char *name = "oxh_batch_norm_depthwise_conv_batch_norm_backward_train";
  DwGeom g;
  OXH_REQUIRE(make_dw_geom(shape, g) && pre_eligible(g), OXH_INVALID_SHAPE,
              std::string(name) + ": not a supported shape "
                                  "(oxh_batch_norm_depthwise_conv_batch_norm_supported)");
  OXH_REQUIRE(gradient && conv_output && bn_weight && saved_mean && saved_inverse_std &&
                  conv_input && conv_weight && pre_input && pre_weight && pre_saved_mean &&
                  pre_saved_inverse_std && bn_weight_gradient && bn_bias_gradient &&
                  conv_bias_gradient && conv_weight_gradient && pre_weight_gradient &&
                  pre_bias_gradient && pre_input_gradient,
              OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  const uint64_t c = g.out.channels;
  const uint64_t in_bytes = c * g.in_samples * 4, out_bytes = c * g.out.samples * 4;
  // every block reads its own channel of the inputs while others write theirs: the gradients
  // overlap none of them
  for (const void *p : {static_cast<const void *>(gradient), static_cast<const void *>(relu_output),
                        static_cast<const void *>(conv_output)}) {
    OXH_REQUIRE(p == nullptr || (!oxh::any_overlap(pre_input_gradient, in_bytes, p, out_bytes) &&
                                 (conv_output_gradient == nullptr ||
                                  !oxh::any_overlap(conv_output_gradient, out_bytes, p, out_bytes))),
                OXH_INVALID_SHAPE, std::string(name) + ": a gradient overlaps an input");
  }
  for (const void *p : {static_cast<const void *>(conv_input), static_cast<const void *>(pre_input)}) {
    OXH_REQUIRE(!oxh::any_overlap(pre_input_gradient, in_bytes, p, in_bytes) &&
                    (conv_output_gradient == nullptr ||
                     !oxh::any_overlap(conv_output_gradient, out_bytes, p, in_bytes)),
                OXH_INVALID_SHAPE, std::string(name) + ": a gradient overlaps an input");
  }
  OXH_REQUIRE(conv_output_gradient == nullptr ||
                  !oxh::any_overlap(conv_output_gradient, out_bytes, pre_input_gradient, in_bytes),
              OXH_INVALID_SHAPE, std::string(name) + ": the gradients overlap");
  // the convolution input's whole gradient (+ addend), each element read then written by one
  // thread: it may equal the addend, and overlaps nothing else
  if (conv_input_gradient != nullptr)
    for (const void *p : {static_cast<const void *>(gradient),
                          static_cast<const void *>(relu_output),
                          static_cast<const void *>(conv_output),
                          static_cast<const void *>(conv_input),
                          static_cast<const void *>(pre_input),
                          static_cast<const void *>(pre_input_gradient),
                          static_cast<const void *>(conv_output_gradient)})
      OXH_REQUIRE(p == nullptr ||
                      !oxh::any_overlap(conv_input_gradient, in_bytes, p,
                                        (p == conv_input || p == pre_input ||
                                         p == pre_input_gradient)
                                            ? in_bytes
                                            : out_bytes),
                  OXH_INVALID_SHAPE,
                  std::string(name) + ": conv_input_gradient overlaps another tensor");
  OXH_REQUIRE(addend == nullptr || addend == conv_input_gradient ||
                  !oxh::any_overlap(pre_input_gradient, in_bytes, addend, in_bytes),
              OXH_INVALID_SHAPE, std::string(name) + ": addend overlaps a gradient");
  hipStream_t st = oxh::as_stream(stream);
  const BackwardArgs a{gradient, relu_output, conv_output, bn_weight, saved_mean,
                       saved_inverse_std, conv_input, conv_weight, addend,
                       conv_output_gradient, bn_weight_gradient, bn_bias_gradient,
                       conv_bias_gradient, conv_weight_gradient, conv_input_gradient};
  const PreBnBackward pre{pre_input, pre_weight, pre_saved_mean, pre_saved_inverse_std,
                          pre_weight_gradient, pre_bias_gradient, pre_input_gradient,
                          pre_input_gradient_sum};
  const int kind = pre_relu ? kPreBnRelu : kPreBn;
  if (relu_output)
    launch_backward<true>(variant(shape), kind, st, g.out.channels, g, a, pre);
  else
    launch_backward<false>(variant(shape), kind, st, g.out.channels, g, a, pre);
  return oxh::launched(name);
}

}  // extern "C"
