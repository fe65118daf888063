// conv.hip -- NCHW fp32 conv2d (groups, square stride and padding) forward, input / weight /
// bias backward, and avg_pool2d forward / backward: the layers a MobileNetV4-Conv-S training
// step needs around the BatchNorm / ReLU / cross-entropy / AdamW hot path.
//
// Reference kernels: conv2d (kernel_module.rs:359-448), conv2d_input_backward (558-658),
// conv2d_weight_backward (660-752), conv2d_bias_backward (754-778), avg_pool2d (450-490),
// avg_pool2d_backward (780-825).  CPU semantics: evaluation.rs:334-445, autograd.rs:412-527.
//
// Summation order.  The forward sums start at the bias and add products in (local input
// channel, ky, kx) order; the input gradient gathers, for one input element, the products of
// every output it feeds in (output channel, oy, ox) order -- the order in which the CPU
// path's scatter loop adds them (oy ascending is ky descending); the pooling kernels follow the
// window order.  These are the CPU path's exact fp32 operation sequences (-ffp-contract=off),
// so the results are bit-identical.  Weight and bias gradients reduce over batch * oh * ow
// terms; one thread per weight element would serialize thousands of dependent adds, so the
// weight gradient splits that range into chunks (each in the CPU order) whose partial sums a
// second launch adds in chunk order, and the bias gradient gives each channel one wave whose
// lane sums a fixed butterfly combines: deterministic, within fp32 rounding of the CPU's single
// running sum.
//
// Kernels (gfx950).  Index arithmetic is 32-bit with multiply-high division (tensors below 2^31
// elements), and the valid kernel taps / output positions of each element are computed in
// closed form, so the inner loops carry no bounds tests.
//   * Pointwise convolutions (1x1, stride 1, no padding, one group) are matrix products
//     Y[oc, (n,p)] = b[oc] + sum_ic W[oc, ic] X[ic, (n,p)], and likewise the input and weight
//     gradients.  They run as LDS-tiled products (32 x 32 or 8 x 8 outputs per block), k-slabs
//     staged through LDS with the next slab's loads in flight during the current slab's
//     arithmetic; each output one serial sum in ascending k from its initial value -- the CPU
//     order, bit-identical.  Products whose grids would leave the chip idle take split tiles
//     (8 x 8 or 16 x 16 outputs, k in four contiguous parts added in order, summed on the
//     matrix cores), as do the weight gradients (k in fixed chunks): deterministic, within
//     1e-5 * sum|terms| of the CPU's serial sum.
//   * Ungrouped K x K convolutions with small planes stage one image's planes and a channel
//     tile's weights in LDS per block; the rest (and depthwise convolutions not fused with
//     their BatchNorm, depthwise_bn.hip) run one output (or input, or weight-chunk) element
//     per thread.
#include <hip/hip_runtime.h>

#include <string>
#include <type_traits>

#include "chunk_sum.h"
#include "common.h"

namespace {

constexpr uint64_t kMaxElems = 1ull << 31;  // 32-bit index arithmetic

struct ConvGeom {
  uint32_t batch, in_c, h, w, out_c, kh, kw, stride, pad, groups;
  uint32_t oh, ow, in_per_group, out_per_group;
  oxh::FastDiv ow_div, oh_div, oc_div, w_div, h_div, ic_div, s_div, ipg_div, opg_div, kw_div,
      kh_div;
};

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const oxh::FastDiv &d) {
  return oxh::fast_div(n, d);
}

// Largest q with q * s <= a for a >= 0; -1 for a < 0.
__device__ __forceinline__ int floor_div(int a, const oxh::FastDiv &s) {
  return a < 0 ? -1 : static_cast<int>(fdiv(static_cast<uint32_t>(a), s));
}
// Smallest q >= 0 with q * s >= a.
__device__ __forceinline__ int ceil_div0(int a, const oxh::FastDiv &s) {
  return a <= 0 ? 0 : static_cast<int>(fdiv(static_cast<uint32_t>(a) + s.d - 1, s));
}

using oxh::tap_mask;
using oxh::tap_operand;
using oxh::tap_term;

typedef float f32x4_t __attribute__((ext_vector_type(4)));  // MFMA accumulators

// ---------------------------------------------------------------- direct kernels

__global__ __launch_bounds__(256) void conv2d_forward_kernel(ConvGeom g, uint32_t total,
                                                             const float *__restrict__ x,
                                                             const float *__restrict__ wt,
                                                             const float *__restrict__ bias,
                                                             float *__restrict__ y) {
  for (uint32_t o = blockIdx.x * 256 + threadIdx.x; o < total; o += gridDim.x * 256) {
    const uint32_t t0 = fdiv(o, g.ow_div), ox = o - t0 * g.ow;
    const uint32_t t1 = fdiv(t0, g.oh_div), oy = t0 - t1 * g.oh;
    const uint32_t n = fdiv(t1, g.oc_div), oc = t1 - n * g.out_c;
    const uint32_t group = fdiv(oc, g.opg_div);
    const int by = static_cast<int>(oy * g.stride) - static_cast<int>(g.pad);
    const int bx = static_cast<int>(ox * g.stride) - static_cast<int>(g.pad);
    // taps with 0 <= by + ky < h and 0 <= bx + kx < w
    const int ky0 = by < 0 ? -by : 0, kx0 = bx < 0 ? -bx : 0;
    const int ky1 = min(static_cast<int>(g.kh), static_cast<int>(g.h) - by);
    const int kx1 = min(static_cast<int>(g.kw), static_cast<int>(g.w) - bx);
    const uint32_t plane = g.h * g.w, taps = g.kh * g.kw;
    const float *xn = x + (n * g.in_c + group * g.in_per_group) * plane;
    const float *wo = wt + oc * g.in_per_group * taps;
    float sum = bias[oc];
    for (uint32_t lc = 0; lc < g.in_per_group; ++lc) {
      const float *xp = xn + lc * plane;
      const float *wp = wo + lc * taps;
      for (int ky = ky0; ky < ky1; ++ky) {
        const float *xr = xp + (by + ky) * static_cast<int>(g.w) + bx;
        const float *wr = wp + ky * static_cast<int>(g.kw);
        for (int kx = kx0; kx < kx1; ++kx) sum += xr[kx] * wr[kx];
      }
    }
    y[o] = sum;
  }
}

// Square K x K kernels with stride S (3 or 5, 1 or 2): the taps unrolled at compile time, each
// tap's input load issued unconditionally (an address inside the plane when the tap is outside
// it) and its product replaced by -0.0f when outside -- x + (-0.0f) == x for every x, so the
// sums equal those that skip the padding taps, in the same order, bit for bit, while all K * K
// loads of a channel are in flight together.
template <int K, int S>
__global__ __launch_bounds__(256) void conv2d_forward_taps_kernel(ConvGeom g, uint32_t total,
                                                                  const float *__restrict__ x,
                                                                  const float *__restrict__ wt,
                                                                  const float *__restrict__ bias,
                                                                  float *__restrict__ y) {
  for (uint32_t o = blockIdx.x * 256 + threadIdx.x; o < total; o += gridDim.x * 256) {
    const uint32_t t0 = fdiv(o, g.ow_div), ox = o - t0 * g.ow;
    const uint32_t t1 = fdiv(t0, g.oh_div), oy = t0 - t1 * g.oh;
    const uint32_t n = fdiv(t1, g.oc_div), oc = t1 - n * g.out_c;
    const uint32_t group = fdiv(oc, g.opg_div);
    const int by = static_cast<int>(oy) * S - static_cast<int>(g.pad);
    const int bx = static_cast<int>(ox) * S - static_cast<int>(g.pad);
    const uint32_t plane = g.h * g.w;
    int row[K], col[K];
    bool vy[K], vx[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      vy[k] = static_cast<uint32_t>(by + k) < g.h;
      vx[k] = static_cast<uint32_t>(bx + k) < g.w;
      row[k] = vy[k] ? (by + k) * static_cast<int>(g.w) : 0;
      col[k] = vx[k] ? bx + k : 0;
    }
    uint32_t mask[K * K];
#pragma unroll
    for (int t = 0; t < K * K; ++t) mask[t] = tap_mask(vy[t / K] && vx[t % K]);
    const float *xn = x + (n * g.in_c + group * g.in_per_group) * plane;
    const float *wo = wt + oc * g.in_per_group * (K * K);
    float sum = bias[oc];
#pragma unroll 2
    for (uint32_t lc = 0; lc < g.in_per_group; ++lc) {
      const float *xp = xn + lc * plane;
      const float *wp = wo + lc * (K * K);
      float xv[K * K], wv[K * K];
#pragma unroll
      for (int t = 0; t < K * K; ++t) {
        xv[t] = xp[row[t / K] + col[t % K]];
        wv[t] = wp[t];
      }
#pragma unroll
      for (int t = 0; t < K * K; ++t) {
        const float p = xv[t] * wv[t];
        sum += tap_term(p, mask[t]);
      }
    }
    y[o] = sum;
  }
}

// Input gradient for square K x K kernels with stride S: the outputs an input element feeds
// are oy = floor(ty / S) - (M - 1) + j, j < M = ceil(K / S) (ascending, as the CPU path adds
// them), each valid when inside the output and its tap ky = ty - oy * S < K; likewise in x.
template <int K, int S>
__global__ __launch_bounds__(256) void conv2d_input_backward_taps_kernel(
    ConvGeom g, uint32_t total, const float *__restrict__ grad, const float *__restrict__ wt,
    const float *addend, float *dx) {
  constexpr int M = (K + S - 1) / S;
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
    const uint32_t t0 = fdiv(i, g.w_div), ix = i - t0 * g.w;
    const uint32_t t1 = fdiv(t0, g.h_div), iy = t0 - t1 * g.h;
    const uint32_t n = fdiv(t1, g.ic_div), ic = t1 - n * g.in_c;
    const uint32_t group = fdiv(ic, g.ipg_div), lc = ic - group * g.in_per_group;
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
    uint32_t mask[M * M];
#pragma unroll
    for (int t = 0; t < M * M; ++t) mask[t] = tap_mask(vy[t / M] && vx[t % M]);
    const uint32_t oplane = g.oh * g.ow;
    float acc = 0.0f;
#pragma unroll 2
    for (uint32_t j = 0; j < g.out_per_group; ++j) {
      const uint32_t oc = group * g.out_per_group + j;
      const float *gp = grad + (n * g.out_c + oc) * oplane;
      const float *wp = wt + (oc * g.in_per_group + lc) * (K * K);
      float gv[M * M], wv[M * M];
#pragma unroll
      for (int t = 0; t < M * M; ++t) {
        gv[t] = gp[grow[t / M] + gcol[t % M]];
        wv[t] = wp[wrow[t / M] + wcol[t % M]];
      }
#pragma unroll
      for (int t = 0; t < M * M; ++t) {
        const float p = gv[t] * wv[t];
        acc += tap_term(p, mask[t]);
      }
    }
    dx[i] = addend != nullptr ? acc + addend[i] : acc;
  }
}

// Ungrouped K x K convolutions on small planes: one block per (image, channel tile) stages the
// image's operand planes and the tile's weights in LDS with coalesced loads (the tap kernels'
// per-lane gathers are bound by the L1 address rate); each thread then computes kLdsR
// channels at one position, reading each staged plane value once for all of them and the
// kLdsR weights as one float4 broadcast (weights staged channel-innermost, the tile padded to
// a multiple of kLdsR with zeros).  Sums run in the CPU path's order; a tap outside the input
// reads a +0 operand (tap_operand: one AND shared by the thread's kLdsR products), so for
// finite weights and gradients the forward and input gradient equal the CPU path's, which skips
// those taps, up to the sign of an exactly zero sum.  kLdsFloats bounds one block's staging.
constexpr uint32_t kLdsFloats = 16384;  // 64 KB
constexpr int kLdsR = 4;

__host__ __device__ __forceinline__ uint32_t round4(uint32_t v) { return (v + 3) & ~3u; }

// Block-wide global -> LDS staging with kStageUnroll loads in flight per thread (a load, a
// wait and a store per element would put one memory latency per element on the block; each
// pass of the loop costs one).  Element i < count is src[src_index(i)], stored at
// dst[dst_index(i)].
#ifndef OXH_STAGE_UNROLL
#define OXH_STAGE_UNROLL 16
#endif
constexpr int kStageUnroll = OXH_STAGE_UNROLL;

template <class SrcMap, class DstMap>
__device__ __forceinline__ void stage(float *dst, const float *src, uint32_t count,
                                      SrcMap src_index, DstMap dst_index) {
  const uint32_t nt = blockDim.x;
  for (uint32_t b = threadIdx.x; b < count; b += nt * kStageUnroll) {
    float v[kStageUnroll];
#pragma unroll
    for (int u = 0; u < kStageUnroll; ++u) {
      const uint32_t i = b + u * nt;
      v[u] = src[src_index(i < count ? i : count - 1)];
    }
#pragma unroll
    for (int u = 0; u < kStageUnroll; ++u) {
      const uint32_t i = b + u * nt;
      if (i < count) dst[dst_index(i)] = v[u];
    }
  }
}
__device__ __forceinline__ uint32_t same_index(uint32_t i) { return i; }
// A contiguous run: 128-bit loads and stores when both ends are 16-byte aligned and the count
// is a multiple of 4 (a block-uniform test), kStageUnroll float4 in flight per thread.
__device__ __forceinline__ void stage_plain(float *dst, const float *src, uint32_t count) {
  if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) != 0 ||
      (count & 3u) != 0) {
    stage(dst, src, count, same_index, same_index);
    return;
  }
  const uint32_t nt = blockDim.x, n4 = count / 4;
  const float4 *s4 = reinterpret_cast<const float4 *>(src);
  float4 *d4 = reinterpret_cast<float4 *>(dst);
  for (uint32_t b = threadIdx.x; b < n4; b += nt * kStageUnroll) {
    float4 v[kStageUnroll];
#pragma unroll
    for (int u = 0; u < kStageUnroll; ++u) {
      const uint32_t i = b + u * nt;
      v[u] = s4[i < n4 ? i : n4 - 1];
    }
#pragma unroll
    for (int u = 0; u < kStageUnroll; ++u) {
      const uint32_t i = b + u * nt;
      if (i < n4) d4[i] = v[u];
    }
  }
}
__device__ __forceinline__ void zero_fill(float *dst, uint32_t count, uint32_t stride,
                                          uint32_t first, uint32_t width) {
  // dst[r * stride + first + c] = 0 for r < count, c < width
  for (uint32_t i = threadIdx.x; i < count * width; i += blockDim.x) {
    const uint32_t r = i / width;
    dst[r * stride + first + (i - r * width)] = 0.0f;
  }
}

template <int K, int S>
__global__ __launch_bounds__(256) void conv2d_forward_lds_kernel(
    ConvGeom g, uint32_t oc_tile, oxh::FastDiv oplane_div, oxh::FastDiv rows_div,
    const float *__restrict__ x, const float *__restrict__ wt, const float *__restrict__ bias,
    float *__restrict__ y) {
  extern __shared__ float lds[];
  constexpr int T = K * K;
  const oxh::BlockTile bt = oxh::xcd_block();
  const uint32_t n = bt.y, oc0 = bt.x * oc_tile;
  const uint32_t ocn = min(oc_tile, g.out_c - oc0), ocp = round4(ocn);
  const uint32_t plane = g.h * g.w, xs = g.in_c * plane;
  float *xl = lds, *wl = lds + round4(xs);  // wl[(ic * T + tap) * ocp + ocl]
  stage_plain(xl, x + static_cast<uint64_t>(n) * xs, xs);
  const uint32_t rows = g.in_c * T;  // r = ic * T + tap
  stage(wl, wt + static_cast<uint64_t>(oc0) * rows, ocn * rows, same_index, [&](uint32_t i) {
    const uint32_t ocl = fdiv(i, rows_div);
    return (i - ocl * rows) * ocp + ocl;
  });
  if (ocp > ocn) zero_fill(wl, rows, ocp, ocn, ocp - ocn);
  __syncthreads();
  const uint32_t oplane = g.oh * g.ow, items = (ocp / kLdsR) * oplane;
  for (uint32_t it = threadIdx.x; it < items; it += blockDim.x) {
    const uint32_t q = fdiv(it, oplane_div), pos = it - q * oplane;
    const uint32_t oy = fdiv(pos, g.ow_div), ox = pos - oy * g.ow;
    const int by = static_cast<int>(oy) * S - static_cast<int>(g.pad);
    const int bx = static_cast<int>(ox) * S - static_cast<int>(g.pad);
    int off[T];
    uint32_t mask[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int iy = by + t / K, ix = bx + t % K;
      const bool v = static_cast<uint32_t>(iy) < g.h && static_cast<uint32_t>(ix) < g.w;
      off[t] = v ? iy * static_cast<int>(g.w) + ix : 0;
      mask[t] = tap_mask(v);
    }
    float acc[kLdsR];
#pragma unroll
    for (int r = 0; r < kLdsR; ++r) {
      const uint32_t ocl = q * kLdsR + r;
      acc[r] = ocl < ocn ? bias[oc0 + ocl] : 0.0f;
    }
    const float *wq = wl + q * kLdsR;
    for (uint32_t ic = 0; ic < g.in_c; ++ic) {
      const float *xp = xl + ic * plane;
      const float *wp = wq + ic * T * ocp;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float4 w4 = *reinterpret_cast<const float4 *>(wp + t * ocp);
        const float xv = tap_operand(xp[off[t]], mask[t]);
        acc[0] += xv * w4.x;
        acc[1] += xv * w4.y;
        acc[2] += xv * w4.z;
        acc[3] += xv * w4.w;
      }
    }
#pragma unroll
    for (int r = 0; r < kLdsR; ++r) {
      const uint32_t ocl = q * kLdsR + r;
      if (ocl < ocn) y[(static_cast<uint64_t>(n) * g.out_c + oc0 + ocl) * oplane + pos] = acc[r];
    }
  }
}

// The forward of an ungrouped K x K convolution whose output plane is small, its input-channel
// sums split: block (output-channel tile of kLdsR-channel groups, image) stages the image and
// the tile's weights as conv2d_forward_lds_kernel; thread (part, item) sums input channels
// [part * in_c / kFwdParts, (part + 1) * in_c / kFwdParts) for the item's kLdsR outputs (part 0
// from the bias), and the parts are added in order.  A quarter of the serial chain per thread
// and four times the waves of the serial kernel.
constexpr int kFwdParts = 4;

template <int K, int S>
__global__ __launch_bounds__(256) void conv2d_forward_split_kernel(
    ConvGeom g, uint32_t oc_tile, uint32_t items, oxh::FastDiv oplane_div,
    oxh::FastDiv rows_div, const float *__restrict__ x, const float *__restrict__ wt,
    const float *__restrict__ bias, float *__restrict__ y) {
  extern __shared__ float lds[];
  constexpr int T = K * K;
  const oxh::BlockTile bt = oxh::xcd_block();
  const uint32_t n = bt.y, oc0 = bt.x * oc_tile;
  const uint32_t ocn = min(oc_tile, g.out_c - oc0), ocp = round4(ocn);
  const uint32_t plane = g.h * g.w, xs = g.in_c * plane;
  const uint32_t rows = g.in_c * T;  // r = ic * T + tap
  float *xl = lds, *wl = lds + round4(xs);  // wl[(ic * T + tap) * ocp + ocl]
  float *red = wl + round4(rows * ocp);     // red[(part - 1) * items * kLdsR + ...]
  stage_plain(xl, x + static_cast<uint64_t>(n) * xs, xs);
  stage(wl, wt + static_cast<uint64_t>(oc0) * rows, ocn * rows, same_index, [&](uint32_t i) {
    const uint32_t ocl = fdiv(i, rows_div);
    return (i - ocl * rows) * ocp + ocl;
  });
  if (ocp > ocn) zero_fill(wl, rows, ocp, ocn, ocp - ocn);
  __syncthreads();
  const uint32_t oplane = g.oh * g.ow;
  const uint32_t it = threadIdx.x % items, part = threadIdx.x / items;
  const bool active = part < kFwdParts;  // threads past parts * items idle
  const uint32_t q = fdiv(it, oplane_div), pos = it - q * oplane;
  float acc[kLdsR] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (active) {
    const uint32_t oy = fdiv(pos, g.ow_div), ox = pos - oy * g.ow;
    const int by = static_cast<int>(oy) * S - static_cast<int>(g.pad);
    const int bx = static_cast<int>(ox) * S - static_cast<int>(g.pad);
    int off[T];
    uint32_t mask[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int iy = by + t / K, ix = bx + t % K;
      const bool v = static_cast<uint32_t>(iy) < g.h && static_cast<uint32_t>(ix) < g.w;
      off[t] = v ? iy * static_cast<int>(g.w) + ix : 0;
      mask[t] = tap_mask(v);
    }
    if (part == 0) {
#pragma unroll
      for (int r = 0; r < kLdsR; ++r) {
        const uint32_t ocl = q * kLdsR + r;
        acc[r] = ocl < ocn ? bias[oc0 + ocl] : 0.0f;
      }
    }
    const uint32_t ic0 = part * g.in_c / kFwdParts, ic1 = (part + 1) * g.in_c / kFwdParts;
    const float *wq = wl + q * kLdsR;
    for (uint32_t ic = ic0; ic < ic1; ++ic) {
      const float *xp = xl + ic * plane;
      const float *wp = wq + ic * T * ocp;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float4 w4 = *reinterpret_cast<const float4 *>(wp + t * ocp);
        const float xv = tap_operand(xp[off[t]], mask[t]);
        acc[0] = __builtin_fmaf(xv, w4.x, acc[0]);
        acc[1] = __builtin_fmaf(xv, w4.y, acc[1]);
        acc[2] = __builtin_fmaf(xv, w4.z, acc[2]);
        acc[3] = __builtin_fmaf(xv, w4.w, acc[3]);
      }
    }
    if (part > 0) {
#pragma unroll
      for (int r = 0; r < kLdsR; ++r) red[((part - 1) * items + it) * kLdsR + r] = acc[r];
    }
  }
  __syncthreads();
  if (!active || part != 0) return;
#pragma unroll
  for (int p = 1; p < kFwdParts; ++p)
#pragma unroll
    for (int r = 0; r < kLdsR; ++r) acc[r] += red[((p - 1) * items + it) * kLdsR + r];
#pragma unroll
  for (int r = 0; r < kLdsR; ++r) {
    const uint32_t ocl = q * kLdsR + r;
    if (ocl < ocn) y[(static_cast<uint64_t>(n) * g.out_c + oc0 + ocl) * oplane + pos] = acc[r];
  }
}

// The forward of an ungrouped K x K convolution on the matrix cores, as an implicit GEMM per
// image: y[oc][p] = bias[oc] + sum over (input channel ic, tap t) of X[ic][iy(p, t)][ix(p, t)] *
// W[oc][ic][t], a tolerance-bar sum (the MFMA's fused roundings, in place of the split
// kernel's fused multiply-adds).  Block (16-channel output tile, image) stages the image with a
// zero halo -- channel ic at xl[ic * cs + yy * wp + xx], yy = iy + pad, xx = ix + pad, a hp x wp
// plane that covers every tap of every output position, so no tap needs a mask -- and the
// tile's weights as wl[(t * C + ic) * 16 + ocl] (zero past the channels).  Wave w takes position
// tile pt = w % pos_tiles and part w / pos_tiles of the input channels (kparts parts: the four
// waves busy when the plane has fewer than three 16-position tiles); per step of 4 channels and
// per tap, v_mfma_f32_16x16x4_f32 with lane (i, q) supplying A[i][q] = X[ic + q] at output
// position 16 pt + i (positions past the plane read position 0 and are not stored) and B[q][i] =
// W[oc0 + i][ic + q][t]; D[4 q + r][i] (lane i + 16 q, register r) is output channel oc0 + i at
// position 16 pt + 4 q + r.  Part 0 starts from the bias; the other parts' sums are added to it
// in part order.  in_c is a multiple of 4; the operands are 16-byte aligned.
struct MfmaForward {
  uint32_t hp, wp, cs, ocs, oc_tile, pos_tiles, kparts;
  oxh::FastDiv plane_div, rows_div;  // rows = in_c * K * K
};

template <int K, int S>
__global__ __launch_bounds__(256) void conv2d_forward_mfma_kernel(
    ConvGeom g, MfmaForward f, const float *__restrict__ x, const float *__restrict__ wt,
    const float *__restrict__ bias, float *__restrict__ y) {
  extern __shared__ float lds[];
  constexpr int T = K * K;
  const oxh::BlockTile bt = oxh::xcd_block();
  const uint32_t n = bt.y, oc0 = bt.x * f.oc_tile;
  const uint32_t ocn = min(f.oc_tile, g.out_c - oc0);
  const uint32_t C = g.in_c, plane = g.h * g.w;
  float *xl = lds, *wl = lds + round4(C * f.cs);
  // Staging, every global load of a round in flight at once (one round for config 5's
  // shapes): the image and the weights as float4, while the LDS image region is zeroed (the
  // halo keeps the zeros) and the weight columns past the channels are cleared; a barrier; then
  // the image's values at ic * cs + (iy + pad) * wp + ix + pad and the weights at
  // (t * C + ic) * ocs + ocl.
  constexpr int U = 8;  // float4 per thread per source per round
  const uint32_t rows = C * T, nt = blockDim.x;
  const float4 *x4 = reinterpret_cast<const float4 *>(x + static_cast<uint64_t>(n) * C * plane);
  const float4 *w4 = reinterpret_cast<const float4 *>(wt + static_cast<uint64_t>(oc0) * rows);
  const uint32_t n4 = C * plane / 4, m4 = ocn * rows / 4;
  const uint32_t most = n4 > m4 ? n4 : m4;
  for (uint32_t b = 0; b < most; b += nt * U) {
    float4 xv[U], wv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t e = b + threadIdx.x + u * nt;
      xv[u] = x4[e < n4 ? e : 0];
      wv[u] = w4[e < m4 ? e : 0];
    }
    if (b == 0) {
      float4 *z = reinterpret_cast<float4 *>(xl);
      for (uint32_t e = threadIdx.x; e < round4(C * f.cs) / 4; e += nt)
        z[e] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (f.ocs > ocn) zero_fill(wl, rows, f.ocs, ocn, f.ocs - ocn);
      __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t e = b + threadIdx.x + u * nt;
      if (e < n4) {
        uint32_t ic = fdiv(4 * e, f.plane_div), rem = 4 * e - ic * plane;
        uint32_t iy = fdiv(rem, g.w_div), ix = rem - iy * g.w;
        const float v[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          xl[ic * f.cs + (iy + g.pad) * f.wp + ix + g.pad] = v[c];
          const bool row_end = ++ix == g.w;
          ix = row_end ? 0 : ix;
          iy += row_end ? 1 : 0;
          const bool plane_end = iy == g.h;
          iy = plane_end ? 0 : iy;
          ic += plane_end ? 1 : 0;
        }
      }
      if (e < m4) {
        uint32_t ocl = fdiv(4 * e, f.rows_div), rem = 4 * e - ocl * rows;
        uint32_t ic = rem / T, t = rem - ic * T;
        const float v[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          wl[(t * C + ic) * f.ocs + ocl] = v[c];
          const bool tap_end = ++t == static_cast<uint32_t>(T);
          t = tap_end ? 0 : t;
          ic += tap_end ? 1 : 0;
          const bool ch_end = ic == C;
          ic = ch_end ? 0 : ic;
          ocl += ch_end ? 1 : 0;
        }
      }
    }
  }
  __syncthreads();
  // wave w: position tile w % pos_tiles, part w / pos_tiles of the input-channel steps
  const uint32_t lane = threadIdx.x % 64, i = lane % 16, q = lane / 16, w = threadIdx.x / 64;
  const uint32_t P = g.oh * g.ow, jobs = f.pos_tiles, parts = f.kparts;
  const uint32_t pt = w % jobs, kp = w / jobs;
  const bool active = w < jobs * parts;
  const uint32_t steps = C / 4, per = (steps + parts - 1) / parts;
  const uint32_t s0 = min(kp * per, steps), s1 = min(s0 + per, steps);
  const uint32_t p = pt * 16 + i, pc = p < P ? p : 0;
  const uint32_t oy = fdiv(pc, g.ow_div), ox = pc - oy * g.ow;
  const uint32_t abase = q * f.cs + oy * S * f.wp + ox * S;
  const uint32_t oc = i;  // this lane's channel of the tile (B column, D column)
  const uint32_t bbase = q * f.ocs + oc;
  const float b0 = kp == 0 && oc < ocn ? bias[oc0 + oc] : 0.0f;
  f32x4_t acc = {b0, b0, b0, b0};
  if (active && s0 < s1) {
    // per step of 4 input channels the K * K taps' MFMAs, the next step's operands read from
    // LDS before them
    const uint32_t astep = 4 * f.cs, bstep = 4 * f.ocs, tstride = C * f.ocs;
    float av[T], bv[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      av[t] = xl[abase + s0 * astep + (t / K) * f.wp + (t % K)];
      bv[t] = wl[bbase + s0 * bstep + t * tstride];
    }
    for (uint32_t j = s0; j < s1; ++j) {
      const uint32_t jn = j + 1 < s1 ? j + 1 : j;
      float an[T], bn[T];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        an[t] = xl[abase + jn * astep + (t / K) * f.wp + (t % K)];
        bn[t] = wl[bbase + jn * bstep + t * tstride];
      }
#pragma unroll
      for (int t = 0; t < T; ++t)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[t], bv[t], acc, 0, 0, 0);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        av[t] = an[t];
        bv[t] = bn[t];
      }
    }
  }
  if (parts > 1) {  // the parts added in order by the part-0 wave
    float *red = wl + rows * f.ocs;  // red[((kp - 1) * jobs + pt) * 256 + r * 64 + lane]
    if (active && kp > 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) red[((kp - 1) * jobs + pt) * 256 + r * 64 + lane] = acc[r];
    }
    __syncthreads();
    if (active && kp == 0) {
      for (uint32_t k = 1; k < parts; ++k) {
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] += red[((k - 1) * jobs + pt) * 256 + r * 64 + lane];
      }
    }
  }
  if (active && kp == 0 && oc < ocn) {
    float *yo = y + (static_cast<uint64_t>(n) * g.out_c + oc0 + oc) * P;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t pos = pt * 16 + 4 * q + r;
      if (pos < P) yo[pos] = acc[r];
    }
  }
}

// Input gradient: block (input-channel tile, image) stages the image's whole output gradient
// and the weights of the tile's input channels as wl[(oc * K * K + tap) * icp + icl].
template <int K, int S>
__global__ __launch_bounds__(256) void conv2d_input_backward_lds_kernel(
    ConvGeom g, uint32_t ic_tile, oxh::FastDiv plane_div, const float *__restrict__ grad,
    const float *__restrict__ wt, const float *addend, float *dx) {
  extern __shared__ float lds[];
  constexpr int T = K * K, M = (K + S - 1) / S;
  const oxh::BlockTile bt = oxh::xcd_block();
  const uint32_t n = bt.y, ic0 = bt.x * ic_tile;
  const uint32_t icn = min(ic_tile, g.in_c - ic0), icp = round4(icn);
  const uint32_t oplane = g.oh * g.ow, gs = g.out_c * oplane;
  float *gl = lds, *wl = lds + round4(gs);
  stage_plain(gl, grad + static_cast<uint64_t>(n) * gs, gs);
  // element i = (oc, icl, tap): per oc the tile's icn * T contiguous weights
  const uint32_t rows = g.out_c * T, run = icn * T;
  const oxh::FastDiv run_div = oxh::make_fastdiv(run);
  stage(
      wl, wt + static_cast<uint64_t>(ic0) * T, g.out_c * run,
      [&](uint32_t i) {
        const uint32_t oc = fdiv(i, run_div);
        return oc * g.in_c * T + (i - oc * run);
      },
      [&](uint32_t i) {
        const uint32_t oc = fdiv(i, run_div), rem = i - oc * run, icl = rem / T;
        return (oc * T + rem - icl * T) * icp + icl;
      });
  if (icp > icn) zero_fill(wl, rows, icp, icn, icp - icn);
  __syncthreads();
  const uint32_t plane = g.h * g.w, items = (icp / kLdsR) * plane;
  for (uint32_t it = threadIdx.x; it < items; it += blockDim.x) {
    const uint32_t q = fdiv(it, plane_div), pos = it - q * plane;
    const uint32_t iy = fdiv(pos, g.w_div), ix = pos - iy * g.w;
    const int ty = static_cast<int>(iy + g.pad), tx = static_cast<int>(ix + g.pad);
    int goff[M * M], woff[M * M];
    uint32_t mask[M * M];
#pragma unroll
    for (int t = 0; t < M * M; ++t) {
      const int oy = ty / S - (M - 1) + t / M, ox = tx / S - (M - 1) + t % M;
      const int ky = ty - oy * S, kx = tx - ox * S;
      const bool v = oy >= 0 && oy < static_cast<int>(g.oh) && ky < K && ox >= 0 &&
                     ox < static_cast<int>(g.ow) && kx < K;
      goff[t] = v ? oy * static_cast<int>(g.ow) + ox : 0;
      woff[t] = v ? (ky * K + kx) * static_cast<int>(icp) : 0;
      mask[t] = tap_mask(v);
    }
    float acc[kLdsR] = {0.0f, 0.0f, 0.0f, 0.0f};
    const float *wq = wl + q * kLdsR;
    for (uint32_t oc = 0; oc < g.out_c; ++oc) {
      const float *gp = gl + oc * oplane;
      const float *wp = wq + oc * T * icp;
#pragma unroll
      for (int t = 0; t < M * M; ++t) {
        const float4 w4 = *reinterpret_cast<const float4 *>(wp + woff[t]);
        const float gv = tap_operand(gp[goff[t]], mask[t]);
        acc[0] += gv * w4.x;
        acc[1] += gv * w4.y;
        acc[2] += gv * w4.z;
        acc[3] += gv * w4.w;
      }
    }
#pragma unroll
    for (int r = 0; r < kLdsR; ++r) {
      const uint32_t icl = q * kLdsR + r;
      if (icl >= icn) continue;
      const uint64_t i = (static_cast<uint64_t>(n) * g.in_c + ic0 + icl) * plane + pos;
      dx[i] = addend != nullptr ? acc[r] + addend[i] : acc[r];
    }
  }
}

// Input gradient of a stride-2 K x K convolution by phase: thread (input channel, phase block
// (a, b)) forms the 2 x 2 input positions (ty, tx) = (2a + py, 2b + px) in padded coordinates
// (iy = ty - pad), whose candidate output positions are the same M x M ones,
// (a - (M - 1) + jy, b - (M - 1) + jx), M = ceil(K / 2), with kernel offset
// ky = py + 2 (M - 1 - jy) (a candidate with ky >= K is no term).  Per output channel, in
// order, and per candidate in (oy, ox) order it adds exactly the valid terms g * w of each of
// the four positions: the CPU path's order and terms, a candidate outside the output plane
// reading the zero halo (a +-0 product; for finite values equal to the CPU path's skipped term
// up to the sign of an exactly zero sum).  The output gradient is staged output-channel-
// innermost around that halo, gl[(py * owp + px) * ocs + oc] (lo rows / columns before the
// plane, enough after it for every candidate; positions ocs = ocp or ocp + 4 floats apart, an
// odd number of 16-byte units, so neighbouring positions' 128-bit reads use different banks),
// and the tile's weights as wl[(icl * T + tap) * ocp + oc]: a group of 4 output channels is one
// 128-bit read per candidate and one per tap (shared by the wave's threads of one channel).
// Each thread's 4 sums use all of its terms (the candidate kernels' threads spend 7 of 16
// candidate terms of a 3 x 3 stride-2 kernel on offsets outside the kernel).
struct PhaseGeom {
  uint32_t lo, ohp, owp, ocp, ocs, ocw, ic_tile, a0, na, nb;
  oxh::FastDiv ab_div, nb_div;
};

template <int K>
__global__ __launch_bounds__(256) void conv2d_input_backward_s2_kernel(
    ConvGeom g, PhaseGeom pg, const float *__restrict__ grad, const float *__restrict__ wt,
    const float *addend, float *dx) {
  extern __shared__ float lds[];
  constexpr int T = K * K, M = (K + 1) / 2;
  const oxh::BlockTile bt = oxh::xcd_block();
  const uint32_t n = bt.y, ic0 = bt.x * pg.ic_tile;
  const uint32_t ocp = pg.ocp, ocs = pg.ocs;
  const uint32_t icn = min(pg.ic_tile, g.in_c - ic0);
  const uint32_t gcount = pg.ohp * pg.owp * ocs, ocw = pg.ocw;
  float *gl = lds, *wl = lds + gcount;  // gcount is a multiple of 4
  {  // the gradient's halo is zero
    float4 *l4 = reinterpret_cast<float4 *>(lds);
    const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t i = threadIdx.x; i < gcount / 4; i += blockDim.x) l4[i] = z;
  }
  __syncthreads();
  const uint32_t oplane = g.oh * g.ow;
  const oxh::FastDiv oplane_div = oxh::make_fastdiv(oplane);
  stage(gl, grad + static_cast<uint64_t>(n) * g.out_c * oplane, g.out_c * oplane, same_index,
        [&](uint32_t e) {
          const uint32_t oc = fdiv(e, oplane_div), opos = e - oc * oplane;
          const uint32_t oy = fdiv(opos, g.ow_div), ox = opos - oy * g.ow;
          return ((oy + pg.lo) * pg.owp + ox + pg.lo) * ocs + oc;
        });
  // the tile's weights as wl[(icl * T + tap) * ocw + oc] (zero for oc past out_c), written as
  // float4 of four output channels: element e = (oc group, r = icl * T + tap), r fastest, so a
  // wave's four loads per element read contiguous runs of r and its 128-bit stores, ocw = 4 mod
  // 32 floats apart, cover all banks
  const uint32_t run = icn * T, groups = ocp / 4, wtotal = run * groups;
  const oxh::FastDiv run_div = oxh::make_fastdiv(run);
  const float *wsrc = wt + static_cast<uint64_t>(ic0) * T;
  const uint32_t wrow = g.in_c * T;
  constexpr int UW = 8;
  for (uint32_t b0 = threadIdx.x; b0 < wtotal; b0 += blockDim.x * UW) {
    float v[UW][4];
#pragma unroll
    for (int u = 0; u < UW; ++u) {
      const uint32_t e = b0 + u * blockDim.x, ec = e < wtotal ? e : 0;
      const uint32_t og = fdiv(ec, run_div), r = ec - og * run;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t oc = 4 * og + c;
        const bool ok = oc < g.out_c;
        v[u][c] = tap_operand(wsrc[ok ? oc * wrow + r : 0], tap_mask(ok));
      }
    }
#pragma unroll
    for (int u = 0; u < UW; ++u) {
      const uint32_t e = b0 + u * blockDim.x;
      if (e < wtotal) {
        const uint32_t og = fdiv(e, run_div), r = e - og * run;
        *reinterpret_cast<float4 *>(wl + r * ocw + 4 * og) =
            make_float4(v[u][0], v[u][1], v[u][2], v[u][3]);
      }
    }
  }
  __syncthreads();
  const uint32_t blocks_ab = pg.na * pg.nb, items = icn * blocks_ab;
  for (uint32_t it = threadIdx.x; it < items; it += blockDim.x) {
    const uint32_t icl = fdiv(it, pg.ab_div), ab = it - icl * blocks_ab;
    const uint32_t ai = fdiv(ab, pg.nb_div), bi = ab - ai * pg.nb;
    const uint32_t a = pg.a0 + ai, b = pg.a0 + bi;
    const float *gp[M][M];
#pragma unroll
    for (int jy = 0; jy < M; ++jy)
#pragma unroll
      for (int jx = 0; jx < M; ++jx)  // (oy + lo, ox + lo) with oy = a - (M - 1) + jy
        gp[jy][jx] = gl + ((a + pg.lo - (M - 1) + jy) * pg.owp + b + pg.lo - (M - 1) + jx) * ocs;
    const float *wq = wl + icl * T * ocw;
    float acc[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
    for (uint32_t oc0 = 0; oc0 < ocp; oc0 += 4) {
      float4 gv[M][M], wv[T];
#pragma unroll
      for (int jy = 0; jy < M; ++jy)
#pragma unroll
        for (int jx = 0; jx < M; ++jx)
          gv[jy][jx] = *reinterpret_cast<const float4 *>(gp[jy][jx] + oc0);
#pragma unroll
      for (int t = 0; t < T; ++t) wv[t] = *reinterpret_cast<const float4 *>(wq + t * ocw + oc0);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int py = 0; py < 2; ++py)
#pragma unroll
          for (int px = 0; px < 2; ++px)
#pragma unroll
            for (int jy = 0; jy < M; ++jy)
#pragma unroll
              for (int jx = 0; jx < M; ++jx) {
                const int ky = py + 2 * (M - 1 - jy), kx = px + 2 * (M - 1 - jx);
                if (ky >= K || kx >= K) continue;
                const float4 &gq = gv[jy][jx];
                const float4 &wt4 = wv[ky * K + kx];
                const float gu = u == 0 ? gq.x : u == 1 ? gq.y : u == 2 ? gq.z : gq.w;
                const float wu = u == 0 ? wt4.x : u == 1 ? wt4.y : u == 2 ? wt4.z : wt4.w;
                acc[py][px] += gu * wu;
              }
    }
#pragma unroll
    for (int py = 0; py < 2; ++py)
#pragma unroll
      for (int px = 0; px < 2; ++px) {
        const uint32_t iy = 2 * a + py - g.pad, ix = 2 * b + px - g.pad;  // wraps below 0
        if (iy >= g.h || ix >= g.w) continue;
        const uint64_t i = ((static_cast<uint64_t>(n) * g.in_c + ic0 + icl) * g.h + iy) * g.w + ix;
        dx[i] = addend != nullptr ? acc[py][px] + addend[i] : acc[py][px];
      }
  }
}

// The stride-2 input gradient of an ungrouped K x K convolution on the matrix cores.  Input
// position (iy, ix) of phase (py, px) = ((iy + pad) & 1, (ix + pad) & 1) receives the taps
// ky = py, py + 2, ... < K (kx likewise) from output (oy, ox) = ((iy + pad - ky) / 2,
// (ix + pad - kx) / 2): per image and phase an implicit GEMM of the phase's positions by the
// input channels over k = (tap, output channel), a tolerance-bar sum (the MFMA's fused
// roundings) in place of the phase-blocked kernel's serial one.  Block (16-channel input tile,
// image) stages the image's output gradient channel-innermost around a zero halo,
// gl[((oy + lo_y) * owp + ox + lo_x) * ocs + oc] (zero past out_c), and the tile's weights as
// wl[(t * ocp + oc) * 16 + icl] (zero past the channels); jobs (phase, 16-position tile) go to
// the waves in turn.  Per tap and step of 4 output channels, v_mfma_f32_16x16x4_f32 with lane
// (i, q) supplying A[i][q] = the gradient of channel oc + q at position 16 mt + i's output for
// the tap (positions past the phase read position 0 and are not stored) and B[q][i] =
// W[oc + q][ic0 + i][t]; D[4 q + r][i] is the input gradient of channel ic0 + i at phase
// position 16 mt + 4 q + r, stored plus the addend.
struct MfmaIg {
  uint32_t lo_y, lo_x, ohp, owp, ocs, ocp;
};

template <int K>
__device__ __forceinline__ void input_backward_mfma_block(
    const ConvGeom &g, const MfmaIg &f, uint32_t tile, uint32_t n, float *lds,
    const float *__restrict__ grad, const float *__restrict__ wt, const float *addend,
    float *dx) {
  constexpr int T = K * K;
  const uint32_t ic0 = tile * 16;
  const uint32_t ocp = f.ocp, ocs = f.ocs, oplane = g.oh * g.ow;
  const uint32_t gcount = f.ohp * f.owp * ocs;  // a multiple of 4
  float *gl = lds, *wl = lds + gcount;
  {  // the gradient's halo and channels past out_c are zero
    float4 *l4 = reinterpret_cast<float4 *>(gl);
    const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t i = threadIdx.x; i < gcount / 4; i += blockDim.x) l4[i] = z;
  }
  __syncthreads();
  const oxh::FastDiv oplane_div = oxh::make_fastdiv(oplane);
  stage(gl, grad + static_cast<uint64_t>(n) * g.out_c * oplane, g.out_c * oplane, same_index,
        [&](uint32_t e) {
          const uint32_t oc = fdiv(e, oplane_div), opos = e - oc * oplane;
          const uint32_t oy = fdiv(opos, g.ow_div), ox = opos - oy * g.ow;
          return ((oy + f.lo_y) * f.owp + ox + f.lo_x) * ocs + oc;
        });
  // weights: element e = (oc * T + t) * 4 + quad, four input channels per 128-bit store
  const uint32_t wtotal = ocp * T * 4, crow = g.in_c * T;
  constexpr int UW = 8;
  for (uint32_t b0 = threadIdx.x; b0 < wtotal; b0 += blockDim.x * UW) {
    float v[UW][4];
#pragma unroll
    for (int u = 0; u < UW; ++u) {
      const uint32_t e = b0 + u * blockDim.x, ec = e < wtotal ? e : 0;
      const uint32_t rest = ec / 4, quad = ec - rest * 4, oc = rest / T, t = rest - oc * T;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t ic = ic0 + 4 * quad + c;
        const bool ok = oc < g.out_c && ic < g.in_c;
        v[u][c] = tap_operand(wt[ok ? oc * crow + ic * T + t : 0], tap_mask(ok));
      }
    }
#pragma unroll
    for (int u = 0; u < UW; ++u) {
      const uint32_t e = b0 + u * blockDim.x;
      if (e < wtotal) {
        const uint32_t rest = e / 4, quad = e - rest * 4, oc = rest / T, t = rest - oc * T;
        *reinterpret_cast<float4 *>(wl + (t * ocp + oc) * 16 + 4 * quad) =
            make_float4(v[u][0], v[u][1], v[u][2], v[u][3]);
      }
    }
  }
  __syncthreads();
  // phases p = 2 py + px: first position (iy0, ix0), extent na x nb, 16-position tiles
  uint32_t na[2], nb[2], tiles[4], first[5];
#pragma unroll
  for (int ph = 0; ph < 2; ++ph) {
    const uint32_t iy0 = (ph + g.pad) & 1u;
    na[ph] = g.h > iy0 ? (g.h - iy0 + 1) / 2 : 0;
    nb[ph] = g.w > iy0 ? (g.w - iy0 + 1) / 2 : 0;
  }
  first[0] = 0;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    tiles[p] = (na[p >> 1] * nb[p & 1] + 15) / 16;
    first[p + 1] = first[p] + tiles[p];
  }
  const uint32_t lane = threadIdx.x % 64, i = lane % 16, q = lane / 16;
  const uint32_t waves = blockDim.x / 64, steps = ocp / 4;
  for (uint32_t job = threadIdx.x / 64; job < first[4]; job += waves) {
    uint32_t p = 0;
#pragma unroll
    for (int u = 1; u < 4; ++u) p += job >= first[u] ? 1u : 0u;
    const uint32_t py = p >> 1, px = p & 1, mt = job - first[p];
    const uint32_t iy0 = (py + g.pad) & 1u, ix0 = (px + g.pad) & 1u;
    const uint32_t mcount = na[py] * nb[px];
    const uint32_t m = mt * 16 + i, mc = m < mcount ? m : 0;
    const uint32_t a = mc / nb[px], b = mc - a * nb[px];
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t ky = py; ky < static_cast<uint32_t>(K); ky += 2) {
      // oy = (iy0 + pad - ky) / 2 + a, exact (same parity); lo_y keeps the row inside the halo
      const uint32_t row = static_cast<uint32_t>(
          (static_cast<int>(iy0 + g.pad) - static_cast<int>(ky)) / 2 + static_cast<int>(a + f.lo_y));
      for (uint32_t kx = px; kx < static_cast<uint32_t>(K); kx += 2) {
        const uint32_t col = static_cast<uint32_t>(
            (static_cast<int>(ix0 + g.pad) - static_cast<int>(kx)) / 2 + static_cast<int>(b + f.lo_x));
        const float *ap = gl + (row * f.owp + col) * ocs + q;
        const float *bp = wl + ((ky * K + kx) * ocp + q) * 16 + i;
        uint32_t s = 0;
        for (; s + 4 <= steps; s += 4) {  // four steps' operands read, then their MFMAs
          float av[4], bv[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            av[u] = ap[4 * (s + u)];
            bv[u] = bp[64 * (s + u)];
          }
#pragma unroll
          for (int u = 0; u < 4; ++u)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u], bv[u], acc, 0, 0, 0);
        }
        for (; s < steps; ++s)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ap[4 * s], bp[64 * s], acc, 0, 0, 0);
      }
    }
    const uint32_t ic = ic0 + i;
    if (ic < g.in_c) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t mo = mt * 16 + 4 * q + r;
        if (mo >= mcount) continue;
        const uint32_t ao = mo / nb[px], bo = mo - ao * nb[px];
        const uint32_t iy = iy0 + 2 * ao, ix = ix0 + 2 * bo;
        const uint64_t o = ((static_cast<uint64_t>(n) * g.in_c + ic) * g.h + iy) * g.w + ix;
        dx[o] = addend != nullptr ? acc[r] + addend[o] : acc[r];
      }
    }
  }
}

template <int K>
__global__ __launch_bounds__(256) void conv2d_input_backward_mfma_kernel(
    ConvGeom g, MfmaIg f, const float *__restrict__ grad, const float *__restrict__ wt,
    const float *addend, float *dx) {
  extern __shared__ float lds[];
  const oxh::BlockTile bt = oxh::xcd_block();
  input_backward_mfma_block<K>(g, f, bt.x, bt.y, lds, grad, wt, addend, dx);
}

// The weight gradient of an ungrouped K x K convolution on the matrix cores:
// dW[oc][ic][t] = sum over images n and output positions p of G[n][oc][p] *
// X[n][ic][iy(p, t)][ix(p, t)], a GEMM of M = out_c rows, N = in_c * K * K columns (ic, t) and
// k = (image, position), summed per chunk of ipc images (a tolerance-bar sum: the MFMA's fused
// roundings; the chunks' partials are then added in chunk order).  Block (job group, chunk)
// stages the chunk's images with a zero halo as conv2d_forward_mfma_kernel does
// (xl[(img * C + ic) * cs + yy * wp + xx]) and the output gradient as
// gl[oc * kpad + img * P + p] (zero past the chunk's positions and the channels).  Job j of the chunk (wave j % 4 of block j / 4)
// is M tile mt = j / ngroups and N tiles [NG * (j % ngroups), + NG): per step of 4 k, lane
// (i, q) supplies A[i][q] = G[16 mt + i][k + q] and, per N tile, B[q][i] = the image value of
// column 16 nt + i = (ic, t) at k + q, xl[o(k + q) + ic * cs + (t / K) * wp + t % K] with
// o(k) = img * C * cs + oy * S * wp + ox * S (columns past the weights and k past the chunk read
// in-range values whose products are not stored or are multiplied by zero); D[4 q + r][i] is dW[16 mt + 4 q + r] at
// column 16 nt + i.  The images and the gradient are 16-byte aligned with C * h * w and
// out_c * oh * ow multiples of 4.
struct MfmaWeight {
  uint32_t hp, wp, cs, ipc, kpad, mtiles, ntiles, ng, ngroups, jobs;
  uint32_t bias;    // 1: column in_c * K * K is the bias gradient (operand 1)
  uint32_t stride;  // floats per chunk: the weights, then (bias) out_c bias sums
  uint32_t kparts;  // > 1 (jobs <= 2): the block's waves split each job's k steps
  oxh::FastDiv plane_div, oplane_div, m_div;
};

template <int K, int S, int NG>
__device__ __forceinline__ void weight_mfma_block(const ConvGeom &g, const MfmaWeight &f,
                                                  uint32_t group, uint32_t chunk, float *lds,
                                                  const float *__restrict__ grad,
                                                  const float *__restrict__ x,
                                                  float *__restrict__ out_w,
                                                  float *__restrict__ out_b) {
  constexpr int T = K * K;
  const uint32_t n0 = chunk * f.ipc;
  const uint32_t imgs = min(f.ipc, g.batch - n0);
  const uint32_t C = g.in_c, M = g.out_c, plane = g.h * g.w, P = g.oh * g.ow;
  const uint32_t xcount = round4(f.ipc * C * f.cs), gcount = f.mtiles * 16 * f.kpad;
  float *xl = lds, *gl = lds + xcount;
  const uint32_t nt_ = blockDim.x;
  // every global load of a round in flight at once while the LDS regions are zeroed
  constexpr int U = 8;
  const float4 *x4 = reinterpret_cast<const float4 *>(x + static_cast<uint64_t>(n0) * C * plane);
  const float4 *g4 = reinterpret_cast<const float4 *>(grad + static_cast<uint64_t>(n0) * M * P);
  const uint32_t n4 = imgs * C * plane / 4, m4 = imgs * M * P / 4;
  const uint32_t most = n4 > m4 ? n4 : m4;
  for (uint32_t b = 0; b < most; b += nt_ * U) {
    float4 xv[U], gv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t e = b + threadIdx.x + u * nt_;
      xv[u] = x4[e < n4 ? e : 0];
      gv[u] = g4[e < m4 ? e : 0];
    }
    if (b == 0) {
      float4 *z = reinterpret_cast<float4 *>(lds);
      for (uint32_t e = threadIdx.x; e < (xcount + gcount) / 4; e += nt_)
        z[e] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t e = b + threadIdx.x + u * nt_;
      if (e < n4) {  // image values: (img, ic) plane index, then row and column, with carries
        uint32_t pl = fdiv(4 * e, f.plane_div), rem = 4 * e - pl * plane;
        uint32_t iy = fdiv(rem, g.w_div), ix = rem - iy * g.w;
        const float v[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          xl[pl * f.cs + (iy + g.pad) * f.wp + ix + g.pad] = v[c];
          const bool row_end = ++ix == g.w;
          ix = row_end ? 0 : ix;
          iy += row_end ? 1 : 0;
          const bool plane_end = iy == g.h;
          iy = plane_end ? 0 : iy;
          pl += plane_end ? 1 : 0;
        }
      }
      if (e < m4) {  // gradient values: image, channel, position, with carries
        const uint32_t pl = fdiv(4 * e, f.oplane_div);
        uint32_t p = 4 * e - pl * P, img = fdiv(pl, f.m_div), oc = pl - img * M;
        const float v[4] = {gv[u].x, gv[u].y, gv[u].z, gv[u].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          gl[oc * f.kpad + img * P + p] = v[c];
          const bool plane_end = ++p == P;
          p = plane_end ? 0 : p;
          oc += plane_end ? 1 : 0;
          const bool image_end = oc == M;
          oc = image_end ? 0 : oc;
          img += image_end ? 1 : 0;
        }
      }
    }
  }
  __syncthreads();
  // wave w: job w % jobs of the group's four (or, with kparts parts, of the chunk's jobs),
  // steps part w / jobs
  const uint32_t w = threadIdx.x / 64;
  const uint32_t job = f.kparts > 1 ? w % f.jobs : group * 4 + w;
  const uint32_t kp = f.kparts > 1 ? w / f.jobs : 0;
  if (job >= f.jobs || kp >= f.kparts) return;  // no barrier follows (kparts 1)
  const uint32_t lane = threadIdx.x % 64, i = lane % 16, q = lane / 16;
  const uint32_t mt = job / f.ngroups, nt0 = (job - mt * f.ngroups) * f.ng;
  const uint32_t cols = C * T;
  // NG N tiles per job (tiles past the last one read in-range values and are not stored); the
  // bias column's operand is 1 (the loaded value's bits replaced)
  uint32_t boff[NG], keep[NG], one[NG];
#pragma unroll
  for (int u = 0; u < NG; ++u) {
    const uint32_t col = (nt0 + u) * 16 + i;
    const uint32_t ic = col / T, t = col - ic * T;
    boff[u] = col < cols ? ic * f.cs + (t / K) * f.wp + (t % K) : 0;
    const bool bias_col = f.bias != 0 && col == cols;
    keep[u] = bias_col ? 0u : 0xFFFFFFFFu;
    one[u] = bias_col ? 0x3F800000u : 0u;
  }
  f32x4_t acc[NG];
#pragma unroll
  for (int u = 0; u < NG; ++u) acc[u] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  // per step of 4 k: lane k = 4 s + q's image offset formed in registers
  const float *ga = gl + (mt * 16 + i) * f.kpad + q;
  const uint32_t kc = imgs * P, per = (f.kpad / 4 + f.kparts - 1) / f.kparts;
  const uint32_t s0 = min(kp * per, f.kpad / 4), s1 = min(s0 + per, f.kpad / 4);
  auto image_offset = [&](uint32_t k) {
    const uint32_t img = fdiv(k, f.oplane_div), p = k - img * P;
    const uint32_t oy = fdiv(p, g.ow_div), ox = p - oy * g.ow;
    const uint32_t off = img * C * f.cs + oy * S * f.wp + ox * S;
    return off & (k < kc ? 0xFFFFFFFFu : 0u);  // k past the chunk: A is zero there
  };
  // two operand sets in turn: the next step's loads are in flight during this step's MFMAs
  auto load = [&](uint32_t st, float &av, float (&bv)[NG]) {
    av = ga[4 * st];
    const uint32_t base = image_offset(4 * st + q);
#pragma unroll
    for (int u = 0; u < NG; ++u)
      bv[u] = __uint_as_float((__float_as_uint(xl[base + boff[u]]) & keep[u]) | one[u]);
  };
  auto step = [&](float av, const float (&bv)[NG]) {
#pragma unroll
    for (int u = 0; u < NG; ++u)
      acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv[u], acc[u], 0, 0, 0);
  };
  float a0, a1, b0[NG], b1[NG];
  if (s0 < s1) {
    load(s0, a0, b0);
    uint32_t s4 = s0;
    for (; s4 + 1 < s1; s4 += 2) {  // sched_barrier: the loads stay ahead of the MFMAs
      load(s4 + 1, a1, b1);
      __builtin_amdgcn_sched_barrier(0);
      step(a0, b0);
      __builtin_amdgcn_sched_barrier(0);
      load(s4 + 2 < s1 ? s4 + 2 : s4 + 1, a0, b0);
      __builtin_amdgcn_sched_barrier(0);
      step(a1, b1);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (s4 < s1) step(a0, b0);
  }
  if (f.kparts > 1) {  // the parts added in order by the part-0 waves (every wave is here)
    float *red = gl + gcount;  // red[(((kp - 1) * jobs + job) * NG + u) * 256 + r * 64 + lane]
    if (kp > 0) {
#pragma unroll
      for (int u = 0; u < NG; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          red[(((kp - 1) * f.jobs + job) * NG + u) * 256 + r * 64 + lane] = acc[u][r];
    }
    __syncthreads();
    if (kp > 0) return;
    for (uint32_t k = 1; k < f.kparts; ++k)
#pragma unroll
      for (int u = 0; u < NG; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[u][r] += red[(((k - 1) * f.jobs + job) * NG + u) * 256 + r * 64 + lane];
  }
  float *ow = out_w + static_cast<uint64_t>(chunk) * f.stride;
  float *ob = out_b + static_cast<uint64_t>(chunk) * f.stride;
#pragma unroll
  for (int u = 0; u < NG; ++u) {
    const uint32_t col = (nt0 + u) * 16 + i;
    if (col > cols || (col == cols && f.bias == 0)) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t oc = mt * 16 + 4 * q + r;
      if (oc >= M) continue;
      if (col < cols)
        ow[oc * cols + col] = acc[u][r];
      else
        ob[oc] = acc[u][r];
    }
  }
}

template <int K, int S, int NG>
__global__ __launch_bounds__(256) void conv2d_weight_mfma_kernel(
    ConvGeom g, MfmaWeight f, const float *__restrict__ grad, const float *__restrict__ x,
    float *__restrict__ out_w, float *__restrict__ out_b) {
  extern __shared__ float lds[];
  weight_mfma_block<K, S, NG>(g, f, blockIdx.x, blockIdx.y, lds, grad, x, out_w, out_b);
}

// A stride-2 K x K convolution's input gradient (blocks [0, ig_blocks): tile, image) and weight
// gradient partials (the rest: job group, chunk) on the matrix cores in one launch, each block
// computing exactly what its own kernel's block computes; each part's blocks remapped over the
// XCDs on their own.
struct MfmaDual {
  uint32_t ig_tiles, ig_blocks, wg_groups, wg_blocks;
};
template <int K, int NG>
__global__ __launch_bounds__(256) void conv2d_backward_mfma_kernel(
    ConvGeom g, MfmaIg fi, MfmaWeight fw, MfmaDual d, const float *__restrict__ grad,
    const float *__restrict__ wt, const float *__restrict__ x, const float *addend, float *dx,
    float *__restrict__ out) {
  extern __shared__ float lds[];
  const uint32_t b = blockIdx.x;
  if (b < d.ig_blocks) {
    const uint32_t r = oxh::xcd_contiguous(b, d.ig_blocks);
    input_backward_mfma_block<K>(g, fi, r % d.ig_tiles, r / d.ig_tiles, lds, grad, wt, addend, dx);
  } else {
    const uint32_t r = oxh::xcd_contiguous(b - d.ig_blocks, d.wg_blocks, d.ig_blocks);
    weight_mfma_block<K, 2, NG>(g, fw, r % d.wg_groups, r / d.wg_groups, lds, grad, x, out,
                                out);
  }
}

// Weight gradient partials: block (output-channel tile of kDwOcTile, image chunk) stages each
// image's input planes and the tile's output-gradient planes position-major
// (gl[pos * kDwOcTile + ocl], zero past the tile).  Thread t < pairs * groups owns one
// (ic, tap) pair for every channel of the tile over one of `groups` position ranges (groups > 1
// when there are few pairs); the ranges' sums are added in range order at the end.  Partials
// over the chunk (the chunk sums then run in chunk order).  With Bias, `groups` more threads
// sum the output gradient itself over the same ranges (the bias gradient: a pair whose operand
// is 1), the weight threads unchanged.  The chunk's weight sums go to out_w + chunk * stride
// ([oc][ic][tap]), its bias sums to out_b + chunk * stride ([oc]).
constexpr int kDwOcTile = 16;
constexpr uint32_t kDwMaxThreads = 512;

template <int K, int S, bool Bias>
__global__ __launch_bounds__(kDwMaxThreads) void conv2d_weight_lds_kernel(
    ConvGeom g, uint32_t per_chunk, uint32_t groups, oxh::FastDiv oplane_div,
    const float *__restrict__ grad, const float *__restrict__ x, float *__restrict__ out_w,
    float *__restrict__ out_b, uint32_t stride) {
  extern __shared__ float lds[];
  constexpr int T = K * K;
  const oxh::BlockTile bt = oxh::xcd_block();
  const uint32_t oc0 = bt.x * kDwOcTile, chunk = bt.y;
  const uint32_t ocn = min(static_cast<uint32_t>(kDwOcTile), g.out_c - oc0);
  const uint32_t plane = g.h * g.w, oplane = g.oh * g.ow, xs = g.in_c * plane;
  const uint32_t pairs = g.in_c * T, wpairs = pairs * groups;
  float *gl = lds, *xl = lds + kDwOcTile * oplane;
  const uint32_t item = threadIdx.x;
  const bool bias_item = Bias && item >= wpairs && item < wpairs + groups;
  const uint32_t grp = bias_item ? item - wpairs : item / pairs;
  const uint32_t pr = bias_item ? pairs : item - grp * pairs;
  const bool active = item < wpairs || bias_item;
  const uint32_t ic = pr / T, tap = pr - ic * T;
  const int ky = static_cast<int>(tap / K) - static_cast<int>(g.pad);
  const int kx = static_cast<int>(tap % K) - static_cast<int>(g.pad);
  const int base = static_cast<int>(ic * plane);
  const uint32_t p0 = active ? grp * oplane / groups : 0;
  const uint32_t p1 = active ? (grp + 1) * oplane / groups : 0;
  const uint32_t oy0 = fdiv(p0, g.ow_div), ox0 = p0 - oy0 * g.ow;
  float acc[kDwOcTile];
#pragma unroll
  for (int o = 0; o < kDwOcTile; ++o) acc[o] = 0.0f;
  const uint32_t n0 = chunk * per_chunk, n1 = min(n0 + per_chunk, g.batch);
  for (uint32_t n = n0; n < n1; ++n) {
    __syncthreads();  // the previous image's planes are read
    stage_plain(xl, x + static_cast<uint64_t>(n) * xs, xs);
    stage(gl, grad + (static_cast<uint64_t>(n) * g.out_c + oc0) * oplane, ocn * oplane,
          same_index, [&](uint32_t i) {
            const uint32_t ocl = fdiv(i, oplane_div);
            return (i - ocl * oplane) * kDwOcTile + ocl;
          });
    if (n == n0 && ocn < kDwOcTile) zero_fill(gl, oplane, kDwOcTile, ocn, kDwOcTile - ocn);
    __syncthreads();
    uint32_t oy = oy0, ox = ox0;
    for (uint32_t pos = p0; pos < p1; ++pos) {
      float gv[kDwOcTile];
      const float4 *g4 = reinterpret_cast<const float4 *>(gl + pos * kDwOcTile);
#pragma unroll
      for (int o = 0; o < kDwOcTile / 4; ++o) {
        const float4 v = g4[o];
        gv[4 * o] = v.x;
        gv[4 * o + 1] = v.y;
        gv[4 * o + 2] = v.z;
        gv[4 * o + 3] = v.w;
      }
      const int iy = static_cast<int>(oy) * S + ky, ix = static_cast<int>(ox) * S + kx;
      const bool ok = static_cast<uint32_t>(iy) < g.h && static_cast<uint32_t>(ix) < g.w;
      // a bias thread's operand is 1 (fma(g, 1, acc) == acc + g exactly)
      const float xv = bias_item ? 1.0f
                                 : tap_operand(xl[ok ? base + iy * static_cast<int>(g.w) + ix : 0],
                                               tap_mask(ok));
#pragma unroll
      for (int o = 0; o < kDwOcTile; ++o) acc[o] = __builtin_fmaf(gv[o], xv, acc[o]);
      if (++ox == g.ow) {
        ox = 0;
        ++oy;
      }
    }
  }
  float *ow = out_w + static_cast<uint64_t>(chunk) * stride;
  float *ob = Bias ? out_b + static_cast<uint64_t>(chunk) * stride : nullptr;
  if (groups == 1) {
    if (!active) return;
#pragma unroll
    for (int o = 0; o < kDwOcTile; ++o) {
      if (static_cast<uint32_t>(o) >= ocn) continue;
      if (bias_item)
        ob[oc0 + o] = acc[o];
      else
        ow[(oc0 + o) * pairs + pr] = acc[o];
    }
    return;
  }
  __syncthreads();  // the staged planes are read: the block's LDS holds the range sums
  float *red = lds;  // red[(grp * pairs + pr) * kDwOcTile + o], the bias ranges after them
  if (active) {
#pragma unroll
    for (int o = 0; o < kDwOcTile; ++o) red[item * kDwOcTile + o] = acc[o];
  }
  __syncthreads();
  const uint32_t total = (pairs + (Bias ? 1 : 0)) * ocn;
  for (uint32_t e = threadIdx.x; e < total; e += blockDim.x) {
    float v = 0.0f;
    if (e < pairs * ocn) {
      const uint32_t o = e / pairs, q = e - o * pairs;
      for (uint32_t r = 0; r < groups; ++r) v += red[(r * pairs + q) * kDwOcTile + o];
      ow[(oc0 + o) * pairs + q] = v;
    } else {
      const uint32_t o = e - pairs * ocn;
      for (uint32_t r = 0; r < groups; ++r) v += red[(wpairs + r) * kDwOcTile + o];
      ob[oc0 + o] = v;
    }
  }
}

// One thread per input element; contributions in (oc, oy, ox) ascending order.
// addend (may be null, may equal dx): dx = sum + addend[i], the gradient accumulation of a
// tensor with a second consumer done in the same pass (the sum is complete before the add).
__global__ __launch_bounds__(256) void conv2d_input_backward_kernel(
    ConvGeom g, uint32_t total, const float *__restrict__ grad, const float *__restrict__ wt,
    const float *addend, float *dx) {
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
    const uint32_t t0 = fdiv(i, g.w_div), ix = i - t0 * g.w;
    const uint32_t t1 = fdiv(t0, g.h_div), iy = t0 - t1 * g.h;
    const uint32_t n = fdiv(t1, g.ic_div), ic = t1 - n * g.in_c;
    const uint32_t group = fdiv(ic, g.ipg_div), lc = ic - group * g.in_per_group;
    // outputs with 0 <= ty - oy * s < kh, ty = iy + pad (and likewise in x)
    const int ty = static_cast<int>(iy + g.pad), tx = static_cast<int>(ix + g.pad);
    const int oy0 = ceil_div0(ty - static_cast<int>(g.kh) + 1, g.s_div);
    const int ox0 = ceil_div0(tx - static_cast<int>(g.kw) + 1, g.s_div);
    const int oy1 = min(floor_div(ty, g.s_div), static_cast<int>(g.oh) - 1);
    const int ox1 = min(floor_div(tx, g.s_div), static_cast<int>(g.ow) - 1);
    const uint32_t oplane = g.oh * g.ow, taps = g.kh * g.kw;
    const int s = static_cast<int>(g.stride);
    float acc = 0.0f;
    for (uint32_t j = 0; j < g.out_per_group; ++j) {
      const uint32_t oc = group * g.out_per_group + j;
      const float *gp = grad + (n * g.out_c + oc) * oplane;
      const float *wp = wt + (oc * g.in_per_group + lc) * taps;
      for (int oy = oy0; oy <= oy1; ++oy) {
        const float *gr = gp + oy * static_cast<int>(g.ow);
        // kx = tx - ox * s
        const float *wr = wp + (ty - oy * s) * static_cast<int>(g.kw) + tx;
        for (int ox = ox0; ox <= ox1; ++ox) acc += gr[ox] * wr[-ox * s];
      }
    }
    dx[i] = addend != nullptr ? acc + addend[i] : acc;
  }
}

// Weight gradient, phase 1: batch chunk c for weight element e (grid-stride over
// chunks * weights), terms in (n, oy, ox) order.
__global__ __launch_bounds__(256) void conv2d_weight_partial_kernel(
    ConvGeom g, uint32_t weights, oxh::FastDiv weights_div, uint32_t chunks,
    const float *__restrict__ grad, const float *__restrict__ x, float *__restrict__ partial) {
  const uint32_t total = weights * chunks;
  const uint32_t per = (g.batch + chunks - 1) / chunks;
  const uint32_t plane = g.h * g.w, oplane = g.oh * g.ow;
  const int s = static_cast<int>(g.stride);
  for (uint32_t t = blockIdx.x * 256 + threadIdx.x; t < total; t += gridDim.x * 256) {
    const uint32_t chunk = fdiv(t, weights_div), e = t - chunk * weights;
    const uint32_t t0 = fdiv(e, g.kw_div), kx = e - t0 * g.kw;
    const uint32_t t1 = fdiv(t0, g.kh_div), ky = t0 - t1 * g.kh;
    const uint32_t oc = fdiv(t1, g.ipg_div), lc = t1 - oc * g.in_per_group;
    const uint32_t ic = fdiv(oc, g.opg_div) * g.in_per_group + lc;
    // outputs with 0 <= oy * s + dy < h, dy = ky - pad (and likewise in x)
    const int dy = static_cast<int>(ky) - static_cast<int>(g.pad);
    const int dx = static_cast<int>(kx) - static_cast<int>(g.pad);
    const int oy0 = ceil_div0(-dy, g.s_div), ox0 = ceil_div0(-dx, g.s_div);
    const int oy1 = min(floor_div(static_cast<int>(g.h) - 1 - dy, g.s_div),
                        static_cast<int>(g.oh) - 1);
    const int ox1 = min(floor_div(static_cast<int>(g.w) - 1 - dx, g.s_div),
                        static_cast<int>(g.ow) - 1);
    const uint32_t n0 = chunk * per, n1 = min(n0 + per, g.batch);
    float acc = 0.0f;
    for (uint32_t n = n0; n < n1; ++n) {
      const float *gp = grad + (n * g.out_c + oc) * oplane;
      const float *xp = x + (n * g.in_c + ic) * plane;
      for (int oy = oy0; oy <= oy1; ++oy) {
        const float *gr = gp + oy * static_cast<int>(g.ow);
        const float *xr = xp + (oy * s + dy) * static_cast<int>(g.w) + dx;
        for (int ox = ox0; ox <= ox1; ++ox) acc += gr[ox] * xr[ox * s];
      }
    }
    partial[t] = acc;
  }
}

// Depthwise weight gradient (one group per channel, square kernels of size 3 or 5): one block
// of Threads per channel (1024 when there are few channels).  Each thread walks the channel's
// output positions j, j + Threads, ... and keeps one partial sum per kernel tap in registers
// (all K * K input loads of a position issued together, taps outside the input adding -0.0f);
// fixed-order wave sums (oxh::wave_sums_rows) and a fixed-order sum over the waves combine them
// (deterministic; within fp32 rounding of the CPU's (n, oy, ox) running sum).  One launch, in
// place of batch-chunk partials and their sum.
template <int K, int Threads>
__global__ __launch_bounds__(Threads) void conv2d_depthwise_weight_kernel(
    ConvGeom g, oxh::FastDiv oplane_div, const float *__restrict__ grad,
    const float *__restrict__ x, float *__restrict__ weight_gradient) {
  constexpr int kTaps = K * K, kWaves = Threads / 64;
  __shared__ float wave_sums[kWaves][kTaps];
  const uint32_t c = blockIdx.x;
  const uint32_t oplane = g.oh * g.ow, plane = g.h * g.w;
  const uint32_t positions = g.batch * oplane;
  float acc[kTaps];
#pragma unroll
  for (int t = 0; t < kTaps; ++t) acc[t] = 0.0f;
  for (uint32_t j = threadIdx.x; j < positions; j += Threads) {
    const uint32_t n = fdiv(j, oplane_div), r = j - n * oplane;
    const uint32_t oy = fdiv(r, g.ow_div), ox = r - oy * g.ow;
    const float gv = grad[(n * g.out_c + c) * oplane + r];
    const float *xp = x + (n * g.in_c + c) * plane;
    const int by = static_cast<int>(oy * g.stride) - static_cast<int>(g.pad);
    const int bx = static_cast<int>(ox * g.stride) - static_cast<int>(g.pad);
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
    for (int t = 0; t < kTaps; ++t) wave_sums[wave][t] = acc[t];
  }
  __syncthreads();
  if (threadIdx.x < kTaps) {
    const int t = threadIdx.x;
    float v = wave_sums[0][t];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) v += wave_sums[w][t];
    weight_gradient[c * kTaps + t] = v;
  }
}

// Bias gradient: one wave per output channel.  Lane l adds the channel's terms l, l + 64, ...
// of the (n, oy, ox) order in fp32; a fixed xor butterfly combines the 64 lane sums
// (deterministic; within fp32 rounding of the CPU's single running sum).  Block b of 256
// threads covers channels 4b .. 4b + 3.
struct BiasArgs {
  const float *grad;
  float *out;
  uint32_t batch, out_c, plane;
  oxh::FastDiv plane_div;
};
__device__ __forceinline__ void bias_block(const BiasArgs &a, uint32_t b) {
  const uint32_t oc = b * 4 + threadIdx.x / 64;
  if (oc >= a.out_c) return;  // wave-uniform
  const uint32_t lane = threadIdx.x % 64, total = a.batch * a.plane;
  float acc = 0.0f;
#pragma unroll 4
  for (uint32_t j = lane; j < total; j += 64) {
    const uint32_t n = fdiv(j, a.plane_div), p = j - n * a.plane;
    acc += a.grad[(n * a.out_c + oc) * a.plane + p];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) a.out[oc] = acc;
}
__global__ __launch_bounds__(256) void conv2d_bias_kernel(BiasArgs a) { bias_block(a, blockIdx.x); }
uint32_t bias_blocks(uint32_t out_c) { return (out_c + 3) / 4; }
BiasArgs bias_args(const ConvGeom &g, const float *gradient, float *bias_gradient) {
  return BiasArgs{gradient, bias_gradient, g.batch, g.out_c, g.oh * g.ow,
                  oxh::make_fastdiv(g.oh * g.ow)};
}

// Weight gradient, phase 2: out[e] = sum over chunks of partial[chunk][e] in a fixed order
// (oxh::sum_chunks_block); elements e >= split go to out2[e - split].
__global__ __launch_bounds__(256) void sum_chunks_kernel(uint32_t count, uint32_t chunks,
                                                         uint32_t lanes,
                                                         const float *__restrict__ partial,
                                                         float *__restrict__ out, uint32_t split,
                                                         float *__restrict__ out2) {
  __shared__ float part[256];
  oxh::sum_chunks_block(blockIdx.x, count, chunks, lanes, partial, out, split, out2, part);
}


// ---------------------------------------------------------------- pointwise product

// Offset of index i along one operand axis: (i / p) * outer + (i % p) * inner.
struct Axis {
  oxh::FastDiv p;
  uint32_t outer, inner;
};

__device__ __forceinline__ uint32_t axis_offset(const Axis &a, uint32_t i) {
  const uint32_t q = fdiv(i, a.p);
  return q * a.outer + (i - q * a.p.d) * a.inner;
}

// Element (r, k) of an operand lies at ptr[offset(row, r) + offset(k, k)].  k_fast: consecutive
// threads load consecutive k (the operand is contiguous along k), else consecutive rows.
struct Operand {
  const float *ptr;
  Axis row, k;
  bool k_fast;
};

struct ProductArgs {
  Operand a, b;       // a: (m, k); b: (n, k)
  float *c;           // c[chunk * c_chunk + offset(cm, m) + offset(cn, n)]
  Axis cm, cn;
  uint32_t c_chunk;
  const float *init;  // initial value per m (the bias), or null for 0
  const float *addend;  // added to each finished sum (indexed as c; one chunk only), or null
  uint32_t M, N, K, k_chunk;
};

// Tilings of the product, each with one serial sum per output: 32 x 32 outputs per 256-thread
// block (2 x 2 per thread) for grids that fill the chip; for small grids, where the serial k
// chain of each thread sets the time, 8 x 8 outputs per 64-thread block (one per thread: a
// quarter of the chain work per thread, four times the blocks, and one wave per CU rather than
// four sharing its LDS), or 16 x 16 per 256 threads with OXH_TINY_TILE=16.
// k per LDS stage of the 32 x 32 tiling: 64 keeps a block's two slabs at ~19 KB (8 blocks per
// CU), where 128-k slabs (~35 KB, 4 per CU) put config 5's largest weight gradient (1200
// blocks) in two rounds of blocks.
#ifndef OXH_TILE32_SLAB
#define OXH_TILE32_SLAB 64
#endif
#ifndef OXH_SMALL_SLAB
#define OXH_SMALL_SLAB 128  // k per LDS stage of the small-grid tilings
#endif
constexpr int kTile = 32;  // the tiling of large grids

template <int Tile, int Threads>
struct TileShape {
  static constexpr int kCols = Threads == 256 ? 16 : 8;       // threads per tile row
  static constexpr int kMicro = Tile / kCols;                  // outputs per thread per axis
  static constexpr int kSlab =  // k per LDS stage
      Tile == kTile ? OXH_TILE32_SLAB : (Tile == 16 && Threads == 64 ? 64 : OXH_SMALL_SLAB);
  static constexpr int kLoads = Tile * kSlab / Threads;        // per thread, per operand
  static_assert(kCols * kCols == Threads && kMicro * kCols == Tile, "tile shape");
  static_assert(Threads % kSlab == 0 || kSlab % Threads == 0, "slab");
};

// One operand's share of a slab load (element e = thread + u * Threads of the slab's
// Tile x kSlab values).  k-fast operands (contiguous along k): e = r * kSlab + kk, so a thread
// keeps kKCols k columns and visits its rows in order; row-fast ones: e = kk * Tile + r, the
// thread's row is fixed and its k step by Threads / Tile.  Row offsets are computed once per
// block.  A load outside the operand reads element 0 instead (no branch per load) and its value
// is never used: the arithmetic stops at the slab's k count, and rows past M or N only feed
// outputs that are not stored.
template <int Tile, int Threads, bool KFast>
struct SlabLoader {
  using S = TileShape<Tile, Threads>;
  static constexpr int kLoads = S::kLoads, kSlab = S::kSlab;
  static constexpr int kKCols = KFast && kSlab > Threads ? kSlab / Threads : 1;
  static constexpr int kRows = KFast ? kLoads / kKCols : 1;  // distinct rows per thread
  static constexpr int kRowStep = KFast ? (kSlab > Threads ? 1 : Threads / kSlab) : 0;
  static constexpr int kKStep = KFast ? Threads : Threads / Tile;
  uint32_t row_off[kRows];
  uint32_t row_ok;  // bit i: row i inside the operand
  int r, kk;        // first (row, k) of the thread

  __device__ __forceinline__ SlabLoader(const Operand &o, uint32_t r0, uint32_t rows, int t) {
    r = KFast ? (kSlab > Threads ? 0 : t / kSlab) : t % Tile;
    kk = KFast ? t % kSlab : t / Tile;
    row_ok = 0;
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      const uint32_t row = r0 + r + i * kRowStep;
      const bool ok = row < rows;
      row_off[i] = ok ? axis_offset(o.row, row) : 0;
      row_ok |= ok ? (1u << i) : 0u;
    }
  }

  // load u: row index u / kKCols, k column u % kKCols (k-fast); k step u (row-fast)
  __device__ __forceinline__ void fetch(const Operand &o, uint32_t k0, uint32_t kc,
                                        float (&v)[kLoads]) const {
    if constexpr (KFast) {
      uint32_t koff[kKCols];
      bool k_ok[kKCols];
#pragma unroll
      for (int j = 0; j < kKCols; ++j) {
        const uint32_t k = static_cast<uint32_t>(kk + j * kKStep);
        k_ok[j] = k < kc;
        koff[j] = axis_offset(o.k, k0 + k);
      }
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        const int i = u / kKCols, j = u % kKCols;
        const bool ok = k_ok[j] && ((row_ok >> i) & 1u);
        v[u] = o.ptr[ok ? row_off[i] + koff[j] : 0];
      }
    } else if (o.k.p.d == 1) {
      // a linear k axis (offset k * outer, the common case): no division per load; the
      // branch is uniform (kernel argument)
      const uint32_t base = row_off[0] + (k0 + static_cast<uint32_t>(kk)) * o.k.outer;
      const uint32_t step = static_cast<uint32_t>(kKStep) * o.k.outer;
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        const uint32_t k = static_cast<uint32_t>(kk + u * kKStep);
        const bool ok = (row_ok & 1u) && k < kc;
        v[u] = o.ptr[ok ? base + static_cast<uint32_t>(u) * step : 0];
      }
    } else {
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        const uint32_t k = static_cast<uint32_t>(kk + u * kKStep);
        const bool ok = (row_ok & 1u) && k < kc;
        v[u] = o.ptr[ok ? row_off[0] + axis_offset(o.k, k0 + k) : 0];
      }
    }
  }

  // LDS tile rows hold k contiguously (s[row][k], rows of kRow floats) so the product reads
  // four k of a row as one 128-bit access.
  template <int kRow>
  __device__ __forceinline__ void stage(const float (&v)[kLoads], float (*s)[kRow]) const {
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      if constexpr (KFast)
        s[r + (u / kKCols) * kRowStep][kk + (u % kKCols) * kKStep] = v[u];
      else
        s[r][kk + u * kKStep] = v[u];
    }
  }
};

// LDS rows of a tiling: kSlab k plus one group of read-ahead, padded by 4 floats (rows start
// in different banks; 16-byte alignment kept).
template <int Tile, int Threads>
struct ProductRow {
  using S = TileShape<Tile, Threads>;
  static constexpr int kG4 = S::kMicro == 1 ? 4 : 2;  // float4 per row per group (16 or 8 k)
  static constexpr int kGroupK = 4 * kG4;
  static constexpr int value = S::kSlab + kGroupK + 4;
};

// sum_{k in [kb, ke), ascending} A[m, k] * B[n, k] added to acc, one serial fp32 sum per
// output (each product rounded, then added: -ffp-contract=off), for the tile at rows m0 (of A)
// and n0 (of B), computed by the Threads threads t = 0 .. Threads - 1 with the LDS operand tiles
// as and bs.  `slabs` stages run (at least ceil((ke - kb) / kSlab); later ones are empty), each
// with two block-wide barriers, so groups of threads sharing a block run equal counts.  Within a
// slab, groups of kG4 float4 (4 k each) per row are read from LDS as 128-bit accesses, the next
// group's reads issued before the current group's arithmetic.
// Fma: each term is added by one fused multiply-add (one rounding in place of the CPU path's
// two: sums that need not follow the CPU path bit for bit -- the weight gradients and the
// split forward -- at half the VALU work).
template <int Tile, int Threads, bool AKFast, bool BKFast, bool Fma = false, int D = 1>
__device__ __forceinline__ void product_sum(
    const ProductArgs &g, uint32_t m0, uint32_t n0, uint32_t kb, uint32_t ke, uint32_t slabs,
    int t, float (&acc)[TileShape<Tile, Threads>::kMicro][TileShape<Tile, Threads>::kMicro],
    float (*as)[ProductRow<Tile, Threads>::value], float (*bs)[ProductRow<Tile, Threads>::value]) {
  using S = TileShape<Tile, Threads>;
  constexpr int kMicro = S::kMicro, kLoads = S::kLoads, kSlab = S::kSlab, kCols = S::kCols;
  constexpr int kG4 = ProductRow<Tile, Threads>::kG4;
  constexpr int kGroupK = ProductRow<Tile, Threads>::kGroupK;
  const int tx = t % kCols, ty = t / kCols;
  const SlabLoader<Tile, Threads, AKFast> la(g.a, m0, g.M, t);
  const SlabLoader<Tile, Threads, BKFast> lb(g.b, n0, g.N, t);
  // a ring of D register slabs: slab s is staged from set s % D, whose loads were issued D
  // slabs earlier
  float va[D][kLoads], vb[D][kLoads];
#pragma unroll
  for (int slot = 0; slot < D; ++slot) {
    const uint32_t k0 = kb + slot * kSlab;
    if (k0 < ke) {
      const uint32_t kc = min(ke - k0, static_cast<uint32_t>(kSlab));
      la.fetch(g.a, k0, kc, va[slot]);
      lb.fetch(g.b, k0, kc, vb[slot]);
    }
  }
  float4 a0[kMicro][kG4], b0[kMicro][kG4], a1[kMicro][kG4], b1[kMicro][kG4];
  auto read_group = [&](uint32_t k, float4 (&av)[kMicro][kG4], float4 (&bv)[kMicro][kG4]) {
#pragma unroll
    for (int i = 0; i < kMicro; ++i)
#pragma unroll
      for (int q = 0; q < kG4; ++q) {
        av[i][q] = *reinterpret_cast<const float4 *>(&as[ty * kMicro + i][k + 4 * q]);
        bv[i][q] = *reinterpret_cast<const float4 *>(&bs[tx * kMicro + i][k + 4 * q]);
      }
  };
  // the group's products first, then each accumulator's adds in ascending k (the adds form
  // the dependent chain; the products stay off it)
  auto add_group = [&](const float4 (&av)[kMicro][kG4], const float4 (&bv)[kMicro][kG4]) {
    if constexpr (Fma) {
#pragma unroll
      for (int q = 0; q < kG4; ++q)
#pragma unroll
        for (int i = 0; i < kMicro; ++i)
#pragma unroll
          for (int j = 0; j < kMicro; ++j) {
            acc[i][j] = __builtin_fmaf(av[i][q].x, bv[j][q].x, acc[i][j]);
            acc[i][j] = __builtin_fmaf(av[i][q].y, bv[j][q].y, acc[i][j]);
            acc[i][j] = __builtin_fmaf(av[i][q].z, bv[j][q].z, acc[i][j]);
            acc[i][j] = __builtin_fmaf(av[i][q].w, bv[j][q].w, acc[i][j]);
          }
      return;
    }
    float p[kMicro][kMicro][4 * kG4];
#pragma unroll
    for (int q = 0; q < kG4; ++q)
#pragma unroll
      for (int i = 0; i < kMicro; ++i)
#pragma unroll
        for (int j = 0; j < kMicro; ++j) {
          p[i][j][4 * q] = av[i][q].x * bv[j][q].x;
          p[i][j][4 * q + 1] = av[i][q].y * bv[j][q].y;
          p[i][j][4 * q + 2] = av[i][q].z * bv[j][q].z;
          p[i][j][4 * q + 3] = av[i][q].w * bv[j][q].w;
        }
#pragma unroll
    for (int u = 0; u < 4 * kG4; ++u)
#pragma unroll
      for (int i = 0; i < kMicro; ++i)
#pragma unroll
        for (int j = 0; j < kMicro; ++j) acc[i][j] += p[i][j][u];
  };
  for (uint32_t s0 = 0; s0 < slabs; s0 += D) {
#pragma unroll
    for (int slot = 0; slot < D; ++slot) {
      const uint32_t s = s0 + slot;
      if (s >= slabs) break;  // block-uniform
      const uint32_t k0 = kb + s * kSlab;
      const uint32_t kc = k0 < ke ? min(ke - k0, static_cast<uint32_t>(kSlab)) : 0;
      if (kc > 0) {
        la.stage(va[slot], as);
        lb.stage(vb[slot], bs);
      }
      __syncthreads();
      const uint32_t k1 = k0 + D * kSlab;
      if (k1 < ke) {  // the next slab's loads overlap this slab's arithmetic
        const uint32_t kc1 = min(ke - k1, static_cast<uint32_t>(kSlab));
        la.fetch(g.a, k1, kc1, va[slot]);
        lb.fetch(g.b, k1, kc1, vb[slot]);
      }
      // whole groups, two per iteration so the read-ahead alternates register sets; a group read
      // starts at k <= kSlab, inside the row
      const uint32_t full = kc / kGroupK * kGroupK;
      uint32_t kk = 0;
      if (full > 0) read_group(0, a0, b0);
      while (kk < full) {
        read_group(kk + kGroupK, a1, b1);
        add_group(a0, b0);
        kk += kGroupK;
        if (kk >= full) break;
        read_group(kk + kGroupK, a0, b0);
        add_group(a1, b1);
        kk += kGroupK;
      }
      for (; kk < kc; ++kk) {
        float av[kMicro], bv[kMicro];
#pragma unroll
        for (int i = 0; i < kMicro; ++i) av[i] = as[ty * kMicro + i][kk];
#pragma unroll
        for (int j = 0; j < kMicro; ++j) bv[j] = bs[tx * kMicro + j][kk];
#pragma unroll
        for (int i = 0; i < kMicro; ++i)
#pragma unroll
          for (int j = 0; j < kMicro; ++j) {
            if constexpr (Fma) acc[i][j] = __builtin_fmaf(av[i], bv[j], acc[i][j]);
            else acc[i][j] += av[i] * bv[j];
          }
      }
      __syncthreads();
    }
  }
}

#ifndef OXH_SPLIT_MFMA
#define OXH_SPLIT_MFMA 1  // 1: the 16 x 16 split tiles sum on the matrix cores
#endif
#ifndef OXH_RING16
#define OXH_RING16 2  // register slabs in flight in the 16 x 16 split tiles' matrix-core sums
#endif
#ifndef OXH_RING32
#define OXH_RING32 1  // ... and in the 32 x 32 tiles'
#endif
#ifndef OXH_RING8
#define OXH_RING8 2  // ... and in the 8 x 8 split tiles'
#endif
#ifndef OXH_RING_SERIAL
#define OXH_RING_SERIAL 1  // ... and in the serial tiles' sums
#endif
#ifndef OXH_TILE32_MFMA
#define OXH_TILE32_MFMA 1  // 1: the 32 x 32 tiles' fused-multiply-add sums on the matrix cores
#endif

// A tile's sum over [kb, ke) on the matrix cores: the Threads threads (t = 0 .. Threads - 1)
// stage Tile x kSlab slabs of both operands as product_sum<Tile, Threads> does (same loads,
// staging and barriers), and wave w = t / 64 sums the 16 x 16 quadrant (w / (Tile / 16),
// w % (Tile / 16)) of the tile.  v_mfma_f32_16x16x4_f32 takes A[i][k] from lane i + 16 k and
// B[k][j] from lane j + 16 k and leaves D[i][j] in lane j + 16 (i / 4), register i % 4 (the
// layout acc uses).  Per 16 k, lane (i, q) reads A[i][k + 4q .. 4q + 3] and B's row i likewise
// as 128-bit LDS accesses and issues four MFMAs, the s-th with component s, so lane group q
// supplies k + 4q + s: the 16 k of the group, each once.  k at or past the slab's count are
// zeroed in both operands.  Each MFMA adds its four products to the accumulator with fused
// roundings: for sums that need not follow the CPU path bit for bit (within 1e-5 * sum|terms|
// of it), as the fused-multiply-add sums they replace.
template <int Tile, int Threads, bool AKFast, bool BKFast, int D = 1>
__device__ __forceinline__ void product_sum_mfma(const ProductArgs &g, uint32_t m0, uint32_t n0,
                                                 uint32_t kb, uint32_t ke, uint32_t slabs, int t,
                                                 f32x4_t &acc,
                                                 float (*as)[ProductRow<Tile, Threads>::value],
                                                 float (*bs)[ProductRow<Tile, Threads>::value]) {
  using S = TileShape<Tile, Threads>;
  constexpr int kLoads = S::kLoads, kSlab = S::kSlab, kQuads = Tile / 16;
  static_assert(Threads == 64 * kQuads * kQuads, "one wave per 16 x 16 quadrant");
  static_assert(kSlab % 16 == 0 && kSlab + 4 <= ProductRow<Tile, Threads>::value, "mfma slab");
  const SlabLoader<Tile, Threads, AKFast> la(g.a, m0, g.M, t);
  const SlabLoader<Tile, Threads, BKFast> lb(g.b, n0, g.N, t);
  // a ring of D register slabs: slab s is staged from set s % D, whose loads were issued D
  // slabs earlier (each slab's global loads take about a memory round trip)
  float va[D][kLoads], vb[D][kLoads];
#pragma unroll
  for (int slot = 0; slot < D; ++slot) {
    const uint32_t k0 = kb + slot * kSlab;
    if (k0 < ke) {
      const uint32_t kc = min(ke - k0, static_cast<uint32_t>(kSlab));
      la.fetch(g.a, k0, kc, va[slot]);
      lb.fetch(g.b, k0, kc, vb[slot]);
    }
  }
  const int w = t / 64, lane = t % 64;
  const int ia = 16 * (w / kQuads) + lane % 16, ib = 16 * (w % kQuads) + lane % 16;
  const int q = lane / 16;
  for (uint32_t s0 = 0; s0 < slabs; s0 += D) {
#pragma unroll
    for (int slot = 0; slot < D; ++slot) {
      const uint32_t s = s0 + slot;
      if (s >= slabs) break;  // block-uniform
      const uint32_t k0 = kb + s * kSlab;
      const uint32_t kc = k0 < ke ? min(ke - k0, static_cast<uint32_t>(kSlab)) : 0;
      if (kc > 0) {
        la.stage(va[slot], as);
        lb.stage(vb[slot], bs);
      }
      __syncthreads();
      const uint32_t k1 = k0 + D * kSlab;
      if (k1 < ke) {
        const uint32_t kc1 = min(ke - k1, static_cast<uint32_t>(kSlab));
        la.fetch(g.a, k1, kc1, va[slot]);
        lb.fetch(g.b, k1, kc1, vb[slot]);
      }
      for (uint32_t kk = 0; kk < kc; kk += 16) {
        float4 a = *reinterpret_cast<const float4 *>(&as[ia][kk + 4 * q]);
        float4 b = *reinterpret_cast<const float4 *>(&bs[ib][kk + 4 * q]);
        if (kk + 16 > kc) {
          const uint32_t k = kk + 4 * static_cast<uint32_t>(q);
          if (k >= kc) a.x = b.x = 0.0f;
          if (k + 1 >= kc) a.y = b.y = 0.0f;
          if (k + 2 >= kc) a.z = b.z = 0.0f;
          if (k + 3 >= kc) a.w = b.w = 0.0f;
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, acc, 0, 0, 0);
      }
      __syncthreads();
    }
  }
}

#ifndef OXH_SPLIT8_MFMA
#define OXH_SPLIT8_MFMA 1  // 1: the 8 x 8 split tiles sum on the matrix cores
#endif

// An 8 x 8 tile's sum over [kb, ke) on the matrix cores (one wave, t = lane), with slab loads,
// staging and barriers as product_sum<8, 64>.  v_mfma_f32_4x4x1f32 runs 16 independent 4 x 4
// outer products: block b takes A_b[i] from lane 4 b + i and B_b[j] from lane 4 b + j and
// leaves D_b[i][j] in lane 4 b + j, register i.  Block b = 4 d + p sums quadrant d (rows
// 4 (d / 2) .. + 3, columns 4 (d % 2) .. + 3) over the k of phase p: per 16 k, lane (b, i)
// reads A's row 4 (d / 2) + i at k + 4p .. 4p + 3 (and B's row 4 (d % 2) + i) as 128-bit LDS
// accesses and issues four MFMAs, the c-th with component c (k + 4p + c).  k at or past the
// slab's count are zeroed in both operands.  acc[i] of lane 4 b + j: phase p's sum for output
// (4 (d / 2) + i, 4 (d % 2) + j) of the tile.
template <bool AKFast, bool BKFast, int D = 1>
__device__ __forceinline__ void product_sum_mfma8(const ProductArgs &g, uint32_t m0, uint32_t n0,
                                                  uint32_t kb, uint32_t ke, uint32_t slabs,
                                                  int t, f32x4_t &acc,
                                                  float (*as)[ProductRow<8, 64>::value],
                                                  float (*bs)[ProductRow<8, 64>::value]) {
  using S = TileShape<8, 64>;
  constexpr int kLoads = S::kLoads, kSlab = S::kSlab;
  static_assert(kSlab % 16 == 0 && kSlab + 4 <= ProductRow<8, 64>::value, "mfma slab");
  const SlabLoader<8, 64, AKFast> la(g.a, m0, g.M, t);
  const SlabLoader<8, 64, BKFast> lb(g.b, n0, g.N, t);
  // a ring of D register slabs: slab s is staged from set s % D, whose loads were issued D
  // slabs earlier
  float va[D][kLoads], vb[D][kLoads];
#pragma unroll
  for (int slot = 0; slot < D; ++slot) {
    const uint32_t k0 = kb + slot * kSlab;
    if (k0 < ke) {
      const uint32_t kc = min(ke - k0, static_cast<uint32_t>(kSlab));
      la.fetch(g.a, k0, kc, va[slot]);
      lb.fetch(g.b, k0, kc, vb[slot]);
    }
  }
  const int d = t / 16, p = (t / 4) % 4, i = t % 4;
  const int ra = 4 * (d / 2) + i, rb = 4 * (d % 2) + i;
  for (uint32_t s0 = 0; s0 < slabs; s0 += D) {
#pragma unroll
    for (int slot = 0; slot < D; ++slot) {
      const uint32_t s = s0 + slot;
      if (s >= slabs) break;  // block-uniform
      const uint32_t k0 = kb + s * kSlab;
      const uint32_t kc = k0 < ke ? min(ke - k0, static_cast<uint32_t>(kSlab)) : 0;
      if (kc > 0) {
        la.stage(va[slot], as);
        lb.stage(vb[slot], bs);
      }
      __syncthreads();
      const uint32_t k1 = k0 + D * kSlab;
      if (k1 < ke) {
        const uint32_t kc1 = min(ke - k1, static_cast<uint32_t>(kSlab));
        la.fetch(g.a, k1, kc1, va[slot]);
        lb.fetch(g.b, k1, kc1, vb[slot]);
      }
      for (uint32_t kk = 0; kk < kc; kk += 16) {
        float4 a = *reinterpret_cast<const float4 *>(&as[ra][kk + 4 * p]);
        float4 b = *reinterpret_cast<const float4 *>(&bs[rb][kk + 4 * p]);
        if (kk + 16 > kc) {
          const uint32_t k = kk + 4 * static_cast<uint32_t>(p);
          if (k >= kc) a.x = b.x = 0.0f;
          if (k + 1 >= kc) a.y = b.y = 0.0f;
          if (k + 2 >= kc) a.z = b.z = 0.0f;
          if (k + 3 >= kc) a.w = b.w = 0.0f;
        }
        acc = __builtin_amdgcn_mfma_f32_4x4x1f32(a.x, b.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_4x4x1f32(a.y, b.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_4x4x1f32(a.z, b.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_4x4x1f32(a.w, b.w, acc, 0, 0, 0);
      }
      __syncthreads();
    }
  }
}

// Output (m, n) of chunk bz: c[bz * c_chunk + offset(cm, m) + offset(cn, n)] = sum (+ addend).
__device__ __forceinline__ void product_store(const ProductArgs &g, uint32_t bz, uint32_t m,
                                              uint32_t n, float sum, float added) {
  if (m >= g.M || n >= g.N) return;
  float *c = g.c + static_cast<uint64_t>(bz) * g.c_chunk;
  c[axis_offset(g.cm, m) + axis_offset(g.cn, n)] = g.addend != nullptr ? sum + added : sum;
}

// C[m, n] = init[m] + sum_{k in chunk bz, ascending} A[m, k] * B[n, k] (+ addend) for the tile
// (bx, by): one serial sum per output, computed by the block's Threads threads.
template <int Tile, int Threads, bool AKFast, bool BKFast, bool Fma = false>
__device__ __forceinline__ void product_tile(const ProductArgs &g, uint32_t bx, uint32_t by,
                                             uint32_t bz,
                                             float (*as)[ProductRow<Tile, Threads>::value],
                                             float (*bs)[ProductRow<Tile, Threads>::value]) {
  using S = TileShape<Tile, Threads>;
  constexpr int kMicro = S::kMicro, kCols = S::kCols;
  const uint32_t m0 = by * Tile, n0 = bx * Tile;
  const uint32_t kb = bz * g.k_chunk;
  const uint32_t ke = min(kb + g.k_chunk, g.K);
  const int t = static_cast<int>(threadIdx.x), tx = t % kCols, ty = t / kCols;
  if constexpr (Fma && Tile == kTile && Threads == 256 && OXH_TILE32_MFMA != 0) {
    // wave w sums quadrant (w / 2, w % 2); lane l holds outputs
    // (m0 + 16 (w / 2) + 4 (l / 16) + r, n0 + 16 (w % 2) + l % 16), r = 0 .. 3
    const int w = t / 64, l = t % 64;
    const uint32_t mq = m0 + 16 * static_cast<uint32_t>(w / 2) + 4 * static_cast<uint32_t>(l / 16);
    const uint32_t n = n0 + 16 * static_cast<uint32_t>(w % 2) + static_cast<uint32_t>(l % 16);
    f32x4_t acc;
    float added[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t m = mq + r;
      acc[r] = g.init != nullptr && m < g.M ? g.init[m] : 0.0f;
      added[r] = g.addend != nullptr && m < g.M && n < g.N
                     ? g.addend[axis_offset(g.cm, m) + axis_offset(g.cn, n)]
                     : 0.0f;
    }
    const uint32_t slabs = kb < ke ? (ke - kb + S::kSlab - 1) / S::kSlab : 0;
    product_sum_mfma<Tile, Threads, AKFast, BKFast, OXH_RING32>(g, m0, n0, kb, ke, slabs, t, acc,
                                                                as, bs);
#pragma unroll
    for (int r = 0; r < 4; ++r) product_store(g, bz, mq + r, n, acc[r], added[r]);
    return;
  }
  float acc[kMicro][kMicro];
#pragma unroll
  for (int i = 0; i < kMicro; ++i) {
    const uint32_t m = m0 + ty * kMicro + i;
    const float v = (g.init != nullptr && m < g.M) ? g.init[m] : 0.0f;
#pragma unroll
    for (int j = 0; j < kMicro; ++j) acc[i][j] = v;
  }
  // the addend is loaded now, with the first slab (after the k loop it would add a memory
  // round trip to the block)
  float added[kMicro][kMicro];
#pragma unroll
  for (int i = 0; i < kMicro; ++i)
#pragma unroll
    for (int j = 0; j < kMicro; ++j) {
      const uint32_t m = m0 + ty * kMicro + i, n = n0 + tx * kMicro + j;
      added[i][j] = g.addend != nullptr && m < g.M && n < g.N
                        ? g.addend[axis_offset(g.cm, m) + axis_offset(g.cn, n)]
                        : 0.0f;
    }
  const uint32_t slabs = kb < ke ? (ke - kb + S::kSlab - 1) / S::kSlab : 0;
  product_sum<Tile, Threads, AKFast, BKFast, Fma, OXH_RING_SERIAL>(g, m0, n0, kb, ke, slabs, t,
                                                                   acc, as, bs);
#pragma unroll
  for (int i = 0; i < kMicro; ++i)
#pragma unroll
    for (int j = 0; j < kMicro; ++j)
      product_store(g, bz, m0 + ty * kMicro + i, n0 + tx * kMicro + j, acc[i][j], added[i][j]);
}

template <int Tile, int Threads, bool AKFast, bool BKFast, bool Fma = false>
__global__ __launch_bounds__(Threads) void pointwise_product_kernel(ProductArgs g) {
  constexpr int kRow = ProductRow<Tile, Threads>::value;
  __shared__ __align__(16) float as[Tile][kRow];
  __shared__ __align__(16) float bs[Tile][kRow];
  const oxh::BlockTile bt = oxh::xcd_block();
  product_tile<Tile, Threads, AKFast, BKFast, Fma>(g, bt.x, bt.y, bt.z, as, bs);
}

// Products whose sums need not follow the serial order (the weight gradient, already reduced in
// k chunks; the forward of a small pointwise convolution): an 8 x 8 tile per kSplitWaves-wave
// block, wave w summing the w-th contiguous part of the chunk's k range serially (wave 0 from
// the initial value), the parts then added in wave order, then the addend.  Four times the
// waves of the one-wave tile and a quarter of its serial chain.
constexpr int kSplitWaves = 4;
constexpr int kSplitThreads = 64 * kSplitWaves;
struct SplitLds {
  float as[kSplitWaves][8][ProductRow<8, 64>::value];
  float bs[kSplitWaves][8][ProductRow<8, 64>::value];
  float part[kSplitWaves][64];
};

template <bool AKFast, bool BKFast>
__device__ __forceinline__ void split_tile(const ProductArgs &g, uint32_t bx, uint32_t by,
                                           uint32_t bz, SplitLds &lds) {
  constexpr int kSlab = TileShape<8, 64>::kSlab;
  const uint32_t m0 = by * 8, n0 = bx * 8;
  const uint32_t kb = bz * g.k_chunk;
  const uint32_t ke = min(kb + g.k_chunk, g.K);
  const uint32_t span = kb < ke ? ke - kb : 0;
  const uint32_t part = (span + kSplitWaves - 1) / kSplitWaves;
  const int w = static_cast<int>(threadIdx.x) / 64, t = static_cast<int>(threadIdx.x) % 64;
  const uint32_t wb = min(kb + w * part, ke), we = min(wb + part, ke);
  const uint32_t slabs = (part + kSlab - 1) / kSlab;  // equal for every wave (barriers)
  const uint32_t m = m0 + t / 8, n = n0 + t % 8;
  if constexpr (OXH_SPLIT8_MFMA != 0) {
    const float init = w == 0 && g.init != nullptr && m < g.M ? g.init[m] : 0.0f;
    const float added = w == 0 && g.addend != nullptr && m < g.M && n < g.N
                            ? g.addend[axis_offset(g.cm, m) + axis_offset(g.cn, n)]
                            : 0.0f;
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    product_sum_mfma8<AKFast, BKFast, OXH_RING8>(g, m0, n0, wb, we, slabs, t, acc, lds.as[w],
                                                 lds.bs[w]);
    // the four k phases of a quadrant (lanes 16 d + 4 p + j, p = 0 .. 3), added as
    // (p0 + p1) + (p2 + p3); lanes of phase 0 then hold the wave's part of the quadrant
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      acc[r] += __shfl_xor(acc[r], 4);
      acc[r] += __shfl_xor(acc[r], 8);
    }
    if ((t / 4) % 4 == 0) {
      const int d = t / 16, j = t % 4;
#pragma unroll
      for (int r = 0; r < 4; ++r) lds.part[w][(4 * (d / 2) + r) * 8 + 4 * (d % 2) + j] = acc[r];
    }
    __syncthreads();
    if (w > 0) return;
    float sum = init;
#pragma unroll
    for (int q = 0; q < kSplitWaves; ++q) sum += lds.part[q][t];
    product_store(g, bz, m, n, sum, added);
    return;
  }
  float acc[1][1] = {{w == 0 && g.init != nullptr && m < g.M ? g.init[m] : 0.0f}};
  const float added = w == 0 && g.addend != nullptr && m < g.M && n < g.N
                          ? g.addend[axis_offset(g.cm, m) + axis_offset(g.cn, n)]
                          : 0.0f;
  product_sum<8, 64, AKFast, BKFast, true>(g, m0, n0, wb, we, slabs, t, acc, lds.as[w],
                                           lds.bs[w]);
  if (w > 0) lds.part[w - 1][t] = acc[0][0];
  __syncthreads();
  if (w > 0) return;
  float sum = acc[0][0];
#pragma unroll
  for (int q = 0; q < kSplitWaves - 1; ++q) sum += lds.part[q][t];
  product_store(g, bz, m, n, sum, added);
}

template <bool AKFast, bool BKFast>
__global__ __launch_bounds__(kSplitThreads) void pointwise_split_kernel(ProductArgs g) {
  __shared__ __align__(16) SplitLds lds;
  const oxh::BlockTile bt = oxh::xcd_block();
  split_tile<AKFast, BKFast>(g, bt.x, bt.y, bt.z, lds);
}

// The split tiles at 16 x 16 outputs, 2 x 2 per lane (product_sum<16, 64>): the same parts of
// k in the same order per output as split_tile, half the operand reads per product (grids of
// many 8 x 8 tiles are bound by those reads).
struct SplitLds16 {
  float as[kSplitWaves][16][ProductRow<16, 64>::value];
  float bs[kSplitWaves][16][ProductRow<16, 64>::value];
  float part[kSplitWaves - 1][4][64];
};

template <bool AKFast, bool BKFast>
__device__ __forceinline__ void split_tile16(const ProductArgs &g, uint32_t bx, uint32_t by,
                                             uint32_t bz, SplitLds16 &lds) {
  using S = TileShape<16, 64>;
  constexpr int kMicro = S::kMicro, kCols = S::kCols;
  const uint32_t m0 = by * 16, n0 = bx * 16;
  const uint32_t kb = bz * g.k_chunk;
  const uint32_t ke = min(kb + g.k_chunk, g.K);
  const uint32_t span = kb < ke ? ke - kb : 0;
  const uint32_t part = (span + kSplitWaves - 1) / kSplitWaves;
  const int w = static_cast<int>(threadIdx.x) / 64, t = static_cast<int>(threadIdx.x) % 64;
  const int tx = t % kCols, ty = t / kCols;
  const uint32_t wb = min(kb + w * part, ke), we = min(wb + part, ke);
  const uint32_t slabs = (part + S::kSlab - 1) / S::kSlab;  // equal for every wave (barriers)
  if constexpr (OXH_SPLIT_MFMA != 0) {
    // lane t holds outputs (m0 + 4 (t / 16) + r, n0 + t % 16), r = 0 .. 3
    const uint32_t n = n0 + static_cast<uint32_t>(t % 16);
    f32x4_t acc;
    float added[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t m = m0 + 4 * static_cast<uint32_t>(t / 16) + r;
      acc[r] = w == 0 && g.init != nullptr && m < g.M ? g.init[m] : 0.0f;
      added[r] = w == 0 && g.addend != nullptr && m < g.M && n < g.N
                     ? g.addend[axis_offset(g.cm, m) + axis_offset(g.cn, n)]
                     : 0.0f;
    }
    product_sum_mfma<16, 64, AKFast, BKFast, OXH_RING16>(g, m0, n0, wb, we, slabs, t, acc,
                                                         lds.as[w], lds.bs[w]);
    if (w > 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) lds.part[w - 1][r][t] = acc[r];
    }
    __syncthreads();
    if (w > 0) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float sum = acc[r];
#pragma unroll
      for (int p = 0; p < kSplitWaves - 1; ++p) sum += lds.part[p][r][t];
      product_store(g, bz, m0 + 4 * static_cast<uint32_t>(t / 16) + r, n, sum, added[r]);
    }
    return;
  }
  float acc[kMicro][kMicro], added[kMicro][kMicro];
#pragma unroll
  for (int i = 0; i < kMicro; ++i)
#pragma unroll
    for (int j = 0; j < kMicro; ++j) {
      const uint32_t m = m0 + ty * kMicro + i, n = n0 + tx * kMicro + j;
      acc[i][j] = w == 0 && g.init != nullptr && m < g.M ? g.init[m] : 0.0f;
      added[i][j] = w == 0 && g.addend != nullptr && m < g.M && n < g.N
                        ? g.addend[axis_offset(g.cm, m) + axis_offset(g.cn, n)]
                        : 0.0f;
    }
  product_sum<16, 64, AKFast, BKFast, true>(g, m0, n0, wb, we, slabs, t, acc, lds.as[w],
                                            lds.bs[w]);
  if (w > 0) {
#pragma unroll
    for (int i = 0; i < kMicro; ++i)
#pragma unroll
      for (int j = 0; j < kMicro; ++j) lds.part[w - 1][i * kMicro + j][t] = acc[i][j];
  }
  __syncthreads();
  if (w > 0) return;
#pragma unroll
  for (int i = 0; i < kMicro; ++i)
#pragma unroll
    for (int j = 0; j < kMicro; ++j) {
      float sum = acc[i][j];
#pragma unroll
      for (int q = 0; q < kSplitWaves - 1; ++q) sum += lds.part[q][i * kMicro + j][t];
      product_store(g, bz, m0 + ty * kMicro + i, n0 + tx * kMicro + j, sum, added[i][j]);
    }
}

template <bool AKFast, bool BKFast>
__global__ __launch_bounds__(kSplitThreads) void pointwise_split16_kernel(ProductArgs g) {
  __shared__ __align__(16) SplitLds16 lds;
  const oxh::BlockTile bt = oxh::xcd_block();
  split_tile16<AKFast, BKFast>(g, bt.x, bt.y, bt.z, lds);
}

// A convolution's input gradient (16 x 16 serial tiles, one output per thread, or with Split1
// the 16 x 16 split tiles its own launch takes for that shape: g1) and weight gradient (8 x 8
// split tiles, or 16 x 16 with S2 == 2, as its own launch takes them: g2) in one launch.  Blocks
// [0, blocks1) take the input gradient's tiles, dispatched first (their chains over the output
// channels are the longer ones), the rest the weight gradient's, each computed exactly as its
// own kernel computes it.
struct DualGrid {
  uint32_t nx1, ny1, blocks1, nx2, ny2, blocks2;
  BiasArgs bias;  // bias.out null: no bias blocks
};

struct SerialTileLds16 {
  float as[16][ProductRow<16, 256>::value];
  float bs[16][ProductRow<16, 256>::value];
};
// The paired launch's LDS: the tiles of the kinds it takes (input gradient S1, weight gradient
// S2) and only those, so each pairing keeps its occupancy.
struct NoLds {};
template <int S1, int S2>
union DualLds {
  SplitLds split;
  std::conditional_t<S1 == 0, SerialTileLds16, NoLds> tile;
  std::conditional_t<S1 == 2 || S2 == 2, SplitLds16, NoLds> split16;
};

template <bool A1, bool B1, bool A2, bool B2, int S1 = 0, int S2 = 0>
__global__ __launch_bounds__(kSplitThreads) void pointwise_dual_kernel(ProductArgs g1,
                                                                       ProductArgs g2,
                                                                       DualGrid d) {
  __shared__ __align__(16) DualLds<S1, S2> lds;
  uint32_t b = blockIdx.x;
  // each part's tiles remapped on their own, so every XCD keeps a share of both parts
  if (b < d.blocks1)
    b = oxh::xcd_contiguous(b, d.blocks1);
  else if (b < d.blocks1 + d.blocks2)
    b = d.blocks1 + oxh::xcd_contiguous(b - d.blocks1, d.blocks2, d.blocks1);
  if (b < d.blocks1) {
    if constexpr (S1 == 2)
      split_tile16<A1, B1>(g1, b % d.nx1, b / d.nx1, 0, lds.split16);
    else if constexpr (S1 == 1)
      split_tile<A1, B1>(g1, b % d.nx1, b / d.nx1, 0, lds.split);
    else
      product_tile<16, 256, A1, B1>(g1, b % d.nx1, b / d.nx1, 0, lds.tile.as, lds.tile.bs);
  } else if (b < d.blocks1 + d.blocks2) {
    b -= d.blocks1;
    const uint32_t plane = d.nx2 * d.ny2, z = b / plane, r = b - z * plane;
    if constexpr (S2 == 2)
      split_tile16<A2, B2>(g2, r % d.nx2, r / d.nx2, z, lds.split16);
    else
      split_tile<A2, B2>(g2, r % d.nx2, r / d.nx2, z, lds.split);
  } else {
    bias_block(d.bias, b - d.blocks1 - d.blocks2);
  }
}

// ---------------------------------------------------------------- pooling

struct PoolGeom {
  uint32_t batch, channels, h, w, kh, kw, sh, sw, oh, ow;
  oxh::FastDiv ow_div, oh_div, w_div, h_div, sh_div, sw_div;
  float denominator;
};

// evaluation.rs:414-444: window sum in (ky, kx) order divided by the window area.
__global__ __launch_bounds__(256) void avg_pool2d_forward_kernel(PoolGeom g, uint32_t total,
                                                                 const float *__restrict__ x,
                                                                 float *__restrict__ y) {
  for (uint32_t o = blockIdx.x * 256 + threadIdx.x; o < total; o += gridDim.x * 256) {
    const uint32_t t0 = fdiv(o, g.ow_div), ox = o - t0 * g.ow;
    const uint32_t plane = fdiv(t0, g.oh_div), oy = t0 - plane * g.oh;
    const float *xp = x + plane * g.h * g.w + oy * g.sh * g.w + ox * g.sw;
    float sum = 0.0f;
    for (uint32_t ky = 0; ky < g.kh; ++ky)
      for (uint32_t kx = 0; kx < g.kw; ++kx) sum += xp[ky * g.w + kx];
    y[o] = sum / g.denominator;
  }
}

// autograd.rs:501-525: each output adds g / area to every input of its window; gathered here per
// input element in (oy, ox) ascending order.
__global__ __launch_bounds__(256) void avg_pool2d_backward_kernel(PoolGeom g, uint32_t total,
                                                                  const float *__restrict__ grad,
                                                                  float *__restrict__ dx) {
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
    const uint32_t t0 = fdiv(i, g.w_div), ix = i - t0 * g.w;
    const uint32_t plane = fdiv(t0, g.h_div), iy = t0 - plane * g.h;
    const float *gp = grad + plane * g.oh * g.ow;
    // outputs oy with oy * sh <= iy < oy * sh + kh
    const int oy0 = ceil_div0(static_cast<int>(iy) - static_cast<int>(g.kh) + 1, g.sh_div);
    const int ox0 = ceil_div0(static_cast<int>(ix) - static_cast<int>(g.kw) + 1, g.sw_div);
    const int oy1 = min(floor_div(static_cast<int>(iy), g.sh_div), static_cast<int>(g.oh) - 1);
    const int ox1 = min(floor_div(static_cast<int>(ix), g.sw_div), static_cast<int>(g.ow) - 1);
    float acc = 0.0f;
    for (int oy = oy0; oy <= oy1; ++oy)
      for (int ox = ox0; ox <= ox1; ++ox)
        acc += gp[oy * static_cast<int>(g.ow) + ox] / g.denominator;
    dx[i] = acc;
  }
}

// ---------------------------------------------------------------- host side

uint32_t grid_for(uint64_t items) {
  uint64_t g = (items + 255) / 256;
  if (g < 1) g = 1;
  if (g > (1u << 20)) g = 1u << 20;
  return static_cast<uint32_t>(g);
}

// The chunk sums of a convolution backward whose caller takes them over (a training program
// launching every convolution's sums at once): while set, launch_sum_chunks records its sum
// here in place of launching it.
thread_local std::vector<oxh::ChunkSum> *deferred_sums = nullptr;

// Elements at or past `split` (default: none) go to out2.
void launch_sum_chunks(hipStream_t s, uint32_t count, uint32_t chunks, const void *partial,
                       float *out, uint32_t split = UINT32_MAX, float *out2 = nullptr) {
  if (split > count) split = count;
  if (deferred_sums != nullptr) {
    deferred_sums->push_back(
        oxh::ChunkSum{static_cast<const float *>(partial), out, out2, count, chunks, split});
    return;
  }
  const uint32_t lanes = oxh::chunk_sum_lanes(chunks);
  const uint32_t per_block = 256 / lanes;
  oxh::launch(sum_chunks_kernel, dim3((count + per_block - 1) / per_block), dim3(256), 0, s,
              count, chunks, lanes, static_cast<const float *>(partial), out, split, out2);
}

uint64_t input_elems(const ConvGeom &g) {
  return static_cast<uint64_t>(g.batch) * g.in_c * g.h * g.w;
}
uint64_t output_elems(const ConvGeom &g) {
  return static_cast<uint64_t>(g.batch) * g.out_c * g.oh * g.ow;
}
uint64_t weight_elems(const ConvGeom &g) {
  return static_cast<uint64_t>(g.out_c) * g.in_per_group * g.kh * g.kw;
}

oxh_status make_conv_geom(const char *name, const oxh_conv2d_shape *s, ConvGeom &g) {
  OXH_REQUIRE(s != nullptr, OXH_INVALID_SHAPE, std::string(name) + ": null shape");
  const uint64_t v[] = {s->batch, s->in_channels, s->height, s->width, s->out_channels,
                        s->kernel_h, s->kernel_w, s->stride, s->groups};
  for (uint64_t d : v)
    OXH_REQUIRE(d > 0 && d < (1ull << 31), OXH_INVALID_SHAPE,
                std::string(name) + ": dimensions must be in 1..2^31");
  OXH_REQUIRE(s->padding < (1ull << 20), OXH_INVALID_SHAPE, std::string(name) + ": padding");
  // nn.rs:257-264: channels divisible by groups
  OXH_REQUIRE(s->in_channels % s->groups == 0 && s->out_channels % s->groups == 0,
              OXH_INVALID_SHAPE,
              std::string(name) + ": invalid Conv2d channel, group, or kernel configuration");
  OXH_REQUIRE(s->height + 2 * s->padding >= s->kernel_h &&
                  s->width + 2 * s->padding >= s->kernel_w,
              OXH_INVALID_SHAPE, std::string(name) + ": kernel larger than the padded input");
  // every tensor, and the index ranges the kernels form, below 2^31
  const uint64_t in_n = s->batch * s->in_channels * s->height * s->width;
  const uint64_t oh = (s->height + 2 * s->padding - s->kernel_h) / s->stride + 1;
  const uint64_t ow = (s->width + 2 * s->padding - s->kernel_w) / s->stride + 1;
  const uint64_t out_n = s->batch * s->out_channels * oh * ow;
  const uint64_t w_n = s->out_channels * (s->in_channels / s->groups) * s->kernel_h * s->kernel_w;
  const uint64_t sizes[] = {s->batch * s->in_channels, s->batch * s->out_channels, in_n, out_n,
                            w_n, s->height + s->padding + s->kernel_h,
                            s->width + s->padding + s->kernel_w};
  for (uint64_t n : sizes)
    OXH_REQUIRE(n < kMaxElems, OXH_INVALID_SHAPE,
                std::string(name) + ": tensors are limited to 2^31 elements");
  g.batch = static_cast<uint32_t>(s->batch);
  g.in_c = static_cast<uint32_t>(s->in_channels);
  g.h = static_cast<uint32_t>(s->height);
  g.w = static_cast<uint32_t>(s->width);
  g.out_c = static_cast<uint32_t>(s->out_channels);
  g.kh = static_cast<uint32_t>(s->kernel_h);
  g.kw = static_cast<uint32_t>(s->kernel_w);
  g.stride = static_cast<uint32_t>(s->stride);
  g.pad = static_cast<uint32_t>(s->padding);
  g.groups = static_cast<uint32_t>(s->groups);
  g.oh = static_cast<uint32_t>(oh);
  g.ow = static_cast<uint32_t>(ow);
  g.in_per_group = g.in_c / g.groups;
  g.out_per_group = g.out_c / g.groups;
  g.ow_div = oxh::make_fastdiv(g.ow);
  g.oh_div = oxh::make_fastdiv(g.oh);
  g.oc_div = oxh::make_fastdiv(g.out_c);
  g.w_div = oxh::make_fastdiv(g.w);
  g.h_div = oxh::make_fastdiv(g.h);
  g.ic_div = oxh::make_fastdiv(g.in_c);
  g.s_div = oxh::make_fastdiv(g.stride);
  g.ipg_div = oxh::make_fastdiv(g.in_per_group);
  g.opg_div = oxh::make_fastdiv(g.out_per_group);
  g.kw_div = oxh::make_fastdiv(g.kw);
  g.kh_div = oxh::make_fastdiv(g.kh);
  return oxh::ok();
}

// Square 3 x 3 or 5 x 5 kernels with stride 1 or 2 take the tap-unrolled direct kernels:
// returns 10 * K + S, or 0 for the generic ones.
int tap_kernel(const ConvGeom &g) {
  if (g.kh != g.kw || (g.kh != 3 && g.kh != 5) || (g.stride != 1 && g.stride != 2)) return 0;
  return static_cast<int>(10 * g.kh + g.stride);
}

// Plans of the LDS-staged per-image kernels: `tile` channels per block (0: not applicable).
struct LdsPlan {
  uint32_t tile = 0, tiles = 0, chunks = 1, per_chunk = 0, lds_bytes = 0;
  uint32_t groups = 1, threads = 256;  // weight gradient position ranges; block size
};

bool lds_eligible(const ConvGeom &g) {
  return g.groups == 1 && tap_kernel(g) != 0 && g.batch <= 65535;
}

// `staged` floats per block plus `per` per tile channel (tiles of kLdsR-channel groups,
// weights padded to a multiple of kLdsR), over `channels` channels of `plane` positions: about
// one group per thread per block, in blocks of as many 64-thread waves as their items fill (at
// most 256 threads).  Every item is a serial sum, so the tiling never changes a result.
LdsPlan channel_tiles(uint64_t staged, uint64_t per, uint64_t channels, uint64_t plane) {
  LdsPlan p;
  staged = (staged + 3) / 4 * 4;
  if (staged + kLdsR * per > kLdsFloats) return p;
  const uint64_t fit = (kLdsFloats - staged) / per / kLdsR * kLdsR;
  uint64_t groups = 256 / plane;
  if (groups < 1) groups = 1;
  uint64_t tile = groups * kLdsR;
  const uint64_t all = (channels + kLdsR - 1) / kLdsR * kLdsR;
  if (tile > all) tile = all;
  if (tile > fit) tile = fit;
  const uint64_t items = tile / kLdsR * plane;
  p.tile = static_cast<uint32_t>(tile);
  p.tiles = static_cast<uint32_t>((channels + tile - 1) / tile);
  p.threads = static_cast<uint32_t>(items >= 256 ? 256 : (items + 63) / 64 * 64);
  p.lds_bytes = static_cast<uint32_t>((staged + tile * per) * 4);
  return p;
}

LdsPlan forward_lds_plan(const ConvGeom &g) {
  if (!lds_eligible(g)) return LdsPlan{};
  const uint64_t taps = g.kh * g.kw;
  return channel_tiles(static_cast<uint64_t>(g.in_c) * g.h * g.w, g.in_c * taps, g.out_c,
                       static_cast<uint64_t>(g.oh) * g.ow);
}

// The split forward: output planes of at most 64 positions, at least 4 input channels per
// part, the serial kernel's grid under 2048 waves (most of the chip idle); tiles of as many
// kLdsR-channel groups as fill 64 items (one per position and group), threads kFwdParts * items
// rounded to waves.  tile == 0: not taken.
#ifndef OXH_FWD_SPLIT
#define OXH_FWD_SPLIT 1  // 0: every K x K forward takes the serial kernels
#endif
LdsPlan forward_split_plan(const ConvGeom &g) {
  LdsPlan p;
  const uint64_t oplane = static_cast<uint64_t>(g.oh) * g.ow;
  if (!OXH_FWD_SPLIT || !lds_eligible(g) || oplane > 64 || g.in_c < 4 * kFwdParts) return p;
  const LdsPlan serial = forward_lds_plan(g);
  if (serial.tile > 0 &&
      static_cast<uint64_t>(serial.tiles) * g.batch * ((serial.threads + 63) / 64) >= 2048)
    return p;
  uint64_t groups = 64 / oplane;
  const uint64_t all = (g.out_c + kLdsR - 1) / kLdsR;
  if (groups > all) groups = all;
  const uint64_t tile = groups * kLdsR, items = groups * oplane;
  const uint64_t taps = static_cast<uint64_t>(g.kh) * g.kw;
  const uint64_t floats = (static_cast<uint64_t>(g.in_c) * g.h * g.w + 3) / 4 * 4 +
                          (g.in_c * taps * tile + 3) / 4 * 4 + (kFwdParts - 1) * items * kLdsR;
  if (floats > kLdsFloats) return p;
  p.tile = static_cast<uint32_t>(tile);
  p.tiles = static_cast<uint32_t>((g.out_c + tile - 1) / tile);
  p.groups = static_cast<uint32_t>(items);  // items per block
  p.threads = static_cast<uint32_t>((kFwdParts * items + 63) / 64 * 64);
  p.lds_bytes = static_cast<uint32_t>(floats * 4);
  return p;
}

// The matrix-core forward takes the split forward's shapes (output planes of <= 64 positions)
// whose input channels are a multiple of 4: blocks of 256 threads over (16-channel tile, image),
// the halo-padded image, the tile's weights and the parts' partial sums within the LDS budget.
// lds_bytes == 0: not taken.
#ifndef OXH_FWD_MFMA
#define OXH_FWD_MFMA 1  // 0: the split forward keeps its fused-multiply-add kernel
#endif
struct MfmaForwardPlan {
  MfmaForward f{};
  uint32_t tiles = 0, lds_bytes = 0;
};
MfmaForwardPlan forward_mfma_plan(const ConvGeom &g) {
  MfmaForwardPlan p;
  if (!OXH_FWD_MFMA || g.in_c % 4 != 0 || forward_split_plan(g).tile == 0) return p;
  MfmaForward &f = p.f;
  f.hp = (g.oh - 1) * g.stride + g.kh;
  f.wp = (g.ow - 1) * g.stride + g.kw;
  f.cs = f.hp * f.wp | 1u;  // odd: the four input-channel lane groups start in different banks
  const uint32_t P = g.oh * g.ow;
  f.pos_tiles = (P + 15) / 16;  // at most 4: the split forward's planes hold <= 64 positions
  f.kparts = f.pos_tiles >= 3 ? 1 : 4 / f.pos_tiles;
  f.oc_tile = 16;
  f.ocs = 16;
  const uint64_t image = round4(g.in_c * f.cs), rows = static_cast<uint64_t>(g.in_c) * g.kh * g.kw;
  const uint64_t red = f.kparts > 1 ? static_cast<uint64_t>(f.kparts - 1) * f.pos_tiles * 256 : 0;
  if (f.pos_tiles > 4 || image + rows * f.ocs + red > kLdsFloats) return p;
  f.plane_div = oxh::make_fastdiv(g.h * g.w);
  f.rows_div = oxh::make_fastdiv(static_cast<uint32_t>(rows));
  p.tiles = (g.out_c + f.oc_tile - 1) / f.oc_tile;
  p.lds_bytes = static_cast<uint32_t>((image + rows * f.ocs + red) * 4);
  return p;
}

// The matrix-core stride-2 input gradient: ungrouped K x K convolutions whose halo-padded
// output gradient and 16-channel weight tile fit the LDS budget.  The halo (lo, the padded
// extents) covers every output position any tap of any input position reads, found by
// enumerating them.  lds_bytes == 0: not taken.
#ifndef OXH_IG_MFMA
#define OXH_IG_MFMA 1  // 0: stride-2 input gradients keep the serial phase-blocked kernel
#endif
struct MfmaIgPlan {
  MfmaIg f{};
  uint32_t tiles = 0, lds_bytes = 0;
};
MfmaIgPlan input_backward_mfma_plan(const ConvGeom &g) {
  MfmaIgPlan p;
  if (!OXH_IG_MFMA || !lds_eligible(g) || g.stride != 2) return p;
  const int K = static_cast<int>(g.kh), pad = static_cast<int>(g.pad);
  auto extent = [&](uint32_t size, uint32_t out, uint32_t &lo, uint32_t &padded) {
    int mn = 0, mx = static_cast<int>(out) - 1;
    for (int i = 0; i < static_cast<int>(size); ++i)
      for (int k = 0; k < K; ++k)
        if (((i + pad - k) & 1) == 0) {
          const int o = (i + pad - k) / 2;
          mn = o < mn ? o : mn;
          mx = o > mx ? o : mx;
        }
    lo = static_cast<uint32_t>(-mn);
    padded = static_cast<uint32_t>(mx - mn + 1);
  };
  MfmaIg &f = p.f;
  extent(g.h, g.oh, f.lo_y, f.ohp);
  extent(g.w, g.ow, f.lo_x, f.owp);
  f.ocp = round4(g.out_c);
  f.ocs = (f.ocp / 4) % 2 == 0 ? f.ocp + 4 : f.ocp;
  const uint64_t floats = static_cast<uint64_t>(f.ohp) * f.owp * f.ocs +
                          static_cast<uint64_t>(g.kh) * g.kw * f.ocp * 16;
  if (floats > kLdsFloats) return p;
  p.tiles = (g.in_c + 15) / 16;
  p.lds_bytes = static_cast<uint32_t>(floats * 4);
  return p;
}

LdsPlan input_backward_lds_plan(const ConvGeom &g) {
  if (!lds_eligible(g)) return LdsPlan{};
  const uint64_t taps = g.kh * g.kw;
  return channel_tiles(static_cast<uint64_t>(g.out_c) * g.oh * g.ow, g.out_c * taps, g.in_c,
                       static_cast<uint64_t>(g.h) * g.w);
}

// The phase-blocked stride-2 input gradient: input channels per block for about 256
// (channel, phase block) items, the halo-padded gradient planes and the tile's weights within
// the LDS budget.  lds_bytes == 0: not taken.
#ifndef OXH_IG_PHASE
#define OXH_IG_PHASE 1  // 0: stride-2 input gradients take the candidate kernels
#endif
struct PhasePlan {
  PhaseGeom pg{};
  uint32_t tiles = 0, threads = 0, lds_bytes = 0;
};
PhasePlan input_backward_s2_plan(const ConvGeom &g) {
  PhasePlan p;
  if (!OXH_IG_PHASE || !lds_eligible(g) || g.stride != 2) return p;
  const uint32_t K = g.kh, M = (K + 1) / 2;
  PhaseGeom &h = p.pg;
  h.a0 = g.pad / 2;
  const uint32_t ay = (g.h - 1 + g.pad) / 2, ax = (g.w - 1 + g.pad) / 2;
  h.na = ay - h.a0 + 1;
  h.nb = ax - h.a0 + 1;
  h.lo = M - 1 > h.a0 ? M - 1 - h.a0 : 0;
  h.ohp = h.lo + (g.oh > ay + 1 ? g.oh : ay + 1);
  h.owp = h.lo + (g.ow > ax + 1 ? g.ow : ax + 1);
  h.ocp = round4(g.out_c);
  h.ocs = (h.ocp / 4) % 2 == 0 ? h.ocp + 4 : h.ocp;
  h.ocw = h.ocp + ((36 - h.ocp % 32) % 32);  // 4 mod 32: conflict-free 128-bit weight stores
  const uint64_t blocks_ab = static_cast<uint64_t>(h.na) * h.nb;
  uint64_t tile = blocks_ab >= 256 ? 1 : 256 / blocks_ab;
  if (tile > g.in_c) tile = g.in_c;
  // smaller tiles where the grid would leave the chip with one block per CU or fewer
  while (tile > 1 && (g.in_c + tile - 1) / tile * static_cast<uint64_t>(g.batch) < 512)
    tile = (tile + 1) / 2;
  const uint64_t gfloats = static_cast<uint64_t>(h.ohp) * h.owp * h.ocs;
  const uint64_t per_ic = static_cast<uint64_t>(K) * K * h.ocw;
  while (tile > 1 && gfloats + tile * per_ic > kLdsFloats) --tile;
  const uint64_t floats = gfloats + tile * per_ic;
  if (floats > kLdsFloats) return p;
  h.ic_tile = static_cast<uint32_t>(tile);
  h.ab_div = oxh::make_fastdiv(static_cast<uint32_t>(blocks_ab));
  h.nb_div = oxh::make_fastdiv(h.nb);
  const uint64_t items = tile * blocks_ab;
  p.tiles = static_cast<uint32_t>((g.in_c + tile - 1) / tile);
  p.threads = static_cast<uint32_t>(items >= 256 ? 256 : (items + 63) / 64 * 64);
  p.lds_bytes = static_cast<uint32_t>(floats * 4);
  return p;
}

// Weight gradient: one thread per (ic, tap) pair and position range (pairs <= kDwMaxThreads;
// ranges so that a block has about 256 threads), the image planes plus a full output-channel
// tile (or the range sums) within the LDS budget; image chunks for about 512 blocks.
// bias: the launch also sums the bias gradient (groups more threads, same ranges); tile == 0
// when that does not fit (the weight plan alone does not depend on it).
LdsPlan weight_lds_plan(const ConvGeom &g, bool bias = false) {
  LdsPlan p;
  if (!lds_eligible(g)) return p;
  const uint64_t pairs = static_cast<uint64_t>(g.in_c) * g.kh * g.kw;
  const uint64_t oplane = static_cast<uint64_t>(g.oh) * g.ow;
  if (pairs > kDwMaxThreads) return p;
  uint64_t groups = 256 / pairs;
  if (groups < 1) groups = 1;
  if (groups > oplane) groups = oplane;
  const uint64_t items = (pairs + (bias ? 1 : 0)) * groups;
  if (items > kDwMaxThreads) return p;
  const uint64_t staged = static_cast<uint64_t>(g.in_c) * g.h * g.w + kDwOcTile * oplane;
  const uint64_t reduce = groups > 1 ? items * kDwOcTile : 0;
  const uint64_t floats = staged > reduce ? staged : reduce;
  if (floats > kLdsFloats) return p;
  p.tile = kDwOcTile;
  p.tiles = (g.out_c + kDwOcTile - 1) / kDwOcTile;
  p.groups = static_cast<uint32_t>(groups);
  p.threads = static_cast<uint32_t>((items + 63) / 64 * 64);
  uint32_t chunks = 512 / p.tiles;
  if (chunks < 1) chunks = 1;
  if (chunks > g.batch) chunks = g.batch;
  while (chunks > 1 && static_cast<uint64_t>(chunks) * weight_elems(g) >= kMaxElems) --chunks;
  p.per_chunk = (g.batch + chunks - 1) / chunks;
  p.chunks = (g.batch + p.per_chunk - 1) / p.per_chunk;
  p.lds_bytes = static_cast<uint32_t>(floats * 4);
  return p;
}

// The matrix-core weight gradient: ungrouped K x K convolutions whose image and gradient runs
// allow 16-byte loads (C * h * w and out_c * oh * ow multiples of 4) and whose chunk of ipc
// images (at least 32 positions) holds at most 256 positions; N tiles per job (1, 3, 6 or 9)
// for about OXH_WGT_JOB_MFMA MFMAs per wave; the images, the gradient and nothing else in LDS.
// bias: one more column, the bias gradient.  lds_bytes == 0: not taken.
#ifndef OXH_WGT_MFMA
#define OXH_WGT_MFMA 1  // 0: K x K weight gradients keep the LDS fused-multiply-add kernel
#endif
#ifndef OXH_WGT_JOB_MFMA
#define OXH_WGT_JOB_MFMA 80
#endif
struct MfmaWeightPlan {
  MfmaWeight f{};
  uint32_t chunks = 0, blocks = 0, lds_bytes = 0;
};
MfmaWeightPlan weight_mfma_plan(const ConvGeom &g, bool bias = false) {
  MfmaWeightPlan p;
  const uint64_t plane = static_cast<uint64_t>(g.h) * g.w, P = static_cast<uint64_t>(g.oh) * g.ow;
  if (!OXH_WGT_MFMA || !lds_eligible(g) || (g.in_c * plane) % 4 != 0 || (g.out_c * P) % 4 != 0 ||
      P > 256)
    return p;
  MfmaWeight &f = p.f;
  f.hp = (g.oh - 1) * g.stride + g.kh;
  f.wp = (g.ow - 1) * g.stride + g.kw;
  f.cs = f.hp * f.wp | 1u;
  uint64_t ipc = (32 + P - 1) / P;
  if (ipc > g.batch) ipc = g.batch;
  f.ipc = static_cast<uint32_t>(ipc);
  f.kpad = static_cast<uint32_t>(round4(static_cast<uint32_t>(ipc * P)));
  if (f.kpad > 256) return p;
  const uint32_t steps = f.kpad / 4;
  const uint32_t weights = g.in_c * g.kh * g.kw;
  f.bias = bias ? 1u : 0u;
  f.stride = static_cast<uint32_t>(weight_elems(g)) + (bias ? g.out_c : 0u);
  f.mtiles = (g.out_c + 15) / 16;
  f.ntiles = (weights + f.bias + 15) / 16;
  // N tiles per job: 1, 3, 6 or 9 (the kernel's instantiations), about OXH_WGT_JOB_MFMA MFMAs
  const uint32_t want = OXH_WGT_JOB_MFMA / steps;
  f.ng = f.ntiles == 1 ? 1 : want >= 9 ? 9 : want >= 6 ? 6 : 3;
  if (f.ng > 3 && (f.ntiles + 2) / 3 * 3 <= f.ng) f.ng = (f.ntiles + 2) / 3 * 3;  // small N
  f.ngroups = (f.ntiles + f.ng - 1) / f.ng;
  f.jobs = f.mtiles * f.ngroups;
  f.kparts = f.jobs <= 2 ? 4 / f.jobs : 1;
  const uint64_t floats = round4(static_cast<uint32_t>(ipc * g.in_c * f.cs)) +
                          static_cast<uint64_t>(f.mtiles) * 16 * f.kpad +
                          static_cast<uint64_t>(f.kparts - 1) * f.jobs * f.ng * 256;
  if (floats > kLdsFloats) return p;
  f.plane_div = oxh::make_fastdiv(static_cast<uint32_t>(plane));
  f.oplane_div = oxh::make_fastdiv(static_cast<uint32_t>(P));
  f.m_div = oxh::make_fastdiv(g.out_c);
  p.chunks = static_cast<uint32_t>((g.batch + ipc - 1) / ipc);
  if (p.chunks > 1 && static_cast<uint64_t>(p.chunks) * f.stride >= kMaxElems) return p;
  p.blocks = (f.jobs + 3) / 4;
  p.lds_bytes = static_cast<uint32_t>(floats * 4);
  return p;
}

// 1x1, stride 1, no padding, one group: the convolution is a matrix product over channels.
bool pointwise(const ConvGeom &g) {
  return g.kh == 1 && g.kw == 1 && g.stride == 1 && g.pad == 0 && g.groups == 1 &&
         (g.out_c + kTile - 1) / kTile <= 65535 && (g.in_c + kTile - 1) / kTile <= 65535;
}

Axis linear(uint32_t stride) { return Axis{oxh::make_fastdiv(1), stride, 0}; }
// (n, p) flattened with p < plane: offset n * (channels * plane) + p.
Axis batch_plane(uint32_t plane, uint32_t channels) {
  return Axis{oxh::make_fastdiv(plane), channels * plane, 1};
}
uint32_t unit_stride(const Axis &a) { return a.p.d == 1 ? a.outer : a.inner; }
Operand operand(const float *ptr, Axis row, Axis k) {
  return Operand{ptr, row, k, unit_stride(k) <= unit_stride(row)};
}


#ifndef OXH_SINGLE_K
#define OXH_SINGLE_K 1024  // weight gradients with at most this many k terms: one pass, no chunks
#endif

#ifndef OXH_TINY_TILE
#define OXH_TINY_TILE 8  // small-grid tiling: 8 (8 x 8, 64 threads) or 16 (16 x 16, 256)
#endif
#ifndef OXH_SMALL_GRID
#define OXH_SMALL_GRID 512  // below this many 32 x 32 blocks the small-grid tiling runs
#endif
constexpr uint64_t kSmallGrid = OXH_SMALL_GRID;

// k chunks of the pointwise weight gradient.  Grids of >= kSmallGrid 32 x 32 tiles (with their
// chunks: about 512 blocks, at least 64 k per chunk, when k > OXH_SINGLE_K) take the serial
// 32 x 32 tiling (serial32); smaller ones the split tiles, chunked for about OXH_SPLIT_TARGET
// waves with at least 4 * 128 k per chunk.  Every chunk is non-empty.
#ifndef OXH_SPLIT_TARGET
#define OXH_SPLIT_TARGET 512
#endif
struct KSplit {
  uint32_t chunks, per;
  bool serial32;
};
KSplit product_split(const ConvGeom &g) {
  const uint64_t tiles = static_cast<uint64_t>((g.out_c + kTile - 1) / kTile) *
                         ((g.in_c + kTile - 1) / kTile);
  const uint64_t k = static_cast<uint64_t>(g.batch) * g.h * g.w;
  const uint64_t weights = static_cast<uint64_t>(g.out_c) * g.in_c;
  uint64_t c = 1;
  if (k > OXH_SINGLE_K) {
    c = (512 + tiles - 1) / tiles;
    const uint64_t by_work = k / 64 > 0 ? k / 64 : 1;
    if (c > by_work) c = by_work;
    if (c > 1024) c = 1024;
  }
  bool serial32 = tiles * c >= kSmallGrid;
  if (!serial32) {
    const uint64_t tiles8 = static_cast<uint64_t>((g.out_c + 7) / 8) * ((g.in_c + 7) / 8);
    c = (OXH_SPLIT_TARGET + tiles8 * kSplitWaves - 1) / (tiles8 * kSplitWaves);
    const uint64_t by_work = k / (kSplitWaves * 128) > 0 ? k / (kSplitWaves * 128) : 1;
    if (c > by_work) c = by_work;
  }
  while (c > 1 && c * weights >= kMaxElems) --c;
  if (c < 1) c = 1;
  const uint64_t per = (k + c - 1) / c;
  return KSplit{static_cast<uint32_t>((k + per - 1) / per), static_cast<uint32_t>(per), serial32};
}


template <int Tile, int Threads, bool Fma = false>
void launch_tiled(hipStream_t s, const ProductArgs &a, uint32_t chunks) {
  const dim3 grid((a.N + Tile - 1) / Tile, (a.M + Tile - 1) / Tile, chunks);
  const dim3 block(Threads);
  if (a.a.k_fast && a.b.k_fast)
    oxh::launch(pointwise_product_kernel<Tile, Threads, true, true, Fma>, grid, block, 0, s, a);
  else if (a.a.k_fast)
    oxh::launch(pointwise_product_kernel<Tile, Threads, true, false, Fma>, grid, block, 0, s, a);
  else if (a.b.k_fast)
    oxh::launch(pointwise_product_kernel<Tile, Threads, false, true, Fma>, grid, block, 0, s, a);
  else
    oxh::launch(pointwise_product_kernel<Tile, Threads, false, false, Fma>, grid, block, 0, s,
                a);
}

template <bool A, bool B>
void launch_split(hipStream_t s, const ProductArgs &a, uint32_t chunks);

// Serial sums (one per output, the CPU path's order): grids of >= kSmallGrid 32 x 32 tiles take
// the 32 x 32 tiling, smaller ones the one-wave 8 x 8 tiles.  With `split`, grids of at most
// kSplitMaxTiles 8 x 8 tiles with at least kSplitMinK terms per sum take the split tiles
// instead (contiguous parts of k added in order: the same sum within a few roundings, a
// quarter of the serial chain, four times the waves of a grid that leaves most of the chip
// idle).
#ifndef OXH_SPLIT_MAX_TILES
#define OXH_SPLIT_MAX_TILES 512
#endif
constexpr uint64_t kSplitMaxTiles = OXH_SPLIT_MAX_TILES;
#ifndef OXH_SPLIT_MIN_K
#define OXH_SPLIT_MIN_K 256
#endif
constexpr uint32_t kSplitMinK = OXH_SPLIT_MIN_K;
// Which tiling a product that may split takes: 0 the serial tiles, 1 the split 8 x 8 tiles
// (grids of at most kSplitMaxTiles of them), 2 the split 16 x 16 tiles (larger grids, still
// under kSmallGrid 32 x 32 tiles: bound by operand reads, which 2 x 2 outputs per lane halve).
#ifndef OXH_SPLIT16
#define OXH_SPLIT16 1
#endif
int split_kind(uint32_t M, uint32_t N, uint32_t k_chunk, uint32_t chunks) {
  const uint64_t big =
      static_cast<uint64_t>((N + kTile - 1) / kTile) * ((M + kTile - 1) / kTile) * chunks;
  const uint64_t tiles8 = static_cast<uint64_t>((N + 7) / 8) * ((M + 7) / 8) * chunks;
  if (big >= kSmallGrid || k_chunk < kSplitMinK) return 0;
  if (tiles8 <= kSplitMaxTiles) return 1;
  return OXH_SPLIT16 ? 2 : 0;
}

// A pointwise input gradient over at least kSplitMinK output channels whose grid would leave
// the chip waiting on the serial chain of every output takes the split tiles of the forward's
// rule (split_kind: 0 serial, 1 split 8 x 8, 2 split 16 x 16), alone and in the paired launch.
#ifndef OXH_IG_SPLIT
#define OXH_IG_SPLIT 2  // the largest split kind the input gradient takes (0: always serial)
#endif
int input_splits(const ProductArgs &x) {
  const int kind = split_kind(x.M, x.N, x.k_chunk, 1);
  return kind <= OXH_IG_SPLIT ? kind : 0;
}

// One-wave 8 x 8 serial tiles hold ~9.5 KB of LDS each: 16 blocks per CU, 4096 on the chip at
// once.  A larger grid would run a second round of blocks; the 16 x 16 serial tiling (four
// waves, 8 blocks per CU, a quarter of the blocks) then takes it: the same sums (one serial
// chain per output in either tiling), one round fewer.
#ifndef OXH_TINY_ROUND
#define OXH_TINY_ROUND 4096  // 8 x 8 blocks per round (0: always 8 x 8)
#endif
bool tiny_grid_rounds(const ProductArgs &a, uint32_t chunks) {
  const uint64_t tiles8 = static_cast<uint64_t>((a.N + 7) / 8) * ((a.M + 7) / 8) * chunks;
  return OXH_TINY_ROUND > 0 && tiles8 > OXH_TINY_ROUND;
}

template <bool A, bool B>
void launch_split16(hipStream_t s, const ProductArgs &a, uint32_t chunks) {
  const dim3 grid((a.N + 15) / 16, (a.M + 15) / 16, chunks);
  oxh::launch(pointwise_split16_kernel<A, B>, grid, dim3(kSplitThreads), 0, s, a);
}

oxh_status launch_product(const char *name, hipStream_t s, const ProductArgs &a,
                          uint32_t chunks, bool split = false) {
  const int kind = split ? split_kind(a.M, a.N, a.k_chunk, chunks) : 0;
  const uint64_t big =
      static_cast<uint64_t>((a.N + kTile - 1) / kTile) * ((a.M + kTile - 1) / kTile) * chunks;
  const bool ak = a.a.k_fast, bk = a.b.k_fast;
  if (big >= kSmallGrid)
    launch_tiled<kTile, 256>(s, a, chunks);
  else if (kind == 1 && ak && bk)
    launch_split<true, true>(s, a, chunks);
  else if (kind == 1 && ak)
    launch_split<true, false>(s, a, chunks);
  else if (kind == 1 && bk)
    launch_split<false, true>(s, a, chunks);
  else if (kind == 1)
    launch_split<false, false>(s, a, chunks);
  else if (kind == 2 && ak && bk)
    launch_split16<true, true>(s, a, chunks);
  else if (kind == 2 && ak)
    launch_split16<true, false>(s, a, chunks);
  else if (kind == 2 && bk)
    launch_split16<false, true>(s, a, chunks);
  else if (kind == 2)
    launch_split16<false, false>(s, a, chunks);
  else if (OXH_TINY_TILE == 8 && !tiny_grid_rounds(a, chunks))
    launch_tiled<8, 64>(s, a, chunks);
  else
    launch_tiled<16, 256>(s, a, chunks);
  return oxh::launched(name);
}

// Batch chunks for the direct weight reduction: about 2^20 threads (short serial chains), at
// most one chunk per batch element.
uint32_t weight_chunks(const ConvGeom &g) {
  const uint64_t weights = weight_elems(g);
  uint64_t c = ((1ull << 20) + weights - 1) / weights;
  if (c > g.batch) c = g.batch;
  while (c > 1 && weights * c >= kMaxElems) --c;
  if (c < 1) c = 1;
  return static_cast<uint32_t>(c);
}
// Depthwise convolutions with 3 x 3 or 5 x 5 kernels take the one-block-per-channel weight
// gradient.
bool depthwise_single_pass(const ConvGeom &g) {
  return g.in_per_group == 1 && g.out_per_group == 1 && g.kh == g.kw &&
         (g.kh == 3 || g.kh == 5) && g.out_c <= 65535 * 16;
}

uint64_t weight_partial_bytes(const ConvGeom &g) {
  if (depthwise_single_pass(g)) return 0;
  // the matrix-core kernel's chunks, or the LDS kernel's with room for the bias sums of a
  // parameter-only oxh_conv2d_backward after each chunk's weights, or (operands the matrix-core
  // kernel does not take) the generic kernel's
  const MfmaWeightPlan mp = weight_mfma_plan(g, true);
  const uint64_t mbytes = mp.lds_bytes > 0 && mp.chunks > 1 ? mp.chunks * mp.f.stride * 4ull : 0;
  const LdsPlan lp = weight_lds_plan(g);
  if (lp.tile > 0) {
    const uint64_t lbytes = lp.chunks > 1 ? lp.chunks * (weight_elems(g) + g.out_c) * 4 : 0;
    return lbytes > mbytes ? lbytes : mbytes;
  }
  if (mp.lds_bytes > 0) {
    const uint64_t generic = weight_elems(g) * weight_chunks(g) * 4;
    return generic > mbytes ? generic : mbytes;
  }
  if (pointwise(g)) {
    const KSplit k = product_split(g);
    return k.chunks > 1 ? static_cast<uint64_t>(k.chunks) * g.out_c * g.in_c * 4 : 0;
  }
  return weight_elems(g) * weight_chunks(g) * 4;
}

oxh_status make_pool_geom(const char *name, const oxh_pool2d_shape *s, PoolGeom &g) {
  OXH_REQUIRE(s != nullptr, OXH_INVALID_SHAPE, std::string(name) + ": null shape");
  const uint64_t v[] = {s->batch, s->channels, s->height, s->width,
                        s->kernel_h, s->kernel_w, s->stride_h, s->stride_w};
  for (uint64_t d : v)
    OXH_REQUIRE(d > 0 && d < (1ull << 31), OXH_INVALID_SHAPE,
                std::string(name) + ": dimensions must be in 1..2^31");
  // tensor/mod.rs:236-250: the window must fit
  OXH_REQUIRE(s->kernel_h <= s->height && s->kernel_w <= s->width, OXH_INVALID_SHAPE,
              std::string(name) + ": avg_pool2d window exceeds the input");
  OXH_REQUIRE(s->batch * s->channels * s->height * s->width < kMaxElems &&
                  s->batch * s->channels < kMaxElems,
              OXH_INVALID_SHAPE, std::string(name) + ": tensors are limited to 2^31 elements");
  g.batch = static_cast<uint32_t>(s->batch);
  g.channels = static_cast<uint32_t>(s->channels);
  g.h = static_cast<uint32_t>(s->height);
  g.w = static_cast<uint32_t>(s->width);
  g.kh = static_cast<uint32_t>(s->kernel_h);
  g.kw = static_cast<uint32_t>(s->kernel_w);
  g.sh = static_cast<uint32_t>(s->stride_h);
  g.sw = static_cast<uint32_t>(s->stride_w);
  g.oh = (g.h - g.kh) / g.sh + 1;
  g.ow = (g.w - g.kw) / g.sw + 1;
  g.denominator = static_cast<float>(static_cast<uint64_t>(g.kh) * g.kw);
  g.ow_div = oxh::make_fastdiv(g.ow);
  g.oh_div = oxh::make_fastdiv(g.oh);
  g.w_div = oxh::make_fastdiv(g.w);
  g.h_div = oxh::make_fastdiv(g.h);
  g.sh_div = oxh::make_fastdiv(g.sh);
  g.sw_div = oxh::make_fastdiv(g.sw);
  return oxh::ok();
}

// dW[oc, ic] = sum_{(n, p)} G[oc, (n, p)] X[ic, (n, p)], k = (n, p) in split.per-sized chunks;
// c is the weight gradient (one chunk) or the chunk partials.
ProductArgs weight_product(const ConvGeom &g, const KSplit &split, const float *gradient,
                           const float *input, float *c) {
  const uint32_t plane = g.h * g.w;
  ProductArgs a{};
  a.a = operand(gradient, linear(plane), batch_plane(plane, g.out_c));
  a.b = operand(input, linear(plane), batch_plane(plane, g.in_c));
  a.c = c;
  a.cm = linear(g.in_c);
  a.cn = linear(1);
  a.c_chunk = g.out_c * g.in_c;
  a.init = nullptr;
  a.M = g.out_c;
  a.N = g.in_c;
  a.K = g.batch * plane;
  a.k_chunk = split.per;
  return a;
}

// dX[ic, (n, p)] = 0 + sum_oc W[oc, ic] G[(n, p), oc], plus the addend when given.
ProductArgs input_product(const ConvGeom &g, const float *gradient, const float *weight,
                          const float *addend, float *input_gradient) {
  const uint32_t plane = g.h * g.w;
  ProductArgs a{};
  a.a = operand(weight, linear(1), linear(g.in_c));
  a.b = operand(gradient, batch_plane(plane, g.out_c), linear(plane));
  a.c = input_gradient;
  a.cm = linear(plane);
  a.cn = batch_plane(plane, g.in_c);
  a.init = nullptr;
  a.addend = addend;
  a.M = g.in_c;
  a.N = g.batch * plane;
  a.K = g.out_c;
  a.k_chunk = a.K;
  return a;
}

uint64_t big_tiles(const ProductArgs &a, uint32_t chunks) {
  return static_cast<uint64_t>((a.N + kTile - 1) / kTile) * ((a.M + kTile - 1) / kTile) * chunks;
}

// The weight-gradient product: the serial 32 x 32 tiling or the split tiles (sums over
// contiguous parts of each chunk, added in order), as product_split chose.
template <bool A, bool B>
void launch_split(hipStream_t s, const ProductArgs &a, uint32_t chunks) {
  const dim3 grid((a.N + 7) / 8, (a.M + 7) / 8, chunks);
  oxh::launch(pointwise_split_kernel<A, B>, grid, dim3(kSplitThreads), 0, s, a);
}

// Weight gradients on split tiles whose 8 x 8 tiles (with their chunks) exceed
// OXH_WEIGHT_SPLIT16 take 16 x 16 split tiles, alone and in the paired launch: a quarter of the
// blocks (a paired launch then fits the chip in one round of blocks: its LDS allows 4 per CU)
// and half the operand reads per output.  0: always 8 x 8.
#ifndef OXH_WEIGHT_SPLIT16
#define OXH_WEIGHT_SPLIT16 512
#endif
bool weight_split16(const ProductArgs &a, uint32_t chunks) {
  const uint64_t tiles8 = static_cast<uint64_t>((a.N + 7) / 8) * ((a.M + 7) / 8) * chunks;
  return OXH_WEIGHT_SPLIT16 > 0 && tiles8 > OXH_WEIGHT_SPLIT16;
}

oxh_status launch_weight_product(const char *name, hipStream_t s, const ProductArgs &a,
                                 const KSplit &split) {
  const uint32_t chunks = split.chunks;
  const bool t16 = weight_split16(a, chunks);
  if (split.serial32) {
    launch_tiled<kTile, 256, true>(s, a, chunks);
  } else if (t16 && a.a.k_fast && a.b.k_fast) {
    launch_split16<true, true>(s, a, chunks);
  } else if (t16 && a.a.k_fast) {
    launch_split16<true, false>(s, a, chunks);
  } else if (t16 && a.b.k_fast) {
    launch_split16<false, true>(s, a, chunks);
  } else if (t16) {
    launch_split16<false, false>(s, a, chunks);
  } else if (a.a.k_fast && a.b.k_fast) {
    launch_split<true, true>(s, a, chunks);
  } else if (a.a.k_fast) {
    launch_split<true, false>(s, a, chunks);
  } else if (a.b.k_fast) {
    launch_split<false, true>(s, a, chunks);
  } else {
    launch_split<false, false>(s, a, chunks);
  }
  return oxh::launched(name);
}

// Both backward products of a pointwise convolution in one launch when together they stay
// below the small-grid threshold (the weight gradient alone would take the split tiles) and
// their operand layouts are the ones a convolution's planes give (plane > 1: weight gradient
// k-fast on both operands, input gradient row-fast on both; plane 1: weight gradient row-fast,
// input gradient k-fast on its second operand).  Every output is the same sum as in the
// separate launches (the input gradient's serial sum does not depend on the tiling).  Returns
// false, launching nothing, otherwise.
// The input gradient x (16 x 16 serial tiles), the weight gradient w (split tiles, per chunk)
// and, when bias.out is set, the bias gradient in one launch.
bool launch_dual(hipStream_t s, const ProductArgs &w, const KSplit &split, const ProductArgs &x,
                 const BiasArgs &bias) {
  if (split.serial32 || big_tiles(w, split.chunks) + big_tiles(x, 1) >= kSmallGrid)
    return false;
  const int s1 = input_splits(x);
  const bool t16 = weight_split16(w, split.chunks);
  const uint32_t t1 = s1 == 1 ? 8 : 16, t2 = t16 ? 16 : 8;  // the two products' tiles
  DualGrid d;
  d.nx1 = (x.N + t1 - 1) / t1;
  d.ny1 = (x.M + t1 - 1) / t1;
  d.blocks1 = d.nx1 * d.ny1;
  d.nx2 = (w.N + t2 - 1) / t2;
  d.ny2 = (w.M + t2 - 1) / t2;
  d.blocks2 = d.nx2 * d.ny2 * split.chunks;
  d.bias = bias;
  const uint32_t blocks3 = bias.out != nullptr ? bias_blocks(bias.out_c) : 0;
  const dim3 grid(d.blocks1 + d.blocks2 + blocks3), block(kSplitThreads);
#define OXH_DUAL(A1, B1, A2, B2)                                                             \
  do {                                                                                       \
    if (s1 == 2 && t16)                                                                      \
      oxh::launch(pointwise_dual_kernel<A1, B1, A2, B2, 2, 2>, grid, block, 0, s, x, w, d);  \
    else if (s1 == 2)                                                                        \
      oxh::launch(pointwise_dual_kernel<A1, B1, A2, B2, 2, 0>, grid, block, 0, s, x, w, d);  \
    else if (s1 == 1 && t16)                                                                 \
      oxh::launch(pointwise_dual_kernel<A1, B1, A2, B2, 1, 2>, grid, block, 0, s, x, w, d);  \
    else if (s1 == 1)                                                                        \
      oxh::launch(pointwise_dual_kernel<A1, B1, A2, B2, 1, 0>, grid, block, 0, s, x, w, d);  \
    else if (t16)                                                                            \
      oxh::launch(pointwise_dual_kernel<A1, B1, A2, B2, 0, 2>, grid, block, 0, s, x, w, d);  \
    else                                                                                     \
      oxh::launch(pointwise_dual_kernel<A1, B1, A2, B2, 0, 0>, grid, block, 0, s, x, w, d);  \
  } while (0)
  if (w.a.k_fast && w.b.k_fast && !x.a.k_fast && !x.b.k_fast)
    OXH_DUAL(false, false, true, true);
  else if (!w.a.k_fast && !w.b.k_fast && !x.a.k_fast && x.b.k_fast)
    OXH_DUAL(false, true, false, false);
  else
    return false;
#undef OXH_DUAL
  return true;
}

oxh_status input_backward_impl(const char *name, oxh_stream stream,
                               const oxh_conv2d_shape *shape, const float *gradient,
                               const float *weight, const float *addend,
                               float *input_gradient) {
  ConvGeom g;
  oxh_status st = make_conv_geom(name, shape, g);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(gradient && weight && input_gradient, OXH_INVALID_SHAPE,
              std::string(name) + ": null pointer");
  const uint64_t in_n = input_elems(g);
  // the addend may be input_gradient itself (each element is read before the same lane
  // writes it), never a part of it
  const uint64_t gx = in_n * 4;
  OXH_REQUIRE(!oxh::any_overlap(input_gradient, gx, gradient, output_elems(g) * 4) &&
                  !oxh::any_overlap(input_gradient, gx, weight, weight_elems(g) * 4),
              OXH_INVALID_SHAPE, std::string(name) + ": input_gradient overlaps an operand");
  OXH_REQUIRE(addend == nullptr || addend == input_gradient ||
                  !oxh::any_overlap(input_gradient, gx, addend, gx),
              OXH_INVALID_SHAPE, std::string(name) + ": addend partially overlaps input_gradient");
  hipStream_t s = oxh::as_stream(stream);
  if (pointwise(g)) {
    const ProductArgs x = input_product(g, gradient, weight, addend, input_gradient);
    return launch_product(name, s, x, 1, input_splits(x) != 0);
  }
  const MfmaIgPlan mp = input_backward_mfma_plan(g);
  if (mp.lds_bytes > 0) {
    const dim3 mgrid(mp.tiles, g.batch), mblock(256);
    if (g.kh == 3)
      oxh::launch(conv2d_input_backward_mfma_kernel<3>, mgrid, mblock, mp.lds_bytes, s, g, mp.f,
                  gradient, weight, addend, input_gradient);
    else
      oxh::launch(conv2d_input_backward_mfma_kernel<5>, mgrid, mblock, mp.lds_bytes, s, g, mp.f,
                  gradient, weight, addend, input_gradient);
    return oxh::launched(name);
  }
  const PhasePlan pp = input_backward_s2_plan(g);
  if (pp.lds_bytes > 0) {
    const dim3 pgrid(pp.tiles, g.batch), pblock(pp.threads);
    if (g.kh == 3)
      oxh::launch(conv2d_input_backward_s2_kernel<3>, pgrid, pblock, pp.lds_bytes, s, g, pp.pg,
                  gradient, weight, addend, input_gradient);
    else
      oxh::launch(conv2d_input_backward_s2_kernel<5>, pgrid, pblock, pp.lds_bytes, s, g, pp.pg,
                  gradient, weight, addend, input_gradient);
    return oxh::launched(name);
  }
  const LdsPlan lp = input_backward_lds_plan(g);
  if (lp.tile > 0) {
    const dim3 lgrid(lp.tiles, g.batch), lblock(lp.threads);
    const oxh::FastDiv pd = oxh::make_fastdiv(g.h * g.w);
    switch (tap_kernel(g)) {
      case 31: oxh::launch(conv2d_input_backward_lds_kernel<3, 1>, lgrid, lblock, lp.lds_bytes, s, g, lp.tile, pd, gradient, weight, addend, input_gradient); break;
      case 32: oxh::launch(conv2d_input_backward_lds_kernel<3, 2>, lgrid, lblock, lp.lds_bytes, s, g, lp.tile, pd, gradient, weight, addend, input_gradient); break;
      case 51: oxh::launch(conv2d_input_backward_lds_kernel<5, 1>, lgrid, lblock, lp.lds_bytes, s, g, lp.tile, pd, gradient, weight, addend, input_gradient); break;
      default: oxh::launch(conv2d_input_backward_lds_kernel<5, 2>, lgrid, lblock, lp.lds_bytes, s, g, lp.tile, pd, gradient, weight, addend, input_gradient);
    }
    return oxh::launched(name);
  }
  const dim3 grid(grid_for(in_n)), block(256);
  const uint32_t total = static_cast<uint32_t>(in_n);
  switch (tap_kernel(g)) {
    case 31: oxh::launch(conv2d_input_backward_taps_kernel<3, 1>, grid, block, 0, s, g, total, gradient, weight, addend, input_gradient); break;
    case 32: oxh::launch(conv2d_input_backward_taps_kernel<3, 2>, grid, block, 0, s, g, total, gradient, weight, addend, input_gradient); break;
    case 51: oxh::launch(conv2d_input_backward_taps_kernel<5, 1>, grid, block, 0, s, g, total, gradient, weight, addend, input_gradient); break;
    case 52: oxh::launch(conv2d_input_backward_taps_kernel<5, 2>, grid, block, 0, s, g, total, gradient, weight, addend, input_gradient); break;
    default: oxh::launch(conv2d_input_backward_kernel, grid, block, 0, s, g, total, gradient, weight, addend, input_gradient);
  }
  return oxh::launched(name);
}

// The weight gradient (oxh_conv2d_weight_backward), and with bias_gradient not null the bias
// gradient in the same launches where the per-image LDS kernels take the shape (bias_done is
// then set; otherwise the caller forms the bias).  partial: the workspace.
oxh_status weight_backward_impl(const char *name, hipStream_t s, const ConvGeom &g,
                                const float *gradient, const float *input, float *weight_gradient,
                                float *bias_gradient, float *partial, bool &bias_done) {
  bias_done = false;
  if (pointwise(g)) {
    const KSplit split = product_split(g);
    oxh_status st = launch_weight_product(
        name, s,
        weight_product(g, split, gradient, input, split.chunks > 1 ? partial : weight_gradient),
        split);
    if (st != OXH_OK || split.chunks == 1) return st;
    const uint32_t count = g.out_c * g.in_c;
    launch_sum_chunks(s, count, split.chunks, partial, weight_gradient);
    return oxh::launched(name);
  }
  if (depthwise_single_pass(g)) {
    const oxh::FastDiv oplane_div = oxh::make_fastdiv(g.oh * g.ow);
    const bool wide = g.out_c <= 128;  // few channels: more threads per channel
    if (g.kh == 3 && wide)
      oxh::launch(conv2d_depthwise_weight_kernel<3, 1024>, dim3(g.out_c), dim3(1024), 0, s, g,
                  oplane_div, gradient, input, weight_gradient);
    else if (g.kh == 3)
      oxh::launch(conv2d_depthwise_weight_kernel<3, 256>, dim3(g.out_c), dim3(256), 0, s, g,
                  oplane_div, gradient, input, weight_gradient);
    else if (wide)
      oxh::launch(conv2d_depthwise_weight_kernel<5, 1024>, dim3(g.out_c), dim3(1024), 0, s, g,
                  oplane_div, gradient, input, weight_gradient);
    else
      oxh::launch(conv2d_depthwise_weight_kernel<5, 256>, dim3(g.out_c), dim3(256), 0, s, g,
                  oplane_div, gradient, input, weight_gradient);
    return oxh::launched(name);
  }
  // the matrix-core kernel where it takes the shape, the bias gradient as one more column
  const MfmaWeightPlan mp = weight_mfma_plan(g, bias_gradient != nullptr);
  if (mp.lds_bytes > 0 && oxh::aligned16(gradient) && oxh::aligned16(input)) {
    const bool chunked = mp.chunks > 1;
    float *ow = chunked ? partial : weight_gradient;
    float *ob = !mp.f.bias ? ow : chunked ? partial + weight_elems(g) : bias_gradient;
    const dim3 mgrid(mp.blocks, mp.chunks), mblock(256);
#define OXH_WGT_MFMA_LAUNCH(KK, SS)                                                            \
  do {                                                                                       \
    if (mp.f.ng == 9)                                                                        \
      oxh::launch(conv2d_weight_mfma_kernel<KK, SS, 9>, mgrid, mblock, mp.lds_bytes, s, g,   \
                  mp.f, gradient, input, ow, ob);                                            \
    else if (mp.f.ng == 6)                                                                   \
      oxh::launch(conv2d_weight_mfma_kernel<KK, SS, 6>, mgrid, mblock, mp.lds_bytes, s, g,   \
                  mp.f, gradient, input, ow, ob);                                            \
    else if (mp.f.ng == 3)                                                                   \
      oxh::launch(conv2d_weight_mfma_kernel<KK, SS, 3>, mgrid, mblock, mp.lds_bytes, s, g,   \
                  mp.f, gradient, input, ow, ob);                                            \
    else                                                                                     \
      oxh::launch(conv2d_weight_mfma_kernel<KK, SS, 1>, mgrid, mblock, mp.lds_bytes, s, g,   \
                  mp.f, gradient, input, ow, ob);                                            \
  } while (0)
    switch (tap_kernel(g)) {
      case 31: OXH_WGT_MFMA_LAUNCH(3, 1); break;
      case 32: OXH_WGT_MFMA_LAUNCH(3, 2); break;
      case 51: OXH_WGT_MFMA_LAUNCH(5, 1); break;
      default: OXH_WGT_MFMA_LAUNCH(5, 2);
    }
#undef OXH_WGT_MFMA_LAUNCH
    oxh_status st = oxh::launched(name);
    if (st != OXH_OK) return st;
    bias_done = mp.f.bias != 0;
    if (!chunked) return st;
    const uint32_t weights = static_cast<uint32_t>(weight_elems(g));
    launch_sum_chunks(s, mp.f.stride, mp.chunks, partial, weight_gradient, weights,
                      mp.f.bias ? bias_gradient : nullptr);
    return oxh::launched(name);
  }
  // the bias sums ride along where their threads fit; else the caller forms the bias
  bool bias = bias_gradient != nullptr && weight_lds_plan(g, true).tile > 0;
  const LdsPlan lp = weight_lds_plan(g, bias);
  if (lp.tile > 0) {
    const uint32_t weights = static_cast<uint32_t>(weight_elems(g));
    const bool chunked = lp.chunks > 1;
    // chunk partials [chunk][weights (+ out_c bias sums)], or the gradients themselves
    const uint32_t stride = weights + (bias ? g.out_c : 0);
    float *ow = chunked ? partial : weight_gradient;
    float *ob = !bias ? nullptr : chunked ? partial + weights : bias_gradient;
    const dim3 lgrid(lp.tiles, lp.chunks), lblock(lp.threads);
    const oxh::FastDiv od = oxh::make_fastdiv(g.oh * g.ow);
#define OXH_WEIGHT_LDS(KK, SS)                                                                \
  do {                                                                                        \
    if (bias)                                                                                 \
      oxh::launch(conv2d_weight_lds_kernel<KK, SS, true>, lgrid, lblock, lp.lds_bytes, s, g,  \
                  lp.per_chunk, lp.groups, od, gradient, input, ow, ob, stride);              \
    else                                                                                      \
      oxh::launch(conv2d_weight_lds_kernel<KK, SS, false>, lgrid, lblock, lp.lds_bytes, s, g, \
                  lp.per_chunk, lp.groups, od, gradient, input, ow, ob, stride);              \
  } while (0)
    switch (tap_kernel(g)) {
      case 31: OXH_WEIGHT_LDS(3, 1); break;
      case 32: OXH_WEIGHT_LDS(3, 2); break;
      case 51: OXH_WEIGHT_LDS(5, 1); break;
      default: OXH_WEIGHT_LDS(5, 2);
    }
#undef OXH_WEIGHT_LDS
    bias_done = bias;
    oxh_status st = oxh::launched(name);
    if (st != OXH_OK || !chunked) return st;
    launch_sum_chunks(s, stride, lp.chunks, partial, weight_gradient, weights, bias_gradient);
    return oxh::launched(name);
  }
  const uint32_t chunks = weight_chunks(g);
  const uint32_t weights = static_cast<uint32_t>(weight_elems(g));
  oxh::launch(conv2d_weight_partial_kernel,
              dim3(grid_for(static_cast<uint64_t>(weights) * chunks)), dim3(256), 0, s, g,
              weights, oxh::make_fastdiv(weights), chunks, gradient, input, partial);
  const oxh_status st = oxh::launched(name);
  if (st != OXH_OK) return st;
  launch_sum_chunks(s, weights, chunks, partial, weight_gradient);
  return oxh::launched(name);
}


}  // namespace

extern "C" {

oxh_status oxh_conv2d_output_size(const oxh_conv2d_shape *shape, uint64_t *out_h,
                                  uint64_t *out_w) {
  ConvGeom g;
  oxh_status st = make_conv_geom("oxh_conv2d_output_size", shape, g);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(out_h && out_w, OXH_INVALID_SHAPE, "null output");
  *out_h = g.oh;
  *out_w = g.ow;
  return oxh::ok();
}

int oxh_conv2d_input_backward_serial(const oxh_conv2d_shape *shape) {
  ConvGeom g;
  if (make_conv_geom("oxh_conv2d_input_backward_serial", shape, g) != OXH_OK) return -1;
  if (!pointwise(g)) return input_backward_mfma_plan(g).lds_bytes > 0 ? 0 : 1;
  return input_splits(input_product(g, nullptr, nullptr, nullptr, nullptr)) != 0 ? 0 : 1;
}

int oxh_conv2d_forward_serial(const oxh_conv2d_shape *shape) {
  ConvGeom g;
  if (make_conv_geom("oxh_conv2d_forward_serial", shape, g) != OXH_OK) return -1;
  if (pointwise(g)) return split_kind(g.out_c, g.batch * g.h * g.w, g.in_c, 1) != 0 ? 0 : 1;
  return forward_split_plan(g).tile > 0 ? 0 : 1;
}

oxh_status oxh_conv2d_forward(oxh_stream stream, const oxh_conv2d_shape *shape,
                              const float *input, const float *weight, const float *bias,
                              float *output) {
  const char *name = "oxh_conv2d_forward";
  ConvGeom g;
  oxh_status st = make_conv_geom(name, shape, g);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(input && weight && bias && output, OXH_INVALID_SHAPE,
              std::string(name) + ": null pointer");
  const uint64_t out_n = output_elems(g), in_n = input_elems(g);
  OXH_REQUIRE(!oxh::any_overlap(output, out_n * 4, input, in_n * 4), OXH_INVALID_SHAPE,
              std::string(name) + ": output overlaps the input");
  hipStream_t s = oxh::as_stream(stream);
  if (pointwise(g)) {
    // Y[oc, (n, p)] = b[oc] + sum_ic W[oc, ic] X[(n, p), ic]
    const uint32_t plane = g.h * g.w;
    ProductArgs a{};
    a.a = operand(weight, linear(g.in_c), linear(1));
    a.b = operand(input, batch_plane(plane, g.in_c), linear(plane));
    a.c = output;
    a.cm = linear(plane);
    a.cn = batch_plane(plane, g.out_c);
    a.init = bias;
    a.M = g.out_c;
    a.N = g.batch * plane;
    a.K = g.in_c;
    a.k_chunk = a.K;
    return launch_product(name, s, a, 1, true);
  }
  const MfmaForwardPlan mp = forward_mfma_plan(g);
  if (mp.lds_bytes > 0 && oxh::aligned16(input) && oxh::aligned16(weight)) {
    const dim3 lgrid(mp.tiles, g.batch), lblock(256);
    switch (tap_kernel(g)) {
      case 31: oxh::launch(conv2d_forward_mfma_kernel<3, 1>, lgrid, lblock, mp.lds_bytes, s, g, mp.f, input, weight, bias, output); break;
      case 32: oxh::launch(conv2d_forward_mfma_kernel<3, 2>, lgrid, lblock, mp.lds_bytes, s, g, mp.f, input, weight, bias, output); break;
      case 51: oxh::launch(conv2d_forward_mfma_kernel<5, 1>, lgrid, lblock, mp.lds_bytes, s, g, mp.f, input, weight, bias, output); break;
      default: oxh::launch(conv2d_forward_mfma_kernel<5, 2>, lgrid, lblock, mp.lds_bytes, s, g, mp.f, input, weight, bias, output);
    }
    return oxh::launched(name);
  }
  const LdsPlan sp = forward_split_plan(g);
  if (sp.tile > 0) {
    const dim3 lgrid(sp.tiles, g.batch), lblock(sp.threads);
    const oxh::FastDiv od = oxh::make_fastdiv(g.oh * g.ow);
    const oxh::FastDiv rd = oxh::make_fastdiv(g.in_c * g.kh * g.kw);
    switch (tap_kernel(g)) {
      case 31: oxh::launch(conv2d_forward_split_kernel<3, 1>, lgrid, lblock, sp.lds_bytes, s, g, sp.tile, sp.groups, od, rd, input, weight, bias, output); break;
      case 32: oxh::launch(conv2d_forward_split_kernel<3, 2>, lgrid, lblock, sp.lds_bytes, s, g, sp.tile, sp.groups, od, rd, input, weight, bias, output); break;
      case 51: oxh::launch(conv2d_forward_split_kernel<5, 1>, lgrid, lblock, sp.lds_bytes, s, g, sp.tile, sp.groups, od, rd, input, weight, bias, output); break;
      default: oxh::launch(conv2d_forward_split_kernel<5, 2>, lgrid, lblock, sp.lds_bytes, s, g, sp.tile, sp.groups, od, rd, input, weight, bias, output);
    }
    return oxh::launched(name);
  }
  const LdsPlan lp = forward_lds_plan(g);
  if (lp.tile > 0) {
    const dim3 lgrid(lp.tiles, g.batch), lblock(lp.threads);
    const oxh::FastDiv od = oxh::make_fastdiv(g.oh * g.ow);
    const oxh::FastDiv rd = oxh::make_fastdiv(g.in_c * g.kh * g.kw);
    switch (tap_kernel(g)) {
      case 31: oxh::launch(conv2d_forward_lds_kernel<3, 1>, lgrid, lblock, lp.lds_bytes, s, g, lp.tile, od, rd, input, weight, bias, output); break;
      case 32: oxh::launch(conv2d_forward_lds_kernel<3, 2>, lgrid, lblock, lp.lds_bytes, s, g, lp.tile, od, rd, input, weight, bias, output); break;
      case 51: oxh::launch(conv2d_forward_lds_kernel<5, 1>, lgrid, lblock, lp.lds_bytes, s, g, lp.tile, od, rd, input, weight, bias, output); break;
      default: oxh::launch(conv2d_forward_lds_kernel<5, 2>, lgrid, lblock, lp.lds_bytes, s, g, lp.tile, od, rd, input, weight, bias, output);
    }
    return oxh::launched(name);
  }
  const dim3 grid(grid_for(out_n)), block(256);
  const uint32_t total = static_cast<uint32_t>(out_n);
  switch (tap_kernel(g)) {
    case 31: oxh::launch(conv2d_forward_taps_kernel<3, 1>, grid, block, 0, s, g, total, input, weight, bias, output); break;
    case 32: oxh::launch(conv2d_forward_taps_kernel<3, 2>, grid, block, 0, s, g, total, input, weight, bias, output); break;
    case 51: oxh::launch(conv2d_forward_taps_kernel<5, 1>, grid, block, 0, s, g, total, input, weight, bias, output); break;
    case 52: oxh::launch(conv2d_forward_taps_kernel<5, 2>, grid, block, 0, s, g, total, input, weight, bias, output); break;
    default: oxh::launch(conv2d_forward_kernel, grid, block, 0, s, g, total, input, weight, bias, output);
  }
  return oxh::launched(name);
}

oxh_status oxh_conv2d_input_backward(oxh_stream stream, const oxh_conv2d_shape *shape,
                                     const float *gradient, const float *weight,
                                     float *input_gradient) {
  return input_backward_impl("oxh_conv2d_input_backward", stream, shape, gradient, weight,
                             nullptr, input_gradient);
}

oxh_status oxh_conv2d_input_backward_accumulate(oxh_stream stream,
                                                const oxh_conv2d_shape *shape,
                                                const float *gradient, const float *weight,
                                                const float *addend, float *input_gradient) {
  const char *name = "oxh_conv2d_input_backward_accumulate";
  OXH_REQUIRE(addend != nullptr, OXH_INVALID_SHAPE, std::string(name) + ": null addend");
  return input_backward_impl(name, stream, shape, gradient, weight, addend, input_gradient);
}

oxh_status oxh_conv2d_weight_backward_workspace_size(const oxh_conv2d_shape *shape,
                                                     uint64_t *bytes) {
  ConvGeom g;
  oxh_status st = make_conv_geom("oxh_conv2d_weight_backward_workspace_size", shape, g);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(bytes != nullptr, OXH_INVALID_SHAPE, "bytes is null");
  *bytes = (weight_partial_bytes(g) + 255) / 256 * 256;
  return oxh::ok();
}

oxh_status oxh_conv2d_weight_backward(oxh_stream stream, const oxh_conv2d_shape *shape,
                                      const float *gradient, const float *input,
                                      float *weight_gradient, void *workspace,
                                      uint64_t workspace_bytes) {
  const char *name = "oxh_conv2d_weight_backward";
  ConvGeom g;
  oxh_status st = make_conv_geom(name, shape, g);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(gradient && input && weight_gradient, OXH_INVALID_SHAPE,
              std::string(name) + ": null pointer");
  const uint64_t need = weight_partial_bytes(g);
  OXH_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need), OXH_INVALID_SHAPE,
              std::string(name) +
                  ": workspace too small (oxh_conv2d_weight_backward_workspace_size)");
  bool bias_done = false;
  return weight_backward_impl(name, oxh::as_stream(stream), g, gradient, input, weight_gradient,
                              nullptr, static_cast<float *>(workspace), bias_done);
}

oxh_status oxh_conv2d_bias_backward(oxh_stream stream, const oxh_conv2d_shape *shape,
                                    const float *gradient, float *bias_gradient,
                                    void *workspace, uint64_t workspace_bytes) {
  const char *name = "oxh_conv2d_bias_backward";
  ConvGeom g;
  oxh_status st = make_conv_geom(name, shape, g);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(gradient && bias_gradient, OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  (void)workspace;  // the single-pass reduction needs none
  (void)workspace_bytes;
  oxh::launch(conv2d_bias_kernel, dim3(bias_blocks(g.out_c)), dim3(256), 0,
              oxh::as_stream(stream), bias_args(g, gradient, bias_gradient));
  return oxh::launched(name);
}

oxh_status oxh_conv2d_backward(oxh_stream stream, const oxh_conv2d_shape *shape,
                               const float *gradient, const float *input, const float *weight,
                               const float *addend, float *input_gradient,
                               float *weight_gradient, float *bias_gradient, void *workspace,
                               uint64_t workspace_bytes) {
  const char *name = "oxh_conv2d_backward";
  ConvGeom g;
  oxh_status st = make_conv_geom(name, shape, g);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(gradient && input && weight && weight_gradient, OXH_INVALID_SHAPE,
              std::string(name) + ": null pointer");
  // a null input_gradient: the parameter gradients only (no addend then)
  OXH_REQUIRE(input_gradient != nullptr || addend == nullptr, OXH_INVALID_SHAPE,
              std::string(name) + ": an addend needs an input gradient");
  const uint64_t need = weight_partial_bytes(g);
  OXH_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need), OXH_INVALID_SHAPE,
              std::string(name) +
                  ": workspace too small (oxh_conv2d_weight_backward_workspace_size)");
  // the two gradients are formed concurrently: neither may overlap what the other reads
  const uint64_t gx = input_elems(g) * 4, gy = output_elems(g) * 4, gw = weight_elems(g) * 4;
  const uint64_t gi = input_gradient != nullptr ? gx : 0;
  const uint64_t gb = bias_gradient != nullptr ? g.out_c * 4ull : 0;
  OXH_REQUIRE(!oxh::any_overlap(input_gradient, gi, gradient, gy) &&
                  !oxh::any_overlap(input_gradient, gi, input, gx) &&
                  !oxh::any_overlap(input_gradient, gi, weight, gw) &&
                  !oxh::any_overlap(input_gradient, gi, weight_gradient, gw) &&
                  !oxh::any_overlap(input_gradient, gi, bias_gradient, gb) &&
                  !oxh::any_overlap(input_gradient, gi, workspace, need) &&
                  !oxh::any_overlap(weight_gradient, gw, weight, gw) &&
                  !oxh::any_overlap(weight_gradient, gw, gradient, gy) &&
                  !oxh::any_overlap(weight_gradient, gw, input, gx) &&
                  !oxh::any_overlap(weight_gradient, gw, bias_gradient, gb) &&
                  !oxh::any_overlap(bias_gradient, gb, gradient, gy) &&
                  !oxh::any_overlap(bias_gradient, gb, workspace, need),
              OXH_INVALID_SHAPE, std::string(name) + ": a gradient overlaps an operand");
  // the addend is read while the other gradients and the workspace are written; it may be
  // input_gradient itself (read before the same lane writes it), never a part of it
  const uint64_t ga = addend != nullptr ? gx : 0;
  OXH_REQUIRE(!oxh::any_overlap(addend, ga, weight_gradient, gw) &&
                  !oxh::any_overlap(addend, ga, bias_gradient, gb) &&
                  !oxh::any_overlap(addend, ga, workspace, need) &&
                  (addend == input_gradient || !oxh::any_overlap(addend, ga, input_gradient, gx)),
              OXH_INVALID_SHAPE, std::string(name) + ": the addend overlaps an output");
  hipStream_t s = oxh::as_stream(stream);
  if (pointwise(g) && input_gradient != nullptr) {
    const KSplit split = product_split(g);
    float *partial = static_cast<float *>(workspace);
    const ProductArgs w =
        weight_product(g, split, gradient, input, split.chunks > 1 ? partial : weight_gradient);
    const ProductArgs x = input_product(g, gradient, weight, addend, input_gradient);
    if (launch_dual(s, w, split, x, bias_args(g, gradient, bias_gradient))) {
      st = oxh::launched(name);
      if (st != OXH_OK || split.chunks == 1) return st;
      const uint32_t count = g.out_c * g.in_c;
      launch_sum_chunks(s, count, split.chunks, partial, weight_gradient);
      return oxh::launched(name);
    }
  }
  // a stride-2 K x K convolution whose two gradients both take the matrix-core kernels: one
  // launch (then the chunk sums and the bias launch)
  if (!pointwise(g) && input_gradient != nullptr && oxh::aligned16(gradient) &&
      oxh::aligned16(input)) {
    const MfmaIgPlan ip = input_backward_mfma_plan(g);
    const MfmaWeightPlan wp = ip.lds_bytes > 0 ? weight_mfma_plan(g) : MfmaWeightPlan{};
    if (ip.lds_bytes > 0 && wp.lds_bytes > 0) {
      float *partial = static_cast<float *>(workspace);
      float *out = wp.chunks > 1 ? partial : weight_gradient;
      const MfmaDual d{ip.tiles, ip.tiles * g.batch, wp.blocks, wp.blocks * wp.chunks};
      const uint32_t lds_bytes = ip.lds_bytes > wp.lds_bytes ? ip.lds_bytes : wp.lds_bytes;
      const dim3 grid(d.ig_blocks + d.wg_blocks), block(256);
#define OXH_KK_DUAL(KK)                                                                     \
  do {                                                                                      \
    if (wp.f.ng == 9)                                                                       \
      oxh::launch(conv2d_backward_mfma_kernel<KK, 9>, grid, block, lds_bytes, s, g, ip.f,    \
                  wp.f, d, gradient, weight, input, addend, input_gradient, out);           \
    else if (wp.f.ng == 6)                                                                  \
      oxh::launch(conv2d_backward_mfma_kernel<KK, 6>, grid, block, lds_bytes, s, g, ip.f,    \
                  wp.f, d, gradient, weight, input, addend, input_gradient, out);           \
    else if (wp.f.ng == 3)                                                                  \
      oxh::launch(conv2d_backward_mfma_kernel<KK, 3>, grid, block, lds_bytes, s, g, ip.f,    \
                  wp.f, d, gradient, weight, input, addend, input_gradient, out);           \
    else                                                                                    \
      oxh::launch(conv2d_backward_mfma_kernel<KK, 1>, grid, block, lds_bytes, s, g, ip.f,    \
                  wp.f, d, gradient, weight, input, addend, input_gradient, out);           \
  } while (0)
      if (g.kh == 3)
        OXH_KK_DUAL(3);
      else
        OXH_KK_DUAL(5);
#undef OXH_KK_DUAL
      st = oxh::launched(name);
      if (st != OXH_OK) return st;
      if (wp.chunks > 1) {
        launch_sum_chunks(s, static_cast<uint32_t>(weight_elems(g)), wp.chunks, partial,
                          weight_gradient);
        st = oxh::launched(name);
        if (st != OXH_OK) return st;
      }
      if (bias_gradient == nullptr) return oxh::ok();
      return oxh_conv2d_bias_backward(stream, shape, gradient, bias_gradient, nullptr, 0);
    }
  }
  // parameter gradients only: the bias sums ride in the weight gradient's launches where its
  // kernel takes them (the full VJP keeps the separate bias launch: equal to
  // oxh_conv2d_bias_backward bit for bit)
  bool bias_done = false;
  st = weight_backward_impl(name, s, g, gradient, input, weight_gradient,
                            input_gradient == nullptr ? bias_gradient : nullptr,
                            static_cast<float *>(workspace), bias_done);
  if (st != OXH_OK) return st;
  if (bias_gradient != nullptr && !bias_done) {
    st = oxh_conv2d_bias_backward(stream, shape, gradient, bias_gradient, nullptr, 0);
    if (st != OXH_OK) return st;
  }
  if (input_gradient == nullptr) return oxh::ok();
  return input_backward_impl(name, stream, shape, gradient, weight, addend, input_gradient);
}

}  // extern "C"

oxh_status oxh::conv2d_backward_deferred(oxh_stream stream, const oxh_conv2d_shape *shape,
                                         const float *gradient, const float *input,
                                         const float *weight, const float *addend,
                                         float *input_gradient, float *weight_gradient,
                                         float *bias_gradient, void *workspace,
                                         uint64_t workspace_bytes,
                                         std::vector<ChunkSum> &deferred) {
  struct Restore {
    ~Restore() { deferred_sums = nullptr; }
  } restore;
  deferred_sums = &deferred;
  return oxh_conv2d_backward(stream, shape, gradient, input, weight, addend, input_gradient,
                             weight_gradient, bias_gradient, workspace, workspace_bytes);
}

extern "C" {

oxh_status oxh_avg_pool2d_forward(oxh_stream stream, const oxh_pool2d_shape *shape,
                                  const float *input, float *output) {
  const char *name = "oxh_avg_pool2d_forward";
  PoolGeom g;
  oxh_status st = make_pool_geom(name, shape, g);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(input && output, OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  const uint64_t out_n = static_cast<uint64_t>(g.batch) * g.channels * g.oh * g.ow;
  oxh::launch(avg_pool2d_forward_kernel, dim3(grid_for(out_n)), dim3(256), 0,
              oxh::as_stream(stream), g, static_cast<uint32_t>(out_n), input, output);
  return oxh::launched(name);
}

oxh_status oxh_avg_pool2d_backward(oxh_stream stream, const oxh_pool2d_shape *shape,
                                   const float *gradient, float *input_gradient) {
  const char *name = "oxh_avg_pool2d_backward";
  PoolGeom g;
  oxh_status st = make_pool_geom(name, shape, g);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(gradient && input_gradient, OXH_INVALID_SHAPE,
              std::string(name) + ": null pointer");
  const uint64_t in_n = static_cast<uint64_t>(g.batch) * g.channels * g.h * g.w;
  oxh::launch(avg_pool2d_backward_kernel, dim3(grid_for(in_n)), dim3(256), 0,
              oxh::as_stream(stream), g, static_cast<uint32_t>(in_n), gradient, input_gradient);
  return oxh::launched(name);
}

}  // extern "C"
