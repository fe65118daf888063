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
// terms; one thread per weight element would serialize thousands of dependent adds, so they are
// split into batch chunks (each chunk in the CPU order) whose partial sums a second launch adds
// in chunk order: deterministic, within fp32 rounding of the CPU's single running sum.
#include <hip/hip_runtime.h>

#include <string>

#include "common.h"

namespace {

struct ConvGeom {
  uint32_t batch, in_c, h, w, out_c, kh, kw, stride, pad, groups;
  uint32_t oh, ow, in_per_group, out_per_group;
};

__global__ __launch_bounds__(256) void conv2d_forward_kernel(ConvGeom g,
                                                             const float *__restrict__ x,
                                                             const float *__restrict__ wt,
                                                             const float *__restrict__ bias,
                                                             float *__restrict__ y) {
  const uint64_t total = static_cast<uint64_t>(g.batch) * g.out_c * g.oh * g.ow;
  for (uint64_t o = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; o < total;
       o += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint32_t ox = static_cast<uint32_t>(o % g.ow);
    const uint32_t oy = static_cast<uint32_t>((o / g.ow) % g.oh);
    const uint32_t oc = static_cast<uint32_t>((o / (static_cast<uint64_t>(g.ow) * g.oh)) % g.out_c);
    const uint64_t n = o / (static_cast<uint64_t>(g.ow) * g.oh * g.out_c);
    const uint32_t group = oc / g.out_per_group;
    float sum = bias[oc];
    for (uint32_t lc = 0; lc < g.in_per_group; ++lc) {
      const uint32_t ic = group * g.in_per_group + lc;
      const float *xp = x + (n * g.in_c + ic) * g.h * g.w;
      const float *wp = wt + (static_cast<uint64_t>(oc) * g.in_per_group + lc) * g.kh * g.kw;
      for (uint32_t ky = 0; ky < g.kh; ++ky) {
        const int iy = static_cast<int>(oy * g.stride + ky) - static_cast<int>(g.pad);
        if (iy < 0 || iy >= static_cast<int>(g.h)) continue;
        for (uint32_t kx = 0; kx < g.kw; ++kx) {
          const int ix = static_cast<int>(ox * g.stride + kx) - static_cast<int>(g.pad);
          if (ix < 0 || ix >= static_cast<int>(g.w)) continue;
          sum += xp[iy * g.w + ix] * wp[ky * g.kw + kx];
        }
      }
    }
    y[o] = sum;
  }
}

// One thread per input element; contributions in (oc, oy, ox) ascending order.
__global__ __launch_bounds__(256) void conv2d_input_backward_kernel(
    ConvGeom g, const float *__restrict__ grad, const float *__restrict__ wt,
    float *__restrict__ dx) {
  const uint64_t total = static_cast<uint64_t>(g.batch) * g.in_c * g.h * g.w;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint32_t ix = static_cast<uint32_t>(i % g.w);
    const uint32_t iy = static_cast<uint32_t>((i / g.w) % g.h);
    const uint32_t ic = static_cast<uint32_t>((i / (static_cast<uint64_t>(g.w) * g.h)) % g.in_c);
    const uint64_t n = i / (static_cast<uint64_t>(g.w) * g.h * g.in_c);
    const uint32_t group = ic / g.in_per_group, lc = ic % g.in_per_group;
    float acc = 0.0f;
    for (uint32_t j = 0; j < g.out_per_group; ++j) {
      const uint32_t oc = group * g.out_per_group + j;
      const float *gp = grad + (n * g.out_c + oc) * g.oh * g.ow;
      const float *wp = wt + (static_cast<uint64_t>(oc) * g.in_per_group + lc) * g.kh * g.kw;
      // oy = (iy + pad - ky) / stride ascends as ky descends
      for (int ky = static_cast<int>(g.kh) - 1; ky >= 0; --ky) {
        const int ty = static_cast<int>(iy + g.pad) - ky;
        if (ty < 0 || ty % static_cast<int>(g.stride) != 0) continue;
        const int oy = ty / static_cast<int>(g.stride);
        if (oy >= static_cast<int>(g.oh)) continue;
        for (int kx = static_cast<int>(g.kw) - 1; kx >= 0; --kx) {
          const int tx = static_cast<int>(ix + g.pad) - kx;
          if (tx < 0 || tx % static_cast<int>(g.stride) != 0) continue;
          const int ox = tx / static_cast<int>(g.stride);
          if (ox >= static_cast<int>(g.ow)) continue;
          acc += gp[oy * g.ow + ox] * wp[ky * g.kw + kx];
        }
      }
    }
    dx[i] = acc;
  }
}

// Weight gradient, phase 1: chunk c of the batch for weight element e (grid-stride over
// chunks * weights), terms in (n, oy, ox) order.
__global__ __launch_bounds__(256) void conv2d_weight_partial_kernel(
    ConvGeom g, uint32_t chunks, const float *__restrict__ grad, const float *__restrict__ x,
    float *__restrict__ partial) {
  const uint64_t weights = static_cast<uint64_t>(g.out_c) * g.in_per_group * g.kh * g.kw;
  const uint64_t total = weights * chunks;
  const uint32_t per = (g.batch + chunks - 1) / chunks;
  for (uint64_t t = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint64_t e = t % weights;
    const uint32_t chunk = static_cast<uint32_t>(t / weights);
    const uint32_t kx = static_cast<uint32_t>(e % g.kw);
    const uint32_t ky = static_cast<uint32_t>((e / g.kw) % g.kh);
    const uint32_t lc = static_cast<uint32_t>((e / (static_cast<uint64_t>(g.kw) * g.kh)) % g.in_per_group);
    const uint32_t oc = static_cast<uint32_t>(e / (static_cast<uint64_t>(g.kw) * g.kh * g.in_per_group));
    const uint32_t ic = (oc / g.out_per_group) * g.in_per_group + lc;
    const uint32_t n0 = chunk * per, n1 = n0 + per < g.batch ? n0 + per : g.batch;
    float acc = 0.0f;
    for (uint32_t n = n0; n < n1; ++n) {
      const float *gp = grad + (static_cast<uint64_t>(n) * g.out_c + oc) * g.oh * g.ow;
      const float *xp = x + (static_cast<uint64_t>(n) * g.in_c + ic) * g.h * g.w;
      for (uint32_t oy = 0; oy < g.oh; ++oy) {
        const int iy = static_cast<int>(oy * g.stride + ky) - static_cast<int>(g.pad);
        if (iy < 0 || iy >= static_cast<int>(g.h)) continue;
        for (uint32_t ox = 0; ox < g.ow; ++ox) {
          const int ix = static_cast<int>(ox * g.stride + kx) - static_cast<int>(g.pad);
          if (ix < 0 || ix >= static_cast<int>(g.w)) continue;
          acc += gp[oy * g.ow + ox] * xp[iy * g.w + ix];
        }
      }
    }
    partial[t] = acc;
  }
}

// Bias gradient, phase 1: chunk c of the batch for output channel oc, terms in (n, oy, ox).
__global__ __launch_bounds__(256) void conv2d_bias_partial_kernel(
    uint32_t batch, uint32_t out_c, uint32_t plane, uint32_t chunks,
    const float *__restrict__ grad, float *__restrict__ partial) {
  const uint64_t total = static_cast<uint64_t>(out_c) * chunks;
  const uint32_t per = (batch + chunks - 1) / chunks;
  for (uint64_t t = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint32_t oc = static_cast<uint32_t>(t % out_c);
    const uint32_t chunk = static_cast<uint32_t>(t / out_c);
    const uint32_t n0 = chunk * per, n1 = n0 + per < batch ? n0 + per : batch;
    float acc = 0.0f;
    for (uint32_t n = n0; n < n1; ++n) {
      const float *gp = grad + (static_cast<uint64_t>(n) * out_c + oc) * plane;
      for (uint32_t i = 0; i < plane; ++i) acc += gp[i];
    }
    partial[t] = acc;
  }
}

// Phase 2 of both: out[e] = sum over chunks of partial[chunk][e], in chunk order.
__global__ __launch_bounds__(256) void sum_chunks_kernel(uint64_t count, uint32_t chunks,
                                                         const float *__restrict__ partial,
                                                         float *__restrict__ out) {
  for (uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < count;
       e += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    float acc = 0.0f;
    for (uint32_t c = 0; c < chunks; ++c) acc += partial[c * count + e];
    out[e] = acc;
  }
}

struct PoolGeom {
  uint32_t batch, channels, h, w, kh, kw, sh, sw, oh, ow;
  float denominator;
};

// evaluation.rs:414-444: window sum in (ky, kx) order divided by the window area.
__global__ __launch_bounds__(256) void avg_pool2d_forward_kernel(PoolGeom g,
                                                                 const float *__restrict__ x,
                                                                 float *__restrict__ y) {
  const uint64_t total = static_cast<uint64_t>(g.batch) * g.channels * g.oh * g.ow;
  for (uint64_t o = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; o < total;
       o += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint32_t ox = static_cast<uint32_t>(o % g.ow);
    const uint32_t oy = static_cast<uint32_t>((o / g.ow) % g.oh);
    const uint64_t plane = o / (static_cast<uint64_t>(g.ow) * g.oh);
    const float *xp = x + plane * g.h * g.w;
    float sum = 0.0f;
    for (uint32_t ky = 0; ky < g.kh; ++ky)
      for (uint32_t kx = 0; kx < g.kw; ++kx)
        sum += xp[(oy * g.sh + ky) * g.w + ox * g.sw + kx];
    y[o] = sum / g.denominator;
  }
}

// autograd.rs:501-525: each output adds g / area to every input of its window; gathered here per
// input element in (oy, ox) ascending order.
__global__ __launch_bounds__(256) void avg_pool2d_backward_kernel(PoolGeom g,
                                                                  const float *__restrict__ grad,
                                                                  float *__restrict__ dx) {
  const uint64_t total = static_cast<uint64_t>(g.batch) * g.channels * g.h * g.w;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint32_t ix = static_cast<uint32_t>(i % g.w);
    const uint32_t iy = static_cast<uint32_t>((i / g.w) % g.h);
    const uint64_t plane = i / (static_cast<uint64_t>(g.w) * g.h);
    const float *gp = grad + plane * g.oh * g.ow;
    // outputs oy with oy * sh <= iy < oy * sh + kh
    const uint32_t oy_lo = iy + 1 > g.kh ? (iy + 1 - g.kh + g.sh - 1) / g.sh : 0;
    const uint32_t ox_lo = ix + 1 > g.kw ? (ix + 1 - g.kw + g.sw - 1) / g.sw : 0;
    float acc = 0.0f;
    for (uint32_t oy = oy_lo; oy < g.oh && oy * g.sh <= iy; ++oy)
      for (uint32_t ox = ox_lo; ox < g.ow && ox * g.sw <= ix; ++ox)
        acc += gp[oy * g.ow + ox] / g.denominator;
    dx[i] = acc;
  }
}

uint32_t grid_for(uint64_t items) {
  uint64_t g = (items + 255) / 256;
  if (g < 1) g = 1;
  if (g > (1u << 20)) g = 1u << 20;
  return static_cast<uint32_t>(g);
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
  g.oh = (g.h + 2 * g.pad - g.kh) / g.stride + 1;
  g.ow = (g.w + 2 * g.pad - g.kw) / g.stride + 1;
  g.in_per_group = g.in_c / g.groups;
  g.out_per_group = g.out_c / g.groups;
  const uint64_t sizes[] = {static_cast<uint64_t>(g.batch) * g.in_c * g.h * g.w,
                            static_cast<uint64_t>(g.batch) * g.out_c * g.oh * g.ow,
                            static_cast<uint64_t>(g.out_c) * g.in_per_group * g.kh * g.kw};
  for (uint64_t n : sizes)
    OXH_REQUIRE(n < (1ull << 40), OXH_INVALID_SHAPE, std::string(name) + ": tensor too large");
  return oxh::ok();
}

// Batch chunks for the weight / bias reductions: enough threads to fill the GPU (~64K), at most
// one chunk per batch element.
uint32_t weight_chunks(const ConvGeom &g) {
  const uint64_t weights = static_cast<uint64_t>(g.out_c) * g.in_per_group * g.kh * g.kw;
  uint64_t c = (65536 + weights - 1) / weights;
  if (c > g.batch) c = g.batch;
  if (c < 1) c = 1;
  return static_cast<uint32_t>(c);
}
uint32_t bias_chunks(uint64_t batch, uint64_t out_c) {
  uint64_t c = (65536 + out_c - 1) / out_c;
  if (c > batch) c = batch;
  if (c < 1) c = 1;
  return static_cast<uint32_t>(c);
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
  OXH_REQUIRE(static_cast<uint64_t>(g.batch) * g.channels * g.h * g.w < (1ull << 40),
              OXH_INVALID_SHAPE, std::string(name) + ": tensor too large");
  return oxh::ok();
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

oxh_status oxh_conv2d_forward(oxh_stream stream, const oxh_conv2d_shape *shape,
                              const float *input, const float *weight, const float *bias,
                              float *output) {
  const char *name = "oxh_conv2d_forward";
  ConvGeom g;
  oxh_status st = make_conv_geom(name, shape, g);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(input && weight && bias && output, OXH_INVALID_SHAPE,
              std::string(name) + ": null pointer");
  const uint64_t out_n = static_cast<uint64_t>(g.batch) * g.out_c * g.oh * g.ow;
  const uint64_t in_n = static_cast<uint64_t>(g.batch) * g.in_c * g.h * g.w;
  OXH_REQUIRE(!oxh::any_overlap(output, out_n * 4, input, in_n * 4), OXH_INVALID_SHAPE,
              std::string(name) + ": output overlaps the input");
  oxh::launch(conv2d_forward_kernel, dim3(grid_for(out_n)), dim3(256), 0,
              oxh::as_stream(stream), g, input, weight, bias, output);
  return oxh::launched(name);
}

oxh_status oxh_conv2d_input_backward(oxh_stream stream, const oxh_conv2d_shape *shape,
                                     const float *gradient, const float *weight,
                                     float *input_gradient) {
  const char *name = "oxh_conv2d_input_backward";
  ConvGeom g;
  oxh_status st = make_conv_geom(name, shape, g);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(gradient && weight && input_gradient, OXH_INVALID_SHAPE,
              std::string(name) + ": null pointer");
  const uint64_t in_n = static_cast<uint64_t>(g.batch) * g.in_c * g.h * g.w;
  oxh::launch(conv2d_input_backward_kernel, dim3(grid_for(in_n)), dim3(256), 0,
              oxh::as_stream(stream), g, gradient, weight, input_gradient);
  return oxh::launched(name);
}

oxh_status oxh_conv2d_weight_backward_workspace_size(const oxh_conv2d_shape *shape,
                                                     uint64_t *bytes) {
  ConvGeom g;
  oxh_status st = make_conv_geom("oxh_conv2d_weight_backward_workspace_size", shape, g);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(bytes != nullptr, OXH_INVALID_SHAPE, "bytes is null");
  const uint64_t weights = static_cast<uint64_t>(g.out_c) * g.in_per_group * g.kh * g.kw;
  const uint64_t wb = weights * weight_chunks(g) * 4;
  const uint64_t bb = static_cast<uint64_t>(g.out_c) * bias_chunks(g.batch, g.out_c) * 4;
  *bytes = ((wb > bb ? wb : bb) + 255) / 256 * 256;
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
  const uint32_t chunks = weight_chunks(g);
  const uint64_t weights = static_cast<uint64_t>(g.out_c) * g.in_per_group * g.kh * g.kw;
  OXH_REQUIRE(workspace != nullptr && workspace_bytes >= weights * chunks * 4,
              OXH_INVALID_SHAPE,
              std::string(name) + ": workspace too small (oxh_conv2d_weight_backward_workspace_size)");
  float *partial = static_cast<float *>(workspace);
  hipStream_t s = oxh::as_stream(stream);
  oxh::launch(conv2d_weight_partial_kernel, dim3(grid_for(weights * chunks)), dim3(256), 0, s,
              g, chunks, gradient, input, partial);
  st = oxh::launched(name);
  if (st != OXH_OK) return st;
  oxh::launch(sum_chunks_kernel, dim3(grid_for(weights)), dim3(256), 0, s, weights, chunks,
              static_cast<const float *>(partial), weight_gradient);
  return oxh::launched(name);
}

oxh_status oxh_conv2d_bias_backward(oxh_stream stream, const oxh_conv2d_shape *shape,
                                    const float *gradient, float *bias_gradient,
                                    void *workspace, uint64_t workspace_bytes) {
  const char *name = "oxh_conv2d_bias_backward";
  ConvGeom g;
  oxh_status st = make_conv_geom(name, shape, g);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(gradient && bias_gradient, OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  const uint32_t chunks = bias_chunks(g.batch, g.out_c);
  OXH_REQUIRE(workspace != nullptr &&
                  workspace_bytes >= static_cast<uint64_t>(g.out_c) * chunks * 4,
              OXH_INVALID_SHAPE,
              std::string(name) + ": workspace too small (oxh_conv2d_weight_backward_workspace_size)");
  float *partial = static_cast<float *>(workspace);
  hipStream_t s = oxh::as_stream(stream);
  oxh::launch(conv2d_bias_partial_kernel,
              dim3(grid_for(static_cast<uint64_t>(g.out_c) * chunks)), dim3(256), 0, s, g.batch,
              g.out_c, g.oh * g.ow, chunks, gradient, partial);
  st = oxh::launched(name);
  if (st != OXH_OK) return st;
  oxh::launch(sum_chunks_kernel, dim3(grid_for(g.out_c)), dim3(256), 0, s,
              static_cast<uint64_t>(g.out_c), chunks, static_cast<const float *>(partial),
              bias_gradient);
  return oxh::launched(name);
}

oxh_status oxh_avg_pool2d_forward(oxh_stream stream, const oxh_pool2d_shape *shape,
                                  const float *input, float *output) {
  const char *name = "oxh_avg_pool2d_forward";
  PoolGeom g;
  oxh_status st = make_pool_geom(name, shape, g);
  if (st != OXH_OK) return st;
  OXH_REQUIRE(input && output, OXH_INVALID_SHAPE, std::string(name) + ": null pointer");
  const uint64_t out_n = static_cast<uint64_t>(g.batch) * g.channels * g.oh * g.ow;
  oxh::launch(avg_pool2d_forward_kernel, dim3(grid_for(out_n)), dim3(256), 0,
              oxh::as_stream(stream), g, input, output);
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
              oxh::as_stream(stream), g, gradient, input_gradient);
  return oxh::launched(name);
}

}  // extern "C"
