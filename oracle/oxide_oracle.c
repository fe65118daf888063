/*
 * oxide_oracle.c -- CPU restatement of oxide-torch's CPU path (tensor hot path).
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for liboxide_hip.so; never linked by the product.
 * See oxide_oracle.h for the list of functions, the reference lines each follows and the checks
 * that pin them.
 *
 * Rust semantics restated here:
 *   - `iter().sum::<f32>()` is a sequential left fold that starts at -0.0 (core's float Sum).
 *   - `f32::max` is IEEE maxNum (a NaN operand yields the other operand) == C fmaxf.
 *   - `f32::exp` / `f32::ln` call the platform libm expf / logf; `sqrt` is correctly rounded,
 *     `recip()` is 1.0 / x.
 *   - `powi(i32)` lowers to compiler-rt's __powisf2 (binary exponentiation, reciprocal for a
 *     negative exponent); restated in oro_powi from that published algorithm.
 *   - No fused multiply-add: rustc never contracts; this file is built with -ffp-contract=off.
 */
#include "oxide_oracle.h"

#include <math.h>
#include <string.h>

#if defined(__FAST_MATH__)
#error "the oracle must not be built with fast-math"
#endif

/* ------------------------------------------------------------------ elementwise */

/* evaluation.rs:21-25 (zip_map at 638-640) and jit.rs:503-507 */
void oro_add(const float *a, const float *b, float *out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

/* evaluation.rs:26-30 and jit.rs:508-512 */
void oro_mul(const float *a, const float *b, float *out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) out[i] = a[i] * b[i];
}

/* evaluation.rs:31-34 (`value.max(0.0)`) and jit.rs:513-517 */
void oro_relu(const float *x, float *out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) out[i] = fmaxf(x[i], 0.0f);
}

/* autograd.rs:123-138: left grad = g * right, right grad = g * left */
void oro_mul_backward(const float *grad, const float *other, float *out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) out[i] = grad[i] * other[i];
}

/* autograd.rs:139-147: g if input > 0 else 0 */
void oro_relu_backward(const float *grad, const float *input, float *out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) out[i] = input[i] > 0.0f ? grad[i] : 0.0f;
}

/* autograd.rs:94-108: an existing gradient is accumulated element by element */
void oro_accumulate(float *current, const float *incoming, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) current[i] += incoming[i];
}

/* jit.rs:463-476 + 479-560: the plan for relu((a+b)*c) is Add -> Mul -> Relu over three
 * workspace buffers; the per-element results equal this direct evaluation. */
void oro_chain_forward(const float *a, const float *b, const float *c, float *y, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) {
    float s = a[i] + b[i];
    float m = s * c[i];
    y[i] = fmaxf(m, 0.0f);
  }
}

/* Upstream ones through Relu (autograd.rs:139-147), Mul (123-138), Add (119-122). */
void oro_chain_backward_ones(const float *a, const float *b, const float *c, float *da, float *db,
                             float *dc, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) {
    float s = a[i] + b[i];
    float m = s * c[i];
    float g_relu = m > 0.0f ? 1.0f : 0.0f;
    float g_left = g_relu * c[i];
    float g_right = g_relu * s;
    da[i] = g_left;
    db[i] = g_left;
    dc[i] = g_right;
  }
}

/* ------------------------------------------------------------------ batch norm */

/* Sequential fp32 sum of a slice, starting at -0.0 (Rust `Sum for f32`). */
static float slice_sum(const float *v, uint64_t n) {
  float acc = -0.0f;
  for (uint64_t i = 0; i < n; ++i) acc += v[i];
  return acc;
}

/* evaluation.rs:490-535 */
int oro_bn_batch_statistics(const float *x, uint64_t batch, uint64_t channels, uint64_t spatial,
                            float epsilon, float *mean, float *inv_std) {
  uint64_t samples = batch * spatial;
  if (samples <= 1) return ORO_EXECUTION; /* evaluation.rs:498-502 */
  float denominator = (float)samples;
  for (uint64_t c = 0; c < channels; ++c) mean[c] = 0.0f;
  for (uint64_t n = 0; n < batch; ++n)
    for (uint64_t c = 0; c < channels; ++c)
      mean[c] += slice_sum(x + (n * channels + c) * spatial, spatial);
  for (uint64_t c = 0; c < channels; ++c) mean[c] /= denominator;
  /* variance accumulates sum((v - mean)^2) per plane; powi(2) is v*v */
  for (uint64_t c = 0; c < channels; ++c) inv_std[c] = 0.0f;
  for (uint64_t n = 0; n < batch; ++n) {
    for (uint64_t c = 0; c < channels; ++c) {
      const float *plane = x + (n * channels + c) * spatial;
      float acc = -0.0f;
      for (uint64_t i = 0; i < spatial; ++i) {
        float d = plane[i] - mean[c];
        acc += d * d;
      }
      inv_std[c] += acc;
    }
  }
  for (uint64_t c = 0; c < channels; ++c) {
    float variance = inv_std[c] / denominator;
    inv_std[c] = 1.0f / sqrtf(variance + epsilon);
  }
  return ORO_OK;
}

/* compiler-rt __powisf2: r = 1; square-and-multiply over |b|; reciprocal if b < 0. */
float oro_powi(float a, int32_t b) {
  const int recip = b < 0;
  float r = 1.0f;
  for (;;) {
    if (b & 1) r *= a;
    b /= 2;
    if (b == 0) break;
    a *= a;
  }
  return recip ? 1.0f / r : r;
}

/* evaluation.rs:537-558 */
int oro_bn_update_running(const float *x, uint64_t batch, uint64_t channels, uint64_t spatial,
                          float momentum, float *running_mean, float *running_var) {
  float mean[channels > 0 ? channels : 1];
  float inv0[channels > 0 ? channels : 1];
  int status = oro_bn_batch_statistics(x, batch, channels, spatial, 0.0f, mean, inv0);
  if (status != ORO_OK) return status;
  uint64_t samples = batch * spatial;
  float unbiased_correction = (float)samples / (float)(samples - 1);
  for (uint64_t c = 0; c < channels; ++c) {
    float biased_variance = oro_powi(inv0[c], -2);
    running_mean[c] = (1.0f - momentum) * running_mean[c] + momentum * mean[c];
    running_var[c] =
        (1.0f - momentum) * running_var[c] + momentum * biased_variance * unbiased_correction;
  }
  return ORO_OK;
}

/* evaluation.rs:560-575 */
void oro_bn_running_statistics(const float *running_var, uint64_t channels, float epsilon,
                               float *inv_std) {
  for (uint64_t c = 0; c < channels; ++c) inv_std[c] = 1.0f / sqrtf(running_var[c] + epsilon);
}

/* evaluation.rs:577-597: ((v - mean) * inv_std) * weight + bias */
void oro_bn_apply(const float *x, uint64_t batch, uint64_t channels, uint64_t spatial,
                  const float *weight, const float *bias, const float *mean, const float *inv_std,
                  float *y) {
  uint64_t total = batch * channels * spatial;
  for (uint64_t i = 0; i < total; ++i) {
    uint64_t c = (i / spatial) % channels;
    y[i] = (x[i] - mean[c]) * inv_std[c] * weight[c] + bias[c];
  }
}

/* evaluation.rs:448-488 (first evaluation of the node: no saved statistics yet). */
int oro_bn_forward(const float *x, uint64_t batch, uint64_t channels, uint64_t spatial,
                   const float *weight, const float *bias, float *running_mean, float *running_var,
                   int training, float momentum, float epsilon, float *y, float *saved_mean,
                   float *saved_inv_std) {
  if (training) {
    int status = oro_bn_batch_statistics(x, batch, channels, spatial, epsilon, saved_mean,
                                         saved_inv_std);
    if (status != ORO_OK) return status;
    status = oro_bn_update_running(x, batch, channels, spatial, momentum, running_mean,
                                   running_var);
    if (status != ORO_OK) return status;
  } else {
    memcpy(saved_mean, running_mean, channels * sizeof(float));
    oro_bn_running_statistics(running_var, channels, epsilon, saved_inv_std);
  }
  oro_bn_apply(x, batch, channels, spatial, weight, bias, saved_mean, saved_inv_std, y);
  return ORO_OK;
}

/* autograd.rs:315-383 */
void oro_bn_backward(const float *grad, const float *x, uint64_t batch, uint64_t channels,
                     uint64_t spatial, const float *weight, const float *mean,
                     const float *inv_std, int training, float *dx, float *dweight, float *dbias) {
  uint64_t samples = batch * spatial;
  float samples_f32 = (float)samples;
  uint64_t total = batch * channels * spatial;
  float gradient_sum[channels > 0 ? channels : 1];
  float gradient_normalized_sum[channels > 0 ? channels : 1];
  for (uint64_t c = 0; c < channels; ++c) {
    dweight[c] = 0.0f;
    dbias[c] = 0.0f;
    gradient_sum[c] = 0.0f;
    gradient_normalized_sum[c] = 0.0f;
  }
  for (uint64_t i = 0; i < total; ++i) {
    uint64_t c = (i / spatial) % channels;
    float normalized = (x[i] - mean[c]) * inv_std[c];
    dweight[c] += grad[i] * normalized;
    dbias[c] += grad[i];
    gradient_sum[c] += grad[i];
    gradient_normalized_sum[c] += grad[i] * normalized;
  }
  for (uint64_t i = 0; i < total; ++i) {
    uint64_t c = (i / spatial) % channels;
    if (training) {
      float normalized = (x[i] - mean[c]) * inv_std[c];
      dx[i] = weight[c] * inv_std[c] / samples_f32 *
              (samples_f32 * grad[i] - gradient_sum[c] - normalized * gradient_normalized_sum[c]);
    } else {
      dx[i] = grad[i] * weight[c] * inv_std[c];
    }
  }
}

/* ------------------------------------------------------------------ cross entropy */

/* evaluation.rs:622-636 */
int oro_class_index(float value, uint64_t classes, uint64_t *index) {
  if (!isfinite(value) || value < 0.0f || (value - truncf(value)) != 0.0f)
    return ORO_INVALID_SHAPE;
  /* `value as usize` saturates: values at or above 2^64 become usize::MAX */
  uint64_t i = value >= 18446744073709551616.0f ? UINT64_MAX : (uint64_t)value;
  if (i >= classes) return ORO_INVALID_SHAPE;
  *index = i;
  return ORO_OK;
}

static float row_max(const float *row, uint64_t classes) {
  float m = -INFINITY; /* fold(f32::NEG_INFINITY, f32::max) */
  for (uint64_t k = 0; k < classes; ++k) m = fmaxf(m, row[k]);
  return m;
}

static float row_normalizer(const float *row, uint64_t classes, float maximum) {
  float acc = -0.0f; /* Sum for f32 */
  for (uint64_t k = 0; k < classes; ++k) acc += expf(row[k] - maximum);
  return acc;
}

/* evaluation.rs:599-620 */
int oro_ce_forward(const float *logits, const float *targets, uint64_t batch, uint64_t classes,
                   float *loss_out) {
  float loss = 0.0f;
  for (uint64_t b = 0; b < batch; ++b) {
    uint64_t target;
    int status = oro_class_index(targets[b], classes, &target);
    if (status != ORO_OK) return status;
    const float *row = logits + b * classes;
    float maximum = row_max(row, classes);
    float normalizer = row_normalizer(row, classes, maximum);
    loss += logf(normalizer) + maximum - row[target];
  }
  *loss_out = loss / (float)batch;
  return ORO_OK;
}

/* autograd.rs:529-554 */
int oro_ce_backward(const float *logits, const float *targets, uint64_t batch, uint64_t classes,
                    float outer_gradient, float *grad) {
  float scale = outer_gradient / (float)batch;
  for (uint64_t b = 0; b < batch; ++b) {
    uint64_t target;
    int status = oro_class_index(targets[b], classes, &target);
    if (status != ORO_OK) return status;
    const float *row = logits + b * classes;
    float maximum = row_max(row, classes);
    float normalizer = row_normalizer(row, classes, maximum);
    for (uint64_t k = 0; k < classes; ++k) {
      float probability = expf(row[k] - maximum) / normalizer;
      grad[b * classes + k] = scale * (probability - (k == target ? 1.0f : 0.0f));
    }
  }
  return ORO_OK;
}

/* ------------------------------------------------------------------ AdamW */

/* optim.rs:98-125 (CPU branch), with the corrections of optim.rs:113-114. */
void oro_adamw_update(float *param, const float *grad, float *first_moment, float *second_moment,
                      uint64_t n, float learning_rate, float weight_decay, float beta1,
                      float beta2, float epsilon, int32_t step) {
  float first_correction = 1.0f - oro_powi(beta1, step);
  float second_correction = 1.0f - oro_powi(beta2, step);
  for (uint64_t i = 0; i < n; ++i) {
    float g = grad[i];
    first_moment[i] = beta1 * first_moment[i] + (1.0f - beta1) * g;
    second_moment[i] = beta2 * second_moment[i] + (1.0f - beta2) * g * g;
    float normalized = (first_moment[i] / first_correction) /
                       (sqrtf(second_moment[i] / second_correction) + epsilon);
    param[i] -= learning_rate * (normalized + weight_decay * param[i]);
  }
}

/* ------------------------------------------------------------------ conv2d / avg_pool2d */

/* evaluation.rs:334-397 */
void oro_conv2d_forward(const float *input, const float *weight, const float *bias,
                        uint64_t batch, uint64_t in_channels, uint64_t height, uint64_t width,
                        uint64_t out_channels, uint64_t kernel_h, uint64_t kernel_w,
                        uint64_t stride, uint64_t padding, uint64_t groups, float *output) {
  uint64_t out_h = (height + 2 * padding - kernel_h) / stride + 1;
  uint64_t out_w = (width + 2 * padding - kernel_w) / stride + 1;
  uint64_t in_per_group = in_channels / groups, out_per_group = out_channels / groups;
  for (uint64_t n = 0; n < batch; ++n)
    for (uint64_t oc = 0; oc < out_channels; ++oc) {
      uint64_t group = oc / out_per_group;
      for (uint64_t oy = 0; oy < out_h; ++oy)
        for (uint64_t ox = 0; ox < out_w; ++ox) {
          float sum = bias[oc];
          for (uint64_t lc = 0; lc < in_per_group; ++lc) {
            uint64_t ic = group * in_per_group + lc;
            for (uint64_t ky = 0; ky < kernel_h; ++ky) {
              uint64_t py = oy * stride + ky;
              if (py < padding || py - padding >= height) continue;
              uint64_t iy = py - padding;
              for (uint64_t kx = 0; kx < kernel_w; ++kx) {
                uint64_t px = ox * stride + kx;
                if (px < padding || px - padding >= width) continue;
                uint64_t ix = px - padding;
                sum += input[((n * in_channels + ic) * height + iy) * width + ix] *
                       weight[((oc * in_per_group + lc) * kernel_h + ky) * kernel_w + kx];
              }
            }
          }
          output[((n * out_channels + oc) * out_h + oy) * out_w + ox] = sum;
        }
    }
}

/* autograd.rs:412-483 */
void oro_conv2d_backward(const float *grad, const float *input, const float *weight,
                         uint64_t batch, uint64_t in_channels, uint64_t height, uint64_t width,
                         uint64_t out_channels, uint64_t kernel_h, uint64_t kernel_w,
                         uint64_t stride, uint64_t padding, uint64_t groups, float *dinput,
                         float *dweight, float *dbias) {
  uint64_t out_h = (height + 2 * padding - kernel_h) / stride + 1;
  uint64_t out_w = (width + 2 * padding - kernel_w) / stride + 1;
  uint64_t in_per_group = in_channels / groups, out_per_group = out_channels / groups;
  memset(dinput, 0, batch * in_channels * height * width * sizeof(float));
  memset(dweight, 0, out_channels * in_per_group * kernel_h * kernel_w * sizeof(float));
  memset(dbias, 0, out_channels * sizeof(float));
  for (uint64_t n = 0; n < batch; ++n)
    for (uint64_t oc = 0; oc < out_channels; ++oc) {
      uint64_t group = oc / out_per_group;
      for (uint64_t oy = 0; oy < out_h; ++oy)
        for (uint64_t ox = 0; ox < out_w; ++ox) {
          float g = grad[((n * out_channels + oc) * out_h + oy) * out_w + ox];
          dbias[oc] += g;
          for (uint64_t lc = 0; lc < in_per_group; ++lc) {
            uint64_t ic = group * in_per_group + lc;
            for (uint64_t ky = 0; ky < kernel_h; ++ky) {
              uint64_t py = oy * stride + ky;
              if (py < padding || py - padding >= height) continue;
              uint64_t iy = py - padding;
              for (uint64_t kx = 0; kx < kernel_w; ++kx) {
                uint64_t px = ox * stride + kx;
                if (px < padding || px - padding >= width) continue;
                uint64_t ix = px - padding;
                uint64_t ii = ((n * in_channels + ic) * height + iy) * width + ix;
                uint64_t wi = ((oc * in_per_group + lc) * kernel_h + ky) * kernel_w + kx;
                dinput[ii] += g * weight[wi];
                dweight[wi] += g * input[ii];
              }
            }
          }
        }
    }
}

/* evaluation.rs:399-445 */
void oro_avg_pool2d_forward(const float *input, uint64_t batch, uint64_t channels,
                            uint64_t height, uint64_t width, uint64_t kernel_h, uint64_t kernel_w,
                            uint64_t stride_h, uint64_t stride_w, float *output) {
  uint64_t out_h = (height - kernel_h) / stride_h + 1, out_w = (width - kernel_w) / stride_w + 1;
  float denominator = (float)(kernel_h * kernel_w);
  for (uint64_t n = 0; n < batch; ++n)
    for (uint64_t c = 0; c < channels; ++c)
      for (uint64_t oy = 0; oy < out_h; ++oy)
        for (uint64_t ox = 0; ox < out_w; ++ox) {
          float sum = 0.0f;
          for (uint64_t ky = 0; ky < kernel_h; ++ky)
            for (uint64_t kx = 0; kx < kernel_w; ++kx)
              sum += input[((n * channels + c) * height + oy * stride_h + ky) * width +
                           ox * stride_w + kx];
          output[((n * channels + c) * out_h + oy) * out_w + ox] = sum / denominator;
        }
}

/* autograd.rs:485-527 */
void oro_avg_pool2d_backward(const float *grad, uint64_t batch, uint64_t channels,
                             uint64_t height, uint64_t width, uint64_t kernel_h,
                             uint64_t kernel_w, uint64_t stride_h, uint64_t stride_w,
                             float *dinput) {
  uint64_t out_h = (height - kernel_h) / stride_h + 1, out_w = (width - kernel_w) / stride_w + 1;
  float denominator = (float)(kernel_h * kernel_w);
  memset(dinput, 0, batch * channels * height * width * sizeof(float));
  for (uint64_t n = 0; n < batch; ++n)
    for (uint64_t c = 0; c < channels; ++c)
      for (uint64_t oy = 0; oy < out_h; ++oy)
        for (uint64_t ox = 0; ox < out_w; ++ox) {
          float contribution = grad[((n * channels + c) * out_h + oy) * out_w + ox] / denominator;
          for (uint64_t ky = 0; ky < kernel_h; ++ky)
            for (uint64_t kx = 0; kx < kernel_w; ++kx)
              dinput[((n * channels + c) * height + oy * stride_h + ky) * width + ox * stride_w +
                     kx] += contribution;
        }
}

/* ------------------------------------------------------------------ model helpers */

/* nn.rs:657-674 */
void oro_initialized_weights(const uint64_t *shape, uint64_t input_channels_per_group,
                             float *out) {
  uint64_t kernel_area = shape[2] * shape[3];
  float fan_in = (float)(input_channels_per_group * kernel_area);
  float scale = sqrtf(2.0f / fan_in);
  uint64_t state = 0x9E3779B9ull;
  for (int d = 0; d < 4; ++d) state ^= shape[d] * 0xBF58476D1CE4E5B9ull;
  state |= 1;
  uint64_t total = shape[0] * shape[1] * shape[2] * shape[3];
  for (uint64_t i = 0; i < total; ++i) {
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    float unit = (float)(uint32_t)(state >> 40) / (float)(1u << 24);
    out[i] = (unit * 2.0f - 1.0f) * scale;
  }
}

/* f32::total_cmp key: flip the magnitude bits of negative values. */
static int32_t total_key(float v) {
  int32_t bits;
  memcpy(&bits, &v, sizeof bits);
  bits ^= (int32_t)(((uint32_t)(bits >> 31)) >> 1);
  return bits;
}

/* mnist_training.rs:201-218: Iterator::max_by keeps the last of equal maxima. */
void oro_argmax_rows(const float *logits, uint64_t rows, uint64_t classes, uint64_t *out) {
  for (uint64_t r = 0; r < rows; ++r) {
    const float *row = logits + r * classes;
    uint64_t best = 0;
    for (uint64_t k = 1; k < classes; ++k)
      if (total_key(row[k]) >= total_key(row[best])) best = k;
    out[r] = best;
  }
}

/* ------------------------------------------------------------------ MNIST data */

/* mnist.rs:118-121 */
void oro_mnist_normalize(const uint8_t *pixels, uint64_t n, float *out) {
  for (uint64_t i = 0; i < n; ++i) out[i] = ((float)pixels[i] / 255.0f - 0.1307f) / 0.3081f;
}

/* mnist.rs:191-199: for index in (1..len).rev(), swap with state % (index + 1). */
void oro_mnist_shuffle(uint64_t *values, uint64_t n) {
  uint64_t state = 0xD1B54A32D192ED03ull;
  for (uint64_t index = n; index-- > 1;) {
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    uint64_t swap_with = state % (index + 1);
    uint64_t t = values[index];
    values[index] = values[swap_with];
    values[swap_with] = t;
  }
}
