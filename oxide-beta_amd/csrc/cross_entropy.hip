// cross_entropy.hip -- row log-softmax cross entropy: mean NLL loss and/or the gradient with
// respect to the logits, from one read of each row.
//
// Reference kernels: cross_entropy_forward (kernel_module.rs:966-1009) runs the whole batch in
// one thread; cross_entropy_backward (1011-1050) re-scans the full row (max and sum of exp) for
// every logit, O(B * C^2).  CPU semantics: evaluation.rs:599-636, autograd.rs:529-554.
//
// Design (gfx950): one workgroup per row.  On the register path (classes % 4 == 0, aligned,
// classes <= 16 * 4 * OXH_CE_BLOCK) the row is loaded once with 128-bit loads into VGPRs (up to
// 16 float4 per lane), the max and the sum of exp(x - max) are block reductions (wave64
// shuffles, then LDS across waves), and the gradient is written from the same registers, so a
// fused loss+gradient moves exactly one read and one write of the logits.  The per-row losses
// go to an fp64 workspace vector and a one-block kernel sums them in row order for the mean (no
// inter-block synchronization: on gfx950 an agent-scope release per block would write back the
// XCD's L2).  Other shapes take a three-pass strided path (max, sum, gradient) whose re-reads of
// a row hit L2.
//
// Per element the fp32 operations follow the CPU path: e = exp(x - max);
// p = e / normalizer; grad = (outer / batch) * (p - onehot); row loss = (ln(normalizer) + max)
// - x[target].  expf / logf are ROCm's device math library (a few ulp from glibc's).
#include <hip/hip_runtime.h>

#include <cmath>
#include <string>

#include "common.h"

namespace {

// Row block shape for wide rows (overridable at build time for tuning sweeps): lanes per row
// and the minimum waves per SIMD the register budget must allow.
#ifndef OXH_CE_BLOCK
#define OXH_CE_BLOCK 512
#endif
#ifndef OXH_CE_MINW
#define OXH_CE_MINW 4
#endif

struct CeArgs {
  const float *logits, *targets, *outer;  // outer: device scalar (may be null when no grad)
  float *loss;                            // may be null (no loss)
  float *grad;                            // may be null (no gradient)
  uint32_t *error_flag;                   // may be null
  double *row_loss;                       // workspace [batch]
  uint64_t batch, classes;
};

// evaluation.rs:622-636: finite, non-negative, integral and below `classes`.
__device__ __forceinline__ bool target_index(float t, uint64_t classes, uint64_t &index) {
  if (!isfinite(t) || t < 0.0f || t - truncf(t) != 0.0f) return false;
  if (t >= 18446744073709551616.0f) return false;
  const uint64_t i = static_cast<uint64_t>(t);
  if (i >= classes) return false;
  index = i;
  return true;
}

template <int BLOCK>
__device__ __forceinline__ float block_max(float v, float *lds) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  constexpr int W = BLOCK / 64;
  const int wave = threadIdx.x / 64;
  if (threadIdx.x % 64 == 0) lds[wave] = v;
  __syncthreads();
  float r = lds[0];
#pragma unroll
  for (int w = 1; w < W; ++w) r = fmaxf(r, lds[w]);
  __syncthreads();
  return r;
}

template <int BLOCK>
__device__ __forceinline__ double block_sum(double v, double *lds) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  constexpr int W = BLOCK / 64;
  const int wave = threadIdx.x / 64;
  if (threadIdx.x % 64 == 0) lds[wave] = v;
  __syncthreads();
  double r = 0.0;
#pragma unroll
  for (int w = 0; w < W; ++w) r += lds[w];
  __syncthreads();
  return r;
}

// Row finished: record its loss for the batch mean.
__device__ __forceinline__ void finish_row(const CeArgs &a, uint64_t row, float row_loss) {
  if (a.loss != nullptr && threadIdx.x == 0) a.row_loss[row] = static_cast<double>(row_loss);
}

// Batch mean of the row losses (one block): thread t adds rows t, t + 1024, ... in order, then a
// fixed-shape tree, so the result is deterministic.  evaluation.rs:616-619 divides the summed
// loss by the batch size in fp32.
constexpr int kMeanBlock = 1024;

__global__ __launch_bounds__(kMeanBlock) void ce_mean_kernel(const double *__restrict__ row_loss,
                                                             uint64_t batch, float *loss) {
  __shared__ double lds[kMeanBlock / 64];
  double s = 0.0;
  for (uint64_t r = threadIdx.x; r < batch; r += kMeanBlock) s += row_loss[r];
  s = block_sum<kMeanBlock>(s, lds);
  if (threadIdx.x == 0) *loss = static_cast<float>(s) / static_cast<float>(batch);
}

// Register path: BLOCK lanes x V float4 hold one row of `classes` (= 4 * c4) logits.  MINW
// (waves per SIMD the compiler must allow) bounds the VGPRs so several rows share a CU and one
// row's memory phase overlaps another's exp / reduction phase.
template <int BLOCK, int V, int MINW>
__global__ __launch_bounds__(BLOCK, MINW) void ce_row_kernel(CeArgs a) {
  __shared__ float lds_f[BLOCK / 64];
  __shared__ double lds_d[BLOCK / 64];
  const uint64_t row = blockIdx.x;
  const uint64_t c4 = a.classes / 4;
  const float4 *x4 = reinterpret_cast<const float4 *>(a.logits + row * a.classes);
  float4 v[V];
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const uint64_t i = threadIdx.x + static_cast<uint64_t>(k) * BLOCK;
    if (i < c4) {
      v[k] = x4[i];
      m = fmaxf(m, fmaxf(fmaxf(v[k].x, v[k].y), fmaxf(v[k].z, v[k].w)));
    }
  }
  const float maximum = block_max<BLOCK>(m, lds_f);
  double s = 0.0;
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const uint64_t i = threadIdx.x + static_cast<uint64_t>(k) * BLOCK;
    if (i < c4) {
      v[k].x = expf(v[k].x - maximum);
      v[k].y = expf(v[k].y - maximum);
      v[k].z = expf(v[k].z - maximum);
      v[k].w = expf(v[k].w - maximum);
      s += static_cast<double>(v[k].x + v[k].y) + static_cast<double>(v[k].z + v[k].w);
    }
  }
  const float normalizer = static_cast<float>(block_sum<BLOCK>(s, lds_d));
  uint64_t target = 0;
  const bool valid = target_index(a.targets[row], a.classes, target);
  if (!valid && threadIdx.x == 0 && a.error_flag) *a.error_flag = 1u;
  if (a.grad) {
    const float scale = *a.outer / static_cast<float>(a.batch);  // autograd.rs:540-541
    // p = e / normalizer (autograd.rs:548) as e * (1 / normalizer): within 1.5 ulp of the
    // correctly rounded quotient, one division per row instead of one per logit.  The target
    // logit keeps the exact quotient because p - 1 cancels.
    const float rinv = 1.0f / normalizer;
    float4 *g4 = reinterpret_cast<float4 *>(a.grad + row * a.classes);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const uint64_t i = threadIdx.x + static_cast<uint64_t>(k) * BLOCK;
      if (i < c4) {
        float4 r;
        if (valid) {
          r.x = scale * (v[k].x * rinv);
          r.y = scale * (v[k].y * rinv);
          r.z = scale * (v[k].z * rinv);
          r.w = scale * (v[k].w * rinv);
          const uint64_t e = 4 * i;
          if (target >= e && target < e + 4) {
            const int t = static_cast<int>(target - e);
            const float et = t == 0 ? v[k].x : t == 1 ? v[k].y : t == 2 ? v[k].z : v[k].w;
            const float gt = scale * (et / normalizer - 1.0f);
            if (t == 0) r.x = gt;
            else if (t == 1) r.y = gt;
            else if (t == 2) r.z = gt;
            else r.w = gt;
          }
        } else {
          r = make_float4(NAN, NAN, NAN, NAN);
        }
        g4[i] = r;
      }
    }
  }
  const float row_loss =
      valid ? logf(normalizer) + maximum - a.logits[row * a.classes + target] : NAN;
  finish_row(a, row, row_loss);
}

// General path: any classes, any alignment; three strided passes over the row.
constexpr int kGenBlock = 256;

__global__ __launch_bounds__(kGenBlock) void ce_row_general_kernel(CeArgs a) {
  __shared__ float lds_f[kGenBlock / 64];
  __shared__ double lds_d[kGenBlock / 64];
  const uint64_t row = blockIdx.x;
  const float *x = a.logits + row * a.classes;
  float m = -INFINITY;
  for (uint64_t i = threadIdx.x; i < a.classes; i += kGenBlock) m = fmaxf(m, x[i]);
  const float maximum = block_max<kGenBlock>(m, lds_f);
  double s = 0.0;
  for (uint64_t i = threadIdx.x; i < a.classes; i += kGenBlock)
    s += static_cast<double>(expf(x[i] - maximum));
  const float normalizer = static_cast<float>(block_sum<kGenBlock>(s, lds_d));
  uint64_t target = 0;
  const bool valid = target_index(a.targets[row], a.classes, target);
  if (!valid && threadIdx.x == 0 && a.error_flag) *a.error_flag = 1u;
  if (a.grad) {
    const float scale = *a.outer / static_cast<float>(a.batch);
    float *g = a.grad + row * a.classes;
    for (uint64_t i = threadIdx.x; i < a.classes; i += kGenBlock) {
      const float p = expf(x[i] - maximum) / normalizer;
      g[i] = valid ? scale * (p - (i == target ? 1.0f : 0.0f)) : NAN;
    }
  }
  const float row_loss = valid ? logf(normalizer) + maximum - x[target] : NAN;
  finish_row(a, row, row_loss);
}

uint64_t ce_workspace_bytes(uint64_t batch) { return (batch * 8 + 255) / 256 * 256; }

oxh_status launch_ce(const char *name, oxh_stream stream, CeArgs a, void *workspace,
                     uint64_t workspace_bytes) {
  OXH_REQUIRE(a.batch > 0 && a.classes > 0, OXH_INVALID_SHAPE,
              std::string(name) + ": empty logits");
  OXH_REQUIRE(a.batch < (1ull << 31) && a.classes < (1ull << 40) &&
                  a.batch * a.classes < (1ull << 42),
              OXH_INVALID_SHAPE, std::string(name) + ": logits too large");
  OXH_REQUIRE(a.logits && a.targets, OXH_INVALID_SHAPE, std::string(name) + ": null input");
  OXH_REQUIRE(!a.grad || a.outer, OXH_INVALID_SHAPE,
              std::string(name) + ": the gradient needs the upstream gradient scalar");
  const uint64_t bytes = a.batch * a.classes * 4;
  if (a.grad)
    OXH_REQUIRE(!oxh::any_overlap(a.grad, bytes, a.logits, bytes), OXH_INVALID_SHAPE,
                std::string(name) + ": gradient overlaps the logits");
  if (a.loss) {
    const uint64_t need = ce_workspace_bytes(a.batch);
    OXH_REQUIRE(workspace != nullptr && workspace_bytes >= need, OXH_INVALID_SHAPE,
                std::string(name) + ": workspace of " + std::to_string(need) +
                    " bytes required (oxh_cross_entropy_workspace_size)");
    OXH_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 7u) == 0, OXH_INVALID_SHAPE,
                std::string(name) + ": workspace must be 8-byte aligned");
    a.row_loss = static_cast<double *>(workspace);
    OXH_REQUIRE(!oxh::any_overlap(workspace, need, a.logits, bytes) &&
                    (!a.grad || !oxh::any_overlap(workspace, need, a.grad, bytes)),
                OXH_INVALID_SHAPE, std::string(name) + ": workspace overlaps the logits or grad");
  }
  hipStream_t s = oxh::as_stream(stream);
  const dim3 grid(static_cast<uint32_t>(a.batch));
  const bool vec = a.classes % 4 == 0 && oxh::aligned16(a.logits) &&
                   (!a.grad || oxh::aligned16(a.grad));
  const uint64_t c4 = a.classes / 4;
  constexpr int B = OXH_CE_BLOCK, W = OXH_CE_MINW;
  if (vec && c4 <= 256) {
    oxh::launch((ce_row_kernel<256, 1, 2>), grid, dim3(256), 0, s, a);
  } else if (vec && c4 <= 256 * 4) {
    oxh::launch((ce_row_kernel<256, 4, 2>), grid, dim3(256), 0, s, a);
  } else if (vec && c4 <= B * 2) {
    oxh::launch((ce_row_kernel<B, 2, W>), grid, dim3(B), 0, s, a);
  } else if (vec && c4 <= B * 4) {
    oxh::launch((ce_row_kernel<B, 4, W>), grid, dim3(B), 0, s, a);
  } else if (vec && c4 <= B * 8) {
    oxh::launch((ce_row_kernel<B, 8, W>), grid, dim3(B), 0, s, a);
  } else if (vec && c4 <= B * 16) {
    oxh::launch((ce_row_kernel<B, 16, (W > 4 ? 4 : W)>), grid, dim3(B), 0, s, a);
  } else if (vec && B <= 256 && c4 <= B * 32) {
    if constexpr (B <= 256)
      oxh::launch((ce_row_kernel<B, 32, (W > 2 ? 2 : W)>), grid, dim3(B), 0, s, a);
  } else {
    oxh::launch(ce_row_general_kernel, grid, dim3(kGenBlock), 0, s, a);
  }
  oxh_status st = oxh::launched(name);
  if (st != OXH_OK || a.loss == nullptr) return st;
  oxh::launch(ce_mean_kernel, dim3(1), dim3(kMeanBlock), 0, s, a.row_loss, a.batch,
                     a.loss);
  return oxh::launched(name);
}

}  // namespace

extern "C" {

oxh_status oxh_cross_entropy_workspace_size(uint64_t batch, uint64_t classes, uint64_t *bytes) {
  OXH_REQUIRE(bytes != nullptr, OXH_INVALID_SHAPE, "bytes is null");
  OXH_REQUIRE(batch > 0 && classes > 0, OXH_INVALID_SHAPE, "empty logits");
  *bytes = ce_workspace_bytes(batch);
  return oxh::ok();
}

oxh_status oxh_cross_entropy_forward(oxh_stream stream, uint64_t batch, uint64_t classes,
                                     const float *logits, const float *targets, float *loss,
                                     uint32_t *error_flag, void *workspace,
                                     uint64_t workspace_bytes) {
  OXH_REQUIRE(loss != nullptr, OXH_INVALID_SHAPE, "oxh_cross_entropy_forward: null loss");
  CeArgs a{logits, targets, nullptr, loss, nullptr, error_flag, nullptr, batch, classes};
  return launch_ce("oxh_cross_entropy_forward", stream, a, workspace, workspace_bytes);
}

oxh_status oxh_cross_entropy_backward(oxh_stream stream, uint64_t batch, uint64_t classes,
                                      const float *logits, const float *targets,
                                      const float *outer_gradient, float *grad,
                                      uint32_t *error_flag) {
  OXH_REQUIRE(grad != nullptr, OXH_INVALID_SHAPE, "oxh_cross_entropy_backward: null grad");
  CeArgs a{logits, targets, outer_gradient, nullptr, grad, error_flag, nullptr, batch, classes};
  return launch_ce("oxh_cross_entropy_backward", stream, a, nullptr, 0);
}

oxh_status oxh_cross_entropy_forward_backward(oxh_stream stream, uint64_t batch,
                                              uint64_t classes, const float *logits,
                                              const float *targets,
                                              const float *outer_gradient, float *loss,
                                              float *grad, uint32_t *error_flag,
                                              void *workspace, uint64_t workspace_bytes) {
  OXH_REQUIRE(loss != nullptr && grad != nullptr, OXH_INVALID_SHAPE,
              "oxh_cross_entropy_forward_backward: null output");
  CeArgs a{logits, targets, outer_gradient, loss, grad, error_flag, nullptr, batch, classes};
  return launch_ce("oxh_cross_entropy_forward_backward", stream, a, workspace,
                   workspace_bytes);
}

}  // extern "C"
