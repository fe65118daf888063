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
#ifndef OXH_CE_NT
#define OXH_CE_NT 3  // ce_row_kernel: 1 non-temporal logit loads, 2 gradient stores, 3 both
#endif
#ifndef OXH_CE_MINW
#define OXH_CE_MINW 4
#endif
#ifndef OXH_CE_MINW16
#define OXH_CE_MINW16 (OXH_CE_MINW > 4 ? 4 : OXH_CE_MINW)  // 16 float4 per lane
#endif
#ifndef OXH_CE_MINW32
#define OXH_CE_MINW32 (OXH_CE_MINW > 2 ? 2 : OXH_CE_MINW)  // 32 float4 per lane
#endif
constexpr int kMinW16 = OXH_CE_MINW16, kMinW32 = OXH_CE_MINW32;
#ifndef OXH_CE_PIPE_BLOCK
#define OXH_CE_PIPE_BLOCK 512  // pipelined path: lanes per row block (0: path off)
#endif
#ifndef OXH_CE_PIPE_GRID
#define OXH_CE_PIPE_GRID 512  // pipelined path: blocks (two rounds of one block per CU)
#endif

// The pipelined path serves rows of 4 * kPipeBlock * kPipeV classes (32 768 at 512 lanes).
constexpr int kPipeBlock = OXH_CE_PIPE_BLOCK > 0 ? OXH_CE_PIPE_BLOCK : 512;
#ifndef OXH_CE_PIPE_V
#define OXH_CE_PIPE_V 16
#endif
constexpr int kPipeV = OXH_CE_PIPE_V;
constexpr uint32_t kPipeGrid = OXH_CE_PIPE_BLOCK > 0 ? OXH_CE_PIPE_GRID : 0xFFFFFFFFu;

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

// Block max: within each row of 16 lanes through DPP moves (xor 1, xor 2, mirrored half, mirrored
// row: every lane then holds its row's max), the four rows through lane reads, then the waves
// through LDS.  max is exact, so the order is immaterial.
template <int BLOCK>
__device__ __forceinline__ float block_max(float v, float *lds) {
  v = fmaxf(v, oxh::dpp_move<0xB1>(v));
  v = fmaxf(v, oxh::dpp_move<0x4E>(v));
  v = fmaxf(v, oxh::dpp_move<0x141>(v));
  v = fmaxf(v, oxh::dpp_move<0x140>(v));
  v = fmaxf(fmaxf(oxh::read_lane(v, 0), oxh::read_lane(v, 16)),
            fmaxf(oxh::read_lane(v, 32), oxh::read_lane(v, 48)));
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

// Block sum in a fixed order: oxh::wave_sums_rows within each wave, then the waves in order.
template <int BLOCK>
__device__ __forceinline__ double block_sum(double v, double *lds) {
  double w[1] = {v};
  oxh::wave_sums_rows(w);
  v = w[0];
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
constexpr int kMeanBlock = 1024, kMeanLoads = 8;

__global__ __launch_bounds__(kMeanBlock) void ce_mean_kernel(const double *__restrict__ row_loss,
                                                             uint64_t batch, float *loss) {
  __shared__ double lds[kMeanBlock / 64];
  double s = 0.0;
  // kMeanLoads loads in flight per round (the row losses come from other XCDs' writes: one
  // memory round trip each), then the adds in row order
  for (uint64_t base = 0; base < batch; base += kMeanBlock * kMeanLoads) {
    double v[kMeanLoads];
#pragma unroll
    for (int i = 0; i < kMeanLoads; ++i) {
      const uint64_t r = base + threadIdx.x + static_cast<uint64_t>(i) * kMeanBlock;
      v[i] = r < batch ? row_loss[r] : 0.0;
    }
#pragma unroll
    for (int i = 0; i < kMeanLoads; ++i)
      if (base + threadIdx.x + static_cast<uint64_t>(i) * kMeanBlock < batch) s += v[i];
  }
  s = block_sum<kMeanBlock>(s, lds);
  if (threadIdx.x == 0) *loss = static_cast<float>(s) / static_cast<float>(batch);
}

// exp(d) for d = x - rowmax <= 0, within ~1.5 ulp: 2^(d * log2 e) with the product carried as
// hi + lo (an exact fma residual plus d times the tail of log2 e), the hardware 2^x (v_exp_f32,
// 1 ulp) on the fraction |f| <= 0.5 + 2^-24, and the integer part applied by ldexp.  NaN
// propagates; d below -200 (including -inf) gives 0, as expf does.
__device__ __forceinline__ float exp_nonpos(float d) {
  constexpr float kLog2eHi = 1.44269502162933349609375f;  // nearest float to log2(e)
  constexpr float kLog2eLo = 1.925963033500011e-08f;      // log2(e) - kLog2eHi
  d = d < -200.0f ? -200.0f : d;
  const float hi = d * kLog2eHi;
  const float lo = fmaf(d, kLog2eLo, fmaf(d, kLog2eHi, -hi));
  const float n = rintf(hi);
  const float f = (hi - n) + lo;  // hi - n is exact
  return ldexpf(__builtin_amdgcn_exp2f(f), static_cast<int>(n));
}

__device__ __forceinline__ float4 exp4_nonpos(const float4 &x, float m) {
  return make_float4(exp_nonpos(x.x - m), exp_nonpos(x.y - m), exp_nonpos(x.z - m),
                     exp_nonpos(x.w - m));
}

// Register path: BLOCK lanes x V float4 hold one row of `classes` (= 4 * c4) logits.  MINW
// (waves per SIMD the compiler must allow) bounds the VGPRs so several rows share a CU and one
// row's memory phase overlaps another's exp / reduction phase.  FULL: c4 == BLOCK * V, so no
// lane needs a bounds check.
template <int BLOCK, int V, int MINW, bool FULL>
__global__ __launch_bounds__(BLOCK, MINW) void ce_row_kernel(CeArgs a) {
  __shared__ float lds_f[BLOCK / 64];
  __shared__ double lds_d[BLOCK / 64];
  const uint64_t row = blockIdx.x;
  const uint32_t c4 = static_cast<uint32_t>(a.classes / 4);
  const float4 *x4 = reinterpret_cast<const float4 *>(a.logits + row * a.classes);
  // loaded with the row (read after the reductions they would add a memory round trip)
  const float target_value = a.targets[row];
  const float outer = a.grad ? *a.outer : 0.0f;
  auto in_row = [&](int k) { return FULL || threadIdx.x + static_cast<uint32_t>(k) * BLOCK < c4; };
  float4 v[V];
#pragma unroll
  for (int k = 0; k < V; ++k)
    v[k] = !in_row(k) ? make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY)
           : (OXH_CE_NT & 1) != 0 ? oxh::load_nt(x4 + threadIdx.x + k * BLOCK)
                                  : x4[threadIdx.x + k * BLOCK];
  // row max: fold(-inf, f32::max) in any order gives the same value (evaluation.rs:609)
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < V; ++k) m = fmaxf(m, fmaxf(fmaxf(v[k].x, v[k].y), fmaxf(v[k].z, v[k].w)));
  const float maximum = block_max<BLOCK>(m, lds_f);
  // e = exp(x - max) kept in place; per-lane pairwise fp32 sums, fp64 across lanes
  float part[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    if (in_row(k)) {
      v[k] = exp4_nonpos(v[k], maximum);
      part[k] = (v[k].x + v[k].y) + (v[k].z + v[k].w);
    } else {
      part[k] = 0.0f;
    }
  }
#pragma unroll
  for (int w = 1; w < V; w *= 2)
#pragma unroll
    for (int k = 0; k + w < V; k += 2 * w) part[k] += part[k + w];
  const float normalizer = static_cast<float>(block_sum<BLOCK>(static_cast<double>(part[0]), lds_d));
  uint64_t target = 0;
  const bool valid = target_index(target_value, a.classes, target);
  if (!valid && threadIdx.x == 0 && a.error_flag) *a.error_flag = 1u;
  if (a.grad) {
    float4 *g4 = reinterpret_cast<float4 *>(a.grad + row * a.classes);
    if (!valid) {
#pragma unroll
      for (int k = 0; k < V; ++k)
        if (in_row(k)) g4[threadIdx.x + k * BLOCK] = make_float4(NAN, NAN, NAN, NAN);
    } else {
      // grad = (outer / B) * (e / normalizer - onehot) (autograd.rs:540-551).  Off-target:
      // e * ((outer / B) / normalizer), within 2.5 ulp of the CPU's scale * (e / normalizer),
      // one multiply per logit.  The target logit keeps scale * (e / normalizer - 1) exactly,
      // since the subtraction cancels.
      const float scale = outer / static_cast<float>(a.batch);
      const float sr = scale / normalizer;
      const uint32_t t4 = static_cast<uint32_t>(target / 4);
      const uint32_t owner = t4 % BLOCK, kt = t4 / BLOCK, ct = static_cast<uint32_t>(target % 4);
#pragma unroll
      for (int k = 0; k < V; ++k) {
        if (!in_row(k)) continue;
        float4 r = make_float4(v[k].x * sr, v[k].y * sr, v[k].z * sr, v[k].w * sr);
        if (static_cast<uint32_t>(k) == kt && threadIdx.x == owner) {
          const float et = ct == 0 ? v[k].x : ct == 1 ? v[k].y : ct == 2 ? v[k].z : v[k].w;
          const float gt = scale * (et / normalizer - 1.0f);
          if (ct == 0) r.x = gt;
          else if (ct == 1) r.y = gt;
          else if (ct == 2) r.z = gt;
          else r.w = gt;
        }
        if constexpr ((OXH_CE_NT & 2) != 0) oxh::store_nt(g4 + threadIdx.x + k * BLOCK, r);
        else g4[threadIdx.x + k * BLOCK] = r;
      }
    }
  }
  const float row_loss =
      valid ? logf(normalizer) + maximum - a.logits[row * a.classes + target] : NAN;
  finish_row(a, row, row_loss);
}

// Pipelined register path for full rows (classes = 4 * BLOCK * V) when the gradient is written:
// a block keeps two rows in VGPRs and walks rows blockIdx.x, blockIdx.x + gridDim.x, ...; the
// next row's loads are issued before the current row's reductions, exp and gradient stores, so
// a CU's memory pipe stays busy through the compute phases (barriers wait only on LDS, never on
// outstanding global loads).  At 227 VGPRs (two waves per SIMD) one 512-lane block fills a CU,
// so the 512-block grid runs as two rounds of 16-row blocks per CU, the second round filling in
// as CUs finish: 357 us, against 366 us for one 32-row block per CU, 367 us for three rounds
// (768 blocks), 373-377 us for four or more (1024, 2048) and 422 us for 384 blocks (half the
// CUs idle in the second round).  Measured at [8192, 32768] fused, one block per CU: 375 us
// against 378-412 us for two independent row blocks per CU (whose load, compute and store
// phases fall into step); a forward alone (reads only) is faster with the two independent
// blocks (160 against 225 us), so it keeps them.  The logits and the gradient move
// through non-temporal buffer loads and stores on a per-row resource (the lane's offset in a
// VGPR, the part's offset k * BLOCK * 16 in a scalar): 364 against 373 us with 64-bit lane
// addresses.  Cache policy sweep (this kernel, [8192, 32768]): the default policy costs 15 us on
// the loads and 35 us on the stores; adding sc0 or sc1 to nt changes nothing (357-358 us).
// The same launch copying the rows without the softmax takes as long (366 us), so
// the arithmetic is hidden and the row-per-CU access pattern sets the rate.  Nothing is read
// from global memory after the next row's loads are in flight: the target logit comes from the
// owner lane's registers, which also writes the row's loss.  Arithmetic per element and per row
// as ce_row_kernel.
constexpr int kBufferNt = 2;  // buffer instruction cache policy: non-temporal
typedef unsigned u32x4_t __attribute__((vector_size(16)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_resource(const float *row, uint64_t classes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(row), 0,
                                           static_cast<int>(classes * 4), 0x00020000);
}

template <int BLOCK, int V>
__device__ __forceinline__ void ce_pipe_load(const CeArgs &a, uint64_t row, float4 (&v)[V],
                                             float &target_value) {
  const __amdgpu_buffer_rsrc_t r = row_resource(a.logits + row * a.classes, a.classes);
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const u32x4_t u =
        __builtin_amdgcn_raw_buffer_load_b128(r, threadIdx.x * 16, k * BLOCK * 16, kBufferNt);
    v[k] = make_float4(__uint_as_float(u[0]), __uint_as_float(u[1]), __uint_as_float(u[2]),
                       __uint_as_float(u[3]));
  }
  target_value = a.targets[row];
}

__device__ __forceinline__ float component(const float4 &v, uint32_t c) {
  return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w;
}

template <int BLOCK, int V>
__device__ __forceinline__ void ce_pipe_row(const CeArgs &a, uint64_t row, float4 (&v)[V],
                                            float target_value, float outer, float *lds_f,
                                            double *lds_d) {
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < V; ++k) m = fmaxf(m, fmaxf(fmaxf(v[k].x, v[k].y), fmaxf(v[k].z, v[k].w)));
  const float maximum = block_max<BLOCK>(m, lds_f);
  uint64_t target = 0;
  const bool valid = target_index(target_value, a.classes, target);
  const uint32_t t4 = static_cast<uint32_t>(target / 4);
  const uint32_t owner = t4 % BLOCK, kt = t4 / BLOCK, ct = static_cast<uint32_t>(target % 4);
  const bool own = valid && threadIdx.x == owner;
  // the target's logit and exp by selects (kt and ct are uniform; only the owner lane's values
  // are used), so no lane diverges
  float xt = 0.0f, et = 0.0f;
#pragma unroll
  for (int k = 0; k < V; ++k) xt = static_cast<uint32_t>(k) == kt ? component(v[k], ct) : xt;
  float part[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    v[k] = exp4_nonpos(v[k], maximum);
    part[k] = (v[k].x + v[k].y) + (v[k].z + v[k].w);
    et = static_cast<uint32_t>(k) == kt ? component(v[k], ct) : et;
  }
#pragma unroll
  for (int w = 1; w < V; w *= 2)
#pragma unroll
    for (int k = 0; k + w < V; k += 2 * w) part[k] += part[k + w];
  const float normalizer =
      static_cast<float>(block_sum<BLOCK>(static_cast<double>(part[0]), lds_d));
  if (!valid && threadIdx.x == 0 && a.error_flag) *a.error_flag = 1u;
  if (a.grad) {
    const __amdgpu_buffer_rsrc_t gr = row_resource(a.grad + row * a.classes, a.classes);
    const float scale = outer / static_cast<float>(a.batch);
    const float sr = scale / normalizer;
    const float gt = scale * (et / normalizer - 1.0f);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      float4 r = valid ? make_float4(v[k].x * sr, v[k].y * sr, v[k].z * sr, v[k].w * sr)
                       : make_float4(NAN, NAN, NAN, NAN);
      const bool here = own && static_cast<uint32_t>(k) == kt;
      r.x = here && ct == 0 ? gt : r.x;
      r.y = here && ct == 1 ? gt : r.y;
      r.z = here && ct == 2 ? gt : r.z;
      r.w = here && ct == 3 ? gt : r.w;
      const u32x4_t u = {__float_as_uint(r.x), __float_as_uint(r.y), __float_as_uint(r.z),
                         __float_as_uint(r.w)};
      __builtin_amdgcn_raw_buffer_store_b128(u, gr, threadIdx.x * 16, k * BLOCK * 16, kBufferNt);
    }
  }
  if (a.loss != nullptr && (valid ? own : threadIdx.x == 0))
    a.row_loss[row] = static_cast<double>(valid ? logf(normalizer) + maximum - xt : NAN);
}

template <int BLOCK, int V>
__global__ __launch_bounds__(BLOCK, 2 * 64 * 4 / BLOCK) void ce_row_pipelined_kernel(CeArgs a) {
  __shared__ float lds_f[BLOCK / 64];
  __shared__ double lds_d[BLOCK / 64];
  const float outer = a.grad ? *a.outer : 0.0f;
  const uint64_t stride = gridDim.x;
  uint64_t row = blockIdx.x;  // < batch: the grid never exceeds the rows
  float4 v0[V], v1[V];
  float t0 = 0.0f, t1 = 0.0f;
  ce_pipe_load<BLOCK, V>(a, row, v0, t0);
  // The trip count depends on blockIdx only (uniform over the block).  Each branch has its own
  // copy of the row body, so the wait before a row's first use of its registers counts only
  // the loads issued after them on that path (a merge of a path with and one without the next
  // row's loads would wait for every outstanding load).
  for (;;) {
    uint64_t next = row + stride;
    if (next < a.batch) {
      ce_pipe_load<BLOCK, V>(a, next, v1, t1);
      ce_pipe_row<BLOCK, V>(a, row, v0, t0, outer, lds_f, lds_d);
    } else {
      ce_pipe_row<BLOCK, V>(a, row, v0, t0, outer, lds_f, lds_d);
      break;
    }
    row = next;
    next = row + stride;
    if (next < a.batch) {
      ce_pipe_load<BLOCK, V>(a, next, v0, t0);
      ce_pipe_row<BLOCK, V>(a, row, v1, t1, outer, lds_f, lds_d);
    } else {
      ce_pipe_row<BLOCK, V>(a, row, v1, t1, outer, lds_f, lds_d);
      break;
    }
    row = next;
  }
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

// Small problems (at most kSmallRows rows of at most kSmallClasses classes, e.g. a batch of
// MNIST logits): one block, one thread per row running the general kernel's per-row steps
// serially, and the batch mean in the same launch -- the fp64 row losses summed in
// ce_mean_kernel's order (thread t holds row t).
constexpr int kSmallRows = 1024;
constexpr uint64_t kSmallClasses = 64;

// One thread per row, the block as many waves as the rows fill.  The row's C <= 64 logits are
// loaded at once (indices clamped into the row, the extra lanes of the array unused), each exp
// is formed once and kept for the gradient; sums in class order (fp64), as the CPU path.  The
// batch loss: wave sums, then the block's waves in order (bit-identical to a block of 1024
// threads whose extra rows add 0).
template <int C>
__global__ __launch_bounds__(kSmallRows) void ce_small_kernel(CeArgs a) {
  __shared__ double lds[kSmallRows / 64];
  const uint64_t row = threadIdx.x;
  double row_loss = 0.0;
  if (row < a.batch) {
    const uint32_t classes = static_cast<uint32_t>(a.classes);
    const float *x = a.logits + row * a.classes;
    float v[C];
#pragma unroll
    for (int i = 0; i < C; ++i) v[i] = x[static_cast<uint32_t>(i) < classes ? i : classes - 1];
    const float target_value = a.targets[row];
    float maximum = -INFINITY;
#pragma unroll
    for (int i = 0; i < C; ++i)
      if (static_cast<uint32_t>(i) < classes) maximum = fmaxf(maximum, v[i]);
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < C; ++i) {
      if (static_cast<uint32_t>(i) < classes) {
        v[i] = expf(v[i] - maximum);  // v now holds e
        s += static_cast<double>(v[i]);
      }
    }
    const float normalizer = static_cast<float>(s);
    uint64_t target = 0;
    const bool valid = target_index(target_value, a.classes, target);
    if (!valid && a.error_flag) *a.error_flag = 1u;
    if (a.grad) {
      const float scale = *a.outer / static_cast<float>(a.batch);
      float *g = a.grad + row * a.classes;
#pragma unroll
      for (int i = 0; i < C; ++i) {
        if (static_cast<uint32_t>(i) < classes) {
          const float p = v[i] / normalizer;
          g[i] = valid ? scale * (p - (static_cast<uint64_t>(i) == target ? 1.0f : 0.0f)) : NAN;
        }
      }
    }
    row_loss = static_cast<double>(valid ? logf(normalizer) + maximum - x[target] : NAN);
  }
  if (a.loss != nullptr) {
    double w[1] = {row_loss};
    oxh::wave_sums_rows(w);
    const uint32_t waves = blockDim.x / 64, wave = threadIdx.x / 64;
    if (threadIdx.x % 64 == 0) lds[wave] = w[0];
    __syncthreads();
    if (threadIdx.x == 0) {
      double total = 0.0;
      for (uint32_t i = 0; i < waves; ++i) total += lds[i];
      *a.loss = static_cast<float>(total) / static_cast<float>(a.batch);
    }
  }
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
  if (a.batch <= static_cast<uint64_t>(kSmallRows) && a.classes <= kSmallClasses) {
    const dim3 block(static_cast<uint32_t>((a.batch + 63) / 64 * 64));
    if (a.classes <= 16) oxh::launch(ce_small_kernel<16>, dim3(1), block, 0, s, a);
    else if (a.classes <= 32) oxh::launch(ce_small_kernel<32>, dim3(1), block, 0, s, a);
    else oxh::launch(ce_small_kernel<64>, dim3(1), block, 0, s, a);
    return oxh::launched(name);
  }
  const dim3 grid(static_cast<uint32_t>(a.batch));
  const bool vec = a.classes % 4 == 0 && oxh::aligned16(a.logits) &&
                   (!a.grad || oxh::aligned16(a.grad));
  const uint64_t c4 = a.classes / 4;
  constexpr int B = OXH_CE_BLOCK, W = OXH_CE_MINW;
  auto row = [&](auto kernel, int block) {
    oxh::launch(kernel, grid, dim3(block), 0, s, a);
  };
  if (vec && c4 == 256) {
    row(ce_row_kernel<256, 1, 2, true>, 256);
  } else if (vec && c4 <= 256) {
    row(ce_row_kernel<256, 1, 2, false>, 256);
  } else if (vec && c4 == 256 * 4) {
    row(ce_row_kernel<256, 4, 2, true>, 256);
  } else if (vec && c4 <= 256 * 4) {
    row(ce_row_kernel<256, 4, 2, false>, 256);
  } else if (vec && c4 <= B * 2) {
    row(ce_row_kernel<B, 2, W, false>, B);
  } else if (vec && c4 <= B * 4) {
    row(ce_row_kernel<B, 4, W, false>, B);
  } else if (vec && c4 == B * 8) {
    row(ce_row_kernel<B, 8, W, true>, B);
  } else if (vec && c4 <= B * 8) {
    row(ce_row_kernel<B, 8, W, false>, B);
  } else if (vec && a.grad && c4 == kPipeBlock * kPipeV && a.batch >= 2 * kPipeGrid) {
    oxh::launch(ce_row_pipelined_kernel<kPipeBlock, kPipeV>, dim3(kPipeGrid), dim3(kPipeBlock),
                0, s, a);
  } else if (vec && c4 == B * 16) {
    row(ce_row_kernel<B, 16, kMinW16, true>, B);
  } else if (vec && c4 <= B * 16) {
    row(ce_row_kernel<B, 16, kMinW16, false>, B);
  } else if (vec && B <= 256 && c4 == B * 32) {
    if constexpr (B <= 256) row(ce_row_kernel<B, 32, kMinW32, true>, B);
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
