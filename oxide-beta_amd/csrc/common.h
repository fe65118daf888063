// common.h -- internal helpers shared by the liboxide_hip.so translation units.
//
// Error reporting (thread-local message + status), host-side argument checks and the launch
// geometry used by the streaming kernels.  gfx950 only: wave64, 256 CUs in 8 XCDs.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "oxide_hip.h"

namespace oxh {

// Looks up this device's copy of the batch-norm static scratch array (the allocation-free
// forward's partials); `device` must be current.  Called by oxh_init.
oxh_status bn_scratch_init(int device);

// Whether a training BatchNorm of this shape runs one block per channel (its backward then
// sums the input gradient per channel in passing: a preceding convolution's bias gradient).
bool batch_norm_single_launch(uint64_t batch, uint64_t channels, uint64_t spatial);

// One weight-gradient chunk sum: out[e] (e < split) or out2[e - split] (split <= e < count)
// = the fixed-order sum over `chunks` of partial[chunk * count + e].
struct ChunkSum {
  const float *partial;
  float *out, *out2;
  uint32_t count, chunks, split;
};

// oxh_conv2d_backward (same arguments and checks) with its weight-gradient chunk sums, if it
// has any, appended to `deferred` in place of launched: the weight (and bias) gradient holds
// its value only once the caller has run them (launch_chunk_sums), and the workspace must stay
// untouched until then.
oxh_status conv2d_backward_deferred(oxh_stream stream, const oxh_conv2d_shape *shape,
                                    const float *gradient, const float *input,
                                    const float *weight, const float *addend,
                                    float *input_gradient, float *weight_gradient,
                                    float *bias_gradient, void *workspace,
                                    uint64_t workspace_bytes, std::vector<ChunkSum> &deferred);

// Every sum of `sums` (each element the same sum as the convolution's own launch forms) in one
// launch per kChunkSumsPerLaunch sums (at least one launch); with `step` not null, the first
// launch also advances the optimizer step counter (*step += 1).
constexpr uint32_t kChunkSumsPerLaunch = 16;
oxh_status launch_chunk_sums(hipStream_t stream, const std::vector<ChunkSum> &sums,
                             int32_t *step);

// oxh_adamw_multi_tensor_table_step without its step counter advance (the caller has
// advanced it, e.g. by launch_chunk_sums).
oxh_status adamw_table_step_advanced(hipStream_t stream, float learning_rate,
                                     float weight_decay, float beta1, float beta2, float epsilon,
                                     const int32_t *step, const oxh_adamw_tensor *device_tensors,
                                     const uint32_t *device_chunk_starts, uint32_t count,
                                     uint64_t total_chunks);

// Records `message` as the calling thread's last error and returns `status`.
oxh_status fail(oxh_status status, const std::string &message);
// Clears the last error; returns OXH_OK.
oxh_status ok();

// Maps a HIP error to OXH_HIP_ERROR with the failing call named.
inline oxh_status hip_status(hipError_t err, const char *what) {
  if (err == hipSuccess) return ok();
  return fail(OXH_HIP_ERROR, std::string(what) + ": " + hipGetErrorString(err));
}

// Launch check: catches a bad launch configuration immediately (asynchronous faults surface
// at the next synchronizing call, as in the reference).
inline oxh_status launched(const char *kernel) { return hip_status(hipGetLastError(), kernel); }

inline hipStream_t as_stream(oxh_stream s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Streaming kernels: 256 threads (4 waves) per block.
constexpr int kBlock = 256;

// Number of compute units on gfx950 (MI355X); used to size reductions so that every CU gets
// several workgroups.
constexpr int kComputeUnits = 256;

// Checks that the n-element buffers do not partially overlap (exact aliasing is allowed for
// in-place elementwise updates).
inline bool partial_overlap(const void *a, const void *b, uint64_t bytes) {
  auto x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  if (x == y) return false;
  return x < y + bytes && y < x + bytes;
}
inline bool any_overlap(const void *a, uint64_t abytes, const void *b, uint64_t bbytes) {
  auto x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + bbytes && y < x + abytes;
}

// Division of a 32-bit dividend below 2^31 by a runtime-invariant divisor d >= 1 with one
// high multiply (Granlund & Montgomery, "Division by invariant integers using
// multiplication", 1994, round-up method): q = (umulhi(n, mul) + n) >> shift.
struct FastDiv {
  uint32_t d, mul, shift;
};

__host__ __device__ inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{d, 0, 0};
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  f.shift = s;
  f.mul = static_cast<uint32_t>(((1ull << 32) * ((1ull << s) - d)) / d + 1);
  return f;
}

__device__ __forceinline__ uint32_t fast_div(uint32_t n, const FastDiv &f) {
  return (__umulhi(n, f.mul) + n) >> f.shift;
}

#ifndef OXH_XCD_REMAP
#define OXH_XCD_REMAP 1  // 1: tiled kernels give each XCD a contiguous run of their tiles
#endif

// Workgroups reach the 8 XCDs round-robin in dispatch order (linear id, x fastest), and each
// XCD has its own L2.  For the ids [base, base + count) of a grid, xcd_contiguous maps the
// local id l (the workgroup base + l, on XCD (base + l) % 8) to the tile it computes so that
// each XCD takes one contiguous run of count / 8 tiles (ids at or past the largest multiple of
// 8 keep theirs).  Neighbouring tiles share operand rows (one image's input, one strip of
// weights), which one L2 then fetches once instead of every XCD fetching all of them.  A
// bijection: XCD s takes l = ((s - base) mod 8) + 8 k, k < count / 8, as tile s * count / 8 + k.
__device__ __forceinline__ uint32_t xcd_contiguous(uint32_t l, uint32_t count,
                                                   uint32_t base = 0) {
  if constexpr (OXH_XCD_REMAP == 0) return l;
  const uint32_t per = count >> 3;
  return l < (per << 3) ? ((base + l) & 7u) * per + (l >> 3) : l;
}
struct BlockTile {
  uint32_t x, y, z;
};
// blockIdx remapped over the whole grid as above.
__device__ __forceinline__ BlockTile xcd_block() {
  const uint32_t gx = gridDim.x, gy = gridDim.y;
  const uint32_t id = (blockIdx.z * gy + blockIdx.y) * gx + blockIdx.x;
  const uint32_t r = xcd_contiguous(id, gx * gy * gridDim.z);
  const uint32_t xy = r % (gx * gy);
  return {xy % gx, xy / gx, r / (gx * gy)};
}

// Convolution tap terms: p where mask is all ones, else -0.0f (x + (-0.0f) == x for every x),
// the term of a tap outside the input, so a sum over all taps equals the CPU path's sum that
// skips them, bit for bit.  Bit operations rather than a select keep the tap's loads
// unconditional (the compiler turns a select on a loaded value into a branch around the load).
__device__ __forceinline__ float tap_term(float p, uint32_t mask) {
  return __uint_as_float((__float_as_uint(p) & mask) | (~mask & 0x80000000u));
}
__device__ __forceinline__ uint32_t tap_mask(bool valid) { return valid ? 0xFFFFFFFFu : 0u; }
// An operand read at a tap outside the input, replaced by +0 (one AND for every product that
// shares it): its products are +-0, which leave a sum unchanged except for the sign of an
// exactly zero sum, when the other factor is finite.
__device__ __forceinline__ float tap_operand(float v, uint32_t mask) {
  return __uint_as_float(__float_as_uint(v) & mask);
}

// Cross-lane moves within rows of 16 lanes through the DPP crossbar (no LDS traffic, unlike
// __shfl_xor's ds_bpermute).  Controls (DPP_CTRL, GCN3 / Vega ISA): quad_perm [1,0,3,2] and
// [2,3,0,1] (lane ^ 1, lane ^ 2), row_half_mirror (7 - i within 8), row_mirror (15 - i within
// 16).  Every lane of the wave must be active.
template <int Ctrl>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xF, 0xF, false));
}
template <int Ctrl>
__device__ __forceinline__ double dpp_move(double v) {
  const unsigned long long b = static_cast<unsigned long long>(__double_as_longlong(v));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
      0, static_cast<int>(static_cast<uint32_t>(b)), Ctrl, 0xF, 0xF, false));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
      0, static_cast<int>(static_cast<uint32_t>(b >> 32)), Ctrl, 0xF, 0xF, false));
  return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}
__device__ __forceinline__ float read_lane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ double read_lane(double v, int lane) {
  const unsigned long long b = static_cast<unsigned long long>(__double_as_longlong(v));
  const uint32_t lo = static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b)), lane));
  const uint32_t hi = static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b >> 32)), lane));
  return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// Wave-wide sums of Count values per lane in one fixed order: within each row of 16 lanes, add
// the partner at lane ^ 1, ^ 2, then the mirrored half and row (each step's operands are
// uniform over the group being combined -- fp addition commutes -- so the mirrors add the same
// values as xor partners 4 and 8); every lane of a row then holds the row's sum, and the total
// is (row 0 + row 1) + (row 2 + row 3), returned in every lane.  The values' steps are
// interleaved.
template <class T, int Count>
__device__ __forceinline__ void wave_sums_rows(T (&v)[Count]) {
#pragma unroll
  for (int i = 0; i < Count; ++i) v[i] += dpp_move<0xB1>(v[i]);
#pragma unroll
  for (int i = 0; i < Count; ++i) v[i] += dpp_move<0x4E>(v[i]);
#pragma unroll
  for (int i = 0; i < Count; ++i) v[i] += dpp_move<0x141>(v[i]);
#pragma unroll
  for (int i = 0; i < Count; ++i) v[i] += dpp_move<0x140>(v[i]);
#pragma unroll
  for (int i = 0; i < Count; ++i)
    v[i] = (read_lane(v[i], 0) + read_lane(v[i], 16)) + (read_lane(v[i], 32) + read_lane(v[i], 48));
}

// 128-bit loads / stores with the non-temporal hint (streamed once: do not keep in cache).
typedef float vf4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 load_nt(const float4 *p) {
  const vf4_t v = __builtin_nontemporal_load(reinterpret_cast<const vf4_t *>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store_nt(float4 *p, const float4 &v) {
  const vf4_t x = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(x, reinterpret_cast<vf4_t *>(p));
}

// Kernel timing hook: oxh_time_next_launch arms the calling thread's next kernel launch to
// record a start / stop event pair around the dispatch itself (hipExtLaunchKernelGGL), the
// same interval a kernel-trace profiler reports.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
LaunchEvents &armed_launch_events();

template <typename Kernel, typename... Args>
inline void launch(Kernel kernel, dim3 grid, dim3 block, uint32_t shared_bytes,
                   hipStream_t stream, Args... args) {
  LaunchEvents &armed = armed_launch_events();
  if (armed.start != nullptr || armed.stop != nullptr) {
    const LaunchEvents ev = armed;
    armed = LaunchEvents{};
    hipExtLaunchKernelGGL(kernel, grid, block, shared_bytes, stream, ev.start, ev.stop, 0u,
                          args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, shared_bytes, stream, args...);
  }
}

}  // namespace oxh

#define OXH_REQUIRE(cond, status, msg) \
  do {                                 \
    if (!(cond)) return ::oxh::fail((status), (msg)); \
  } while (0)

#define OXH_HIP_CHECK(call)                                   \
  do {                                                        \
    hipError_t oxh_err_ = (call);                             \
    if (oxh_err_ != hipSuccess) return ::oxh::hip_status(oxh_err_, #call); \
  } while (0)
