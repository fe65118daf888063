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

#include "oxide_hip.h"

namespace oxh {

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

// Convolution tap terms: p where mask is all ones, else -0.0f (x + (-0.0f) == x for every x),
// the term of a tap outside the input, so a sum over all taps equals the CPU path's sum that
// skips them, bit for bit.  Bit operations rather than a select keep the tap's loads
// unconditional (the compiler turns a select on a loaded value into a branch around the load).
__device__ __forceinline__ float tap_term(float p, uint32_t mask) {
  return __uint_as_float((__float_as_uint(p) & mask) | (~mask & 0x80000000u));
}
__device__ __forceinline__ uint32_t tap_mask(bool valid) { return valid ? 0xFFFFFFFFu : 0u; }

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
