// runtime.hip -- device selection, streams, buffers, errors and graph capture/replay.
//
// Mirrors the cuda-core calls the reference adapter makes (runtime.rs:46-105,
// cuda/jit.rs:25-99) and the CudaGraphExec wrapper (cuda_graph.rs:47-179), on HIP directly:
// the gfx950 code object is linked into this library, so "loading kernels" is selecting the
// device.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <string>

#include "common.h"

namespace oxh {

namespace {
thread_local std::string g_last_error;
}

oxh_status fail(oxh_status status, const std::string &message) {
  g_last_error = message;
  return status;
}

oxh_status ok() {
  g_last_error.clear();
  return OXH_OK;
}

LaunchEvents &armed_launch_events() {
  thread_local LaunchEvents armed;
  return armed;
}

}  // namespace oxh

struct oxh_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

extern "C" {

const char *oxh_last_error(void) { return oxh::g_last_error.c_str(); }

const char *oxh_version(void) { return "oxide-hip 0.1.0 (gfx950)"; }

oxh_status oxh_device_count(int *count) {
  OXH_REQUIRE(count != nullptr, OXH_INVALID_SHAPE, "count is null");
  OXH_HIP_CHECK(hipGetDeviceCount(count));
  return oxh::ok();
}

oxh_status oxh_init(int device) {
  int count = 0;
  OXH_HIP_CHECK(hipGetDeviceCount(&count));
  OXH_REQUIRE(device >= 0 && device < count, OXH_INVALID_SHAPE,
              "device " + std::to_string(device) + " is outside 0.." + std::to_string(count));
  OXH_HIP_CHECK(hipSetDevice(device));
  hipDeviceProp_t prop;
  OXH_HIP_CHECK(hipGetDeviceProperties(&prop, device));
  std::string arch = prop.gcnArchName;
  OXH_REQUIRE(arch.rfind("gfx950", 0) == 0, OXH_EXECUTION,
              "liboxide_hip is built for gfx950, device reports " + arch);
  return oxh::bn_scratch_init(device);
}

oxh_status oxh_stream_create(oxh_stream *stream) {
  OXH_REQUIRE(stream != nullptr, OXH_INVALID_SHAPE, "stream is null");
  hipStream_t s = nullptr;
  // Default priority, non-blocking with respect to the null stream: capturable.
  OXH_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return oxh::ok();
}

oxh_status oxh_stream_destroy(oxh_stream stream) {
  if (stream == nullptr) return oxh::ok();
  OXH_HIP_CHECK(hipStreamDestroy(oxh::as_stream(stream)));
  return oxh::ok();
}

oxh_status oxh_stream_synchronize(oxh_stream stream) {
  OXH_HIP_CHECK(hipStreamSynchronize(oxh::as_stream(stream)));
  return oxh::ok();
}

oxh_status oxh_alloc(void **ptr, uint64_t bytes) {
  OXH_REQUIRE(ptr != nullptr, OXH_INVALID_SHAPE, "ptr is null");
  *ptr = nullptr;
  if (bytes == 0) return oxh::ok();
  OXH_HIP_CHECK(hipMalloc(ptr, bytes));
  return oxh::ok();
}

oxh_status oxh_free(void *ptr) {
  if (ptr == nullptr) return oxh::ok();
  OXH_HIP_CHECK(hipFree(ptr));
  return oxh::ok();
}

namespace {
// Zero fill as a kernel rather than hipMemsetAsync, so that a caller may record it into a
// graph (memset nodes have given wrong results on replays after the first on gfx950 boxes).
// `head` bytes up to 16-byte alignment, `body` 16-byte words, then `tail` bytes.
__global__ __launch_bounds__(256) void zero_bytes_kernel(uint8_t *p, uint32_t head, uint64_t body,
                                                         uint32_t tail) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  const uint64_t first = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (first < head) p[first] = 0;
  uint4 *words = reinterpret_cast<uint4 *>(p + head);
  for (uint64_t i = first; i < body; i += stride) words[i] = make_uint4(0u, 0u, 0u, 0u);
  if (first < tail) p[head + body * 16 + first] = 0;
}
}  // namespace

oxh_status oxh_memset0_async(void *ptr, uint64_t bytes, oxh_stream stream) {
  if (bytes == 0) return oxh::ok();
  OXH_REQUIRE(ptr != nullptr, OXH_INVALID_SHAPE, "ptr is null");
  const uint32_t head =
      static_cast<uint32_t>(std::min<uint64_t>(bytes, (16 - reinterpret_cast<uintptr_t>(ptr) % 16) % 16));
  const uint64_t body = (bytes - head) / 16;
  const uint32_t tail = static_cast<uint32_t>((bytes - head) % 16);
  const uint64_t blocks = std::max<uint64_t>(1, std::min<uint64_t>((body + 255) / 256, 4096));
  oxh::launch(zero_bytes_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
              oxh::as_stream(stream), static_cast<uint8_t *>(ptr), head, body, tail);
  return oxh::launched("oxh_memset0_async");
}

oxh_status oxh_memcpy_h2d_async(void *dst, const void *src, uint64_t bytes, oxh_stream stream) {
  if (bytes == 0) return oxh::ok();
  OXH_REQUIRE(dst != nullptr && src != nullptr, OXH_INVALID_SHAPE, "null pointer");
  OXH_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, oxh::as_stream(stream)));
  return oxh::ok();
}

oxh_status oxh_memcpy_d2h(void *dst, const void *src, uint64_t bytes, oxh_stream stream) {
  if (bytes == 0) return oxh::ok();
  OXH_REQUIRE(dst != nullptr && src != nullptr, OXH_INVALID_SHAPE, "null pointer");
  OXH_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, oxh::as_stream(stream)));
  OXH_HIP_CHECK(hipStreamSynchronize(oxh::as_stream(stream)));
  return oxh::ok();
}

oxh_status oxh_memcpy_d2d_async(void *dst, const void *src, uint64_t bytes, oxh_stream stream) {
  if (bytes == 0) return oxh::ok();
  OXH_REQUIRE(dst != nullptr && src != nullptr, OXH_INVALID_SHAPE, "null pointer");
  OXH_HIP_CHECK(
      hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, oxh::as_stream(stream)));
  return oxh::ok();
}

// ---------------------------------------------------------------- model initialization

oxh_status oxh_initialized_weights(const uint64_t shape[4], uint64_t input_channels_per_group,
                                   float *out) {
  OXH_REQUIRE(shape != nullptr && out != nullptr, OXH_INVALID_SHAPE, "null argument");
  OXH_REQUIRE(input_channels_per_group > 0 && shape[2] * shape[3] > 0, OXH_INVALID_SHAPE,
              "oxh_initialized_weights: empty kernel or channel group");
  // nn.rs:657-674: fan_in = in_per_group * kh * kw as f32; scale = sqrt(2 / fan_in); the state
  // starts at 0x9E3779B9, xors every dimension times 0xBF58476D1CE4E5B9, is forced odd, then
  // advances by xorshift64 (<< 13, >> 7, << 17) once per element; the top 24 bits give a
  // uniform in [0, 1) mapped to [-scale, scale).
  const float fan_in = static_cast<float>(input_channels_per_group * shape[2] * shape[3]);
  const float scale = std::sqrt(2.0f / fan_in);
  uint64_t state = 0x9E3779B9ull;
  for (int d = 0; d < 4; ++d) state ^= shape[d] * 0xBF58476D1CE4E5B9ull;
  state |= 1;
  const uint64_t total = shape[0] * shape[1] * shape[2] * shape[3];
  for (uint64_t i = 0; i < total; ++i) {
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    const float unit = static_cast<float>(static_cast<uint32_t>(state >> 40)) /
                       static_cast<float>(1u << 24);
    out[i] = (unit * 2.0f - 1.0f) * scale;
  }
  return oxh::ok();
}

// ---------------------------------------------------------------- kernel timing

oxh_status oxh_event_create(oxh_event *event) {
  OXH_REQUIRE(event != nullptr, OXH_INVALID_SHAPE, "event is null");
  hipEvent_t e = nullptr;
  OXH_HIP_CHECK(hipEventCreate(&e));
  *event = e;
  return oxh::ok();
}

oxh_status oxh_event_destroy(oxh_event event) {
  if (event == nullptr) return oxh::ok();
  OXH_HIP_CHECK(hipEventDestroy(static_cast<hipEvent_t>(event)));
  return oxh::ok();
}

oxh_status oxh_event_elapsed_ms(oxh_event start, oxh_event stop, float *ms) {
  OXH_REQUIRE(start && stop && ms, OXH_INVALID_SHAPE, "null argument");
  OXH_HIP_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
  OXH_HIP_CHECK(
      hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
  return oxh::ok();
}

oxh_status oxh_time_next_launch(oxh_event start, oxh_event stop) {
  OXH_REQUIRE(start != nullptr || stop != nullptr, OXH_INVALID_SHAPE, "no event given");
  oxh::armed_launch_events() =
      oxh::LaunchEvents{static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)};
  return oxh::ok();
}

// ---------------------------------------------------------------- graphs

oxh_status oxh_graph_begin(oxh_stream stream) {
  OXH_REQUIRE(stream != nullptr, OXH_INVALID_SHAPE,
              "the null stream cannot be captured; use oxh_stream_create");
  // cuda_graph.rs:77 synchronizes before capture so earlier work is not part of the graph.
  OXH_HIP_CHECK(hipStreamSynchronize(oxh::as_stream(stream)));
  OXH_HIP_CHECK(hipStreamBeginCapture(oxh::as_stream(stream), hipStreamCaptureModeThreadLocal));
  return oxh::ok();
}

oxh_status oxh_graph_abort(oxh_stream stream) {
  // cuda_graph.rs:84-97: end capture even on a recording error and destroy what was recorded,
  // so the stream stays usable.
  hipGraph_t discarded = nullptr;
  hipError_t err = hipStreamEndCapture(oxh::as_stream(stream), &discarded);
  if (discarded != nullptr) (void)hipGraphDestroy(discarded);
  (void)hipGetLastError();
  if (err != hipSuccess && err != hipErrorStreamCaptureInvalidated)
    return oxh::hip_status(err, "hipStreamEndCapture");
  return oxh::ok();
}

oxh_status oxh_graph_end(oxh_stream stream, oxh_graph **out) {
  OXH_REQUIRE(out != nullptr, OXH_INVALID_SHAPE, "graph out-pointer is null");
  *out = nullptr;
  hipGraph_t graph = nullptr;
  hipError_t err = hipStreamEndCapture(oxh::as_stream(stream), &graph);
  if (err != hipSuccess) {
    if (graph != nullptr) (void)hipGraphDestroy(graph);
    return oxh::hip_status(err, "hipStreamEndCapture");
  }
  OXH_REQUIRE(graph != nullptr, OXH_EXECUTION, "capture returned a null graph");
  hipGraphExec_t exec = nullptr;
  err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (err != hipSuccess) {
    (void)hipGraphDestroy(graph);
    return oxh::hip_status(err, "hipGraphInstantiate");
  }
  *out = new oxh_graph{graph, exec};
  return oxh::ok();
}

oxh_status oxh_graph_launch(const oxh_graph *graph, oxh_stream stream) {
  OXH_REQUIRE(graph != nullptr, OXH_INVALID_SHAPE, "graph is null");
  OXH_HIP_CHECK(hipGraphLaunch(graph->exec, oxh::as_stream(stream)));
  return oxh::ok();
}

oxh_status oxh_graph_destroy(oxh_graph *graph) {
  if (graph == nullptr) return oxh::ok();
  // cuda_graph.rs:167-179: executable first, then its source graph.
  hipError_t e1 = graph->exec ? hipGraphExecDestroy(graph->exec) : hipSuccess;
  hipError_t e2 = graph->graph ? hipGraphDestroy(graph->graph) : hipSuccess;
  delete graph;
  OXH_HIP_CHECK(e1);
  OXH_HIP_CHECK(e2);
  return oxh::ok();
}

}  // extern "C"
