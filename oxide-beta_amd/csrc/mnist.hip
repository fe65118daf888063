// mnist.hip -- the canonical uncompressed MNIST IDX files: parsing and validation, the
// deterministic shuffle, and batch normalization (crates/oxide-torch/src/data/mnist.rs), with
// the batch assembly also on the device.
//
// Host side (data/mnist.rs:26-49,103-133,144-199): the four IDX files are read and checked as
// the reference checks them (magic 2051 / 2049 big-endian, 28 x 28 images, exact payload
// lengths, labels <= 9, equal image and label counts); MnistBatches' index order comes from
// deterministic_shuffle (xorshift64 13/7/17 from 0xD1B54A32D192ED03, Fisher-Yates from the
// end, swap partner state % (index + 1)); a batch is (pixel / 255 - 0.1307) / 0.3081 in fp32 and
// the labels as fp32.
//
// Device side: the dataset's bytes live in HBM (47 MB for the training split) and one launch
// gathers a batch by index and normalizes it straight into the training step's input and
// target buffers -- the same fp32 operations, so the values equal the host batch bit for bit --
// instead of assembling every batch on the host and copying it over PCIe.
#include <hip/hip_runtime.h>

#include <cerrno>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

#include "common.h"

struct oxh_mnist {
  std::vector<uint8_t> train_images, train_labels, test_images, test_labels;  // file bytes
  uint64_t train_count = 0, test_count = 0;
};

namespace {

constexpr uint32_t kRows = 28, kColumns = 28, kPixels = kRows * kColumns;
constexpr uint32_t kImageMagic = 2051, kLabelMagic = 2049;
constexpr uint64_t kImageHeader = 16, kLabelHeader = 8;

bool be_u32(const uint8_t *bytes, uint64_t len, uint64_t offset, uint32_t *value) {
  if (offset + 4 > len) return false;
  *value = (static_cast<uint32_t>(bytes[offset]) << 24) |
           (static_cast<uint32_t>(bytes[offset + 1]) << 16) |
           (static_cast<uint32_t>(bytes[offset + 2]) << 8) | static_cast<uint32_t>(bytes[offset + 3]);
  return true;
}

// data/mnist.rs:145-170
oxh_status parse_images(const uint8_t *bytes, uint64_t len, uint64_t *count) {
  uint32_t magic = 0, n = 0, rows = 0, columns = 0;
  if (bytes == nullptr || len < kImageHeader || !be_u32(bytes, len, 0, &magic) ||
      magic != kImageMagic)
    return oxh::fail(OXH_EXECUTION, "invalid MNIST image IDX header");
  be_u32(bytes, len, 4, &n);
  be_u32(bytes, len, 8, &rows);
  be_u32(bytes, len, 12, &columns);
  if (rows != kRows || columns != kColumns)
    return oxh::fail(OXH_EXECUTION, "expected 28x28 MNIST images, got " + std::to_string(rows) +
                                        "x" + std::to_string(columns));
  if (len != kImageHeader + static_cast<uint64_t>(n) * kPixels)
    return oxh::fail(OXH_EXECUTION, "invalid MNIST image payload length");
  *count = n;
  return oxh::ok();
}

// data/mnist.rs:172-183
oxh_status parse_labels(const uint8_t *bytes, uint64_t len, uint64_t *count) {
  uint32_t magic = 0, n = 0;
  if (bytes == nullptr || len < kLabelHeader || !be_u32(bytes, len, 0, &magic) ||
      magic != kLabelMagic)
    return oxh::fail(OXH_EXECUTION, "invalid MNIST label IDX header");
  be_u32(bytes, len, 4, &n);
  bool valid = len == kLabelHeader + static_cast<uint64_t>(n);
  for (uint64_t i = kLabelHeader; valid && i < len; ++i) valid = bytes[i] <= 9;
  if (!valid) return oxh::fail(OXH_EXECUTION, "invalid MNIST label payload");
  *count = n;
  return oxh::ok();
}

oxh_status read_file(const std::string &path, std::vector<uint8_t> &out) {
  std::ifstream in(path, std::ios::binary);
  if (!in)
    return oxh::fail(OXH_EXECUTION,
                     "failed to read MNIST file " + path + ": " + std::strerror(errno));
  in.seekg(0, std::ios::end);
  const std::streamoff size = in.tellg();
  in.seekg(0, std::ios::beg);
  if (size < 0) return oxh::fail(OXH_EXECUTION, "failed to read MNIST file " + path);
  out.resize(static_cast<size_t>(size));
  if (size > 0 && !in.read(reinterpret_cast<char *>(out.data()), size))
    return oxh::fail(OXH_EXECUTION, "failed to read MNIST file " + path);
  return oxh::ok();
}

// (pixel / 255 - 0.1307) / 0.3081 in fp32 (data/mnist.rs:118-121)
__host__ __device__ inline float normalize_pixel(uint8_t pixel) {
  return (static_cast<float>(pixel) / 255.0f - 0.1307f) / 0.3081f;
}

// One thread per 4 pixels of one image (784 = 196 * 4).  An index outside the split writes a
// NaN image and label (never read out of bounds); the host checks indices it owns.
__global__ __launch_bounds__(256) void mnist_gather_kernel(const uint8_t *__restrict__ images,
                                                           const uint8_t *__restrict__ labels,
                                                           uint64_t count,
                                                           const uint32_t *__restrict__ indices,
                                                           uint32_t batch,
                                                           float *__restrict__ out_images,
                                                           float *__restrict__ out_labels) {
  constexpr uint32_t kQuads = kPixels / 4;
  const uint32_t t = blockIdx.x * 256 + threadIdx.x;
  if (t >= batch * kQuads) return;
  const uint32_t b = t / kQuads, q = t - b * kQuads;
  const uint32_t index = indices[b];
  float4 v;
  if (index < count) {
    const uchar4 p = reinterpret_cast<const uchar4 *>(images + static_cast<uint64_t>(index) *
                                                                   kPixels)[q];
    v = make_float4(normalize_pixel(p.x), normalize_pixel(p.y), normalize_pixel(p.z),
                    normalize_pixel(p.w));
  } else {
    const float nan = __int_as_float(0x7fc00000);
    v = make_float4(nan, nan, nan, nan);
  }
  reinterpret_cast<float4 *>(out_images + static_cast<uint64_t>(b) * kPixels)[q] = v;
  if (q == 0)
    out_labels[b] = index < count ? static_cast<float>(labels[index]) : __int_as_float(0x7fc00000);
}

}  // namespace

extern "C" {

oxh_status oxh_idx_parse_images(const uint8_t *bytes, uint64_t len, uint64_t *count) {
  OXH_REQUIRE(count != nullptr, OXH_INVALID_SHAPE, "count is null");
  return parse_images(bytes, len, count);
}

oxh_status oxh_idx_parse_labels(const uint8_t *bytes, uint64_t len, uint64_t *count) {
  OXH_REQUIRE(count != nullptr, OXH_INVALID_SHAPE, "count is null");
  return parse_labels(bytes, len, count);
}

oxh_status oxh_mnist_load(const char *directory, oxh_mnist **out) {
  OXH_REQUIRE(directory != nullptr && out != nullptr, OXH_INVALID_SHAPE,
              "oxh_mnist_load: null argument");
  *out = nullptr;
  auto *m = new oxh_mnist();
  const std::string dir(directory);
  auto join = [&](const char *name) { return dir + "/" + name; };
  uint64_t train_labels = 0, test_labels = 0;
  oxh_status st = read_file(join("train-images-idx3-ubyte"), m->train_images);
  if (st == OXH_OK) st = parse_images(m->train_images.data(), m->train_images.size(), &m->train_count);
  if (st == OXH_OK) st = read_file(join("train-labels-idx1-ubyte"), m->train_labels);
  if (st == OXH_OK) st = parse_labels(m->train_labels.data(), m->train_labels.size(), &train_labels);
  if (st == OXH_OK) st = read_file(join("t10k-images-idx3-ubyte"), m->test_images);
  if (st == OXH_OK) st = parse_images(m->test_images.data(), m->test_images.size(), &m->test_count);
  if (st == OXH_OK) st = read_file(join("t10k-labels-idx1-ubyte"), m->test_labels);
  if (st == OXH_OK) st = parse_labels(m->test_labels.data(), m->test_labels.size(), &test_labels);
  if (st == OXH_OK && (m->train_count != train_labels || m->test_count != test_labels))
    st = oxh::fail(OXH_EXECUTION, "MNIST image and label counts do not match");
  if (st != OXH_OK) {
    delete m;
    return st;
  }
  *out = m;
  return oxh::ok();
}

oxh_status oxh_mnist_free(oxh_mnist *mnist) {
  delete mnist;  // the last error stays untouched
  return OXH_OK;
}

oxh_status oxh_mnist_split(const oxh_mnist *mnist, int test, const uint8_t **images,
                           const uint8_t **labels, uint64_t *count) {
  OXH_REQUIRE(mnist && images && labels && count, OXH_INVALID_SHAPE,
              "oxh_mnist_split: null argument");
  const auto &im = test ? mnist->test_images : mnist->train_images;
  const auto &lb = test ? mnist->test_labels : mnist->train_labels;
  *images = im.data() + kImageHeader;
  *labels = lb.data() + kLabelHeader;
  *count = test ? mnist->test_count : mnist->train_count;
  return oxh::ok();
}

oxh_status oxh_mnist_batch_order(uint64_t count, int shuffle, uint64_t *indices) {
  OXH_REQUIRE(count == 0 || indices != nullptr, OXH_INVALID_SHAPE, "indices is null");
  for (uint64_t i = 0; i < count; ++i) indices[i] = i;
  if (!shuffle) return oxh::ok();
  // data/mnist.rs:191-199
  uint64_t state = 0xD1B54A32D192ED03ull;
  for (uint64_t index = count > 0 ? count - 1 : 0; index >= 1; --index) {
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    const uint64_t partner = state % (index + 1);
    const uint64_t t = indices[index];
    indices[index] = indices[partner];
    indices[partner] = t;
  }
  return oxh::ok();
}

oxh_status oxh_mnist_batch_host(const uint8_t *images, const uint8_t *labels, uint64_t count,
                                const uint64_t *indices, uint64_t batch, float *out_images,
                                float *out_labels) {
  OXH_REQUIRE(batch > 0, OXH_INVALID_SHAPE, "batch_size must be non-zero");
  OXH_REQUIRE(images && labels && indices && out_images && out_labels, OXH_INVALID_SHAPE,
              "oxh_mnist_batch_host: null argument");
  for (uint64_t b = 0; b < batch; ++b)
    OXH_REQUIRE(indices[b] < count, OXH_INVALID_SHAPE, "MNIST index out of range");
  for (uint64_t b = 0; b < batch; ++b) {
    const uint8_t *src = images + indices[b] * kPixels;
    for (uint32_t p = 0; p < kPixels; ++p) out_images[b * kPixels + p] = normalize_pixel(src[p]);
    out_labels[b] = static_cast<float>(labels[indices[b]]);
  }
  return oxh::ok();
}

oxh_status oxh_mnist_gather_batch(oxh_stream stream, const uint8_t *images, const uint8_t *labels,
                                  uint64_t count, const uint32_t *indices, uint64_t batch,
                                  float *out_images, float *out_labels) {
  const char *name = "oxh_mnist_gather_batch";
  OXH_REQUIRE(batch > 0 && batch < (1ull << 24), OXH_INVALID_SHAPE,
              std::string(name) + ": batch must be in 1..2^24");
  OXH_REQUIRE(images && labels && indices && out_images && out_labels, OXH_INVALID_SHAPE,
              std::string(name) + ": null argument");
  OXH_REQUIRE(oxh::aligned16(out_images) && (reinterpret_cast<uintptr_t>(images) & 3u) == 0,
              OXH_INVALID_SHAPE,
              std::string(name) + ": images must be 4-byte and out_images 16-byte aligned");
  const uint64_t threads = batch * (kPixels / 4);
  oxh::launch(mnist_gather_kernel, dim3(static_cast<uint32_t>((threads + 255) / 256)), dim3(256),
              0, oxh::as_stream(stream), images, labels, count, indices,
              static_cast<uint32_t>(batch), out_images, out_labels);
  return oxh::launched(name);
}

}  // extern "C"
