// checkpoint.hip -- the OXTR little-endian checkpoint format that MobileNetV4ConvSmall::save
// writes and load_mnist reads (crates/oxide-torch-models/src/models/mobilenet_v4.rs:217-264,
// 386-428).  Host code only.
//
// Layout: magic "OXTR\x01"; u64 tensor count; per tensor: u64 rank, rank x u64 dimensions,
// u64 value count, that many f32 values.  All integers little-endian (the host is).  The
// reader validates structure only, like the reference's read_checkpoint (the value count is
// not tied to the shape; a model loader compares shapes), but never trusts a count from the
// file for an allocation: every declared size is checked against the bytes that remain.
#include <cerrno>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

#include "common.h"

struct oxh_checkpoint {
  std::vector<std::vector<uint64_t>> shapes;
  std::vector<std::vector<float>> values;
};

namespace {

constexpr char kMagic[5] = {'O', 'X', 'T', 'R', '\x01'};

struct Reader {
  const std::vector<uint8_t> &bytes;
  uint64_t pos = 0;
  uint64_t left() const { return bytes.size() - pos; }
  bool u64(uint64_t *v) {
    if (left() < 8) return false;
    std::memcpy(v, bytes.data() + pos, 8);
    pos += 8;
    return true;
  }
};

oxh_status truncated() {
  return oxh::fail(OXH_EXECUTION, "checkpoint read failed: unexpected end of file");
}

}  // namespace

extern "C" {

oxh_status oxh_checkpoint_save(const char *path, const oxh_checkpoint_tensor *tensors,
                               uint64_t count) {
  OXH_REQUIRE(path != nullptr, OXH_INVALID_SHAPE, "oxh_checkpoint_save: null path");
  OXH_REQUIRE(count == 0 || tensors != nullptr, OXH_INVALID_SHAPE,
              "oxh_checkpoint_save: null tensors");
  for (uint64_t i = 0; i < count; ++i)
    OXH_REQUIRE((tensors[i].rank == 0 || tensors[i].shape != nullptr) &&
                    (tensors[i].len == 0 || tensors[i].data != nullptr),
                OXH_INVALID_SHAPE, "oxh_checkpoint_save: null shape or data");
  std::ofstream out(path, std::ios::binary | std::ios::trunc);
  if (!out)
    return oxh::fail(OXH_EXECUTION, std::string("failed to create checkpoint ") + path + ": " +
                                        std::strerror(errno));
  auto put = [&](const void *p, size_t n) { out.write(static_cast<const char *>(p), n); };
  put(kMagic, sizeof kMagic);
  put(&count, 8);
  for (uint64_t i = 0; i < count; ++i) {
    const oxh_checkpoint_tensor &t = tensors[i];
    put(&t.rank, 8);
    put(t.shape, t.rank * 8);
    put(&t.len, 8);
    put(t.data, t.len * 4);
  }
  out.flush();
  if (!out) return oxh::fail(OXH_EXECUTION, "checkpoint write failed");
  return oxh::ok();
}

oxh_status oxh_checkpoint_load(const char *path, oxh_checkpoint **out) {
  OXH_REQUIRE(path != nullptr && out != nullptr, OXH_INVALID_SHAPE,
              "oxh_checkpoint_load: null argument");
  *out = nullptr;
  std::ifstream in(path, std::ios::binary);
  if (!in)
    return oxh::fail(OXH_EXECUTION, std::string("failed to open checkpoint ") + path + ": " +
                                        std::strerror(errno));
  std::vector<uint8_t> bytes((std::istreambuf_iterator<char>(in)),
                             std::istreambuf_iterator<char>());
  if (bytes.size() < sizeof kMagic) return truncated();
  if (std::memcmp(bytes.data(), kMagic, sizeof kMagic) != 0)
    return oxh::fail(OXH_EXECUTION, "invalid OXTR checkpoint header");
  Reader r{bytes, sizeof kMagic};
  uint64_t count = 0;
  if (!r.u64(&count)) return truncated();
  auto *ck = new oxh_checkpoint();
  for (uint64_t i = 0; i < count; ++i) {
    uint64_t rank = 0, len = 0;
    if (!r.u64(&rank) || rank > r.left() / 8) {
      delete ck;
      return truncated();
    }
    std::vector<uint64_t> shape(rank);
    for (auto &d : shape) r.u64(&d);
    if (!r.u64(&len) || len > r.left() / 4) {
      delete ck;
      return truncated();
    }
    std::vector<float> values(len);
    if (len != 0) std::memcpy(values.data(), bytes.data() + r.pos, len * 4);
    r.pos += len * 4;
    ck->shapes.push_back(std::move(shape));
    ck->values.push_back(std::move(values));
  }
  *out = ck;
  return oxh::ok();
}

oxh_status oxh_checkpoint_count(const oxh_checkpoint *checkpoint, uint64_t *count) {
  OXH_REQUIRE(checkpoint && count, OXH_INVALID_SHAPE, "oxh_checkpoint_count: null argument");
  *count = checkpoint->shapes.size();
  return oxh::ok();
}

oxh_status oxh_checkpoint_entry(const oxh_checkpoint *checkpoint, uint64_t index,
                                 uint64_t *rank, const uint64_t **shape, uint64_t *len,
                                 const float **data) {
  OXH_REQUIRE(checkpoint && rank && shape && len && data, OXH_INVALID_SHAPE,
              "oxh_checkpoint_entry: null argument");
  OXH_REQUIRE(index < checkpoint->shapes.size(), OXH_INVALID_SHAPE,
              "oxh_checkpoint_entry: index out of range");
  *rank = checkpoint->shapes[index].size();
  *shape = checkpoint->shapes[index].data();
  *len = checkpoint->values[index].size();
  *data = checkpoint->values[index].data();
  return oxh::ok();
}

// Leaves the calling thread's last error untouched (it runs on error paths too).
oxh_status oxh_checkpoint_free(oxh_checkpoint *checkpoint) {
  delete checkpoint;
  return OXH_OK;
}

}  // extern "C"
