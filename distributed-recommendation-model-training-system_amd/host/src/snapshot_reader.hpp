// snapshot_reader.hpp -- streaming reader of the reference's shard snapshot
// files (formats 1 and 2).
//
// The byte stream is the one snapshot_writer.hpp writes (the reference's
// src/store/snapshot.cpp:29-98 encodings: little-endian u64, IEEE floats that
// must be finite, strings of at most 1024 bytes, then per table the definition
// -- with the weight-bounds flag in format 2 only -- the optimizer clock and
// the rows) followed by the FNV-1a checksum of every byte before it.  The
// reader checks the same things the reference's ReadSnapshot does
// (:223-268): the magic, the identity and table schema, finite state,
// non-negative second moments, the checksum and the absence of trailing
// bytes.  Rows are handed out one at a time, so a file of any size streams
// through a fixed buffer; the checksum is known only at Finish(), so callers
// commit nothing before it.
#pragma once

#include <fcntl.h>
#include <unistd.h>

#include <bit>
#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <filesystem>
#include <string>
#include <vector>

#include "job_queue.hpp"

namespace eps::hipbk {

static_assert(std::endian::native == std::endian::little, "snapshot rows are read as little-endian bytes");

class SnapshotReader {
 public:
  struct Table {
    TableDefinition definition;
    std::uint64_t optimizer_sequence = 0;
    float beta1_power = 0, beta2_power = 0;
    std::uint64_t rows = 0;
  };

  explicit SnapshotReader(const std::filesystem::path& file) : buffer_(kChunk) {
    fd_ = ::open(file.c_str(), O_RDONLY);
    Expect(fd_ >= 0, "cannot open snapshot", Error::Code::unavailable);
    const std::uint64_t magic = U64();
    Expect(magic == kFormat1 || magic == kFormat2, "not a shard snapshot (unknown magic)");
    version = magic == kFormat2 ? 2 : 1;
    const std::uint64_t n = U64();
    Expect(n <= 1024, "snapshot run identifier is too long");
    run.resize(n);
    Read(run.data(), n);
    shard = U64();
    shard_count = U64();
    epoch = U64();
    tables = U64();
    Expect(tables <= 1024, "snapshot holds too many tables");
  }
  ~SnapshotReader() {
    if (fd_ >= 0) ::close(fd_);
  }
  SnapshotReader(const SnapshotReader&) = delete;
  SnapshotReader& operator=(const SnapshotReader&) = delete;

  // Header of the next table; its rows follow (Row() `rows` times).
  Table NextTable() {
    Table t;
    TableDefinition& d = t.definition;
    const std::uint64_t id = U64(), dim = U64(), count = U64();
    Expect(id <= UINT32_MAX && dim >= 1 && dim <= 65536 && count == shard_count,
           "snapshot table definition is invalid");
    d.id = TableId(id);
    d.dimension = std::uint32_t(dim);
    d.shard_count = std::uint32_t(count);
    d.partition_epoch = U64();
    Expect(d.partition_epoch == epoch, "snapshot table epoch differs from the shard's");
    OptimizerConfig& o = d.optimizer;
    o.learning_rate = F32();
    o.beta1 = F32();
    o.beta2 = F32();
    o.epsilon = F32();
    o.initial_beta1_power = F32();
    o.initial_beta2_power = F32();
    if (version == 2) {
      const std::uint64_t bounded = U64();
      Expect(bounded <= 1, "snapshot weight-bounds flag is invalid");
      if (bounded) {
        const float lo = F32();
        o.weight_bounds = WeightBounds{lo, F32()};
      }
    }
    d.initialization_min = F32();
    d.initialization_max = F32();
    d.initialization_seed = U64();
    t.optimizer_sequence = U64();
    t.beta1_power = F32();
    t.beta2_power = F32();
    Expect(t.beta1_power >= 0 && t.beta1_power < 1 && t.beta2_power >= 0 && t.beta2_power < 1,
           "snapshot optimizer powers are out of range");
    t.rows = U64();
    return t;
  }

  // One row: its key, update counter and [w | m | v] (3 x dim floats).
  void Row(std::uint32_t dim, Key& key, std::uint64_t& updates, float* wmv) {
    key = U64();
    updates = U64();
    Read(wmv, std::size_t(dim) * 12);
    for (std::uint32_t i = 0; i < 3 * dim; ++i) Expect(std::isfinite(wmv[i]), "snapshot holds non-finite state");
    for (std::uint32_t i = 2 * dim; i < 3 * dim; ++i) Expect(wmv[i] >= 0.f, "snapshot holds a negative second moment");
  }

  // Checks the trailing checksum and that nothing follows it.
  void Finish() {
    const std::uint64_t expected = hash_;
    hashing_ = false;
    const std::uint64_t stored = U64();
    Expect(stored == expected, "snapshot checksum mismatch");
    Expect(Available() == 0 && Refill() == 0, "snapshot has trailing bytes");
  }

  std::string run;
  std::uint64_t shard = 0, shard_count = 0, epoch = 0, tables = 0;
  std::uint32_t version = 0;

 private:
  static constexpr std::uint64_t kFormat1 = 0x3153504541524853ULL;
  static constexpr std::uint64_t kFormat2 = 0x3253504541524853ULL;
  static constexpr std::size_t kChunk = 4u << 20;

  std::size_t Available() const { return end_ - at_; }
  std::size_t Refill() {
    at_ = 0;
    end_ = 0;
    for (;;) {
      const ssize_t n = ::read(fd_, buffer_.data(), buffer_.size());
      if (n < 0 && errno == EINTR) continue;
      Expect(n >= 0, "snapshot read failed", Error::Code::unavailable);
      end_ = std::size_t(n);
      return end_;
    }
  }
  void Read(void* out, std::size_t size) {
    auto* dst = static_cast<unsigned char*>(out);
    while (size) {
      if (!Available()) Expect(Refill() > 0, "snapshot is truncated", Error::Code::unavailable);
      const std::size_t n = std::min(size, Available());
      const unsigned char* src = buffer_.data() + at_;
      if (hashing_) {
        std::uint64_t h = hash_;
        for (std::size_t i = 0; i < n; ++i) h = (h ^ src[i]) * 1099511628211ULL;
        hash_ = h;
      }
      std::memcpy(dst, src, n);
      at_ += n;
      dst += n;
      size -= n;
    }
  }
  std::uint64_t U64() {
    unsigned char b[8];
    Read(b, 8);
    std::uint64_t v = 0;
    for (int i = 7; i >= 0; --i) v = (v << 8) | b[i];
    return v;
  }
  float F32() {
    unsigned char b[4];
    Read(b, 4);
    std::uint32_t u = 0;
    for (int i = 3; i >= 0; --i) u = (u << 8) | b[i];
    float x;
    std::memcpy(&x, &u, 4);
    Expect(std::isfinite(x), "snapshot holds non-finite state");
    return x;
  }

  int fd_ = -1;
  std::vector<unsigned char> buffer_;
  std::size_t at_ = 0, end_ = 0;
  std::uint64_t hash_ = 14695981039346656037ULL;
  bool hashing_ = true;
};

}  // namespace eps::hipbk
