// snapshot_writer.hpp -- the reference's snapshot byte stream, written to a
// staging file and published atomically.
//
// Format (src/store/snapshot.cpp:29-76,159-194): little-endian u64 and IEEE
// float fields, strings as a u64 length plus their bytes, and a trailing u64
// FNV-1a checksum of every byte before it.  Publication follows WriteSnapshot:
// the bytes go to "<file>.pending" (created exclusively), are fsync'ed, hard
// linked to <file> (which must not exist yet), the staging name is removed
// and the directory fsync'ed.  I/O failures are Error::Code::unavailable.
// The checksum is byte-serial, so the caller's thread only hashes and fills
// buffers; a second thread writes the full ones.
#pragma once

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <bit>
#include <cerrno>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <filesystem>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "eps/hip_cache_backend.hpp"
#include "job_queue.hpp"

namespace eps::hipbk {

static_assert(std::endian::native == std::endian::little,
              "snapshot rows are copied as little-endian bytes");

class SnapshotWriter {
 public:
  static constexpr std::uint64_t kMagicV2 = 0x3253504541524853ULL;  // "SHRAEPS2"

  explicit SnapshotWriter(std::filesystem::path file)
      : file_(std::move(file)), pending_(file_.string() + ".pending") {
    std::error_code ec;
    if (file_.has_parent_path()) std::filesystem::create_directories(file_.parent_path(), ec);
    fd_ = ::open(pending_.c_str(), O_WRONLY | O_CREAT | O_EXCL, 0600);
    Expect(fd_ >= 0, "cannot create snapshot staging file", Error::Code::unavailable);
    for (auto& b : buffers_) b.resize(kBuffer);
    io_ = std::thread([this] { Drain(); });
  }
  ~SnapshotWriter() {
    Stop();
    if (fd_ >= 0) ::close(fd_);
    if (!published_) ::unlink(pending_.c_str());
  }
  SnapshotWriter(const SnapshotWriter&) = delete;
  SnapshotWriter& operator=(const SnapshotWriter&) = delete;

  void U64(std::uint64_t v) { Bytes(&v, 8); }
  void F32(float x) { Bytes(&x, 4); }
  void String(const std::string& s) {
    U64(s.size());
    Bytes(s.data(), s.size());
  }
  // Hashed bytes, appended as they lie in memory (little-endian host).
  void Bytes(const void* data, std::size_t size) {
    const auto* p = static_cast<const unsigned char*>(data);
    std::uint64_t h = hash_;
    for (std::size_t i = 0; i < size; ++i) h = (h ^ p[i]) * kPrime;
    hash_ = h;
    Append(p, size);
  }
  std::uint64_t bytes() const { return written_ + filled_; }

  // Appends the checksum, makes the file durable and publishes it.
  std::uint64_t Publish() {
    const std::uint64_t checksum = hash_;
    Append(&checksum, 8);
    Hand();
    Stop();
    Expect(!io_failed_, "snapshot write failed", Error::Code::unavailable);
    Expect(::fsync(fd_) == 0, "snapshot fsync failed", Error::Code::unavailable);
    ::close(fd_);
    fd_ = -1;
    Expect(::link(pending_.c_str(), file_.c_str()) == 0,
            "snapshot already exists or cannot be published", Error::Code::unavailable);
    published_ = true;
    ::unlink(pending_.c_str());
    const auto dir = file_.has_parent_path() ? file_.parent_path() : std::filesystem::path(".");
    const int d = ::open(dir.c_str(), O_RDONLY);
    Expect(d >= 0, "cannot open snapshot directory", Error::Code::unavailable);
    const int rc = ::fsync(d);
    ::close(d);
    Expect(rc == 0, "snapshot fsync failed", Error::Code::unavailable);
    return checksum;
  }

 private:
  static constexpr std::uint64_t kOffset = 14695981039346656037ULL;
  static constexpr std::uint64_t kPrime = 1099511628211ULL;
  static constexpr std::size_t kBuffer = 4u << 20;

  void Append(const void* data, std::size_t size) {
    const auto* p = static_cast<const unsigned char*>(data);
    while (size) {
      auto& buffer = buffers_[current_];
      const std::size_t n = std::min(size, buffer.size() - filled_);
      std::memcpy(buffer.data() + filled_, p, n);
      filled_ += n;
      p += n;
      size -= n;
      if (filled_ == buffer.size()) Hand();
    }
  }
  // Passes the current buffer to the writing thread and waits for the other.
  void Hand() {
    std::unique_lock<std::mutex> lock(mutex_);
    idle_.wait(lock, [&] { return !busy_; });
    Expect(!io_failed_, "snapshot write failed", Error::Code::unavailable);
    ready_ = current_;
    ready_bytes_ = filled_;
    busy_ = true;
    written_ += filled_;
    filled_ = 0;
    current_ ^= 1;
    wake_.notify_one();
  }
  void Drain() {
    std::unique_lock<std::mutex> lock(mutex_);
    for (;;) {
      wake_.wait(lock, [&] { return busy_ || stop_; });
      if (!busy_) return;
      const unsigned char* data = buffers_[ready_].data();
      const std::size_t size = ready_bytes_;
      lock.unlock();
      bool ok = true;
      for (std::size_t pos = 0; pos < size && ok;) {
        const ssize_t n = ::write(fd_, data + pos, size - pos);
        if (n < 0 && errno == EINTR) continue;
        ok = n > 0;
        if (ok) pos += std::size_t(n);
      }
      lock.lock();
      io_failed_ = io_failed_ || !ok;
      busy_ = false;
      idle_.notify_one();
    }
  }
  void Stop() {
    if (!io_.joinable()) return;
    {
      std::unique_lock<std::mutex> lock(mutex_);
      idle_.wait(lock, [&] { return !busy_; });
      stop_ = true;
    }
    wake_.notify_one();
    io_.join();
  }

  std::filesystem::path file_;
  std::string pending_;
  std::vector<unsigned char> buffers_[2];
  unsigned current_ = 0, ready_ = 0;
  std::size_t filled_ = 0, ready_bytes_ = 0;
  std::uint64_t written_ = 0, hash_ = kOffset;
  int fd_ = -1;
  bool published_ = false;
  std::mutex mutex_;
  std::condition_variable wake_, idle_;
  bool busy_ = false, stop_ = false, io_failed_ = false;
  std::thread io_;
};

// The stream's fields in WriteSnapshot's order (src/store/snapshot.cpp:164-185):
// the identity and table count, then per table Binary::Definition (:77-98,
// with the weight-bounds flag of format 2), the optimizer clock and the row
// count, then per row its key, update counter and 3 x dim floats [w | m | v].
inline void WriteSnapshotHeader(SnapshotWriter& out, const SnapshotIdentity& id, std::uint64_t tables) {
  out.U64(SnapshotWriter::kMagicV2);
  out.String(id.run);
  out.U64(id.shard);
  out.U64(id.shard_count);
  out.U64(id.epoch);
  out.U64(tables);
}
inline void WriteSnapshotTable(SnapshotWriter& out, const SnapshotTable& t) {
  const auto& d = t.definition;
  const auto& o = d.optimizer;
  out.U64(d.id);
  out.U64(d.dimension);
  out.U64(d.shard_count);
  out.U64(d.partition_epoch);
  out.F32(o.learning_rate);
  out.F32(o.beta1);
  out.F32(o.beta2);
  out.F32(o.epsilon);
  out.F32(o.initial_beta1_power);
  out.F32(o.initial_beta2_power);
  out.U64(o.weight_bounds ? 1 : 0);
  if (o.weight_bounds) {
    out.F32(o.weight_bounds->minimum);
    out.F32(o.weight_bounds->maximum);
  }
  out.F32(d.initialization_min);
  out.F32(d.initialization_max);
  out.U64(d.initialization_seed);
  out.U64(t.optimizer_sequence);
  out.F32(t.beta1_power);
  out.F32(t.beta2_power);
  out.U64(t.keys.size());
}
// One row whose [w | m | v] floats lie contiguously (the device layout).
inline void WriteSnapshotRow(SnapshotWriter& out, Key key, std::uint64_t updates, const float* wmv,
                             std::uint32_t dim) {
  out.U64(key);
  out.U64(updates);
  out.Bytes(wmv, std::size_t(dim) * 12);
}
// One row held as three vectors (a CPU store's RowState).
inline void WriteSnapshotRow(SnapshotWriter& out, const RowState& row) {
  out.U64(row.row.key);
  out.U64(row.row_updates);
  out.Bytes(row.weights.data(), row.weights.size() * 4);
  out.Bytes(row.first_moment.data(), row.first_moment.size() * 4);
  out.Bytes(row.second_moment.data(), row.second_moment.size() * 4);
}

}  // namespace eps::hipbk
