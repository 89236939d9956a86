// packet.cpp -- CSR gradient packet checks and host expansion.
#include "packet.hpp"

#include <cmath>
#include <unordered_set>

#include "job_queue.hpp"

namespace eps::hipbk {
namespace {

constexpr std::uint64_t kPacketLimit = 16ull << 20;

struct RowKeyHash {
  std::size_t operator()(const RowKey& r) const noexcept {
    return std::hash<std::uint64_t>()(r.key * 0x9e3779b97f4a7c15ull ^ r.table);
  }
};

}  // namespace

std::uint64_t PacketBytes(const CompactGradients& p) {
  const std::uint64_t words = p.row_offsets.size() + p.source_rows.size();
  const std::uint64_t floats = p.source_values.size() + p.scales.size();
  return p.rows.size() * sizeof(RowKey) + floats * sizeof(float) + words * sizeof(std::uint64_t);
}

void CheckPacket(const CompactGradients& p) {
  Expect(p.dimension >= 1 && p.dimension <= 4096 && p.rows.size() <= (1ull << 20),
         "compact packet: dimension or row count out of range");
  const std::uint64_t refs = p.source_rows.size();
  bool shape = p.source_values.size() % p.dimension == 0 && p.scales.size() == refs &&
               p.row_offsets.size() == p.rows.size() + 1 && p.row_offsets.front() == 0 &&
               p.row_offsets.back() == refs;
  for (std::size_t r = 1; shape && r < p.row_offsets.size(); ++r) shape = p.row_offsets[r - 1] <= p.row_offsets[r];
  Expect(shape, "compact packet: malformed row offsets");
  Expect(PacketBytes(p) <= kPacketLimit, "compact packet exceeds 16 MiB", Error::Code::capacity_exceeded);
  std::unordered_set<RowKey, RowKeyHash> rows(p.rows.begin(), p.rows.end());
  Expect(rows.size() == p.rows.size(), "compact packet names a row twice");
  const std::uint64_t sources = p.source_values.size() / p.dimension;
  for (std::uint64_t s : p.source_rows) Expect(s < sources, "compact packet reference past its source rows");
  for (float v : p.source_values) Expect(std::isfinite(v), "compact packet holds a non-finite gradient value");
  for (float s : p.scales) Expect(std::isfinite(s) && s >= 0.f, "compact packet scale is negative or non-finite");
}

RowGradients ExpandPacket(const CompactGradients& p) {
  CheckPacket(p);
  const std::uint32_t dim = p.dimension;
  Expect(p.rows.size() * std::uint64_t(dim) * 4 <= kPacketLimit, "expanded packet exceeds 16 MiB",
         Error::Code::capacity_exceeded);
  RowGradients out{p.rows, std::vector<float>(p.rows.size() * dim, 0.f)};
  float* dst = out.values.data();
  for (std::size_t r = 0; r < p.rows.size(); ++r, dst += dim) {
    for (std::uint64_t ref = p.row_offsets[r]; ref < p.row_offsets[r + 1]; ++ref) {
      const float* src = p.source_values.data() + p.source_rows[ref] * dim;
      const float scale = p.scales[ref];
      for (std::uint32_t d = 0; d < dim; ++d) {
        const float term = src[d] * scale;  // rounded, then added: no contraction
        dst[d] = dst[d] + term;
      }
    }
    for (std::uint32_t d = 0; d < dim; ++d) Expect(std::isfinite(dst[d]), "compact packet sum overflows");
  }
  return out;
}

}  // namespace eps::hipbk
