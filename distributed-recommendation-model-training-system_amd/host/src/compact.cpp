// compact.cpp -- validation and host expansion of CSR gradient packets.
#include <algorithm>
#include <cmath>
#include <set>
#include <utility>

#include "executor.hpp"

namespace eps::hip_detail {

std::uint64_t CompactBytes(const CompactGradients& p) {
  return p.rows.size() * sizeof(RowKey) + (p.source_values.size() + p.scales.size()) * 4 +
         (p.row_offsets.size() + p.source_rows.size()) * 8;
}

// src/access/compact_gradients.cpp:10-22: shape, 16 MiB packet limit, unique
// rows, in-range references, finite values and finite non-negative scales.
void ValidateCompact(const CompactGradients& p) {
  Require(p.dimension > 0 && p.dimension <= 4096 && p.rows.size() <= (1ULL << 20),
          "invalid compact gradient dimensions");
  Require(p.source_values.size() % p.dimension == 0 && p.row_offsets.size() == p.rows.size() + 1 &&
              p.source_rows.size() == p.scales.size() && p.row_offsets.front() == 0 &&
              p.row_offsets.back() == p.source_rows.size() &&
              std::is_sorted(p.row_offsets.begin(), p.row_offsets.end()),
          "invalid compact gradient offsets");
  Require(CompactBytes(p) <= (16ULL << 20), "compact gradient exceeds byte limit",
          Error::Code::capacity_exceeded);
  std::set<std::pair<TableId, Key>> seen;
  for (const auto& row : p.rows)
    Require(seen.emplace(row.table, row.key).second, "duplicate compact parameter row");
  const std::uint64_t sources = p.source_values.size() / p.dimension;
  for (auto s : p.source_rows) Require(s < sources, "compact gradient reference is out of bounds");
  for (auto v : p.source_values) Require(std::isfinite(v), "non-finite compact gradient value");
  for (auto s : p.scales) Require(std::isfinite(s) && s >= 0, "invalid compact gradient scale");
}

// src/access/compact_gradients.cpp:27-39.
RowGradients ExpandCompact(const CompactGradients& p) {
  ValidateCompact(p);
  Require(p.rows.size() <= (16ULL << 20) / (p.dimension * 4ULL), "expanded gradient exceeds byte limit",
          Error::Code::capacity_exceeded);
  RowGradients out{p.rows, std::vector<float>(p.rows.size() * p.dimension, 0.f)};
  for (std::size_t r = 0; r < p.rows.size(); ++r) {
    for (std::uint32_t d = 0; d < p.dimension; ++d) {
      float sum = 0.f;
      for (auto ref = p.row_offsets[r]; ref < p.row_offsets[r + 1]; ++ref) {
        const float term = p.source_values[p.source_rows[ref] * p.dimension + d] * p.scales[ref];
        sum = sum + term;
      }
      Require(std::isfinite(sum), "compact gradient reduction overflow");
      out.values[r * p.dimension + d] = sum;
    }
  }
  return out;
}

}  // namespace eps::hip_detail
