// guard.hpp -- the pieces of the fused update that decide before anything is
// written: the overflow guard's bounds and the range checks of the indices the
// update kernels take from a prepared workspace.  Plain arithmetic on scalars,
// compiled for the device (adam.hip) and for the host (the unit test of these
// functions), so both evaluate exactly the same expressions.
#pragma once
#include <cstdint>
#include <cmath>

#if defined(__HIPCC__)
#define EPS_HD __host__ __device__ __forceinline__
#else
#define EPS_HD inline
#endif

namespace eps_hip {

constexpr uint32_t kGuardRefRowBits = 27;  // gradient row bits of a reference word
constexpr double kGuardLimit = 1e30;       // every bound must stay below this (far below FLT_MAX)
constexpr double kGuardWiden = 1.01;       // each bound is widened by 1%

// Bound G >= |g| for every reduced gradient: the largest gradient magnitude
// times the largest scale (at least 1) times the references summed into one
// row, times the rounding growth (1 + 2^-24)^(refs + 2) of a sequential fp32
// sum, widened by 1%.
EPS_HD double GuardGradBound(double max_grad, double max_scale, double refs) {
  const double scale = max_scale > 1.0 ? max_scale : 1.0;
  return max_grad * scale * refs * std::exp((refs + 2.0) * 0x1.0p-24) * kGuardWiden;
}

// Whether one table's update cannot overflow, given the bounds-domain maxima
// W >= |w|, M >= |m|, V >= v before the update and G: |m'| <= b1*M + (1-b1)*G,
// v' <= b2*V + (1-b2)*G^2, |w'| <= W + lr_t*|m'|/eps (sqrt(v') + eps >= eps),
// each widened by 1% and required below 1e30.
EPS_HD bool GuardTableSafe(double b1, double b2, double lr, double eps, double W, double M,
                           double V, double G) {
  const double mbound = (b1 * M + (1.0 - b1) * G) * kGuardWiden;
  const double vbound = (b2 * V + (1.0 - b2) * G * G) * kGuardWiden;
  const double wbound = (W + lr * mbound / eps) * kGuardWiden;
  return mbound < kGuardLimit && vbound < kGuardLimit && wbound < kGuardLimit && eps > 0.0;
}

// A sorted key is (table key index << row_bits | slot); a reference word is
// (scale bits << 32 | feature << 27 | gradient row).  The update kernels take
// both from a prepared workspace; every table index, slot, feature and
// gradient row they name is checked against the push before it is used as an
// address.
struct KeyParts { uint32_t table, slot; };
EPS_HD KeyParts SplitKey(uint32_t key, uint32_t row_bits) {
  if (row_bits >= 32) return KeyParts{0u, key};
  return KeyParts{key >> row_bits, key & ((1u << row_bits) - 1u)};
}
EPS_HD bool KeyInRange(KeyParts k, uint32_t tables, uint64_t rows_of_table) {
  return k.table < tables && uint64_t(k.slot) < rows_of_table;
}
struct RefParts { uint32_t feature, row; };
EPS_HD RefParts SplitRef(uint64_t word) {
  const uint32_t ref = uint32_t(word);
  return RefParts{ref >> kGuardRefRowBits, ref & ((1u << kGuardRefRowBits) - 1u)};
}
EPS_HD bool RefInRange(RefParts r, uint32_t features, uint64_t rows_of_feature) {
  return r.feature < features && uint64_t(r.row) < rows_of_feature;
}

}  // namespace eps_hip
