// prepare.hpp -- host-side description of a push shared by prepare.hip and adam.hip.
#pragma once
#include <array>

#include "common.hpp"

namespace eps_hip {

// Lanes per row of the vector kernels: G = dim/4 rounded up to a power of two
// (4..64); classes 0..4 are log2(G)-2, class 5 is the generic scalar shape.
inline uint32_t DimClass(uint32_t dim) {
  if (dim % 4 != 0 || dim > 256) return 5;
  uint32_t log2g = 2;
  while ((1u << log2g) < dim / 4) ++log2g;
  return log2g - 2;
}

// Positions of the sorted reference array handled by one block of the fused
// update, per class: two segments' worth per sub-wavefront group.
inline uint32_t PositionsPerBlock(uint32_t cls) {
  return cls == 5 ? 8u : 2u * (kBlock >> (cls + 2));
}

struct PushPlan {
  uint64_t occurrences = 0;           // total over features (holes included)
  uint32_t row_bits = 0, key_bits = 0, passes = 0;
  std::array<uint32_t, kMaxPasses> shift{}, bits{};
  // Fixed-size, so planning a push allocates nothing.
  std::array<uint32_t, EPS_HIP_MAX_TABLES> key_index{};    // call table index -> key index (class order)
  std::array<uint32_t, EPS_HIP_MAX_TABLES> table_of_key{}; // key index -> call table index
  std::array<uint32_t, kClasses + 1> class_start{};  // first key index of each class
  std::array<uint64_t, kClasses> class_occurrences{};  // upper bound of sorted positions
};

// eps_hip_push with every kernel on `stream` (the hot-row kernel before the
// row kernels): no side stream or event is created or waited on.
int PushOneStream(const eps_hip_table* tables, const eps_hip_optimizer* optimizers, uint32_t table_count,
                  const eps_hip_push_feature* features, uint32_t feature_count, void* workspace,
                  uint64_t workspace_bytes, void* bounds, void* stream);

// eps_hip_prepare with the occurrence indices carried through the sort (the
// sorted position -> occurrence map eps_hip_unique and eps_hip_reduce use).
int PrepareWithOccurrences(const eps_hip_table* tables, uint32_t table_count,
                           const eps_hip_push_feature* features, uint32_t feature_count, void* workspace,
                           uint64_t workspace_bytes, void* stream);

int PlanPush(const eps_hip_table* tables, uint32_t table_count,
             const eps_hip_push_feature* features, uint32_t feature_count, PushPlan& plan);

}  // namespace eps_hip
