// eps/types.hpp -- value types of the parameter-shard backend contract.
//
// Source-compatible restatement of the types the cache-backend interface uses
// (reference: include/eps/types.hpp:10-258).  Names, member order and member
// types are kept identical because callers brace-initialise these aggregates
// (e.g. tests/cuda_tests.cpp:16,106 of the reference); request/reply types of
// the RPC service that no backend operation takes are not restated.
#pragma once

#include <cstdint>
#include <memory>
#include <optional>
#include <string>
#include <variant>
#include <vector>

namespace eps {

using TableId = std::uint32_t;
using ShardId = std::uint32_t;
using AgentId = std::uint32_t;
using Key = std::uint64_t;

// Error codes in this order; the C runtime reports code + 1.
struct Error {
  enum class Code {
    invalid_argument,
    unavailable,
    stale_generation,
    retired_request,
    capacity_exceeded,
    run_failed
  };
  Code code;
  std::string message;
};

template <typename T>
using Result = std::variant<T, Error>;

struct Ack {};

enum class Phase { lookup, push, release, maintenance };
enum class Pooling { sum, mean, sequence };
enum class Placement { cpu, loading, gpu, draining };
enum class AccessRoute { cpu_pool, transfer_unique, resident_gpu };

struct RequestId {
  std::string run;
  std::uint32_t learner;
  std::uint64_t sequence;
  Phase phase;
  bool operator==(const RequestId&) const = default;
};

struct RowKey {
  TableId table;
  Key key;
  bool operator==(const RowKey&) const = default;
};

struct WeightBounds {
  float minimum;
  float maximum;
  bool operator==(const WeightBounds&) const = default;
};

// Sparse LazyAdam over fp32 weight, first- and second-moment rows.
struct OptimizerConfig {
  float learning_rate;
  float beta1;
  float beta2;
  float epsilon;
  float initial_beta1_power;
  float initial_beta2_power;
  std::optional<WeightBounds> weight_bounds = std::nullopt;
  bool operator==(const OptimizerConfig&) const = default;
};

struct TableDefinition {
  TableId id;
  std::uint32_t dimension;
  std::uint32_t shard_count;
  std::uint64_t partition_epoch;
  OptimizerConfig optimizer;
  float initialization_min;
  float initialization_max;
  std::uint64_t initialization_seed;
  bool operator==(const TableDefinition&) const = default;
};

// One lookup feature: keys, bag offsets (padding already removed) and the
// original bag lengths that a mean divides by once.
struct FeatureInput {
  TableId table;
  std::uint32_t feature;
  Pooling pooling;
  std::vector<Key> keys;
  std::vector<std::uint64_t> offsets;
  std::vector<std::uint64_t> valid_lengths;
};

struct TensorBlock {
  std::uint32_t feature;
  std::vector<std::uint64_t> shape;
  std::vector<float> values;
};

struct DeviceTensor;
struct DeviceTensorBlock {
  std::uint32_t feature;
  std::vector<std::uint64_t> shape;
  std::shared_ptr<DeviceTensor> tensor;
};

struct LocatedRow {
  RowKey row;
  ShardId home;
  Placement placement;
  AgentId agent;
  std::uint64_t generation;
  std::uint64_t slot;
};

// Rows one agent serves for one feature; occurrence_to_unique maps every key
// occurrence to an index of `rows` (UINT64_MAX: served elsewhere).
struct AgentWork {
  std::uint32_t feature;
  AccessRoute route;
  AgentId agent;
  std::vector<LocatedRow> rows;
  std::vector<std::uint64_t> occurrence_to_unique;
  std::vector<float> transferred_weights;
};

struct RowState {
  RowKey row;
  std::vector<float> weights;
  std::vector<float> first_moment;
  std::vector<float> second_moment;
  std::uint64_t row_updates;
};

// Learning rate and the bias-correction powers of one table for one update.
struct UpdateContext {
  RequestId original_request;
  ShardId shard;
  TableId table;
  std::uint64_t optimizer_sequence;
  float learning_rate;
  float beta1_power;
  float beta2_power;
};

struct RowGradients {
  std::vector<RowKey> rows;
  std::vector<float> values;  // row-major, one reduced gradient per unique row
};

// CSR from each unique row to the feature-gradient rows contributing to it;
// repeated ids keep repeated, ordered references.
struct CompactGradients {
  std::vector<RowKey> rows;
  std::uint32_t dimension;
  std::vector<float> source_values;
  std::vector<std::uint64_t> row_offsets;
  std::vector<std::uint64_t> source_rows;
  std::vector<float> scales;
};

struct MigrationPlan {
  std::string id;
  AgentId agent;
  std::vector<LocatedRow> rows;
  Placement destination;
  std::uint64_t estimated_bytes;
  std::uint64_t reserve_slots = 0;
};

}  // namespace eps
