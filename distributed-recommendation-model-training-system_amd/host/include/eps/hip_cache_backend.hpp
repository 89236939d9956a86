// eps/hip_cache_backend.hpp -- MI355X (gfx950) implementation of the GPU cache
// agent.
//
// Drop-in for the reference's CudaCacheBackend
// (include/eps/cuda_cache_backend.hpp:5-37): same operations, options and
// statistics, same error behaviour, one FIFO worker per backend.  Device work
// goes through the C ABI of include/eps_hip.h (libeps_hip.so); this class owns
// the AoS [w | m | v] tables with a device key -> slot index each, the slot
// stacks, the row generations and update counters, pinned staging, one stream
// and the device-output budget.
#pragma once

#include <filesystem>
#include <future>
#include <memory>
#include <string>
#include <vector>

#include "eps/cache_agent.hpp"
#include "eps/device_features.hpp"

namespace eps {

// CudaCacheOptions field for field, with MI355X-sized limits: rows_per_table
// up to 2^31 and transfer_bytes up to 2 GiB (288 GB of HBM per device).
struct HipCacheOptions {
  AgentId agent = 0;
  int device = 0;
  std::uint64_t state_bytes = 64ULL << 20;
  std::uint64_t rows_per_table = 4096;
  std::uint64_t transfer_bytes = 16ULL << 20;
  std::uint64_t outstanding_output_bytes = 64ULL << 20;
  std::uint32_t output_alignment = 4;
};

struct HipMemoryStats {
  std::uint64_t resident_state_bytes;
  std::uint64_t staging_device_bytes;
  std::uint64_t outstanding_output_bytes;
  std::uint64_t output_allocations;
  std::uint64_t index_rebuilds = 0;  // key-index rebuilds after eviction churn, all tables
  bool operator==(const HipMemoryStats&) const = default;
};

// Identity of a shard snapshot and one of its tables, as the shard holds them
// (the fields WriteSnapshot takes from ShardStore, src/store/snapshot.cpp:159-194).
struct SnapshotIdentity {
  std::string run;
  ShardId shard;
  std::uint32_t shard_count;
  std::uint64_t epoch;
};
struct SnapshotTable {
  TableDefinition definition;
  std::uint64_t optimizer_sequence;
  float beta1_power, beta2_power;
  std::vector<Key> keys;  // row order of the file (the shard's key order)
};
struct SnapshotFile {
  std::uint64_t bytes, checksum, device_rows;
  bool operator==(const SnapshotFile&) const = default;
};

class HipCacheBackend final : public GpuCacheAgent {
 public:
  explicit HipCacheBackend(HipCacheOptions options = {});
  ~HipCacheBackend() override;
  std::future<Result<Ack>> Define(TableDefinition) override;
  std::future<Result<std::uint64_t>> FreeSlots(TableId) override;
  std::future<Result<std::vector<LocatedRow>>> Load(MigrationPlan, std::vector<RowState>) override;
  std::future<Result<std::vector<TensorBlock>>> GatherHost(std::vector<AgentWork>,
                                                           std::vector<FeatureInput>) override;
  std::future<Result<std::vector<DeviceTensorBlock>>> GatherDevice(
      std::vector<AgentWork>, std::vector<FeatureInput>) override;
  std::future<Result<Ack>> ApplyHost(UpdateContext, RowGradients) override;
  std::future<Result<Ack>> ApplyCompact(UpdateContext, CompactGradients) override;
  std::future<Result<std::vector<RowState>>> ReadBack(MigrationPlan) override;
  std::future<Result<Ack>> CommitEviction(MigrationPlan) override;
  std::future<Result<HipMemoryStats>> MemoryStats();
  std::future<Result<std::vector<DeviceTensorBlock>>> AssembleFeatures(DeviceAssemblyRequest);

  // Device-resident push of this agent's rows: per-feature gradients that are
  // already on this device ((bags, or occurrences for a sequence feature) x
  // dimension, matched to the work by feature id), with the lookup's work and
  // layouts and one UpdateContext per table.  Duplicate ids are aggregated in
  // (feature, bag, position) order and LazyAdam is applied once per unique
  // row, all on the device and all-or-nothing over the call.  The reference
  // has no device entry for this: it copies device gradients to the host
  // (adapters/entropy/runtime_c.cpp:200-204), reduces them there
  // (src/access/batch_access.cpp:54-97) and applies each table's rows through
  // ApplyHost (src/cuda/cache_backend.cu:501-513); the results are the same.
  std::future<Result<Ack>> PushDevice(std::vector<UpdateContext> contexts, std::vector<AgentWork> work,
                                      std::vector<FeatureInput> layouts,
                                      std::vector<DeviceTensorBlock> gradients);

  // Snapshot format 2 of a shard whose rows live in this backend, written
  // straight from HBM: the same bytes as the reference's WriteSnapshot
  // (src/store/snapshot.cpp:159-194) of a store holding these tables and rows,
  // with the same staging-file publication.  Each key is a row resident here
  // or one of `host_rows` (rows the shard's CPU store holds).  The reference
  // first moves every GPU row back to the CPU store, 64 rows per request
  // (src/server/service.cpp:599-612), then writes from there.
  std::future<Result<SnapshotFile>> WriteSnapshot(std::filesystem::path file, SnapshotIdentity identity,
                                                  std::vector<SnapshotTable> tables,
                                                  std::vector<RowState> host_rows);

  // Device restore from a shard snapshot file (formats 1 and 2): the plan's
  // rows are read from the file (the reference's ReadSnapshot checks,
  // src/store/snapshot.cpp:223-268: identity, schema, finite state,
  // non-negative second moments, checksum, no trailing bytes) and admitted
  // straight into HBM with their update counters, as Load admits rows
  // (src/cuda/cache_backend.cu:390-462: same plan checks, slot reserve and
  // LIFO slots, all-or-nothing).  `identity` names the checkpoint (the file's
  // run, shard, shard count and epoch must equal it); each plan row's table
  // must be defined here as the file defines it.  The reference restores into
  // its CPU store and moves GPU rows back with Load, 64 rows per request.
  std::future<Result<std::vector<LocatedRow>>> RestoreSnapshot(std::filesystem::path file,
                                                               SnapshotIdentity identity,
                                                               MigrationPlan plan);

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

}  // namespace eps
