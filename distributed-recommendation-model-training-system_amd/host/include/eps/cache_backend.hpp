// eps/cache_backend.hpp -- the backend plugin interface of a parameter shard.
//
// Source-compatible restatement of the reference interface
// (include/eps/cache_backend.hpp:12-29): every operation is asynchronous and
// resolves to Result<T>; arguments are taken by value.
#pragma once

#include <future>
#include <memory>
#include <vector>

#include "eps/types.hpp"

namespace eps {

class CacheBackend {
 public:
  virtual ~CacheBackend() = default;
  virtual std::future<Result<Ack>> Define(TableDefinition table) = 0;
  virtual std::future<Result<std::uint64_t>> FreeSlots(TableId table) = 0;
  virtual std::future<Result<std::vector<LocatedRow>>> Load(MigrationPlan plan,
                                                            std::vector<RowState> states) = 0;
  virtual std::future<Result<std::vector<TensorBlock>>> GatherHost(
      std::vector<AgentWork> work, std::vector<FeatureInput> layouts) = 0;
  virtual std::future<Result<Ack>> ApplyHost(UpdateContext context, RowGradients gradients) = 0;
  // Default: expand the CSR on the host and apply it as ApplyHost.
  virtual std::future<Result<Ack>> ApplyCompact(UpdateContext context, CompactGradients packet);
  // Read-back keeps the rows resident; CommitEviction releases their slots.
  virtual std::future<Result<std::vector<RowState>>> ReadBack(MigrationPlan plan) = 0;
  virtual std::future<Result<Ack>> CommitEviction(MigrationPlan plan) = 0;
};

}  // namespace eps
