// hip_cache_backend.cpp -- eps::HipCacheBackend over the gfx950 kernel library.
//
// Behaviour follows the reference CudaCacheBackend (src/cuda/cache_backend.cu)
// operation by operation -- validation before mutation, the same error codes
// and messages' meaning, LIFO slot reuse, row generations, atomic Load with
// rollback, device outputs that outlive the backend -- while the device work is
// the C ABI of include/eps_hip.h:
//   GatherHost / GatherDevice -> eps_hip_gather (all features in one launch)
//   ApplyHost                 -> eps_hip_adam_rows (guarded single pass)
//   ApplyCompact              -> eps_hip_adam_compact (CSR reduce fused with Adam)
//   Load / ReadBack           -> eps_hip_scatter_rows / eps_hip_gather_rows
//   AssembleFeatures          -> eps_hip_fill_u32, eps_hip_add_contribution,
//                                eps_hip_normalize_mean
//   PushDevice                -> eps_hip_prepare + eps_hip_push (device gradients)
//   WriteSnapshot             -> eps_hip_gather_rows into pinned staging, double buffered
// Occurrence slots are resolved once per unique row (the reference looks the
// row up in a hash map once per occurrence, src/cuda/cache_backend.cu:279-291).
#include "eps/hip_cache_backend.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <limits>
#include <map>
#include <numeric>
#include <set>
#include <unordered_map>
#include <utility>

#include "eps_hip.h"
#include "executor.hpp"
#include "snapshot_writer.hpp"

namespace eps {
namespace {

using hip_detail::Failure;
using hip_detail::Require;

void Hip(hipError_t status) {
  if (status != hipSuccess)
    throw Failure({status == hipErrorOutOfMemory ? Error::Code::capacity_exceeded
                                                 : Error::Code::run_failed,
                   hipGetErrorString(status)});
}

// C ABI status: 0 ok, else Error::Code + 1.
void Abi(int rc) {
  if (rc == EPS_HIP_OK) return;
  const int code = rc >= EPS_HIP_INVALID_ARGUMENT && rc <= EPS_HIP_RUN_FAILED ? rc - 1
                                                                              : int(Error::Code::run_failed);
  throw Failure({Error::Code(code), eps_hip_last_error()});
}

struct Memory {
  void* pointer = nullptr;
  int device = 0;
  bool pinned = false;
  Memory() = default;
  Memory(const Memory&) = delete;
  Memory& operator=(const Memory&) = delete;
  ~Memory() { Reset(); }
  void Reset() noexcept {
    if (!pointer) return;
    (void)hipSetDevice(device);
    if (pinned) (void)hipHostFree(pointer); else (void)hipFree(pointer);
    pointer = nullptr;
  }
  void Allocate(std::uint64_t bytes, int ordinal, bool host = false) {
    device = ordinal;
    pinned = host;
    Hip(hipSetDevice(device));
    if (!bytes) return;
    if (host) Hip(hipHostMalloc(&pointer, bytes, hipHostMallocDefault));
    else Hip(hipMalloc(&pointer, bytes));
  }
  template <typename T>
  T* As() const { return static_cast<T*>(pointer); }
};

struct Stream {
  hipStream_t value = nullptr;
  int device;
  explicit Stream(int d) : device(d) {
    Hip(hipSetDevice(d));
    Hip(hipStreamCreateWithFlags(&value, hipStreamNonBlocking));
  }
  ~Stream() {
    (void)hipSetDevice(device);
    if (value) (void)hipStreamDestroy(value);
  }
};

struct Event {
  hipEvent_t value = nullptr;
  int device;
  explicit Event(int d) : device(d) {
    Hip(hipSetDevice(d));
    Hip(hipEventCreateWithFlags(&value, hipEventDisableTiming));
  }
  ~Event() {
    (void)hipSetDevice(device);
    if (value) (void)hipEventDestroy(value);
  }
};

struct OutputBudget {
  std::atomic<std::uint64_t> used{0};
  std::atomic<std::uint64_t> allocations{0};
  std::uint64_t limit = 0;
};

// One device output allocation, charged to the backend's budget until the last
// view of it is released (possibly after the backend itself is gone).
struct Allocation {
  Memory memory;
  Event ready;
  std::shared_ptr<OutputBudget> budget;
  std::uint64_t bytes;
  Allocation(int device, std::uint64_t n, std::shared_ptr<OutputBudget> b)
      : ready(device), budget(std::move(b)), bytes(n) {
    Require(n <= budget->limit, "device output is too large", Error::Code::capacity_exceeded);
    const auto before = budget->used.fetch_add(n);
    if (before > budget->limit - n) {
      budget->used.fetch_sub(n);
      throw Failure({Error::Code::capacity_exceeded, "outstanding device output budget exhausted"});
    }
    try {
      memory.Allocate(n, device);
      ++budget->allocations;
    } catch (...) {
      budget->used.fetch_sub(n);
      throw;
    }
  }
  ~Allocation() {
    memory.Reset();
    budget->used.fetch_sub(bytes);
  }
};

class TensorView final : public DeviceTensor {
 public:
  TensorView(std::shared_ptr<Allocation> owner, std::uint64_t offset, std::uint64_t count)
      : owner_(std::move(owner)), offset_(offset), count_(count) {}
  void* data() const override {
    return owner_->memory.pointer ? owner_->memory.As<float>() + offset_ : nullptr;
  }
  std::uint64_t elements() const override { return count_; }
  int device() const override { return owner_->memory.device; }
  void WaitOnStream(void* stream) const override {
    Hip(hipSetDevice(device()));
    Hip(hipStreamWaitEvent(static_cast<hipStream_t>(stream), owner_->ready.value, 0));
  }
  std::vector<float> CopyToHost() const override {
    Hip(hipSetDevice(device()));
    Hip(hipEventSynchronize(owner_->ready.value));
    std::vector<float> values(count_);
    if (count_) Hip(hipMemcpy(values.data(), data(), count_ * 4, hipMemcpyDeviceToHost));
    return values;
  }

 private:
  std::shared_ptr<Allocation> owner_;
  std::uint64_t offset_, count_;
};

uint32_t PoolingCode(Pooling p) {
  switch (p) {
    case Pooling::sum: return EPS_HIP_POOL_SUM;
    case Pooling::mean: return EPS_HIP_POOL_MEAN;
    default: return EPS_HIP_POOL_SEQUENCE;
  }
}

}  // namespace

struct HipCacheBackend::Impl {
  struct Entry {
    LocatedRow location;
    std::uint64_t updates;
  };
  struct Table {
    TableDefinition definition;
    Memory state;
    std::vector<std::uint64_t> free;  // LIFO: slot 0 is handed out first
    std::unordered_map<Key, Entry> rows;
    eps_hip_table abi{};
  };
  struct GatherPart {
    std::uint32_t feature;
    Table* table;
    Pooling pooling;
    std::uint64_t slot_offset, offsets_offset, output_offset, rows;
    const float* source;
    std::uint64_t stride, source_rows;
  };

  explicit Impl(HipCacheOptions o)
      : options(o), stream((Validate(o), o.device)), done(o.device),
        output_budget(std::make_shared<OutputBudget>()) {
    Abi(eps_hip_device_check(o.device));
    output_budget->limit = o.outstanding_output_bytes;
    host_values.Allocate(o.transfer_bytes, o.device, true);
    host_indices.Allocate(o.transfer_bytes, o.device, true);
    device_values.Allocate(o.transfer_bytes, o.device);
    device_indices.Allocate(o.transfer_bytes, o.device);
    device_transient.Allocate(o.transfer_bytes, o.device);
    workspace.Allocate(eps_hip_update_workspace_bytes(), o.device);
    bounds.Allocate(eps_hip_bounds_bytes(), o.device);
    gather_status.Allocate(256, o.device);
    Abi(eps_hip_bounds_reset(bounds.pointer, stream.value));
    Finish();
    worker = std::make_unique<hip_detail::Worker>(128);
  }
  ~Impl() {
    worker.reset();
    (void)hipSetDevice(options.device);
    (void)hipStreamSynchronize(stream.value);
  }

  // CudaCacheOptions limits (src/cuda/cache_backend.cu:208-214), widened for
  // MI355X: 2^31 rows per table and 2 GiB of staging.
  static void Validate(const HipCacheOptions& o) {
    Require(o.output_alignment >= 4 && o.output_alignment <= 256 &&
                (o.output_alignment & (o.output_alignment - 1)) == 0 && o.rows_per_table > 0 &&
                o.rows_per_table <= (1ULL << 31) && o.transfer_bytes >= 1024 &&
                o.transfer_bytes <= (2ULL << 30),
            "invalid HIP cache limits");
  }

  void Activate() { Hip(hipSetDevice(options.device)); }
  void Finish() {
    Hip(hipEventRecord(done.value, stream.value));
    Hip(hipEventSynchronize(done.value));
  }
  Table& Get(TableId id) {
    auto it = tables.find(id);
    Require(it != tables.end(), "unknown HIP cache table");
    return *it->second;
  }
  Entry& Find(const LocatedRow& loc) {
    auto& t = Get(loc.row.table);
    auto it = t.rows.find(loc.row.key);
    Require(it != t.rows.end() && loc.agent == options.agent &&
                it->second.location.generation == loc.generation &&
                it->second.location.slot == loc.slot && it->second.location.home == loc.home,
            "HIP cache generation mismatch", Error::Code::stale_generation);
    return it->second;
  }
  void Limit(std::uint64_t bytes) const {
    Require(bytes <= options.transfer_bytes, "HIP staging budget exceeded", Error::Code::capacity_exceeded);
  }
  void CopyIn(void* device, const void* host, std::uint64_t bytes) {
    if (bytes) Hip(hipMemcpyAsync(device, host, bytes, hipMemcpyHostToDevice, stream.value));
  }

  // Occurrence slots + bag offsets into the index staging, transferred unique
  // vectors into the transient buffer (src/cuda/cache_backend.cu:251-308).
  std::pair<std::vector<GatherPart>, std::uint64_t> PrepareGather(
      const std::vector<AgentWork>& work, const std::vector<FeatureInput>& layouts) {
    std::vector<GatherPart> parts;
    parts.reserve(work.size());
    std::uint64_t indices = 0, values = 0, transferred = 0;
    auto* index = host_indices.As<std::uint64_t>();
    std::vector<std::uint64_t> slot_of;
    for (const auto& task : work) {
      auto it = std::find_if(layouts.begin(), layouts.end(),
                             [&](const FeatureInput& f) { return f.feature == task.feature; });
      Require(it != layouts.end() && task.agent == options.agent &&
                  (task.route == AccessRoute::resident_gpu ||
                   task.route == AccessRoute::transfer_unique),
              "invalid HIP gather work");
      const FeatureInput& f = *it;
      Table& table = Get(f.table);
      const std::uint64_t dim = table.definition.dimension;
      const bool transfer = task.route == AccessRoute::transfer_unique;
      Require(transfer ? task.transferred_weights.size() == task.rows.size() * dim
                       : task.transferred_weights.empty(),
              "invalid HIP transferred weights");
      const std::uint64_t transfer_offset = transferred;
      if (transfer) {
        Limit((transferred + task.transferred_weights.size()) * 4);
        for (float value : task.transferred_weights)
          Require(std::isfinite(value), "non-finite transferred weight");
        std::copy(task.transferred_weights.begin(), task.transferred_weights.end(),
                  host_values.As<float>() + transferred);
        transferred += task.transferred_weights.size();
      }
      Require(task.occurrence_to_unique.size() == f.keys.size() && !f.offsets.empty() &&
                  f.offsets.front() == 0 && f.offsets.back() == f.keys.size() &&
                  std::is_sorted(f.offsets.begin(), f.offsets.end()),
              "invalid HIP gather layout");
      Limit((indices + f.keys.size() + f.offsets.size()) * 8);
      const std::uint64_t slot_offset = indices;
      constexpr std::uint64_t kUnresolved = std::numeric_limits<std::uint64_t>::max() - 1;
      slot_of.assign(task.rows.size(), kUnresolved);
      for (std::size_t i = 0; i < f.keys.size(); ++i) {
        const std::uint64_t unique = task.occurrence_to_unique[i];
        if (unique == UINT64_MAX) {
          index[indices++] = UINT64_MAX;
          continue;
        }
        Require(unique < task.rows.size() && task.rows[unique].row == RowKey{f.table, f.keys[i]},
                "invalid HIP occurrence map");
        if (slot_of[unique] == kUnresolved) {
          if (transfer) {
            Require(task.rows[unique].placement == Placement::cpu, "transferred row is not CPU-owned");
            slot_of[unique] = unique;
          } else {
            slot_of[unique] = Find(task.rows[unique]).location.slot;
          }
        }
        index[indices++] = slot_of[unique];
      }
      const std::uint64_t offsets_offset = indices;
      std::copy(f.offsets.begin(), f.offsets.end(), index + indices);
      indices += f.offsets.size();
      const std::uint64_t rows = f.pooling == Pooling::sequence ? f.keys.size() : f.offsets.size() - 1;
      Limit((values + rows * dim) * 4);
      parts.push_back({f.feature, &table, f.pooling, slot_offset, offsets_offset, values, rows,
                       transfer ? device_transient.As<float>() + transfer_offset : table.state.As<float>(),
                       transfer ? dim : dim * 3, transfer ? task.rows.size() : options.rows_per_table});
      values += rows * dim;
    }
    CopyIn(device_indices.pointer, host_indices.pointer, indices * 8);
    CopyIn(device_transient.pointer, host_values.pointer, transferred * 4);
    return {std::move(parts), values};
  }

  // Unnormalised pooled sums (the mean divide happens once, at assembly or in
  // the client), all parts of the call in launches of up to 16 features.
  void LaunchGather(const std::vector<GatherPart>& parts, float* output) {
    auto* status = gather_status.As<uint32_t>();
    Abi(eps_hip_fill_u32(status, 0, 1, stream.value));
    std::vector<eps_hip_gather_part> abi;
    abi.reserve(parts.size());
    for (const auto& p : parts) {
      if (!p.rows) continue;
      eps_hip_gather_part g{};
      g.source = p.source;
      g.indices = device_indices.As<std::uint64_t>() + p.slot_offset;
      g.offsets = device_indices.As<std::uint64_t>() + p.offsets_offset;
      g.output = output + p.output_offset;
      g.stride = p.stride;
      g.rows = p.rows;
      g.source_rows = p.source_rows;
      g.dim = p.table->definition.dimension;
      g.pooling = PoolingCode(p.pooling);
      abi.push_back(g);
    }
    for (std::size_t i = 0; i < abi.size(); i += EPS_HIP_MAX_GATHER_PARTS) {
      const auto n = std::min<std::size_t>(EPS_HIP_MAX_GATHER_PARTS, abi.size() - i);
      Abi(eps_hip_gather(abi.data() + i, uint32_t(n), status, stream.value));
    }
  }
  void CheckGatherStatus() {
    uint32_t status = 0;
    Hip(hipMemcpy(&status, gather_status.pointer, 4, hipMemcpyDeviceToHost));
    Require(status == 0, "HIP gather met an out-of-range slot", Error::Code::run_failed);
  }

  // src/cuda/cache_backend.cu:321-333.
  Table& CheckContext(const UpdateContext& c) {
    Table& t = Get(c.table);
    Require(std::isfinite(c.learning_rate) && c.learning_rate > 0 && c.beta1_power >= 0 &&
                c.beta1_power < 1 && c.beta2_power >= 0 && c.beta2_power < 1,
            "invalid HIP update context");
    return t;
  }
  static void CheckOwner(const UpdateContext& c, const Entry& e) {
    Require(e.location.home == c.shard && e.updates != UINT64_MAX, "invalid HIP gradient owner/counter");
  }
  Table& ValidateUpdate(const UpdateContext& c, const std::vector<RowKey>& rows) {
    Table& t = CheckContext(c);
    Limit(rows.size() * std::uint64_t(t.definition.dimension) * 4);
    std::set<Key> unique;
    for (const auto& row : rows) {
      auto it = t.rows.find(row.key);
      Require(row.table == c.table && unique.insert(row.key).second && it != t.rows.end(),
              "invalid HIP gradient owner/counter");
      CheckOwner(c, it->second);
    }
    return t;
  }
  eps_hip_optimizer Optimizer(const Table& t, const UpdateContext& c) const {
    const auto& o = t.definition.optimizer;
    eps_hip_optimizer opt{};
    opt.learning_rate = c.learning_rate;
    opt.beta1 = o.beta1;
    opt.beta2 = o.beta2;
    opt.epsilon = o.epsilon;
    opt.beta1_power = c.beta1_power;
    opt.beta2_power = c.beta2_power;
    opt.bounded = o.weight_bounds ? 1 : 0;
    opt.weight_min = o.weight_bounds ? o.weight_bounds->minimum : 0.f;
    opt.weight_max = o.weight_bounds ? o.weight_bounds->maximum : 0.f;
    return opt;
  }
  // All-or-nothing: the device status says whether anything was written.
  void CheckStatus(void* ws) {
    uint32_t status = 0;
    Abi(eps_hip_read_status(ws, &status, stream.value));
    Require((status & EPS_HIP_STATUS_NONFINITE_GRAD) == 0, "non-finite gradient");
    Require((status & EPS_HIP_STATUS_REDUCE_OVERFLOW) == 0, "gradient reduction overflow");
    Require((status & (EPS_HIP_STATUS_BAD_INDEX | EPS_HIP_STATUS_ADAM_OVERFLOW)) == 0,
            "HIP optimizer state would overflow");
    Require((status & EPS_HIP_STATUS_STALLED) == 0, "HIP hot-row update did not complete",
            Error::Code::run_failed);
  }
  void FinishUpdate(Table& t, const std::vector<RowKey>& rows) {
    CheckStatus(workspace.pointer);
    for (const auto& row : rows) ++t.rows.at(row.key).updates;
  }
  // The device push workspace grows to the largest call seen (the stream is
  // idle between operations, so the old one can go).
  void ReservePush(std::uint64_t bytes) {
    if (bytes <= push_bytes) return;
    push_workspace.Reset();
    push_bytes = 0;
    push_workspace.Allocate(bytes, options.device);
    push_bytes = bytes;
  }

  HipCacheOptions options;
  Stream stream;
  Event done;
  Memory host_values, host_indices, device_values, device_indices, device_transient, workspace,
      bounds, gather_status, push_workspace;
  std::uint64_t push_bytes = 0;
  std::map<TableId, std::unique_ptr<Table>> tables;
  std::uint64_t allocated_state = 0;
  std::shared_ptr<OutputBudget> output_budget;
  std::unique_ptr<hip_detail::Worker> worker;
};

HipCacheBackend::HipCacheBackend(HipCacheOptions options) : impl_(std::make_unique<Impl>(options)) {}
HipCacheBackend::~HipCacheBackend() { impl_->worker->Stop(); }

std::future<Result<Ack>> HipCacheBackend::Define(TableDefinition d) {
  return impl_->worker->Submit<Ack>([this, d] {
    if (d.optimizer.weight_bounds) {
      const auto b = *d.optimizer.weight_bounds;
      Require(std::isfinite(b.minimum) && std::isfinite(b.maximum) && b.minimum <= b.maximum,
              "invalid optimizer weight bounds");
    }
    impl_->Activate();
    Require(d.dimension > 0 && d.dimension <= 65536, "invalid HIP dimension");
    if (auto it = impl_->tables.find(d.id); it != impl_->tables.end()) {
      Require(it->second->definition == d, "HIP table configuration mismatch");
      return Ack{};
    }
    const std::uint64_t rows = impl_->options.rows_per_table;
    const std::uint64_t bytes = rows * (std::uint64_t(d.dimension) * 12 + 8);
    Require(bytes <= impl_->options.state_bytes - impl_->allocated_state,
            "HIP table state budget exhausted", Error::Code::capacity_exceeded);
    auto t = std::make_unique<Impl::Table>();
    t->definition = d;
    t->state.Allocate(rows * std::uint64_t(d.dimension) * 12, impl_->options.device);
    t->free.resize(rows);
    std::iota(t->free.rbegin(), t->free.rend(), 0);
    t->abi = eps_hip_table{t->state.As<float>(), rows, d.dimension, d.id};
    impl_->tables.emplace(d.id, std::move(t));
    impl_->allocated_state += bytes;
    return Ack{};
  });
}

std::future<Result<std::uint64_t>> HipCacheBackend::FreeSlots(TableId id) {
  return impl_->worker->Submit<std::uint64_t>(
      [this, id] { return std::uint64_t(impl_->Get(id).free.size()); });
}

std::future<Result<std::vector<LocatedRow>>> HipCacheBackend::Load(MigrationPlan plan,
                                                                   std::vector<RowState> states) {
  return impl_->worker->Submit<std::vector<LocatedRow>>(
      [this, plan = std::move(plan), states = std::move(states)] {
        impl_->Activate();
        Require(plan.agent == impl_->options.agent && plan.rows.size() == states.size() &&
                    plan.destination == Placement::gpu,
                "invalid HIP load plan");
        std::map<TableId, std::vector<std::size_t>> groups;
        std::set<std::pair<TableId, Key>> unique;
        std::uint64_t bytes = 0;
        for (std::size_t i = 0; i < states.size(); ++i) {
          const auto& row = states[i];
          auto& t = impl_->Get(row.row.table);
          const auto dim = t.definition.dimension;
          Require(row.row == plan.rows[i].row && !t.rows.count(row.row.key) &&
                      unique.emplace(row.row.table, row.row.key).second,
                  "duplicate/existing HIP load row");
          Require(row.weights.size() == dim && row.first_moment.size() == dim &&
                      row.second_moment.size() == dim,
                  "HIP load shape mismatch");
          for (const auto* v : {&row.weights, &row.first_moment, &row.second_moment})
            for (float x : *v) Require(std::isfinite(x), "non-finite HIP load state");
          for (float x : row.second_moment) Require(x >= 0, "negative HIP second moment");
          bytes += std::uint64_t(dim) * 12;
          groups[row.row.table].push_back(i);
        }
        impl_->Limit(bytes);
        impl_->Limit(states.size() * 8);
        for (const auto& [id, rows] : groups) {
          auto& t = impl_->Get(id);
          Require(plan.reserve_slots <= t.free.size() && rows.size() <= t.free.size() - plan.reserve_slots,
                  "HIP cache slots or reserve exhausted", Error::Code::capacity_exceeded);
          t.rows.reserve(t.rows.size() + rows.size());
        }
        std::vector<LocatedRow> result(states.size());
        std::vector<std::pair<TableId, Key>> inserted;
        inserted.reserve(states.size());
        struct Group { Impl::Table* table; std::uint64_t values, slots, count; };
        std::vector<Group> copies;
        std::uint64_t value_offset = 0, slot_offset = 0;
        try {
          for (const auto& [id, rows] : groups) {
            auto& t = impl_->Get(id);
            const auto dim = t.definition.dimension;
            copies.push_back({&t, value_offset, slot_offset, rows.size()});
            for (auto i : rows) {
              const std::uint64_t slot = t.free.back();
              LocatedRow loc = plan.rows[i];
              loc.slot = slot;
              loc.agent = impl_->options.agent;
              loc.placement = Placement::gpu;
              t.rows.emplace(loc.row.key, Impl::Entry{loc, states[i].row_updates});
              t.free.pop_back();
              inserted.emplace_back(id, loc.row.key);
              result[i] = loc;
              impl_->host_indices.As<std::uint64_t>()[slot_offset++] = slot;
              for (const auto* v : {&states[i].weights, &states[i].first_moment, &states[i].second_moment}) {
                std::copy(v->begin(), v->end(), impl_->host_values.As<float>() + value_offset);
                value_offset += dim;
              }
            }
          }
          impl_->CopyIn(impl_->device_values.pointer, impl_->host_values.pointer, bytes);
          impl_->CopyIn(impl_->device_indices.pointer, impl_->host_indices.pointer, slot_offset * 8);
          for (const auto& c : copies) {
            if (!c.count) continue;
            Abi(eps_hip_scatter_rows(&c.table->abi, impl_->device_indices.As<std::uint64_t>() + c.slots,
                                     impl_->device_values.As<float>() + c.values, c.count,
                                     impl_->bounds.pointer, impl_->stream.value));
          }
          impl_->Finish();
          return result;
        } catch (...) {
          (void)hipStreamSynchronize(impl_->stream.value);
          for (auto [id, key] : inserted) {
            auto& t = impl_->Get(id);
            t.free.push_back(t.rows.at(key).location.slot);
            t.rows.erase(key);
          }
          throw;
        }
      });
}

std::future<Result<std::vector<TensorBlock>>> HipCacheBackend::GatherHost(
    std::vector<AgentWork> work, std::vector<FeatureInput> layouts) {
  return impl_->worker->Submit<std::vector<TensorBlock>>(
      [this, work = std::move(work), layouts = std::move(layouts)] {
        impl_->Activate();
        auto [parts, values] = impl_->PrepareGather(work, layouts);
        impl_->LaunchGather(parts, impl_->device_values.As<float>());
        if (values)
          Hip(hipMemcpyAsync(impl_->host_values.pointer, impl_->device_values.pointer, values * 4,
                             hipMemcpyDeviceToHost, impl_->stream.value));
        impl_->Finish();
        impl_->CheckGatherStatus();
        std::vector<TensorBlock> out;
        out.reserve(parts.size());
        for (const auto& p : parts) {
          const std::uint64_t dim = p.table->definition.dimension;
          const float* begin = impl_->host_values.As<float>() + p.output_offset;
          out.push_back({p.feature, {p.rows, dim}, {begin, begin + p.rows * dim}});
        }
        return out;
      });
}

std::future<Result<std::vector<DeviceTensorBlock>>> HipCacheBackend::GatherDevice(
    std::vector<AgentWork> work, std::vector<FeatureInput> layouts) {
  return impl_->worker->Submit<std::vector<DeviceTensorBlock>>(
      [this, work = std::move(work), layouts = std::move(layouts)] {
        impl_->Activate();
        auto [parts, values] = impl_->PrepareGather(work, layouts);
        auto allocation = std::make_shared<Allocation>(impl_->options.device, values * 4, impl_->output_budget);
        std::vector<DeviceTensorBlock> out;
        out.reserve(parts.size());
        for (const auto& p : parts) {
          const std::uint64_t dim = p.table->definition.dimension;
          out.push_back({p.feature, {p.rows, dim},
                         std::make_shared<TensorView>(allocation, p.output_offset, p.rows * dim)});
        }
        impl_->LaunchGather(parts, allocation->memory.As<float>());
        Hip(hipEventRecord(allocation->ready.value, impl_->stream.value));
        impl_->Finish();  // index staging is reusable once the launch is done
        impl_->CheckGatherStatus();
        return out;
      });
}

std::future<Result<Ack>> HipCacheBackend::ApplyHost(UpdateContext context, RowGradients g) {
  return impl_->worker->Submit<Ack>([this, context, g = std::move(g)] {
    impl_->Activate();
    auto& t = impl_->ValidateUpdate(context, g.rows);
    const std::uint64_t dim = t.definition.dimension;
    Require(g.values.size() == g.rows.size() * dim, "invalid HIP gradient shape");
    impl_->Limit(g.rows.size() * 8);
    if (g.rows.empty()) return Ack{};
    auto* slots = impl_->host_indices.As<std::uint64_t>();
    for (std::size_t i = 0; i < g.rows.size(); ++i) slots[i] = t.rows.at(g.rows[i].key).location.slot;
    std::copy(g.values.begin(), g.values.end(), impl_->host_values.As<float>());
    impl_->CopyIn(impl_->device_values.pointer, impl_->host_values.pointer, g.values.size() * 4);
    impl_->CopyIn(impl_->device_indices.pointer, slots, g.rows.size() * 8);
    const eps_hip_optimizer opt = impl_->Optimizer(t, context);
    Abi(eps_hip_adam_rows(&t.abi, &opt, impl_->device_indices.As<std::uint64_t>(),
                          impl_->device_values.As<float>(), g.rows.size(), impl_->workspace.pointer,
                          impl_->bounds.pointer, impl_->stream.value));
    impl_->FinishUpdate(t, g.rows);
    return Ack{};
  });
}

std::future<Result<Ack>> HipCacheBackend::ApplyCompact(UpdateContext context, CompactGradients p) {
  return impl_->worker->Submit<Ack>([this, context, p = std::move(p)] {
    impl_->Activate();
    hip_detail::ValidateCompact(p);
    auto& t = impl_->ValidateUpdate(context, p.rows);
    const std::uint64_t dim = t.definition.dimension;
    Require(p.dimension == dim, "compact HIP table dimension mismatch");
    const std::uint64_t slots_offset = p.row_offsets.size() + p.source_rows.size();
    const std::uint64_t index_count = slots_offset + p.rows.size();
    const std::uint64_t value_count = p.source_values.size() + p.scales.size();
    impl_->Limit(index_count * 8);
    impl_->Limit(value_count * 4);
    if (p.rows.empty()) return Ack{};
    auto* indices = impl_->host_indices.As<std::uint64_t>();
    std::copy(p.row_offsets.begin(), p.row_offsets.end(), indices);
    std::copy(p.source_rows.begin(), p.source_rows.end(), indices + p.row_offsets.size());
    for (std::size_t i = 0; i < p.rows.size(); ++i)
      indices[slots_offset + i] = t.rows.at(p.rows[i].key).location.slot;
    auto* values = impl_->host_values.As<float>();
    std::copy(p.source_values.begin(), p.source_values.end(), values);
    std::copy(p.scales.begin(), p.scales.end(), values + p.source_values.size());
    impl_->CopyIn(impl_->device_transient.pointer, values, value_count * 4);
    impl_->CopyIn(impl_->device_indices.pointer, indices, index_count * 8);
    const auto* dev_index = impl_->device_indices.As<std::uint64_t>();
    const auto* dev_value = impl_->device_transient.As<float>();
    const eps_hip_optimizer opt = impl_->Optimizer(t, context);
    Abi(eps_hip_adam_compact(&t.abi, &opt, dev_index + slots_offset, p.rows.size(), dev_index,
                             dev_index + p.row_offsets.size(), dev_value + p.source_values.size(),
                             dev_value, p.source_values.size() / dim, p.source_rows.size(),
                             impl_->workspace.pointer, impl_->bounds.pointer, impl_->stream.value));
    impl_->FinishUpdate(t, p.rows);
    return Ack{};
  });
}

std::future<Result<std::vector<RowState>>> HipCacheBackend::ReadBack(MigrationPlan plan) {
  return impl_->worker->Submit<std::vector<RowState>>([this, plan = std::move(plan)] {
    impl_->Activate();
    std::map<TableId, std::vector<std::size_t>> groups;
    std::uint64_t bytes = 0;
    std::vector<RowState> out(plan.rows.size());
    for (std::size_t i = 0; i < plan.rows.size(); ++i) {
      const auto& loc = plan.rows[i];
      auto& entry = impl_->Find(loc);
      const std::uint64_t dim = impl_->Get(loc.row.table).definition.dimension;
      out[i] = {loc.row, std::vector<float>(dim), std::vector<float>(dim), std::vector<float>(dim),
                entry.updates};
      groups[loc.row.table].push_back(i);
      bytes += dim * 12;
    }
    impl_->Limit(bytes);
    impl_->Limit(plan.rows.size() * 8);
    struct Part { Impl::Table* table; std::uint64_t values, slots, count; };
    std::vector<Part> parts;
    std::uint64_t values = 0, slots = 0;
    for (const auto& [id, members] : groups) {
      auto& t = impl_->Get(id);
      parts.push_back({&t, values, slots, members.size()});
      for (auto i : members) {
        impl_->host_indices.As<std::uint64_t>()[slots++] = impl_->Find(plan.rows[i]).location.slot;
        values += std::uint64_t(t.definition.dimension) * 3;
      }
    }
    impl_->CopyIn(impl_->device_indices.pointer, impl_->host_indices.pointer, slots * 8);
    for (const auto& p : parts) {
      if (!p.count) continue;
      Abi(eps_hip_gather_rows(&p.table->abi, impl_->device_indices.As<std::uint64_t>() + p.slots,
                              impl_->device_values.As<float>() + p.values, p.count, impl_->stream.value));
    }
    if (bytes)
      Hip(hipMemcpyAsync(impl_->host_values.pointer, impl_->device_values.pointer, bytes,
                         hipMemcpyDeviceToHost, impl_->stream.value));
    impl_->Finish();
    std::uint64_t offset = 0;
    for (const auto& [id, members] : groups) {
      const std::uint64_t dim = impl_->Get(id).definition.dimension;
      for (auto i : members) {
        for (auto* v : {&out[i].weights, &out[i].first_moment, &out[i].second_moment}) {
          std::copy_n(impl_->host_values.As<float>() + offset, dim, v->begin());
          offset += dim;
        }
      }
    }
    return out;
  });
}

std::future<Result<Ack>> HipCacheBackend::CommitEviction(MigrationPlan plan) {
  return impl_->worker->Submit<Ack>([this, plan = std::move(plan)] {
    std::set<std::pair<TableId, Key>> unique;
    for (const auto& loc : plan.rows) {
      impl_->Find(loc);
      Require(unique.emplace(loc.row.table, loc.row.key).second, "duplicate HIP eviction row");
    }
    for (const auto& loc : plan.rows) {
      auto& t = impl_->Get(loc.row.table);
      t.free.push_back(loc.slot);
      t.rows.erase(loc.row.key);
    }
    return Ack{};
  });
}

// Device feature assembly (src/cuda/cache_backend.cu:600-697): a zeroed output
// per feature, host partial sums added (scattered to sequence positions when
// projected), device contributions added after their producers' events, then
// one mean divide by the original bag lengths.
std::future<Result<std::vector<DeviceTensorBlock>>> HipCacheBackend::AssembleFeatures(
    DeviceAssemblyRequest request) {
  return impl_->worker->Submit<std::vector<DeviceTensorBlock>>([this, request = std::move(request)] {
    impl_->Activate();
    const auto& o = impl_->options;
    Require(request.host.size() == request.layouts.size() && !request.host.empty(),
            "invalid device assembly features");
    struct Target {
      std::uint64_t offset, rows, compact_rows;
      std::uint32_t dim;
      const SequenceProjection* projection;
    };
    struct Source {
      const DeviceTensor* tensor;
      std::size_t target;
      std::vector<std::uint64_t> positions;
    };
    std::map<std::uint32_t, const SequenceProjection*> projections;
    for (const auto& p : request.projections)
      Require(projections.emplace(p.feature, &p).second, "duplicate device output projection");
    std::vector<Target> targets;
    std::map<std::uint32_t, std::size_t> indices;
    std::uint64_t total = 0;
    for (std::size_t i = 0; i < request.host.size(); ++i) {
      const auto& host = request.host[i];
      const auto& layout = request.layouts[i];
      Require(layout.pooling == Pooling::sum || layout.pooling == Pooling::mean ||
                  layout.pooling == Pooling::sequence,
              "invalid device assembly pooling");
      Require(host.feature == layout.feature && host.shape.size() == 2 && host.shape[1] > 0 &&
                  host.shape[1] <= UINT32_MAX && indices.emplace(host.feature, i).second,
              "invalid device assembly schema");
      const std::uint64_t rows =
          layout.pooling == Pooling::sequence ? layout.keys.size() : layout.valid_lengths.size();
      Require(host.shape[0] == rows && rows <= o.transfer_bytes / (4 * host.shape[1]) &&
                  host.values.size() == rows * host.shape[1],
              "device assembly host shape mismatch");
      const SequenceProjection* p = nullptr;
      if (projections.count(host.feature)) {
        p = projections.at(host.feature);
        Require(layout.pooling == Pooling::sequence && p->positions.size() == rows,
                "invalid sequence output projection");
        for (std::size_t j = 0; j < p->positions.size(); ++j)
          Require(p->positions[j] < p->rows && (!j || p->positions[j - 1] < p->positions[j]),
                  "invalid output sequence position");
        impl_->Limit(p->positions.size() * 8);
      }
      const std::uint64_t output_rows = p ? p->rows : rows;
      const std::uint64_t alignment = o.output_alignment / 4;
      total = (total + alignment - 1) / alignment * alignment;
      Require(output_rows <= o.transfer_bytes / (4 * host.shape[1]), "device assembly output exceeds limit",
              Error::Code::capacity_exceeded);
      impl_->Limit((total + output_rows * host.shape[1]) * 4);
      targets.push_back({total, output_rows, rows, std::uint32_t(host.shape[1]), p});
      total += output_rows * host.shape[1];
      if (layout.pooling == Pooling::mean) impl_->Limit(layout.valid_lengths.size() * 8);
    }
    for (const auto& [id, p] : projections)
      Require(indices.count(id) > 0, "unknown device output projection");
    std::vector<Source> sources;
    sources.reserve(request.device.size());
    for (const auto& contribution : request.device) {
      const auto& block = contribution.block;
      Require(indices.count(block.feature) && bool(block.tensor), "unknown/null device contribution");
      const std::size_t ti = indices.at(block.feature);
      const Target& target = targets[ti];
      Require(block.shape.size() == 2 && block.shape[1] == target.dim &&
                  block.shape[0] <= o.transfer_bytes / (4ULL * target.dim) &&
                  block.tensor->elements() == block.shape[0] * target.dim &&
                  block.tensor->device() == o.device,
              "native contribution device/layout mismatch");
      Source source{block.tensor.get(), ti, {}};
      if (contribution.projected) {
        Require(request.layouts[ti].pooling == Pooling::sequence &&
                    contribution.positions.size() == block.shape[0],
                "invalid projected device contribution");
        source.positions.reserve(contribution.positions.size());
        for (std::size_t j = 0; j < contribution.positions.size(); ++j) {
          const std::uint64_t position = contribution.positions[j];
          Require(position < target.compact_rows && (!j || contribution.positions[j - 1] < position),
                  "invalid device contribution position");
          source.positions.push_back(target.projection ? target.projection->positions[position] : position);
        }
      } else {
        Require(contribution.positions.empty() && block.shape[0] == target.compact_rows,
                "device contribution row mismatch");
        if (target.projection) source.positions = target.projection->positions;
      }
      impl_->Limit(source.positions.size() * 8);
      sources.push_back(std::move(source));
    }
    auto allocation = std::make_shared<Allocation>(o.device, total * 4, impl_->output_budget);
    std::vector<DeviceTensorBlock> output;
    output.reserve(targets.size());
    for (std::size_t i = 0; i < targets.size(); ++i) {
      const Target& target = targets[i];
      output.push_back({request.host[i].feature, {target.rows, target.dim},
                        std::make_shared<TensorView>(allocation, target.offset, target.rows * target.dim)});
    }
    hipStream_t s = impl_->stream.value;
    float* base = allocation->memory.As<float>();
    try {
      if (total) Abi(eps_hip_fill_u32(reinterpret_cast<uint32_t*>(base), 0, total, s));
      for (std::size_t i = 0; i < targets.size(); ++i) {
        const Target& target = targets[i];
        const auto& host = request.host[i];
        if (host.values.empty()) continue;
        float* destination = base + target.offset;
        if (!target.projection) {
          Hip(hipMemcpyAsync(destination, host.values.data(), host.values.size() * 4,
                             hipMemcpyHostToDevice, s));
        } else {
          Hip(hipMemcpyAsync(impl_->device_values.pointer, host.values.data(), host.values.size() * 4,
                             hipMemcpyHostToDevice, s));
          Hip(hipMemcpyAsync(impl_->device_indices.pointer, target.projection->positions.data(),
                             target.projection->positions.size() * 8, hipMemcpyHostToDevice, s));
          Abi(eps_hip_add_contribution(destination, impl_->device_values.As<float>(),
                                       impl_->device_indices.As<std::uint64_t>(), host.values.size(),
                                       target.dim, s));
        }
      }
      for (const auto& source : sources) {
        const std::uint64_t n = source.tensor->elements();
        if (!n) continue;
        const Target& target = targets[source.target];
        source.tensor->WaitOnStream(s);
        const std::uint64_t* positions = nullptr;
        if (!source.positions.empty()) {
          Hip(hipMemcpyAsync(impl_->device_indices.pointer, source.positions.data(),
                             source.positions.size() * 8, hipMemcpyHostToDevice, s));
          positions = impl_->device_indices.As<std::uint64_t>();
        }
        Abi(eps_hip_add_contribution(base + target.offset, static_cast<const float*>(source.tensor->data()),
                                     positions, n, target.dim, s));
      }
      for (std::size_t i = 0; i < targets.size(); ++i) {
        if (request.layouts[i].pooling != Pooling::mean) continue;
        const Target& target = targets[i];
        if (!target.rows) continue;
        const auto& lengths = request.layouts[i].valid_lengths;
        Hip(hipMemcpyAsync(impl_->device_indices.pointer, lengths.data(), lengths.size() * 8,
                           hipMemcpyHostToDevice, s));
        Abi(eps_hip_normalize_mean(base + target.offset, impl_->device_indices.As<std::uint64_t>(),
                                   target.rows, target.dim, s));
      }
      Hip(hipEventRecord(allocation->ready.value, s));
      impl_->Finish();
    } catch (...) {
      (void)hipStreamSynchronize(s);
      throw;
    }
    return output;
  });
}

// Device-resident push.  Host work is the slot translation of the lookup's
// occurrence maps (once per unique row, as in PrepareGather) and the owner and
// counter checks of ValidateUpdate (src/cuda/cache_backend.cu:321-333); the
// gradients never leave the device.  eps_hip_prepare sorts the occurrences by
// (table, slot) and eps_hip_push runs ReduceGradients
// (src/access/batch_access.cpp:54-97: non-finite inputs rejected, scale
// 1/valid_length for mean, sums in (feature, bag, position) order, overflow of
// a sum rejected) fused with LazyAdam (src/update/lazy_adam.cpp:7-42), writing
// nothing unless the whole call is valid.
std::future<Result<Ack>> HipCacheBackend::PushDevice(std::vector<UpdateContext> contexts,
                                                     std::vector<AgentWork> work,
                                                     std::vector<FeatureInput> layouts,
                                                     std::vector<DeviceTensorBlock> gradients) {
  return impl_->worker->Submit<Ack>([this, contexts = std::move(contexts), work = std::move(work),
                                     layouts = std::move(layouts), gradients = std::move(gradients)] {
    Impl& I = *impl_;
    I.Activate();
    struct PushTable {
      Impl::Table* table;
      const UpdateContext* context;
      std::uint32_t index;
      std::vector<Key> rows;  // unique rows touched, first-touch order
      std::unordered_map<Key, std::uint64_t> slots;
    };
    std::map<TableId, PushTable> tables;
    for (const auto& c : contexts) {
      Impl::Table& t = I.CheckContext(c);
      Require(tables.emplace(c.table, PushTable{&t, &c, UINT32_MAX, {}, {}}).second,
              "duplicate HIP update context");
    }
    std::map<std::uint32_t, const DeviceTensorBlock*> gradient_of;
    for (const auto& g : gradients)
      Require(gradient_of.emplace(g.feature, &g).second, "duplicate gradient feature");
    Require(gradients.size() == work.size(), "gradient feature count mismatch");
    Require(work.size() <= EPS_HIP_MAX_FEATURES, "too many features for one HIP push",
            Error::Code::capacity_exceeded);
    struct Part {
      PushTable* table;
      const FeatureInput* layout;
      const DeviceTensor* gradient;
      std::uint64_t slots, offsets, lengths;
    };
    std::vector<Part> parts;
    parts.reserve(work.size());
    auto* index = I.host_indices.As<std::uint64_t>();
    std::uint64_t used = 0, occurrences = 0;
    std::uint32_t table_count = 0;
    std::set<std::uint32_t> features;
    for (const auto& task : work) {
      auto it = std::find_if(layouts.begin(), layouts.end(),
                             [&](const FeatureInput& f) { return f.feature == task.feature; });
      Require(features.insert(task.feature).second, "duplicate HIP push feature");
      Require(it != layouts.end() && task.agent == I.options.agent &&
                  task.route == AccessRoute::resident_gpu && task.transferred_weights.empty(),
              "invalid HIP push work");
      const FeatureInput& f = *it;
      auto pt = tables.find(f.table);
      Require(pt != tables.end(), "missing HIP update context");
      PushTable& target = pt->second;
      const std::uint64_t dim = target.table->definition.dimension;
      Require(task.occurrence_to_unique.size() == f.keys.size() && !f.offsets.empty() &&
                  f.offsets.front() == 0 && f.offsets.back() == f.keys.size() &&
                  std::is_sorted(f.offsets.begin(), f.offsets.end()) &&
                  f.valid_lengths.size() + 1 == f.offsets.size(),
              "invalid HIP push layout");
      auto g = gradient_of.find(f.feature);
      Require(g != gradient_of.end(), "missing feature gradient");
      const DeviceTensorBlock& block = *g->second;
      const std::uint64_t rows = f.pooling == Pooling::sequence ? f.keys.size() : f.valid_lengths.size();
      Require(block.tensor && block.shape == std::vector<std::uint64_t>{rows, dim} &&
                  block.tensor->elements() == rows * dim && block.tensor->device() == I.options.device &&
                  (rows == 0 || block.tensor->data() != nullptr),
              "gradient tensor layout mismatch");
      I.Limit((used + f.keys.size() + f.offsets.size() + f.valid_lengths.size()) * 8);
      if (target.index == UINT32_MAX) target.index = table_count++;
      Part part{&target, &f, block.tensor.get(), used, 0, 0};
      constexpr std::uint64_t kUnresolved = std::numeric_limits<std::uint64_t>::max() - 1;
      std::vector<std::uint64_t> slot_of(task.rows.size(), kUnresolved);
      for (std::size_t i = 0; i < f.keys.size(); ++i) {
        const std::uint64_t unique = task.occurrence_to_unique[i];
        if (unique == UINT64_MAX) {
          index[used++] = UINT64_MAX;
          continue;
        }
        Require(unique < task.rows.size() && task.rows[unique].row == RowKey{f.table, f.keys[i]},
                "invalid HIP occurrence map");
        if (slot_of[unique] == kUnresolved) {
          const Impl::Entry& e = I.Find(task.rows[unique]);
          Impl::CheckOwner(*target.context, e);
          slot_of[unique] = e.location.slot;
          if (target.slots.emplace(f.keys[i], e.location.slot).second) target.rows.push_back(f.keys[i]);
        }
        index[used++] = slot_of[unique];
      }
      occurrences += f.keys.size();
      part.offsets = used;
      std::copy(f.offsets.begin(), f.offsets.end(), index + used);
      used += f.offsets.size();
      part.lengths = used;
      std::copy(f.valid_lengths.begin(), f.valid_lengths.end(), index + used);
      used += f.valid_lengths.size();
      parts.push_back(part);
    }
    if (!occurrences) return Ack{};
    std::vector<eps_hip_table> abi_tables(table_count);
    std::vector<eps_hip_optimizer> optimizers(table_count);
    for (auto& [id, t] : tables) {
      if (t.index == UINT32_MAX) continue;
      abi_tables[t.index] = t.table->abi;
      optimizers[t.index] = I.Optimizer(*t.table, *t.context);
    }
    const std::uint64_t bytes = eps_hip_push_workspace_bytes(occurrences);
    I.ReservePush(bytes);
    hipStream_t s = I.stream.value;
    try {
      I.CopyIn(I.device_indices.pointer, I.host_indices.pointer, used * 8);
      const auto* device = I.device_indices.As<std::uint64_t>();
      std::vector<eps_hip_push_feature> features;
      features.reserve(parts.size());
      for (const auto& p : parts) {
        p.gradient->WaitOnStream(s);
        const FeatureInput& f = *p.layout;
        eps_hip_push_feature x{};
        x.indices = device + p.slots;
        x.offsets = device + p.offsets;
        x.valid_lengths = f.pooling == Pooling::mean ? device + p.lengths : nullptr;
        x.gradients = static_cast<const float*>(p.gradient->data());
        x.occurrences = f.keys.size();
        x.bags = f.valid_lengths.size();
        x.table = p.table->index;
        x.pooling = PoolingCode(f.pooling);
        features.push_back(x);
      }
      Abi(eps_hip_prepare(abi_tables.data(), table_count, features.data(), std::uint32_t(features.size()),
                          I.push_workspace.pointer, bytes, s));
      Abi(eps_hip_push(abi_tables.data(), optimizers.data(), table_count, features.data(),
                       std::uint32_t(features.size()), I.push_workspace.pointer, bytes, I.bounds.pointer, s));
      I.CheckStatus(I.push_workspace.pointer);
    } catch (...) {
      (void)hipStreamSynchronize(s);
      throw;
    }
    for (auto& [id, t] : tables)
      for (Key key : t.rows) ++t.table->rows.at(key).updates;
    return Ack{};
  });
}

// Snapshot writeback.  Rows are encoded in file order chunk by chunk: the
// device rows of chunk c + 1 are gathered into one half of the pinned staging
// (eps_hip_gather_rows writes host memory directly) while the host hashes and
// writes chunk c from the other half.  The checksum, a byte-serial FNV-1a, is
// the host's share and bounds the rate.
std::future<Result<SnapshotFile>> HipCacheBackend::WriteSnapshot(std::filesystem::path file,
                                                                 SnapshotIdentity identity,
                                                                 std::vector<SnapshotTable> tables,
                                                                 std::vector<RowState> host_rows) {
  return impl_->worker->Submit<SnapshotFile>([this, file = std::move(file), identity = std::move(identity),
                                              tables = std::move(tables),
                                              host_rows = std::move(host_rows)] {
    Impl& I = *impl_;
    I.Activate();
    // The identity and schema checks the reference reader applies
    // (src/store/snapshot.cpp:201-206,230-245), so a written file restores.
    Require(!identity.run.empty() && identity.run.size() <= 1024 && identity.shard_count > 0 &&
                identity.shard < identity.shard_count && identity.epoch > 0 && tables.size() <= 1024,
            "invalid snapshot identity");
    std::map<std::pair<TableId, Key>, const RowState*> host;
    for (const auto& r : host_rows)
      Require(host.emplace(std::make_pair(r.row.table, r.row.key), &r).second, "duplicate snapshot host row");
    std::set<TableId> ids;
    std::uint64_t device_rows = 0;
    for (const auto& t : tables) {
      const auto& d = t.definition;
      Require(ids.insert(d.id).second && d.dimension > 0 && d.dimension <= 65536 &&
                  d.shard_count == identity.shard_count && d.partition_epoch == identity.epoch &&
                  t.beta1_power >= 0 && t.beta1_power < 1 && t.beta2_power >= 0 && t.beta2_power < 1,
              "invalid snapshot table");
      auto it = I.tables.find(d.id);
      Require(it == I.tables.end() || it->second->definition == d, "HIP table configuration mismatch");
      std::set<Key> keys;
      for (Key key : t.keys) {
        Require(keys.insert(key).second, "duplicate snapshot row");
        const bool resident = it != I.tables.end() && it->second->rows.count(key);
        auto h = host.find({d.id, key});
        Require(resident != (h != host.end()), "snapshot row must be held by exactly one store");
        if (resident) {
          ++device_rows;
        } else {
          const RowState& r = *h->second;
          Require(r.weights.size() == d.dimension && r.first_moment.size() == d.dimension &&
                      r.second_moment.size() == d.dimension,
                  "snapshot host row shape mismatch");
        }
      }
      Require(it == I.tables.end() || 2 * std::uint64_t(d.dimension) * 12 <= I.options.transfer_bytes,
              "snapshot row exceeds the staging buffer", Error::Code::capacity_exceeded);
    }

    hip_detail::SnapshotWriter out(file);
    hip_detail::WriteSnapshotHeader(out, identity, tables.size());
    Event ready[2] = {Event(I.options.device), Event(I.options.device)};
    const std::uint64_t half_bytes = I.options.transfer_bytes / 2;
    for (const auto& t : tables) {
      const auto& d = t.definition;
      hip_detail::WriteSnapshotTable(out, t);
      auto it = I.tables.find(d.id);
      Impl::Table* table = it == I.tables.end() ? nullptr : it->second.get();
      const std::uint64_t floats = std::uint64_t(d.dimension) * 3;
      const std::uint64_t cap = table ? std::min(half_bytes / (floats * 4), half_bytes / 8) : 0;
      // Chunks: [begin, end) of the key list holding at most `cap` device rows.
      std::vector<std::pair<std::size_t, std::size_t>> chunks;
      for (std::size_t b = 0; b < t.keys.size();) {
        std::size_t e = b;
        std::uint64_t n = 0;
        while (e < t.keys.size() && (!table || !table->rows.count(t.keys[e]) || n < cap)) {
          if (table && table->rows.count(t.keys[e])) ++n;
          ++e;
        }
        chunks.emplace_back(b, e);
        b = e;
      }
      auto issue = [&](std::size_t c) {
        const int h = int(c % 2);
        auto* slots = I.host_indices.As<std::uint64_t>() + h * (half_bytes / 8);
        std::uint64_t n = 0;
        for (std::size_t i = chunks[c].first; i < chunks[c].second; ++i)
          if (table)
            if (auto r = table->rows.find(t.keys[i]); r != table->rows.end()) slots[n++] = r->second.location.slot;
        if (n) {
          auto* dslots = I.device_indices.As<std::uint64_t>() + h * (half_bytes / 8);
          I.CopyIn(dslots, slots, n * 8);
          Abi(eps_hip_gather_rows(&table->abi, dslots,
                                  reinterpret_cast<float*>(I.host_values.As<unsigned char>() + h * half_bytes), n,
                                  I.stream.value));
        }
        Hip(hipEventRecord(ready[h].value, I.stream.value));
      };
      try {
        if (!chunks.empty()) issue(0);
        for (std::size_t c = 0; c < chunks.size(); ++c) {
          if (c + 1 < chunks.size()) issue(c + 1);
          const int h = int(c % 2);
          Hip(hipEventSynchronize(ready[h].value));
          const float* staged = reinterpret_cast<const float*>(I.host_values.As<unsigned char>() + h * half_bytes);
          std::uint64_t n = 0;
          for (std::size_t i = chunks[c].first; i < chunks[c].second; ++i) {
            const Key key = t.keys[i];
            const Impl::Entry* entry = nullptr;
            if (table)
              if (auto r = table->rows.find(key); r != table->rows.end()) entry = &r->second;
            if (entry) {
              hip_detail::WriteSnapshotRow(out, key, entry->updates, staged + n * floats, d.dimension);
              ++n;
            } else {
              hip_detail::WriteSnapshotRow(out, *host.at({d.id, key}));
            }
          }
        }
      } catch (...) {
        (void)hipStreamSynchronize(I.stream.value);
        throw;
      }
    }
    const std::uint64_t bytes = out.bytes() + 8;
    const std::uint64_t checksum = out.Publish();
    return SnapshotFile{bytes, checksum, device_rows};
  });
}

std::future<Result<HipMemoryStats>> HipCacheBackend::MemoryStats() {
  return impl_->worker->Submit<HipMemoryStats>([this] {
    std::uint64_t state = 0;
    for (const auto& [id, table] : impl_->tables)
      state += impl_->options.rows_per_table * std::uint64_t(table->definition.dimension) * 12;
    const std::uint64_t staging = impl_->options.transfer_bytes * 3 + eps_hip_update_workspace_bytes() +
                                  eps_hip_bounds_bytes() + 256 + impl_->push_bytes;
    return HipMemoryStats{state, staging, impl_->output_budget->used.load(),
                          impl_->output_budget->allocations.load()};
  });
}

}  // namespace eps
