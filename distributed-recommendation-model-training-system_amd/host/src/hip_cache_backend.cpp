// hip_cache_backend.cpp -- eps::HipCacheBackend: the GPU cache agent of a
// parameter shard on one MI355X, over the kernel library's C ABI.
//
// Operation          device work (include/eps_hip.h)
//   Define           device table + key index (eps_hip_index_clear)
//   Load             eps_hip_scatter_rows, eps_hip_index_insert
//   GatherHost/Device eps_hip_resolve (key index), eps_hip_gather
//   ApplyHost        eps_hip_adam_rows
//   ApplyCompact     eps_hip_adam_compact
//   ReadBack         eps_hip_gather_rows
//   CommitEviction   eps_hip_index_remove
//   AssembleFeatures eps_hip_fill_u32, eps_hip_add_contribution, eps_hip_normalize_mean
//   PushDevice       eps_hip_resolve, eps_hip_prepare, eps_hip_push
//   WriteSnapshot    eps_hip_gather_rows into pinned staging, double buffered
//   RestoreSnapshot  eps_hip_scatter_rows, eps_hip_index_insert
//
// The observable contract is the reference CudaCacheBackend's
// (src/cuda/cache_backend.cu; include/eps/cache_backend.hpp:12-29): the same
// checks before any state changes and the same error codes, slots handed out
// from slot 0 and reused last-freed first, row generations and update counters
// kept by the agent, atomic loads, device outputs that outlive the backend.
// The design is this file's: every request is resolved against the host-side
// residency of its unique rows only (generation, owner, counter checks: O(rows),
// not O(occurrences)), its arrays are carved out of one pinned + device
// transfer area and uploaded with one copy, and each key occurrence is turned
// into a slot on the device by the table's key index, which also checks the
// caller's occurrence map.  Gathers and pushes share that resolution and
// build their kernel descriptors from it.
#include "eps/hip_cache_backend.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <cmath>
#include <cstring>
#include <limits>
#include <map>
#include <optional>
#include <set>
#include <unordered_map>
#include <unordered_set>
#include <utility>

#include "eps_hip.h"
#include "job_queue.hpp"
#include "packet.hpp"
#include "snapshot_reader.hpp"
#include "snapshot_writer.hpp"

namespace eps {
namespace {

using hipbk::Expect;
using hipbk::Raise;
using Code = Error::Code;

constexpr std::uint64_t kHole = ~0ull;
constexpr std::size_t kQueueDepth = 128;
constexpr std::uint32_t kFailureBits = 0x7f;

void HipOk(hipError_t e, const char* what) {
  if (e == hipSuccess) return;
  Raise(e == hipErrorOutOfMemory ? Code::capacity_exceeded : Code::run_failed,
        std::string(what) + ": " + hipGetErrorString(e));
}

// A C ABI result (0, or Error::Code + 1).
void AbiOk(int rc) {
  if (rc == EPS_HIP_OK) return;
  const bool known = rc >= EPS_HIP_INVALID_ARGUMENT && rc <= EPS_HIP_RUN_FAILED;
  Raise(known ? Code(rc - 1) : Code::run_failed, eps_hip_last_error());
}

std::uint64_t RoundUp(std::uint64_t x, std::uint64_t to) { return (x + to - 1) / to * to; }

// ---------------------------------------------------------------------------
// Memory the backend owns: device memory or pinned host memory.
class Memory {
 public:
  Memory() = default;
  Memory(const Memory&) = delete;
  Memory& operator=(const Memory&) = delete;
  ~Memory() { Release(); }
  void Acquire(int device, std::uint64_t bytes, bool pinned) {
    Release();
    device_ = device;
    pinned_ = pinned;
    bytes_ = bytes;
    HipOk(hipSetDevice(device), "select device");
    if (!bytes) return;
    if (pinned) HipOk(hipHostMalloc(&p_, bytes, hipHostMallocDefault), "pinned host allocation");
    else HipOk(hipMalloc(&p_, bytes), "device allocation");
  }
  void Release() noexcept {
    if (!p_) return;
    (void)hipSetDevice(device_);
    if (pinned_) (void)hipHostFree(p_);
    else (void)hipFree(p_);
    p_ = nullptr;
  }
  template <typename T = void>
  T* Get() const { return static_cast<T*>(p_); }
  std::uint64_t bytes() const { return bytes_; }

 private:
  void* p_ = nullptr;
  int device_ = 0;
  bool pinned_ = false;
  std::uint64_t bytes_ = 0;
};

// ---------------------------------------------------------------------------
// The staging of one request: a pinned host area and a device area of the
// same size, carved front to back.  Inputs are written into the host side
// and uploaded with one copy; device-only pieces (kernel outputs) follow them.
class Transfer {
 public:
  template <typename T>
  struct Piece {
    T* host;
    T* device;
    std::uint64_t count;
  };

  void Open(int device, std::uint64_t bytes) {
    host_.Acquire(device, bytes, true);
    device_.Acquire(device, bytes, false);
    capacity_ = bytes;
  }
  void Reset() { used_ = uploaded_ = 0; }
  std::uint64_t capacity() const { return capacity_; }
  std::uint64_t device_bytes() const { return device_.bytes(); }

  template <typename T>
  Piece<T> Take(std::uint64_t count) {
    const std::uint64_t at = RoundUp(used_, 256);
    Expect(count <= (capacity_ - std::min(at, capacity_)) / sizeof(T), "request exceeds the transfer staging",
           Code::capacity_exceeded);
    used_ = at + count * sizeof(T);
    auto* h = reinterpret_cast<T*>(host_.Get<unsigned char>() + at);
    auto* d = reinterpret_cast<T*>(device_.Get<unsigned char>() + at);
    return {h, d, count};
  }
  template <typename T>
  Piece<T> Copy(const std::vector<T>& values) {
    Piece<T> p = Take<T>(values.size());
    if (!values.empty()) std::memcpy(p.host, values.data(), values.size() * sizeof(T));
    return p;
  }
  // Copies everything taken since the last upload to the device.
  void Upload(hipStream_t stream) {
    if (used_ > uploaded_)
      HipOk(hipMemcpyAsync(device_.Get<unsigned char>() + uploaded_, host_.Get<unsigned char>() + uploaded_,
                           used_ - uploaded_, hipMemcpyHostToDevice, stream),
            "staging upload");
    uploaded_ = used_;
  }
  // Marks what was taken so far as device-only (it is not uploaded).
  void Skip() { uploaded_ = used_; }
  template <typename T>
  void Download(const Piece<T>& p, hipStream_t stream) {
    if (p.count)
      HipOk(hipMemcpyAsync(p.host, p.device, p.count * sizeof(T), hipMemcpyDeviceToHost, stream), "staging download");
  }

 private:
  Memory host_, device_;
  std::uint64_t capacity_ = 0, used_ = 0, uploaded_ = 0;
};

// ---------------------------------------------------------------------------
// Device outputs: one allocation per request, viewed by one tensor per
// feature; the allocation lives while any view does (past the backend) and
// is charged to the backend's outstanding-output budget meanwhile.
struct OutputLedger {
  std::atomic<std::uint64_t> used{0}, blocks{0};
  std::uint64_t limit = 0;
};

class OutputBlock {
 public:
  OutputBlock(std::shared_ptr<OutputLedger> ledger, int device, std::uint64_t bytes)
      : ledger_(std::move(ledger)), device_(device), bytes_(bytes) {
    Expect(bytes <= ledger_->limit, "device output larger than the output budget", Code::capacity_exceeded);
    std::uint64_t seen = ledger_->used.load();
    do {
      Expect(seen <= ledger_->limit - bytes, "outstanding device outputs exhaust the budget",
             Code::capacity_exceeded);
    } while (!ledger_->used.compare_exchange_weak(seen, seen + bytes));
    try {
      memory_.Acquire(device, bytes, false);
      HipOk(hipEventCreateWithFlags(&ready_, hipEventDisableTiming), "output event");
    } catch (...) {
      memory_.Release();
      ledger_->used.fetch_sub(bytes);
      throw;
    }
    ledger_->blocks.fetch_add(1);
  }
  ~OutputBlock() {
    memory_.Release();
    if (ready_) {
      (void)hipSetDevice(device_);
      (void)hipEventDestroy(ready_);
    }
    ledger_->used.fetch_sub(bytes_);
  }
  float* data() const { return memory_.Get<float>(); }
  hipEvent_t ready() const { return ready_; }
  int device() const { return device_; }

 private:
  std::shared_ptr<OutputLedger> ledger_;
  int device_;
  std::uint64_t bytes_;
  Memory memory_;
  hipEvent_t ready_ = nullptr;
};

class OutputSlice final : public DeviceTensor {
 public:
  OutputSlice(std::shared_ptr<OutputBlock> block, std::uint64_t offset, std::uint64_t count)
      : block_(std::move(block)), offset_(offset), count_(count) {}
  void* data() const override { return block_->data() ? block_->data() + offset_ : nullptr; }
  std::uint64_t elements() const override { return count_; }
  int device() const override { return block_->device(); }
  void WaitOnStream(void* stream) const override {
    HipOk(hipSetDevice(block_->device()), "select device");
    HipOk(hipStreamWaitEvent(static_cast<hipStream_t>(stream), block_->ready(), 0), "wait for device output");
  }
  std::vector<float> CopyToHost() const override {
    HipOk(hipSetDevice(block_->device()), "select device");
    HipOk(hipEventSynchronize(block_->ready()), "wait for device output");
    std::vector<float> out(count_);
    if (count_) HipOk(hipMemcpy(out.data(), data(), count_ * 4, hipMemcpyDeviceToHost), "device output copy");
    return out;
  }

 private:
  std::shared_ptr<OutputBlock> block_;
  std::uint64_t offset_, count_;
};

// ---------------------------------------------------------------------------
// One table on the device: the AoS [w | m | v] rows, the key index, the slot
// stack (its back is the next slot handed out) and the residency of every
// row the agent holds.
struct Resident {
  LocatedRow where;
  std::uint64_t updates;
};

struct SlotTable {
  TableDefinition definition;
  eps_hip_table abi{};
  Memory state, index;
  std::uint64_t index_capacity = 0;
  std::uint64_t removed_since_rebuild = 0;  // key removals since the index was last built
  std::vector<std::uint64_t> free_slots;
  std::unordered_map<Key, Resident> rows;

  std::uint32_t dim() const { return definition.dimension; }
  std::uint64_t TakeSlot() {
    const std::uint64_t s = free_slots.back();
    free_slots.pop_back();
    return s;
  }
};

bool Finite(const std::vector<float>& v) {
  return std::all_of(v.begin(), v.end(), [](float x) { return std::isfinite(x); });
}

}  // namespace

// ---------------------------------------------------------------------------
struct HipCacheBackend::Impl {
  explicit Impl(const HipCacheOptions& o) : options(o), ledger(std::make_shared<OutputLedger>()) {
    Expect(o.output_alignment >= 4 && o.output_alignment <= 256 && (o.output_alignment & (o.output_alignment - 1)) == 0 &&
               o.rows_per_table > 0 && o.rows_per_table <= (1ull << 31) && o.transfer_bytes >= 1024 &&
               o.transfer_bytes <= (2ull << 30),
           "invalid HIP cache options");
    ledger->limit = o.outstanding_output_bytes;
    AbiOk(eps_hip_device_check(o.device));
    HipOk(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "create stream");
    transfer.Open(o.device, o.transfer_bytes);
    bounds.Acquire(o.device, eps_hip_bounds_bytes(), false);
    AbiOk(eps_hip_bounds_reset(bounds.Get(), stream));
    update_ws.Acquire(o.device, eps_hip_update_workspace_bytes(), false);
    AbiOk(eps_hip_fill_u32(update_ws.Get<std::uint32_t>(), 0, update_ws.bytes() / 4, stream));
    flags.Acquire(o.device, 256, false);
    flags_host.Acquire(o.device, 256, true);
    Await();
    queue = std::make_unique<hipbk::JobQueue>(kQueueDepth);
  }
  ~Impl() {
    queue.reset();  // runs what was queued, then stops
    (void)hipSetDevice(options.device);
    if (stream) {
      (void)hipStreamSynchronize(stream);
      (void)hipStreamDestroy(stream);
    }
  }

  // Set when a device push may have been applied in part (a stalled hot-row
  // hand-over, or a prepared workspace naming rows or gradients the push does
  // not have): the tables can no longer be trusted, so every later operation
  // fails with run_failed.  Recovery is a fresh backend and RestoreSnapshot.
  bool stopped = false;
  void Activate() {
    HipOk(hipSetDevice(options.device), "select device");
    if (stopped) Raise(Code::run_failed, "HIP agent stopped after a device push that may be partial; restore a snapshot");
  }
  void Await() { HipOk(hipStreamSynchronize(stream), "device work"); }

  SlotTable& Table(TableId id) {
    auto it = tables.find(id);
    Expect(it != tables.end(), "table is not defined on this HIP agent");
    return *it->second;
  }

  // The residency of a located row, which must be this agent's current copy.
  Resident& Locate(const LocatedRow& loc) {
    SlotTable& t = Table(loc.row.table);
    auto it = t.rows.find(loc.row.key);
    const bool current = it != t.rows.end() && loc.agent == options.agent &&
                         it->second.where.generation == loc.generation && it->second.where.slot == loc.slot &&
                         it->second.where.home == loc.home;
    Expect(current, "row is not resident at this generation on this HIP agent", Code::stale_generation);
    return it->second;
  }

  // A removed key leaves a kGone bucket wherever later keys may sit past it;
  // inserts reuse such buckets but nothing empties them, so under admission
  // and eviction churn they would pile up and lengthen every probe that
  // misses.  Once a table has seen removals to a quarter of its buckets, its
  // index is built again from the resident map: cleared, then every resident
  // key inserted with its slot.  Probe chains then stay bounded by the live
  // load (at most half the buckets), at a cost of one insert per resident row
  // per capacity/4 removals.  A rebuild that fails part-way leaves keys
  // unfindable, so it stops the agent.
  void RebuildIndexIfWorn(SlotTable& t) {
    if (t.removed_since_rebuild <= t.index_capacity / 4) return;
    try {
      Await();  // the staging area may still feed earlier work
      AbiOk(eps_hip_index_clear(t.index.Get(), t.index_capacity, stream));
      ClearFlag();
      const std::uint64_t piece = (transfer.capacity() - 2 * 256) / 16;
      std::uint64_t left = t.rows.size();
      auto it = t.rows.begin();
      while (left) {
        const std::uint64_t n = std::min(piece, left);
        Await();  // the previous piece's upload has left the host staging
        transfer.Reset();
        auto keys = transfer.Take<std::uint64_t>(n);
        auto slots = transfer.Take<std::uint64_t>(n);
        for (std::uint64_t j = 0; j < n; ++j, ++it) {
          keys.host[j] = it->first;
          slots.host[j] = it->second.where.slot;
        }
        transfer.Upload(stream);
        AbiOk(eps_hip_index_insert(t.index.Get(), t.index_capacity, keys.device, slots.device, n, Flag(), stream));
        left -= n;
      }
      Expect(!(ReadFlag(Flag()) & EPS_HIP_STATUS_BAD_INDEX), "HIP key index rebuild overflowed", Code::run_failed);
      transfer.Reset();
      t.removed_since_rebuild = 0;
      ++index_rebuilds;
    } catch (...) {
      stopped = true;
      throw;
    }
  }
  std::uint64_t index_rebuilds = 0;

  // Status flags of one request: word 0 collects the resolution and index
  // results; the push and update workspaces hold their own.
  std::uint32_t* Flag() { return flags.Get<std::uint32_t>(); }
  void ClearFlag() { AbiOk(eps_hip_fill_u32(Flag(), 0, 1, stream)); }
  std::uint32_t ReadFlag(const std::uint32_t* device_word) {
    HipOk(hipMemcpyAsync(flags_host.Get(), device_word, 4, hipMemcpyDeviceToHost, stream), "status copy");
    Await();
    return *flags_host.Get<std::uint32_t>();
  }

  // Failure bits of an update -> the reference's error for the same case:
  // non-finite inputs and overflow are request errors (invalid_argument,
  // src/update/lazy_adam.cpp:7-23, src/access/batch_access.cpp:23-95); a bad
  // slot or a stalled hand-over is this agent's own failure.
  static void UpdateVerdict(std::uint32_t status) {
    if (!(status & kFailureBits)) return;
    if (status & (EPS_HIP_STATUS_STALLED | EPS_HIP_STATUS_BAD_INDEX))
      Raise(Code::run_failed, "HIP update failed on the device");
    if (status & EPS_HIP_STATUS_NONFINITE_GRAD) Raise(Code::invalid_argument, "non-finite gradient");
    if (status & EPS_HIP_STATUS_BAD_SCALE) Raise(Code::invalid_argument, "invalid gradient scale");
    Raise(Code::invalid_argument, "optimizer state would overflow");
  }

  eps_hip_optimizer Optimizer(const SlotTable& t, float lr, float b1p, float b2p) const {
    const OptimizerConfig& o = t.definition.optimizer;
    eps_hip_optimizer x{};
    x.learning_rate = lr;
    x.beta1 = o.beta1;
    x.beta2 = o.beta2;
    x.epsilon = o.epsilon;
    x.beta1_power = b1p;
    x.beta2_power = b2p;
    x.bounded = o.weight_bounds ? 1 : 0;
    x.weight_min = o.weight_bounds ? o.weight_bounds->minimum : 0.f;
    x.weight_max = o.weight_bounds ? o.weight_bounds->maximum : 0.f;
    return x;
  }

  static void CheckContext(const UpdateContext& c) {
    // src/cuda/cache_backend.cu:321-325.
    Expect(std::isfinite(c.learning_rate) && c.learning_rate > 0 && c.beta1_power >= 0 && c.beta1_power < 1 &&
               c.beta2_power >= 0 && c.beta2_power < 1,
           "invalid update context");
  }

  // Rows of one update: in the context's table, distinct, held here for the
  // context's shard, counters not saturated.  Returns their residencies.
  std::vector<Resident*> UpdateRows(const UpdateContext& c, SlotTable& t, const std::vector<RowKey>& rows) {
    std::vector<Resident*> out;
    out.reserve(rows.size());
    std::unordered_set<Key> seen;
    for (const RowKey& r : rows) {
      auto it = t.rows.find(r.key);
      Expect(r.table == c.table && seen.insert(r.key).second && it != t.rows.end() &&
                 it->second.where.home == c.shard && it->second.updates != UINT64_MAX,
             "update row is not a distinct row this agent holds for the shard");
      out.push_back(&it->second);
    }
    return out;
  }

  // ---- request resolution shared by gathers and pushes ----
  struct Resolved {
    const AgentWork* work;
    const FeatureInput* layout;
    SlotTable* table;
    bool carried;            // transfer_unique: rows travel with the request
    std::uint64_t rows;      // output rows (bags, or occurrences for sequence)
    std::uint64_t occurrences;
    std::uint64_t* slots;    // device: per occurrence slot (or unique index when carried), kHole elsewhere
    std::uint64_t* offsets;  // device: bags + 1
    std::uint64_t* lengths;  // device: bags
    const float* carried_rows;  // device: unique rows x dim (carried only)
    std::vector<const Resident*> unique;  // resident unique rows
  };

  std::vector<Resolved> ResolveWork(const std::vector<AgentWork>& work, const std::vector<FeatureInput>& layouts,
                                    bool allow_carried) {
    std::unordered_map<std::uint32_t, const FeatureInput*> by_feature;
    for (const auto& f : layouts) by_feature.emplace(f.feature, &f);
    std::unordered_set<std::uint32_t> served;
    std::vector<Resolved> out;
    out.reserve(work.size());
    struct Staged {
      Transfer::Piece<std::uint64_t> keys, occ, unique_keys;
    };
    std::vector<Staged> staged;
    staged.reserve(work.size());
    transfer.Reset();
    for (const AgentWork& w : work) {
      auto f = by_feature.find(w.feature);
      const bool carried = w.route == AccessRoute::transfer_unique;
      Expect(f != by_feature.end() && served.insert(w.feature).second && w.agent == options.agent &&
                 (w.route == AccessRoute::resident_gpu || (allow_carried && carried)),
             "invalid HIP agent work");
      const FeatureInput& L = *f->second;
      SlotTable& t = Table(L.table);
      const std::uint32_t dim = t.dim();
      const bool seq = L.pooling == Pooling::sequence;
      // Mean pooling needs every bag's original length (its gradient scale).
      bool layout_ok = w.occurrence_to_unique.size() == L.keys.size() && !L.offsets.empty() &&
                       L.offsets.front() == 0 && L.offsets.back() == L.keys.size() &&
                       std::is_sorted(L.offsets.begin(), L.offsets.end()) &&
                       (L.pooling != Pooling::mean || L.valid_lengths.size() + 1 == L.offsets.size());
      Expect(layout_ok, "invalid HIP lookup layout");
      Resolved r{&w, &L, &t, carried, seq ? L.keys.size() : L.offsets.size() - 1, L.keys.size(),
                 nullptr, nullptr, nullptr, nullptr, {}};
      if (carried) {
        Expect(w.transferred_weights.size() == w.rows.size() * std::uint64_t(dim),
               "transferred weights do not match the work rows");
        Expect(Finite(w.transferred_weights), "non-finite transferred weight");
        for (const LocatedRow& loc : w.rows)
          Expect(loc.placement == Placement::cpu && loc.row.table == L.table, "transferred row is not CPU-owned");
      } else {
        Expect(w.transferred_weights.empty(), "resident work carries weights");
        r.unique.reserve(w.rows.size());
        for (const LocatedRow& loc : w.rows) {
          Expect(loc.row.table == L.table, "work row belongs to another table");
          r.unique.push_back(&Locate(loc));
        }
      }
      Staged s{transfer.Copy(L.keys), transfer.Copy(w.occurrence_to_unique), transfer.Take<std::uint64_t>(w.rows.size())};
      for (std::size_t u = 0; u < w.rows.size(); ++u) s.unique_keys.host[u] = w.rows[u].row.key;
      auto offsets = transfer.Copy(L.offsets);
      auto lengths = transfer.Copy(L.valid_lengths);
      r.offsets = offsets.device;
      r.lengths = L.valid_lengths.empty() ? nullptr : lengths.device;
      if (carried) r.carried_rows = transfer.Copy(w.transferred_weights).device;
      staged.push_back(s);
      out.push_back(std::move(r));
    }
    transfer.Upload(stream);
    for (auto& r : out) r.slots = transfer.Take<std::uint64_t>(r.occurrences).device;
    transfer.Skip();
    ClearFlag();
    for (std::size_t i = 0; i < out.size(); ++i) {
      Resolved& r = out[i];
      const Staged& s = staged[i];
      AbiOk(eps_hip_resolve(r.carried ? nullptr : r.table->index.Get(), r.table->index_capacity, s.keys.device,
                            s.occ.device, s.unique_keys.device, s.unique_keys.count, r.occurrences, r.slots, Flag(),
                            stream));
    }
    return out;
  }

  // Pooled gather of resolved features into `output` (dim-wide rows, feature
  // after feature at the given float offsets).
  void Gather(const std::vector<Resolved>& parts, float* output, const std::vector<std::uint64_t>& at) {
    std::vector<eps_hip_gather_part> abi;
    abi.reserve(parts.size());
    for (std::size_t i = 0; i < parts.size(); ++i) {
      const Resolved& r = parts[i];
      const std::uint32_t dim = r.table->dim();
      eps_hip_gather_part g{};
      g.source = r.carried ? r.carried_rows : r.table->abi.state;
      g.indices = r.occurrences ? r.slots : nullptr;
      g.offsets = r.layout->pooling == Pooling::sequence ? nullptr : r.offsets;
      g.output = output + at[i];
      g.stride = r.carried ? dim : 3ull * dim;
      g.rows = r.rows;
      g.source_rows = r.carried ? r.work->rows.size() : options.rows_per_table;
      g.dim = dim;
      g.pooling = r.layout->pooling == Pooling::sum ? EPS_HIP_POOL_SUM
                  : r.layout->pooling == Pooling::mean ? EPS_HIP_POOL_MEAN
                                                       : EPS_HIP_POOL_SEQUENCE;
      abi.push_back(g);
    }
    for (std::size_t b = 0; b < abi.size(); b += EPS_HIP_MAX_GATHER_PARTS) {
      const auto n = std::uint32_t(std::min<std::size_t>(EPS_HIP_MAX_GATHER_PARTS, abi.size() - b));
      AbiOk(eps_hip_gather(abi.data() + b, n, Flag(), stream));
    }
  }

  void CheckResolution() {
    Expect(!(ReadFlag(Flag()) & EPS_HIP_STATUS_BAD_INDEX), "occurrence map does not match the lookup");
  }

  // Grows the push workspace to `occurrences`; a fresh one is zero-filled.
  void ReservePush(std::uint64_t occurrences) {
    const std::uint64_t need = eps_hip_push_workspace_bytes(occurrences);
    if (need <= push_ws.bytes()) return;
    Await();
    push_ws.Acquire(options.device, need, false);
    AbiOk(eps_hip_fill_u32(push_ws.Get<std::uint32_t>(), 0, need / 4, stream));
  }

  // Admits rows: allocates their slots (all or none), scatters their packed
  // state, indexes their keys.  `pack(i, dst)` writes row i's [w | m | v].
  // Rows stream through the transfer area in pieces; the residency is
  // committed only after every piece landed, so a failure leaves no trace.
  template <typename Pack>
  std::vector<LocatedRow> Admit(const MigrationPlan& plan, const std::vector<std::uint64_t>& updates, Pack pack) {
    std::map<TableId, std::vector<std::size_t>> by_table;
    for (std::size_t i = 0; i < plan.rows.size(); ++i) by_table[plan.rows[i].row.table].push_back(i);
    for (const auto& [id, members] : by_table) RebuildIndexIfWorn(Table(id));
    for (const auto& [id, members] : by_table) {
      const SlotTable& t = Table(id);
      Expect(plan.reserve_slots <= t.free_slots.size() && members.size() <= t.free_slots.size() - plan.reserve_slots,
             "HIP cache slots or slot reserve exhausted", Code::capacity_exceeded);
      const std::uint64_t per_row = 12ull * t.dim() + 16;
      Expect(transfer.capacity() >= 3 * 256 + per_row, "admitted row exceeds the transfer staging",
             Code::capacity_exceeded);
    }
    std::vector<LocatedRow> result(plan.rows.size());
    std::vector<std::pair<SlotTable*, std::uint64_t>> taken;
    for (const auto& [id, members] : by_table) {
      SlotTable& t = Table(id);
      for (std::size_t i : members) {
        const std::uint64_t slot = t.TakeSlot();
        taken.emplace_back(&t, slot);
        LocatedRow loc = plan.rows[i];
        loc.slot = slot;
        loc.agent = options.agent;
        loc.placement = Placement::gpu;
        result[i] = loc;
      }
    }
    // Keys indexed so far, per table (removed again if the admission fails).
    std::vector<std::pair<SlotTable*, std::vector<Key>>> indexed;
    try {
      ClearFlag();
      for (const auto& [id, members] : by_table) {
        SlotTable& t = Table(id);
        const std::uint64_t width = 3ull * t.dim();
        const std::uint64_t piece = (transfer.capacity() - 3 * 256) / (width * 4 + 16);
        indexed.emplace_back(&t, std::vector<Key>());
        for (std::size_t b = 0; b < members.size(); b += piece) {
          const std::size_t n = std::min<std::size_t>(piece, members.size() - b);
          Await();  // the previous piece's upload has left the host staging
          transfer.Reset();
          auto rows = transfer.Take<float>(n * width);
          auto slots = transfer.Take<std::uint64_t>(n);
          auto keys = transfer.Take<std::uint64_t>(n);
          for (std::size_t j = 0; j < n; ++j) {
            const std::size_t i = members[b + j];
            pack(i, rows.host + j * width);
            slots.host[j] = result[i].slot;
            keys.host[j] = result[i].row.key;
          }
          transfer.Upload(stream);
          AbiOk(eps_hip_scatter_rows(&t.abi, slots.device, rows.device, n, bounds.Get(), stream));
          indexed.back().second.insert(indexed.back().second.end(), keys.host, keys.host + n);
          AbiOk(eps_hip_index_insert(t.index.Get(), t.index_capacity, keys.device, slots.device, n, Flag(), stream));
        }
      }
      Expect(!(ReadFlag(Flag()) & EPS_HIP_STATUS_BAD_INDEX), "HIP key index is full", Code::run_failed);
    } catch (...) {
      // Nothing of the admission stays: its keys leave the index (those that
      // never made it in are simply not found) and its slots go back on top
      // of their stacks in the order they were taken.
      (void)hipStreamSynchronize(stream);
      for (auto& [t, keys] : indexed) {
        for (std::size_t b = 0; b < keys.size(); b += transfer.capacity() / 8) {
          const std::size_t n = std::min<std::size_t>(transfer.capacity() / 8, keys.size() - b);
          transfer.Reset();
          auto piece = transfer.Take<std::uint64_t>(n);
          std::memcpy(piece.host, keys.data() + b, n * 8);
          transfer.Upload(stream);
          (void)eps_hip_index_remove(t->index.Get(), t->index_capacity, piece.device, n, nullptr, stream);
          (void)hipStreamSynchronize(stream);
          t->removed_since_rebuild += n;
        }
      }
      for (auto it = taken.rbegin(); it != taken.rend(); ++it) it->first->free_slots.push_back(it->second);
      throw;
    }
    for (std::size_t i = 0; i < result.size(); ++i)
      Table(result[i].row.table).rows.emplace(result[i].row.key, Resident{result[i], updates[i]});
    return result;
  }

  // The checks every admission applies before anything moves (Load's, with
  // the row shapes checked by the caller): this agent, a GPU destination,
  // distinct rows not held here yet, tables defined.
  void CheckAdmission(const MigrationPlan& plan) {
    Expect(plan.agent == options.agent && plan.destination == Placement::gpu, "invalid HIP admission plan");
    std::set<std::pair<TableId, Key>> seen;
    for (const LocatedRow& loc : plan.rows) {
      const SlotTable& t = Table(loc.row.table);
      Expect(seen.emplace(loc.row.table, loc.row.key).second && !t.rows.count(loc.row.key),
             "admitted row is duplicated or already held here");
    }
  }

  HipCacheOptions options;
  hipStream_t stream = nullptr;
  Transfer transfer;
  Memory bounds, update_ws, push_ws, flags, flags_host;
  std::shared_ptr<OutputLedger> ledger;
  std::map<TableId, std::unique_ptr<SlotTable>> tables;
  std::uint64_t state_charged = 0;
  std::unique_ptr<hipbk::JobQueue> queue;
};

// ---------------------------------------------------------------------------
HipCacheBackend::HipCacheBackend(HipCacheOptions options) : impl_(std::make_unique<Impl>(options)) {}
HipCacheBackend::~HipCacheBackend() { impl_->queue->Close(); }

std::future<Result<Ack>> HipCacheBackend::Define(TableDefinition d) {
  return impl_->queue->Post<Ack>([this, d] {
    Impl& I = *impl_;
    I.Activate();
    // ValidateWeightBounds (src/common/optimizer_bounds.hpp:7-13).
    if (const auto& b = d.optimizer.weight_bounds)
      Expect(std::isfinite(b->minimum) && std::isfinite(b->maximum) && b->minimum <= b->maximum,
             "invalid optimizer weight bounds");
    Expect(d.dimension >= 1 && d.dimension <= 65536, "invalid HIP table dimension");
    if (auto it = I.tables.find(d.id); it != I.tables.end()) {
      Expect(it->second->definition == d, "HIP table is already defined differently");
      return Ack{};
    }
    // The state budget counts 12 bytes per element and 8 per row, as the
    // reference's (src/cuda/cache_backend.cu:372-374).
    const std::uint64_t rows = I.options.rows_per_table;
    const std::uint64_t charge = rows * (std::uint64_t(d.dimension) * 12 + 8);
    Expect(charge <= I.options.state_bytes - std::min(I.state_charged, I.options.state_bytes),
           "HIP table state budget exhausted", Code::capacity_exceeded);
    auto t = std::make_unique<SlotTable>();
    t->definition = d;
    t->state.Acquire(I.options.device, rows * d.dimension * 12ull, false);
    t->abi = eps_hip_table{t->state.Get<float>(), rows, d.dimension, d.id};
    t->index_capacity = 64;
    while (t->index_capacity < 2 * rows) t->index_capacity <<= 1;
    t->index.Acquire(I.options.device, eps_hip_index_bytes(t->index_capacity), false);
    AbiOk(eps_hip_index_clear(t->index.Get(), t->index_capacity, I.stream));
    t->free_slots.reserve(rows);
    for (std::uint64_t s = rows; s-- > 0;) t->free_slots.push_back(s);  // slot 0 first
    I.Await();
    I.tables.emplace(d.id, std::move(t));
    I.state_charged += charge;
    return Ack{};
  });
}

std::future<Result<std::uint64_t>> HipCacheBackend::FreeSlots(TableId id) {
  return impl_->queue->Post<std::uint64_t>([this, id] { return std::uint64_t(impl_->Table(id).free_slots.size()); });
}

std::future<Result<std::vector<LocatedRow>>> HipCacheBackend::Load(MigrationPlan plan, std::vector<RowState> states) {
  return impl_->queue->Post<std::vector<LocatedRow>>([this, plan = std::move(plan), states = std::move(states)] {
    Impl& I = *impl_;
    I.Activate();
    Expect(plan.rows.size() == states.size(), "invalid HIP admission plan");
    I.CheckAdmission(plan);
    std::vector<std::uint64_t> updates(states.size());
    for (std::size_t i = 0; i < states.size(); ++i) {
      const RowState& s = states[i];
      const std::uint32_t dim = I.Table(s.row.table).dim();
      Expect(s.row == plan.rows[i].row, "admitted state does not match its plan row");
      Expect(s.weights.size() == dim && s.first_moment.size() == dim && s.second_moment.size() == dim,
             "admitted state has the wrong shape");
      Expect(Finite(s.weights) && Finite(s.first_moment) && Finite(s.second_moment), "admitted state is not finite");
      Expect(std::all_of(s.second_moment.begin(), s.second_moment.end(), [](float v) { return v >= 0.f; }),
             "admitted second moment is negative");
      updates[i] = s.row_updates;
    }
    return I.Admit(plan, updates, [&](std::size_t i, float* dst) {
      const RowState& s = states[i];
      const std::size_t dim = s.weights.size();
      std::memcpy(dst, s.weights.data(), dim * 4);
      std::memcpy(dst + dim, s.first_moment.data(), dim * 4);
      std::memcpy(dst + 2 * dim, s.second_moment.data(), dim * 4);
    });
  });
}

std::future<Result<std::vector<TensorBlock>>> HipCacheBackend::GatherHost(std::vector<AgentWork> work,
                                                                          std::vector<FeatureInput> layouts) {
  return impl_->queue->Post<std::vector<TensorBlock>>([this, work = std::move(work), layouts = std::move(layouts)] {
    Impl& I = *impl_;
    I.Activate();
    auto parts = I.ResolveWork(work, layouts, true);
    std::vector<std::uint64_t> at;
    std::uint64_t floats = 0;
    for (const auto& r : parts) {
      at.push_back(floats);
      floats += r.rows * r.table->dim();
    }
    auto out = I.transfer.Take<float>(floats);
    I.transfer.Skip();
    I.Gather(parts, out.device, at);
    I.transfer.Download(out, I.stream);
    I.CheckResolution();
    std::vector<TensorBlock> blocks;
    blocks.reserve(parts.size());
    for (std::size_t i = 0; i < parts.size(); ++i) {
      const std::uint64_t dim = parts[i].table->dim(), n = parts[i].rows * dim;
      blocks.push_back({parts[i].layout->feature, {parts[i].rows, dim}, {out.host + at[i], out.host + at[i] + n}});
    }
    return blocks;
  });
}

std::future<Result<std::vector<DeviceTensorBlock>>> HipCacheBackend::GatherDevice(std::vector<AgentWork> work,
                                                                                  std::vector<FeatureInput> layouts) {
  return impl_->queue->Post<std::vector<DeviceTensorBlock>>([this, work = std::move(work),
                                                             layouts = std::move(layouts)] {
    Impl& I = *impl_;
    I.Activate();
    auto parts = I.ResolveWork(work, layouts, true);
    std::vector<std::uint64_t> at;
    std::uint64_t floats = 0;
    for (const auto& r : parts) {
      at.push_back(floats);
      floats += r.rows * r.table->dim();
    }
    auto block = std::make_shared<OutputBlock>(I.ledger, I.options.device, floats * 4);
    I.Gather(parts, block->data(), at);
    HipOk(hipEventRecord(block->ready(), I.stream), "output ready event");
    I.CheckResolution();  // also drains the staging's users
    std::vector<DeviceTensorBlock> out;
    out.reserve(parts.size());
    for (std::size_t i = 0; i < parts.size(); ++i) {
      const std::uint64_t dim = parts[i].table->dim();
      out.push_back({parts[i].layout->feature, {parts[i].rows, dim},
                     std::make_shared<OutputSlice>(block, at[i], parts[i].rows * dim)});
    }
    return out;
  });
}

std::future<Result<Ack>> HipCacheBackend::ApplyHost(UpdateContext context, RowGradients g) {
  return impl_->queue->Post<Ack>([this, context, g = std::move(g)] {
    Impl& I = *impl_;
    I.Activate();
    Impl::CheckContext(context);
    SlotTable& t = I.Table(context.table);
    auto rows = I.UpdateRows(context, t, g.rows);
    Expect(g.values.size() == rows.size() * std::uint64_t(t.dim()), "gradient values do not match the rows");
    if (rows.empty()) return Ack{};
    I.transfer.Reset();
    auto slots = I.transfer.Take<std::uint64_t>(rows.size());
    for (std::size_t i = 0; i < rows.size(); ++i) slots.host[i] = rows[i]->where.slot;
    auto values = I.transfer.Copy(g.values);
    I.transfer.Upload(I.stream);
    const eps_hip_optimizer o = I.Optimizer(t, context.learning_rate, context.beta1_power, context.beta2_power);
    AbiOk(eps_hip_adam_rows(&t.abi, &o, slots.device, values.device, rows.size(), I.update_ws.Get(),
                            I.bounds.Get(), I.stream));
    Impl::UpdateVerdict(I.ReadFlag(eps_hip_status_word(I.update_ws.Get())));
    for (Resident* r : rows) ++r->updates;
    return Ack{};
  });
}

std::future<Result<Ack>> HipCacheBackend::ApplyCompact(UpdateContext context, CompactGradients p) {
  return impl_->queue->Post<Ack>([this, context, p = std::move(p)] {
    Impl& I = *impl_;
    I.Activate();
    hipbk::CheckPacket(p);
    Impl::CheckContext(context);
    SlotTable& t = I.Table(context.table);
    auto rows = I.UpdateRows(context, t, p.rows);
    Expect(p.dimension == t.dim(), "compact packet dimension differs from the table's");
    if (rows.empty()) return Ack{};
    I.transfer.Reset();
    auto slots = I.transfer.Take<std::uint64_t>(rows.size());
    for (std::size_t i = 0; i < rows.size(); ++i) slots.host[i] = rows[i]->where.slot;
    auto offsets = I.transfer.Copy(p.row_offsets);
    auto sources = I.transfer.Copy(p.source_rows);
    auto scales = I.transfer.Copy(p.scales);
    auto values = I.transfer.Copy(p.source_values);
    I.transfer.Upload(I.stream);
    const eps_hip_optimizer o = I.Optimizer(t, context.learning_rate, context.beta1_power, context.beta2_power);
    AbiOk(eps_hip_adam_compact(&t.abi, &o, slots.device, rows.size(), offsets.device, sources.device, scales.device,
                               values.device, p.source_values.size() / p.dimension, p.source_rows.size(),
                               I.update_ws.Get(), I.bounds.Get(), I.stream));
    Impl::UpdateVerdict(I.ReadFlag(eps_hip_status_word(I.update_ws.Get())));
    for (Resident* r : rows) ++r->updates;
    return Ack{};
  });
}

std::future<Result<std::vector<RowState>>> HipCacheBackend::ReadBack(MigrationPlan plan) {
  return impl_->queue->Post<std::vector<RowState>>([this, plan = std::move(plan)] {
    Impl& I = *impl_;
    I.Activate();
    std::vector<const Resident*> held;
    std::map<TableId, std::vector<std::size_t>> by_table;
    for (std::size_t i = 0; i < plan.rows.size(); ++i) {
      held.push_back(&I.Locate(plan.rows[i]));
      by_table[plan.rows[i].row.table].push_back(i);
    }
    I.transfer.Reset();
    struct TableRun {
      SlotTable* t;
      Transfer::Piece<std::uint64_t> slots;
      const std::vector<std::size_t>* members;
    };
    std::vector<TableRun> runs;
    for (const auto& [id, members] : by_table) {
      TableRun run{&I.Table(id), I.transfer.Take<std::uint64_t>(members.size()), &members};
      for (std::size_t j = 0; j < members.size(); ++j) run.slots.host[j] = held[members[j]]->where.slot;
      runs.push_back(run);
    }
    I.transfer.Upload(I.stream);
    std::vector<Transfer::Piece<float>> packed;
    for (const TableRun& run : runs) packed.push_back(I.transfer.Take<float>(run.slots.count * 3ull * run.t->dim()));
    I.transfer.Skip();
    for (std::size_t k = 0; k < runs.size(); ++k) {
      AbiOk(eps_hip_gather_rows(&runs[k].t->abi, runs[k].slots.device, packed[k].device, runs[k].slots.count,
                                I.stream));
      I.transfer.Download(packed[k], I.stream);
    }
    I.Await();
    std::vector<RowState> out(plan.rows.size());
    for (std::size_t k = 0; k < runs.size(); ++k) {
      const std::size_t dim = runs[k].t->dim();
      for (std::size_t j = 0; j < runs[k].members->size(); ++j) {
        const std::size_t i = (*runs[k].members)[j];
        const float* src = packed[k].host + j * 3 * dim;
        out[i] = RowState{plan.rows[i].row, {src, src + dim}, {src + dim, src + 2 * dim}, {src + 2 * dim, src + 3 * dim},
                          held[i]->updates};
      }
    }
    return out;
  });
}

std::future<Result<Ack>> HipCacheBackend::CommitEviction(MigrationPlan plan) {
  return impl_->queue->Post<Ack>([this, plan = std::move(plan)] {
    Impl& I = *impl_;
    I.Activate();
    std::set<std::pair<TableId, Key>> seen;
    std::map<TableId, std::vector<Key>> by_table;
    for (const LocatedRow& loc : plan.rows) {
      I.Locate(loc);
      Expect(seen.emplace(loc.row.table, loc.row.key).second, "evicted row is named twice");
      by_table[loc.row.table].push_back(loc.row.key);
    }
    I.transfer.Reset();
    std::vector<std::pair<SlotTable*, Transfer::Piece<std::uint64_t>>> removals;
    for (const auto& [id, keys] : by_table) removals.emplace_back(&I.Table(id), I.transfer.Copy(keys));
    I.transfer.Upload(I.stream);
    I.ClearFlag();
    for (auto& [t, keys] : removals)
      AbiOk(eps_hip_index_remove(t->index.Get(), t->index_capacity, keys.device, keys.count, I.Flag(), I.stream));
    Expect(!(I.ReadFlag(I.Flag()) & EPS_HIP_STATUS_BAD_INDEX), "HIP key index lost a resident row", Code::run_failed);
    for (const LocatedRow& loc : plan.rows) {
      SlotTable& t = I.Table(loc.row.table);
      t.free_slots.push_back(loc.slot);
      t.rows.erase(loc.row.key);
    }
    for (auto& [t, keys] : removals) {
      t->removed_since_rebuild += keys.count;
      I.RebuildIndexIfWorn(*t);
    }
    return Ack{};
  });
}

std::future<Result<std::vector<DeviceTensorBlock>>> HipCacheBackend::AssembleFeatures(DeviceAssemblyRequest request) {
  return impl_->queue->Post<std::vector<DeviceTensorBlock>>([this, request = std::move(request)] {
    Impl& I = *impl_;
    I.Activate();
    const std::uint64_t cap = I.options.transfer_bytes;
    Expect(!request.host.empty() && request.host.size() == request.layouts.size(), "invalid device assembly");
    std::unordered_map<std::uint32_t, const SequenceProjection*> projection;
    for (const auto& p : request.projections)
      Expect(projection.emplace(p.feature, &p).second, "feature projected twice");
    // One output per feature: its rows before and after projection, its
    // offset in the shared allocation.
    struct Out {
      std::uint64_t at, rows, compact, dim;
      const SequenceProjection* projection;
    };
    std::vector<Out> outs;
    std::unordered_map<std::uint32_t, std::size_t> slot_of;
    const std::uint64_t align = I.options.output_alignment / 4;
    std::uint64_t floats = 0;
    for (std::size_t i = 0; i < request.host.size(); ++i) {
      const TensorBlock& h = request.host[i];
      const FeatureInput& L = request.layouts[i];
      Expect(h.feature == L.feature && h.shape.size() == 2 && h.shape[1] >= 1 && h.shape[1] <= UINT32_MAX &&
                 slot_of.emplace(h.feature, i).second,
             "device assembly host part does not match its layout");
      const std::uint64_t dim = h.shape[1];
      const std::uint64_t compact = L.pooling == Pooling::sequence ? L.keys.size() : L.valid_lengths.size();
      Expect(h.shape[0] == compact && compact <= cap / (4 * dim) && h.values.size() == compact * dim,
             "device assembly host part has the wrong shape");
      const SequenceProjection* p = nullptr;
      if (auto it = projection.find(h.feature); it != projection.end()) {
        p = it->second;
        bool ok = L.pooling == Pooling::sequence && p->positions.size() == compact;
        for (std::size_t j = 0; ok && j < p->positions.size(); ++j)
          ok = p->positions[j] < p->rows && (j == 0 || p->positions[j - 1] < p->positions[j]);
        Expect(ok, "invalid sequence projection");
      }
      const std::uint64_t rows = p ? p->rows : compact;
      Expect(rows <= cap / (4 * dim), "device assembly output exceeds the transfer limit", Code::capacity_exceeded);
      floats = RoundUp(floats, align);
      outs.push_back({floats, rows, compact, dim, p});
      floats += rows * dim;
    }
    for (const auto& [feature, p] : projection) Expect(slot_of.count(feature), "projection of an unknown feature");
    // Device contributions and where their rows land.
    struct Add {
      const DeviceTensor* tensor;
      std::size_t out;
      std::vector<std::uint64_t> positions;
    };
    std::vector<Add> adds;
    for (const DeviceContribution& c : request.device) {
      auto it = slot_of.find(c.block.feature);
      Expect(it != slot_of.end() && c.block.tensor, "device contribution of an unknown feature");
      const Out& o = outs[it->second];
      const DeviceTensorBlock& b = c.block;
      Expect(b.shape.size() == 2 && b.shape[1] == o.dim && b.shape[0] <= cap / (4 * o.dim) &&
                 b.tensor->elements() == b.shape[0] * o.dim && b.tensor->device() == I.options.device,
             "device contribution layout or device mismatch");
      Add a{b.tensor.get(), it->second, {}};
      if (c.projected) {
        bool ok = request.layouts[it->second].pooling == Pooling::sequence && c.positions.size() == b.shape[0];
        for (std::size_t j = 0; ok && j < c.positions.size(); ++j)
          ok = c.positions[j] < o.compact && (j == 0 || c.positions[j - 1] < c.positions[j]);
        Expect(ok, "invalid projected device contribution");
        for (std::uint64_t q : c.positions) a.positions.push_back(o.projection ? o.projection->positions[q] : q);
      } else {
        Expect(c.positions.empty() && b.shape[0] == o.compact, "device contribution row count mismatch");
        if (o.projection) a.positions = o.projection->positions;
      }
      adds.push_back(std::move(a));
    }
    auto block = std::make_shared<OutputBlock>(I.ledger, I.options.device, floats * 4);
    float* base = block->data();
    try {
      // Stage what the kernels read: projected host parts and their
      // positions, contribution positions, mean lengths.
      I.transfer.Reset();
      struct HostAdd {
        Transfer::Piece<float> values;
        Transfer::Piece<std::uint64_t> positions;
      };
      std::vector<std::optional<HostAdd>> host_adds(outs.size());
      std::vector<Transfer::Piece<std::uint64_t>> add_positions, lengths(outs.size());
      for (std::size_t i = 0; i < outs.size(); ++i)
        if (outs[i].projection && !request.host[i].values.empty())
          host_adds[i] = HostAdd{I.transfer.Copy(request.host[i].values), I.transfer.Copy(outs[i].projection->positions)};
      for (const Add& a : adds) add_positions.push_back(I.transfer.Copy(a.positions));
      for (std::size_t i = 0; i < outs.size(); ++i)
        if (request.layouts[i].pooling == Pooling::mean) lengths[i] = I.transfer.Copy(request.layouts[i].valid_lengths);
      I.transfer.Upload(I.stream);
      if (floats) AbiOk(eps_hip_fill_u32(reinterpret_cast<std::uint32_t*>(base), 0, floats, I.stream));
      // Host parts: a plain part is copied over the zeroed output, a
      // projected one is added at its positions (src/cuda/cache_backend.cu:664-676).
      for (std::size_t i = 0; i < outs.size(); ++i) {
        const auto& values = request.host[i].values;
        if (values.empty()) continue;
        float* dst = base + outs[i].at;
        if (host_adds[i])
          AbiOk(eps_hip_add_contribution(dst, host_adds[i]->values.device, host_adds[i]->positions.device,
                                         values.size(), std::uint32_t(outs[i].dim), I.stream));
        else
          HipOk(hipMemcpyAsync(dst, values.data(), values.size() * 4, hipMemcpyHostToDevice, I.stream), "host part");
      }
      // Device contributions, after their producers' work.
      for (std::size_t k = 0; k < adds.size(); ++k) {
        const Add& a = adds[k];
        const std::uint64_t n = a.tensor->elements();
        if (!n) continue;
        a.tensor->WaitOnStream(I.stream);
        AbiOk(eps_hip_add_contribution(base + outs[a.out].at, static_cast<const float*>(a.tensor->data()),
                                       a.positions.empty() ? nullptr : add_positions[k].device, n,
                                       std::uint32_t(outs[a.out].dim), I.stream));
      }
      // Means divide once by the original bag lengths.
      for (std::size_t i = 0; i < outs.size(); ++i)
        if (request.layouts[i].pooling == Pooling::mean && outs[i].rows)
          AbiOk(eps_hip_normalize_mean(base + outs[i].at, lengths[i].device, outs[i].rows, std::uint32_t(outs[i].dim),
                                       I.stream));
      HipOk(hipEventRecord(block->ready(), I.stream), "output ready event");
      I.Await();
    } catch (...) {
      (void)hipStreamSynchronize(I.stream);
      throw;
    }
    std::vector<DeviceTensorBlock> result;
    result.reserve(outs.size());
    for (std::size_t i = 0; i < outs.size(); ++i)
      result.push_back({request.host[i].feature, {outs[i].rows, outs[i].dim},
                        std::make_shared<OutputSlice>(block, outs[i].at, outs[i].rows * outs[i].dim)});
    return result;
  });
}

std::future<Result<Ack>> HipCacheBackend::PushDevice(std::vector<UpdateContext> contexts, std::vector<AgentWork> work,
                                                     std::vector<FeatureInput> layouts,
                                                     std::vector<DeviceTensorBlock> gradients) {
  return impl_->queue->Post<Ack>([this, contexts = std::move(contexts), work = std::move(work),
                                  layouts = std::move(layouts), gradients = std::move(gradients)] {
    Impl& I = *impl_;
    I.Activate();
    // One context per pushed table; one gradient block per pushed feature.
    std::map<TableId, const UpdateContext*> context_of;
    for (const auto& c : contexts) {
      Impl::CheckContext(c);
      Expect(context_of.emplace(c.table, &c).second, "two update contexts for one table");
    }
    std::unordered_map<std::uint32_t, const DeviceTensorBlock*> gradient_of;
    for (const auto& g : gradients) Expect(gradient_of.emplace(g.feature, &g).second, "two gradients for one feature");
    Expect(work.size() <= EPS_HIP_MAX_FEATURES, "too many features in one device push");
    auto parts = I.ResolveWork(work, layouts, false);
    // Call tables in first-use order; the push's per-table optimizers.
    std::vector<TableId> order;
    std::map<TableId, std::uint32_t> index_of;
    std::vector<eps_hip_table> tables;
    std::vector<eps_hip_optimizer> optimizers;
    std::vector<eps_hip_push_feature> features;
    std::uint64_t occurrences = 0;
    for (const auto& r : parts) {
      const FeatureInput& L = *r.layout;
      auto c = context_of.find(L.table);
      Expect(c != context_of.end(), "device push without a context for its table");
      auto g = gradient_of.find(L.feature);
      const std::uint64_t dim = r.table->dim();
      Expect(g != gradient_of.end() && g->second->tensor && g->second->shape.size() == 2 &&
                 g->second->shape[0] == r.rows && g->second->shape[1] == dim &&
                 g->second->tensor->elements() == r.rows * dim && g->second->tensor->device() == I.options.device,
             "device gradient does not match its feature");
      auto [it, fresh] = index_of.emplace(L.table, std::uint32_t(tables.size()));
      if (fresh) {
        order.push_back(L.table);
        tables.push_back(r.table->abi);
        optimizers.push_back(I.Optimizer(*r.table, c->second->learning_rate, c->second->beta1_power,
                                         c->second->beta2_power));
      }
      g->second->tensor->WaitOnStream(I.stream);
      eps_hip_push_feature f{};
      f.indices = r.occurrences ? r.slots : nullptr;
      f.offsets = r.offsets;
      f.valid_lengths = r.lengths;
      f.gradients = static_cast<const float*>(g->second->tensor->data());
      f.occurrences = r.occurrences;
      f.bags = L.pooling == Pooling::sequence ? 1 : r.rows;
      f.table = it->second;
      f.pooling = L.pooling == Pooling::sum ? EPS_HIP_POOL_SUM
                  : L.pooling == Pooling::mean ? EPS_HIP_POOL_MEAN
                                               : EPS_HIP_POOL_SEQUENCE;
      if (L.pooling == Pooling::sequence) {  // one bag holding every occurrence
        f.offsets = nullptr;
        f.valid_lengths = nullptr;
      }
      features.push_back(f);
      occurrences += r.occurrences;
    }
    Expect(tables.size() <= EPS_HIP_MAX_TABLES, "too many tables in one device push");
    // Every unique row the push updates, once per table.
    std::vector<Resident*> updated;
    {
      std::set<std::pair<TableId, Key>> seen;
      for (const auto& r : parts)
        for (const Resident* u : r.unique) {
          Expect(u->updates != UINT64_MAX && u->where.home == context_of.at(u->where.row.table)->shard,
                 "device push row is not this shard's");
          if (seen.emplace(u->where.row.table, u->where.row.key).second) updated.push_back(const_cast<Resident*>(u));
        }
    }
    I.CheckResolution();
    if (features.empty()) return Ack{};
    I.ReservePush(occurrences);
    void* ws = I.push_ws.Get();
    const std::uint64_t bytes = I.push_ws.bytes();
    AbiOk(eps_hip_prepare(tables.data(), std::uint32_t(tables.size()), features.data(), std::uint32_t(features.size()),
                          ws, bytes, I.stream));
    AbiOk(eps_hip_push(tables.data(), optimizers.data(), std::uint32_t(tables.size()), features.data(),
                       std::uint32_t(features.size()), ws, bytes, I.bounds.Get(), I.stream));
    const std::uint32_t status = I.ReadFlag(eps_hip_status_word(ws));
    if (status & (EPS_HIP_STATUS_STALLED | EPS_HIP_STATUS_BAD_INDEX)) I.stopped = true;
    Impl::UpdateVerdict(status);
    for (Resident* r : updated) ++r->updates;
    return Ack{};
  });
}

std::future<Result<SnapshotFile>> HipCacheBackend::WriteSnapshot(std::filesystem::path file, SnapshotIdentity identity,
                                                                 std::vector<SnapshotTable> tables,
                                                                 std::vector<RowState> host_rows) {
  return impl_->queue->Post<SnapshotFile>([this, file = std::move(file), identity = std::move(identity),
                                           tables = std::move(tables), host_rows = std::move(host_rows)] {
    Impl& I = *impl_;
    I.Activate();
    // The identity and schema checks the reference reader applies
    // (src/store/snapshot.cpp:201-206,230-245), so a written file restores.
    Expect(!identity.run.empty() && identity.run.size() <= 1024 && identity.shard_count > 0 &&
               identity.shard < identity.shard_count && identity.epoch > 0 && tables.size() <= 1024,
           "invalid snapshot identity");
    std::map<std::pair<TableId, Key>, const RowState*> host;
    for (const auto& r : host_rows)
      Expect(host.emplace(std::make_pair(r.row.table, r.row.key), &r).second, "a host row is given twice");
    std::set<TableId> ids;
    std::uint64_t device_rows = 0;
    for (const auto& t : tables) {
      const auto& d = t.definition;
      Expect(ids.insert(d.id).second && d.dimension > 0 && d.dimension <= 65536 &&
                 d.shard_count == identity.shard_count && d.partition_epoch == identity.epoch &&
                 t.beta1_power >= 0 && t.beta1_power < 1 && t.beta2_power >= 0 && t.beta2_power < 1,
             "invalid snapshot table");
      auto it = I.tables.find(d.id);
      Expect(it == I.tables.end() || it->second->definition == d, "snapshot table is defined differently here");
      std::unordered_set<Key> keys;
      for (Key key : t.keys) {
        Expect(keys.insert(key).second, "snapshot names a row twice");
        const bool resident = it != I.tables.end() && it->second->rows.count(key);
        auto h = host.find({d.id, key});
        Expect(resident != (h != host.end()), "a snapshot row must be held by exactly one store");
        if (resident) {
          ++device_rows;
        } else {
          const RowState& r = *h->second;
          Expect(r.weights.size() == d.dimension && r.first_moment.size() == d.dimension &&
                     r.second_moment.size() == d.dimension,
                 "snapshot host row has the wrong shape");
        }
      }
      Expect(it == I.tables.end() || I.options.transfer_bytes / 2 / 256 * 256 >= 256 + std::uint64_t(d.dimension) * 12 + 8,
             "snapshot row exceeds the transfer staging", Code::capacity_exceeded);
    }

    hipbk::SnapshotWriter out(file);
    hipbk::WriteSnapshotHeader(out, identity, tables.size());
    // Device rows come back in chunks through two halves of the transfer
    // area: the device fills one half while the host hashes the other.
    hipEvent_t ready[2] = {nullptr, nullptr};
    for (auto& e : ready) HipOk(hipEventCreateWithFlags(&e, hipEventDisableTiming), "snapshot event");
    struct EventGuard {
      hipEvent_t* e;
      ~EventGuard() {
        for (int i = 0; i < 2; ++i)
          if (e[i]) (void)hipEventDestroy(e[i]);
      }
    } guard{ready};
    I.transfer.Reset();
    const std::uint64_t half = I.transfer.capacity() / 2 / 256 * 256;
    auto halves = std::array<Transfer::Piece<unsigned char>, 2>{I.transfer.Take<unsigned char>(half),
                                                               I.transfer.Take<unsigned char>(half)};
    try {
      for (const auto& t : tables) {
        const auto& d = t.definition;
        hipbk::WriteSnapshotTable(out, t);
        auto it = I.tables.find(d.id);
        SlotTable* table = it == I.tables.end() ? nullptr : it->second.get();
        const std::uint64_t width = 3ull * d.dimension;
        // A chunk's slots (rounded up to 256 bytes) and rows fit in a half.
        const std::uint64_t per_chunk = table ? (half - 256) / (width * 4 + 8) : 0;
        auto resident = [&](Key key) -> const Resident* {
          if (!table) return nullptr;
          auto r = table->rows.find(key);
          return r == table->rows.end() ? nullptr : &r->second;
        };
        // Chunks: [begin, end) of the key list with at most per_chunk device rows.
        std::vector<std::pair<std::size_t, std::size_t>> chunks;
        for (std::size_t b = 0; b < t.keys.size();) {
          std::size_t e = b;
          for (std::uint64_t n = 0; e < t.keys.size(); ++e) {
            if (!resident(t.keys[e])) continue;
            if (n == per_chunk) break;
            ++n;
          }
          chunks.emplace_back(b, e);
          b = e;
        }
        auto issue = [&](std::size_t c) {
          const auto& h = halves[c % 2];
          auto* slots = reinterpret_cast<std::uint64_t*>(h.host);
          auto* dslots = reinterpret_cast<std::uint64_t*>(h.device);
          std::uint64_t n = 0;
          for (std::size_t i = chunks[c].first; i < chunks[c].second; ++i)
            if (const Resident* r = resident(t.keys[i])) slots[n++] = r->where.slot;
          if (n) {
            float* rows = reinterpret_cast<float*>(h.host + RoundUp(n * 8, 256));
            HipOk(hipMemcpyAsync(dslots, slots, n * 8, hipMemcpyHostToDevice, I.stream), "snapshot slots");
            AbiOk(eps_hip_gather_rows(&table->abi, dslots, rows, n, I.stream));
          }
          HipOk(hipEventRecord(ready[c % 2], I.stream), "snapshot event");
        };
        if (!chunks.empty()) issue(0);
        for (std::size_t c = 0; c < chunks.size(); ++c) {
          if (c + 1 < chunks.size()) issue(c + 1);
          HipOk(hipEventSynchronize(ready[c % 2]), "snapshot rows");
          const auto& h = halves[c % 2];
          std::uint64_t n = 0;
          for (std::size_t i = chunks[c].first; i < chunks[c].second; ++i)
            if (resident(t.keys[i])) ++n;
          const float* rows = reinterpret_cast<const float*>(h.host + RoundUp(n * 8, 256));
          std::uint64_t k = 0;
          for (std::size_t i = chunks[c].first; i < chunks[c].second; ++i) {
            const Key key = t.keys[i];
            if (const Resident* r = resident(key)) {
              hipbk::WriteSnapshotRow(out, key, r->updates, rows + k * width, d.dimension);
              ++k;
            } else {
              hipbk::WriteSnapshotRow(out, *host.at({d.id, key}));
            }
          }
        }
      }
    } catch (...) {
      (void)hipStreamSynchronize(I.stream);
      throw;
    }
    const std::uint64_t bytes = out.bytes() + 8;
    const std::uint64_t checksum = out.Publish();
    return SnapshotFile{bytes, checksum, device_rows};
  });
}

std::future<Result<std::vector<LocatedRow>>> HipCacheBackend::RestoreSnapshot(std::filesystem::path file,
                                                                              SnapshotIdentity identity,
                                                                              MigrationPlan plan) {
  return impl_->queue->Post<std::vector<LocatedRow>>([this, file = std::move(file), identity = std::move(identity),
                                                      plan = std::move(plan)] {
    Impl& I = *impl_;
    I.Activate();
    I.CheckAdmission(plan);
    std::map<std::pair<TableId, Key>, std::size_t> wanted;
    for (std::size_t i = 0; i < plan.rows.size(); ++i) wanted[{plan.rows[i].row.table, plan.rows[i].row.key}] = i;
    hipbk::SnapshotReader in(file);
    Expect(in.run == identity.run && in.shard == identity.shard && in.shard_count == identity.shard_count &&
               in.epoch == identity.epoch && in.shard_count >= 1 && in.shard < in.shard_count && in.epoch >= 1,
           "snapshot is not the named checkpoint");
    // Every wanted row's state, read in file order (the checksum is checked
    // before anything is admitted).
    std::vector<std::vector<float>> states(plan.rows.size());
    std::vector<std::uint64_t> updates(plan.rows.size());
    std::vector<bool> found(plan.rows.size(), false);
    std::set<TableId> tables_seen;
    std::vector<float> scratch;
    for (std::uint64_t k = 0; k < in.tables; ++k) {
      const auto t = in.NextTable();
      const TableId id = t.definition.id;
      Expect(tables_seen.insert(id).second, "snapshot defines a table twice");
      auto here = I.tables.find(id);
      const bool used = std::any_of(plan.rows.begin(), plan.rows.end(), [&](const LocatedRow& r) { return r.row.table == id; });
      if (used) Expect(here != I.tables.end() && here->second->definition == t.definition,
                       "snapshot table is defined differently here");
      scratch.resize(3ull * t.definition.dimension);
      for (std::uint64_t j = 0; j < t.rows; ++j) {
        Key key = 0;
        std::uint64_t counter = 0;
        in.Row(t.definition.dimension, key, counter, scratch.data());
        auto w = wanted.find({id, key});
        if (w == wanted.end()) continue;
        Expect(!found[w->second], "snapshot holds a row twice");
        found[w->second] = true;
        states[w->second] = scratch;
        updates[w->second] = counter;
      }
    }
    in.Finish();
    Expect(std::all_of(found.begin(), found.end(), [](bool f) { return f; }), "a planned row is not in the snapshot");
    return I.Admit(plan, updates, [&](std::size_t i, float* dst) {
      std::memcpy(dst, states[i].data(), states[i].size() * 4);
    });
  });
}

std::future<Result<HipMemoryStats>> HipCacheBackend::MemoryStats() {
  return impl_->queue->Post<HipMemoryStats>([this] {
    const Impl& I = *impl_;
    std::uint64_t state = 0, indexes = 0;
    for (const auto& [id, t] : I.tables) {
      state += I.options.rows_per_table * std::uint64_t(t->dim()) * 12;
      indexes += t->index.bytes();
    }
    const std::uint64_t staging = I.transfer.device_bytes() + I.update_ws.bytes() + I.push_ws.bytes() +
                                  I.bounds.bytes() + I.flags.bytes() + indexes;
    return HipMemoryStats{state, staging, I.ledger->used.load(), I.ledger->blocks.load(), I.index_rebuilds};
  });
}

}  // namespace eps
