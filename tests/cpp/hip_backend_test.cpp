// hip_backend_test.cpp -- eps::HipCacheBackend against the oracle, on a GPU.
//
// Re-expresses the scenarios of the reference's tests/cuda_tests.cpp (device
// backend vs the protocol reference backend): multi-table pooled gathers with
// holes, a sequence feature and an empty bag; the transfer_unique route;
// device results and their lifetime beyond the backend; seven ApplyHost and
// two ApplyCompact steps on a bounded table (clipping exercised); overflow
// rejection that leaves every row untouched; slot reclamation and stale
// generations after reuse; the atomic slot reserve of concurrent loads; plus
// device feature assembly (tests/device_pull_tests.cpp's ReferenceAssembly);
// the device-resident push (ReduceGradients + LazyAdam on the device); and the
// snapshot writeback from HBM, read back and rewritten by the oracle's
// restatement of src/store/snapshot.cpp, which must give the same bytes.
// Expected values come from the oracle (oracle/eps_oracle.h, the CPU
// restatement of the reference shard) and are compared bit for bit.
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <limits>
#include <map>
#include <set>
#include <stdexcept>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "eps/hip_cache_backend.hpp"
#include "eps_hip.h"
#include "eps_oracle.h"

using namespace eps;

namespace {

int g_checks = 0;

void Check(bool ok, const std::string& why) {
  ++g_checks;
  if (!ok) throw std::runtime_error(why);
}

template <typename T>
T Take(std::future<Result<T>> f) {
  auto r = f.get();
  if (auto e = std::get_if<Error>(&r)) throw std::runtime_error("backend error: " + e->message);
  return std::get<T>(std::move(r));
}

template <typename T>
Error::Code Fails(std::future<Result<T>> f, const std::string& what) {
  auto r = f.get();
  Check(std::holds_alternative<Error>(r), what + " was accepted");
  return std::get<Error>(r).code;
}

bool SameBits(const std::vector<float>& a, const std::vector<float>& b) {
  return a.size() == b.size() && (a.empty() || std::memcmp(a.data(), b.data(), a.size() * 4) == 0);
}

constexpr float kLr = 0.01f, kBeta1 = 0.9f, kBeta2 = 0.999f, kEps = 1e-8f;
constexpr float kMin = -0.015f, kMax = 0.015f;

TableDefinition Table(TableId id, std::uint32_t dim) {
  TableDefinition t{id, dim, 1, 1, {kLr, kBeta1, kBeta2, kEps, 0.9f, 0.999f}, -0.1f, 0.1f, 42};
  if (id == 1) t.optimizer.weight_bounds = WeightBounds{kMin, kMax};
  return t;
}

// Deterministic initial rows: table 1 keys 1..4 (dim 128), table 2 keys 1..2 (dim 64).
std::vector<RowState> States() {
  std::vector<RowState> rows;
  for (TableId table : {1u, 2u}) {
    const std::uint32_t dim = table == 1 ? 128 : 64;
    for (Key key = 1; key <= (table == 1 ? 4u : 2u); ++key) {
      RowState r{{table, key}, std::vector<float>(dim), std::vector<float>(dim), std::vector<float>(dim), 3};
      for (std::uint32_t d = 0; d < dim; ++d) {
        r.weights[d] = 0.04f * std::cos(float(key * 5 + d * 3 + table));
        r.first_moment[d] = 0.002f * float((d + key) % 7);
        r.second_moment[d] = 0.001f * float(1 + (d + 2 * key) % 4);
      }
      rows.push_back(std::move(r));
    }
  }
  return rows;
}

MigrationPlan Plan(const std::vector<RowState>& rows, const std::string& id = "load") {
  MigrationPlan p{id, 0, {}, Placement::gpu, 0};
  for (const auto& r : rows) p.rows.push_back({r.row, 0, Placement::loading, 0, 1, 0});
  return p;
}

// Mean with a hole (key 999 served elsewhere), a sequence, and a sum with an empty bag.
std::vector<FeatureInput> Layouts() {
  return {{1, 0, Pooling::mean, {2, 1, 999, 2, 4}, {0, 3, 5}, {3, 2}},
          {1, 1, Pooling::sequence, {3, 1, 3}, {0, 2, 3}, {2, 1}},
          {2, 2, Pooling::sum, {2, 1, 2}, {0, 3, 3}, {3, 0}}};
}

const LocatedRow& Locate(const std::vector<LocatedRow>& located, TableId table, Key key) {
  return *std::find_if(located.begin(), located.end(),
                       [&](const LocatedRow& l) { return l.row == RowKey{table, key}; });
}

std::vector<AgentWork> Work(const std::vector<LocatedRow>& l) {
  return {{0, AccessRoute::resident_gpu, 0, {Locate(l, 1, 2), Locate(l, 1, 1), Locate(l, 1, 4)},
           {0, 1, UINT64_MAX, 0, 2}, {}},
          {1, AccessRoute::resident_gpu, 0, {Locate(l, 1, 3), Locate(l, 1, 1)}, {0, 1, 0}, {}},
          {2, AccessRoute::resident_gpu, 0, {Locate(l, 2, 2), Locate(l, 2, 1)}, {0, 1, 0}, {}}};
}

// Host copy of the rows the backend holds, advanced with the oracle.
struct Model {
  std::map<std::pair<TableId, Key>, RowState> rows;
  const RowState& Get(TableId t, Key k) const { return rows.at({t, k}); }
};

// GatherHost of one work item: HostCacheBackend semantics via the oracle.
TensorBlock Expected(const Model& model, const AgentWork& task, const FeatureInput& f, std::uint32_t dim) {
  eps_or_feature of{f.keys.data(), f.keys.size(), f.offsets.data(), f.valid_lengths.data(), nullptr,
                    f.valid_lengths.size(), uint32_t(f.pooling), f.feature};
  std::vector<const float*> unique;
  for (const auto& loc : task.rows) unique.push_back(model.Get(loc.row.table, loc.row.key).weights.data());
  const std::uint64_t rows = f.pooling == Pooling::sequence ? f.keys.size() : f.offsets.size() - 1;
  TensorBlock out{f.feature, {rows, dim}, std::vector<float>(rows * dim)};
  Check(eps_or_gather_host(&of, dim, task.occurrence_to_unique.data(), task.rows.size(), unique.data(),
                           out.values.data()) == 0,
        "oracle gather failed");
  return out;
}

void CompareGather(const std::vector<TensorBlock>& got, const Model& model, const std::vector<AgentWork>& work,
                   const std::vector<FeatureInput>& layouts, const char* what) {
  Check(got.size() == work.size(), std::string(what) + ": block count");
  for (std::size_t i = 0; i < work.size(); ++i) {
    const auto& f = layouts[i];
    const std::uint32_t dim = f.table == 1 ? 128 : 64;
    const TensorBlock want = Expected(model, work[i], f, dim);
    Check(got[i].feature == want.feature && got[i].shape == want.shape, std::string(what) + ": layout");
    Check(SameBits(got[i].values, want.values), std::string(what) + ": values differ from the oracle");
  }
}

void CompareStates(const std::vector<RowState>& got, const Model& model, const char* what) {
  for (const auto& r : got) {
    const RowState& want = model.Get(r.row.table, r.row.key);
    Check(r.row_updates == want.row_updates, std::string(what) + ": update counter");
    Check(SameBits(r.weights, want.weights) && SameBits(r.first_moment, want.first_moment) &&
              SameBits(r.second_moment, want.second_moment),
          std::string(what) + ": state differs from the oracle");
  }
}

void ApplyModel(Model& model, TableId table, const std::vector<Key>& keys, const std::vector<float>& g,
                float b1p, float b2p) {
  const std::uint32_t dim = table == 1 ? 128 : 64;
  for (std::size_t i = 0; i < keys.size(); ++i) {
    auto& r = model.rows.at({table, keys[i]});
    Check(eps_or_adam_rows_ctx(r.weights.data(), r.first_moment.data(), r.second_moment.data(),
                               g.data() + i * dim, 1, dim, kBeta1, kBeta2, kEps, kLr, b1p, b2p,
                               table == 1, kMin, kMax) == 0,
          "oracle Adam rejected a valid update");
    ++r.row_updates;
  }
}

// A caller-owned device gradient (the training framework's tensor), written
// synchronously, so there is nothing to wait for.
class DeviceBuffer final : public DeviceTensor {
 public:
  explicit DeviceBuffer(const std::vector<float>& values) : count_(values.size()) {
    if (!count_) return;
    Check(hipMalloc(&pointer_, count_ * 4) == hipSuccess &&
              hipMemcpy(pointer_, values.data(), count_ * 4, hipMemcpyHostToDevice) == hipSuccess,
          "device gradient upload");
  }
  ~DeviceBuffer() override {
    if (pointer_) (void)hipFree(pointer_);
  }
  void* data() const override { return pointer_; }
  std::uint64_t elements() const override { return count_; }
  int device() const override { return 0; }
  void WaitOnStream(void*) const override {}
  std::vector<float> CopyToHost() const override {
    std::vector<float> values(count_);
    if (count_) Check(hipMemcpy(values.data(), pointer_, count_ * 4, hipMemcpyDeviceToHost) == hipSuccess, "download");
    return values;
  }

 private:
  void* pointer_ = nullptr;
  std::uint64_t count_;
};

// Per-feature gradients of the Layouts() lookup: (bags, or keys for the
// sequence feature) x dimension.
std::vector<std::vector<float>> PushGradients(const std::vector<FeatureInput>& layouts, int step) {
  std::vector<std::vector<float>> out;
  for (const auto& f : layouts) {
    const std::uint32_t dim = f.table == 1 ? 128 : 64;
    const std::uint64_t rows = f.pooling == Pooling::sequence ? f.keys.size() : f.valid_lengths.size();
    std::vector<float> g(rows * dim);
    for (std::size_t i = 0; i < g.size(); ++i)
      g[i] = 0.03f * std::sin(float(i * 7 + f.feature * 11 + step * 5)) - 0.004f * float(i % 3);
    out.push_back(std::move(g));
  }
  return out;
}

std::vector<DeviceTensorBlock> Upload(const std::vector<FeatureInput>& layouts,
                                      const std::vector<std::vector<float>>& g) {
  std::vector<DeviceTensorBlock> out;
  for (std::size_t i = 0; i < layouts.size(); ++i) {
    const std::uint64_t dim = layouts[i].table == 1 ? 128 : 64;
    out.push_back({layouts[i].feature, {g[i].size() / dim, dim}, std::make_shared<DeviceBuffer>(g[i])});
  }
  return out;
}

// The reference push of the same gradients: ReduceGradients per table over all
// of the lookup's features (the hole key 999 is reduced too and then routed
// elsewhere), LazyAdam on this agent's rows.
void ApplyPushModel(Model& model, const std::vector<FeatureInput>& layouts,
                    const std::vector<std::vector<float>>& g, const std::map<TableId, std::pair<float, float>>& powers) {
  for (const auto& [table, p] : powers) {
    const std::uint32_t dim = table == 1 ? 128 : 64;
    eps_or_table_def def{};
    def.id = table;
    def.dim = dim;
    def.shard_count = 1;
    eps_or_store* store = eps_or_create(&def);
    std::vector<eps_or_feature> features;
    std::vector<const float*> grads;
    std::uint64_t keys = 0;
    for (std::size_t i = 0; i < layouts.size(); ++i) {
      const auto& f = layouts[i];
      if (f.table != table) continue;
      features.push_back({f.keys.data(), f.keys.size(), f.offsets.data(), f.valid_lengths.data(), nullptr,
                          f.valid_lengths.size(), uint32_t(f.pooling), f.feature});
      grads.push_back(g[i].data());
      keys += f.keys.size();
    }
    std::vector<std::uint64_t> row_keys(keys);
    std::vector<float> values(keys * dim);
    std::uint64_t count = 0;
    const int rc = eps_or_reduce_gradients(store, features.data(), grads.data(), uint32_t(features.size()),
                                           row_keys.data(), values.data(), &count);
    eps_or_destroy(store);
    Check(rc == 0, "oracle gradient reduction failed");
    std::vector<Key> mine;
    std::vector<float> mine_values;
    for (std::uint64_t u = 0; u < count; ++u) {
      if (!model.rows.count({table, row_keys[u]})) continue;  // served by another owner
      mine.push_back(row_keys[u]);
      mine_values.insert(mine_values.end(), values.begin() + u * dim, values.begin() + (u + 1) * dim);
    }
    ApplyModel(model, table, mine, mine_values, p.first, p.second);
  }
}

HipCacheOptions SmallOptions(std::uint64_t rows_per_table) {
  HipCacheOptions o;
  o.rows_per_table = rows_per_table;
  o.state_bytes = 1 << 20;
  o.transfer_bytes = 1 << 20;
  o.outstanding_output_bytes = 1 << 20;
  return o;
}

// Two loads racing for a slot reserve: the second is refused whole.
void AtomicReserve() {
  HipCacheOptions o = SmallOptions(3);
  o.state_bytes = 96;  // exactly one dim-2 table of 3 rows
  HipCacheBackend gpu(o);
  Take(gpu.Define(Table(99, 2)));
  auto load = [&](Key first, std::size_t count) {
    std::vector<RowState> states;
    for (std::size_t n = 0; n < count; ++n) states.push_back({{99, first + n}, {0.1f, 0.2f}, {0, 0}, {0, 0}, 0});
    auto plan = Plan(states);
    plan.reserve_slots = 1;
    return gpu.Load(std::move(plan), std::move(states));
  };
  auto first = load(1, 2), second = load(3, 1);
  Take(std::move(first));
  Check(Fails(std::move(second), "load into the reserve") == Error::Code::capacity_exceeded,
        "reserve refusal code");
  Check(Take(gpu.FreeSlots(99)) == 1, "concurrent load consumed the slot reserve");
  Check(Fails(gpu.Define(Table(100, 2)), "define beyond the state budget") == Error::Code::capacity_exceeded,
        "state budget code");
}

void Assembly(HipCacheBackend& gpu, const std::vector<LocatedRow>& located, const Model& model) {
  // Device part of a mean feature and of a projected sequence feature, plus
  // host partial sums; the mean divides once by the original lengths.
  const std::vector<FeatureInput> layouts = {
      {2, 7, Pooling::mean, {1, 2, 2}, {0, 2, 3}, {4, 1}},
      {2, 8, Pooling::sequence, {2, 1}, {0, 2}, {2}}};
  std::vector<AgentWork> work = {
      {7, AccessRoute::resident_gpu, 0, {Locate(located, 2, 1), Locate(located, 2, 2)}, {0, 1, 1}, {}},
      {8, AccessRoute::resident_gpu, 0, {Locate(located, 2, 2), Locate(located, 2, 1)}, {0, 1}, {}}};
  auto device = Take(gpu.GatherDevice(work, layouts));
  std::vector<TensorBlock> host = {{7, {2, 64}, std::vector<float>(2 * 64)}, {8, {2, 64}, std::vector<float>(2 * 64)}};
  for (std::size_t i = 0; i < host[0].values.size(); ++i) host[0].values[i] = 0.001f * float(i % 13);
  for (std::size_t i = 0; i < host[1].values.size(); ++i) host[1].values[i] = -0.002f * float(i % 5);
  DeviceAssemblyRequest request;
  request.host = host;
  request.layouts = layouts;
  request.device = {{device[0], {}, false}, {device[1], {}, false}};
  request.projections = {{8, 5, {1, 3}}};  // sequence rows land at positions 1 and 3 of 5
  auto assembled = Take(gpu.AssembleFeatures(request));
  Check(assembled.size() == 2 && assembled[1].shape == std::vector<std::uint64_t>{5, 64}, "assembly layout");
  // Expected (src/cuda/cache_backend.cu:664-692): a non-projected host part is
  // copied over the zeroed output, a projected one is added to it; device
  // parts are added after; the mean divides last.
  std::vector<float> mean(2 * 64, 0.f), seq(5 * 64, 0.f);
  const TensorBlock dm = Expected(model, work[0], layouts[0], 64), ds = Expected(model, work[1], layouts[1], 64);
  for (std::size_t i = 0; i < mean.size(); ++i) {
    float v = host[0].values[i];
    v = v + dm.values[i];
    const std::uint64_t len = layouts[0].valid_lengths[i / 64];
    mean[i] = len ? v / float(len) : v;
  }
  for (std::size_t r = 0; r < 2; ++r) {
    const std::uint64_t at = request.projections[0].positions[r];
    for (std::size_t d = 0; d < 64; ++d) {
      float v = 0.f;
      v = v + host[1].values[r * 64 + d];
      v = v + ds.values[r * 64 + d];
      seq[at * 64 + d] = v;
    }
  }
  assembled[0].tensor->WaitOnStream(nullptr);
  Check(SameBits(assembled[0].tensor->CopyToHost(), mean), "assembled mean feature");
  Check(SameBits(assembled[1].tensor->CopyToHost(), seq), "assembled projected sequence feature");
}

// Device-resident push: two steps over both tables (mean with a hole, a
// sequence, a sum with an empty bag) against the oracle's ReduceGradients +
// LazyAdam, then rejections that leave every row as it was.
void DevicePush(HipCacheBackend& gpu, const std::vector<LocatedRow>& located, Model& model,
                float& b1, float& b2) {
  const auto layouts = Layouts();
  const auto work = Work(located);
  float t2b1 = 0.9f, t2b2 = 0.999f;
  for (int step = 0; step < 2; ++step) {
    const auto g = PushGradients(layouts, step);
    std::vector<UpdateContext> contexts = {{{"hip-push", 0, std::uint64_t(step), Phase::push}, 0, 1, 0, kLr, b1, b2},
                                           {{"hip-push", 0, std::uint64_t(step), Phase::push}, 0, 2, 0, kLr, t2b1, t2b2}};
    Take(gpu.PushDevice(contexts, work, layouts, Upload(layouts, g)));
    ApplyPushModel(model, layouts, g, {{1, {b1, b2}}, {2, {t2b1, t2b2}}});
    b1 *= 0.9f;
    b2 *= 0.999f;
    t2b1 *= 0.9f;
    t2b2 *= 0.999f;
    CompareStates(Take(gpu.ReadBack({"read", 0, located, Placement::cpu, 0})), model, "state after device push");
  }
  const std::vector<UpdateContext> contexts = {{{"hip-push", 0, 9, Phase::push}, 0, 1, 0, kLr, b1, b2},
                                               {{"hip-push", 0, 9, Phase::push}, 0, 2, 0, kLr, t2b1, t2b2}};
  auto g = PushGradients(layouts, 3);
  g[2][64 + 5] = std::numeric_limits<float>::quiet_NaN();  // the empty bag's gradient row
  Check(Fails(gpu.PushDevice(contexts, work, layouts, Upload(layouts, g)), "non-finite device gradient") ==
            Error::Code::invalid_argument,
        "non-finite gradient code");
  g = PushGradients(layouts, 3);
  std::fill(g[1].begin(), g[1].end(), std::numeric_limits<float>::max());
  Fails(gpu.PushDevice(contexts, work, layouts, Upload(layouts, g)), "overflowing device push");
  g = PushGradients(layouts, 3);
  auto short_blocks = Upload(layouts, g);
  short_blocks[1].shape[0] = 2;
  Check(Fails(gpu.PushDevice(contexts, work, layouts, short_blocks), "mis-shaped device gradient") ==
            Error::Code::invalid_argument,
        "gradient shape code");
  Fails(gpu.PushDevice({contexts[0]}, work, layouts, Upload(layouts, g)), "push without a table context");
  auto twice = work;
  twice[1] = work[0];  // feature 0 twice, feature 1's gradient unused
  Fails(gpu.PushDevice(contexts, twice, layouts, Upload(layouts, g)), "a feature pushed twice");
  auto stale = work;
  stale[2].rows[0].generation += 1;
  Check(Fails(gpu.PushDevice(contexts, stale, layouts, Upload(layouts, g)), "stale device push") ==
            Error::Code::stale_generation,
        "stale push code");
  CompareStates(Take(gpu.ReadBack({"read", 0, located, Placement::cpu, 0})), model,
                "state after rejected device pushes");
}

// Device push at scale: three tables of 60,000 rows (dims 64, 64 bounded,
// 128), four features (two on one table; mean and sum) of 2,048 bags of 1..20
// skewed ids, so the hottest rows take thousands of references (the
// hot-row kernel) and the rest the row-run kernel; ids past the loaded rows
// are served elsewhere (holes).  Every touched row must match the oracle's
// ReduceGradients + LazyAdam bit for bit, and an untouched row stays as it was.
RowState MakeRow(TableId table, Key key, std::uint32_t dim);

void DevicePushAtScale() {
  HipCacheOptions o = SmallOptions(60000);
  o.state_bytes = 256ull << 20;
  o.transfer_bytes = 64ull << 20;  // a table's touched rows read back in one call
  HipCacheBackend gpu(o);
  std::vector<TableDefinition> defs = {Table(11, 64), Table(12, 64), Table(13, 128)};
  defs[1].optimizer.weight_bounds = WeightBounds{-0.03f, 0.03f};
  constexpr Key kLoaded = 59000, kIds = 60000;
  std::map<std::pair<TableId, Key>, RowState> model;
  std::map<std::pair<TableId, Key>, LocatedRow> where;
  for (const auto& d : defs) {
    Take(gpu.Define(d));
    for (Key b = 0; b < kLoaded; b += 10000) {
      std::vector<RowState> part;
      for (Key k = b; k < std::min(kLoaded, b + 10000); ++k) {
        RowState r = MakeRow(d.id, k, d.dimension);
        model[{d.id, k}] = r;
        part.push_back(r);
      }
      for (const auto& loc : Take(gpu.Load(Plan(part), part))) where[{loc.row.table, loc.row.key}] = loc;
    }
  }
  std::uint64_t state = 12345;
  auto next = [&]() {  // SplitMix64 stream
    state += 0x9e3779b97f4a7c15ull;
    std::uint64_t z = state;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  };
  struct Spec { TableId table; std::uint32_t feature; Pooling pooling; };
  const std::vector<Spec> specs = {{11, 0, Pooling::mean}, {11, 1, Pooling::sum}, {12, 2, Pooling::sum},
                                   {13, 3, Pooling::mean}};
  std::vector<FeatureInput> layouts;
  std::vector<AgentWork> work;
  std::vector<std::vector<float>> grads;
  for (const auto& sp : specs) {
    FeatureInput f{sp.table, sp.feature, sp.pooling, {}, {0}, {}};
    for (int b = 0; b < 2048; ++b) {
      const std::uint64_t len = 1 + next() % 20;
      for (std::uint64_t i = 0; i < len; ++i) {
        const double u = double(next() >> 11) * 0x1.0p-53;
        f.keys.push_back(Key(double(kIds) * u * u * u * u));  // skewed: key 0 is the hottest
      }
      f.offsets.push_back(f.keys.size());
      f.valid_lengths.push_back(len + (b % 7 == 0 ? 2 : 0));  // some bags lost positions elsewhere
    }
    AgentWork w{sp.feature, AccessRoute::resident_gpu, 0, {}, std::vector<std::uint64_t>(f.keys.size()), {}};
    std::map<Key, std::uint64_t> unique;
    for (std::size_t i = 0; i < f.keys.size(); ++i) {
      if (f.keys[i] >= kLoaded) { w.occurrence_to_unique[i] = UINT64_MAX; continue; }
      auto [it, fresh] = unique.emplace(f.keys[i], w.rows.size());
      if (fresh) w.rows.push_back(where.at({sp.table, f.keys[i]}));
      w.occurrence_to_unique[i] = it->second;
    }
    const std::uint32_t dim = sp.table == 13 ? 128 : 64;
    std::vector<float> g(f.valid_lengths.size() * dim);
    for (auto& x : g) x = float(std::int64_t(next() % 2001) - 1000) * 1e-4f;
    layouts.push_back(std::move(f));
    work.push_back(std::move(w));
    grads.push_back(std::move(g));
  }
  std::vector<UpdateContext> contexts;
  std::map<TableId, std::pair<float, float>> powers;
  for (const auto& d : defs) {
    contexts.push_back({{"scale", 0, 1, Phase::push}, 0, d.id, 1, kLr, 0.81f, 0.998f});
    powers[d.id] = {0.81f, 0.998f};
  }
  std::vector<DeviceTensorBlock> blocks;
  for (std::size_t i = 0; i < layouts.size(); ++i) {
    const std::uint64_t dim = layouts[i].table == 13 ? 128 : 64;
    blocks.push_back({layouts[i].feature, {grads[i].size() / dim, dim}, std::make_shared<DeviceBuffer>(grads[i])});
  }
  Take(gpu.PushDevice(contexts, work, layouts, blocks));
  // Expected: the reference's per-table reduce over every feature of the table, then Adam.
  std::size_t touched = 0;
  for (const auto& d : defs) {
    eps_or_table_def def{};
    def.id = d.id; def.dim = d.dimension; def.shard_count = 1;
    eps_or_store* store = eps_or_create(&def);
    std::vector<eps_or_feature> fs;
    std::vector<const float*> gs;
    std::uint64_t keys = 0;
    for (std::size_t i = 0; i < layouts.size(); ++i) {
      if (layouts[i].table != d.id) continue;
      const auto& f = layouts[i];
      fs.push_back({f.keys.data(), f.keys.size(), f.offsets.data(), f.valid_lengths.data(), nullptr,
                    f.valid_lengths.size(), uint32_t(f.pooling), f.feature});
      gs.push_back(grads[i].data());
      keys += f.keys.size();
    }
    std::vector<std::uint64_t> row_keys(keys);
    std::vector<float> values(keys * d.dimension);
    std::uint64_t count = 0;
    Check(eps_or_reduce_gradients(store, fs.data(), gs.data(), uint32_t(fs.size()), row_keys.data(),
                                  values.data(), &count) == 0,
          "oracle reduce at scale");
    eps_or_destroy(store);
    MigrationPlan read{"read", 0, {}, Placement::cpu, 0};
    std::vector<std::uint64_t> mine;
    for (std::uint64_t u = 0; u < count; ++u) {
      if (row_keys[u] >= kLoaded) continue;
      RowState& r = model.at({d.id, row_keys[u]});
      Check(eps_or_adam_rows_ctx(r.weights.data(), r.first_moment.data(), r.second_moment.data(),
                                 values.data() + u * d.dimension, 1, d.dimension, kBeta1, kBeta2, kEps, kLr,
                                 powers[d.id].first, powers[d.id].second, d.optimizer.weight_bounds ? 1 : 0,
                                 -0.03f, 0.03f) == 0,
            "oracle Adam at scale");
      ++r.row_updates;
      read.rows.push_back(where.at({d.id, row_keys[u]}));
    }
    read.rows.push_back(where.at({d.id, kLoaded - 1}));  // untouched (ids near the end are rare)
    for (const auto& got : Take(gpu.ReadBack(read))) {
      const RowState& want = model.at({got.row.table, got.row.key});
      Check(SameBits(got.weights, want.weights) && SameBits(got.first_moment, want.first_moment) &&
                SameBits(got.second_moment, want.second_moment) && got.row_updates == want.row_updates,
            "device push at scale differs from the oracle (table " + std::to_string(d.id) + ", key " +
                std::to_string(got.row.key) + ")");
      ++touched;
    }
  }
  Check(touched > 10000, "device push at scale touched too few rows");
}

std::string FileBytes(const std::filesystem::path& p) {
  std::ifstream in(p, std::ios::binary);
  return {std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>()};
}

RowState MakeRow(TableId table, Key key, std::uint32_t dim) {
  RowState r{{table, key}, std::vector<float>(dim), std::vector<float>(dim), std::vector<float>(dim),
             key % 13};
  for (std::uint32_t d = 0; d < dim; ++d) {
    r.weights[d] = 0.01f * std::sin(float(key * 7 + d));
    r.first_moment[d] = 1e-4f * std::cos(float(key + 3 * d));
    r.second_moment[d] = 1e-6f * float(1 + (key + d) % 5);
  }
  return r;
}

// Snapshot writeback: 2,000 device rows of a bounded table interleaved with
// CPU-store rows in the file's key order (several staging chunks), a table the
// backend defines but holds no rows of, and a table only the CPU store holds.
void SnapshotWriteback() {
  const auto dir = std::filesystem::temp_directory_path() / ("eps-snapshot-" + std::to_string(::getpid()));
  std::filesystem::remove_all(dir);
  HipCacheOptions o = SmallOptions(4096);
  o.transfer_bytes = 64 << 10;  // 170 rows of dim 16 per staging half
  o.state_bytes = 64 << 20;
  HipCacheBackend gpu(o);
  TableDefinition big{5, 16, 1, 1, {0.01f, 0.9f, 0.999f, 1e-8f, 0.9f, 0.999f}, -0.1f, 0.1f, 77};
  big.optimizer.weight_bounds = WeightBounds{-0.5f, 0.5f};
  const TableDefinition empty = Table(2, 64), host_only = Table(9, 8);
  Take(gpu.Define(big));
  Take(gpu.Define(empty));
  std::map<std::pair<TableId, Key>, RowState> expect;
  std::vector<RowState> host_rows;
  std::vector<Key> order;
  for (Key k = 0; k < 3000; ++k) order.push_back((k * 1777) % 3001 + 1);  // a permutation of 1..3001 minus one
  std::vector<RowState> device;
  for (Key key : order) {
    RowState r = MakeRow(5, key, 16);
    expect[{5, key}] = r;
    (key % 3 == 0 ? host_rows : device).push_back(r);
  }
  std::map<Key, LocatedRow> where;  // table 5 rows as the backend placed them
  for (std::size_t b = 0; b < device.size(); b += 300) {
    std::vector<RowState> part(device.begin() + b, device.begin() + std::min(device.size(), b + 300));
    for (const auto& loc : Take(gpu.Load(Plan(part), part))) where[loc.row.key] = loc;
  }
  std::vector<Key> keys2 = {40, 8, 16}, keys9 = {3, 1, 2};
  for (Key key : keys2) host_rows.push_back(expect[{2, key}] = MakeRow(2, key, 64));
  for (Key key : keys9) host_rows.push_back(expect[{9, key}] = MakeRow(9, key, 8));
  std::vector<SnapshotTable> tables = {{big, 12, 0.2f, 0.3f, order}, {empty, 0, 0.9f, 0.999f, keys2},
                                       {host_only, 5, 0.5f, 0.6f, keys9}};
  const SnapshotIdentity id{"run-hip", 0, 1, 1};
  const auto file = dir / "step" / "shard-0.bin";
  const SnapshotFile written = Take(gpu.WriteSnapshot(file, id, tables, host_rows));
  Check(written.device_rows == device.size() && written.bytes == std::filesystem::file_size(file) &&
            !std::filesystem::exists(file.string() + ".pending"),
        "snapshot file summary");

  // The oracle reads it back (checksum, identity, schema, every row) ...
  char run[1025];
  std::uint64_t shard = 0, count = 0, epoch = 0, checksum = 0;
  std::uint32_t version = 0, ntables = 0;
  eps_or_store* stores[8] = {};
  Check(eps_or_snapshot_read(file.c_str(), run, sizeof run, &shard, &count, &epoch, &version, stores, 8,
                             &ntables, &checksum) == 0,
        std::string("oracle rejected the snapshot: ") + eps_or_last_error());
  Check(std::string(run) == id.run && shard == 0 && count == 1 && epoch == 1 && version == 2 &&
            ntables == 3 && checksum == written.checksum,
        "snapshot identity");
  for (std::uint32_t t = 0; t < ntables; ++t) {
    const auto& want = tables[t];
    float b1 = 0, b2 = 0;
    std::uint64_t seq = 0;
    eps_or_powers(stores[t], &b1, &b2, &seq);
    Check(b1 == want.beta1_power && b2 == want.beta2_power && seq == want.optimizer_sequence &&
              eps_or_row_count(stores[t]) == want.keys.size(),
          "snapshot table clock");
    const std::uint32_t dim = want.definition.dimension;
    for (std::size_t i = 0; i < want.keys.size(); ++i) {
      const Key key = want.keys[i];
      Check(eps_or_key_at(stores[t], i) == key, "snapshot row order");
      std::vector<float> w(dim), m(dim), v(dim);
      std::uint64_t updates = 0;
      Check(eps_or_read(stores[t], key, w.data(), m.data(), v.data(), &updates) == 0, "snapshot row missing");
      const RowState& r = expect.at({want.definition.id, key});
      Check(SameBits(w, r.weights) && SameBits(m, r.first_moment) && SameBits(v, r.second_moment) &&
                updates == r.row_updates,
            "snapshot row differs");
    }
  }
  // ... and its own writer, given the same content, produces the same bytes.
  const auto again = dir / "oracle.bin";
  Check(eps_or_snapshot_write(again.c_str(), run, shard, count, epoch, stores, ntables) == 0, "oracle writer");
  Check(FileBytes(again) == FileBytes(file), "snapshot bytes differ from the oracle writer's");

  // Restore and resume (tests/core_tests.cpp:107-129): a fresh backend
  // restores every row of the file straight into HBM (RestoreSnapshot) and
  // takes the same update as the original; both end bit-identical, counters
  // included.  Refused restores (another checkpoint, a row the file lacks, a
  // damaged copy) admit nothing.
  {
    HipCacheBackend restored(o);
    Take(restored.Define(big));
    MigrationPlan plan{"restore", 0, {}, Placement::gpu, 0};
    for (Key key : order) plan.rows.push_back({{5, key}, 0, Placement::loading, 0, 1, 0});
    Check(Fails(restored.RestoreSnapshot(file, {"other-run", 0, 1, 1}, plan), "restore of another checkpoint") ==
              Error::Code::invalid_argument,
          "wrong checkpoint code");
    auto too_many = plan;
    too_many.rows.push_back({{5, 5000}, 0, Placement::loading, 0, 1, 0});
    Fails(restored.RestoreSnapshot(file, id, too_many), "restore of a row the file lacks");
    const auto damaged = dir / "damaged.bin";
    {
      std::string bytes = FileBytes(file);
      bytes[bytes.size() / 3] ^= 0x01;
      std::ofstream(damaged, std::ios::binary) << bytes;
    }
    Fails(restored.RestoreSnapshot(damaged, id, plan), "restore of a damaged file");
    Check(Take(restored.FreeSlots(5)) == 4096, "a refused restore admitted rows");
    std::map<Key, LocatedRow> where_restored;
    for (const auto& loc : Take(restored.RestoreSnapshot(file, id, plan))) where_restored[loc.row.key] = loc;
    Check(where_restored.size() == order.size() && Take(restored.FreeSlots(5)) == 4096 - order.size(),
          "restored rows");
    for (std::size_t b = 0; b < order.size(); b += 300) {  // ReadBack is bounded by the staging
      MigrationPlan some{"read", 0, {}, Placement::cpu, 0};
      for (std::size_t i = b; i < std::min(order.size(), b + 300); ++i) some.rows.push_back(where_restored.at(order[i]));
      for (const auto& r : Take(restored.ReadBack(some))) {
        const RowState& want = expect.at({5, r.row.key});
        Check(SameBits(r.weights, want.weights) && SameBits(r.first_moment, want.first_moment) &&
                  SameBits(r.second_moment, want.second_moment) && r.row_updates == want.row_updates,
              "restored row differs from the snapshot");
      }
    }
    RowGradients g;
    MigrationPlan before{"read", 0, {}, Placement::cpu, 0}, after = before;
    for (std::size_t i = 0; i < device.size(); i += 97) {
      g.rows.push_back(device[i].row);
      for (int d = 0; d < 16; ++d) g.values.push_back(0.3f * std::cos(float(i + d)));
      before.rows.push_back(where.at(device[i].row.key));
      after.rows.push_back(where_restored.at(device[i].row.key));
    }
    const UpdateContext c{{"resume", 0, 12, Phase::push}, 0, 5, 12, 0.01f, 0.2f, 0.3f};
    Take(gpu.ApplyHost(c, g));
    Take(restored.ApplyHost(c, g));
    const auto a = Take(gpu.ReadBack(before)), b = Take(restored.ReadBack(after));
    for (std::size_t i = 0; i < a.size(); ++i)
      Check(a[i].row == b[i].row && SameBits(a[i].weights, b[i].weights) &&
                SameBits(a[i].first_moment, b[i].first_moment) &&
                SameBits(a[i].second_moment, b[i].second_moment) && a[i].row_updates == b[i].row_updates &&
                a[i].row_updates == expect.at({5, a[i].row.key}).row_updates + 1,
            "resumed training diverged from the original");
  }
  for (std::uint32_t t = 0; t < ntables; ++t) eps_or_destroy(stores[t]);

  // Published files are immutable; bad requests are refused before any I/O.
  const std::string before = FileBytes(file);
  Check(Fails(gpu.WriteSnapshot(file, id, tables, host_rows), "overwrite") == Error::Code::unavailable,
        "snapshot overwrite code");
  Check(FileBytes(file) == before && !std::filesystem::exists(file.string() + ".pending"),
        "refused overwrite changed the snapshot");
  auto dup = tables;
  dup[2].keys.push_back(3);
  Check(Fails(gpu.WriteSnapshot(dir / "dup.bin", id, dup, host_rows), "duplicate key") ==
            Error::Code::invalid_argument,
        "duplicate key code");
  auto twice = host_rows;
  twice.push_back(MakeRow(5, order[0] % 3 == 0 ? order[1] : order[0], 16));
  Fails(gpu.WriteSnapshot(dir / "twice.bin", id, tables, twice), "row held twice");
  auto missing = tables;
  missing[1].keys.push_back(77);
  Fails(gpu.WriteSnapshot(dir / "missing.bin", id, missing, host_rows), "missing row");
  Fails(gpu.WriteSnapshot(dir / "bad.bin", {"run-hip", 1, 1, 1}, tables, host_rows), "shard out of range");
  for (const char* name : {"dup.bin", "twice.bin", "missing.bin", "bad.bin"})
    Check(!std::filesystem::exists(dir / name), "refused snapshot left a file");
  std::filesystem::remove_all(dir);
}

eps_or_table_def OracleDef(const TableDefinition& d) {
  eps_or_table_def def{};
  def.id = d.id;
  def.dim = d.dimension;
  def.shard = 0;
  def.shard_count = 1;
  def.learning_rate = d.optimizer.learning_rate;
  def.beta1 = d.optimizer.beta1;
  def.beta2 = d.optimizer.beta2;
  def.epsilon = d.optimizer.epsilon;
  def.initial_beta1_power = d.optimizer.initial_beta1_power;
  def.initial_beta2_power = d.optimizer.initial_beta2_power;
  def.bounded = d.optimizer.weight_bounds ? 1 : 0;
  if (d.optimizer.weight_bounds) {
    def.weight_min = d.optimizer.weight_bounds->minimum;
    def.weight_max = d.optimizer.weight_bounds->maximum;
  }
  def.init_min = d.initialization_min;
  def.init_max = d.initialization_max;
  def.init_seed = d.initialization_seed;
  return def;
}

eps_or_feature AsOracle(const FeatureInput& f) {
  return {f.keys.data(), f.keys.size(), f.offsets.data(), f.valid_lengths.data(), nullptr,
          f.valid_lengths.size(), uint32_t(f.pooling), f.feature};
}

// The feature restricted to the occurrences `keep` accepts: bags keep their
// place and their original lengths (the mean scale), as a shard sees its part
// of a lookup (src/access/prepared_lookup.cpp:47-83).
template <typename Keep>
FeatureInput Restrict(const FeatureInput& f, Keep keep) {
  FeatureInput out{f.table, f.feature, f.pooling, {}, {0}, f.valid_lengths};
  for (std::size_t b = 0; b + 1 < f.offsets.size(); ++b) {
    for (std::uint64_t i = f.offsets[b]; i < f.offsets[b + 1]; ++i)
      if (keep(f.keys[i])) out.keys.push_back(f.keys[i]);
    out.offsets.push_back(out.keys.size());
  }
  return out;
}

// A push over rows of mixed ownership, as the shard service runs it
// (src/server/service.cpp:236-331): one lookup ticket of three features over
// two tables; keys k % 3 == 0 live in the shard's CPU store, the others on
// this agent.  Every step the service reduces the ticket's gradients per
// table, applies LazyAdam to its CPU rows and sends the agent its rows'
// gradients, compact (CSR) when that is smaller than the expanded rows and
// the expanded rows exceed 20 bytes per row + 8 (:279-295), else expanded;
// the powers advance once per table.  Odd steps take the device-resident
// route instead: PushDevice for the agent's rows (the CPU keys are holes) and
// the CPU rows through the shard's own push.  After every step each row,
// wherever it lives, and each table's powers equal one CPU shard that held
// every row and took the same pushes.
void MixedPush() {
  HipCacheOptions o = SmallOptions(4096);
  o.state_bytes = 64ull << 20;
  o.transfer_bytes = 8ull << 20;
  HipCacheBackend gpu(o);
  const std::vector<TableDefinition> defs = {Table(21, 64), Table(22, 32)};
  constexpr Key kKeys = 3000;
  auto on_cpu = [](Key k) { return k % 3 == 0; };
  std::vector<eps_or_store*> truth, cpu;
  std::map<std::pair<TableId, Key>, LocatedRow> where;
  for (const auto& d : defs) {
    Take(gpu.Define(d));
    const eps_or_table_def def = OracleDef(d);
    truth.push_back(eps_or_create(&def));
    cpu.push_back(eps_or_create(&def));
    std::vector<RowState> agent_rows;
    for (Key k = 0; k < kKeys; ++k) {
      Check(eps_or_ensure(truth.back(), k) >= 0, "oracle first touch");
      RowState r{{d.id, k}, std::vector<float>(d.dimension), std::vector<float>(d.dimension),
                 std::vector<float>(d.dimension), 0};
      Check(eps_or_read(truth.back(), k, r.weights.data(), r.first_moment.data(), r.second_moment.data(),
                        &r.row_updates) == 0,
            "oracle read");
      if (on_cpu(k)) {
        Check(eps_or_import(cpu.back(), k, r.weights.data(), r.first_moment.data(), r.second_moment.data(), 0) == 0,
              "oracle import");
      } else {
        agent_rows.push_back(std::move(r));
      }
    }
    for (const auto& loc : Take(gpu.Load(Plan(agent_rows), agent_rows))) where[{loc.row.table, loc.row.key}] = loc;
  }
  std::uint64_t state = 99;
  auto next = [&]() {
    state += 0x9e3779b97f4a7c15ull;
    std::uint64_t z = state;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  };
  int compact_sends = 0, expanded_sends = 0;
  for (int step = 0; step < 4; ++step) {
    // The ticket: feature 0 (table 21, mean), 1 (table 21, sum), 2 (table 22, sum).
    std::vector<FeatureInput> layouts;
    std::vector<std::vector<float>> grads;
    const std::pair<std::size_t, Pooling> spec[] = {{0, Pooling::mean}, {0, Pooling::sum}, {1, Pooling::sum}};
    for (std::uint32_t fi = 0; fi < 3; ++fi) {
      const TableDefinition& d = defs[spec[fi].first];
      FeatureInput f{d.id, fi, spec[fi].second, {}, {0}, {}};
      // Step 2's bags hold one id each: every agent row has its own source
      // row, so the CSR is larger than the expanded rows and goes expanded.
      const int bags = step == 2 ? 120 : 300;
      for (int b = 0; b < bags; ++b) {
        const std::uint64_t len = step == 2 ? 1 : 1 + next() % 12;
        for (std::uint64_t i = 0; i < len; ++i) {
          const double u = double(next() >> 11) * 0x1.0p-53;
          f.keys.push_back(Key(double(kKeys) * u * u * u));
        }
        f.offsets.push_back(f.keys.size());
        f.valid_lengths.push_back(len + (b % 5 == 0 ? 1 : 0));
      }
      std::vector<float> g(f.valid_lengths.size() * d.dimension);
      for (auto& x : g) x = float(std::int64_t(next() % 2001) - 1000) * 2e-5f;
      layouts.push_back(std::move(f));
      grads.push_back(std::move(g));
    }
    std::vector<eps_or_feature> of;
    std::vector<const float*> og;
    std::vector<std::uint32_t> store_of;
    for (std::size_t i = 0; i < layouts.size(); ++i) {
      of.push_back(AsOracle(layouts[i]));
      og.push_back(grads[i].data());
      store_of.push_back(layouts[i].table == 21 ? 0 : 1);
    }
    // The context of each table: the shard's powers before this push.
    std::vector<UpdateContext> contexts;
    for (std::size_t t = 0; t < defs.size(); ++t) {
      float b1 = 0, b2 = 0;
      std::uint64_t seq = 0;
      eps_or_powers(cpu[t], &b1, &b2, &seq);
      contexts.push_back({{"mixed", 0, std::uint64_t(step), Phase::push}, 0, defs[t].id, seq, kLr, b1, b2});
    }
    Check(eps_or_push(truth.data(), 2, of.data(), store_of.data(), og.data(), 3) == 0, "oracle push (all rows)");
    if (step % 2 == 0) {
      for (std::size_t t = 0; t < defs.size(); ++t) {
        const std::uint32_t dim = defs[t].dimension;
        std::vector<eps_or_feature> tf;
        std::vector<const float*> tg;
        std::uint64_t n = 0;
        for (std::size_t i = 0; i < layouts.size(); ++i)
          if (store_of[i] == t) {
            tf.push_back(of[i]);
            tg.push_back(og[i]);
            n += of[i].key_count;
          }
        std::vector<std::uint64_t> keys(n + 1);
        std::vector<float> values((n + 1) * dim);
        std::uint64_t count = 0;
        Check(eps_or_reduce_gradients(truth[t], tf.data(), tg.data(), uint32_t(tf.size()), keys.data(), values.data(),
                                      &count) == 0,
              "oracle reduce");
        std::vector<std::uint64_t> cpu_keys, gpu_keys;
        std::vector<float> cpu_values, gpu_values;
        for (std::uint64_t u = 0; u < count; ++u) {
          auto& k = on_cpu(keys[u]) ? cpu_keys : gpu_keys;
          auto& v = on_cpu(keys[u]) ? cpu_values : gpu_values;
          k.push_back(keys[u]);
          v.insert(v.end(), values.begin() + u * dim, values.begin() + (u + 1) * dim);
        }
        // The agent's packet (service.cpp:279-295).
        const std::uint64_t expanded = gpu_values.size() * 4;
        bool sent = false;
        if (!gpu_keys.empty() && expanded > gpu_keys.size() * 20 + 8) {
          std::vector<float> source(n * dim + 1);
          std::vector<std::uint64_t> offsets(gpu_keys.size() + 1), refs(n + 1);
          std::vector<float> scales(n + 1);
          std::uint64_t sources = 0, references = 0;
          if (eps_or_build_compact(tf.data(), tg.data(), uint32_t(tf.size()), dim, gpu_keys.data(), gpu_keys.size(),
                                   source.data(), &sources, offsets.data(), refs.data(), scales.data(),
                                   &references) == 0) {
            const std::uint64_t bytes = eps_or_compact_bytes(gpu_keys.size(), sources, references) -
                                        gpu_keys.size() * sizeof(RowKey);
            if (bytes < expanded) {
              CompactGradients packet{{}, dim, {source.begin(), source.begin() + sources}, offsets,
                                      {refs.begin(), refs.begin() + references},
                                      {scales.begin(), scales.begin() + references}};
              for (Key k : gpu_keys) packet.rows.push_back({defs[t].id, k});
              Take(gpu.ApplyCompact(contexts[t], packet));
              sent = true;
              ++compact_sends;
            }
          }
        }
        if (!sent && !gpu_keys.empty()) {
          RowGradients rg{{}, gpu_values};
          for (Key k : gpu_keys) rg.rows.push_back({defs[t].id, k});
          Take(gpu.ApplyHost(contexts[t], rg));
          ++expanded_sends;
        }
        // CPU rows last; the table's powers advance once, rows or not (:325).
        Check(eps_or_validate_lazy_adam(cpu[t], cpu_keys.data(), cpu_values.data(), cpu_keys.size()) == 0,
              "oracle validate");
        eps_or_apply_lazy_adam(cpu[t], cpu_keys.data(), cpu_values.data(), cpu_keys.size());
      }
    } else {
      std::vector<AgentWork> work;
      for (const auto& f : layouts) {
        AgentWork w{f.feature, AccessRoute::resident_gpu, 0, {}, std::vector<std::uint64_t>(f.keys.size()), {}};
        std::map<Key, std::uint64_t> unique;
        for (std::size_t i = 0; i < f.keys.size(); ++i) {
          if (on_cpu(f.keys[i])) {
            w.occurrence_to_unique[i] = UINT64_MAX;
            continue;
          }
          auto [it, fresh] = unique.emplace(f.keys[i], w.rows.size());
          if (fresh) w.rows.push_back(where.at({f.table, f.keys[i]}));
          w.occurrence_to_unique[i] = it->second;
        }
        work.push_back(std::move(w));
      }
      std::vector<DeviceTensorBlock> blocks;
      for (std::size_t i = 0; i < layouts.size(); ++i) {
        const std::uint64_t dim = layouts[i].table == 21 ? 64 : 32;
        blocks.push_back({layouts[i].feature, {layouts[i].valid_lengths.size(), dim},
                          std::make_shared<DeviceBuffer>(grads[i])});
      }
      Take(gpu.PushDevice(contexts, work, layouts, blocks));
      std::vector<FeatureInput> mine;
      std::vector<eps_or_feature> cf;
      for (const auto& f : layouts) mine.push_back(Restrict(f, on_cpu));
      for (const auto& f : mine) cf.push_back(AsOracle(f));
      Check(eps_or_push(cpu.data(), 2, cf.data(), store_of.data(), og.data(), 3) == 0, "oracle push (CPU rows)");
    }
    // Every row against the single-shard truth.
    for (std::size_t t = 0; t < defs.size(); ++t) {
      float b1 = 0, b2 = 0, c1 = 0, c2 = 0;
      std::uint64_t s1 = 0, s2 = 0;
      eps_or_powers(truth[t], &b1, &b2, &s1);
      eps_or_powers(cpu[t], &c1, &c2, &s2);
      Check(b1 == c1 && b2 == c2 && s1 == s2, "powers advanced other than once per push");
      const std::uint32_t dim = defs[t].dimension;
      MigrationPlan read{"read", 0, {}, Placement::cpu, 0};
      for (Key k = 0; k < kKeys; ++k) {
        std::vector<float> w(dim), m(dim), v(dim), cw(dim), cm(dim), cv(dim);
        std::uint64_t updates = 0, cu = 0;
        Check(eps_or_read(truth[t], k, w.data(), m.data(), v.data(), &updates) == 0, "truth row");
        if (on_cpu(k)) {
          Check(eps_or_read(cpu[t], k, cw.data(), cm.data(), cv.data(), &cu) == 0 && SameBits(w, cw) &&
                    SameBits(m, cm) && SameBits(v, cv) && cu == updates,
                "CPU row of the mixed push differs");
        } else {
          read.rows.push_back(where.at({defs[t].id, k}));
        }
      }
      for (const auto& r : Take(gpu.ReadBack(read))) {
        std::vector<float> w(dim), m(dim), v(dim);
        std::uint64_t updates = 0;
        Check(eps_or_read(truth[t], r.row.key, w.data(), m.data(), v.data(), &updates) == 0, "truth row");
        Check(SameBits(r.weights, w) && SameBits(r.first_moment, m) && SameBits(r.second_moment, v) &&
                  r.row_updates == updates,
              "agent row of the mixed push differs (step " + std::to_string(step) + ", table " +
                  std::to_string(defs[t].id) + ", key " + std::to_string(r.row.key) + ")");
      }
    }
  }
  Check(compact_sends > 0 && expanded_sends > 0, "the service's packet choice took only one form");
  for (auto* s : truth) eps_or_destroy(s);
  for (auto* s : cpu) eps_or_destroy(s);
}

// GatherDevice and PushDevice at the occurrence count of the 4 x 12.5M x 128
// workload: 4 mean features of 262,144 bags x 32 ids (33.5 M occurrences),
// Zipf(1.1) ids over 60,000 keys per table, of which this agent holds the
// first 50,000 (the rest are served elsewhere: holes).  Every occurrence is
// resolved to its slot on the device.  Checked against the oracle on 1,024
// sampled bags of each feature (pull) and, after the push, on the 16 hottest
// and 240 random held rows of each table (the oracle reduces every occurrence
// of those keys, in order, with the full bags' mean scales).
void LargeOccurrences() {
  constexpr std::uint32_t kDim = 128, kBags = 262144, kLen = 32, kTables = 4;
  constexpr Key kHeld = 50000, kIds = 60000;
  HipCacheOptions o = SmallOptions(65536);
  o.state_bytes = 8ull << 30;
  o.transfer_bytes = 1ull << 30;
  o.outstanding_output_bytes = 1ull << 30;
  HipCacheBackend gpu(o);
  std::vector<double> cdf(kIds);
  double total = 0;
  for (Key r = 0; r < kIds; ++r) cdf[r] = total += std::pow(double(r + 1), -1.1);
  std::uint64_t state = 4;
  auto next = [&]() {
    state += 0x9e3779b97f4a7c15ull;
    std::uint64_t z = state;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  };
  std::vector<TableDefinition> defs;
  std::map<std::pair<TableId, Key>, RowState> model;
  std::map<std::pair<TableId, Key>, LocatedRow> where;
  std::vector<FeatureInput> layouts;
  std::vector<AgentWork> work;
  std::vector<std::vector<float>> grads;
  for (std::uint32_t t = 0; t < kTables; ++t) {
    defs.push_back(Table(40 + t, kDim));
    Take(gpu.Define(defs.back()));
    for (Key b = 0; b < kHeld; b += 10000) {
      std::vector<RowState> part;
      for (Key k = b; k < b + 10000; ++k) part.push_back(model[{40 + t, k}] = MakeRow(40 + t, k, kDim));
      for (const auto& loc : Take(gpu.Load(Plan(part), part))) where[{loc.row.table, loc.row.key}] = loc;
    }
    FeatureInput f{40 + t, t, Pooling::mean, std::vector<Key>(std::uint64_t(kBags) * kLen), {}, {}};
    f.offsets.resize(kBags + 1);
    f.valid_lengths.assign(kBags, kLen);
    for (std::uint64_t b = 0; b <= kBags; ++b) f.offsets[b] = b * kLen;
    // Rank -> key through a fixed odd multiplier, so the hot keys are spread.
    for (auto& k : f.keys) {
      const double u = double(next() >> 11) * 0x1.0p-53 * total;
      const Key rank = Key(std::lower_bound(cdf.begin(), cdf.end(), u) - cdf.begin());
      k = (std::min(rank, kIds - 1) * 7919 + 13) % kIds;
    }
    AgentWork w{t, AccessRoute::resident_gpu, 0, {}, std::vector<std::uint64_t>(f.keys.size()), {}};
    std::vector<std::uint64_t> unique(kIds, UINT64_MAX);
    for (std::size_t i = 0; i < f.keys.size(); ++i) {
      const Key k = f.keys[i];
      if (k >= kHeld) {
        w.occurrence_to_unique[i] = UINT64_MAX;
        continue;
      }
      if (unique[k] == UINT64_MAX) {
        unique[k] = w.rows.size();
        w.rows.push_back(where.at({40 + t, k}));
      }
      w.occurrence_to_unique[i] = unique[k];
    }
    std::vector<float> g(std::uint64_t(kBags) * kDim);
    for (auto& x : g) x = float(std::int64_t(next() % 2001) - 1000) * 1e-5f;
    layouts.push_back(std::move(f));
    work.push_back(std::move(w));
    grads.push_back(std::move(g));
  }
  auto pulled = Take(gpu.GatherDevice(work, layouts));
  for (std::uint32_t t = 0; t < kTables; ++t) {
    const FeatureInput& f = layouts[t];
    const std::vector<float> got = pulled[t].tensor->CopyToHost();
    Check(pulled[t].shape == std::vector<std::uint64_t>{kBags, kDim}, "large pull shape");
    for (int s = 0; s < 1024; ++s) {
      const std::uint64_t b = next() % kBags;
      std::vector<float> want(kDim, 0.f);
      for (std::uint64_t i = f.offsets[b]; i < f.offsets[b + 1]; ++i) {
        if (f.keys[i] >= kHeld) continue;
        const auto& w = model.at({40 + t, f.keys[i]}).weights;
        for (std::uint32_t d = 0; d < kDim; ++d) want[d] = want[d] + w[d];
      }
      Check(std::memcmp(want.data(), got.data() + b * kDim, kDim * 4) == 0,
            "large pull bag differs (table " + std::to_string(t) + ", bag " + std::to_string(b) + ")");
    }
  }
  std::vector<UpdateContext> contexts;
  std::vector<DeviceTensorBlock> blocks;
  for (std::uint32_t t = 0; t < kTables; ++t) {
    contexts.push_back({{"large", 0, 1, Phase::push}, 0, 40 + t, 0, kLr, 0.9f, 0.999f});
    blocks.push_back({t, {kBags, kDim}, std::make_shared<DeviceBuffer>(grads[t])});
  }
  Take(gpu.PushDevice(contexts, work, layouts, blocks));
  for (std::uint32_t t = 0; t < kTables; ++t) {
    const FeatureInput& f = layouts[t];
    std::vector<std::uint64_t> counts(kHeld, 0);
    for (Key k : f.keys)
      if (k < kHeld) ++counts[k];
    std::vector<Key> by_count;
    for (Key k = 0; k < kHeld; ++k)
      if (counts[k]) by_count.push_back(k);
    std::sort(by_count.begin(), by_count.end(), [&](Key a, Key b) { return counts[a] > counts[b]; });
    std::set<Key> sample(by_count.begin(), by_count.begin() + 16);
    while (sample.size() < 256) sample.insert(by_count[next() % by_count.size()]);
    const FeatureInput part = Restrict(f, [&](Key k) { return sample.count(k) > 0; });
    eps_or_table_def def = OracleDef(defs[t]);
    eps_or_store* store = eps_or_create(&def);
    const eps_or_feature of = AsOracle(part);
    const float* og = grads[t].data();
    std::vector<std::uint64_t> keys(part.keys.size() + 1);
    std::vector<float> values((part.keys.size() + 1) * kDim);
    std::uint64_t count = 0;
    Check(eps_or_reduce_gradients(store, &of, &og, 1, keys.data(), values.data(), &count) == 0 && count == sample.size(),
          "oracle reduce (large)");
    eps_or_destroy(store);
    MigrationPlan read{"read", 0, {}, Placement::cpu, 0};
    for (std::uint64_t u = 0; u < count; ++u) {
      RowState& r = model.at({40 + t, keys[u]});
      Check(eps_or_adam_rows_ctx(r.weights.data(), r.first_moment.data(), r.second_moment.data(),
                                 values.data() + u * kDim, 1, kDim, kBeta1, kBeta2, kEps, kLr, 0.9f, 0.999f, 0, 0, 0) == 0,
            "oracle Adam (large)");
      ++r.row_updates;
      read.rows.push_back(where.at({40 + t, keys[u]}));
    }
    for (const auto& got : Take(gpu.ReadBack(read))) {
      const RowState& want = model.at({got.row.table, got.row.key});
      Check(SameBits(got.weights, want.weights) && SameBits(got.first_moment, want.first_moment) &&
                SameBits(got.second_moment, want.second_moment) && got.row_updates == want.row_updates,
            "large push row differs (table " + std::to_string(t) + ", key " + std::to_string(got.row.key) + ", " +
                std::to_string(counts[got.row.key]) + " references)");
    }
  }
}

// A device push whose hot-row hand-over times out (forced from the host with a
// spin limit of 0: the hot-row kernel runs for a push with a table of 65,536
// or more references) may have been applied in part -- the row kernels beside
// it keep writing -- so the agent stops: that push fails with run_failed, and
// so does every later operation on the agent.
void StalledPushStops() {
  HipCacheOptions o = SmallOptions(4096);
  o.state_bytes = 64ull << 20;
  o.transfer_bytes = 16ull << 20;
  HipCacheBackend gpu(o);
  constexpr TableId kTable = 21;
  Take(gpu.Define(Table(kTable, 64)));
  std::vector<RowState> part;
  for (Key k = 0; k < 3000; ++k) part.push_back(MakeRow(kTable, k, 64));
  std::map<Key, LocatedRow> where;
  for (const auto& loc : Take(gpu.Load(Plan(part), part))) where[loc.row.key] = loc;
  // 70,000 single-id bags: key 0 in every tenth bag (a hot row), the rest spread.
  FeatureInput f{kTable, 0, Pooling::sum, {}, {0}, {}};
  AgentWork w{0, AccessRoute::resident_gpu, 0, {}, {}, {}};
  std::map<Key, std::uint64_t> unique;
  for (std::uint64_t b = 0; b < 70000; ++b) {
    const Key key = b % 10 == 0 ? 0 : 1 + b % 2999;
    f.keys.push_back(key);
    f.offsets.push_back(b + 1);
    f.valid_lengths.push_back(1);
    auto [it, fresh] = unique.emplace(key, w.rows.size());
    if (fresh) w.rows.push_back(where.at(key));
    w.occurrence_to_unique.push_back(it->second);
  }
  std::vector<float> g(70000 * 64);
  for (std::size_t i = 0; i < g.size(); ++i) g[i] = 1e-3f * float(int(i % 17) - 8);
  const std::vector<UpdateContext> contexts = {{{"stall", 0, 1, Phase::push}, 0, kTable, 1, kLr, 0.81f, 0.998f}};
  const std::vector<FeatureInput> layouts = {f};
  const std::vector<AgentWork> work = {w};
  std::vector<DeviceTensorBlock> blocks = {{0, {70000, 64}, std::make_shared<DeviceBuffer>(g)}};
  Check(eps_hip_debug_set_spin_limit(0) == 0, "spin limit");
  const auto code = Fails(gpu.PushDevice(contexts, work, layouts, blocks), "stalled device push");
  Check(eps_hip_debug_set_spin_limit(1u << 22) == 0, "spin limit");
  Check(code == Error::Code::run_failed, "a stalled push is the agent's own failure");
  Check(Fails(gpu.PushDevice(contexts, work, layouts, blocks), "push after a stall") == Error::Code::run_failed,
        "the agent stopped after a stalled push");
  Check(Fails(gpu.GatherHost(work, layouts), "gather after a stall") == Error::Code::run_failed,
        "a stopped agent serves no gathers");
}

// Admission and eviction churn on a 256-row table (a 512-bucket key index):
// 40 rounds each admit 150 fresh keys beside 50 that stay, gather a sum over
// all of them and evict the 150 again, 6,000 removals in all.  Every gather
// resolves each occurrence through the index (a key it lost fails the
// gather) and must match the oracle bit for bit; the index must have been
// rebuilt along the way, and the rows that stay must still read back whole.
void EvictionChurn() {
  HipCacheBackend gpu(SmallOptions(256));
  Take(gpu.Define(Table(2, 64)));
  auto state = [](Key key) {
    RowState r{{2, key}, std::vector<float>(64), std::vector<float>(64, 0.f), std::vector<float>(64, 0.f), 0};
    for (std::uint32_t d = 0; d < 64; ++d) r.weights[d] = 0.001f * float((key * 7 + d) % 97);
    return r;
  };
  Model model;
  std::vector<RowState> stay;
  for (Key k = 1; k <= 50; ++k) stay.push_back(state(k * 7919));
  const auto stay_at = Take(gpu.Load(Plan(stay), stay));
  for (const auto& r : stay) model.rows[{2, r.row.key}] = r;
  for (int round = 0; round < 40; ++round) {
    std::vector<RowState> churn;
    for (Key j = 0; j < 150; ++j) churn.push_back(state(1000003ull * Key(round + 1) + j * 131));
    const auto churn_at = Take(gpu.Load(Plan(churn), churn));
    for (const auto& r : churn) model.rows[{2, r.row.key}] = r;
    // Bag b sums churned row b and staying row b % 50.
    AgentWork w{0, AccessRoute::resident_gpu, 0, stay_at, {}, {}};
    w.rows.insert(w.rows.end(), churn_at.begin(), churn_at.end());
    FeatureInput f{2, 0, Pooling::sum, {}, {0}, {}};
    for (std::uint64_t b = 0; b < 150; ++b) {
      f.keys.push_back(churn[b].row.key);
      w.occurrence_to_unique.push_back(50 + b);
      f.keys.push_back(stay[b % 50].row.key);
      w.occurrence_to_unique.push_back(b % 50);
      f.offsets.push_back(2 * (b + 1));
      f.valid_lengths.push_back(2);
    }
    CompareGather(Take(gpu.GatherHost({w}, {f})), model, {w}, {f}, "gather under eviction churn");
    Take(gpu.CommitEviction(MigrationPlan{"evict", 0, churn_at, Placement::cpu, 0}));
    for (const auto& r : churn) model.rows.erase({2, r.row.key});
  }
  Check(Take(gpu.MemoryStats()).index_rebuilds >= 30, "key index not rebuilt under eviction churn");
  Check(Take(gpu.FreeSlots(2)) == 206, "slots after eviction churn");
  CompareStates(Take(gpu.ReadBack(MigrationPlan{"read", 0, stay_at, Placement::cpu, 0})), model,
                "staying rows after eviction churn");
}

void Main() {
  EvictionChurn();
  AtomicReserve();
  SnapshotWriteback();
  DevicePushAtScale();
  MixedPush();
  LargeOccurrences();
  StalledPushStops();
  auto gpu = std::make_shared<HipCacheBackend>(SmallOptions(8));
  for (const auto& t : {Table(1, 128), Table(2, 64)}) Take(gpu->Define(t));
  Take(gpu->Define(Table(1, 128)));  // identical redefinition is accepted
  Check(Fails(gpu->Define(Table(1, 64)), "conflicting redefinition") == Error::Code::invalid_argument,
        "redefinition code");
  auto rows = States();
  Model model;
  for (const auto& r : rows) model.rows[{r.row.table, r.row.key}] = r;
  auto plan = Plan(rows);
  auto located = Take(gpu->Load(plan, rows));
  Check(located[0].slot == 0 && located[1].slot == 1 && located[0].placement == Placement::gpu,
        "slots are handed out from the bottom of the free list");
  Check(Take(gpu->FreeSlots(1)) == 4 && Take(gpu->FreeSlots(2)) == 6, "free slots after load");
  auto work = Work(located);
  auto layouts = Layouts();
  CompareGather(Take(gpu->GatherHost(work, layouts)), model, work, layouts, "resident gather");

  // CPU-owned unique vectors travel with the request and use the same pooling.
  auto cold = work;
  for (auto& task : cold) {
    task.route = AccessRoute::transfer_unique;
    for (auto& loc : task.rows) {
      loc.placement = Placement::cpu;
      const auto& w = model.Get(loc.row.table, loc.row.key).weights;
      task.transferred_weights.insert(task.transferred_weights.end(), w.begin(), w.end());
    }
  }
  CompareGather(Take(gpu->GatherHost(cold, layouts)), model, work, layouts, "transfer_unique gather");
  auto poisoned = cold;
  poisoned[0].transferred_weights[3] = std::numeric_limits<float>::infinity();
  Check(Fails(gpu->GatherHost(poisoned, layouts), "non-finite transferred weight") == Error::Code::invalid_argument,
        "transferred weight code");

  auto device = Take(gpu->GatherDevice(work, layouts));
  std::vector<TensorBlock> before;
  for (std::size_t i = 0; i < work.size(); ++i)
    before.push_back(Expected(model, work[i], layouts[i], layouts[i].table == 1 ? 128 : 64));
  for (std::size_t i = 0; i < device.size(); ++i) {
    device[i].tensor->WaitOnStream(nullptr);
    Check(SameBits(device[i].tensor->CopyToHost(), before[i].values), "device gather result");
  }

  float b1 = 0.9f, b2 = 0.999f;
  const std::vector<Key> keys = {1, 2, 3, 4};
  for (std::uint64_t step = 0; step < 7; ++step) {
    UpdateContext c{{"hip-test", 0, step, Phase::push}, 0, 1, step, kLr, b1, b2};
    RowGradients g;
    for (Key key : keys) {
      g.rows.push_back({1, key});
      for (int d = 0; d < 128; ++d) g.values.push_back(0.05f * std::sin(float(key * 3 + d + 2 * step)));
    }
    Take(gpu->ApplyHost(c, g));
    ApplyModel(model, 1, keys, g.values, b1, b2);
    b1 *= 0.9f;
    b2 *= 0.999f;
    CompareGather(Take(gpu->GatherHost(work, layouts)), model, work, layouts, "gather after ApplyHost");
  }
  CompactGradients compact{{{1, 1}, {1, 2}, {1, 3}, {1, 4}}, 128, {}, {0, 3, 4, 6, 7},
                           {0, 1, 0, 2, 1, 2, 0}, {1.0f / 3, 0.5f, 1.0f / 3, 1, 0.25f, 0.25f, 1}};
  for (int source = 0; source < 3; ++source)
    for (int d = 0; d < 128; ++d) compact.source_values.push_back(0.02f * std::cos(float(source * 7 + d)));
  for (std::uint64_t step = 7; step < 9; ++step) {
    UpdateContext c{{"hip-test", 0, step, Phase::push}, 0, 1, step, kLr, b1, b2};
    Take(gpu->ApplyCompact(c, compact));
    std::vector<float> g(4 * 128);
    const std::vector<std::uint64_t> row_keys = {1, 2, 3, 4};
    Check(eps_or_expand_compact(4, row_keys.data(), 128, compact.source_values.data(),
                                compact.source_values.size(), compact.row_offsets.data(),
                                compact.source_rows.data(), compact.scales.data(), compact.source_rows.size(),
                                g.data()) == 0,
          "oracle CSR expansion failed");
    ApplyModel(model, 1, keys, g, b1, b2);
    b1 *= 0.9f;
    b2 *= 0.999f;
  }
  MigrationPlan readback{"read", 0, located, Placement::cpu, 0};
  std::reverse(readback.rows.begin(), readback.rows.end());
  auto original = Take(gpu->ReadBack(readback));
  CompareStates(original, model, "ReadBack after 7 ApplyHost + 2 ApplyCompact");
  bool clipped = false;
  for (const auto& r : original)
    if (r.row.table == 1)
      for (float w : r.weights) {
        Check(w >= kMin && w <= kMax, "bounded weight escaped its interval");
        clipped = clipped || w == kMin || w == kMax;
      }
  Check(clipped, "the updates did not exercise clipping");

  // Updates that would overflow are rejected whole: no row changes.
  UpdateContext bad{{"hip-test", 0, 9, Phase::push}, 0, 1, 9, kLr, b1, b2};
  auto overflow_compact = compact;
  std::fill(overflow_compact.source_values.begin(), overflow_compact.source_values.end(),
            std::numeric_limits<float>::max());
  Fails(gpu->ApplyCompact(bad, overflow_compact), "overflowing compact update");
  CompareStates(Take(gpu->ReadBack(readback)), model, "state after rejected compact update");
  RowGradients overflow{{{1, 1}, {1, 3}}, std::vector<float>(2 * 128, 1.f)};
  overflow.values.back() = std::numeric_limits<float>::max();
  Fails(gpu->ApplyHost(bad, overflow), "overflowing update");
  CompareStates(Take(gpu->ReadBack(readback)), model, "state after rejected update");
  RowGradients duplicate{{{1, 1}, {1, 1}}, std::vector<float>(2 * 128, 0.f)};
  Check(Fails(gpu->ApplyHost(bad, duplicate), "duplicate rows") == Error::Code::invalid_argument, "duplicate code");
  UpdateContext invalid = bad;
  invalid.learning_rate = 0.f;
  Fails(gpu->ApplyHost(invalid, RowGradients{{{1, 2}}, std::vector<float>(128, 0.f)}), "zero learning rate");
  auto bad_csr = compact;
  bad_csr.source_rows[2] = 3;  // only three source rows exist
  Fails(gpu->ApplyCompact(bad, bad_csr), "out-of-range CSR reference");
  CompareStates(Take(gpu->ReadBack(readback)), model, "state after rejected requests");

  for (std::size_t i = 0; i < device.size(); ++i)
    Check(SameBits(device[i].tensor->CopyToHost(), before[i].values), "device result changed after updates");

  DevicePush(*gpu, located, model, b1, b2);

  Assembly(*gpu, located, model);
  auto stats = Take(gpu->MemoryStats());
  Check(stats.resident_state_bytes == 8ull * (128 + 64) * 12, "resident state bytes");

  Take(gpu->CommitEviction(readback));
  Check(Take(gpu->FreeSlots(1)) == 8 && Take(gpu->FreeSlots(2)) == 8, "slots reclaimed by eviction");
  for (auto& r : rows) r = model.Get(r.row.table, r.row.key);
  for (auto& loc : plan.rows) loc.generation += 2;
  auto reloaded = Take(gpu->Load(plan, rows));
  Check(Fails(gpu->GatherHost(work, layouts), "stale slot") == Error::Code::stale_generation,
        "stale generation code");
  auto fresh = Work(reloaded);
  CompareGather(Take(gpu->GatherHost(fresh, layouts)), model, fresh, layouts, "gather after reload");

  gpu.reset();  // device results own their memory and outlive the backend
  for (std::size_t i = 0; i < device.size(); ++i)
    Check(SameBits(device[i].tensor->CopyToHost(), before[i].values), "device result after backend release");
}

}  // namespace

int main() {
  try {
    Main();
    std::cout << "PASS HIP backend: " << g_checks
              << " checks (gathers, optimizer states, device push, snapshot writeback, atomic "
                 "rejection, slot reuse, eviction churn, assembly, device-result lifetime)\n";
    return 0;
  } catch (const std::exception& e) {
    std::cerr << "FAIL HIP backend: " << e.what() << '\n';
    return 1;
  }
}
