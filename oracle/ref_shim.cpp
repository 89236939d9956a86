// ref_shim.cpp -- C entry points over the reference's own CPU shard sources.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together with
// the reference's unmodified sources (src/store/shard_store.cpp,
// src/access/batch_access.cpp, src/access/compact_gradients.cpp,
// src/update/lazy_adam.cpp, src/cache/host_backend.cpp, src/store/snapshot.cpp)
// where they lie in the
// reference checkout, into oracle/_ref/libeps_ref.so.  Tests use it to pin the
// C restatement in oracle/eps_oracle.c; bench.py may time it as the CPU
// baseline.  Nothing here is part of the product.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "access/batch_access.hpp"
#include "common/error.hpp"
#include "eps/cache_backend.hpp"
#include "eps/compact_gradients.hpp"
#include "store/shard_store.hpp"
#include "store/snapshot.hpp"
#include "update/lazy_adam.hpp"

#include "eps_oracle.h"

using namespace eps;

namespace {
thread_local std::string g_error;
int Code(const Error& e) { g_error = e.message; return int(e.code) + 1; }
template <typename F> int Guard(F&& f) {
  try { f(); return 0; }
  catch (const detail::Failure& e) { return Code(e.error()); }
  catch (const std::exception& e) { g_error = e.what(); return int(Error::Code::run_failed) + 1; }
}
Pooling Mode(std::uint32_t p) { return static_cast<Pooling>(p); }
FeatureInput Input(std::uint32_t table, const eps_or_feature& f) {
  FeatureInput in{table, f.feature, Mode(f.pooling), {f.keys, f.keys + f.key_count},
                  {f.offsets, f.offsets + f.bag_count + 1},
                  {f.valid_lengths, f.valid_lengths + f.bag_count}};
  return in;
}
TableDefinition Definition(const eps_or_table_def& t) {
  TableDefinition d{t.id, t.dim, t.shard_count, 1,
                    {t.learning_rate, t.beta1, t.beta2, t.epsilon,
                     t.initial_beta1_power, t.initial_beta2_power},
                    t.init_min, t.init_max, t.init_seed};
  if (t.bounded) d.optimizer.weight_bounds = WeightBounds{t.weight_min, t.weight_max};
  return d;
}
struct Shard {
  detail::ShardStore store;
  std::vector<detail::PreparedFeature> prepared;
  Shard(std::uint32_t shard, std::uint32_t count) : store(shard, count, 1, ~0ULL >> 1) {}
};
template <typename T> T Take(std::future<Result<T>> f) {
  auto r = f.get();
  if (auto* e = std::get_if<Error>(&r)) throw detail::Failure(*e);
  return std::get<T>(std::move(r));
}
}  // namespace

extern "C" {
const char* ref_last_error(void) { return g_error.c_str(); }

void* ref_shard_create(std::uint32_t shard, std::uint32_t count) {
  return new Shard(shard, count);
}
void ref_shard_destroy(void* h) { delete static_cast<Shard*>(h); }

// WriteSnapshot of the shard (format 2; the file must not exist yet).
int ref_shard_write_snapshot(void* h, const char* path, const char* run) {
  return Guard([&] { detail::WriteSnapshot(path, run, static_cast<Shard*>(h)->store); });
}

int ref_shard_create_table(void* h, const eps_or_table_def* t) {
  return Guard([&] { static_cast<Shard*>(h)->store.Create(Definition(*t)); });
}

// ShardStore::Ensure for a key (first-touch slot); returns the slot.
int ref_shard_ensure(void* h, std::uint32_t table, std::uint64_t key, std::uint64_t* slot) {
  return Guard([&] { *slot = static_cast<Shard*>(h)->store.Ensure(table, key); });
}

int ref_shard_import(void* h, std::uint32_t table, std::uint64_t key, const float* w,
                     const float* m, const float* v, std::uint64_t updates) {
  return Guard([&] {
    auto& s = static_cast<Shard*>(h)->store;
    const auto dim = s.Table(table).definition.dimension;
    s.Import({{table, key}, {w, w + dim}, {m, m + dim}, {v, v + dim}, updates});
  });
}

int ref_shard_read(void* h, std::uint32_t table, std::uint64_t key, float* w, float* m,
                   float* v, std::uint64_t* updates) {
  return Guard([&] {
    auto row = static_cast<Shard*>(h)->store.Read(table, key);
    std::memcpy(w, row.weights.data(), row.weights.size() * 4);
    std::memcpy(m, row.first_moment.data(), row.first_moment.size() * 4);
    std::memcpy(v, row.second_moment.data(), row.second_moment.size() * 4);
    *updates = row.row_updates;
  });
}

void ref_shard_powers(void* h, std::uint32_t table, float* b1p, float* b2p,
                      std::uint64_t* sequence) {
  auto& t = static_cast<Shard*>(h)->store.Table(table);
  *b1p = t.beta1_power; *b2p = t.beta2_power; *sequence = t.optimizer_sequence;
}

// PrepareFeature (batch_access.cpp:25-52); the prepared feature is retained in
// the shard so a later ref_shard_push can reduce against it (the ticket).
int ref_shard_prepare(void* h, std::uint32_t table, const eps_or_feature* f,
                      std::uint64_t* unique_slots, std::uint64_t* unique_count,
                      std::uint64_t* occurrence_to_unique, float* contribution) {
  return Guard([&] {
    auto* s = static_cast<Shard*>(h);
    auto in = Input(table, *f);
    detail::ValidateFeature(in, s->store);
    auto p = detail::PrepareFeature(std::move(in), s->store);
    std::copy(p.unique_slots.begin(), p.unique_slots.end(), unique_slots);
    *unique_count = p.unique_slots.size();
    std::copy(p.occurrence_to_unique.begin(), p.occurrence_to_unique.end(), occurrence_to_unique);
    std::copy(p.contribution.values.begin(), p.contribution.values.end(), contribution);
    s->prepared.push_back(std::move(p));
  });
}
void ref_shard_clear_prepared(void* h) { static_cast<Shard*>(h)->prepared.clear(); }

// Reduce the retained prepared features against `gradients` (one block per
// prepared feature, in preparation order) for `table`, in ReduceGradients'
// first-occurrence row order (batch_access.cpp:54-97).
int ref_shard_reduce(void* h, std::uint32_t table, const float* const* gradients,
                     std::uint64_t* row_keys, float* row_values, std::uint64_t* row_count) {
  return Guard([&] {
    auto* s = static_cast<Shard*>(h);
    std::vector<TensorBlock> g;
    for (std::size_t i = 0; i < s->prepared.size(); ++i) {
      const auto& c = s->prepared[i].contribution;
      g.push_back({c.feature, c.shape, {gradients[i], gradients[i] + c.values.size()}});
    }
    auto reduced = detail::ReduceGradients(s->prepared, g, s->store);
    auto it = reduced.find(table);
    *row_count = 0;
    if (it == reduced.end()) return;
    const auto& r = it->second;
    for (std::size_t i = 0; i < r.rows.size(); ++i) row_keys[i] = r.rows[i].key;
    std::copy(r.values.begin(), r.values.end(), row_values);
    *row_count = r.rows.size();
  });
}

// One Push on CPU-owned rows (service.cpp:256-267,324-325): ReduceGradients,
// ValidateLazyAdam per table, then ApplyLazyAdam per table.  Clears the ticket.
int ref_shard_push(void* h, const float* const* gradients) {
  return Guard([&] {
    auto* s = static_cast<Shard*>(h);
    std::vector<TensorBlock> g;
    for (std::size_t i = 0; i < s->prepared.size(); ++i) {
      const auto& c = s->prepared[i].contribution;
      g.push_back({c.feature, c.shape, {gradients[i], gradients[i] + c.values.size()}});
    }
    auto reduced = detail::ReduceGradients(s->prepared, g, s->store);
    for (const auto& [table, rows] : reduced) detail::ValidateLazyAdam(s->store.Table(table), rows);
    for (const auto& [table, rows] : reduced) detail::ApplyLazyAdam(s->store.Table(table), rows);
    s->prepared.clear();
  });
}

// ExpandCompactGradients (compact_gradients.cpp:27-39) on one table's packet.
int ref_expand_compact(std::uint32_t table, std::uint64_t rows, const std::uint64_t* row_keys,
                       std::uint32_t dim, const float* source_values,
                       std::uint64_t source_value_count, const std::uint64_t* row_offsets,
                       const std::uint64_t* source_rows, const float* scales,
                       std::uint64_t references, float* out) {
  return Guard([&] {
    CompactGradients p{{}, dim, {source_values, source_values + source_value_count},
                       {row_offsets, row_offsets + rows + 1},
                       {source_rows, source_rows + references}, {scales, scales + references}};
    for (std::uint64_t r = 0; r < rows; ++r) p.rows.push_back({table, row_keys[r]});
    auto e = ExpandCompactGradients(p);
    std::copy(e.values.begin(), e.values.end(), out);
  });
}

// BuildCompactGradients (compact_gradients.cpp:43-72) over the retained
// prepared features of the shard.
int ref_shard_build_compact(void* h, std::uint32_t table, const float* const* gradients,
                            const std::uint64_t* row_keys, std::uint64_t rows,
                            float* source_values, std::uint64_t* source_value_count,
                            std::uint64_t* row_offsets, std::uint64_t* source_rows,
                            float* scales, std::uint64_t* references) {
  return Guard([&] {
    auto* s = static_cast<Shard*>(h);
    std::vector<TensorBlock> g;
    for (std::size_t i = 0; i < s->prepared.size(); ++i) {
      const auto& c = s->prepared[i].contribution;
      g.push_back({c.feature, c.shape, {gradients[i], gradients[i] + c.values.size()}});
    }
    std::vector<RowKey> targets;
    for (std::uint64_t r = 0; r < rows; ++r) targets.push_back({table, row_keys[r]});
    const auto dim = s->store.Table(table).definition.dimension;
    auto p = detail::BuildCompactGradients(s->prepared, g, targets, dim);
    std::copy(p.source_values.begin(), p.source_values.end(), source_values);
    *source_value_count = p.source_values.size();
    std::copy(p.row_offsets.begin(), p.row_offsets.end(), row_offsets);
    std::copy(p.source_rows.begin(), p.source_rows.end(), source_rows);
    std::copy(p.scales.begin(), p.scales.end(), scales);
    *references = p.source_rows.size();
  });
}

// ---- HostCacheBackend (src/cache/host_backend.cpp) ----
void* ref_host_backend_create(std::uint32_t agent, std::uint64_t bytes) {
  return new HostCacheBackend(agent, bytes);
}
void ref_host_backend_destroy(void* h) { delete static_cast<HostCacheBackend*>(h); }

int ref_host_backend_define(void* h, const eps_or_table_def* t) {
  return Guard([&] { Take(static_cast<HostCacheBackend*>(h)->Define(Definition(*t))); });
}

// Load rows (w|m|v packed per row) and return the assigned slots.
int ref_host_backend_load(void* h, std::uint32_t table, std::uint32_t dim,
                          const std::uint64_t* keys, std::uint64_t rows, const float* packed,
                          const std::uint64_t* updates, std::uint64_t* slots) {
  return Guard([&] {
    MigrationPlan plan{"load", 0, {}, Placement::gpu, 0};
    std::vector<RowState> states;
    for (std::uint64_t i = 0; i < rows; ++i) {
      const float* p = packed + i * dim * 3;
      states.push_back({{table, keys[i]}, {p, p + dim}, {p + dim, p + 2 * dim},
                        {p + 2 * dim, p + 3 * dim}, updates[i]});
      plan.rows.push_back({{table, keys[i]}, 0, Placement::loading, 0, 1, 0});
    }
    auto located = Take(static_cast<HostCacheBackend*>(h)->Load(plan, states));
    for (std::uint64_t i = 0; i < rows; ++i) slots[i] = located[i].slot;
  });
}

int ref_host_backend_apply(void* h, std::uint32_t table, float learning_rate, float b1p,
                           float b2p, const std::uint64_t* keys, std::uint64_t rows,
                           const float* values, std::uint32_t dim) {
  return Guard([&] {
    UpdateContext c{{"ref", 0, 0, Phase::push}, 0, table, 0, learning_rate, b1p, b2p};
    RowGradients g;
    for (std::uint64_t i = 0; i < rows; ++i) g.rows.push_back({table, keys[i]});
    g.values.assign(values, values + rows * dim);
    Take(static_cast<HostCacheBackend*>(h)->ApplyHost(c, std::move(g)));
  });
}

int ref_host_backend_read(void* h, std::uint32_t table, std::uint32_t dim,
                          const std::uint64_t* keys, const std::uint64_t* slots,
                          std::uint64_t rows, float* packed, std::uint64_t* updates) {
  return Guard([&] {
    MigrationPlan plan{"read", 0, {}, Placement::cpu, 0};
    for (std::uint64_t i = 0; i < rows; ++i)
      plan.rows.push_back({{table, keys[i]}, 0, Placement::gpu, 0, 1, slots[i]});
    auto states = Take(static_cast<HostCacheBackend*>(h)->ReadBack(plan));
    for (std::uint64_t i = 0; i < rows; ++i) {
      float* p = packed + i * dim * 3;
      std::copy(states[i].weights.begin(), states[i].weights.end(), p);
      std::copy(states[i].first_moment.begin(), states[i].first_moment.end(), p + dim);
      std::copy(states[i].second_moment.begin(), states[i].second_moment.end(), p + 2 * dim);
      updates[i] = states[i].row_updates;
    }
  });
}
}  // extern "C"
