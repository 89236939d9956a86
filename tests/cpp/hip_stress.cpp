// hip_stress.cpp -- concurrent checked reads of one eps::HipCacheBackend, on a GPU.
//
// The scenario of the reference's tests/cuda_stress.cpp:35-105: one table of
// `rows` rows (default 262,144) of dimension `dim` (128) whose weights have
// the closed form 0.001 * (key % 17 + d % 13); `workers` caller threads (8)
// each issue `batches` (64) GatherHost calls of 4,096 keys in sum-pooled bags
// of 16, 95% of the keys drawn from the first 32,768 rows, and every pooled
// value is compared with the sequential fp32 sum of the closed form.
// Requires a maximum absolute error of 0 and MemoryStats unchanged by the
// reads.
//
// Then the job-queue rule of the backend (at most 128 operations wait,
// src/cuda/cache_backend.cu:222; src/common/executor.hpp): behind one gather
// of 131,072 keys, a burst of 1,000 MemoryStats calls from one thread must see
// refusals with capacity_exceeded, every accepted call must resolve to the
// same statistics, and the backend must serve again afterwards.
//
// Prints one JSON line: the read phase's wall time (including the checks, as
// the reference reports it) and the queue burst's counts.  Any failure prints
// FAIL and exits 1.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <iostream>
#include <mutex>
#include <random>
#include <stdexcept>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "eps/hip_cache_backend.hpp"

using namespace eps;

namespace {

constexpr std::uint32_t kKeysPerBatch = 4096;
constexpr std::uint64_t kBag = 16;

void Check(bool ok, const std::string& why) {
  if (!ok) throw std::runtime_error(why);
}

template <typename T>
T Take(std::future<Result<T>> f) {
  auto r = f.get();
  if (auto e = std::get_if<Error>(&r)) throw std::runtime_error("backend error: " + e->message);
  return std::get<T>(std::move(r));
}

float Weight(Key key, std::uint32_t d) { return 0.001f * (float(key % 17) + float(d % 13)); }

struct Query {
  std::vector<AgentWork> work;
  std::vector<FeatureInput> layouts;
};

// One feature of `keys` keys in bags of 16; the work lists each distinct row
// once, in first-occurrence order.
Query MakeQuery(const std::vector<LocatedRow>& rows, std::uint32_t keys, std::mt19937_64& random) {
  FeatureInput layout{1, 0, Pooling::sum, {}, {0}, {}};
  AgentWork work{0, AccessRoute::resident_gpu, 0, {}, {}, {}};
  std::unordered_map<Key, std::uint64_t> unique;
  unique.reserve(keys);
  for (std::uint32_t i = 0; i < keys; ++i) {
    const std::size_t hot = std::min<std::size_t>(rows.size(), 32768);
    const std::size_t limit = random() % 100 < 95 ? hot : rows.size();
    const LocatedRow& row = rows[random() % limit];
    layout.keys.push_back(row.row.key);
    auto [it, added] = unique.try_emplace(row.row.key, work.rows.size());
    if (added) work.rows.push_back(row);
    work.occurrence_to_unique.push_back(it->second);
    if ((i + 1) % kBag == 0) {
      layout.offsets.push_back(i + 1);
      layout.valid_lengths.push_back(kBag);
    }
  }
  return {{std::move(work)}, {std::move(layout)}};
}

// Largest |expected - actual| over one result; expected is the sequential
// fp32 sum of the closed-form weights of each bag.
float MaxError(const Query& q, const std::vector<TensorBlock>& result, std::uint32_t dim) {
  Check(result.size() == 1, "stress result count");
  const FeatureInput& in = q.layouts[0];
  const std::uint64_t bags = in.valid_lengths.size();
  Check(result[0].values.size() == bags * dim, "stress output shape");
  float worst = 0.f;
  for (std::uint64_t bag = 0; bag < bags; ++bag)
    for (std::uint32_t d = 0; d < dim; ++d) {
      float expected = 0.f;
      for (std::uint64_t i = in.offsets[bag]; i < in.offsets[bag + 1]; ++i) expected += Weight(in.keys[i], d);
      const float actual = result[0].values[bag * dim + d];
      Check(std::isfinite(actual), "non-finite stress result");
      worst = std::max(worst, std::fabs(expected - actual));
    }
  return worst;
}

int Run(std::uint64_t rows, std::uint32_t dim, int workers, int batches) {
  Check(rows >= 32768 && rows <= (1u << 20) && dim >= 1 && dim <= 512 && workers >= 1 && workers <= 32 &&
            batches >= 1 && batches <= 1000,
        "invalid stress dimensions");
  HipCacheOptions options;
  options.rows_per_table = rows;
  options.state_bytes = rows * (std::uint64_t(dim) * 12 + 8);
  options.transfer_bytes = 64ull << 20;
  HipCacheBackend backend(options);
  Take(backend.Define({1, dim, 1, 1, {0.01f, 0.9f, 0.999f, 1e-8f, 0.9f, 0.999f}, 0.f, 0.f, 42}));

  std::vector<LocatedRow> located;
  located.reserve(rows);
  const std::uint64_t chunk = 4096;
  for (std::uint64_t begin = 0; begin < rows; begin += chunk) {
    MigrationPlan plan{"stress-load", 0, {}, Placement::gpu, 0};
    std::vector<RowState> states;
    for (std::uint64_t i = begin; i < std::min(rows, begin + chunk); ++i) {
      RowState r{{1, i + 1}, std::vector<float>(dim), std::vector<float>(dim, 0.f), std::vector<float>(dim, 0.f), 0};
      for (std::uint32_t d = 0; d < dim; ++d) r.weights[d] = Weight(i + 1, d);
      plan.rows.push_back({r.row, 0, Placement::loading, 0, 1, 0});
      states.push_back(std::move(r));
    }
    auto got = Take(backend.Load(std::move(plan), std::move(states)));
    located.insert(located.end(), got.begin(), got.end());
  }

  std::mt19937_64 warm_random(1);
  Query warm = MakeQuery(located, kKeysPerBatch, warm_random);
  Check(MaxError(warm, Take(backend.GatherHost(warm.work, warm.layouts)), dim) == 0.f, "warm-up gather");
  const HipMemoryStats before = Take(backend.MemoryStats());

  std::atomic<bool> go{false};
  std::atomic<int> ready{0};
  std::mutex mutex;
  std::string failure;
  float worst = 0.f;
  std::vector<std::thread> callers;
  for (int w = 0; w < workers; ++w)
    callers.emplace_back([&, w] {
      ++ready;
      while (!go.load()) std::this_thread::yield();
      try {
        std::mt19937_64 random(42 + w);
        float local = 0.f;
        for (int b = 0; b < batches; ++b) {
          Query q = MakeQuery(located, kKeysPerBatch, random);
          local = std::max(local, MaxError(q, Take(backend.GatherHost(q.work, q.layouts)), dim));
        }
        std::lock_guard<std::mutex> lock(mutex);
        worst = std::max(worst, local);
      } catch (const std::exception& e) {
        std::lock_guard<std::mutex> lock(mutex);
        failure = e.what();
      }
    });
  while (ready.load() != workers) std::this_thread::yield();
  const auto start = std::chrono::steady_clock::now();
  go = true;
  for (auto& t : callers) t.join();
  const double seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count();
  Check(failure.empty(), failure);
  Check(worst == 0.f, "stress gather differs from the closed form by " + std::to_string(worst));
  const HipMemoryStats after = Take(backend.MemoryStats());
  Check(before == after, "checked reads changed the backend's device memory statistics");

  // Queue rule: a long gather first, then a burst that outruns the worker.
  std::mt19937_64 big_random(7);
  Query big = MakeQuery(located, 131072, big_random);
  auto long_gather = backend.GatherHost(big.work, big.layouts);
  std::vector<std::future<Result<HipMemoryStats>>> burst;
  burst.reserve(1000);
  for (int i = 0; i < 1000; ++i) burst.push_back(backend.MemoryStats());
  int refused = 0, served = 0;
  for (auto& f : burst) {
    auto r = f.get();
    if (auto e = std::get_if<Error>(&r)) {
      Check(e->code == Error::Code::capacity_exceeded, "burst refusal code: " + e->message);
      ++refused;
    } else {
      Check(std::get<HipMemoryStats>(r) == after, "burst statistics");
      ++served;
    }
  }
  Check(MaxError(big, Take(std::move(long_gather)), dim) == 0.f, "long gather");
  Check(refused > 0, "a burst of 1,000 calls behind a long gather was never refused");
  Check(served >= 128, "fewer than 128 queued calls were served");
  Check(Take(backend.MemoryStats()) == after, "backend serves after the burst");
  Check(MaxError(warm, Take(backend.GatherHost(warm.work, warm.layouts)), dim) == 0.f, "gather after the burst");

  std::printf(
      "{\"test\": \"hip_checked_read_stress\", \"rows\": %llu, \"dimension\": %u, \"workers\": %d, "
      "\"checked_batches\": %d, \"key_occurrences\": %llu, \"maximum_absolute_error\": %g, "
      "\"backend_state_bytes\": %llu, \"backend_staging_bytes\": %llu, "
      "\"wall_seconds_including_reference_checks\": %.4f, \"queue_burst\": 1000, \"queue_refused\": %d, "
      "\"queue_served\": %d}\n",
      (unsigned long long)rows, dim, workers, workers * batches,
      (unsigned long long)workers * batches * kKeysPerBatch, double(worst),
      (unsigned long long)after.resident_state_bytes, (unsigned long long)after.staging_device_bytes, seconds,
      refused, served);
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    const std::uint64_t rows = argc > 1 ? std::stoull(argv[1]) : 262144;
    const std::uint32_t dim = argc > 2 ? std::stoul(argv[2]) : 128;
    const int workers = argc > 3 ? std::stoi(argv[3]) : 8;
    const int batches = argc > 4 ? std::stoi(argv[4]) : 64;
    return Run(rows, dim, workers, batches);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "FAIL hip stress: %s\n", e.what());
    return 1;
  }
}
