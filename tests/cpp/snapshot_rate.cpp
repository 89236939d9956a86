// snapshot_rate.cpp -- rate of HipCacheBackend::WriteSnapshot against the CPU
// writer (the oracle's restatement of src/store/snapshot.cpp:159-194) on the
// same rows, and the FNV-1a checksum alone (the format's byte-serial floor).
//
//   tests/cpp/_build/snapshot_rate [rows=1000000] [dim=64] [dir=/tmp]
//
// Prints one JSON line.  The files written are compared byte for byte and
// removed.  Rows are synthetic (deterministic per key), loaded into one table.
#include <unistd.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

#include "eps/hip_cache_backend.hpp"
#include "eps_oracle.h"

using namespace eps;
using Clock = std::chrono::steady_clock;

namespace {

template <typename T>
T Take(std::future<Result<T>> f) {
  auto r = f.get();
  if (auto e = std::get_if<Error>(&r)) {
    std::cerr << "backend error: " << e->message << "\n";
    std::exit(1);
  }
  return std::get<T>(std::move(r));
}

double Seconds(Clock::time_point a) { return std::chrono::duration<double>(Clock::now() - a).count(); }

std::string Bytes(const std::filesystem::path& p) {
  std::ifstream in(p, std::ios::binary);
  return {std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>()};
}

}  // namespace

int main(int argc, char** argv) {
  const std::uint64_t rows = argc > 1 ? std::stoull(argv[1]) : 1000000;
  const std::uint32_t dim = argc > 2 ? std::uint32_t(std::stoul(argv[2])) : 64;
  const std::filesystem::path dir =
      std::filesystem::path(argc > 3 ? argv[3] : "/tmp") / ("eps-snapshot-rate-" + std::to_string(::getpid()));
  std::filesystem::remove_all(dir);
  HipCacheOptions o;
  o.rows_per_table = rows;
  o.state_bytes = rows * (std::uint64_t(dim) * 12 + 8);
  o.transfer_bytes = 256ull << 20;
  HipCacheBackend gpu(o);
  TableDefinition d{1, dim, 1, 1, {0.01f, 0.9f, 0.999f, 1e-8f, 0.9f, 0.999f}, -0.05f, 0.05f, 3001};
  Take(gpu.Define(d));
  eps_or_table_def od{};
  od.id = 1; od.dim = dim; od.shard = 0; od.shard_count = 1;
  od.learning_rate = 0.01f; od.beta1 = 0.9f; od.beta2 = 0.999f; od.epsilon = 1e-8f;
  od.initial_beta1_power = 0.9f; od.initial_beta2_power = 0.999f;
  od.init_min = -0.05f; od.init_max = 0.05f; od.init_seed = 3001;
  eps_or_store* store = eps_or_create(&od);
  const std::uint64_t per_load = (o.transfer_bytes / (std::uint64_t(dim) * 12)) / 2;
  std::vector<Key> keys(rows);
  for (std::uint64_t i = 0; i < rows; ++i) keys[i] = (i * 2654435761ull) % (rows * 4) + 1;
  for (std::uint64_t b = 0; b < rows; b += per_load) {
    const std::uint64_t n = std::min(per_load, rows - b);
    MigrationPlan plan{"load", 0, {}, Placement::gpu, 0};
    std::vector<RowState> states;
    states.reserve(n);
    for (std::uint64_t i = b; i < b + n; ++i) {
      RowState r{{1, keys[i]}, std::vector<float>(dim), std::vector<float>(dim), std::vector<float>(dim), i % 7};
      for (std::uint32_t j = 0; j < dim; ++j) {
        r.weights[j] = 0.01f * std::sin(float(i + j));
        r.first_moment[j] = 1e-4f * float((i + j) % 5);
        r.second_moment[j] = 1e-6f * float((i * 3 + j) % 7);
      }
      eps_or_import(store, r.row.key, r.weights.data(), r.first_moment.data(), r.second_moment.data(),
                    r.row_updates);
      plan.rows.push_back({r.row, 0, Placement::loading, 0, 1, 0});
      states.push_back(std::move(r));
    }
    Take(gpu.Load(std::move(plan), std::move(states)));
  }
  const SnapshotIdentity id{"rate", 0, 1, 1};
  // The oracle store's clock is its initial one: write the same here.
  const std::vector<SnapshotTable> tables = {{d, 0, 0.9f, 0.999f, keys}};
  const auto gpu_file = dir / "gpu.bin", cpu_file = dir / "cpu.bin";
  auto t0 = Clock::now();
  const SnapshotFile f = Take(gpu.WriteSnapshot(gpu_file, id, tables, {}));
  const double gpu_s = Seconds(t0);
  t0 = Clock::now();
  eps_or_store* const stores[1] = {store};
  if (eps_or_snapshot_write(cpu_file.c_str(), "rate", 0, 1, 1, stores, 1) != 0) {
    std::cerr << "oracle writer failed: " << eps_or_last_error() << "\n";
    return 1;
  }
  const double cpu_s = Seconds(t0);
  const std::string a = Bytes(gpu_file), b = Bytes(cpu_file);
  t0 = Clock::now();
  const std::uint64_t h = eps_or_fnv1a(14695981039346656037ull, a.data(), a.size() - 8);
  const double hash_s = Seconds(t0);
  const bool same = a == b && h == f.checksum;
  std::filesystem::remove_all(dir);
  eps_or_destroy(store);
  std::printf("{\"rows\": %llu, \"dim\": %u, \"bytes\": %llu, \"identical\": %s, \"gpu_write_s\": %.4f, "
              "\"gpu_MBps\": %.1f, \"cpu_writer_s\": %.4f, \"cpu_MBps\": %.1f, \"fnv1a_only_s\": %.4f, "
              "\"fnv1a_MBps\": %.1f}\n",
              (unsigned long long)rows, dim, (unsigned long long)f.bytes, same ? "true" : "false", gpu_s,
              f.bytes / gpu_s / 1e6, cpu_s, f.bytes / cpu_s / 1e6, hash_s, f.bytes / hash_s / 1e6);
  return same ? 0 : 1;
}
