// snapshot_format_test.cpp -- the backend's snapshot encoder on the CPU.
//
// The encoder HipCacheBackend::WriteSnapshot drives (host/src/snapshot_writer.hpp:
// byte stream, FNV-1a, staging-file publication, field order) writes stores'
// content; the oracle's restatement of the reference's WriteSnapshot
// (src/store/snapshot.cpp:159-194) writes the same content; the files must be
// byte-identical.  Publication: an existing file is never replaced, and no
// staging file is left behind on success or failure.  The reader that
// HipCacheBackend::RestoreSnapshot streams files through (snapshot_reader.hpp)
// reads that file back to the oracle's rows and clocks, reads the reference's
// own format-1 fixture (tests/fixtures/snapshot-v1-unbounded.bin, copied to
// tests/golden/), and refuses a flipped byte, a truncation and trailing bytes
// as the reference's ReadSnapshot does.  No GPU is used.
#include <unistd.h>

#include <cmath>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

#include "eps_oracle.h"
#include "snapshot_reader.hpp"
#include "snapshot_writer.hpp"

using namespace eps;

namespace {

int g_checks = 0;
void Check(bool ok, const std::string& why) {
  ++g_checks;
  if (!ok) throw std::runtime_error(why);
}

std::string Bytes(const std::filesystem::path& p) {
  std::ifstream in(p, std::ios::binary);
  return {std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>()};
}

struct Table {
  eps_or_table_def def;
  TableDefinition definition;
  eps_or_store* store;
};

Table Make(std::uint32_t id, std::uint32_t dim, bool bounded) {
  Table t{};
  t.def.id = id; t.def.dim = dim; t.def.shard = 1; t.def.shard_count = 3;
  t.def.learning_rate = 0.05f; t.def.beta1 = 0.8f; t.def.beta2 = 0.99f; t.def.epsilon = 1e-7f;
  t.def.initial_beta1_power = 0.8f; t.def.initial_beta2_power = 0.99f;
  t.def.bounded = bounded; t.def.weight_min = -0.25f; t.def.weight_max = 0.5f;
  t.def.init_min = -0.1f; t.def.init_max = 0.1f; t.def.init_seed = 1234 + id;
  t.definition = {id, dim, 3, 7, {0.05f, 0.8f, 0.99f, 1e-7f, 0.8f, 0.99f}, -0.1f, 0.1f, 1234ull + id};
  if (bounded) t.definition.optimizer.weight_bounds = WeightBounds{-0.25f, 0.5f};
  t.store = eps_or_create(&t.def);
  Check(t.store != nullptr, "oracle store");
  return t;
}

}  // namespace

int main() {
  try {
    const auto dir = std::filesystem::temp_directory_path() / ("eps-format-" + std::to_string(::getpid()));
    std::filesystem::remove_all(dir);
    std::vector<Table> tables = {Make(4, 3, true), Make(2, 16, false)};
    // Rows: first-touch initialised ones and imported ones, keys of shard 1 of 3.
    for (auto& t : tables) {
      for (Key k = 1; k < 60; k += 3) Check(eps_or_ensure(t.store, k) >= 0, "ensure");
      std::vector<float> w(t.def.dim), m(t.def.dim), v(t.def.dim);
      for (std::uint32_t d = 0; d < t.def.dim; ++d) {
        w[d] = std::sin(float(d + t.def.id)); m[d] = -1e-3f * d; v[d] = 1e-20f * (d + 1);
      }
      Check(eps_or_import(t.store, 301, w.data(), m.data(), v.data(), 17) == 0, "import");
    }
    // One push advances the second table's clock (sequence 1, powers squared).
    const std::uint64_t keys[] = {4, 7, 4}, offsets[] = {0, 3}, lengths[] = {3};
    eps_or_feature f{keys, 3, offsets, lengths, nullptr, 1, 1 /* mean */, 0};
    std::vector<float> g(16, 0.125f);
    const float* grads[] = {g.data()};
    eps_or_store* stores[] = {tables[1].store};
    const std::uint32_t feature_store[] = {0};
    Check(eps_or_push(stores, 1, &f, feature_store, grads, 1) == 0, "oracle push");

    // The backend's encoder, fed as WriteSnapshot feeds it.
    const SnapshotIdentity id{"format-run", 1, 3, 7};
    const auto ours = dir / "ours" / "shard-1.bin";
    std::uint64_t checksum = 0;
    {
      hipbk::SnapshotWriter out(ours);
      hipbk::WriteSnapshotHeader(out, id, tables.size());
      for (const auto& t : tables) {
        SnapshotTable st{t.definition, 0, 0, 0, {}};
        eps_or_powers(t.store, &st.beta1_power, &st.beta2_power, &st.optimizer_sequence);
        const std::uint64_t rows = eps_or_row_count(t.store);
        for (std::uint64_t r = 0; r < rows; ++r) st.keys.push_back(eps_or_key_at(t.store, r));
        hipbk::WriteSnapshotTable(out, st);
        std::vector<float> wmv(3 * t.def.dim);
        for (std::size_t i = 0; i < st.keys.size(); ++i) {
          std::uint64_t updates = 0;
          Check(eps_or_read(t.store, st.keys[i], wmv.data(), wmv.data() + t.def.dim,
                            wmv.data() + 2 * t.def.dim, &updates) == 0,
                "oracle read");
          if (i % 2) {
            hipbk::WriteSnapshotRow(out, st.keys[i], updates, wmv.data(), t.def.dim);
          } else {  // the CPU-store form of a row
            RowState row{{t.def.id, st.keys[i]}, {wmv.begin(), wmv.begin() + t.def.dim},
                         {wmv.begin() + t.def.dim, wmv.begin() + 2 * t.def.dim},
                         {wmv.begin() + 2 * t.def.dim, wmv.end()}, updates};
            hipbk::WriteSnapshotRow(out, row);
          }
        }
      }
      checksum = out.Publish();
    }
    // The oracle writes the stores in the same order; the tables carry partition epoch 7.
    const auto theirs = dir / "oracle.bin";
    eps_or_store* const both[] = {tables[0].store, tables[1].store};
    Check(eps_or_snapshot_write(theirs.c_str(), "format-run", 1, 3, 7, both, 2) == 0, "oracle writer");
    Check(Bytes(ours) == Bytes(theirs), "encoder bytes differ from the oracle writer's");
    const std::string data = Bytes(ours);

    // The reader gives back every table clock and row of the stores.
    {
      hipbk::SnapshotReader in(ours);
      Check(in.version == 2 && in.run == id.run && in.shard == 1 && in.shard_count == 3 && in.epoch == 7 &&
                in.tables == 2,
            "reader identity");
      for (const auto& t : tables) {
        const auto header = in.NextTable();
        float b1 = 0, b2 = 0;
        std::uint64_t seq = 0;
        eps_or_powers(t.store, &b1, &b2, &seq);
        Check(header.definition == t.definition && header.optimizer_sequence == seq && header.beta1_power == b1 &&
                  header.beta2_power == b2 && header.rows == eps_or_row_count(t.store),
              "reader table header");
        std::vector<float> got(3 * t.def.dim), want(3 * t.def.dim);
        for (std::uint64_t r = 0; r < header.rows; ++r) {
          Key key = 0;
          std::uint64_t updates = 0, want_updates = 0;
          in.Row(t.def.dim, key, updates, got.data());
          Check(key == eps_or_key_at(t.store, r), "reader row order");
          Check(eps_or_read(t.store, key, want.data(), want.data() + t.def.dim, want.data() + 2 * t.def.dim,
                            &want_updates) == 0 &&
                    got == want && updates == want_updates,
                "reader row");
        }
      }
      in.Finish();
    }
    // The reference's format-1 fixture: run "legacy-unbounded", one row
    // [0.25, 0.25 | 0, 0 | 0, 0] (tests/fixtures/README.md of the reference).
    {
      const auto fixture = std::filesystem::canonical("/proc/self/exe").parent_path() / ".." / ".." / "golden" /
                           "snapshot-v1-unbounded.bin";
      hipbk::SnapshotReader in(fixture);
      Check(in.version == 1 && in.run == "legacy-unbounded" && in.tables == 1, "fixture identity");
      const auto header = in.NextTable();
      Check(header.rows == 1 && header.definition.dimension == 2 && !header.definition.optimizer.weight_bounds,
            "fixture table");
      std::vector<float> wmv(6);
      Key key = 0;
      std::uint64_t updates = 0;
      in.Row(2, key, updates, wmv.data());
      Check(wmv == std::vector<float>{0.25f, 0.25f, 0, 0, 0, 0}, "fixture row");
      in.Finish();
    }
    // Damaged files are refused: a flipped byte, a truncation, trailing bytes.
    auto refuses = [&](const std::string& bytes, Error::Code code, const char* what) {
      const auto bad = dir / "damaged.bin";
      std::filesystem::remove(bad);
      std::ofstream(bad, std::ios::binary) << bytes;
      bool refused = false;
      try {
        hipbk::SnapshotReader in(bad);
        for (std::uint64_t t = 0; t < in.tables; ++t) {
          const auto header = in.NextTable();
          std::vector<float> wmv(3 * header.definition.dimension);
          Key key;
          std::uint64_t updates;
          for (std::uint64_t r = 0; r < header.rows; ++r) in.Row(header.definition.dimension, key, updates, wmv.data());
        }
        in.Finish();
      } catch (const hipbk::Fault& e) {
        refused = e.error.code == code;
      }
      Check(refused, what);
    };
    std::string flipped = data;
    flipped[data.size() / 2] ^= 0x10;
    refuses(flipped, Error::Code::invalid_argument, "a flipped byte was accepted");
    refuses(data.substr(0, data.size() - 3), Error::Code::unavailable, "a truncated snapshot was accepted");
    refuses(data + "x", Error::Code::invalid_argument, "trailing bytes were accepted");
    Check(eps_or_fnv1a(14695981039346656037ull, data.data(), data.size() - 8) == checksum,
          "returned checksum");
    Check(!std::filesystem::exists(ours.string() + ".pending"), "staging file left after publish");

    // A published file is never replaced; the refused attempt leaves no staging file.
    bool refused = false;
    try {
      hipbk::SnapshotWriter again(ours);
      again.U64(1);
      again.Publish();
    } catch (const hipbk::Fault& e) {
      refused = e.error.code == Error::Code::unavailable;
    }
    Check(refused && Bytes(ours) == data && !std::filesystem::exists(ours.string() + ".pending"),
          "an existing snapshot was replaced");
    // A writer dropped before publication removes its staging file.
    { hipbk::SnapshotWriter dropped(dir / "dropped.bin"); dropped.U64(5); }
    Check(!std::filesystem::exists(dir / "dropped.bin") &&
              !std::filesystem::exists((dir / "dropped.bin").string() + ".pending"),
          "unpublished snapshot left files");
    for (auto& t : tables) eps_or_destroy(t.store);
    std::filesystem::remove_all(dir);
    std::cout << "PASS snapshot format: " << g_checks << " checks\n";
    return 0;
  } catch (const std::exception& e) {
    std::cerr << "FAIL snapshot format: " << e.what() << '\n';
    return 1;
  }
}
