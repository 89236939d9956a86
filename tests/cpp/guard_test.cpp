// Host unit test of csrc/guard.hpp: the overflow guard's bounds and the range
// checks of sorted keys and reference words, the same functions the update
// kernels evaluate on the device.
//
//  * soundness of the gradient bound: for random fp32 sequences, the
//    sequential sum of (x * scale) products (each rounded, as the reference's
//    ReduceGradients does, src/access/batch_access.cpp:73-93) never exceeds G;
//  * soundness of the table check: whenever GuardTableSafe says a table is
//    safe, one fp32 Adam step (src/update/lazy_adam.cpp:31-35) of any state
//    inside the bounds and any gradient inside G stays finite and below the
//    limit; near the limit both answers occur, and each of the three bounds
//    decides alone on a case built for it.  (The check is deliberately loose:
//    |w'| is bounded with sqrt(v') dropped, so the gradient's share of the m
//    bound never decides an outcome that the v bound leaves safe.)
//  * key and reference decode: boundaries of every field.
// Exits non-zero on the first failure.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <limits>

#include "guard.hpp"

using namespace eps_hip;

namespace {

int failures = 0;
#define EXPECT(cond, ...)                                   \
  do {                                                      \
    if (!(cond)) {                                          \
      std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
      std::fprintf(stderr, __VA_ARGS__);                    \
      std::fprintf(stderr, "\n");                           \
      if (++failures > 20) std::exit(1);                    \
    }                                                       \
  } while (0)

struct Rng {
  uint64_t s;
  uint64_t next() {  // SplitMix64
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  }
  double uniform() { return double(next() >> 11) * 0x1.0p-53; }
  double log_uniform(double lo, double hi) { return std::pow(10.0, lo + (hi - lo) * uniform()); }
  double sign() { return (next() & 1) ? 1.0 : -1.0; }
};

void TestGradBound(Rng& rng) {
  int checked = 0;
  for (int trial = 0; trial < 400; ++trial) {
    const int n = 1 + int(rng.next() % (trial < 200 ? 64 : 5000));
    const float max_grad = float(rng.log_uniform(-8, 30));
    const float max_scale = float(rng.log_uniform(-3, 2));
    float sum = 0.f, seen_g = 0.f, seen_s = 0.f;
    // Worst case: same-sign terms at the maxima, or random ones.
    const bool worst = trial % 3 == 0;
    for (int i = 0; i < n; ++i) {
      const float x = worst ? max_grad : float(rng.sign() * rng.uniform() * max_grad);
      const float s = worst ? max_scale : float(rng.uniform() * max_scale);
      const volatile float product = x * s;
      sum = sum + product;
      seen_g = std::fmax(seen_g, std::fabs(x));
      seen_s = std::fmax(seen_s, s);
    }
    if (!std::isfinite(sum)) continue;
    const double G = GuardGradBound(seen_g, seen_s, double(n));
    EXPECT(std::fabs(double(sum)) <= G, "gradient bound %g below |sum| %g (n %d)", G, double(sum), n);
    ++checked;
  }
  // A long same-sign run whose every addition rounds up: 2^22 additions of
  // 0.69f end 5.4% above the exact sum, beyond a plain 1% widening, so the
  // rounding growth term must cover it.
  float sum = 0.f;
  const int n = 1 << 22;
  for (int i = 0; i < n; ++i) sum = sum + 0.69f;
  EXPECT(double(sum) > 1.05 * double(0.69f) * n, "long run did not round up (%g)", double(sum));
  EXPECT(double(sum) <= GuardGradBound(0.69f, 1.0, n), "long run %g", double(sum));
  EXPECT(checked > 300, "only %d finite gradient cases", checked);
  // Scales below 1 are bounded by 1 (the bound never shrinks below max|g| * refs).
  EXPECT(GuardGradBound(2.0, 0.25, 3.0) >= 6.0, "scale floor");
}

// One fp32 Adam element exactly as the update kernels compute it.
void AdamStep(float b1, float b2, float lr, float eps, float g, float& w, float& m, float& v) {
  const float omb1 = 1.0f - b1, omb2 = 1.0f - b2;
  const volatile float mn = b1 * m + omb1 * g;
  const volatile float t = omb2 * g;
  const volatile float vn = b2 * v + t * g;
  const volatile float den = std::sqrt(float(vn)) + eps;
  const volatile float step = lr * mn;
  w = w - step / den;
  m = mn;
  v = vn;
}

void TestTableSafe(Rng& rng) {
  int safe = 0, unsafe = 0;
  for (int trial = 0; trial < 200000; ++trial) {
    const float b1 = float(0.5 + 0.499 * rng.uniform());
    const float b2 = float(0.9 + 0.0999 * rng.uniform());
    const float lr = float(rng.log_uniform(-6, 0));
    const float eps = float(rng.log_uniform(-10, -3));
    // Magnitudes concentrated near the limit so both answers occur.
    const float W = float(rng.log_uniform(0, 30.5));
    const float M = float(rng.log_uniform(10, 30));
    const float V = float(rng.log_uniform(0, 30.5));
    const float Gf = float(rng.log_uniform(0, 16));
    const double G = GuardGradBound(Gf, 1.0, 1.0);
    const bool ok = GuardTableSafe(b1, b2, lr, eps, W, M, V, G);
    (ok ? safe : unsafe)++;
    if (!ok) continue;
    // Any state inside the bounds: the extremes and a random point.
    for (int corner = 0; corner < 3; ++corner) {
      float w = corner == 2 ? float(rng.sign() * rng.uniform() * W) : float(corner ? W : -W);
      float m = corner == 2 ? float(rng.sign() * rng.uniform() * M) : float(corner ? M : -M);
      float v = corner == 2 ? float(rng.uniform() * V) : V;
      const float g = corner == 2 ? float(rng.sign() * rng.uniform() * Gf) : float(corner ? Gf : -Gf);
      AdamStep(b1, b2, lr, eps, g, w, m, v);
      const bool finite = std::isfinite(w) && std::isfinite(m) && std::isfinite(v);
      EXPECT(finite && std::fabs(w) < kGuardLimit && std::fabs(m) < kGuardLimit && v < kGuardLimit,
             "safe table overflowed: b1 %g b2 %g lr %g eps %g W %g M %g V %g G %g -> w %g m %g v %g",
             b1, b2, lr, eps, W, M, V, Gf, w, m, v);
    }
  }
  EXPECT(safe > 1000 && unsafe > 1000, "safe %d unsafe %d: the sampler misses one side", safe, unsafe);
  // The three bounds each decide on their own.
  EXPECT(GuardTableSafe(0.9, 0.999, 1e-3, 1e-8, 0, 0, 0, 1.0), "small values");
  EXPECT(!GuardTableSafe(0.9, 0.999, 1e-3, 1e-8, 0, 2e30, 0, 0), "m bound");
  EXPECT(!GuardTableSafe(0.9, 0.999, 1e-3, 1e-8, 0, 0, 2e30, 0), "v bound");
  EXPECT(!GuardTableSafe(0.9, 0.999, 1e-3, 1e-8, 0.995e30, 0, 0, 0), "w bound (widening)");
  EXPECT(!GuardTableSafe(0.9, 0.999, 1e-3, 1e-8, 0, 1e26, 0, 0), "w bound through lr*m/eps");
  EXPECT(GuardTableSafe(0.9, 0.999, 1e-3, 1e-8, 0, 1e20, 0, 0), "w bound through lr*m/eps (small)");
  EXPECT(!GuardTableSafe(0.9, 0.999, 1e-3, 0.0, 0, 0, 0, 0), "eps 0");
  EXPECT(!GuardTableSafe(0.9, 0.999, 1e-3, 1e-8, 0, 0, 0, 1e17), "gradient squared in v");
  EXPECT(GuardTableSafe(0.9, 0.999, 1e-3, 1e-8, 0, 0, 0, 1e16), "gradient squared in v (small)");
}

void TestDecode() {
  // row_bits 20: key index above, slot below.
  const uint32_t rb = 20;
  KeyParts k = SplitKey((3u << rb) | 5u, rb);
  EXPECT(k.table == 3 && k.slot == 5, "split key");
  EXPECT(!KeyInRange(k, 3, 100), "table index == tables");
  EXPECT(KeyInRange(k, 4, 6), "in range");
  EXPECT(!KeyInRange(k, 4, 5), "slot == rows");
  k = SplitKey((1u << rb) - 1u, rb);
  EXPECT(k.table == 0 && k.slot == (1u << rb) - 1u, "largest slot");
  EXPECT(KeyInRange(k, 1, 1u << rb) && !KeyInRange(k, 1, (1u << rb) - 1u), "largest slot bounds");
  k = SplitKey(0xffffffffu, 32);
  EXPECT(k.table == 0 && k.slot == 0xffffffffu, "32 row bits");
  k = SplitKey(0xffffffffu, 31);
  EXPECT(k.table == 1 && k.slot == 0x7fffffffu, "31 row bits");
  // Reference words: scale bits above, feature and gradient row below.
  const uint64_t word = (uint64_t(0x3f800000u) << 32) | (uint64_t(31) << 27) | ((1u << 27) - 1u);
  RefParts r = SplitRef(word);
  EXPECT(r.feature == 31 && r.row == (1u << 27) - 1u, "split ref");
  EXPECT(!RefInRange(r, 31, 1ull << 27), "feature == features");
  EXPECT(RefInRange(r, 32, 1ull << 27), "feature and row in range");
  EXPECT(!RefInRange(r, 32, (1ull << 27) - 1), "row == rows");
  r = SplitRef((uint64_t(0xffffffffu) << 32) | 7u);
  EXPECT(r.feature == 0 && r.row == 7, "scale bits do not leak into the reference");
}

}  // namespace

int main() {
  Rng rng{0x5eed5eedull};
  TestGradBound(rng);
  TestTableSafe(rng);
  TestDecode();
  if (failures) {
    std::fprintf(stderr, "%d failure(s)\n", failures);
    return 1;
  }
  std::printf("guard_test: ok\n");
  return 0;
}
