// Shared by the C++ self-checks under tests/cpp: a failure counter in the
// style of the reference's bench/bench.cc:35-43, the repo's seeded generator
// and the normwise error of the parity bar.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <vector>

static int failures = 0;
#define CHECK(cond, ...)                      \
  do {                                        \
    if (!(cond)) {                            \
      ++failures;                             \
      std::printf("FAIL %d: ", __LINE__);     \
      std::printf(__VA_ARGS__);               \
      std::printf("\n");                      \
    }                                         \
  } while (0)

// splitmix64 -> Box-Muller, the repo's generator (molot_amd/synth.py)
struct Rng {
  uint64_t s, i = 0;
  explicit Rng(uint64_t seed) : s(seed) {}
  uint64_t next() {
    uint64_t z = s + (++i) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  void normal(std::vector<float>& v) {
    for (size_t k = 0; k < v.size(); k += 2) {
      const double u1 = ((double)(next() >> 11) + 1.0) / 9007199254740992.0;
      const double u2 = (double)(next() >> 11) / 9007199254740992.0;
      const double r = std::sqrt(-2.0 * std::log(u1));
      v[k] = (float)(r * std::cos(2 * M_PI * u2));
      if (k + 1 < v.size()) v[k + 1] = (float)(r * std::sin(2 * M_PI * u2));
    }
  }
};

static double normwise(const std::vector<float>& got, const std::vector<float>& ref) {
  double num = 0, den = 0;
  for (size_t i = 0; i < ref.size(); ++i) {
    num = std::fmax(num, std::fabs((double)got[i] - ref[i]));
    den = std::fmax(den, std::fabs((double)ref[i]));
  }
  return den > 0 ? num / den : num;
}

