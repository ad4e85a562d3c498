// Known-answer vectors of the random-number calls generate_speculative and
// generate_advanced make (layer.cpp:1249, 1369-1371, 1394, 1493-1498,
// 1596-1597), produced by the C++ standard library itself: std::mt19937
// outputs, std::uniform_real_distribution<float>(0, 1) draws,
// std::generate_canonical<double, 53> draws and std::discrete_distribution
// <size_t> draws over double weights, interleaved as the speculative loop
// interleaves them.  Output: JSON on stdout (make_mt19937_kat.sh).
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

static uint32_t fbits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
static uint64_t dbits(double d) { uint64_t u; std::memcpy(&u, &d, 8); return u; }

int main() {
  std::printf("{\n");
  // raw outputs
  std::printf("  \"raw\": [\n");
  const uint32_t seeds[] = {0u, 1u, 5489u, 42u, 4294967295u};
  for (int si = 0; si < 5; ++si) {
    std::mt19937 g(seeds[si]);
    std::printf("    {\"seed\": %u, \"out\": [", seeds[si]);
    for (int i = 0; i < 1300; ++i) {
      const uint32_t v = g();
      if (i < 8 || i == 623 || i == 624 || i == 1247 || i == 1248 || i == 1299)
        std::printf("%s[%d, %u]", (i ? ", " : ""), i, v);
    }
    std::printf("]}%s\n", si < 4 ? "," : "");
  }
  std::printf("  ],\n");
  {
    std::mt19937 d;
    for (int i = 1; i < 10000; ++i) d();
    std::printf("  \"default_10000th\": %u,\n", (unsigned)d());
  }
  // a stream of mixed draws: per step kind 0 = uniform_real_distribution
  // <float>(0, 1), 1 = generate_canonical<double, 53>, 2 = discrete over w
  std::printf("  \"mixed\": [\n");
  const double w[] = {0.1, 0.0, 0.25, 0.05, 0.3, 0.0, 0.2, 0.1};
  for (int si = 0; si < 3; ++si) {
    const uint32_t seed = si == 0 ? 7u : si == 1 ? 1234u : 99999u;
    std::mt19937 g(seed);
    std::printf("    {\"seed\": %u, \"draws\": [", seed);
    for (int i = 0; i < 700; ++i) {
      const int kind = (i * 7 + si) % 3;
      if (i) std::printf(", ");
      if (kind == 0) {
        std::uniform_real_distribution<float> u(0.0f, 1.0f);
        std::printf("[0, %u]", fbits(u(g)));
      } else if (kind == 1) {
        std::printf("[1, %llu]", (unsigned long long)dbits(std::generate_canonical<double, 53>(g)));
      } else {
        std::discrete_distribution<size_t> dd(w, w + 8);
        std::printf("[2, %zu]", dd(g));
      }
    }
    std::printf("]}%s\n", si < 2 ? "," : "");
  }
  std::printf("  ],\n");
  // discrete_distribution boundaries: weights whose cumulative sums land on
  // the draws exactly are not reproducible by value, so check the lower_bound
  // rule on a wide vector with many draws
  std::printf("  \"discrete\": {\"seed\": 2024, \"weights\": [");
  std::vector<double> wv(50);
  for (int i = 0; i < 50; ++i) wv[i] = (i % 7 == 3) ? 0.0 : 1.0 / (1.0 + i % 11);
  for (int i = 0; i < 50; ++i) std::printf("%s%.17g", i ? ", " : "", wv[i]);
  std::printf("], \"draws\": [");
  std::mt19937 g(2024u);
  for (int i = 0; i < 400; ++i) {
    std::discrete_distribution<size_t> dd(wv.begin(), wv.end());
    std::printf("%s%zu", i ? ", " : "", dd(g));
  }
  std::printf("]}\n}\n");
  return 0;
}
