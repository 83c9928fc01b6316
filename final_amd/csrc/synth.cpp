// Seeded synthetic workload generator (host).  See include/moe_synth.h.
#include "moe_synth.h"

#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

namespace {

int g_threads = 0;

inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

// Normal pair number p of (seed, stream): Box-Muller on two 53-bit uniforms,
// u1 in (0,1], u2 in [0,1), evaluated in double and rounded once to float.
inline void normal_pair(uint64_t key, uint64_t p, double out[2]) {
  const uint64_t h1 = mix64(key + 2 * p + 0x632be59bd9b4e019ULL);
  const uint64_t h2 = mix64(key + 2 * p + 1 + 0x632be59bd9b4e019ULL);
  const double u1 = (double)((h1 >> 11) + 1) * 0x1.0p-53;
  const double u2 = (double)(h2 >> 11) * 0x1.0p-53;
  const double r = std::sqrt(-2.0 * std::log(u1));
  const double a = 6.283185307179586476925286766559 * u2;
  out[0] = r * std::cos(a);
  out[1] = r * std::sin(a);
}

void fill_range(uint64_t key, float sd, uint64_t first, float *out, size_t n) {
  size_t i = 0;
  while (i < n) {
    const uint64_t g = first + i;  // global element index
    double z[2];
    normal_pair(key, g >> 1, z);
    out[i] = (float)((double)sd * z[g & 1]);
    ++i;
    if ((g & 1) == 0 && i < n) {
      out[i] = (float)((double)sd * z[1]);
      ++i;
    }
  }
}

}  // namespace

extern "C" {

void moe_synth_set_threads(int n) { g_threads = n; }

void moe_synth_normal(uint64_t seed, uint64_t stream, float std_dev,
                      uint64_t first, float *out, size_t n) {
  if (!out || n == 0) return;
  const uint64_t key = mix64(mix64(seed) ^ (stream * 0x9E3779B97F4A7C15ULL));
  unsigned hw = std::thread::hardware_concurrency();
  int nt = g_threads > 0 ? g_threads : (int)std::min(hw ? hw : 1u, 16u);
  const size_t chunk = 1 << 20;
  if (nt <= 1 || n < 2 * chunk) {
    fill_range(key, std_dev, first, out, n);
    return;
  }
  nt = (int)std::min<size_t>((size_t)nt, (n + chunk - 1) / chunk);
  std::vector<std::thread> pool;
  const size_t per = ((n / (size_t)nt) + 1) & ~(size_t)1;  // even split points
  for (int t = 0; t < nt; ++t) {
    const size_t lo = std::min(n, per * (size_t)t);
    const size_t hi = (t == nt - 1) ? n : std::min(n, per * (size_t)(t + 1));
    if (hi <= lo) continue;
    pool.emplace_back(fill_range, key, std_dev, first + lo, out + lo, hi - lo);
  }
  for (auto &th : pool) th.join();
}

uint64_t moe_synth_stream_gate(void) { return 0; }
uint64_t moe_synth_stream_bias(void) { return 1; }
uint64_t moe_synth_stream_w1(int e) { return 2 + 3 * (uint64_t)e; }
uint64_t moe_synth_stream_w3(int e) { return 3 + 3 * (uint64_t)e; }
uint64_t moe_synth_stream_w2(int e) { return 4 + 3 * (uint64_t)e; }
uint64_t moe_synth_stream_x(int num_experts) { return 2 + 3 * (uint64_t)num_experts; }

}  // extern "C"
