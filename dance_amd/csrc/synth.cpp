// Deterministic synthetic workloads for the BASELINE configurations.
//
// Every row r of sub-stream `stream` draws from its own xoshiro256** generator
// seeded through splitmix64 from (seed, stream, r), so rows can be generated
// in parallel and any subset of rows can be regenerated alone. Centers use the
// reserved stream 0xC0DE. Normals come from the Box-Muller transform in double
// precision. Per row, the first draw picks the mixture component uniformly
// (next() % num_centers); the row is then c_k + sigma * eps with eps ~ N(0, I).
//   fp32: optionally L2-normalised in double, then rounded to fp32.
//   uint8: clip(floor(64 + 24 z + 0.5), 0, 255).
// num_centers = 0 draws x ~ N(0, I) directly (config 1).

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/dance_hip.h"

namespace {

inline uint64_t splitmix64(uint64_t& s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

struct Xoshiro {
  uint64_t s[4];
  Xoshiro(uint64_t seed, uint64_t stream, uint64_t row) {
    uint64_t sm = seed ^ (stream * 0xD1B54A32D192ED03ull) ^ ((row + 1) * 0x8CB92BA72F3D8DD7ull);
    for (auto& w : s) w = splitmix64(sm);
  }
  uint64_t next() {
    const uint64_t r = rotl(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return r;
  }
  double uniform() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }  // [0,1)
  // Box-Muller: a pair of independent normals.
  void normal2(double& z0, double& z1) {
    const double u1 = 1.0 - uniform();  // (0,1]
    const double u2 = uniform();
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double th = 6.283185307179586 * u2;
    z0 = r * std::cos(th);
    z1 = r * std::sin(th);
  }
  void normals(double* out, uint32_t n) {
    uint32_t i = 0;
    for (; i + 1 < n; i += 2) normal2(out[i], out[i + 1]);
    if (i < n) {
      double z1;
      normal2(out[i], z1);
    }
  }
};

constexpr uint64_t kCenterStream = 0xC0DEull;

std::vector<double> make_centers(uint64_t seed, uint32_t k, uint32_t dim) {
  std::vector<double> c((size_t)k * dim);
  for (uint32_t i = 0; i < k; ++i) {
    Xoshiro g(seed, kCenterStream, i);
    g.normals(&c[(size_t)i * dim], dim);
  }
  return c;
}

template <typename Fn>
void parallel_rows(uint32_t n, Fn&& fn) {
  unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (n < 4096) nt = 1;
  std::vector<std::thread> th;
  const uint32_t per = (n + nt - 1) / nt;
  for (unsigned t = 0; t < nt; ++t) {
    const uint32_t b = t * per, e = std::min(n, b + per);
    if (b >= e) break;
    th.emplace_back([=, &fn] {
      std::vector<double> buf;
      for (uint32_t r = b; r < e; ++r) fn(r, buf);
    });
  }
  for (auto& x : th) x.join();
}

void mixture_row(uint64_t seed, uint32_t stream, uint32_t r, uint32_t dim, uint32_t k, double sigma,
                 const std::vector<double>& centers, std::vector<double>& z) {
  Xoshiro g(seed, stream, r);
  z.resize(dim);
  if (k == 0) {
    g.normals(z.data(), dim);
    return;
  }
  const uint32_t comp = (uint32_t)(g.next() % k);
  g.normals(z.data(), dim);
  const double* c = &centers[(size_t)comp * dim];
  for (uint32_t e = 0; e < dim; ++e) z[e] = c[e] + sigma * z[e];
}

}  // namespace

extern "C" {

int dance_synth_f32(uint64_t seed, uint32_t stream, uint32_t num_points, uint32_t dim, uint32_t num_centers,
                    float sigma, int normalize, float* out) {
  if (out == nullptr || dim == 0 || stream == kCenterStream) return -1;
  const std::vector<double> centers = make_centers(seed, num_centers, dim);
  parallel_rows(num_points, [&](uint32_t r, std::vector<double>& z) {
    mixture_row(seed, stream, r, dim, num_centers, sigma, centers, z);
    double scale = 1.0;
    if (normalize) {
      double ss = 0;
      for (double v : z) ss += v * v;
      scale = ss > 0 ? 1.0 / std::sqrt(ss) : 1.0;
    }
    float* o = out + (size_t)r * dim;
    for (uint32_t e = 0; e < dim; ++e) o[e] = (float)(z[e] * scale);
  });
  return 0;
}

int dance_synth_u8(uint64_t seed, uint32_t stream, uint32_t num_points, uint32_t dim, uint32_t num_centers,
                   float sigma, uint8_t* out) {
  if (out == nullptr || dim == 0 || stream == kCenterStream) return -1;
  const std::vector<double> centers = make_centers(seed, num_centers, dim);
  parallel_rows(num_points, [&](uint32_t r, std::vector<double>& z) {
    mixture_row(seed, stream, r, dim, num_centers, sigma, centers, z);
    uint8_t* o = out + (size_t)r * dim;
    for (uint32_t e = 0; e < dim; ++e) {
      const double v = std::floor(64.0 + 24.0 * z[e] + 0.5);
      o[e] = (uint8_t)std::min(255.0, std::max(0.0, v));
    }
  });
  return 0;
}

}  // extern "C"
