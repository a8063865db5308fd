// Quantized lower bound on the canonical distance, used to skip exact
// distance gathers whose result cannot change the search state.
//
// Each vector row x gets a 128-byte companion row (one cache line):
//   chunk 0      header {float s, float r, float a, unused}
//   chunks 1..7  int8 codes q (16 dimensions per chunk, zero padded)
// with x ~ s*q, a ~ s^2 * sum(q^2) (rounded to fp32) and r >= ||x - s*q||_2
// (rounded up). For a pair (x, y) with code dot product c (an exact integer),
//   Q = s_x^2 A_x + s_y^2 A_y - 2 s_x s_y c = ||s_x q_x - s_y q_y||^2,
// and the triangle inequality gives ||x - y|| >= sqrt(Q) - r_x - r_y.
//
// The canonical fp32 distance (fmaf per lane over n_lane non-negative terms,
// then the three-level octet tree) satisfies dist >= D (1 - u)^(n_lane + 5)
// - eta, with D the exact squared distance, u = 2^-24 and eta an underflow
// slack, so D >= (T + 1e-30)(1 + kappa2), kappa2 = 2 (n_lane + 8) u, proves
// dist >= T. That holds when Q >= (sqrt((T + 1e-30)(1 + kappa2)) + r_x +
// r_y)^2. The test is evaluated in fp32 with explicit slack factors 2^-19,
// 32 times the accumulated rounding (|Q_computed - Q| <= 6 u (a_x + a_y),
// since 2 s_x s_y |c| <= a_x + a_y). A candidate proved this way would be
// rejected by the pool's threshold test, so skipping its exact distance
// leaves every result bit-identical. Rows with non-finite values, or whose
// scale leaves [2^-60, 2^50], get r = +inf and are never skipped.
#pragma once

#include "wave.h"

namespace dance {

constexpr uint32_t kQChunks = 8;                      // 16-byte chunks per code row
constexpr uint32_t kQMaxDim = (kQChunks - 1u) * 16u;  // dimensions a code row holds
constexpr float kQSlack = 0x1p-19f;

struct QBoundSet {
  const uint4* rows;  // N x kQChunks chunks; nullptr disables the bound
  float kappa2;       // 2 (n_lane + 8) 2^-24 for the row type and width
};

// One thread per row: codes, scale, radius. Reads `dim` elements of the row.
template <int DT>
__global__ void k_quantize(RowSet rs, uint32_t N, uint32_t dim, uint4* __restrict__ out) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const uint4* row = rs.rows + (size_t)i * rs.stride16;
  auto elem = [&](uint32_t d) -> float {
    if constexpr (DT == DANCE_F32) {
      const uint32_t* w = reinterpret_cast<const uint32_t*>(row);
      return __uint_as_float(w[d]);
    } else {
      const uint16_t* h = reinterpret_cast<const uint16_t*>(row);
      return (float)__builtin_bit_cast(_Float16, h[d]);
    }
  };
  float mx = 0.0f;
  bool finite = true;
  for (uint32_t d = 0; d < dim; ++d) {
    const float v = elem(d);
    finite = finite && __builtin_isfinite(v);
    mx = fmaxf(mx, fabsf(v));
  }
  float s = mx / 127.0f;
  // all-zero rows are exact with s = 0; other scales must stay in range
  const bool usable = finite && (mx == 0.0f || (s >= 0x1p-60f && s <= 0x1p50f));
  if (!usable || mx == 0.0f) s = 0.0f;
  int64_t A = 0;
  double err = 0.0;
  uint32_t words[(kQChunks - 1) * 4];
#pragma unroll
  for (uint32_t w = 0; w < (kQChunks - 1) * 4; ++w) {
    uint32_t word = 0u;
#pragma unroll
    for (uint32_t b = 0; b < 4; ++b) {
      const uint32_t d = 4u * w + b;
      if (d < dim) {
        const float v = elem(d);
        int q = 0;
        if (s > 0.0f) q = (int)fminf(127.0f, fmaxf(-127.0f, rintf(v / s)));
        A += (int64_t)q * q;
        const double e = (double)v - (double)s * (double)q;
        err = fma(e, e, err);
        word |= ((uint32_t)(q & 0xFF)) << (8u * b);
      }
    }
    words[w] = word;
  }
  float r = __builtin_inff();
  if (usable) {
    const double rd = sqrt(err) * (1.0 + 0x1p-40);
    r = (float)rd;
    if ((double)r < rd) r = __uint_as_float(__float_as_uint(r) + 1u);  // r >= 0: next float up
  }
  const float a = (float)((double)s * (double)s * (double)A);
  uint4* o = out + (size_t)i * kQChunks;
  o[0] = make_uint4(__float_as_uint(s), __float_as_uint(r), __float_as_uint(a), 0u);
#pragma unroll
  for (uint32_t c = 1; c < kQChunks; ++c)
    o[c] = make_uint4(words[4 * (c - 1)], words[4 * (c - 1) + 1], words[4 * (c - 1) + 2], words[4 * (c - 1) + 3]);
}

// The querying row's header (scalars) and code row address.
struct QSelf {
  const uint4* row;
  float s, r, a;
};

__device__ __forceinline__ void q_load_self(const QBoundSet& qb, uint32_t id, QSelf& me) {
  const uint4* p = qb.rows + (size_t)id * kQChunks;
  me.row = p;
  const uint4 h = p[0];  // same address in every lane: kept as scalars
  me.s = __uint_as_float(uni_u(h.x));
  me.r = __uint_as_float(uni_u(h.y));
  me.a = __uint_as_float(uni_u(h.z));
}

// Upper bound of sqrt((T + 1e-30)(1 + kappa2)) + r_self (uniform).
__device__ __forceinline__ float q_threshold(const QBoundSet& qb, const QSelf& me, float T) {
  const float t = (T + 1e-30f) * (1.0f + qb.kappa2);
  return uni_f((__builtin_sqrtf(t) + me.r) * (1.0f + kQSlack));
}

// Chunk `sub` of the code row of candidate `id` (zero when inactive).
__device__ __forceinline__ uint4 q_load(const QBoundSet& qb, uint32_t id, bool active, uint32_t sub) {
  return active ? qb.rows[(size_t)id * kQChunks + sub] : make_uint4(0u, 0u, 0u, 0u);
}

// Octet test for a candidate: every lane of the octet holds one chunk `b` of
// its code row (q_load); the lane with sub == 0 (which holds the header)
// returns whether the bound proves dist >= T. `code` is chunk `sub` of the
// querying row. Must be called by all 64 lanes.
__device__ __forceinline__ bool q_proves_reject(const QSelf& me, const uint4& code, float sT, const uint4& b,
                                                bool active, uint32_t sub) {
  int c = 0;
  c = __builtin_amdgcn_sdot4((int)code.x, (int)b.x, c, false);
  c = __builtin_amdgcn_sdot4((int)code.y, (int)b.y, c, false);
  c = __builtin_amdgcn_sdot4((int)code.z, (int)b.z, c, false);
  c = __builtin_amdgcn_sdot4((int)code.w, (int)b.w, c, false);
  if (sub == 0) c = 0;  // chunk 0 is the header
  c += dpp<kDppHalfMirror>(0, c);
  c += dpp<kDppQuadXor2>(0, c);
  c += dpp<kDppQuadXor1>(0, c);
  const float sy = __uint_as_float(b.x);
  const float ry = __uint_as_float(b.y);
  const float sa = me.a + __uint_as_float(b.z);
  const float q = __builtin_fmaf(-2.0f * (me.s * sy), (float)c, sa) - kQSlack * sa - 1e-30f;
  const float w = (sT + ry) * (1.0f + kQSlack);
  return active && q >= w * w * (1.0f + kQSlack);
}

// Threshold of the prune's bound for a candidate at stored distance sd: a
// pair distance d >= T gives fl(alpha * d) >= fl(alpha * T) > sd, so the
// candidate survives. Returns sqrt((T + 1e-30)(1 + kappa2)) rounded up, the
// per-candidate part of q_threshold; +inf (never skipped) for sd < 1e-30 or
// non-finite sd, where the relative slack would not cover rounding.
__device__ __forceinline__ float prune_bound_root(const QBoundSet& qb, float sd, float alpha) {
  if (!(sd >= 1e-30f) || !(sd <= FLT_MAX)) return __builtin_inff();
  const float T = sd / alpha * (1.0f + 0x1p-20f);
  const float t = (T + 1e-30f) * (1.0f + qb.kappa2);
  return __builtin_sqrtf(t) * (1.0f + kQSlack);
}

// Bits 0, 8, ..., 56 of a ballot -> bits 0..7.
__device__ __forceinline__ uint32_t octet_bits(uint64_t m) {
  return (uint32_t)(((m & 0x0101010101010101ull) * 0x0102040810204080ull) >> 56);
}

}  // namespace dance
