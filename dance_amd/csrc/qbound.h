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
// - 1e-30, with D the exact squared distance, u = 2^-24 and 1e-30 an
// underflow slack, so D >= (T + eta)(1 + kappa2), kappa2 = 2 (n_lane + 8) u,
// eta = 1e-30, proves dist >= T. The fp16 distance rounds each difference and
// square to binary16 (unit 2^-11): a term t^2 becomes at least
// t^2 (1 - 3 2^-11) - 2^-24 (the absolute part covers the subnormal range),
// so for fp16 rows kappa2 = 2 (3 2^-11 + (n_lane + 8) u) and
// eta = 1e-30 + dim 2^-24. The test holds when Q >= (sqrt((T + eta)
// (1 + kappa2)) + r_x + r_y)^2. The test is evaluated in fp32 with explicit slack factors 2^-19,
// 32 times the accumulated rounding (|Q_computed - Q| <= 6 u (a_x + a_y),
// since 2 s_x s_y |c| <= a_x + a_y). A candidate proved this way would be
// rejected by the pool's threshold test, so skipping its exact distance
// leaves every result bit-identical. Rows with non-finite values, or whose
// scale leaves [2^-60, 2^50], get r = +inf and are never skipped.
// The same rows give an upper bound, sqrt(Q) + r_x + r_y >= ||x - y||
// (q_pair_ub), which proves pair tests of the form fl(alpha * dist) <= T0.
#pragma once

#include "wave.h"

namespace dance {

constexpr uint32_t kQChunks = 8;                      // 16-byte chunks per code row
constexpr uint32_t kQMaxDim = (kQChunks - 1u) * 16u;  // dimensions a code row holds
constexpr float kQSlack = 0x1p-19f;

struct QBoundSet {
  const uint4* rows;  // N x kQChunks chunks; nullptr disables the bound
  float kappa2;       // relative rounding slack of the row type and width
  float eta;          // absolute slack (underflow; binary16 subnormals)
};

// One octet per row (8 rows per wave): lane sub owns code words sub, sub+8,
// sub+16, sub+24 (word w = dimensions 4w..4w+3), so every load and store of
// an octet covers contiguous bytes. Computes codes, scale and radius from the
// first `dim` elements of the row.
template <int DT>
__global__ __launch_bounds__(256) void k_quantize(RowSet rs, uint32_t N, uint32_t dim, uint4* __restrict__ out) {
  constexpr uint32_t kWords = (kQChunks - 1) * 4;  // 28 code words
  constexpr uint32_t kEB = DT == DANCE_F32 ? 4u : 2u;  // element bytes
  const uint32_t lane = threadIdx.x & 63u, sub = lane & 7u;
  const uint32_t row = (blockIdx.x * 256u + threadIdx.x) >> 3;
  const bool act = row < N;
  const uint8_t* rb = reinterpret_cast<const uint8_t*>(rs.rows + (size_t)(act ? row : 0u) * rs.stride16);
  const uint32_t row_bytes = rs.stride16 * 16u;
  float v[4][4];
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) {
    const uint32_t w = sub + 8u * k;
    const bool in = act && w < kWords && 4u * w < dim && (4u * w + 4u) * kEB <= row_bytes;
    if constexpr (DT == DANCE_F32) {
      const uint4 c = in ? *reinterpret_cast<const uint4*>(rb + 16u * w) : make_uint4(0u, 0u, 0u, 0u);
      v[k][0] = __uint_as_float(c.x);
      v[k][1] = __uint_as_float(c.y);
      v[k][2] = __uint_as_float(c.z);
      v[k][3] = __uint_as_float(c.w);
    } else {
      const uint2 c = in ? *reinterpret_cast<const uint2*>(rb + 8u * w) : make_uint2(0u, 0u);
      v[k][0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(c.x & 0xFFFFu));
      v[k][1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(c.x >> 16));
      v[k][2] = (float)__builtin_bit_cast(_Float16, (uint16_t)(c.y & 0xFFFFu));
      v[k][3] = (float)__builtin_bit_cast(_Float16, (uint16_t)(c.y >> 16));
    }
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e)
      if (4u * w + e >= dim) v[k][e] = 0.0f;  // padding inside a word
  }
  float mx = 0.0f;
  int fin = 1;
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k)
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e) {
      fin &= __builtin_isfinite(v[k][e]) ? 1 : 0;
      mx = fmaxf(mx, fabsf(v[k][e]));
    }
  // octet reductions (every lane of the octet ends with the result)
  mx = fmaxf(mx, __int_as_float(dpp<kDppQuadXor1>(0, __float_as_int(mx))));
  mx = fmaxf(mx, __int_as_float(dpp<kDppQuadXor2>(0, __float_as_int(mx))));
  mx = fmaxf(mx, __int_as_float(dpp<kDppHalfMirror>(0, __float_as_int(mx))));
  fin &= dpp<kDppQuadXor1>(1, fin);
  fin &= dpp<kDppQuadXor2>(1, fin);
  fin &= dpp<kDppHalfMirror>(1, fin);
  float s = mx / 127.0f;
  // all-zero rows are exact with s = 0; other scales must stay in range
  const bool usable = fin && (mx == 0.0f || (s >= 0x1p-60f && s <= 0x1p50f));
  if (!usable || mx == 0.0f) s = 0.0f;
  int A = 0;
  double err = 0.0;
  uint32_t words[4];
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) {
    uint32_t word = 0u;
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e) {
      int qv = 0;
      if (s > 0.0f) qv = (int)fminf(127.0f, fmaxf(-127.0f, rintf(v[k][e] / s)));
      A += qv * qv;
      const double d = (double)v[k][e] - (double)s * (double)qv;
      err = fma(d, d, err);
      word |= ((uint32_t)(qv & 0xFF)) << (8u * e);
    }
    words[k] = word;
  }
  A += dpp<kDppQuadXor1>(0, A);
  A += dpp<kDppQuadXor2>(0, A);
  A += dpp<kDppHalfMirror>(0, A);
  err += __shfl_xor(err, 1);
  err += __shfl_xor(err, 2);
  err += __shfl_xor(err, 4);
  if (!act) return;
  uint32_t* o = reinterpret_cast<uint32_t*>(out + (size_t)row * kQChunks);
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) {
    const uint32_t w = sub + 8u * k;
    if (w < kWords) o[4u + w] = words[k];
  }
  if (sub == 0) {
    float r = __builtin_inff();
    if (usable) {
      const double rd = sqrt(err) * (1.0 + 0x1p-40);
      r = (float)rd;
      if ((double)r < rd) r = __uint_as_float(__float_as_uint(r) + 1u);  // r >= 0: next float up
    }
    const float a = (float)((double)s * (double)s * (double)A);
    reinterpret_cast<uint4*>(o)[0] = make_uint4(__float_as_uint(s), __float_as_uint(r), __float_as_uint(a), 0u);
  }
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

// Upper bound of sqrt((T + eta)(1 + kappa2)) + r_self (uniform).
__device__ __forceinline__ float q_threshold(const QBoundSet& qb, const QSelf& me, float T) {
  const float t = (T + qb.eta) * (1.0f + qb.kappa2);
  return uni_f((__builtin_sqrtf(t) + me.r) * (1.0f + kQSlack));
}

// Chunk `sub` of the code row of candidate `id`. An inactive lane loads
// nothing and the value is left unset (as in load_row): `active` is the same
// on the 8 lanes of an octet and q_proves_reject returns false for it.
__device__ __forceinline__ uint4 q_load(const QBoundSet& qb, uint32_t id, bool active, uint32_t sub) {
  uint4 b;
  if (active) b = qb.rows[(size_t)id * kQChunks + sub];
  return b;
}

// The bound's test for one pair: the querying row's scale s and a, the
// candidate's header (sy, ry, ay), sT from q_threshold (or the prune's root)
// and the exact integer code dot c. Every caller evaluates this expression,
// so a decision does not depend on how c was computed.
__device__ __forceinline__ bool q_pair_proves(float s, float a, float sT, float sy, float ry, float ay, int c) {
  const float sa = a + ay;
  const float q = __builtin_fmaf(-2.0f * (s * sy), (float)c, sa) - kQSlack * sa - 1e-30f;
  const float w = (sT + ry) * (1.0f + kQSlack);
  return q >= w * w * (1.0f + kQSlack);
}

// q_pair_proves with the querying row's scale passed as m2s = -2 s. Scaling
// by -2 commutes with rounding for the scales k_quantize keeps ([2^-60,
// 2^50], or 0), so fl(m2s * sy) = -2 fl(s * sy) and the decision is that of
// q_pair_proves on the same inputs.
__device__ __forceinline__ bool q_pair_proves_m2(float m2s, float a, float sT, float sy, float ry, float ay, int c) {
  const float sa = a + ay;
  const float q = __builtin_fmaf(m2s * sy, (float)c, sa) - kQSlack * sa - 1e-30f;
  const float w = (sT + ry) * (1.0f + kQSlack);
  return q >= w * w * (1.0f + kQSlack);
}

// Exact integer code dot of two rows whose chunk `sub` every lane of an
// octet holds (chunk 0, the header, left out); every lane of the octet
// receives it. Must be called by all 64 lanes.
__device__ __forceinline__ int q_octet_dot(const uint4& code, const uint4& b, uint32_t sub) {
  int c = 0;
  c = __builtin_amdgcn_sdot4((int)code.x, (int)b.x, c, false);
  c = __builtin_amdgcn_sdot4((int)code.y, (int)b.y, c, false);
  c = __builtin_amdgcn_sdot4((int)code.z, (int)b.z, c, false);
  c = __builtin_amdgcn_sdot4((int)code.w, (int)b.w, c, false);
  if (sub == 0) c = 0;  // chunk 0 is the header
  c += dpp<kDppHalfMirror>(0, c);
  c += dpp<kDppQuadXor2>(0, c);
  c += dpp<kDppQuadXor1>(0, c);
  return c;
}

// Octet test for a candidate: every lane of the octet holds one chunk `b` of
// its code row (q_load); the lane with sub == 0 (which holds the header)
// returns whether the bound proves dist >= T. `code` is chunk `sub` of the
// querying row. Must be called by all 64 lanes.
__device__ __forceinline__ bool q_proves_reject(const QSelf& me, const uint4& code, float sT, const uint4& b,
                                                bool active, uint32_t sub) {
  const int c = q_octet_dot(code, b, sub);
  return active && q_pair_proves(me.s, me.a, sT, __uint_as_float(b.x), __uint_as_float(b.y), __uint_as_float(b.z), c);
}

// The upper-bound side, for a pair test fl(alpha * dist) <= T0 (the online
// insert's occlusion test). The canonical distance satisfies dist <= D (1 +
// u)^(n_lane + 5) + 1e-30 <= D (1 + kappa2) + eta' by the rounding argument of
// the lower side (binary16 terms: at most t^2 (1 + 2^-11)^3 + 2^-24 each),
// with eta' <= 2 eta, and fl(alpha * dist) <= alpha dist (1 + u). So D <=
// (T0 / (alpha (1 + u)) - 2 eta) / (1 + kappa2) proves the test. q_ub_root
// returns the square root of that bound on D, rounded down (every step's
// rounding absorbed by the 2^-20 and kQSlack factors), or -1 (never proved)
// when T0 is below 1e-30 or not finite or the bound is not a positive finite
// number.
__device__ __forceinline__ float q_ub_root(const QBoundSet& qb, float T0, float alpha) {
  if (!(T0 >= 1e-30f) || !(T0 <= FLT_MAX)) return -1.0f;
  const float t = T0 / alpha * (1.0f - 0x1p-20f);
  const float t2 = (t - 2.0f * qb.eta) / (1.0f + qb.kappa2) * (1.0f - kQSlack);
  if (!(t2 > 0.0f) || !(t2 <= FLT_MAX)) return -1.0f;
  return __builtin_sqrtf(t2) * (1.0f - kQSlack);
}
// q_ub_root for rows of type DT. The binary16 distance squares each
// difference in binary16, which overflows to +inf past 65504; D <= 254^2
// keeps every term finite (a difference of at most 254 (1 + 2^-11) squares
// to below 65504), so the root is capped there for fp16 rows.
template <int DT>
__device__ __forceinline__ float q_ub_root_of(const QBoundSet& qb, float T0, float alpha) {
  const float r = q_ub_root(qb, T0, alpha);
  return DT == DANCE_F16 ? fminf(r, 254.0f) : r;
}
// Proves D <= root_ub^2 for the pair (querying row s, a, r; candidate
// header sy, ry, ay; code dot c): by the triangle inequality ||x - y|| <=
// sqrt(Q) + r_x + r_y, and Q <= Q_computed + 6 u (a_x + a_y); the fp32
// evaluation adds kQSlack (a_x + a_y) + 1e-30 instead and rounds the sum up
// by kQSlack. Rows with r = +inf are never proved.
__device__ __forceinline__ bool q_pair_ub(float s, float a, float r, float root_ub, float sy, float ry, float ay,
                                          int c) {
  const float sa = a + ay;
  const float q = __builtin_fmaf(-2.0f * (s * sy), (float)c, sa) + kQSlack * sa + 1e-30f;
  const float lhs = (__builtin_sqrtf(fmaxf(q, 0.0f)) + r + ry) * (1.0f + kQSlack);
  return lhs <= root_ub;
}

// Threshold of the prune's bound for a candidate at stored distance sd: a
// pair distance d >= T gives fl(alpha * d) >= fl(alpha * T) > sd, so the
// candidate survives. Returns sqrt((T + eta)(1 + kappa2)) rounded up, the
// per-candidate part of q_threshold; +inf (never skipped) for sd < 1e-30 or
// non-finite sd, where the relative slack would not cover rounding.
__device__ __forceinline__ float prune_bound_root(const QBoundSet& qb, float sd, float alpha) {
  if (!(sd >= 1e-30f) || !(sd <= FLT_MAX)) return __builtin_inff();
  const float T = sd / alpha * (1.0f + 0x1p-20f);
  const float t = (T + qb.eta) * (1.0f + qb.kappa2);
  return __builtin_sqrtf(t) * (1.0f + kQSlack);
}

// Bits 0, 8, ..., 56 of a ballot -> bits 0..7.
__device__ __forceinline__ uint32_t octet_bits(uint64_t m) {
  return (uint32_t)(((m & 0x0101010101010101ull) * 0x0102040810204080ull) >> 56);
}

}  // namespace dance
