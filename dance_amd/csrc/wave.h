// Wave64 primitives and the canonical distance for gfx950 (CDNA4).
//
// Distances are computed by "octets": 8 consecutive lanes cooperate on one
// vector pair, each lane owning the 16-byte chunks sub, sub+8, sub+16, ... of
// the row (sub = lane & 7). One wave therefore evaluates 8 distances per pass,
// and every 8-lane load instruction reads whole 128-byte lines.
//
// Canonical arithmetic (shared bit for bit with the CPU oracle):
//   fp32: p = fmaf(t, t, p), t = a - b, in ascending element order within the
//   lane's chunks.
//   fp16: the reference's element arithmetic (gpu_vamana_vnew2.cu:391-418,
//   gpu_vamana_filtered.cu:4036-4047): per pair of elements (one 32-bit word)
//   the difference and the square are binary16 operations (round to nearest
//   even, overflow to inf), the two squares are widened and added in fp32,
//   and that pair sum is added to p. For odd dim the last element is widened
//   first and squared in fp32 (p = fmaf(t, t, p)), as the reference does.
//   Words in ascending order within the lane's chunks.
//   Then, for both, the DPP tree half-row mirror (lane j + lane 7-j), quad
//   swap 2, quad swap 1: ((p0+p7)+(p2+p5)) + ((p1+p6)+(p3+p4)); every lane of
//   the octet holds it.
//   uint8: exact integer sum of (a-b)^2, converted to fp32 once.
// The value is symmetric in (a, b): a-b and b-a differ only in sign, in
// binary16 as in fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <float.h>
#include <limits.h>
#include <type_traits>

#define DANCE_INV 0xFFFFFFFFu

enum DanceDType : int { DANCE_F32 = 0, DANCE_U8 = 1, DANCE_F16 = 2 };

__device__ __forceinline__ uint32_t lane_id() {
  return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}
__device__ __forceinline__ uint64_t wballot(bool p) { return (uint64_t)__ballot(p); }
__device__ __forceinline__ uint32_t mbcnt64(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}
__device__ __forceinline__ int ffs64(uint64_t m) { return __ffsll((unsigned long long)m) - 1; }
// Lanes [0, n) as a mask (n >= 64: every lane).
__device__ __forceinline__ uint64_t lanes_below(uint32_t n) { return n >= 64u ? ~0ull : ((1ull << n) - 1ull); }
// Lane 8 g of each octet g (the lanes that hold an octet's result).
constexpr uint64_t kOctetLeads = 0x0101010101010101ull;
__device__ __forceinline__ uint32_t popc64(uint64_t m) { return (uint32_t)__popcll((unsigned long long)m); }

__device__ __forceinline__ int uni_i(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uint32_t uni_u(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ float uni_f(float v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ __forceinline__ uint32_t rdlane_u(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
__device__ __forceinline__ float rdlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Index of this wave in its workgroup, as a scalar: everything derived from it
// (LDS bases, vertex ids, row addresses) then lives in SGPRs.
__device__ __forceinline__ uint32_t wave_index() { return uni_u(threadIdx.x >> 6); }

// Orders LDS traffic between lanes of one wave (the wave runs in lockstep;
// this keeps the compiler from reordering and drains outstanding LDS ops).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// DPP controls (gfx9 encoding).
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <- lane 7-i within 8
constexpr int kDppRowMirror = 0x140;   // lane i <- lane 15-i within 16
constexpr int kDppBcast15 = 0x142;     // lane 15 of each row -> next row
constexpr int kDppBcast31 = 0x143;     // lane 31 -> rows 2 and 3

template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ int dpp(int old, int v) {
  return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWS, 0xF, false);
}

// Wave-wide reductions with DPP; max/min and integer sums are exact, so the
// tree shape does not matter. The full result lands in lane 63 and is read back as a scalar.
template <typename Op>
__device__ __forceinline__ int wave_reduce_i(int v, int ident, Op op) {
  v = op(v, dpp<kDppQuadXor1>(ident, v));
  v = op(v, dpp<kDppQuadXor2>(ident, v));
  v = op(v, dpp<kDppHalfMirror>(ident, v));
  v = op(v, dpp<kDppRowMirror>(ident, v));
  v = op(v, dpp<kDppBcast15, 0xA>(ident, v));
  v = op(v, dpp<kDppBcast31, 0xC>(ident, v));
  return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ int wave_max_i(int v) {
  return wave_reduce_i(v, INT_MIN, [](int a, int b) { return max(a, b); });
}
__device__ __forceinline__ int wave_min_i(int v) {
  return wave_reduce_i(v, INT_MAX, [](int a, int b) { return min(a, b); });
}
__device__ __forceinline__ uint32_t wave_sum_u(uint32_t v) {
  return (uint32_t)wave_reduce_i((int)v, 0, [](int a, int b) { return (int)((uint32_t)a + (uint32_t)b); });
}
__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
  return (uint32_t)wave_reduce_i((int)v, 0, [](int a, int b) { return (int)max((uint32_t)a, (uint32_t)b); });
}
__device__ __forceinline__ uint32_t wave_min_u(uint32_t v) {
  return (uint32_t)wave_reduce_i((int)v, -1, [](int a, int b) { return (int)min((uint32_t)a, (uint32_t)b); });
}

// Exclusive prefix sum over the 64 lanes.
__device__ __forceinline__ uint32_t wave_excl_scan_u(uint32_t v) {
  uint32_t x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t y = (uint32_t)__shfl_up((int)x, (unsigned int)d);
    if (lane_id() >= (uint32_t)d) x += y;
  }
  return x - v;
}

// Workgroup index of a launch of up to 2^32 workgroups. A dispatch holds
// fewer than 2^32 work-items per dimension, so larger launches are 2-D
// (grid_dims): gx x gy workgroups, dispatched in row-major order.
__device__ __forceinline__ uint32_t grid_block() { return blockIdx.y * gridDim.x + blockIdx.x; }
__device__ __forceinline__ uint32_t grid_blocks() { return gridDim.x * gridDim.y; }

// Workgroup -> logical block. Workgroups are dispatched round-robin over the 8
// XCDs; this mapping hands XCD k the contiguous logical range
// [k*per, (k+1)*per) so each XCD's L2 walks one region of the processing
// order. nb_pad is the launched grid size, a multiple of 8.
__device__ __forceinline__ uint32_t xcd_block(uint32_t b, uint32_t nb_pad) {
  const uint32_t per = nb_pad >> 3;
  return (b & 7u) * per + (b >> 3);
}

// Reference hashes: vnew2.cu:169-191.
__device__ __forceinline__ uint32_t d_hash_u32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}
__device__ __forceinline__ uint32_t d_det_neighbor(uint32_t node, uint32_t k, uint32_t N) {
  if (N <= 1) return DANCE_INV;
  uint32_t v = d_hash_u32(node * 0x9e3779b1u + k * 0x85ebca6bu + 17u) % N;
  if (v == node) v = (v + 1u) % N;
  return v;
}

// ---------------------------------------------------------------------------
// Octet distance.
// ---------------------------------------------------------------------------
struct RowSet {
  const uint4* rows;  // device rows, each padded to stride16 16-byte chunks
  uint32_t stride16;  // chunks per row (row stride / 16 bytes)
  uint32_t nch;       // chunks that hold data (ceil(dim * elem_bytes / 16))
  int32_t tail16;     // fp16 rows of odd dim: index of the 32-bit word holding
                      // the last element (its upper half is padding); else -1
};

// Chunks sub, sub + 8, ... of row `id`. Rows are padded with zeros to the
// chunk group (nch == 8 CPL, see setup_rows), so every slot holds data. An
// inactive lane loads nothing and v keeps whatever it held (callers pass
// freshly declared arrays): `active` is the same on the 8 lanes of an octet,
// so inactive values only reach the distances of inactive candidates, which
// every caller discards. Leaving them unset spares the 4 zeroing moves per
// chunk that a defined value costs in front of each masked load.
template <int CPL>
__device__ __forceinline__ void load_row(const RowSet& rs, uint32_t id, bool active, uint32_t sub,
                                         uint4 (&v)[CPL]) {
  const uint4* p = rs.rows + (size_t)id * rs.stride16;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    if (active) v[c] = p[sub + 8u * (uint32_t)c];
  }
}

__device__ __forceinline__ float fma_sq(float a, float b, float acc) {
  const float t = a - b;
  return __builtin_fmaf(t, t, acc);
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2_t as_half2(uint32_t w) { return __builtin_bit_cast(half2_t, w); }

// One word of fp16 elements: binary16 difference and square, widened pair sum.
__device__ __forceinline__ float h2_pair_sq(uint32_t a, uint32_t b) {
  const half2_t t = as_half2(a) - as_half2(b);
  const half2_t q = t * t;
  return (float)q.x + (float)q.y;
}

// The odd-dim tail word: only the lower half holds data (the upper half is
// padding, zero in every row); widened first, squared in fp32.
__device__ __forceinline__ float h2_tail_fma(uint32_t a, uint32_t b, float acc) {
  const float t = (float)as_half2(a).x - (float)as_half2(b).x;
  return __builtin_fmaf(t, t, acc);
}

template <int DT, int CPL>
__device__ __forceinline__ float octet_partial_f(const RowSet& rs, uint32_t sub, const uint4 (&a)[CPL],
                                                 const uint4 (&b)[CPL]) {
  float acc = 0.0f;
  if constexpr (DT == DANCE_F32) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      acc = fma_sq(__uint_as_float(a[c].x), __uint_as_float(b[c].x), acc);
      acc = fma_sq(__uint_as_float(a[c].y), __uint_as_float(b[c].y), acc);
      acc = fma_sq(__uint_as_float(a[c].z), __uint_as_float(b[c].z), acc);
      acc = fma_sq(__uint_as_float(a[c].w), __uint_as_float(b[c].w), acc);
    }
  } else if (rs.tail16 < 0) {  // kernel argument: a uniform branch
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      acc += h2_pair_sq(a[c].x, b[c].x);
      acc += h2_pair_sq(a[c].y, b[c].y);
      acc += h2_pair_sq(a[c].z, b[c].z);
      acc += h2_pair_sq(a[c].w, b[c].w);
    }
  } else {
    // Word (c, w) of this lane is word 4*sub + 32*c + w of the row.
    const int tl = rs.tail16 - 4 * (int)sub;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const uint32_t wa[4] = {a[c].x, a[c].y, a[c].z, a[c].w};
      const uint32_t wb[4] = {b[c].x, b[c].y, b[c].z, b[c].w};
#pragma unroll
      for (int w = 0; w < 4; ++w)
        acc = tl == 32 * c + w ? h2_tail_fma(wa[w], wb[w], acc) : acc + h2_pair_sq(wa[w], wb[w]);
    }
  }
  return acc;
}

// The lane's share of sum a^2 over a uint8 row: the part of a pair's partial
// that depends on `a` alone. Loops that pair one cached row with many others
// compute it once (the search's vertex row, the online insert's expanded
// row) instead of per pair.
template <int CPL>
__device__ __forceinline__ uint32_t u8_self_sq(const uint4 (&a)[CPL]) {
  uint32_t sq = 0u;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    sq = __builtin_amdgcn_udot4(a[c].x, a[c].x, sq, false);
    sq = __builtin_amdgcn_udot4(a[c].y, a[c].y, sq, false);
    sq = __builtin_amdgcn_udot4(a[c].z, a[c].z, sq, false);
    sq = __builtin_amdgcn_udot4(a[c].w, a[c].w, sq, false);
  }
  return sq;
}

// Sum over the lane's bytes of a^2 + b^2 - 2ab given a_sq = u8_self_sq(a):
// exact in 32-bit integers (wrap-around included), so the grouping of the
// terms never changes the value.
template <int CPL>
__device__ __forceinline__ int octet_partial_u8(const uint4 (&a)[CPL], const uint4 (&b)[CPL], uint32_t a_sq) {
  uint32_t sq = a_sq, cr = 0u;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    sq = __builtin_amdgcn_udot4(b[c].x, b[c].x, sq, false);
    cr = __builtin_amdgcn_udot4(a[c].x, b[c].x, cr, false);
    sq = __builtin_amdgcn_udot4(b[c].y, b[c].y, sq, false);
    cr = __builtin_amdgcn_udot4(a[c].y, b[c].y, cr, false);
    sq = __builtin_amdgcn_udot4(b[c].z, b[c].z, sq, false);
    cr = __builtin_amdgcn_udot4(a[c].z, b[c].z, cr, false);
    sq = __builtin_amdgcn_udot4(b[c].w, b[c].w, sq, false);
    cr = __builtin_amdgcn_udot4(a[c].w, b[c].w, cr, false);
  }
  return (int)(sq - 2u * cr);
}
template <int CPL>
__device__ __forceinline__ int octet_partial_u8(const uint4 (&a)[CPL], const uint4 (&b)[CPL]) {
  return octet_partial_u8<CPL>(a, b, u8_self_sq<CPL>(a));
}

// Canonical octet combination of per-lane partial sums (see the header).
__device__ __forceinline__ float octet_combine(float p) {
  p += __int_as_float(dpp<kDppHalfMirror>(0, __float_as_int(p)));
  p += __int_as_float(dpp<kDppQuadXor2>(0, __float_as_int(p)));
  p += __int_as_float(dpp<kDppQuadXor1>(0, __float_as_int(p)));
  return p;
}

// Full distance of a pair held by an octet; every lane of the octet returns it.
// Must be called by all 64 lanes (the butterfly crosses lanes). a_sq is
// u8_self_sq(a) for uint8 rows (unused otherwise).
template <int DT, int CPL>
__device__ __forceinline__ float octet_finish(const RowSet& rs, uint32_t sub, const uint4 (&a)[CPL],
                                              const uint4 (&b)[CPL], uint32_t a_sq) {
  if constexpr (DT == DANCE_U8) {
    int p = octet_partial_u8<CPL>(a, b, a_sq);
    p += dpp<kDppHalfMirror>(0, p);
    p += dpp<kDppQuadXor2>(0, p);
    p += dpp<kDppQuadXor1>(0, p);
    return (float)(uint32_t)p;
  } else {
    return octet_combine(octet_partial_f<DT, CPL>(rs, sub, a, b));
  }
}
template <int DT, int CPL>
__device__ __forceinline__ float octet_finish(const RowSet& rs, uint32_t sub, const uint4 (&a)[CPL],
                                              const uint4 (&b)[CPL]) {
  return octet_finish<DT, CPL>(rs, sub, a, b, DT == DANCE_U8 ? u8_self_sq<CPL>(a) : 0u);
}

// The per-lane self term octet_finish takes for a row cached in registers.
template <int DT, int CPL>
__device__ __forceinline__ uint32_t self_term(const uint4 (&a)[CPL]) {
  if constexpr (DT == DANCE_U8)
    return u8_self_sq<CPL>(a);
  else
    return 0u;
}

// Float ordering keys for wave reductions over non-negative distances.
// NaN never wins, matching the reference's strict float comparisons.
__device__ __forceinline__ int fkey(float d) { return __float_as_int(d); }

// Distances from a cached vector `av` to up to 64 ids lst[0..n) -> lsd[0..n).
// Two passes of 8 octets are kept in flight (one for a last group of <= 8).
// lst holds 64 entries; every index read stays below 64. Returns after lsd
// is visible.
template <int DT, int CPL>
__device__ __forceinline__ void batch_dist(const RowSet& rs, const uint4 (&av)[CPL], uint32_t a_sq,
                                           const uint32_t* lst, float* lsd, uint32_t n, uint32_t grp,
                                           uint32_t sub) {
  uint32_t p = 0;
  for (; p + 8 < n; p += 16) {
    const uint32_t k0 = p + grp, k1 = p + 8 + grp;
    const bool a0 = k0 < n, a1 = k1 < n;
    const uint32_t id0 = lst[k0], id1 = lst[k1];  // k0, k1 < 64: in bounds; inactive ids are not loaded
    uint4 b0[CPL], b1[CPL];
    load_row<CPL>(rs, id0, a0, sub, b0);
    load_row<CPL>(rs, id1, a1, sub, b1);
    const float d0 = octet_finish<DT, CPL>(rs, sub, av, b0, a_sq);
    const float d1 = octet_finish<DT, CPL>(rs, sub, av, b1, a_sq);
    if (sub == 0) {
      if (a0) lsd[k0] = d0;
      if (a1) lsd[k1] = d1;
    }
  }
  if (p < n) {  // a last group of at most 8: one pass
    const uint32_t k0 = p + grp;
    const bool a0 = k0 < n;
    uint4 b0[CPL];
    load_row<CPL>(rs, lst[k0], a0, sub, b0);
    const float d0 = octet_finish<DT, CPL>(rs, sub, av, b0, a_sq);
    if (sub == 0 && a0) lsd[k0] = d0;
  }
  wave_sync();
}
template <int DT, int CPL>
__device__ __forceinline__ void batch_dist(const RowSet& rs, const uint4 (&av)[CPL], const uint32_t* lst,
                                           float* lsd, uint32_t n, uint32_t grp, uint32_t sub) {
  batch_dist<DT, CPL>(rs, av, self_term<DT, CPL>(av), lst, lsd, n, grp, sub);
}

// ---------------------------------------------------------------------------
// int8 MFMA operands (v_mfma_i32_32x32x32_i8: 16 bytes of K per lane).
// ---------------------------------------------------------------------------
typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef int v16i_t __attribute__((ext_vector_type(16)));

// v_writelane_b32: lane L of `words` takes the wave-uniform value v; the
// other lanes keep theirs.
template <uint32_t L>
__device__ __forceinline__ uint32_t write_lane(uint32_t words, uint32_t v) {
  static_assert(L < 64u, "lane index");
  asm volatile("v_writelane_b32 %0, %1, %2" : "+v"(words) : "s"(v), "n"(L));
  return words;
}

// f(integral_constant<uint32_t, 0>) ... f(integral_constant<uint32_t, N-1>).
template <uint32_t I, uint32_t N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<uint32_t, I>{});
    static_for<I + 1, N>(f);
  }
}

// Bytes 32 step + 16 (lane / 32) .. +16 of uint8 row `id`, shifted by -128
// (b ^ 0x80 maps [0, 255] onto int8): one MFMA operand fragment, row id
// supplied by lane l for tile row l % 32. Rows are zero padded to their
// chunk group (8 CPL chunks), so steps < 4 CPL stay inside the row; padding
// bytes become -128 in every row and add nothing to a pair's distance.
__device__ __forceinline__ v4i_t u8_frag(const RowSet& rs, uint32_t id, uint32_t step, uint32_t lane) {
  const uint4 c = rs.rows[(size_t)id * rs.stride16 + 2u * step + (lane >> 5)];
  return v4i_t{(int)(c.x ^ 0x80808080u), (int)(c.y ^ 0x80808080u), (int)(c.z ^ 0x80808080u),
               (int)(c.w ^ 0x80808080u)};
}

// acc + the sum of squares of a fragment's 16 int8 values (exact).
__device__ __forceinline__ int i8_sq4(const v4i_t& f, int acc) {
  acc = __builtin_amdgcn_sdot4(f.x, f.x, acc, false);
  acc = __builtin_amdgcn_sdot4(f.y, f.y, acc, false);
  acc = __builtin_amdgcn_sdot4(f.z, f.z, acc, false);
  return __builtin_amdgcn_sdot4(f.w, f.w, acc, false);
}

// Exact uint8 squared distance from a Gram entry: |a'|^2 + |b'|^2 - 2 a'.b'
// over the shifted rows equals sum (a - b)^2 as an integer (32-bit
// wrap-around included), converted to float once, as octet_finish does.
__device__ __forceinline__ float u8_gram_dist(int na, int nb, int dot) {
  return (float)((uint32_t)na + (uint32_t)nb - 2u * (uint32_t)dot);
}

