// CPU oracle for the DANCE GPU Vamana construction path.
//
// TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP build in
// dance_amd/: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
// leg may load it. No product code links or calls it.
//
// It restates, sequentially and per vertex, the algorithm of the reference
// standard builder ("vnew2"), /root/reference/src/gpu_vamana_vnew2.cu, with the
// effective compile-time configuration of include/gpu_vamana_config.h (QUALITY
// and FAST_SMALL profiles). Every function cites the reference lines it follows.
//
// Two points are fixed by this build rather than by the reference:
//  * Canonical distance arithmetic (dist_* below). The reference's fp32 sums
//    depend on warp-shuffle order and NVCC contraction; the HIP kernels and this
//    oracle both implement the order specified here, so they agree bit for bit.
//  * Canonical reverse-edge order: the reference fills its reverse CSR through
//    atomic cursors (vnew2.cu:1632-1661), so segment order is arrival order.
//    Here every segment is in ascending source id (the order a stable device
//    radix sort produces).
//
// Parity status per function is recorded in the header of oracle/oracle.py.

#include <algorithm>
#include <atomic>
#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <numeric>
#include <vector>
#include <omp.h>

namespace {

constexpr uint32_t INV = 0xFFFFFFFFu;
enum DType : int { DT_F32 = 0, DT_U8 = 1, DT_F16 = 2 };

// ---------------------------------------------------------------------------
// Hashes (vnew2.cu:169-191).
// ---------------------------------------------------------------------------
inline uint32_t hash_u32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

inline uint32_t det_neighbor(uint32_t node, uint32_t k, uint32_t N) {
  if (N <= 1) return INV;
  uint32_t h = hash_u32(node * 0x9e3779b1u + k * 0x85ebca6bu + 17u);
  uint32_t v = h % N;
  if (v == node) v = (v + 1u) % N;
  return v;
}

// ---------------------------------------------------------------------------
// Canonical squared-L2 distance.
//
// The row is cut into 16-byte chunks (4 fp32, 8 fp16 or 16 uint8 elements).
// Sub-lane j in [0,8) owns chunks j, j+8, j+16, ... and walks its elements in
// ascending order.
//  * fp32 accumulates p_j = fmaf(t, t, p_j) with t = a_e - b_e rounded to fp32.
//  * fp16 follows the reference's element arithmetic (vnew2.cu:391-418,
//    filtered.cu:4036-4047): for each pair of elements (2e, 2e+1), the
//    differences and squares are binary16 operations (__hsub2, __hmul2: round
//    to nearest even, overflow to inf); the two squares are widened and added
//    in fp32 and that pair sum is added to p_j. For odd dim the last element is
//    widened first: t = float(a) - float(b), p_j = fmaf(t, t, p_j) (the
//    reference's `sum += delta * delta` tail, :404-410).
//  * The eight partials are combined as ((p0+p7)+(p2+p5)) + ((p1+p6)+(p3+p4)),
//    the DPP tree of the HIP kernels (half-row mirror, then quad swaps by 2
//    and by 1).
//  * uint8 sums (a-b)^2 exactly in integers, like the reference's dp4a form
//    xx+yy-2xy (vnew2.cu:268-290), and converts once.
// ---------------------------------------------------------------------------
inline float half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      // subnormal half -> normal float
      int e = -1;
      do { man <<= 1; ++e; } while ((man & 0x400u) == 0);
      man &= 0x3FFu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 0x1F) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

inline float combine8(const float p[8]) {
  return ((p[0] + p[7]) + (p[2] + p[5])) + ((p[1] + p[6]) + (p[3] + p[4]));
}

float dist_f32(const float* a, const float* b, uint32_t dim) {
  const uint32_t E = 4;
  const uint32_t nch = (dim + E - 1) / E;
  float p[8];
  for (uint32_t j = 0; j < 8; ++j) {
    float acc = 0.0f;
    for (uint32_t c = j; c < nch; c += 8) {
      const uint32_t e1 = std::min(c * E + E, dim);
      for (uint32_t e = c * E; e < e1; ++e) {
        float t = a[e] - b[e];
        acc = fmaf(t, t, acc);
      }
    }
    p[j] = acc;
  }
  return combine8(p);
}

// IEEE binary16 rounding (to nearest, ties to even) of a double. Every value
// rounded here is exact in double (a difference or product of two binary16
// values), so this is the single rounding of the binary16 operation.
uint16_t half_round(double x) {
  const uint16_t sign = std::signbit(x) ? 0x8000u : 0u;
  if (std::isnan(x)) return (uint16_t)(sign | 0x7E00u);
  const double ax = std::fabs(x);
  if (ax >= 65520.0) return (uint16_t)(sign | 0x7C00u);  // max finite 65504; the tie 65520 goes to even (inf)
  if (ax < 0x1p-14) {
    // subnormal range: multiples of 2^-24; 1024 * 2^-24 is the smallest
    // normal, whose encoding 0x0400 the integer already is
    return (uint16_t)(sign | (uint16_t)std::nearbyint(ax * 0x1p24));
  }
  int e = 0;
  std::frexp(ax, &e);  // ax in [2^(e-1), 2^e)
  int E = e - 1;
  double m = std::nearbyint(std::ldexp(ax, 10 - E));  // [1024, 2048]
  if (m >= 2048.0) {
    m = 1024.0;
    ++E;
  }
  if (E > 15) return (uint16_t)(sign | 0x7C00u);
  return (uint16_t)(sign | (uint16_t)((E + 15) << 10) | (uint16_t)((int)m - 1024));
}

// __hmul2(__hsub2(a, b), same) on one element, widened.
inline float half_sq_of_diff(uint16_t a, uint16_t b) {
  const uint16_t t = half_round((double)half_to_float(a) - (double)half_to_float(b));
  const double tf = (double)half_to_float(t);
  return half_to_float(half_round(tf * tf));
}

float dist_f16(const uint16_t* a, const uint16_t* b, uint32_t dim) {
  const uint32_t E = 8;
  const uint32_t nch = (dim + E - 1) / E;
  float p[8];
  for (uint32_t j = 0; j < 8; ++j) {
    float acc = 0.0f;
    for (uint32_t c = j; c < nch; c += 8) {
      const uint32_t e1 = std::min(c * E + E, dim);
      for (uint32_t e = c * E; e < e1; e += 2) {
        if (e + 1 == dim) {  // odd dim: the last element alone, in fp32
          const float t = half_to_float(a[e]) - half_to_float(b[e]);
          acc = fmaf(t, t, acc);
        } else {
          acc = acc + (half_sq_of_diff(a[e], b[e]) + half_sq_of_diff(a[e + 1], b[e + 1]));
        }
      }
    }
    p[j] = acc;
  }
  return combine8(p);
}

float dist_u8(const uint8_t* a, const uint8_t* b, uint32_t dim) {
  int64_t s = 0;
  for (uint32_t e = 0; e < dim; ++e) {
    int d = (int)a[e] - (int)b[e];
    s += d * d;
  }
  return (float)(uint32_t)s;
}

}  // namespace

extern "C" uint16_t oracle_half_round(double x) { return half_round(x); }
extern "C" float oracle_half_sq_of_diff(uint16_t a, uint16_t b) { return half_sq_of_diff(a, b); }

namespace {

struct Data {
  const void* ptr;
  int dtype;
  uint32_t N;
  uint32_t dim;
  float operator()(uint32_t a, uint32_t b) const {
    switch (dtype) {
      case DT_F32: {
        const float* p = (const float*)ptr;
        return dist_f32(p + (size_t)a * dim, p + (size_t)b * dim, dim);
      }
      case DT_U8: {
        const uint8_t* p = (const uint8_t*)ptr;
        return dist_u8(p + (size_t)a * dim, p + (size_t)b * dim, dim);
      }
      default: {
        const uint16_t* p = (const uint16_t*)ptr;
        return dist_f16(p + (size_t)a * dim, p + (size_t)b * dim, dim);
      }
    }
  }
};

inline bool valid_for(uint32_t id, uint32_t N, uint32_t node) {
  return id != INV && id < N && id != node;
}

// ---------------------------------------------------------------------------
// Bounded top-L candidate pool (vnew2.cu:520-734): ids, dists, expanded flags,
// running max (largest dist, lowest slot on ties). Early reject is on
// (ENABLE_TOPL_EARLY_REJECT=1, gpu_vamana_config.h:169-171).
// ---------------------------------------------------------------------------
struct Pool {
  uint32_t L;
  std::vector<uint32_t> ids;
  std::vector<float> d;
  std::vector<uint8_t> exp;
  uint32_t size = 0;
  int max_pos = -1;
  float max_d = -FLT_MAX;

  explicit Pool(uint32_t L_) : L(L_), ids(L_, INV), d(L_, FLT_MAX), exp(L_, 0) {}

  // recompute_max_pos_size_warp, vnew2.cu:554-596
  void recompute_max() {
    float m = -FLT_MAX;
    int p = -1;
    for (uint32_t i = 0; i < size; ++i) {
      if (ids[i] == INV) continue;
      if (d[i] > m) {
        m = d[i];
        p = (int)i;
      }
    }
    max_pos = p;
    max_d = m;
  }

  // insert_top_l_state_warp, vnew2.cu:598-697
  void insert(uint32_t id, float dist) {
    if (id == INV) return;
    if (size >= L && max_pos >= 0 && dist >= max_d) return;
    int same = -1;
    for (uint32_t i = 0; i < size; ++i)
      if (ids[i] == id) {
        same = (int)i;
        break;
      }
    if (same >= 0) {
      if (dist < d[same]) {
        d[same] = dist;
        exp[same] = 0;
        if (same == max_pos) recompute_max();
      }
      return;
    }
    if (size < L) {
      uint32_t pos = size;
      ids[pos] = id;
      d[pos] = dist;
      exp[pos] = 0;
      size++;
      if (max_pos < 0 || dist > max_d) {
        max_pos = (int)pos;
        max_d = dist;
      }
      return;
    }
    if (max_pos >= 0 && dist < max_d) {
      ids[max_pos] = id;
      d[max_pos] = dist;
      exp[max_pos] = 0;
      recompute_max();
    }
  }

  // select_next_unexpanded_size_warp, vnew2.cu:699-734
  int select() const {
    float m = FLT_MAX;
    int p = -1;
    for (uint32_t i = 0; i < size; ++i) {
      if (ids[i] != INV && exp[i] == 0 && d[i] < m) {
        m = d[i];
        p = (int)i;
      }
    }
    return p;
  }
};

// cur rows are `cs` entries apart: R for vnew2's packed current graph, C for
// the v8 builder's double-buffered C-stride graphs (0 means R). The prune
// writes cur only when it is given (v8 prunes in place in the work graph).
struct Graph {
  uint32_t N, R, C;
  uint32_t* cur;
  uint32_t* deg_cur;
  uint32_t* work;
  uint32_t* deg_work;
  float* wd;
  uint32_t cs = 0;
  size_t stride() const { return cs ? cs : R; }
};

// dynamic_robust_insert_C_warp, vnew2.cu:759-877 (ENABLE_FAST_ONLINE_REPLACE=0)
void robust_insert_row(const Data& D, uint32_t N, uint32_t C, uint32_t node, uint32_t x, float d_px, float alpha,
                       uint32_t* row, float* drow, uint32_t& deg_io) {
  if (x == INV || x >= N || x == node) return;
  uint32_t deg = std::min(deg_io, C);
  for (uint32_t i = 0; i < deg; ++i)
    if (row[i] == x) return;
  bool occluded = false;
  for (uint32_t i = 0; i < deg && !occluded; ++i) {
    uint32_t y = row[i];
    if (!valid_for(y, N, node)) continue;
    float d_py = drow[i];
    if (d_py <= d_px) {
      float d_yx = D(y, x);
      if (alpha * d_yx <= d_px) occluded = true;
    }
  }
  if (occluded) return;
  int worst_pos = -1;
  float worst_d = -FLT_MAX;
  int victim_pos = -1;
  float victim_d = -FLT_MAX;
  for (uint32_t i = 0; i < deg; ++i) {
    uint32_t y = row[i];
    if (!valid_for(y, N, node)) continue;
    float d_py = drow[i];
    if (d_py > worst_d) {
      worst_d = d_py;
      worst_pos = (int)i;
    }
    if (d_py > d_px) {
      float d_xy = D(x, y);
      if (alpha * d_xy <= d_py && d_py > victim_d) {
        victim_d = d_py;
        victim_pos = (int)i;
      }
    }
  }
  if (victim_pos >= 0) {
    row[victim_pos] = x;
    drow[victim_pos] = d_px;
  } else if (deg < C) {
    row[deg] = x;
    drow[deg] = d_px;
    deg_io = deg + 1;
  } else if (worst_pos >= 0 && d_px < worst_d) {
    row[worst_pos] = x;
    drow[worst_pos] = d_px;
  }
}

void robust_insert(const Data& D, Graph& g, uint32_t node, uint32_t x, float d_px, float alpha) {
  robust_insert_row(D, g.N, g.C, node, x, d_px, alpha, g.work + (size_t)node * g.C, g.wd + (size_t)node * g.C,
                    g.deg_work[node]);
}

// search_prune_kernel_shared, vnew2.cu:1119-1439 (one entry point,
// INIT_RANDOM_SEEDS=8, no active/important masks on the release path).
uint64_t search_one(const Data& D, Graph& g, uint32_t node, uint32_t L, uint32_t steps, float alpha,
                    uint32_t start, uint64_t* n_dist) {
  const uint32_t N = g.N, R = g.R, C = g.C;
  const size_t cb = (size_t)node * g.stride(), wb = (size_t)node * C;
  uint32_t deg_self = std::min(g.deg_cur[node], R);
  // Work row := current row with stored distances (vnew2.cu:1186-1212).
  for (uint32_t i = 0; i < C; ++i) {
    uint32_t nb = INV;
    float dist = FLT_MAX;
    if (i < deg_self) {
      nb = g.cur[cb + i];
      if (valid_for(nb, N, node))
        dist = g.wd[wb + i];
      else
        nb = INV;
    }
    g.work[wb + i] = nb;
    g.wd[wb + i] = dist;
  }
  g.deg_work[node] = deg_self;

  Pool pool(L);
  uint64_t nd = 0;
  if (start < N && start != node) {
    pool.insert(start, D(node, start));
    ++nd;
  }
  for (uint32_t i = 0; i < deg_self; ++i) {
    uint32_t nb = g.cur[cb + i];
    if (valid_for(nb, N, node)) pool.insert(nb, g.wd[wb + i]);
  }
  for (uint32_t k = 0; k < 8; ++k) {
    uint32_t s = det_neighbor(node, k + 1024u, N);
    if (!valid_for(s, N, node)) continue;
    pool.insert(s, D(node, s));
    ++nd;
  }
  uint32_t max_steps = std::min(steps, L);
  uint64_t expansions = 0;
  for (uint32_t step = 0; step < max_steps; ++step) {
    int pos = pool.select();
    if (pos < 0) break;
    uint32_t x = pool.ids[pos];
    float dx = pool.d[pos];
    pool.exp[pos] = 1;
    if (x == INV || x >= N) break;
    ++expansions;
    robust_insert(D, g, node, x, dx, alpha);
    uint32_t deg = std::min(g.deg_cur[x], R);
    const size_t xb = (size_t)x * g.stride();
    for (uint32_t j = 0; j < deg; ++j) {
      uint32_t c = g.cur[xb + j];
      if (!valid_for(c, N, node)) continue;
      pool.insert(c, D(node, c));
      ++nd;
    }
  }
  if (n_dist) *n_dist += nd;
  return expansions;
}

// Reverse-edge CSR (reverse_count_csr_kernel / reverse_fill_csr_kernel,
// vnew2.cu:1604-1661) with segments in ascending source order, then
// reverse_merge_csr_kernel (vnew2.cu:1722-1814).
void reverse_merge(const Data& D, Graph& g, uint32_t heavy_threshold, uint32_t heavy_sample,
                   std::vector<uint32_t>* offsets_out, std::vector<uint32_t>* ids_out) {
  const uint32_t N = g.N, R = g.R, C = g.C;
  std::vector<uint32_t> off((size_t)N + 1, 0);
  for (uint32_t s = 0; s < N; ++s) {
    uint32_t deg = std::min(g.deg_work[s], R);
    const size_t b = (size_t)s * C;
    for (uint32_t i = 0; i < deg; ++i) {
      uint32_t t = g.work[b + i];
      if (t != INV && t < N && t != s) off[(size_t)t + 1]++;
    }
  }
  for (uint32_t t = 0; t < N; ++t) off[(size_t)t + 1] += off[t];
  std::vector<uint32_t> ids(off[N]);
  std::vector<uint32_t> cursor(off.begin(), off.end() - 1);
  for (uint32_t s = 0; s < N; ++s) {  // ascending source = canonical order
    uint32_t deg = std::min(g.deg_work[s], R);
    const size_t b = (size_t)s * C;
    for (uint32_t i = 0; i < deg; ++i) {
      uint32_t t = g.work[b + i];
      if (t != INV && t < N && t != s) ids[cursor[t]++] = s;
    }
  }
#pragma omp parallel for schedule(dynamic, 256)
  for (int64_t tt = 0; tt < (int64_t)N; ++tt) {
    uint32_t t = (uint32_t)tt;
    uint32_t* row = g.work + (size_t)t * C;
    float* drow = g.wd + (size_t)t * C;
    uint32_t deg = std::min(g.deg_work[t], C);
    uint32_t begin = off[t], end = off[(size_t)t + 1];
    uint32_t indeg = end - begin;
    uint32_t count = indeg;
    if (heavy_threshold != 0 && indeg > heavy_threshold) {
      count = std::min(heavy_sample, indeg);
      if (count == 0) count = 1;
    }
    for (uint32_t si = 0; si < count; ++si) {
      uint32_t i = begin + si;
      if (count < indeg) i = begin + (uint32_t)(((uint64_t)si * indeg) / count);
      uint32_t src = ids[i];
      if (src == INV || src >= N || src == t) continue;
      bool found = false;
      for (uint32_t p = 0; p < deg; ++p)
        if (row[p] == src) {
          found = true;
          break;
        }
      if (found) continue;
      float dist = D(t, src);
      if (deg < C) {
        row[deg] = src;
        drow[deg] = dist;
        deg++;
        continue;
      }
      float wdist = -FLT_MAX;
      int wpos = -1;
      for (uint32_t p = 0; p < C; ++p)
        if (drow[p] > wdist) {
          wdist = drow[p];
          wpos = (int)p;
        }
      if (wpos >= 0 && dist < wdist) {
        row[wpos] = src;
        drow[wpos] = dist;
      }
    }
    g.deg_work[t] = deg;
  }
  if (offsets_out) *offsets_out = std::move(off);
  if (ids_out) *ids_out = std::move(ids);
}

// final_prune_kernel_shared, vnew2.cu:1893-2147: RobustPrune of the work row
// to R with alpha, plus the minimum-degree fill used in the last iteration.
void prune_one(const Data& D, Graph& g, uint32_t node, uint32_t min_degree, float alpha) {
  const uint32_t N = g.N, R = g.R, C = g.C;
  const size_t wb = (size_t)node * C, cb = (size_t)node * g.stride();
  uint32_t deg = std::min(g.deg_work[node], C);
  std::vector<uint32_t> sid(C);
  std::vector<float> sd(C);
  std::vector<uint8_t> rem(C);
  for (uint32_t i = 0; i < C; ++i) {
    uint32_t id = INV;
    float dist = FLT_MAX;
    uint8_t r = 1;
    if (i < deg) {
      id = g.work[wb + i];
      dist = g.wd[wb + i];
      if (valid_for(id, N, node) && dist < FLT_MAX)
        r = 0;
      else
        id = INV;
    }
    sid[i] = id;
    sd[i] = dist;
    rem[i] = r;
  }
  std::vector<uint32_t> out_id;
  std::vector<float> out_d;
  out_id.reserve(R);
  out_d.reserve(R);
  for (uint32_t round = 0; round < R; ++round) {
    float bd = FLT_MAX;
    int bp = -1;
    for (uint32_t p = 0; p < C; ++p) {
      if (rem[p] != 0) continue;
      uint32_t id = sid[p];
      if (!valid_for(id, N, node)) continue;
      if (sd[p] < bd || (sd[p] == bd && bp < 0)) {
        bd = sd[p];
        bp = (int)p;
      }
    }
    if (bp < 0) break;
    uint32_t sel = sid[bp];
    float seld = sd[bp];
    if (!valid_for(sel, N, node)) break;
    out_id.push_back(sel);
    out_d.push_back(seld);
    if (out_id.size() >= R) break;
    for (uint32_t i = 0; i < C; ++i)
      if (rem[i] == 0 && sid[i] == sel) rem[i] = 1;
    for (uint32_t q = 0; q < C; ++q) {
      if (rem[q] != 0) continue;
      uint32_t qid = sid[q];
      if (!valid_for(qid, N, node)) continue;
      float qd = sd[q];
      if (seld <= qd) {
        float dsq = D(sel, qid);
        if (alpha * dsq <= qd) rem[q] = 1;
      }
    }
  }
  uint32_t md = std::min(min_degree, R);
  while (out_id.size() < md) {
    float bd = FLT_MAX;
    int bp = -1;
    for (uint32_t p = 0; p < C; ++p) {
      uint32_t id = sid[p];
      if (!valid_for(id, N, node)) continue;
      bool dup = false;
      for (uint32_t o : out_id)
        if (o == id) {
          dup = true;
          break;
        }
      if (dup) continue;
      if (sd[p] < bd || (sd[p] == bd && bp < 0)) {
        bd = sd[p];
        bp = (int)p;
      }
    }
    if (bp < 0) break;
    out_id.push_back(sid[bp]);
    out_d.push_back(sd[bp]);
    sid[bp] = INV;
  }
  const uint32_t oc = (uint32_t)out_id.size();
  for (uint32_t i = 0; i < C; ++i) {
    g.work[wb + i] = i < oc ? out_id[i] : INV;
    g.wd[wb + i] = i < oc ? out_d[i] : FLT_MAX;
  }
  if (g.cur)
    for (uint32_t i = 0; i < R; ++i) g.cur[cb + i] = i < oc ? out_id[i] : INV;
  g.deg_work[node] = oc;
  if (g.deg_cur) g.deg_cur[node] = oc;
}

// medoid_score_kernel_warp + host top-1, vnew2.cu:1032-1064, 2359-2479.
uint32_t medoid(const Data& D, float* scores_out, uint32_t* cand_out) {
  const uint32_t N = D.N;
  uint32_t nc = std::min<uint32_t>(1024u, N), ns = std::min<uint32_t>(4096u, N);
  std::vector<float> sc(nc);
  std::vector<uint32_t> ci(nc);
#pragma omp parallel for schedule(dynamic, 8)
  for (int64_t ww = 0; ww < (int64_t)nc; ++ww) {
    uint32_t w = (uint32_t)ww;
    uint32_t c = hash_u32(w * 9973u + 17u) % N;
    float sum = 0.0f;
    for (uint32_t s = 0; s < ns; ++s) {
      uint32_t smp = hash_u32(s * 10007u + 131u) % N;
      if (smp == c) continue;
      sum += D(c, smp);
    }
    sc[w] = sum / (float)ns;
    ci[w] = c;
  }
  uint32_t best = INV;
  float bs = FLT_MAX;
  for (uint32_t i = 0; i < nc; ++i)
    if (sc[i] < bs) {
      bs = sc[i];
      best = i;
    }
  if (scores_out) std::memcpy(scores_out, sc.data(), nc * sizeof(float));
  if (cand_out) std::memcpy(cand_out, ci.data(), nc * sizeof(uint32_t));
  return best == INV ? 0u : ci[best];
}

// init_random_graph, vnew2.cu:1066-1117.
void init_graph(const Data& D, Graph& g) {
  const uint32_t N = g.N, R = g.R, C = g.C;
#pragma omp parallel for schedule(static)
  for (int64_t nn = 0; nn < (int64_t)N; ++nn) {
    uint32_t node = (uint32_t)nn;
    const size_t cb = (size_t)node * g.stride(), wb = (size_t)node * C;
    for (uint32_t i = 0; i < C; ++i) {
      g.work[wb + i] = INV;
      g.wd[wb + i] = FLT_MAX;
      if (i < g.stride()) g.cur[cb + i] = INV;
    }
    for (uint32_t i = 0; i < R; ++i) {
      uint32_t nb = det_neighbor(node, i, N);
      if (N <= 1 || nb == INV || nb >= N || nb == node) nb = INV;
      float dist = FLT_MAX;
      if (nb != INV) dist = D(node, nb);
      g.cur[cb + i] = nb;
      g.work[wb + i] = nb;
      g.wd[wb + i] = dist;
    }
    uint32_t deg = N > 1 ? R : 0;
    g.deg_cur[node] = deg;
    g.deg_work[node] = deg;
  }
}

// gpu_vamana_alpha_for_iter, vnew2.cu:201-213: alpha from iteration
// `from` on (default: the last iteration only; 0 = USE_ALPHA_FROM_FIRST_ITER,
// k = VAMANA_ALPHA_FINAL_FROM_ITER=k).
float alpha_for_iter(uint32_t iter, uint32_t from, float alpha) { return iter >= from ? alpha : 1.0f; }

}  // namespace

// ===========================================================================
// extern "C" surface used by oracle/oracle.py
// ===========================================================================
extern "C" {

uint32_t oracle_hash_u32(uint32_t x) { return hash_u32(x); }
uint32_t oracle_det_neighbor(uint32_t node, uint32_t k, uint32_t N) { return det_neighbor(node, k, N); }

// Canonical distance of two rows given by pointer (a query row and a base row).
float oracle_distance_rows(const void* a, const void* b, int dtype, uint32_t dim) {
  switch (dtype) {
    case DT_F32: return dist_f32((const float*)a, (const float*)b, dim);
    case DT_U8: return dist_u8((const uint8_t*)a, (const uint8_t*)b, dim);
    default: return dist_f16((const uint16_t*)a, (const uint16_t*)b, dim);
  }
}

float oracle_distance(const void* data, int dtype, uint32_t dim, uint32_t a, uint32_t b) {
  Data D{data, dtype, 0xFFFFFFFFu, dim};
  return D(a, b);
}

void oracle_distance_many(const void* data, int dtype, uint32_t dim, const uint32_t* a, const uint32_t* b,
                          uint64_t n, float* out) {
  Data D{data, dtype, 0xFFFFFFFFu, dim};
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)n; ++i) out[i] = D(a[i], b[i]);
}

uint32_t oracle_medoid(const void* data, int dtype, uint32_t N, uint32_t dim, float* scores,
                       uint32_t* cands) {
  Data D{data, dtype, N, dim};
  return medoid(D, scores, cands);
}

void oracle_init_graph(const void* data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t C,
                       uint32_t* cur, uint32_t* deg_cur, uint32_t* work, uint32_t* deg_work, float* wd) {
  Data D{data, dtype, N, dim};
  Graph g{N, R, C, cur, deg_cur, work, deg_work, wd};
  init_graph(D, g);
}

// One search + online-insert pass over every vertex (vnew2.cu:2538-2561).
uint64_t oracle_search(const void* data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t L,
                       uint32_t C, uint32_t steps, float alpha, uint32_t start, uint32_t* cur,
                       uint32_t* deg_cur, uint32_t* work, uint32_t* deg_work, float* wd) {
  Data D{data, dtype, N, dim};
  Graph g{N, R, C, cur, deg_cur, work, deg_work, wd};
  uint64_t total = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : total)
  for (int64_t nn = 0; nn < (int64_t)N; ++nn) {
    uint64_t nd = 0;
    search_one(D, g, (uint32_t)nn, L, steps, alpha, start, &nd);
    total += nd;
  }
  return total;
}

// One online robust insert of x (distance d_px to node) into node's work
// row (ids, dists, degree) of capacity C (vnew2.cu:759-877), for the tests.
void oracle_robust_insert(const void* data, int dtype, uint32_t N, uint32_t dim, uint32_t C, uint32_t node,
                          uint32_t x, float d_px, float alpha, uint32_t* row, float* drow, uint32_t* deg) {
  Data D{data, dtype, N, dim};
  robust_insert_row(D, N, C, node, x, d_px, alpha, row, drow, *deg);
}

// Reverse CSR + merge (vnew2.cu:2569-2611). offsets (N+1) and ids (<= N*R)
// receive the canonical CSR when non-null.
uint64_t oracle_reverse_merge(const void* data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t C,
                              uint32_t* work, uint32_t* deg_work, float* wd, uint32_t heavy_threshold,
                              uint32_t heavy_sample, uint32_t* offsets, uint32_t* ids) {
  Data D{data, dtype, N, dim};
  Graph g{N, R, C, nullptr, nullptr, work, deg_work, wd};
  std::vector<uint32_t> off, rid;
  reverse_merge(D, g, heavy_threshold, heavy_sample, &off, &rid);
  if (offsets) std::memcpy(offsets, off.data(), off.size() * sizeof(uint32_t));
  if (ids) std::memcpy(ids, rid.data(), rid.size() * sizeof(uint32_t));
  return rid.size();
}

void oracle_prune(const void* data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t C,
                  uint32_t min_degree, float alpha, uint32_t* work, uint32_t* deg_work, float* wd,
                  uint32_t* cur, uint32_t* deg_cur) {
  Data D{data, dtype, N, dim};
  Graph g{N, R, C, cur, deg_cur, work, deg_work, wd};
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t nn = 0; nn < (int64_t)N; ++nn) prune_one(D, g, (uint32_t)nn, min_degree, alpha);
}

// Full standard build (gpu_vamana_build_impl, vnew2.cu:2170-2855).
// Returns 0 on success, -1 on invalid parameters (same checks as vnew2.cu:2176-2204).
int oracle_vnew2_build(const void* data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t L,
                       uint32_t C, uint32_t STEPS, uint32_t iters, float alpha, uint32_t alpha_from,
                       uint32_t heavy_threshold, uint32_t heavy_sample, uint32_t* graph_out, uint32_t* degree_out,
                       uint32_t* medoid_out) {
  if (data == nullptr || graph_out == nullptr || degree_out == nullptr) return -1;
  if (N == 0 || dim == 0 || R == 0 || L == 0 || C == 0 || STEPS == 0) return -1;
  if (C < R) return -1;
  if (STEPS > L) STEPS = L;
  Data D{data, dtype, N, dim};
  std::vector<uint32_t> work((size_t)N * C), deg_work(N), deg_cur(N);
  std::vector<float> wd((size_t)N * C);
  Graph g{N, R, C, graph_out, deg_cur.data(), work.data(), deg_work.data(), wd.data()};
  uint32_t start = medoid(D, nullptr, nullptr);
  init_graph(D, g);
  for (uint32_t it = 0; it < iters; ++it) {
    float a = alpha_for_iter(it, alpha_from, alpha);
    uint32_t steps = STEPS;
    // ENABLE_COARSE_TO_FINE_STEPS: WARMUP_EXPAND_STEPS=64 for COARSE_WARMUP_ITERS=2 (config.h:66-77).
    if (it < 2 && steps > 64) steps = 64;
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t nn = 0; nn < (int64_t)N; ++nn) search_one(D, g, (uint32_t)nn, L, steps, a, start, nullptr);
    reverse_merge(D, g, heavy_threshold, heavy_sample, nullptr, nullptr);
    uint32_t md = (it + 1 == iters) ? 64u : 0u;
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t nn = 0; nn < (int64_t)N; ++nn) prune_one(D, g, (uint32_t)nn, md, a);
  }
  std::memcpy(degree_out, deg_cur.data(), (size_t)N * sizeof(uint32_t));
  if (medoid_out) *medoid_out = start;
  return 0;
}

// Full v8 build (gpu_vamana_build_impl, gpu_vamana_uint8.cu:2437-3090) with
// its own buffer scheme: two C-stride graphs initialised alike and one
// distance array (init_random_graph, uint8.cu:1074-1121); each search copies
// the current graph's row into the next graph (uint8.cu:1173-1198) and expands
// the current graph's C-stride rows; the reverse merge (reverse_merge_csr_kernel,
// uint8.cu:1795-1940, no heavy cap: v8 has none) and the prune
// (final_prune_kernel_shared, uint8.cu:2020-2298) work in place on the next
// graph; the graphs swap after every iteration (uint8.cu:2936-2942). The
// output is the first R entries of every current row (cudaMemcpy2D,
// uint8.cu:3046). Parameter checks as uint8.cu:2443-2466.
int oracle_v8_build(const void* data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t L, uint32_t C,
                    uint32_t STEPS, uint32_t iters, float alpha, uint32_t alpha_from, uint32_t* graph_out,
                    uint32_t* degree_out, uint32_t* medoid_out) {
  if (data == nullptr || graph_out == nullptr || degree_out == nullptr) return -1;
  if (N == 0 || dim == 0 || R == 0 || L == 0 || C == 0 || STEPS == 0) return -1;
  if (C < R) return -1;
  if (STEPS > L) STEPS = L;
  Data D{data, dtype, N, dim};
  std::vector<uint32_t> ga((size_t)N * C), gb((size_t)N * C), da(N), db(N);
  std::vector<float> dists((size_t)N * C);
  uint32_t start = medoid(D, nullptr, nullptr);
  {
    Graph g0{N, R, C, ga.data(), da.data(), gb.data(), db.data(), dists.data(), C};
    init_graph(D, g0);
  }
  uint32_t *cur = ga.data(), *dcur = da.data(), *next = gb.data(), *dnext = db.data();
  for (uint32_t it = 0; it < iters; ++it) {
    float a = alpha_for_iter(it, alpha_from, alpha);
    uint32_t steps = STEPS;
    if (it < 2 && steps > 64) steps = 64;  // ENABLE_COARSE_TO_FINE_STEPS (uint8.cu:2788-2791)
    Graph g{N, R, C, cur, dcur, next, dnext, dists.data(), C};
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t nn = 0; nn < (int64_t)N; ++nn) search_one(D, g, (uint32_t)nn, L, steps, a, start, nullptr);
    reverse_merge(D, g, 0, 0, nullptr, nullptr);
    Graph gp{N, R, C, nullptr, nullptr, next, dnext, dists.data(), C};
    const uint32_t md = (it + 1 == iters) ? 64u : 0u;  // FINAL_MIN_DEGREE in the last iteration (uint8.cu:2871-2874)
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t nn = 0; nn < (int64_t)N; ++nn) prune_one(D, gp, (uint32_t)nn, md, a);
    std::swap(cur, next);
    std::swap(dcur, dnext);
  }
  for (uint32_t n = 0; n < N; ++n)
    std::memcpy(graph_out + (size_t)n * R, cur + (size_t)n * C, (size_t)R * sizeof(uint32_t));
  std::memcpy(degree_out, dcur, (size_t)N * sizeof(uint32_t));
  if (medoid_out) *medoid_out = start;
  return 0;
}

int oracle_num_threads(void) { return omp_get_max_threads(); }

}  // extern "C"
