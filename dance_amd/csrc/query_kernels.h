// Query-time best-first search over a built graph (DiskANN
// search_memory_index semantics, optional single-label filter) for gfx950.
//
// One wave64 per query. The candidate list holds the L smallest
// (distance, id) seen so far, PS slots per lane (entry p = slot p / 64 of
// lane p % 64; PS = 1 .. 16 covers L up to 1024), unsorted: the worst entry
// is tracked for rejection and replacement, and expansion takes the smallest
// unexpanded entry, which is exactly the first unexpanded position of
// DiskANN's sorted list. The
// visited set is a forgetful LDS cache; it is transparent because a node
// still in the list is found by the duplicate check and a node that left the
// list (or never entered it) is rejected again: once the list is full its
// worst entry only falls.
#pragma once

#include "wave.h"

namespace dance {
namespace qs {

constexpr uint32_t kVisBits = 11;
constexpr uint32_t kVis = 1u << kVisBits;
constexpr uint32_t kWaves = 4;
constexpr uint32_t kBlock = 64 * kWaves;
constexpr uint32_t kLds = kVis + 128u;  // words per wave
constexpr uint32_t kMaxK = 64;

template <int PS>
struct QPool {
  uint32_t id[PS];
  float d[PS];
  uint32_t ex;  // bit s: slot s expanded
  uint32_t count, cap;
  int wlane, wslot;
  float wd;
  uint32_t wid;

  __device__ __forceinline__ void init(uint32_t c) {
#pragma unroll
    for (int s = 0; s < PS; ++s) {
      id[s] = DANCE_INV;
      d[s] = FLT_MAX;
    }
    ex = 0;
    count = 0;
    cap = c;
    wlane = -1;
    wslot = 0;
    wd = -FLT_MAX;
    wid = 0;
  }
  __device__ __forceinline__ bool valid(int s, uint32_t lane) const { return (uint32_t)s * 64u + lane < count; }

  __device__ __forceinline__ void recompute_worst(uint32_t lane) {
    int lk = INT_MIN, ls = 0;
    uint32_t li = 0;
#pragma unroll
    for (int s = 0; s < PS; ++s) {
      if (valid(s, lane)) {
        const int k = fkey(d[s]);
        if (k > lk || (k == lk && id[s] > li)) {
          lk = k;
          li = id[s];
          ls = s;
        }
      }
    }
    const int M = wave_max_i(lk);
    if (M == INT_MIN) {
      wlane = -1;
      return;
    }
    const uint32_t W = wave_max_u(lk == M ? li : 0u);
    wlane = ffs64(wballot(lk == M && li == W));
    wslot = __builtin_amdgcn_readlane(ls, wlane);
    wd = __int_as_float(M);
    wid = W;
  }
  __device__ __forceinline__ bool full_reject(float nd, uint32_t nid) const {
    return count >= cap && !(nd < wd || (nd == wd && nid < wid));
  }
  __device__ __forceinline__ void insert(uint32_t nid, float nd, uint32_t lane) {
    uint64_t dup = 0;
#pragma unroll
    for (int s = 0; s < PS; ++s) dup |= wballot(valid(s, lane) && id[s] == nid);
    if (dup) return;
    if (count < cap) {
      const uint32_t p = count;
      if (lane == (p & 63u)) {
#pragma unroll
        for (int s = 0; s < PS; ++s)
          if ((uint32_t)s == (p >> 6)) {
            id[s] = nid;
            d[s] = nd;
          }
        ex &= ~(1u << (p >> 6));
      }
      ++count;
      if (wlane < 0 || nd > wd || (nd == wd && nid > wid)) {
        wlane = (int)(p & 63u);
        wslot = (int)(p >> 6);
        wd = nd;
        wid = nid;
      }
      return;
    }
    if (!(nd < wd || (nd == wd && nid < wid))) return;
    if ((int)lane == wlane) {
#pragma unroll
      for (int s = 0; s < PS; ++s)
        if (s == wslot) {
          id[s] = nid;
          d[s] = nd;
        }
      ex &= ~(1u << wslot);
    }
    recompute_worst(lane);
  }
  // Smallest unexpanded (distance, id): returns the lane, slot in *slot, or -1.
  __device__ __forceinline__ int select(uint32_t lane, int* slot, uint32_t* sid) const {
    int lk = INT_MAX, ls = 0;
    uint32_t li = DANCE_INV;
#pragma unroll
    for (int s = 0; s < PS; ++s) {
      if (valid(s, lane) && !((ex >> s) & 1u)) {
        const int k = fkey(d[s]);
        if (k < lk || (k == lk && id[s] < li)) {
          lk = k;
          li = id[s];
          ls = s;
        }
      }
    }
    const uint64_t any = wballot(lk != INT_MAX || li != DANCE_INV);
    if (!any) return -1;
    const int M = wave_min_i(lk);
    const uint32_t I = wave_min_u(lk == M ? li : DANCE_INV);
    const int l = ffs64(wballot(lk == M && li == I && ((any >> lane) & 1ull)));
    *slot = __builtin_amdgcn_readlane(ls, l);
    *sid = I;
    return l;
  }
};

struct QArgs {
  uint32_t N, R;
  const uint32_t* g;
  const uint32_t* deg;
  const uint32_t* starts;
  uint32_t nstarts;
  const uint32_t* start_off;  // nq + 1 (nullptr: starts[0] shared, or starts[q])
  uint32_t nq, k, L, max_expansions;
  const uint32_t* off;   // label CSR (nullptr: no filter)
  const uint32_t* lab;
  const uint32_t* qlab;  // one label per query
  uint32_t* out_ids;     // nq x k
  float* out_d;
  unsigned long long* ctr;  // distances, expansions, capped queries
};

__device__ __forceinline__ bool q_has_label(const QArgs& a, uint32_t p, uint32_t l) {
  const uint32_t e = a.off[p + 1];
  for (uint32_t i = a.off[p]; i < e; ++i) {
    const uint32_t v = a.lab[i];
    if (v == l) return true;
    if (v > l) break;
  }
  return false;
}

template <int DT, int CPL, int PS>
__global__ __launch_bounds__(kBlock) void k_query(RowSet base, RowSet qrows, QArgs a) {
  extern __shared__ uint32_t smem[];
  const uint32_t w = wave_index();
  const uint32_t q = blockIdx.x * kWaves + w;
  if (q >= a.nq) return;
  const uint32_t lane = lane_id(), grp = lane >> 3, sub = lane & 7u;
  uint32_t* vis = smem + w * kLds;
  uint32_t* lst = vis + kVis;
  float* lsd = reinterpret_cast<float*>(lst + 64);
  for (uint32_t i = lane; i < kVis; i += 64) vis[i] = DANCE_INV;
  uint4 av[CPL];
  load_row<CPL>(qrows, q, true, sub, av);
  wave_sync();
  QPool<PS> P;
  P.init(a.L);
  const bool filt = a.off != nullptr;
  const uint32_t ql = filt ? a.qlab[q] : DANCE_INV;
  uint32_t ndist = 0, nexp = 0;
  // One batch of candidates (lane order = insertion order); start nodes skip
  // the label check.
  auto batch = [&](uint32_t c, bool check_label) {
    const bool v = c < a.N && (!filt || !check_label || q_has_label(a, c, ql));
    const uint32_t slot = (c * 0x9E3779B1u) >> (32 - kVisBits);
    const bool need = v && vis[slot] != c;
    const uint64_t m = wballot(need);
    if (m) {
      const uint32_t n = popc64(m);
      if (need) lst[mbcnt64(m)] = c;
      wave_sync();
      batch_dist<DT, CPL>(base, av, lst, lsd, n, grp, sub);
      ndist += n;
      const uint32_t ck = lane < n ? lst[lane] : DANCE_INV;
      const float dk = lane < n ? lsd[lane] : FLT_MAX;
      uint64_t km = wballot(lane < n && !P.full_reject(dk, ck));
      while (km) {
        const int k = ffs64(km);
        km &= km - 1;
        P.insert(rdlane_u(ck, k), rdlane_f(dk, k), lane);
      }
    }
    if (need) vis[slot] = c;
    wave_sync();
  };
  // The start nodes (the label's entry points) go in first, 64 at a time,
  // without the label check.
  {
    const uint32_t b0 = a.start_off ? a.start_off[q] : (a.nstarts == 1 ? 0u : q);
    const uint32_t b1 = a.start_off ? a.start_off[q + 1] : b0 + 1u;
    for (uint32_t b = b0; b < b1; b += 64) batch(b + lane < b1 ? a.starts[b + lane] : DANCE_INV, false);
  }
  bool capped = false;
  while (true) {
    int slot;
    uint32_t u;
    const int l = P.select(lane, &slot, &u);
    if (l < 0) break;
    if (nexp >= a.max_expansions) {
      capped = true;
      break;
    }
    if ((int)lane == l) P.ex |= 1u << slot;
    ++nexp;
    const uint32_t du = min(a.deg[u], a.R);
    const size_t b = (size_t)u * a.R;
    for (uint32_t j = 0; j < du; j += 64) batch(j + lane < du ? a.g[b + j + lane] : DANCE_INV, true);
  }
  // k best in (distance, id) order: lane i receives the i-th.
  uint32_t taken = 0, oid = DANCE_INV;
  float od = FLT_MAX;
  for (uint32_t i = 0; i < a.k; ++i) {
    int lk = INT_MAX, ls = 0;
    uint32_t li = DANCE_INV;
#pragma unroll
    for (int s = 0; s < PS; ++s) {
      if (P.valid(s, lane) && !((taken >> s) & 1u)) {
        const int k = fkey(P.d[s]);
        if (k < lk || (k == lk && P.id[s] < li)) {
          lk = k;
          li = P.id[s];
          ls = s;
        }
      }
    }
    const uint64_t any = wballot(li != DANCE_INV);
    if (!any) break;
    const int M = wave_min_i(lk);
    const uint32_t I = wave_min_u(lk == M ? li : DANCE_INV);
    const int l = ffs64(wballot(lk == M && li == I && li != DANCE_INV));
    const int s = __builtin_amdgcn_readlane(ls, l);
    if ((int)lane == l) taken |= 1u << s;
    if (lane == i) {
      oid = I;
      od = __int_as_float(M);
    }
  }
  if (lane < a.k) {
    a.out_ids[(size_t)q * a.k + lane] = oid;
    a.out_d[(size_t)q * a.k + lane] = od;
  }
  if (a.ctr && lane == 0) {
    atomicAdd(a.ctr + 0, (unsigned long long)ndist);
    atomicAdd(a.ctr + 1, (unsigned long long)nexp);
    if (capped) atomicAdd(a.ctr + 2, 1ull);
  }
}

}  // namespace qs
}  // namespace dance
