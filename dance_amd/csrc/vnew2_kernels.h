// Device kernels of the standard GPU Vamana build, written for gfx950.
//
// One wave64 owns one vertex. Per-vertex state lives where CDNA4 keeps it
// cheapest: the top-L candidate pool in VGPRs (PS slots per lane, slot
// s = r*64 + lane), the C-wide work row and scratch lists in LDS, a forgetful
// visited cache in LDS that skips distance gathers for ids already handled in
// this search, and the vertex's own vector in VGPRs. Distances are gathered by
// octets (see wave.h), 16 pairs in flight per wave.
//
// Semantics follow /root/reference/src/gpu_vamana_vnew2.cu exactly; each
// kernel cites the reference kernel it replaces. The visited cache never
// changes a result: re-inserting an id the pool has already handled is a no-op
// in the reference's pool (the pool maximum never rises once the pool is full,
// and distances are a deterministic function of the id).
#pragma once

#include <type_traits>

#include "locality.h"
#include "qbound.h"
#include "wave.h"

// Opt-in per-phase cycle counters of the search kernel (the analogue of the
// reference's ENABLE_SEARCH_PRUNE_TIMING, vnew2.cu:100-102). Off by default.
#ifndef DANCE_SEARCH_TIMING
#define DANCE_SEARCH_TIMING 0
#endif

namespace dance {

__device__ __forceinline__ uint64_t dclock() {
#if DANCE_SEARCH_TIMING
  return __builtin_amdgcn_s_memtime();
#else
  return 0;
#endif
}

// 768 slots: a search wave's LDS (visited cache, work row, batch, order) is
// then 5 KB at C <= 128, which still lets the register budget, not LDS, set
// the waves per SIMD (8 for the uint8 rows of width 128, 7 for the exact
// fp32 search: 8 x 4 waves of 5 KB fill the 160 KB of a CU). 1024 slots
// cost the fp32 search a wave per SIMD and were slower (c3 iterations 1-2:
// 543 and 663 ms against 499 and 624 ms with 512 slots, kernels of that
// time); 768 against 512 saves 14 ms of the c4 build and 7 ms of c3. The
// cache never changes a result, only how many exact distances repeat. A
// slot count that is not a power of two hashes by a multiply-high.
#ifndef DANCE_VIS_BITS
#define DANCE_VIS_BITS 9
#endif
#ifndef DANCE_VIS_SLOTS
#define DANCE_VIS_SLOTS 768u
#endif
constexpr uint32_t kVisBits = DANCE_VIS_BITS;  // used when the slot count is 2^kVisBits
constexpr uint32_t kVis = DANCE_VIS_SLOTS;     // visited cache slots per wave
static_assert(kVis % 64u == 0u && kVis >= 128u, "visited cache: whole 64-slot rows");
constexpr uint32_t kWavesPerBlock = 4;
constexpr uint32_t kBlock = 64 * kWavesPerBlock;
constexpr uint32_t kQInFlight = 4;  // bound-filter passes whose loads are in flight together

struct VCounters {
  unsigned long long search_dist;   // distances computed for pool candidates
  unsigned long long insert_dist;   // distances computed by the online insert
  unsigned long long expansions;    // expanded pool entries
  unsigned long long vis_skips;     // candidates skipped by the visited cache
  unsigned long long insert_mut;    // online-insert mutations of the work row
  unsigned long long insert_try;    // online-insert attempts
  unsigned long long merge_dist;    // reverse-merge candidates (distance from the slot snapshot)
  unsigned long long prune_dist;    // prune pair distances
  unsigned long long reverse_edges; // reverse proposals
  unsigned long long touched_rows;  // targets with at least one reverse edge
  // DANCE_SEARCH_TIMING: cycles in select / online insert / candidate
  // distances / ordered pool inserts / seeding, summed over waves.
  unsigned long long cyc_select, cyc_insert, cyc_dist, cyc_pool, cyc_seed, cyc_total;
  unsigned long long bound_checks;  // candidates tested with the quantized lower bound
  unsigned long long bound_skips;   // candidates whose exact distance the bound made unnecessary
  unsigned long long prune_bound_checks, prune_bound_skips;  // the same for prune pairs
  unsigned long long prune_rounds, prune_exact_rounds;       // selection rounds; those with exact pairs
  // DANCE_SEARCH_TIMING: k_prune_rank phase cycles, summed over waves.
  unsigned long long cyc_prune_rank, cyc_prune_gram, cyc_prune_rounds, cyc_prune_fill;
  unsigned long long insert_bound_checks;  // online-insert occlusion pairs tested with the code-row bounds
  unsigned long long insert_bound_skips;   // those whose exact distance the bounds made unnecessary
};


// Counters are striped over kCtrStripes copies (by workgroup) so that the
// per-wave atomics of millions of waves do not serialise on one address; the
// host sums the stripes.
constexpr uint32_t kCtrStripes = 64;
__device__ __forceinline__ VCounters* ctr_stripe(VCounters* base) {
  return base + (blockIdx.x & (kCtrStripes - 1u));
}

// Sums the counter stripes into one VCounters (a snapshot after a launch).
static __global__ void k_ctr_sum(const VCounters* __restrict__ stripes, VCounters* __restrict__ out) {
  constexpr uint32_t nf = sizeof(VCounters) / sizeof(unsigned long long);
  static_assert(nf <= 64, "one thread of the 64-thread launch per field");
  const uint32_t f = threadIdx.x;
  if (f >= nf) return;
  unsigned long long s = 0;
  for (uint32_t k = 0; k < kCtrStripes; ++k) s += reinterpret_cast<const unsigned long long*>(stripes + k)[f];
  reinterpret_cast<unsigned long long*>(out)[f] = s;
}


struct GraphBufs {
  uint32_t N, R, C;
  uint32_t* cur;       // N x R
  uint32_t* deg_cur;   // N
  uint32_t* work;      // N x C
  uint32_t* deg_work;  // N
  float* wd;           // N x C
};

__device__ __forceinline__ bool valid_for(uint32_t id, uint32_t N, uint32_t node) {
  return id != DANCE_INV && id < N && id != node;
}

// ---------------------------------------------------------------------------
// Register-resident bounded top-L pool (vnew2.cu:520-734).
//
// Slot p = r*64 + lane lives in register r of that lane. Besides the id, each
// slot keeps two ordering keys so that the max and the selection are one
// wave reduction each, with no per-slot validity tests:
//   mkey: the distance bits (an order-preserving int for non-negative floats)
//         of a valid entry with a non-NaN distance, INT_MIN otherwise; the
//         largest mkey, lowest slot, is the pool's worst entry.
//   skey: mkey of an entry that can still be expanded (not expanded,
//         distance < FLT_MAX), INT_MAX otherwise; the smallest skey, lowest
//         slot, is the next entry to expand.
// Distances are non-negative (squared L2), so mkey also stores the distance
// itself; NaN entries (mkey INT_MIN) are never read back as distances.
// ---------------------------------------------------------------------------
constexpr int kSelLimit = 0x7F7FFFFF;  // bits of FLT_MAX: keys below it are selectable

__device__ __forceinline__ int pool_mkey(float d) { return d == d ? __float_as_int(d) : INT_MIN; }
__device__ __forceinline__ int pool_skey(int mk) { return mk != INT_MIN && mk < kSelLimit ? mk : INT_MAX; }

template <int PS>
struct RegPool {
  uint32_t id[PS];
  int mkey[PS];
  int skey[PS];
  uint32_t size;
  int max_pos;
  float max_d;
  uint32_t L;

  __device__ __forceinline__ void init(uint32_t L_) {
#pragma unroll
    for (int r = 0; r < PS; ++r) {
      id[r] = DANCE_INV;
      mkey[r] = INT_MIN;
      skey[r] = INT_MAX;
    }
    size = 0u;
    max_pos = -1;
    max_d = -FLT_MAX;
    L = L_;
  }

  __device__ __forceinline__ uint32_t get_id(int pos) const {
    uint32_t v = DANCE_INV;
#pragma unroll
    for (int r = 0; r < PS; ++r)
      if (r == (pos >> 6)) v = id[r];
    return rdlane_u(v, pos & 63);
  }
  // Distance of a valid slot (NaN for a NaN entry).
  __device__ __forceinline__ float get_d(int pos) const {
    int v = INT_MIN;
#pragma unroll
    for (int r = 0; r < PS; ++r)
      if (r == (pos >> 6)) v = mkey[r];
    const int k = __builtin_amdgcn_readlane(v, pos & 63);
    return k == INT_MIN ? __builtin_nanf("") : __int_as_float(k);
  }
  // Whether this lane's register r holds slot pos (never for pos < 0): one
  // vector compare of the lane against the uniform pos - 64 r, which lies in
  // [0, 64) only for the register that holds the slot.
  static __device__ __forceinline__ bool at_slot(uint32_t lane, int r, int pos) {
    return lane == (uint32_t)pos - 64u * (uint32_t)r;
  }
  // Slot updates are select instructions on every lane (no divergent
  // branch, so no register copies at the merge).
  __device__ __forceinline__ void set_slot(int pos, uint32_t nid, float nd, uint32_t lane) {
    const int mk = pool_mkey(nd), sk = pool_skey(mk);
#pragma unroll
    for (int r = 0; r < PS; ++r) {
      const bool h = at_slot(lane, r, pos);
      id[r] = h ? nid : id[r];
      mkey[r] = h ? mk : mkey[r];
      skey[r] = h ? sk : skey[r];
    }
  }
  __device__ __forceinline__ void set_d(int pos, float nd, uint32_t lane) {
    const int mk = pool_mkey(nd), sk = pool_skey(mk);
#pragma unroll
    for (int r = 0; r < PS; ++r) {
      const bool h = at_slot(lane, r, pos);
      mkey[r] = h ? mk : mkey[r];
      skey[r] = h ? sk : skey[r];
    }
  }
  __device__ __forceinline__ void set_expanded(int pos, uint32_t lane) {
#pragma unroll
    for (int r = 0; r < PS; ++r) skey[r] = at_slot(lane, r, pos) ? INT_MAX : skey[r];
  }

  // recompute_max_pos_size_warp: largest distance, lowest slot on ties.
  // kHasNumber: the caller knows some slot holds a non-NaN distance, so the
  // empty case (every mkey INT_MIN) cannot occur and is not tested.
  template <bool kHasNumber = false>
  __device__ __forceinline__ void recompute_max() {
    int best = mkey[0];
#pragma unroll
    for (int r = 1; r < PS; ++r) best = max(best, mkey[r]);
    const int M = wave_max_i(best);
    if (!kHasNumber && M == INT_MIN) {
      max_pos = -1;
      max_d = -FLT_MAX;
      return;
    }
    int pos = -1;
#pragma unroll
    for (int r = 0; r < PS; ++r) {
      if (pos < 0) {
        const uint64_t m = wballot(mkey[r] == M);
        if (m) pos = r * 64 + ffs64(m);
      }
    }
    // wave-uniform: keep the loop-carried pool state in scalar registers
    max_pos = uni_i(pos);
    max_d = uni_f(__int_as_float(M));
  }

  // insert_top_l_state_warp with ENABLE_TOPL_EARLY_REJECT=1. `nid`/`nd` are uniform.
  __device__ __forceinline__ void insert(uint32_t nid, float nd, uint32_t lane) {
    if (nid == DANCE_INV) return;
    if (size >= L && max_pos >= 0 && nd >= max_d) return;
    int same = -1;
#pragma unroll
    for (int r = PS - 1; r >= 0; --r) {
      const uint64_t m = wballot(id[r] == nid);
      same = m ? r * 64 + ffs64(m) : same;  // the lowest register wins
    }
    same = uni_i(same);
    // One of: refresh a duplicate's distance, append, replace the worst.
    // The slot registers change by selects on one path (see insert_full).
    const bool refresh = same >= 0 && nd < get_d(same);
    const bool append = same < 0 && size < L;
    const bool replace = same < 0 && size >= L && max_pos >= 0 && nd < max_d;
    const int pos = same >= 0 ? same : (append ? (int)size : max_pos);
    const int mk = pool_mkey(nd), sk = pool_skey(mk);
    const bool any = refresh || append || replace;
#pragma unroll
    for (int r = 0; r < PS; ++r) {
      const bool h = any && at_slot(lane, r, pos);
      id[r] = h ? nid : id[r];  // a duplicate keeps its id
      mkey[r] = h ? mk : mkey[r];
      skey[r] = h ? sk : skey[r];
    }
    if (append) {
      size = uni_u(size + 1u);
      if (max_pos < 0 || nd > max_d) {
        max_pos = uni_i(pos);
        max_d = uni_f(nd);
      }
    } else if (replace || (refresh && same == max_pos)) {
      recompute_max<true>();  // nd is a number
    }
  }

  // insert() for a pool with size >= L and max_pos >= 0 (which every path
  // below preserves) and a valid candidate id.
  // The slot registers are updated by selects (no branch around them), so
  // the compiler keeps them in place instead of copying them at every join;
  // the uniform branches are the rare refresh of a duplicate and the max
  // recomputation.
  //
  // An id already in the pool (rare: the visited cache filters repeats until
  // it forgets them) refreshes its slot when closer. A new id replaces the
  // worst slot; its distance is below max_d, so not NaN: its mkey is its bits
  // and its skey those bits unless the distance is FLT_MAX or more (below an
  // infinite worst entry), which pool_skey marks unselectable.
  __device__ __forceinline__ void insert_full(uint32_t nid, float nd, uint32_t lane) {
    if (!(nd < max_d)) return;  // uniform; a NaN distance changes nothing either
    uint64_t dup = 0;
#pragma unroll
    for (int r = 0; r < PS; ++r) dup |= wballot(id[r] == nid);
    // Both outcomes write one slot through the same selects below; only the
    // uniform slot and whether the max moves differ, so the slot registers
    // are not copied between the two paths.
    int pos = max_pos;
    bool moved = true;
    if (dup) {
      int same = -1;
#pragma unroll
      for (int r = PS - 1; r >= 0; --r) {
        const uint64_t m = wballot(id[r] == nid);
        same = m ? r * 64 + ffs64(m) : same;  // the lowest register wins
      }
      same = uni_i(same);
      if (!(nd < get_d(same))) return;
      pos = same;  // a duplicate keeps its id (nid)
      moved = same == max_pos;
    }
    const int mk = __float_as_int(nd);
    const int sk = mk < kSelLimit ? mk : INT_MAX;
#pragma unroll
    for (int r = 0; r < PS; ++r) {
      const bool h = at_slot(lane, r, pos);
      id[r] = h ? nid : id[r];
      mkey[r] = h ? mk : mkey[r];
      skey[r] = h ? sk : skey[r];
    }
    if (moved) recompute_max<true>();  // nd is a number
  }

  // select_next_unexpanded_size_warp: smallest distance among unexpanded
  // entries with distance < FLT_MAX, lowest slot on ties; -1 if none. The
  // selected entry's distance goes to *dist (its skey holds the bits).
  __device__ __forceinline__ int select(float* dist) const {
    int best = skey[0];
#pragma unroll
    for (int r = 1; r < PS; ++r) best = min(best, skey[r]);
    const int M = wave_min_i(best);
    if (M == INT_MAX) return -1;
    *dist = __int_as_float(M);
    int pos = -1;
#pragma unroll
    for (int r = 0; r < PS; ++r) {
      if (pos < 0) {
        const uint64_t m = wballot(skey[r] == M);
        if (m) pos = r * 64 + ffs64(m);
      }
    }
    return pos;
  }
};

__device__ __forceinline__ uint32_t vis_slot(uint32_t id) {
  if constexpr (kVis == (1u << kVisBits)) return (id * 0x9E3779B1u) >> (32 - kVisBits);
  return __umulhi(id * 0x9E3779B1u, kVis);
}

// Neighbour i of `node` in the random initial graph: the cur rows k_init
// writes (init_random_graph, vnew2.cu:1066-1117).
__device__ __forceinline__ uint32_t init_neighbor(uint32_t node, uint32_t i, uint32_t N) {
  const uint32_t nb = d_det_neighbor(node, i, N);
  return (N <= 1 || nb == DANCE_INV || nb >= N || nb == node) ? DANCE_INV : nb;
}

struct SearchArgs {
  RowSet rs;
  GraphBufs g;
  uint32_t L, steps, start;
  float alpha;
  const uint32_t* order;  // optional processing order (vertex = order[wave])
  VCounters* ctr;
  QBoundSet qb;  // quantized lower bound (qb.rows == nullptr: exact distances only)
};

// Per-wave LDS words of the search kernel: visited cache, work row (ids,
// dists), candidate batch (ids, dists), work-row order.
__host__ __device__ constexpr uint32_t search_lds_words(uint32_t Cp) { return kVis + 3u * Cp + 128u; }

// QB compiles the quantized-bound path in (the launcher picks QB = true only
// when the bound is on for the launch); QB = false kernels carry no bound code
// and keep their register budget for the exact path.
// IB (with QB, fp32/fp16 rows and C <= 128 only) adds the insert bound: the
// online insert's occlusion test decides pairs on the code rows first. HC
// (the first iteration, whose graph is the random initial one) takes an
// expanded vertex's neighbours from init_neighbor instead of gathering its
// cur row and degree: the same values, without three random cache lines per
// expansion; and it computes the vertex's own initial row and distances as
// k_init would, so that the build skips k_init.
template <int DT, int CPL, int PS, bool QB, bool IB = false, bool HC = false>
struct SearchWave {
  const SearchArgs& a;
  uint32_t node, lane, grp, sub, Cp;
  uint32_t *vis, *wid, *lst, *ord;
  float *wdd, *lsd;
  uint4 av[CPL];
  uint32_t av_sq;  // self_term(av): the vertex row's share of every pair distance
  RegPool<PS> P;
  QSelf qme;
  uint32_t wdeg;
  uint32_t n_search, n_insert, n_skip, n_mut, n_try, n_bchk, n_bskip, n_ibchk, n_ibskip;
  uint64_t c_select = 0, c_insert = 0, c_dist = 0, c_pool = 0;

  __device__ SearchWave(const SearchArgs& args, uint32_t node_, uint32_t* base, uint32_t Cp_)
      : a(args), node(node_), Cp(Cp_) {
    lane = lane_id();
    grp = lane >> 3;
    sub = lane & 7u;
    vis = base;
    wid = vis + kVis;
    wdd = reinterpret_cast<float*>(wid + Cp);
    lst = reinterpret_cast<uint32_t*>(wdd + Cp);
    lsd = reinterpret_cast<float*>(lst + 64);
    ord = reinterpret_cast<uint32_t*>(lsd + 64);
    n_search = n_insert = n_skip = n_mut = n_try = n_bchk = n_bskip = n_ibchk = n_ibskip = 0;
  }

  // Drops from lst[0..n) the candidates whose distance the quantized bound
  // proves >= the pool threshold (they would be rejected unseen); keeps the
  // others in order and returns their count.
  __device__ __forceinline__ uint32_t bound_filter(uint32_t n) {
    const float sT = q_threshold(a.qb, qme, P.max_d);
    const uint4 code = qme.row[sub];
    uint64_t keep = 0;
    for (uint32_t p = 0; p < n; p += 8 * kQInFlight) {
      uint4 b[kQInFlight];
#pragma unroll
      for (uint32_t u = 0; u < kQInFlight; ++u) {
        const uint32_t k = p + 8 * u + grp;
        b[u] = q_load(a.qb, lst[k], k < n, sub);  // k < 64 (p steps by 8 kQInFlight, which divides 64)
      }
      bool rej[kQInFlight];
#pragma unroll
      for (uint32_t u = 0; u < kQInFlight; ++u)
        rej[u] = q_proves_reject(qme, code, sT, b[u], p + 8 * u + grp < n, sub);
#pragma unroll
      for (uint32_t u = 0; u < kQInFlight; ++u)
        keep |= (uint64_t)octet_bits(wballot(sub == 0 && p + 8 * u + grp < n && !rej[u])) << (p + 8 * u);
    }
    const uint32_t nk = popc64(keep);
    n_bchk += n;
    n_bskip += n - nk;
    if (nk < n) {
      const uint32_t ck = lst[lane];
      wave_sync();
      if ((keep >> lane) & 1ull) lst[mbcnt64(keep)] = ck;
      wave_sync();
    }
    return nk;
  }

  // Handles one batch of <= 64 candidates given in insertion order (one per
  // lane; DANCE_INV = none): visited filter, distances, ordered inserts.
  __device__ __forceinline__ void process_batch(uint32_t c) {
    const uint32_t N = a.g.N;
    const uint32_t slot = vis_slot(c);
    const uint32_t at = vis[slot];
    // Masks from ballots of single compares (c < N also excludes DANCE_INV).
    const uint64_t mv = wballot(c < N) & wballot(c != node);
    const uint64_t ms = mv & wballot(at == c);
    const uint64_t m = mv & ~ms;
    const bool need = c < N && c != node && at != c;
    const uint32_t n = popc64(m);
    n_skip += popc64(ms);
    if (n == 0) return;
    if (need) lst[mbcnt64(m)] = c;
    wave_sync();
    const uint64_t t0 = dclock();
    const bool full = P.size >= P.L && P.max_pos >= 0;
    const uint32_t nx = (QB && full && a.qb.rows) ? bound_filter(n) : n;
    if (nx) batch_dist<DT, CPL>(a.rs, av, av_sq, lst, lsd, nx, grp, sub);
    n_search += nx;
    const uint64_t t1 = dclock();
    c_dist += t1 - t0;
    const uint32_t ck = lst[lane];  // read only where lane < nx (keep below)
    const float dk = lsd[lane];
    uint64_t km = lanes_below(nx);
    if (full) km &= wballot(dk < P.max_d);
    if (full) {
      // A pool that starts the batch full stays full with a valid worst
      // entry, so insert() reduces to: reject unless below the worst,
      // refresh a duplicate, else replace the worst slot.
      while (km) {
        const int k = ffs64(km);
        km &= ~(1ull << k);
        P.insert_full(rdlane_u(ck, k), rdlane_f(dk, k), lane);
      }
    } else {
      while (km) {
        const int k = ffs64(km);
        km &= ~(1ull << k);
        P.insert(rdlane_u(ck, k), rdlane_f(dk, k), lane);
      }
    }
    if (need) vis[slot] = c;
    wave_sync();
    c_pool += dclock() - t1;
  }

  // Work-row order: ord[r] is the slot of rank r over [0, wdeg), ascending by
  // (usable, distance, slot descending), where unusable entries (invalid id
  // or NaN distance) rank lowest. Reading it from the top gives the usable
  // entries by (distance descending, slot ascending): the worst entry first,
  // then the victim candidates in the order the online insert tries them.
  __device__ __forceinline__ bool usable(uint32_t j) const {
    return valid_for(wid[j], a.g.N, node) && wdd[j] == wdd[j];
  }
  // Whether slot j orders before a usable entry (d, s).
  __device__ __forceinline__ bool before(uint32_t j, float d, uint32_t s) const {
    if (!usable(j)) return true;
    const float dj = wdd[j];
    return dj < d || (dj == d && j > s);
  }
  // Ranks by counting, over one 64-bit key per slot: (usable, distance bits,
  // ~slot) for usable entries and (0, ~slot) for the others, so that key_j <
  // key_i exactly when j orders before i (distances are non-negative, their
  // bits ascend with their values). The keys are staged in the visited cache's
  // LDS, which run() clears afterwards; rows longer than it holds count on the
  // row itself.
  __device__ __forceinline__ void ord_init() {
    if (2u * wdeg <= kVis) {
      uint64_t* key = reinterpret_cast<uint64_t*>(vis);
      for (uint32_t i = lane; i < wdeg; i += 64) {
        const uint32_t hi = usable(i) ? (0x80000000u | __float_as_uint(wdd[i])) : 0u;
        key[i] = ((uint64_t)hi << 32) | (uint64_t)(0xFFFFFFFFu - i);
      }
      wave_sync();
      for (uint32_t i = lane; i < wdeg; i += 64) {
        const uint64_t ki = key[i];
        uint32_t r = 0;
        for (uint32_t j = 0; j < wdeg; ++j) r += key[j] < ki ? 1u : 0u;
        ord[r] = i;
      }
      wave_sync();
      return;
    }
    for (uint32_t i = lane; i < wdeg; i += 64) {
      const bool ui = usable(i);
      const float di = wdd[i];
      uint32_t r = 0;
      for (uint32_t j = 0; j < wdeg; ++j) {
        if (j == i) continue;
        const bool uj = usable(j);
        r += ui ? (!uj || wdd[j] < di || (wdd[j] == di && j > i)) : (!uj && j > i);
      }
      ord[r] = i;
    }
    wave_sync();
  }
  // Slot s now holds a usable entry of distance d; it left rank rold (deg - 1
  // when appended: the new slot is appended at the top); deg is the row
  // length after the change. rnew is its new rank when the caller knows it
  // (no other entry has distance d), else kRankUnknown: then it is counted.
  static constexpr uint32_t kRankUnknown = 0xFFFFFFFFu;
  __device__ __forceinline__ void ord_update(uint32_t s, float d, uint32_t rold, uint32_t rnew, uint32_t deg) {
    if (rnew == kRankUnknown) {
      rnew = 0;
      for (uint32_t b = 0; b < deg; b += 64) {
        const uint32_t j = b + lane;
        rnew += popc64(wballot(j < deg && j != s && before(j, d, s)));
      }
    }
    // ranks between rnew and rold move one step toward rold; rnew receives s.
    // Chunks of 64 are read before they are written and walk away from the
    // ranks they read, so every rank is read before it is overwritten.
    if (rnew < rold) {
      for (int top = (int)rold; top > (int)rnew; top -= 64) {
        const int i = top - (int)lane;
        const bool ok = i > (int)rnew;
        const uint32_t v = ok ? ord[i - 1] : 0u;
        wave_sync();
        if (ok) ord[i] = v;
        wave_sync();
      }
    } else if (rnew > rold) {
      for (uint32_t bot = rold; bot < rnew; bot += 64) {
        const uint32_t i = bot + lane;
        const bool ok = i < rnew;
        const uint32_t v = ok ? ord[i + 1] : 0u;
        wave_sync();
        if (ok) ord[i] = v;
        wave_sync();
      }
    }
    if (lane == 0) ord[rnew] = s;
    wave_sync();
  }

  // The occlusion test of robust_insert with the insert bound: a pass of 8
  // candidates first tests its pairs on the code rows (x's chunk in xcode).
  // An upper bound that proves fl(alpha * d(y, x)) <= d_px proves an
  // occluder and ends the test; pairs whose lower bound proves the opposite
  // need nothing more; the others collect their ids in lst and lsd (128
  // words, unused during the insert; nA <= C <= 128) and get exact
  // distances, in passes of 8, once the bound passes end. The answer is the
  // exact test's: every decision the bounds make is the one the exact
  // distance would give, and the answer does not depend on the order.
  __device__ __forceinline__ bool occlusion_bounded(uint32_t x, float dpx, const uint4& xcode, uint32_t nU,
                                                    uint32_t nA) {
    // x's header: lane 0 holds chunk 0 of its code row
    const float xs = __uint_as_float(rdlane_u(xcode.x, 0));
    const float xr = __uint_as_float(rdlane_u(xcode.y, 0));
    const float xa = __uint_as_float(rdlane_u(xcode.z, 0));
    const float ub = q_ub_root_of<DT>(a.qb, dpx, a.alpha);
    const float lbT = (prune_bound_root(a.qb, dpx, a.alpha) + xr) * (1.0f + kQSlack);
    uint32_t* pend = lst;
    uint32_t nopen = 0;
    for (uint32_t p = 0; p < nA; p += 8) {
      const uint32_t k0 = p + grp;
      const bool a0 = k0 < nA;
      const uint32_t y0 = a0 ? wid[ord[nU + k0]] : 0u;
      const uint4 b = q_load(a.qb, y0, a0, sub);
      const int c = q_octet_dot(xcode, b, sub);
      const float sy = __uint_as_float(b.x), ry = __uint_as_float(b.y), ay = __uint_as_float(b.z);
      const bool lead = sub == 0u && a0;
      const uint32_t np = min(8u, nA - p);
      n_ibchk += np;
      if (wballot(lead && q_pair_ub(xs, xa, xr, ub, sy, ry, ay, c))) {
        n_ibskip += np;
        return true;
      }
      const uint64_t und = wballot(lead && !q_pair_proves(xs, xa, lbT, sy, ry, ay, c));
      n_ibskip += np - popc64(und);
      if (lead && ((und >> lane) & 1ull)) pend[nopen + popc64(und & lanes_below(lane))] = y0;
      nopen += popc64(und);
    }
    if (nopen == 0) return false;
    wave_sync();
    uint4 xv[CPL];
    load_row<CPL>(a.rs, x, true, sub, xv);
    bool occ = false;
    uint32_t q = 0;
    for (; q < nopen && !occ; q += 8) {
      const uint32_t k = q + grp;
      const bool act = k < nopen;
      uint4 b0[CPL];
      load_row<CPL>(a.rs, pend[act ? k : 0u], act, sub, b0);
      const float d0 = octet_finish<DT, CPL>(a.rs, sub, xv, b0, self_term<DT, CPL>(xv));
      occ = (wballot(a.alpha * d0 <= dpx) & kOctetLeads & lanes_below(8u * (nopen - q))) != 0;
    }
    n_insert += min(q, nopen);  // distances of the passes made
    wave_sync();
    return occ;
  }

  // dynamic_robust_insert_C_warp (vnew2.cu:759-877) on the LDS work row.
  __device__ __forceinline__ void robust_insert(uint32_t x, float dpx) {
    const uint32_t N = a.g.N, C = a.g.C;
    if (x == DANCE_INV || x >= N || x == node) return;
    n_try++;
    // With the insert bound the occlusion test starts from x's code chunk
    // and x's row is loaded where exact distances are needed; otherwise x's
    // row is requested first (x < N), so its load overlaps the pass below (a
    // repeated x leaves it unused).
    constexpr bool kIB = QB && IB && DT != DANCE_U8;
    uint4 xv[CPL];
    uint4 xcode;
    if constexpr (kIB)
      xcode = a.qb.rows[(size_t)x * kQChunks + sub];  // launched only with code rows present
    else
      load_row<CPL>(a.rs, x, true, sub, xv);
    // One pass over the row: x already there ends the insert; otherwise the
    // usable entries nearer than x (nA, of which nL strictly) and farther
    // (nB); dpx is a number, so a usable entry is exactly one of nA and nB.
    // The rest (nU), unusable, rank lowest in the order.
    uint32_t nA = 0, nL = 0, nB = 0;
    for (uint32_t b = 0; b < wdeg; b += 64) {
      const uint32_t i = b + lane;  // < Cp: b < wdeg <= Cp, both multiples of 64
      const uint64_t in = lanes_below(wdeg - b);
      const uint32_t y = wid[i];
      if (in & wballot(y == x)) return;
      const float dpy = wdd[i];
      const uint64_t v = in & wballot(y < N) & wballot(y != node);
      nA += popc64(v & wballot(dpy <= dpx));
      nL += popc64(v & wballot(dpy < dpx));
      nB += popc64(v & wballot(dpy > dpx));
    }
    const uint32_t nU = wdeg - nA - nB;
    // Occlusion: exists y with d_py <= d_px and alpha * d(y, x) <= d_px. The
    // answer does not depend on the order; the candidates are the order's
    // ranks [nU, nU + nA) (usable entries with d_py <= d_px, nearest to the
    // vertex first), and the test stops at the first pass of 8 that finds an
    // occluder.
    bool occluded = false;
    uint32_t p = 0;
    if constexpr (kIB) {
      occluded = occlusion_bounded(x, dpx, xcode, nU, nA);
      if (occluded) return;
      load_row<CPL>(a.rs, x, true, sub, xv);  // for the victim test
    } else {
      const uint32_t xv_sq = self_term<DT, CPL>(xv);
      for (; p < nA && !occluded; p += 8) {
        const uint32_t k0 = p + grp;
        const bool a0 = k0 < nA;
        const uint32_t y0 = a0 ? wid[ord[nU + k0]] : 0u;
        uint4 b0[CPL];
        load_row<CPL>(a.rs, y0, a0, sub, b0);
        const float d0 = octet_finish<DT, CPL>(a.rs, sub, xv, b0, xv_sq);
        occluded = (wballot(a.alpha * d0 <= dpx) & kOctetLeads & lanes_below(8u * (nA - p))) != 0;
      }
      n_insert += min(p, nA);  // distances of the passes made
      if (occluded) return;
    }
    const uint32_t xv_sq = self_term<DT, CPL>(xv);
    // Worst usable entry (largest d_py, lowest slot): the top of the order.
    int wpos = -1;
    float wdist = -FLT_MAX;
    if (wdeg > 0) {
      const uint32_t top = ord[wdeg - 1];
      if (usable(top)) {
        wpos = (int)top;
        wdist = wdd[top];
      }
    }
    // Victim: the largest d_py (lowest slot on ties) among y with d_py > d_px
    // and alpha * d(x, y) <= d_py. The nB candidates are the top nB ranks of
    // the order, already in that sequence, so only a prefix is gathered.
    int vpos = -1;
    uint32_t vrank = 0;
    for (p = 0; p < nB && vpos < 0; p += 8) {
      const uint32_t k0 = p + grp;
      const bool a0 = k0 < nB;
      const uint32_t s0 = a0 ? ord[wdeg - 1u - k0] : 0u;
      const uint32_t y0 = a0 ? wid[s0] : 0u;
      uint4 b0[CPL];
      load_row<CPL>(a.rs, y0, a0, sub, b0);
      const float d0 = octet_finish<DT, CPL>(a.rs, sub, xv, b0, xv_sq);
      const uint64_t hit = wballot(a.alpha * d0 <= wdd[s0]) & kOctetLeads & lanes_below(8u * (nB - p));
      if (hit) {
        const int l = ffs64(hit);  // lane 8 g + 0 of the first octet that hit
        vpos = (int)rdlane_u(s0, l);
        vrank = wdeg - 1u - (p + ((uint32_t)l >> 3));
      }
    }
    n_insert += min(p, nB);
    // The changed slot and the rank its old entry held: the victim's, the
    // top rank for the worst entry, the new top for an appended slot.
    int mslot = -1;
    uint32_t rold = 0;
    bool appended = false;
    if (vpos >= 0) {
      mslot = vpos;
      rold = vrank;
    } else if (wdeg < C) {
      mslot = (int)wdeg;
      rold = wdeg;
      appended = true;
    } else if (wpos >= 0 && dpx < wdist) {
      mslot = wpos;
      rold = wdeg - 1u;
    }
    if (mslot >= 0) {
      wave_sync();
      if (lane == 0) {
        wid[mslot] = x;
        wdd[mslot] = dpx;
      }
      if (appended) wdeg++;
      n_mut++;
      wave_sync();
      // Its new rank: the unusable entries and the usable ones strictly
      // nearer than x rank below it (the replaced entry was farther); ties
      // at distance dpx are ordered by slot, which only a count resolves.
      ord_update((uint32_t)mslot, dpx, rold, nA == nL ? nU + nL : kRankUnknown, wdeg);
    }
  }

  __device__ void run() {
    const uint64_t t_run = dclock();
    const GraphBufs& g = a.g;
    const uint32_t N = g.N, R = g.R, C = g.C;
    load_row<CPL>(a.rs, node, true, sub, av);
    av_sq = self_term<DT, CPL>(av);
    if (QB && a.qb.rows) q_load_self(a.qb, node, qme);
    // Work row := current row with its stored distances (vnew2.cu:1186-1212).
    // With HC the current row is the random initial graph's, computed here
    // with its distances as k_init computes them (init_neighbor, batch_dist
    // from the cached row), so the build needs no k_init launch.
    const uint32_t deg_self = HC ? (N > 1u ? R : 0u) : min(g.deg_cur[node], R);
    const size_t wb = (size_t)node * C;
    if constexpr (HC) {
      for (uint32_t b = 0; b < Cp; b += 64) {  // Cp is a multiple of 64
        const uint32_t i = b + lane;
        const uint32_t nb = i < deg_self ? init_neighbor(node, i, N) : DANCE_INV;
        const bool v = nb != DANCE_INV;
        const uint64_t m = wballot(v);
        const uint32_t n = popc64(m);
        if (v) lst[mbcnt64(m)] = nb;
        wave_sync();
        if (n) batch_dist<DT, CPL>(a.rs, av, av_sq, lst, lsd, n, grp, sub);
        wid[i] = nb;
        wdd[i] = v ? lsd[mbcnt64(m)] : FLT_MAX;
        wave_sync();
      }
    } else {
      const size_t cb = (size_t)node * R;
      for (uint32_t i = lane; i < Cp; i += 64) {
        uint32_t nb = DANCE_INV;
        float dist = FLT_MAX;
        if (i < deg_self) {
          nb = g.cur[cb + i];
          if (valid_for(nb, N, node))
            dist = g.wd[wb + i];
          else
            nb = DANCE_INV;
        }
        wid[i] = nb;
        wdd[i] = dist;
      }
    }
    wdeg = deg_self;
    P.init(a.L);
    wave_sync();
    ord_init();
    for (uint32_t i = lane; i < kVis; i += 64) vis[i] = DANCE_INV;
    wave_sync();
    // Entry point (vnew2.cu:1223-1244).
    process_batch(lane == 0 && a.start < N && a.start != node ? a.start : DANCE_INV);
    // Own neighbours with stored distances (vnew2.cu:1246-1278), inserted in
    // row order. When they fit in one batch, the pool holds at most the entry
    // point, no two of them (nor one and the entry point) share a visited
    // slot and none has a NaN distance, the inserts are plain appends: they
    // go in as one batch (slots in row order, the running max as the
    // sequential appends leave it). Otherwise one insert after another.
    bool appended = false;
    if (deg_self <= 64u && P.size <= 1u) {
      const uint32_t nb = lane < deg_self ? wid[lane] : DANCE_INV;
      const float dd = lane < deg_self ? wdd[lane] : FLT_MAX;
      const bool v = nb != DANCE_INV;
      const uint64_t m = wballot(v);
      const uint32_t n = popc64(m);
      const uint32_t p0 = P.get_id(0);  // the entry point, or DANCE_INV
      const uint32_t slot = vis_slot(nb);
      if (v) vis[slot] = lane;
      wave_sync();
      const bool clash = v && (vis[slot] != lane || nb == p0 || dd != dd);
      wave_sync();
      if (!wballot(clash) && P.size + n <= P.L) {
        const uint32_t base = P.size;
        if (v) {
          lst[mbcnt64(m)] = nb;
          lsd[mbcnt64(m)] = dd;
        }
        wave_sync();
#pragma unroll
        for (int r = 0; r < PS; ++r) {
          const uint32_t p = (uint32_t)r * 64u + lane;
          if (p >= base && p < base + n) {
            const float d = lsd[p - base];
            P.id[r] = lst[p - base];
            P.mkey[r] = pool_mkey(d);
            P.skey[r] = pool_skey(P.mkey[r]);
          }
        }
        // sequential appends keep the first strictly larger distance
        const int M = wave_max_i(v ? fkey(dd) : INT_MIN);
        if (n > 0 && (P.max_pos < 0 || __int_as_float(M) > P.max_d)) {
          const int first = ffs64(wballot(v && fkey(dd) == M));  // lowest lane holding the max
          P.max_pos = uni_i((int)(base + popc64(m & ((1ull << first) - 1ull))));
          P.max_d = uni_f(__int_as_float(M));
        }
        P.size = uni_u(base + n);
        if (v) vis[slot] = nb;
        wave_sync();
        appended = true;
      }
    }
    for (uint32_t b = 0; !appended && b < deg_self; b += 64) {
      const uint32_t i = b + lane;
      const uint32_t nb = i < deg_self ? wid[i] : DANCE_INV;
      const float dd = i < deg_self ? wdd[i] : FLT_MAX;
      const bool v = nb != DANCE_INV;
      uint64_t m = wballot(v);
      while (m) {
        const int k = ffs64(m);
        m &= m - 1;
        P.insert(rdlane_u(nb, k), rdlane_f(dd, k), lane);
      }
      if (v) vis[vis_slot(nb)] = nb;
      wave_sync();
    }
    // INIT_RANDOM_SEEDS hashed seeds (vnew2.cu:1280-1300).
    process_batch(lane < 8 ? d_det_neighbor(node, lane + 1024u, N) : DANCE_INV);
    const uint32_t max_steps = min(a.steps, a.L);
    uint32_t n_exp = 0;
    const uint64_t t_seed = dclock() - t_run;
    (void)t_seed;
    for (uint32_t step = 0; step < max_steps; ++step) {
      const uint64_t ts0 = dclock();
      float dx;
      const int pos = P.select(&dx);
      if (pos < 0) break;
      const uint32_t x = P.get_id(pos);
      P.set_expanded(pos, lane);
      if (x == DANCE_INV || x >= N) break;
      n_exp++;
      // Issue the adjacency gather of x before the online insert.
      const uint32_t degx = HC ? (N > 1u ? R : 0u) : min(g.deg_cur[x], R);
      const size_t xb = (size_t)x * R;
      uint32_t c0 = DANCE_INV;
      if (lane < degx) c0 = HC ? init_neighbor(x, lane, N) : g.cur[xb + lane];
      const uint64_t ts1 = dclock();
      c_select += ts1 - ts0;
      robust_insert(x, dx);
      c_insert += dclock() - ts1;
      process_batch(c0);
      for (uint32_t b = 64; b < degx; b += 64) {
        const uint32_t pidx = b + lane;
        process_batch(pidx < degx ? (HC ? init_neighbor(x, pidx, N) : g.cur[xb + pidx]) : DANCE_INV);
      }
    }
    for (uint32_t i = lane; i < C; i += 64) {
      g.work[wb + i] = wid[i];
      g.wd[wb + i] = wdd[i];
    }
    if (lane == 0) g.deg_work[node] = wdeg;
    if (a.ctr) {
      const uint64_t m = wballot(true);
      if (lane == (uint32_t)ffs64(m)) {
        atomicAdd(&ctr_stripe(a.ctr)->search_dist, (unsigned long long)n_search);
        atomicAdd(&ctr_stripe(a.ctr)->insert_dist, (unsigned long long)n_insert);
        atomicAdd(&ctr_stripe(a.ctr)->expansions, (unsigned long long)n_exp);
        atomicAdd(&ctr_stripe(a.ctr)->vis_skips, (unsigned long long)n_skip);
        atomicAdd(&ctr_stripe(a.ctr)->insert_mut, (unsigned long long)n_mut);
        atomicAdd(&ctr_stripe(a.ctr)->insert_try, (unsigned long long)n_try);
        if (QB && a.qb.rows) {
          atomicAdd(&ctr_stripe(a.ctr)->bound_checks, (unsigned long long)n_bchk);
          atomicAdd(&ctr_stripe(a.ctr)->bound_skips, (unsigned long long)n_bskip);
          if constexpr (IB) {
            atomicAdd(&ctr_stripe(a.ctr)->insert_bound_checks, (unsigned long long)n_ibchk);
            atomicAdd(&ctr_stripe(a.ctr)->insert_bound_skips, (unsigned long long)n_ibskip);
          }
        }
#if DANCE_SEARCH_TIMING
        atomicAdd(&ctr_stripe(a.ctr)->cyc_select, (unsigned long long)c_select);
        atomicAdd(&ctr_stripe(a.ctr)->cyc_insert, (unsigned long long)c_insert);
        atomicAdd(&ctr_stripe(a.ctr)->cyc_dist, (unsigned long long)c_dist);
        atomicAdd(&ctr_stripe(a.ctr)->cyc_pool, (unsigned long long)c_pool);
        atomicAdd(&ctr_stripe(a.ctr)->cyc_seed, (unsigned long long)t_seed);
        atomicAdd(&ctr_stripe(a.ctr)->cyc_total, (unsigned long long)(dclock() - t_run));
#endif
      }
    }
  }
};

// Waves per SIMD the register allocator must leave room for, for the
// narrow-row, L <= 128 variants (the common case): DANCE_SEARCH_WAVES_QB
// (default 5) with the bound compiled in (the allocator would otherwise
// settle at 4 by a few registers), and DANCE_SEARCH_WAVES (default 6)
// without it; the exact search fits in 68 registers and runs 7 waves per
// SIMD (asking for 7 changes nothing); the first-iteration exact variants of
// one and two chunks per lane (uint8 rows of up to 256 bytes) ask for 8,
// which their LDS allows at C <= 128, so that the neighbour hash does not
// push the scalar registers past the 8-wave limit. The insert-bound variants
// ask for DANCE_SEARCH_WAVES_IB (default 6: 79-80 registers at 3 chunks per
// lane, no spills). No constraint elsewhere.
#ifndef DANCE_SEARCH_WAVES
#define DANCE_SEARCH_WAVES 6
#endif
#ifndef DANCE_SEARCH_WAVES_QB
#define DANCE_SEARCH_WAVES_QB 5
#endif
#ifndef DANCE_SEARCH_WAVES_IB
#define DANCE_SEARCH_WAVES_IB 6
#endif
template <int CPL, int PS, bool QB, bool IB, bool HC>
constexpr int kSearchMinWaves =
    (CPL <= 3 && PS == 2)
        ? (IB ? DANCE_SEARCH_WAVES_IB : QB ? DANCE_SEARCH_WAVES_QB : (CPL <= 2 && HC) ? 8 : DANCE_SEARCH_WAVES)
        : 1;

// search_prune_kernel_shared (vnew2.cu:1119-1439).
template <int DT, int CPL, int PS, bool QB, bool IB = false, bool HC = false>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(kSearchMinWaves<CPL, PS, QB, IB, HC>))) void k_search(SearchArgs a, uint32_t Cp) {
  extern __shared__ uint32_t smem[];
  const uint32_t w = wave_index();
  const uint32_t gw = xcd_block(grid_block(), grid_blocks()) * kWavesPerBlock + w;
  if (gw >= a.g.N) return;
  const uint32_t node = a.order ? a.order[gw] : gw;
  SearchWave<DT, CPL, PS, QB, IB, HC> sw(a, node, smem + w * search_lds_words(Cp), Cp);
  sw.run();
}

// ---------------------------------------------------------------------------
// RobustPrune with alpha and the last-iteration degree fill
// (final_prune_kernel_shared, vnew2.cu:1893-2147).
// ---------------------------------------------------------------------------
struct PruneArgs {
  RowSet rs;
  GraphBufs g;
  uint32_t min_degree;
  float alpha;
  const uint32_t* order;
  VCounters* ctr;
  QBoundSet qb;  // quantized lower bound (qb.rows == nullptr: exact distances only)
};

__host__ __device__ constexpr uint32_t prune_lds_words(uint32_t Cp, uint32_t Rp) { return 5u * Cp + 2u * Rp; }

constexpr uint32_t PR_REMOVED = 1u, PR_INOUT = 2u;

template <int DT, int CPL>
__global__ __launch_bounds__(kBlock) void k_prune(PruneArgs a, uint32_t Cp, uint32_t Rp) {
  extern __shared__ uint32_t smem[];
  const uint32_t w = wave_index();
  const uint32_t gw = xcd_block(grid_block(), grid_blocks()) * kWavesPerBlock + w;
  const GraphBufs& g = a.g;
  if (gw >= g.N) return;
  const uint32_t node = a.order ? a.order[gw] : gw;
  const uint32_t N = g.N, R = g.R, C = g.C;
  const uint32_t lane = lane_id(), grp = lane >> 3, sub = lane & 7u;
  uint32_t* sid = smem + w * prune_lds_words(Cp, Rp);
  float* sd = reinterpret_cast<float*>(sid + Cp);
  uint32_t* fl = sid + 2 * Cp;
  uint32_t* lst = sid + 3 * Cp;
  uint32_t* oid = sid + 4 * Cp;
  float* od = reinterpret_cast<float*>(oid + Rp);
  float* sroot = od + Rp;  // prune_bound_root of each candidate
  const size_t wb = (size_t)node * C, cb = (size_t)node * R;
  const uint32_t deg = min(g.deg_work[node], C);
  const bool qon = a.qb.rows != nullptr;
  for (uint32_t i = lane; i < Cp; i += 64) {
    uint32_t id = DANCE_INV;
    float dist = FLT_MAX;
    uint32_t f = PR_REMOVED;
    if (i < deg) {
      id = g.work[wb + i];
      dist = g.wd[wb + i];
      if (valid_for(id, N, node) && dist < FLT_MAX)
        f = 0u;
      else
        id = DANCE_INV;
    }
    sid[i] = id;
    sd[i] = dist;
    fl[i] = f;
    lst[i] = 0u;  // every entry a valid index, so lst reads need no guard
    if (qon) sroot[i] = prune_bound_root(a.qb, dist, a.alpha);
  }
  wave_sync();
  uint32_t oc = 0, npair = 0, nbchk = 0, nbskip = 0, nround = 0, nexact = 0;
  for (uint32_t round = 0; round < R; ++round) {
    // smallest distance, lowest index on ties: each lane keeps its first
    // entry of its smallest key (entries ascend per lane)
    int best = INT_MAX;
    uint32_t cand = 0xFFFFFFFFu;
    for (uint32_t i = lane; i < Cp; i += 64) {
      const int k = fkey(sd[i]);
      const bool ok = (fl[i] & PR_REMOVED) == 0u && sid[i] != DANCE_INV && k < best;
      best = ok ? k : best;
      cand = ok ? i : cand;
    }
    const int M = wave_min_i(best);
    if (M == INT_MAX) break;
    const uint32_t pos = wave_min_u(best == M ? cand : 0xFFFFFFFFu);
    const uint32_t sel = uni_u(sid[pos]);
    const float seld = uni_f(sd[pos]);
    if (lane == 0) {
      oid[oc] = sel;
      od[oc] = seld;
    }
    oc++;
    nround++;
    if (oc >= R) break;
    uint32_t nq = 0;
    for (uint32_t b = 0; b < Cp; b += 64) {
      const uint32_t i = b + lane;
      const uint32_t id = sid[i];
      uint32_t f = fl[i];
      if (id == sel) f |= PR_REMOVED | PR_INOUT;
      fl[i] = f;
      const bool q = (f & PR_REMOVED) == 0u && id != DANCE_INV && seld <= sd[i];
      const uint64_t m = wballot(q);
      if (q) lst[nq + mbcnt64(m)] = i;
      nq += popc64(m);
    }
    wave_sync();
    if (nq == 0) continue;
    if (qon) {
      // Drop the candidates whose pair distance the bound proves large
      // enough to keep them; their exact distance cannot remove them.
      const uint4* qs = a.qb.rows + (size_t)sel * kQChunks;
      const uint4 code = qs[sub];
      const QSelf me{qs, __uint_as_float(uni_u(rdlane_u(code.x, 0))), __uint_as_float(uni_u(rdlane_u(code.y, 0))),
                     __uint_as_float(uni_u(rdlane_u(code.z, 0)))};
      uint32_t nk = 0;
      for (uint32_t base = 0; base < nq; base += 64) {  // lst holds up to C entries
        const uint32_t nb = min(64u, nq - base);
        uint64_t keep = 0;
        for (uint32_t p = 0; p < nb; p += 8 * kQInFlight) {
          uint4 b[kQInFlight];
          uint32_t si[kQInFlight];
#pragma unroll
          for (uint32_t u = 0; u < kQInFlight; ++u) {
            const uint32_t k = p + 8 * u + grp;
            si[u] = lst[min(base + k, Cp - 1u)];
            b[u] = q_load(a.qb, sid[si[u]], k < nb, sub);
          }
#pragma unroll
          for (uint32_t u = 0; u < kQInFlight; ++u) {
            const uint32_t k = p + 8 * u + grp;
            const float sT = (sroot[si[u]] + me.r) * (1.0f + kQSlack);
            const bool prove = q_proves_reject(me, code, sT, b[u], k < nb, sub);
            keep |= (uint64_t)octet_bits(wballot(sub == 0 && k < nb && !prove)) << (p + 8 * u);
          }
        }
        // compact in place: writes land at or below the entries just read
        const uint32_t v = lane < nb ? lst[base + lane] : 0u;
        wave_sync();
        if ((keep >> lane) & 1ull) lst[nk + mbcnt64(keep)] = v;
        wave_sync();
        nk += popc64(keep);
      }
      nbchk += nq;
      nbskip += nq - nk;
      nq = nk;
      if (nq == 0) continue;
    }
    uint4 sv[CPL];
    load_row<CPL>(a.rs, sel, true, sub, sv);
    nexact++;
    for (uint32_t p = 0; p < nq; p += 16) {
      const uint32_t k0 = p + grp, k1 = p + 8 + grp;
      const bool a0 = k0 < nq, a1 = k1 < nq;
      const uint32_t s0 = lst[min(k0, Cp - 1u)], s1 = lst[min(k1, Cp - 1u)];
      uint4 b0[CPL], b1[CPL];
      load_row<CPL>(a.rs, sid[s0], a0, sub, b0);
      load_row<CPL>(a.rs, sid[s1], a1, sub, b1);
      const float d0 = octet_finish<DT, CPL>(a.rs, sub, sv, b0);
      const float d1 = octet_finish<DT, CPL>(a.rs, sub, sv, b1);
      if (sub == 0) {
        if (a0 && a.alpha * d0 <= sd[s0]) fl[s0] |= PR_REMOVED;
        if (a1 && a.alpha * d1 <= sd[s1]) fl[s1] |= PR_REMOVED;
      }
    }
    npair += nq;
    wave_sync();
  }
  // Degree fill to min(min_degree, R) with the nearest unused candidates,
  // occluded ones included (vnew2.cu:2076-2126).
  const uint32_t md = min(a.min_degree, R);
  while (oc < md) {
    int best = INT_MAX;
    for (uint32_t i = lane; i < Cp; i += 64) {
      const bool ok = sid[i] != DANCE_INV && (fl[i] & PR_INOUT) == 0u;
      if (ok) best = min(best, fkey(sd[i]));
    }
    const int M = wave_min_i(best);
    if (M == INT_MAX) break;
    uint32_t cand = 0xFFFFFFFFu;
    for (uint32_t i = lane; i < Cp; i += 64) {
      const bool ok = sid[i] != DANCE_INV && (fl[i] & PR_INOUT) == 0u && fkey(sd[i]) == M;
      if (ok) cand = min(cand, i);
    }
    const uint32_t pos = wave_min_u(cand);
    const uint32_t pick = uni_u(sid[pos]);
    if (lane == 0) {
      oid[oc] = pick;
      od[oc] = sd[pos];
    }
    oc++;
    for (uint32_t i = lane; i < Cp; i += 64)
      if (sid[i] == pick) fl[i] |= PR_INOUT;
    wave_sync();
  }
  wave_sync();
  for (uint32_t i = lane; i < C; i += 64) {
    g.work[wb + i] = i < oc ? oid[i] : DANCE_INV;
    g.wd[wb + i] = i < oc ? od[i] : FLT_MAX;
  }
  for (uint32_t i = lane; i < R; i += 64) g.cur[cb + i] = i < oc ? oid[i] : DANCE_INV;
  if (lane == 0) {
    g.deg_work[node] = oc;
    g.deg_cur[node] = oc;
  }
  if (a.ctr && lane == 0) {
    atomicAdd(&ctr_stripe(a.ctr)->prune_dist, (unsigned long long)npair);
    atomicAdd(&ctr_stripe(a.ctr)->prune_rounds, (unsigned long long)nround);
    atomicAdd(&ctr_stripe(a.ctr)->prune_exact_rounds, (unsigned long long)nexact);
    if (qon) {
      atomicAdd(&ctr_stripe(a.ctr)->prune_bound_checks, (unsigned long long)nbchk);
      atomicAdd(&ctr_stripe(a.ctr)->prune_bound_skips, (unsigned long long)nbskip);
    }
  }
}

// ---------------------------------------------------------------------------
// The same RobustPrune for rows of at most 128 candidates, organised around
// one sort (k_prune_rank).
//
// A round selects the remaining candidate of smallest (distance, index), and
// removal never changes a distance, so the candidates are ranked once by
// (distance, index) and everything after works on 128-bit masks over ranks,
// held in scalar registers: a round selects the lowest remaining rank; the
// candidates it tests (d_sel <= d) are exactly the remaining ranks; the fill
// takes the lowest ranks not yet output. With the quantized bound, its
// decision for every pair (selected rank i, candidate rank j > i) is made
// before the rounds: the exact integer code dots of all pairs come from int8
// MFMA tiles (v_mfma_i32_32x32x32_i8, 32 x 32 pairs per tile, K = 4 x 32 code
// bytes), and each pair is tested with the expression of q_pair_proves on the
// same inputs as the per-round test of k_prune. The pairs the bound leaves
// open are then listed and their exact distances computed in one batch (all
// loads of a pass in flight together), and the occlusion decision of every
// pair is a bit in LDS, so the rounds run on masks alone: a round removes
// occ[selected] from the remaining ranks. The decisions are those the rounds
// would make one pair at a time (same distance, operands in the same order,
// same test), so the graph is that of k_prune. More pairs are computed than
// the rounds would test (some open pairs involve ranks already removed), in
// exchange for no gather inside a round. Rows whose open pairs exceed the
// list (4 Cq) fall back to exact tests inside the rounds; without the bound
// every round tests its remaining ranks exactly. uint8 rows need no bound:
// their exact distance of every pair comes from int8 MFMA Gram tiles of the
// rows themselves (see kRankGram), so every decision is in LDS before the
// rounds and no pair is gathered twice.
// ---------------------------------------------------------------------------
constexpr uint32_t kRankCap = 128;  // candidates per row this kernel takes (C <= 128)

// How k_prune_rank decides its pairs: each round tests its remaining ranks
// exactly (kRankExact); the quantized bound's MFMA tiles first, then one
// exact batch for the pairs it leaves open (kRankBound); or, for uint8 rows,
// the exact distance of every pair from MFMA Gram tiles (kRankGram).
enum : int { kRankExact = 0, kRankBound = 1, kRankGram = 2 };

// Per-wave LDS: arrays of Cq = C rounded up to 32 entries (ids of the
// exact-test list; rid, rd by rank; the exact-test list of ranks; per-rank
// flags), and with MFMA tiles (bound or Gram) 4 words per rank of headers
// (the bound's {-2 s, r, a, root}, later the open-pair list; the Gram's
// squared row norms) and 4 mask words per rank.
__host__ __device__ constexpr uint32_t prune_rank_lds_words(uint32_t Cq, bool tiles) {
  return 5u * Cq + (tiles ? 8u * Cq : 0u);
}

// 16 code bytes of rank row `row` for MFMA K-step `step`: code chunk
// 1 + 2 step + lane/32 (chunk 0 is the header; chunks past 7 are zero).
// Both operands of a Gram tile take their rows this way, so the tile sums
// every code byte of a pair exactly once (layout checked on gfx950: lane l
// supplies row l % 32, and D[i][j] sits in accumulator v of lane l with
// j = l % 32, i = 8 (v / 4) + 4 (l / 32) + v % 4).
__device__ __forceinline__ v4i_t code_frag(const QBoundSet& qb, const uint32_t* rid, uint32_t row, uint32_t nvalid,
                                           uint32_t step, uint32_t lane) {
  const uint32_t chunk = 1u + 2u * step + (lane >> 5);
  v4i_t v = {0, 0, 0, 0};
  if (row < nvalid && chunk < kQChunks) {
    const uint4 c = qb.rows[(size_t)rid[row] * kQChunks + chunk];
    v = v4i_t{(int)c.x, (int)c.y, (int)c.z, (int)c.w};
  }
  return v;
}

__device__ __forceinline__ uint32_t ffs128(uint64_t m0, uint64_t m1) {
  return m0 ? (uint32_t)ffs64(m0) : (m1 ? 64u + (uint32_t)ffs64(m1) : 0xFFFFFFFFu);
}

// Occupancy floor: the bound's variant holds every code fragment of up to 96
// ranks (48 registers) next to its MFMA accumulators, which fits 5 waves per
// SIMD; the variant without it fits 6 at rows of up to 4 chunks per lane.
// Wider rows (and fp16 rows of 4 chunks per lane, whose tail selects take a
// few more registers) get no floor, so no variant spills.
template <int DT, int CPL, int PM>
constexpr int kRankMinWaves = PM != kRankExact ? 5 : (CPL < 4 || (CPL == 4 && DT != DANCE_F16)) ? 6 : 1;
template <int DT, int CPL, int PM>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(kRankMinWaves<DT, CPL, PM>, 8))) void k_prune_rank(PruneArgs a, uint32_t Cq) {
  constexpr bool QB = PM == kRankBound, XG = PM == kRankGram;
  static_assert(!XG || DT == DANCE_U8, "Gram tiles give exact distances of uint8 rows only");
  extern __shared__ uint32_t smem[];
  const uint32_t w = wave_index();
  const uint32_t gw = xcd_block(grid_block(), grid_blocks()) * kWavesPerBlock + w;
  const GraphBufs& g = a.g;
  if (gw >= g.N) return;
  const uint32_t node = a.order ? a.order[gw] : gw;
  const uint32_t N = g.N, R = g.R, C = g.C;
  const uint32_t lane = lane_id(), grp = lane >> 3, sub = lane & 7u;
  uint32_t* const base = smem + w * prune_rank_lds_words(Cq, PM != kRankExact);
  uint32_t* sid = base;                               // ids of the exact-test list (rounds)
  uint32_t* rid = base + Cq;                          // rank -> id
  float* rd = reinterpret_cast<float*>(base + 2 * Cq);  // rank -> distance
  uint32_t* lst = base + 3 * Cq;                      // ranks needing an exact distance
  uint32_t* rmf = base + 4 * Cq;                      // per rank: removed this round / repeated id
  // QB: per rank {-2 s, r, a, root} (a = -inf past the valid ranks), reused
  // after the bound tiles as the list of open pairs; then per rank 4 words:
  // the candidate ranks the bound proves kept, later those it occludes.
  float4* hq = reinterpret_cast<float4*>(base + 5 * Cq);
  uint32_t* plist = reinterpret_cast<uint32_t*>(hq);
  uint32_t* pm = reinterpret_cast<uint32_t*>(hq + Cq);
  const bool lo_in = lane < Cq, hi_in = lane + 64u < Cq;  // this lane's two slots exist

  const size_t wb = (size_t)node * C, cb = (size_t)node * R;
  const uint32_t deg = min(g.deg_work[node], C);
  [[maybe_unused]] const uint64_t t0 = dclock();
  // 1. candidates (a lane holds indices lane and lane + 64)
  uint32_t myid[2];
  int mykey[2];
  float mydist[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t i = lane + 64u * (uint32_t)h;
    uint32_t id = DANCE_INV;
    float dist = FLT_MAX;
    if (i < deg) {
      id = g.work[wb + i];
      dist = g.wd[wb + i];
      if (!(valid_for(id, N, node) && dist < FLT_MAX)) id = DANCE_INV;
    }
    if (i < Cq) {
      rmf[i] = 0u;
      lst[i] = 0u;
    }
    myid[h] = id;
    mydist[h] = dist;
    mykey[h] = fkey(dist);
  }
  // 2. rank = number of candidates before it in (distance, index) order; an
  // id met twice marks both copies. Candidate k is read from lane k % 64 of
  // slot k / 64 (wave-uniform k, so the reads are register reads).
  // Repeats are counted, not or-ed: a counter is one add per step, where a
  // carried flag costs the compiler a 0/1 register and its re-test.
  uint32_t myrank[2] = {0u, 0u};
  uint32_t ndup[2] = {0u, 0u};
  const uint32_t dlo = min(deg, 64u);
  for (uint32_t k = 0; k < dlo; ++k) {  // k < 64 <= index of slot 1
    const uint32_t idk = (uint32_t)__builtin_amdgcn_readlane((int)myid[0], (int)k);
    if (idk == DANCE_INV) continue;
    const int kk = __builtin_amdgcn_readlane(mykey[0], (int)k);
    myrank[0] += (kk < mykey[0] || (kk == mykey[0] && k < lane)) ? 1u : 0u;
    myrank[1] += kk <= mykey[1] ? 1u : 0u;
    ndup[0] += (idk == myid[0] && k != lane) ? 1u : 0u;
    ndup[1] += idk == myid[1] ? 1u : 0u;
  }
  for (uint32_t k = 64; k < deg; ++k) {  // k >= 64 > index of slot 0
    const uint32_t idk = (uint32_t)__builtin_amdgcn_readlane((int)myid[1], (int)(k - 64u));
    if (idk == DANCE_INV) continue;
    const int kk = __builtin_amdgcn_readlane(mykey[1], (int)(k - 64u));
    myrank[0] += kk < mykey[0] ? 1u : 0u;
    myrank[1] += (kk < mykey[1] || (kk == mykey[1] && k - 64u < lane)) ? 1u : 0u;
    ndup[0] += idk == myid[0] ? 1u : 0u;
    ndup[1] += (idk == myid[1] && k - 64u != lane) ? 1u : 0u;
  }
  const bool mydup[2] = {ndup[0] != 0u, ndup[1] != 0u};
  const uint64_t v0 = wballot(myid[0] != DANCE_INV), v1 = wballot(myid[1] != DANCE_INV);
  const uint32_t nvalid = popc64(v0) + popc64(v1);
#pragma unroll
  for (int h = 0; h < 2; ++h)
    if (myid[h] != DANCE_INV) {
      rid[myrank[h]] = myid[h];
      rd[myrank[h]] = mydist[h];
      rmf[myrank[h]] = mydup[h] ? 2u : 0u;
    }
  wave_sync();
  const uint64_t dup0 = wballot(lo_in && (rmf[lane] & 2u) != 0u);
  const uint64_t dup1 = wballot(hi_in && (rmf[lane + 64] & 2u) != 0u);
  const uint64_t all0 = nvalid >= 64 ? ~0ull : ((1ull << nvalid) - 1ull);
  const uint64_t all1 = nvalid >= 128 ? ~0ull : (nvalid > 64 ? ((1ull << (nvalid - 64)) - 1ull) : 0ull);
  if (lo_in) rmf[lane] = 0u;
  if (hi_in) rmf[lane + 64] = 0u;
  wave_sync();
  [[maybe_unused]] const uint64_t t1 = dclock();

  uint32_t npair = 0, nbchk = 0, nbskip = 0;
  bool batched = false;  // every needed pair decision is in pm before the rounds
  if constexpr (QB) {
    // 3. the bound's decision for every pair (i, j > i), from int8 MFMA Gram
    // tiles of the code rows: bit j of pm[4 i ..] = pair proven kept.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t r = lane + 64u * (uint32_t)h;
      if (r < Cq) {
        float4 v = make_float4(0.0f, 0.0f, -__builtin_inff(), 0.0f);
        if (r < nvalid) {
          const uint4 hd = a.qb.rows[(size_t)rid[r] * kQChunks];
          v = make_float4(-2.0f * __uint_as_float(hd.x), __uint_as_float(hd.y), __uint_as_float(hd.z),
                          prune_bound_root(a.qb, rd[r], a.alpha));
        }
        hq[r] = v;
      }
    }
    wave_sync();
    const uint32_t nt = (nvalid + 31u) >> 5;
    const uint32_t jl = lane & 31u, ih = 4u * (lane >> 5);
    // One 32 x 32 tile of pair decisions: rows ti, columns tj >= ti.
    auto tile = [&](uint32_t ti, uint32_t tj, const v4i_t(&fa)[4], const v4i_t(&fb)[4]) {
      v16i_t acc = {};
#pragma unroll
      for (uint32_t s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[s], fb[s], acc, 0, 0, 0);
      // j-side values per lane; i-side per accumulator from LDS. Invalid
      // ranks carry a = -inf, which fails the test.
      const uint32_t j = tj * 32u + jl;
      const float4 hj = hq[j];
      const float sy = -0.5f * hj.x, ry = hj.y, ay = hj.z, rootj = hj.w;
      uint32_t words = 0u;  // lane l < 32 collects the proof word of tile row l
      static_for<0, 16>([&](auto vc) {
        constexpr uint32_t v = decltype(vc)::value, ir = 8u * (v >> 2) + (v & 3u);
        const uint32_t i = ti * 32u + ir + ih;
        const float4 hi = hq[i];
        const float sT = (rootj + hi.y) * (1.0f + kQSlack);
        const bool pr = i < j && q_pair_proves_m2(hi.x, hi.z, sT, sy, ry, ay, acc[v]);
        const uint64_t m = wballot(pr);
        words = write_lane<ir>(words, (uint32_t)m);
        words = write_lane<ir + 4u>(words, (uint32_t)(m >> 32));
      });
      if (lane < 32u) pm[4u * (ti * 32u + lane) + tj] = words;
    };
    if (nt <= 3u) {
      // up to 96 ranks: every code fragment loaded at once, then the tiles
      v4i_t F[3][4];
      static_for<0, 3>([&](auto tc) {
        constexpr uint32_t t = decltype(tc)::value;
#pragma unroll
        for (uint32_t s = 0; s < 4; ++s) F[t][s] = code_frag(a.qb, rid, t * 32u + jl, nvalid, s, lane);
      });
      static_for<0, 3>([&](auto ic) {
        constexpr uint32_t ti = decltype(ic)::value;
        static_for<ti, 3>([&](auto jc) {
          constexpr uint32_t tj = decltype(jc)::value;
          if (tj < nt) tile(ti, tj, F[ti], F[tj]);
        });
      });
    } else {
      for (uint32_t ti = 0; ti < nt; ++ti) {
        v4i_t fa[4];
#pragma unroll
        for (uint32_t s = 0; s < 4; ++s) fa[s] = code_frag(a.qb, rid, ti * 32u + jl, nvalid, s, lane);
        tile(ti, ti, fa, fa);
        for (uint32_t tj = ti + 1u; tj < nt; ++tj) {
          v4i_t fb[4];
#pragma unroll
          for (uint32_t s = 0; s < 4; ++s) fb[s] = code_frag(a.qb, rid, tj * 32u + jl, nvalid, s, lane);
          tile(ti, tj, fa, fb);
        }
      }
    }
    // Words of tiles below the diagonal or past the last tile stay unset:
    // every reader masks them (open pairs keep j > i, j < nvalid; the rounds
    // keep only remaining ranks, which lie above the selected one).
    wave_sync();
    // 3b. open pairs (valid j > i that the bound leaves undecided): listed
    // and computed exactly in one batch when they fit the list (4 Cq pairs),
    // so the rounds read their decisions from LDS. The occlusion bits
    // replace the proof words: bit j of pm[4 i ..] = i occludes j.
    uint32_t op[2][4], cnt[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t i = lane + 64u * (uint32_t)h;
      cnt[h] = 0u;
#pragma unroll
      for (uint32_t q = 0; q < 4; ++q) {
        uint32_t m = 0u;
        if (i < nvalid) {
          const uint32_t lo = 32u * q;
          // j in [max(i + 1, lo), min(nvalid, lo + 32)) of this word
          const uint32_t b = i + 1u > lo ? i + 1u - lo : 0u, e = nvalid > lo ? min(nvalid - lo, 32u) : 0u;
          const uint32_t span = b < e ? ((e - b == 32u ? 0xFFFFFFFFu : ((1u << (e - b)) - 1u)) << b) : 0u;
          m = span & ~pm[4u * i + q];
        }
        op[h][q] = m;
        cnt[h] += __builtin_popcount(m);
      }
    }
    const uint32_t c0 = wave_reduce_i((int)cnt[0], 0, [](int x, int y) { return x + y; });
    const uint32_t c1 = wave_reduce_i((int)cnt[1], 0, [](int x, int y) { return x + y; });
    const uint32_t T = c0 + c1;
    nbchk = nvalid > 1u ? nvalid * (nvalid - 1u) / 2u : 0u;
    nbskip = nbchk - T;
    batched = T <= 4u * Cq;
    if (batched) {
      uint32_t w0 = wave_excl_scan_u(cnt[0]), w1 = c0 + wave_excl_scan_u(cnt[1]);
      wave_sync();  // the open masks are in registers: pm becomes the occlusion words
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t i = lane + 64u * (uint32_t)h;
        if (i < Cq) {
          pm[4u * i + 0] = 0u;
          pm[4u * i + 1] = 0u;
          pm[4u * i + 2] = 0u;
          pm[4u * i + 3] = 0u;
        }
        uint32_t& wp = h == 0 ? w0 : w1;
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
          uint32_t m = op[h][q];
          while (m) {
            const uint32_t bj = (uint32_t)__builtin_ctz(m);
            m &= m - 1u;
            plist[wp++] = i | ((32u * q + bj) << 8);
          }
        }
      }
      wave_sync();
      // exact distances, two pairs per octet in flight; the distance of
      // (i, j) is taken with i's row first, as the rounds would take it
      for (uint32_t p = 0; p < T; p += 16) {
        const uint32_t k0 = p + grp, k1 = p + 8 + grp;
        const bool a0 = k0 < T, a1 = k1 < T;
        const uint32_t e0 = plist[min(k0, T - 1u)], e1 = plist[min(k1, T - 1u)];
        const uint32_t i0 = e0 & 0xFFu, j0 = e0 >> 8, i1 = e1 & 0xFFu, j1 = e1 >> 8;
        uint4 x0[CPL], y0[CPL], x1[CPL], y1[CPL];
        load_row<CPL>(a.rs, rid[i0], a0, sub, x0);
        load_row<CPL>(a.rs, rid[j0], a0, sub, y0);
        load_row<CPL>(a.rs, rid[i1], a1, sub, x1);
        load_row<CPL>(a.rs, rid[j1], a1, sub, y1);
        const float d0 = octet_finish<DT, CPL>(a.rs, sub, x0, y0);
        const float d1 = octet_finish<DT, CPL>(a.rs, sub, x1, y1);
        if (sub == 0) {
          if (a0 && a.alpha * d0 <= rd[j0]) atomicOr(&pm[4u * i0 + (j0 >> 5)], 1u << (j0 & 31u));
          if (a1 && a.alpha * d1 <= rd[j1]) atomicOr(&pm[4u * i1 + (j1 >> 5)], 1u << (j1 & 31u));
        }
      }
      npair = T;
      wave_sync();
    }
  } else if constexpr (XG) {
    // 3'. uint8 rows: the exact distance of every pair from int8 MFMA Gram
    // tiles of the rows themselves. Bytes shifted by -128 (b ^ 0x80) fit
    // int8, and |a - b|^2 = |a'|^2 + |b'|^2 - 2 a'.b' holds in 32-bit
    // integers, so each distance is the integer of the octet sum, converted
    // to float the same way (padding bytes are -128 in both rows and add
    // nothing). Bit j of pm[4 i ..] = i occludes j, for valid j > i: the test
    // the rounds would make (alpha d <= d(node, j)); every pair is decided
    // before the rounds, and each candidate row is gathered once.
    constexpr uint32_t S = 4u * CPL;  // K-steps of 32 bytes over the padded row
    int* nrm = reinterpret_cast<int*>(hq);  // |row'|^2 by rank
    const uint32_t nt = (nvalid + 31u) >> 5;
    const uint32_t jl = lane & 31u, ih = 4u * (lane >> 5);
    // 16 shifted bytes of rank `row` for K-step `step` (chunk 2 step + lane/32)
    auto frag = [&](uint32_t row, uint32_t step) -> v4i_t {
      return row < nvalid ? u8_frag(a.rs, rid[row], step, lane) : v4i_t{0, 0, 0, 0};
    };
    auto sq4 = [](const v4i_t& f, int acc) { return i8_sq4(f, acc); };
    // lanes l and l + 32 hold the two halves of row t * 32 + l % 32
    auto put_norm = [&](uint32_t t, int part) {
      const int n = part + __shfl_xor(part, 32);
      if (lane < 32u) nrm[t * 32u + lane] = n;
    };
    auto decide = [&](uint32_t ti, uint32_t tj, const v16i_t& acc) {
      const uint32_t j = tj * 32u + jl;  // < nt * 32 <= Cq
      const bool jv = j < nvalid;
      const int nj = nrm[j];
      const float dj = rd[j];
      uint32_t words = 0u;  // lane l < 32 collects the occlusion word of tile row l
      static_for<0, 16>([&](auto vc) {
        constexpr uint32_t v = decltype(vc)::value, ir = 8u * (v >> 2) + (v & 3u);
        const uint32_t i = ti * 32u + ir + ih;
        const float d = u8_gram_dist(nrm[i], nj, acc[v]);
        const uint64_t m = wballot(jv && i < j && a.alpha * d <= dj);
        words = write_lane<ir>(words, (uint32_t)m);
        words = write_lane<ir + 4u>(words, (uint32_t)(m >> 32));
      });
      if (lane < 32u) pm[4u * (ti * 32u + lane) + tj] = words;
    };
    if (CPL == 1 && nt <= 3u) {
      // up to 96 ranks of 128-byte rows: every fragment loaded at once
      v4i_t F[3][S];
      static_for<0, 3>([&](auto tc) {
        constexpr uint32_t t = decltype(tc)::value;
#pragma unroll
        for (uint32_t s = 0; s < S; ++s) F[t][s] = frag(t * 32u + jl, s);
      });
      static_for<0, 3>([&](auto tc) {
        constexpr uint32_t t = decltype(tc)::value;
        int part = 0;
#pragma unroll
        for (uint32_t s = 0; s < S; ++s) part = sq4(F[t][s], part);
        put_norm(t, part);
      });
      wave_sync();
      static_for<0, 3>([&](auto ic) {
        constexpr uint32_t ti = decltype(ic)::value;
        static_for<ti, 3>([&](auto jc) {
          constexpr uint32_t tj = decltype(jc)::value;
          if (tj < nt) {
            v16i_t acc = {};
#pragma unroll
            for (uint32_t s = 0; s < S; ++s) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(F[ti][s], F[tj][s], acc, 0, 0, 0);
            decide(ti, tj, acc);
          }
        });
      });
    } else {
      for (uint32_t t = 0; t < nt; ++t) {
        int part = 0;
#pragma unroll
        for (uint32_t s = 0; s < S; ++s) part = sq4(frag(t * 32u + jl, s), part);
        put_norm(t, part);
      }
      wave_sync();
      for (uint32_t ti = 0; ti < nt; ++ti)
        for (uint32_t tj = ti; tj < nt; ++tj) {
          v16i_t acc = {};
#pragma unroll
          for (uint32_t s = 0; s < S; ++s)
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(frag(ti * 32u + jl, s), frag(tj * 32u + jl, s), acc, 0, 0, 0);
          decide(ti, tj, acc);
        }
    }
    // Words of tiles below the diagonal or past the last tile stay unset:
    // the rounds keep only remaining ranks, which lie above the selected one.
    npair = nvalid > 1u ? nvalid * (nvalid - 1u) / 2u : 0u;
    batched = true;
    wave_sync();
  }

  // 4. selection rounds on rank masks. Rank r's id, distance and (batched)
  // occlusion words sit in lane r % 64 of register slot r / 64, read with
  // v_readlane; outputs collect in registers (output k in lane k % 64 of
  // slot k / 64). The exact-test path of the rounds keeps its lists in LDS.
  [[maybe_unused]] const uint64_t t2 = dclock();
  uint32_t r_id[2], r_occ[2][4];
  float r_d[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t r = min(lane + 64u * (uint32_t)h, Cq - 1u);
    r_id[h] = rid[r];
    r_d[h] = rd[r];
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) r_occ[h][q] = 0u;
    if constexpr (QB || XG) {
      if (batched) {
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) r_occ[h][q] = pm[4u * r + q];
      }
    }
  }
  auto rank_u = [&](const uint32_t (&v)[2], uint32_t r) -> uint32_t {
    return (uint32_t)__builtin_amdgcn_readlane((int)(r < 64u ? v[0] : v[1]), (int)(r & 63u));
  };
  uint32_t o_id[2] = {DANCE_INV, DANCE_INV};
  float o_d[2] = {FLT_MAX, FLT_MAX};
  auto emit = [&](uint32_t k, uint32_t id, float d) {  // output k (uniform)
    if (k < 64u) {
      o_id[0] = lane == k ? id : o_id[0];
      o_d[0] = lane == k ? d : o_d[0];
    } else {
      o_id[1] = lane == k - 64u ? id : o_id[1];
      o_d[1] = lane == k - 64u ? d : o_d[1];
    }
  };
  uint64_t rem0 = all0, rem1 = all1, io0 = 0ull, io1 = 0ull;
  uint32_t oc = 0, nround = 0, nexact = 0;
  auto drop_same_id = [&](uint32_t id) {  // every copy of id leaves and counts as output
    const uint64_t s0 = wballot(lane < nvalid && r_id[0] == id);
    const uint64_t s1 = wballot(lane + 64u < nvalid && r_id[1] == id);
    rem0 &= ~s0;
    rem1 &= ~s1;
    io0 |= s0;
    io1 |= s1;
  };
  while (oc < R) {
    const uint32_t r = ffs128(rem0, rem1);
    if (r == 0xFFFFFFFFu) break;
    const uint32_t sel = rank_u(r_id, r);
    const float seld = __uint_as_float(rank_u(reinterpret_cast<const uint32_t(&)[2]>(r_d), r));
    emit(oc, sel, seld);
    oc++;
    nround++;
    if (r < 64) {
      rem0 &= ~(1ull << r);
      io0 |= 1ull << r;
    } else {
      rem1 &= ~(1ull << (r - 64));
      io1 |= 1ull << (r - 64);
    }
    if ((r < 64 ? (dup0 >> r) : (dup1 >> (r - 64))) & 1ull) drop_same_id(sel);
    if (oc >= R) break;
    if (batched) {  // bound or Gram tiles: every needed decision is in r_occ
      const uint32_t l = r & 63u;
      const bool hi = r >= 64u;
      const uint32_t w0 = (uint32_t)__builtin_amdgcn_readlane((int)(hi ? r_occ[1][0] : r_occ[0][0]), (int)l);
      const uint32_t w1 = (uint32_t)__builtin_amdgcn_readlane((int)(hi ? r_occ[1][1] : r_occ[0][1]), (int)l);
      const uint32_t w2 = (uint32_t)__builtin_amdgcn_readlane((int)(hi ? r_occ[1][2] : r_occ[0][2]), (int)l);
      const uint32_t w3 = (uint32_t)__builtin_amdgcn_readlane((int)(hi ? r_occ[1][3] : r_occ[0][3]), (int)l);
      rem0 &= ~((uint64_t)w0 | ((uint64_t)w1 << 32));
      rem1 &= ~((uint64_t)w2 | ((uint64_t)w3 << 32));
      continue;
    }
    uint64_t need0 = rem0, need1 = rem1;
    if (need0 == 0 && need1 == 0) continue;
    if constexpr (QB) {
      const uint64_t p0 = (uint64_t)uni_u(pm[4 * r + 0]) | ((uint64_t)uni_u(pm[4 * r + 1]) << 32);
      const uint64_t p1 = (uint64_t)uni_u(pm[4 * r + 2]) | ((uint64_t)uni_u(pm[4 * r + 3]) << 32);
      need0 &= ~p0;
      need1 &= ~p1;
      if (need0 == 0 && need1 == 0) continue;
    }
    uint4 sv[CPL];  // the selected row, in flight while the list is built
    load_row<CPL>(a.rs, sel, true, sub, sv);
    nexact++;
    const uint32_t n0 = popc64(need0), nn = n0 + popc64(need1);
    // the list holds each rank and, in sid, its id
    if ((need0 >> lane) & 1ull) lst[mbcnt64(need0)] = lane;
    if ((need1 >> lane) & 1ull) lst[n0 + mbcnt64(need1)] = lane + 64u;
    if ((need0 >> lane) & 1ull) sid[mbcnt64(need0)] = r_id[0];
    if ((need1 >> lane) & 1ull) sid[n0 + mbcnt64(need1)] = r_id[1];
    wave_sync();
    for (uint32_t p = 0; p < nn; p += 16) {
      const uint32_t k0 = p + grp, k1 = p + 8 + grp;
      const bool a0 = k0 < nn, a1 = k1 < nn;
      const uint32_t r0 = min(lst[min(k0, Cq - 1u)], Cq - 1u);
      const uint32_t r1 = min(lst[min(k1, Cq - 1u)], Cq - 1u);
      uint4 b0[CPL], b1[CPL];
      load_row<CPL>(a.rs, sid[min(k0, Cq - 1u)], a0, sub, b0);
      load_row<CPL>(a.rs, sid[min(k1, Cq - 1u)], a1, sub, b1);
      const float d0 = octet_finish<DT, CPL>(a.rs, sub, sv, b0);
      const float d1 = octet_finish<DT, CPL>(a.rs, sub, sv, b1);
      if (sub == 0) {
        if (a0 && a.alpha * d0 <= rd[r0]) rmf[r0] = 1u;
        if (a1 && a.alpha * d1 <= rd[r1]) rmf[r1] = 1u;
      }
    }
    npair += nn;
    wave_sync();
    const bool f0 = lo_in && rmf[lane] != 0u, f1 = hi_in && rmf[lane + 64] != 0u;
    rem0 &= ~wballot(f0);
    rem1 &= ~wballot(f1);
    if (f0) rmf[lane] = 0u;
    if (f1) rmf[lane + 64] = 0u;
    wave_sync();
  }
  // 5. degree fill to min(min_degree, R): lowest ranks not yet output,
  // occluded ones included (vnew2.cu:2076-2126)
  [[maybe_unused]] const uint64_t t3 = dclock();
  const uint32_t md = min(a.min_degree, R);
  while (oc < md) {
    const uint32_t r = ffs128(all0 & ~io0, all1 & ~io1);
    if (r == 0xFFFFFFFFu) break;
    const uint32_t pick = rank_u(r_id, r);
    emit(oc, pick, __uint_as_float(rank_u(reinterpret_cast<const uint32_t(&)[2]>(r_d), r)));
    oc++;
    if (r < 64)
      io0 |= 1ull << r;
    else
      io1 |= 1ull << (r - 64);
    if ((r < 64 ? (dup0 >> r) : (dup1 >> (r - 64))) & 1ull) drop_same_id(pick);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t i = lane + 64u * (uint32_t)h;
    if (i < C) {
      g.work[wb + i] = i < oc ? o_id[h] : DANCE_INV;
      g.wd[wb + i] = i < oc ? o_d[h] : FLT_MAX;
    }
    if (i < R) g.cur[cb + i] = i < oc ? o_id[h] : DANCE_INV;
  }
  if (lane == 0) {
    g.deg_work[node] = oc;
    g.deg_cur[node] = oc;
  }
  if (a.ctr && lane == 0) {
    VCounters* c = ctr_stripe(a.ctr);
    atomicAdd(&c->prune_dist, (unsigned long long)npair);
    atomicAdd(&c->prune_rounds, (unsigned long long)nround);
    atomicAdd(&c->prune_exact_rounds, (unsigned long long)nexact);
    if (QB) {
      atomicAdd(&c->prune_bound_checks, (unsigned long long)nbchk);
      atomicAdd(&c->prune_bound_skips, (unsigned long long)nbskip);
    }
#if DANCE_SEARCH_TIMING
    const uint64_t t4 = dclock();
    atomicAdd(&c->cyc_prune_rank, (unsigned long long)(t1 - t0));
    atomicAdd(&c->cyc_prune_gram, (unsigned long long)(t2 - t1));
    atomicAdd(&c->cyc_prune_rounds, (unsigned long long)(t3 - t2));
    atomicAdd(&c->cyc_prune_fill, (unsigned long long)(t4 - t3));
#endif
  }
}

// ---------------------------------------------------------------------------
// Reverse edges. k_rev_keys emits one (target, slot) item per forward slot j =
// s*R + i in source order and snapshots that slot's stored distance; a stable
// LSD radix sort by target then yields every segment in ascending source
// order. k_merge is reverse_merge_csr_kernel (vnew2.cu:1722-1814) over those
// canonical segments. The reference recomputes d(t, s) for each reverse
// candidate; here it is read from the snapshot of s's forward entry, which
// holds d(s, t): every writer of a work row stores the canonical distance of
// the row's vertex to the entry (init, search, online insert, merge, prune
// keep them), and the canonical distance is bitwise symmetric (a-b and b-a
// differ only in sign). The snapshot is taken before any merge writes rows.
// ---------------------------------------------------------------------------
// Sources [s_lo, s_lo + items / R): item j covers forward slot s_lo R + j.
// With s_lo = 0 and items = N R this is the whole graph (item = slot); a
// graph of 2^32 or more slots is done in parts of fewer (see k_wide_gather).
static __global__ void k_rev_keys(const uint32_t* __restrict__ work, const uint32_t* __restrict__ deg_work,
                                  const float* __restrict__ wd, uint32_t N, uint32_t R, uint32_t C, uint32_t s_lo,
                                  size_t items, uint32_t* __restrict__ keys, uint32_t* __restrict__ vals,
                                  float* __restrict__ snap) {
  const size_t j = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= items) return;
  const uint32_t s = s_lo + (uint32_t)(j / R), i = (uint32_t)(j % R);
  const uint32_t deg = min(deg_work[s], R);
  const size_t wi = (size_t)s * C + i;
  const uint32_t t = i < deg ? work[wi] : DANCE_INV;
  const bool v = t != DANCE_INV && t < N && t != s;
  keys[j] = v ? t : N;
  vals[j] = (uint32_t)j;
  snap[(size_t)s_lo * R + j] = v ? wd[wi] : FLT_MAX;
}

// Graphs of 2^32 or more forward slots: the sources are split into P parts
// of fewer than 2^32 slots each, and each part is sorted by target on its
// own (32-bit items, as for smaller graphs). A target's sources are then the
// concatenation of its part segments in part order, which is still ascending
// source order. k_wide_offsets adds the parts' offsets (64-bit), and
// k_wide_gather (one wave per target) writes each segment's sources and
// slot snapshots in that order, so the merge reads them by sorted position.
constexpr uint32_t kMaxRevParts = 16;
struct WideParts {
  uint32_t P;
  uint32_t s_lo[kMaxRevParts];    // first source of each part
  size_t vbase[kMaxRevParts];     // each part's sorted local slots start here in pvals
};
static __global__ void k_wide_offsets(uint32_t N, WideParts wp, const uint32_t* __restrict__ poffs,
                                      uint64_t* __restrict__ offs64) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t > N) return;
  uint64_t sum = 0;
  for (uint32_t p = 0; p < wp.P; ++p) sum += poffs[(size_t)p * (N + 1) + t];
  offs64[t] = sum;
}
static __global__ __launch_bounds__(256) void k_wide_gather(uint32_t N, uint32_t R, WideParts wp,
                                                            const uint32_t* __restrict__ poffs,
                                                            const uint32_t* __restrict__ pvals,
                                                            const float* __restrict__ snap,
                                                            const uint64_t* __restrict__ offs64,
                                                            uint32_t* __restrict__ src_sorted,
                                                            float* __restrict__ snap_sorted) {
  const uint32_t t = grid_block() * 4u + (threadIdx.x >> 6), lane = threadIdx.x & 63u;
  if (t >= N) return;
  uint64_t out = offs64[t];
  for (uint32_t p = 0; p < wp.P; ++p) {
    const uint32_t* po = poffs + (size_t)p * (N + 1);
    const uint32_t b = po[t], e = po[t + 1];
    for (uint32_t k = b + lane; k < e; k += 64u) {
      const uint32_t local = pvals[wp.vbase[p] + k];
      src_sorted[out + (k - b)] = wp.s_lo[p] + local / R;
      snap_sorted[out + (k - b)] = snap[(size_t)wp.s_lo[p] * R + local];
    }
    out += e - b;
  }
}

// CSR offsets from the sorted keys (invalid items carry key N and sort last):
// offs[t] = first index whose key is >= t, for t in [0, N]. Item i fills the
// targets after its predecessor's key up to its own; i = n closes the range.
static __global__ void k_seg_offsets(const uint32_t* __restrict__ keys, size_t n, uint32_t N,
                                     uint32_t* __restrict__ offs) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i > n) return;
  const uint32_t lo = i == 0 ? 0u : keys[i - 1] + 1u;
  const uint32_t hi = i == n ? N : min(keys[i], N);
  for (uint32_t t = lo; t <= hi && t <= N; ++t) offs[t] = (uint32_t)i;
}

struct MergeArgs {
  RowSet rs;
  GraphBufs g;
  const uint32_t* offsets;  // N+1
  const uint32_t* srcs;     // sorted forward slots s*R + i
  const float* snap;        // distance of forward slot j
  uint32_t heavy_threshold, heavy_sample;
  const uint32_t* order;
  VCounters* ctr;
  // Graphs of 2^32 or more slots (k_wide_gather): 64-bit offsets, and srcs /
  // snap hold each sorted position's source and distance. nullptr otherwise.
  const uint64_t* offsets64;
  // Source and snapshot distance of sorted position idx.
  __device__ __forceinline__ void at(size_t idx, uint32_t R, uint32_t& src, float& d) const {
    if (offsets64) {
      src = srcs[idx];
      d = snap[idx];
    } else {
      const uint32_t slot = srcs[idx];
      src = slot / R;
      d = snap[slot];
    }
  }
  __device__ __forceinline__ void segment(uint32_t t, size_t& begin, size_t& end) const {
    if (offsets64) {
      begin = offsets64[t];
      end = offsets64[t + 1];
    } else {
      begin = offsets[t];
      end = offsets[t + 1];
    }
  }
};

__host__ __device__ constexpr uint32_t merge_lds_words(uint32_t Cp) { return 2u * Cp + 128u; }

template <int DT, int CPL>
__global__ __launch_bounds__(kBlock) void k_merge(MergeArgs a, uint32_t Cp) {
  extern __shared__ uint32_t smem[];
  const uint32_t w = wave_index();
  const uint32_t gw = xcd_block(grid_block(), grid_blocks()) * kWavesPerBlock + w;
  const GraphBufs& g = a.g;
  if (gw >= g.N) return;
  const uint32_t t = a.order ? a.order[gw] : gw;
  const uint32_t N = g.N, C = g.C, R = g.R;
  const uint32_t lane = lane_id();
  uint32_t* wid = smem + w * merge_lds_words(Cp);
  float* wdd = reinterpret_cast<float*>(wid + Cp);
  uint32_t* lst = wid + 2 * Cp;
  float* lsd = reinterpret_cast<float*>(lst + 64);
  size_t begin, end;
  a.segment(t, begin, end);
  const uint32_t indeg = (uint32_t)(end - begin);
  if (indeg == 0) return;
  uint32_t count = indeg;
  if (a.heavy_threshold != 0 && indeg > a.heavy_threshold) {
    count = min(a.heavy_sample, indeg);
    if (count == 0) count = 1;
  }
  const size_t wb = (size_t)t * C;
  uint32_t deg = min(g.deg_work[t], C);
  for (uint32_t i = lane; i < Cp; i += 64) {
    wid[i] = i < C ? g.work[wb + i] : DANCE_INV;
    wdd[i] = i < C ? g.wd[wb + i] : -FLT_MAX;
  }
  wave_sync();
  bool worst_ok = false;
  int wpos = -1;
  float wdist = -FLT_MAX;
  uint32_t ncand = 0;
  for (uint32_t b = 0; b < count; b += 64) {
    const uint32_t k = b + lane;
    uint32_t src = DANCE_INV;
    float dsrc = FLT_MAX;
    if (k < count) {
      const size_t idx = count < indeg ? begin + (size_t)(((unsigned long long)k * indeg) / count) : begin + k;
      a.at(idx, R, src, dsrc);
    }
    const bool v = valid_for(src, N, t);
    bool inrow = false;
    for (uint32_t j = 0; j < deg; ++j) inrow |= wid[j] == src;
    const bool need = v && !inrow;
    const uint64_t m = wballot(need);
    const uint32_t n = popc64(m);
    if (n == 0) continue;
    if (need) {
      lst[mbcnt64(m)] = src;
      lsd[mbcnt64(m)] = dsrc;
    }
    wave_sync();
    ncand += n;
    const uint32_t ck = lane < n ? lst[lane] : DANCE_INV;
    const float dk = lane < n ? lsd[lane] : FLT_MAX;
    wave_sync();
    for (uint32_t kk = 0; kk < n; ++kk) {
      const uint32_t s = rdlane_u(ck, (int)kk);
      const float ds = rdlane_f(dk, (int)kk);
      bool dup = false;
      for (uint32_t bb = 0; bb < deg && !dup; bb += 64) {
        const uint32_t i = bb + lane;
        dup = wballot(i < deg && wid[i] == s) != 0;
      }
      if (dup) continue;
      if (deg < C) {
        if (lane == 0) {
          wid[deg] = s;
          wdd[deg] = ds;
        }
        deg++;
        worst_ok = false;
        wave_sync();
        continue;
      }
      if (!worst_ok) {
        int best = INT_MIN;
        for (uint32_t i = lane; i < C; i += 64)
          if (wdd[i] == wdd[i]) best = max(best, fkey(wdd[i]));
        const int M = wave_max_i(best);
        wpos = -1;
        wdist = -FLT_MAX;
        if (M != INT_MIN && __int_as_float(M) > -FLT_MAX) {
          uint32_t cand = 0xFFFFFFFFu;
          for (uint32_t i = lane; i < C; i += 64)
            if (wdd[i] == wdd[i] && fkey(wdd[i]) == M) cand = min(cand, i);
          wpos = (int)wave_min_u(cand);
          wdist = __int_as_float(M);
        }
        worst_ok = true;
      }
      if (wpos >= 0 && ds < wdist) {
        if (lane == 0) {
          wid[wpos] = s;
          wdd[wpos] = ds;
        }
        worst_ok = false;
        wave_sync();
      }
    }
  }
  wave_sync();
  for (uint32_t i = lane; i < C; i += 64) {
    g.work[wb + i] = wid[i];
    g.wd[wb + i] = wdd[i];
  }
  if (lane == 0) {
    g.deg_work[t] = deg;
    if (a.ctr) {
      atomicAdd(&ctr_stripe(a.ctr)->merge_dist, (unsigned long long)ncand);
      atomicAdd(&ctr_stripe(a.ctr)->reverse_edges, (unsigned long long)indeg);
      atomicAdd(&ctr_stripe(a.ctr)->touched_rows, 1ull);
    }
  }
}

// Register-resident variant of k_merge for C <= 64*MS: the work row lives in
// MS VGPRs per lane (entry i = lane i % 64, slot i / 64), so membership tests
// are ballots and the worst-slot search is one wave reduction. Same decisions
// as k_merge (reverse_merge_csr_kernel, vnew2.cu:1722-1814): per candidate in
// source order, skip if present, append while deg < C, else replace the
// largest distance (lowest slot on ties) when strictly closer.
template <int MS>
struct MergeRow {
  uint32_t id[MS];
  float d[MS];
  __device__ __forceinline__ uint32_t id_at(uint32_t i) const {
    uint32_t v = id[0];
#pragma unroll
    for (int s = 1; s < MS; ++s)
      if ((i >> 6) == (uint32_t)s) v = id[s];
    return rdlane_u(v, (int)(i & 63u));
  }
  __device__ __forceinline__ bool contains(uint32_t x, uint32_t deg, uint32_t lane) const {
    uint64_t m = 0;
#pragma unroll
    for (int s = 0; s < MS; ++s) m |= wballot((uint32_t)s * 64u + lane < deg && id[s] == x);
    return m != 0;
  }
  __device__ __forceinline__ void set(uint32_t i, uint32_t x, float dist, uint32_t lane) {
    if (lane == (i & 63u)) {
#pragma unroll
      for (int s = 0; s < MS; ++s)
        if ((i >> 6) == (uint32_t)s) {
          id[s] = x;
          d[s] = dist;
        }
    }
  }
  // Largest non-NaN distance over [0, C) and its lowest slot; -1 when none
  // exceeds -FLT_MAX.
  __device__ __forceinline__ int worst(uint32_t C, uint32_t lane, float* wdist) const {
    int best = INT_MIN;
    uint32_t bi = 0xFFFFFFFFu;
#pragma unroll
    for (int s = 0; s < MS; ++s) {
      const uint32_t i = (uint32_t)s * 64u + lane;
      if (i < C && d[s] == d[s]) {
        const int k = fkey(d[s]);
        if (k > best) {
          best = k;
          bi = i;
        }
      }
    }
    const int M = wave_max_i(best);
    *wdist = -FLT_MAX;
    if (M == INT_MIN || !(__int_as_float(M) > -FLT_MAX)) return -1;
    *wdist = __int_as_float(M);
    return (int)wave_min_u(best == M ? bi : 0xFFFFFFFFu);
  }
};

template <int DT, int CPL, int MS>
__global__ __launch_bounds__(kBlock) void k_merge_reg(MergeArgs a) {
  const uint32_t w = wave_index();
  const uint32_t gw = xcd_block(grid_block(), grid_blocks()) * kWavesPerBlock + w;
  const GraphBufs& g = a.g;
  if (gw >= g.N) return;
  const uint32_t t = a.order ? a.order[gw] : gw;
  const uint32_t N = g.N, C = g.C, R = g.R;
  const uint32_t lane = lane_id();
  size_t begin, end;
  a.segment(t, begin, end);
  const uint32_t indeg = (uint32_t)(end - begin);
  if (indeg == 0) return;
  uint32_t count = indeg;
  if (a.heavy_threshold != 0 && indeg > a.heavy_threshold) {
    count = min(a.heavy_sample, indeg);
    if (count == 0) count = 1;
  }
  const size_t wb = (size_t)t * C;
  uint32_t deg = min(g.deg_work[t], C);
  MergeRow<MS> row;
#pragma unroll
  for (int s = 0; s < MS; ++s) {
    const uint32_t i = (uint32_t)s * 64u + lane;
    row.id[s] = i < C ? g.work[wb + i] : DANCE_INV;
    row.d[s] = i < C ? g.wd[wb + i] : -FLT_MAX;
  }
  bool worst_ok = false;
  int wpos = -1;
  float wdist = -FLT_MAX;
  uint32_t ncand = 0;
  for (uint32_t b = 0; b < count; b += 64) {
    const uint32_t k = b + lane;
    uint32_t src = DANCE_INV;
    float dsrc = FLT_MAX;
    if (k < count) {
      const size_t idx = count < indeg ? begin + (size_t)(((unsigned long long)k * indeg) / count) : begin + k;
      a.at(idx, R, src, dsrc);
    }
    const bool v = valid_for(src, N, t);
    const float dsv = v ? dsrc : FLT_MAX;
    ncand += popc64(wballot(v));
    // Once the row is full its worst only decreases, so a source that does
    // not beat the batch-start worst is rejected at its turn as well: the
    // batch walks only the others (hub targets reject most of their list).
    if (deg == C && !worst_ok) {
      wpos = row.worst(C, lane, &wdist);
      worst_ok = true;
    }
    uint64_t m = wballot(v && (deg < C || (wpos >= 0 && dsv < wdist)));
    while (m) {
      const int kk = ffs64(m);
      m &= m - 1;
      const uint32_t s = rdlane_u(src, kk);
      const float ds = rdlane_f(dsv, kk);
      if (deg == C && worst_ok && !(wpos >= 0 && ds < wdist)) continue;  // rejected either way
      if (row.contains(s, deg, lane)) continue;
      if (deg < C) {
        row.set(deg, s, ds, lane);
        ++deg;
        worst_ok = false;
        continue;
      }
      if (!worst_ok) {
        wpos = row.worst(C, lane, &wdist);
        worst_ok = true;
      }
      if (wpos >= 0 && ds < wdist) {
        row.set((uint32_t)wpos, s, ds, lane);
        worst_ok = false;
      }
    }
  }
#pragma unroll
  for (int s = 0; s < MS; ++s) {
    const uint32_t i = (uint32_t)s * 64u + lane;
    if (i < C) {
      g.work[wb + i] = row.id[s];
      g.wd[wb + i] = row.d[s];
    }
  }
  if (lane == 0) {
    g.deg_work[t] = deg;
    if (a.ctr) {
      atomicAdd(&ctr_stripe(a.ctr)->merge_dist, (unsigned long long)ncand);
      atomicAdd(&ctr_stripe(a.ctr)->reverse_edges, (unsigned long long)indeg);
      atomicAdd(&ctr_stripe(a.ctr)->touched_rows, 1ull);
    }
  }
}

// ---------------------------------------------------------------------------
// Approximate medoid (medoid_score_kernel_warp, vnew2.cu:1032-1064): one
// wave per candidate; distances by octets, summed in sample order by lane 0.
// ---------------------------------------------------------------------------
template <int DT, int CPL>
__global__ __launch_bounds__(kBlock) void k_medoid(RowSet rs, uint32_t N, uint32_t nc, uint32_t ns,
                                                   float* scores, uint32_t* cands) {
  __shared__ float buf[kWavesPerBlock][512];
  const uint32_t w = wave_index();
  const uint32_t cw = grid_block() * kWavesPerBlock + w;
  if (cw >= nc) return;
  const uint32_t lane = lane_id(), grp = lane >> 3, sub = lane & 7u;
  const uint32_t c = d_hash_u32(cw * 9973u + 17u) % N;
  uint4 cv[CPL];
  load_row<CPL>(rs, c, true, sub, cv);
  float sum = 0.0f;
  for (uint32_t base = 0; base < ns; base += 512) {
    const uint32_t cnt = min(512u, ns - base);
    for (uint32_t p = 0; p < cnt; p += 16) {
      const uint32_t k0 = p + grp, k1 = p + 8 + grp;
      const bool a0 = k0 < cnt, a1 = k1 < cnt;
      const uint32_t s0 = d_hash_u32((base + k0) * 10007u + 131u) % N;
      const uint32_t s1 = d_hash_u32((base + k1) * 10007u + 131u) % N;
      uint4 b0[CPL], b1[CPL];
      load_row<CPL>(rs, s0, a0, sub, b0);
      load_row<CPL>(rs, s1, a1, sub, b1);
      const float d0 = octet_finish<DT, CPL>(rs, sub, cv, b0);
      const float d1 = octet_finish<DT, CPL>(rs, sub, cv, b1);
      if (sub == 0) {
        if (a0) buf[w][k0] = d0;
        if (a1) buf[w][k1] = d1;
      }
    }
    wave_sync();
    if (lane == 0) {
      for (uint32_t k = 0; k < cnt; ++k) {
        const uint32_t smp = d_hash_u32((base + k) * 10007u + 131u) % N;
        if (smp == c) continue;
        sum += buf[w][k];
      }
    }
    wave_sync();
  }
  if (lane == 0) {
    scores[cw] = sum / (float)ns;
    cands[cw] = c;
  }
}

// init_random_graph (vnew2.cu:1066-1117): R hashed neighbours per vertex.
template <int DT, int CPL>
__global__ __launch_bounds__(kBlock) void k_init(RowSet rs, GraphBufs g) {
  __shared__ uint32_t lstb[kWavesPerBlock][64];
  __shared__ float lsdb[kWavesPerBlock][64];
  const uint32_t w = wave_index();
  const uint32_t node = grid_block() * kWavesPerBlock + w;
  const uint32_t N = g.N, R = g.R, C = g.C;
  if (node >= N) return;
  const uint32_t lane = lane_id(), grp = lane >> 3, sub = lane & 7u;
  const size_t cb = (size_t)node * R, wb = (size_t)node * C;
  for (uint32_t i = lane; i < C; i += 64) {
    g.work[wb + i] = DANCE_INV;
    g.wd[wb + i] = FLT_MAX;
  }
  uint4 nv[CPL];
  load_row<CPL>(rs, node, true, sub, nv);
  for (uint32_t b = 0; b < R; b += 64) {
    const uint32_t i = b + lane;
    const uint32_t nb = i < R ? init_neighbor(node, i, N) : DANCE_INV;
    const bool v = i < R && nb != DANCE_INV;
    const uint64_t m = wballot(v);
    const uint32_t n = popc64(m);
    if (v) lstb[w][mbcnt64(m)] = nb;
    wave_sync();
    batch_dist<DT, CPL>(rs, nv, lstb[w], lsdb[w], n, grp, sub);
    const float dist = v ? lsdb[w][mbcnt64(m)] : FLT_MAX;
    if (i < R) {
      g.cur[cb + i] = nb;
      g.work[wb + i] = nb;
      g.wd[wb + i] = dist;
    }
    wave_sync();
  }
  if (lane == 0) {
    const uint32_t deg = N > 1 ? R : 0u;
    g.deg_cur[node] = deg;
    g.deg_work[node] = deg;
  }
}

// Approximate nearest pivots for the locality schedule, from integer codes:
// one thread per vertex, pivot codes staged in LDS 64 at a time. U8 = false
// reads the quantized rows (header {s, r, a} + 7 chunks of int8 codes;
// distance ~ a_x + a_p - 2 s_x s_p <q_x, q_p>); U8 = true reads uint8 rows of
// at most 8 chunks (exact squared distance from unsigned dot products). Only
// the processing order depends on the result, never the graph.
template <bool U8>
__global__ __launch_bounds__(256) void k_cells_q(const uint4* __restrict__ rows, uint32_t stride16, uint32_t nch,
                                                 uint32_t N, const uint32_t* __restrict__ pivots, uint32_t K,
                                                 uint32_t levels, uint32_t* __restrict__ cell,
                                                 uint32_t* __restrict__ vid) {
  constexpr uint32_t NC = U8 ? 8u : 7u;  // code chunks per row
  constexpr uint32_t OFF = U8 ? 0u : 1u;  // q-rows keep their header in chunk 0
  __shared__ uint4 pc[64][NC];
  __shared__ float pn[64], psc[64];
  const uint32_t v = blockIdx.x * 256u + threadIdx.x;
  const bool act = v < N;
  const uint32_t have = U8 ? nch : 8u;
  uint4 xc[NC];
  float sx = 1.0f, ax = 0.0f;
  {
    const uint4* r = rows + (size_t)(act ? v : 0u) * stride16;
#pragma unroll
    for (uint32_t c = 0; c < NC; ++c) xc[c] = (act && OFF + c < have) ? r[OFF + c] : make_uint4(0u, 0u, 0u, 0u);
    if constexpr (U8) {
      uint32_t n2 = 0;
#pragma unroll
      for (uint32_t c = 0; c < NC; ++c) {
        n2 = __builtin_amdgcn_udot4(xc[c].x, xc[c].x, n2, false);
        n2 = __builtin_amdgcn_udot4(xc[c].y, xc[c].y, n2, false);
        n2 = __builtin_amdgcn_udot4(xc[c].z, xc[c].z, n2, false);
        n2 = __builtin_amdgcn_udot4(xc[c].w, xc[c].w, n2, false);
      }
      ax = (float)n2;
    } else if (act) {
      const uint4 h = r[0];
      sx = __uint_as_float(h.x);
      ax = __uint_as_float(h.z);
    }
  }
  Nearest3 nb;
  for (uint32_t k0 = 0; k0 < K; k0 += 64) {
    const uint32_t np = min(64u, K - k0);
    __syncthreads();
    if (threadIdx.x < np) {
      const uint4* r = rows + (size_t)pivots[k0 + threadIdx.x] * stride16;
      uint32_t n2 = 0;
#pragma unroll
      for (uint32_t c = 0; c < NC; ++c) {
        const uint4 w = OFF + c < have ? r[OFF + c] : make_uint4(0u, 0u, 0u, 0u);
        pc[threadIdx.x][c] = w;
        if constexpr (U8) {
          n2 = __builtin_amdgcn_udot4(w.x, w.x, n2, false);
          n2 = __builtin_amdgcn_udot4(w.y, w.y, n2, false);
          n2 = __builtin_amdgcn_udot4(w.z, w.z, n2, false);
          n2 = __builtin_amdgcn_udot4(w.w, w.w, n2, false);
        }
      }
      if constexpr (U8) {
        pn[threadIdx.x] = (float)n2;
        psc[threadIdx.x] = 1.0f;
      } else {
        const uint4 h = r[0];
        pn[threadIdx.x] = __uint_as_float(h.z);
        psc[threadIdx.x] = __uint_as_float(h.x);
      }
    }
    __syncthreads();
    for (uint32_t p = 0; p < np; ++p) {
      float d;
      if constexpr (U8) {
        uint32_t dot = 0;
#pragma unroll
        for (uint32_t c = 0; c < NC; ++c) {
          const uint4 w = pc[p][c];
          dot = __builtin_amdgcn_udot4(xc[c].x, w.x, dot, false);
          dot = __builtin_amdgcn_udot4(xc[c].y, w.y, dot, false);
          dot = __builtin_amdgcn_udot4(xc[c].z, w.z, dot, false);
          dot = __builtin_amdgcn_udot4(xc[c].w, w.w, dot, false);
        }
        d = ax + pn[p] - 2.0f * (float)dot;
      } else {
        int dot = 0;
#pragma unroll
        for (uint32_t c = 0; c < NC; ++c) {
          const uint4 w = pc[p][c];
          dot = __builtin_amdgcn_sdot4((int)xc[c].x, (int)w.x, dot, false);
          dot = __builtin_amdgcn_sdot4((int)xc[c].y, (int)w.y, dot, false);
          dot = __builtin_amdgcn_sdot4((int)xc[c].z, (int)w.z, dot, false);
          dot = __builtin_amdgcn_sdot4((int)xc[c].w, (int)w.w, dot, false);
        }
        d = ax + pn[p] - 2.0f * sx * psc[p] * (float)dot;
      }
      nb.add(d, k0 + p);
    }
  }
  if (act) {
    cell[v] = cell_key(nb.k1, nb.k2, nb.k3, K, levels);
    vid[v] = v;
  }
}

// k_cells_q on the matrix cores, for code rows (U8 = false) and uint8 rows of
// one chunk group (128 bytes, U8 = true): one wave per 32 vertices, int8 MFMA
// tiles of 32 pivots (rows) x 32 vertices (columns) over the 128 bytes (code
// chunks 1-7, or the uint8 bytes shifted by -128). Lane l holds, for vertex
// l % 32, pivots 8 (v >> 2) + (v & 3) + 4 (l >> 5) of each tile (v < 16), in
// ascending order, keeps its own three nearest (first on ties), and the two
// halves of a vertex merge by (distance, pivot) at the end. The distances
// are k_cells_q's exactly (the same fp32 expression on the same integer dot
// for code rows; the integer squared distance for uint8 rows, which
// k_cells_q's fp32 expression also yields below 2^24), so the cells are too.
template <bool U8>
__global__ __launch_bounds__(256) void k_cells_mfma(const uint4* __restrict__ rows, uint32_t stride16, uint32_t N,
                                                    const uint32_t* __restrict__ pivots, uint32_t K,
                                                    uint32_t levels, uint32_t* __restrict__ cell,
                                                    uint32_t* __restrict__ vid) {
  __shared__ int pn_i[4][32];    // uint8 rows: |pivot'|^2
  __shared__ float pn_f[4][32];  // code rows: a and s of the pivot
  __shared__ float ps_f[4][32];
  const uint32_t w = wave_index(), lane = lane_id(), jl = lane & 31u, half = lane >> 5;
  const uint32_t v0 = (blockIdx.x * 4u + w) * 32u;
  if (v0 >= N) return;  // the whole wave; no block-wide barrier follows
  const uint32_t v = v0 + jl;
  const bool act = v < N;
  // 16 bytes of row `id` for K-step s: chunk 2 s + half of the uint8 row, or
  // chunk 1 + 2 s + half of the code row (chunk 8 would be past the row: 0)
  auto frag = [&](uint32_t id, bool ok, uint32_t step) -> v4i_t {
    const uint32_t c = (U8 ? 0u : 1u) + 2u * step + half;
    if (!ok || c >= 8u) return v4i_t{0, 0, 0, 0};
    const uint4 q = rows[(size_t)id * stride16 + c];
    if constexpr (U8)
      return v4i_t{(int)(q.x ^ 0x80808080u), (int)(q.y ^ 0x80808080u), (int)(q.z ^ 0x80808080u),
                   (int)(q.w ^ 0x80808080u)};
    else
      return v4i_t{(int)q.x, (int)q.y, (int)q.z, (int)q.w};
  };
  v4i_t B[4];
#pragma unroll
  for (uint32_t st = 0; st < 4; ++st) B[st] = frag(v, act, st);
  int xn = 0;
  float xa = 0.0f, xs = 1.0f;
  if constexpr (U8) {
    int part = 0;
#pragma unroll
    for (uint32_t st = 0; st < 4; ++st) part = i8_sq4(B[st], part);
    xn = part + __shfl_xor(part, 32);
  } else if (act) {
    const uint4 h = rows[(size_t)v * stride16];
    xs = __uint_as_float(h.x);
    xa = __uint_as_float(h.z);
  }
  Nearest3 nb;
  for (uint32_t t0 = 0; t0 < K; t0 += 32) {
    const uint32_t pi = t0 + jl;
    const bool pok = pi < K;
    const uint32_t pid = pok ? pivots[pi] : 0u;
    v4i_t A[4];
#pragma unroll
    for (uint32_t st = 0; st < 4; ++st) A[st] = frag(pid, pok, st);
    wave_sync();  // the previous tile's reads of the pivot terms are done
    if constexpr (U8) {
      int part = 0;
#pragma unroll
      for (uint32_t st = 0; st < 4; ++st) part = i8_sq4(A[st], part);
      part += __shfl_xor(part, 32);
      if (lane < 32u) pn_i[w][jl] = part;
    } else {
      if (lane < 32u && pok) {
        const uint4 h = rows[(size_t)pid * stride16];
        pn_f[w][jl] = __uint_as_float(h.z);
        ps_f[w][jl] = __uint_as_float(h.x);
      }
    }
    v16i_t acc = {};
#pragma unroll
    for (uint32_t st = 0; st < 4; ++st) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[st], B[st], acc, 0, 0, 0);
    wave_sync();
    static_for<0, 16>([&](auto vc) {
      constexpr uint32_t vv = decltype(vc)::value, ir0 = 8u * (vv >> 2) + (vv & 3u);
      const uint32_t ir = ir0 + 4u * half, k = t0 + ir;
      if (k < K) {
        float d;
        if constexpr (U8)
          d = u8_gram_dist(xn, pn_i[w][ir], acc[vv]);
        else
          d = xa + pn_f[w][ir] - 2.0f * xs * ps_f[w][ir] * (float)acc[vv];
        nb.add(d, k);
      }
    });
  }
  // merge the upper half's three into the lower half's, by (distance, pivot)
  const float e1 = __shfl_xor(nb.d1, 32), e2 = __shfl_xor(nb.d2, 32), e3 = __shfl_xor(nb.d3, 32);
  const uint32_t f1 = (uint32_t)__shfl_xor((int)nb.k1, 32), f2 = (uint32_t)__shfl_xor((int)nb.k2, 32),
                 f3 = (uint32_t)__shfl_xor((int)nb.k3, 32);
  if (half == 0u && act) {
    // two sorted lists of three, popped from the front by selects
    float a1 = nb.d1, a2 = nb.d2, a3 = nb.d3, b1 = e1, b2 = e2, b3 = e3;
    uint32_t ka1 = nb.k1, ka2 = nb.k2, ka3 = nb.k3, kb1 = f1, kb2 = f2, kb3 = f3;
    uint32_t out[3];
#pragma unroll
    for (int o = 0; o < 3; ++o) {
      const bool ta = a1 < b1 || (a1 == b1 && ka1 < kb1);
      out[o] = ta ? ka1 : kb1;
      a1 = ta ? a2 : a1;
      ka1 = ta ? ka2 : ka1;
      a2 = ta ? a3 : a2;
      ka2 = ta ? ka3 : ka2;
      b1 = ta ? b1 : b2;
      kb1 = ta ? kb1 : kb2;
      b2 = ta ? b2 : b3;
      kb2 = ta ? kb2 : kb3;
    }
    cell[v] = cell_key(out[0], out[1], out[2], K, levels);
    vid[v] = v;
  }
}

}  // namespace dance
