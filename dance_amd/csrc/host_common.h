// Host-side helpers shared by the build translation units: error macros,
// RAII device buffers, the scan / radix-sort drivers, row upload into the
// padded 16-byte layout and compile-time dispatch over dtype and row width.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <thread>
#include <type_traits>
#include <vector>

#include "prims.h"
#include "wave.h"

namespace dance {

inline double now_sec() {
  return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

inline bool verbose() {
  const char* e = std::getenv("DANCE_VERBOSE");
  return e && e[0] && e[0] != '0';
}


#define DHIP(call)                                                                                  \
  do {                                                                                              \
    hipError_t e_ = (call);                                                                         \
    if (e_ != hipSuccess) {                                                                         \
      std::fprintf(stderr, "[dance_hip] HIP error '%s' at %s:%d\n", hipGetErrorString(e_), __FILE__, \
                   __LINE__);                                                                       \
      return -1;                                                                                    \
    }                                                                                               \
  } while (0)

#define DCHECK(call)            \
  do {                          \
    if ((call) != 0) return -1; \
  } while (0)

inline uint32_t elem_bytes(int dtype) { return dtype == DANCE_F32 ? 4u : dtype == DANCE_F16 ? 2u : 1u; }

// Smallest compiled chunks-per-lane count covering nch chunks.
// Grid of at least `blocks` workgroups of `threads` work-items, rounded up
// to a multiple of `mult` (8 for xcd_block): 1-D while it holds fewer than
// 2^32 work-items, else 2^20 x gy (kernels index with grid_block()).
inline dim3 grid_dims(uint64_t blocks, uint32_t threads, uint32_t mult = 1) {
  blocks = (blocks + mult - 1) / mult * mult;
  if (blocks * threads < (1ull << 32)) return dim3((uint32_t)std::max<uint64_t>(blocks, 1));
  const uint64_t gx = 1ull << 20;
  return dim3((uint32_t)gx, (uint32_t)((blocks + gx - 1) / gx));
}

inline int pick_cpl(uint32_t nch) {
  const uint32_t need = (nch + 7u) / 8u;
  static const int opts[] = {1, 2, 3, 4, 8, 16};
  for (int o : opts)
    if ((uint32_t)o >= need) return o;
  return -1;
}

template <int V>
using IC = std::integral_constant<int, V>;

template <typename Fn>
inline int with_cpl(int cpl, Fn&& fn) {
  switch (cpl) {
    case 1: return fn(IC<1>{});
    case 2: return fn(IC<2>{});
    case 3: return fn(IC<3>{});
    case 4: return fn(IC<4>{});
    case 8: return fn(IC<8>{});
    case 16: return fn(IC<16>{});
  }
  std::fprintf(stderr, "[dance_hip] unsupported vector width\n");
  return -1;
}

template <typename Fn>
inline int with_dt_cpl(int dtype, int cpl, Fn&& fn) {
  switch (dtype) {
    case DANCE_F32: return with_cpl(cpl, [&](auto c) { return fn(IC<DANCE_F32>{}, c); });
    case DANCE_U8: return with_cpl(cpl, [&](auto c) { return fn(IC<DANCE_U8>{}, c); });
    case DANCE_F16: return with_cpl(cpl, [&](auto c) { return fn(IC<DANCE_F16>{}, c); });
  }
  std::fprintf(stderr, "[dance_hip] unsupported dtype %d\n", dtype);
  return -1;
}

// ---------------------------------------------------------------------------
// Device memory: RAII buffers, or slices of a caller's arena.
// ---------------------------------------------------------------------------

// Bump allocator over device memory owned by someone else (the allocation-free
// build's scratch array). While an ArenaScope is alive on a thread, every
// DevBuf::alloc on that thread takes its bytes from the arena instead of
// hipMalloc, and nothing is freed: the arena's contents end with the scope.
struct Arena {
  char* base = nullptr;
  size_t cap = 0;
  size_t used = 0;
};
inline thread_local Arena* tl_arena = nullptr;
struct ArenaScope {
  Arena* prev;
  explicit ArenaScope(Arena* a) : prev(tl_arena) { tl_arena = a; }
  ~ArenaScope() { tl_arena = prev; }
  ArenaScope(const ArenaScope&) = delete;
  ArenaScope& operator=(const ArenaScope&) = delete;
};

struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  bool borrowed = false;  // a slice of an arena (never freed here)
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() {
    if (p && !borrowed) (void)hipFree(p);
  }
  int alloc(size_t b) {
    if (p) {
      if (!borrowed) (void)hipFree(p);
      p = nullptr;
    }
    borrowed = false;
    bytes = b;
    if (b == 0) return 0;
    if (Arena* a = tl_arena) {
      const size_t off = (a->used + 255u) & ~(size_t)255u;
      if (off > a->cap || b > a->cap - off) {
        std::fprintf(stderr, "[dance_hip] scratch arena exhausted: %zu bytes requested, %zu of %zu in use\n", b,
                     a->used, a->cap);
        return -1;
      }
      p = a->base + off;
      a->used = off + b;
      borrowed = true;
      return 0;
    }
    hipError_t e = hipMalloc(&p, b);
    if (e != hipSuccess) {
      std::fprintf(stderr, "[dance_hip] hipMalloc(%zu) failed: %s\n", b, hipGetErrorString(e));
      p = nullptr;
      return -1;
    }
    return 0;
  }
  void* release() {
    void* q = p;
    p = nullptr;
    return q;
  }
  template <typename T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

// ---------------------------------------------------------------------------
// Scan / sort drivers.
// ---------------------------------------------------------------------------
struct ScanWorkspace {
  DevBuf buf;
  std::vector<size_t> level_off;
  int prepare(size_t n) {
    level_off.clear();
    size_t total = 0, m = n;
    while (true) {
      const size_t tiles = (m + kScanTile - 1) / kScanTile;
      level_off.push_back(total);
      total += tiles;
      if (tiles <= 1) break;
      m = tiles;
    }
    if (buf.bytes >= total * 4) return 0;
    return buf.alloc(std::max<size_t>(total * 4, 256));
  }
};

inline int scan_exclusive_level(uint32_t* d, size_t n, ScanWorkspace& ws, size_t level, hipStream_t s) {
  if (n == 0) return 0;
  const size_t tiles = (n + kScanTile - 1) / kScanTile;
  uint32_t* partial = ws.buf.as<uint32_t>() + ws.level_off[level];
  hipLaunchKernelGGL(k_scan_tile, dim3((uint32_t)tiles), dim3(kScanThreads), 0, s, d, n, partial);
  DHIP(hipGetLastError());
  if (tiles > 1) {
    DCHECK(scan_exclusive_level(partial, tiles, ws, level + 1, s));
    hipLaunchKernelGGL(k_scan_add, dim3((uint32_t)tiles), dim3(kScanThreads), 0, s, d, n, partial);
    DHIP(hipGetLastError());
  }
  return 0;
}

inline int scan_exclusive(uint32_t* d, size_t n, ScanWorkspace& ws, hipStream_t s) {
  DCHECK(ws.prepare(n));
  return scan_exclusive_level(d, n, ws, 0, s);
}

struct SortWorkspace {
  DevBuf hist;
  ScanWorkspace scan;
};

// Stable sort of (keys, vals) by the low key_bits bits. Returns the index
// (0 or 1) of the buffer pair holding the result.
inline int radix_sort_pairs(uint32_t* keys[2], uint32_t* vals[2], size_t n, uint32_t key_bits, SortWorkspace& ws,
                            hipStream_t s, int* result_index) {
  int cur = 0;
  if (n == 0 || key_bits == 0) {
    *result_index = 0;
    return 0;
  }
  const size_t tiles = (n + kRadixTile - 1) / kRadixTile;
  if (ws.hist.bytes < tiles * 256 * 4) DCHECK(ws.hist.alloc(tiles * 256 * 4));
  for (uint32_t shift = 0; shift < key_bits; shift += 8) {
    hipLaunchKernelGGL(k_radix_hist, dim3((uint32_t)tiles), dim3(kRadixThreads), 0, s, keys[cur], n, shift,
                       (uint32_t)tiles, ws.hist.as<uint32_t>());
    DHIP(hipGetLastError());
    DCHECK(scan_exclusive(ws.hist.as<uint32_t>(), tiles * 256, ws.scan, s));
    hipLaunchKernelGGL(k_radix_scatter, dim3((uint32_t)tiles), dim3(kRadixThreads), 0, s, keys[cur], vals[cur], n,
                       shift, (uint32_t)tiles, ws.hist.as<uint32_t>(), keys[cur ^ 1], vals[cur ^ 1]);
    DHIP(hipGetLastError());
    cur ^= 1;
  }
  *result_index = cur;
  return 0;
}

inline uint32_t bit_length(uint32_t x) {
  uint32_t b = 0;
  while (x) {
    ++b;
    x >>= 1;
  }
  return b;
}

// ---------------------------------------------------------------------------
// Vector upload into the padded row layout.
// ---------------------------------------------------------------------------
struct Rows {
  DevBuf owned;
  RowSet rs{};
  int dtype = DANCE_F32;
  uint32_t N = 0, dim = 0;
  uint32_t vbytes() const { return dim * elem_bytes(dtype); }
};

static __global__ void k_f32_to_f16_rows(const float* __restrict__ src, uint32_t N, uint32_t dim,
                                  _Float16* __restrict__ dst, uint32_t dst_stride_elems) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)N * dim) return;
  const size_t r = i / dim, c = i % dim;
  dst[r * dst_stride_elems + c] = (_Float16)src[i];  // round to nearest even
}

// Copies between pageable host memory and device memory through pinned
// staging buffers. A hipMemcpy from or to pageable memory moves about
// 8 GB/s here (a 2.56 GB graph took 0.31 s); instead up to kCopyThreads host
// threads each own a pinned buffer and a stream and move whole chunks, so
// the DMA of one chunk overlaps the host-side copy of another. Synchronous:
// returns after every byte has arrived. The pinned buffers are allocated on
// first use and kept for the life of the process (kCopyThreads x kCopyChunk
// bytes); copies below two chunks take one plain hipMemcpy.
constexpr size_t kCopyChunk = 32ull << 20;
constexpr unsigned kCopyThreads = 8;

inline int pinned_stage(unsigned k, void** out) {
  static std::mutex mu;
  static void* bufs[kCopyThreads] = {};
  std::lock_guard<std::mutex> lock(mu);
  if (!bufs[k]) DHIP(hipHostMalloc(&bufs[k], kCopyChunk, hipHostMallocPortable));
  *out = bufs[k];
  return 0;
}

inline int copy_pageable(void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
  if (bytes < 2 * kCopyChunk) {
    DHIP(hipMemcpy(dst, src, bytes, kind));
    return 0;
  }
  int dev = 0;
  DHIP(hipGetDevice(&dev));
  const size_t chunks = (bytes + kCopyChunk - 1) / kCopyChunk;
  const unsigned T = (unsigned)std::min<size_t>(kCopyThreads, chunks);
  static std::mutex copy_mu;  // concurrent copies would share the staging buffers
  std::lock_guard<std::mutex> lock(copy_mu);
  std::atomic<size_t> next{0};
  std::atomic<int> failed{0};
  auto worker = [&](unsigned t) {
    void* stage = nullptr;
    hipStream_t st = nullptr;
    if (hipSetDevice(dev) != hipSuccess || pinned_stage(t, &stage) != 0 || hipStreamCreate(&st) != hipSuccess) {
      failed = 1;
      return;
    }
    for (size_t c = next++; c < chunks && !failed; c = next++) {
      const size_t off = c * kCopyChunk, len = std::min(kCopyChunk, bytes - off);
      if (kind == hipMemcpyDeviceToHost) {
        if (hipMemcpyAsync(stage, static_cast<const char*>(src) + off, len, kind, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess) {
          failed = 1;
          break;
        }
        std::memcpy(static_cast<char*>(dst) + off, stage, len);
      } else {
        std::memcpy(stage, static_cast<const char*>(src) + off, len);
        if (hipMemcpyAsync(static_cast<char*>(dst) + off, stage, len, kind, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess) {
          failed = 1;
          break;
        }
      }
    }
    if (hipStreamDestroy(st) != hipSuccess) failed = 1;
  };
  std::vector<std::thread> pool;
  for (unsigned t = 1; t < T; ++t) pool.emplace_back(worker, t);
  worker(0);
  for (auto& th : pool) th.join();
  if (failed) {
    std::fprintf(stderr, "[dance_hip] staged %s copy of %zu bytes failed\n",
                 kind == hipMemcpyDeviceToHost ? "device-to-host" : "host-to-device", bytes);
    return -1;
  }
  return 0;
}

inline int setup_rows(Rows& out, const void* src, bool src_on_device, int src_dtype, int store_dtype, uint32_t N,
                      uint32_t dim, hipStream_t s) {
  out.dtype = store_dtype;
  out.N = N;
  out.dim = dim;
  const size_t row_bytes = (size_t)dim * elem_bytes(store_dtype);
  // Rows are padded with zeros to the compiled chunk group (8 lanes x CPL
  // chunks of 16 bytes), so every chunk slot of a row holds data and row
  // loads need no per-chunk bounds test; zeros add nothing to a distance.
  const uint32_t data_chunks = (uint32_t)((row_bytes + 15) / 16);
  const int cpl = pick_cpl(data_chunks);
  const uint32_t nch = cpl > 0 ? 8u * (uint32_t)cpl : data_chunks;
  const size_t stride = (size_t)nch * 16;
  out.rs.stride16 = nch;
  out.rs.nch = nch;
  out.rs.tail16 = (store_dtype == DANCE_F16 && (dim & 1u)) ? (int32_t)((dim - 1u) / 2u) : -1;
  const size_t src_row_bytes = (size_t)dim * elem_bytes(src_dtype);
  if (src_dtype == store_dtype && src_on_device && stride == row_bytes &&
      (reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
    out.rs.rows = static_cast<const uint4*>(src);
    return 0;
  }
  DCHECK(out.owned.alloc(stride * N));
  if (src_dtype == store_dtype) {
    if (stride == row_bytes) {
      if (src_on_device)
        DHIP(hipMemcpyAsync(out.owned.p, src, row_bytes * N, hipMemcpyDeviceToDevice, s));
      else
        DCHECK(copy_pageable(out.owned.p, src, row_bytes * N, hipMemcpyHostToDevice));
    } else {
      // Pitched copies from pageable host memory go row by row (6 s for
      // 250 MB measured): upload contiguously, then pad on the device.
      DevBuf tmp;
      const void* dsrc = src;
      if (!src_on_device) {
        DCHECK(tmp.alloc(row_bytes * N));
        DCHECK(copy_pageable(tmp.p, src, row_bytes * N, hipMemcpyHostToDevice));
        dsrc = tmp.p;
      }
      DHIP(hipMemsetAsync(out.owned.p, 0, stride * N, s));
      DHIP(hipMemcpy2DAsync(out.owned.p, stride, dsrc, row_bytes, row_bytes, N, hipMemcpyDeviceToDevice, s));
      DHIP(hipStreamSynchronize(s));  // tmp is freed on return
    }
  } else {
    // fp32 input stored as fp16 (FAST_SMALL): upload, convert on device.
    DevBuf tmp;
    const void* fsrc = src;
    if (!src_on_device) {
      DCHECK(tmp.alloc(src_row_bytes * N));
      DCHECK(copy_pageable(tmp.p, src, src_row_bytes * N, hipMemcpyHostToDevice));
      fsrc = tmp.p;
    }
    DHIP(hipMemsetAsync(out.owned.p, 0, stride * N, s));
    const size_t total = (size_t)N * dim;
    hipLaunchKernelGGL(k_f32_to_f16_rows, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s,
                       static_cast<const float*>(fsrc), N, dim, out.owned.as<_Float16>(), (uint32_t)(stride / 2));
    DHIP(hipGetLastError());
    DHIP(hipStreamSynchronize(s));
  }
  out.rs.rows = out.owned.as<const uint4>();
  return 0;
}


}  // namespace dance
