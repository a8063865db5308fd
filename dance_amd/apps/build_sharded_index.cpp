// build_sharded_index: the GPU shard path of DiskANN's
// build_merged_vamana_index (reference:
// integrations/dance-diskann-78256bba.patch:1209-1560, with
// DISKANN_USE_GPU_SHARD_BUILD=1) up to the merged Vamana graph that DiskANN
// then lays out on disk.
//
//   --data_type uint8|float --data_path <bin> --index_path_prefix P
//   [--max_degree|-R 64] [--Lbuild|-L 100] [--num_shards K | --budget_gb G]
//   [--sampling_rate p] [--k_base 2] [--seed 42] [--kmeans_reps 10]
//
// Steps:
//   1. partition (DiskANN partition_with_ram_budget, upstream partition.cpp):
//      a Bernoulli(p) sample of the rows (p defaults to 256000 / N, at most
//      1), k-means++ seeding and at most kmeans_reps Lloyd iterations on it
//      (stopping when the residual improves by less than 1e-5 of itself;
//      an empty cluster keeps its center). The assignment step runs on the
//      GPU (dance_partition_assign); centers are fp64 means of their points,
//      summed in point order. Without --num_shards the number of parts starts
//      at 3 and grows by 2 until the largest shard, estimated from the sample
//      with k_base assignments, fits G GB of device memory for its build.
//      Finally every row goes to its k_base nearest centers.
//   2. per shard (patch:2811-2984): the shard's rows in ascending id order,
//      built with the v8 builder gpu_vamana_build[_float] (or vnew2's
//      gpu_vamana_vnew2_build[_float] when DISKANN_GPU_VAMANA_VERSION=vnew2 or
//      DISKANN_USE_GPU_VAMANA_VNEW2 is set and not 0, patch:2576-2584), with
//      that builder's medoid (patch:2947), at shard_R = 2R/3
//      (DISKANN_GPU_SHARD_R caps it at R), C = max(2 shard_R, shard_R + 32)
//      (DISKANN_GPU_C), STEPS = min(L, 20) (DISKANN_GPU_STEPS), C at least
//      shard_R and STEPS at most L (patch:3271-3335); saved with the builder's
//      medoid, width shard_R and rows cut to that width (patch:419-480).
//   3. diskann::merge_shards_gpu into P and P_medoids.bin.
// Files: P_centroids.bin (K x dim fp32), P_tempFiles_subshard-<p>_ids_uint32.bin,
// P_tempFiles_subshard-<p>_mem.index, P, P_medoids.bin.
// The seeds make the run deterministic; DiskANN seeds from std::random_device.
// Exit status: 0 ok, 255 (-1) on any error.

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <random>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

#include "dance_hip.h"
#include "gpu_merge.h"
#include "gpu_vamana_builder.h"

namespace {

double now_sec() {
  return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

struct Options {
  std::string data_type, data_path, prefix;
  uint32_t R = 64, L = 100, num_shards = 0, k_base = 2, kmeans_reps = 10;
  double budget_gb = 0.0, sampling_rate = 0.0;
  uint64_t seed = 42;
};

uint32_t to_u32(const std::string& v, const std::string& k) {
  char* end = nullptr;
  const unsigned long long x = std::strtoull(v.c_str(), &end, 10);
  if (v.empty() || *end || x > 0xFFFFFFFFull) throw std::runtime_error("bad value for " + k + ": " + v);
  return (uint32_t)x;
}

double to_f64(const std::string& v, const std::string& k) {
  char* end = nullptr;
  const double x = std::strtod(v.c_str(), &end);
  if (v.empty() || *end || !std::isfinite(x)) throw std::runtime_error("bad value for " + k + ": " + v);
  return x;
}

Options parse(int argc, char** argv) {
  Options o;
  for (int i = 1; i < argc; ++i) {
    const std::string k = argv[i];
    if (i + 1 >= argc) throw std::runtime_error("missing value for " + k);
    const std::string v = argv[++i];
    if (k == "--data_type") o.data_type = v;
    else if (k == "--data_path") o.data_path = v;
    else if (k == "--index_path_prefix") o.prefix = v;
    else if (k == "--max_degree" || k == "-R") o.R = to_u32(v, k);
    else if (k == "--Lbuild" || k == "-L") o.L = to_u32(v, k);
    else if (k == "--num_shards") o.num_shards = to_u32(v, k);
    else if (k == "--budget_gb") o.budget_gb = to_f64(v, k);
    else if (k == "--sampling_rate") o.sampling_rate = to_f64(v, k);
    else if (k == "--k_base") o.k_base = to_u32(v, k);
    else if (k == "--seed") o.seed = to_u32(v, k);
    else if (k == "--kmeans_reps") o.kmeans_reps = to_u32(v, k);
    else throw std::runtime_error("unknown argument " + k);
  }
  if (o.data_type != "uint8" && o.data_type != "float")
    throw std::runtime_error("--data_type must be uint8 or float");
  if (o.data_path.empty() || o.prefix.empty()) throw std::runtime_error("--data_path and --index_path_prefix are required");
  if (o.R < 2 || o.L == 0) throw std::runtime_error("--max_degree must be at least 2 and --Lbuild positive");
  if (o.num_shards == 0 && !(o.budget_gb > 0.0)) throw std::runtime_error("give --num_shards or a positive --budget_gb");
  if (o.k_base == 0 || o.k_base > 8) throw std::runtime_error("--k_base must be 1..8");
  if (o.num_shards != 0 && o.num_shards < o.k_base) throw std::runtime_error("--num_shards must be at least --k_base");
  if (o.sampling_rate < 0.0 || o.sampling_rate > 1.0) throw std::runtime_error("--sampling_rate must be in [0, 1]");
  return o;
}

template <typename T>
std::vector<T> read_matrix(const std::string& path, uint32_t& n, uint32_t& dim) {
  std::ifstream in(path, std::ios::binary);
  if (!in) throw std::runtime_error("cannot open " + path);
  uint32_t hdr[2];
  in.read(reinterpret_cast<char*>(hdr), 8);
  if (!in) throw std::runtime_error("short header in " + path);
  n = hdr[0];
  dim = hdr[1];
  in.seekg(0, std::ios::end);
  const uint64_t want = 8 + (uint64_t)n * dim * sizeof(T), have = (uint64_t)in.tellg();
  if (have != want)
    throw std::runtime_error(path + ": file size " + std::to_string(have) + " != expected " + std::to_string(want));
  if (n == 0 || dim == 0) throw std::runtime_error(path + " holds no points");
  in.seekg(8);
  std::vector<T> x((size_t)n * dim);
  in.read(reinterpret_cast<char*>(x.data()), (std::streamsize)(x.size() * sizeof(T)));
  return x;
}

void write_file(const std::string& path, const void* a, size_t an, const void* b, size_t bn) {
  std::ofstream f(path, std::ios::binary);
  if (!f) throw std::runtime_error("cannot write " + path);
  f.write(static_cast<const char*>(a), (std::streamsize)an);
  if (bn) f.write(static_cast<const char*>(b), (std::streamsize)bn);
  if (!f) throw std::runtime_error("write failed: " + path);
}

// DiskANN .bin with a uint32 header (rows, cols).
template <typename T>
void write_bin(const std::string& path, const T* data, uint32_t rows, uint32_t cols) {
  const uint32_t hdr[2] = {rows, cols};
  write_file(path, hdr, 8, data, (size_t)rows * cols * sizeof(T));
}

uint32_t env_u32(const char* name, uint32_t fallback) {
  const char* e = std::getenv(name);
  return e ? (uint32_t)std::atoi(e) : fallback;
}

// Shard builder choice (patch:2576-2584): v8 unless DISKANN_GPU_VAMANA_VERSION
// is "vnew2" or DISKANN_USE_GPU_VAMANA_VNEW2 is set, non-empty and not "0".
bool use_vnew2() {
  const char* v = std::getenv("DISKANN_GPU_VAMANA_VERSION");
  if (v != nullptr && std::strcmp(v, "vnew2") == 0) return true;
  const char* e = std::getenv("DISKANN_USE_GPU_VAMANA_VNEW2");
  return e != nullptr && e[0] != '\0' && std::strcmp(e, "0") != 0;
}

template <typename T>
double sq_dist(const T* x, const double* c, uint32_t dim) {
  double acc = 0.0;
  for (uint32_t j = 0; j < dim; ++j) {
    const double d = (double)x[j] - c[j];
    acc = std::fma(d, d, acc);
  }
  return acc;
}

template <typename T>
int dtype_code() {
  return std::is_same<T, float>::value ? DANCE_DTYPE_F32 : DANCE_DTYPE_U8;
}

template <typename T>
void assign(const T* x, uint64_t n, uint32_t dim, const std::vector<double>& centers, uint32_t K, uint32_t k_base,
            std::vector<uint32_t>& out) {
  std::vector<float> cf(centers.begin(), centers.end());
  out.assign((size_t)n * k_base, 0);
  if (dance_partition_assign(x, dtype_code<T>(), n, dim, cf.data(), K, k_base, out.data()) != 0)
    throw std::runtime_error("dance_partition_assign failed");
}

// DiskANN kmeans::kmeanspp_selecting_pivots (upstream): the first pivot
// uniform, each next one drawn with probability proportional to the squared
// distance to the nearest pivot so far (redrawn if already picked, unless
// every distance is 0).
template <typename T>
std::vector<double> kmeanspp(const std::vector<T>& s, uint64_t ns, uint32_t dim, uint32_t K, std::mt19937_64& rng) {
  std::vector<double> piv((size_t)K * dim);
  std::uniform_real_distribution<double> uni(0.0, 1.0);
  std::uniform_int_distribution<uint64_t> first(0, ns - 1);
  std::vector<uint64_t> picked{first(rng)};
  for (uint32_t j = 0; j < dim; ++j) piv[j] = (double)s[picked[0] * dim + j];
  std::vector<double> dist(ns);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)ns; ++i) dist[i] = sq_dist(&s[(size_t)i * dim], piv.data(), dim);
  while (picked.size() < K) {
    double sum = 0.0;
    for (uint64_t i = 0; i < ns; ++i) sum += dist[i];
    const bool all_zero = sum == 0.0;
    const double dart = uni(rng) * sum;
    double prefix = 0.0;
    uint64_t pick = ns - 1;
    for (uint64_t i = 0; i < ns; ++i) {
      if (dart >= prefix && dart < prefix + dist[i]) {
        pick = i;
        break;
      }
      prefix += dist[i];
    }
    if (all_zero) pick = first(rng);
    if (!all_zero && std::find(picked.begin(), picked.end(), pick) != picked.end()) continue;
    double* c = &piv[picked.size() * dim];
    for (uint32_t j = 0; j < dim; ++j) c[j] = (double)s[pick * dim + j];
    picked.push_back(pick);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)ns; ++i) dist[i] = std::min(dist[i], sq_dist(&s[(size_t)i * dim], c, dim));
  }
  return piv;
}

// DiskANN kmeans::run_lloyds (upstream) with the assignment on the GPU.
// Centers are rounded to fp32 for the assignment, as DiskANN keeps them.
template <typename T>
void lloyds(const std::vector<T>& s, uint64_t ns, uint32_t dim, uint32_t K, uint32_t reps, std::vector<double>& c) {
  std::vector<uint32_t> a;
  double old_res = 0.0;
  for (uint32_t rep = 0; rep < reps; ++rep) {
    for (double& v : c) v = (double)(float)v;
    assign(s.data(), ns, dim, c, K, 1, a);
    std::vector<double> sum((size_t)K * dim, 0.0);
    std::vector<uint64_t> cnt(K, 0);
    double res = 0.0;
    for (uint64_t i = 0; i < ns; ++i) {
      const uint32_t k = a[i];
      if (k >= K) continue;
      ++cnt[k];
      const T* x = &s[i * dim];
      res += sq_dist(x, &c[(size_t)k * dim], dim);
      for (uint32_t j = 0; j < dim; ++j) sum[(size_t)k * dim + j] += (double)x[j];
    }
    for (uint32_t k = 0; k < K; ++k)
      if (cnt[k])
        for (uint32_t j = 0; j < dim; ++j) c[(size_t)k * dim + j] = sum[(size_t)k * dim + j] / (double)cnt[k];
    std::cout << "[partition] lloyd rep " << rep << " residual " << res << std::endl;
    if (rep > 0 && (res == 0.0 || (old_res - res) / res < 1e-5)) break;
    old_res = res;
  }
  for (double& v : c) v = (double)(float)v;
}

// Device bytes of one shard's build (rows, graph, candidate rows with
// distances, radix double buffers, degrees and flags), per point.
double shard_device_bytes(uint64_t npts, uint32_t dim, uint32_t elem, uint32_t R, uint32_t C) {
  const double row = (double)((dim * elem + 15) / 16 * 16);
  return (double)npts * (row + 4.0 * R + 8.0 * C + 16.0 * R + 32.0);
}

template <typename T>
int run(const Options& o) {
  const double t0 = now_sec();
  uint32_t n = 0, dim = 0;
  const std::vector<T> x = read_matrix<T>(o.data_path, n, dim);
  const uint32_t elem = sizeof(T);

  // shard build parameters (patch:3271-3335)
  uint32_t shard_R = 2 * o.R / 3;
  if (env_u32("DISKANN_GPU_SHARD_R", 0) > 0) shard_R = std::min(env_u32("DISKANN_GPU_SHARD_R", 0), o.R);
  uint32_t C = env_u32("DISKANN_GPU_C", 0);
  if (C == 0) C = std::max(2 * shard_R, shard_R + 32);
  uint32_t steps = env_u32("DISKANN_GPU_STEPS", 0);
  if (steps == 0) steps = std::min<uint32_t>(o.L, 20);
  C = std::max(C, shard_R);
  steps = std::min(steps, o.L);
  std::cout << "[GPU shard] shard_R=" << shard_R << " L=" << o.L << " C=" << C << " STEPS=" << steps << std::endl;

  // 1. partition
  std::mt19937_64 rng(o.seed);
  const double p = o.sampling_rate > 0.0 ? o.sampling_rate : std::min(1.0, 256000.0 / n);
  std::bernoulli_distribution take(p);
  std::vector<T> sample;
  uint64_t ns = 0;
  for (uint32_t i = 0; i < n; ++i)
    if (take(rng)) {
      sample.insert(sample.end(), x.begin() + (size_t)i * dim, x.begin() + (size_t)(i + 1) * dim);
      ++ns;
    }
  uint32_t K = o.num_shards ? o.num_shards : 3;
  if (ns < std::max<uint32_t>(K, o.k_base))
    throw std::runtime_error("the sample holds " + std::to_string(ns) + " points, fewer than the shards; raise --sampling_rate");
  std::vector<double> centers;
  const double t_part = now_sec();
  while (true) {
    if (K > ns) throw std::runtime_error("no partition fits the budget with " + std::to_string(ns) + " sampled points");
    centers = kmeanspp(sample, ns, dim, K, rng);
    lloyds(sample, ns, dim, K, o.kmeans_reps, centers);
    if (o.num_shards) break;
    std::vector<uint32_t> a;
    assign(sample.data(), ns, dim, centers, K, std::min(o.k_base, K), a);
    std::vector<uint64_t> sizes(K, 0);
    for (uint32_t v : a)
      if (v < K) ++sizes[v];
    double worst = 0.0;
    for (uint64_t sz : sizes) worst = std::max(worst, shard_device_bytes((uint64_t)(sz / p), dim, elem, shard_R, C));
    std::cout << "[partition] parts=" << K << " largest shard estimate " << worst / (1u << 30) << " GB, budget "
              << o.budget_gb << " GB" << std::endl;
    if (worst <= o.budget_gb * (double)(1u << 30)) break;
    K += 2;
  }
  if (o.k_base > K) throw std::runtime_error("--k_base exceeds the number of shards");
  std::vector<float> cf(centers.begin(), centers.end());
  write_bin(o.prefix + "_centroids.bin", cf.data(), K, dim);
  std::vector<uint32_t> a;
  assign(x.data(), n, dim, centers, K, o.k_base, a);
  std::vector<std::vector<uint32_t>> shards(K);
  for (uint32_t i = 0; i < n; ++i)
    for (uint32_t r = 0; r < o.k_base; ++r) {
      const uint32_t k = a[(size_t)i * o.k_base + r];
      if (k < K) shards[k].push_back(i);
    }
  const double t_built_part = now_sec();
  std::cout << "[partition] " << K << " shards, sample " << ns << " points, " << (t_built_part - t_part) << " s"
            << std::endl;

  // 2. per-shard GPU builds
  const bool vnew2 = use_vnew2();
  const std::string tmp = o.prefix + "_tempFiles_subshard-";
  for (uint32_t k = 0; k < K; ++k) {
    const std::vector<uint32_t>& ids = shards[k];
    write_bin(tmp + std::to_string(k) + "_ids_uint32.bin", ids.data(), (uint32_t)ids.size(), 1);
    const uint32_t m = (uint32_t)ids.size();
    std::vector<uint32_t> graph((size_t)std::max(m, 1u) * shard_R, 0xFFFFFFFFu), degree(std::max(m, 1u), 0);
    uint32_t medoid = 0;
    if (m > 0) {
      std::vector<T> rows((size_t)m * dim);
      for (uint32_t i = 0; i < m; ++i)
        std::memcpy(&rows[(size_t)i * dim], &x[(size_t)ids[i] * dim], (size_t)dim * sizeof(T));
      std::cout << "[GPU shard] build start: shard=" << k << " type=" << (std::is_same<T, float>::value ? "float" : "uint8")
                << " builder=" << (vnew2 ? "vnew2" : "v8") << " npts=" << m << " dim=" << dim << " R=" << shard_R
                << " L=" << o.L << " C=" << C << " STEPS=" << steps << std::endl;
      const double tb = now_sec();
      int rc;
      if (std::is_same<T, float>::value) {
        const float* r = reinterpret_cast<const float*>(rows.data());
        rc = vnew2 ? gpu_vamana_vnew2_build_float(r, m, dim, shard_R, o.L, C, steps, graph.data(), degree.data())
                   : gpu_vamana_build_float(r, m, dim, shard_R, o.L, C, steps, graph.data(), degree.data());
      } else {
        const uint8_t* r = reinterpret_cast<const uint8_t*>(rows.data());
        rc = vnew2 ? gpu_vamana_vnew2_build(r, m, dim, shard_R, o.L, C, steps, graph.data(), degree.data())
                   : gpu_vamana_build(r, m, dim, shard_R, o.L, C, steps, graph.data(), degree.data());
      }
      if (rc != 0) throw std::runtime_error("gpu_vamana_build failed for shard " + std::to_string(k));
      medoid = vnew2 ? gpu_vamana_vnew2_get_last_medoid() : gpu_vamana_get_last_medoid();
      if (medoid >= m) medoid = 0;
      std::cout << "[gpu_shard_timing] shard=" << k << " npts=" << m << " gpu_vamana_call_seconds=" << (now_sec() - tb)
                << std::endl;
    }
    // save_gpu_vamana_graph_for_merge (patch:419-480)
    std::string body;
    uint64_t size = 24;
    for (uint32_t i = 0; i < m; ++i) size += 4 + 4ull * std::min(degree[i], shard_R);
    body.reserve(size);
    const uint64_t frozen = 0;
    body.append(reinterpret_cast<const char*>(&size), 8);
    body.append(reinterpret_cast<const char*>(&shard_R), 4);
    body.append(reinterpret_cast<const char*>(&medoid), 4);
    body.append(reinterpret_cast<const char*>(&frozen), 8);
    for (uint32_t i = 0; i < m; ++i) {
      const uint32_t d = std::min(degree[i], shard_R);
      body.append(reinterpret_cast<const char*>(&d), 4);
      body.append(reinterpret_cast<const char*>(&graph[(size_t)i * shard_R]), 4ull * d);
    }
    write_file(tmp + std::to_string(k) + "_mem.index", body.data(), body.size(), nullptr, 0);
    std::cout << "[GPU shard] shard " << k << " npts=" << m << " medoid=" << medoid << std::endl;
  }
  const double t_shards = now_sec();

  // 3. merge
  const int rc = diskann::merge_shards_gpu(tmp, "_mem.index", tmp, "_ids_uint32.bin", K, o.R, o.prefix,
                                           o.prefix + "_medoids.bin");
  if (rc != 0) throw std::runtime_error("merge_shards_gpu failed with code " + std::to_string(rc));
  const double t_end = now_sec();
  std::cout << "[build_sharded_index] N=" << n << " dim=" << dim << " shards=" << K << " partition_s="
            << (t_built_part - t0) << " shard_builds_s=" << (t_shards - t_built_part) << " merge_s="
            << (t_end - t_shards) << " total_s=" << (t_end - t0) << std::endl;
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    const Options o = parse(argc, argv);
    return o.data_type == "float" ? run<float>(o) : run<uint8_t>(o);
  } catch (const std::exception& e) {
    std::cerr << "build_sharded_index: " << e.what() << std::endl;
    return -1;
  }
}
