// build_memory_index --gpu_filtered: builds a label-filtered DiskANN in-memory
// index with the GPU-FilteredVamana builder (libdance_hip.so).
//
// Drop-in for the DANCE-patched DiskANN app (reference:
// integrations/dance-diskann-78256bba.patch:120-160 for the option, and
// :20243-20530 for the GPU branch of Index::build_filtered_index). Only the
// --gpu_filtered path is provided; without it the app exits with an error,
// because DiskANN's CPU build is not part of this library.
//
//   --data_type uint8|float --dist_fn l2 --data_path <bin>
//   --index_path_prefix PATH --label_file <txt> [--universal_label NAME]
//   [--max_degree|-R 64] [--Lbuild|-L 100] [--FilteredLbuild 0] [--alpha 1.2]
//   [--num_threads|-T N] [--label_type uint] [--build_PQ_bytes 0] --gpu_filtered
//
// Steps:
//   1. labels: one row per point, comma-separated names; names are numbered
//      1, 2, ... in order of first appearance, the universal label is 0
//      (DiskANN convert_labels_string_to_int, upstream); rows become sorted
//      unique id lists (the canonical CSR, patch:20269-20286);
//   2. entry points: global start = the point nearest to the centroid of all
//      points; label starts by Filtered-DiskANN's load-balanced FindMedoid
//      (25 random carriers per label, the least-loaded wins; see
//      balanced_label_starts), or with DANCE_LABEL_STARTS=centroid the carrier
//      nearest to the centroid of the label's carriers (squared L2 in fp64,
//      ties to the lower id);
//   3. gpu_vamana_filtered_build_{uint8,float} with the internal degree
//      R_b = max(max_degree, 64) (or max(max_degree,
//      DISKANN_GPU_FILTERED_INTERNAL_DEGREE)), L = Lbuild, filtered_L =
//      FilteredLbuild or Lbuild, C = 750 (DiskANN's default max occlusion
//      size), STEPS = min(64, L) or DISKANN_GPU_FILTERED_STEPS; when R_b
//      exceeds max_degree the library's publish step prunes the graph to
//      max_degree (DISKANN_GPU_FILTERED_PUBLISH_DEGREE is set to max_degree,
//      and unset otherwise) (patch:20368-20398);
//   4. with DISKANN_GPU_FILTERED_RESELECT_LABEL_STARTS=common_degree, label
//      starts are reselected from the raw graph (patch:20447-20504);
//      install: per row drop invalid / self / repeated ids, an empty row of a
//      multi-point index gets (i + 1) mod N (patch:20506-20521);
//   5. save: <prefix> (graph: u64 file bytes, u32 max degree, u32 start,
//      u64 frozen 0, rows), <prefix>.data, <prefix>_labels.txt,
//      <prefix>_label_formatted.txt, <prefix>_labels_map.txt,
//      <prefix>_labels_to_medoids.txt and, with a universal label,
//      <prefix>_universal_label.txt.
// DISKANN_GPU_FILTERED_GPU_PUBLISH=0 with R_b above max_degree asks for
// DiskANN's CPU prune and reverse repair instead of the publish step
// (patch:20527-20537); that CPU code is not part of this library, so the app
// then exits with an error. Exit status: 0 ok, 255 (-1) on any error.

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <iterator>
#include <limits>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

#include "diskann_io.h"
#include "gpu_vamana_filtered.h"

namespace {

constexpr uint32_t kInvalid = 0xFFFFFFFFu;
constexpr uint32_t kMinInternalDegree = 64;  // patch:20367-20370
constexpr uint32_t kDefaultMaxC = 750;       // DiskANN IndexWriteParameters default

double now_sec() {
  return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

struct Options {
  std::string data_type, dist_fn = "l2", data_path, prefix, label_file, universal_label, label_type = "uint";
  uint32_t R = 64, L = 100, Lf = 0, threads = 0, pq_bytes = 0;
  float alpha = 1.2f;
  bool gpu_filtered = false, use_opq = false;
};

Options parse(int argc, char** argv) {
  Options o;
  dio::ArgTable t;
  auto str = [](std::string* dst) { return [dst](const std::string& v, const std::string&) { *dst = v; }; };
  auto u32 = [](uint32_t* dst) {
    return [dst](const std::string& v, const std::string& k) { *dst = dio::parse_u32(v, k, true); };
  };
  t.flag({"--gpu_filtered"}, &o.gpu_filtered);
  t.flag({"--use_opq"}, &o.use_opq);
  t.value({"--data_type"}, str(&o.data_type));
  t.value({"--dist_fn"}, str(&o.dist_fn));
  t.value({"--data_path"}, str(&o.data_path));
  t.value({"--index_path_prefix"}, str(&o.prefix));
  t.value({"--label_file"}, str(&o.label_file));
  t.value({"--universal_label"}, str(&o.universal_label));
  t.value({"--label_type"}, str(&o.label_type));
  t.value({"--max_degree", "-R"}, u32(&o.R));
  t.value({"--Lbuild", "-L"}, u32(&o.L));
  t.value({"--FilteredLbuild", "-Lf"}, u32(&o.Lf));
  t.value({"--num_threads", "-T"}, u32(&o.threads));
  t.value({"--build_PQ_bytes"}, u32(&o.pq_bytes));
  t.value({"--alpha"}, [&](const std::string& v, const std::string& k) { o.alpha = dio::parse_positive_float(v, k); });
  t.parse(argc, argv);
  if (o.data_type.empty() || o.data_path.empty() || o.prefix.empty())
    throw std::runtime_error("--data_type, --data_path and --index_path_prefix are required");
  if (!o.gpu_filtered)
    throw std::runtime_error("only the --gpu_filtered build is provided (DiskANN's CPU build is not part of this library)");
  if (o.data_type != "float" && o.data_type != "uint8")
    throw std::runtime_error("--gpu_filtered supports only float and uint8 data");
  if (o.label_file.empty()) throw std::runtime_error("--gpu_filtered requires --label_file");
  if (o.dist_fn != "l2") throw std::runtime_error("--gpu_filtered builds with --dist_fn l2 only");
  if (o.label_type != "uint") throw std::runtime_error("--gpu_filtered supports --label_type uint only");
  if (o.pq_bytes != 0 || o.use_opq)
    throw std::runtime_error("[GPU filtered] first version supports only static memory indices without tags or PQ build");
  if (o.R == 0 || o.L == 0) throw std::runtime_error("--max_degree and --Lbuild must be positive");
  return o;
}

// Label rows with ids 1.. by first appearance (the universal label, when
// named, is 0), tokens in file order with repeats, plus the canonical CSR
// (sorted unique ids per row).
struct Labels {
  dio::LabelRows rows;
  std::vector<uint32_t> offsets, ids;
  uint32_t universal = kInvalid;
  uint32_t count() const { return (uint32_t)rows.names.size(); }
};

Labels read_labels(const Options& o, uint32_t n) {
  Labels lb;
  lb.rows = dio::read_labels(o.label_file, {o.universal_label, "", false, false});
  lb.universal = lb.rows.universal;
  if (lb.rows.rows.size() != n)
    throw std::runtime_error("label file has " + std::to_string(lb.rows.rows.size()) + " rows for " +
                             std::to_string(n) + " points");
  dio::canonical_csr(lb.rows, lb.offsets, lb.ids);
  return lb;
}

// Index of the row nearest (fp64 squared L2, ties to the lower id) to the
// centroid of the listed rows.
template <typename T>
uint32_t nearest_to_centroid(const std::vector<T>& x, uint32_t dim, const uint32_t* rows, size_t count,
                             std::vector<double>& cent) {
  cent.assign(dim, 0.0);
  for (size_t i = 0; i < count; ++i) {
    const T* v = x.data() + (size_t)rows[i] * dim;
    for (uint32_t d = 0; d < dim; ++d) cent[d] += (double)v[d];
  }
  for (uint32_t d = 0; d < dim; ++d) cent[d] /= (double)count;
  uint32_t best = kInvalid;
  double best_d = std::numeric_limits<double>::infinity();
  for (size_t i = 0; i < count; ++i) {
    const T* v = x.data() + (size_t)rows[i] * dim;
    double s = 0.0;
    for (uint32_t d = 0; d < dim; ++d) {
      const double t = (double)v[d] - cent[d];
      s += t * t;
    }
    if (s < best_d || (s == best_d && rows[i] < best)) {
      best_d = s;
      best = rows[i];
    }
  }
  return best;
}

// Label starts by Filtered-DiskANN's load-balanced FindMedoid, as upstream
// DiskANN's Index::build_filtered_index picks them right before the patch's
// GPU branch (patch:20239, `_medoid_counts[best_medoid]++`, is that loop's
// last line; the starts reach the builder at :20288-20296): per label, in
// ascending id order, draw kStartCands carriers uniformly with replacement,
// keep the first drawn among those that already start the fewest labels, and
// count it once more. Carriers of the universal label carry every label. The
// draws are splitmix64 outputs modulo the carrier count, seeded with
// DISKANN_GPU_FILTERED_LABEL_START_SEED (default 1), in place of rand().
constexpr uint32_t kStartCands = 25;

uint64_t splitmix64(uint64_t& s) {
  uint64_t z = (s += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

std::vector<uint32_t> balanced_label_starts(const Labels& lb, uint32_t n, uint64_t seed) {
  const uint32_t num_labels = lb.count();
  std::vector<uint32_t> loff, pts;
  dio::postings(lb.offsets, lb.ids, num_labels, loff, pts);
  std::vector<uint32_t> universal;  // carriers of the universal label, ascending
  if (lb.universal < num_labels)
    universal.assign(pts.begin() + loff[lb.universal], pts.begin() + loff[lb.universal + 1]);
  std::vector<uint32_t> load(n, 0), starts(num_labels, kInvalid), carriers;
  uint64_t state = seed;
  for (uint32_t l = 0; l < num_labels; ++l) {
    carriers.clear();
    std::set_union(pts.begin() + loff[l], pts.begin() + loff[l + 1], universal.begin(), universal.end(),
                   std::back_inserter(carriers));
    if (carriers.empty()) continue;
    uint32_t best = kInvalid, best_load = kInvalid;
    for (uint32_t c = 0; c < kStartCands; ++c) {
      const uint32_t cand = carriers[splitmix64(state) % carriers.size()];
      if (load[cand] < best_load) {
        best_load = load[cand];
        best = cand;
      }
    }
    starts[l] = best;
    ++load[best];
  }
  return starts;
}

// The global start is the point nearest to the centroid (DiskANN
// calculate_entry_point, patch:20267). Label starts follow the rule above, or
// with DANCE_LABEL_STARTS=centroid the carrier of each label nearest to the
// centroid of its carriers.
template <typename T>
void entry_points(const std::vector<T>& x, uint32_t n, uint32_t dim, const Labels& lb, uint32_t& global_start,
                  std::vector<uint32_t>& label_start) {
  std::vector<uint32_t> all(n);
  for (uint32_t i = 0; i < n; ++i) all[i] = i;
  std::vector<double> cent;
  global_start = nearest_to_centroid(x, dim, all.data(), n, cent);
  const char* rule = std::getenv("DANCE_LABEL_STARTS");
  if (!(rule && std::string(rule) == "centroid")) {
    if (rule && rule[0] && std::string(rule) != "balanced")
      throw std::runtime_error(std::string("DANCE_LABEL_STARTS=") + rule + " is neither balanced nor centroid");
    const char* seed_env = std::getenv("DISKANN_GPU_FILTERED_LABEL_START_SEED");
    const uint64_t seed = seed_env && seed_env[0] ? std::strtoull(seed_env, nullptr, 10) : 1ull;
    label_start = balanced_label_starts(lb, n, seed);
    return;
  }
  const uint32_t num_labels = lb.count();
  std::vector<uint32_t> loff, pts;
  dio::postings(lb.offsets, lb.ids, num_labels, loff, pts);
  label_start.assign(num_labels, kInvalid);
#pragma omp parallel for schedule(dynamic, 16)
  for (uint32_t l = 0; l < num_labels; ++l) {
    const size_t c = loff[l + 1] - loff[l];
    if (c == 0) continue;
    std::vector<double> cl;
    label_start[l] = nearest_to_centroid(x, dim, pts.data() + loff[l], c, cl);
  }
}

// Internal degree and publish choice (patch:20368-20384); sets or clears
// DISKANN_GPU_FILTERED_PUBLISH_DEGREE for the library.
void publish_plan(uint32_t R, uint32_t& builder_R, bool& gpu_publish) {
  builder_R = std::max(R, kMinInternalDegree);
  const char* internal_env = std::getenv("DISKANN_GPU_FILTERED_INTERNAL_DEGREE");
  if (internal_env && std::atoi(internal_env) > 0) builder_R = std::max(R, (uint32_t)std::atoi(internal_env));
  const char* publish_env = std::getenv("DISKANN_GPU_FILTERED_GPU_PUBLISH");
  gpu_publish = builder_R > R && (!publish_env || std::atoi(publish_env) != 0);
  if (builder_R > R && !gpu_publish)
    throw std::runtime_error("[GPU filtered] DISKANN_GPU_FILTERED_GPU_PUBLISH=0 with internal degree " +
                             std::to_string(builder_R) + " above --max_degree " + std::to_string(R) +
                             " needs DiskANN's CPU prune, which this build does not provide");
  if (gpu_publish)
    setenv("DISKANN_GPU_FILTERED_PUBLISH_DEGREE", std::to_string(R).c_str(), 1);
  else
    unsetenv("DISKANN_GPU_FILTERED_PUBLISH_DEGREE");
}

template <typename T>
int run(const Options& o) {
  const double t0 = now_sec();
  uint32_t builder_R = 0;
  bool gpu_publish = false;
  publish_plan(o.R, builder_R, gpu_publish);
  const uint32_t R = gpu_publish ? o.R : builder_R;  // row width of the returned graph
  uint32_t n = 0, dim = 0;
  std::vector<T> x = dio::read_bin<T>(o.data_path, n, dim);
  Labels lb = read_labels(o, n);
  uint32_t global_start = 0;
  std::vector<uint32_t> starts;
  entry_points(x, n, dim, lb, global_start, starts);
  const double t_prep = now_sec();

  const uint32_t L = o.L, Lf = o.Lf == 0 ? o.L : o.Lf;
  const char* steps_env = std::getenv("DISKANN_GPU_FILTERED_STEPS");
  const uint32_t steps = steps_env ? (uint32_t)std::max(1, std::atoi(steps_env)) : std::min<uint32_t>(64, L);
  std::cout << "[GPU filtered] requested_R=" << o.R << " internal_R=" << builder_R
            << " publish_backend=" << (gpu_publish ? "gpu_warp_exact_csr" : "direct") << std::endl;
  std::cout << "[GPU filtered] N=" << n << " dim=" << dim << " labels=" << lb.count() - 1
            << " label_slots=" << lb.ids.size() << " global_start=" << global_start << " L=" << L
            << " filtered_L=" << Lf << " C=" << kDefaultMaxC << " steps=" << steps << " alpha=" << o.alpha
            << std::endl;
  std::vector<uint32_t> graph((size_t)n * builder_R, kInvalid), degree(n, 0);
  int rc;
  if (std::is_same<T, uint8_t>::value)
    rc = gpu_vamana_filtered_build_uint8(reinterpret_cast<const uint8_t*>(x.data()), n, dim, builder_R, L, Lf,
                                         kDefaultMaxC,
                                         steps, o.alpha, lb.offsets.data(), lb.ids.data(), (uint32_t)lb.ids.size(),
                                         starts.data(), (uint32_t)starts.size(), lb.universal, global_start, nullptr,
                                         nullptr, 0, graph.data(), degree.data());
  else
    rc = gpu_vamana_filtered_build_float(reinterpret_cast<const float*>(x.data()), n, dim, builder_R, L, Lf,
                                         kDefaultMaxC,
                                         steps, o.alpha, lb.offsets.data(), lb.ids.data(), (uint32_t)lb.ids.size(),
                                         starts.data(), (uint32_t)starts.size(), lb.universal, global_start, nullptr,
                                         nullptr, 0, graph.data(), degree.data());
  if (rc != 0) throw std::runtime_error("[GPU filtered] gpu_vamana_filtered_build failed with code " + std::to_string(rc));
  GPUFilteredVamanaStats st;
  gpu_vamana_filtered_get_last_stats(&st);
  std::cout << "[GPU filtered] stats semantic_complete=" << st.semantic_complete
            << " gpu_build_seconds=" << st.gpu_build_seconds << " peak_gpu_mem_gb=" << st.peak_gpu_mem_gb
            << " avg_common_label_out_degree=" << st.avg_common_label_out_degree
            << " label_reject_count=" << st.label_reject_count
            << " invalid_neighbor_count=" << st.invalid_neighbor_count
            << " self_loop_count=" << st.self_loop_count << std::endl;
  const double t_build = now_sec();

  // DISKANN_GPU_FILTERED_RESELECT_LABEL_STARTS=common_degree (patch:20447-20504):
  // each label's start becomes the carrier with the most neighbours carrying
  // the label (or the universal label) in the raw graph, then the larger raw
  // degree, then the lower id. Labels without a carrier keep their start.
  const char* reselect = std::getenv("DISKANN_GPU_FILTERED_RESELECT_LABEL_STARTS");
  if (reselect && std::string(reselect) == "common_degree") {
    auto has = [&](uint32_t p, uint32_t label) {
      return std::binary_search(lb.ids.begin() + lb.offsets[p], lb.ids.begin() + lb.offsets[p + 1], label);
    };
    const size_t nl = starts.size();
    std::vector<uint32_t> best(nl, kInvalid), best_common(nl, 0), best_out(nl, 0);
    for (uint32_t node = 0; node < n; ++node)
      for (uint32_t q = lb.offsets[node]; q < lb.offsets[node + 1]; ++q) {
        const uint32_t label = lb.ids[q];
        if (label == lb.universal || label >= nl) continue;
        uint32_t common = 0;
        for (uint32_t j = 0; j < degree[node] && j < R; ++j) {
          const uint32_t nb = graph[(size_t)node * R + j];
          if (nb < n && nb != node && (has(nb, label) || (lb.universal != kInvalid && has(nb, lb.universal))))
            ++common;
        }
        if (best[label] == kInvalid || common > best_common[label] ||
            (common == best_common[label] && degree[node] > best_out[label])) {
          best[label] = node;
          best_common[label] = common;
          best_out[label] = degree[node];
        }
      }
    uint32_t reselected = 0, changed = 0;
    for (size_t l = 0; l < nl; ++l)
      if (best[l] != kInvalid) {
        ++reselected;
        changed += starts[l] != best[l];
        starts[l] = best[l];
      }
    std::cout << "[GPU filtered] reselected label starts mode=common_degree labels=" << reselected
              << " changed=" << changed << std::endl;
  }

  // Install (patch:20506-20521): per row drop invalid / self / repeated ids;
  // an empty row of a multi-point index gets (i + 1) mod N.
  const dio::RowFn installed = [&](uint32_t i, std::vector<uint32_t>& row) {
    for (uint32_t j = 0; j < degree[i] && j < R; ++j) {
      const uint32_t nb = graph[(size_t)i * R + j];
      if (nb != kInvalid && nb < n && nb != i && std::find(row.begin(), row.end(), nb) == row.end())
        row.push_back(nb);
    }
    if (row.empty() && n > 1) row.push_back((i + 1) % n);
  };
  dio::File gf(o.prefix, O_WRONLY | O_CREAT | O_TRUNC);
  if (!gf.ok()) throw std::runtime_error("failed to write " + o.prefix);
  const dio::GraphSummary gs = dio::write_graph(gf, n, global_start, installed);
  gf.close_checked();
  const uint64_t edges = gs.edges;
  const uint32_t max_deg = gs.max_degree;
  {
    dio::File d(o.prefix + ".data", O_WRONLY | O_CREAT | O_TRUNC);
    if (!d.ok()) throw std::runtime_error("failed to write " + o.prefix + ".data");
    dio::write_bin(d, n, dim, x.data());
    d.close_checked();
  }
  const auto& tokens = lb.rows.rows;
  dio::write_text(o.prefix + "_labels.txt", dio::id_rows_text(n, [&](size_t i, std::vector<uint32_t>& r) {
                    r.assign(lb.ids.begin() + lb.offsets[i], lb.ids.begin() + lb.offsets[i + 1]);
                  }));
  dio::write_text(o.prefix + "_label_formatted.txt",
                  dio::id_rows_text(n, [&](size_t i, std::vector<uint32_t>& r) { r = tokens[i]; }));
  std::string map, medoids;
  for (uint32_t l = lb.universal == 0 ? 0 : 1; l < lb.count(); ++l)
    map += lb.rows.names[l] + "\t" + std::to_string(l) + "\n";
  for (uint32_t l = 0; l < starts.size(); ++l)
    if (starts[l] != kInvalid) medoids += std::to_string(l) + ", " + std::to_string(starts[l]) + "\n";
  dio::write_text(o.prefix + "_labels_map.txt", map);
  dio::write_text(o.prefix + "_labels_to_medoids.txt", medoids);
  if (lb.universal == 0) dio::write_text(o.prefix + "_universal_label.txt", "0\n");
  const double t_end = now_sec();
  std::cout << "[GPU filtered] graph installed: edges=" << edges << " max_degree=" << max_deg
            << " prepare_seconds=" << t_prep - t0 << " build_seconds=" << t_build - t_prep
            << " save_seconds=" << t_end - t_build << " total_seconds=" << t_end - t0 << std::endl;
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    const Options o = parse(argc, argv);
    std::cout << "Starting index build with R: " << o.R << "  Lbuild: " << o.L << "  alpha: " << o.alpha
              << "  #threads: " << o.threads << std::endl;
    return o.data_type == "uint8" ? run<uint8_t>(o) : run<float>(o);
  } catch (const std::exception& e) {
    std::cerr << "Index build failed: " << e.what() << std::endl;
    return -1;
  }
}
