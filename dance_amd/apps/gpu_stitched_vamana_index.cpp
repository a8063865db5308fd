// gpu_stitched_vamana_index: StitchedVamana for labelled data with the GPU
// Vamana builder (libdance_hip.so).
//
// Same command line, file formats and exit codes as the reference app
// (/root/reference/apps/utils/gpu_stitched_vamana_index.cpp):
//   --data_type uint8|float --data_path <bin> --label_file <txt>
//   --index_path_prefix PATH [--universal_label S] [--timing_json PATH]
//   [--Rsmall 32] [--Lsmall 100] [--Rstitched 64] [--C 96] [--steps 64]
//   [--num_threads|-T 32] [--alpha 1.2]
// Labels (:111-160): one line per point, comma-separated names, spaces and
// CR removed, repeats within a line dropped; ids 1.. by first appearance;
// empty rows / tokens and the universal label are errors.
// Build (:241-341): per label in id order, a vnew2 build of the label's points
// (ascending point ids) with Rsmall/Lsmall/C/steps; the label medoid is the
// global id of the local medoid; local rows are remapped to global ids (at
// most Rstitched entries taken per label, invalid / self / repeated ids
// dropped) and appended to the point's row.
// Output (:162-229): <prefix> DiskANN graph (start 0, no frozen points),
// <prefix>.data (copy of the input), <prefix>_labels.txt,
// <prefix>_label_formatted.txt, <prefix>_labels_map.txt,
// <prefix>_labels_to_medoids.txt; optional timing JSON.
// The reference then runs DiskANN's CPU prune_all_neighbors when some row has
// more than one label (:349-372); that CPU step belongs to upstream DiskANN
// and is not part of this library: such inputs write <prefix>_full (the
// unpruned graph, as the reference does before pruning) and exit with 3.
// Exit codes: 0 ok, 1 error, 2 unsupported data type, 3 prune unavailable.

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <iostream>
#include <limits>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <unordered_map>
#include <vector>

#include "gpu_vamana_builder.h"

namespace {

constexpr uint32_t kInvalid = std::numeric_limits<uint32_t>::max();

struct Args {
  std::string data_type, data_path, label_file, index_path_prefix, universal_label, timing_json;
  uint32_t r_small = 32, l_small = 100, r_out = 64, c = 96, steps = 64, threads = 32;
  float alpha = 1.2f;
};

double now_sec() {
  static const auto t0 = std::chrono::steady_clock::now();
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

void usage(std::ostream& os) {
  os << "gpu_stitched_vamana_index: Build GPU StitchedVamana for single- or multi-label data.\n"
     << "  --data_type uint8|float        (required)\n"
     << "  --data_path PATH               (required)\n"
     << "  --label_file PATH              (required)\n"
     << "  --index_path_prefix PATH       (required)\n"
     << "  --universal_label NAME         (default none)\n"
     << "  --timing_json PATH             (default none)\n"
     << "  --Rsmall N (32) --Lsmall N (100) --Rstitched N (64) --C N (96) --steps N (64)\n"
     << "  --num_threads|-T N (32) --alpha F (1.2)\n";
}

uint32_t to_u32(const std::string& v, const std::string& k) {
  if (v.empty() || v.find_first_not_of("0123456789") != std::string::npos)
    throw std::runtime_error("the argument ('" + v + "') for option '" + k + "' is invalid");
  const unsigned long long x = std::stoull(v);
  if (x > std::numeric_limits<uint32_t>::max())
    throw std::runtime_error("the argument ('" + v + "') for option '" + k + "' is invalid");
  return (uint32_t)x;
}

float to_f32(const std::string& v, const std::string& k) {
  size_t used = 0;
  float f = 0;
  try {
    f = std::stof(v, &used);
  } catch (...) {
    used = 0;
  }
  if (used == 0 || used != v.size())
    throw std::runtime_error("the argument ('" + v + "') for option '" + k + "' is invalid");
  return f;
}

// Accepts "--name value" and "--name=value" (and -h, -T), like
// boost::program_options; all four path options are required.
Args parse_args(int argc, char** argv) {
  Args a;
  bool seen_type = false, seen_data = false, seen_labels = false, seen_prefix = false;
  for (int i = 1; i < argc; ++i) {
    std::string k = argv[i], v;
    if (k == "--help" || k == "-h") {
      usage(std::cout);
      std::exit(0);
    }
    const size_t eq = k.find('=');
    if (k.rfind("--", 0) == 0 && eq != std::string::npos) {
      v = k.substr(eq + 1);
      k = k.substr(0, eq);
    } else {
      if (i + 1 >= argc) throw std::runtime_error("the required argument for option '" + k + "' is missing");
      v = argv[++i];
    }
    if (k == "--data_type") a.data_type = v, seen_type = true;
    else if (k == "--data_path") a.data_path = v, seen_data = true;
    else if (k == "--label_file") a.label_file = v, seen_labels = true;
    else if (k == "--index_path_prefix") a.index_path_prefix = v, seen_prefix = true;
    else if (k == "--universal_label") a.universal_label = v;
    else if (k == "--timing_json") a.timing_json = v;
    else if (k == "--Rsmall") a.r_small = to_u32(v, k);
    else if (k == "--Lsmall") a.l_small = to_u32(v, k);
    else if (k == "--Rstitched") a.r_out = to_u32(v, k);
    else if (k == "--C") a.c = to_u32(v, k);
    else if (k == "--steps") a.steps = to_u32(v, k);
    else if (k == "--num_threads" || k == "-T") a.threads = to_u32(v, k);
    else if (k == "--alpha") a.alpha = to_f32(v, k);
    else throw std::runtime_error("unrecognised option '" + k + "'");
  }
  if (!seen_type) throw std::runtime_error("the option '--data_type' is required but missing");
  if (!seen_data) throw std::runtime_error("the option '--data_path' is required but missing");
  if (!seen_labels) throw std::runtime_error("the option '--label_file' is required but missing");
  if (!seen_prefix) throw std::runtime_error("the option '--index_path_prefix' is required but missing");
  if (a.r_out < a.r_small) a.r_out = a.r_small;
  return a;
}

// DiskANN matrix file: int32 npts, int32 dim, payload (:90-106).
template <typename T>
std::vector<T> load_bin(const std::string& path, uint32_t& npts, uint32_t& dim) {
  std::ifstream in(path, std::ios::binary);
  if (!in) throw std::runtime_error("failed to open data file: " + path);
  int32_t hdr[2] = {0, 0};
  in.read(reinterpret_cast<char*>(hdr), sizeof(hdr));
  if (!in) throw std::runtime_error("failed to read data payload: " + path);
  npts = (uint32_t)hdr[0];
  dim = (uint32_t)hdr[1];
  std::vector<T> data((size_t)npts * dim);
  in.read(reinterpret_cast<char*>(data.data()), (std::streamsize)(data.size() * sizeof(T)));
  if (!in) throw std::runtime_error("failed to read data payload: " + path);
  return data;
}

void copy_file(const std::string& src, const std::string& dst) {
  std::ifstream in(src, std::ios::binary);
  std::ofstream out(dst, std::ios::binary);
  out << in.rdbuf();
}

struct LabelTable {
  std::vector<std::vector<std::string>> point_names;  // per point, first-appearance order
  std::unordered_map<std::string, uint32_t> id_of;   // name -> 1-based id
  std::vector<std::string> names;                     // id-1 -> name
  std::vector<std::vector<uint32_t>> points;          // id-1 -> ascending point ids
};

LabelTable parse_labels(const std::string& path, const std::string& universal) {
  std::ifstream in(path);
  if (!in) throw std::runtime_error("failed to open label file: " + path);
  LabelTable t;
  std::string line;
  while (std::getline(in, line)) {
    line.erase(std::remove_if(line.begin(), line.end(), [](unsigned char ch) { return ch == '\r' || ch == ' '; }),
               line.end());
    if (line.empty()) throw std::runtime_error("empty label row is not supported");
    std::vector<std::string> row;
    size_t start = 0;
    while (true) {
      const size_t comma = line.find(',', start);
      const std::string name = line.substr(start, comma == std::string::npos ? std::string::npos : comma - start);
      if (name.empty()) throw std::runtime_error("empty label token is not supported");
      if (!universal.empty() && name == universal)
        throw std::runtime_error("GPU StitchedMVP does not support universal-label rows");
      if (std::find(row.begin(), row.end(), name) == row.end()) row.push_back(name);
      if (comma == std::string::npos) break;
      start = comma + 1;
    }
    const uint32_t pid = (uint32_t)t.point_names.size();
    for (const auto& name : row) {
      auto it = t.id_of.find(name);
      if (it == t.id_of.end()) {
        it = t.id_of.emplace(name, (uint32_t)t.names.size() + 1).first;
        t.names.push_back(name);
        t.points.emplace_back();
      }
      t.points[it->second - 1].push_back(pid);
    }
    t.point_names.push_back(std::move(row));
  }
  return t;
}

void write_sidecars(const Args& a, const LabelTable& t, const std::vector<uint32_t>& medoids) {
  copy_file(a.data_path, a.index_path_prefix + ".data");
  {
    std::ofstream labels(a.index_path_prefix + "_labels.txt");
    std::ofstream formatted(a.index_path_prefix + "_label_formatted.txt");
    for (const auto& row : t.point_names) {
      for (size_t j = 0; j < row.size(); ++j) {
        if (j) {
          labels << ',';
          formatted << ',';
        }
        const uint32_t id = t.id_of.at(row[j]);
        labels << id;
        formatted << id;
      }
      labels << "\n";
      formatted << "\n";
    }
  }
  {
    std::ofstream map(a.index_path_prefix + "_labels_map.txt");
    for (uint32_t i = 0; i < t.names.size(); ++i) map << t.names[i] << "\t" << (i + 1) << "\n";
  }
  {
    std::ofstream med(a.index_path_prefix + "_labels_to_medoids.txt");
    for (uint32_t i = 0; i < medoids.size(); ++i) med << (i + 1) << ", " << medoids[i] << "\n";
  }
}

// DiskANN graph file with start 0 and no frozen points (:201-229).
uint64_t write_graph(const std::string& path, const std::vector<std::vector<uint32_t>>& graph) {
  uint64_t bytes = 2 * sizeof(uint64_t) + 2 * sizeof(uint32_t), edges = 0;
  uint32_t max_degree = 0;
  for (const auto& row : graph) {
    max_degree = std::max<uint32_t>(max_degree, (uint32_t)row.size());
    bytes += sizeof(uint32_t) + row.size() * sizeof(uint32_t);
    edges += row.size();
  }
  const uint32_t start = 0;
  const uint64_t frozen = 0;
  std::ofstream out(path, std::ios::binary);
  out.write(reinterpret_cast<const char*>(&bytes), sizeof(bytes));
  out.write(reinterpret_cast<const char*>(&max_degree), sizeof(max_degree));
  out.write(reinterpret_cast<const char*>(&start), sizeof(start));
  out.write(reinterpret_cast<const char*>(&frozen), sizeof(frozen));
  for (const auto& row : graph) {
    const uint32_t deg = (uint32_t)row.size();
    out.write(reinterpret_cast<const char*>(&deg), sizeof(deg));
    if (deg) out.write(reinterpret_cast<const char*>(row.data()), (std::streamsize)deg * sizeof(uint32_t));
  }
  if (!out) throw std::runtime_error("failed to write graph " + path);
  std::cout << "[GPU stitched] wrote graph bytes=" << bytes << " edges=" << edges
            << " avg_degree=" << (graph.empty() ? 0.0 : (double)edges / (double)graph.size())
            << " max_degree=" << max_degree << std::endl;
  return edges;
}

template <typename T>
int build_stitched(const Args& a) {
  const double t0 = now_sec();
  uint32_t npts = 0, dim = 0;
  std::vector<T> data = load_bin<T>(a.data_path, npts, dim);
  LabelTable t = parse_labels(a.label_file, a.universal_label);
  if (t.point_names.size() != npts) throw std::runtime_error("number of label rows does not match data points");
  const size_t nlabels = t.points.size();
  std::vector<std::vector<uint32_t>> graph(npts);
  std::vector<uint32_t> medoids(nlabels, 0);
  double build_s = 0, max_build_s = 0, materialize_s = 0, remap_s = 0;
  uint64_t memberships = 0, bad_local = 0, self_loops = 0, dup_edges = 0;
  uint32_t min_pts = std::numeric_limits<uint32_t>::max(), max_pts = 0;
  std::cout << "[GPU stitched] enabled labels=" << nlabels << " N=" << npts << " dim=" << dim
            << " Rsmall=" << a.r_small << " Lsmall=" << a.l_small << " Rstitched=" << a.r_out << " C=" << a.c
            << std::endl;
  std::vector<T> local;
  std::vector<uint32_t> lgraph, ldeg;
  for (size_t lid = 0; lid < nlabels; ++lid) {
    const auto& ids = t.points[lid];
    if (ids.empty()) continue;
    const uint32_t n = (uint32_t)ids.size();
    min_pts = std::min(min_pts, n);
    max_pts = std::max(max_pts, n);
    memberships += n;
    const double mt = now_sec();
    local.resize((size_t)n * dim);
    for (uint32_t i = 0; i < n; ++i) std::copy_n(data.data() + (size_t)ids[i] * dim, dim, local.data() + (size_t)i * dim);
    materialize_s += now_sec() - mt;
    lgraph.assign((size_t)n * a.r_small, kInvalid);
    ldeg.assign(n, 0);
    const double lt = now_sec();
    int rc;
    if constexpr (std::is_same<T, uint8_t>::value)
      rc = gpu_vamana_vnew2_build(local.data(), n, dim, a.r_small, a.l_small, a.c, a.steps, lgraph.data(),
                                  ldeg.data());
    else
      rc = gpu_vamana_vnew2_build_float(local.data(), n, dim, a.r_small, a.l_small, a.c, a.steps, lgraph.data(),
                                        ldeg.data());
    if (rc != 0) throw std::runtime_error("gpu_vamana_vnew2_build failed for label " + t.names[lid]);
    const double bs = now_sec() - lt;
    build_s += bs;
    max_build_s = std::max(max_build_s, bs);
    uint32_t med = gpu_vamana_vnew2_get_last_medoid();
    if (med >= n) med = 0;
    medoids[lid] = ids[med];
    const double rt = now_sec();
    for (uint32_t i = 0; i < n; ++i) {
      auto& row = graph[ids[i]];
      const uint32_t deg = std::min(ldeg[i], a.r_out);
      for (uint32_t j = 0; j < deg; ++j) {
        const uint32_t nb = lgraph[(size_t)i * a.r_small + j];
        if (nb == kInvalid || nb >= n) {
          ++bad_local;
          continue;
        }
        if (ids[nb] == ids[i]) {
          ++self_loops;
          continue;
        }
        const uint32_t g = ids[nb];
        if (std::find(row.begin(), row.end(), g) == row.end())
          row.push_back(g);
        else
          ++dup_edges;
      }
    }
    remap_s += now_sec() - rt;
    std::cout << "[GPU stitched] label=" << t.names[lid] << " points=" << n << " medoid=" << medoids[lid]
              << " seconds=" << (now_sec() - lt) << std::endl;
  }
  const double wt = now_sec();
  const uint64_t out_edges = write_graph(a.index_path_prefix, graph);
  const double write_s = now_sec() - wt;
  const double mt = now_sec();
  write_sidecars(a, t, medoids);
  const double meta_s = now_sec() - mt;
  const bool single = std::all_of(t.point_names.begin(), t.point_names.end(),
                                  [](const std::vector<std::string>& r) { return r.size() == 1; });
  int exit_code = 0;
  if (single && a.r_small <= a.r_out) {
    std::cout << "[GPU stitched] global label-aware prune is a no-op: single-label rows and Rsmall <= Rstitched"
              << std::endl;
  } else {
    copy_file(a.index_path_prefix, a.index_path_prefix + "_full");
    std::cerr << "[GPU stitched] rows with several labels need DiskANN's CPU prune_all_neighbors(Rstitched, 750, "
                 "alpha), which this library does not provide; the unpruned graph is "
              << a.index_path_prefix << "_full" << std::endl;
    exit_code = 3;
  }
  const double total_s = now_sec() - t0;
  if (min_pts == std::numeric_limits<uint32_t>::max()) min_pts = 0;
  const double mean_pts = nlabels ? (double)memberships / (double)nlabels : 0.0;
  std::cout << "[GPU stitched] total_seconds=" << total_s << " gpu_label_build_seconds=" << build_s
            << " output_edges=" << out_edges << std::endl;
  if (!a.timing_json.empty()) {
    std::ofstream js(a.timing_json);
    js << "{\n"
       << "  \"num_labels\": " << nlabels << ",\n"
       << "  \"npts_per_label_min\": " << min_pts << ",\n"
       << "  \"npts_per_label_mean\": " << mean_pts << ",\n"
       << "  \"npts_per_label_max\": " << max_pts << ",\n"
       << "  \"total_label_memberships\": " << memberships << ",\n"
       << "  \"processed_label_memberships\": " << memberships << ",\n"
       << "  \"remap_invalid_local_ids\": " << bad_local << ",\n"
       << "  \"remap_self_loops\": " << self_loops << ",\n"
       << "  \"remap_duplicate_edges\": " << dup_edges << ",\n"
       << "  \"label_data_materialization_seconds\": " << materialize_s << ",\n"
       << "  \"per_label_gpu_build_sum_seconds\": " << build_s << ",\n"
       << "  \"per_label_gpu_build_max_seconds\": " << max_build_s << ",\n"
       << "  \"local_to_global_remap_seconds\": " << remap_s << ",\n"
       << "  \"write_index_seconds\": " << write_s << ",\n"
       << "  \"final_prune_seconds\": 0,\n"
       << "  \"metadata_seconds\": " << meta_s << ",\n"
       << "  \"total_seconds\": " << total_s << ",\n"
       << "  \"output_edges\": " << out_edges << "\n"
       << "}\n";
  }
  return exit_code;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    const Args a = parse_args(argc, argv);
    if (a.data_type == "uint8") return build_stitched<uint8_t>(a);
    if (a.data_type == "float") return build_stitched<float>(a);
    std::cerr << "GPU StitchedMVP supports uint8 and float in this version" << std::endl;
    return 2;
  } catch (const std::exception& e) {
    std::cerr << "[GPU stitched] failed: " << e.what() << std::endl;
    return 1;
  }
}
