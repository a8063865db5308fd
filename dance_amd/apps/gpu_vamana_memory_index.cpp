// gpu_vamana_memory_index: builds a DiskANN in-memory index with the GPU
// Vamana builder (libdance_hip.so).
//
// Same command line, file formats, validation rules, JSON report and exit
// codes as the reference app (/root/reference/apps/utils/gpu_vamana_memory_index.cpp):
//   --data_path <bin> [--data_type uint8|float] [--offset N] [--npts N|0=all]
//   [--index_prefix PATH] [--R 42] [--L 100] [--C 80] [--STEPS 64] [--builder vnew2|v8]
// Input: DiskANN matrix file (uint32 N, uint32 dim, row-major payload), the
// size checked exactly (:157-195). Output (only for a valid graph, :349-386):
// <prefix> = DiskANN graph (uint64 file bytes, uint32 max degree, uint32
// medoid, uint64 frozen points, then per node uint32 k + k ids) and
// <prefix>.data, both written to temporaries and renamed, never overwriting
// (:197-297). Exit codes: 0 ok, 2 usage/input error, 3 invalid graph, else the
// builder's return code (:423-449).

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <fstream>
#include <iostream>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

#include "gpu_vamana_builder.h"

namespace {

struct Options {
  std::string data_path, data_type = "uint8", index_prefix, builder = "vnew2";
  uint64_t offset = 0;
  uint32_t npts = 0, R = 42, L = 100, C = 80, STEPS = 64;
};

double seconds_since_start() {
  static const auto t0 = std::chrono::steady_clock::now();
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

std::string json_string(const std::string& s) {
  std::string out;
  for (unsigned char c : s) {
    switch (c) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\b': out += "\\b"; break;
      case '\f': out += "\\f"; break;
      case '\n': out += "\\n"; break;
      case '\r': out += "\\r"; break;
      case '\t': out += "\\t"; break;
      default:
        if (c < 0x20) throw std::runtime_error("control character in JSON path");
        out.push_back((char)c);
    }
  }
  return out;
}

uint64_t to_u64(const std::string& v, const std::string& opt) {
  if (v.empty() || v.find_first_not_of("0123456789") != std::string::npos)
    throw std::runtime_error(opt + " must be an unsigned integer");
  try {
    size_t used = 0;
    unsigned long long x = std::stoull(v, &used, 10);
    if (used != v.size()) throw std::runtime_error("");
    return x;
  } catch (...) {
    throw std::runtime_error(opt + " must be an unsigned integer");
  }
}

uint32_t to_u32(const std::string& v, const std::string& opt, bool zero_ok) {
  const uint64_t x = to_u64(v, opt);
  if (x > std::numeric_limits<uint32_t>::max() || (!zero_ok && x == 0))
    throw std::runtime_error(opt + (zero_ok ? " is out of uint32 range" : " must be in [1, UINT32_MAX]"));
  return (uint32_t)x;
}

void print_usage(const char* prog) {
  std::cerr << "Usage: " << prog
            << " --data_path <bin> [--data_type uint8|float] [--offset N] [--npts N|0=all]"
            << " [--index_prefix PATH] [--R 42] [--L 100] [--C 80] [--STEPS 64] [--builder vnew2|v8]\n";
}

Options parse(int argc, char** argv) {
  Options o;
  static const char* known[] = {"--data_path", "--data_type", "--index_prefix", "--offset", "--npts",
                                "--R",         "--L",         "--C",            "--STEPS",  "--builder"};
  for (int i = 1; i < argc; ++i) {
    const std::string k = argv[i];
    if (std::find(std::begin(known), std::end(known), k) == std::end(known))
      throw std::runtime_error("unknown argument: " + k);
    if (i + 1 >= argc) throw std::runtime_error("missing value for " + k);
    const std::string v = argv[++i];
    if (k == "--data_path") o.data_path = v;
    else if (k == "--data_type") o.data_type = v;
    else if (k == "--index_prefix") o.index_prefix = v;
    else if (k == "--offset") o.offset = to_u64(v, k);
    else if (k == "--npts") o.npts = to_u32(v, k, true);
    else if (k == "--R") o.R = to_u32(v, k, false);
    else if (k == "--L") o.L = to_u32(v, k, false);
    else if (k == "--C") o.C = to_u32(v, k, false);
    else if (k == "--STEPS") o.STEPS = to_u32(v, k, false);
    else o.builder = v;
  }
  if (o.data_path.empty()) throw std::runtime_error("--data_path is required");
  if (o.data_type != "uint8" && o.data_type != "float") throw std::runtime_error("--data_type must be uint8 or float");
  if (o.builder != "vnew2" && o.builder != "v8") throw std::runtime_error("--builder must be vnew2 or v8");
  (void)json_string(o.data_path);
  (void)json_string(o.index_prefix);
  return o;
}

template <typename T>
std::vector<T> read_slice(const Options& o, uint32_t& dim, uint64_t& total, uint32_t& count) {
  std::ifstream in(o.data_path, std::ios::binary);
  if (!in) throw std::runtime_error("failed to open " + o.data_path);
  uint32_t hdr[2] = {0, 0};
  in.read(reinterpret_cast<char*>(hdr), sizeof(hdr));
  if (!in) throw std::runtime_error("failed to read DiskANN matrix header");
  total = hdr[0];
  dim = hdr[1];
  if (dim == 0 || total > (std::numeric_limits<uint64_t>::max() - 8) / ((uint64_t)dim * sizeof(T)))
    throw std::runtime_error("DiskANN matrix shape overflows its byte-size calculation");
  in.seekg(0, std::ios::end);
  const std::streamoff bytes = in.tellg();
  if (bytes < 0 || (uint64_t)bytes != 8 + total * (uint64_t)dim * sizeof(T))
    throw std::runtime_error("DiskANN matrix header does not match exact file size");
  const uint64_t left = total - std::min<uint64_t>(o.offset, total);
  const uint64_t want = o.npts == 0 ? left : o.npts;
  if (o.offset > total || want > left || want > std::numeric_limits<uint32_t>::max())
    throw std::runtime_error("requested slice exceeds base file point count");
  if (want == 0) throw std::runtime_error("requested slice and dimension must be nonzero");
  count = (uint32_t)want;
  std::vector<T> v((size_t)count * dim);
  in.seekg((std::streamoff)(8 + o.offset * (uint64_t)dim * sizeof(T)), std::ios::beg);
  in.read(reinterpret_cast<char*>(v.data()), (std::streamsize)(v.size() * sizeof(T)));
  if (!in) throw std::runtime_error("failed to read requested slice");
  return v;
}

bool exists(const std::string& p) { return (bool)std::ifstream(p, std::ios::binary); }

template <typename T>
void write_index(const Options& o, const std::vector<T>& data, uint32_t n, uint32_t dim,
                 const std::vector<uint32_t>& graph, const std::vector<uint32_t>& degree, uint32_t medoid) {
  if (o.index_prefix.empty()) return;
  const std::string graph_path = o.index_prefix, data_path = o.index_prefix + ".data";
  const std::string graph_tmp = o.index_prefix + ".tmp", data_tmp = data_path + ".tmp";
  if (exists(graph_path) || exists(data_path) || exists(graph_tmp) || exists(data_tmp))
    throw std::runtime_error("refusing to overwrite existing memory-index output");
  size_t edges = 0;
  for (uint32_t d : degree) edges += std::min(d, o.R);
  const uint32_t max_deg = *std::max_element(degree.begin(), degree.end());
  const size_t frozen = 0;
  const size_t header = sizeof(size_t) + 2 * sizeof(uint32_t) + sizeof(size_t);
  const size_t graph_bytes = header + (size_t)n * 4 + edges * 4;
  const size_t data_bytes = 8 + data.size() * sizeof(T);
  auto cleanup = [&](bool with_data) {
    std::remove(graph_tmp.c_str());
    if (with_data) std::remove(data_tmp.c_str());
  };
  {
    std::ofstream out(graph_tmp, std::ios::binary | std::ios::trunc);
    if (!out) throw std::runtime_error("failed to create graph temporary output " + graph_tmp);
    out.write(reinterpret_cast<const char*>(&graph_bytes), sizeof(graph_bytes));
    out.write(reinterpret_cast<const char*>(&max_deg), 4);
    out.write(reinterpret_cast<const char*>(&medoid), 4);
    out.write(reinterpret_cast<const char*>(&frozen), sizeof(frozen));
    for (uint32_t v = 0; v < n; ++v) {
      const uint32_t k = std::min(degree[v], o.R);
      out.write(reinterpret_cast<const char*>(&k), 4);
      out.write(reinterpret_cast<const char*>(graph.data() + (size_t)v * o.R), (std::streamsize)k * 4);
    }
    out.close();
    if (!out) {
      cleanup(false);
      throw std::runtime_error("failed while writing graph temporary output " + graph_tmp);
    }
  }
  {
    std::ofstream out(data_tmp, std::ios::binary | std::ios::trunc);
    if (!out) {
      cleanup(true);
      throw std::runtime_error("failed to create vector temporary output " + data_tmp);
    }
    out.write(reinterpret_cast<const char*>(&n), 4);
    out.write(reinterpret_cast<const char*>(&dim), 4);
    out.write(reinterpret_cast<const char*>(data.data()), (std::streamsize)(data.size() * sizeof(T)));
    out.close();
    if (!out) {
      cleanup(true);
      throw std::runtime_error("failed while writing vector temporary output " + data_tmp);
    }
  }
  std::ifstream g(graph_tmp, std::ios::binary | std::ios::ate), d(data_tmp, std::ios::binary | std::ios::ate);
  if (!g || g.tellg() != (std::streamoff)graph_bytes || !d || d.tellg() != (std::streamoff)data_bytes) {
    cleanup(true);
    throw std::runtime_error("serialized temporary output size does not match its DiskANN layout");
  }
  if (std::rename(data_tmp.c_str(), data_path.c_str()) != 0) {
    cleanup(true);
    throw std::runtime_error("failed to publish vector output " + data_path);
  }
  if (std::rename(graph_tmp.c_str(), graph_path.c_str()) != 0) {
    std::remove(graph_tmp.c_str());
    std::remove(data_path.c_str());
    throw std::runtime_error("failed to publish graph output " + graph_path);
  }
}

template <typename T>
int run(const Options& o) {
  uint32_t dim = 0, n = 0;
  uint64_t total = 0;
  const double t_load = seconds_since_start();
  std::vector<T> data = read_slice<T>(o, dim, total, n);
  const double load_s = seconds_since_start() - t_load;
  if ((size_t)n > std::numeric_limits<size_t>::max() / 4 / o.R)
    throw std::runtime_error("N * R overflows the host graph allocation");
  std::vector<uint32_t> graph((size_t)n * o.R), degree(n);
  const double t_gpu = seconds_since_start();
  int rc;
  if constexpr (std::is_same<T, uint8_t>::value)
    rc = o.builder == "vnew2" ? gpu_vamana_vnew2_build(data.data(), n, dim, o.R, o.L, o.C, o.STEPS, graph.data(), degree.data())
                              : gpu_vamana_build(data.data(), n, dim, o.R, o.L, o.C, o.STEPS, graph.data(), degree.data());
  else
    rc = o.builder == "vnew2"
             ? gpu_vamana_vnew2_build_float(data.data(), n, dim, o.R, o.L, o.C, o.STEPS, graph.data(), degree.data())
             : gpu_vamana_build_float(data.data(), n, dim, o.R, o.L, o.C, o.STEPS, graph.data(), degree.data());
  const double gpu_s = seconds_since_start() - t_gpu;
  GPUVamanaStats st{};
  uint32_t medoid;
  if (o.builder == "vnew2") {
    medoid = gpu_vamana_vnew2_get_last_medoid();
    gpu_vamana_vnew2_get_last_stats(&st);
  } else {
    medoid = gpu_vamana_get_last_medoid();
    gpu_vamana_get_last_stats(&st);
  }
  uint64_t edges = 0, invalid = 0, self = 0, dup = 0, overflow = 0;
  uint32_t max_deg = 0;
  std::vector<uint32_t> row;
  for (uint32_t v = 0; v < n; ++v) {
    const uint32_t d = degree[v];
    edges += d;
    max_deg = std::max(max_deg, d);
    if (d > o.R) ++overflow;
    row.clear();
    for (uint32_t j = 0; j < std::min(d, o.R); ++j) {
      const uint32_t u = graph[(size_t)v * o.R + j];
      if (u >= n) {
        ++invalid;
        continue;
      }
      if (u == v) ++self;
      row.push_back(u);
    }
    std::sort(row.begin(), row.end());
    dup += (uint64_t)(row.end() - std::unique(row.begin(), row.end()));
  }
  const bool valid = rc == 0 && invalid == 0 && self == 0 && dup == 0 && overflow == 0 && medoid < n;
  if (valid) write_index(o, data, n, dim, graph, degree, medoid);
  std::ostringstream js;
  js << "{\n"
     << "  \"data_path\": \"" << json_string(o.data_path) << "\",\n"
     << "  \"data_type\": \"" << o.data_type << "\",\n"
     << "  \"base_npts\": " << total << ",\n"
     << "  \"offset\": " << o.offset << ",\n"
     << "  \"npts\": " << n << ",\n"
     << "  \"dim\": " << dim << ",\n"
     << "  \"R\": " << o.R << ",\n"
     << "  \"L\": " << o.L << ",\n"
     << "  \"C\": " << o.C << ",\n"
     << "  \"STEPS\": " << o.STEPS << ",\n"
     << "  \"builder\": \"" << o.builder << "\",\n"
     << "  \"index_prefix\": \"" << json_string(o.index_prefix) << "\",\n"
     << "  \"memory_index_serialized\": " << (!o.index_prefix.empty() && valid ? "true" : "false") << ",\n"
     << "  \"load_seconds\": " << load_s << ",\n"
     << "  \"gpu_call_seconds\": " << gpu_s << ",\n"
     << "  \"stats_gpu_build_seconds\": " << st.gpu_build_seconds << ",\n"
     << "  \"stats_h2d_seconds\": " << st.h2d_seconds << ",\n"
     << "  \"stats_search_online_insert_seconds\": " << st.search_online_insert_seconds << ",\n"
     << "  \"stats_reverse_seconds\": " << st.reverse_seconds << ",\n"
     << "  \"stats_final_prune_seconds\": " << st.final_prune_seconds << ",\n"
     << "  \"stats_d2h_seconds\": " << st.d2h_seconds << ",\n"
     << "  \"selective_active_nodes\": " << st.selective_active_nodes << ",\n"
     << "  \"medoid\": " << medoid << ",\n"
     << "  \"edge_count\": " << edges << ",\n"
     << "  \"avg_degree\": " << (double)edges / (double)n << ",\n"
     << "  \"max_degree\": " << max_deg << ",\n"
     << "  \"invalid_neighbor_count\": " << invalid << ",\n"
     << "  \"self_loop_count\": " << self << ",\n"
     << "  \"duplicate_edge_count\": " << dup << ",\n"
     << "  \"degree_overflow_count\": " << overflow << ",\n"
     << "  \"graph_valid\": " << (valid ? "true" : "false") << ",\n"
     << "  \"return_code\": " << rc << "\n"
     << "}\n";
  std::cout << js.str();
  return valid ? 0 : (rc != 0 ? rc : 3);
}

}  // namespace

int main(int argc, char** argv) {
  try {
    const Options o = parse(argc, argv);
    std::string exe = argc > 0 ? argv[0] : "";
    const size_t slash = exe.find_last_of("/\\");
    if (slash != std::string::npos) exe = exe.substr(slash + 1);
    if (exe == "gpu_vamana_memory_index" && o.index_prefix.empty())
      throw std::runtime_error("gpu_vamana_memory_index requires --index_prefix");
    if (exe == "gpu_vamana_memory_index" && o.builder != "vnew2")
      throw std::runtime_error("gpu_vamana_memory_index requires --builder vnew2");
    return o.data_type == "uint8" ? run<uint8_t>(o) : run<float>(o);
  } catch (const std::exception& e) {
    print_usage(argc > 0 ? argv[0] : "gpu_vamana_memory_index");
    std::cerr << "error: " << e.what() << std::endl;
    return 2;
  }
}
