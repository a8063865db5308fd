// gpu_vamana_memory_index: one standard GPU Vamana build of a slice of a
// DiskANN .bin matrix, audited and saved as a DiskANN in-memory index.
//
// Command line, report and files are those of the reference app
// (apps/utils/gpu_vamana_memory_index.cpp): options --data_path,
// --data_type uint8|float, --offset, --npts (0 = to the end),
// --index_prefix, --R 42, --L 100, --C 80, --STEPS 64, --builder vnew2|v8; a
// JSON report on stdout; <prefix> (graph) and <prefix>.data when the graph
// passes its audit; exit 0 when it does, the builder's code when the build
// failed, 3 when the audit failed, 2 on a usage or input error. Run under
// the name gpu_vamana_memory_index it requires --index_prefix and the vnew2
// builder, as the reference does.
//
// Flow: read the slice (pread of exactly the requested rows) -> one call of
// gpu_vamana[_vnew2]_build[_float] -> audit every row (ids, self loops,
// repeats, degree cap) -> publish both files through temporaries.

#include <chrono>
#include <cstdint>
#include <iostream>
#include <string>
#include <type_traits>
#include <vector>

#include "diskann_io.h"
#include "gpu_vamana_builder.h"

namespace {

struct Job {
  std::string data_path, data_type = "uint8", prefix, builder = "vnew2";
  uint64_t offset = 0;
  uint32_t npts = 0;  // 0: every row from the offset on
  uint32_t R = 42, L = 100, C = 80, STEPS = 64;
};

const char* kUsage =
    " --data_path <bin> [--data_type uint8|float] [--offset N] [--npts N|0=all] [--index_prefix PATH]"
    " [--R 42] [--L 100] [--C 80] [--STEPS 64] [--builder vnew2|v8]\n";

Job read_job(int argc, char** argv) {
  Job j;
  dio::ArgTable t;
  t.value({"--data_path"}, [&](const std::string& v, const std::string&) { j.data_path = v; });
  t.value({"--data_type"}, [&](const std::string& v, const std::string&) { j.data_type = v; });
  t.value({"--index_prefix"}, [&](const std::string& v, const std::string&) { j.prefix = v; });
  t.value({"--builder"}, [&](const std::string& v, const std::string&) { j.builder = v; });
  t.value({"--offset"}, [&](const std::string& v, const std::string& k) { j.offset = dio::parse_u64(v, k); });
  t.value({"--npts"}, [&](const std::string& v, const std::string& k) { j.npts = dio::parse_u32(v, k, true); });
  uint32_t* dims[] = {&j.R, &j.L, &j.C, &j.STEPS};
  const char* names[] = {"--R", "--L", "--C", "--STEPS"};
  for (int k = 0; k < 4; ++k) {
    uint32_t* dst = dims[k];
    t.value({names[k]}, [dst](const std::string& v, const std::string& key) { *dst = dio::parse_u32(v, key, false); });
  }
  t.parse(argc, argv);
  if (j.data_path.empty()) throw std::runtime_error("--data_path is required");
  if (j.data_type != "uint8" && j.data_type != "float") throw std::runtime_error("--data_type must be uint8 or float");
  if (j.builder != "vnew2" && j.builder != "v8") throw std::runtime_error("--builder must be vnew2 or v8");
  // paths go into the JSON report: reject what it cannot carry
  for (const std::string* p : {&j.data_path, &j.prefix})
    for (unsigned char c : *p)
      if (c < 0x20 && c != '\b' && c != '\f' && c != '\n' && c != '\r' && c != '\t')
        throw std::runtime_error("control character in JSON path");
  return j;
}

template <typename T>
struct Slice {
  uint64_t file_rows = 0;
  uint32_t dim = 0, n = 0;
  std::vector<T> rows;
};

template <typename T>
Slice<T> load_slice(const Job& j) {
  dio::File f(j.data_path, O_RDONLY);
  if (!f.ok()) throw std::runtime_error("failed to open " + j.data_path);
  const dio::MatrixShape shape = dio::bin_shape(f, sizeof(T));
  Slice<T> s;
  s.file_rows = shape.rows;
  s.dim = shape.dim;
  const uint64_t left = j.offset <= shape.rows ? shape.rows - j.offset : 0;
  const uint64_t want = j.npts ? j.npts : left;
  if (j.offset > shape.rows || want > left || want > 0xFFFFFFFFull)
    throw std::runtime_error("requested slice exceeds base file point count");
  if (want == 0) throw std::runtime_error("requested slice and dimension must be nonzero");
  s.n = (uint32_t)want;
  s.rows = dio::read_bin_rows<T>(f, shape, j.offset, want);
  return s;
}

struct Audit {
  uint64_t edges = 0, invalid = 0, self_loops = 0, repeats = 0, overflows = 0;
  uint32_t max_degree = 0;
  bool clean() const { return invalid == 0 && self_loops == 0 && repeats == 0 && overflows == 0; }
};

// Per row: degree above R is an overflow; within the first min(degree, R)
// slots, ids >= n are invalid, the row's own id is a self loop, and every
// extra copy of a valid id is a repeat.
Audit audit(const std::vector<uint32_t>& graph, const std::vector<uint32_t>& degree, uint32_t n, uint32_t R) {
  Audit a;
  std::vector<uint32_t> ids;
  for (uint32_t v = 0; v < n; ++v) {
    const uint32_t d = degree[v];
    a.edges += d;
    a.max_degree = std::max(a.max_degree, d);
    a.overflows += d > R;
    ids.clear();
    for (uint32_t s = 0; s < std::min(d, R); ++s) {
      const uint32_t u = graph[(size_t)v * R + s];
      if (u >= n) {
        ++a.invalid;
        continue;
      }
      a.self_loops += u == v;
      ids.push_back(u);
    }
    std::sort(ids.begin(), ids.end());
    for (size_t k = 1; k < ids.size(); ++k) a.repeats += ids[k] == ids[k - 1];
  }
  return a;
}

// <prefix>: the graph (rows cut at R), start = medoid, no frozen points;
// <prefix>.data: the slice. Written to temporaries, checked, renamed.
template <typename T>
void save_index(const Job& j, const Slice<T>& s, const std::vector<uint32_t>& graph,
                const std::vector<uint32_t>& degree, uint32_t medoid) {
  const std::string data_path = j.prefix + ".data";
  for (const std::string& p : {j.prefix, data_path, j.prefix + ".tmp", data_path + ".tmp"})
    if (dio::exists(p)) throw std::runtime_error("refusing to overwrite existing memory-index output");
  dio::Publisher pub;
  const dio::RowFn rows = dio::padded_rows(graph.data(), degree.data(), j.R, j.R);
  dio::File& g = pub.open(j.prefix);
  pub.expect(dio::write_graph(g, s.n, medoid, rows).bytes);
  dio::File& d = pub.open(data_path);
  dio::write_bin(d, s.n, s.dim, s.rows.data());
  pub.expect(8 + (uint64_t)s.n * s.dim * sizeof(T));
  pub.commit("DiskANN");
}

double seconds_since(std::chrono::steady_clock::time_point t) {
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t).count();
}

template <typename T>
int build(const Job& j) {
  auto t = std::chrono::steady_clock::now();
  const Slice<T> s = load_slice<T>(j);
  const double load_s = seconds_since(t);
  std::vector<uint32_t> graph((size_t)s.n * j.R), degree(s.n);

  const bool v8 = j.builder == "v8";
  t = std::chrono::steady_clock::now();
  int rc;
  if constexpr (std::is_same<T, uint8_t>::value)
    rc = (v8 ? gpu_vamana_build : gpu_vamana_vnew2_build)(s.rows.data(), s.n, s.dim, j.R, j.L, j.C, j.STEPS,
                                                         graph.data(), degree.data());
  else
    rc = (v8 ? gpu_vamana_build_float : gpu_vamana_vnew2_build_float)(s.rows.data(), s.n, s.dim, j.R, j.L, j.C,
                                                                     j.STEPS, graph.data(), degree.data());
  const double call_s = seconds_since(t);
  GPUVamanaStats st{};
  (v8 ? gpu_vamana_get_last_stats : gpu_vamana_vnew2_get_last_stats)(&st);
  const uint32_t medoid = (v8 ? gpu_vamana_get_last_medoid : gpu_vamana_vnew2_get_last_medoid)();

  const Audit a = audit(graph, degree, s.n, j.R);
  const bool valid = rc == 0 && a.clean() && medoid < s.n;
  if (valid && !j.prefix.empty()) save_index(j, s, graph, degree, medoid);

  dio::JsonReport r;
  r.str("data_path", j.data_path).str("data_type", j.data_type).num("base_npts", s.file_rows)
      .num("offset", j.offset).num("npts", s.n).num("dim", s.dim).num("R", j.R).num("L", j.L).num("C", j.C)
      .num("STEPS", j.STEPS).str("builder", j.builder).str("index_prefix", j.prefix)
      .boolean("memory_index_serialized", valid && !j.prefix.empty()).num("load_seconds", load_s)
      .num("gpu_call_seconds", call_s).num("stats_gpu_build_seconds", st.gpu_build_seconds)
      .num("stats_h2d_seconds", st.h2d_seconds).num("stats_search_online_insert_seconds", st.search_online_insert_seconds)
      .num("stats_reverse_seconds", st.reverse_seconds).num("stats_final_prune_seconds", st.final_prune_seconds)
      .num("stats_d2h_seconds", st.d2h_seconds).num("selective_active_nodes", st.selective_active_nodes)
      .num("medoid", medoid).num("edge_count", a.edges).num("avg_degree", (double)a.edges / (double)s.n)
      .num("max_degree", a.max_degree).num("invalid_neighbor_count", a.invalid)
      .num("self_loop_count", a.self_loops).num("duplicate_edge_count", a.repeats)
      .num("degree_overflow_count", a.overflows).boolean("graph_valid", valid).num("return_code", rc);
  std::cout << r.text();
  if (valid) return 0;
  return rc != 0 ? rc : 3;
}

std::string base_name(const char* path) {
  const std::string p = path ? path : "";
  const size_t k = p.find_last_of("/\\");
  return k == std::string::npos ? p : p.substr(k + 1);
}

}  // namespace

int main(int argc, char** argv) {
  try {
    const Job j = read_job(argc, argv);
    if (base_name(argc > 0 ? argv[0] : nullptr) == "gpu_vamana_memory_index") {
      if (j.prefix.empty()) throw std::runtime_error("gpu_vamana_memory_index requires --index_prefix");
      if (j.builder != "vnew2") throw std::runtime_error("gpu_vamana_memory_index requires --builder vnew2");
    }
    return j.data_type == "uint8" ? build<uint8_t>(j) : build<float>(j);
  } catch (const std::exception& e) {
    std::cerr << "Usage: " << (argc > 0 ? argv[0] : "gpu_vamana_memory_index") << kUsage;
    std::cerr << "error: " << e.what() << std::endl;
    return 2;
  }
}
