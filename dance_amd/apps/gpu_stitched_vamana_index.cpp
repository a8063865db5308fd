// gpu_stitched_vamana_index: StitchedVamana over labelled data. Each label's
// points get their own standard GPU build; the local graphs are stitched into
// one global graph on the device (dance_stitched_build) and saved with the
// DiskANN label sidecars.
//
// Interface of the reference app (apps/utils/gpu_stitched_vamana_index.cpp):
// options --data_type uint8|float, --data_path, --label_file,
// --index_path_prefix (all required), --universal_label, --timing_json,
// --Rsmall 32, --Lsmall 100, --Rstitched 64 (raised to Rsmall when below it),
// --C 96, --steps 64, --num_threads/-T 32, --alpha 1.2 (both for the global
// prune); "--name value" and "--name=value". Labels: one line per point,
// comma-separated names, '\r' and ' ' removed, repeats within a line
// dropped, ids 1, 2, ... by first appearance, empty rows / tokens and the
// universal label rejected. Outputs: <prefix> (graph, start 0, no frozen
// points), <prefix>.data (the input file), <prefix>_labels.txt,
// _label_formatted.txt, _labels_map.txt, _labels_to_medoids.txt; the
// "[GPU stitched] wrote graph ..." and "[GPU stitched timing] ..." log lines
// and the timing JSON keys are the reference's. Exit codes: 0 ok, 1 error,
// 2 unsupported data type.
//
// The reference ends with DiskANN's CPU Index::prune_all_neighbors when some
// row carries several labels (or Rsmall > Rstitched). That upstream CPU
// routine is not part of this library: such inputs write <prefix>_full (the
// unpruned graph, which the reference also writes first) and exit with 3.

#include <chrono>
#include <cstdint>
#include <iostream>
#include <string>
#include <type_traits>
#include <vector>

#include "dance_hip.h"
#include "diskann_io.h"

namespace {

struct Opts {
  std::string data_type, data_path, label_file, prefix, universal, timing_json;
  uint32_t r_small = 32, l_small = 100, r_out = 64, c = 96, steps = 64, threads = 32;
  float alpha = 1.2f;
};

const char* kHelp =
    "gpu_stitched_vamana_index: Build GPU StitchedVamana for single- or multi-label data.\n"
    "  --data_type uint8|float   --data_path PATH   --label_file PATH   --index_path_prefix PATH   (required)\n"
    "  --universal_label NAME    --timing_json PATH\n"
    "  --Rsmall 32  --Lsmall 100  --Rstitched 64  --C 96  --steps 64  --num_threads|-T 32  --alpha 1.2\n";

Opts read_opts(int argc, char** argv) {
  Opts o;
  bool help = false;
  dio::ArgTable t;
  auto invalid = [](const std::string& v, const std::string& k) {
    return std::runtime_error("the argument ('" + v + "') for option '" + k + "' is invalid");
  };
  auto as_u32 = [&](uint32_t* dst) {
    return [dst, invalid](const std::string& v, const std::string& k) {
      try {
        *dst = dio::parse_u32(v, k, true);
      } catch (const std::exception&) {
        throw invalid(v, k);
      }
    };
  };
  auto as_str = [](std::string* dst) { return [dst](const std::string& v, const std::string&) { *dst = v; }; };
  t.flag({"--help", "-h"}, &help);
  t.value({"--data_type"}, as_str(&o.data_type));
  t.value({"--data_path"}, as_str(&o.data_path));
  t.value({"--label_file"}, as_str(&o.label_file));
  t.value({"--index_path_prefix"}, as_str(&o.prefix));
  t.value({"--universal_label"}, as_str(&o.universal));
  t.value({"--timing_json"}, as_str(&o.timing_json));
  t.value({"--Rsmall"}, as_u32(&o.r_small));
  t.value({"--Lsmall"}, as_u32(&o.l_small));
  t.value({"--Rstitched"}, as_u32(&o.r_out));
  t.value({"--C"}, as_u32(&o.c));
  t.value({"--steps"}, as_u32(&o.steps));
  t.value({"--num_threads", "-T"}, as_u32(&o.threads));
  t.value({"--alpha"}, [&](const std::string& v, const std::string& k) {
    char* end = nullptr;
    o.alpha = std::strtof(v.c_str(), &end);
    if (v.empty() || end != v.c_str() + v.size()) throw invalid(v, k);
  });
  dio::ArgStyle style;
  style.equals_form = true;
  style.unknown = [](const std::string& k) { return "unrecognised option '" + k + "'"; };
  style.missing = [](const std::string& k) { return "the required argument for option '" + k + "' is missing"; };
  const std::vector<std::string> seen = t.parse(argc, argv, style);
  if (help) {
    std::cout << kHelp;
    std::exit(0);
  }
  for (const char* req : {"--data_type", "--data_path", "--label_file", "--index_path_prefix"})
    if (std::find(seen.begin(), seen.end(), req) == seen.end())
      throw std::runtime_error(std::string("the option '") + req + "' is required but missing");
  o.r_out = std::max(o.r_out, o.r_small);
  return o;
}

double now_sec() {
  static const auto t0 = std::chrono::steady_clock::now();
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

template <typename T>
std::vector<T> read_vectors(const std::string& path, uint32_t& n, uint32_t& dim) {
  dio::File f(path, O_RDONLY);
  if (!f.ok()) throw std::runtime_error("failed to open data file: " + path);
  int32_t hdr[2] = {0, 0};
  if (f.size() < 8) throw std::runtime_error("failed to read data payload: " + path);
  f.read_at(hdr, 8, 0);
  n = (uint32_t)hdr[0];
  dim = (uint32_t)hdr[1];
  const uint64_t bytes = (uint64_t)n * dim * sizeof(T);
  if (f.size() < 8 + bytes) throw std::runtime_error("failed to read data payload: " + path);
  std::vector<T> x((size_t)n * dim);
  f.read_at(x.data(), bytes, 8);
  return x;
}

// Comma-joined label ids per row (ids in the row's order), one line each.
std::string label_rows_text(const dio::LabelRows& lr) {
  return dio::id_rows_text(lr.rows.size(), [&](size_t i, std::vector<uint32_t>& r) { r = lr.rows[i]; });
}

template <typename T>
int run(const Opts& o) {
  const double t0 = now_sec();
  uint32_t n = 0, dim = 0;
  const std::vector<T> x = read_vectors<T>(o.data_path, n, dim);
  const dio::LabelRows lr = dio::read_labels(
      o.label_file, {o.universal, "GPU StitchedMVP does not support universal-label rows", true, true});
  if (lr.rows.size() != n) throw std::runtime_error("number of label rows does not match data points");
  const uint32_t num_labels = (uint32_t)lr.names.size() - 1;  // ids 1..num_labels

  // label -> ascending points; label l (id l + 1) is built l-th
  std::vector<uint32_t> loff(num_labels + 1, 0), pts;
  uint32_t most = 0;
  for (const auto& r : lr.rows) {
    for (uint32_t id : r) ++loff[id];
    most = std::max(most, (uint32_t)r.size());
  }
  for (uint32_t l = 0; l < num_labels; ++l) loff[l + 1] += loff[l];
  pts.resize(loff[num_labels]);
  {
    std::vector<uint32_t> cur(loff.begin(), loff.end() - 1);
    for (uint32_t p = 0; p < n; ++p)
      for (uint32_t id : lr.rows[p]) pts[cur[id - 1]++] = p;
  }
  uint32_t lmin = 0, lmax = 0;
  for (uint32_t l = 0; l < num_labels; ++l) {
    const uint32_t m = loff[l + 1] - loff[l];
    lmin = l ? std::min(lmin, m) : m;
    lmax = std::max(lmax, m);
  }
  std::cout << "[GPU stitched] enabled labels=" << num_labels << " N=" << n << " dim=" << dim
            << " Rsmall=" << o.r_small << " Lsmall=" << o.l_small << " Rstitched=" << o.r_out << " C=" << o.c
            << std::endl;

  const uint32_t cap = std::max(1u, most * std::min(o.r_small, o.r_out));
  std::vector<uint32_t> graph((size_t)n * cap), degree(n), medoids(std::max(1u, num_labels));
  const int dtype = std::is_same<T, uint8_t>::value ? 1 : 0;
  const int rc = dance_stitched_build(x.data(), dtype, n, dim, loff.data(), pts.data(), num_labels, o.r_small,
                                      o.l_small, o.c, o.steps, o.r_out, cap, graph.data(), degree.data(),
                                      medoids.data());
  if (rc != 0) throw std::runtime_error("dance_stitched_build failed with code " + std::to_string(rc));
  DanceStitchedStats st{};
  dance_get_last_stitched_stats(&st);

  const double tw = now_sec();
  dio::File gf(o.prefix, O_WRONLY | O_CREAT | O_TRUNC);
  if (!gf.ok()) throw std::runtime_error("failed to write " + o.prefix);
  const dio::GraphSummary gs = dio::write_graph(gf, n, 0, dio::padded_rows(graph.data(), degree.data(), cap, cap));
  gf.close_checked();
  std::cout << "[GPU stitched] wrote graph bytes=" << gs.bytes << " edges=" << gs.edges
            << " avg_degree=" << (double)gs.edges / (double)n << " max_degree=" << gs.max_degree << std::endl;
  const double write_index_s = now_sec() - tw;

  const double tm = now_sec();
  dio::copy_file(o.data_path, o.prefix + ".data");
  const std::string rows_text = label_rows_text(lr);
  dio::write_text(o.prefix + "_labels.txt", rows_text);
  dio::write_text(o.prefix + "_label_formatted.txt", rows_text);
  std::string map, med;
  for (uint32_t l = 1; l <= num_labels; ++l) {
    map += lr.names[l] + "\t" + std::to_string(l) + "\n";
    med += std::to_string(l) + ", " + std::to_string(medoids[l - 1]) + "\n";
  }
  dio::write_text(o.prefix + "_labels_map.txt", map);
  dio::write_text(o.prefix + "_labels_to_medoids.txt", med);
  const double metadata_s = now_sec() - tm;

  for (uint32_t l = 0; l < num_labels; ++l)
    std::cout << "[GPU stitched] label=" << lr.names[l + 1] << " points=" << loff[l + 1] - loff[l]
              << " medoid=" << medoids[l] << std::endl;
  const bool needs_prune = most > 1 || o.r_small > o.r_out;
  if (needs_prune) {
    dio::copy_file(o.prefix, o.prefix + "_full");
    std::cerr << "[GPU stitched] rows carry several labels: the global label-aware prune is DiskANN's CPU "
                 "Index::prune_all_neighbors, which this build does not provide; unpruned graph written to "
              << o.prefix << "_full" << std::endl;
    return 3;
  }
  std::cout << "[GPU stitched] global label-aware prune is a no-op: single-label rows and Rsmall <= Rstitched"
            << std::endl;
  const double total_s = now_sec() - t0;
  const double mean = num_labels ? (double)st.memberships / num_labels : 0.0;
  std::cout << "[GPU stitched] total_seconds=" << total_s << " gpu_label_build_seconds=" << st.build_sum_seconds
            << " output_edges=" << gs.edges << std::endl;
  std::cout << "[GPU stitched timing] num_labels=" << num_labels << " npts_per_label_min=" << lmin
            << " npts_per_label_mean=" << mean << " npts_per_label_max=" << lmax
            << " total_label_memberships=" << st.memberships << " processed_label_memberships=" << st.memberships
            << " remap_invalid_local_ids=" << st.remap_invalid_local_ids << " remap_self_loops=" << st.remap_self_loops
            << " remap_duplicate_edges=" << st.remap_duplicate_edges
            << " label_data_materialization_seconds=" << st.materialize_seconds
            << " per_label_gpu_build_sum_seconds=" << st.build_sum_seconds
            << " per_label_gpu_build_max_seconds=" << st.build_max_seconds
            << " local_to_global_remap_seconds=" << st.remap_seconds << " write_index_seconds=" << write_index_s
            << " final_prune_seconds=0 metadata_seconds=" << metadata_s << " total_seconds=" << total_s
            << " peak_gpu_mem_gb=" << st.peak_gpu_mem_gb << " output_edges=" << gs.edges << std::endl;
  if (!o.timing_json.empty()) {
    dio::JsonReport j;
    j.num("num_labels", num_labels).num("npts_per_label_min", lmin).num("npts_per_label_mean", mean)
        .num("npts_per_label_max", lmax).num("total_label_memberships", st.memberships)
        .num("processed_label_memberships", st.memberships).num("remap_invalid_local_ids", st.remap_invalid_local_ids)
        .num("remap_self_loops", st.remap_self_loops).num("remap_duplicate_edges", st.remap_duplicate_edges)
        .num("label_data_materialization_seconds", st.materialize_seconds)
        .num("per_label_gpu_build_sum_seconds", st.build_sum_seconds)
        .num("per_label_gpu_build_max_seconds", st.build_max_seconds)
        .num("local_to_global_remap_seconds", st.remap_seconds).num("write_index_seconds", write_index_s)
        .num("final_prune_seconds", 0).num("metadata_seconds", metadata_s).num("total_seconds", total_s)
        .num("peak_gpu_mem_gb", st.peak_gpu_mem_gb).num("output_edges", gs.edges);
    dio::write_text(o.timing_json, j.text());
  }
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    const Opts o = read_opts(argc, argv);
    if (o.data_type == "uint8") return run<uint8_t>(o);
    if (o.data_type == "float") return run<float>(o);
    std::cerr << "GPU StitchedMVP supports uint8 and float in this version" << std::endl;
    return 2;
  } catch (const std::exception& e) {
    std::cerr << "[GPU stitched] failed: " << e.what() << std::endl;
    return 1;
  }
}
