// DiskANN file formats and command-line plumbing shared by the apps
// (gpu_vamana_memory_index, gpu_stitched_vamana_index, build_memory_index,
// build_sharded_index).
//
// Formats (DiskANN's, as the reference apps read and write them):
//   .bin matrix   u32 rows, u32 dim, then rows x dim elements, row-major
//   graph file    u64 file bytes, u32 max degree, u32 start, u64 frozen
//                 points, then per row: u32 degree, degree x u32 ids
//   label sidecars (text): <prefix>_labels.txt, _label_formatted.txt,
//                 _labels_map.txt, _labels_to_medoids.txt,
//                 _universal_label.txt
#pragma once

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <limits>
#include <map>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace dio {

constexpr uint32_t kNone = 0xFFFFFFFFu;

// ---------------------------------------------------------------------------
// Command line: a table of options, each with a setter. Values are parsed
// strictly (decimal digits only for integers).
// ---------------------------------------------------------------------------
// How a command line spells its options and errors.
struct ArgStyle {
  bool equals_form = false;  // also accept "--name=value"
  std::function<std::string(const std::string&)> unknown = [](const std::string& k) {
    return "unknown argument: " + k;
  };
  std::function<std::string(const std::string&)> missing = [](const std::string& k) {
    return "missing value for " + k;
  };
};

class ArgTable {
 public:
  using Setter = std::function<void(const std::string& value, const std::string& key)>;

  void value(std::initializer_list<const char*> names, Setter set) {
    const size_t id = setters_.size();
    setters_.push_back(std::move(set));
    for (const char* n : names) index_[n] = {id, true};
  }
  void flag(std::initializer_list<const char*> names, bool* target) {
    const size_t id = setters_.size();
    setters_.push_back([target](const std::string&, const std::string&) { *target = true; });
    for (const char* n : names) index_[n] = {id, false};
  }
  // Returns the keys seen, in order.
  std::vector<std::string> parse(int argc, char** argv, const ArgStyle& style = ArgStyle()) const {
    std::vector<std::string> seen;
    for (int i = 1; i < argc; ++i) {
      std::string key = argv[i], v;
      bool inline_value = false;
      const size_t eq = key.find('=');
      if (style.equals_form && key.rfind("--", 0) == 0 && eq != std::string::npos) {
        v = key.substr(eq + 1);
        key = key.substr(0, eq);
        inline_value = true;
      }
      const auto it = index_.find(key);
      if (it == index_.end()) throw std::runtime_error(style.unknown(key));
      if (it->second.second && !inline_value) {
        if (i + 1 >= argc) throw std::runtime_error(style.missing(key));
        v = argv[++i];
      }
      setters_[it->second.first](v, key);
      seen.push_back(key);
    }
    return seen;
  }

 private:
  std::vector<Setter> setters_;
  std::map<std::string, std::pair<size_t, bool>> index_;  // name -> (setter, takes a value)
};

inline uint64_t parse_u64(const std::string& text, const std::string& key) {
  const bool digits = !text.empty() && text.find_first_not_of("0123456789") == std::string::npos;
  errno = 0;
  char* end = nullptr;
  const unsigned long long v = digits ? std::strtoull(text.c_str(), &end, 10) : 0;
  if (!digits || errno == ERANGE || end != text.c_str() + text.size())
    throw std::runtime_error(key + " must be an unsigned integer");
  return (uint64_t)v;
}

// allow_zero false: the value must be in [1, UINT32_MAX].
inline uint32_t parse_u32(const std::string& text, const std::string& key, bool allow_zero) {
  const uint64_t v = parse_u64(text, key);
  if (v > std::numeric_limits<uint32_t>::max())
    throw std::runtime_error(key + (allow_zero ? " is out of uint32 range" : " must be in [1, UINT32_MAX]"));
  if (!allow_zero && v == 0) throw std::runtime_error(key + " must be in [1, UINT32_MAX]");
  return (uint32_t)v;
}

inline float parse_positive_float(const std::string& text, const std::string& key) {
  char* end = nullptr;
  const float v = std::strtof(text.c_str(), &end);
  if (text.empty() || end != text.c_str() + text.size() || !(v > 0.0f))
    throw std::runtime_error(key + " must be a positive number");
  return v;
}

// ---------------------------------------------------------------------------
// Files: a small RAII descriptor with full-length pread / write loops.
// ---------------------------------------------------------------------------
class File {
 public:
  File(const std::string& path, int flags, mode_t mode = 0644) : path_(path), fd_(::open(path.c_str(), flags, mode)) {}
  ~File() {
    if (fd_ >= 0) ::close(fd_);
  }
  File(const File&) = delete;
  File& operator=(const File&) = delete;
  bool ok() const { return fd_ >= 0; }
  const std::string& path() const { return path_; }

  uint64_t size() const {
    struct stat st;
    if (::fstat(fd_, &st) != 0) throw std::runtime_error("failed to stat " + path_);
    return (uint64_t)st.st_size;
  }
  void read_at(void* dst, uint64_t bytes, uint64_t offset) const {
    char* p = static_cast<char*>(dst);
    while (bytes > 0) {
      const ssize_t r = ::pread(fd_, p, (size_t)std::min<uint64_t>(bytes, 1ull << 30), (off_t)offset);
      if (r <= 0) throw std::runtime_error("failed to read " + path_);
      p += r;
      bytes -= (uint64_t)r;
      offset += (uint64_t)r;
    }
  }
  void append(const void* src, uint64_t bytes) {
    const char* p = static_cast<const char*>(src);
    while (bytes > 0) {
      const ssize_t w = ::write(fd_, p, (size_t)std::min<uint64_t>(bytes, 1ull << 30));
      if (w <= 0) throw std::runtime_error("failed to write " + path_);
      p += w;
      bytes -= (uint64_t)w;
    }
  }
  void close_checked() {
    if (fd_ >= 0 && ::close(fd_) != 0) {
      fd_ = -1;
      throw std::runtime_error("failed to close " + path_);
    }
    fd_ = -1;
  }

 private:
  std::string path_;
  int fd_;
};

inline bool exists(const std::string& path) {
  struct stat st;
  return ::stat(path.c_str(), &st) == 0;
}

// ---------------------------------------------------------------------------
// .bin matrices
// ---------------------------------------------------------------------------
struct MatrixShape {
  uint64_t rows = 0;  // rows in the file
  uint32_t dim = 0;
};

// Reads the header and requires the file to be exactly 8 + rows*dim*elem bytes.
inline MatrixShape bin_shape(const File& f, size_t elem) {
  uint32_t hdr[2] = {0, 0};
  if (f.size() < 8) throw std::runtime_error("failed to read DiskANN matrix header");
  f.read_at(hdr, 8, 0);
  MatrixShape s{hdr[0], hdr[1]};
  if (s.dim == 0 || s.rows > (std::numeric_limits<uint64_t>::max() - 8) / ((uint64_t)s.dim * elem))
    throw std::runtime_error("DiskANN matrix shape overflows its byte-size calculation");
  if (f.size() != 8 + s.rows * s.dim * elem)
    throw std::runtime_error("DiskANN matrix header does not match exact file size");
  return s;
}

// Rows [first, first + count) of a .bin matrix of T.
template <typename T>
std::vector<T> read_bin_rows(const File& f, const MatrixShape& s, uint64_t first, uint64_t count) {
  std::vector<T> out((size_t)(count * s.dim));
  f.read_at(out.data(), out.size() * sizeof(T), 8 + first * s.dim * sizeof(T));
  return out;
}

template <typename T>
std::vector<T> read_bin(const std::string& path, uint32_t& rows, uint32_t& dim) {
  File f(path, O_RDONLY);
  if (!f.ok()) throw std::runtime_error("failed to open " + path);
  const MatrixShape s = bin_shape(f, sizeof(T));
  if (s.rows == 0 || s.rows > std::numeric_limits<uint32_t>::max())
    throw std::runtime_error("matrix of " + path + " has no rows or too many");
  rows = (uint32_t)s.rows;
  dim = s.dim;
  return read_bin_rows<T>(f, s, 0, s.rows);
}

template <typename T>
void write_bin(File& out, uint32_t rows, uint32_t dim, const T* data) {
  const uint32_t hdr[2] = {rows, dim};
  out.append(hdr, 8);
  out.append(data, (uint64_t)rows * dim * sizeof(T));
}

// ---------------------------------------------------------------------------
// Graph files
// ---------------------------------------------------------------------------
struct GraphSummary {
  uint64_t bytes = 0, edges = 0;
  uint32_t max_degree = 0;
};

// Row source: for row i, fills `row` with its neighbour list.
using RowFn = std::function<void(uint32_t i, std::vector<uint32_t>& row)>;

inline GraphSummary graph_summary(uint32_t n, const RowFn& rows) {
  GraphSummary s;
  s.bytes = 24;
  std::vector<uint32_t> r;
  for (uint32_t i = 0; i < n; ++i) {
    r.clear();
    rows(i, r);
    s.bytes += 4 + 4ull * r.size();
    s.edges += r.size();
    s.max_degree = std::max<uint32_t>(s.max_degree, (uint32_t)r.size());
  }
  return s;
}

// Writes the graph file; the header's byte count and max degree come from a
// first pass over the rows. Rows are written in batches.
inline GraphSummary write_graph(File& out, uint32_t n, uint32_t start, const RowFn& rows) {
  const GraphSummary s = graph_summary(n, rows);
  const uint64_t frozen = 0;
  out.append(&s.bytes, 8);
  out.append(&s.max_degree, 4);
  out.append(&start, 4);
  out.append(&frozen, 8);
  std::vector<uint32_t> buf, r;
  buf.reserve(1 << 20);
  for (uint32_t i = 0; i < n; ++i) {
    r.clear();
    rows(i, r);
    buf.push_back((uint32_t)r.size());
    buf.insert(buf.end(), r.begin(), r.end());
    if (buf.size() >= (1u << 20)) {
      out.append(buf.data(), 4ull * buf.size());
      buf.clear();
    }
  }
  out.append(buf.data(), 4ull * buf.size());
  return s;
}

// Rows of a padded N x stride graph with per-row degrees, cut at `cap`.
inline RowFn padded_rows(const uint32_t* graph, const uint32_t* degree, uint32_t stride, uint32_t cap) {
  return [=](uint32_t i, std::vector<uint32_t>& row) {
    const uint32_t k = std::min(degree[i], cap);
    row.assign(graph + (size_t)i * stride, graph + (size_t)i * stride + k);
  };
}

// ---------------------------------------------------------------------------
// Publishing: outputs are written to temporaries, checked for their expected
// sizes, then renamed into place; any failure removes what was written.
// ---------------------------------------------------------------------------
class Publisher {
 public:
  struct Item {
    std::string final_path, temp_path;
    uint64_t expect_bytes;
  };
  ~Publisher() {
    if (!done_)
      for (const Item& it : items_) std::remove(it.temp_path.c_str());
  }
  // Opens the temporary of `final_path` for writing.
  File& open(const std::string& final_path) {
    items_.push_back({final_path, final_path + ".tmp", 0});
    files_.emplace_back(new File(items_.back().temp_path, O_WRONLY | O_CREAT | O_TRUNC));
    if (!files_.back()->ok()) throw std::runtime_error("failed to create temporary output " + items_.back().temp_path);
    return *files_.back();
  }
  void expect(uint64_t bytes) { items_.back().expect_bytes = bytes; }
  // Closes, checks the sizes, renames in order (last opened first).
  void commit(const std::string& what) {
    for (auto& f : files_) f->close_checked();
    for (const Item& it : items_) {
      struct stat st;
      if (::stat(it.temp_path.c_str(), &st) != 0 || (uint64_t)st.st_size != it.expect_bytes)
        throw std::runtime_error("serialized temporary output size does not match its " + what + " layout");
    }
    for (size_t k = items_.size(); k-- > 0;) {
      if (std::rename(items_[k].temp_path.c_str(), items_[k].final_path.c_str()) != 0) {
        for (size_t j = k + 1; j < items_.size(); ++j) std::remove(items_[j].final_path.c_str());
        throw std::runtime_error("failed to publish output " + items_[k].final_path);
      }
    }
    done_ = true;
  }

 private:
  std::vector<Item> items_;
  std::vector<std::unique_ptr<File>> files_;
  bool done_ = false;
};

inline void write_text(const std::string& path, const std::string& body) {
  File f(path, O_WRONLY | O_CREAT | O_TRUNC);
  if (!f.ok()) throw std::runtime_error("failed to write " + path);
  f.append(body.data(), body.size());
  f.close_checked();
}

inline void copy_file(const std::string& src, const std::string& dst) {
  File in(src, O_RDONLY);
  if (!in.ok()) throw std::runtime_error("failed to open " + src);
  File out(dst, O_WRONLY | O_CREAT | O_TRUNC);
  if (!out.ok()) throw std::runtime_error("failed to write " + dst);
  const uint64_t total = in.size();
  std::vector<char> buf(std::min<uint64_t>(total, 64ull << 20));
  for (uint64_t off = 0; off < total;) {
    const uint64_t k = std::min<uint64_t>(buf.size(), total - off);
    in.read_at(buf.data(), k, off);
    out.append(buf.data(), k);
    off += k;
  }
  out.close_checked();
}

// ---------------------------------------------------------------------------
// JSON report: keys in insertion order, one per line.
// ---------------------------------------------------------------------------
inline std::string json_quote(const std::string& s) {
  static const char* hex = "0123456789abcdef";
  std::string out = "\"";
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
        if (c < 0x20) {
          out += "\\u00";
          out += hex[c >> 4];
          out += hex[c & 15];
        } else {
          out.push_back((char)c);
        }
    }
  }
  return out + "\"";
}

class JsonReport {
 public:
  template <typename V>
  JsonReport& num(const std::string& key, V v) {
    std::ostringstream s;
    s << v;
    fields_.emplace_back(key, s.str());
    return *this;
  }
  JsonReport& str(const std::string& key, const std::string& v) {
    fields_.emplace_back(key, json_quote(v));
    return *this;
  }
  JsonReport& boolean(const std::string& key, bool v) {
    fields_.emplace_back(key, v ? "true" : "false");
    return *this;
  }
  std::string text() const {
    std::string out = "{\n";
    for (size_t i = 0; i < fields_.size(); ++i)
      out += "  " + json_quote(fields_[i].first) + ": " + fields_[i].second + (i + 1 < fields_.size() ? ",\n" : "\n");
    return out + "}\n";
  }

 private:
  std::vector<std::pair<std::string, std::string>> fields_;
};

// ---------------------------------------------------------------------------
// Label files: one row per point, comma-separated label names.
// ---------------------------------------------------------------------------
struct LabelRows {
  std::vector<std::string> names;            // id -> name; ids follow first appearance
  std::vector<std::vector<uint32_t>> rows;   // per point: ids in file order
  uint32_t first_id = 1;                     // id of the first named label
  uint32_t universal = kNone;                // id of the universal label (0) when one is named
};

struct LabelParse {
  std::string universal;        // name of the universal label ("" = none)
  std::string universal_error;  // non-empty: the universal label may not appear in a row (message)
  bool drop_repeats;            // keep the first occurrence of a name within a row
  bool strip_spaces;            // remove ' ' as well as '\r' from each line
};

// Names are numbered 1, 2, ... in order of first appearance; a universal
// label, when named and allowed, is id 0.
inline LabelRows read_labels(const std::string& path, const LabelParse& how) {
  File f(path, O_RDONLY);
  if (!f.ok()) throw std::runtime_error("failed to open label file: " + path);
  std::string text((size_t)f.size(), '\0');
  f.read_at(&text[0], text.size(), 0);
  LabelRows out;
  std::unordered_map<std::string, uint32_t> id_of;
  out.names.push_back(how.universal);  // slot 0: the universal label, or unused
  if (!how.universal.empty() && how.universal_error.empty()) {
    id_of.emplace(how.universal, 0u);
    out.universal = 0;
  }
  size_t pos = 0;
  while (pos < text.size()) {
    size_t eol = text.find('\n', pos);
    if (eol == std::string::npos) eol = text.size();
    std::string line = text.substr(pos, eol - pos);
    pos = eol + 1;
    line.erase(std::remove_if(line.begin(), line.end(),
                              [&](char c) { return c == '\r' || (how.strip_spaces && c == ' '); }),
               line.end());
    const std::string where = "label row " + std::to_string(out.rows.size());
    if (line.empty()) throw std::runtime_error("empty label row is not supported (" + where + " is empty)");
    if (line.back() == ',') throw std::runtime_error("empty label token is not supported (" + where + ")");
    std::vector<uint32_t> row;
    size_t a = 0;
    while (true) {
      const size_t b = line.find(',', a);
      const std::string name = line.substr(a, b == std::string::npos ? std::string::npos : b - a);
      if (name.empty()) throw std::runtime_error("empty label token is not supported (" + where + ")");
      if (!how.universal_error.empty() && !how.universal.empty() && name == how.universal)
        throw std::runtime_error(how.universal_error);
      auto it = id_of.find(name);
      if (it == id_of.end()) {
        it = id_of.emplace(name, (uint32_t)out.names.size()).first;
        out.names.push_back(name);
      }
      if (!how.drop_repeats || std::find(row.begin(), row.end(), it->second) == row.end()) row.push_back(it->second);
      if (b == std::string::npos) break;
      a = b + 1;
    }
    out.rows.push_back(std::move(row));
  }
  return out;
}

// Sorted unique ids per row in CSR form (the canonical label CSR).
inline void canonical_csr(const LabelRows& lr, std::vector<uint32_t>& offsets, std::vector<uint32_t>& ids) {
  offsets.assign(lr.rows.size() + 1, 0);
  ids.clear();
  for (size_t i = 0; i < lr.rows.size(); ++i) {
    std::vector<uint32_t> r = lr.rows[i];
    std::sort(r.begin(), r.end());
    r.erase(std::unique(r.begin(), r.end()), r.end());
    offsets[i] = (uint32_t)ids.size();
    ids.insert(ids.end(), r.begin(), r.end());
  }
  offsets[lr.rows.size()] = (uint32_t)ids.size();
}

// label -> points (ascending point ids) for labels [0, num_labels).
inline void postings(const std::vector<uint32_t>& offsets, const std::vector<uint32_t>& ids, uint32_t num_labels,
                     std::vector<uint32_t>& loff, std::vector<uint32_t>& pts) {
  loff.assign(num_labels + 1, 0);
  for (uint32_t l : ids)
    if (l < num_labels) ++loff[l + 1];
  for (uint32_t l = 0; l < num_labels; ++l) loff[l + 1] += loff[l];
  pts.assign(loff[num_labels], 0);
  std::vector<uint32_t> cur(loff.begin(), loff.end() - 1);
  for (size_t i = 0; i + 1 < offsets.size(); ++i)
    for (uint32_t p = offsets[i]; p < offsets[i + 1]; ++p)
      if (ids[p] < num_labels) pts[cur[ids[p]]++] = (uint32_t)i;
}

// Comma-joined rows of ids, one line per row.
inline std::string id_rows_text(size_t n, const std::function<void(size_t, std::vector<uint32_t>&)>& row_of) {
  std::string out;
  std::vector<uint32_t> r;
  for (size_t i = 0; i < n; ++i) {
    r.clear();
    row_of(i, r);
    for (size_t j = 0; j < r.size(); ++j) {
      if (j) out.push_back(',');
      out += std::to_string(r[j]);
    }
    out.push_back('\n');
  }
  return out;
}

}  // namespace dio
