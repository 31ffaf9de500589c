// tq.cpp -- the .tq container of quantized bases (host side).
//
// Layout (tier.cpp:273-292 reads it, tier.cpp:2716-2744 and quant.py:60-105
// write it): a text header of hb bytes, NUL padded, then the matrices.
//   line 1            "TQB1 <hb> <n>"
//   meta lines        "#<key> <value>"
//   one line each     "<name> <type> <rows> <cols> <offset> <bytes> [err]"
// hb = ceil((n*200 + 4096) / 4096) * 4096; matrix data starts at hb, each
// matrix at a 4096-aligned offset, its rows of q_row_bytes(type, cols) bytes
// back to back.  A reader accepts 64 <= hb <= 64 MiB, skips empty and '#'
// lines, and rejects an unknown type, columns that are not whole blocks, or a
// byte count other than rows * q_row_bytes.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cinttypes>
#include <cstdio>
#include <cstring>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "tm_host.h"

using namespace tiermm;

struct tiermm_tq {
  struct Mat {
    std::string name;
    int qtype, rows, cols;
    uint64_t offset, bytes;
    size_t rb;
    double err;  // -1 when the file gives none
  };
  std::string path;
  std::vector<Mat> mats;
  std::map<std::string, int> index;
  std::vector<std::pair<std::string, std::string>> meta;
};

namespace {

const BlockInfo* info_by_name(const char* name) {
  for (int t = 0; t < 256; ++t) {
    const BlockInfo* b = block_info(t);
    if (b && !std::strcmp(b->name, name)) return b;
  }
  return nullptr;
}

bool pread_all(int fd, void* dst, size_t n, uint64_t off) {
  uint8_t* p = (uint8_t*)dst;
  while (n) {
    const ssize_t r = pread(fd, p, n, (off_t)off);
    if (r <= 0) return false;
    p += r;
    n -= (size_t)r;
    off += (uint64_t)r;
  }
  return true;
}

bool pwrite_all(int fd, const void* src, size_t n, uint64_t off) {
  const uint8_t* p = (const uint8_t*)src;
  while (n) {
    const ssize_t r = pwrite(fd, p, n, (off_t)off);
    if (r <= 0) return false;
    p += r;
    n -= (size_t)r;
    off += (uint64_t)r;
  }
  return true;
}

}  // namespace

extern "C" {

int tiermm_tq_open(const char* path, tiermm_tq** out) {
  if (!path || !out) return set_error(TIERMM_EINVAL, "tiermm_tq_open: null argument");
  *out = nullptr;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return set_error(TIERMM_EINVAL, "tiermm_tq_open: %s: %s", path, std::strerror(errno));
  char first[128] = {0};
  const ssize_t got = pread(fd, first, sizeof first - 1, 0);
  size_t hb = 0, n = 0;
  if (got < 8 || std::sscanf(first, "TQB1 %zu %zu", &hb, &n) != 2 || hb < 64 || hb > (64ull << 20)) {
    close(fd);
    return set_error(TIERMM_EINVAL, "tiermm_tq_open: %s is not a .tq file", path);
  }
  std::string h(hb, '\0');
  const bool ok = pread_all(fd, &h[0], hb, 0);
  close(fd);
  if (!ok) return set_error(TIERMM_EINVAL, "tiermm_tq_open: %s: header shorter than %zu bytes", path, hb);
  h.resize(std::strlen(h.c_str()));
  auto* tq = new tiermm_tq;
  tq->path = path;
  std::istringstream is(h);
  std::string line;
  std::getline(is, line);  // the TQB1 line
  while (std::getline(is, line)) {
    if (line.empty()) continue;
    if (line[0] == '#') {
      const size_t sp = line.find(' ');
      tq->meta.emplace_back(line.substr(1, sp == std::string::npos ? std::string::npos : sp - 1),
                            sp == std::string::npos ? std::string() : line.substr(sp + 1));
      continue;
    }
    char nm[256], ty[32];
    int rows, cols;
    unsigned long long off, sz;
    double err = -1.0;
    const int f = std::sscanf(line.c_str(), "%255s %31s %d %d %llu %llu %lf", nm, ty, &rows, &cols, &off, &sz, &err);
    if (f < 6) continue;
    if (f < 7) err = -1.0;
    const BlockInfo* b = info_by_name(ty);
    if (!b || rows < 0 || cols <= 0 || cols % b->elems ||
        (uint64_t)(cols / b->elems) * b->bytes * (uint64_t)rows != sz) {
      delete tq;
      return set_error(TIERMM_EINVAL, "tiermm_tq_open: %s: matrix %s of type %s does not parse", path, nm, ty);
    }
    tiermm_tq::Mat m{nm, b->type, rows, cols, off, sz, (size_t)(cols / b->elems) * b->bytes, err};
    auto it = tq->index.find(m.name);
    if (it != tq->index.end()) {
      tq->mats[it->second] = m;  // a repeated name replaces the earlier line, as the reference's map does
    } else {
      tq->index[m.name] = (int)tq->mats.size();
      tq->mats.push_back(m);
    }
  }
  if (tq->mats.empty()) {
    delete tq;
    return set_error(TIERMM_EINVAL, "tiermm_tq_open: %s holds no matrices", path);
  }
  *out = tq;
  return TIERMM_OK;
}

void tiermm_tq_close(tiermm_tq* tq) { delete tq; }

int tiermm_tq_count(const tiermm_tq* tq) { return tq ? (int)tq->mats.size() : 0; }

int tiermm_tq_find(const tiermm_tq* tq, const char* name) {
  if (!tq || !name) return -1;
  auto it = tq->index.find(name);
  return it == tq->index.end() ? -1 : it->second;
}

int tiermm_tq_info(const tiermm_tq* tq, int i, const char** name, int* qtype, int* rows, int* cols,
                   uint64_t* offset, uint64_t* bytes, size_t* rb, double* err) {
  if (!tq || i < 0 || i >= (int)tq->mats.size()) return set_error(TIERMM_EINVAL, "tiermm_tq_info: index %d", i);
  const auto& m = tq->mats[i];
  if (name) *name = m.name.c_str();
  if (qtype) *qtype = m.qtype;
  if (rows) *rows = m.rows;
  if (cols) *cols = m.cols;
  if (offset) *offset = m.offset;
  if (bytes) *bytes = m.bytes;
  if (rb) *rb = m.rb;
  if (err) *err = m.err;
  return TIERMM_OK;
}

int tiermm_tq_meta_count(const tiermm_tq* tq) { return tq ? (int)tq->meta.size() : 0; }

int tiermm_tq_meta(const tiermm_tq* tq, int i, const char** key, const char** value) {
  if (!tq || i < 0 || i >= (int)tq->meta.size()) return set_error(TIERMM_EINVAL, "tiermm_tq_meta: index %d", i);
  if (key) *key = tq->meta[i].first.c_str();
  if (value) *value = tq->meta[i].second.c_str();
  return TIERMM_OK;
}

int tiermm_tq_read_rows(const tiermm_tq* tq, int i, size_t r0, size_t nrows, void* dst) {
  if (!tq || i < 0 || i >= (int)tq->mats.size()) return set_error(TIERMM_EINVAL, "tiermm_tq_read_rows: index %d", i);
  const auto& m = tq->mats[i];
  if (r0 > (size_t)m.rows || nrows > (size_t)m.rows - r0)
    return set_error(TIERMM_EINVAL, "tiermm_tq_read_rows: rows [%zu, %zu) of %d", r0, r0 + nrows, m.rows);
  if (nrows == 0) return TIERMM_OK;
  if (!dst) return set_error(TIERMM_EINVAL, "tiermm_tq_read_rows: null destination");
  const int fd = open(tq->path.c_str(), O_RDONLY);
  if (fd < 0) return set_error(TIERMM_EINVAL, "tiermm_tq_read_rows: %s: %s", tq->path.c_str(), std::strerror(errno));
  const bool ok = pread_all(fd, dst, nrows * m.rb, m.offset + (uint64_t)r0 * m.rb);
  close(fd);
  if (!ok) return set_error(TIERMM_EINVAL, "tiermm_tq_read_rows: %s: short read of %s", tq->path.c_str(), m.name.c_str());
  return TIERMM_OK;
}

int tiermm_tq_write(const char* path, int n, const char* const* names, const int* qtypes, const int* rows,
                    const int* cols, const void* const* data, const double* errs, int nmeta,
                    const char* const* keys, const char* const* values) {
  if (!path || n <= 0 || !names || !qtypes || !rows || !cols || !data || (nmeta > 0 && (!keys || !values)))
    return set_error(TIERMM_EINVAL, "tiermm_tq_write: null argument or no matrices");
  const uint64_t hb = ((uint64_t)n * 200 + 4096 + 4095) / 4096 * 4096;
  std::vector<uint64_t> off(n), size(n);
  uint64_t end = hb;
  for (int i = 0; i < n; ++i) {
    const BlockInfo* b = block_info(qtypes[i]);
    if (!b || rows[i] < 0 || cols[i] <= 0 || cols[i] % b->elems || !names[i] || !*names[i] ||
        std::strpbrk(names[i], " \t\n"))
      return set_error(TIERMM_EINVAL, "tiermm_tq_write: matrix %d (%s) has a bad name, type or shape", i,
                       names[i] ? names[i] : "?");
    size[i] = (uint64_t)(cols[i] / b->elems) * b->bytes * (uint64_t)rows[i];
    off[i] = end;
    end += (size[i] + 4095) / 4096 * 4096;
  }
  std::string h = "TQB1 " + std::to_string(hb) + " " + std::to_string(n) + "\n";
  for (int j = 0; j < nmeta; ++j) h += std::string("#") + keys[j] + " " + values[j] + "\n";
  char line[512];
  for (int i = 0; i < n; ++i) {
    char e[32];
    if (errs) std::snprintf(e, sizeof e, "%.6f", errs[i]);
    else std::snprintf(e, sizeof e, "-1");
    std::snprintf(line, sizeof line, "%s %s %d %d %" PRIu64 " %" PRIu64 " %s\n", names[i], block_info(qtypes[i])->name,
                  rows[i], cols[i], off[i], size[i], e);
    h += line;
  }
  if (h.size() >= hb) return set_error(TIERMM_EINVAL, "tiermm_tq_write: header of %zu bytes does not fit", h.size());
  h.resize(hb, '\0');
  const std::string tmp = std::string(path) + ".part";
  const int fd = open(tmp.c_str(), O_RDWR | O_CREAT | O_TRUNC, 0644);
  if (fd < 0) return set_error(TIERMM_EINVAL, "tiermm_tq_write: %s: %s", tmp.c_str(), std::strerror(errno));
  bool ok = ftruncate(fd, (off_t)end) == 0;
  for (int i = 0; ok && i < n; ++i) ok = size[i] == 0 || pwrite_all(fd, data[i], size[i], off[i]);
  ok = ok && pwrite_all(fd, h.data(), hb, 0) && fsync(fd) == 0;
  close(fd);
  if (!ok || std::rename(tmp.c_str(), path) != 0) {
    std::remove(tmp.c_str());
    return set_error(TIERMM_EINVAL, "tiermm_tq_write: writing %s failed", path);
  }
  return TIERMM_OK;
}

}  // extern "C"
