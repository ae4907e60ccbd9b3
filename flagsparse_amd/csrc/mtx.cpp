// Matrix Market coordinate reader (host code): the on-disk format the reference's SuiteSparse
// test drivers load (tests/test_spmv.py:29-103, tests/test_spmm_coo.py:156-249,
// tests/test_spmv_coo.py:257-305).  It returns the raw entries; expansion of symmetric /
// skew-symmetric / hermitian storage, pattern values and duplicate summation are done by the
// caller (flagsparse_amd/mtx.py), as the reference's loaders do after parsing.
//
// The whole file is read into memory and scanned once with a hand-written tokenizer (no
// per-line allocation), so a SuiteSparse file of tens of millions of entries loads at disk
// speed rather than at Python-parsing speed.
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "fsp_internal.hpp"

namespace fsp {
namespace {

struct Cursor {
  const char* p;
  const char* end;
};

bool at_eol(const Cursor& c) { return c.p >= c.end || *c.p == '\n' || *c.p == '\r'; }

void skip_blanks(Cursor& c) {
  while (c.p < c.end && (*c.p == ' ' || *c.p == '\t')) ++c.p;
}

void next_line(Cursor& c) {
  while (c.p < c.end && *c.p != '\n') ++c.p;
  if (c.p < c.end) ++c.p;
}

// One whitespace-separated token of the current line as [b, e); false at end of line.
bool token(Cursor& c, const char** b, const char** e) {
  skip_blanks(c);
  if (at_eol(c)) return false;
  *b = c.p;
  while (c.p < c.end && *c.p != ' ' && *c.p != '\t' && *c.p != '\n' && *c.p != '\r') ++c.p;
  *e = c.p;
  return true;
}

std::string lower(const char* b, const char* e) {
  std::string s(b, e);
  for (auto& ch : s) ch = (char)((ch >= 'A' && ch <= 'Z') ? ch - 'A' + 'a' : ch);
  return s;
}

bool parse_i64(const char* b, const char* e, int64_t* out) {
  std::string s(b, e);
  char* endp = nullptr;
  errno = 0;
  const long long v = std::strtoll(s.c_str(), &endp, 10);
  if (errno || endp != s.c_str() + s.size()) return false;
  *out = v;
  return true;
}

bool parse_f64(const char* b, const char* e, double* out) {
  char buf[64];
  const size_t n = (size_t)(e - b);
  if (n == 0 || n >= sizeof(buf)) return false;
  std::memcpy(buf, b, n);
  buf[n] = '\0';
  char* endp = nullptr;
  *out = std::strtod(buf, &endp);
  return endp == buf + n;
}

}  // namespace
}  // namespace fsp

using namespace fsp;

// info[0..7): n_rows, n_cols, nnz (header), field (0 real/integer/double, 1 pattern,
// 2 complex), symmetry (0 general, 1 symmetric, 2 skew-symmetric, 3 hermitian), entries read,
// entries read without a value (stored as 0; pattern files need none).
extern "C" int fsp_mtx_read(const char* path, int64_t* info, int64_t* rows, int64_t* cols,
                            double* vals, int64_t capacity) {
  if (!path || !info) return set_error(FSP_EINVAL, "fsp_mtx_read: null path or info");
  if (rows && (!cols || !vals || capacity < 0))
    return set_error(FSP_EINVAL, "fsp_mtx_read: rows given without cols/vals/capacity");
  FILE* f = std::fopen(path, "rb");
  if (!f) return set_error(FSP_EINVAL, std::string("fsp_mtx_read: cannot open ") + path);
  std::vector<char> buf;
  {
    char chunk[1 << 16];
    size_t n;
    while ((n = std::fread(chunk, 1, sizeof(chunk), f)) > 0) buf.insert(buf.end(), chunk, chunk + n);
  }
  std::fclose(f);
  Cursor c{buf.data(), buf.data() + buf.size()};
  int64_t field = 0, symmetry = 0;
  bool have_size = false;
  int64_t n_rows = 0, n_cols = 0, nnz = 0, n_read = 0, n_missing = 0;
  while (c.p < c.end) {
    skip_blanks(c);
    if (at_eol(c)) {  // blank line
      next_line(c);
      continue;
    }
    if (*c.p == '%') {
      // "%%MatrixMarket matrix coordinate <field> <symmetry>" (case-insensitive)
      if (c.end - c.p >= 14 && std::strncmp(c.p, "%%MatrixMarket", 14) == 0) {
        const char *b, *e;
        std::vector<std::string> t;
        while (token(c, &b, &e)) t.push_back(lower(b, e));
        if (t.size() >= 3 && t[2] == "array")
          return set_error(FSP_ENOTSUP, "fsp_mtx_read: dense 'array' files are not supported");
        if (t.size() >= 5) {
          field = t[3] == "pattern" ? 1 : t[3] == "complex" ? 2 : 0;
          symmetry = t[4] == "symmetric" ? 1 : t[4] == "skew-symmetric" ? 2
                     : t[4] == "hermitian" ? 3 : 0;
        }
      }
      next_line(c);
      continue;
    }
    const char *b, *e;
    if (!have_size) {
      int64_t v[3] = {0, 0, 0};
      int k = 0;
      while (k < 3 && token(c, &b, &e)) {
        if (!parse_i64(b, e, &v[k]))
          return set_error(FSP_EINVAL, "fsp_mtx_read: cannot parse the size line");
        ++k;
      }
      if (k < 2) return set_error(FSP_EINVAL, "fsp_mtx_read: cannot parse the size line");
      n_rows = v[0];
      n_cols = v[1];
      nnz = v[2];
      have_size = true;
      next_line(c);
      if (!rows) break;  // header only
      continue;
    }
    if (n_read >= nnz || n_read >= capacity) break;  // only the first nnz entry lines count
    int64_t r = 0, col = 0;
    double vr = 0.0, vi = 0.0;
    int k = 0;
    bool ok = true;
    while (token(c, &b, &e)) {
      if (k == 0) ok = ok && parse_i64(b, e, &r);
      else if (k == 1) ok = ok && parse_i64(b, e, &col);
      else if (k == 2) ok = ok && parse_f64(b, e, &vr);
      else if (k == 3) ok = ok && parse_f64(b, e, &vi);
      ++k;
    }
    if (!ok) return set_error(FSP_EINVAL, "fsp_mtx_read: cannot parse an entry line");
    if (k >= 2) {  // a line with fewer than two tokens is skipped, as the reference does
      rows[n_read] = r - 1;
      cols[n_read] = col - 1;
      if (field == 2) {
        vals[2 * n_read] = vr;
        vals[2 * n_read + 1] = vi;
      } else {
        vals[n_read] = (k >= 3) ? vr : (field == 1 ? 1.0 : 0.0);
      }
      if (field != 1 && k < (field == 2 ? 4 : 3)) ++n_missing;
      ++n_read;
    }
    next_line(c);
  }
  if (!have_size) return set_error(FSP_EINVAL, "fsp_mtx_read: cannot parse .mtx header");
  info[0] = n_rows;
  info[1] = n_cols;
  info[2] = nnz;
  info[3] = field;
  info[4] = symmetry;
  info[5] = n_read;
  info[6] = n_missing;
  return FSP_OK;
}
