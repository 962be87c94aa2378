// checkpoint.cpp -- loading a Hugging Face Qwen3 checkpoint into a context:
// the safetensors reader (safetensors/safetensors.go, repo.go), the loader's
// per-tensor conversions (weights/weights.go:552-627, weights/convert.go:41-131)
// and the Qwen3 weight map (model/qwen3.go:54-205). The header of a file is
// treated as hostile input and every refusal names the tensor, in the
// reference's words; tensors are converted one at a time so host memory holds
// one plane and its working copies.
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>

#include <algorithm>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../../include/tgohip.h"

namespace tgohip {
int fail(int code, const std::string& msg);
}
using tgohip::fail;

namespace {

// ---------------------------------------------------------------------------
// A small JSON reader: enough of RFC 8259 to parse a safetensors header, an
// index and a config. Integers keep their exact int64 value when they have
// one; depth is bounded, since the text comes from a downloaded file.
// ---------------------------------------------------------------------------
struct JVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  bool is_int = false;  // NUM: integer syntax whose value fits int64
  int64_t i = 0;
  double d = 0;
  std::string s;
  std::vector<JVal> a;
  std::vector<std::pair<std::string, JVal>> o;  // in text order; later keys win
};

struct JParser {
  const char* p;
  const char* e;
  std::string err;
  int depth = 0;

  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
  }
  bool fail_at(const std::string& m) {
    if (err.empty()) err = m;
    return false;
  }
  static void put_utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xC0 | (cp >> 6));
      out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += (char)(0xE0 | (cp >> 12));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    } else {
      out += (char)(0xF0 | (cp >> 18));
      out += (char)(0x80 | ((cp >> 12) & 0x3F));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t& v) {
    if (e - p < 4) return fail_at("truncated \\u escape");
    v = 0;
    for (int k = 0; k < 4; k++) {
      const char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return fail_at("invalid \\u escape");
    }
    return true;
  }
  bool str(std::string& out) {
    if (p >= e || *p != '"') return fail_at("expected a string");
    p++;
    out.clear();
    while (true) {
      if (p >= e) return fail_at("unterminated string");
      const unsigned char c = (unsigned char)*p++;
      if (c == '"') return true;
      if (c < 0x20) return fail_at("control character in string");
      if (c != '\\') {
        out += (char)c;
        continue;
      }
      if (p >= e) return fail_at("unterminated escape");
      const char x = *p++;
      switch (x) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00 && e - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            const char* save = p;
            p += 2;
            uint32_t lo;
            if (!hex4(lo)) return false;
            if (lo >= 0xDC00 && lo < 0xE000) cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            else { p = save; cp = 0xFFFD; }
          } else if (cp >= 0xD800 && cp < 0xE000) {
            cp = 0xFFFD;
          }
          put_utf8(out, cp);
          break;
        }
        default: return fail_at("invalid escape");
      }
    }
  }
  bool num(JVal& v) {
    const char* s0 = p;
    if (p < e && *p == '-') p++;
    if (p >= e || !(*p >= '0' && *p <= '9')) return fail_at("invalid number");
    if (*p == '0') p++;
    else while (p < e && *p >= '0' && *p <= '9') p++;
    bool frac = false;
    if (p < e && *p == '.') {
      frac = true;
      p++;
      if (p >= e || !(*p >= '0' && *p <= '9')) return fail_at("invalid number");
      while (p < e && *p >= '0' && *p <= '9') p++;
    }
    if (p < e && (*p == 'e' || *p == 'E')) {
      frac = true;
      p++;
      if (p < e && (*p == '+' || *p == '-')) p++;
      if (p >= e || !(*p >= '0' && *p <= '9')) return fail_at("invalid number");
      while (p < e && *p >= '0' && *p <= '9') p++;
    }
    const std::string t(s0, p);
    v.kind = JVal::NUM;
    v.d = strtod(t.c_str(), nullptr);
    v.is_int = false;
    if (!frac) {
      // exact int64 or nothing: accumulate with an overflow check
      const bool neg = t[0] == '-';
      uint64_t mag = 0;
      bool ok = true;
      for (size_t k = neg ? 1 : 0; k < t.size(); k++) {
        const uint64_t dgt = (uint64_t)(t[k] - '0');
        if (mag > (UINT64_MAX - dgt) / 10) { ok = false; break; }
        mag = mag * 10 + dgt;
      }
      const uint64_t lim = neg ? (uint64_t)INT64_MAX + 1 : (uint64_t)INT64_MAX;
      if (ok && mag <= lim) {
        v.is_int = true;
        v.i = neg ? (int64_t)(0 - mag) : (int64_t)mag;
      }
    }
    return true;
  }
  bool lit(const char* w, size_t n) {
    if ((size_t)(e - p) < n || memcmp(p, w, n) != 0) return fail_at("invalid literal");
    p += n;
    return true;
  }
  bool val(JVal& v) {
    ws();
    if (p >= e) return fail_at("unexpected end of JSON input");
    if (++depth > 64) return fail_at("nested too deeply");
    bool ok = true;
    const char c = *p;
    if (c == '{') {
      v.kind = JVal::OBJ;
      p++;
      ws();
      if (p < e && *p == '}') {
        p++;
      } else {
        while (ok) {
          ws();
          std::string k;
          if (!str(k)) { ok = false; break; }
          ws();
          if (p >= e || *p != ':') { ok = fail_at("expected ':'"); break; }
          p++;
          JVal x;
          if (!val(x)) { ok = false; break; }
          bool dup = false;
          for (auto& kv : v.o)
            if (kv.first == k) { kv.second = std::move(x); dup = true; break; }
          if (!dup) v.o.emplace_back(std::move(k), std::move(x));
          ws();
          if (p < e && *p == ',') { p++; continue; }
          if (p < e && *p == '}') { p++; break; }
          ok = fail_at("expected ',' or '}'");
        }
      }
    } else if (c == '[') {
      v.kind = JVal::ARR;
      p++;
      ws();
      if (p < e && *p == ']') {
        p++;
      } else {
        while (ok) {
          JVal x;
          if (!val(x)) { ok = false; break; }
          v.a.push_back(std::move(x));
          ws();
          if (p < e && *p == ',') { p++; continue; }
          if (p < e && *p == ']') { p++; break; }
          ok = fail_at("expected ',' or ']'");
        }
      }
    } else if (c == '"') {
      v.kind = JVal::STR;
      ok = str(v.s);
    } else if (c == 't') {
      v.kind = JVal::BOOL;
      v.b = true;
      ok = lit("true", 4);
    } else if (c == 'f') {
      v.kind = JVal::BOOL;
      ok = lit("false", 5);
    } else if (c == 'n') {
      v.kind = JVal::NUL;
      ok = lit("null", 4);
    } else {
      ok = num(v);
    }
    depth--;
    return ok;
  }
};

// Parses a whole document; trailing non-space text is an error.
bool json_parse(const char* s, size_t n, JVal& out, std::string& err) {
  JParser jp{s, s + n, {}};
  if (!jp.val(out)) {
    err = jp.err;
    return false;
  }
  jp.ws();
  if (jp.p != jp.e) {
    err = "invalid character after top-level value";
    return false;
  }
  return true;
}

bool ieq(const std::string& a, const char* b) {
  const size_t n = strlen(b);
  if (a.size() != n) return false;
  for (size_t k = 0; k < n; k++)
    if (tolower((unsigned char)a[k]) != tolower((unsigned char)b[k])) return false;
  return true;
}

std::string shape_str(const std::vector<int64_t>& s) {  // Go's %v of a slice
  std::string r = "[";
  for (size_t k = 0; k < s.size(); k++) r += (k ? " " : "") + std::to_string(s[k]);
  return r + "]";
}

int64_t dtype_size(const std::string& d) {  // safetensors.go:49-53
  static const std::map<std::string, int64_t> m = {{"F64", 8}, {"F32", 4}, {"F16", 2}, {"BF16", 2},
                                                   {"I64", 8}, {"I32", 4}, {"I16", 2}, {"I8", 1},
                                                   {"U8", 1},  {"BOOL", 1}};
  auto it = m.find(d);
  return it == m.end() ? 0 : it->second;
}

}  // namespace

// ---------------------------------------------------------------------------
// safetensors.File (safetensors/safetensors.go:116-263)
// ---------------------------------------------------------------------------
struct StEntry {
  std::string dtype;
  std::vector<int64_t> shape;
  int64_t begin = 0, end = 0;
};

struct tgohip_st {
  std::string path;
  FILE* f = nullptr;
  int64_t data_start = 0, data_len = 0;
  std::map<std::string, StEntry> entries;
  std::vector<std::string> names;  // sorted
  ~tgohip_st() {
    if (f) fclose(f);
  }
};

// The header cap: the length prefix is read before anything else is known.
static int64_t g_max_header = 100ll << 20;

static int st_error(const std::string& msg) { return fail(TGOHIP_EINVAL, "safetensors: " + msg); }

// One header record against the data region (safetensors.go:196-241).
static int st_entry(tgohip_st* f, const std::string& name, const JVal& rec, StEntry& out) {
  const std::string at = f->path + ": " + name + ": ";
  std::string dtype;
  std::vector<int64_t> shape, offs;
  if (rec.kind != JVal::OBJ && rec.kind != JVal::NUL)
    return st_error(at + "parse entry: the record is not an object");
  for (const auto& kv : rec.o) {
    const JVal& v = kv.second;
    auto ints = [&](std::vector<int64_t>& dst, const char* field) -> bool {
      dst.clear();
      if (v.kind == JVal::NUL) return true;
      if (v.kind != JVal::ARR) return false;
      for (const JVal& x : v.a) {
        if (x.kind != JVal::NUM || !x.is_int) return false;
        dst.push_back(x.i);
      }
      (void)field;
      return true;
    };
    if (ieq(kv.first, "dtype")) {
      if (v.kind == JVal::STR) dtype = v.s;
      else if (v.kind != JVal::NUL) return st_error(at + "parse entry: dtype is not a string");
    } else if (ieq(kv.first, "shape")) {
      if (!ints(shape, "shape")) return st_error(at + "parse entry: shape is not a list of integers");
    } else if (ieq(kv.first, "data_offsets")) {
      if (!ints(offs, "data_offsets"))
        return st_error(at + "parse entry: data_offsets is not a list of integers");
    }
  }
  const int64_t width = dtype_size(dtype);
  if (!width) return st_error(at + "unknown dtype \"" + dtype + "\"");
  if (offs.size() != 2)
    return st_error(at + "data_offsets has " + std::to_string(offs.size()) + " elements, want 2");
  const int64_t begin = offs[0], end = offs[1];
  if (end < begin)
    return st_error(at + "data_offsets end " + std::to_string(end) + " is before begin " +
                    std::to_string(begin));
  if (begin < 0 || end > f->data_len)
    return st_error(at + "data_offsets [" + std::to_string(begin) + "," + std::to_string(end) +
                    ") lie outside the " + std::to_string(f->data_len) + "-byte data region");
  int64_t count = 1;
  for (size_t k = 0; k < shape.size(); k++) {
    const int64_t d = shape[k];
    if (d < 0)
      return st_error(at + "shape dimension " + std::to_string(k) + " is negative (" +
                      std::to_string(d) + ")");
    if (d != 0 && count > INT64_MAX / d)
      return st_error(at + "shape " + shape_str(shape) + " is larger than this platform can index");
    count *= d;
  }
  if (count > INT64_MAX / width)
    return st_error(at + "shape " + shape_str(shape) + " of dtype " + dtype +
                    " is larger than this platform can index");
  if (count * width != end - begin)
    return st_error(at + "shape " + shape_str(shape) + " of dtype " + dtype + " needs " +
                    std::to_string(count * width) + " bytes, but data_offsets span " +
                    std::to_string(end - begin));
  out.dtype = dtype;
  out.shape = shape;
  out.begin = begin;
  out.end = end;
  return 0;
}

extern "C" tgohip_st* tgohip_st_open(const char* path) {
  if (!path) {
    fail(TGOHIP_EINVAL, "safetensors: no path");
    return nullptr;
  }
  std::unique_ptr<tgohip_st> f(new tgohip_st);
  f->path = path;
  struct stat sb;
  if (stat(path, &sb) != 0) {
    fail(TGOHIP_EINVAL, std::string("safetensors: open ") + path + ": no such file");
    return nullptr;
  }
  if (!S_ISREG(sb.st_mode)) {
    fail(TGOHIP_EINVAL, std::string("safetensors: ") + path + ": is not a regular file");
    return nullptr;
  }
  f->f = fopen(path, "rb");
  if (!f->f) {
    fail(TGOHIP_EINVAL, std::string("safetensors: open ") + path + ": cannot read");
    return nullptr;
  }
  const int64_t size = (int64_t)sb.st_size;
  if (size < 8) {
    st_error(f->path + ": file is " + std::to_string(size) +
             " bytes, shorter than the 8-byte header length");
    return nullptr;
  }
  uint8_t pre[8];
  if (fread(pre, 1, 8, f->f) != 8) {
    st_error(f->path + ": read header length");
    return nullptr;
  }
  uint64_t n = 0;
  for (int k = 7; k >= 0; k--) n = (n << 8) | pre[k];
  if (n > (uint64_t)(size - 8)) {
    st_error(f->path + ": header length " + std::to_string(n) + " exceeds the " +
             std::to_string(size - 8) + " bytes that follow it");
    return nullptr;
  }
  if (n > (uint64_t)g_max_header) {
    st_error(f->path + ": header length " + std::to_string(n) + " exceeds the " +
             std::to_string(g_max_header) + "-byte limit");
    return nullptr;
  }
  std::string hdr((size_t)n, '\0');
  if (n && fread(&hdr[0], 1, (size_t)n, f->f) != (size_t)n) {
    st_error(f->path + ": read header");
    return nullptr;
  }
  JVal root;
  std::string jerr;
  if (!json_parse(hdr.data(), hdr.size(), root, jerr)) {
    st_error(f->path + ": parse header: " + jerr);
    return nullptr;
  }
  if (root.kind != JVal::OBJ) {
    st_error(f->path + ": parse header: the header is not a JSON object");
    return nullptr;
  }
  f->data_start = 8 + (int64_t)n;
  f->data_len = size - 8 - (int64_t)n;
  // Validate in name order, so a file with two faults refuses the same way
  // every time (safetensors.go:171-178).
  std::vector<const std::pair<std::string, JVal>*> recs;
  for (const auto& kv : root.o) recs.push_back(&kv);
  std::sort(recs.begin(), recs.end(), [](auto* a, auto* b) { return a->first < b->first; });
  for (auto* kv : recs) {
    if (kv->first == "__metadata__") {
      bool ok = kv->second.kind == JVal::OBJ || kv->second.kind == JVal::NUL;
      for (const auto& m : kv->second.o) ok = ok && m.second.kind == JVal::STR;
      if (!ok) {
        st_error(f->path + ": __metadata__ is not a map of strings");
        return nullptr;
      }
      continue;
    }
    StEntry e;
    if (st_entry(f.get(), kv->first, kv->second, e)) return nullptr;
    f->entries[kv->first] = e;
    f->names.push_back(kv->first);
  }
  // No two tensors share a byte; empty tensors own none (safetensors.go:246-277).
  struct Span {
    const std::string* name;
    int64_t b, e;
  };
  std::vector<Span> sp;
  for (const auto& nm : f->names) {
    const StEntry& e = f->entries[nm];
    if (e.end != e.begin) sp.push_back({&nm, e.begin, e.end});
  }
  std::stable_sort(sp.begin(), sp.end(), [](const Span& a, const Span& b) { return a.b < b.b; });
  for (size_t k = 1; k < sp.size(); k++)
    if (sp[k].b < sp[k - 1].e) {
      st_error(f->path + ": " + *sp[k].name + " [" + std::to_string(sp[k].b) + "," +
               std::to_string(sp[k].e) + ") overlaps " + *sp[k - 1].name + " [" +
               std::to_string(sp[k - 1].b) + "," + std::to_string(sp[k - 1].e) + ")");
      return nullptr;
    }
  return f.release();
}

extern "C" void tgohip_st_close(tgohip_st* f) { delete f; }

extern "C" int tgohip_st_count(const tgohip_st* f) { return f ? (int)f->names.size() : 0; }

extern "C" int tgohip_st_entry(const tgohip_st* f, int i, const char** name, const char** dtype,
                               int* rank, int64_t* shape, int64_t* begin, int64_t* end) {
  if (!f || i < 0 || i >= (int)f->names.size())
    return fail(TGOHIP_EINVAL, "safetensors: entry index out of range");
  const std::string& nm = f->names[(size_t)i];
  const StEntry& e = f->entries.at(nm);
  if (name) *name = nm.c_str();
  if (dtype) *dtype = e.dtype.c_str();
  if (rank) *rank = (int)e.shape.size();
  if (shape)
    for (size_t k = 0; k < e.shape.size() && k < 8; k++) shape[k] = e.shape[k];
  if (begin) *begin = e.begin;
  if (end) *end = e.end;
  return 0;
}

static int64_t st_read(const tgohip_st* f, const std::string& name, void* dst, int64_t cap) {
  auto it = f->entries.find(name);
  if (it == f->entries.end())
    return st_error(f->path + ": no tensor named \"" + name + "\"");
  const int64_t n = it->second.end - it->second.begin;
  if (n > cap) return st_error(f->path + ": " + name + ": the destination is too small");
  if (n == 0) return 0;
  if (fseeko(f->f, (off_t)(f->data_start + it->second.begin), SEEK_SET) != 0 ||
      fread(dst, 1, (size_t)n, f->f) != (size_t)n)
    return st_error(f->path + ": " + name + ": read plane: the file is shorter than its header says");
  return n;
}

extern "C" int64_t tgohip_st_read(const tgohip_st* f, const char* name, void* dst, int64_t cap) {
  if (!f || !name) return fail(TGOHIP_EINVAL, "safetensors: no file or name");
  return st_read(f, name, dst, cap);
}

// Lowers the header cap (tests exercise the refusal without a 100 MB file).
extern "C" void tgohip_st_set_max_header(int64_t bytes) {
  g_max_header = bytes > 0 ? bytes : (100ll << 20);
}

// ---------------------------------------------------------------------------
// safetensors.Repo (safetensors/repo.go:48-196)
// ---------------------------------------------------------------------------
struct tgohip_repo {
  std::string dir;
  std::map<std::string, std::unique_ptr<tgohip_st>> files;  // shard name -> file
  std::map<std::string, std::string> shard_of;                // tensor -> shard
};

static bool read_file(const std::string& path, std::string& out, bool& missing) {
  missing = false;
  struct stat sb;
  if (stat(path.c_str(), &sb) != 0) {
    missing = true;
    return false;
  }
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) return false;
  out.assign((size_t)sb.st_size, '\0');
  const bool ok = fread(&out[0], 1, out.size(), f) == out.size();
  fclose(f);
  return ok;
}

static bool shard_name_ok(const std::string& s) {  // repo.go:188-196
  return !(s.empty() || s == "." || s == ".." || s.find('/') != std::string::npos ||
           s.find('\\') != std::string::npos);
}

extern "C" tgohip_repo* tgohip_repo_open(const char* dir_c) {
  if (!dir_c) {
    fail(TGOHIP_EINVAL, "safetensors: no directory");
    return nullptr;
  }
  std::unique_ptr<tgohip_repo> r(new tgohip_repo);
  r->dir = dir_c;
  const std::string dir = r->dir;
  std::string cfg;
  bool missing;
  if (read_file(dir + "/config.json", cfg, missing)) {
    JVal v;
    std::string err;
    if (!json_parse(cfg.data(), cfg.size(), v, err)) {
      st_error(dir + ": config.json is not valid JSON");
      return nullptr;
    }
  } else if (!missing) {
    st_error(dir + ": read config");
    return nullptr;
  }
  const std::string idx_path = dir + "/model.safetensors.index.json";
  std::string idx;
  if (!read_file(idx_path, idx, missing)) {
    if (!missing) {
      st_error(dir + ": read index");
      return nullptr;
    }
    // unsharded
    struct stat sb;
    if (stat((dir + "/model.safetensors").c_str(), &sb) != 0) {
      st_error(dir + ": no model.safetensors and no model.safetensors.index.json");
      return nullptr;
    }
    tgohip_st* f = tgohip_st_open((dir + "/model.safetensors").c_str());
    if (!f) return nullptr;
    for (const auto& nm : f->names) r->shard_of[nm] = "model.safetensors";
    r->files["model.safetensors"].reset(f);
    return r.release();
  }
  JVal v;
  std::string err;
  if (!json_parse(idx.data(), idx.size(), v, err) || v.kind != JVal::OBJ) {
    st_error(idx_path + ": parse index: " + (err.empty() ? "not an object" : err));
    return nullptr;
  }
  std::map<std::string, std::string> wm;
  for (const auto& kv : v.o) {
    if (!ieq(kv.first, "weight_map")) continue;
    if (kv.second.kind == JVal::NUL) continue;
    if (kv.second.kind != JVal::OBJ) {
      st_error(idx_path + ": parse index: weight_map is not an object");
      return nullptr;
    }
    for (const auto& m : kv.second.o) {
      if (m.second.kind != JVal::STR) {
        st_error(idx_path + ": parse index: weight_map values are file names");
        return nullptr;
      }
      wm[m.first] = m.second.s;
    }
  }
  if (wm.empty()) {
    st_error(idx_path + ": weight_map is empty or absent");
    return nullptr;
  }
  for (const auto& kv : wm) {  // name order
    if (!shard_name_ok(kv.second)) {
      st_error(idx_path + ": " + kv.first + ": shard \"" + kv.second +
               "\" is not a file name in the model directory");
      return nullptr;
    }
    if (r->files.count(kv.second)) continue;
    struct stat sb;
    const std::string sp = dir + "/" + kv.second;
    if (stat(sp.c_str(), &sb) != 0) {
      st_error(idx_path + ": " + kv.first + ": shard " + kv.second + " is missing");
      return nullptr;
    }
    tgohip_st* f = tgohip_st_open(sp.c_str());
    if (!f) return nullptr;
    r->files[kv.second].reset(f);
  }
  for (const auto& kv : wm) {
    if (!r->files[kv.second]->entries.count(kv.first)) {
      st_error(idx_path + ": " + kv.first + ": shard " + kv.second + " has no such tensor");
      return nullptr;
    }
    r->shard_of[kv.first] = kv.second;
  }
  for (const auto& fs : r->files)  // shard-name order
    for (const auto& nm : fs.second->names) {
      auto it = wm.find(nm);
      if (it == wm.end() || it->second != fs.first) {
        st_error(idx_path + ": " + nm + " in shard " + fs.first + " has no entry in the index");
        return nullptr;
      }
    }
  return r.release();
}

extern "C" void tgohip_repo_close(tgohip_repo* r) { delete r; }

static const tgohip_st* repo_file(const tgohip_repo* r, const std::string& name, StEntry* e) {
  auto it = r->shard_of.find(name);
  if (it == r->shard_of.end()) return nullptr;
  const tgohip_st* f = r->files.at(it->second).get();
  if (e) *e = f->entries.at(name);
  return f;
}

extern "C" int tgohip_repo_has(const tgohip_repo* r, const char* name) {
  return r && name && r->shard_of.count(name) ? 1 : 0;
}

// ---------------------------------------------------------------------------
// The loader's conversions (weights/weights.go:552-627, convert.go:41-131)
// ---------------------------------------------------------------------------
static float f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16, ex = (h >> 10) & 0x1f, m = h & 0x3ff;
  uint32_t u;
  if (ex == 0) {
    if (m == 0) {
      u = sign;
    } else {  // subnormal: normalise
      int sh = 0;
      uint32_t mm = m;
      while (!(mm & 0x400)) { mm <<= 1; sh++; }
      u = sign | ((uint32_t)(113 - sh) << 23) | ((mm & 0x3ff) << 13);
    }
  } else if (ex == 31) {
    u = sign | 0x7f800000u | (m << 13);
  } else {
    u = sign | ((ex + 112) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// decodeF32: BF16 widens by a 16-bit shift, F16 exactly, F32 as is; integer
// planes are refused rather than reinterpreted.
static int decode_f32(const std::string& name, const std::string& dt, const std::vector<uint8_t>& raw,
                      float* dst, size_t n) {
  const size_t w = (size_t)dtype_size(dt);
  if (dt != "BF16" && dt != "F16" && dt != "F32")
    return fail(TGOHIP_EINVAL, "weights: \"" + name + "\": dtype " + dt +
                                   " is not a float plane this loader converts; a weight must be "
                                   "BF16, F16 or F32");
  if (raw.size() != n * w)
    return fail(TGOHIP_EINVAL, "weights: \"" + name + "\": " + dt + " plane is " +
                                   std::to_string(raw.size()) + " bytes, but " + std::to_string(n) +
                                   " elements need " + std::to_string(n * w));
  for (size_t k = 0; k < n; k++) {
    if (dt == "BF16") {
      const uint32_t u = (uint32_t)(raw[2 * k] | (raw[2 * k + 1] << 8)) << 16;
      memcpy(&dst[k], &u, 4);
    } else if (dt == "F16") {
      dst[k] = f16_bits_to_f32((uint16_t)(raw[2 * k] | (raw[2 * k + 1] << 8)));
    } else {
      uint32_t u = 0;
      for (int b = 3; b >= 0; b--) u = (u << 8) | raw[4 * k + (size_t)b];
      memcpy(&dst[k], &u, 4);
    }
  }
  return 0;
}

// The f32 plane of one tensor after decode, transpose and head permutation.
static int repo_plane(const tgohip_repo* r, const std::string& name, bool transpose, int head_dim,
                      std::vector<float>& out) {
  StEntry e;
  const tgohip_st* f = repo_file(r, name, &e);
  if (!f)
    return fail(TGOHIP_EINVAL, "weights: the model declares \"" + name +
                                   "\", which this checkpoint does not contain");
  if (e.shape.size() != 1 && e.shape.size() != 2)
    return fail(TGOHIP_EINVAL, "weights: \"" + name + "\" has rank " +
                                   std::to_string(e.shape.size()) +
                                   "; a weight this loader converts is a matrix or a gain vector");
  if (transpose && e.shape.size() != 2)
    return fail(TGOHIP_EINVAL, "weights: \"" + name + "\" is declared transposed but has shape " +
                                   shape_str(e.shape) + "; only a matrix has axes to exchange");
  size_t n = 1;
  for (int64_t d : e.shape) n *= (size_t)d;
  if (n == 0)
    return fail(TGOHIP_EINVAL, "weights: \"" + name + "\" has shape " + shape_str(e.shape) +
                                   ", which holds no elements");
  std::vector<uint8_t> raw((size_t)(e.end - e.begin));
  if (st_read(f, name, raw.data(), (int64_t)raw.size()) < 0) return TGOHIP_EINVAL;
  std::vector<float> plane(n);
  if (int rc = decode_f32(name, e.dtype, raw, plane.data(), n)) return rc;
  std::vector<uint8_t>().swap(raw);
  const size_t last = transpose ? (size_t)e.shape[0] : (size_t)e.shape.back();
  if (transpose) {
    const size_t rows = (size_t)e.shape[0], cols = (size_t)e.shape[1];
    out.assign(n, 0.f);
    for (size_t rr = 0; rr < rows; rr++)
      for (size_t c = 0; c < cols; c++) out[c * rows + rr] = plane[rr * cols + c];
  } else {
    out.swap(plane);
  }
  if (head_dim > 0) {
    if (head_dim % 2)
      return fail(TGOHIP_EINVAL, "weights: \"" + name + "\": head dim " + std::to_string(head_dim) +
                                     " must be positive and even; RoPE rotates pairs");
    if (last % (size_t)head_dim)
      return fail(TGOHIP_EINVAL, "weights: \"" + name + "\": output axis " + std::to_string(last) +
                                     " is not a multiple of head dim " + std::to_string(head_dim) +
                                     ", so it does not divide into heads");
    const size_t half = (size_t)head_dim / 2;
    std::vector<float> tmp((size_t)head_dim);
    for (size_t off = 0; off < out.size(); off += (size_t)head_dim) {
      std::copy(out.begin() + (long)off, out.begin() + (long)(off + head_dim), tmp.begin());
      for (size_t i = 0; i < half; i++) {
        out[off + 2 * i] = tmp[i];
        out[off + 2 * i + 1] = tmp[i + half];
      }
    }
  }
  return 0;
}

extern "C" int tgohip_repo_plane(const tgohip_repo* r, const char* name, int transpose, int head_dim,
                                 float* out, int64_t n) {
  if (!r || !name || !out) return fail(TGOHIP_EINVAL, "weights: no repo, name or output");
  std::vector<float> p;
  if (int rc = repo_plane(r, name, transpose != 0, head_dim, p)) return rc;
  if ((int64_t)p.size() != n)
    return fail(TGOHIP_EINVAL, "weights: \"" + std::string(name) + "\" holds " +
                                   std::to_string(p.size()) + " elements, not " + std::to_string(n));
  memcpy(out, p.data(), p.size() * 4);
  return 0;
}

// ---------------------------------------------------------------------------
// The Qwen3 weight map (model/qwen3.go:54-205) and weights.Load
// ---------------------------------------------------------------------------
namespace {
struct Spec {
  std::string tensor, port;
  std::vector<int64_t> shape;  // as the file stores it
  int kind;                    // 0 gain, 1 projection, 2 embedding, 3 head
  bool transpose;
  int head_dim;                // > 0: permute heads of this width
};
}  // namespace

static int load_projection(tgohip_ctx* ctx, const Spec& s, const std::vector<float>& p, int form,
                           int64_t K, int64_t N, double max_sat, int64_t* saturated) {
  const size_t n = p.size();
  if (form == TGOHIP_FORM_F16) {
    std::vector<uint16_t> h(n);
    const size_t sat = tgohip_to_f16(p.data(), h.data(), n);
    if ((double)sat / (double)n > max_sat)
      return fail(TGOHIP_EINVAL, "weights: \"" + s.tensor + "\" saturated " + std::to_string(sat) +
                                     " of " + std::to_string(n) +
                                     " elements to +-65504, over the threshold: this checkpoint "
                                     "holds values f16 cannot represent, and int8 is not a fix "
                                     "for it either");
    if (saturated) *saturated += (int64_t)sat;
    return tgohip_weight(ctx, s.port.c_str(), form, (int)K, (int)N, h.data(), nullptr, nullptr);
  }
  if (form == TGOHIP_FORM_I8 || form == TGOHIP_FORM_I4_TGO)  // quantized on the device
    return tgohip_weight_f32(ctx, s.port.c_str(), form, (int)K, (int)N, p.data());
  return fail(TGOHIP_EINVAL, "weights: load form " + std::to_string(form) +
                                 " is not F16, I8 or the int4 pack tgo stores (I4_TGO)");
}

extern "C" int tgohip_load_qwen3(tgohip_ctx* ctx, const tgohip_repo* r, int form, int tie,
                                 int64_t* saturated) {
  if (!ctx || !r) return fail(TGOHIP_EINVAL, "weights: Load needs a context and a repo");
  tgohip_model_cfg c;
  if (int rc = tgohip_get_config(ctx, &c)) return rc;
  if (form != TGOHIP_FORM_F16 && form != TGOHIP_FORM_I8 && form != TGOHIP_FORM_I4_TGO)
    return fail(TGOHIP_EINVAL, "weights: load form " + std::to_string(form) +
                                   " is not F16, I8 or the int4 pack tgo stores (I4_TGO)");
  const int64_t d = c.hidden, qw = (int64_t)c.heads * c.head_dim, kvw = (int64_t)c.kv_heads * c.head_dim,
                f = c.ffn, V = c.vocab, dh = c.head_dim;
  std::vector<Spec> specs;
  specs.push_back({"model.embed_tokens.weight", "embed", {V, d}, 2, false, 0});
  for (int l = 0; l < c.layers; l++) {
    const std::string pre = "model.layers." + std::to_string(l) + ".", pl = std::to_string(l) + ".";
    specs.push_back({pre + "input_layernorm.weight", pl + "attn_norm", {d}, 0, false, 0});
    specs.push_back({pre + "self_attn.q_proj.weight", pl + "wq", {qw, d}, 1, true, (int)dh});
    specs.push_back({pre + "self_attn.k_proj.weight", pl + "wk", {kvw, d}, 1, true, (int)dh});
    specs.push_back({pre + "self_attn.v_proj.weight", pl + "wv", {kvw, d}, 1, true, 0});
    specs.push_back({pre + "self_attn.o_proj.weight", pl + "wo", {d, qw}, 1, true, 0});
    specs.push_back({pre + "self_attn.q_norm.weight", pl + "qnorm", {dh}, 0, false, (int)dh});
    specs.push_back({pre + "self_attn.k_norm.weight", pl + "knorm", {dh}, 0, false, (int)dh});
    specs.push_back({pre + "post_attention_layernorm.weight", pl + "ffn_norm", {d}, 0, false, 0});
    specs.push_back({pre + "mlp.gate_proj.weight", pl + "wgate", {f, d}, 1, true, 0});
    specs.push_back({pre + "mlp.up_proj.weight", pl + "wup", {f, d}, 1, true, 0});
    specs.push_back({pre + "mlp.down_proj.weight", pl + "wdown", {d, f}, 1, true, 0});
  }
  specs.push_back({"model.norm.weight", "final_norm", {d}, 0, false, 0});
  // A tied head is a second plane from the embedding tensor; a tied
  // checkpoint must not also ship lm_head.weight (model/qwen3.go:194-204).
  if (tie && r->shard_of.count("lm_head.weight"))
    return fail(TGOHIP_EINVAL, "weights: the config ties the head to the embedding, and the "
                               "checkpoint also ships \"lm_head.weight\"");
  specs.push_back({tie ? "model.embed_tokens.weight" : "lm_head.weight", "lm_head", {V, d}, 3, true, 0});

  // Every declared tensor is present with the declared shape before any
  // conversion starts (weights.go planLoad; model.go checkAgainst).
  for (const Spec& s : specs) {
    StEntry e;
    if (!repo_file(r, s.tensor, &e))
      return fail(TGOHIP_EINVAL, "weights: the model declares \"" + s.tensor +
                                     "\", which this checkpoint does not contain");
    if (e.shape != s.shape)
      return fail(TGOHIP_EINVAL, "weights: \"" + s.tensor + "\" has shape " + shape_str(e.shape) +
                                     " and the config declares " + shape_str(s.shape));
  }
  const double max_sat = 1e-5;  // weights.go:205
  if (saturated) *saturated = 0;
  for (const Spec& s : specs) {
    std::vector<float> p;
    if (int rc = repo_plane(r, s.tensor, s.transpose, s.head_dim, p)) return rc;
    int rc = 0;
    if (s.kind == 0) {
      rc = tgohip_gain(ctx, s.port.c_str(), p.data(), (int)p.size());
    } else if (s.kind == 2) {
      // A gathered table cannot pack: under int4 it is int8 (weights.go:538-546).
      const int ef = form == TGOHIP_FORM_F16 ? TGOHIP_FORM_F16 : TGOHIP_FORM_I8;
      rc = load_projection(ctx, s, p, ef, V, d, max_sat, saturated);
    } else {
      const int64_t K = s.shape[1], N = s.shape[0];  // [out, in] -> [in, out]
      rc = load_projection(ctx, s, p, form, K, N, max_sat, saturated);
    }
    if (rc) return rc;
  }
  return 0;
}
