// .safetensors reader: readHeader / readTensor (src/weights/safetensors.ts:28-70) on a file descriptor.
//
// The header is parsed and validated up front, with the reference's checks in the reference's order and
// its messages; tensor bytes are read only on request, with positional reads (pread) straight into the
// caller's memory (typically pinned host memory that a stream copy then moves to HBM). A large read is
// split over several threads: one thread copying out of the page cache does a few GB/s, several come
// closer to what the host link to the GPU takes.
//
// The file is untrusted: the JSON parser bounds nesting depth and never reads past the header, every
// number is checked before use, and reads are checked against the tensor's extent.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "we.h"

namespace we {
void set_no_ctx_error(const char* msg);  // runtime.cpp: we_last_error(NULL) of this thread
}

namespace {

int st_fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  we::set_no_ctx_error(buf);
  return code;
}

// ---- minimal JSON (RFC 8259) -------------------------------------------------------------------------

struct JVal {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;  // insertion order; a repeated key keeps its first place
  const JVal* get(const std::string& k) const {
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

class JParser {
 public:
  JParser(const char* p, size_t n) : p_(p), end_(p + n) {}
  bool parse_document(JVal& out) {
    if (end_ - p_ >= 3 && (unsigned char)p_[0] == 0xEF && (unsigned char)p_[1] == 0xBB && (unsigned char)p_[2] == 0xBF)
      p_ += 3;  // a UTF-8 byte-order mark is dropped when the header bytes are decoded as text
    ws();
    if (!value(out, 0)) return false;
    ws();
    return p_ == end_;
  }

 private:
  static constexpr int kMaxDepth = 256;
  const char* p_;
  const char* end_;

  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
  }
  bool lit(const char* s) {
    const size_t n = strlen(s);
    if ((size_t)(end_ - p_) < n || memcmp(p_, s, n) != 0) return false;
    p_ += n;
    return true;
  }
  bool value(JVal& v, int depth) {
    if (depth > kMaxDepth || p_ >= end_) return false;
    switch (*p_) {
      case '{': return object(v, depth);
      case '[': return array(v, depth);
      case '"': v.kind = JVal::Str; return string(v.str);
      case 't': v.kind = JVal::Bool; v.b = true; return lit("true");
      case 'f': v.kind = JVal::Bool; v.b = false; return lit("false");
      case 'n': v.kind = JVal::Null; return lit("null");
      default: v.kind = JVal::Num; return number(v.num);
    }
  }
  bool object(JVal& v, int depth) {
    v.kind = JVal::Obj;
    p_++;
    ws();
    if (p_ < end_ && *p_ == '}') {
      p_++;
      return true;
    }
    for (;;) {
      ws();
      if (p_ >= end_ || *p_ != '"') return false;
      std::string key;
      if (!string(key)) return false;
      ws();
      if (p_ >= end_ || *p_ != ':') return false;
      p_++;
      ws();
      JVal item;
      if (!value(item, depth + 1)) return false;
      bool replaced = false;
      for (auto& kv : v.obj)
        if (kv.first == key) {
          kv.second = std::move(item);
          replaced = true;
          break;
        }
      if (!replaced) v.obj.emplace_back(std::move(key), std::move(item));
      ws();
      if (p_ >= end_) return false;
      if (*p_ == ',') {
        p_++;
        continue;
      }
      if (*p_ == '}') {
        p_++;
        return true;
      }
      return false;
    }
  }
  bool array(JVal& v, int depth) {
    v.kind = JVal::Arr;
    p_++;
    ws();
    if (p_ < end_ && *p_ == ']') {
      p_++;
      return true;
    }
    for (;;) {
      ws();
      JVal item;
      if (!value(item, depth + 1)) return false;
      v.arr.push_back(std::move(item));
      ws();
      if (p_ >= end_) return false;
      if (*p_ == ',') {
        p_++;
        continue;
      }
      if (*p_ == ']') {
        p_++;
        return true;
      }
      return false;
    }
  }
  static void utf8(std::string& s, uint32_t cp) {
    if (cp < 0x80) {
      s += (char)cp;
    } else if (cp < 0x800) {
      s += (char)(0xC0 | (cp >> 6));
      s += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      s += (char)(0xE0 | (cp >> 12));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    } else {
      s += (char)(0xF0 | (cp >> 18));
      s += (char)(0x80 | ((cp >> 12) & 0x3F));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t& cp) {
    if (end_ - p_ < 4) return false;
    cp = 0;
    for (int i = 0; i < 4; i++) {
      const char c = *p_++;
      cp <<= 4;
      if (c >= '0' && c <= '9') cp |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') cp |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') cp |= (uint32_t)(c - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string& s) {
    p_++;  // opening quote
    for (;;) {
      if (p_ >= end_) return false;
      const unsigned char c = (unsigned char)*p_++;
      if (c == '"') return true;
      if (c < 0x20) return false;  // raw control characters are not allowed inside strings
      if (c != '\\') {
        s += (char)c;
        continue;
      }
      if (p_ >= end_) return false;
      const char e = *p_++;
      switch (e) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
            const char* save = p_;
            p_ += 2;
            uint32_t lo;
            if (hex4(lo) && lo >= 0xDC00 && lo < 0xE000) cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            else p_ = save;  // a lone surrogate stays one code unit
          }
          utf8(s, cp);
          break;
        }
        default: return false;
      }
    }
  }
  bool number(double& out) {
    const char* s = p_;
    if (p_ < end_ && *p_ == '-') p_++;
    if (p_ >= end_) return false;
    if (*p_ == '0') {
      p_++;
    } else if (*p_ >= '1' && *p_ <= '9') {
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
    } else {
      return false;
    }
    if (p_ < end_ && *p_ == '.') {
      p_++;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      p_++;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) p_++;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
    }
    const std::string text(s, p_);
    out = strtod(text.c_str(), nullptr);  // overflow gives +-inf, as JSON.parse does
    return true;
  }
};

// ---- JavaScript's number / String() formatting, for messages identical to the reference's -------------

std::string js_number(double v) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v > 0 ? "Infinity" : "-Infinity";
  if (v == 0.0) return "0";
  char buf[64];
  if (v == std::floor(v) && std::fabs(v) < 1e21) {
    snprintf(buf, sizeof buf, "%.0f", v);
    return buf;
  }
  for (int prec = 1; prec <= 17; prec++) {  // shortest text that reads back as the same double
    snprintf(buf, sizeof buf, "%.*g", prec, v);
    if (strtod(buf, nullptr) == v) break;
  }
  std::string s = buf;
  const size_t e = s.find('e');
  if (e != std::string::npos) {  // 1e+21 style: no leading zeros in the exponent
    std::string mant = s.substr(0, e), ex = s.substr(e + 1);
    const char sign = ex[0] == '-' ? '-' : '+';
    size_t i = (ex[0] == '-' || ex[0] == '+') ? 1 : 0;
    while (i + 1 < ex.size() && ex[i] == '0') i++;
    s = mant + "e" + sign + ex.substr(i);
  }
  return s;
}

std::string js_string(const JVal* v) {
  if (!v) return "undefined";
  switch (v->kind) {
    case JVal::Null: return "null";
    case JVal::Bool: return v->b ? "true" : "false";
    case JVal::Num: return js_number(v->num);
    case JVal::Str: return v->str;
    case JVal::Arr: {
      std::string s;
      for (size_t i = 0; i < v->arr.size(); i++) {
        if (i) s += ',';
        if (v->arr[i].kind != JVal::Null) s += js_string(&v->arr[i]);
      }
      return s;
    }
    default: return "[object Object]";
  }
}

// Number.isSafeInteger(n) && n >= 0
bool is_count(const JVal& v) {
  return v.kind == JVal::Num && std::isfinite(v.num) && v.num == std::floor(v.num) && v.num >= 0.0 &&
         v.num <= 9007199254740991.0;
}

// JavaScript visits an object's integer-like keys ("0", "17"; canonical, below 2^32 - 1) first, in numeric
// order, then the other keys in insertion order: the order Object.entries gives the reference's loop.
bool array_index(const std::string& k, uint64_t& idx) {
  if (k.empty() || k.size() > 10) return false;
  if (k.size() > 1 && k[0] == '0') return false;
  idx = 0;
  for (char c : k) {
    if (c < '0' || c > '9') return false;
    idx = idx * 10 + (uint64_t)(c - '0');
  }
  return idx < 4294967295ull;
}

struct DtypeBytes {
  const char* name;
  uint32_t bytes;
};
// DTYPE_BYTES (src/weights/safetensors.ts:8-11)
constexpr DtypeBytes kDtypes[] = {{"F64", 8}, {"F32", 4}, {"F16", 2},   {"BF16", 2},    {"F8_E4M3", 1},
                                  {"F8_E5M2", 1}, {"I64", 8}, {"I32", 4}, {"I16", 2}, {"I8", 1},
                                  {"U64", 8}, {"U32", 4}, {"U16", 2},   {"U8", 1},      {"BOOL", 1}};
constexpr uint64_t kMaxHeader = 100000000;  // MAX_HEADER (src/weights/safetensors.ts:13)

}  // namespace

struct we_safetensors {
  int fd = -1;
  uint64_t file_size = 0;
  struct Tensor {
    std::string name, dtype;
    std::vector<uint64_t> shape;
    uint64_t offset = 0, size = 0;
  };
  std::vector<Tensor> tensors;  // in the reference's Map order
  std::map<std::string, uint32_t> by_name;
  std::vector<std::pair<std::string, std::string>> metadata;  // string values of __metadata__
};

namespace {

int read_all(int fd, uint64_t off, uint64_t n, char* dst) {
  while (n > 0) {
    const size_t want = (size_t)std::min<uint64_t>(n, 1ull << 30);
    const ssize_t got = pread(fd, dst, want, (off_t)off);
    if (got < 0) {
      if (errno == EINTR) continue;
      return errno ? errno : EIO;
    }
    if (got == 0) return EIO;  // the file shrank under us
    dst += got;
    off += (uint64_t)got;
    n -= (uint64_t)got;
  }
  return 0;
}

// readHeader (src/weights/safetensors.ts:28-65)
int parse_header(we_safetensors& st) {
  if (st.file_size < 8) return st_fail(WE_EFORMAT, "File is too small to be a .safetensors file");
  unsigned char size8[8];
  if (int e = read_all(st.fd, 0, 8, (char*)size8)) return st_fail(WE_EIO, "read failed: %s", strerror(e));
  uint64_t header_size = 0;
  for (int i = 7; i >= 0; i--) header_size = (header_size << 8) | size8[i];
  if (header_size > kMaxHeader || 8 + header_size > st.file_size)
    return st_fail(WE_EFORMAT, "Bad header size: %s", js_number((double)header_size).c_str());

  std::string text((size_t)header_size, '\0');
  if (header_size)
    if (int e = read_all(st.fd, 8, header_size, &text[0])) return st_fail(WE_EIO, "read failed: %s", strerror(e));
  JVal header;
  if (!JParser(text.data(), text.size()).parse_document(header)) return st_fail(WE_EFORMAT, "Header is not valid JSON");
  if (header.kind != JVal::Obj) return st_fail(WE_EFORMAT, "Header is not an object");

  const uint64_t start = 8 + header_size;
  const uint64_t data_size = st.file_size - start;

  // Object.entries order, __metadata__ set aside
  std::vector<const std::pair<std::string, JVal>*> entries;
  for (const auto& kv : header.obj) entries.push_back(&kv);
  std::stable_sort(entries.begin(), entries.end(), [](const auto* a, const auto* b) {
    uint64_t ia, ib;
    const bool xa = array_index(a->first, ia), xb = array_index(b->first, ib);
    if (xa != xb) return xa;
    return xa && ia < ib;
  });

  for (const auto* kv : entries) {
    const std::string& name = kv->first;
    const JVal& entry = kv->second;
    if (name == "__metadata__") {
      if (entry.kind == JVal::Obj)
        for (const auto& m : entry.obj)
          if (m.second.kind == JVal::Str) st.metadata.emplace_back(m.first, m.second.str);
      continue;
    }
    const bool is_obj = entry.kind == JVal::Obj;
    const JVal* dtype = is_obj ? entry.get("dtype") : nullptr;
    const JVal* shape = is_obj ? entry.get("shape") : nullptr;
    const JVal* offsets = is_obj ? entry.get("data_offsets") : nullptr;
    uint32_t elem = 0;
    if (dtype && dtype->kind == JVal::Str)
      for (const auto& d : kDtypes)
        if (dtype->str == d.name) elem = d.bytes;
    if (!elem) return st_fail(WE_EFORMAT, "%s: unknown dtype %s", name.c_str(), js_string(dtype).c_str());
    if (!shape || shape->kind != JVal::Arr || !std::all_of(shape->arr.begin(), shape->arr.end(), is_count))
      return st_fail(WE_EFORMAT, "%s: bad shape", name.c_str());
    if (!offsets || offsets->kind != JVal::Arr || offsets->arr.size() != 2 ||
        !std::all_of(offsets->arr.begin(), offsets->arr.end(), is_count))
      return st_fail(WE_EFORMAT, "%s: bad data_offsets", name.c_str());
    const double begin = offsets->arr[0].num, end = offsets->arr[1].num;
    double expected = 1.0;  // the reference multiplies in doubles
    for (const JVal& s : shape->arr) expected *= s.num;
    expected *= elem;
    if (end - begin != expected)
      return st_fail(WE_EFORMAT, "%s: has %s bytes, its shape needs %s bytes", name.c_str(), js_number(end - begin).c_str(),
                     js_number(expected).c_str());
    if (end > (double)data_size) return st_fail(WE_EFORMAT, "%s: data goes past the end of the file", name.c_str());
    we_safetensors::Tensor t;
    t.name = name;
    t.dtype = dtype->str;
    for (const JVal& s : shape->arr) t.shape.push_back((uint64_t)s.num);
    t.offset = start + (uint64_t)begin;
    t.size = (uint64_t)end - (uint64_t)begin;
    st.by_name[name] = (uint32_t)st.tensors.size();
    st.tensors.push_back(std::move(t));
  }

  // no two tensors share bytes (a stable sort by offset, as the reference's)
  std::vector<uint32_t> order(st.tensors.size());
  for (uint32_t i = 0; i < order.size(); i++) order[i] = i;
  std::stable_sort(order.begin(), order.end(),
                   [&](uint32_t a, uint32_t b) { return st.tensors[a].offset < st.tensors[b].offset; });
  for (size_t i = 1; i < order.size(); i++) {
    const auto& prev = st.tensors[order[i - 1]];
    const auto& cur = st.tensors[order[i]];
    if (cur.offset < prev.offset + prev.size)
      return st_fail(WE_EFORMAT, "%s and %s overlap", prev.name.c_str(), cur.name.c_str());
  }
  return WE_OK;
}

}  // namespace

extern "C" {

int we_st_open(const char* path, we_safetensors** out) {
  if (!path || !out) return st_fail(WE_EINVAL, "we_st_open: path and out must not be NULL");
  *out = nullptr;
  std::unique_ptr<we_safetensors> st(new we_safetensors);
  st->fd = open(path, O_RDONLY | O_CLOEXEC);
  if (st->fd < 0) return st_fail(WE_EIO, "cannot open %s: %s", path, strerror(errno));
  struct stat sb;
  if (fstat(st->fd, &sb) != 0) {
    const int e = errno;
    close(st->fd);
    return st_fail(WE_EIO, "cannot stat %s: %s", path, strerror(e));
  }
  st->file_size = (uint64_t)sb.st_size;
  const int rc = parse_header(*st);
  if (rc != WE_OK) {
    close(st->fd);
    return rc;
  }
  *out = st.release();
  return WE_OK;
}

int we_st_close(we_safetensors* st) {
  if (!st) return WE_OK;
  if (st->fd >= 0) close(st->fd);
  delete st;
  return WE_OK;
}

int we_st_count(const we_safetensors* st, uint32_t* n) {
  if (!st || !n) return st_fail(WE_EINVAL, "we_st_count: NULL argument");
  *n = (uint32_t)st->tensors.size();
  return WE_OK;
}

int we_st_info(const we_safetensors* st, uint32_t index, we_tensor_info* out) {
  if (!st || !out) return st_fail(WE_EINVAL, "we_st_info: NULL argument");
  if (index >= st->tensors.size())
    return st_fail(WE_EINVAL, "tensor index %u out of range (%zu tensors)", index, st->tensors.size());
  const auto& t = st->tensors[index];
  out->name = t.name.c_str();
  out->dtype = t.dtype.c_str();
  out->ndim = (uint32_t)t.shape.size();
  out->shape = t.shape.empty() ? nullptr : t.shape.data();
  out->offset = t.offset;
  out->size = t.size;
  return WE_OK;
}

int we_st_find(const we_safetensors* st, const char* name, uint32_t* index) {
  if (!st || !name || !index) return st_fail(WE_EINVAL, "we_st_find: NULL argument");
  const auto it = st->by_name.find(name);
  if (it == st->by_name.end()) return st_fail(WE_ENOTFOUND, "Missing tensor %s", name);
  *index = it->second;
  return WE_OK;
}

int we_st_metadata_count(const we_safetensors* st, uint32_t* n) {
  if (!st || !n) return st_fail(WE_EINVAL, "we_st_metadata_count: NULL argument");
  *n = (uint32_t)st->metadata.size();
  return WE_OK;
}

int we_st_metadata_at(const we_safetensors* st, uint32_t index, const char** key, const char** value) {
  if (!st || !key || !value) return st_fail(WE_EINVAL, "we_st_metadata_at: NULL argument");
  if (index >= st->metadata.size())
    return st_fail(WE_EINVAL, "metadata index %u out of range (%zu entries)", index, st->metadata.size());
  *key = st->metadata[index].first.c_str();
  *value = st->metadata[index].second.c_str();
  return WE_OK;
}

int we_st_read(const we_safetensors* st, uint32_t index, uint64_t begin, uint64_t bytes, void* dst, uint32_t threads) {
  if (!st || (!dst && bytes)) return st_fail(WE_EINVAL, "we_st_read: NULL argument");
  if (index >= st->tensors.size())
    return st_fail(WE_EINVAL, "tensor index %u out of range (%zu tensors)", index, st->tensors.size());
  const auto& t = st->tensors[index];
  if (begin > t.size || bytes > t.size - begin)
    return st_fail(WE_EINVAL, "%s: bytes [%llu, %llu) are outside its %llu bytes", t.name.c_str(),
                   (unsigned long long)begin, (unsigned long long)(begin + bytes), (unsigned long long)t.size);
  if (bytes == 0) return WE_OK;
  constexpr uint64_t kPiece = 8ull << 20;  // a thread reads at least this much
  uint64_t n = threads ? threads : 8;
  n = std::max<uint64_t>(1, std::min<uint64_t>(n, (bytes + kPiece - 1) / kPiece));
  const uint64_t off0 = t.offset + begin;
  char* d = (char*)dst;
  if (n == 1) {
    if (int e = read_all(st->fd, off0, bytes, d)) return st_fail(WE_EIO, "%s: read failed: %s", t.name.c_str(), strerror(e));
    return WE_OK;
  }
  // page-aligned pieces of ceil(bytes / n), so n pieces always cover the range; the last piece also runs to the
  // end of the range, whatever the rounding
  const uint64_t per = ((bytes + n - 1) / n + 4095) & ~4095ull;
  std::vector<int> errs(n, 0);
  std::vector<std::thread> pool;
  for (uint64_t i = 0; i < n; i++) {
    const uint64_t b = std::min(bytes, i * per), e = i + 1 == n ? bytes : std::min(bytes, b + per);
    if (b >= e) break;
    pool.emplace_back([&, i, b, e] { errs[i] = read_all(st->fd, off0 + b, e - b, d + b); });
  }
  for (auto& th : pool) th.join();
  for (int e : errs)
    if (e) return st_fail(WE_EIO, "%s: read failed: %s", t.name.c_str(), strerror(e));
  return WE_OK;
}

}  // extern "C"
