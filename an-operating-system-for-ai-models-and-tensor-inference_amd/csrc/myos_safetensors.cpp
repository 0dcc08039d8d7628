// SafeTensors reader. The format is the `safetensors` crate's (pinned 0.8.0 in
// the reference's Cargo.lock:101-103): u64 LE header size N, N bytes of JSON
// {name: {"dtype", "shape", "data_offsets": [begin, end]}, "__metadata__": {...}},
// then the payload. Offsets are relative to the payload start, must tile it
// without gaps or overlap and end at the file end (the crate's validate step).
#include "myos_safetensors.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>

#include "../../include/myos_hip.h"

namespace myos {
namespace {

// Minimal JSON reader: enough for SafeTensors headers (objects, arrays,
// strings with escapes, non-negative integers, and skipping other scalars).
struct Json {
  const char *p, *end;
  bool ok = true;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
  }
  bool lit(char c) {
    ws();
    if (p < end && *p == c) {
      p++;
      return true;
    }
    return false;
  }
  bool str(std::string &out) {
    ws();
    if (p >= end || *p != '"') return ok = false;
    p++;
    out.clear();
    while (p < end && *p != '"') {
      char c = *p++;
      if (c == '\\') {
        if (p >= end) return ok = false;
        char e = *p++;
        switch (e) {
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          case '/': out += '/'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {
            if (end - p < 4) return ok = false;
            unsigned v = 0;
            for (int i = 0; i < 4; i++) {
              char h = *p++;
              v <<= 4;
              if (h >= '0' && h <= '9') v |= h - '0';
              else if (h >= 'a' && h <= 'f') v |= h - 'a' + 10;
              else if (h >= 'A' && h <= 'F') v |= h - 'A' + 10;
              else return ok = false;
            }
            // names here are ASCII in practice; encode the BMP code point as UTF-8
            if (v < 0x80) out += (char)v;
            else if (v < 0x800) {
              out += (char)(0xC0 | (v >> 6));
              out += (char)(0x80 | (v & 0x3F));
            } else {
              out += (char)(0xE0 | (v >> 12));
              out += (char)(0x80 | ((v >> 6) & 0x3F));
              out += (char)(0x80 | (v & 0x3F));
            }
            break;
          }
          default: return ok = false;
        }
      } else {
        out += c;
      }
    }
    if (p >= end) return ok = false;
    p++;
    return true;
  }
  bool uint(uint64_t &v) {
    ws();
    if (p >= end || *p < '0' || *p > '9') return ok = false;
    v = 0;
    while (p < end && *p >= '0' && *p <= '9') {
      uint64_t nv = v * 10 + (uint64_t)(*p - '0');
      if (nv / 10 != v) return ok = false;  // overflow
      v = nv;
      p++;
    }
    return true;
  }
  bool skip() {  // any JSON value
    ws();
    if (p >= end) return ok = false;
    if (*p == '"') {
      std::string s;
      return str(s);
    }
    if (*p == '{') {
      p++;
      if (lit('}')) return true;
      do {
        std::string k;
        if (!str(k) || !lit(':') || !skip()) return ok = false;
      } while (lit(','));
      return lit('}') || (ok = false);
    }
    if (*p == '[') {
      p++;
      if (lit(']')) return true;
      do {
        if (!skip()) return ok = false;
      } while (lit(','));
      return lit(']') || (ok = false);
    }
    const char *s = p;
    while (p < end && (std::isalnum((unsigned char)*p) || *p == '-' || *p == '+' || *p == '.'))
      p++;
    return p > s || (ok = false);
  }
  bool uint_array(std::vector<uint64_t> &out) {
    out.clear();
    if (!lit('[')) return ok = false;
    if (lit(']')) return true;
    do {
      uint64_t v;
      if (!uint(v)) return ok = false;
      out.push_back(v);
    } while (lit(','));
    return lit(']') || (ok = false);
  }
};

struct Entry {
  std::string name;
  std::string dtype;
  std::vector<uint64_t> shape, offsets;
};

}  // namespace

SafeTensorsFile::~SafeTensorsFile() {
  if (map_) munmap(map_, len_);
}

int SafeTensorsFile::open(const char *path) {
  int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return MYOS_E_IO;
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    return MYOS_E_IO;
  }
  len_ = (size_t)st.st_size;
  if (len_ > 0) {
    map_ = mmap(nullptr, len_, PROT_READ, MAP_PRIVATE, fd, 0);
    if (map_ == MAP_FAILED) {
      map_ = nullptr;
      ::close(fd);
      return MYOS_E_IO;
    }
  }
  ::close(fd);
  const uint8_t *b = (const uint8_t *)map_;
  if (len_ < 8) return MYOS_E_PARSE;
  uint64_t n = 0;
  for (int i = 7; i >= 0; i--) n = (n << 8) | b[i];
  if (n > len_ - 8) return MYOS_E_PARSE;
  Json js{(const char *)b + 8, (const char *)b + 8 + n};
  const uint8_t *payload = b + 8 + n;
  const size_t payload_len = len_ - 8 - (size_t)n;
  std::vector<Entry> entries;
  if (!js.lit('{')) return MYOS_E_PARSE;
  if (!js.lit('}')) {
    do {
      Entry e;
      if (!js.str(e.name) || !js.lit(':')) return MYOS_E_PARSE;
      if (e.name == "__metadata__") {
        if (!js.skip()) return MYOS_E_PARSE;
        continue;
      }
      if (!js.lit('{')) return MYOS_E_PARSE;
      bool have_d = false, have_s = false, have_o = false;
      if (!js.lit('}')) {
        do {
          std::string key;
          if (!js.str(key) || !js.lit(':')) return MYOS_E_PARSE;
          if (key == "dtype") {
            if (!js.str(e.dtype)) return MYOS_E_PARSE;
            have_d = true;
          } else if (key == "shape") {
            if (!js.uint_array(e.shape)) return MYOS_E_PARSE;
            have_s = true;
          } else if (key == "data_offsets") {
            if (!js.uint_array(e.offsets) || e.offsets.size() != 2) return MYOS_E_PARSE;
            have_o = true;
          } else if (!js.skip()) {
            return MYOS_E_PARSE;
          }
        } while (js.lit(','));
        if (!js.lit('}')) return MYOS_E_PARSE;
      }
      if (!have_d || !have_s || !have_o) return MYOS_E_PARSE;
      entries.push_back(std::move(e));
    } while (js.lit(','));
    if (!js.lit('}')) return MYOS_E_PARSE;
  }
  js.ws();
  if (!js.ok) return MYOS_E_PARSE;
  // offsets must tile the payload exactly
  std::vector<const Entry *> order;
  for (auto &e : entries) order.push_back(&e);
  std::sort(order.begin(), order.end(), [](const Entry *a, const Entry *b) {
    return a->offsets[0] < b->offsets[0] ||
           (a->offsets[0] == b->offsets[0] && a->offsets[1] < b->offsets[1]);
  });
  uint64_t cursor = 0;
  for (const Entry *e : order) {
    if (e->offsets[0] != cursor || e->offsets[1] < e->offsets[0]) return MYOS_E_PARSE;
    cursor = e->offsets[1];
  }
  if (cursor != payload_len) return MYOS_E_PARSE;
  for (auto &e : entries) {
    StTensor t;
    size_t esize;
    if (e.dtype == "F32") {
      t.dtype = StDType::F32;
      esize = 4;
    } else if (e.dtype == "F16") {
      t.dtype = StDType::F16;
      esize = 2;
    } else if (e.dtype == "BF16") {
      t.dtype = StDType::BF16;
      esize = 2;
    } else {
      return MYOS_E_PARSE;  // WeightError::UnsupportedDType
    }
    if (e.name.empty()) return MYOS_E_PARSE;  // WeightError::EmptyName
    size_t numel = 1;
    for (uint64_t d : e.shape) {
      t.shape.push_back((size_t)d);
      if (d && numel > SIZE_MAX / d) return MYOS_E_W_LENGTH;
      numel *= (size_t)d;
    }
    if (numel > SIZE_MAX / esize) return MYOS_E_W_LENGTH;
    t.nbytes = (size_t)(e.offsets[1] - e.offsets[0]);
    if (t.nbytes != numel * esize) return MYOS_E_W_LENGTH;  // LengthMismatch
    t.data = payload + e.offsets[0];
    if (!tensors_.emplace(e.name, t).second) return MYOS_E_PARSE;  // Duplicate
  }
  return MYOS_OK;
}

const StTensor *SafeTensorsFile::find(const std::string &name) const {
  auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

int SafeTensorsFile::bf16(const std::string &name, const std::vector<size_t> &expect,
                          const uint16_t **out) const {
  const StTensor *t = find(name);
  if (!t) return MYOS_E_W_MISSING;
  if (t->dtype != StDType::BF16) return MYOS_E_W_DTYPE;
  if (t->shape != expect) return MYOS_E_W_SHAPE;
  if (out) *out = (const uint16_t *)t->data;
  return MYOS_OK;
}

}  // namespace myos
