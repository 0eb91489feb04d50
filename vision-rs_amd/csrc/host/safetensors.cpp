// Local safetensors reader for weight ingestion.
//
// Format (safetensors 0.x): an 8-byte little-endian header length N, N bytes
// of UTF-8 JSON mapping each tensor name to {"dtype", "shape", "data_offsets"
// [begin, end)} (offsets relative to the byte after the header), an optional
// "__metadata__" object of strings, then the raw little-endian tensor bytes.
// The reference reads the same files through teeny-data
// (examples/yolo26.rs:3403-3550, `SafeTensors::from_pretrained`, `tensors()`,
// `tensor(key).data()`); only the parse is restated here, the file comes from
// local disk.
#include <cstdio>
#include <cstring>

#include "vrs_internal.h"

namespace vrs {
namespace {

// Minimal JSON reader for the header: objects, arrays, strings (with escapes),
// integers and the literals; numbers with a fraction or exponent are skipped
// (they occur only in metadata).
struct Json {
  const char* p;
  const char* end;
  bool ok = true;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool eat(char c) {
    ws();
    if (p < end && *p == c) { ++p; return true; }
    return false;
  }
  bool str(std::string& out) {
    ws();
    if (p >= end || *p != '"') return ok = false;
    ++p;
    out.clear();
    while (p < end && *p != '"') {
      char c = *p++;
      if (c == '\\') {
        if (p >= end) return ok = false;
        const char e = *p++;
        switch (e) {
          case '"': case '\\': case '/': c = e; break;
          case 'b': c = '\b'; break;
          case 'f': c = '\f'; break;
          case 'n': c = '\n'; break;
          case 'r': c = '\r'; break;
          case 't': c = '\t'; break;
          case 'u': {
            if (end - p < 4) return ok = false;
            unsigned v = 0;
            for (int i = 0; i < 4; ++i) {
              const char h = *p++;
              v = v * 16 + (h >= '0' && h <= '9' ? h - '0' : h >= 'a' && h <= 'f' ? h - 'a' + 10
                                                   : h >= 'A' && h <= 'F' ? h - 'A' + 10 : 99);
              if (v > 0xffff) return ok = false;
            }
            // UTF-8 of the BMP code point (surrogate pairs are kept as two units)
            if (v < 0x80) { out += (char)v; }
            else if (v < 0x800) { out += (char)(0xc0 | (v >> 6)); out += (char)(0x80 | (v & 0x3f)); }
            else {
              out += (char)(0xe0 | (v >> 12));
              out += (char)(0x80 | ((v >> 6) & 0x3f));
              out += (char)(0x80 | (v & 0x3f));
            }
            continue;
          }
          default: return ok = false;
        }
      }
      out += c;
    }
    if (p >= end) return ok = false;
    ++p;
    return true;
  }
  bool integer(int64_t& v) {
    ws();
    bool neg = false;
    if (p < end && *p == '-') { neg = true; ++p; }
    if (p >= end || *p < '0' || *p > '9') return ok = false;
    v = 0;
    while (p < end && *p >= '0' && *p <= '9') {
      if (v > (INT64_MAX - 9) / 10) return ok = false;
      v = v * 10 + (*p++ - '0');
    }
    if (neg) v = -v;
    return true;
  }
  // skip any value
  bool skip(int depth = 0) {
    if (depth > 64) return ok = false;
    ws();
    if (p >= end) return ok = false;
    if (*p == '"') { std::string s; return str(s); }
    if (*p == '{' || *p == '[') {
      const char close = *p == '{' ? '}' : ']';
      const bool obj = *p == '{';
      ++p;
      if (eat(close)) return true;
      do {
        if (obj) {
          std::string k;
          if (!str(k) || !eat(':')) return ok = false;
        }
        if (!skip(depth + 1)) return false;
      } while (eat(','));
      return eat(close) || (ok = false);
    }
    // number or literal
    const char* s = p;
    while (p < end && *p != ',' && *p != '}' && *p != ']' && *p != ' ' && *p != '\n' && *p != '\r' && *p != '\t') ++p;
    return p > s || (ok = false);
  }
};

int dtype_size(const std::string& d) {
  if (d == "F32" || d == "I32" || d == "U32") return 4;
  if (d == "F16" || d == "BF16" || d == "I16" || d == "U16") return 2;
  if (d == "F64" || d == "I64" || d == "U64") return 8;
  if (d == "I8" || d == "U8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
  return 0;
}

float half_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = s;
    } else {  // subnormal: normalise
      int sh = 0;
      uint32_t mm = m;
      while (!(mm & 0x400)) { mm <<= 1; ++sh; }
      bits = s | ((uint32_t)(127 - 15 - sh + 1) << 23) | ((mm & 0x3ff) << 13);
    }
  } else if (e == 31) {
    bits = s | 0x7f800000u | (m << 13);
  } else {
    bits = s | ((e + 127 - 15) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

}  // namespace

int st_open(const char* path, StFile& f) {
  f = StFile{};
  FILE* fp = fopen(path, "rb");
  if (!fp) return fail(VRS_EINVAL, "safetensors: cannot open '%s'", path);
  if (fseek(fp, 0, SEEK_END) != 0) { fclose(fp); return fail(VRS_EINVAL, "safetensors: cannot seek '%s'", path); }
  const long sz = ftell(fp);
  rewind(fp);
  if (sz < 8) { fclose(fp); return fail(VRS_EBADSHAPE, "safetensors: '%s' is too short", path); }
  f.bytes.resize((size_t)sz);
  const size_t got = fread(f.bytes.data(), 1, (size_t)sz, fp);
  fclose(fp);
  if (got != (size_t)sz) return fail(VRS_EINVAL, "safetensors: short read of '%s'", path);
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | (unsigned char)f.bytes[i];
  if (n > (uint64_t)sz - 8) return fail(VRS_EBADSHAPE, "safetensors: header length %llu exceeds the file", (unsigned long long)n);
  f.data_begin = 8 + (size_t)n;
  Json j{f.bytes.data() + 8, f.bytes.data() + 8 + n};
  if (!j.eat('{')) return fail(VRS_EBADSHAPE, "safetensors: header is not a JSON object");
  if (!j.eat('}')) {
    do {
      std::string name;
      if (!j.str(name) || !j.eat(':')) return fail(VRS_EBADSHAPE, "safetensors: malformed header");
      if (name == "__metadata__") {
        if (!j.skip()) return fail(VRS_EBADSHAPE, "safetensors: malformed metadata");
        continue;
      }
      StTensor t;
      bool have_off = false, have_dt = false, have_shape = false;
      if (!j.eat('{')) return fail(VRS_EBADSHAPE, "safetensors: entry '%s' is not an object", name.c_str());
      if (!j.eat('}')) {
        do {
          std::string key;
          if (!j.str(key) || !j.eat(':')) return fail(VRS_EBADSHAPE, "safetensors: malformed entry '%s'", name.c_str());
          if (key == "dtype") {
            if (!j.str(t.dtype)) return fail(VRS_EBADSHAPE, "safetensors: '%s' dtype", name.c_str());
            have_dt = true;
          } else if (key == "shape") {
            if (!j.eat('[')) return fail(VRS_EBADSHAPE, "safetensors: '%s' shape", name.c_str());
            if (!j.eat(']')) {
              do {
                int64_t d;
                if (!j.integer(d) || d < 0) return fail(VRS_EBADSHAPE, "safetensors: '%s' shape", name.c_str());
                t.shape.push_back(d);
              } while (j.eat(','));
              if (!j.eat(']')) return fail(VRS_EBADSHAPE, "safetensors: '%s' shape", name.c_str());
            }
            have_shape = true;
          } else if (key == "data_offsets") {
            int64_t a = -1, b = -1;
            if (!j.eat('[') || !j.integer(a) || !j.eat(',') || !j.integer(b) || !j.eat(']'))
              return fail(VRS_EBADSHAPE, "safetensors: '%s' data_offsets", name.c_str());
            if (a < 0 || b < a) return fail(VRS_EBADSHAPE, "safetensors: '%s' data_offsets", name.c_str());
            t.begin = (size_t)a;
            t.end = (size_t)b;
            have_off = true;
          } else if (!j.skip()) {
            return fail(VRS_EBADSHAPE, "safetensors: malformed entry '%s'", name.c_str());
          }
        } while (j.eat(','));
        if (!j.eat('}')) return fail(VRS_EBADSHAPE, "safetensors: malformed entry '%s'", name.c_str());
      }
      if (!have_off || !have_dt || !have_shape)
        return fail(VRS_EBADSHAPE, "safetensors: entry '%s' lacks dtype/shape/data_offsets", name.c_str());
      // element and byte counts of an untrusted header: every product is
      // checked before it is formed (a crafted shape must not overflow)
      int64_t numel = 1;
      for (int64_t d : t.shape) {
        if (d > 0 && numel > INT64_MAX / d)
          return fail(VRS_EBADSHAPE, "safetensors: '%s' shape overflows 64-bit element counts", name.c_str());
        numel *= d;
      }
      const int es = dtype_size(t.dtype);
      if (es == 0) return fail(VRS_EUNSUPPORTED, "safetensors: '%s' has unknown dtype %s", name.c_str(), t.dtype.c_str());
      if (numel > INT64_MAX / es)
        return fail(VRS_EBADSHAPE, "safetensors: '%s' byte size overflows", name.c_str());
      if ((int64_t)(t.end - t.begin) != numel * es)
        return fail(VRS_EBADSHAPE, "safetensors: '%s' spans %zu bytes for %lld %s values", name.c_str(),
                    t.end - t.begin, (long long)numel, t.dtype.c_str());
      if (f.data_begin + t.end > f.bytes.size())
        return fail(VRS_EBADSHAPE, "safetensors: '%s' runs past the end of the file", name.c_str());
      t.numel = numel;
      f.tensors[name] = t;
    } while (j.eat(','));
    if (!j.eat('}')) return fail(VRS_EBADSHAPE, "safetensors: malformed header");
  }
  return VRS_OK;
}

const StTensor* st_find(const StFile& f, const std::string& name) {
  auto it = f.tensors.find(name);
  return it == f.tensors.end() ? nullptr : &it->second;
}

int st_to_f32(const StFile& f, const std::string& name, const StTensor& t, std::vector<float>& out) {
  const unsigned char* src = reinterpret_cast<const unsigned char*>(f.bytes.data() + f.data_begin + t.begin);
  out.resize((size_t)t.numel);
  if (t.dtype == "F32") {
    memcpy(out.data(), src, (size_t)t.numel * 4);   // little-endian host
  } else if (t.dtype == "F16") {
    for (int64_t i = 0; i < t.numel; ++i) out[i] = half_to_f32((uint16_t)(src[2 * i] | (src[2 * i + 1] << 8)));
  } else if (t.dtype == "BF16") {
    for (int64_t i = 0; i < t.numel; ++i) {
      const uint32_t bits = (uint32_t)(src[2 * i] | (src[2 * i + 1] << 8)) << 16;
      memcpy(&out[i], &bits, 4);
    }
  } else if (t.dtype == "F64") {
    for (int64_t i = 0; i < t.numel; ++i) {
      double d;
      memcpy(&d, src + 8 * i, 8);
      out[i] = (float)d;
    }
  } else {
    return fail(VRS_EUNSUPPORTED, "safetensors: '%s' is %s (F32, F16, BF16 or F64 expected)", name.c_str(),
                t.dtype.c_str());
  }
  return VRS_OK;
}

}  // namespace vrs
