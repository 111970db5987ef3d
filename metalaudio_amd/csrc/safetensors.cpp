// SafeTensors reader: header parsing with bounds and overflow checks, fp32 conversion.
// Follows SafeTensorsLoader.swift:401-660 (parseHeader, loadRawTensorData, convertToFloat32,
// validateWeights); the JSON reader below covers the header grammar (objects, arrays, strings
// with escapes, numbers, true/false/null) and nothing else.
#include "safetensors.hpp"

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>

#include "common.hpp"

namespace mnn {

namespace {

[[noreturn]] void bad_file(const std::string& what) { fail(MNN_ERR_INVALID_FILE, what); }

// ------------------------------------------------------------------ minimal JSON
struct JVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  double num = 0.0;
  bool is_int = false;
  int64_t inum = 0;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
};

class JParser {
 public:
  JParser(const char* p, size_t n) : p_(p), end_(p + n) {}
  JVal parse_document() {
    JVal v = value(0);
    ws();
    if (p_ != end_) bad_file("invalid header JSON: trailing characters");
    return v;
  }

 private:
  static constexpr int kMaxDepth = 64;
  const char* p_;
  const char* end_;

  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  char peek() {
    ws();
    if (p_ >= end_) bad_file("invalid header JSON: unexpected end");
    return *p_;
  }
  void expect(char c) {
    if (peek() != c) bad_file(std::string("invalid header JSON: expected '") + c + "'");
    ++p_;
  }
  bool literal(const char* lit) {
    const size_t n = std::strlen(lit);
    if ((size_t)(end_ - p_) >= n && std::memcmp(p_, lit, n) == 0) {
      p_ += n;
      return true;
    }
    return false;
  }
  static void put_utf8(std::string& s, uint32_t cp) {
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
  uint32_t hex4() {
    if (end_ - p_ < 4) bad_file("invalid header JSON: short \\u escape");
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else bad_file("invalid header JSON: bad \\u escape");
    }
    return v;
  }
  std::string string() {
    expect('"');
    std::string s;
    while (true) {
      if (p_ >= end_) bad_file("invalid header JSON: unterminated string");
      const char c = *p_++;
      if (c == '"') return s;
      if ((unsigned char)c < 0x20) bad_file("invalid header JSON: control character in string");
      if (c != '\\') {
        s += c;
        continue;
      }
      if (p_ >= end_) bad_file("invalid header JSON: unterminated escape");
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
          uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            if (!literal("\\u")) bad_file("invalid header JSON: lone surrogate");
            const uint32_t lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) bad_file("invalid header JSON: bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            bad_file("invalid header JSON: lone surrogate");
          }
          put_utf8(s, cp);
          break;
        }
        default: bad_file("invalid header JSON: bad escape");
      }
    }
  }
  JVal number() {
    const char* s = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    bool frac = false;
    while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' ||
                         *p_ == '+' || *p_ == '-')) {
      if (*p_ == '.' || *p_ == 'e' || *p_ == 'E') frac = true;
      ++p_;
    }
    const std::string tok(s, p_);
    if (tok.empty() || tok == "-") bad_file("invalid header JSON: bad number");
    JVal v;
    v.kind = JVal::NUM;
    char* stop = nullptr;
    v.num = std::strtod(tok.c_str(), &stop);
    if (stop != tok.c_str() + tok.size()) bad_file("invalid header JSON: bad number '" + tok + "'");
    if (!frac) {
      errno = 0;
      const long long i = std::strtoll(tok.c_str(), &stop, 10);
      if (errno == 0 && stop == tok.c_str() + tok.size()) {
        v.is_int = true;
        v.inum = i;
      }
    }
    return v;
  }
  JVal value(int depth) {
    if (depth > kMaxDepth) bad_file("invalid header JSON: nesting too deep");
    const char c = peek();
    JVal v;
    if (c == '{') {
      ++p_;
      v.kind = JVal::OBJ;
      if (peek() == '}') {
        ++p_;
        return v;
      }
      while (true) {
        std::string k = string();
        expect(':');
        v.obj.emplace_back(std::move(k), value(depth + 1));
        if (peek() == ',') {
          ++p_;
          continue;
        }
        expect('}');
        return v;
      }
    }
    if (c == '[') {
      ++p_;
      v.kind = JVal::ARR;
      if (peek() == ']') {
        ++p_;
        return v;
      }
      while (true) {
        v.arr.push_back(value(depth + 1));
        if (peek() == ',') {
          ++p_;
          continue;
        }
        expect(']');
        return v;
      }
    }
    if (c == '"') {
      v.kind = JVal::STR;
      v.str = string();
      return v;
    }
    if (literal("true")) {
      v.kind = JVal::BOOL;
      v.num = 1;
      return v;
    }
    if (literal("false")) {
      v.kind = JVal::BOOL;
      return v;
    }
    if (literal("null")) return v;
    return number();
  }
};

bool valid_utf8(const unsigned char* s, size_t n) {
  size_t i = 0;
  while (i < n) {
    const unsigned char c = s[i];
    int len;
    uint32_t cp;
    if (c < 0x80) {
      ++i;
      continue;
    } else if ((c & 0xE0) == 0xC0) {
      len = 2;
      cp = c & 0x1F;
    } else if ((c & 0xF0) == 0xE0) {
      len = 3;
      cp = c & 0x0F;
    } else if ((c & 0xF8) == 0xF0) {
      len = 4;
      cp = c & 0x07;
    } else {
      return false;
    }
    if (i + len > n) return false;
    for (int k = 1; k < len; ++k) {
      if ((s[i + k] & 0xC0) != 0x80) return false;
      cp = (cp << 6) | (s[i + k] & 0x3F);
    }
    if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) ||
        cp > 0x10FFFF || (cp >= 0xD800 && cp < 0xE000))
      return false;
    i += len;
  }
  return true;
}

bool dtype_from_string(const std::string& s, StDType& t) {
  static const std::pair<const char*, StDType> kNames[] = {
      {"F32", ST_F32}, {"F16", ST_F16}, {"BF16", ST_BF16}, {"I32", ST_I32}, {"I64", ST_I64},
      {"I16", ST_I16}, {"I8", ST_I8},   {"U8", ST_U8},     {"BOOL", ST_BOOL}};
  for (const auto& kv : kNames)
    if (s == kv.first) {
      t = kv.second;
      return true;
    }
  return false;
}

template <class T>
T load_le(const unsigned char* p) {
  T v;
  std::memcpy(&v, p, sizeof(T));  // x86-64 and gfx950 hosts are little-endian
  return v;
}

}  // namespace

size_t st_dtype_size(StDType t) {
  switch (t) {
    case ST_F32:
    case ST_I32: return 4;
    case ST_F16:
    case ST_BF16:
    case ST_I16: return 2;
    case ST_I64: return 8;
    default: return 1;
  }
}

int64_t StTensorInfo::count() const {
  MNN_REQUIRE(end >= begin, MNN_ERR_INVALID_FILE,
              "tensor byte range [" << begin << ", " << end << ") is reversed");
  return (int64_t)((end - begin) / st_dtype_size(dtype));
}

float st_half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1F, man = h & 0x3FF;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {  // subnormal: man * 2^-24, renormalised
      int e = -1;
      uint32_t m = man;
      do {
        ++e;
        m <<= 1;
      } while ((m & 0x400) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3FF) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);  // inf / nan (payload kept)
  } else {
    bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

SafeTensorsFile::SafeTensorsFile(const std::string& path) : path_(path) {
  f_ = std::fopen(path.c_str(), "rb");
  MNN_REQUIRE(f_, MNN_ERR_FILE_NOT_FOUND, "SafeTensors file not found at: " << path);
  try {
    MNN_REQUIRE(std::fseek(f_, 0, SEEK_END) == 0, MNN_ERR_INVALID_FILE, "cannot seek " << path);
    const long fsz = std::ftell(f_);
    MNN_REQUIRE(fsz >= 0, MNN_ERR_INVALID_FILE, "cannot size " << path);
    std::rewind(f_);
    unsigned char len8[8];
    if ((uint64_t)fsz < 8 || std::fread(len8, 1, 8, f_) != 8)
      bad_file("invalid header JSON: cannot read header size");
    const uint64_t hlen = load_le<uint64_t>(len8);
    MNN_REQUIRE(hlen <= kMaxHeader, MNN_ERR_INVALID_FILE,
                "header size " << hlen << " exceeds maximum " << kMaxHeader);
    if (hlen > (uint64_t)fsz - 8) bad_file("invalid header JSON: header truncated");
    std::vector<unsigned char> hdr(hlen);
    if (hlen && std::fread(hdr.data(), 1, hlen, f_) != hlen)
      bad_file("invalid header JSON: header truncated");
    if (!valid_utf8(hdr.data(), hdr.size())) bad_file("header is not valid UTF-8");
    JParser jp(reinterpret_cast<const char*>(hdr.data()), hdr.size());
    const JVal root = jp.parse_document();
    if (root.kind != JVal::OBJ) bad_file("invalid header JSON: not an object");
    data_start_ = 8 + hlen;
    data_size_ = (uint64_t)fsz - data_start_;
    for (const auto& kv : root.obj) {
      if (kv.first == "__metadata__") {
        if (kv.second.kind == JVal::OBJ)
          for (const auto& m : kv.second.obj)
            if (m.second.kind == JVal::STR) meta_[m.first] = m.second.str;
        continue;
      }
      // malformed entries and unknown dtypes are skipped, as the reference does
      // (SafeTensorsLoader.swift:448-466)
      const JVal& e = kv.second;
      if (e.kind != JVal::OBJ) continue;
      const JVal *dt = nullptr, *sh = nullptr, *off = nullptr;
      for (const auto& f : e.obj) {
        if (f.first == "dtype") dt = &f.second;
        else if (f.first == "shape") sh = &f.second;
        else if (f.first == "data_offsets") off = &f.second;
      }
      if (!dt || dt->kind != JVal::STR || !sh || sh->kind != JVal::ARR || !off ||
          off->kind != JVal::ARR || off->arr.size() != 2)
        continue;
      StTensorInfo ti;
      if (!dtype_from_string(dt->str, ti.dtype)) continue;
      bool ok = true;
      for (const JVal& d : sh->arr) {
        if (d.kind != JVal::NUM || !d.is_int || d.inum < 0) ok = false;
        else ti.shape.push_back(d.inum);
      }
      for (const JVal& o : off->arr)
        if (o.kind != JVal::NUM || !o.is_int || o.inum < 0) ok = false;
      if (!ok) continue;
      ti.begin = (uint64_t)off->arr[0].inum;
      ti.end = (uint64_t)off->arr[1].inum;
      infos_[kv.first] = ti;
      names_.push_back(kv.first);
    }
    std::sort(names_.begin(), names_.end());
  } catch (...) {
    std::fclose(f_);
    f_ = nullptr;
    throw;
  }
}

SafeTensorsFile::~SafeTensorsFile() {
  if (f_) std::fclose(f_);
}

const StTensorInfo& SafeTensorsFile::info(const std::string& name) const {
  auto it = infos_.find(name);
  MNN_REQUIRE(it != infos_.end(), MNN_ERR_TENSOR_NOT_FOUND,
              "Tensor '" << name << "' not found in SafeTensors file");
  return it->second;
}

void SafeTensorsFile::read_f32(const std::string& name, float* out, size_t count) const {
  const StTensorInfo& ti = info(name);
  const size_t es = st_dtype_size(ti.dtype);
  MNN_REQUIRE(ti.end >= ti.begin && ti.end <= data_size_, MNN_ERR_INVALID_FILE,
              "Tensor '" << name << "' offset " << ti.end << " exceeds data size " << data_size_);
  const uint64_t bytes = ti.end - ti.begin;
  MNN_REQUIRE(bytes % es == 0, MNN_ERR_INVALID_FILE,
              "Tensor '" << name << "' data truncated: " << bytes << " bytes is not a multiple of "
                         << es);
  const uint64_t n = bytes / es;
  MNN_REQUIRE(n == count, MNN_ERR_BUFFER_SIZE_MISMATCH,
              "Tensor '" << name << "' holds " << n << " values, the destination " << count);
  MNN_REQUIRE(out || n == 0, MNN_ERR_INVALID_ARGUMENT, "null destination");
  std::vector<unsigned char> raw(bytes);
  if (bytes) {
    MNN_REQUIRE(std::fseek(f_, (long)(data_start_ + ti.begin), SEEK_SET) == 0,
                MNN_ERR_INVALID_FILE, "cannot seek to tensor '" << name << "'");
    MNN_REQUIRE(std::fread(raw.data(), 1, bytes, f_) == bytes, MNN_ERR_INVALID_FILE,
                "Tensor '" << name << "' data truncated");
  }
  const unsigned char* p = raw.data();
  for (uint64_t i = 0; i < n; ++i, p += es) {
    float v;
    switch (ti.dtype) {
      case ST_F32: v = load_le<float>(p); break;
      case ST_F16: v = st_half_to_float(load_le<uint16_t>(p)); break;
      case ST_BF16: {
        const uint32_t b = (uint32_t)load_le<uint16_t>(p) << 16;
        std::memcpy(&v, &b, 4);
        break;
      }
      case ST_I32: v = (float)load_le<int32_t>(p); break;
      case ST_I64: v = (float)load_le<int64_t>(p); break;
      case ST_I16: v = (float)load_le<int16_t>(p); break;
      case ST_I8: v = (float)load_le<int8_t>(p); break;
      case ST_U8: v = (float)*p; break;
      default: v = *p ? 1.f : 0.f; break;
    }
    MNN_REQUIRE(!std::isnan(v), MNN_ERR_INVALID_CONFIGURATION,
                "Corrupted weights in '" << name << "': Contains NaN");
    MNN_REQUIRE(!std::isinf(v), MNN_ERR_INVALID_CONFIGURATION,
                "Corrupted weights in '" << name << "': Contains Inf");
    out[i] = v;
  }
}

}  // namespace mnn

// ------------------------------------------------------------------ MTLA
namespace mnn {

uint32_t crc32_ieee(const unsigned char* p, size_t n, uint32_t crc) {
  static const auto table = [] {
    std::vector<uint32_t> t(256);
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int k = 0; k < 8; ++k) c = (c & 1) ? (c >> 1) ^ 0xEDB88320u : (c >> 1);
      t[i] = c;
    }
    return t;
  }();
  crc = ~crc;
  for (size_t i = 0; i < n; ++i) crc = table[(crc ^ p[i]) & 0xFF] ^ (crc >> 8);
  return ~crc;
}

MtlaFile::MtlaFile(const std::string& path) {
  FILE* f = std::fopen(path.c_str(), "rb");
  MNN_REQUIRE(f, MNN_ERR_FILE_NOT_FOUND, "model file not found at: " << path);
  std::vector<unsigned char> d;
  {
    std::unique_ptr<FILE, int (*)(FILE*)> guard(f, &std::fclose);
    MNN_REQUIRE(std::fseek(f, 0, SEEK_END) == 0, MNN_ERR_INVALID_FILE, "cannot seek " << path);
    const long n = std::ftell(f);
    MNN_REQUIRE(n >= 0, MNN_ERR_INVALID_FILE, "cannot size " << path);
    std::rewind(f);
    d.resize((size_t)n);
    MNN_REQUIRE(d.empty() || std::fread(d.data(), 1, d.size(), f) == d.size(),
                MNN_ERR_INVALID_FILE, "cannot read " << path);
  }
  size_t off = 0;
  auto need = [&](size_t n) {
    MNN_REQUIRE(n <= d.size() && off <= d.size() - n, MNN_ERR_INVALID_FILE,
                "Unexpected end of file at offset " << off << ": needed " << n
                                                    << " bytes, file size is " << d.size());
    const size_t at = off;
    off += n;
    return at;
  };
  auto u32 = [&] { return load_le<uint32_t>(d.data() + need(4)); };
  MNN_REQUIRE(d.size() >= 16, MNN_ERR_INVALID_FILE,
              "File too small: expected at least 16 bytes, got " << d.size());
  const uint32_t magic = u32();
  MNN_REQUIRE(magic == kMagic, MNN_ERR_INVALID_FILE, "Invalid magic number: 0x" << std::hex
                                                                              << magic);
  const uint32_t version = u32();
  MNN_REQUIRE(version == 1 || version == 2, MNN_ERR_INVALID_FILE,
              "Unsupported version " << version << ", only version 2 is supported");
  const uint32_t count = u32();
  if (version == 1) {
    (void)u32();  // reserved
  } else {
    MNN_REQUIRE(d.size() >= 20, MNN_ERR_INVALID_FILE,
                "File too small: expected at least 20 bytes, got " << d.size());
    const uint32_t stored = u32();
    (void)u32();  // reserved
    const uint32_t actual = crc32_ieee(d.data() + 20, d.size() - 20);
    MNN_REQUIRE(stored == actual, MNN_ERR_INVALID_FILE,
                "Checksum mismatch: expected 0x" << std::hex << stored << ", got 0x" << actual);
  }
  for (uint32_t k = 0; k < count; ++k) {
    const uint32_t name_len = u32(), rank = u32();
    (void)u32();  // data type: f32
    const uint32_t bytes = u32();
    MNN_REQUIRE(name_len < 1024, MNN_ERR_INVALID_FILE, "Invalid tensor name (too long)");
    MNN_REQUIRE(rank <= 16, MNN_ERR_INVALID_CONFIGURATION,
                "tensor has " << rank << " dimensions, maximum 16 allowed");
    const size_t at = need(name_len);
    MNN_REQUIRE(valid_utf8(d.data() + at, name_len), MNN_ERR_INVALID_FILE,
                "Invalid tensor name (not valid UTF-8)");
    std::string name(reinterpret_cast<const char*>(d.data() + at), name_len);
    std::vector<int64_t> shape;
    uint64_t elems = 1;
    for (uint32_t r = 0; r < rank; ++r) {
      const uint32_t dim = u32();
      shape.push_back(dim);
      MNN_REQUIRE(dim == 0 || elems <= UINT64_MAX / dim, MNN_ERR_INVALID_FILE,
                  "tensor shape in model file overflows");
      elems *= dim;
    }
    MNN_REQUIRE(elems <= UINT64_MAX / 4 && (uint64_t)bytes == elems * 4, MNN_ERR_INVALID_FILE,
                "Tensor '" << name << "' declares " << bytes << " bytes but shape requires "
                           << elems * 4 << " bytes");
    const size_t dat = need(bytes);
    std::vector<float> v((size_t)elems);
    if (bytes) std::memcpy(v.data(), d.data() + dat, bytes);
    t_[name] = {std::move(shape), std::move(v)};
  }
  for (const auto& kv : t_) names_.push_back(kv.first);  // map order: sorted
}

const std::vector<int64_t>& MtlaFile::shape(const std::string& name) const {
  auto it = t_.find(name);
  MNN_REQUIRE(it != t_.end(), MNN_ERR_TENSOR_NOT_FOUND, "Tensor '" << name << "' not found");
  return it->second.first;
}

const std::vector<float>& MtlaFile::data(const std::string& name) const {
  auto it = t_.find(name);
  MNN_REQUIRE(it != t_.end(), MNN_ERR_TENSOR_NOT_FOUND, "Tensor '" << name << "' not found");
  return it->second.second;
}

void mtla_write(const std::string& path,
                const std::map<std::string, std::pair<std::vector<int64_t>, std::vector<float>>>& t) {
  std::vector<unsigned char> body;
  auto put32 = [&](uint32_t v) {
    unsigned char b[4];
    std::memcpy(b, &v, 4);
    body.insert(body.end(), b, b + 4);
  };
  for (const auto& kv : t) {  // std::map: name order, as the reference's sorted keys
    const auto& shape = kv.second.first;
    const auto& v = kv.second.second;
    MNN_REQUIRE(kv.first.size() < 1024 && shape.size() <= 16, MNN_ERR_INVALID_ARGUMENT,
                "tensor '" << kv.first << "': name or rank too large");
    uint64_t elems = 1;
    for (int64_t dmn : shape) {
      MNN_REQUIRE(dmn >= 0 && dmn <= UINT32_MAX, MNN_ERR_INVALID_ARGUMENT, "bad dimension");
      elems *= (uint64_t)dmn;
    }
    MNN_REQUIRE(elems == v.size() && elems * 4 <= UINT32_MAX, MNN_ERR_INVALID_ARGUMENT,
                "tensor '" << kv.first << "': data does not match its shape");
    put32((uint32_t)kv.first.size());
    put32((uint32_t)shape.size());
    put32(0);
    put32((uint32_t)(elems * 4));
    body.insert(body.end(), kv.first.begin(), kv.first.end());
    for (int64_t dmn : shape) put32((uint32_t)dmn);
    const auto* p = reinterpret_cast<const unsigned char*>(v.data());
    body.insert(body.end(), p, p + elems * 4);
  }
  std::vector<unsigned char> out;
  const uint32_t hdr[5] = {MtlaFile::kMagic, 2u, (uint32_t)t.size(),
                           crc32_ieee(body.data(), body.size()), 0u};
  const auto* hp = reinterpret_cast<const unsigned char*>(hdr);
  out.insert(out.end(), hp, hp + sizeof(hdr));
  out.insert(out.end(), body.begin(), body.end());
  FILE* f = std::fopen(path.c_str(), "wb");
  MNN_REQUIRE(f, MNN_ERR_INVALID_ARGUMENT, "cannot write " << path);
  const size_t wrote = std::fwrite(out.data(), 1, out.size(), f);
  const int closed = std::fclose(f);
  MNN_REQUIRE(wrote == out.size() && closed == 0, MNN_ERR_INVALID_ARGUMENT,
              "write to " << path << " failed");
}

}  // namespace mnn
