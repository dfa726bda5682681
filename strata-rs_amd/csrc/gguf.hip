// GGUF v3 reader (host code): see gguf.hpp. Follows
// crates/strata-gguf/src/reader.rs:22-353 step for step, including its
// limits (strings of at most 65,535 bytes, arrays of at most 2^24 items,
// nesting of at most two array levels, 1..4 dims) and its choices (a
// duplicate metadata key keeps the last value; only integer-typed
// `general.alignment` values count, and a u64 one reads as 0 as in
// MetaValue::as_int, so it falls back to 32).
#include "gguf.hpp"

#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <unordered_set>

namespace sh {

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF"
constexpr uint32_t kVersion = 3;
constexpr uint64_t kMaxArrayLen = uint64_t(1) << 24;
constexpr uint64_t kKeepAllBelow = uint64_t(1) << 20;  // reader.rs:166-170
constexpr uint64_t kItemsKept = 64;                     // metadata.rs MAX_ARRAY_ITEMS_KEPT

enum : uint32_t {
  kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kString, kArray, kU64, kI64, kF64,
};

std::string fmt(const char* f, unsigned long long a, unsigned long long b = 0) {
  char buf[160];
  snprintf(buf, sizeof buf, f, a, b);
  return buf;
}

// Rust's str::from_utf8 acceptance (no overlongs, no surrogates, <= U+10FFFF).
bool valid_utf8(const uint8_t* p, uint64_t n) {
  uint64_t i = 0;
  while (i < n) {
    const uint8_t c = p[i];
    if (c < 0x80) {
      ++i;
      continue;
    }
    int len;
    uint8_t lo = 0x80, hi = 0xBF;
    if (c >= 0xC2 && c <= 0xDF) {
      len = 2;
    } else if (c >= 0xE0 && c <= 0xEF) {
      len = 3;
      if (c == 0xE0) lo = 0xA0;
      if (c == 0xED) hi = 0x9F;
    } else if (c >= 0xF0 && c <= 0xF4) {
      len = 4;
      if (c == 0xF0) lo = 0x90;
      if (c == 0xF4) hi = 0x8F;
    } else {
      return false;
    }
    if (n - i < uint64_t(len)) return false;
    if (p[i + 1] < lo || p[i + 1] > hi) return false;
    for (int k = 2; k < len; ++k)
      if (p[i + k] < 0x80 || p[i + k] > 0xBF) return false;
    i += len;
  }
  return true;
}

struct Cursor {
  const uint8_t* d;
  uint64_t n;
  uint64_t pos = 0;
  GgufErr err = GgufErr::kOk;
  std::string msg;

  bool need(uint64_t k) {
    if (k > n - pos) {  // pos <= n always
      err = GgufErr::kTruncated;
      msg = fmt("truncated: expected %llu bytes, found %llu", k, n - pos);
      return false;
    }
    return true;
  }
  template <class T>
  bool get(T* v) {
    if (!need(sizeof(T))) return false;
    memcpy(v, d + pos, sizeof(T));  // little-endian host
    pos += sizeof(T);
    return true;
  }
  bool string(std::string* s) {
    uint64_t len;
    if (!get(&len)) return false;
    if (len > 65535) {
      err = GgufErr::kBadKeyLength;
      msg = fmt("bad key length %llu", len);
      return false;
    }
    if (!need(len)) return false;
    if (!valid_utf8(d + pos, len)) {
      err = GgufErr::kStringNotUtf8;
      msg = "string is not UTF-8";
      return false;
    }
    s->assign(reinterpret_cast<const char*>(d + pos), size_t(len));
    pos += len;
    return true;
  }
  bool bad_type(uint32_t t) {
    err = GgufErr::kBadValueType;
    msg = fmt("bad metadata value type %llu", t);
    return false;
  }
  // reader.rs:123-176
  bool value(uint32_t ty, int depth, GgufMeta* v) {
    if (depth > 2) return bad_type(9);
    v->ty = ty;
    switch (ty) {
      case kU8: { uint8_t x; if (!get(&x)) return false; v->i = x; return true; }
      case kI8: { int8_t x; if (!get(&x)) return false; v->i = x; return true; }
      case kU16: { uint16_t x; if (!get(&x)) return false; v->i = x; return true; }
      case kI16: { int16_t x; if (!get(&x)) return false; v->i = x; return true; }
      case kU32: { uint32_t x; if (!get(&x)) return false; v->i = x; return true; }
      case kI32: { int32_t x; if (!get(&x)) return false; v->i = x; return true; }
      case kF32: { float x; if (!get(&x)) return false; v->f = x; return true; }
      case kBool: { uint8_t x; if (!get(&x)) return false; v->i = x != 0; return true; }
      case kString: return string(&v->s);
      case kU64: return get(&v->u);
      case kI64: return get(&v->i);
      case kF64: return get(&v->f);
      case kArray: {
        uint32_t elem;
        if (!get(&elem)) return false;
        if (elem > kF64) return bad_type(elem);
        uint64_t count;
        if (!get(&count)) return false;
        if (count > kMaxArrayLen) return bad_type(9);
        v->elem = elem;
        v->count = count;
        // the reference parses every item of arrays up to 2^20 long and the
        // first 64 of longer ones (reader.rs:159-172)
        const uint64_t keep = count <= kKeepAllBelow ? count : kItemsKept;
        GgufMeta item;
        for (uint64_t k = 0; k < keep; ++k)
          if (!value(elem, depth + 1, &item)) return false;
        return true;
      }
      default: return bad_type(ty);
    }
  }
};

}  // namespace

GgufFile::~GgufFile() {
  if (map) munmap(const_cast<uint8_t*>(map), size_t(size));
}

void gguf_type_geometry(uint32_t ty, uint64_t* block, uint64_t* bytes) {
  uint64_t b = 0, s = 0;
  switch (ty) {
    case 0: b = 1; s = 4; break;    // F32
    case 1: b = 1; s = 2; break;    // F16
    case 30: b = 1; s = 2; break;   // BF16
    case 24: b = 1; s = 1; break;   // I8
    case 2: b = 32; s = 18; break;  // Q4_0
    case 3: b = 32; s = 20; break;  // Q4_1
    case 6: b = 32; s = 22; break;  // Q5_0
    case 7: b = 32; s = 24; break;  // Q5_1
    case 8: b = 32; s = 34; break;  // Q8_0
    case 9: b = 32; s = 36; break;  // Q8_1
    case 20: b = 32; s = 18; break; // IQ4_NL
    case 39: b = 32; s = 17; break; // MXFP4
    case 10: b = 256; s = 84; break;   // Q2_K
    case 11: b = 256; s = 110; break;  // Q3_K
    case 12: b = 256; s = 144; break;  // Q4_K
    case 13: b = 256; s = 176; break;  // Q5_K
    case 14: b = 256; s = 210; break;  // Q6_K
    case 16: b = 256; s = 66; break;   // IQ2_XXS
    case 17: b = 256; s = 74; break;   // IQ2_XS
    case 18: b = 256; s = 98; break;   // IQ3_XXS
    case 21: b = 256; s = 110; break;  // IQ3_S
    case 22: b = 256; s = 82; break;   // IQ2_S
    case 23: b = 256; s = 136; break;  // IQ4_XS
    case 29: b = 256; s = 56; break;   // IQ1_M
    case 40: b = 64; s = 36; break;    // NVFP4
    case 41: b = 128; s = 18; break;   // Q1_0
    case 42: b = 64; s = 18; break;    // Q2_0
    default: break;
  }
  *block = b;
  *bytes = s;
}

GgufErr gguf_open(const char* path, GgufFile** out, std::string* msg) {
  *out = nullptr;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    *msg = std::string("cannot open ") + path + ": " + strerror(errno);
    return GgufErr::kIo;
  }
  struct stat st;
  if (fstat(fd, &st) != 0) {
    *msg = std::string("cannot stat ") + path + ": " + strerror(errno);
    close(fd);
    return GgufErr::kIo;
  }
  GgufFile* f = new GgufFile;
  f->size = uint64_t(st.st_size);
  if (f->size > 0) {
    void* m = mmap(nullptr, size_t(f->size), PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
      *msg = std::string("cannot map ") + path + ": " + strerror(errno);
      close(fd);
      delete f;
      return GgufErr::kIo;
    }
    f->map = static_cast<const uint8_t*>(m);
  }
  close(fd);

  Cursor c{f->map, f->size};
  auto failed = [&](GgufErr e, const std::string& m) {
    *msg = m;
    delete f;
    return e;
  };
  uint32_t magic = 0, version = 0;
  uint64_t n_tensors = 0, n_kv = 0;
  if (!c.get(&magic)) return failed(c.err, c.msg);
  if (magic != kMagic) return failed(GgufErr::kBadMagic, fmt("bad magic 0x%08llx", magic));
  if (!c.get(&version)) return failed(c.err, c.msg);
  if (version != kVersion) return failed(GgufErr::kUnsupportedVersion, fmt("unsupported GGUF version %llu", version));
  if (!c.get(&n_tensors) || !c.get(&n_kv)) return failed(c.err, c.msg);
  for (uint64_t k = 0; k < n_kv; ++k) {
    std::string key;
    uint32_t ty;
    GgufMeta v;
    if (!c.string(&key) || !c.get(&ty)) return failed(c.err, c.msg);
    if (ty > kF64) {
      c.bad_type(ty);
      return failed(c.err, c.msg);
    }
    if (!c.value(ty, 0, &v)) return failed(c.err, c.msg);
    f->meta[key] = std::move(v);  // a repeated key keeps the last value
  }
  std::unordered_set<std::string> names;
  for (uint64_t k = 0; k < n_tensors; ++k) {
    GgufTensor t;
    uint32_t nd;
    if (!c.string(&t.name)) return failed(c.err, c.msg);
    if (!names.insert(t.name).second) return failed(GgufErr::kDuplicateTensor, "duplicate tensor " + t.name);
    if (!c.get(&nd)) return failed(c.err, c.msg);
    if (nd == 0 || nd > 4)
      return failed(GgufErr::kWrongTensorDims, t.name + ": " + fmt("%llu dims (1..4 allowed)", nd));
    t.shape.resize(nd);
    for (uint32_t d = 0; d < nd; ++d)
      if (!c.get(&t.shape[d])) return failed(c.err, c.msg);
    if (!c.get(&t.ty) || !c.get(&t.offset)) return failed(c.err, c.msg);
    f->index[t.name] = f->tensors.size();
    f->tensors.push_back(std::move(t));
  }
  // alignment: general.alignment when it is an integer type and positive
  uint64_t align = 32;
  auto it = f->meta.find("general.alignment");
  if (it != f->meta.end()) {
    const GgufMeta& m = it->second;
    const bool integer = m.ty != kF32 && m.ty != kF64 && m.ty != kString && m.ty != kArray;
    if (integer && m.i > 0) align = uint64_t(m.i);
  }
  f->alignment = align;
  const uint64_t pos = c.pos;
  uint64_t start;
  const bool overflow = __builtin_add_overflow(pos, align - 1, &start);
  start = overflow ? ~uint64_t(0) : start / align * align;
  if (overflow || start > f->size) {
    if (!f->tensors.empty())
      return failed(GgufErr::kTruncated, fmt("truncated: data starts at %llu, the file has %llu bytes",
                                             overflow ? ~0ull : start, f->size));
    start = f->size;  // a metadata-only shard
  }
  f->version = version;
  f->data_start = start;
  f->n_kv = n_kv;
  *out = f;
  return GgufErr::kOk;
}

GgufErr gguf_payload_bytes(const GgufTensor& t, uint64_t* bytes, std::string* msg) {
  if (t.shape.empty()) {
    *msg = t.name + ": no dims";
    return GgufErr::kWrongTensorDims;
  }
  uint64_t block, size;
  gguf_type_geometry(t.ty, &block, &size);
  if (block == 0) {
    *msg = fmt("unsupported quant type id %llu", t.ty);
    return GgufErr::kUnsupportedQuant;
  }
  uint64_t n = 1;
  for (uint64_t d : t.shape) {
    if (d == 0 || n > ~uint64_t(0) / d) {
      *msg = t.name + ": a zero or overflowing dim";
      return GgufErr::kTruncated;
    }
    n *= d;
  }
  const uint64_t n_blocks = n / block;  // the reference divides (reader.rs:418)
  if (__builtin_mul_overflow(n_blocks, size, bytes)) {
    *msg = t.name + ": payload size overflows";
    return GgufErr::kTruncated;
  }
  return GgufErr::kOk;
}

GgufErr gguf_tensor_data(const GgufFile& f, const GgufTensor& t, const uint8_t** data, uint64_t* bytes,
                         std::string* msg) {
  uint64_t nb;
  GgufErr e = gguf_payload_bytes(t, &nb, msg);
  if (e != GgufErr::kOk) return e;
  uint64_t start, end;
  if (__builtin_add_overflow(f.data_start, t.offset, &start) || __builtin_add_overflow(start, nb, &end) ||
      end > f.size) {
    *msg = t.name + ": " + fmt("payload of %llu bytes runs past the end of the file (%llu bytes)", nb, f.size);
    return GgufErr::kTruncated;
  }
  *data = f.map + start;
  *bytes = nb;
  return GgufErr::kOk;
}

static bool is_digit(char c) { return c >= '0' && c <= '9'; }

GgufErr gguf_split_paths(const std::string& s, std::vector<std::string>* out, std::string* msg) {
  out->clear();
  const size_t at = s.rfind("-of-");
  const bool shape = at != std::string::npos && at >= 6 && s[at - 6] == '-' && s.size() == at + 14 &&
                     s.compare(at + 9, 5, ".gguf") == 0;
  size_t no = 0, n = 0;
  bool digits = shape;
  for (int i = 0; shape && i < 5; ++i) {
    const char a = s[at - 5 + i], b = s[at + 4 + i];
    if (!is_digit(a) || !is_digit(b)) {
      digits = false;
      break;
    }
    no = no * 10 + size_t(a - '0');
    n = n * 10 + size_t(b - '0');
  }
  if (!digits || n < 1 || no < 1 || no > n) {
    out->push_back(s);
    return GgufErr::kOk;
  }
  for (size_t i = 1; i <= n; ++i) {
    char num[8];
    snprintf(num, sizeof num, "%05zu", i);
    std::string p = s;
    p.replace(at - 5, 5, num);
    struct stat st;
    if (stat(p.c_str(), &st) != 0) {
      out->clear();
      *msg = p + ": missing model shard " + std::to_string(i) + " of " + std::to_string(n) +
             " (is the download complete?)";
      return GgufErr::kIo;
    }
    out->push_back(p);
  }
  return GgufErr::kOk;
}

GgufModel::~GgufModel() {
  for (GgufFile* f : shards) delete f;
}

GgufErr gguf_model_open(const char* any_shard, GgufModel** out, std::string* msg) {
  *out = nullptr;
  std::vector<std::string> paths;
  GgufErr e = gguf_split_paths(any_shard, &paths, msg);
  if (e != GgufErr::kOk) return e;
  GgufModel* m = new GgufModel;
  for (const std::string& p : paths) {
    GgufFile* f = nullptr;
    e = gguf_open(p.c_str(), &f, msg);
    if (e != GgufErr::kOk) {
      delete m;
      return e;
    }
    m->shards.push_back(f);
  }
  for (size_t si = 0; si < m->shards.size(); ++si) {
    const std::vector<GgufTensor>& ts = m->shards[si]->tensors;
    for (size_t ti = 0; ti < ts.size(); ++ti) {
      if (!m->index.emplace(ts[ti].name, std::make_pair(si, ti)).second) {
        *msg = "tensor " + ts[ti].name + " is in two shards";
        delete m;
        return GgufErr::kDuplicateTensor;
      }
    }
  }
  *out = m;
  return GgufErr::kOk;
}

}  // namespace sh
