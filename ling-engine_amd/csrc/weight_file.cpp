// The on-disk kernel-order weight file: an offline compiler from a (sharded) safetensors checkpoint to the
// tiled blobs the GEMMs read, and its loader. Host code only; no GPU is touched.
//
// The reference builds the tiled layout at every load, on the GPU (src/core/model.cu:131-186 upload_tiled /
// upload_nvfp4 over retile_* of src/core/stream_gemm.cu:705-780), from a checkpoint mapped by its safetensors
// reader (src/core/safetensors.hpp:14-52). Its README's offline compiler ("ling-compile") was never built.
// This file does that step once: each quantized linear's tiled blob is written byte-identical to what the
// device retile produces, next to its scale side tables, so that a load is a copy of aligned sections.
//
// File layout (little-endian; every section starts on a 4096-byte boundary):
//   FileHeader (64 B) | Entry[count] (192 B each) | string table (names, NUL-terminated) | data sections
// Each entry names its blob (tiled weight), aux (coded NVFP4: raw scale copy, 128 B per block; FP8: FP32
// per-channel [N] or block [ceil(N/128)][ceil(K/128)] scales) and table (coded NVFP4: the 64-byte code table)
// sections with a 64-bit hash of each; the header holds a hash of the entries and strings.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <set>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "ling_gemm.h"
#include "lq_quantize.hpp"

namespace lq {
int fail(int code, const std::string& msg);
}

namespace {

constexpr int kChunk = 128;
constexpr size_t kAlign = 4096;
constexpr char kMagic[8] = {'L', 'Q', 'W', 'F', 'I', 'L', 'E', '1'};
constexpr uint32_t kVersion = 1;

struct IoError : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct ArgError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// ---------------- 64-bit section hash ----------------
// FNV-1a over little-endian 64-bit words (a tail shorter than 8 bytes is zero-padded), seeded with the byte
// count: h = (h ^ word) * 0x100000001b3 from h = 0xcbf29ce484222325 ^ n.
uint64_t hash64(const uint8_t* p, size_t n) {
  uint64_t h = 0xcbf29ce484222325ull ^ static_cast<uint64_t>(n);
  size_t i = 0;
  for (; i + 8 <= n; i += 8) {
    uint64_t w;
    std::memcpy(&w, p + i, 8);
    h = (h ^ w) * 0x100000001b3ull;
  }
  if (i < n) {
    uint64_t w = 0;
    std::memcpy(&w, p + i, n - i);
    h = (h ^ w) * 0x100000001b3ull;
  }
  return h;
}

// ---------------- minimal JSON (what safetensors headers and index files use) ----------------
struct Json {
  enum Type { kNull, kBool, kNum, kStr, kArr, kObj } type = kNull;
  bool b = false;
  double num = 0;
  int64_t inum = 0;
  bool integral = false;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;

  const Json* get(const std::string& key) const {
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

class JsonParser {
 public:
  JsonParser(const char* p, size_t n) : p_(p), e_(p + n) {}
  Json parse() {
    Json v = value(0);
    ws();
    if (p_ != e_) bad("trailing characters");
    return v;
  }

 private:
  const char* p_;
  const char* e_;

  [[noreturn]] void bad(const char* what) { throw IoError(std::string("malformed JSON: ") + what); }
  void ws() {
    while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if (size_t(e_ - p_) < n || std::memcmp(p_, s, n) != 0) return false;
    p_ += n;
    return true;
  }
  static void put_utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += char(cp);
    } else if (cp < 0x800) {
      out += char(0xc0 | (cp >> 6));
      out += char(0x80 | (cp & 0x3f));
    } else if (cp < 0x10000) {
      out += char(0xe0 | (cp >> 12));
      out += char(0x80 | ((cp >> 6) & 0x3f));
      out += char(0x80 | (cp & 0x3f));
    } else {
      out += char(0xf0 | (cp >> 18));
      out += char(0x80 | ((cp >> 12) & 0x3f));
      out += char(0x80 | ((cp >> 6) & 0x3f));
      out += char(0x80 | (cp & 0x3f));
    }
  }
  uint32_t hex4() {
    if (e_ - p_ < 4) bad("short \\u escape");
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= uint32_t(c - '0');
      else if (c >= 'a' && c <= 'f') v |= uint32_t(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= uint32_t(c - 'A' + 10);
      else bad("bad \\u escape");
    }
    return v;
  }
  std::string string() {
    if (p_ >= e_ || *p_ != '"') bad("expected a string");
    ++p_;
    std::string out;
    while (true) {
      if (p_ >= e_) bad("unterminated string");
      const char c = *p_++;
      if (c == '"') break;
      if (static_cast<unsigned char>(c) < 0x20) bad("control character in string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (p_ >= e_) bad("unterminated escape");
      const char x = *p_++;
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
          uint32_t cp = hex4();
          if (cp >= 0xd800 && cp < 0xdc00) {
            if (!lit("\\u")) bad("lone surrogate");
            const uint32_t lo = hex4();
            if (lo < 0xdc00 || lo >= 0xe000) bad("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
          }
          put_utf8(out, cp);
          break;
        }
        default: bad("bad escape");
      }
    }
    return out;
  }
  Json number() {
    Json v;
    v.type = Json::kNum;
    const char* s = p_;
    if (p_ < e_ && *p_ == '-') ++p_;
    bool frac = false;
    while (p_ < e_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' ||
                       *p_ == '-')) {
      if (*p_ == '.' || *p_ == 'e' || *p_ == 'E') frac = true;
      ++p_;
    }
    const std::string text(s, p_);
    if (text.empty() || text == "-") bad("bad number");
    char* end = nullptr;
    v.num = std::strtod(text.c_str(), &end);
    if (end != text.c_str() + text.size()) bad("bad number");
    if (!frac) {
      errno = 0;
      v.inum = std::strtoll(text.c_str(), &end, 10);
      v.integral = errno == 0 && end == text.c_str() + text.size();
    }
    return v;
  }
  Json value(int depth) {
    if (depth > 64) bad("nesting too deep");
    ws();
    if (p_ >= e_) bad("unexpected end");
    Json v;
    const char c = *p_;
    if (c == '{') {
      ++p_;
      v.type = Json::kObj;
      ws();
      if (p_ < e_ && *p_ == '}') {
        ++p_;
        return v;
      }
      while (true) {
        ws();
        std::string k = string();
        ws();
        if (p_ >= e_ || *p_ != ':') bad("expected ':'");
        ++p_;
        v.obj.emplace_back(std::move(k), value(depth + 1));
        ws();
        if (p_ < e_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < e_ && *p_ == '}') {
          ++p_;
          return v;
        }
        bad("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p_;
      v.type = Json::kArr;
      ws();
      if (p_ < e_ && *p_ == ']') {
        ++p_;
        return v;
      }
      while (true) {
        v.arr.push_back(value(depth + 1));
        ws();
        if (p_ < e_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < e_ && *p_ == ']') {
          ++p_;
          return v;
        }
        bad("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.type = Json::kStr;
      v.str = string();
      return v;
    }
    if (lit("true")) {
      v.type = Json::kBool;
      v.b = true;
      return v;
    }
    if (lit("false")) {
      v.type = Json::kBool;
      return v;
    }
    if (lit("null")) return v;
    return number();
  }
};

// ---------------- mapped files and the safetensors checkpoint ----------------
class Mapping {
 public:
  // writable = a private (copy-on-write) mapping, so callers may wrap it in writable buffer objects
  Mapping(const std::string& path, bool writable) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) throw IoError("cannot open " + path + ": " + std::strerror(errno));
    struct stat st {};
    if (::fstat(fd_, &st) != 0) throw IoError("cannot stat " + path);
    size_ = static_cast<size_t>(st.st_size);
    if (size_ == 0) return;
    void* p = ::mmap(nullptr, size_, writable ? (PROT_READ | PROT_WRITE) : PROT_READ, MAP_PRIVATE, fd_, 0);
    if (p == MAP_FAILED) throw IoError("cannot map " + path);
    data_ = static_cast<uint8_t*>(p);
  }
  ~Mapping() {
    if (data_) ::munmap(data_, size_);
    if (fd_ >= 0) ::close(fd_);
  }
  Mapping(const Mapping&) = delete;
  Mapping& operator=(const Mapping&) = delete;
  uint8_t* data() const { return data_; }
  size_t size() const { return size_; }

 private:
  int fd_ = -1;
  uint8_t* data_ = nullptr;
  size_t size_ = 0;
};

struct Tensor {
  std::string dtype;
  std::vector<int64_t> shape;
  const uint8_t* data = nullptr;
  size_t bytes = 0;
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
  }
};

size_t dtype_size(const std::string& d) {
  static const std::map<std::string, size_t> sizes = {
      {"BOOL", 1}, {"U8", 1},  {"I8", 1},  {"F8_E4M3", 1}, {"F8_E5M2", 1}, {"I16", 2}, {"U16", 2}, {"F16", 2},
      {"BF16", 2}, {"I32", 4}, {"U32", 4}, {"F32", 4},     {"I64", 8},     {"U64", 8}, {"F64", 8}};
  auto it = sizes.find(d);
  return it == sizes.end() ? 0 : it->second;
}

// A checkpoint directory: model.safetensors.index.json and its shards, or one model.safetensors; every
// tensor is a view into its shard's mapping (the reference's Checkpoint, src/core/safetensors.cpp:39-79).
class Checkpoint {
 public:
  explicit Checkpoint(const std::string& dir) {
    std::set<std::string> shards;
    const std::string index = dir + "/model.safetensors.index.json";
    if (::access(index.c_str(), R_OK) == 0) {
      Mapping m(index, false);
      const Json j = JsonParser(reinterpret_cast<const char*>(m.data()), m.size()).parse();
      const Json* wm = j.get("weight_map");
      if (!wm || wm->type != Json::kObj) throw IoError(index + ": no weight_map object");
      for (const auto& kv : wm->obj) {
        if (kv.second.type != Json::kStr) throw IoError(index + ": weight_map value is not a string");
        const std::string& s = kv.second.str;
        if (s.empty() || s.find('/') != std::string::npos) throw IoError(index + ": bad shard name " + s);
        shards.insert(s);
      }
    } else if (::access((dir + "/model.safetensors").c_str(), R_OK) == 0) {
      shards.insert("model.safetensors");
    } else {
      throw IoError("no model.safetensors.index.json or model.safetensors in " + dir);
    }
    for (const std::string& shard : shards) load_shard(dir + "/" + shard, shard);
  }

  const std::map<std::string, Tensor>& tensors() const { return tensors_; }
  const Tensor* find(const std::string& name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
  }

 private:
  std::vector<std::unique_ptr<Mapping>> files_;
  std::map<std::string, Tensor> tensors_;

  void load_shard(const std::string& path, const std::string& shard) {
    auto file = std::make_unique<Mapping>(path, false);
    if (file->size() < 8) throw IoError("truncated shard " + shard);
    uint64_t hlen = 0;
    std::memcpy(&hlen, file->data(), 8);
    if (hlen > file->size() - 8) throw IoError("bad header length in " + shard);
    const Json h = JsonParser(reinterpret_cast<const char*>(file->data() + 8), hlen).parse();
    if (h.type != Json::kObj) throw IoError("header of " + shard + " is not an object");
    const uint8_t* base = file->data() + 8 + hlen;
    const size_t avail = file->size() - 8 - hlen;
    for (const auto& kv : h.obj) {
      if (kv.first == "__metadata__") continue;
      const Json& info = kv.second;
      const Json* dt = info.get("dtype");
      const Json* sh = info.get("shape");
      const Json* off = info.get("data_offsets");
      if (!dt || dt->type != Json::kStr || !sh || sh->type != Json::kArr || !off || off->type != Json::kArr ||
          off->arr.size() != 2)
        throw IoError("bad entry " + kv.first + " in " + shard);
      if (kv.first.empty() || kv.first.find('\0') != std::string::npos) throw IoError("bad tensor name in " + shard);
      Tensor t;
      t.dtype = dt->str;
      uint64_t numel = 1;
      for (const Json& d : sh->arr) {
        if (d.type != Json::kNum || !d.integral || d.inum < 0) throw IoError("bad shape of " + kv.first);
        if (__builtin_mul_overflow(numel, static_cast<uint64_t>(d.inum), &numel) || numel > (uint64_t(1) << 48))
          throw IoError("shape of " + kv.first + " is too large");
        t.shape.push_back(d.inum);
      }
      for (const Json& o : off->arr)
        if (o.type != Json::kNum || !o.integral || o.inum < 0) throw IoError("bad offsets of " + kv.first);
      const uint64_t b0 = static_cast<uint64_t>(off->arr[0].inum), b1 = static_cast<uint64_t>(off->arr[1].inum);
      if (b1 < b0 || b1 > avail) throw IoError("offsets of " + kv.first + " are out of " + shard);
      const size_t es = dtype_size(t.dtype);
      if (es && static_cast<uint64_t>(t.numel()) * es != b1 - b0)
        throw IoError(kv.first + ": " + std::to_string(b1 - b0) + " bytes do not match its shape and dtype");
      t.data = base + b0;
      t.bytes = b1 - b0;
      if (tensors_.count(kv.first)) throw IoError("tensor " + kv.first + " appears in two shards");
      tensors_[kv.first] = t;
    }
    files_.push_back(std::move(file));
  }
};

float half_to_f32(uint16_t h) {
  const uint32_t s = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 0) v = std::ldexp(float(m), -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = std::ldexp(float(m | 1024), int(e) - 25);
  return s ? -v : v;
}

// element i of a float tensor as FP32 (F32 exact; BF16 and F16 widened exactly)
float element_f32(const Tensor& t, size_t i, const std::string& name) {
  if (t.dtype == "F32") {
    float v;
    std::memcpy(&v, t.data + 4 * i, 4);
    return v;
  }
  if (t.dtype == "BF16") {
    uint16_t b;
    std::memcpy(&b, t.data + 2 * i, 2);
    const uint32_t u = uint32_t(b) << 16;
    float v;
    std::memcpy(&v, &u, 4);
    return v;
  }
  if (t.dtype == "F16") {
    uint16_t b;
    std::memcpy(&b, t.data + 2 * i, 2);
    return half_to_f32(b);
  }
  throw ArgError(name + " is " + t.dtype + ", expected F32, BF16 or F16");
}

float scalar_f32(const Tensor& t, const std::string& name) {
  if (t.numel() != 1) throw ArgError(name + " is not a scalar");
  return element_f32(t, 0, name);
}

// ---------------- host retile (CPU threads; byte-identical to the device retile) ----------------
void parallel_for(size_t n, const std::function<void(size_t, size_t)>& fn) {
  const size_t want = n / 4096 + 1;  // at least 4096 blocks per thread
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const size_t nt = std::min<size_t>({want, size_t(hw), size_t(16)});
  if (nt <= 1) {
    fn(0, n);
    return;
  }
  std::vector<std::thread> ts;
  for (size_t t = 0; t < nt; ++t) ts.emplace_back([&fn, n, nt, t] { fn(n * t / nt, n * (t + 1) / nt); });
  for (auto& th : ts) th.join();
}

// FP8 block (tile, chunk): 16-byte piece ((h*2+q)*8+g)*4+t holds W[16 tile + g + 8h][128 chunk + 32t + 16q, +16)
void host_retile_fp8(const uint8_t* w, uint8_t* out, int N, int K) {
  const size_t C = size_t(K) / kChunk, blocks = size_t(N / 16) * C;
  parallel_for(blocks, [&](size_t b0, size_t b1) {
    for (size_t blk = b0; blk < b1; ++blk) {
      const size_t row0 = (blk / C) * 16, k0 = (blk % C) * kChunk;
      uint8_t* o = out + blk * 2048;
      for (int p = 0; p < 128; ++p) {
        const int t = p & 3, g = (p >> 2) & 7, q = (p >> 5) & 1, h = p >> 6;
        std::memcpy(o + p * 16, w + (row0 + g + 8 * h) * size_t(K) + k0 + 32 * t + 16 * q, 16);
      }
    }
  });
}

// NVFP4 block: slot r*4+t holds the 16 value bytes of W[16 tile + r][128 chunk + 32t, +32) and its two E4M3
// scales at 1024 + 2 slot (coded: values at a 1024-byte stride, the scales to `raw` at 128 bytes per block)
void host_retile_nvfp4_values(const uint8_t* w, const uint8_t* sc, uint8_t* out, size_t stride, uint8_t* raw,
                              int N, int K) {
  const size_t C = size_t(K) / kChunk, blocks = size_t(N / 16) * C;
  parallel_for(blocks, [&](size_t b0, size_t b1) {
    for (size_t blk = b0; blk < b1; ++blk) {
      const size_t row0 = (blk / C) * 16, c = blk % C;
      uint8_t* o = out + blk * stride;
      uint8_t* so = raw ? raw + blk * 128 : o + 1024;
      for (int s = 0; s < 64; ++s) {
        const int r = s >> 2, t = s & 3;
        const size_t n = row0 + r;
        std::memcpy(o + s * 16, w + n * (K / 2) + c * 64 + t * 16, 16);
        std::memcpy(so + s * 2, sc + n * (K / 16) + c * 8 + t * 2, 2);
      }
    }
  });
}

// coded NVFP4: after the value blocks, 96 code bytes per block; slot s < 32 puts its 12-bit code pair
// (first scale low, 6 bits each) in byte 2s and the low nibble of 64 + s, slot 32 + L in byte 2L + 1 and
// the high nibble of 64 + L
void host_retile_nvfp4_coded(const uint8_t* w, const uint8_t* sc, const uint8_t* code_of, uint8_t* out, uint8_t* raw,
                             int N, int K) {
  const size_t C = size_t(K) / kChunk, blocks = size_t(N / 16) * C;
  host_retile_nvfp4_values(w, sc, out, 1024, raw, N, K);
  uint8_t* codes = out + blocks * 1024;
  parallel_for(blocks, [&](size_t b0, size_t b1) {
    for (size_t blk = b0; blk < b1; ++blk) {
      const uint8_t* r = raw + blk * 128;
      uint8_t* cd = codes + blk * 96;
      for (int L = 0; L < 32; ++L) {
        const uint32_t f0 = uint32_t(code_of[r[2 * L]]) | (uint32_t(code_of[r[2 * L + 1]]) << 6);
        const uint32_t f1 = uint32_t(code_of[r[2 * (L + 32)]]) | (uint32_t(code_of[r[2 * (L + 32) + 1]]) << 6);
        cd[2 * L] = static_cast<uint8_t>(f0 & 0xff);
        cd[2 * L + 1] = static_cast<uint8_t>(f1 & 0xff);
        cd[64 + L] = static_cast<uint8_t>((f0 >> 8) | ((f1 >> 8) << 4));
      }
    }
  });
}

void check_tiling(int N, int K, const std::string& what) {
  if (N <= 0 || K <= 0 || N % 16 != 0 || K % kChunk != 0)
    throw ArgError(what + ": N % 16 and K % 128 must be 0 (N=" + std::to_string(N) + ", K=" + std::to_string(K) + ")");
}

// ---------------- on-disk records ----------------
struct FileHeader {
  char magic[8];
  uint32_t version;
  uint32_t count;
  uint64_t entries_off;
  uint64_t strings_off;
  uint64_t strings_bytes;
  uint64_t data_off;
  uint64_t file_bytes;
  uint64_t meta_hash;  // hash64 of the entry records and the string table
};
static_assert(sizeof(FileHeader) == 64, "FileHeader is 64 bytes");

struct Entry {
  uint64_t name_off;
  uint32_t name_len;
  uint32_t kind;
  uint32_t scale_kind;
  int32_t N;
  int32_t K;
  uint32_t ndim;
  float weight_scale;
  float input_scale;
  uint32_t flags;
  uint32_t reserved0;
  char dtype[16];
  int64_t shape[4];
  uint64_t blob_off, blob_bytes;
  uint64_t aux_off, aux_bytes;
  uint64_t table_off, table_bytes;
  uint64_t blob_hash, aux_hash, table_hash;
  uint64_t reserved1[3];
};
static_assert(sizeof(Entry) == 192, "Entry is 192 bytes");

// ---------------- the compiler ----------------
struct Plan {
  std::string name;
  Entry e{};
  std::function<void(uint8_t* blob, uint8_t* aux, uint8_t* table)> fill;
};

const Tensor& need(const Checkpoint& ck, const std::string& name) {
  const Tensor* t = ck.find(name);
  if (!t) throw ArgError("tensor not in checkpoint: " + name);
  return *t;
}

void set_dtype(Entry& e, const std::string& d) {
  std::memset(e.dtype, 0, sizeof e.dtype);
  std::memcpy(e.dtype, d.data(), std::min(d.size(), sizeof e.dtype - 1));
}

constexpr int kQuantFlags = LQ_WFILE_QUANT_FP8 | LQ_WFILE_QUANT_FP8_BLOCK | LQ_WFILE_QUANT_NVFP4;

// A high-precision linear weight quantized here (LQ_WFILE_QUANT_*): a 2-D P.weight in BF16, F16 or F32 with no
// scale tensors of its own, N % 16 == 0 and K % 128 == 0, and a name naming neither an embedding nor a norm (those
// are lookups and vectors, not GEMM operands) nor a MoE router. Anything else is left to the passthrough. NVFP4 takes BF16 values
// (the reference's quantize_nvfp4, src/core/model.cu:188-249, rounds BF16): F16 and F32 weights are rounded to
// BF16 first. FP8 quantizes the exact FP32 values.
void plan_quantized(const Checkpoint& ck, const std::string& name, const std::string& prefix, const Tensor& w,
                    int flags, std::vector<Plan>& plans, std::set<std::string>& consumed) {
  int dt;
  if (w.dtype == "BF16") dt = LQ_DT_BF16;
  else if (w.dtype == "F16") dt = LQ_DT_F16;
  else if (w.dtype == "F32") dt = LQ_DT_F32;
  else return;
  if (w.shape.size() != 2 || ck.find(prefix + ".weight_scale") || ck.find(prefix + ".weight_scale_inv")) return;
  if (name.find("embed") != std::string::npos || name.find("norm") != std::string::npos) return;
  // MoE routers (P = "....gate" or a name with "router") stay in their own precision: their outputs pick the
  // experts, and the reference quantizes only the projections it streams (src/core/drafter.cpp:93-100)
  const std::string gate_suffix = ".gate";
  if (prefix.find("router") != std::string::npos ||
      (prefix.size() >= gate_suffix.size() &&
       prefix.compare(prefix.size() - gate_suffix.size(), gate_suffix.size(), gate_suffix) == 0))
    return;
  if (w.shape[0] <= 0 || w.shape[1] <= 0 || w.shape[0] > (int64_t(1) << 30) || w.shape[1] > (int64_t(1) << 29)) return;
  const int N = static_cast<int>(w.shape[0]), K = static_cast<int>(w.shape[1]);
  if (N % 16 != 0 || K % kChunk != 0) return;
  Plan p;
  p.name = prefix;
  Entry& e = p.e;
  e.N = N;
  e.K = K;
  e.ndim = 2;
  e.shape[0] = N;
  e.shape[1] = K;
  e.flags |= LQ_WENTRY_QUANTIZED;
  set_dtype(e, w.dtype);
  const Tensor* in = ck.find(prefix + ".input_scale");
  if (in) {
    e.input_scale = scalar_f32(*in, prefix + ".input_scale");
    e.flags |= LQ_WENTRY_HAS_INPUT_SCALE;
    consumed.insert(prefix + ".input_scale");
  }
  consumed.insert(name);
  const uint8_t* src = w.data;
  if (flags & LQ_WFILE_QUANT_NVFP4) {
    // BF16 values: F16 / F32 elements are rounded to BF16 as they are read, so no copy of the weight is made. The
    // block scales decide here whether the blob is coded, and are made again when the entry is filled: a plan keeps
    // only its 64-byte code table, so planning a whole checkpoint holds no per-weight buffers.
    const int vdt = dt == LQ_DT_BF16 ? dt : (dt | lq::hostq::kRoundBf16);
    float g;
    uint8_t table[64], code_of[256];
    bool coded;
    {
      std::vector<uint8_t> scl(size_t(N) * K / 16);
      g = lq::hostq::nvfp4_scales(src, vdt, N, K, scl.data());
      coded = !(flags & LQ_WFILE_NO_CODES) && lq_scale_code_table(scl.data(), scl.size(), table, code_of) == 1;
    }
    e.weight_scale = g;
    if (coded) {
      e.kind = LQ_WENTRY_NVFP4_CODED;
      e.blob_bytes = lq_tiled_bytes_nvfp4_coded(N, K);
      e.aux_bytes = size_t(N) * K / 16;
      e.table_bytes = 64;
    } else {
      e.kind = LQ_WENTRY_NVFP4;
      e.blob_bytes = lq_tiled_bytes_nvfp4(N, K);
    }
    std::vector<uint8_t> tab(table, table + 64), map(code_of, code_of + 256);
    p.fill = [=](uint8_t* blob, uint8_t* aux, uint8_t* tb) {
      std::vector<uint8_t> scl(size_t(N) * K / 16), v(size_t(N) * K / 2);
      (void)lq::hostq::nvfp4_scales(src, vdt, N, K, scl.data());
      (void)lq::hostq::nvfp4_values(src, vdt, N, K, g, scl.data(), v.data());
      if (coded) {
        host_retile_nvfp4_coded(v.data(), scl.data(), map.data(), blob, aux, N, K);
        std::memcpy(tb, tab.data(), 64);
      } else {
        host_retile_nvfp4_values(v.data(), scl.data(), blob, 1152, nullptr, N, K);
      }
    };
  } else {
    const bool block = (flags & LQ_WFILE_QUANT_FP8_BLOCK) != 0;
    e.kind = LQ_WENTRY_FP8;
    e.blob_bytes = lq_tiled_bytes_fp8(N, K);
    e.scale_kind = block ? LQ_WSCALE_BLOCK128 : LQ_WSCALE_CHANNEL;
    e.aux_bytes = block ? size_t((N + 127) / 128) * ((K + 127) / 128) * 4 : size_t(N) * 4;
    p.fill = [=](uint8_t* blob, uint8_t* aux, uint8_t*) {
      std::vector<uint8_t> q(size_t(N) * K);
      if (block) lq::hostq::fp8_block128(src, dt, N, K, q.data(), reinterpret_cast<float*>(aux));
      else lq::hostq::fp8_channel(src, dt, N, K, q.data(), reinterpret_cast<float*>(aux));
      host_retile_fp8(q.data(), blob, N, K);
    };
  }
  plans.push_back(std::move(p));
}

std::vector<Plan> plan_checkpoint(const Checkpoint& ck, int flags, std::set<std::string>& consumed) {
  std::vector<Plan> plans;
  const std::string suffix = ".weight";
  for (const auto& kv : ck.tensors()) {
    const std::string& name = kv.first;
    const Tensor& w = kv.second;
    if (name.size() <= suffix.size() || name.compare(name.size() - suffix.size(), suffix.size(), suffix) != 0) continue;
    const std::string prefix = name.substr(0, name.size() - suffix.size());
    const Tensor* ws = ck.find(prefix + ".weight_scale");
    const bool nvfp4 = w.dtype == "U8" && ws && ws->dtype == "F8_E4M3";
    const bool fp8 = w.dtype == "F8_E4M3";
    if (!nvfp4 && !fp8) {
      if (flags & kQuantFlags) plan_quantized(ck, name, prefix, w, flags, plans, consumed);
      continue;
    }
    if (w.shape.size() != 2) throw ArgError(name + ": a quantized weight must be 2-D");
    // N and K are int in the kernels' interface (and K = 2 x the packed NVFP4 width)
    if (w.shape[0] > (int64_t(1) << 30) || w.shape[1] > (int64_t(1) << 29))
      throw ArgError(name + ": dimensions too large for the GEMM interface");
    Plan p;
    p.name = prefix;
    Entry& e = p.e;
    e.N = static_cast<int32_t>(w.shape[0]);
    e.ndim = 2;
    const Tensor* in = ck.find(prefix + ".input_scale");
    if (in) {
      e.input_scale = scalar_f32(*in, prefix + ".input_scale");
      e.flags |= LQ_WENTRY_HAS_INPUT_SCALE;
      consumed.insert(prefix + ".input_scale");
    }
    consumed.insert(name);
    if (nvfp4) {
      e.K = static_cast<int32_t>(w.shape[1] * 2);
      check_tiling(e.N, e.K, prefix);
      if (ws->shape.size() != 2 || ws->shape[0] != e.N || ws->shape[1] != e.K / 16)
        throw ArgError(prefix + ".weight_scale: expected [N][K/16] E4M3 block scales");
      e.weight_scale = scalar_f32(need(ck, prefix + ".weight_scale_2"), prefix + ".weight_scale_2");
      consumed.insert(prefix + ".weight_scale");
      consumed.insert(prefix + ".weight_scale_2");
      e.shape[0] = w.shape[0];
      e.shape[1] = w.shape[1];
      set_dtype(e, "U8");
      uint8_t table[64], code_of[256];
      const bool coded = !(flags & LQ_WFILE_NO_CODES) && lq_scale_code_table(ws->data, ws->bytes, table, code_of) == 1;
      const int N = e.N, K = e.K;
      const uint8_t* vals = w.data;
      const uint8_t* scl = ws->data;
      if (coded) {
        e.kind = LQ_WENTRY_NVFP4_CODED;
        e.blob_bytes = lq_tiled_bytes_nvfp4_coded(N, K);
        e.aux_bytes = size_t(N) * K / 16;
        e.table_bytes = 64;
        std::vector<uint8_t> tab(table, table + 64), map(code_of, code_of + 256);
        p.fill = [=](uint8_t* blob, uint8_t* aux, uint8_t* tb) {
          host_retile_nvfp4_coded(vals, scl, map.data(), blob, aux, N, K);
          std::memcpy(tb, tab.data(), 64);
        };
      } else {
        e.kind = LQ_WENTRY_NVFP4;
        e.blob_bytes = lq_tiled_bytes_nvfp4(N, K);
        p.fill = [=](uint8_t* blob, uint8_t*, uint8_t*) { host_retile_nvfp4_values(vals, scl, blob, 1152, nullptr, N, K); };
      }
    } else {
      e.K = static_cast<int32_t>(w.shape[1]);
      check_tiling(e.N, e.K, prefix);
      e.kind = LQ_WENTRY_FP8;
      e.shape[0] = w.shape[0];
      e.shape[1] = w.shape[1];
      set_dtype(e, "F8_E4M3");
      const int N = e.N, K = e.K;
      e.blob_bytes = lq_tiled_bytes_fp8(N, K);
      const uint8_t* vals = w.data;
      const Tensor* inv = ck.find(prefix + ".weight_scale_inv");
      const Tensor* src = nullptr;
      std::string src_name;
      if (inv) {
        const int64_t bn = (N + 127) / 128, bk = (K + 127) / 128;
        if (inv->shape.size() != 2 || inv->shape[0] != bn || inv->shape[1] != bk)
          throw ArgError(prefix + ".weight_scale_inv: expected [ceil(N/128)][ceil(K/128)] block scales");
        e.scale_kind = LQ_WSCALE_BLOCK128;
        e.aux_bytes = size_t(bn * bk) * 4;
        src = inv;
        src_name = prefix + ".weight_scale_inv";
        consumed.insert(src_name);
      } else if (ws) {
        src_name = prefix + ".weight_scale";
        consumed.insert(src_name);
        if (ws->numel() == 1) {
          e.scale_kind = LQ_WSCALE_TENSOR;
          e.weight_scale = scalar_f32(*ws, src_name);
        } else if (ws->numel() == N && (ws->shape.size() == 1 || (ws->shape.size() == 2 && ws->shape[1] == 1))) {
          e.scale_kind = LQ_WSCALE_CHANNEL;
          e.aux_bytes = size_t(N) * 4;
          src = ws;
        } else {
          throw ArgError(src_name + ": expected a scalar or [N] per-channel scales");
        }
      } else {
        throw ArgError(prefix + ": FP8 weight without weight_scale or weight_scale_inv");
      }
      p.fill = [=](uint8_t* blob, uint8_t* aux, uint8_t*) {
        host_retile_fp8(vals, blob, N, K);
        if (src)
          for (size_t i = 0; i < size_t(src->numel()); ++i) {
            const float v = element_f32(*src, i, src_name);
            std::memcpy(aux + 4 * i, &v, 4);
          }
      };
    }
    plans.push_back(std::move(p));
  }
  if (flags & LQ_WFILE_PASSTHROUGH) {
    for (const auto& kv : ck.tensors()) {
      if (consumed.count(kv.first)) continue;
      const Tensor& t = kv.second;
      if (t.shape.size() > 4) throw ArgError(kv.first + ": more than 4 dimensions");
      Plan p;
      p.name = kv.first;
      p.e.kind = LQ_WENTRY_RAW;
      p.e.ndim = static_cast<uint32_t>(t.shape.size());
      for (size_t d = 0; d < t.shape.size(); ++d) p.e.shape[d] = t.shape[d];
      set_dtype(p.e, t.dtype);
      p.e.blob_bytes = t.bytes;
      const uint8_t* src = t.data;
      const size_t n = t.bytes;
      p.fill = [=](uint8_t* blob, uint8_t*, uint8_t*) { std::memcpy(blob, src, n); };
      plans.push_back(std::move(p));
    }
  }
  return plans;
}

void pwrite_all(int fd, const void* p, size_t n, uint64_t off, const std::string& path) {
  const uint8_t* b = static_cast<const uint8_t*>(p);
  while (n) {
    const ssize_t w = ::pwrite(fd, b, std::min<size_t>(n, size_t(1) << 30), static_cast<off_t>(off));
    if (w < 0) {
      if (errno == EINTR) continue;
      throw IoError("write to " + path + " failed: " + std::strerror(errno));
    }
    b += w;
    off += static_cast<uint64_t>(w);
    n -= static_cast<size_t>(w);
  }
}

void compile_file(const std::string& dir, const std::string& out, int flags, int* count_out) {
  Checkpoint ck(dir);
  std::set<std::string> consumed;
  std::vector<Plan> plans = plan_checkpoint(ck, flags, consumed);
  if (plans.empty()) throw ArgError(dir + ": no quantized linear weights (FP8 or NVFP4) found");
  std::string strings;
  for (Plan& p : plans) {
    p.e.name_off = strings.size();
    p.e.name_len = static_cast<uint32_t>(p.name.size());
    strings += p.name;
    strings += '\0';
  }
  FileHeader h{};
  std::memcpy(h.magic, kMagic, 8);
  h.version = kVersion;
  h.count = static_cast<uint32_t>(plans.size());
  h.entries_off = sizeof(FileHeader);
  h.strings_off = h.entries_off + plans.size() * sizeof(Entry);
  h.strings_bytes = strings.size();
  h.data_off = align_up(h.strings_off + h.strings_bytes);
  uint64_t off = h.data_off;
  for (Plan& p : plans) {
    Entry& e = p.e;
    e.blob_off = off;
    off = align_up(off + e.blob_bytes);
    if (e.aux_bytes) {
      e.aux_off = off;
      off = align_up(off + e.aux_bytes);
    }
    if (e.table_bytes) {
      e.table_off = off;
      off = align_up(off + e.table_bytes);
    }
  }
  h.file_bytes = off;

  const std::string tmp = out + ".partial";
  const int fd = ::open(tmp.c_str(), O_WRONLY | O_CREAT | O_TRUNC, 0644);
  if (fd < 0) throw IoError("cannot create " + tmp + ": " + std::strerror(errno));
  try {
    if (::ftruncate(fd, static_cast<off_t>(h.file_bytes)) != 0) throw IoError("cannot size " + tmp);
    std::vector<uint8_t> blob, aux, table;
    for (Plan& p : plans) {
      Entry& e = p.e;
      blob.assign(e.blob_bytes, 0);
      aux.assign(e.aux_bytes, 0);
      table.assign(e.table_bytes, 0);
      p.fill(blob.data(), aux.data(), table.data());
      e.blob_hash = hash64(blob.data(), blob.size());
      e.aux_hash = hash64(aux.data(), aux.size());
      e.table_hash = hash64(table.data(), table.size());
      pwrite_all(fd, blob.data(), blob.size(), e.blob_off, tmp);
      if (e.aux_bytes) pwrite_all(fd, aux.data(), aux.size(), e.aux_off, tmp);
      if (e.table_bytes) pwrite_all(fd, table.data(), table.size(), e.table_off, tmp);
    }
    std::vector<uint8_t> meta(plans.size() * sizeof(Entry) + strings.size());
    for (size_t i = 0; i < plans.size(); ++i) std::memcpy(meta.data() + i * sizeof(Entry), &plans[i].e, sizeof(Entry));
    std::memcpy(meta.data() + plans.size() * sizeof(Entry), strings.data(), strings.size());
    h.meta_hash = hash64(meta.data(), meta.size());
    pwrite_all(fd, meta.data(), meta.size(), h.entries_off, tmp);
    pwrite_all(fd, &h, sizeof h, 0, tmp);
    if (::fsync(fd) != 0) throw IoError("fsync of " + tmp + " failed");
  } catch (...) {
    ::close(fd);
    ::unlink(tmp.c_str());
    throw;
  }
  ::close(fd);
  if (::rename(tmp.c_str(), out.c_str()) != 0) {
    ::unlink(tmp.c_str());
    throw IoError("cannot rename " + tmp + " to " + out);
  }
  if (count_out) *count_out = static_cast<int>(plans.size());
}

}  // namespace

// the loaded file (opaque to callers)
struct lq_wfile {
  std::unique_ptr<Mapping> map;
  const FileHeader* h = nullptr;
  const Entry* entries = nullptr;
  const char* strings = nullptr;
  std::map<std::string, int> index;
};

namespace {

// The section sizes a GEMM will read for this entry's kind and shape: a blob shorter than its tiled size would make
// a GEMM read past the mapping.
bool sizes_match(const Entry& e) {
  if (e.kind == LQ_WENTRY_RAW) return true;
  if (e.N <= 0 || e.K <= 0 || e.N % 16 != 0 || e.K % kChunk != 0) return false;
  const size_t N = size_t(e.N), K = size_t(e.K);
  switch (e.kind) {
    case LQ_WENTRY_FP8: {
      size_t aux = 0;
      if (e.scale_kind == LQ_WSCALE_CHANNEL) aux = N * 4;
      else if (e.scale_kind == LQ_WSCALE_BLOCK128) aux = ((N + 127) / 128) * ((K + 127) / 128) * 4;
      else if (e.scale_kind != LQ_WSCALE_TENSOR && e.scale_kind != LQ_WSCALE_NONE) return false;
      return e.blob_bytes == lq_tiled_bytes_fp8(e.N, e.K) && e.aux_bytes == aux && e.table_bytes == 0;
    }
    case LQ_WENTRY_NVFP4:
      return e.blob_bytes == lq_tiled_bytes_nvfp4(e.N, e.K) && e.aux_bytes == 0 && e.table_bytes == 0;
    default:  // coded NVFP4
      return e.blob_bytes == lq_tiled_bytes_nvfp4_coded(e.N, e.K) && e.aux_bytes == N * K / 16 && e.table_bytes == 64;
  }
}

lq_wfile* open_file(const std::string& path) {
  auto f = std::make_unique<lq_wfile>();
  f->map = std::make_unique<Mapping>(path, true);
  const size_t n = f->map->size();
  const uint8_t* d = f->map->data();
  if (n < sizeof(FileHeader)) throw IoError(path + ": not a kernel-order weight file (too short)");
  f->h = reinterpret_cast<const FileHeader*>(d);
  const FileHeader& h = *f->h;
  if (std::memcmp(h.magic, kMagic, 8) != 0) throw IoError(path + ": not a kernel-order weight file (bad magic)");
  if (h.version != kVersion) throw IoError(path + ": unsupported version " + std::to_string(h.version));
  if (h.file_bytes != n) throw IoError(path + ": truncated or padded (" + std::to_string(n) + " bytes, header says " +
                                       std::to_string(h.file_bytes) + ")");
  // every sum below is checked against the mapped size before it is formed, so a crafted header cannot wrap
  if (h.entries_off != sizeof(FileHeader) || h.count > (n - sizeof(FileHeader)) / sizeof(Entry) ||
      h.strings_off != h.entries_off + uint64_t(h.count) * sizeof(Entry) || h.data_off > n ||
      h.strings_off > h.data_off || h.strings_bytes > h.data_off - h.strings_off)
    throw IoError(path + ": bad section offsets");
  if (hash64(d + h.entries_off, h.strings_off + h.strings_bytes - h.entries_off) != h.meta_hash)
    throw IoError(path + ": entry table hash mismatch");
  f->entries = reinterpret_cast<const Entry*>(d + h.entries_off);
  f->strings = reinterpret_cast<const char*>(d + h.strings_off);
  auto in_data = [&](uint64_t off, uint64_t bytes) { return bytes == 0 || (off >= h.data_off && off <= n && bytes <= n - off); };
  for (uint32_t i = 0; i < h.count; ++i) {
    const Entry& e = f->entries[i];
    if (e.name_off >= h.strings_bytes || e.name_len >= h.strings_bytes - e.name_off ||
        f->strings[e.name_off + e.name_len] != '\0')
      throw IoError(path + ": bad name of entry " + std::to_string(i));
    if (!in_data(e.blob_off, e.blob_bytes) || !in_data(e.aux_off, e.aux_bytes) || !in_data(e.table_off, e.table_bytes))
      throw IoError(path + ": section of entry " + std::to_string(i) + " is out of the file");
    if (e.kind < LQ_WENTRY_FP8 || e.kind > LQ_WENTRY_RAW) throw IoError(path + ": bad kind of entry " + std::to_string(i));
    if (!sizes_match(e)) throw IoError(path + ": section sizes of entry " + std::to_string(i) + " do not fit its shape");
    f->index[std::string(f->strings + e.name_off, e.name_len)] = static_cast<int>(i);
  }
  return f.release();
}

template <class F>
int guarded(F&& fn) {
  try {
    return fn();
  } catch (const ArgError& e) {
    return lq::fail(LQ_ERR_ARG, e.what());
  } catch (const IoError& e) {
    return lq::fail(LQ_ERR_IO, e.what());
  } catch (const std::bad_alloc&) {
    return lq::fail(LQ_ERR_IO, "out of host memory");
  } catch (const std::exception& e) {
    return lq::fail(LQ_ERR_IO, e.what());
  }
}

}  // namespace

extern "C" {

int lq_host_retile_fp8(const uint8_t* w, uint8_t* out, int N, int K) {
  return guarded([&] {
    check_tiling(N, K, "host_retile_fp8");
    if (!w || !out) throw ArgError("host_retile_fp8: null pointer");
    host_retile_fp8(w, out, N, K);
    return LQ_OK;
  });
}

int lq_host_retile_nvfp4(const uint8_t* w, const uint8_t* wscale, uint8_t* out, int N, int K) {
  return guarded([&] {
    check_tiling(N, K, "host_retile_nvfp4");
    if (!w || !wscale || !out) throw ArgError("host_retile_nvfp4: null pointer");
    host_retile_nvfp4_values(w, wscale, out, 1152, nullptr, N, K);
    return LQ_OK;
  });
}

int lq_host_retile_nvfp4_coded(const uint8_t* w, const uint8_t* wscale, const uint8_t* code_of256, uint8_t* out,
                               uint8_t* raw_scales, int N, int K) {
  return guarded([&] {
    check_tiling(N, K, "host_retile_nvfp4_coded");
    if (!w || !wscale || !code_of256 || !out || !raw_scales) throw ArgError("host_retile_nvfp4_coded: null pointer");
    host_retile_nvfp4_coded(w, wscale, code_of256, out, raw_scales, N, K);
    return LQ_OK;
  });
}

int lq_wfile_compile(const char* checkpoint_dir, const char* out_path, int flags, int* entries_written) {
  return guarded([&] {
    if (!checkpoint_dir || !out_path) throw ArgError("wfile_compile: null path");
    if (flags & ~(LQ_WFILE_NO_CODES | LQ_WFILE_PASSTHROUGH | kQuantFlags)) throw ArgError("wfile_compile: unknown flags");
    const int q = flags & kQuantFlags;
    if (q & (q - 1)) throw ArgError("wfile_compile: at most one LQ_WFILE_QUANT_* flag");
    compile_file(checkpoint_dir, out_path, flags, entries_written);
    return LQ_OK;
  });
}

int lq_wfile_open(const char* path, lq_wfile** out) {
  return guarded([&] {
    if (!path || !out) throw ArgError("wfile_open: null pointer");
    *out = nullptr;
    *out = open_file(path);
    return LQ_OK;
  });
}

void lq_wfile_close(lq_wfile* f) { delete f; }

int lq_wfile_count(const lq_wfile* f) { return f ? static_cast<int>(f->h->count) : 0; }

int lq_wfile_find(const lq_wfile* f, const char* name) {
  if (!f || !name) return -1;
  auto it = f->index.find(name);
  return it == f->index.end() ? -1 : it->second;
}

int lq_wfile_entry(const lq_wfile* f, int i, lq_wentry* out) {
  return guarded([&] {
    if (!f || !out) throw ArgError("wfile_entry: null pointer");
    if (i < 0 || i >= static_cast<int>(f->h->count)) throw ArgError("wfile_entry: index out of range");
    const Entry& e = f->entries[i];
    uint8_t* base = f->map->data();
    std::memset(out, 0, sizeof *out);
    out->name = f->strings + e.name_off;
    out->kind = static_cast<int>(e.kind);
    out->scale_kind = static_cast<int>(e.scale_kind);
    out->N = e.N;
    out->K = e.K;
    out->weight_scale = e.weight_scale;
    out->input_scale = e.input_scale;
    out->flags = static_cast<int>(e.flags);
    std::memcpy(out->dtype, e.dtype, sizeof out->dtype);
    out->dtype[sizeof out->dtype - 1] = '\0';
    out->ndim = static_cast<int>(e.ndim);
    for (int d = 0; d < 4; ++d) out->shape[d] = e.shape[d];
    out->blob = e.blob_bytes ? base + e.blob_off : nullptr;
    out->blob_bytes = e.blob_bytes;
    out->aux = e.aux_bytes ? base + e.aux_off : nullptr;
    out->aux_bytes = e.aux_bytes;
    out->table = e.table_bytes ? base + e.table_off : nullptr;
    out->table_bytes = e.table_bytes;
    return LQ_OK;
  });
}

int lq_wfile_verify(const lq_wfile* f, int i) {
  return guarded([&] {
    if (!f) throw ArgError("wfile_verify: null pointer");
    if (i < 0 || i >= static_cast<int>(f->h->count)) throw ArgError("wfile_verify: index out of range");
    const Entry& e = f->entries[i];
    const uint8_t* base = f->map->data();
    const std::string name(f->strings + e.name_off, e.name_len);
    if (hash64(base + e.blob_off, e.blob_bytes) != e.blob_hash) throw IoError(name + ": blob hash mismatch");
    if (hash64(base + e.aux_off, e.aux_bytes) != e.aux_hash) throw IoError(name + ": scale table hash mismatch");
    if (hash64(base + e.table_off, e.table_bytes) != e.table_hash) throw IoError(name + ": code table hash mismatch");
    return LQ_OK;
  });
}

}  // extern "C"
