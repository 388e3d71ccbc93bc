// weights.cpp -- safetensors shards (memory-mapped) and their upload: the C ABI
// of include/imq_weights.h.  Host code; device work is copies only.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <dirent.h>

#include <algorithm>
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <set>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "ctx.hpp"
#include "imq.h"
#include "imq_weights.h"

using namespace imq::detail;

namespace {

// ---------------------------------------------------------------- JSON ----
// Enough JSON for safetensors headers and index files: objects, arrays,
// strings (with escapes), integers, true/false/null.  Fractions and exponents
// are accepted and kept as doubles (they never appear where integers are read).
struct JVal {
  enum Kind { kNull, kBool, kNum, kStr, kArr, kObj } kind = kNull;
  bool b = false;
  double num = 0.0;
  int64_t inum = 0;
  bool is_int = false;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;

  const JVal* get(const std::string& key) const {
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

class JParser {
 public:
  JParser(const char* p, size_t n) : p_(p), e_(p + n) {}

  bool parse(JVal& out, std::string& err) {
    if (!value(out, 0)) {
      err = err_.empty() ? "malformed JSON" : err_;
      return false;
    }
    ws();
    if (p_ != e_) {
      err = "trailing bytes after the JSON value";
      return false;
    }
    return true;
  }

 private:
  const char* p_;
  const char* e_;
  std::string err_;

  bool bad(const char* what) {
    err_ = what;
    return false;
  }
  void ws() {
    while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char* s) {
    const size_t n = strlen(s);
    if ((size_t)(e_ - p_) < n || memcmp(p_, s, n) != 0) return false;
    p_ += n;
    return true;
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
  bool hex4(uint32_t& v) {
    if (e_ - p_ < 4) return false;
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string& s) {
    if (p_ >= e_ || *p_ != '"') return bad("expected a string");
    ++p_;
    while (true) {
      if (p_ >= e_) return bad("unterminated string");
      const char c = *p_++;
      if (c == '"') return true;
      if ((unsigned char)c < 0x20) return bad("control character in a string");
      if (c != '\\') {
        s += c;
        continue;
      }
      if (p_ >= e_) return bad("unterminated escape");
      const char x = *p_++;
      switch (x) {
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
          if (!hex4(cp)) return bad("bad \\u escape");
          if (cp >= 0xD800 && cp < 0xDC00) {
            uint32_t lo;
            if (!lit("\\u") || !hex4(lo) || lo < 0xDC00 || lo >= 0xE000)
              return bad("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(s, cp);
          break;
        }
        default: return bad("bad escape");
      }
    }
  }
  bool number(JVal& v) {
    const char* s = p_;
    if (p_ < e_ && *p_ == '-') ++p_;
    if (p_ >= e_ || !(*p_ >= '0' && *p_ <= '9')) return bad("bad number");
    while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
    bool integral = true;
    if (p_ < e_ && *p_ == '.') {
      integral = false;
      ++p_;
      while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < e_ && (*p_ == 'e' || *p_ == 'E')) {
      integral = false;
      ++p_;
      if (p_ < e_ && (*p_ == '+' || *p_ == '-')) ++p_;
      while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    const std::string t(s, p_);
    v.kind = JVal::kNum;
    v.num = strtod(t.c_str(), nullptr);
    if (integral) {
      errno = 0;
      const long long ll = strtoll(t.c_str(), nullptr, 10);
      if (errno == ERANGE) return bad("integer out of range");
      v.inum = ll;
      v.is_int = true;
    }
    return true;
  }
  bool value(JVal& v, int depth) {
    if (depth > 64) return bad("JSON nested too deeply");
    ws();
    if (p_ >= e_) return bad("unexpected end of JSON");
    const char c = *p_;
    if (c == '{') {
      ++p_;
      v.kind = JVal::kObj;
      ws();
      if (p_ < e_ && *p_ == '}') {
        ++p_;
        return true;
      }
      while (true) {
        ws();
        std::string key;
        if (!string(key)) return false;
        ws();
        if (p_ >= e_ || *p_ != ':') return bad("expected ':'");
        ++p_;
        JVal child;
        if (!value(child, depth + 1)) return false;
        v.obj.emplace_back(std::move(key), std::move(child));
        ws();
        if (p_ < e_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < e_ && *p_ == '}') {
          ++p_;
          return true;
        }
        return bad("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p_;
      v.kind = JVal::kArr;
      ws();
      if (p_ < e_ && *p_ == ']') {
        ++p_;
        return true;
      }
      while (true) {
        JVal child;
        if (!value(child, depth + 1)) return false;
        v.arr.push_back(std::move(child));
        ws();
        if (p_ < e_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < e_ && *p_ == ']') {
          ++p_;
          return true;
        }
        return bad("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = JVal::kStr;
      return string(v.str);
    }
    if (lit("true")) {
      v.kind = JVal::kBool;
      v.b = true;
      return true;
    }
    if (lit("false")) {
      v.kind = JVal::kBool;
      return true;
    }
    if (lit("null")) return true;
    return number(v);
  }
};

// ------------------------------------------------------------ dtypes ----
struct DtypeName {
  const char* name;
  size_t size;
};
constexpr DtypeName kDtypes[] = {
    {"BOOL", 1}, {"U8", 1},  {"I8", 1},  {"U16", 2}, {"I16", 2},     {"F16", 2},    {"BF16", 2},
    {"U32", 4},  {"I32", 4}, {"F32", 4}, {"U64", 8}, {"I64", 8},     {"F64", 8},    {"F8_E4M3", 1},
    {"F8_E5M2", 1}};
constexpr int kNumDtypes = (int)(sizeof(kDtypes) / sizeof(kDtypes[0]));

int dtype_of(const std::string& s) {
  for (int i = 0; i < kNumDtypes; ++i)
    if (s == kDtypes[i].name) return i;
  return -1;
}

// ------------------------------------------------------------ shards ----
struct Tensor {
  std::string name;
  int dtype = 0;
  std::vector<int64_t> shape;
  const uint8_t* data = nullptr;
  size_t bytes = 0;
  int shard = 0;
};

struct Shard {
  std::string path;
  void* map = nullptr;
  size_t size = 0;
  std::vector<std::pair<std::string, std::string>> metadata;
};

thread_local std::string g_open_error;

int open_fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int open_fail(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_open_error = buf;
  return IMQ_EINVAL;
}

bool mul_ok(size_t a, size_t b, size_t& out) {
  if (a != 0 && b > SIZE_MAX / a) return false;
  out = a * b;
  return true;
}

}  // namespace

struct imq_st {
  std::vector<Shard> shards;
  std::vector<Tensor> tensors;  // sorted by name
  std::unordered_map<std::string, int> index;
  mutable std::mutex mu;
  mutable std::string err;

  ~imq_st() {
    for (auto& s : shards)
      if (s.map && s.map != MAP_FAILED) munmap(s.map, s.size);
  }

  int fail(const char* fmt, ...) const __attribute__((format(printf, 2, 3))) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    std::lock_guard<std::mutex> lk(mu);
    err = buf;
    return IMQ_EINVAL;
  }
};

namespace {

// Map one shard and parse + validate its header; tensors are appended to
// `found` (name -> tensor, a later shard replacing an earlier entry).
int load_shard(imq_st* st, const std::string& path, std::unordered_map<std::string, Tensor>& found) {
  const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return open_fail("%s: cannot open: %s", path.c_str(), strerror(errno));
  struct stat sb;
  if (fstat(fd, &sb) != 0) {
    close(fd);
    return open_fail("%s: cannot stat: %s", path.c_str(), strerror(errno));
  }
  const size_t size = (size_t)sb.st_size;
  if (size < 8) {
    close(fd);
    return open_fail("%s: %zu bytes, too short for a safetensors header", path.c_str(), size);
  }
  void* map = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (map == MAP_FAILED) return open_fail("%s: mmap failed: %s", path.c_str(), strerror(errno));
  Shard shard;
  shard.path = path;
  shard.map = map;
  shard.size = size;
  const int shard_id = (int)st->shards.size();
  st->shards.push_back(shard);  // owns the mapping from here on

  const auto* base = static_cast<const uint8_t*>(map);
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | base[i];
  if (hlen > size - 8)
    return open_fail("%s: header length %llu exceeds the file (%zu bytes)", path.c_str(),
                     (unsigned long long)hlen, size);
  JVal root;
  std::string jerr;
  JParser parser(reinterpret_cast<const char*>(base + 8), (size_t)hlen);
  if (!parser.parse(root, jerr)) return open_fail("%s: header: %s", path.c_str(), jerr.c_str());
  if (root.kind != JVal::kObj) return open_fail("%s: header is not a JSON object", path.c_str());
  const uint8_t* buffer = base + 8 + hlen;
  const size_t buf_size = size - 8 - (size_t)hlen;

  std::vector<std::pair<size_t, size_t>> spans;
  for (const auto& kv : root.obj) {
    if (kv.first == "__metadata__") {
      if (kv.second.kind != JVal::kObj)
        return open_fail("%s: __metadata__ is not an object", path.c_str());
      for (const auto& m : kv.second.obj) {
        if (m.second.kind != JVal::kStr)
          return open_fail("%s: __metadata__[%s] is not a string", path.c_str(), m.first.c_str());
        st->shards[shard_id].metadata.emplace_back(m.first, m.second.str);
      }
      continue;
    }
    const JVal& t = kv.second;
    const char* name = kv.first.c_str();
    const JVal* dt = t.kind == JVal::kObj ? t.get("dtype") : nullptr;
    const JVal* sh = t.kind == JVal::kObj ? t.get("shape") : nullptr;
    const JVal* off = t.kind == JVal::kObj ? t.get("data_offsets") : nullptr;
    if (!dt || dt->kind != JVal::kStr || !sh || sh->kind != JVal::kArr || !off ||
        off->kind != JVal::kArr)
      return open_fail("%s: tensor %s: needs dtype, shape and data_offsets", path.c_str(), name);
    const int dtype = dtype_of(dt->str);
    if (dtype < 0)
      return open_fail("%s: tensor %s: unknown dtype %s", path.c_str(), name, dt->str.c_str());
    if (sh->arr.size() > IMQ_ST_MAX_DIMS)
      return open_fail("%s: tensor %s: %zu dims (at most %d)", path.c_str(), name, sh->arr.size(),
                       IMQ_ST_MAX_DIMS);
    Tensor tensor;
    tensor.name = kv.first;
    tensor.dtype = dtype;
    tensor.shard = shard_id;
    size_t count = 1;
    for (const JVal& d : sh->arr) {
      if (d.kind != JVal::kNum || !d.is_int || d.inum < 0)
        return open_fail("%s: tensor %s: bad shape entry", path.c_str(), name);
      tensor.shape.push_back(d.inum);
      if (!mul_ok(count, (size_t)d.inum, count))
        return open_fail("%s: tensor %s: element count overflows", path.c_str(), name);
    }
    if (off->arr.size() != 2 || off->arr[0].kind != JVal::kNum || !off->arr[0].is_int ||
        off->arr[1].kind != JVal::kNum || !off->arr[1].is_int || off->arr[0].inum < 0 ||
        off->arr[1].inum < off->arr[0].inum)
      return open_fail("%s: tensor %s: bad data_offsets", path.c_str(), name);
    const size_t b0 = (size_t)off->arr[0].inum, b1 = (size_t)off->arr[1].inum;
    if (b1 > buf_size)
      return open_fail("%s: tensor %s: data_offsets [%zu, %zu) past the %zu-byte buffer",
                       path.c_str(), name, b0, b1, buf_size);
    size_t want = 0;
    if (!mul_ok(count, kDtypes[dtype].size, want) || want != b1 - b0)
      return open_fail("%s: tensor %s: %zu bytes for %zu elements of %s", path.c_str(), name,
                       b1 - b0, count, kDtypes[dtype].name);
    tensor.data = buffer + b0;
    tensor.bytes = b1 - b0;
    if (tensor.bytes) spans.emplace_back(b0, b1);
    found[tensor.name] = std::move(tensor);
  }
  std::sort(spans.begin(), spans.end());
  for (size_t i = 1; i < spans.size(); ++i)
    if (spans[i].first < spans[i - 1].second)
      return open_fail("%s: tensor data ranges overlap at byte %zu", path.c_str(), spans[i].first);
  return IMQ_OK;
}

int finish_open(imq_st* st, std::unordered_map<std::string, Tensor>& found, imq_st** out) {
  st->tensors.reserve(found.size());
  for (auto& kv : found) st->tensors.push_back(std::move(kv.second));
  std::sort(st->tensors.begin(), st->tensors.end(),
            [](const Tensor& a, const Tensor& b) { return a.name < b.name; });
  for (size_t i = 0; i < st->tensors.size(); ++i) st->index[st->tensors[i].name] = (int)i;
  *out = st;
  return IMQ_OK;
}

void fill_info(const Tensor& t, imq_st_info* out) {
  out->name = t.name.c_str();
  out->dtype = t.dtype;
  out->ndim = (int)t.shape.size();
  for (int i = 0; i < IMQ_ST_MAX_DIMS; ++i) out->shape[i] = i < out->ndim ? t.shape[i] : 0;
  out->data = t.data;
  out->bytes = t.bytes;
  out->shard = t.shard;
}

bool read_file(const std::string& path, std::string& out) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) return false;
  char buf[65536];
  size_t n;
  while ((n = fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
  const bool ok = !ferror(f);
  fclose(f);
  return ok;
}

// ------------------------------------------------------------ upload ----
float bf16_to_f32(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t f32_to_f16(float f) {
  const _Float16 h = (_Float16)f;  // round to nearest even, with subnormals and overflow to inf
  uint16_t u;
  memcpy(&u, &h, 2);
  return u;
}

float f16_to_f32(uint16_t u) {
  _Float16 h;
  memcpy(&h, &u, 2);
  return (float)h;
}

// Element conversion from a stored safetensors dtype into a library dtype.
enum class Conv { kCopy, kBf16ToF16, kBf16ToF32, kF16ToF32 };

// Elements [i0, i1) of one chunk into the staging buffer, converted.
void fill_stage(uint8_t* stage, const uint8_t* s, size_t i0, size_t i1, size_t src_es,
                Conv conv) {
  switch (conv) {
    case Conv::kCopy: memcpy(stage + i0 * src_es, s + i0 * src_es, (i1 - i0) * src_es); break;
    case Conv::kBf16ToF16: {
      auto* o = reinterpret_cast<uint16_t*>(stage);
      for (size_t i = i0; i < i1; ++i) {
        uint16_t h;
        memcpy(&h, s + 2 * i, 2);
        o[i] = f32_to_f16(bf16_to_f32(h));
      }
      break;
    }
    case Conv::kBf16ToF32:
    case Conv::kF16ToF32: {
      auto* o = reinterpret_cast<float*>(stage);
      for (size_t i = i0; i < i1; ++i) {
        uint16_t h;
        memcpy(&h, s + 2 * i, 2);
        o[i] = conv == Conv::kBf16ToF32 ? bf16_to_f32(h) : f16_to_f32(h);
      }
      break;
    }
  }
}

// Threads that fill one staging chunk (the caller and kCopyThreads - 1
// workers) and the smallest part worth a thread.
constexpr int kCopyThreads = 4;
constexpr size_t kMinPartBytes = 1u << 20;

// Copy (and convert) `count` elements in chunks through the pinned buffers.
// Chunk i waits for the copy that last read its buffer, is filled on the host
// and then copied asynchronously on `stream`.
int staged_copy(imq_ctx* ctx, const char* fn, uint8_t* dst, const uint8_t* src, size_t count,
                size_t src_es, size_t dst_es, Conv conv, hipStream_t stream) {
  std::lock_guard<std::mutex> lk(ctx->staging_mu);
  for (int i = 0; i < imq_ctx::kStagingBuffers; ++i) {
    if (!ctx->staging[i]) {
      hipError_t e = hipHostMalloc(&ctx->staging[i], imq_ctx::kStagingBytes, hipHostMallocDefault);
      if (e != hipSuccess) {
        ctx->staging[i] = nullptr;
        return hip_fail(ctx, e, "pinned staging buffer");
      }
      e = hipEventCreateWithFlags(&ctx->staging_done[i], hipEventDisableTiming);
      if (e != hipSuccess) {
        ctx->staging_done[i] = nullptr;
        return hip_fail(ctx, e, "staging event");
      }
    }
  }
  if (!ctx->copy_pool) {
    ctx->copy_pool.reset(new (std::nothrow) imq::CopyPool(kCopyThreads - 1));
    if (!ctx->copy_pool) return fail(ctx, IMQ_ENOMEM, "%s: out of host memory", fn);
  }
  const size_t per_chunk = imq_ctx::kStagingBytes / std::max(src_es, dst_es);
  for (size_t e0 = 0; e0 < count; e0 += per_chunk) {
    const size_t n = std::min(per_chunk, count - e0);
    const int b = ctx->staging_next;
    ctx->staging_next = (b + 1) % imq_ctx::kStagingBuffers;
    hipError_t e = hipEventSynchronize(ctx->staging_done[b]);
    if (e != hipSuccess) return hip_fail(ctx, e, fn);
    auto* stage = static_cast<uint8_t*>(ctx->staging[b]);
    const uint8_t* s = src + e0 * src_es;
    const int parts = (int)std::min<size_t>(kCopyThreads, std::max<size_t>(1, n * src_es / kMinPartBytes));
    if (parts == 1) {
      fill_stage(stage, s, 0, n, src_es, conv);
    } else {
      // Part boundaries on 64-element multiples (whole cache lines either side).
      const size_t step = (n / parts + 63) / 64 * 64;
      ctx->copy_pool->run(parts, [&](int i) {
        const size_t i0 = std::min(n, (size_t)i * step);
        const size_t i1 = (i == parts - 1) ? n : std::min(n, i0 + step);
        fill_stage(stage, s, i0, i1, src_es, conv);
      });
    }
    e = hipMemcpyAsync(dst + e0 * dst_es, stage, n * dst_es, hipMemcpyHostToDevice, stream);
    if (e != hipSuccess) return hip_fail(ctx, e, fn);
    e = hipEventRecord(ctx->staging_done[b], stream);
    if (e != hipSuccess) return hip_fail(ctx, e, fn);
  }
  return IMQ_OK;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// The conversion from stored dtype `from` to `to` (both imq_st_dtype), if allowed.
bool conversion(int from, int to, Conv& conv) {
  if (from == to) conv = Conv::kCopy;
  else if (from == IMQ_ST_BF16 && to == IMQ_ST_F16) conv = Conv::kBf16ToF16;
  else if (from == IMQ_ST_BF16 && to == IMQ_ST_F32) conv = Conv::kBf16ToF32;
  else if (from == IMQ_ST_F16 && to == IMQ_ST_F32) conv = Conv::kF16ToF32;
  else return false;
  return true;
}

int st_dtype_of(imq_dtype d) { return d == IMQ_BF16 ? IMQ_ST_BF16 : d == IMQ_F16 ? IMQ_ST_F16 : IMQ_ST_F32; }

}  // namespace

extern "C" {

int imq_st_open(const char* const* paths, int n_paths, imq_st** out) {
  if (!out) return open_fail("imq_st_open: null output pointer");
  *out = nullptr;
  if (!paths || n_paths <= 0) return open_fail("imq_st_open: no shard paths");
  auto* st = new (std::nothrow) imq_st;
  if (!st) {
    open_fail("imq_st_open: out of host memory");
    return IMQ_ENOMEM;
  }
  std::unordered_map<std::string, Tensor> found;
  for (int i = 0; i < n_paths; ++i) {
    if (!paths[i]) {
      delete st;
      return open_fail("imq_st_open: null path %d", i);
    }
    const int rc = load_shard(st, paths[i], found);
    if (rc != IMQ_OK) {
      delete st;
      return rc;
    }
  }
  return finish_open(st, found, out);
}

int imq_st_open_dir(const char* directory, imq_st** out) {
  if (!out) return open_fail("imq_st_open_dir: null output pointer");
  *out = nullptr;
  if (!directory) return open_fail("imq_st_open_dir: null directory");
  const std::string dir = directory;
  const std::string sep = (!dir.empty() && dir.back() == '/') ? "" : "/";
  std::vector<std::string> names;
  std::string index_text;
  bool from_index = false;
  if (read_file(dir + sep + "model.safetensors.index.json", index_text)) {
    // SafetensorsLoader.swift:9-15: an unreadable or malformed index, or one
    // without a string weight_map, falls through to the directory listing.
    JVal root;
    std::string jerr;
    JParser parser(index_text.data(), index_text.size());
    if (parser.parse(root, jerr) && root.kind == JVal::kObj) {
      const JVal* map = root.get("weight_map");
      bool all_strings = map && map->kind == JVal::kObj;
      if (all_strings)
        for (const auto& kv : map->obj) all_strings = all_strings && kv.second.kind == JVal::kStr;
      if (all_strings) {
        std::set<std::string> files;
        for (const auto& kv : map->obj) files.insert(kv.second.str);
        names.assign(files.begin(), files.end());
        from_index = true;
      }
    }
  }
  if (!from_index) {
    DIR* d = opendir(directory);
    if (!d) return open_fail("imq_st_open_dir: %s: %s", directory, strerror(errno));
    while (dirent* ent = readdir(d)) {
      const std::string n = ent->d_name;
      const std::string ext = ".safetensors";
      if (n.size() > ext.size() && n.compare(n.size() - ext.size(), ext.size(), ext) == 0)
        names.push_back(n);
    }
    closedir(d);
    std::sort(names.begin(), names.end());
  }
  if (names.empty())
    return open_fail("imq_st_open_dir: weights not found in %s (no *.safetensors)", directory);
  std::vector<std::string> paths;
  std::vector<const char*> ptrs;
  for (const auto& n : names) paths.push_back(dir + sep + n);
  for (const auto& p : paths) ptrs.push_back(p.c_str());
  return imq_st_open(ptrs.data(), (int)ptrs.size(), out);
}

int imq_st_close(imq_st* st) {
  delete st;
  return IMQ_OK;
}

const char* imq_st_last_error(const imq_st* st) {
  if (!st) return g_open_error.c_str();
  std::lock_guard<std::mutex> lk(st->mu);
  return st->err.c_str();
}

int imq_st_shard_count(const imq_st* st) { return st ? (int)st->shards.size() : 0; }

const char* imq_st_shard_path(const imq_st* st, int shard) {
  if (!st || shard < 0 || shard >= (int)st->shards.size()) return nullptr;
  return st->shards[shard].path.c_str();
}

const char* imq_st_metadata(const imq_st* st, int shard, const char* key) {
  if (!st || !key || shard < 0 || shard >= (int)st->shards.size()) return nullptr;
  for (const auto& kv : st->shards[shard].metadata)
    if (kv.first == key) return kv.second.c_str();
  return nullptr;
}

int imq_st_count(const imq_st* st) { return st ? (int)st->tensors.size() : 0; }

int imq_st_info_at(const imq_st* st, int index, imq_st_info* out) {
  if (!st || !out) return open_fail("imq_st_info_at: null argument");
  if (index < 0 || index >= (int)st->tensors.size())
    return st->fail("imq_st_info_at: index %d out of range [0, %zu)", index, st->tensors.size());
  fill_info(st->tensors[index], out);
  return IMQ_OK;
}

int imq_st_find(const imq_st* st, const char* name, imq_st_info* out) {
  if (!st || !name || !out) return open_fail("imq_st_find: null argument");
  const auto it = st->index.find(name);
  if (it == st->index.end()) return st->fail("missing tensor %s", name);
  fill_info(st->tensors[it->second], out);
  return IMQ_OK;
}

int imq_upload(imq_ctx* ctx, void* dst, const void* src, size_t bytes, imq_stream stream) {
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "imq_upload: null context");
  if (bytes == 0) return IMQ_OK;
  if (!dst || !src) return fail(ctx, IMQ_EINVAL, "imq_upload: null pointer");
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  return staged_copy(ctx, "imq_upload", static_cast<uint8_t*>(dst),
                     static_cast<const uint8_t*>(src), bytes, 1, 1, Conv::kCopy,
                     static_cast<hipStream_t>(stream));
}

int imq_st_upload(imq_ctx* ctx, const imq_st* st, const char* name, int dst_dtype, void* dst,
                  size_t dst_bytes, imq_stream stream) {
  const char* fn = "imq_st_upload";
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "%s: null context", fn);
  if (!st || !name || !dst) return fail(ctx, IMQ_EINVAL, "%s: null argument", fn);
  const auto it = st->index.find(name);
  if (it == st->index.end()) return fail(ctx, IMQ_EINVAL, "missing tensor %s", name);
  const Tensor& t = st->tensors[it->second];
  Conv conv = Conv::kCopy;
  if (dst_dtype < 0 || dst_dtype >= kNumDtypes || !conversion(t.dtype, dst_dtype, conv))
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: %s: %s to dtype %d", fn, name, kDtypes[t.dtype].name,
                dst_dtype);
  const size_t src_es = kDtypes[t.dtype].size;
  const size_t dst_es = kDtypes[dst_dtype].size;
  const size_t count = t.bytes / src_es;
  if (dst_bytes != count * dst_es)
    return fail(ctx, IMQ_EINVAL, "%s: %s: destination holds %zu bytes, the tensor needs %zu", fn,
                name, dst_bytes, count * dst_es);
  if (count == 0) return IMQ_OK;
  const int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  return staged_copy(ctx, fn, static_cast<uint8_t*>(dst), t.data, count, src_es, dst_es, conv,
                     static_cast<hipStream_t>(stream));
}

int imq_load_qlinear_cat(imq_ctx* ctx, const imq_st* st, const char* const* prefixes, int count,
                         imq_dtype param_dtype, imq_qweight* out, imq_stream stream) {
  const char* fn = "imq_load_qlinear_cat";
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "%s: null context", fn);
  if (!st || !prefixes || count <= 0 || !out) return fail(ctx, IMQ_EINVAL, "%s: null argument", fn);
  memset(out, 0, sizeof *out);
  if (param_dtype != IMQ_BF16 && param_dtype != IMQ_F16 && param_dtype != IMQ_F32)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: dtype %d", fn, (int)param_dtype);
  // Every part: its three tensors, checked; all parts share K and the scale type.
  struct Part {
    const Tensor* t[3];
    int64_t n;
  };
  std::vector<Part> parts((size_t)count);
  const char* suffix[3] = {".weight", ".scales", ".biases"};
  int64_t k = 0, n_total = 0;
  int src_dtype = -1;
  for (int pi = 0; pi < count; ++pi) {
    const char* prefix = prefixes[pi];
    if (!prefix) return fail(ctx, IMQ_EINVAL, "%s: null prefix %d", fn, pi);
    const std::string p = prefix;
    Part& part = parts[(size_t)pi];
    for (int i = 0; i < 3; ++i) {
      const auto it = st->index.find(p + suffix[i]);
      if (it == st->index.end())
        return fail(ctx, IMQ_EINVAL, "missing tensor %s%s", prefix, suffix[i]);
      part.t[i] = &st->tensors[it->second];
    }
    const Tensor* const* t = part.t;
    if (t[0]->dtype != IMQ_ST_U32 || t[0]->shape.size() != 2)
      return fail(ctx, IMQ_EINVAL, "%s: %s.weight must be U32 [N, K/8]", fn, prefix);
    const int64_t n = t[0]->shape[0];
    const int64_t kk = t[0]->shape[1] * 8;
    if (n <= 0 || kk <= 0 || kk % 64 != 0 || n > INT32_MAX || kk > INT32_MAX)
      return fail(ctx, IMQ_EINVAL, "%s: %s: bad packed shape [%lld, %lld]", fn, prefix,
                  (long long)n, (long long)t[0]->shape[1]);
    if (pi == 0) {
      k = kk;
      src_dtype = t[1]->dtype;
    } else if (kk != k) {
      return fail(ctx, IMQ_EINVAL, "%s: %s has K=%lld, %s has K=%lld", fn, prefix, (long long)kk,
                  prefixes[0], (long long)k);
    }
    for (int i = 1; i < 3; ++i) {
      if (t[i]->dtype != src_dtype ||
          (src_dtype != IMQ_ST_BF16 && src_dtype != IMQ_ST_F16 && src_dtype != IMQ_ST_F32))
        return fail(ctx, IMQ_EINVAL, "%s: %s scales and biases must share BF16, F16 or F32 (and "
                    "the first projection's type)", fn, prefix);
      if (t[i]->shape.size() != 2 || t[i]->shape[0] != n || t[i]->shape[1] != k / 64)
        return fail(ctx, IMQ_EINVAL, "%s: %s%s must be [%lld, %lld]", fn, prefix, suffix[i],
                    (long long)n, (long long)(k / 64));
    }
    part.n = n;
    n_total += n;
  }
  if (n_total > INT32_MAX)
    return fail(ctx, IMQ_EINVAL, "%s: %lld rows in all", fn, (long long)n_total);
  Conv conv = Conv::kCopy;
  if (!conversion(src_dtype, st_dtype_of(param_dtype), conv))
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: %s scales to dtype %d", fn, kDtypes[src_dtype].name,
                (int)param_dtype);
  const size_t src_es = kDtypes[src_dtype].size;
  const size_t dst_es = elem_size(param_dtype);
  const size_t row_w = (size_t)k / 2, row_p = (size_t)(k / 64);
  const size_t w_bytes = (size_t)n_total * row_w;
  const size_t n_params = (size_t)n_total * row_p;
  const size_t s_off = align_up(w_bytes, 256);
  const size_t b_off = s_off + align_up(n_params * dst_es, 256);
  const size_t total = b_off + n_params * dst_es;
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  void* base = nullptr;
  hipError_t e = hipMalloc(&base, total);
  if (e == hipErrorOutOfMemory)
    return fail(ctx, IMQ_ENOMEM, "%s: %zu bytes: out of device memory", fn, total);
  if (e != hipSuccess) return hip_fail(ctx, e, fn);
  auto* b8 = static_cast<uint8_t*>(base);
  const auto st_ = static_cast<hipStream_t>(stream);
  size_t row0 = 0;
  for (const Part& part : parts) {
    const size_t np = (size_t)part.n * row_p;
    rc = staged_copy(ctx, fn, b8 + row0 * row_w, part.t[0]->data, part.t[0]->bytes, 1, 1,
                     Conv::kCopy, st_);
    if (rc == IMQ_OK)
      rc = staged_copy(ctx, fn, b8 + s_off + row0 * row_p * dst_es, part.t[1]->data, np, src_es,
                       dst_es, conv, st_);
    if (rc == IMQ_OK)
      rc = staged_copy(ctx, fn, b8 + b_off + row0 * row_p * dst_es, part.t[2]->data, np, src_es,
                       dst_es, conv, st_);
    if (rc != IMQ_OK) break;
    row0 += (size_t)part.n;
  }
  if (rc != IMQ_OK) {
    (void)hipStreamSynchronize(st_);
    (void)hipFree(base);
    return rc;
  }
  out->w = reinterpret_cast<uint32_t*>(b8);
  out->scales = b8 + s_off;
  out->biases = b8 + b_off;
  out->n = (int)n_total;
  out->k = (int)k;
  out->dtype = param_dtype;
  out->base = base;
  return IMQ_OK;
}

int imq_load_qlinear(imq_ctx* ctx, const imq_st* st, const char* prefix, imq_dtype param_dtype,
                     imq_qweight* out, imq_stream stream) {
  if (!prefix) {
    if (out) memset(out, 0, sizeof *out);
    return fail(ctx, IMQ_EINVAL, "imq_load_qlinear: null argument");
  }
  const int rc = imq_load_qlinear_cat(ctx, st, &prefix, 1, param_dtype, out, stream);
  if (rc != IMQ_OK && ctx) {
    // Report under the entry point the caller used.
    std::lock_guard<std::mutex> lk(ctx->mu);
    const std::string cat = "imq_load_qlinear_cat";
    if (ctx->err.compare(0, cat.size(), cat) == 0) ctx->err.replace(0, cat.size(), "imq_load_qlinear");
  }
  return rc;
}

int imq_qweight_free(imq_ctx* ctx, imq_qweight* q) {
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "imq_qweight_free: null context");
  if (!q || !q->base) return IMQ_OK;
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  const hipError_t e = hipFree(q->base);
  memset(q, 0, sizeof *q);
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, "imq_qweight_free");
}

}  // extern "C"
