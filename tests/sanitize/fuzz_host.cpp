// fuzz_host.cpp -- bounded, seeded fuzz of libimq's host code under
// AddressSanitizer and UndefinedBehaviorSanitizer (no GPU): the safetensors
// reader (header JSON, entry validation, shard discovery from an index file)
// and the argument checks of the C entry points.
//
// TEST INFRASTRUCTURE ONLY (built by tests/sanitize/Makefile, run by
// tests/test_sanitize_cpu.py).  Usage: fuzz_host <work dir> <iterations> <seed>
// Prints "fuzz_host: <n> files, <m> opened, <k> rejected, <c> abi checks" and
// exits 0; any sanitizer report aborts with a non-zero status.
#include <dirent.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cinttypes>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "imq.h"
#include "imq_step.h"
#include "imq_weights.h"

namespace {

std::mt19937_64 rng;

uint64_t rnd(uint64_t n) { return n ? rng() % n : 0; }

const char* kDtypes[] = {"BOOL", "U8",  "I8",  "U16", "I16", "F16",     "BF16",    "U32",
                         "I32",  "F32", "U64", "I64", "F64", "F8_E4M3", "F8_E5M2"};
const int kSizes[] = {1, 1, 1, 2, 2, 2, 2, 4, 4, 4, 8, 8, 8, 1, 1};

// A well-formed shard: a few tensors of random dtype and shape, packed in order.
std::string valid_shard(int* n_tensors) {
  const int nt = 1 + (int)rnd(5);
  std::string json = "{";
  size_t off = 0;
  for (int t = 0; t < nt; ++t) {
    const int d = (int)rnd(15);
    const int nd = (int)rnd(4);
    std::string shape = "[";
    size_t count = 1;
    for (int i = 0; i < nd; ++i) {
      const int e = 1 + (int)rnd(6);
      count *= (size_t)e;
      shape += (i ? "," : "") + std::to_string(e);
    }
    shape += "]";
    const size_t bytes = count * (size_t)kSizes[d];
    char ent[256];
    snprintf(ent, sizeof ent, "%s\"t%d\":{\"dtype\":\"%s\",\"shape\":%s,\"data_offsets\":[%zu,%zu]}",
             t ? "," : "", t, kDtypes[d], shape.c_str(), off, off + bytes);
    json += ent;
    off += bytes;
  }
  json += ",\"__metadata__\":{\"format\":\"pt\",\"k\":\"v\\u00e9\"}}";
  std::string out(8, '\0');
  const uint64_t h = json.size();
  memcpy(&out[0], &h, 8);
  out += json;
  for (size_t i = 0; i < off; ++i) out += (char)rnd(256);
  *n_tensors = nt;
  return out;
}

// Random JSON-ish text: nesting, escapes, numbers, truncation.  At most one
// nested value per level (the text stays linear in the depth).
std::string junk_json(int depth) {
  static const char* atoms[] = {"null", "true", "false", "0", "-1", "1e400", "18446744073709551616",
                                "\"\\u12\"", "\"\\ud800\"", "\"a\\\"b\"", "[", "{", "\"dtype\"",
                                "\"data_offsets\"", "[0,99999999999]", "\"BF16\"", "-", "\"\\"};
  std::string s;
  const int parts = 1 + (int)rnd(8);
  const int nest = (int)rnd(parts);  // the one part that nests
  for (int i = 0; i < parts; ++i) {
    const int k = (int)rnd(2);
    if (i == nest && depth < 300 && k == 0) s += "{\"x\":" + junk_json(depth + 1) + "}";
    else if (i == nest && depth < 300) s += "[" + junk_json(depth + 1) + "]";
    else s += atoms[rnd(sizeof atoms / sizeof *atoms)];
    if (rnd(2)) s += ",";
  }
  return s;
}

std::string mutate(std::string f) {
  switch (rnd(7)) {
    case 0:  // truncate
      f.resize(rnd(f.size() + 1));
      break;
    case 1:  // flip bytes anywhere
      for (int i = 0, n = 1 + (int)rnd(8); i < n && !f.empty(); ++i) f[rnd(f.size())] ^= (char)(1 + rnd(255));
      break;
    case 2: {  // random header length
      const uint64_t choices[] = {0, 1, 7, (uint64_t)f.size(), (uint64_t)f.size() + 1, UINT64_MAX,
                                  (uint64_t)1 << 40, rnd(1 << 20)};
      const uint64_t h = choices[rnd(8)];
      if (f.size() >= 8) memcpy(&f[0], &h, 8);
      break;
    }
    case 3: {  // replace the header with junk of the stated length
      const std::string j = "{" + junk_json(0) + "}";
      std::string out(8, '\0');
      const uint64_t h = j.size();
      memcpy(&out[0], &h, 8);
      f = out + j + std::string(rnd(64), 'x');
      break;
    }
    case 4: {  // overlapping / out-of-range offsets, bad shapes, unknown dtypes
      static const char* ents[] = {
          "{\"a\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[0,8]},"
          "\"b\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[4,12]}}",
          "{\"a\":{\"dtype\":\"F32\",\"shape\":[-1],\"data_offsets\":[0,4]}}",
          "{\"a\":{\"dtype\":\"F32\",\"shape\":[4294967296,4294967296],\"data_offsets\":[0,4]}}",
          "{\"a\":{\"dtype\":\"Q4\",\"shape\":[1],\"data_offsets\":[0,1]}}",
          "{\"a\":{\"dtype\":\"U8\",\"shape\":[3],\"data_offsets\":[2,1]}}",
          "{\"a\":{\"dtype\":\"U8\",\"shape\":[1,1,1,1,1,1,1,1,1],\"data_offsets\":[0,1]}}",
          "{\"a\":{\"dtype\":\"U8\",\"shape\":[2],\"data_offsets\":[0,2]},\"a\":{\"dtype\":\"U8\","
          "\"shape\":[2],\"data_offsets\":[0,2]}}",
          "{\"a\":{\"dtype\":\"U8\",\"shape\":[1.5],\"data_offsets\":[0,1]}}",
          "{\"__metadata__\":{\"k\":7}}",
          "{\"a\":{\"dtype\":\"U8\",\"shape\":[16],\"data_offsets\":[0,16]}}"};
      const std::string j = ents[rnd(sizeof ents / sizeof *ents)];
      std::string out(8, '\0');
      const uint64_t h = j.size();
      memcpy(&out[0], &h, 8);
      f = out + j + std::string(rnd(20), 'y');
      break;
    }
    case 5:  // header padded with spaces (allowed), then garbage
      if (f.size() > 8) f.insert(f.size() / 2, std::string(rnd(16), ' '));
      break;
    default:
      break;
  }
  return f;
}

void write_file(const std::string& path, const std::string& bytes) {
  FILE* fp = fopen(path.c_str(), "wb");
  if (!fp) {
    perror(path.c_str());
    exit(2);
  }
  if (!bytes.empty() && fwrite(bytes.data(), 1, bytes.size(), fp) != bytes.size()) exit(2);
  fclose(fp);
}

// Touch every byte the reader exposes, so a bad offset trips the sanitizer
// (or the kernel) here rather than going unnoticed.
uint64_t walk(const imq_st* st) {
  uint64_t sum = 0;
  const int n = imq_st_count(st);
  for (int i = 0; i < n; ++i) {
    imq_st_info info;
    if (imq_st_info_at(st, i, &info) != IMQ_OK) continue;
    const auto* p = static_cast<const unsigned char*>(info.data);
    for (size_t b = 0; b < info.bytes; ++b) sum += p[b];
    imq_st_info again;
    if (imq_st_find(st, info.name, &again) != IMQ_OK || again.data != info.data) {
      fprintf(stderr, "fuzz_host: find(%s) disagrees with info_at\n", info.name);
      exit(3);
    }
    sum += strlen(info.name) + (uint64_t)info.ndim;
  }
  imq_st_info none;
  if (imq_st_find(st, "no such tensor", &none) == IMQ_OK) exit(3);
  for (int s = 0; s < imq_st_shard_count(st); ++s) {
    const char* m = imq_st_metadata(st, s, "format");
    if (m) sum += strlen(m);
    if (imq_st_shard_path(st, s) == nullptr) exit(3);
  }
  sum += strlen(imq_st_last_error(st));
  return sum;
}

int abi_checks() {
  int n = 0;
  auto expect = [&](int got, int want, const char* what) {
    ++n;
    if (got != want) {
      fprintf(stderr, "fuzz_host: %s returned %d, expected %d\n", what, got, want);
      exit(4);
    }
  };
  uint32_t w[16] = {};
  uint16_t s[4] = {}, y[4] = {};
  expect(imq_qmm_t(nullptr, w, s, s, s, y, 64, 1, 1, 64, 4, IMQ_BF16, nullptr), IMQ_EINVAL,
         "imq_qmm_t(null ctx)");
  expect(imq_qmm_t_noalloc(nullptr, w, s, s, s, y, 64, 1, 1, 64, 4, IMQ_BF16, nullptr), IMQ_EINVAL,
         "imq_qmm_t_noalloc(null ctx)");
  expect(imq_qgemv(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0, 0, IMQ_BF16,
                   nullptr),
         IMQ_EINVAL, "imq_qgemv(null)");
  expect(imq_qgemm(nullptr, w, s, s, s, y, -64, 1, 1, 64, 4, IMQ_F16, nullptr), IMQ_EINVAL,
         "imq_qgemm(null ctx)");
  expect(imq_dequantize(nullptr, w, s, s, y, 64, 1, 64, 4, IMQ_BF16, nullptr), IMQ_EINVAL,
         "imq_dequantize(null ctx)");
  expect(imq_cast_prescale(nullptr, nullptr, y, 4, 16.0f, IMQ_F16, nullptr), IMQ_EINVAL,
         "imq_cast_prescale(null ctx)");
  expect(imq_qmm_postscale(nullptr, w, s, s, s, nullptr, 64, 1, 1, 1.0f, 64, 4, IMQ_F16, nullptr),
         IMQ_EINVAL, "imq_qmm_postscale(null ctx)");
  expect(imq_qmm_gate_add(nullptr, w, s, s, s, nullptr, nullptr, nullptr, 64, 1, 1, 1.0f, 64, 4,
                          IMQ_F16, nullptr),
         IMQ_EINVAL, "imq_qmm_gate_add(null ctx)");
  expect(imq_qmm_swiglu(nullptr, w, s, s, s, y, 1, 64, 2, 1, 1, 0, 1, 1.0f, 1.0f, 64, 4, IMQ_F16,
                        nullptr),
         IMQ_EINVAL, "imq_qmm_swiglu(null ctx)");
  imq_plan plan;
  expect(imq_qmm_plan(nullptr, IMQ_ENTRY_QMM_T, 64, 1, 1, IMQ_BF16, &plan), IMQ_EINVAL,
         "imq_qmm_plan(null ctx)");
  expect(imq_stream_sync(nullptr, nullptr), IMQ_EINVAL, "imq_stream_sync(null)");
  expect(imq_malloc(nullptr, 16, nullptr), IMQ_EINVAL, "imq_malloc(null)");
  expect(imq_free(nullptr, nullptr), IMQ_EINVAL, "imq_free(null)");
  expect(imq_memcpy_h2d(nullptr, y, s, 4, nullptr), IMQ_EINVAL, "imq_memcpy_h2d(null)");
  expect(imq_upload(nullptr, y, s, 4, nullptr), IMQ_EINVAL, "imq_upload(null)");
  expect(imq_st_upload(nullptr, nullptr, "x", 0, y, 4, nullptr), IMQ_EINVAL, "imq_st_upload(null)");
  imq_qweight q;
  expect(imq_load_qlinear(nullptr, nullptr, "x", IMQ_BF16, &q, nullptr), IMQ_EINVAL,
         "imq_load_qlinear(null)");
  const char* names[2] = {"a", nullptr};
  expect(imq_load_qlinear_cat(nullptr, nullptr, names, 2, IMQ_BF16, &q, nullptr), IMQ_EINVAL,
         "imq_load_qlinear_cat(null)");
  expect(imq_qweight_free(nullptr, &q), IMQ_EINVAL, "imq_qweight_free(null)");
  imq_dit_dims d = {64, 32, 256, 256, 1, 1};
  imq_dit_step* stp = nullptr;
  expect(imq_dit_step_create(nullptr, &d, nullptr, 0, IMQ_F16, &stp), IMQ_EINVAL,
         "imq_dit_step_create(null ctx)");
  expect(imq_dit_step_run(nullptr, nullptr, nullptr, nullptr, 1, nullptr), IMQ_EINVAL,
         "imq_dit_step_run(null)");
  expect(imq_dit_step_denoise(nullptr, nullptr, nullptr, nullptr, 0.1f, 1, nullptr), IMQ_EINVAL,
         "imq_dit_step_denoise(null)");
  expect(imq_dit_step_set_head(nullptr, nullptr, nullptr), IMQ_EINVAL, "imq_dit_step_set_head(null)");
  expect(imq_dit_step_set_conditioning(nullptr, nullptr, nullptr, nullptr), IMQ_EINVAL,
         "imq_dit_step_set_conditioning(null)");
  expect(imq_dit_step_destroy(nullptr), IMQ_OK, "imq_dit_step_destroy(null)");
  expect(imq_dit_step_launches(nullptr), 0, "imq_dit_step_launches(null)");
  imq_ctx* ctx = nullptr;
  expect(imq_create(0, nullptr), IMQ_EINVAL, "imq_create(null out)");
  const int rc = imq_create(-1, &ctx);  // no device: EHIP (count fails) or EINVAL (out of range)
  ++n;
  if (rc == IMQ_OK || ctx != nullptr) {
    fprintf(stderr, "fuzz_host: imq_create(-1) succeeded\n");
    exit(4);
  }
  if (strlen(imq_last_error(nullptr)) == 0) exit(4);
  for (int st = -3; st < 8; ++st) n += imq_status_string(st) != nullptr;
  expect(imq_abi_version(), IMQ_ABI_VERSION, "imq_abi_version");
  expect(imq_destroy(nullptr), IMQ_OK, "imq_destroy(null)");
  return n;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 4) {
    fprintf(stderr, "usage: fuzz_host <work dir> <iterations> <seed>\n");
    return 2;
  }
  const std::string dir = argv[1];
  const int iters = atoi(argv[2]);
  rng.seed(strtoull(argv[3], nullptr, 10));
  mkdir(dir.c_str(), 0755);
  int files = 0, opened = 0, rejected = 0;
  uint64_t sum = 0;
  for (int it = 0; it < iters; ++it) {
    int nt = 0;
    std::string f = valid_shard(&nt);
    const bool clean = it % 4 == 0;
    if (!clean) f = mutate(f);
    const std::string path = dir + "/" + std::to_string(it % 8) + ".safetensors";
    write_file(path, f);
    ++files;
    const char* paths[1] = {path.c_str()};
    imq_st* st = nullptr;
    const int rc = imq_st_open(paths, 1, &st);
    if (rc == IMQ_OK) {
      ++opened;
      if (clean && imq_st_count(st) != nt) {
        fprintf(stderr, "fuzz_host: clean shard %d: %d tensors, wrote %d\n", it, imq_st_count(st), nt);
        return 3;
      }
      sum += walk(st);
      imq_st_close(st);
    } else {
      ++rejected;
      if (clean) {
        fprintf(stderr, "fuzz_host: clean shard %d rejected: %s\n", it, imq_st_last_error(nullptr));
        return 3;
      }
      if (st != nullptr || strlen(imq_st_last_error(nullptr)) == 0) return 3;
    }
    // Every 16th iteration: a directory with an index file (maybe malformed)
    // naming some of the shards written so far, and maybe missing ones.
    if (it % 16 == 15) {
      const std::string sub = dir + "/d" + std::to_string(it);
      mkdir(sub.c_str(), 0755);
      write_file(sub + "/a.safetensors", valid_shard(&nt));
      write_file(sub + "/b.safetensors", rnd(2) ? valid_shard(&nt) : mutate(valid_shard(&nt)));
      std::string idx;
      switch (rnd(4)) {
        case 0: idx = "{\"weight_map\":{\"t0\":\"a.safetensors\",\"t1\":\"b.safetensors\"}}"; break;
        case 1: idx = "{\"weight_map\":{\"t0\":\"missing.safetensors\"}}"; break;
        case 2: idx = "{" + junk_json(0); break;
        default: idx = "{\"weight_map\":{\"t0\":\"../a.safetensors\",\"t1\":7}}"; break;
      }
      write_file(sub + "/model.safetensors.index.json", idx);
      imq_st* ds = nullptr;
      if (imq_st_open_dir(sub.c_str(), &ds) == IMQ_OK) {
        sum += walk(ds);
        imq_st_close(ds);
      }
      for (const char* name : {"a.safetensors", "b.safetensors", "model.safetensors.index.json"})
        unlink((sub + "/" + name).c_str());
      rmdir(sub.c_str());
    }
  }
  imq_st* none = nullptr;
  if (imq_st_open_dir((dir + "/does-not-exist").c_str(), &none) == IMQ_OK) return 3;
  if (imq_st_open(nullptr, 0, &none) == IMQ_OK) return 3;
  const int checks = abi_checks();
  for (int i = 0; i < 8; ++i) unlink((dir + "/" + std::to_string(i) + ".safetensors").c_str());
  printf("fuzz_host: %d files, %d opened, %d rejected, %d abi checks (checksum %" PRIu64 ")\n",
         files, opened, rejected, checks, sum);
  return 0;
}
