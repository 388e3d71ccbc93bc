// ctx.hpp -- the library context and error helpers shared by the C-ABI
// translation units (not part of the public interface).
#pragma once

#include <hip/hip_runtime.h>

#include <mutex>
#include <string>
#include <unordered_map>

#include "imq.h"

struct imq_ctx {
  static constexpr int kStagingBuffers = 2;
  static constexpr size_t kStagingBytes = 32u << 20;

  int device = 0;
  mutable std::mutex mu;
  std::string err;
  // Pinned bounce buffers of imq_upload (allocated on first use), each with
  // the event of the last copy that read it.
  std::mutex staging_mu;
  void* staging[kStagingBuffers] = {};
  hipEvent_t staging_done[kStagingBuffers] = {};
  int staging_next = 0;
  // Split-K workspaces of the qGEMM, one per stream: calls on one stream run
  // in order, so they never overlap on a workspace.  Grown (never shrunk) on
  // demand outside stream capture.
  std::mutex ws_mu;
  std::unordered_map<hipStream_t, std::pair<void*, size_t>> split_ws;

  ~imq_ctx();
};

namespace imq {
namespace detail {

// Record a failure on ctx (or, with ctx == nullptr, in the calling thread's
// pre-context slot) and return status.
int fail(imq_ctx* ctx, int status, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
int hip_fail(imq_ctx* ctx, hipError_t e, const char* what);
bool aligned(const void* p, size_t a);
size_t elem_size(imq_dtype dtype);
int bind_device(imq_ctx* ctx);

}  // namespace detail
}  // namespace imq
