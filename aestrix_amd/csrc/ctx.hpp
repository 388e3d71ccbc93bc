// ctx.hpp -- the library context and error helpers shared by the C-ABI
// translation units (not part of the public interface).
#pragma once

#include <hip/hip_runtime.h>

#include <condition_variable>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "imq.h"

namespace imq {

// A few host threads that fill the pinned staging buffers together: one
// thread's memcpy into pinned memory (about 30 GB/s) is half of what the
// host-to-device DMA takes (about 58 GB/s), two to four threads match it.
class CopyPool {
 public:
  explicit CopyPool(int workers);
  ~CopyPool();
  // fn(i) for every i in [0, parts), on the workers and the calling thread;
  // returns when all parts are done.  One run at a time.
  void run(int parts, const std::function<void(int)>& fn);

 private:
  void work();
  std::vector<std::thread> threads_;
  std::mutex mu_;
  std::condition_variable start_cv_, done_cv_;
  const std::function<void(int)>* fn_ = nullptr;
  int parts_ = 0, next_ = 0, remaining_ = 0;
  unsigned long gen_ = 0;
  bool stop_ = false;
};

}  // namespace imq

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
  std::unique_ptr<imq::CopyPool> copy_pool;  // created with the staging buffers
  // Split-K workspaces of the qGEMM, one per stream: calls on one stream run
  // in order, so they never overlap on a workspace.  Grown (never shrunk) on
  // demand outside stream capture; an outgrown one is kept until the context
  // is destroyed (graphs captured earlier may still address it).
  std::mutex ws_mu;
  std::unordered_map<hipStream_t, std::pair<void*, size_t>> split_ws;
  std::vector<void*> retired_ws;  // outgrown workspaces, freed with the context
  // Device address of the library's static split-K scratch on this device
  // (imq_qmm_t_noalloc), looked up at imq_create.
  void* static_scratch = nullptr;

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
