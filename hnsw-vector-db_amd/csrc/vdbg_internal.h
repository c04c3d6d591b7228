// vdbg_internal.h -- host-side structures shared by the C ABI and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/vdbg.h"

namespace vdbg {

// Status codes, numbered as vdb::Status::Code (include/vdb/status.h:14-26).
enum Code : int {
  kOk = VDBG_OK,
  kInvalidArgument = VDBG_INVALID_ARGUMENT,
  kNotFound = VDBG_NOT_FOUND,
  kFailedPrecondition = VDBG_FAILED_PRECONDITION,
  kResourceExhausted = VDBG_RESOURCE_EXHAUSTED,
  kNotSupported = VDBG_NOT_SUPPORTED,
  kInternal = VDBG_INTERNAL,
};

int SetError(int code, const std::string& msg);  // records the thread's message, returns code

#define VDBG_HIP(expr)                                                                  \
  do {                                                                                  \
    hipError_t e_ = (expr);                                                             \
    if (e_ != hipSuccess)                                                               \
      return ::vdbg::SetError(e_ == hipErrorOutOfMemory ? ::vdbg::kResourceExhausted    \
                                                        : ::vdbg::kInternal,            \
                              std::string(#expr) + ": " + hipGetErrorString(e_));      \
  } while (0)

#define VDBG_RETURN_IF_ERROR(expr) \
  do {                             \
    int rc_ = (expr);              \
    if (rc_ != 0) return rc_;      \
  } while (0)

// Value statistics of a resident row set, used to decide when the GEMM formulation is
// exact (integer-valued data with bounded sums) and to bound its rounding otherwise.
struct RowStats {
  float lo = 0.f, hi = 0.f;  // min and max over all stored values (padding included)
  float max_abs = 0.f;
  float xn_max = 0.f;        // largest row norm ||x||^2
  int all_int = 1;           // every value is an integer
};

// Grow-only device scratch, carved into aligned slices per call.
struct Workspace {
  void* base = nullptr;
  size_t cap = 0;
  size_t used = 0;
  int reserve(size_t bytes);  // makes `bytes` available (may reallocate; call before carving)
  template <class T>
  T* take(size_t count) {
    size_t off = (used + 255) & ~size_t(255);
    used = off + count * sizeof(T);
    return reinterpret_cast<T*>(static_cast<char*>(base) + off);
  }
  void release();
};

struct ProfEntry {
  std::string name;
  hipEvent_t start, stop;
};

struct Ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::recursive_mutex mu;
  Workspace ws;   // per-call scratch
  Workspace ws2;  // scratch of the exact re-scan that runs while ws is live
  uint32_t* host_pinned = nullptr;  // small pinned staging for counters
  bool profiling = false;
  std::vector<ProfEntry> pending;
  std::vector<hipEvent_t> free_events;
  std::map<std::string, std::pair<double, uint64_t>> prof;  // name -> (ms, launches)
  uint64_t last_fallbacks = 0;
  int device_arch_ok = 1;
};

struct Dataset {
  Ctx* ctx = nullptr;
  float* rows = nullptr;   // n x pd
  float* norms = nullptr;  // n row norms (fp32, ||x||^2)
  size_t n = 0, dim = 0, pd = 0;
  int metric = 0;
  RowStats stats;
};

// Brackets a launch with events when the context is profiling.
class ProfScope {
 public:
  ProfScope(Ctx* c, const char* name, hipStream_t s);
  ~ProfScope();

 private:
  Ctx* c_;
  hipStream_t s_;
  ProfEntry e_;
  bool on_;
};

// ---------------------------------------------------------------- launchers

int LaunchRowStats(Ctx* c, hipStream_t s, const float* rows, size_t n, size_t pd,
                   float* norms, RowStats* out);

struct FlatPlan;
// Flat exact search over a resident dataset; queries/outputs/allow are device pointers.
int FlatSearch(Dataset* ds, const float* Q, size_t nq, size_t k, const uint64_t* allow,
               uint32_t* out_ids, float* out_d, hipStream_t s);

}  // namespace vdbg

struct vdbg_ctx {
  vdbg::Ctx c;
};
struct vdbg_dataset {
  vdbg::Dataset d;
};
