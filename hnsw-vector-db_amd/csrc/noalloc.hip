// noalloc.hip -- the allocation-free flat search: vdbg_flat_search_device's pipeline with all
// of its scratch in a static device array, for callers that cannot allocate device memory
// (tight serving loops, harnesses that forbid hipMalloc).  It is not capturable into a HIP
// graph: like vdbg_flat_search_device it reads the count of uncertified queries back on the
// host before it queues their exact re-scan.
#include <mutex>
#include <string>

#include "gemm.h"
#include "vdbg_internal.h"

namespace vdbg {

// The array's size and its split: the scan pipeline's buffers (query terms, sample minima,
// candidate buffers, operands) in the first part, the exact re-scan of uncertified queries in
// the last kNoAllocExactBytes.  Every GPU the library runs on holds one copy until the process
// ends.
constexpr size_t kNoAllocBytes = size_t(32) << 20;
constexpr size_t kNoAllocExactBytes = size_t(8) << 20;
constexpr int kNoAllocMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

namespace {

struct DeviceScratch {
  std::mutex mu;                 // one call's host part at a time on this device
  bool ready = false;
  unsigned char* ptr = nullptr;  // this device's address of `scratch`
  Workspace ws, ws2;             // fixed workspaces over ptr
};

DeviceScratch g_scratch[kNoAllocMaxDevices];
std::mutex g_init_mu;

}  // namespace

// Looks up this device's address of `scratch` (each device holds its own copy of the array
// at its own address) and sets the fixed workspaces over it, once per device.  Called by
// vdbg_ctx_create with `device` current.  From here on only the looked-up address is used:
// the array's name in host code is a host-side stand-in, not a device address.
int InitNoAllocScratch(int device) {
  if (device < 0 || device >= kNoAllocMaxDevices) return kOk;  // the entry point refuses it
  std::lock_guard<std::mutex> g(g_init_mu);
  DeviceScratch& d = g_scratch[device];
  if (d.ready) return kOk;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr)
    return SetError(kInternal, std::string("allocation-free scratch address: ") +
                                   hipGetErrorString(e));
  hipEvent_t e1 = nullptr, e2 = nullptr;
  if (hipEventCreateWithFlags(&e1, hipEventDisableTiming) != hipSuccess)
    return SetError(kInternal, "allocation-free scratch event");
  if (hipEventCreateWithFlags(&e2, hipEventDisableTiming) != hipSuccess) {
    (void)hipEventDestroy(e1);
    return SetError(kInternal, "allocation-free scratch event");
  }
  d.ptr = static_cast<unsigned char*>(p);
  d.ws.base = d.ptr;
  d.ws.cap = kNoAllocBytes - kNoAllocExactBytes;
  d.ws.fixed = true;
  d.ws.name = "vdbg_flat_search_device_noalloc (scan)";
  d.ws.done = e1;
  d.ws2.base = d.ptr + (kNoAllocBytes - kNoAllocExactBytes);
  d.ws2.cap = kNoAllocExactBytes;
  d.ws2.fixed = true;
  d.ws2.name = "vdbg_flat_search_device_noalloc (exact re-scan)";
  d.ws2.done = e2;
  d.ready = true;
  return kOk;
}

}  // namespace vdbg

using namespace vdbg;

extern "C" {

int vdbg_flat_search_device_noalloc(vdbg_dataset* ds, const float* queries, size_t nq,
                                    size_t k, const uint64_t* allow_words, uint32_t* out_ids,
                                    float* out_dists, void* stream) {
  if (ds == nullptr) return SetError(kInvalidArgument, "null dataset");
  if (nq > 0 && k > 0 && (queries == nullptr || out_ids == nullptr || out_dists == nullptr))
    return SetError(kInvalidArgument, "null pointer");
  if (nq > 0x7fffffffull) return SetError(kInvalidArgument, "too many queries");
  if (k > 240)
    return SetError(kInvalidArgument,
                    "vdbg_flat_search_device_noalloc: k must be at most 240 (larger k sorts "
                    "every row and needs allocated scratch: use vdbg_flat_search_device)");
  Ctx* c = ds->d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  if (c->device < 0 || c->device >= kNoAllocMaxDevices)
    return SetError(kNotSupported, "vdbg_flat_search_device_noalloc: device index too large");
  DeviceScratch& d = g_scratch[c->device];
  std::lock_guard<std::mutex> gd(d.mu);
  if (!d.ready) return SetError(kFailedPrecondition, "allocation-free scratch is not set up");
  VDBG_HIP(hipSetDevice(c->device));
  ScanSource* src = &ds->d.src;
  if (src->N >= 1024 && GemmSupported(src->pd) && src->Smax == 0)
    return SetError(kFailedPrecondition, "the dataset has no threshold sample");
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : c->stream;
  // no row compaction under a filter (it would need scratch sized by the rows): the scan
  // tests the filter words per row, with the same results
  return RunScan(c, src, queries, nq, k, allow_words, out_ids, out_dists, s, &d.ws, &d.ws2);
}

}  // extern "C"
