// vdbg_api.hip -- the C ABI (include/vdbg.h): contexts, resident datasets, profiling and
// the flat search entry points.
#include <cstring>
#include <new>
#include <string>

#include "vdbg_internal.h"

namespace vdbg {

namespace {
thread_local std::string g_error;
}

int SetError(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

int Workspace::reserve(size_t bytes) {
  if (bytes <= cap) return kOk;
  if (base != nullptr) {
    // Earlier launches may still read the old block.
    VDBG_HIP(hipDeviceSynchronize());
    VDBG_HIP(hipFree(base));
    base = nullptr;
    cap = 0;
  }
  size_t want = bytes + bytes / 4 + (1u << 20);
  VDBG_HIP(hipMalloc(&base, want));
  cap = want;
  used = 0;
  return kOk;
}

void Workspace::release() {
  if (base != nullptr) (void)hipFree(base);
  base = nullptr;
  cap = used = 0;
}

ProfScope::ProfScope(Ctx* c, const char* name, hipStream_t s) : c_(c), s_(s), on_(c->profiling) {
  if (!on_) return;
  e_.name = name;
  auto grab = [&]() {
    hipEvent_t ev;
    if (!c_->free_events.empty()) {
      ev = c_->free_events.back();
      c_->free_events.pop_back();
    } else if (hipEventCreate(&ev) != hipSuccess) {
      ev = nullptr;
    }
    return ev;
  };
  e_.start = grab();
  e_.stop = grab();
  if (e_.start == nullptr || e_.stop == nullptr) {
    on_ = false;
    return;
  }
  (void)hipEventRecord(e_.start, s_);
}

ProfScope::~ProfScope() {
  if (!on_) return;
  (void)hipEventRecord(e_.stop, s_);
  c_->pending.push_back(e_);
}

static void DrainProfile(Ctx* c) {
  for (auto& p : c->pending) {
    float ms = 0.f;
    if (hipEventSynchronize(p.stop) == hipSuccess &&
        hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
      auto& slot = c->prof[p.name];
      slot.first += ms;
      slot.second += 1;
    }
    c->free_events.push_back(p.start);
    c->free_events.push_back(p.stop);
  }
  c->pending.clear();
}

static int CheckDims(size_t dim, size_t pd) {
  if (dim == 0 || pd < dim || pd % 16 != 0)
    return SetError(kInvalidArgument, "padded_dim must be a multiple of 16 and >= dim > 0");
  return kOk;
}

static int CreateDataset(vdbg_ctx* ctx, const float* rows, bool rows_on_device, size_t n,
                         size_t dim, size_t pd, int metric, vdbg_dataset** out) {
  if (ctx == nullptr || out == nullptr) return SetError(kInvalidArgument, "null argument");
  VDBG_RETURN_IF_ERROR(CheckDims(dim, pd));
  if (metric < 0 || metric > 2) return SetError(kInvalidArgument, "unknown metric");
  if (n > 0xfffffffeull) return SetError(kInvalidArgument, "more rows than InternalId holds");
  if (n > 0 && rows == nullptr) return SetError(kInvalidArgument, "null rows");
  Ctx* c = &ctx->c;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  auto* ds = new (std::nothrow) vdbg_dataset;
  if (ds == nullptr) return SetError(kResourceExhausted, "out of host memory");
  Dataset& d = ds->d;
  d.ctx = c;
  d.n = n;
  d.dim = dim;
  d.pd = pd;
  d.metric = metric;
  const size_t bytes = n * pd * sizeof(float);
  if (n > 0) {
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&d.rows), bytes);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&d.norms), n * sizeof(float));
    if (e == hipSuccess)
      e = hipMemcpyAsync(d.rows, rows, bytes,
                         rows_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                         c->stream);
    if (e != hipSuccess) {
      (void)hipFree(d.rows);
      (void)hipFree(d.norms);
      delete ds;
      return SetError(e == hipErrorOutOfMemory ? kResourceExhausted : kInternal,
                      std::string("dataset upload: ") + hipGetErrorString(e));
    }
  }
  int rc = LaunchRowStats(c, c->stream, d.rows, n, pd, d.norms, &d.stats);
  if (rc != kOk) {
    (void)hipFree(d.rows);
    (void)hipFree(d.norms);
    delete ds;
    return rc;
  }
  *out = ds;
  return kOk;
}

}  // namespace vdbg

using namespace vdbg;

extern "C" {

int vdbg_version(void) { return (0 << 16) | 1; }

const char* vdbg_last_error(void) { return g_error.c_str(); }

int vdbg_ctx_create(int device, vdbg_ctx** out) {
  if (out == nullptr) return SetError(kInvalidArgument, "null out");
  int n = 0;
  VDBG_HIP(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return SetError(kInvalidArgument, "no such device");
  VDBG_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  VDBG_HIP(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return SetError(kFailedPrecondition,
                    std::string("vdbg is built for gfx950, device is ") + prop.gcnArchName);
  auto* ctx = new (std::nothrow) vdbg_ctx;
  if (ctx == nullptr) return SetError(kResourceExhausted, "out of host memory");
  ctx->c.device = device;
  hipError_t e = hipStreamCreateWithFlags(&ctx->c.stream, hipStreamNonBlocking);
  if (e == hipSuccess)
    e = hipHostMalloc(reinterpret_cast<void**>(&ctx->c.host_pinned), 4096, hipHostMallocDefault);
  if (e != hipSuccess) {
    if (ctx->c.stream) (void)hipStreamDestroy(ctx->c.stream);
    delete ctx;
    return SetError(kInternal, std::string("context: ") + hipGetErrorString(e));
  }
  *out = ctx;
  return kOk;
}

int vdbg_ctx_destroy(vdbg_ctx* ctx) {
  if (ctx == nullptr) return kOk;
  Ctx& c = ctx->c;
  (void)hipSetDevice(c.device);
  (void)hipStreamSynchronize(c.stream);
  DrainProfile(&c);
  for (auto ev : c.free_events) (void)hipEventDestroy(ev);
  c.ws.release();
  c.ws2.release();
  if (c.host_pinned) (void)hipHostFree(c.host_pinned);
  (void)hipStreamDestroy(c.stream);
  delete ctx;
  return kOk;
}

void* vdbg_ctx_stream(vdbg_ctx* ctx) { return ctx ? static_cast<void*>(ctx->c.stream) : nullptr; }

int vdbg_ctx_synchronize(vdbg_ctx* ctx) {
  if (ctx == nullptr) return SetError(kInvalidArgument, "null ctx");
  VDBG_HIP(hipSetDevice(ctx->c.device));
  VDBG_HIP(hipStreamSynchronize(ctx->c.stream));
  return kOk;
}

int vdbg_profile_enable(vdbg_ctx* ctx, int enable) {
  if (ctx == nullptr) return SetError(kInvalidArgument, "null ctx");
  std::lock_guard<std::recursive_mutex> g(ctx->c.mu);
  ctx->c.profiling = enable != 0;
  return kOk;
}

int vdbg_profile_reset(vdbg_ctx* ctx) {
  if (ctx == nullptr) return SetError(kInvalidArgument, "null ctx");
  std::lock_guard<std::recursive_mutex> g(ctx->c.mu);
  VDBG_HIP(hipSetDevice(ctx->c.device));
  DrainProfile(&ctx->c);
  ctx->c.prof.clear();
  return kOk;
}

int vdbg_profile_get(vdbg_ctx* ctx, const char* name, double* total_ms, uint64_t* launches) {
  if (ctx == nullptr || name == nullptr) return SetError(kInvalidArgument, "null argument");
  std::lock_guard<std::recursive_mutex> g(ctx->c.mu);
  VDBG_HIP(hipSetDevice(ctx->c.device));
  DrainProfile(&ctx->c);
  auto it = ctx->c.prof.find(name);
  if (total_ms) *total_ms = it == ctx->c.prof.end() ? 0.0 : it->second.first;
  if (launches) *launches = it == ctx->c.prof.end() ? 0 : it->second.second;
  return kOk;
}

int vdbg_dataset_create(vdbg_ctx* ctx, const float* rows, size_t n, size_t dim,
                        size_t padded_dim, int metric, vdbg_dataset** out) {
  return CreateDataset(ctx, rows, false, n, dim, padded_dim, metric, out);
}

int vdbg_dataset_create_device(vdbg_ctx* ctx, const float* rows_dev, size_t n, size_t dim,
                               size_t padded_dim, int metric, vdbg_dataset** out) {
  return CreateDataset(ctx, rows_dev, true, n, dim, padded_dim, metric, out);
}

int vdbg_dataset_destroy(vdbg_dataset* ds) {
  if (ds == nullptr) return kOk;
  Ctx* c = ds->d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  (void)hipSetDevice(c->device);
  (void)hipDeviceSynchronize();
  (void)hipFree(ds->d.rows);
  (void)hipFree(ds->d.norms);
  delete ds;
  return kOk;
}

const float* vdbg_dataset_rows(vdbg_dataset* ds) { return ds ? ds->d.rows : nullptr; }

int vdbg_flat_search_device(vdbg_dataset* ds, const float* queries, size_t nq, size_t k,
                            const uint64_t* allow_words, uint32_t* out_ids, float* out_dists,
                            void* stream) {
  if (ds == nullptr) return SetError(kInvalidArgument, "null dataset");
  if (nq > 0 && k > 0 && (queries == nullptr || out_ids == nullptr || out_dists == nullptr))
    return SetError(kInvalidArgument, "null pointer");
  if (nq > 0x7fffffffull) return SetError(kInvalidArgument, "too many queries");
  Ctx* c = ds->d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : c->stream;
  return FlatSearch(&ds->d, queries, nq, k, allow_words, out_ids, out_dists, s);
}

int vdbg_flat_search_host(vdbg_dataset* ds, const float* queries, size_t nq, size_t k,
                          const uint64_t* allow_words, uint32_t* out_ids, float* out_dists,
                          uint64_t* dist_comps) {
  if (ds == nullptr) return SetError(kInvalidArgument, "null dataset");
  if (nq == 0 || k == 0) {
    if (dist_comps) *dist_comps = 0;
    return kOk;
  }
  if (queries == nullptr || out_ids == nullptr || out_dists == nullptr)
    return SetError(kInvalidArgument, "null pointer");
  Ctx* c = ds->d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  const size_t pd = ds->d.pd;
  const size_t words = (ds->d.n + 63) / 64;
  float* dq = nullptr;
  uint64_t* dm = nullptr;
  uint32_t* di = nullptr;
  float* dd = nullptr;
  auto cleanup = [&]() {
    (void)hipFreeAsync(dq, s);
    (void)hipFreeAsync(dm, s);
    (void)hipFreeAsync(di, s);
    (void)hipFreeAsync(dd, s);
  };
  hipError_t e = hipMallocAsync(reinterpret_cast<void**>(&dq), nq * pd * sizeof(float), s);
  if (e == hipSuccess && allow_words)
    e = hipMallocAsync(reinterpret_cast<void**>(&dm), words * sizeof(uint64_t) + 8, s);
  if (e == hipSuccess) e = hipMallocAsync(reinterpret_cast<void**>(&di), nq * k * 4, s);
  if (e == hipSuccess) e = hipMallocAsync(reinterpret_cast<void**>(&dd), nq * k * 4, s);
  if (e == hipSuccess)
    e = hipMemcpyAsync(dq, queries, nq * pd * sizeof(float), hipMemcpyHostToDevice, s);
  if (e == hipSuccess && allow_words)
    e = hipMemcpyAsync(dm, allow_words, words * sizeof(uint64_t), hipMemcpyHostToDevice, s);
  if (e != hipSuccess) {
    cleanup();
    return SetError(e == hipErrorOutOfMemory ? kResourceExhausted : kInternal,
                    std::string("flat search staging: ") + hipGetErrorString(e));
  }
  int rc = FlatSearch(&ds->d, dq, nq, k, allow_words ? dm : nullptr, di, dd, s);
  if (rc == kOk) {
    e = hipMemcpyAsync(out_ids, di, nq * k * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipMemcpyAsync(out_dists, dd, nq * k * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) rc = SetError(kInternal, std::string("flat search: ") + hipGetErrorString(e));
  }
  cleanup();
  if (rc == kOk && dist_comps) *dist_comps = uint64_t(nq) * ds->d.n;
  return rc;
}

int vdbg_last_fallbacks(vdbg_ctx* ctx, uint64_t* fallback_queries) {
  if (ctx == nullptr || fallback_queries == nullptr)
    return SetError(kInvalidArgument, "null argument");
  *fallback_queries = ctx->c.last_fallbacks;
  return kOk;
}

}  // extern "C"
