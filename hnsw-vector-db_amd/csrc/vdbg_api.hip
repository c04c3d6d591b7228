// vdbg_api.hip -- the C ABI (include/vdbg.h): contexts, resident datasets, profiling and
// the flat search entry points.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "gemm.h"
#include "hnsw_host.h"
#include "vdbg_device.h"
#include "vdbg_internal.h"

namespace vdbg {

namespace {
thread_local std::string g_error;
}

int SetError(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

__global__ void k_publish_words(const uint32_t* __restrict__ src, int n, uint32_t* dst,
                                uint32_t seq) {
  const int i = threadIdx.x;
  if (i < n) dst[1 + i] = src[i];
  __threadfence_system();
  __syncthreads();
  if (i == 0) __hip_atomic_store(dst, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

uint32_t NextFlagSeq(Ctx* c) { return ++c->flag_seq == 0 ? ++c->flag_seq : c->flag_seq; }

int ReadWords(Ctx* c, const uint32_t* dev, int n, hipStream_t s, uint32_t* out) {
  if (n <= 0 || n > 64) return SetError(kInternal, "ReadWords: 1..64 words");
  std::lock_guard<std::mutex> g(c->flag_mu);
  const uint32_t seq = NextFlagSeq(c);
  k_publish_words<<<1, 64, 0, s>>>(dev, n, c->host_flag_dev, seq);
  VDBG_HIP(hipGetLastError());
  VDBG_RETURN_IF_ERROR(WaitWords(c, seq, dev, n, s));
  for (int i = 0; i < n; ++i) out[i] = c->host_pinned[i];
  return kOk;
}

int WaitWords(Ctx* c, uint32_t seq, const uint32_t* dev, int n, hipStream_t s) {
  volatile uint32_t* f = c->host_flag;
  for (uint32_t spin = 0;; ++spin) {
    if (__atomic_load_n(&c->host_flag[0], __ATOMIC_ACQUIRE) == seq) {
      for (int i = 0; i < n; ++i) c->host_pinned[i] = f[1 + i];
      return kOk;
    }
    if ((spin & 1023u) == 1023u) {  // every ~1k polls: has the stream ended or failed?
      const hipError_t q = hipStreamQuery(s);
      if (q != hipErrorNotReady) {
        VDBG_HIP(q);
        if (__atomic_load_n(&c->host_flag[0], __ATOMIC_ACQUIRE) != seq) {
          // the stream is done but the number did not show: copy the words the slow way
          VDBG_HIP(hipMemcpy(c->host_pinned, dev, size_t(n) * 4, hipMemcpyDeviceToHost));
          return kOk;
        }
      }
    }
    __builtin_ia32_pause();
  }
}

// ------------------------------------------------------------ host staging

// Inputs: the device reads the mapped pinned block (16-byte vectors, grid-strided).
__global__ void k_stage_in(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n16) {
  const size_t step = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += step)
    dst[i] = src[i];
}

// Results: every block writes its share into the mapped pinned block and fences at system
// scope; the last block to finish (a device counter, reset by that block) raises the flag.
struct StageOutArgs {
  const uint4* src[3];
  uint4* dst[3];
  size_t n16[3];
  int n;
  uint32_t* counter;
  uint32_t* flag;
  uint32_t seq;
};

__global__ void k_stage_out(StageOutArgs a) {
  const size_t step = size_t(gridDim.x) * blockDim.x;
  for (int r = 0; r < a.n; ++r)
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < a.n16[r]; i += step)
      a.dst[r][i] = a.src[r][i];
  __threadfence_system();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t before =
        __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (before == gridDim.x - 1) {
      __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __threadfence_system();
      __hip_atomic_store(a.flag, a.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

// Grows the pinned block to `host` bytes and the device block to kStageAlign + `dev` bytes.
// An outgrown pinned block stays allocated until the context ends (a kernel may have read
// it); an outgrown device block is freed once the stream has drained.
static int StageReserve(Ctx* c, size_t host, size_t dev, hipStream_t s) {
  if (host > c->stage_h_cap) {
    const size_t want = std::max<size_t>(host + host / 2, size_t(1) << 20);
    uint8_t* h = nullptr;
    uint8_t* hd = nullptr;
    hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&h), want,
                                 hipHostMallocMapped | hipHostMallocCoherent);
    if (e == hipSuccess) e = hipHostGetDevicePointer(reinterpret_cast<void**>(&hd), h, 0);
    if (e != hipSuccess) {
      if (h != nullptr) (void)hipHostFree(h);
      return SetError(e == hipErrorOutOfMemory ? kResourceExhausted : kInternal,
                      std::string("staging (host): ") + hipGetErrorString(e));
    }
    if (c->stage_h != nullptr) c->stage_h_retired.push_back(c->stage_h);
    c->stage_h = h;
    c->stage_h_dev = hd;
    c->stage_h_cap = want;
  }
  if (kStageAlign + dev > c->stage_d_cap) {
    const size_t want = kStageAlign + std::max<size_t>(dev + dev / 2, size_t(1) << 20);
    if (c->stage_d != nullptr) {
      VDBG_HIP(hipStreamSynchronize(s));
      VDBG_HIP(hipFree(c->stage_d));
      c->stage_d = nullptr;
      c->stage_d_cap = 0;
    }
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&c->stage_d), want);
    if (e == hipSuccess) e = hipMemset(c->stage_d, 0, kStageAlign);  // the completion counter
    if (e != hipSuccess) {
      if (c->stage_d != nullptr) (void)hipFree(c->stage_d);
      c->stage_d = nullptr;
      return SetError(e == hipErrorOutOfMemory ? kResourceExhausted : kInternal,
                      std::string("staging (device): ") + hipGetErrorString(e));
    }
    c->stage_d_cap = want;
  }
  return kOk;
}

int StageIn(Ctx* c, const void* const* src, const size_t* bytes, int nin, size_t out,
            hipStream_t s, uint8_t** dev) {
  size_t in = 0;
  for (int i = 0; i < nin; ++i) in += StageSpan(bytes[i]);
  VDBG_RETURN_IF_ERROR(StageReserve(c, std::max(in, out), in + out, s));
  uint8_t* h = c->stage_h;
  for (int i = 0; i < nin; ++i) {
    if (bytes[i] > 0) std::memcpy(h, src[i], bytes[i]);
    std::memset(h + bytes[i], 0, StageSpan(bytes[i]) - bytes[i]);
    h += StageSpan(bytes[i]);
  }
  uint8_t* base = c->stage_d + kStageAlign;
  const size_t n16 = in / 16;
  const unsigned blocks = unsigned(std::min<size_t>(256, (n16 + 255) / 256));
  k_stage_in<<<blocks, 256, 0, s>>>(reinterpret_cast<const uint4*>(c->stage_h_dev),
                                    reinterpret_cast<uint4*>(base), n16);
  VDBG_HIP(hipGetLastError());
  *dev = base;
  return kOk;
}

int StageOut(Ctx* c, const uint8_t* const* src, const size_t* bytes, void* const* dst, int nout,
             hipStream_t s) {
  if (nout < 1 || nout > 3) return SetError(kInternal, "StageOut: 1 to 3 regions");
  // the results land at the start of the pinned block (the inputs there have been read: the
  // copy-in kernel ran before everything queued after it)
  StageOutArgs a{};
  a.n = nout;
  size_t off = 0, total16 = 0;
  for (int r = 0; r < nout; ++r) {
    a.src[r] = reinterpret_cast<const uint4*>(src[r]);
    a.dst[r] = reinterpret_cast<uint4*>(c->stage_h_dev + off);
    a.n16[r] = (bytes[r] + 15) / 16;
    total16 += a.n16[r];
    off += StageRound(bytes[r]);
  }
  VDBG_RETURN_IF_ERROR(StageReserve(c, off, 0, s));  // (reserved by StageIn already)
  a.counter = reinterpret_cast<uint32_t*>(c->stage_d);
  std::lock_guard<std::mutex> g(c->flag_mu);
  a.flag = c->host_flag_dev;
  a.seq = NextFlagSeq(c);
  const unsigned blocks = unsigned(std::max<size_t>(1, std::min<size_t>(64, (total16 + 255) / 256)));
  k_stage_out<<<blocks, 256, 0, s>>>(a);
  VDBG_HIP(hipGetLastError());
  bool seen = false;
  for (uint32_t spin = 0; !seen; ++spin) {
    if (__atomic_load_n(&c->host_flag[0], __ATOMIC_ACQUIRE) == a.seq) {
      seen = true;
      break;
    }
    if ((spin & 1023u) == 1023u) {  // has the stream ended or failed?
      const hipError_t q = hipStreamQuery(s);
      if (q != hipErrorNotReady) {
        VDBG_HIP(q);
        if (__atomic_load_n(&c->host_flag[0], __ATOMIC_ACQUIRE) == a.seq) {
          seen = true;
          break;
        }
        // the stream is done but the flag did not show: copy the results the slow way
        for (int r = 0; r < nout; ++r)
          VDBG_HIP(hipMemcpy(dst[r], src[r], bytes[r], hipMemcpyDeviceToHost));
        return kOk;
      }
    }
    __builtin_ia32_pause();
  }
  off = 0;
  for (int r = 0; r < nout; ++r) {
    std::memcpy(dst[r], c->stage_h + off, bytes[r]);
    off += StageRound(bytes[r]);
  }
  return kOk;
}

int Workspace::reserve(size_t bytes) {
  if (bytes <= cap) return kOk;
  if (fixed)
    return SetError(kResourceExhausted,
                    std::string(name) + ": the call needs " + std::to_string(bytes) +
                        " bytes of scratch, more than the " + std::to_string(cap) +
                        " this path holds");
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
  if (base != nullptr && !fixed) (void)hipFree(base);
  if (done != nullptr) (void)hipEventDestroy(done);
  done = nullptr;
  last = nullptr;
  used_once = false;
  base = nullptr;
  cap = used = 0;
}

WsUse::WsUse(Workspace* w, hipStream_t s) : w_(w), s_(s) {
  if (w_->done == nullptr &&
      hipEventCreateWithFlags(&w_->done, hipEventDisableTiming) != hipSuccess) {
    w_->done = nullptr;
    rc_ = SetError(kInternal, "workspace event");
    return;
  }
  // the previous user's launches on this same stream are ordered by the stream itself
  if (!(w_->used_once && w_->last == s_) && hipStreamWaitEvent(s_, w_->done, 0) != hipSuccess)
    rc_ = SetError(kInternal, "workspace event wait");
}

WsUse::~WsUse() {
  if (w_->done != nullptr && hipEventRecord(w_->done, s_) == hipSuccess) {
    w_->last = s_;
    w_->used_once = true;
  }
}

// External ids of appended rows given none: each row's own row number.
__global__ void k_iota64(uint64_t* __restrict__ p, uint64_t first, size_t n) {
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = first + i;
}

__global__ void k_fill32(uint32_t* __restrict__ p, uint32_t v, size_t n) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i < n) p[i] = v;
}

int Fill32(void* p, uint32_t v, size_t n, hipStream_t s) {
  if (n == 0) return kOk;
  k_fill32<<<dim3(unsigned((n + 255) / 256)), 256, 0, s>>>(static_cast<uint32_t*>(p), v, n);
  VDBG_HIP(hipGetLastError());
  return kOk;
}

ProfScope::ProfScope(Ctx* c, const char* name, hipStream_t s) : c_(c), s_(s), on_(c->profiling) {
  if (!on_) return;
  e_.name = name;
  std::lock_guard<std::mutex> g(c_->prof_mu);
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
  std::lock_guard<std::mutex> g(c_->prof_mu);
  c_->pending.push_back(e_);
}

static void DrainProfile(Ctx* c) {
  std::lock_guard<std::mutex> g(c->prof_mu);
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
    // device rows may still be in production on any stream of the caller: wait for the
    // whole device before copying (the copy has completed when this call returns)
    if (e == hipSuccess && rows_on_device) e = hipDeviceSynchronize();
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
  if (n > 0) {
    if (c->fp16_gemm)
      rc = MakeRows16(c, c->stream, d.rows, n, pd, &d.rows16_parts, &d.rows16_exp,
                      &d.rows16_approx, d.stats, &d.rows16);
    if (rc != kOk) {
      (void)hipFree(d.rows);
      (void)hipFree(d.norms);
      delete ds;
      return rc;
    }
  }
  // (float rows ranking on the fp16 h halves need no int8 copy)
  if (n > 0 && c->fp16_gemm && c->int8_gemm && d.rows16 != nullptr && !d.rows16_approx) {
    if (d.rows16_parts == 1) {
      rc = MakeRows8(c, c->stream, d.rows, n, pd, metric, d.stats, &d.rows8, &d.init8, &d.c8);
    } else {
      rc = MakeRows8Split(c, c->stream, d.rows, n, pd, d.stats, &d.rows8, &d.rows8_exp,
                          &d.rows8_l1max, &d.rows8_l2max);
      d.rows8_parts = 2;
    }
    if (rc != kOk) {
      (void)hipFree(d.rows16);
      (void)hipFree(d.rows);
      (void)hipFree(d.norms);
      delete ds;
      return rc;
    }
  }
  d.src.kind = 0;
  d.src.X = d.rows;
  d.src.X16 = d.rows16;
  d.src.X8 = d.rows8;
  d.src.init8 = d.init8;
  d.src.c8 = d.c8;
  d.src.x8_parts = d.rows8_parts;
  d.src.x8_exp = d.rows8_exp;
  d.src.x8_l1max = d.rows8_l1max;
  d.src.x8_l2max = d.rows8_l2max;
  d.src.x16_parts = d.rows16_parts;
  d.src.x16_exp = d.rows16_exp;
  d.src.x16_approx = d.rows16_approx;
  d.src.rn = d.norms;
  d.src.N = static_cast<uint32_t>(n);
  d.src.pd = static_cast<int>(pd);
  d.src.metric = metric;
  d.src.rmag = d.stats.xn_max;
  d.src.stats = d.stats;
  // The threshold sample of the GEMM path is gathered now, so that no search allocates it
  // (the allocation-free flat search relies on this).
  if (n >= 1024 && GemmSupported(pd)) {
    rc = BuildSample(c, &d.src, c->stream);
    if (rc == kOk && hipStreamSynchronize(c->stream) != hipSuccess)
      rc = SetError(kInternal, "dataset sample");
    if (rc != kOk) {
      FreeSample(&d.src);
      (void)hipFree(d.rows8);
      (void)hipFree(d.init8);
      (void)hipFree(d.rows16);
      (void)hipFree(d.rows);
      (void)hipFree(d.norms);
      delete ds;
      return rc;
    }
  }
  ++c->live_datasets;
  *out = ds;
  return kOk;
}

// The SQ8 search: top max(depth, k) by the SQ8 distance, then (depth > 0) Rerank with the
// fp32 rows to k, as HnswSq8Index::search does with its beam
// (src/index/hnsw/hnsw_index.cc:82-100).
static int Sq8Search(Sq8Index* x, const float* Q, size_t nq, size_t k, size_t depth,
                     const uint64_t* allow, uint32_t* out_ids, float* out_d, hipStream_t s) {
  Ctx* c = x->ds->ctx;
  if (nq == 0 || k == 0) return kOk;
  if (depth == 0) return ScanMasked(c, &x->src, Q, nq, k, allow, out_ids, out_d, s);
  const size_t kk = std::max(depth, k);
  uint32_t* ti = nullptr;
  float* td = nullptr;
  hipError_t e = hipMallocAsync(reinterpret_cast<void**>(&ti), nq * kk * 4, s);
  if (e == hipSuccess) e = hipMallocAsync(reinterpret_cast<void**>(&td), nq * kk * 4, s);
  if (e != hipSuccess) {
    (void)hipFreeAsync(ti, s);
    return SetError(kResourceExhausted, std::string("sq8 search: ") + hipGetErrorString(e));
  }
  int rc = ScanMasked(c, &x->src, Q, nq, kk, allow, ti, td, s);
  if (rc == kOk)
    rc = Rerank(c, x->ds->rows, int(x->ds->pd), x->ds->metric, Q, nq, ti, kk, k, out_ids, out_d,
                s, &x->ds->src);
  (void)hipFreeAsync(ti, s);
  (void)hipFreeAsync(td, s);
  return rc;
}

__global__ void k_check_cand(const uint32_t* __restrict__ cand, size_t n, uint32_t rows,
                             int* __restrict__ bad) {
  const size_t t = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (t < n && cand[t] != kNoId && cand[t] >= rows) *bad = 1;
}

__global__ void k_count_cand(const uint32_t* __restrict__ cand, size_t nq, size_t depth,
                             uint64_t* __restrict__ dc) {
  const size_t q = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (q >= nq) return;
  uint64_t n = 0;
  for (size_t i = 0; i < depth; ++i) n += cand[q * depth + i] != kNoId ? 1 : 0;
  dc[q] = n;
}

// Rerank (src/index/index.cc:89-95) on a batch: candidates [nq][depth] (UINT32_MAX = none),
// rows checked against the dataset first; dist_comps[q] = the query's candidate count.
__global__ void k_pad_results(uint32_t* ids, float* d, size_t n) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i < n) {
    ids[i] = kNoId;
    d[i] = __builtin_inff();
  }
}

static int RerankChecked(Ctx* c, Dataset* d, const float* Q, size_t nq, const uint32_t* cand,
                         size_t depth, size_t k, uint32_t* out_ids, float* out_d,
                         uint64_t* dist_comps, hipStream_t s, bool host_checked = false) {
  if (depth > 0 && !host_checked) {
    int* bad = nullptr;
    VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&bad), sizeof(int), s));
    VDBG_HIP(hipMemsetAsync(bad, 0, sizeof(int), s));
    k_check_cand<<<dim3(unsigned((nq * depth + 255) / 256)), 256, 0, s>>>(cand, nq * depth,
                                                                         uint32_t(d->n), bad);
    VDBG_HIP(hipGetLastError());
    VDBG_HIP(hipMemcpyAsync(c->host_pinned, bad, sizeof(int), hipMemcpyDeviceToHost, s));
    VDBG_HIP(hipStreamSynchronize(s));
    (void)hipFreeAsync(bad, s);
    if (c->host_pinned[0] != 0) return SetError(kInvalidArgument, "candidate row out of range");
  }
  if (depth == 0) {
    k_pad_results<<<dim3(unsigned((nq * k + 255) / 256)), 256, 0, s>>>(out_ids, out_d, nq * k);
    VDBG_HIP(hipGetLastError());
  } else {
    VDBG_RETURN_IF_ERROR(Rerank(c, d->rows, int(d->pd), d->metric, Q, nq, cand, depth, k,
                                out_ids, out_d, s, &d->src));
  }
  if (dist_comps != nullptr) {
    if (depth == 0) {
      VDBG_HIP(hipMemsetAsync(dist_comps, 0, nq * 8, s));
    } else {
      k_count_cand<<<dim3(unsigned((nq + 255) / 256)), 256, 0, s>>>(cand, nq, depth, dist_comps);
      VDBG_HIP(hipGetLastError());
    }
  }
  return kOk;
}

}  // namespace vdbg

using namespace vdbg;

extern "C" {

int vdbg_version(void) { return (0 << 16) | 1; }

const char* vdbg_last_error(void) { return g_error.c_str(); }

static const char* const kKsetNames[] = {"scalar", "avx2", "avx512"};

static int BestHostKset() { return vdbg::BestHostKernelSet(); }

static int KsetByName(const char* name) {
  for (int i = 0; i < 3; ++i)
    if (std::strcmp(name, kKsetNames[i]) == 0) return i <= BestHostKset() ? i : -1;
  return -1;
}

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
  VDBG_RETURN_IF_ERROR(InitNoAllocScratch(device));
  auto* ctx = new (std::nothrow) vdbg_ctx;
  if (ctx == nullptr) return SetError(kResourceExhausted, "out of host memory");
  ctx->c.device = device;
  ctx->c.cu_count = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
  ctx->c.handle = ctx;
  // Kernels() (cpu_features.cc:27-34): VDB_KERNELS when it names an available set, else the
  // best set of this CPU, so distances match a vdb process on the same host.
  ctx->c.kset = BestHostKset();
  if (const char* env = std::getenv("VDB_KERNELS"); env != nullptr && *env != '\0') {
    const int k = KsetByName(env);
    if (k >= 0) ctx->c.kset = k;
  }
  hipError_t e = hipStreamCreateWithFlags(&ctx->c.stream, hipStreamNonBlocking);
  if (e == hipSuccess)
    e = hipHostMalloc(reinterpret_cast<void**>(&ctx->c.host_pinned), 4096, hipHostMallocDefault);
  if (e == hipSuccess)
    e = hipHostMalloc(reinterpret_cast<void**>(&ctx->c.host_flag), 4096,
                      hipHostMallocMapped | hipHostMallocCoherent);
  if (e == hipSuccess) {
    ctx->c.host_flag[0] = 0;
    e = hipHostGetDevicePointer(reinterpret_cast<void**>(&ctx->c.host_flag_dev), ctx->c.host_flag, 0);
  }
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&ctx->c.fb_dev), 256);
  if (e == hipSuccess) e = hipMemset(ctx->c.fb_dev, 0, 256);
  if (e != hipSuccess) {
    if (ctx->c.fb_dev) (void)hipFree(ctx->c.fb_dev);
    if (ctx->c.host_flag) (void)hipHostFree(ctx->c.host_flag);
    if (ctx->c.host_pinned) (void)hipHostFree(ctx->c.host_pinned);
    if (ctx->c.stream) (void)hipStreamDestroy(ctx->c.stream);
    delete ctx;
    return SetError(kInternal, std::string("context: ") + hipGetErrorString(e));
  }
  *out = ctx;
  return kOk;
}

int vdbg_ctx_set_kernels(vdbg_ctx* ctx, const char* name) {
  if (ctx == nullptr || name == nullptr) return SetError(kInvalidArgument, "null argument");
  const int k = KsetByName(name);
  if (k < 0) return SetError(kInvalidArgument, std::string("unknown or unavailable kernel set ") + name);
  std::lock_guard<std::recursive_mutex> g(ctx->c.mu);
  ctx->c.kset = k;
  return kOk;
}

const char* vdbg_ctx_kernels(vdbg_ctx* ctx) {
  return ctx == nullptr ? "" : kKsetNames[ctx->c.kset];
}

int vdbg_ctx_set_fp16_gemm(vdbg_ctx* ctx, int enable) {
  if (ctx == nullptr) return SetError(kInvalidArgument, "null ctx");
  std::lock_guard<std::recursive_mutex> g(ctx->c.mu);
  ctx->c.fp16_gemm = enable != 0;
  return kOk;
}

int vdbg_ctx_set_int8_gemm(vdbg_ctx* ctx, int enable) {
  if (ctx == nullptr) return SetError(kInvalidArgument, "null ctx");
  std::lock_guard<std::recursive_mutex> g(ctx->c.mu);
  ctx->c.int8_gemm = enable != 0;
  return kOk;
}

int vdbg_ctx_set_ivf_row_sums(vdbg_ctx* ctx, int enable) {
  if (ctx == nullptr) return SetError(kInvalidArgument, "null ctx");
  std::lock_guard<std::recursive_mutex> g(ctx->c.mu);
  ctx->c.ivf_row_sums = enable != 0;
  return kOk;
}

int vdbg_ctx_set_int8_float_min_work(vdbg_ctx* ctx, double work) {
  if (ctx == nullptr) return SetError(kInvalidArgument, "null ctx");
  if (!(work >= 0.0)) return SetError(kInvalidArgument, "work must be >= 0");
  std::lock_guard<std::recursive_mutex> g(ctx->c.mu);
  ctx->c.int8_float_min_work = work;
  return kOk;
}

int vdbg_ctx_set_host_threads(vdbg_ctx* ctx, int n) {
  if (ctx == nullptr) return SetError(kInvalidArgument, "null ctx");
  std::lock_guard<std::recursive_mutex> g(ctx->c.mu);
  ctx->c.host_threads = n > 0 ? n : 0;
  return kOk;
}

int vdbg_ctx_set_fp16_single(vdbg_ctx* ctx, int enable) {
  if (ctx == nullptr) return SetError(kInvalidArgument, "null ctx");
  std::lock_guard<std::recursive_mutex> g(ctx->c.mu);
  ctx->c.fp16_single = enable != 0;
  return kOk;
}

int vdbg_ctx_set_collection_schedule(vdbg_ctx* ctx, int combine, int lanes, int threaded) {
  if (ctx == nullptr) return SetError(kInvalidArgument, "null ctx");
  if (lanes < 0 || lanes > 16) return SetError(kInvalidArgument, "lanes must be in 0..16");
  std::lock_guard<std::recursive_mutex> g(ctx->c.mu);
  ctx->c.combine_segments = combine != 0;
  ctx->c.collection_lanes = lanes;
  ctx->c.lane_threads = threaded != 0;
  return kOk;
}

int vdbg_ctx_set_gated_fallbacks(vdbg_ctx* ctx, int enable) {
  if (ctx == nullptr) return SetError(kInvalidArgument, "null ctx");
  std::lock_guard<std::recursive_mutex> g(ctx->c.mu);
  ctx->c.gate_fallbacks = enable != 0;
  return kOk;
}

int vdbg_ctx_set_test_fallbacks(vdbg_ctx* ctx, int level) {
  if (ctx == nullptr) return SetError(kInvalidArgument, "null ctx");
  if (level < 0 || level > 2) return SetError(kInvalidArgument, "level must be 0, 1 or 2");
  std::lock_guard<std::recursive_mutex> g(ctx->c.mu);
  ctx->c.test_fallbacks = level;
  return kOk;
}

int vdbg_ctx_destroy(vdbg_ctx* ctx) {
  if (ctx == nullptr) return kOk;
  Ctx& c = ctx->c;
  {
    std::lock_guard<std::recursive_mutex> g(c.mu);
    if (c.live_datasets > 0)
      return SetError(kInvalidArgument, "context still has datasets: destroy them first");
  }
  (void)hipSetDevice(c.device);
  (void)hipStreamSynchronize(c.stream);
  DrainProfile(&c);
  for (auto ev : c.free_events) (void)hipEventDestroy(ev);
  for (ScanScratch* l : c.lanes) {
    (void)hipStreamSynchronize(l->stream);
    delete l;
  }
  c.lanes.clear();
  c.ws.release();
  c.ws2.release();
  c.wsc.release();
  c.wcomb.release();
  if (c.wcomb_done) (void)hipEventDestroy(c.wcomb_done);
  if (c.wsc_done) (void)hipEventDestroy(c.wsc_done);
  if (c.host_pinned) (void)hipHostFree(c.host_pinned);
  if (c.stage_h) (void)hipHostFree(c.stage_h);
  for (uint8_t* h : c.stage_h_retired) (void)hipHostFree(h);
  if (c.stage_d) (void)hipFree(c.stage_d);
  if (c.fb_dev) (void)hipFree(c.fb_dev);
  if (c.host_flag) (void)hipHostFree(c.host_flag);
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

int vdbg_dataset_open_vectors(vdbg_ctx* ctx, const void* file, size_t len, size_t dim,
                              int metric, uint64_t rows, int verify_crc, vdbg_dataset** out) {
  if (ctx == nullptr || out == nullptr || (file == nullptr && len > 0))
    return SetError(kInvalidArgument, "null argument");
  if (dim == 0) return SetError(kInvalidArgument, "dim must be > 0");
  if (metric < 0 || metric > 2) return SetError(kInvalidArgument, "unknown metric");
  const float* data = nullptr;
  uint64_t n = 0;
  VDBG_RETURN_IF_ERROR(CheckSegmentVectors(file, len, dim, metric, rows, verify_crc, &data, &n));
  return CreateDataset(ctx, data, false, size_t(n), dim, (dim + 15) / 16 * 16, metric, out);
}

int vdbg_dataset_create_device(vdbg_ctx* ctx, const float* rows_dev, size_t n, size_t dim,
                               size_t padded_dim, int metric, vdbg_dataset** out) {
  return CreateDataset(ctx, rows_dev, true, n, dim, padded_dim, metric, out);
}

// MutableSegment (src/engine/mutable_segment.cc:10-40): an empty dataset whose rows arrive
// by vdbg_dataset_append.  Capacity is reserved up front and doubles when exceeded.
int vdbg_dataset_create_appendable(vdbg_ctx* ctx, size_t dim, size_t pd, int metric,
                                   size_t capacity, vdbg_dataset** out) {
  if (ctx == nullptr || out == nullptr) return SetError(kInvalidArgument, "null argument");
  VDBG_RETURN_IF_ERROR(CheckDims(dim, pd));
  if (metric < 0 || metric > 2) return SetError(kInvalidArgument, "unknown metric");
  if (capacity > 0xfffffffeull) return SetError(kInvalidArgument, "more rows than InternalId holds");
  Ctx* c = &ctx->c;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  auto* ds = new (std::nothrow) vdbg_dataset;
  if (ds == nullptr) return SetError(kResourceExhausted, "out of host memory");
  Dataset& d = ds->d;
  d.ctx = c;
  d.n = 0;
  d.dim = dim;
  d.pd = pd;
  d.metric = metric;
  d.appendable = true;
  d.cap = std::max<size_t>(capacity, 1024);
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&d.rows), d.cap * pd * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&d.norms), d.cap * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&d.ext_ids), d.cap * 8);
  if (e != hipSuccess) {
    (void)hipFree(d.rows);
    (void)hipFree(d.norms);
    (void)hipFree(d.ext_ids);
    delete ds;
    return SetError(e == hipErrorOutOfMemory ? kResourceExhausted : kInternal,
                    std::string("appendable dataset: ") + hipGetErrorString(e));
  }
  d.src.kind = 0;
  d.src.X = d.rows;
  d.src.rn = d.norms;
  d.src.N = 0;
  d.src.pd = int(pd);
  d.src.metric = metric;
  ++c->live_datasets;
  *out = ds;
  return kOk;
}

// MutableSegment::Append (mutable_segment.cc:24-44) for n rows at once: the rows (n x pd,
// host), their external ids (host; null gives each new row its row number), published
// together when the call returns.  *first_row (nullable) receives the row number of the first.
// Only growth past the reserved capacity waits for the whole device (old buffers are freed
// once no search can read them); otherwise the call waits only for its own copies and the
// statistics of the new rows on the context's stream.
int vdbg_dataset_append(vdbg_dataset* ds, const float* rows, size_t n, const uint64_t* ext_ids,
                        uint64_t* first_row) {
  if (ds == nullptr || (n > 0 && rows == nullptr)) return SetError(kInvalidArgument, "null argument");
  Dataset& d = ds->d;
  Ctx* c = d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  if (!d.appendable)
    return SetError(kFailedPrecondition, "rows are appended only to a dataset made by "
                                         "vdbg_dataset_create_appendable");
  if (d.live_indexes > 0)
    return SetError(kFailedPrecondition, "an appendable dataset with an index takes no rows");
  if (d.n + n > 0xfffffffeull) return SetError(kResourceExhausted, "mutable segment is full");
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  if (first_row != nullptr) *first_row = d.n;
  if (n == 0) return kOk;
  if (d.n + n > d.cap) {  // grow: every search queued on any stream finishes first
    const size_t cap = std::max(2 * d.cap, d.n + n);
    float *nr = nullptr, *nn = nullptr;
    uint64_t* ne = nullptr;
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&nr), cap * d.pd * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&nn), cap * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&ne), cap * 8);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess && d.n > 0)
      e = hipMemcpyAsync(nr, d.rows, d.n * d.pd * sizeof(float), hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess && d.n > 0)
      e = hipMemcpyAsync(nn, d.norms, d.n * sizeof(float), hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess && d.n > 0)
      e = hipMemcpyAsync(ne, d.ext_ids, d.n * 8, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
      (void)hipFree(nr);
      (void)hipFree(nn);
      (void)hipFree(ne);
      return SetError(e == hipErrorOutOfMemory ? kResourceExhausted : kInternal,
                      std::string("append: ") + hipGetErrorString(e));
    }
    (void)hipFree(d.rows);
    (void)hipFree(d.norms);
    (void)hipFree(d.ext_ids);
    for (void* p : d.retired) (void)hipFree(p);
    d.retired.clear();
    d.rows = nr;
    d.norms = nn;
    d.ext_ids = ne;
    d.cap = cap;
  }
  float* at = d.rows + d.n * d.pd;
  VDBG_HIP(hipMemcpyAsync(at, rows, n * d.pd * sizeof(float), hipMemcpyHostToDevice, s));
  if (ext_ids != nullptr) {
    VDBG_HIP(hipMemcpyAsync(d.ext_ids + d.n, ext_ids, n * 8, hipMemcpyHostToDevice, s));
  } else {
    k_iota64<<<dim3(unsigned((n + 255) / 256)), 256, 0, s>>>(d.ext_ids + d.n, d.n, n);
    VDBG_HIP(hipGetLastError());
  }
  RowStats st;  // (reads the statistics back: the copies above have completed on return)
  VDBG_RETURN_IF_ERROR(LaunchRowStats(c, s, at, n, d.pd, d.norms + d.n, &st));
  if (d.n == 0) {
    d.stats = st;
  } else {
    d.stats.lo = std::min(d.stats.lo, st.lo);
    d.stats.hi = std::max(d.stats.hi, st.hi);
    d.stats.max_abs = std::max(d.stats.max_abs, st.max_abs);
    d.stats.xn_max = std::max(d.stats.xn_max, st.xn_max);
    d.stats.all_int = d.stats.all_int & st.all_int;
  }
  d.n += n;
  d.src.X = d.rows;
  d.src.rn = d.norms;
  d.src.N = uint32_t(d.n);
  d.src.stats = d.stats;
  d.src.rmag = d.stats.xn_max;
  // The threshold sample: any rows of the set give a valid threshold, and RunScan sizes its
  // rank by the rows the sample spans, so a sample that trails the rows stays correct; it is
  // gathered anew once the rows have doubled since (or reached 1024), which keeps the
  // refreshes logarithmic in the appends.  The replaced sample is kept until the device is
  // next idle, since searches queued earlier on any stream may still read it.
  if (d.n >= 1024 && GemmSupported(d.pd) &&
      (d.src.Smax == 0 || d.n >= 2 * size_t(d.src.SN))) {
    if (d.src.Sbuf != nullptr) {
      d.retired.push_back(d.src.Sbuf);
      d.src.Sbuf = nullptr;  // FreeSample then only forgets it
    }
    FreeSample(&d.src);
    VDBG_RETURN_IF_ERROR(BuildSample(c, &d.src, s));
    // searches on other streams read the new sample only after its gather has completed
    VDBG_HIP(hipStreamSynchronize(s));
  }
  return kOk;
}

int vdbg_dataset_size(vdbg_dataset* ds, uint64_t* rows) {
  if (ds == nullptr || rows == nullptr) return SetError(kInvalidArgument, "null argument");
  std::lock_guard<std::recursive_mutex> g(ds->d.ctx->mu);
  *rows = ds->d.n;
  return kOk;
}

int vdbg_dataset_destroy(vdbg_dataset* ds) {
  if (ds == nullptr) return kOk;
  Ctx* c = ds->d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  if (ds->d.live_indexes > 0)
    return SetError(kInvalidArgument, "dataset still has SQ8/IVF-PQ indexes: destroy them first");
  (void)hipSetDevice(c->device);
  (void)hipDeviceSynchronize();
  --c->live_datasets;
  FreeSample(&ds->d.src);
  for (void* p : ds->d.retired) (void)hipFree(p);
  (void)hipFree(ds->d.rows);
  (void)hipFree(ds->d.norms);
  if (ds->d.rows16 != nullptr) (void)hipFree(ds->d.rows16);
  if (ds->d.ext_ids != nullptr) (void)hipFree(ds->d.ext_ids);
  if (ds->d.rows8 != nullptr) (void)hipFree(ds->d.rows8);
  if (ds->d.init8 != nullptr) (void)hipFree(ds->d.init8);
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
  return ScanMasked(c, &ds->d.src, queries, nq, k, allow_words, out_ids, out_dists, s);
}

int vdbg_flat_search_host(vdbg_dataset* ds, const float* queries, size_t nq, size_t k,
                          const uint64_t* allow_words, uint32_t* out_ids, float* out_dists,
                          uint64_t* dist_comps) {
  if (ds == nullptr) return SetError(kInvalidArgument, "null dataset");
  if (dist_comps) *dist_comps = 0;
  if (nq == 0 || k == 0) return kOk;
  if (queries == nullptr || out_ids == nullptr || out_dists == nullptr)
    return SetError(kInvalidArgument, "null pointer");
  Ctx* c = ds->d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  Dataset* d = &ds->d;
  int rc = StageHost(c, d->n, d->pd, queries, nq, k, allow_words, out_ids, out_dists, nullptr,
                     [&](const float* dq, const uint64_t* dm, uint32_t* di, float* dd,
                         uint64_t*, hipStream_t s) {
                       return ScanMasked(c, &d->src, dq, nq, k, dm, di, dd, s);
                     });
  if (rc == kOk && dist_comps) *dist_comps = uint64_t(nq) * d->n;
  return rc;
}

int vdbg_sq8_train(vdbg_dataset* ds, float* vmin_out, float* scale_out) {
  if (ds == nullptr || vmin_out == nullptr || scale_out == nullptr)
    return SetError(kInvalidArgument, "null argument");
  Ctx* c = ds->d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  const size_t pd = ds->d.pd;
  float* dv = nullptr;
  VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&dv), 2 * pd * sizeof(float), s));
  int rc = Sq8Train(c, &ds->d, dv, dv + pd, s);
  if (rc == kOk) {
    hipError_t e = hipMemcpyAsync(vmin_out, dv, pd * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipMemcpyAsync(scale_out, dv + pd, pd * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) rc = SetError(kInternal, std::string("sq8 train: ") + hipGetErrorString(e));
  }
  (void)hipFreeAsync(dv, s);
  return rc;
}

// vdbg_sq8_create (codes == nullptr: encode the rows) and vdbg_sq8_load (codes: an index
// file's n x pd code bytes on the host, uploaded as they are).
static int CreateSq8(vdbg_dataset* ds, const float* vmin, const float* scale,
                     const uint8_t* codes, vdbg_sq8** out) {
  Ctx* c = ds->d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  Dataset& d = ds->d;
  const size_t pd = d.pd, n = d.n;
  auto* h = new (std::nothrow) vdbg_sq8;
  if (h == nullptr) return SetError(kResourceExhausted, "out of host memory");
  Sq8Index& x = h->q;
  x.ds = &d;
  x.vmin_h.assign(vmin, vmin + pd);
  x.scale_h.assign(scale, scale + pd);
  auto fail = [&](int rc) {
    (void)hipFree(x.codes16);
    (void)hipFree(x.codes);
    (void)hipFree(x.yn);
    (void)hipFree(x.vmin);
    delete h;
    return rc;
  };
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&x.vmin), 2 * pd * sizeof(float));
  if (e == hipSuccess && n > 0) e = hipMalloc(reinterpret_cast<void**>(&x.codes), n * pd);
  if (e == hipSuccess && n > 0) e = hipMalloc(reinterpret_cast<void**>(&x.yn), n * sizeof(float));
  if (e != hipSuccess)
    return fail(SetError(e == hipErrorOutOfMemory ? kResourceExhausted : kInternal,
                         std::string("sq8 create: ") + hipGetErrorString(e)));
  x.scale = x.vmin + pd;
  e = hipMemcpyAsync(x.vmin, vmin, pd * 4, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipMemcpyAsync(x.scale, scale, pd * 4, hipMemcpyHostToDevice, s);
  if (e == hipSuccess && codes != nullptr && n > 0)
    e = hipMemcpyAsync(x.codes, codes, n * pd, hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return fail(SetError(kInternal, hipGetErrorString(e)));
  int rc = Sq8Encode(c, &d, x.vmin, x.scale, x.codes, x.yn, s, codes != nullptr);
  if (rc != kOk) return fail(rc);
  // magnitude term of the rounding bound: max ||code*scale||^2, a bound on the decoded
  // row norm, and ||vmin||^2
  std::vector<float> yn(n);
  if (n > 0) {
    e = hipMemcpyAsync(yn.data(), x.yn, n * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail(SetError(kInternal, hipGetErrorString(e)));
  }
  double ymax = 0, xhat = 0, vn = 0;
  for (float v : yn) ymax = std::max(ymax, double(v));
  for (size_t i = 0; i < pd; ++i) {
    const double a = std::fabs(double(vmin[i]));
    const double b = std::fabs(double(vmin[i]) + 255.0 * double(scale[i]));
    xhat += std::max(a, b) * std::max(a, b);
    vn += double(vmin[i]) * vmin[i];
  }
  x.src.kind = 1;
  x.src.C = x.codes;
  x.src.rn = x.yn;
  x.src.vmin = x.vmin;
  x.src.scale = x.scale;
  x.src.N = static_cast<uint32_t>(n);
  x.src.pd = static_cast<int>(pd);
  x.src.metric = d.metric;
  x.src.rmag = float(ymax + xhat + vn);
  x.src.rn_max = float(ymax);
  rc = MakeCodes16(c, s, x.codes, n, pd, &x.codes16);
  if (rc != kOk) return fail(rc);
  x.src.X16 = x.codes16;
  ++d.live_indexes;
  *out = h;
  return kOk;
}

int vdbg_sq8_create(vdbg_dataset* ds, const float* vmin, const float* scale, vdbg_sq8** out) {
  if (ds == nullptr || vmin == nullptr || scale == nullptr || out == nullptr)
    return SetError(kInvalidArgument, "null argument");
  return CreateSq8(ds, vmin, scale, nullptr, out);
}

// LoadIndex's framing check (src/index/index.cc:47-56) and HnswSq8Index::load
// (src/index/hnsw/hnsw_index.cc:117-129): u64 rows, the serialised Sq8Quantizer
// (src/index/quant/sq8.cc:43-63: u32 dim, u32 padded dim, vmin, scale), rows x padded_dim
// code bytes, then the graph (HnswGraph::Deserialize, hnsw_graph.h:368-413), kept on the host
// with a host copy of the codes for the walk.
int vdbg_sq8_load(vdbg_dataset* ds, const void* file, size_t len, vdbg_sq8** out) {
  if (ds == nullptr || out == nullptr || (file == nullptr && len > 0))
    return SetError(kInvalidArgument, "null argument");
  const auto* b = static_cast<const uint8_t*>(file);
  if (len < 12) return SetError(VDBG_CORRUPTION, "index file too short");
  uint32_t stored;
  std::memcpy(&stored, b + len - 4, 4);
  if (Crc32c(b, len - 4) != stored) return SetError(VDBG_CORRUPTION, "index file checksum mismatch");
  if (std::memcmp(b, "VDBHSQ81", 8) != 0)
    return SetError(VDBG_CORRUPTION, "not an hnsw-sq8 index file (magic VDBHSQ81)");
  const uint8_t* p = b + 8;
  size_t left = len - 12;
  auto take = [&](void* dst, size_t n) {
    if (left < n) return false;
    if (dst != nullptr) std::memcpy(dst, p, n);
    p += n;
    left -= n;
    return true;
  };
  const Dataset& d = ds->d;
  uint64_t n = 0;
  uint32_t qd = 0, qp = 0;
  if (!take(&n, 8) || n != d.n || !take(&qd, 4) || !take(&qp, 4) || qd > qp || qp % 16 != 0 ||
      qp != d.pd)
    return SetError(VDBG_CORRUPTION, "hnsw-sq8 index does not match the segment");
  std::vector<float> vmin(qp), scale(qp);
  if (!take(vmin.data(), qp * 4) || !take(scale.data(), qp * 4))
    return SetError(VDBG_CORRUPTION, "hnsw-sq8 index does not match the segment");
  const uint8_t* codes = p;
  if (!take(nullptr, size_t(n) * d.pd)) return SetError(VDBG_CORRUPTION, "truncated sq8 codes");
  HnswGraph* graph = nullptr;
  size_t used = 0;
  const char* err = nullptr;
  if (HnswParse(p, left, n, &graph, &used, &err) != 0) return SetError(VDBG_CORRUPTION, err);
  std::vector<uint8_t> codes_h;
  try {
    codes_h.assign(codes, codes + size_t(n) * d.pd);
  } catch (...) {
    HnswFree(graph);
    return SetError(kResourceExhausted, "out of host memory for the sq8 codes");
  }
  const int rc = CreateSq8(ds, vmin.data(), scale.data(), codes, out);
  if (rc != kOk) {
    HnswFree(graph);
    return rc;
  }
  (*out)->q.graph = graph;
  (*out)->q.codes_h = std::move(codes_h);
  return kOk;
}

int vdbg_sq8_graph_info(vdbg_sq8* sq, int64_t out[5]) {
  if (sq == nullptr || out == nullptr) return SetError(kInvalidArgument, "null argument");
  if (sq->q.graph == nullptr)
    return SetError(kFailedPrecondition, "the index has no graph (made by vdbg_sq8_create)");
  HnswInfo(sq->q.graph, out);
  return kOk;
}

namespace {

// HnswSq8Index::search's depth and beam width (src/index/hnsw/hnsw_index.cc:88-89).
void HnswDepth(size_t k, size_t ef, int rerank, size_t* depth, size_t* beam) {
  *depth = rerank < 0 ? std::max(ef, k) : size_t(rerank);
  *beam = std::max({ef, k, *depth});
}

// The walk of every query on the host (no lock held: the graph and host codes are read-only).
// cand: nq x kk ids and SQ8 distances, padded; dc: the walk's distance computations.
void WalkBatch(const Sq8Index& x, int kset, int threads, const float* Qh, size_t nq, size_t kk,
               size_t beam, const uint64_t* allow_h, std::vector<uint32_t>* cand,
               std::vector<float>* cand_d, std::vector<uint32_t>* found,
               std::vector<uint64_t>* dc) {
  const Dataset& d = *x.ds;
  cand->resize(nq * kk);
  cand_d->resize(nq * kk);
  found->resize(nq);
  dc->resize(nq);
  HnswWalkArgs a{x.graph, x.codes_h.data(), x.vmin_h.data(), x.scale_h.data(), d.pd,
                 HostSq8Kernel(kset, d.metric), Qh, nq, kk, beam, allow_h, cand->data(),
                 cand_d->data(), found->data(), dc->data(),
                 threads > 0 ? threads : DefaultHostThreads()};
  HnswWalk(a);
}

int CheckHnswArgs(vdbg_sq8* sq, size_t nq, size_t k, const void* queries, const void* ids,
                  const void* dists) {
  if (sq == nullptr) return SetError(kInvalidArgument, "null index");
  if (sq->q.graph == nullptr)
    return SetError(kFailedPrecondition, "the index has no graph (made by vdbg_sq8_create)");
  if (nq > 0 && k > 0 && (queries == nullptr || ids == nullptr || dists == nullptr))
    return SetError(kInvalidArgument, "null pointer");
  if (k > 10000) return SetError(kInvalidArgument, "k must be in 1..10000");
  if (nq > 0x7fffffffull) return SetError(kInvalidArgument, "too many queries");
  return kOk;
}

}  // namespace

int vdbg_sq8_hnsw_search_host(vdbg_sq8* sq, const float* queries, size_t nq, size_t k,
                              size_t ef, int rerank, const uint64_t* allow_words,
                              uint32_t* out_ids, float* out_dists, uint64_t* dist_comps) {
  VDBG_RETURN_IF_ERROR(CheckHnswArgs(sq, nq, k, queries, out_ids, out_dists));
  if (nq == 0) return kOk;
  Sq8Index& x = sq->q;
  Dataset& d = *x.ds;
  Ctx* c = d.ctx;
  if (k == 0) {
    if (dist_comps != nullptr) std::fill(dist_comps, dist_comps + nq, uint64_t(0));
    return kOk;
  }
  int kset, threads;
  {
    std::lock_guard<std::recursive_mutex> g(c->mu);
    kset = c->kset;
    threads = c->host_threads;
  }
  size_t depth, beam;
  HnswDepth(k, ef, rerank, &depth, &beam);
  const size_t kk = depth == 0 ? k : std::max(depth, k);
  std::vector<uint32_t> cand, found;
  std::vector<float> cand_d;
  std::vector<uint64_t> dc;
  WalkBatch(x, kset, threads, queries, nq, kk, beam, allow_words, &cand, &cand_d, &found, &dc);
  if (depth == 0) {  // the beam's k best by SQ8 distance (hnsw_index.cc:90-91)
    for (size_t i = 0; i < nq; ++i) {
      std::memcpy(out_ids + i * k, cand.data() + i * kk, k * 4);
      std::memcpy(out_dists + i * k, cand_d.data() + i * kk, k * 4);
      if (dist_comps != nullptr) dist_comps[i] = dc[i];
    }
    return kOk;
  }
  // Rerank of every query's beam on the GPU (hnsw_index.cc:93-94, index.cc:89-95): the
  // queries and the beams go in through the staging block
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  const int rc = StageRegions(c, queries, nq * d.pd * 4, cand.data(), nq * kk * 4, nq, k,
                              out_ids, out_dists, nullptr,
                              [&](const float* dq, const void* dx, uint32_t* di, float* dd,
                                  uint64_t*, hipStream_t st) {
                                return Rerank(c, d.rows, int(d.pd), d.metric, dq, nq,
                                              static_cast<const uint32_t*>(dx), kk, k, di, dd,
                                              st, &d.src);
                              });
  if (rc == kOk && dist_comps != nullptr)
    for (size_t i = 0; i < nq; ++i) dist_comps[i] = dc[i] + found[i];
  return rc;
}

int vdbg_sq8_hnsw_search_device(vdbg_sq8* sq, const float* queries, size_t nq, size_t k,
                                size_t ef, int rerank, const uint64_t* allow_words,
                                uint32_t* out_ids, float* out_dists, uint64_t* dist_comps,
                                void* stream) {
  VDBG_RETURN_IF_ERROR(CheckHnswArgs(sq, nq, k, queries, out_ids, out_dists));
  if (nq == 0) return kOk;
  Sq8Index& x = sq->q;
  Dataset& d = *x.ds;
  Ctx* c = d.ctx;
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : c->stream;
  int kset, threads;
  std::vector<float> qh(nq * d.pd);
  std::vector<uint64_t> allow_h;
  {  // the queries (and the filter) to the host for the walk
    std::lock_guard<std::recursive_mutex> g(c->mu);
    VDBG_HIP(hipSetDevice(c->device));
    kset = c->kset;
    threads = c->host_threads;
    VDBG_HIP(hipMemcpyAsync(qh.data(), queries, qh.size() * 4, hipMemcpyDeviceToHost, s));
    if (allow_words != nullptr) {
      allow_h.resize((d.n + 63) / 64);
      if (!allow_h.empty())
        VDBG_HIP(hipMemcpyAsync(allow_h.data(), allow_words, allow_h.size() * 8,
                                hipMemcpyDeviceToHost, s));
    }
    VDBG_HIP(hipStreamSynchronize(s));
  }
  std::vector<uint64_t> dch(nq, 0);
  size_t depth, beam;
  HnswDepth(k, ef, rerank, &depth, &beam);
  const size_t kk = depth == 0 ? k : std::max(depth, k);
  std::vector<uint32_t> cand, found;
  std::vector<float> cand_d;
  std::vector<uint64_t> dc;
  if (k > 0)
    WalkBatch(x, kset, threads, qh.data(), nq, kk, beam,
              allow_words != nullptr ? allow_h.data() : nullptr, &cand, &cand_d, &found, &dc);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  if (k == 0) {
    if (dist_comps != nullptr) {
      VDBG_HIP(hipMemcpyAsync(dist_comps, dch.data(), nq * 8, hipMemcpyHostToDevice, s));
      VDBG_HIP(hipStreamSynchronize(s));
    }
    return kOk;
  }
  for (size_t i = 0; i < nq; ++i) dch[i] = dc[i] + (depth == 0 ? 0 : found[i]);
  if (depth == 0) {
    for (size_t i = 0; i < nq; ++i) {  // compact [nq][kk] to [nq][k] (kk == k here)
      VDBG_HIP(hipMemcpyAsync(out_ids + i * k, cand.data() + i * kk, k * 4,
                              hipMemcpyHostToDevice, s));
      VDBG_HIP(hipMemcpyAsync(out_dists + i * k, cand_d.data() + i * kk, k * 4,
                              hipMemcpyHostToDevice, s));
    }
  } else {
    uint32_t* dcand = nullptr;
    VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&dcand), nq * kk * 4, s));
    hipError_t e = hipMemcpyAsync(dcand, cand.data(), nq * kk * 4, hipMemcpyHostToDevice, s);
    int rc = e == hipSuccess ? kOk : SetError(kInternal, hipGetErrorString(e));
    if (rc == kOk)
      rc = Rerank(c, d.rows, int(d.pd), d.metric, queries, nq, dcand, kk, k, out_ids, out_dists,
                  s, &d.src);
    (void)hipFreeAsync(dcand, s);
    VDBG_RETURN_IF_ERROR(rc);
  }
  if (dist_comps != nullptr)
    VDBG_HIP(hipMemcpyAsync(dist_comps, dch.data(), nq * 8, hipMemcpyHostToDevice, s));
  // the host vectors above are sources of queued copies: wait before they go away
  VDBG_HIP(hipStreamSynchronize(s));
  return kOk;
}

int vdbg_sq8_destroy(vdbg_sq8* sq) {
  if (sq == nullptr) return kOk;
  Ctx* c = sq->q.ds->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  (void)hipSetDevice(c->device);
  (void)hipDeviceSynchronize();
  --sq->q.ds->live_indexes;
  HnswFree(sq->q.graph);
  FreeSample(&sq->q.src);
  (void)hipFree(sq->q.codes);
  (void)hipFree(sq->q.codes16);
  (void)hipFree(sq->q.yn);
  (void)hipFree(sq->q.vmin);
  delete sq;
  return kOk;
}

int vdbg_sq8_codes(vdbg_sq8* sq, uint8_t* codes_out) {
  if (sq == nullptr || codes_out == nullptr) return SetError(kInvalidArgument, "null argument");
  Ctx* c = sq->q.ds->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  const size_t bytes = sq->q.ds->n * sq->q.ds->pd;
  if (bytes == 0) return kOk;
  VDBG_HIP(hipMemcpyAsync(codes_out, sq->q.codes, bytes, hipMemcpyDeviceToHost, c->stream));
  VDBG_HIP(hipStreamSynchronize(c->stream));
  return kOk;
}

int vdbg_sq8_search_device(vdbg_sq8* sq, const float* queries, size_t nq, size_t k,
                           size_t depth, const uint64_t* allow_words, uint32_t* out_ids,
                           float* out_dists, void* stream) {
  if (sq == nullptr) return SetError(kInvalidArgument, "null index");
  if (nq > 0 && k > 0 && (queries == nullptr || out_ids == nullptr || out_dists == nullptr))
    return SetError(kInvalidArgument, "null pointer");
  Ctx* c = sq->q.ds->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : c->stream;
  return Sq8Search(&sq->q, queries, nq, k, depth, allow_words, out_ids, out_dists, s);
}

int vdbg_sq8_search_host(vdbg_sq8* sq, const float* queries, size_t nq, size_t k, size_t depth,
                         const uint64_t* allow_words, uint32_t* out_ids, float* out_dists,
                         uint64_t* dist_comps) {
  if (sq == nullptr) return SetError(kInvalidArgument, "null index");
  if (dist_comps) *dist_comps = 0;
  if (nq == 0 || k == 0) return kOk;
  if (queries == nullptr || out_ids == nullptr || out_dists == nullptr)
    return SetError(kInvalidArgument, "null pointer");
  Ctx* c = sq->q.ds->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  Sq8Index* x = &sq->q;
  int rc = StageHost(c, x->ds->n, x->ds->pd, queries, nq, k, allow_words, out_ids, out_dists,
                     nullptr,
                     [&](const float* dq, const uint64_t* dm, uint32_t* di, float* dd,
                         uint64_t*, hipStream_t s) {
                       return Sq8Search(x, dq, nq, k, depth, dm, di, dd, s);
                     });
  if (rc == kOk && dist_comps)
    *dist_comps = uint64_t(nq) * (x->ds->n + (depth > 0 ? std::min(std::max(depth, k), x->ds->n) : 0));
  return rc;
}

int vdbg_rerank_device(vdbg_dataset* ds, const float* queries, size_t nq, const uint32_t* cand,
                       size_t depth, size_t k, uint32_t* out_ids, float* out_dists,
                       uint64_t* dist_comps, void* stream) {
  if (ds == nullptr) return SetError(kInvalidArgument, "null dataset");
  if (nq == 0 || k == 0) return kOk;
  if (queries == nullptr || out_ids == nullptr || out_dists == nullptr ||
      (depth > 0 && cand == nullptr))
    return SetError(kInvalidArgument, "null pointer");
  if (k > 10000) return SetError(kInvalidArgument, "k must be in 1..10000");
  Dataset* d = &ds->d;
  Ctx* c = d->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : c->stream;
  return RerankChecked(c, d, queries, nq, cand, depth, k, out_ids, out_dists, dist_comps, s);
}

int vdbg_rerank_host(vdbg_dataset* ds, const float* queries, size_t nq, const uint32_t* cand,
                     size_t depth, size_t k, uint32_t* out_ids, float* out_dists,
                     uint64_t* dist_comps) {
  if (ds == nullptr) return SetError(kInvalidArgument, "null dataset");
  if (nq == 0 || k == 0) return kOk;
  if (queries == nullptr || out_ids == nullptr || out_dists == nullptr ||
      (depth > 0 && cand == nullptr))
    return SetError(kInvalidArgument, "null pointer");
  if (k > 10000) return SetError(kInvalidArgument, "k must be in 1..10000");
  Dataset* d = &ds->d;
  for (size_t i = 0; i < nq * depth; ++i)
    if (cand[i] != kNoId && cand[i] >= d->n) return SetError(kInvalidArgument, "candidate row out of range");
  Ctx* c = d->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  // (a zero-length candidate region still gets a device address: RerankChecked reads none)
  static const uint32_t kNone = kNoId;
  return StageRegions(c, queries, nq * d->pd * 4, depth > 0 ? static_cast<const void*>(cand) : &kNone,
                      depth > 0 ? nq * depth * 4 : 4, nq, k, out_ids, out_dists, dist_comps,
                      [&](const float* dq, const void* dx, uint32_t* di, float* dd,
                          uint64_t* ddc, hipStream_t st) {
                        return RerankChecked(c, d, dq, nq, static_cast<const uint32_t*>(dx),
                                             depth, k, di, dd, ddc, st, true);
                      });
}

int vdbg_last_gemm_bits(vdbg_ctx* ctx) {
  if (ctx == nullptr) return 0;
  Ctx& c = ctx->c;
  std::lock_guard<std::recursive_mutex> g(c.mu);
  if (c.last_gemm_gate != nullptr) {  // chosen on the device: read the flag
    std::vector<int> v(size_t(std::max(c.last_gemm_gate_n.load(), 1)), 0);
    // (the scan may have run on any stream)
    if (hipSetDevice(c.device) != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(v.data(), c.last_gemm_gate, size_t(c.last_gemm_gate_n) * sizeof(int),
                  hipMemcpyDeviceToHost) != hipSuccess)
      return 0;
    bool all = true;
    for (int i = 0; i < c.last_gemm_gate_n; ++i) all = all && v[size_t(i)] != 0;
    c.last_gemm_bits = all ? 8 : 32;
    c.last_gemm_gate = nullptr;
  }
  return c.last_gemm_bits;
}

int vdbg_last_fallbacks(vdbg_ctx* ctx, uint64_t* fallback_queries) {
  if (ctx == nullptr || fallback_queries == nullptr)
    return SetError(kInvalidArgument, "null argument");
  Ctx& c = ctx->c;
  std::lock_guard<std::recursive_mutex> g(c.mu);
  uint64_t n = c.last_fallbacks;
  if (c.fb_dev_used) {  // passes queued without a host read: their count is on the device
    VDBG_HIP(hipSetDevice(c.device));
    VDBG_HIP(hipDeviceSynchronize());
    uint32_t v = 0;
    VDBG_HIP(hipMemcpy(&v, c.fb_dev, 4, hipMemcpyDeviceToHost));
    VDBG_HIP(hipMemset(c.fb_dev, 0, 4));
    c.fb_dev_used = false;
    n += v;
  }
  *fallback_queries = n;
  return kOk;
}

}  // extern "C"
