// pqflat.hip -- PqFlatIndex (src/index/quant/ivf_pq.h:12-36, ivf_pq.cc:41-98) on gfx950.
//
// Every row's PQ code is scored by ADC against the query's table, the max(depth, k) best
// by (ADC, id) kept, then FinishSearch (:28-36): the float Rerank of those candidates, or
// with depth 0 the best k by ADC.  Per query:
//   table[j][c] = L2SqAny(q_j, C_j[c])  (L2)  or  -DotAny(q_j, C_j[c])  (inner product,
//                 cosine)                                  ProductQuantizer::compute_table
//   adc(code)   = four accumulators over j mod 4           pq.h:36-46
//   depth       = rerank < 0 ? max(10 k, 100) : rerank     RerankDepth, ivf_pq.cc:16-19
//   distance_computations = rows (+ the candidates reranked)
// The tables are built on the device ([nq][m x 256] floats), the scan is the exact-score
// scan of the flat path with the ADC as its score (row splits with a wave top-k each, then
// a merge; a segmented sort beyond 240), the rerank the flat path's k_rerank.
//
// Bound: HBM.  Each query streams the n x m code bytes (plus its 16 KB table, L2-resident).
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "vdbg_device.h"
#include "vdbg_internal.h"

namespace vdbg {
namespace {

constexpr int kKsub = 256;

// compute_table (pq.cc:63-73) for nq queries: one thread per (query, subspace, centroid).
__global__ void k_pq_tables(const float* __restrict__ Q, int pd, int nq,
                            const float* __restrict__ cen, int m, int dsub, int l2,
                            float* __restrict__ T) {
  const size_t t = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  const size_t ts = size_t(m) * kKsub;
  if (t >= size_t(nq) * ts) return;
  const size_t q = t / ts;
  const int e = int(t - q * ts);
  const int j = e / kKsub;
  const float* qs = Q + q * pd + size_t(j) * dsub;
  const float* cc = cen + size_t(e) * dsub;
  T[t] = l2 ? l2sq_any(qs, cc, dsub) : -dot_any(qs, cc, dsub);
}

// distance_computations of PqFlatIndex::search: every row, plus the candidates handed to
// Rerank (ivf_pq.cc:76-79).
__global__ void k_pqflat_dc(const uint32_t* __restrict__ cand, int kk, int nq, uint64_t rows,
                            int reranked, uint64_t* __restrict__ dc) {
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= nq) return;
  uint64_t v = rows;
  if (reranked)
    for (int i = 0; i < kk; ++i) v += cand[size_t(q) * kk + i] != kNoId ? 1 : 0;
  dc[q] = v;
}

// A device buffer released on the stream when the call ends.
struct Tmp {
  void* p = nullptr;
  hipStream_t s = nullptr;
  ~Tmp() {
    if (p != nullptr) (void)hipFreeAsync(p, s);
  }
};

int PqFlatSearch(PqFlatIndex* x, const float* Q, size_t nq, size_t k, int rerank,
                 const uint64_t* allow, uint32_t* out_ids, float* out_d, uint64_t* dc,
                 hipStream_t s) {
  Dataset* ds = x->ds;
  Ctx* c = ds->ctx;
  const size_t n = ds->n;
  if (nq == 0) return kOk;
  if (n == 0 || k == 0) {  // ivf_pq.cc:62: nothing searched, nothing counted
    if (k > 0) {
      ScanSource none;
      VDBG_RETURN_IF_ERROR(ScoreScan(c, none, Q, nq, k, nullptr, out_ids, out_d, s));
    }
    if (dc != nullptr) VDBG_HIP(hipMemsetAsync(dc, 0, nq * 8, s));
    return kOk;
  }
  const size_t depth = rerank < 0 ? std::max<size_t>(10 * k, 100) : size_t(rerank);
  const size_t kk = std::max(depth, k);
  const size_t ts = size_t(x->m) * kKsub;
  Tmp tables;
  tables.s = s;
  VDBG_HIP(hipMallocAsync(&tables.p, nq * ts * sizeof(float), s));
  {
    ProfScope ps(c, "pq_tables", s);
    const size_t total = nq * ts;
    k_pq_tables<<<dim3(unsigned((total + 255) / 256)), 256, 0, s>>>(
        Q, int(ds->pd), int(nq), x->cen, x->m, x->dsub, ds->metric == 0 ? 1 : 0,
        static_cast<float*>(tables.p));
    VDBG_HIP(hipGetLastError());
  }
  ScanSource src;
  src.kind = 2;
  src.C = x->codes;
  src.pq_m = x->m;
  src.N = uint32_t(n);
  src.pd = int(ts);
  src.metric = ds->metric;
  const float* T = static_cast<const float*>(tables.p);
  // the scan keeps at most n candidates, as a TopK of any capacity over n rows does (depth
  // may exceed vdb's largest k: max(10 k, 100) at k = 10,000)
  const size_t keep = std::min(kk, std::max<size_t>(n, k));
  if (depth == 0) {
    VDBG_RETURN_IF_ERROR(ScoreScan(c, src, T, nq, k, allow, out_ids, out_d, s));
    if (dc != nullptr)
      k_pqflat_dc<<<dim3(unsigned((nq + 255) / 256)), 256, 0, s>>>(out_ids, int(k), int(nq), n, 0,
                                                                   dc);
    VDBG_HIP(hipGetLastError());
    return kOk;
  }
  Tmp ci, cd;
  ci.s = cd.s = s;
  VDBG_HIP(hipMallocAsync(&ci.p, nq * keep * 4, s));
  VDBG_HIP(hipMallocAsync(&cd.p, nq * keep * 4, s));
  uint32_t* cand = static_cast<uint32_t*>(ci.p);
  VDBG_RETURN_IF_ERROR(ScoreScan(c, src, T, nq, keep, allow, cand, static_cast<float*>(cd.p), s));
  VDBG_RETURN_IF_ERROR(Rerank(c, ds->rows, int(ds->pd), ds->metric, Q, nq, cand, keep, k, out_ids,
                              out_d, s, &ds->src));
  if (dc != nullptr)
    k_pqflat_dc<<<dim3(unsigned((nq + 255) / 256)), 256, 0, s>>>(cand, int(keep), int(nq), n, 1,
                                                                 dc);
  VDBG_HIP(hipGetLastError());
  return kOk;
}

void FreePqFlat(PqFlatIndex* x) {
  (void)hipFree(x->cen);
  (void)hipFree(x->codes);
  x->cen = nullptr;
  x->codes = nullptr;
}

// Uploads the codebook (and codes, when given on the host) of an index over ds.
int InstallPqFlat(Ctx* c, PqFlatIndex* x, const uint8_t* codes_h, hipStream_t s) {
  const size_t n = x->ds->n;
  if (!x->cen_h.empty()) {
    VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&x->cen), x->cen_h.size() * sizeof(float)));
    VDBG_HIP(hipMemcpyAsync(x->cen, x->cen_h.data(), x->cen_h.size() * sizeof(float),
                            hipMemcpyHostToDevice, s));
  }
  if (n > 0 && x->codes == nullptr) {
    VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&x->codes), n * x->m));
    if (codes_h != nullptr)
      VDBG_HIP(hipMemcpyAsync(x->codes, codes_h, n * x->m, hipMemcpyHostToDevice, s));
  }
  VDBG_HIP(hipStreamSynchronize(s));
  return kOk;
}

}  // namespace
}  // namespace vdbg

using namespace vdbg;

extern "C" {

int vdbg_pqflat_build(vdbg_dataset* ds, size_t pq_m, uint64_t seed,
                      size_t max_points_per_centroid, size_t kmeans_iters, vdbg_pqflat** out) {
  if (ds == nullptr || out == nullptr) return SetError(kInvalidArgument, "null argument");
  Dataset& d = ds->d;
  if (pq_m == 0 || d.dim % pq_m != 0)
    return SetError(kInvalidArgument, "pq_m must divide the dimension");  // index.cc:27-29
  Ctx* c = d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  auto* h = new (std::nothrow) vdbg_pqflat;
  if (h == nullptr) return SetError(kResourceExhausted, "out of host memory");
  PqFlatIndex& x = h->p;
  x.ds = &d;
  x.m = int(pq_m);
  x.dsub = int(d.dim / pq_m);
  auto fail = [&](int rc) {
    FreePqFlat(&x);
    delete h;
    return rc;
  };
  // PqFlatIndex::build (ivf_pq.cc:45-57): nothing is trained over no rows
  if (d.n > 0) {
    int rc = PqTrainRows(c, d.rows, d.n, d.pd, d.dim, pq_m, seed, max_points_per_centroid,
                         kmeans_iters, &x.cen_h, s);
    if (rc != kOk) return fail(rc);
    x.trained = true;
  }
  int rc = InstallPqFlat(c, &x, nullptr, s);
  if (rc != kOk) return fail(rc);
  if (d.n > 0) {
    rc = PqEncode(c, d.rows, uint32_t(d.n), int(d.pd), int(d.dim), nullptr, nullptr, x.cen, x.m,
                  x.dsub, x.codes, s);
    if (rc != kOk) return fail(rc);
    if (hipStreamSynchronize(s) != hipSuccess) return fail(SetError(kInternal, "pq encode"));
  }
  ++d.live_indexes;
  *out = h;
  return kOk;
}

// LoadIndex of a VDBPQFL1 file (index.cc:38-87, 76-77) and PqFlatIndex::load (ivf_pq.cc:
// 89-98): u64 rows, the ProductQuantizer (pq.cc:75-92: u32 dim, u32 m, centroids), then rows
// x m code bytes.
int vdbg_pqflat_load(vdbg_dataset* ds, const void* file, size_t len, vdbg_pqflat** out) {
  if (ds == nullptr || out == nullptr || (file == nullptr && len > 0))
    return SetError(kInvalidArgument, "null argument");
  const auto* b = static_cast<const uint8_t*>(file);
  if (len < 12) return SetError(VDBG_CORRUPTION, "index file too short");
  uint32_t stored;
  std::memcpy(&stored, b + len - 4, 4);
  if (Crc32c(b, len - 4) != stored) return SetError(VDBG_CORRUPTION, "index file checksum mismatch");
  if (std::memcmp(b, "VDBPQFL1", 8) != 0)
    return SetError(VDBG_CORRUPTION, "not a pq-flat index file (magic VDBPQFL1)");
  const uint8_t* p = b + 8;
  size_t left = len - 12;
  auto take = [&](void* dst, size_t n) {
    if (left < n) return false;
    if (dst != nullptr && n > 0) std::memcpy(dst, p, n);
    p += n;
    left -= n;
    return true;
  };
  Dataset& d = ds->d;
  uint64_t n = 0;
  uint32_t dim = 0, m = 0;
  const char* mismatch = "pq index does not match the segment";
  if (!take(&n, 8) || n != d.n || !take(&dim, 4) || !take(&m, 4) || m == 0 || dim % m != 0)
    return SetError(VDBG_CORRUPTION, mismatch);
  const size_t dsub = dim / m;
  std::vector<float> cen(size_t(m) * kKsub * dsub);
  if (!take(cen.data(), cen.size() * sizeof(float)) || dim != d.dim)
    return SetError(VDBG_CORRUPTION, mismatch);
  const uint8_t* codes = p;
  if (!take(nullptr, size_t(n) * m)) return SetError(VDBG_CORRUPTION, "truncated pq codes");
  Ctx* c = d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  auto* h = new (std::nothrow) vdbg_pqflat;
  if (h == nullptr) return SetError(kResourceExhausted, "out of host memory");
  PqFlatIndex& x = h->p;
  x.ds = &d;
  x.m = int(m);
  x.dsub = int(dsub);
  x.cen_h = std::move(cen);
  x.trained = true;
  const int rc = InstallPqFlat(c, &x, codes, c->stream);
  if (rc != kOk) {
    FreePqFlat(&x);
    delete h;
    return rc;
  }
  ++d.live_indexes;
  *out = h;
  return kOk;
}

// PqFlatIndex::save (ivf_pq.cc:81-87) through WriteIndexFile (index.cc:40-46).
int vdbg_pqflat_save(vdbg_pqflat* ix, void* buf, size_t cap, size_t* len) {
  if (ix == nullptr || len == nullptr) return SetError(kInvalidArgument, "null argument");
  PqFlatIndex& x = ix->p;
  Dataset& d = *x.ds;
  const size_t n = d.n;
  std::string out("VDBPQFL1");
  auto put = [&](const void* v, size_t bytes) {
    out.append(static_cast<const char*>(v), bytes);
  };
  const uint64_t rows = n;
  const uint32_t dim = uint32_t(d.dim), m = uint32_t(x.m);
  put(&rows, 8);
  put(&dim, 4);
  put(&m, 4);
  put(x.cen_h.data(), x.cen_h.size() * sizeof(float));
  const size_t at = out.size();
  out.resize(at + n * x.m);
  if (n > 0) {
    Ctx* c = d.ctx;
    std::lock_guard<std::recursive_mutex> g(c->mu);
    VDBG_HIP(hipSetDevice(c->device));
    VDBG_HIP(hipMemcpyAsync(&out[at], x.codes, n * x.m, hipMemcpyDeviceToHost, c->stream));
    VDBG_HIP(hipStreamSynchronize(c->stream));
  }
  const uint32_t crc = Crc32c(out.data(), out.size());
  put(&crc, 4);
  *len = out.size();
  if (buf != nullptr) {
    if (cap < out.size()) return SetError(kResourceExhausted, "buffer too small for the index file");
    std::memcpy(buf, out.data(), out.size());
  }
  return kOk;
}

int vdbg_pqflat_destroy(vdbg_pqflat* ix) {
  if (ix == nullptr) return kOk;
  Ctx* c = ix->p.ds->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  (void)hipSetDevice(c->device);
  (void)hipDeviceSynchronize();
  --ix->p.ds->live_indexes;
  FreePqFlat(&ix->p);
  delete ix;
  return kOk;
}

int vdbg_pqflat_info(vdbg_pqflat* ix, size_t* m, float* centroids_out) {
  if (ix == nullptr || m == nullptr) return SetError(kInvalidArgument, "null argument");
  *m = size_t(ix->p.m);
  if (centroids_out != nullptr && !ix->p.cen_h.empty())
    std::memcpy(centroids_out, ix->p.cen_h.data(), ix->p.cen_h.size() * sizeof(float));
  return kOk;
}

int vdbg_pqflat_codes(vdbg_pqflat* ix, uint8_t* codes_out) {
  if (ix == nullptr || codes_out == nullptr) return SetError(kInvalidArgument, "null argument");
  const size_t bytes = ix->p.ds->n * size_t(ix->p.m);
  if (bytes == 0) return kOk;
  Ctx* c = ix->p.ds->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  VDBG_HIP(hipMemcpyAsync(codes_out, ix->p.codes, bytes, hipMemcpyDeviceToHost, c->stream));
  VDBG_HIP(hipStreamSynchronize(c->stream));
  return kOk;
}

int vdbg_pqflat_search_device(vdbg_pqflat* ix, const float* queries, size_t nq, size_t k,
                              int rerank, const uint64_t* allow_words, uint32_t* out_ids,
                              float* out_dists, uint64_t* dist_comps, void* stream) {
  if (ix == nullptr) return SetError(kInvalidArgument, "null index");
  if (nq > 0 && k > 0 && (queries == nullptr || out_ids == nullptr || out_dists == nullptr))
    return SetError(kInvalidArgument, "null pointer");
  if (k > 10000) return SetError(kInvalidArgument, "k must be in 1..10000");
  Ctx* c = ix->p.ds->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : c->stream;
  return PqFlatSearch(&ix->p, queries, nq, k, rerank, allow_words, out_ids, out_dists,
                      dist_comps, s);
}

int vdbg_pqflat_search_host(vdbg_pqflat* ix, const float* queries, size_t nq, size_t k,
                            int rerank, const uint64_t* allow_words, uint32_t* out_ids,
                            float* out_dists, uint64_t* dist_comps) {
  if (ix == nullptr) return SetError(kInvalidArgument, "null index");
  if (nq == 0 || k == 0) {
    if (dist_comps != nullptr) std::fill(dist_comps, dist_comps + nq, uint64_t(0));
    return kOk;
  }
  if (queries == nullptr || out_ids == nullptr || out_dists == nullptr)
    return SetError(kInvalidArgument, "null pointer");
  if (k > 10000) return SetError(kInvalidArgument, "k must be in 1..10000");
  Dataset& d = *ix->p.ds;
  Ctx* c = d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  return StageHost(c, d.n, d.pd, queries, nq, k, allow_words, out_ids, out_dists, dist_comps,
                   [&](const float* dq, const uint64_t* dm, uint32_t* di, float* dd,
                       uint64_t* ddc, hipStream_t st) {
                     return PqFlatSearch(&ix->p, dq, nq, k, rerank, dm, di, dd, ddc, st);
                   });
}

}  // extern "C"
