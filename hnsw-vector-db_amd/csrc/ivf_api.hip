// ivf_api.hip -- the IVF-PQ part of the C ABI: vdb's VDBIVFP1 index file in and out,
// resident lists and tables, and IvfPqIndex::search on the GPU.
#include <algorithm>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "vdbg_internal.h"

namespace vdbg {


int IvfTerm2(Ctx* c, const float* coarse, int nlist, int pd, const float* cen, int m, int dsub,
             float* term2, hipStream_t s);
int IvfQtabRs(Ctx* c, const float* Q, int pd, int nq, const float* cen, int m, int dsub,
              float* qtab, float* qmax, hipStream_t s);
int IvfRowSums(Ctx* c, const uint32_t* off, int nlist, const uint8_t* codes, int m,
               const float* term2, float* rowsum, float* t2abs, hipStream_t s);
int IvfQtab(Ctx* c, const float* Q, int pd, int nq, const float* cen, int m, int dsub,
            int twice, float* qtab, hipStream_t s);
int IvfScan(Ctx* c, const IvfScanArgs& a, hipStream_t s, void* scratch);
size_t IvfScanScratchBytes(size_t nq, size_t nprobe);
int IvfScanDeep(Ctx* c, const IvfScanArgs& a, hipStream_t s);

namespace {

struct Reader {
  const uint8_t* p;
  const uint8_t* end;
  bool ok = true;
  template <class T>
  bool get(T* v) {
    if (!ok || size_t(end - p) < sizeof(T)) return ok = false;
    std::memcpy(v, p, sizeof(T));
    p += sizeof(T);
    return true;
  }
  bool bytes(size_t n, const uint8_t** out) {
    if (!ok || size_t(end - p) < n) return ok = false;
    *out = p;
    p += n;
    return true;
  }
};

template <class T>
void Put(std::string* s, const T& v) {
  s->append(reinterpret_cast<const char*>(&v), sizeof(T));
}

constexpr size_t kMaxPrecomputedBytes = size_t{1} << 30;  // ivf_pq.h:61

}  // namespace

void FreeIvf(IvfIndex* x) {
  if (x->coarse_ds != nullptr) vdbg_dataset_destroy(x->coarse_ds);
  (void)hipFree(x->cen);
  (void)hipFree(x->off);
  (void)hipFree(x->ids);
  (void)hipFree(x->codes);
  (void)hipFree(x->term2);
  (void)hipFree(x->rowsum);
  (void)hipFree(x->t2abs);
  x->rowsum = nullptr;
  x->t2abs = nullptr;
  x->coarse_ds = nullptr;
  x->cen = nullptr;
  x->term2 = nullptr;
  x->off = nullptr;
  x->ids = nullptr;
  x->codes = nullptr;
}

// Makes coarse centroids, codebook and offsets resident (ids/codes are already on the
// device) and derives the precomputed tables, as IvfPqIndex::load does after reading
// (ivf_pq.cc:251-278) and build does at its end (:140-148).
int InstallIvf(Ctx* c, IvfIndex* x, hipStream_t s) {
  const size_t pd = x->pd, nlist = x->nlist;
  const size_t cen_n = size_t(x->m) * 256 * x->dsub;
  VDBG_RETURN_IF_ERROR(vdbg_dataset_create(c->handle, x->coarse_h.data(), nlist, x->dim, pd,
                                           x->metric, &x->coarse_ds));
  VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&x->cen), cen_n * sizeof(float)));
  VDBG_HIP(hipMemcpyAsync(x->cen, x->cen_h.data(), cen_n * sizeof(float), hipMemcpyHostToDevice, s));
  if (x->off == nullptr) {
    VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&x->off), (nlist + 1) * sizeof(uint32_t)));
    VDBG_HIP(hipMemcpyAsync(x->off, x->off_h.data(), (nlist + 1) * sizeof(uint32_t),
                            hipMemcpyHostToDevice, s));
  }
  // precompute_tables (ivf_pq.cc:152-167): L2 only, while nlist * m * 256 floats <= 1 GiB
  if (x->metric == 0 && nlist > 0 && nlist * x->m * 256 * sizeof(float) <= kMaxPrecomputedBytes) {
    VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&x->term2), nlist * x->m * 256 * sizeof(float)));
    VDBG_RETURN_IF_ERROR(IvfTerm2(c, x->coarse_ds->d.rows, int(nlist), int(pd), x->cen, x->m,
                                  x->dsub, x->term2, s));
    // the scan's ranking inputs: term-2 sums per row and their per-list bound
    const size_t n = x->off_h.empty() ? 0 : x->off_h.back();  // CSR entries
    VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&x->rowsum), std::max<size_t>(1, n) * sizeof(float)));
    VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&x->t2abs), nlist * sizeof(float)));
    VDBG_RETURN_IF_ERROR(IvfRowSums(c, x->off, int(nlist), x->codes, x->m, x->term2, x->rowsum,
                                    x->t2abs, s));
  }
  VDBG_HIP(hipStreamSynchronize(s));
  return kOk;
}

// IvfPqIndex::load (ivf_pq.cc:251-278) after LoadIndex's framing check (index.cc:38-56).
static int LoadIvf(Ctx* c, IvfIndex* x, const uint8_t* bytes, size_t len, hipStream_t s) {
  if (len < 12) return SetError(VDBG_CORRUPTION, "index file too short");
  uint32_t stored;
  std::memcpy(&stored, bytes + len - 4, 4);
  if (Crc32c(bytes, len - 4) != stored) return SetError(VDBG_CORRUPTION, "index file checksum mismatch");
  if (std::memcmp(bytes, "VDBIVFP1", 8) != 0) return SetError(VDBG_CORRUPTION, "unknown index file magic");
  Reader r{bytes + 8, bytes + len - 4};
  uint64_t n = 0;
  uint32_t pd = 0, nl = 0;
  if (!r.get(&n) || !r.get(&pd) || !r.get(&nl) || n != x->ds->n || pd != x->ds->pd)
    return SetError(VDBG_CORRUPTION, "ivf-pq index does not match the segment");
  const uint8_t* b = nullptr;
  if (!r.bytes(size_t(nl) * pd * sizeof(float), &b))
    return SetError(VDBG_CORRUPTION, "truncated ivf centroids");
  x->nlist = int(nl);
  x->pd = int(pd);
  x->coarse_h.resize(size_t(nl) * pd);
  std::memcpy(x->coarse_h.data(), b, x->coarse_h.size() * sizeof(float));
  // ProductQuantizer::deserialize (pq.cc:82-92)
  uint32_t d = 0, m = 0;
  if (!r.get(&d) || !r.get(&m) || m == 0 || d % m != 0 || d != x->ds->dim)
    return SetError(VDBG_CORRUPTION, "bad pq codebook");
  x->dim = int(d);
  x->m = int(m);
  x->dsub = int(d / m);
  if (!r.bytes(size_t(m) * 256 * x->dsub * sizeof(float), &b))
    return SetError(VDBG_CORRUPTION, "bad pq codebook");
  x->cen_h.resize(size_t(m) * 256 * x->dsub);
  std::memcpy(x->cen_h.data(), b, x->cen_h.size() * sizeof(float));
  std::vector<uint32_t> ids;
  std::vector<uint8_t> codes;
  ids.reserve(n);
  codes.reserve(n * m);
  x->off_h.assign(1, 0);
  for (uint32_t l = 0; l < nl; ++l) {
    uint64_t sz = 0;
    if (!r.get(&sz) || sz > n) return SetError(VDBG_CORRUPTION, "bad ivf list size");
    if (!r.bytes(sz * sizeof(uint32_t), &b)) return SetError(VDBG_CORRUPTION, "truncated ivf ids");
    const size_t at = ids.size();
    ids.resize(at + sz);
    std::memcpy(ids.data() + at, b, sz * sizeof(uint32_t));
    for (size_t i = at; i < ids.size(); ++i)
      if (ids[i] >= n) return SetError(VDBG_CORRUPTION, "ivf id out of range");
    if (!r.bytes(sz * m, &b)) return SetError(VDBG_CORRUPTION, "truncated ivf codes");
    codes.insert(codes.end(), b, b + sz * m);
    if (ids.size() > 0xffffffffull) return SetError(VDBG_CORRUPTION, "too many list entries");
    x->off_h.push_back(uint32_t(ids.size()));
  }
  VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&x->ids), std::max<size_t>(1, ids.size()) * 4));
  VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&x->codes), std::max<size_t>(1, codes.size())));
  if (!ids.empty()) {
    VDBG_HIP(hipMemcpyAsync(x->ids, ids.data(), ids.size() * 4, hipMemcpyHostToDevice, s));
    VDBG_HIP(hipMemcpyAsync(x->codes, codes.data(), codes.size(), hipMemcpyHostToDevice, s));
  }
  return InstallIvf(c, x, s);
}

// IvfPqIndex::save (ivf_pq.cc:236-249) + WriteIndexFile (index.cc:110-117).
static int SaveIvf(Ctx* c, IvfIndex* x, std::string* out, hipStream_t s) {
  const size_t total = x->off_h.empty() ? 0 : x->off_h.back();
  std::vector<uint32_t> ids(total);
  std::vector<uint8_t> codes(total * x->m);
  if (total > 0) {
    VDBG_HIP(hipMemcpyAsync(ids.data(), x->ids, total * 4, hipMemcpyDeviceToHost, s));
    VDBG_HIP(hipMemcpyAsync(codes.data(), x->codes, codes.size(), hipMemcpyDeviceToHost, s));
    VDBG_HIP(hipStreamSynchronize(s));
  }
  std::string& f = *out;
  f.clear();
  f.append("VDBIVFP1", 8);
  Put<uint64_t>(&f, x->ds->n);
  Put<uint32_t>(&f, uint32_t(x->pd));
  Put<uint32_t>(&f, uint32_t(x->nlist));
  f.append(reinterpret_cast<const char*>(x->coarse_h.data()), x->coarse_h.size() * sizeof(float));
  Put<uint32_t>(&f, uint32_t(x->dim));
  Put<uint32_t>(&f, uint32_t(x->m));
  f.append(reinterpret_cast<const char*>(x->cen_h.data()), x->cen_h.size() * sizeof(float));
  for (int l = 0; l < x->nlist; ++l) {
    const uint32_t b = x->off_h[l], e = x->off_h[l + 1];
    Put<uint64_t>(&f, uint64_t(e - b));
    f.append(reinterpret_cast<const char*>(ids.data() + b), size_t(e - b) * 4);
    f.append(reinterpret_cast<const char*>(codes.data() + size_t(b) * x->m), size_t(e - b) * x->m);
  }
  Put<uint32_t>(&f, Crc32c(f.data(), f.size()));
  return kOk;
}

// IvfPqIndex::search (ivf_pq.cc:169-222) for a batch: coarse probe (the exact scan over the
// centroids, top nprobe by (dist, list id)), per-query tables, the ADC scan into
// TopK(max(R, k)), then FinishSearch (:28-36): depth 0 truncates, otherwise Rerank.
static int IvfSearch(IvfIndex* x, const float* Q, size_t nq, size_t k, size_t nprobe_req,
                     int rerank, const uint64_t* allow, uint32_t* out_ids, float* out_d,
                     uint64_t* dc_dev, hipStream_t s) {
  Ctx* c = x->ds->ctx;
  if (nq == 0 || k == 0) return kOk;
  if (x->nlist == 0) {  // an empty segment's index returns nothing (ivf_pq.cc:172)
    VDBG_HIP(hipMemsetAsync(out_ids, 0xff, nq * k * 4, s));
    std::vector<float> inf(nq * k, __builtin_inff());
    VDBG_HIP(hipMemcpyAsync(out_d, inf.data(), nq * k * 4, hipMemcpyHostToDevice, s));
    if (dc_dev) VDBG_HIP(hipMemsetAsync(dc_dev, 0, nq * 8, s));
    return hipStreamSynchronize(s) == hipSuccess ? kOk : SetError(kInternal, "sync");
  }
  const size_t nprobe = std::clamp<size_t>(nprobe_req, 1, size_t(x->nlist));
  const size_t depth = rerank < 0 ? std::max<size_t>(10 * k, 100) : size_t(rerank);
  const size_t R = std::max(depth, k);
  if (k > 10000) return SetError(kInvalidArgument, "k must be in 1..10000");
  const bool l2 = x->metric == 0;
  const bool pre = l2 && x->term2 != nullptr;
  const size_t ts = size_t(x->m) * 256;
  // the row-sum scan (k_ivf_scan_rs) also takes each query's per-subspace table maxima
  const bool rs = pre && c->ivf_row_sums && x->rowsum != nullptr && R <= 256 &&
                  (x->m == 4 || x->m == 8 || x->m == 16);
  const bool want_qtab = pre || !l2;
  void* buf = nullptr;
  const size_t scan_bytes = R <= 256 ? IvfScanScratchBytes(nq, nprobe) : 0;
  const size_t bytes = nq * nprobe * 8 + (want_qtab ? nq * ts * 4 : 0) + (rs ? nq * x->m * 4 : 0) +
                       nq * R * 8 + scan_bytes + 4096 + 256;
  VDBG_HIP(hipMallocAsync(&buf, bytes, s));
  char* p = static_cast<char*>(buf);
  auto take = [&](size_t b) {
    char* r = p;
    p += (b + 255) & ~size_t(255);
    return r;
  };
  uint32_t* probe = reinterpret_cast<uint32_t*>(take(nq * nprobe * 4));
  float* probe_d = reinterpret_cast<float*>(take(nq * nprobe * 4));
  float* qtab = want_qtab ? reinterpret_cast<float*>(take(nq * ts * 4)) : nullptr;
  float* qmax = rs ? reinterpret_cast<float*>(take(nq * x->m * 4)) : nullptr;
  uint32_t* ti = R == k ? out_ids : reinterpret_cast<uint32_t*>(take(nq * R * 4));
  float* td = R == k ? out_d : reinterpret_cast<float*>(take(nq * R * 4));
  // the scan's own scratch, allocated here with the rest (no allocation between the coarse
  // probe and the scan)
  void* scan_scratch = scan_bytes != 0 ? take(scan_bytes) : nullptr;
  // the tables depend on the queries alone: queued first, they keep the GPU busy while the
  // host plans and queues the coarse probe
  int rc = kOk;
  if (rs)
    rc = IvfQtabRs(c, Q, x->pd, int(nq), x->cen, x->m, x->dsub, qtab, qmax, s);
  else if (qtab != nullptr)
    rc = IvfQtab(c, Q, x->pd, int(nq), x->cen, x->m, x->dsub, pre ? 1 : 0, qtab, s);
  if (rc == kOk) rc = RunScan(c, &x->coarse_ds->d.src, Q, nq, nprobe, nullptr, probe, probe_d, s);
  if (rc == kOk) {
    IvfScanArgs a{Q, x->pd, x->dim, x->m, x->dsub, x->metric, x->coarse_ds->d.rows, x->cen,
                  x->off, x->ids, x->codes, x->term2, qtab, probe, probe_d, int(nprobe),
                  int(nq), allow, int(R), ti, td, dc_dev, uint64_t(x->nlist), depth > 0 ? 1 : 0};
    a.nlist = uint32_t(x->nlist);
    if (rs) {
      a.rowsum = x->rowsum;
      a.t2abs = x->t2abs;
      a.qmax = qmax;
    }
    rc = R <= 256 ? IvfScan(c, a, s, scan_scratch) : IvfScanDeep(c, a, s);
  }
  if (rc == kOk && depth > 0) {
    rc = Rerank(c, x->ds->rows, x->pd, x->metric, Q, nq, ti, R, k, out_ids, out_d, s,
                &x->ds->src);
  }
  (void)hipFreeAsync(buf, s);
  return rc;
}

}  // namespace vdbg

using namespace vdbg;

extern "C" {

int vdbg_ivfpq_load(vdbg_dataset* ds, const void* file, size_t len, vdbg_ivfpq** out) {
  if (ds == nullptr || out == nullptr || (file == nullptr && len > 0))
    return SetError(kInvalidArgument, "null argument");
  Ctx* c = ds->d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  auto* h = new (std::nothrow) vdbg_ivfpq;
  if (h == nullptr) return SetError(kResourceExhausted, "out of host memory");
  h->x.ds = &ds->d;
  h->x.metric = ds->d.metric;
  int rc = LoadIvf(c, &h->x, static_cast<const uint8_t*>(file), len, c->stream);
  if (rc != kOk) {
    FreeIvf(&h->x);
    delete h;
    return rc;
  }
  ++ds->d.live_indexes;
  *out = h;
  return kOk;
}

int vdbg_ivfpq_save(vdbg_ivfpq* ix, void* buf, size_t cap, size_t* len) {
  if (ix == nullptr || len == nullptr) return SetError(kInvalidArgument, "null argument");
  Ctx* c = ix->x.ds->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  std::string f;
  VDBG_RETURN_IF_ERROR(SaveIvf(c, &ix->x, &f, c->stream));
  *len = f.size();
  if (buf == nullptr) return kOk;
  if (cap < f.size()) return SetError(kInvalidArgument, "buffer too small for the index file");
  std::memcpy(buf, f.data(), f.size());
  return kOk;
}

int vdbg_ivfpq_destroy(vdbg_ivfpq* ix) {
  if (ix == nullptr) return kOk;
  Ctx* c = ix->x.ds->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  (void)hipSetDevice(c->device);
  (void)hipDeviceSynchronize();
  --ix->x.ds->live_indexes;
  FreeIvf(&ix->x);
  delete ix;
  return kOk;
}

int vdbg_ivfpq_info(vdbg_ivfpq* ix, size_t* nlist, size_t* m, int* precomputed_tables) {
  if (ix == nullptr) return SetError(kInvalidArgument, "null index");
  if (nlist) *nlist = size_t(ix->x.nlist);
  if (m) *m = size_t(ix->x.m);
  if (precomputed_tables) *precomputed_tables = ix->x.term2 != nullptr;
  return kOk;
}

int vdbg_ivfpq_list_sizes(vdbg_ivfpq* ix, uint64_t* sizes) {
  if (ix == nullptr || sizes == nullptr) return SetError(kInvalidArgument, "null argument");
  for (int l = 0; l < ix->x.nlist; ++l) sizes[l] = ix->x.off_h[l + 1] - ix->x.off_h[l];
  return kOk;
}

int vdbg_ivfpq_search_device(vdbg_ivfpq* ix, const float* queries, size_t nq, size_t k,
                             size_t nprobe, int rerank, const uint64_t* allow_words,
                             uint32_t* out_ids, float* out_dists, uint64_t* codes_scanned,
                             void* stream) {
  if (ix == nullptr) return SetError(kInvalidArgument, "null index");
  if (nq > 0 && k > 0 && (queries == nullptr || out_ids == nullptr || out_dists == nullptr))
    return SetError(kInvalidArgument, "null pointer");
  Ctx* c = ix->x.ds->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : c->stream;
  return IvfSearch(&ix->x, queries, nq, k, nprobe, rerank, allow_words, out_ids, out_dists,
                   codes_scanned, s);
}

int vdbg_ivfpq_search_host(vdbg_ivfpq* ix, const float* queries, size_t nq, size_t k,
                           size_t nprobe, int rerank, const uint64_t* allow_words,
                           uint32_t* out_ids, float* out_dists, uint64_t* dist_comps) {
  if (ix == nullptr) return SetError(kInvalidArgument, "null index");
  if (dist_comps) std::fill(dist_comps, dist_comps + nq, 0);
  if (nq == 0 || k == 0) return kOk;
  if (queries == nullptr || out_ids == nullptr || out_dists == nullptr)
    return SetError(kInvalidArgument, "null pointer");
  Ctx* c = ix->x.ds->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  IvfIndex* x = &ix->x;
  // IndexSearchStats::distance_computations per query (ivf_pq.cc:199, 241, 243): nlist +
  // codes scanned + candidates re-ranked, returned with the results when asked for
  return StageHost(c, x->ds->n, x->pd, queries, nq, k, allow_words, out_ids, out_dists,
                   dist_comps,
                   [&](const float* dq, const uint64_t* dm, uint32_t* di, float* dd,
                       uint64_t* ddc, hipStream_t st) {
                     return IvfSearch(x, dq, nq, k, nprobe, rerank, dm, di, dd, ddc, st);
                   });
}

}  // extern "C"
