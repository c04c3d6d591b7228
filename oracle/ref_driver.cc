// ref_driver.cc -- a C-ABI driver over the reference's own hot-path sources.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together with the
// reference's src/util, src/distance and src/index files, read where they lie under
// /root/reference, into oracle/_ref/libvdbref.so (never committed).  It is used to pin
// the C restatement (vdb_oracle.c) and, in bench.py, as the timed CPU baseline.  Every
// entry point calls the reference's real code.  The one loop restated here is the
// collection read path of ref_filtered_collection_search (planner.cc needs CRoaring, which
// is absent): it still runs the reference's distance kernels, TopK and NormalizeVector.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <unordered_set>
#include <vector>

#include "distance/distance.h"
#include "index/flat_index.h"
#include "index/hnsw/hnsw_index.h"
#include "index/index.h"
#include "index/quant/ivf_pq.h"
#include "index/quant/kmeans.h"
#include "index/quant/pq.h"
#include "index/quant/sq8.h"
#include "storage/env.h"
#include "util/crc32c.h"
#include "util/dataset.h"
#include "util/thread_pool.h"
#include "util/topk.h"

using namespace vdb;

namespace {

const KernelSet* PickSet(const char* name) {
  if (name == nullptr || *name == '\0') return &Kernels();
  const KernelSet* k = FindKernels(name);
  return k != nullptr ? k : &Kernels();
}

DistFn Fn(const KernelSet* ks, int metric) { return metric == 0 ? ks->l2 : ks->ip; }
Sq8DistFn Sq8Fn(const KernelSet* ks, int metric) { return metric == 0 ? ks->sq8_l2 : ks->sq8_ip; }

class DenseFilter final : public RowFilter {
 public:
  explicit DenseFilter(const uint64_t* w) : w_(w) {}
  bool allowed(InternalId id) const override { return (w_[id >> 6] >> (id & 63)) & 1u; }

 private:
  const uint64_t* w_;
};

class StringSink final : public WritableFile {
 public:
  Status append(std::span<const std::byte> data) override {
    s.append(reinterpret_cast<const char*>(data.data()), data.size());
    return Status::OK();
  }
  Status sync() override { return Status::OK(); }
  Status close() override { return Status::OK(); }
  uint64_t size() const override { return s.size(); }
  std::string s;
};

void WritePadded(const std::vector<Neighbor>& v, size_t k, float* od, uint32_t* oi) {
  for (size_t i = 0; i < k; ++i) {
    od[i] = i < v.size() ? v[i].dist : std::numeric_limits<float>::infinity();
    oi[i] = i < v.size() ? v[i].id : UINT32_MAX;
  }
}

std::string g_last_file;

}  // namespace

extern "C" {

const char* ref_best_kernels() { return Kernels().name; }
int ref_has_kernels(const char* name) { return FindKernels(name) != nullptr; }

float ref_l2(const char* ks, const float* a, const float* b, size_t d) { return PickSet(ks)->l2(a, b, d); }
float ref_dot(const char* ks, const float* a, const float* b, size_t d) { return PickSet(ks)->dot(a, b, d); }
float ref_sq8_l2(const char* ks, const float* q, const uint8_t* c, const float* vmin,
                 const float* scale, size_t d) {
  return PickSet(ks)->sq8_l2(q, c, vmin, scale, d);
}
float ref_sq8_ip(const char* ks, const float* q, const uint8_t* c, const float* vmin,
                 const float* scale, size_t d) {
  return PickSet(ks)->sq8_ip(q, c, vmin, scale, d);
}
float ref_l2sq_any(const float* a, const float* b, size_t d) { return L2SqAny(a, b, d); }
float ref_dot_any(const float* a, const float* b, size_t d) { return DotAny(a, b, d); }

size_t ref_topk(const float* dist, const uint32_t* id, size_t n, size_t k, float* od,
                uint32_t* oi) {
  TopK top(k);
  for (size_t i = 0; i < n; ++i) top.push(dist[i], id[i]);
  auto s = top.sorted();
  for (size_t i = 0; i < s.size(); ++i) {
    od[i] = s[i].dist;
    oi[i] = s[i].id;
  }
  return s.size();
}

// FlatIndex::search semantics (FlatSearch without a pool) with the named kernel set, one
// call per query, queries fanned over a ThreadPool as CollectionImpl::SearchBatch does.
void ref_flat_search_batch(const char* ks, int metric, const float* base, size_t rows,
                           size_t dim, size_t pd, const float* queries, size_t nq, size_t k,
                           const uint64_t* allow, float* od, uint32_t* oi, int nthreads) {
  VectorView v{base, rows, dim, pd};
  DistFn fn = Fn(PickSet(ks), metric);
  DenseFilter f(allow);
  ThreadPool pool(nthreads <= 0 ? 1 : static_cast<size_t>(nthreads));
  pool.parallel_for(0, nq, [&](size_t q) {
    std::vector<Neighbor> out;
    FlatSearch(v, fn, queries + q * pd, k, allow ? &f : nullptr, out, nullptr);
    WritePadded(out, k, od + q * k, oi + q * k);
  });
}

// The reference's FlatIndex class itself (default kernel set), fanned over a pool: the
// CPU baseline bench.py times.
void ref_flat_index_batch(int metric, const float* base, size_t rows, size_t dim, size_t pd,
                          const float* queries, size_t nq, size_t k, float* od, uint32_t* oi,
                          int nthreads) {
  VectorView v{base, rows, dim, pd};
  FlatIndex idx(static_cast<Metric>(metric), v);
  ThreadPool pool(nthreads <= 0 ? 1 : static_cast<size_t>(nthreads));
  SearchParams p;
  pool.parallel_for(0, nq, [&](size_t q) {
    std::vector<Neighbor> out;
    idx.search(queries + q * pd, k, p, nullptr, out, nullptr);
    WritePadded(out, k, od + q * k, oi + q * k);
  });
}

// FlatSearchBatch (flat_index.cc:41-68).
void ref_flat_search_blocked(const char* ks, int metric, const float* base, size_t rows,
                             size_t dim, size_t pd, const float* queries, size_t nq, size_t k,
                             float* od, uint32_t* oi, int nthreads) {
  VectorView v{base, rows, dim, pd};
  ThreadPool pool(nthreads <= 0 ? 1 : static_cast<size_t>(nthreads));
  std::vector<std::vector<Neighbor>> out;
  FlatSearchBatch(v, Fn(PickSet(ks), metric), queries, nq, k, out, &pool);
  for (size_t q = 0; q < nq; ++q) WritePadded(out[q], k, od + q * k, oi + q * k);
}

void ref_rerank(const char* ks, int metric, const float* base, size_t rows, size_t dim,
                size_t pd, const float* q, const uint32_t* cand, size_t ncand, size_t k,
                float* od, uint32_t* oi) {
  VectorView v{base, rows, dim, pd};
  std::vector<Neighbor> c(ncand), out;
  for (size_t i = 0; i < ncand; ++i) c[i] = Neighbor{0.f, cand[i]};
  Rerank(v, Fn(PickSet(ks), metric), q, c, k, out, nullptr);
  WritePadded(out, k, od, oi);
}

void ref_sq8_train_encode(const float* base, size_t rows, size_t dim, size_t pd, float* vmin,
                          float* scale, uint8_t* codes) {
  VectorView v{base, rows, dim, pd};
  Sq8Quantizer sq;
  sq.train(v);
  std::memcpy(vmin, sq.vmin(), pd * sizeof(float));
  std::memcpy(scale, sq.scale(), pd * sizeof(float));
  if (codes != nullptr)
    for (size_t r = 0; r < rows; ++r) sq.encode(v.row(r), codes + r * pd);
}

// HnswSq8Index::build + save (src/index/hnsw/hnsw_index.cc:66-79, 108-115): the VDBHSQ81
// file a segment of that index type holds.  Returns the file size; writes it when it fits
// in cap bytes.
size_t ref_hnsw_sq8_file(int metric, const float* base, size_t rows, size_t dim, size_t pd,
                         size_t M, size_t ef_construction, uint64_t seed, char* buf, size_t cap) {
  VectorView v{base, rows, dim, pd};
  IndexOptions o;
  o.type = IndexType::HnswSq8;
  o.M = M;
  o.ef_construction = ef_construction;
  o.seed = seed;
  HnswSq8Index idx(o, static_cast<Metric>(metric), v);
  if (!idx.build(nullptr).ok()) return 0;
  StringSink sink;
  if (!idx.save(sink).ok()) return 0;
  if (buf != nullptr && sink.s.size() <= cap) std::memcpy(buf, sink.s.data(), sink.s.size());
  return sink.s.size();
}

// HnswIndex::build + save (src/index/hnsw/hnsw_index.cc:18-40): the VDBHNSW1 file a segment
// of vdb's default index type (IndexType::Hnsw, options.h:22) holds.  Returns the file size;
// writes it when it fits in cap bytes.
size_t ref_hnsw_file(int metric, const float* base, size_t rows, size_t dim, size_t pd,
                     size_t M, size_t ef_construction, uint64_t seed, char* buf, size_t cap) {
  VectorView v{base, rows, dim, pd};
  IndexOptions o;
  o.type = IndexType::Hnsw;
  o.M = M;
  o.ef_construction = ef_construction;
  o.seed = seed;
  HnswIndex idx(o, static_cast<Metric>(metric), v);
  if (!idx.build(nullptr).ok()) return 0;
  StringSink sink;
  if (!idx.save(sink).ok()) return 0;
  if (buf != nullptr && sink.s.size() <= cap) std::memcpy(buf, sink.s.data(), sink.s.size());
  return sink.s.size();
}

// LoadIndex of a VDBHNSW1 file (index.cc:63-67) and HnswIndex::search per query, under a
// RowFilter given as dense words (nullable).  Returns 0, or 1 when the file does not load.
int ref_hnsw_search_batch(int metric, const char* file, size_t file_len, const float* base,
                          size_t rows, size_t dim, size_t pd, const float* queries, size_t nq,
                          size_t k, size_t ef, const uint64_t* allow_words, float* od,
                          uint32_t* oi, uint64_t* dc, int nthreads) {
  VectorView v{base, rows, dim, pd};
  IndexOptions o;
  o.type = IndexType::Hnsw;
  auto idx = LoadIndex(std::string_view(file, file_len), o, static_cast<Metric>(metric), v);
  if (!idx.ok() || (*idx)->type() != IndexType::Hnsw) return 1;
  const Index& ix = **idx;
  SearchParams p;
  p.ef = ef;
  DenseFilter filt(allow_words);
  ThreadPool pool(nthreads <= 0 ? 1 : static_cast<size_t>(nthreads));
  pool.parallel_for(0, nq, [&](size_t qi) {
    std::vector<Neighbor> out;
    IndexSearchStats st;
    ix.search(queries + qi * pd, k, p, allow_words != nullptr ? &filt : nullptr, out, &st);
    WritePadded(out, k, od + qi * k, oi + qi * k);
    if (dc != nullptr) dc[qi] = st.distance_computations;
  });
  return 0;
}

// ref_hnsw_sq8_file with the build on a thread pool of nthreads (HnswSq8Index::build(pool),
// as vdb builds a segment's graph): the graph depends on the threads' interleaving, so two
// builds may differ; the file is what the segment would hold.
size_t ref_hnsw_sq8_file_mt(int metric, const float* base, size_t rows, size_t dim, size_t pd,
                            size_t M, size_t ef_construction, uint64_t seed, int nthreads,
                            const char** file) {
  VectorView v{base, rows, dim, pd};
  IndexOptions o;
  o.type = IndexType::HnswSq8;
  o.M = M;
  o.ef_construction = ef_construction;
  o.seed = seed;
  HnswSq8Index idx(o, static_cast<Metric>(metric), v);
  ThreadPool pool(nthreads <= 0 ? 1 : static_cast<size_t>(nthreads));
  if (!idx.build(&pool).ok()) return 0;
  StringSink sink;
  if (!idx.save(sink).ok()) return 0;
  g_last_file = std::move(sink.s);
  *file = g_last_file.data();
  return g_last_file.size();
}

// LoadIndex of a VDBHSQ81 file (index.cc:38-87) and HnswSq8Index::search
// (src/index/hnsw/hnsw_index.cc:82-100) per query: graph beam over the codes with the
// reference's own kernel set, then Rerank.  allow_words (nullable) is the RowFilter (bit r of
// word r / 64 = row r allowed).  Returns 0, or 1 when the file does not load.
int ref_hnsw_sq8_search_batch(int metric, const char* file, size_t file_len, const float* base,
                              size_t rows, size_t dim, size_t pd, const float* queries,
                              size_t nq, size_t k, size_t ef, int rerank,
                              const uint64_t* allow_words, float* od, uint32_t* oi,
                              uint64_t* dc, int nthreads) {
  VectorView v{base, rows, dim, pd};
  IndexOptions o;
  o.type = IndexType::HnswSq8;
  auto idx = LoadIndex(std::string_view(file, file_len), o, static_cast<Metric>(metric), v);
  if (!idx.ok()) return 1;
  const Index& ix = **idx;
  SearchParams p;
  p.ef = ef;
  p.rerank = rerank;
  DenseFilter filt(allow_words);
  ThreadPool pool(nthreads <= 0 ? 1 : static_cast<size_t>(nthreads));
  pool.parallel_for(0, nq, [&](size_t qi) {
    std::vector<Neighbor> out;
    IndexSearchStats st;
    ix.search(queries + qi * pd, k, p, allow_words != nullptr ? &filt : nullptr, out, &st);
    WritePadded(out, k, od + qi * k, oi + qi * k);
    if (dc != nullptr) dc[qi] = st.distance_computations;
  });
  return 0;
}

// PqFlatIndex::build + save (src/index/quant/ivf_pq.cc:45-57, 81-87) through CreateIndex
// (index.cc:16-36): the VDBPQFL1 file.  Returns its size (0 on failure); writes it when it
// fits in cap bytes.
size_t ref_pqflat_file(int metric, const float* base, size_t rows, size_t dim, size_t pd,
                       size_t m, uint64_t seed, size_t max_points, char* buf, size_t cap) {
  VectorView v{base, rows, dim, pd};
  IndexOptions o;
  o.type = IndexType::PqFlat;
  o.pq_m = m;
  o.seed = seed;
  o.max_train_points_per_centroid = max_points;
  auto idx = CreateIndex(o, static_cast<Metric>(metric), v);
  if (!idx.ok() || !(*idx)->build(nullptr).ok()) return 0;
  StringSink sink;
  if (!(*idx)->save(sink).ok()) return 0;
  if (buf != nullptr && sink.s.size() <= cap) std::memcpy(buf, sink.s.data(), sink.s.size());
  return sink.s.size();
}

// LoadIndex of a VDBPQFL1 file and PqFlatIndex::search (ivf_pq.cc:59-79) per query.
int ref_pqflat_search_batch(int metric, const char* file, size_t file_len, const float* base,
                            size_t rows, size_t dim, size_t pd, const float* queries, size_t nq,
                            size_t k, int rerank, const uint64_t* allow_words, float* od,
                            uint32_t* oi, uint64_t* dc, int nthreads) {
  VectorView v{base, rows, dim, pd};
  IndexOptions o;
  o.type = IndexType::PqFlat;
  auto idx = LoadIndex(std::string_view(file, file_len), o, static_cast<Metric>(metric), v);
  if (!idx.ok()) return 1;
  const Index& ix = **idx;
  SearchParams p;
  p.rerank = rerank;
  DenseFilter filt(allow_words);
  ThreadPool pool(nthreads <= 0 ? 1 : static_cast<size_t>(nthreads));
  pool.parallel_for(0, nq, [&](size_t qi) {
    std::vector<Neighbor> out;
    IndexSearchStats st;
    ix.search(queries + qi * pd, k, p, allow_words != nullptr ? &filt : nullptr, out, &st);
    WritePadded(out, k, od + qi * k, oi + qi * k);
    if (dc != nullptr) dc[qi] = st.distance_computations;
  });
  return 0;
}

// SQ8 scan + rerank composed from the reference's parts (Sq8 kernel into TopK, Rerank).
void ref_sq8_search_batch(const char* ks, int metric, const float* base, const uint8_t* codes,
                          size_t rows, size_t dim, size_t pd, const float* vmin,
                          const float* scale, const float* queries, size_t nq, size_t k,
                          size_t depth, float* od, uint32_t* oi, int nthreads) {
  VectorView v{base, rows, dim, pd};
  const KernelSet* set = PickSet(ks);
  Sq8DistFn sfn = Sq8Fn(set, metric);
  DistFn fn = Fn(set, metric);
  ThreadPool pool(nthreads <= 0 ? 1 : static_cast<size_t>(nthreads));
  pool.parallel_for(0, nq, [&](size_t qi) {
    const float* q = queries + qi * pd;
    TopK top(std::max(depth, k));
    for (size_t r = 0; r < rows; ++r)
      top.push(sfn(q, codes + r * pd, vmin, scale, pd), static_cast<InternalId>(r));
    std::vector<Neighbor> out;
    if (depth == 0) {
      top.sorted_into(&out);
      if (out.size() > k) out.resize(k);
    } else {
      Rerank(v, fn, q, top.sorted(), k, out, nullptr);
    }
    WritePadded(out, k, od + qi * k, oi + qi * k);
  });
}

static std::string PqBytes(const float* centroids, size_t dim, size_t m) {
  std::string b;
  PutU32(&b, static_cast<uint32_t>(dim));
  PutU32(&b, static_cast<uint32_t>(m));
  PutBytes(&b, centroids, m * ProductQuantizer::kCentroids * (dim / m) * sizeof(float));
  return b;
}

static bool LoadPq(const float* centroids, size_t dim, size_t m, ProductQuantizer* pq) {
  std::string b = PqBytes(centroids, dim, m);
  ByteReader r(b);
  return pq->deserialize(r);
}

int ref_pq_train(const float* data, size_t n, size_t dim, size_t stride, size_t m,
                 uint64_t seed, size_t max_points, float* centroids) {
  ProductQuantizer pq(dim, m);
  KMeansOptions o;
  o.seed = seed;
  o.max_points_per_centroid = max_points;
  if (!pq.train(data, n, stride, o, nullptr).ok()) return 1;
  const size_t dsub = dim / m;
  for (size_t j = 0; j < m; ++j)
    for (size_t c = 0; c < ProductQuantizer::kCentroids; ++c)
      std::memcpy(centroids + (j * ProductQuantizer::kCentroids + c) * dsub, pq.centroid(j, c),
                  dsub * sizeof(float));
  return 0;
}

int ref_pq_encode(const float* centroids, size_t dim, size_t m, const float* x, size_t n,
                  size_t stride, uint8_t* codes) {
  ProductQuantizer pq;
  if (!LoadPq(centroids, dim, m, &pq)) return 1;
  for (size_t i = 0; i < n; ++i) pq.encode(x + i * stride, codes + i * m);
  return 0;
}

int ref_pq_table(const float* centroids, size_t dim, size_t m, const float* q, int metric,
                 float* table) {
  ProductQuantizer pq;
  if (!LoadPq(centroids, dim, m, &pq)) return 1;
  pq.compute_table(q, static_cast<Metric>(metric), table);
  return 0;
}

float ref_pq_adc(const float* centroids, size_t dim, size_t m, const float* table,
                 const uint8_t* code) {
  ProductQuantizer pq;
  if (!LoadPq(centroids, dim, m, &pq)) return -1.f;
  return pq.adc(table, code);
}

int ref_kmeans(const float* data, size_t n, size_t d, size_t stride, size_t k, size_t iters,
               uint64_t seed, size_t max_points, int kmeanspp, float* centroids) {
  KMeansOptions o;
  o.iters = iters;
  o.seed = seed;
  o.max_points_per_centroid = max_points;
  o.kmeanspp = kmeanspp != 0;
  std::vector<float> cen;
  if (!KMeans(data, n, d, stride, k, o, nullptr, &cen).ok()) return 1;
  std::memcpy(centroids, cen.data(), cen.size() * sizeof(float));
  return 0;
}

void ref_assign_nearest(const float* data, size_t n, size_t d, size_t stride,
                        const float* centroids, size_t k, uint32_t* assign, float* dist) {
  AssignNearest(data, n, d, stride, centroids, k, nullptr, assign, dist);
}

// Builds an IvfPqIndex over the rows and returns its VDBIVFP1 file (Index::save).  The
// bytes stay valid until the next call.
int ref_ivfpq_build(int metric, const float* base, size_t rows, size_t dim, size_t pd,
                    size_t nlist, size_t m, uint64_t seed, size_t max_points,
                    const char** file, size_t* file_len, int nthreads) {
  VectorView v{base, rows, dim, pd};
  IndexOptions o;
  o.type = IndexType::IvfPq;
  o.pq_m = m;
  o.nlist = nlist;
  o.seed = seed;
  o.max_train_points_per_centroid = max_points;
  auto idx = CreateIndex(o, static_cast<Metric>(metric), v);
  if (!idx.ok()) return 1;
  ThreadPool pool(nthreads <= 0 ? 1 : static_cast<size_t>(nthreads));
  if (!(*idx)->build(&pool).ok()) return 2;
  StringSink sink;
  if (!(*idx)->save(sink).ok()) return 3;
  g_last_file = std::move(sink.s);
  *file = g_last_file.data();
  *file_len = g_last_file.size();
  return 0;
}

// Loads a VDBIVFP1 file with LoadIndex and runs IvfPqIndex::search for every query.
int ref_ivfpq_search_batch(int metric, const char* file, size_t file_len, const float* base,
                           size_t rows, size_t dim, size_t pd, const float* queries, size_t nq,
                           size_t k, size_t nprobe, int rerank, const uint64_t* allow,
                           float* od, uint32_t* oi, uint64_t* dc, int nthreads) {
  VectorView v{base, rows, dim, pd};
  IndexOptions o;
  o.type = IndexType::IvfPq;
  auto idx = LoadIndex(std::string_view(file, file_len), o, static_cast<Metric>(metric), v);
  if (!idx.ok()) return 1;
  SearchParams p;
  p.nprobe = nprobe;
  p.rerank = rerank;
  DenseFilter f(allow);
  ThreadPool pool(nthreads <= 0 ? 1 : static_cast<size_t>(nthreads));
  const Index& ix = **idx;
  pool.parallel_for(0, nq, [&](size_t q) {
    std::vector<Neighbor> out;
    IndexSearchStats st;
    ix.search(queries + q * pd, k, p, allow ? &f : nullptr, out, &st);
    WritePadded(out, k, od + q * k, oi + q * k);
    if (dc != nullptr) dc[q] = st.distance_computations;
  });
  return 0;
}

int ref_normalize(float* v, size_t dim) { return NormalizeVector(v, dim) ? 1 : 0; }
uint32_t ref_crc32c(const void* data, size_t n) { return crc32c::Value(data, n); }

// The filtered read path of CollectionImpl::Search over disk segments with flat indexes,
// per query and fanned over a pool as SearchBatch does (collection_impl.cc:1121-1135):
// PrepareQuery (:1023-1034, with the reference's NormalizeVector), for every segment the
// prefilter exact scan ExactOverBitmap (planner.cc:31-38: allowed rows ascending, the
// default kernel set's DistFn, the reference's TopK), then the merge of :1076-1112
// (sort by (dist, part, row), first hit per external id).  The planner itself and the
// roaring bitmaps need libraries absent here, so the allowed rows arrive as dense words
// and this loop restates theirs.  Returns 1 (InvalidArgument) for a query PrepareQuery
// rejects.
int ref_filtered_collection_search(int metric, const float* const* seg_rows,
                                   const size_t* seg_n, size_t nseg, size_t dim, size_t pd,
                                   const uint64_t* const* allow, const uint64_t* ext,
                                   const float* raw_queries, size_t nq, size_t k,
                                   uint64_t* out_ext, float* out_d, int nthreads) {
  DistFn fn = Fn(&Kernels(), metric);
  std::vector<size_t> seg_off(nseg + 1, 0);
  for (size_t p = 0; p < nseg; ++p) seg_off[p + 1] = seg_off[p] + seg_n[p];
  std::atomic<int> bad{0};
  ThreadPool pool(nthreads <= 0 ? 1 : static_cast<size_t>(nthreads));
  pool.parallel_for(0, nq, [&](size_t qi) {
    std::vector<float> q(pd, 0.f);
    const float* v = raw_queries + qi * dim;
    for (size_t i = 0; i < dim; ++i) {
      if (!std::isfinite(v[i])) {
        bad = 1;
        return;
      }
      q[i] = v[i];
    }
    if (metric == 2 && !NormalizeVector(q.data(), dim)) {
      bad = 1;
      return;
    }
    struct Cand {
      float dist;
      uint32_t part;
      uint32_t row;
    };
    std::vector<Cand> all;
    std::vector<Neighbor> hits;
    for (size_t p = 0; p < nseg; ++p) {
      TopK top(k);
      const uint64_t* w = allow[p];
      for (size_t wi = 0; wi < (seg_n[p] + 63) / 64; ++wi) {
        uint64_t bits = w[wi];
        while (bits != 0) {
          const uint32_t r = static_cast<uint32_t>(wi * 64 + __builtin_ctzll(bits));
          bits &= bits - 1;
          if (r >= seg_n[p]) break;
          top.push(fn(q.data(), seg_rows[p] + static_cast<size_t>(r) * pd, pd), r);
        }
      }
      top.sorted_into(&hits);
      for (const Neighbor& h : hits) all.push_back({h.dist, static_cast<uint32_t>(p), h.id});
    }
    std::sort(all.begin(), all.end(), [](const Cand& a, const Cand& b) {
      if (a.dist != b.dist) return a.dist < b.dist;
      if (a.part != b.part) return a.part < b.part;
      return a.row < b.row;
    });
    std::unordered_set<uint64_t> seen;
    size_t out = 0;
    for (const Cand& c : all) {
      const uint64_t e = ext[seg_off[c.part] + c.row];
      if (!seen.insert(e).second) continue;
      out_ext[qi * k + out] = e;
      out_d[qi * k + out] = c.dist;
      if (++out >= k) break;
    }
    for (; out < k; ++out) {
      out_ext[qi * k + out] = UINT64_MAX;
      out_d[qi * k + out] = std::numeric_limits<float>::infinity();
    }
  });
  return bad ? 1 : 0;
}

}  // extern "C"
