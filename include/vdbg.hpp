// vdbg.hpp -- C++20 host classes over the C ABI in vdbg.h, shaped like vdb's index interface.
//
// vdb's search path is `class Index` (src/index/index.h:36-55): search(q, k, params, filter,
// out, stats) per query, with SearchParams (include/vdb/options.h:59-67), RowFilter
// (index.h:23-27), IndexSearchStats (index.h:29-32) and results as ascending Neighbor
// (include/vdb/types.h:19-28).  The classes below keep those names, argument meanings and
// result order so that a vdb Index adapter (or any C++ caller) is a thin forwarding layer:
//
//   GpuFlatIndex   FlatIndex (src/index/flat_index.h:20-39) + FlatSearchBatch (:17-18)
//   GpuSq8Index    the SQ8 codes and scan of HnswSq8Index (src/index/hnsw/hnsw_index.h:44-95)
//                  with the graph beam replaced by an exhaustive scan
//   GpuIvfPqIndex  IvfPqIndex (src/index/quant/ivf_pq.h:42-81), file format VDBIVFP1
//   SearchSegments the read path of CollectionImpl::Search over flat segments
//                  (src/engine/collection_impl.cc:1036-1112): PrepareQuery, per-segment
//                  filtered scan, (dist, part, row) merge with one hit per external id
//   GpuSegment     Segment::Open (src/storage/segment_reader.cc:20-122) straight into HBM:
//                  vectors.f32, ids.u64, the index file by magic, deletes-<n>.roar
//   SearchCollection  CollectionImpl::SearchBatch over GpuSegments of any index type with
//                  SearchDiskSegment's plan per segment (src/engine/planner.cc:42-129), one
//                  device batch and one merge
//   Coalescer      concurrent Index::search calls of one index (one query each, from vdb's
//                  pool workers) answered as device batches, each call's result unchanged
//
// Differences, all forced by the device: filters are dense bitmasks (DenseRowFilter) rather
// than a virtual allowed() per row; searches return a Status (vdb's return void), since a
// device call can fail; every search also has a batched form.  Header-only; link libvdbg.so.
#pragma once

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <memory>
#include <span>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

#include "vdbg.h"

namespace vdbg {

// ---------------------------------------------------------------- vocabulary (vdb's)

enum class Metric : uint8_t { L2 = 0, InnerProduct = 1, Cosine = 2 };  // types.h:13-17
using InternalId = uint32_t;
using VectorId = uint64_t;
constexpr InternalId kNoRow = 0xffffffffu;

// Neighbor::operator< (types.h:23-25): distance, then id.
struct Neighbor {
  float dist = 0.f;
  InternalId id = 0;
  bool operator<(const Neighbor& o) const { return dist < o.dist || (dist == o.dist && id < o.id); }
  bool operator==(const Neighbor& o) const = default;
};

constexpr size_t PaddedDim(size_t dim) { return (dim + 15) / 16 * 16; }  // types.h:30-32

enum class FilterStrategy : uint8_t { Auto = 0, PreFilter = 1, Graph = 2, PostFilter = 3 };  // options.h:57

// SearchParams (options.h:59-67).
struct SearchParams {
  size_t ef = 64;      // SQ8: depth = max(ef, k) when rerank < 0 (hnsw_index.cc:88)
  size_t nprobe = 16;  // IVF lists to scan
  int rerank = -1;     // -1 = auto, 0 = none
  FilterStrategy strategy = FilterStrategy::Auto;  // the planner's (planner.cc:66-80)
  size_t prefilter_threshold = 10000;              // matches at or below -> exact
  size_t post_filter_alpha = 10;                   // post filter searches k * alpha
};

// The fields of IndexOptions (options.h:20-33) the builds read, plus the k-means iteration
// count (KMeansOptions::iters, src/index/quant/kmeans.h:13-20; vdb's build uses 25).
struct IndexOptions {
  size_t pq_m = 16;
  size_t nlist = 1024;
  size_t max_train_points_per_centroid = 256;
  uint64_t seed = 42;
  size_t kmeans_iters = 25;
};

struct IndexSearchStats {  // index.h:29-32
  uint64_t distance_computations = 0;
  size_t ef = 0;
};

// A segment's float rows: VectorView (src/util/aligned_buffer.h:56-63).
struct VectorView {
  const float* data = nullptr;
  size_t rows = 0, dim = 0, padded_dim = 0;
  const float* row(size_t r) const { return data + r * padded_dim; }
};

// vdb::Status with the same code numbering (include/vdb/status.h:14-26).
class Status {
 public:
  Status() = default;
  Status(int code, std::string msg) : code_(code), msg_(std::move(msg)) {}
  static Status OK() { return {}; }
  // The status of a C ABI call: its return code and the thread's last message.
  static Status FromCall(int rc) { return rc == VDBG_OK ? Status() : Status(rc, vdbg_last_error()); }
  bool ok() const { return code_ == VDBG_OK; }
  int code() const { return code_; }
  const std::string& message() const { return msg_; }
  std::string ToString() const { return ok() ? "OK" : std::to_string(code_) + ": " + msg_; }

 private:
  int code_ = VDBG_OK;
  std::string msg_;
};

#define VDBG_CXX_RETURN_IF_ERROR(expr)   \
  do {                                   \
    ::vdbg::Status s_ = (expr);          \
    if (!s_.ok()) return s_;             \
  } while (0)

// RowFilter as a dense bitmask: bit r of word r / 64 set = row r allowed.  DeleteFilter
// (src/engine/planner.cc:12-19) is FromDeleted(DeleteBits words); BitmapFilter (:21-29) is the
// roaring result minus deletes, expanded with Allow().
class DenseRowFilter {
 public:
  DenseRowFilter() = default;
  explicit DenseRowFilter(size_t rows, bool all = false)
      : rows_(rows), words_((rows + 63) / 64, all ? ~uint64_t(0) : 0) {}
  static DenseRowFilter FromWords(const uint64_t* words, size_t rows) {
    DenseRowFilter f(rows);
    std::memcpy(f.words_.data(), words, f.words_.size() * sizeof(uint64_t));
    return f;
  }
  // A view of words the caller keeps alive (no copy); Allow/Deny copy them first.
  static DenseRowFilter View(const uint64_t* words, size_t rows) {
    DenseRowFilter f;
    f.rows_ = rows;
    f.view_ = words;
    return f;
  }
  // Every row not set in the deletion words (DeleteBits::test, delete_bits.h:50-55).
  static DenseRowFilter FromDeleted(const uint64_t* deleted_words, size_t rows) {
    DenseRowFilter f(rows);
    for (size_t i = 0; i < f.words_.size(); ++i) f.words_[i] = ~deleted_words[i];
    return f;
  }
  void Allow(InternalId r) {
    own();
    words_[r >> 6] |= uint64_t(1) << (r & 63);
  }
  void Deny(InternalId r) {
    own();
    words_[r >> 6] &= ~(uint64_t(1) << (r & 63));
  }
  bool allowed(InternalId r) const { return r < rows_ && ((words()[r >> 6] >> (r & 63)) & 1u); }
  const uint64_t* words() const { return view_ != nullptr ? view_ : words_.data(); }
  size_t rows() const { return rows_; }

 private:
  void own() {
    if (view_ != nullptr) {
      words_.assign(view_, view_ + (rows_ + 63) / 64);
      view_ = nullptr;
    }
  }
  size_t rows_ = 0;
  std::vector<uint64_t> words_;
  const uint64_t* view_ = nullptr;
};

// ---------------------------------------------------------------- device

// One GPU, its stream and workspace (vdbg_ctx).  Calls on one Device are serialised; for
// concurrent one-query calls on one index use a Coalescer, or one Device per thread.
class Device {
 public:
  static Status Open(int ordinal, std::unique_ptr<Device>* out) {
    vdbg_ctx* c = nullptr;
    VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(vdbg_ctx_create(ordinal, &c)));
    out->reset(new Device(c));
    return Status::OK();
  }
  ~Device() { vdbg_ctx_destroy(ctx_); }
  Device(const Device&) = delete;
  Device& operator=(const Device&) = delete;
  vdbg_ctx* get() const { return ctx_; }
  // Queries whose certificate failed in the last flat/SQ8 search and were re-scanned exactly.
  uint64_t last_fallbacks() const {
    uint64_t n = 0;
    vdbg_last_fallbacks(ctx_, &n);
    return n;
  }
  // Ranking on fp16 MFMA (default on; results are identical either way).  Datasets created
  // while it is on keep an fp16 copy of their rows.
  Status set_fp16_gemm(bool enable) {
    return Status::FromCall(vdbg_ctx_set_fp16_gemm(ctx_, enable ? 1 : 0));
  }
  // Ranking of integer rows spanning at most 256 values on int8 MFMA (default on; results
  // are identical either way).
  Status set_int8_gemm(bool enable) {
    return Status::FromCall(vdbg_ctx_set_int8_gemm(ctx_, enable ? 1 : 0));
  }
  // Smallest rows x queries x padded_dim of a float-row batch ranked on int8 MFMA.
  Status set_int8_float_min_work(double work) {
    return Status::FromCall(vdbg_ctx_set_int8_float_min_work(ctx_, work));
  }
  // The distance kernel set exact distances follow ("scalar", "avx2", "avx512").
  Status set_kernels(const char* name) { return Status::FromCall(vdbg_ctx_set_kernels(ctx_, name)); }

 private:
  explicit Device(vdbg_ctx* c) : ctx_(c) {}
  vdbg_ctx* ctx_;
};

namespace detail {

// [nq][k] padded ids/dists -> one ascending Neighbor list per query (padding dropped).
inline void Unpack(const std::vector<uint32_t>& ids, const std::vector<float>& d, size_t nq,
                   size_t k, std::vector<std::vector<Neighbor>>& out) {
  out.assign(nq, {});
  for (size_t q = 0; q < nq; ++q) {
    auto& o = out[q];
    o.reserve(k);
    for (size_t i = 0; i < k && ids[q * k + i] != kNoRow; ++i) o.push_back({d[q * k + i], ids[q * k + i]});
  }
}

struct DatasetDeleter {
  void operator()(vdbg_dataset* d) const { vdbg_dataset_destroy(d); }
};
using DatasetPtr = std::unique_ptr<vdbg_dataset, DatasetDeleter>;

inline Status MakeDataset(Device& dev, Metric m, const VectorView& v, DatasetPtr* out) {
  vdbg_dataset* d = nullptr;
  VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(
      vdbg_dataset_create(dev.get(), v.data, v.rows, v.dim, v.padded_dim, int(m), &d)));
  out->reset(d);
  return Status::OK();
}

}  // namespace detail

// ---------------------------------------------------------------- flat

// FlatIndex: exact search over the resident rows (flat_index.cc:11-39, 70-83).
class GpuFlatIndex {
 public:
  static Status Create(Device& dev, Metric metric, const VectorView& v,
                       std::unique_ptr<GpuFlatIndex>* out) {
    detail::DatasetPtr d;
    VDBG_CXX_RETURN_IF_ERROR(detail::MakeDataset(dev, metric, v, &d));
    out->reset(new GpuFlatIndex(dev, metric, v, std::move(d)));
    return Status::OK();
  }
  const char* type() const { return "flat"; }
  Status build() { return Status::OK(); }  // nothing to train: rows are resident
  size_t size() const { return view_.rows; }
  size_t memory_bytes() const { return 0; }  // FlatIndex holds no structures beyond the rows
  Metric metric() const { return metric_; }
  const VectorView& view() const { return view_; }
  vdbg_dataset* dataset() const { return ds_.get(); }

  // FlatIndex::search: the k nearest allowed rows, closest first; stats as :75-76 counts.
  Status search(const float* q, size_t k, const SearchParams& p, const DenseRowFilter* filter,
                std::vector<Neighbor>& out, IndexSearchStats* stats) const {
    std::vector<std::vector<Neighbor>> all;
    VDBG_CXX_RETURN_IF_ERROR(search_batch(q, 1, k, p, filter, all, stats));
    out = std::move(all[0]);
    return Status::OK();
  }
  // FlatSearchBatch (flat_index.cc:41-68): the same results as search() per query.
  Status search_batch(const float* queries, size_t nq, size_t k, const SearchParams&,
                      const DenseRowFilter* filter, std::vector<std::vector<Neighbor>>& out,
                      IndexSearchStats* stats) const {
    std::vector<uint32_t> ids(nq * k);
    std::vector<float> d(nq * k);
    uint64_t dc = 0;
    VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(vdbg_flat_search_host(
        ds_.get(), queries, nq, k, filter ? filter->words() : nullptr, ids.data(), d.data(), &dc)));
    detail::Unpack(ids, d, nq, k, out);
    if (stats) stats->distance_computations += dc;
    return Status::OK();
  }
  // Rerank (src/index/index.cc:89-95) of candidates found elsewhere, e.g. by vdb's CPU
  // HNSW-SQ8 beam or an IVF-PQ top-R: cand is [nq][depth] rows (kNoRow = none); the exact
  // distances on the resident rows, the k best per query; stats add the candidate counts.
  Status rerank_batch(const float* queries, size_t nq, const uint32_t* cand, size_t depth,
                      size_t k, std::vector<std::vector<Neighbor>>& out,
                      IndexSearchStats* stats) const {
    std::vector<uint32_t> ids(nq * k);
    std::vector<float> d(nq * k);
    std::vector<uint64_t> dc(nq);
    VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(vdbg_rerank_host(
        ds_.get(), queries, nq, cand, depth, k, ids.data(), d.data(), dc.data())));
    detail::Unpack(ids, d, nq, k, out);
    if (stats)
      for (uint64_t c : dc) stats->distance_computations += c;
    return Status::OK();
  }

 private:
  GpuFlatIndex(Device& dev, Metric m, const VectorView& v, detail::DatasetPtr d)
      : dev_(dev), metric_(m), view_(v), ds_(std::move(d)) {}
  Device& dev_;
  Metric metric_;
  VectorView view_;
  detail::DatasetPtr ds_;
};

// ---------------------------------------------------------------- SQ8

// HnswSq8Index's quantized scan (hnsw_index.h:44-95, hnsw_index.cc:66-100) without the graph:
// build() trains Sq8Quantizer on the rows and encodes them; search scores every code with
// the asymmetric SQ8 distance into TopK(depth), depth = rerank < 0 ? max(ef, k) : rerank,
// then reranks with the float rows (depth 0: top k by SQ8 distance).
class GpuSq8Index {
 public:
  static Status Create(Device& dev, Metric metric, const VectorView& v,
                       std::unique_ptr<GpuSq8Index>* out) {
    detail::DatasetPtr d;
    VDBG_CXX_RETURN_IF_ERROR(detail::MakeDataset(dev, metric, v, &d));
    out->reset(new GpuSq8Index(dev, metric, v, std::move(d)));
    return Status::OK();
  }
  ~GpuSq8Index() {
    if (sq_) vdbg_sq8_destroy(sq_);
  }
  const char* type() const { return "sq8_scan"; }
  Status build() {
    vmin_.assign(view_.padded_dim, 0.f);
    scale_.assign(view_.padded_dim, 0.f);
    VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(vdbg_sq8_train(ds_.get(), vmin_.data(), scale_.data())));
    return encode();
  }
  // A deserialised quantizer (Sq8Quantizer::deserialize, sq8.cc:48-63) instead of training.
  Status build_with(std::span<const float> vmin, std::span<const float> scale) {
    vmin_.assign(vmin.begin(), vmin.end());
    scale_.assign(scale.begin(), scale.end());
    return encode();
  }
  size_t size() const { return view_.rows; }
  size_t code_bytes() const { return view_.rows * view_.padded_dim; }
  size_t memory_bytes() const { return code_bytes() + 2 * view_.padded_dim * sizeof(float); }
  const std::vector<float>& vmin() const { return vmin_; }
  const std::vector<float>& scale() const { return scale_; }
  vdbg_sq8* handle() const { return sq_; }  // nullptr before build()
  Status codes(std::vector<uint8_t>* out) const {
    out->resize(code_bytes());
    return Status::FromCall(vdbg_sq8_codes(sq_, out->data()));
  }
  static size_t Depth(const SearchParams& p, size_t k) {
    return p.rerank < 0 ? std::max(p.ef, k) : size_t(p.rerank);
  }

  Status search(const float* q, size_t k, const SearchParams& p, const DenseRowFilter* filter,
                std::vector<Neighbor>& out, IndexSearchStats* stats) const {
    std::vector<std::vector<Neighbor>> all;
    VDBG_CXX_RETURN_IF_ERROR(search_batch(q, 1, k, p, filter, all, stats));
    out = std::move(all[0]);
    return Status::OK();
  }
  Status search_batch(const float* queries, size_t nq, size_t k, const SearchParams& p,
                      const DenseRowFilter* filter, std::vector<std::vector<Neighbor>>& out,
                      IndexSearchStats* stats) const {
    if (sq_ == nullptr) return Status(VDBG_FAILED_PRECONDITION, "build() first");
    std::vector<uint32_t> ids(nq * k);
    std::vector<float> d(nq * k);
    uint64_t dc = 0;
    VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(
        vdbg_sq8_search_host(sq_, queries, nq, k, Depth(p, k), filter ? filter->words() : nullptr,
                             ids.data(), d.data(), &dc)));
    detail::Unpack(ids, d, nq, k, out);
    if (stats) stats->distance_computations += dc;
    return Status::OK();
  }

 private:
  GpuSq8Index(Device& dev, Metric m, const VectorView& v, detail::DatasetPtr d)
      : dev_(dev), metric_(m), view_(v), ds_(std::move(d)) {}
  Status encode() {
    if (sq_) vdbg_sq8_destroy(sq_);
    sq_ = nullptr;
    return Status::FromCall(vdbg_sq8_create(ds_.get(), vmin_.data(), scale_.data(), &sq_));
  }
  Device& dev_;
  Metric metric_;
  VectorView view_;
  detail::DatasetPtr ds_;
  vdbg_sq8* sq_ = nullptr;
  std::vector<float> vmin_, scale_;
};

// HnswSq8Index (src/index/hnsw/hnsw_index.h:64-97) loaded from its VDBHSQ81 file: the graph
// walk stays on the host (HnswGraph::search), the float rerank of each beam runs on the GPU
// (hnsw_index.cc:82-100).  The graph is built by vdb's own CPU code; this class only serves it.
class GpuHnswSq8Index {
 public:
  static Status Load(Device& dev, Metric metric, const VectorView& v, std::string_view file,
                     std::unique_ptr<GpuHnswSq8Index>* out) {
    detail::DatasetPtr d;
    VDBG_CXX_RETURN_IF_ERROR(detail::MakeDataset(dev, metric, v, &d));
    vdbg_sq8* sq = nullptr;
    VDBG_CXX_RETURN_IF_ERROR(
        Status::FromCall(vdbg_sq8_load(d.get(), file.data(), file.size(), &sq)));
    out->reset(new GpuHnswSq8Index(v, std::move(d), sq));
    return Status::OK();
  }
  ~GpuHnswSq8Index() {
    if (sq_) vdbg_sq8_destroy(sq_);
  }
  const char* type() const { return "hnsw_sq8"; }
  size_t size() const { return view_.rows; }
  size_t code_bytes() const { return view_.rows * view_.padded_dim; }

  Status search(const float* q, size_t k, const SearchParams& p, const DenseRowFilter* filter,
                std::vector<Neighbor>& out, IndexSearchStats* stats) const {
    std::vector<std::vector<Neighbor>> all;
    VDBG_CXX_RETURN_IF_ERROR(search_batch(q, 1, k, p, filter, all, stats));
    out = std::move(all[0]);
    return Status::OK();
  }
  Status search_batch(const float* queries, size_t nq, size_t k, const SearchParams& p,
                      const DenseRowFilter* filter, std::vector<std::vector<Neighbor>>& out,
                      IndexSearchStats* stats) const {
    std::vector<uint32_t> ids(nq * k);
    std::vector<float> d(nq * k);
    std::vector<uint64_t> dc(nq);
    VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(vdbg_sq8_hnsw_search_host(
        sq_, queries, nq, k, p.ef, p.rerank, filter ? filter->words() : nullptr, ids.data(),
        d.data(), dc.data())));
    detail::Unpack(ids, d, nq, k, out);
    if (stats)
      for (uint64_t x : dc) stats->distance_computations += x;
    return Status::OK();
  }
  vdbg_sq8* handle() const { return sq_; }

 private:
  GpuHnswSq8Index(const VectorView& v, detail::DatasetPtr d, vdbg_sq8* sq)
      : view_(v), ds_(std::move(d)), sq_(sq) {}
  VectorView view_;
  detail::DatasetPtr ds_;
  vdbg_sq8* sq_ = nullptr;
};

// ---------------------------------------------------------------- IVF-PQ

// IvfPqIndex (ivf_pq.h:42-81): build() trains and fills the lists on the GPU, Load() reads a
// VDBIVFP1 file (LoadIndex + IvfPqIndex::load, index.cc:38-87, ivf_pq.cc:251-278), Save()
// writes one (Index::save, ivf_pq.cc:236-249); search follows ivf_pq.cc:169-222.
class GpuIvfPqIndex {
 public:
  static Status Create(Device& dev, const IndexOptions& opts, Metric metric, const VectorView& v,
                       std::unique_ptr<GpuIvfPqIndex>* out) {
    if (opts.pq_m == 0 || v.dim % opts.pq_m != 0)
      return Status(VDBG_INVALID_ARGUMENT, "pq_m must divide dim");  // index.cc:27-29
    detail::DatasetPtr d;
    VDBG_CXX_RETURN_IF_ERROR(detail::MakeDataset(dev, metric, v, &d));
    out->reset(new GpuIvfPqIndex(dev, opts, metric, v, std::move(d)));
    return Status::OK();
  }
  ~GpuIvfPqIndex() {
    if (ix_) vdbg_ivfpq_destroy(ix_);
  }
  const char* type() const { return "ivf_pq"; }
  Status build() {
    reset();
    return Status::FromCall(vdbg_ivfpq_build(ds_.get(), opts_.nlist, opts_.pq_m, opts_.seed,
                                             opts_.max_train_points_per_centroid,
                                             opts_.kmeans_iters, &ix_));
  }
  Status Load(std::string_view file) {
    reset();
    return Status::FromCall(vdbg_ivfpq_load(ds_.get(), file.data(), file.size(), &ix_));
  }
  Status Save(std::string* file) const {
    size_t len = 0;
    VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(vdbg_ivfpq_save(ix_, nullptr, 0, &len)));
    file->resize(len);
    return Status::FromCall(vdbg_ivfpq_save(ix_, file->data(), len, &len));
  }
  size_t size() const { return view_.rows; }
  size_t nlist() const { return info().nlist; }
  size_t m() const { return info().m; }
  bool precomputed_tables() const { return info().pre != 0; }
  std::vector<uint64_t> list_sizes() const {
    std::vector<uint64_t> s(nlist());
    vdbg_ivfpq_list_sizes(ix_, s.data());
    return s;
  }
  size_t code_bytes() const { return view_.rows * m(); }
  vdbg_ivfpq* handle() const { return ix_; }  // nullptr before build() or Load()

  Status search(const float* q, size_t k, const SearchParams& p, const DenseRowFilter* filter,
                std::vector<Neighbor>& out, IndexSearchStats* stats) const {
    std::vector<std::vector<Neighbor>> all;
    VDBG_CXX_RETURN_IF_ERROR(search_batch(q, 1, k, p, filter, all, stats));
    out = std::move(all[0]);
    return Status::OK();
  }
  Status search_batch(const float* queries, size_t nq, size_t k, const SearchParams& p,
                      const DenseRowFilter* filter, std::vector<std::vector<Neighbor>>& out,
                      IndexSearchStats* stats) const {
    if (ix_ == nullptr) return Status(VDBG_FAILED_PRECONDITION, "build() or Load() first");
    std::vector<uint32_t> ids(nq * k);
    std::vector<float> d(nq * k);
    std::vector<uint64_t> dc(nq);
    VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(vdbg_ivfpq_search_host(
        ix_, queries, nq, k, p.nprobe, p.rerank, filter ? filter->words() : nullptr, ids.data(),
        d.data(), dc.data())));
    detail::Unpack(ids, d, nq, k, out);
    if (stats)
      for (uint64_t c : dc) stats->distance_computations += c;
    return Status::OK();
  }

 private:
  struct Info {
    size_t nlist = 0, m = 0;
    int pre = 0;
  };
  GpuIvfPqIndex(Device& dev, const IndexOptions& o, Metric metric, const VectorView& v,
                detail::DatasetPtr d)
      : dev_(dev), opts_(o), metric_(metric), view_(v), ds_(std::move(d)) {}
  Info info() const {
    Info i;
    if (ix_) vdbg_ivfpq_info(ix_, &i.nlist, &i.m, &i.pre);
    return i;
  }
  void reset() {
    if (ix_) vdbg_ivfpq_destroy(ix_);
    ix_ = nullptr;
  }
  Device& dev_;
  IndexOptions opts_;
  Metric metric_;
  VectorView view_;
  detail::DatasetPtr ds_;
  vdbg_ivfpq* ix_ = nullptr;
};

// ---------------------------------------------------------------- coalesced one-query calls

// Concurrent one-query searches of one index gathered into device batches (vdbg_coalescer_*).
// vdb's pool workers call Index::search once per query (src/engine/collection_impl.cc:
// 1120-1130); a Coalescer answers each such call with exactly what the index's own search()
// returns, while concurrent calls that share k, the parameters the index reads and the
// filter's words pointer run as one batch.  A filter expanded per call has a pointer of its
// own and runs alone: keep one set of words per segment state (deletes) and pass it as a
// view.  Destroy the Coalescer before its index.
class Coalescer {
 public:
  struct Options {
    size_t max_batch = 32;     // queries per device batch, 1..4096
    uint32_t max_wait_us = 50;  // longest wait for the previous batch's callers to call again
  };
  static Status Create(const GpuFlatIndex& ix, const Options& o, std::unique_ptr<Coalescer>* out) {
    vdbg_coalescer* c = nullptr;
    const int rc = vdbg_coalescer_create_flat(ix.dataset(), o.max_batch, o.max_wait_us, &c);
    return Make(Kind::Flat, rc, c, out);
  }
  static Status Create(const GpuSq8Index& ix, const Options& o, std::unique_ptr<Coalescer>* out) {
    vdbg_coalescer* c = nullptr;
    const int rc = vdbg_coalescer_create_sq8(ix.handle(), o.max_batch, o.max_wait_us, &c);
    return Make(Kind::Sq8, rc, c, out);
  }
  static Status Create(const GpuHnswSq8Index& ix, const Options& o,
                       std::unique_ptr<Coalescer>* out) {
    vdbg_coalescer* c = nullptr;
    const int rc = vdbg_coalescer_create_sq8_hnsw(ix.handle(), o.max_batch, o.max_wait_us, &c);
    return Make(Kind::HnswSq8, rc, c, out);
  }
  static Status Create(const GpuIvfPqIndex& ix, const Options& o, std::unique_ptr<Coalescer>* out) {
    vdbg_coalescer* c = nullptr;
    const int rc = vdbg_coalescer_create_ivfpq(ix.handle(), o.max_batch, o.max_wait_us, &c);
    return Make(Kind::IvfPq, rc, c, out);
  }
  // PqFlatIndex (src/index/quant/ivf_pq.cc:59-79) through its C handle (vdbg_pqflat_*).
  static Status Create(vdbg_pqflat* ix, const Options& o, std::unique_ptr<Coalescer>* out) {
    vdbg_coalescer* c = nullptr;
    const int rc = vdbg_coalescer_create_pqflat(ix, o.max_batch, o.max_wait_us, &c);
    return Make(Kind::PqFlat, rc, c, out);
  }
  ~Coalescer() { vdbg_coalescer_destroy(co_); }
  Coalescer(const Coalescer&) = delete;
  Coalescer& operator=(const Coalescer&) = delete;

  // The index's search() for one query (padded_dim floats): the same neighbours, order and
  // distance computations.  Blocks until the query's batch is done.
  Status search(const float* q, size_t k, const SearchParams& p, const DenseRowFilter* filter,
                std::vector<Neighbor>& out, IndexSearchStats* stats) const {
    size_t param = 0;
    if (kind_ == Kind::Sq8) param = GpuSq8Index::Depth(p, k);
    if (kind_ == Kind::HnswSq8) param = p.ef;
    if (kind_ == Kind::IvfPq) param = p.nprobe;
    std::vector<uint32_t> ids(k);
    std::vector<float> d(k);
    uint64_t dc = 0;
    VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(vdbg_coalescer_search(
        co_, q, k, param, p.rerank, filter ? filter->words() : nullptr, ids.data(), d.data(), &dc)));
    out.clear();
    for (size_t i = 0; i < k && ids[i] != kNoRow; ++i) out.push_back({d[i], ids[i]});
    if (stats) stats->distance_computations += dc;
    return Status::OK();
  }
  // Batches run so far and the queries they held.
  void counts(uint64_t* batches, uint64_t* queries) const { vdbg_coalescer_stats(co_, batches, queries); }

 private:
  enum class Kind { Flat, Sq8, HnswSq8, IvfPq, PqFlat };
  static Status Make(Kind kind, int rc, vdbg_coalescer* c, std::unique_ptr<Coalescer>* out) {
    VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(rc));
    out->reset(new Coalescer(kind, c));
    return Status::OK();
  }
  Coalescer(Kind kind, vdbg_coalescer* co) : kind_(kind), co_(co) {}
  Kind kind_;
  vdbg_coalescer* co_;
};

// ---------------------------------------------------------------- collection read path

// A flat segment as CollectionImpl::Search sees it: its index, the rows a query may return
// (deletes and filter applied; nullptr = all) and the external id of every row.
struct SegmentRef {
  const GpuFlatIndex* index = nullptr;
  const DenseRowFilter* allowed = nullptr;
  const VectorId* external_ids = nullptr;
};

struct SearchHit {  // include/vdb/types.h SearchHit: id, distance, score
  VectorId id = 0;
  float distance = 0.f;
  float score = 0.f;  // -distance for inner product and cosine, distance for L2
};

// CollectionImpl::Search (collection_impl.cc:1036-1112) for nq raw queries of dim floats
// over flat segments of one metric: PrepareQuery (:1023-1034), each segment's filtered
// exact scan, the merge by (dist, part, row) keeping the first hit of each external id.
inline Status SearchSegments(Device& dev, std::span<const SegmentRef> segs, Metric metric,
                             const float* raw_queries, size_t nq, size_t dim, size_t k,
                             std::vector<std::vector<SearchHit>>& out,
                             IndexSearchStats* stats = nullptr) {
  if (k == 0 || k > 10000) return Status(VDBG_INVALID_ARGUMENT, "k must be in 1..10000");
  const size_t pd = PaddedDim(dim);
  std::vector<float> q(nq * pd);
  VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(
      vdbg_prepare_queries_host(dev.get(), raw_queries, nq, dim, pd, int(metric), q.data())));
  const size_t np = segs.size();
  std::vector<float> pdist(np * nq * k);
  std::vector<uint32_t> prow(np * nq * k);
  std::vector<uint64_t> ext, off(np);
  for (size_t p = 0; p < np; ++p) {
    const GpuFlatIndex* ix = segs[p].index;
    uint64_t dc = 0;
    VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(vdbg_flat_search_host(
        ix->dataset(), q.data(), nq, k, segs[p].allowed ? segs[p].allowed->words() : nullptr,
        prow.data() + p * nq * k, pdist.data() + p * nq * k, &dc)));
    if (stats) stats->distance_computations += dc;
    off[p] = ext.size();
    ext.insert(ext.end(), segs[p].external_ids, segs[p].external_ids + ix->size());
  }
  std::vector<uint64_t> oe(nq * k);
  std::vector<float> od(nq * k);
  VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(
      vdbg_merge_parts_host(dev.get(), nq, np, k, pdist.data(), prow.data(), ext.data(),
                            ext.size(), off.data(), oe.data(), od.data())));
  out.assign(nq, {});
  for (size_t i = 0; i < nq; ++i)
    for (size_t j = 0; j < k && oe[i * k + j] != ~uint64_t(0); ++j)
      out[i].push_back({oe[i * k + j], od[i * k + j],
                        metric == Metric::L2 ? od[i * k + j] : -od[i * k + j]});
  return Status::OK();
}

// ---------------------------------------------------------------- segments on disk

enum class IndexType : uint8_t { Flat = 0, Hnsw = 1, HnswSq8 = 2, PqFlat = 3, IvfPq = 4 };  // options.h:13

inline const char* IndexTypeName(IndexType t) {  // src/util/status.cc:55-64
  switch (t) {
    case IndexType::Flat: return "flat";
    case IndexType::Hnsw: return "hnsw";
    case IndexType::HnswSq8: return "hnsw_sq8";
    case IndexType::PqFlat: return "pq";
    case IndexType::IvfPq: return "ivf_pq";
  }
  return "unknown";
}

// The fields of SegmentMeta (src/storage/manifest.h) that Segment::Open reads.
struct SegmentMeta {
  uint32_t id = 0;
  uint64_t rows = 0;
  std::string deletes_file;  // "deletes-<n>.roar", empty = none persisted
};

// The fields of CollectionOptions (options.h:35-41) that Segment::Open reads.
struct CollectionOptions {
  size_t dim = 0;
  Metric metric = Metric::L2;
  IndexType index_type = IndexType::Flat;
};

namespace detail {

// A whole file mapped read-only (Env::map_file, src/storage/env.h), unmapped on destruction.
class MappedFile {
 public:
  ~MappedFile() {
    if (p_ != nullptr && p_ != MAP_FAILED) munmap(p_, n_);
  }
  Status Open(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return Status(VDBG_IO_ERROR, path + ": cannot open");
    struct stat st;
    if (fstat(fd, &st) != 0) {
      ::close(fd);
      return Status(VDBG_IO_ERROR, path + ": cannot stat");
    }
    n_ = size_t(st.st_size);
    if (n_ > 0) p_ = mmap(nullptr, n_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (p_ == MAP_FAILED) return Status(VDBG_IO_ERROR, path + ": cannot map");
    return Status::OK();
  }
  const void* data() const { return p_; }
  size_t size() const { return n_; }

 private:
  void* p_ = nullptr;
  size_t n_ = 0;
};

inline std::string JoinPath(const std::string& a, const std::string& b) {
  return a.empty() || a.back() == '/' ? a + b : a + "/" + b;
}

}  // namespace detail

// Segment::Open (src/storage/segment_reader.cc:20-122) for what a search reads, made resident
// on the device: vectors.f32 (header and CRC checks, the rows uploaded), ids.u64 (kept on
// the host and resident for the merge), the index file (LoadIndex by magic, index.cc:38-87:
// VDBFLAT1 needs nothing more, VDBHSQ81 brings its SQ8 codes and its graph, walked on the
// host with the rerank on the GPU, VDBIVFP1 its lists, VDBPQFL1 its codebook and codes; a
// float-row HNSW index is NotSupported: vdb keeps such a segment on its CPU path and hands
// its hits to SearchCollection as a host part) and the persisted delete set.  meta.bin is not read: filters arrive already evaluated, as dense words.  Errors are
// the reference's Corruption messages, prefixed with the file or directory.
class GpuSegment {
 public:
  static Status Open(Device& dev, const std::string& dir, const SegmentMeta& meta,
                     const CollectionOptions& opts, bool verify_crc,
                     std::unique_ptr<GpuSegment>* out) {
    std::unique_ptr<GpuSegment> s(new GpuSegment());
    s->id_ = meta.id;
    s->dim_ = opts.dim;
    s->metric_ = opts.metric;
    // ---- vectors.f32 (:37-59)
    {
      const std::string vpath = detail::JoinPath(dir, "vectors.f32");
      detail::MappedFile f;
      VDBG_CXX_RETURN_IF_ERROR(f.Open(vpath));
      vdbg_dataset* d = nullptr;
      Status st = Status::FromCall(vdbg_dataset_open_vectors(dev.get(), f.data(), f.size(), opts.dim,
                                                             int(opts.metric), meta.rows,
                                                             verify_crc ? 1 : 0, &d));
      if (!st.ok()) return Status(st.code(), dir + "/" + st.message());
      s->ds_.reset(d);
      s->rows_ = meta.rows;
    }
    // ---- ids.u64 (:61-66)
    {
      std::string bytes;
      VDBG_CXX_RETURN_IF_ERROR(ReadFile(detail::JoinPath(dir, "ids.u64"), &bytes));
      size_t off = 0, len = 0;
      Status st = Status::FromCall(vdbg_blob_decode(bytes.data(), bytes.size(), "VDBIDS01", &off, &len));
      if (!st.ok()) return Status(st.code(), detail::JoinPath(dir, "ids.u64") + ": " + st.message());
      if (len != s->rows_ * sizeof(VectorId)) return Status(VDBG_CORRUPTION, dir + ": ids.u64 size mismatch");
      s->ids_.resize(s->rows_);
      if (len > 0) std::memcpy(s->ids_.data(), bytes.data() + off, len);
      VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(vdbg_dataset_set_external_ids(s->ds_.get(), s->ids_.data())));
    }
    // ---- index.<type> (:90-99)
    {
      std::string bytes;
      VDBG_CXX_RETURN_IF_ERROR(
          ReadFile(detail::JoinPath(dir, std::string("index.") + IndexTypeName(opts.index_type)), &bytes));
      Status st = s->LoadIndex(bytes);
      if (!st.ok()) return Status(st.code(), dir + ": " + st.message());
    }
    // ---- deletes (:102-117)
    s->deleted_.assign((s->rows_ + 63) / 64, 0);
    if (!meta.deletes_file.empty()) {
      std::string bytes;
      VDBG_CXX_RETURN_IF_ERROR(ReadFile(detail::JoinPath(dir, meta.deletes_file), &bytes));
      uint64_t n = 0;
      Status st = Status::FromCall(vdbg_deletes_decode(bytes.data(), bytes.size(), s->rows_,
                                                       s->deleted_.data(), &n));
      if (!st.ok()) return Status(st.code(), dir + ": " + st.message());
      s->deleted_count_ = n;
    }
    *out = std::move(s);
    return Status::OK();
  }
  ~GpuSegment() {
    if (sq8_) vdbg_sq8_destroy(sq8_);
    if (ivf_) vdbg_ivfpq_destroy(ivf_);
    if (pqf_) vdbg_pqflat_destroy(pqf_);
  }

  uint32_t id() const { return id_; }
  size_t rows() const { return rows_; }
  size_t dim() const { return dim_; }
  Metric metric() const { return metric_; }
  IndexType index_type() const { return type_; }
  VectorId external_id(InternalId r) const { return ids_[r]; }
  // DeleteBits (src/util/delete_bits.h:18-114) as dense words, bit r = row r deleted.
  const std::vector<uint64_t>& deleted_words() const { return deleted_; }
  size_t deleted_count() const { return deleted_count_; }
  size_t live_rows() const { return rows_ - std::min(rows_, deleted_count_); }
  // DeleteBits::set: later searches skip the row.
  void Delete(InternalId r) {
    if (r >= rows_) return;
    uint64_t& w = deleted_[r >> 6];
    const uint64_t bit = uint64_t(1) << (r & 63);
    if (!(w & bit)) ++deleted_count_;
    w |= bit;
  }
  vdbg_dataset* dataset() const { return ds_.get(); }
  vdbg_sq8* sq8() const { return sq8_; }
  vdbg_ivfpq* ivfpq() const { return ivf_; }
  vdbg_pqflat* pqflat() const { return pqf_; }

  static Status ReadFile(const std::string& path, std::string* out) {
    detail::MappedFile f;
    VDBG_CXX_RETURN_IF_ERROR(f.Open(path));
    out->assign(static_cast<const char*>(f.data()), f.size());
    return Status::OK();
  }

 private:
  GpuSegment() = default;
  // LoadIndex (index.cc:38-87): CRC32C footer, then the magic picks the index.
  Status LoadIndex(const std::string& bytes) {
    if (bytes.size() < 12) return Status(VDBG_CORRUPTION, "index file too short");
    uint32_t stored;
    std::memcpy(&stored, bytes.data() + bytes.size() - 4, 4);
    if (vdbg_crc32c_extend(0, bytes.data(), bytes.size() - 4) != stored)
      return Status(VDBG_CORRUPTION, "index file checksum mismatch");
    const std::string_view magic(bytes.data(), 8);
    if (magic == "VDBFLAT1") {
      type_ = IndexType::Flat;
      return Status::OK();
    }
    if (magic == "VDBHSQ81") {
      type_ = IndexType::HnswSq8;
      return Status::FromCall(vdbg_sq8_load(ds_.get(), bytes.data(), bytes.size(), &sq8_));
    }
    if (magic == "VDBIVFP1") {
      type_ = IndexType::IvfPq;
      return Status::FromCall(vdbg_ivfpq_load(ds_.get(), bytes.data(), bytes.size(), &ivf_));
    }
    if (magic == "VDBPQFL1") {
      type_ = IndexType::PqFlat;
      return Status::FromCall(vdbg_pqflat_load(ds_.get(), bytes.data(), bytes.size(), &pqf_));
    }
    if (magic == "VDBHNSW1")
      return Status(VDBG_NOT_SUPPORTED, "float-row HNSW index files are searched on the CPU");
    return Status(VDBG_CORRUPTION, "unknown index file magic");
  }

  uint32_t id_ = 0;
  size_t rows_ = 0, dim_ = 0;
  Metric metric_ = Metric::L2;
  IndexType type_ = IndexType::Flat;
  detail::DatasetPtr ds_;
  vdbg_sq8* sq8_ = nullptr;
  vdbg_ivfpq* ivf_ = nullptr;
  vdbg_pqflat* pqf_ = nullptr;
  std::vector<VectorId> ids_;
  std::vector<uint64_t> deleted_;
  size_t deleted_count_ = 0;
};

// The hits of a disk segment searched on the host: vdb's own SearchDiskSegment
// (planner.cc:42-129) over an index this library does not hold, such as HnswIndex over a
// VDBHNSW1 file (vdb's default IndexType::Hnsw, options.h:22; GpuSegment::Open is
// NotSupported for it).  [nq][k] each: per query ascending (dist, row), kNoRow after the last
// hit, and each hit's external id.
struct HostSegmentHits {
  std::vector<float> dists;
  std::vector<InternalId> rows;
  std::vector<VectorId> ids;
  std::vector<uint64_t> dist_comps;  // [nq] SegmentExplain::distance_computations, or empty
};

// One disk segment of a snapshot: on the device, or searched on the host.
struct DiskPart {
  const GpuSegment* gpu = nullptr;
  const HostSegmentHits* host = nullptr;
};

// CollectionImpl::SearchBatch (collection_impl.cc:1121-1135) over a snapshot's disk segments,
// as one device batch (vdbg_collection_search_host): PrepareQuery, SearchDiskSegment's plan
// per segment (planner.cc:42-129), the merge with one hit per external id.  parts are in the
// snapshot's order; a host part's hits merge in its place.  filters: null for a request
// without a filter, else one filter per part (the request's filter evaluated on that
// segment; deletes are removed here; a host part's entry is not read).  plans (optional)
// receives each part's SegmentExplain::strategy ("host" for a host part).
inline Status SearchCollection(Device& dev, std::span<const DiskPart> parts, size_t dim,
                               Metric metric, const float* raw_queries, size_t nq, size_t k,
                               const SearchParams& p,
                               const std::vector<const DenseRowFilter*>* filters,
                               std::vector<std::vector<SearchHit>>& out,
                               std::vector<uint64_t>* dist_comps = nullptr,
                               std::vector<std::string>* plans = nullptr) {
  if (filters != nullptr && filters->size() != parts.size())
    return Status(VDBG_INVALID_ARGUMENT, "one filter per segment");
  std::vector<vdbg_segment> v(parts.size());
  for (size_t i = 0; i < parts.size(); ++i) {
    if (const HostSegmentHits* h = parts[i].host) {
      if (h->dists.size() != nq * k || h->rows.size() != nq * k || h->ids.size() != nq * k ||
          (!h->dist_comps.empty() && h->dist_comps.size() != nq))
        return Status(VDBG_INVALID_ARGUMENT, "host segment hits are [nq][k]");
      v[i].host_dists = h->dists.data();
      v[i].host_rows = h->rows.data();
      v[i].host_ext = h->ids.data();
      v[i].host_dist_comps = h->dist_comps.empty() ? nullptr : h->dist_comps.data();
      // (a null pointer would read as "not searched on the host")
      static const InternalId kNone = kNoRow;
      if (nq * k == 0) v[i].host_rows = &kNone;
      continue;
    }
    if (parts[i].gpu == nullptr) return Status(VDBG_INVALID_ARGUMENT, "empty disk part");
    const GpuSegment& g = *parts[i].gpu;
    v[i].rows = g.dataset();
    v[i].sq8 = g.sq8();
    v[i].ivfpq = g.ivfpq();
    v[i].pqflat = g.pqflat();
    v[i].deleted_words = g.deleted_count() > 0 ? g.deleted_words().data() : nullptr;
    v[i].filter_words = filters != nullptr ? (*filters)[i]->words() : nullptr;
  }
  const vdbg_search_params sp{p.ef, p.nprobe, p.rerank, int(p.strategy), p.prefilter_threshold,
                              p.post_filter_alpha};
  std::vector<uint64_t> ids(nq * k), dc(nq);
  std::vector<float> d(nq * k);
  std::vector<int> pl(parts.size());
  VDBG_CXX_RETURN_IF_ERROR(Status::FromCall(vdbg_collection_search_host(
      dev.get(), v.data(), v.size(), dim, int(metric), raw_queries, nq, k, &sp, ids.data(),
      d.data(), dc.data(), pl.data())));
  out.assign(nq, {});
  for (size_t i = 0; i < nq; ++i)
    for (size_t j = 0; j < k && ids[i * k + j] != ~uint64_t(0); ++j)
      out[i].push_back({ids[i * k + j], d[i * k + j],
                        metric == Metric::L2 ? d[i * k + j] : -d[i * k + j]});
  if (dist_comps != nullptr) *dist_comps = dc;
  if (plans != nullptr) {
    static const char* const kNames[] = {"index", "empty", "prefilter_exact", "filtered_index",
                                         "filtered_index+exact_fallback", "post_filter", "scan",
                                         "scan_filter", "host"};
    plans->clear();
    for (int x : pl) plans->push_back(kNames[x]);
  }
  return Status::OK();
}

// The same over segments that are all on the device.
inline Status SearchCollection(Device& dev, std::span<const GpuSegment* const> segs, size_t dim,
                               Metric metric, const float* raw_queries, size_t nq, size_t k,
                               const SearchParams& p,
                               const std::vector<const DenseRowFilter*>* filters,
                               std::vector<std::vector<SearchHit>>& out,
                               std::vector<uint64_t>* dist_comps = nullptr,
                               std::vector<std::string>* plans = nullptr) {
  std::vector<DiskPart> parts(segs.size());
  for (size_t i = 0; i < segs.size(); ++i) parts[i].gpu = segs[i];
  return SearchCollection(dev, std::span<const DiskPart>(parts), dim, metric, raw_queries, nq, k,
                          p, filters, out, dist_comps, plans);
}

}  // namespace vdbg
