// gpu_index_test.cc -- the C++20 host classes (include/vdbg.hpp) on the GPU, checked against the
// oracle (oracle/vdb_oracle.h).  The cases follow the reference's own tests:
// tests/flat_test.cc (every metric, batched == single, filter, k > rows), tests/index_test.cc
// (build/search/save/load, pq_m must divide dim), tests/pq_test.cc (small segments shrink
// nlist, IVF-PQ inner product) and tests/filter_test.cc (exact filtered search at several
// selectivities).  Results must equal the oracle's bit for bit.
//
// Run: tests/cpp/gpu_index_test  (exit status 0 = all passed).  Needs a gfx950 GPU.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <functional>
#include <string>
#include <thread>
#include <vector>

#include "../../include/vdbg.hpp"
#include "../../oracle/vdb_oracle.h"

namespace {

int g_failed = 0;
int g_checks = 0;
std::string g_test;

#define CHECK(cond)                                                                    \
  do {                                                                                 \
    ++g_checks;                                                                        \
    if (!(cond)) {                                                                     \
      ++g_failed;                                                                      \
      std::fprintf(stderr, "  %s:%d: %s: CHECK(%s) failed\n", __FILE__, __LINE__,      \
                   g_test.c_str(), #cond);                                             \
    }                                                                                  \
  } while (0)
#define CHECK_OK(expr)                                                                 \
  do {                                                                                 \
    vdbg::Status s_ = (expr);                                                          \
    ++g_checks;                                                                        \
    if (!s_.ok()) {                                                                    \
      ++g_failed;                                                                      \
      std::fprintf(stderr, "  %s:%d: %s: %s -> %s\n", __FILE__, __LINE__, g_test.c_str(), \
                   #expr, s_.ToString().c_str());                                      \
      return;                                                                          \
    }                                                                                  \
  } while (0)

// SplitMix64 rows: a clustered mixture (centres U[0,1)^d scaled, row = centre + 0.1 noise),
// optionally normalised, like test::MakeClustered's role in the reference tests.
struct Rng {
  uint64_t s;
  uint64_t next() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  float uni() { return float(next() >> 40) * (1.0f / 16777216.0f); }
};

struct Data {
  size_t rows = 0, dim = 0, pd = 0;
  std::vector<float> v;
  vdbg::VectorView view() const { return {v.data(), rows, dim, pd}; }
  const float* row(size_t r) const { return v.data() + r * pd; }
};

Data Clustered(size_t n, size_t dim, size_t clusters, uint64_t seed, bool unit) {
  Data d;
  d.rows = n;
  d.dim = dim;
  d.pd = vdbg::PaddedDim(dim);
  d.v.assign(n * d.pd, 0.f);
  Rng c{1000 + clusters}, r{seed};
  std::vector<float> cen(clusters * dim);
  for (auto& x : cen) x = c.uni();
  for (size_t i = 0; i < n; ++i) {
    const size_t k = r.next() % clusters;
    for (size_t j = 0; j < dim; ++j) d.v[i * d.pd + j] = cen[k * dim + j] + 0.1f * (r.uni() - 0.5f);
    if (unit) or_normalize(d.v.data() + i * d.pd, dim);
  }
  return d;
}

int Kset() { return OR_KSET_AVX512; }

// Oracle flat search over rows with an optional dense filter, as ascending Neighbor lists.
std::vector<std::vector<vdbg::Neighbor>> OracleFlat(const Data& b, const float* q, size_t nq,
                                                    size_t k, vdbg::Metric m,
                                                    const vdbg::DenseRowFilter* f) {
  std::vector<float> d(nq * k);
  std::vector<uint32_t> id(nq * k);
  or_flat_search_batch(Kset(), int(m), b.v.data(), b.rows, b.pd, q, nq, k, f ? f->words() : nullptr,
                       d.data(), id.data(), 8);
  std::vector<std::vector<vdbg::Neighbor>> out(nq);
  for (size_t i = 0; i < nq; ++i)
    for (size_t j = 0; j < k && id[i * k + j] != UINT32_MAX; ++j) out[i].push_back({d[i * k + j], id[i * k + j]});
  return out;
}

bool Same(const std::vector<vdbg::Neighbor>& a, const std::vector<vdbg::Neighbor>& b) {
  if (a.size() != b.size()) return false;
  for (size_t i = 0; i < a.size(); ++i)
    if (a[i].id != b[i].id || std::memcmp(&a[i].dist, &b[i].dist, 4) != 0) return false;
  return true;
}

vdbg::Device* g_dev = nullptr;

// ---------------------------------------------------------------- flat (flat_test.cc)

void FlatMatchesOracleForEveryMetric() {
  for (vdbg::Metric m : {vdbg::Metric::L2, vdbg::Metric::InnerProduct, vdbg::Metric::Cosine}) {
    const bool unit = m == vdbg::Metric::Cosine;
    Data base = Clustered(30000, 37, 10, 1, unit), qs = Clustered(64, 37, 10, 2, unit);
    std::unique_ptr<vdbg::GpuFlatIndex> ix;
    CHECK_OK(vdbg::GpuFlatIndex::Create(*g_dev, m, base.view(), &ix));
    std::vector<std::vector<vdbg::Neighbor>> got;
    vdbg::IndexSearchStats st;
    CHECK_OK(ix->search_batch(qs.v.data(), qs.rows, 20, {}, nullptr, got, &st));
    auto want = OracleFlat(base, qs.v.data(), qs.rows, 20, m, nullptr);
    for (size_t q = 0; q < qs.rows; ++q) {
      CHECK(got[q].size() == 20u);
      CHECK(Same(got[q], want[q]));
      for (size_t i = 1; i < got[q].size(); ++i) CHECK(!(got[q][i] < got[q][i - 1]));
    }
    CHECK(st.distance_computations == qs.rows * base.rows);  // flat_index.cc:75-76
  }
}

void FlatBatchedMatchesSingleQuery() {
  Data base = Clustered(20000, 64, 20, 3, false), qs = Clustered(130, 64, 20, 4, false);
  std::unique_ptr<vdbg::GpuFlatIndex> ix;
  CHECK_OK(vdbg::GpuFlatIndex::Create(*g_dev, vdbg::Metric::L2, base.view(), &ix));
  std::vector<std::vector<vdbg::Neighbor>> batch;
  CHECK_OK(ix->search_batch(qs.v.data(), qs.rows, 10, {}, nullptr, batch, nullptr));
  std::vector<vdbg::Neighbor> single;
  for (size_t q = 0; q < qs.rows; ++q) {
    CHECK_OK(ix->search(qs.row(q), 10, {}, nullptr, single, nullptr));
    CHECK(single == batch[q]);
  }
}

void FlatFilterIsRespected() {
  Data base = Clustered(1000, 16, 4, 5, false);
  vdbg::DenseRowFilter odd(base.rows);
  for (uint32_t r = 1; r < base.rows; r += 2) odd.Allow(r);
  std::unique_ptr<vdbg::GpuFlatIndex> ix;
  CHECK_OK(vdbg::GpuFlatIndex::Create(*g_dev, vdbg::Metric::L2, base.view(), &ix));
  std::vector<vdbg::Neighbor> out;
  CHECK_OK(ix->search(base.row(0), 50, {}, &odd, out, nullptr));
  CHECK(out.size() == 50u);
  for (const auto& n : out) CHECK(n.id % 2 == 1u);
  CHECK(Same(out, OracleFlat(base, base.row(0), 1, 50, vdbg::Metric::L2, &odd)[0]));
}

void FlatKLargerThanRows() {
  Data base = Clustered(5, 8, 1, 6, false);
  std::unique_ptr<vdbg::GpuFlatIndex> ix;
  CHECK_OK(vdbg::GpuFlatIndex::Create(*g_dev, vdbg::Metric::L2, base.view(), &ix));
  std::vector<vdbg::Neighbor> out;
  CHECK_OK(ix->search(base.row(0), 100, {}, nullptr, out, nullptr));
  CHECK(out.size() == 5u);
  CHECK(!out.empty() && out[0].id == 0u);
}

void RerankMatchesOracle() {
  Data base = Clustered(20000, 48, 25, 15, false), qs = Clustered(30, 48, 25, 16, false);
  std::unique_ptr<vdbg::GpuFlatIndex> ix;
  CHECK_OK(vdbg::GpuFlatIndex::Create(*g_dev, vdbg::Metric::L2, base.view(), &ix));
  for (size_t depth : {size_t(80), size_t(600)}) {
    Rng r{depth};
    std::vector<uint32_t> cand(qs.rows * depth);
    for (auto& c : cand) c = uint32_t(r.next() % base.rows);
    for (size_t q = 0; q < qs.rows; q += 4) cand[q * depth + depth - 1] = vdbg::kNoRow;
    std::vector<std::vector<vdbg::Neighbor>> got;
    vdbg::IndexSearchStats st;
    CHECK_OK(ix->rerank_batch(qs.v.data(), qs.rows, cand.data(), depth, 10, got, &st));
    uint64_t want_dc = 0;
    for (size_t q = 0; q < qs.rows; ++q) {
      std::vector<uint32_t> c;
      for (size_t i = 0; i < depth; ++i)
        if (cand[q * depth + i] != vdbg::kNoRow) c.push_back(cand[q * depth + i]);
      want_dc += c.size();
      std::vector<float> d(10);
      std::vector<uint32_t> id(10);
      const size_t n = or_rerank(Kset(), 0, base.v.data(), base.pd, qs.row(q), c.data(), c.size(), 10,
                                 d.data(), id.data());
      std::vector<vdbg::Neighbor> w;
      for (size_t j = 0; j < n; ++j) w.push_back({d[j], id[j]});
      CHECK(Same(got[q], w));
    }
    CHECK(st.distance_computations == want_dc);
  }
}

// ---------------------------------------------------------------- SQ8

void Sq8CodesAndSearchMatchOracle() {
  Data base = Clustered(25000, 96, 30, 7, false), qs = Clustered(48, 96, 30, 8, false);
  std::unique_ptr<vdbg::GpuSq8Index> ix;
  CHECK_OK(vdbg::GpuSq8Index::Create(*g_dev, vdbg::Metric::L2, base.view(), &ix));
  CHECK_OK(ix->build());
  std::vector<float> vmin(base.pd), scale(base.pd);
  or_sq8_train(base.v.data(), base.rows, base.dim, base.pd, vmin.data(), scale.data());
  CHECK(std::memcmp(vmin.data(), ix->vmin().data(), 4 * base.pd) == 0);
  CHECK(std::memcmp(scale.data(), ix->scale().data(), 4 * base.pd) == 0);
  std::vector<uint8_t> codes, want(base.rows * base.pd);
  CHECK_OK(ix->codes(&codes));
  or_sq8_encode_rows(base.v.data(), base.rows, base.dim, base.pd, vmin.data(), scale.data(), want.data());
  CHECK(codes == want);
  for (int rerank : {-1, 0, 60}) {
    vdbg::SearchParams p;
    p.ef = 40;
    p.rerank = rerank;
    const size_t k = 10, depth = vdbg::GpuSq8Index::Depth(p, k);
    std::vector<std::vector<vdbg::Neighbor>> got;
    CHECK_OK(ix->search_batch(qs.v.data(), qs.rows, k, p, nullptr, got, nullptr));
    std::vector<float> d(qs.rows * k);
    std::vector<uint32_t> id(qs.rows * k);
    or_sq8_search_batch(Kset(), 0, base.v.data(), codes.data(), base.rows, base.pd, vmin.data(),
                        scale.data(), qs.v.data(), qs.rows, k, depth, nullptr, d.data(), id.data(), 8);
    for (size_t q = 0; q < qs.rows; ++q) {
      std::vector<vdbg::Neighbor> w;
      for (size_t j = 0; j < k; ++j) w.push_back({d[q * k + j], id[q * k + j]});
      CHECK(Same(got[q], w));
    }
  }
}

// ---------------------------------------------------------------- IVF-PQ (index_test.cc, pq_test.cc)

struct IvfFile {
  size_t nlist = 0, pd = 0, dim = 0, m = 0;
  std::vector<float> coarse, cen;
  std::vector<uint64_t> off{0};
  std::vector<uint32_t> ids;
  std::vector<uint8_t> codes;
};

// VDBIVFP1 body (ivf_pq.cc:236-249): rows u64, pd u32, nlist u32, coarse, dim u32, m u32,
// codebook, per list (size u64, ids, codes); CRC32C footer.
bool ParseIvf(const std::string& f, IvfFile* o) {
  if (f.size() < 12 || f.compare(0, 8, "VDBIVFP1") != 0) return false;
  size_t p = 8;
  auto rd = [&](void* dst, size_t n) {
    std::memcpy(dst, f.data() + p, n);
    p += n;
  };
  uint64_t rows;
  uint32_t pd, nlist, dim, m;
  rd(&rows, 8);
  rd(&pd, 4);
  rd(&nlist, 4);
  o->pd = pd;
  o->nlist = nlist;
  o->coarse.resize(size_t(nlist) * pd);
  rd(o->coarse.data(), o->coarse.size() * 4);
  rd(&dim, 4);
  rd(&m, 4);
  o->dim = dim;
  o->m = m;
  o->cen.resize(size_t(m) * 256 * (dim / m));
  rd(o->cen.data(), o->cen.size() * 4);
  for (uint32_t l = 0; l < nlist; ++l) {
    uint64_t sz;
    rd(&sz, 8);
    const size_t b = o->ids.size();
    o->ids.resize(b + sz);
    rd(o->ids.data() + b, sz * 4);
    o->codes.resize((b + sz) * m);
    rd(o->codes.data() + b * m, sz * m);
    o->off.push_back(o->off.back() + sz);
  }
  return p + 4 == f.size() && or_crc32c(0, f.data(), p) == *reinterpret_cast<const uint32_t*>(f.data() + p);
}

void IvfPqBuildSearchSaveLoad() {
  Data base = Clustered(40000, 64, 50, 9, false), qs = Clustered(64, 64, 50, 10, false);
  vdbg::IndexOptions opts;
  opts.nlist = 256;
  opts.pq_m = 16;
  std::unique_ptr<vdbg::GpuIvfPqIndex> ix;
  CHECK_OK(vdbg::GpuIvfPqIndex::Create(*g_dev, opts, vdbg::Metric::L2, base.view(), &ix));
  CHECK_OK(ix->build());
  CHECK(ix->nlist() == 256u && ix->m() == 16u && ix->precomputed_tables());
  uint64_t total = 0;
  for (uint64_t s : ix->list_sizes()) total += s;
  CHECK(total == base.rows);
  std::string file;
  CHECK_OK(ix->Save(&file));
  IvfFile f;
  CHECK(ParseIvf(file, &f));
  for (int rerank : {0, 100}) {
    vdbg::SearchParams p;
    p.nprobe = 12;
    p.rerank = rerank;
    std::vector<std::vector<vdbg::Neighbor>> got;
    vdbg::IndexSearchStats st;
    CHECK_OK(ix->search_batch(qs.v.data(), qs.rows, 10, p, nullptr, got, &st));
    std::vector<float> term2(f.nlist * f.m * 256), d(qs.rows * 10);
    std::vector<uint32_t> id(qs.rows * 10);
    std::vector<uint64_t> dc(qs.rows);
    or_ivfpq_term2(f.coarse.data(), f.nlist, f.pd, f.cen.data(), f.m, f.dim / f.m, term2.data());
    or_ivfpq_search_batch(Kset(), 0, base.v.data(), base.dim, base.pd, f.coarse.data(), f.nlist,
                          f.cen.data(), f.m, f.off.data(), f.ids.data(), f.codes.data(), term2.data(),
                          qs.v.data(), qs.rows, 10, p.nprobe, p.rerank, nullptr, d.data(), id.data(),
                          dc.data(), 8);
    uint64_t want_dc = 0;
    for (size_t q = 0; q < qs.rows; ++q) {
      std::vector<vdbg::Neighbor> w;
      for (size_t j = 0; j < 10 && id[q * 10 + j] != UINT32_MAX; ++j) w.push_back({d[q * 10 + j], id[q * 10 + j]});
      CHECK(Same(got[q], w));
      want_dc += dc[q];
    }
    CHECK(st.distance_computations == want_dc);
  }
  // load into a fresh index: the same file back, the same answers
  std::unique_ptr<vdbg::GpuIvfPqIndex> re;
  CHECK_OK(vdbg::GpuIvfPqIndex::Create(*g_dev, opts, vdbg::Metric::L2, base.view(), &re));
  CHECK_OK(re->Load(file));
  std::string again;
  CHECK_OK(re->Save(&again));
  CHECK(again == file);
  vdbg::SearchParams p;
  p.nprobe = 8;
  std::vector<std::vector<vdbg::Neighbor>> a, b;
  CHECK_OK(ix->search_batch(qs.v.data(), qs.rows, 10, p, nullptr, a, nullptr));
  CHECK_OK(re->search_batch(qs.v.data(), qs.rows, 10, p, nullptr, b, nullptr));
  CHECK(a == b);
  // a corrupted byte is rejected as Corruption (index.cc:47-56)
  std::string bad = file;
  bad[bad.size() / 2] ^= 0x5a;
  std::unique_ptr<vdbg::GpuIvfPqIndex> c;
  CHECK_OK(vdbg::GpuIvfPqIndex::Create(*g_dev, opts, vdbg::Metric::L2, base.view(), &c));
  CHECK(c->Load(bad).code() == VDBG_CORRUPTION);
}

void IvfPqExhaustiveWithFullRerankEqualsFlat() {
  // nprobe = nlist and a rerank depth covering every row: the answer is the exact one
  Data base = Clustered(250, 32, 5, 11, false), qs = Clustered(40, 32, 5, 12, false);
  vdbg::IndexOptions opts;
  opts.nlist = 6;
  opts.pq_m = 8;
  std::unique_ptr<vdbg::GpuIvfPqIndex> ix;
  CHECK_OK(vdbg::GpuIvfPqIndex::Create(*g_dev, opts, vdbg::Metric::L2, base.view(), &ix));
  CHECK_OK(ix->build());
  vdbg::SearchParams p;
  p.nprobe = ix->nlist();
  p.rerank = 256;
  std::vector<std::vector<vdbg::Neighbor>> got;
  CHECK_OK(ix->search_batch(qs.v.data(), qs.rows, 10, p, nullptr, got, nullptr));
  auto want = OracleFlat(base, qs.v.data(), qs.rows, 10, vdbg::Metric::L2, nullptr);
  for (size_t q = 0; q < qs.rows; ++q) CHECK(Same(got[q], want[q]));
}

void IvfPqSmallSegmentsShrinkNlist() {
  Data base = Clustered(390, 16, 4, 13, false);
  vdbg::IndexOptions opts;
  opts.nlist = 1024;
  opts.pq_m = 4;
  std::unique_ptr<vdbg::GpuIvfPqIndex> ix;
  CHECK_OK(vdbg::GpuIvfPqIndex::Create(*g_dev, opts, vdbg::Metric::L2, base.view(), &ix));
  CHECK_OK(ix->build());
  CHECK(ix->nlist() == 10u);  // clamp(nlist, 1, n / 39), ivf_pq.cc:104
}

void IvfPqMustDivideDim() {
  Data base = Clustered(100, 30, 2, 14, false);
  vdbg::IndexOptions opts;
  opts.pq_m = 7;
  std::unique_ptr<vdbg::GpuIvfPqIndex> ix;
  CHECK(vdbg::GpuIvfPqIndex::Create(*g_dev, opts, vdbg::Metric::L2, base.view(), &ix).code() ==
        VDBG_INVALID_ARGUMENT);
}

// ---------------------------------------------------------------- collection read path

void CollectionSearchMatchesOracleAtEverySelectivity() {
  const size_t dim = 48, k = 10, nq = 32;
  std::vector<Data> segs;
  std::vector<std::unique_ptr<vdbg::GpuFlatIndex>> idx;
  std::vector<std::vector<uint64_t>> ext;
  uint64_t next = 100;
  for (size_t s = 0; s < 3; ++s) {
    segs.push_back(Clustered(5000 + 1500 * s, dim, 12, 20 + s, true));
    idx.emplace_back();
    CHECK_OK(vdbg::GpuFlatIndex::Create(*g_dev, vdbg::Metric::Cosine, segs[s].view(), &idx[s]));
    ext.emplace_back();
    for (size_t r = 0; r < segs[s].rows; ++r) ext[s].push_back(next++);
  }
  for (size_t r = 0; r < 50; ++r) ext[2][r] = ext[0][r];  // an upsert visible in two segments
  Data raw = Clustered(nq, dim, 12, 30, false);
  for (float sel : {0.01f, 0.1f, 0.5f, 1.0f}) {
    std::vector<vdbg::DenseRowFilter> allow;
    std::vector<vdbg::SegmentRef> refs;
    Rng r{uint64_t(sel * 1000)};
    for (size_t s = 0; s < 3; ++s) {
      allow.emplace_back(segs[s].rows);
      for (uint32_t row = 0; row < segs[s].rows; ++row)
        if (r.uni() < sel) allow[s].Allow(row);
    }
    for (size_t s = 0; s < 3; ++s) refs.push_back({idx[s].get(), &allow[s], ext[s].data()});
    std::vector<float> rq(nq * dim);
    for (size_t q = 0; q < nq; ++q) std::memcpy(&rq[q * dim], raw.row(q), dim * 4);
    std::vector<std::vector<vdbg::SearchHit>> got;
    CHECK_OK(vdbg::SearchSegments(*g_dev, refs, vdbg::Metric::Cosine, rq.data(), nq, dim, k, got));
    // oracle: prepare, per-segment filtered search, merge
    const size_t pd = vdbg::PaddedDim(dim);
    std::vector<float> q(nq * pd, 0.f);
    for (size_t i = 0; i < nq; ++i) {
      std::memcpy(&q[i * pd], &rq[i * dim], dim * 4);
      or_normalize(&q[i * pd], dim);
    }
    std::vector<uint64_t> all_ext, off;
    std::vector<std::vector<std::vector<vdbg::Neighbor>>> parts;
    for (size_t s = 0; s < 3; ++s) {
      off.push_back(all_ext.size());
      all_ext.insert(all_ext.end(), ext[s].begin(), ext[s].end());
      parts.push_back(OracleFlat(segs[s], q.data(), nq, k, vdbg::Metric::Cosine, &allow[s]));
    }
    for (size_t i = 0; i < nq; ++i) {
      std::vector<float> pdist(3 * k, INFINITY), od(k);
      std::vector<uint32_t> prow(3 * k, UINT32_MAX);
      std::vector<uint64_t> oe(k);
      for (size_t s = 0; s < 3; ++s)
        for (size_t j = 0; j < parts[s][i].size(); ++j) {
          pdist[s * k + j] = parts[s][i][j].dist;
          prow[s * k + j] = parts[s][i][j].id;
        }
      const size_t n = or_merge_parts(3, k, pdist.data(), prow.data(), all_ext.data(), off.data(),
                                      od.data(), oe.data());
      CHECK(got[i].size() == n);
      for (size_t j = 0; j < std::min(n, got[i].size()); ++j) {
        CHECK(got[i][j].id == oe[j]);
        CHECK(std::memcmp(&got[i][j].distance, &od[j], 4) == 0);
        CHECK(got[i][j].score == -od[j]);
      }
    }
  }
  // PrepareQuery's errors (collection_impl.cc:1026-1031)
  std::vector<float> bad(dim, 1.f);
  bad[3] = NAN;
  std::vector<std::vector<vdbg::SearchHit>> out;
  std::vector<vdbg::SegmentRef> refs{{idx[0].get(), nullptr, ext[0].data()}};
  CHECK(vdbg::SearchSegments(*g_dev, refs, vdbg::Metric::Cosine, bad.data(), 1, dim, k, out).code() ==
        VDBG_INVALID_ARGUMENT);
  std::vector<float> zero(dim, 0.f);
  CHECK(vdbg::SearchSegments(*g_dev, refs, vdbg::Metric::Cosine, zero.data(), 1, dim, k, out).code() ==
        VDBG_INVALID_ARGUMENT);
}

// ---------------------------------------------------------------- segment files (segment_reader.cc)

// File writers, field by field from the reference's layouts (segment_writer.cc:58-75,
// file_format.cc:8-18, index.cc:38-45, hnsw_index.cc:108-115, the portable roaring format).
template <class T>
void Put(std::string* s, T v) {
  s->append(reinterpret_cast<const char*>(&v), sizeof(T));
}

void WriteFile(const std::string& path, const std::string& bytes) {
  std::ofstream f(path, std::ios::binary);
  f.write(bytes.data(), std::streamsize(bytes.size()));
}

std::string Blob(const char* magic, const std::string& payload) {
  std::string b(magic, 8);
  Put<uint32_t>(&b, 1);
  Put<uint32_t>(&b, or_crc32c(0, payload.data(), payload.size()));
  Put<uint64_t>(&b, payload.size());
  return b + payload;
}

std::string IndexFile(const char* magic, const std::string& body) {
  std::string f = std::string(magic, 8) + body;
  Put<uint32_t>(&f, or_crc32c(0, f.data(), f.size()));
  return f;
}

std::string VectorsFile(const Data& d, vdbg::Metric m) {
  std::string h(4096, '\0');
  std::memcpy(h.data(), "VDBSEG01", 8);
  const uint64_t len = d.rows * d.pd * 4;
  auto put = [&](size_t off, auto v) { std::memcpy(h.data() + off, &v, sizeof(v)); };
  put(8, uint32_t(1));
  put(12, uint32_t(m));
  put(16, uint64_t(d.rows));
  put(24, uint32_t(d.dim));
  put(28, uint32_t(d.pd));
  put(32, uint64_t(4096));
  put(40, len);
  put(48, or_crc32c(0, d.v.data(), len));
  put(64, uint64_t(9));
  put(4092, or_crc32c(0, h.data(), 4092));
  return h + std::string(reinterpret_cast<const char*>(d.v.data()), len);
}

// A roaring bitmap of `rows` (ascending) in the portable format with array containers only
// (every container of at most 4096 rows): cookie 12346, count, (key, card - 1), offsets, values.
std::string RoaringArrays(const std::vector<uint32_t>& rows) {
  std::vector<std::pair<uint16_t, std::vector<uint16_t>>> cont;
  for (uint32_t r : rows) {
    if (cont.empty() || cont.back().first != (r >> 16)) cont.push_back({uint16_t(r >> 16), {}});
    cont.back().second.push_back(uint16_t(r & 0xffff));
  }
  std::string s;
  Put<uint32_t>(&s, 12346);
  Put<uint32_t>(&s, uint32_t(cont.size()));
  for (auto& [key, v] : cont) {
    Put<uint16_t>(&s, key);
    Put<uint16_t>(&s, uint16_t(v.size() - 1));
  }
  uint32_t off = uint32_t(s.size() + 4 * cont.size());
  for (auto& c : cont) {
    Put<uint32_t>(&s, off);
    off += uint32_t(2 * c.second.size());
  }
  for (auto& c : cont)
    for (uint16_t x : c.second) Put<uint16_t>(&s, x);
  return s;
}

struct SegFiles {
  Data rows;
  std::vector<uint64_t> ext;
  std::vector<uint32_t> deleted;
  std::vector<float> vmin, scale;  // HNSW-SQ8
  std::vector<uint8_t> codes;
  std::string file;                // the VDBHSQ81 index file
  IvfFile ivf;                     // IVF-PQ
};

// A small valid HNSW graph in HnswGraph::serialize's layout (hnsw_graph.h:352-366): every node
// on layer 0 only, linked to the nodes up to four places before and after it (M = 4, M0 = 8).
std::string ChainGraph(size_t rows) {
  const uint32_t M = 4, M0 = 2 * M;
  std::string g;
  Put<uint64_t>(&g, rows);
  Put<uint64_t>(&g, rows);
  Put<uint32_t>(&g, M);
  Put<uint32_t>(&g, 40);
  Put<uint64_t>(&g, 42);
  Put<uint32_t>(&g, 0);  // top layer
  Put<uint32_t>(&g, 0);  // entry point
  g.append(rows, '\0');  // levels
  for (size_t i = 0; i < rows; ++i) {
    std::vector<uint32_t> nb;
    for (int d = 1; d <= 4; ++d) {
      if (i + d < rows) nb.push_back(uint32_t(i + d));
      if (i >= size_t(d)) nb.push_back(uint32_t(i - d));
    }
    Put<uint32_t>(&g, uint32_t(nb.size()));
    for (uint32_t j = 0; j < M0; ++j) Put<uint32_t>(&g, j < nb.size() ? nb[j] : 0u);
  }
  return g;
}

std::string MakeSegmentDir(const std::string& root, uint32_t id, vdbg::IndexType t, vdbg::Metric m,
                           SegFiles& sf, uint64_t first_ext) {
  const std::string dir = root + "/seg-" + std::to_string(id);
  std::filesystem::create_directories(dir);
  WriteFile(dir + "/vectors.f32", VectorsFile(sf.rows, m));
  for (size_t r = 0; r < sf.rows.rows; ++r) sf.ext.push_back(first_ext + 5 * r);
  WriteFile(dir + "/ids.u64", Blob("VDBIDS01", std::string(reinterpret_cast<const char*>(sf.ext.data()),
                                                          sf.ext.size() * 8)));
  const Data& b = sf.rows;
  std::string file;
  if (t == vdbg::IndexType::Flat) {
    file = IndexFile("VDBFLAT1", "");
  } else if (t == vdbg::IndexType::HnswSq8) {
    sf.vmin.resize(b.pd);
    sf.scale.resize(b.pd);
    sf.codes.resize(b.rows * b.pd);
    or_sq8_train(b.v.data(), b.rows, b.dim, b.pd, sf.vmin.data(), sf.scale.data());
    or_sq8_encode_rows(b.v.data(), b.rows, b.dim, b.pd, sf.vmin.data(), sf.scale.data(), sf.codes.data());
    std::string body;
    Put<uint64_t>(&body, b.rows);
    Put<uint32_t>(&body, uint32_t(b.dim));
    Put<uint32_t>(&body, uint32_t(b.pd));
    body.append(reinterpret_cast<const char*>(sf.vmin.data()), b.pd * 4);
    body.append(reinterpret_cast<const char*>(sf.scale.data()), b.pd * 4);
    body.append(reinterpret_cast<const char*>(sf.codes.data()), sf.codes.size());
    body += ChainGraph(b.rows);
    file = IndexFile("VDBHSQ81", body);
    sf.file = file;
  } else {
    std::unique_ptr<vdbg::GpuIvfPqIndex> ix;
    vdbg::IndexOptions o;
    o.nlist = 40;
    o.pq_m = 8;
    o.kmeans_iters = 8;
    if (!vdbg::GpuIvfPqIndex::Create(*g_dev, o, m, b.view(), &ix).ok() || !ix->build().ok() ||
        !ix->Save(&file).ok())
      return "";
    ParseIvf(file, &sf.ivf);
  }
  WriteFile(dir + "/index." + vdbg::IndexTypeName(t), file);
  if (!sf.deleted.empty())
    WriteFile(dir + "/deletes-000003.roar", Blob("VDBDEL01", RoaringArrays(sf.deleted)));
  return dir;
}

// The oracle's view of one segment's index search (flat / SQ8 scan + rerank / IVF-PQ) for
// every query, allowed rows only.
std::vector<std::vector<vdbg::Neighbor>> OracleSegment(const SegFiles& sf, vdbg::IndexType t,
                                                       vdbg::Metric m, const float* q, size_t nq,
                                                       size_t k, const vdbg::SearchParams& p,
                                                       const vdbg::DenseRowFilter* allow) {
  if (t == vdbg::IndexType::Flat) return OracleFlat(sf.rows, q, nq, k, m, allow);
  const Data& b = sf.rows;
  std::vector<float> d(nq * k);
  std::vector<uint32_t> id(nq * k);
  if (t == vdbg::IndexType::HnswSq8) {  // HnswSq8Index::search over the file's graph
    CHECK(or_hnsw_sq8_search_file(Kset(), int(m), reinterpret_cast<const uint8_t*>(sf.file.data()),
                                  sf.file.size(), b.v.data(), b.rows, b.pd, q, nq, k, p.ef,
                                  p.rerank, allow && !sf.deleted.empty() ? allow->words() : nullptr,
                                  d.data(), id.data(), nullptr, 8) == 0);
  } else {
    const IvfFile& f = sf.ivf;
    std::vector<float> term2(f.nlist * f.m * 256);
    or_ivfpq_term2(f.coarse.data(), f.nlist, f.pd, f.cen.data(), f.m, f.dim / f.m, term2.data());
    std::vector<uint64_t> dc(nq);
    or_ivfpq_search_batch(Kset(), int(m), b.v.data(), b.dim, b.pd, f.coarse.data(), f.nlist,
                          f.cen.data(), f.m, f.off.data(), f.ids.data(), f.codes.data(),
                          m == vdbg::Metric::L2 ? term2.data() : nullptr, q, nq, k, p.nprobe,
                          p.rerank, allow ? allow->words() : nullptr, d.data(), id.data(),
                          dc.data(), 8);
  }
  std::vector<std::vector<vdbg::Neighbor>> out(nq);
  for (size_t i = 0; i < nq; ++i)
    for (size_t j = 0; j < k && id[i * k + j] != UINT32_MAX; ++j) out[i].push_back({d[i * k + j], id[i * k + j]});
  return out;
}

void SegmentOpenAndCollectionSearch() {
  char tmpl[] = "/tmp/vdbg_segments_XXXXXX";
  const char* root_c = mkdtemp(tmpl);
  CHECK(root_c != nullptr);
  if (root_c == nullptr) return;
  const std::string root = root_c;
  const size_t dim = 40, k = 10, nq = 24;
  const vdbg::Metric m = vdbg::Metric::L2;
  const vdbg::IndexType types[3] = {vdbg::IndexType::Flat, vdbg::IndexType::HnswSq8,
                                    vdbg::IndexType::IvfPq};
  std::vector<SegFiles> sf(3);
  std::vector<std::unique_ptr<vdbg::GpuSegment>> seg(3);
  for (size_t s = 0; s < 3; ++s) {
    sf[s].rows = Clustered(3000 + 2000 * s, dim, 16, 50 + s, false);
    if (s != 1)
      for (uint32_t r = 7; r < sf[s].rows.rows; r += 31) sf[s].deleted.push_back(r);
    const std::string dir = MakeSegmentDir(root, uint32_t(s), types[s], m, sf[s], 1000000 * (s + 1));
    CHECK(!dir.empty());
    vdbg::SegmentMeta meta{uint32_t(s), sf[s].rows.rows, sf[s].deleted.empty() ? "" : "deletes-000003.roar"};
    vdbg::CollectionOptions opts{dim, m, types[s]};
    CHECK_OK(vdbg::GpuSegment::Open(*g_dev, dir, meta, opts, true, &seg[s]));
    CHECK(seg[s]->index_type() == types[s]);
    CHECK(seg[s]->deleted_count() == sf[s].deleted.size());
    CHECK(seg[s]->external_id(3) == sf[s].ext[3]);
  }
  Data raw = Clustered(nq, dim, 16, 70, false);
  std::vector<float> rq(nq * dim);
  for (size_t q = 0; q < nq; ++q) std::memcpy(&rq[q * dim], raw.row(q), dim * 4);
  std::vector<const vdbg::GpuSegment*> segs{seg[0].get(), seg[1].get(), seg[2].get()};
  vdbg::SearchParams p;
  p.nprobe = 6;
  {  // GpuHnswSq8Index on its own over segment 1's file: graph walk + GPU rerank
    std::unique_ptr<vdbg::GpuHnswSq8Index> hx;
    CHECK_OK(vdbg::GpuHnswSq8Index::Load(*g_dev, m, sf[1].rows.view(), sf[1].file, &hx));
    const size_t pd = vdbg::PaddedDim(dim);
    std::vector<float> q(nq * pd, 0.f);
    for (size_t i = 0; i < nq; ++i) std::memcpy(&q[i * pd], &rq[i * dim], dim * 4);
    for (int rr : {-1, 0, 25}) {
      vdbg::SearchParams hp;
      hp.ef = 20;
      hp.rerank = rr;
      std::vector<std::vector<vdbg::Neighbor>> got;
      CHECK_OK(hx->search_batch(q.data(), nq, k, hp, nullptr, got, nullptr));
      const auto want = OracleSegment(sf[1], vdbg::IndexType::HnswSq8, m, q.data(), nq, k, hp, nullptr);
      for (size_t i = 0; i < nq; ++i) {
        CHECK(got[i].size() == want[i].size());
        for (size_t j = 0; j < std::min(got[i].size(), want[i].size()); ++j)
          CHECK(got[i][j].id == want[i][j].id && std::memcmp(&got[i][j].dist, &want[i][j].dist, 4) == 0);
      }
    }
  }
  for (int with_filter = 0; with_filter < 2; ++with_filter) {
    std::vector<vdbg::DenseRowFilter> filt;
    std::vector<const vdbg::DenseRowFilter*> fp;
    std::vector<vdbg::DenseRowFilter> allow;  // what each segment's search may return
    for (size_t s = 0; s < 3; ++s) {
      filt.emplace_back(sf[s].rows.rows);
      Rng r{900 + s};
      for (uint32_t row = 0; row < sf[s].rows.rows; ++row)
        if (r.uni() < 0.4f) filt[s].Allow(row);
      allow.push_back(with_filter ? filt[s] : vdbg::DenseRowFilter(sf[s].rows.rows, true));
      for (uint32_t d : sf[s].deleted) allow[s].Deny(d);
    }
    for (auto& f : filt) fp.push_back(&f);
    std::vector<std::vector<vdbg::SearchHit>> got;
    std::vector<uint64_t> dc;
    std::vector<std::string> plans;
    CHECK_OK(vdbg::SearchCollection(*g_dev, segs, dim, m, rq.data(), nq, k, p,
                                    with_filter ? &fp : nullptr, got, &dc, &plans));
    // every segment matches > 1000 rows but fewer than the 10,000 threshold: exact under a
    // filter; otherwise each segment's own index under its deletes
    for (size_t s = 0; s < 3; ++s) CHECK(plans[s] == (with_filter ? "prefilter_exact" : "index"));
    const size_t pd = vdbg::PaddedDim(dim);
    std::vector<float> q(nq * pd, 0.f);
    for (size_t i = 0; i < nq; ++i) std::memcpy(&q[i * pd], &rq[i * dim], dim * 4);
    std::vector<std::vector<std::vector<vdbg::Neighbor>>> parts;
    std::vector<uint64_t> all_ext, off;
    for (size_t s = 0; s < 3; ++s) {
      parts.push_back(with_filter ? OracleFlat(sf[s].rows, q.data(), nq, k, m, &allow[s])
                                  : OracleSegment(sf[s], types[s], m, q.data(), nq, k, p, &allow[s]));
      off.push_back(all_ext.size());
      all_ext.insert(all_ext.end(), sf[s].ext.begin(), sf[s].ext.end());
    }
    for (size_t i = 0; i < nq; ++i) {
      std::vector<float> pdist(3 * k, INFINITY), od(k);
      std::vector<uint32_t> prow(3 * k, UINT32_MAX);
      std::vector<uint64_t> oe(k);
      for (size_t s = 0; s < 3; ++s)
        for (size_t j = 0; j < parts[s][i].size(); ++j) {
          pdist[s * k + j] = parts[s][i][j].dist;
          prow[s * k + j] = parts[s][i][j].id;
        }
      const size_t n = or_merge_parts(3, k, pdist.data(), prow.data(), all_ext.data(), off.data(),
                                      od.data(), oe.data());
      CHECK(got[i].size() == n);
      for (size_t j = 0; j < std::min(n, got[i].size()); ++j) {
        CHECK(got[i][j].id == oe[j]);
        CHECK(std::memcmp(&got[i][j].distance, &od[j], 4) == 0);
      }
    }
  }
  // deletes after open: DeleteBits::set hides the row from the next search
  std::vector<std::vector<vdbg::SearchHit>> a, b;
  CHECK_OK(vdbg::SearchCollection(*g_dev, segs, dim, m, rq.data(), 1, 1, p, nullptr, a));
  CHECK(a.size() == 1 && a[0].size() == 1);
  for (size_t s = 0; s < 3; ++s)
    for (uint32_t r = 0; r < seg[s]->rows(); ++r)
      if (seg[s]->external_id(r) == a[0][0].id) seg[s]->Delete(r);
  CHECK_OK(vdbg::SearchCollection(*g_dev, segs, dim, m, rq.data(), 1, 1, p, nullptr, b));
  CHECK(b[0].size() == 1 && b[0][0].id != a[0][0].id);

  // what Segment::Open rejects
  std::unique_ptr<vdbg::GpuSegment> bad;
  const std::string d0 = root + "/seg-0";
  vdbg::CollectionOptions flat{dim, m, vdbg::IndexType::Flat};
  CHECK(vdbg::GpuSegment::Open(*g_dev, root + "/none", {9, 3000, ""}, flat, true, &bad).code() == VDBG_IO_ERROR);
  CHECK(vdbg::GpuSegment::Open(*g_dev, d0, {0, 3001, ""}, flat, true, &bad).code() == VDBG_CORRUPTION);
  vdbg::CollectionOptions wrong_dim{dim + 1, m, vdbg::IndexType::Flat};
  CHECK(vdbg::GpuSegment::Open(*g_dev, d0, {0, 3000, ""}, wrong_dim, true, &bad).code() == VDBG_CORRUPTION);
  WriteFile(d0 + "/deletes-000004.roar", Blob("VDBDEL01", RoaringArrays({1, 2, 5000})));
  CHECK(vdbg::GpuSegment::Open(*g_dev, d0, {0, 3000, "deletes-000004.roar"}, flat, true, &bad).code() ==
        VDBG_CORRUPTION);  // a deleted row past the segment's end
  WriteFile(d0 + "/index.hnsw", IndexFile("VDBHNSW1", std::string(8, '\0')));
  vdbg::CollectionOptions hnsw{dim, m, vdbg::IndexType::Hnsw};
  CHECK(vdbg::GpuSegment::Open(*g_dev, d0, {0, 3000, ""}, hnsw, true, &bad).code() == VDBG_NOT_SUPPORTED);
  WriteFile(d0 + "/ids.u64", Blob("VDBIDS01", std::string(8 * 2999, '\0')));
  CHECK(vdbg::GpuSegment::Open(*g_dev, d0, {0, 3000, ""}, flat, true, &bad).code() == VDBG_CORRUPTION);
  seg.clear();
  std::filesystem::remove_all(root);
}

}  // namespace

// ---------------------------------------------------------------- coalesced one-query calls

// T threads each send one query at a time through a Coalescer, as vdb's pool workers call
// Index::search; every answer must equal the index's own search() of that query, neighbours,
// order, distance bits and distance computations.
template <class Ix>
void ConcurrentCallsMatch(const Ix& ix, const Data& qs, const std::vector<vdbg::SearchParams>& ps,
                          const vdbg::DenseRowFilter* filter, size_t max_batch) {
  std::unique_ptr<vdbg::Coalescer> co;
  CHECK_OK(vdbg::Coalescer::Create(ix, {max_batch, 20}, &co));
  struct Call {
    size_t q, k, p;
    bool filtered;
  };
  std::vector<Call> calls;
  for (size_t q = 0; q < qs.rows; ++q)
    for (size_t p = 0; p < ps.size(); ++p)
      for (size_t k : {size_t(1), size_t(10)})
        for (bool f : {false, true}) calls.push_back({q, k, p, f && filter != nullptr});
  std::vector<std::vector<vdbg::Neighbor>> got(calls.size());
  std::vector<uint64_t> dc(calls.size());
  std::vector<std::string> errs(16);
  std::vector<std::thread> pool;
  for (size_t t = 0; t < 16; ++t)
    pool.emplace_back([&, t] {
      for (size_t i = t; i < calls.size(); i += 16) {
        const Call& c = calls[i];
        vdbg::IndexSearchStats st;
        const vdbg::Status s = co->search(qs.row(c.q), c.k, ps[c.p], c.filtered ? filter : nullptr,
                                          got[i], &st);
        if (!s.ok()) {
          errs[t] = s.ToString();
          return;
        }
        dc[i] = st.distance_computations;
      }
    });
  for (auto& t : pool) t.join();
  for (const auto& e : errs) {
    CHECK(e.empty());
    if (!e.empty()) std::fprintf(stderr, "  %s: %s\n", g_test.c_str(), e.c_str());
  }
  for (size_t i = 0; i < calls.size(); ++i) {
    const Call& c = calls[i];
    std::vector<vdbg::Neighbor> want;
    vdbg::IndexSearchStats st;
    CHECK_OK(ix.search(qs.row(c.q), c.k, ps[c.p], c.filtered ? filter : nullptr, want, &st));
    CHECK(Same(got[i], want));
    CHECK(dc[i] == st.distance_computations);
  }
  uint64_t batches = 0, queries = 0;
  co->counts(&batches, &queries);
  CHECK(queries == calls.size() && batches >= 1 && batches <= queries);
}

void CoalescedCallsMatchSearch() {
  Data base = Clustered(20000, 64, 40, 21, false), qs = Clustered(40, 64, 40, 22, false);
  vdbg::DenseRowFilter some(base.rows);
  for (uint32_t r = 0; r < base.rows; ++r)
    if (r % 3 != 1) some.Allow(r);
  {
    std::unique_ptr<vdbg::GpuFlatIndex> ix;
    CHECK_OK(vdbg::GpuFlatIndex::Create(*g_dev, vdbg::Metric::L2, base.view(), &ix));
    ConcurrentCallsMatch(*ix, qs, {vdbg::SearchParams{}}, &some, 8);
    // and the oracle, for the unfiltered k = 10 answers
    std::unique_ptr<vdbg::Coalescer> co;
    CHECK_OK(vdbg::Coalescer::Create(*ix, {}, &co));
    auto want = OracleFlat(base, qs.v.data(), qs.rows, 10, vdbg::Metric::L2, nullptr);
    for (size_t q = 0; q < qs.rows; ++q) {
      std::vector<vdbg::Neighbor> out;
      CHECK_OK(co->search(qs.row(q), 10, {}, nullptr, out, nullptr));
      CHECK(Same(out, want[q]));
    }
  }
  {
    std::unique_ptr<vdbg::GpuSq8Index> ix;
    CHECK_OK(vdbg::GpuSq8Index::Create(*g_dev, vdbg::Metric::L2, base.view(), &ix));
    CHECK_OK(ix->build());
    vdbg::SearchParams a, b;
    a.ef = 40;
    b.rerank = 0;
    ConcurrentCallsMatch(*ix, qs, {a, b}, &some, 16);
  }
  {
    vdbg::IndexOptions opts;
    opts.nlist = 64;
    opts.pq_m = 16;
    std::unique_ptr<vdbg::GpuIvfPqIndex> ix;
    CHECK_OK(vdbg::GpuIvfPqIndex::Create(*g_dev, opts, vdbg::Metric::L2, base.view(), &ix));
    CHECK_OK(ix->build());
    vdbg::SearchParams a, b;
    a.nprobe = 8;
    a.rerank = 0;
    b.nprobe = 16;
    b.rerank = 50;
    ConcurrentCallsMatch(*ix, qs, {a, b}, &some, 12);
  }
}

int main() {
  std::unique_ptr<vdbg::Device> dev;
  vdbg::Status s = vdbg::Device::Open(0, &dev);
  if (!s.ok()) {
    std::fprintf(stderr, "no device: %s\n", s.ToString().c_str());
    return 2;
  }
  g_dev = dev.get();
  const std::pair<const char*, std::function<void()>> tests[] = {
      {"FlatTest.MatchesOracleForEveryMetric", FlatMatchesOracleForEveryMetric},
      {"FlatTest.BatchedMatchesSingleQuery", FlatBatchedMatchesSingleQuery},
      {"FlatTest.FilterIsRespected", FlatFilterIsRespected},
      {"FlatTest.KLargerThanRows", FlatKLargerThanRows},
      {"RerankTest.MatchesOracle", RerankMatchesOracle},
      {"Sq8Test.CodesAndSearchMatchOracle", Sq8CodesAndSearchMatchOracle},
      {"IndexTest.IvfPqBuildSearchSaveLoad", IvfPqBuildSearchSaveLoad},
      {"IndexTest.IvfPqExhaustiveWithFullRerankEqualsFlat", IvfPqExhaustiveWithFullRerankEqualsFlat},
      {"PqTest.SmallSegmentsShrinkNlist", IvfPqSmallSegmentsShrinkNlist},
      {"IndexTest.PqMustDivideDim", IvfPqMustDivideDim},
      {"FilteredSearchTest.CollectionSearchMatchesOracleAtEverySelectivity",
       CollectionSearchMatchesOracleAtEverySelectivity},
      {"SegmentTest.OpenFromFilesAndSearchCollection", SegmentOpenAndCollectionSearch},
      {"CoalescerTest.ConcurrentCallsMatchSearch", CoalescedCallsMatchSearch},
  };
  for (const auto& [name, fn] : tests) {
    g_test = name;
    const int before = g_failed;
    std::printf("[ RUN      ] %s\n", name);
    std::fflush(stdout);
    fn();
    std::printf("[ %s ] %s\n", g_failed == before ? "      OK" : " FAILED ", name);
    std::fflush(stdout);
  }
  std::printf("%d checks, %d failed\n", g_checks, g_failed);
  return g_failed == 0 ? 0 : 1;
}
