// collection.hip -- CollectionImpl::Search (src/engine/collection_impl.cc:1036-1112) over a
// snapshot's disk segments for a whole batch of queries, in one call on one stream.
//
// vdb runs SearchBatch (:1121-1135) as one Search per query on a thread pool, each calling
// SearchDiskSegment (src/engine/planner.cc:42-129) per segment and merging.  Here the batch
// stays on the device: PrepareQuery once for all queries, one device search per segment into
// a [segment][query][k] hit array (the planner's choice is per segment: it depends only on
// the segment's filter and deletes, not on the query), one merge kernel that reads each
// segment's resident external ids, one copy back.  A segment whose index this library does
// not hold (vdb's float-row HNSW) is searched by the caller on the host; its hits take the
// segment's place in the merge.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "vdbg_device.h"
#include "vdbg_internal.h"

namespace vdbg {
namespace {

size_t CountRows(const uint64_t* w, size_t rows) {
  size_t n = 0;
  for (size_t i = 0; i < rows / 64; ++i) n += size_t(__builtin_popcountll(w[i]));
  if (rows % 64) n += size_t(__builtin_popcountll(w[rows / 64] & ((uint64_t(1) << (rows % 64)) - 1)));
  return n;
}

// A device buffer freed on the stream when the call ends.
struct DevBuf {
  void* p = nullptr;
  hipStream_t s = nullptr;
  ~DevBuf() {
    if (p != nullptr) (void)hipFreeAsync(p, s);
  }
};

int Alloc(DevBuf* b, size_t bytes, hipStream_t s) {
  b->s = s;
  VDBG_HIP(hipMallocAsync(&b->p, std::max<size_t>(bytes, 256), s));
  return kOk;
}

struct SegPlan {
  int plan = VDBG_PLAN_INDEX;
  std::vector<uint64_t> allow;  // host words handed to the device search; empty = none
  size_t matches = 0;
  size_t nprobe = 0;
  int64_t allowed = -1;         // rows the words allow, when the scan may take it as known
};

// Lanes of the collection search: flat scans of different segments run side by side, each
// on its own stream with its own scratch (a segment's scan alone is too small to fill the
// GPU, and lanes keep the host from waiting on one before queuing the next).
int EnsureLanes(Ctx* c, int n) {
  while (int(c->lanes.size()) < n) {
    auto* l = new (std::nothrow) ScanScratch;
    if (l == nullptr) return SetError(kResourceExhausted, "out of host memory");
    if (hipStreamCreateWithFlags(&l->stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&l->done, hipEventDisableTiming) != hipSuccess) {
      delete l;
      return SetError(kInternal, "collection search lane");
    }
    c->lanes.push_back(l);
  }
  return kOk;
}

}  // namespace
}  // namespace vdbg

using namespace vdbg;

extern "C" {

int vdbg_dataset_set_external_ids(vdbg_dataset* ds, const uint64_t* ids) {
  if (ds == nullptr || (ids == nullptr && ds->d.n > 0)) return SetError(kInvalidArgument, "null argument");
  Dataset& d = ds->d;
  Ctx* c = d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  if (d.n == 0) return kOk;
  if (d.ext_ids == nullptr) VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&d.ext_ids), d.n * 8));
  VDBG_HIP(hipMemcpyAsync(d.ext_ids, ids, d.n * 8, hipMemcpyHostToDevice, c->stream));
  // whether every row has its own external id (the combined scan of the collection search
  // relies on it; vdb's segments hold each id once)
  std::vector<uint64_t> sorted(ids, ids + d.n);
  std::sort(sorted.begin(), sorted.end());
  d.ext_unique = std::adjacent_find(sorted.begin(), sorted.end()) == sorted.end();
  VDBG_HIP(hipStreamSynchronize(c->stream));
  return kOk;
}

}  // extern "C"

namespace {

// Largest number of allowed rows, over all segments, scanned as one combined source (past it,
// gathering the rows costs more than the separate scans' fixed costs: measured at 8 x 625,000
// x 384, 49k rows 1.09 ms combined against 1.50 on lanes, 490k rows 4.28 against 3.66).
constexpr size_t kCombinedMaxRows = size_t(1) << 18;

// A collection of flat segments whose allowed rows are few in all, scanned as one source:
// every segment's allowed rows (ascending, segment by segment) gathered into one row set with
// their external ids, one scan for the top k x nseg of that set by (dist, index), then the
// merge keeping the first hit of each external id, k of them.  The index order is the
// (part, row) order, so the order is vdb's merge order.  With every external id held once
// inside its segment, the first k distinct ids of all rows in that order are the first k of
// vdb's merge of per-segment top-k lists (a hit in the answer has fewer than k hits of its
// own segment before it: each is either in the answer or repeats an answer id held by another
// segment), and every one of them is among the first k x nseg rows of the order (at most
// nseg rows carry each answer id).
int CombinedScan(Ctx* c, const vdbg_segment* segs, size_t nseg, const std::vector<int64_t>& rows,
                 const std::vector<const uint64_t*>& allow, const float* q, size_t nq,
                 size_t k, uint64_t* out_ext, float* out_d, hipStream_t s) {
  const Dataset& d0 = segs[0].rows->d;
  const ScanSource& s0 = d0.src;
  const size_t pd = d0.pd;
  const size_t kk = k * nseg;
  size_t total = 0;
  for (int64_t r : rows) total += size_t(r);
  ScanSource cs;
  cs.kind = 0;
  cs.N = uint32_t(total);
  cs.pd = int(pd);
  cs.metric = s0.metric;
  cs.x16_parts = s0.x16_parts;
  cs.x16_exp = s0.x16_exp;
  cs.x16_approx = s0.x16_approx;
  cs.X16 = s0.X16;  // (non-null while the sample is sized: the sample keeps an fp16 part)
  cs.stats = s0.stats;
  cs.rmag = s0.rmag;
  for (size_t p = 1; p < nseg; ++p) {
    const ScanSource& sp = segs[p].rows->d.src;
    cs.stats.lo = std::min(cs.stats.lo, sp.stats.lo);
    cs.stats.hi = std::max(cs.stats.hi, sp.stats.hi);
    cs.stats.max_abs = std::max(cs.stats.max_abs, sp.stats.max_abs);
    cs.stats.xn_max = std::max(cs.stats.xn_max, sp.stats.xn_max);
    cs.stats.all_int &= sp.stats.all_int;
    cs.rmag = std::max(cs.rmag, sp.rmag);
  }
  const size_t row16 = s0.X16 != nullptr ? pd * size_t(s0.x16_parts) * 2 : 0;
  const size_t sample_bytes = SampleBytes(cs, SampleRows(uint32_t(total)));
  Workspace& w = c->wcomb;
  if (c->wcomb_done != nullptr) VDBG_HIP(hipStreamWaitEvent(s, c->wcomb_done, 0));
  w.used = 0;
  const size_t bytes = total * (4 + 8 + pd * 4 + row16 + 4) + sample_bytes +
                       nq * kk * 8 + 12 * 256;
  VDBG_RETURN_IF_ERROR(w.reserve(bytes));
  uint32_t* ids = w.take<uint32_t>(total);
  uint64_t* ext = w.take<uint64_t>(total);
  float* X = w.take<float>(total * pd);
  uint16_t* X16 = row16 != 0 ? reinterpret_cast<uint16_t*>(w.take<char>(total * row16)) : nullptr;
  float* rn = w.take<float>(total);
  void* sample = w.take<char>(sample_bytes);
  uint32_t* cids = w.take<uint32_t>(nq * kk);
  float* cd = w.take<float>(nq * kk);
  {
    ProfScope ps(c, "compact", s);
    // the segments' masks compacted in one launch and their rows gathered in another, up to
    // kMultiParts segments at a time
    CompactMulti cm{};
    GatherMulti gm{};
    auto flush = [&]() -> int {
      VDBG_RETURN_IF_ERROR(CompactGatherMulti(cm, gm, s));
      cm.n = 0;
      gm.n = 0;
      return kOk;
    };
    size_t at = 0;
    for (size_t p = 0; p < nseg; ++p) {
      const Dataset& d = segs[p].rows->d;
      const uint32_t n = uint32_t(rows[p]);
      if (n == 0) continue;
      if (cm.n == kMultiParts || gm.n == kMultiParts) VDBG_RETURN_IF_ERROR(flush());
      if (allow[p] != nullptr) {
        const size_t nwords = (d.n + 63) / 64;
        if (nwords > size_t(kCompactBlockWords) || n > kCompactBlockIds)
          return SetError(kInternal, "combined scan: mask too large");
        cm.w[cm.n] = allow[p];
        cm.ids[cm.n] = ids + at;
        cm.nwords[cm.n] = uint32_t(nwords);
        cm.N[cm.n] = uint32_t(d.n);
        ++cm.n;
      }
      GatherParts g{};
      g.a = reinterpret_cast<const uint4*>(d.src.X);
      g.ao = reinterpret_cast<uint4*>(X + at * pd);
      g.wa = uint32_t(pd * 4 / 16);
      if (row16 != 0) {
        g.b = reinterpret_cast<const uint4*>(d.src.X16);
        g.bo = reinterpret_cast<uint4*>(reinterpret_cast<char*>(X16) + at * row16);
        g.wb = uint32_t(row16 / 16);
      }
      g.rn = d.src.rn;
      g.rno = rn + at;
      g.ext = d.ext_ids;
      g.exto = ext + at;
      g.ids = allow[p] != nullptr ? ids + at : nullptr;
      g.n = n;
      gm.g[gm.n] = g;
      gm.start[gm.n + 1] = gm.start[gm.n] + uint64_t(n) * (g.wa + g.wb + g.wc + 1);
      ++gm.n;
      at += n;
    }
    VDBG_RETURN_IF_ERROR(flush());
  }
  cs.X = X;
  cs.X16 = X16;
  cs.rn = rn;
  cs.Sbuf = nullptr;
  // only as many sample rows as the one scan below uses
  VDBG_RETURN_IF_ERROR(GatherSample(c, &cs, s, sample, SampleWant(c, cs, nq, kk)));
  int rc = RunScan(c, &cs, q, nq, kk, nullptr, cids, cd, s);
  if (rc == kOk) {
    MergeArgs a{int(nq), 1, int(kk), cd, cids, ext, nullptr, out_ext, out_d};
    a.kout = int(k);
    rc = MergeParts(c, a, s);
  }
  if (c->wcomb_done == nullptr &&
      hipEventCreateWithFlags(&c->wcomb_done, hipEventDisableTiming) != hipSuccess)
    c->wcomb_done = nullptr;
  if (c->wcomb_done == nullptr || hipEventRecord(c->wcomb_done, s) != hipSuccess)
    (void)hipStreamSynchronize(s);  // no event: drain before the rows are reused
  FreeSample(&cs);  // (the sample lives in the workspace: nothing is freed)
  return rc;
}

// The collection search of vdbg_collection_search_host (queries and results in host memory)
// and vdbg_collection_search_device (in device memory, on `stream`).
int CollectionSearch(vdbg_ctx* ctx, const vdbg_segment* segs, size_t nseg, size_t dim,
                     int metric, const float* queries, size_t nq, size_t k,
                     const vdbg_search_params* params, uint64_t* out_ids, float* out_dists,
                     uint64_t* dist_comps, int* seg_plans, bool device_io, void* stream) {
  if (ctx == nullptr || params == nullptr || (nseg > 0 && segs == nullptr) ||
      (nq > 0 && (queries == nullptr || out_ids == nullptr || out_dists == nullptr)))
    return SetError(kInvalidArgument, "null argument");
  // collection_impl.cc:1038-1039
  if (k == 0 || k > 10000) return SetError(kInvalidArgument, "k must be in 1..10000");
  if (dim == 0 || metric < 0 || metric > 2) return SetError(kInvalidArgument, "bad dim or metric");
  if (params->strategy < VDBG_STRATEGY_AUTO || params->strategy > VDBG_STRATEGY_POST_FILTER)
    return SetError(kInvalidArgument, "unknown filter strategy");
  if (nq > 0x7fffffffull) return SetError(kInvalidArgument, "too many queries");
  const size_t pd = (dim + 15) / 16 * 16;
  Ctx* c = &ctx->c;
  for (size_t p = 0; p < nseg; ++p) {
    const vdbg_segment& g = segs[p];
    if (g.host_rows != nullptr) {  // searched on the host: its lists are checked below
      if (g.memory_part)
        return SetError(kInvalidArgument, "an in-memory part is searched here, not on the host");
      if (nq > 0 && (g.host_dists == nullptr || g.host_ext == nullptr))
        return SetError(kInvalidArgument, "host-searched segment without distances or ids");
      for (size_t i = 0; i < nq; ++i) {
        const float* d = g.host_dists + i * k;
        const uint32_t* r = g.host_rows + i * k;
        size_t j = 0;
        for (; j < k && r[j] != kNoId; ++j) {
          if (std::isnan(d[j]))
            return SetError(kInvalidArgument, "host-searched segment: NaN distance");
          if (j > 0 && (d[j] < d[j - 1] || (d[j] == d[j - 1] && r[j] <= r[j - 1])))
            return SetError(kInvalidArgument, "host-searched segment: hits not in ascending "
                                              "(dist, row) order");
        }
        for (; j < k; ++j)
          if (r[j] != kNoId)
            return SetError(kInvalidArgument, "host-searched segment: a hit after the end of "
                                              "its list");
      }
      continue;
    }
    if (g.rows == nullptr) return SetError(kInvalidArgument, "segment without rows");
    const Dataset& d = g.rows->d;
    if (d.ctx != c) return SetError(kInvalidArgument, "segment on another context");
    if (d.dim != dim || d.pd != pd || d.metric != metric)
      return SetError(kInvalidArgument, "segment dim or metric differs from the collection's");
    if (int(g.sq8 != nullptr) + int(g.ivfpq != nullptr) + int(g.pqflat != nullptr) > 1)
      return SetError(kInvalidArgument, "a segment has one index: sq8, ivfpq or pqflat");
    if (g.memory_part && (g.sq8 != nullptr || g.ivfpq != nullptr || g.pqflat != nullptr))
      return SetError(kInvalidArgument, "an in-memory part has no index");
    if ((g.sq8 != nullptr && g.sq8->q.ds != &d) || (g.ivfpq != nullptr && g.ivfpq->x.ds != &d) ||
        (g.pqflat != nullptr && g.pqflat->p.ds != &d))
      return SetError(kInvalidArgument, "index does not belong to the segment's rows");
    if (d.n > 0 && d.ext_ids == nullptr)
      return SetError(kFailedPrecondition, "segment has no external ids (vdbg_dataset_set_external_ids)");
  }
  std::lock_guard<std::recursive_mutex> lk(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = device_io && stream != nullptr ? static_cast<hipStream_t>(stream) : c->stream;
  if (dist_comps != nullptr) std::fill(dist_comps, dist_comps + nq, uint64_t(0));

  // ---- the plan of every segment (SearchDiskSegment, planner.cc:53-128)
  const vdbg_search_params& P = *params;
  std::vector<SegPlan> plan(nseg);
  size_t allow_words_total = 0;
  for (size_t p = 0; p < nseg; ++p) {
    const vdbg_segment& g = segs[p];
    if (g.host_rows != nullptr) {
      plan[p].plan = VDBG_PLAN_HOST;
      continue;
    }
    const size_t rows = g.rows->d.n, nw = (rows + 63) / 64;
    const size_t deleted = g.deleted_words ? CountRows(g.deleted_words, rows) : 0;
    const size_t live = rows - std::min(rows, deleted);
    SegPlan& sp = plan[p];
    sp.nprobe = P.nprobe;
    if (g.memory_part) {
      // SearchMutable (planner.cc:131-151): MutableSegment::Search scores every row that is
      // not deleted and matches the filter (mutable_segment.cc:46-64)
      sp.plan = g.filter_words != nullptr ? VDBG_PLAN_SCAN_FILTER : VDBG_PLAN_SCAN;
      if (g.filter_words != nullptr || deleted > 0) {
        sp.allow.assign(nw, ~uint64_t(0));
        if (g.filter_words != nullptr)
          for (size_t i = 0; i < nw; ++i) sp.allow[i] &= g.filter_words[i];
        if (deleted > 0)
          for (size_t i = 0; i < nw; ++i) sp.allow[i] &= ~g.deleted_words[i];
        if (rows % 64 && nw > 0) sp.allow[nw - 1] &= (uint64_t(1) << (rows % 64)) - 1;
        sp.matches = CountRows(sp.allow.data(), rows);
      } else {
        sp.matches = rows;
      }
      sp.allowed = int64_t(sp.matches);
      allow_words_total += sp.allow.size();
      continue;
    }
    if (g.filter_words == nullptr) {
      sp.plan = VDBG_PLAN_INDEX;  // :56-62, DeleteFilter when rows are deleted
      if (deleted > 0) {
        sp.allow.resize(nw);
        for (size_t i = 0; i < nw; ++i) sp.allow[i] = ~g.deleted_words[i];
        sp.allowed = int64_t(live);
      }
    } else {
      sp.allow.assign(g.filter_words, g.filter_words + nw);  // Evaluate, minus deletes (:64-65)
      if (deleted > 0)
        for (size_t i = 0; i < nw; ++i) sp.allow[i] &= ~g.deleted_words[i];
      if (rows % 64 && nw > 0) sp.allow[nw - 1] &= (uint64_t(1) << (rows % 64)) - 1;
      sp.matches = CountRows(sp.allow.data(), rows);
      sp.allowed = int64_t(sp.matches);
      const double sel = live == 0 ? 0.0 : double(sp.matches) / double(live);
      int strat = P.strategy;
      const bool flat = g.sq8 == nullptr && g.ivfpq == nullptr && g.pqflat == nullptr;
      if (strat == VDBG_STRATEGY_AUTO) {  // :70-80
        const double sv = std::max(sel, 1e-9);
        const double graph_cost = 10.0 * double(std::max(P.ef, k)) / sv;
        strat = (sp.matches <= P.prefilter_threshold || double(sp.matches) <= graph_cost || flat)
                    ? VDBG_STRATEGY_PREFILTER
                    : VDBG_STRATEGY_GRAPH;
      }
      if (sp.matches == 0) {
        sp.plan = VDBG_PLAN_EMPTY;
        sp.allow.clear();
      } else if (strat == VDBG_STRATEGY_PREFILTER) {
        sp.plan = VDBG_PLAN_PREFILTER_EXACT;
      } else if (strat == VDBG_STRATEGY_GRAPH) {
        sp.plan = VDBG_PLAN_FILTERED_INDEX;
        if (P.strategy == VDBG_STRATEGY_AUTO)  // :92-99
          sp.nprobe = std::max(P.nprobe, size_t(std::ceil(double(P.nprobe) / std::max(sel, 1e-9))));
      } else {
        sp.plan = VDBG_PLAN_POST_FILTER;
      }
    }
    allow_words_total += sp.allow.size();
  }

  if (nq == 0) {
    if (seg_plans != nullptr)
      for (size_t p = 0; p < nseg; ++p) seg_plans[p] = plan[p].plan;
    return kOk;
  }

  // ---- PrepareQuery for the batch (collection_impl.cc:1023-1034)
  DevBuf raw, Q, hits_d, hits_r, allow_dev, dcb, extp, oe, od;
  const float* raw_q = queries;
  if (!device_io) {
    VDBG_RETURN_IF_ERROR(Alloc(&raw, nq * dim * 4, s));
    VDBG_HIP(hipMemcpyAsync(raw.p, queries, nq * dim * 4, hipMemcpyHostToDevice, s));
    raw_q = static_cast<const float*>(raw.p);
  }
  VDBG_RETURN_IF_ERROR(Alloc(&Q, nq * pd * 4, s));
  // the preparation runs while the host sets up the rest; its status is checked before any
  // search is queued
  PrepPending prep;
  VDBG_RETURN_IF_ERROR(PrepareQueriesLaunch(c, raw_q, nq, dim, pd, metric,
                                            static_cast<float*>(Q.p), s, &prep));
  const float* q = static_cast<const float*>(Q.p);

  const size_t np = std::max<size_t>(nseg, 1), slice = nq * k;
  VDBG_RETURN_IF_ERROR(Alloc(&hits_d, np * slice * 4, s));
  VDBG_RETURN_IF_ERROR(Alloc(&hits_r, np * slice * 4, s));
  VDBG_RETURN_IF_ERROR(Alloc(&allow_dev, allow_words_total * 8, s));
  VDBG_RETURN_IF_ERROR(Alloc(&dcb, nq * 8, s));
  std::vector<uint64_t> allow_all;
  allow_all.reserve(allow_words_total);
  std::vector<size_t> allow_at(nseg);
  for (size_t p = 0; p < nseg; ++p) {
    allow_at[p] = allow_all.size();
    allow_all.insert(allow_all.end(), plan[p].allow.begin(), plan[p].allow.end());
  }
  if (!allow_all.empty())
    VDBG_HIP(hipMemcpyAsync(allow_dev.p, allow_all.data(), allow_all.size() * 8,
                            hipMemcpyHostToDevice, s));
  VDBG_RETURN_IF_ERROR(PrepareQueriesCheck(&prep));
  std::vector<uint64_t> dch(nq);

  // One index search of segment p into (ids, dists) [nq][kk] with the given allow words:
  // Index::search of the segment's index type, adding its distance computations.
  auto index_search = [&](size_t p, size_t kk, size_t nprobe, const uint64_t* allow,
                          uint32_t* ids, float* dd, size_t ef) -> int {
    const vdbg_segment& g = segs[p];
    const size_t rows = g.rows->d.n;
    if (g.pqflat != nullptr) {  // PqFlatIndex::search (ivf_pq.cc:59-79)
      VDBG_RETURN_IF_ERROR(vdbg_pqflat_search_device(g.pqflat, q, nq, kk, P.rerank, allow, ids, dd,
                                                     static_cast<uint64_t*>(dcb.p), s));
      VDBG_HIP(hipMemcpyAsync(dch.data(), dcb.p, nq * 8, hipMemcpyDeviceToHost, s));
      VDBG_HIP(hipStreamSynchronize(s));
      if (dist_comps != nullptr)
        for (size_t i = 0; i < nq; ++i) dist_comps[i] += dch[i];
    } else if (g.ivfpq != nullptr) {
      VDBG_RETURN_IF_ERROR(vdbg_ivfpq_search_device(g.ivfpq, q, nq, kk, nprobe, P.rerank, allow,
                                                    ids, dd, static_cast<uint64_t*>(dcb.p), s));
      VDBG_HIP(hipMemcpyAsync(dch.data(), dcb.p, nq * 8, hipMemcpyDeviceToHost, s));
      VDBG_HIP(hipStreamSynchronize(s));
      if (dist_comps != nullptr)
        for (size_t i = 0; i < nq; ++i) dist_comps[i] += dch[i];
    } else if (g.sq8 != nullptr && g.sq8->q.graph != nullptr) {
      // HnswSq8Index::search (hnsw_index.cc:82-100): the graph walk on the host, the rerank
      // on the device; ef as the caller's plan sets it
      VDBG_RETURN_IF_ERROR(vdbg_sq8_hnsw_search_device(g.sq8, q, nq, kk, ef, P.rerank, allow, ids,
                                                       dd, static_cast<uint64_t*>(dcb.p), s));
      VDBG_HIP(hipMemcpyAsync(dch.data(), dcb.p, nq * 8, hipMemcpyDeviceToHost, s));
      VDBG_HIP(hipStreamSynchronize(s));
      if (dist_comps != nullptr)
        for (size_t i = 0; i < nq; ++i) dist_comps[i] += dch[i];
    } else if (g.sq8 != nullptr) {
      // this library's SQ8 scan index (vdbg_sq8_create, no graph): every code, with
      // HnswSq8Index::search's depth rule (hnsw_index.cc:88)
      const size_t depth = P.rerank < 0 ? std::max(ef, kk) : size_t(P.rerank);
      VDBG_RETURN_IF_ERROR(vdbg_sq8_search_device(g.sq8, q, nq, kk, depth, allow, ids, dd, s));
      if (dist_comps != nullptr)
        for (size_t i = 0; i < nq; ++i)
          dist_comps[i] += rows + (depth > 0 ? std::min(std::max(depth, kk), rows) : 0);
    } else {
      VDBG_RETURN_IF_ERROR(vdbg_flat_search_device(g.rows, q, nq, kk, allow, ids, dd, s));
      if (dist_comps != nullptr)
        for (size_t i = 0; i < nq; ++i) dist_comps[i] += rows;  // flat_index.cc:75-76
    }
    return kOk;
  };
  // ExactOverBitmap (planner.cc:31-38): the exact scan of the allowed rows.
  auto exact = [&](size_t p, const uint64_t* allow, uint32_t* ids, float* dd) -> int {
    VDBG_RETURN_IF_ERROR(vdbg_flat_search_device(segs[p].rows, q, nq, k, allow, ids, dd, s));
    if (dist_comps != nullptr)
      for (size_t i = 0; i < nq; ++i) dist_comps[i] += plan[p].matches;
    return kOk;
  };

  // flat scans (in-memory parts, flat segments under their index plan, the exact scan of a
  // prefilter plan) go to the lanes; every other plan runs on s in turn
  auto on_lane = [&](size_t p) {
    const int pl = plan[p].plan;
    const vdbg_segment& g = segs[p];
    return pl == VDBG_PLAN_SCAN || pl == VDBG_PLAN_SCAN_FILTER || pl == VDBG_PLAN_PREFILTER_EXACT ||
           (pl == VDBG_PLAN_INDEX && g.sq8 == nullptr && g.ivfpq == nullptr && g.pqflat == nullptr);
  };

  // ---- every segment a flat scan and few allowed rows in all: one combined scan
  {
    bool ok = c->combine_segments && nseg >= 2 && nq >= 3 && k * nseg <= 240;
    std::vector<int64_t> rows(nseg, 0);
    std::vector<const uint64_t*> allow_p(nseg, nullptr);
    size_t total = 0;
    const ScanSource* s0 = nseg > 0 && segs[0].host_rows == nullptr ? &segs[0].rows->d.src : nullptr;
    for (size_t p = 0; p < nseg && ok; ++p) {
      const vdbg_segment& g = segs[p];
      ok = g.host_rows == nullptr && on_lane(p);
      if (!ok) break;
      const Dataset& d = g.rows->d;
      const ScanSource& sp = d.src;
      ok = d.ext_unique && sp.kind == 0 && sp.Xmap == nullptr && s0 != nullptr &&
           (sp.X16 == nullptr) == (s0->X16 == nullptr) && sp.x16_parts == s0->x16_parts &&
           sp.x16_exp == s0->x16_exp && sp.x16_approx == s0->x16_approx;
      if (!ok) break;
      const SegPlan& pl = plan[p];
      if (pl.allow.empty()) {
        rows[p] = int64_t(d.n);
      } else {
        rows[p] = pl.allowed;
        allow_p[p] = static_cast<const uint64_t*>(allow_dev.p) + allow_at[p];
        ok = pl.allowed >= 0 && uint64_t(pl.allowed) <= kCompactBlockIds &&
             (d.n + 63) / 64 <= size_t(kCompactBlockWords);
      }
      total += size_t(std::max<int64_t>(rows[p], 0));
    }
    if (ok && total >= 1 && total <= kCombinedMaxRows) {
      for (size_t p = 0; p < nseg; ++p) {
        if (dist_comps != nullptr) {
          const size_t n = plan[p].plan == VDBG_PLAN_INDEX ? segs[p].rows->d.n : plan[p].matches;
          for (size_t i = 0; i < nq; ++i) dist_comps[i] += n;  // flat_index.cc:75-76
        }
      }
      uint64_t* merge_ext = device_io ? out_ids : nullptr;
      float* merge_d = device_io ? out_dists : nullptr;
      if (!device_io) {
        VDBG_RETURN_IF_ERROR(Alloc(&oe, slice * 8, s));
        VDBG_RETURN_IF_ERROR(Alloc(&od, slice * 4, s));
        merge_ext = static_cast<uint64_t*>(oe.p);
        merge_d = static_cast<float*>(od.p);
      }
      VDBG_RETURN_IF_ERROR(ResetFallbacks(c, s));
      VDBG_RETURN_IF_ERROR(CombinedScan(c, segs, nseg, rows, allow_p, q, nq, k, merge_ext,
                                        merge_d, s));
      if (!device_io) {
        VDBG_HIP(hipMemcpyAsync(out_ids, oe.p, slice * 8, hipMemcpyDeviceToHost, s));
        VDBG_HIP(hipMemcpyAsync(out_dists, od.p, slice * 4, hipMemcpyDeviceToHost, s));
      }
      VDBG_HIP(hipStreamSynchronize(s));
      if (seg_plans != nullptr)
        for (size_t p = 0; p < nseg; ++p) seg_plans[p] = plan[p].plan;
      return kOk;
    }
  }
  size_t nlane_segs = 0;
  for (size_t p = 0; p < nseg; ++p) nlane_segs += on_lane(p) ? 1 : 0;
  const int nlanes = nlane_segs >= 2 && c->collection_lanes > 1
                         ? int(std::min<size_t>(size_t(c->collection_lanes), nlane_segs))
                         : 0;
  hipEvent_t fork = nullptr;
  if (nlanes > 0) {
    VDBG_RETURN_IF_ERROR(EnsureLanes(c, nlanes));
    VDBG_HIP(hipEventCreateWithFlags(&fork, hipEventDisableTiming));
    VDBG_HIP(hipEventRecord(fork, s));  // the prepared queries and the allow words
    for (int l = 0; l < nlanes; ++l) VDBG_HIP(hipStreamWaitEvent(c->lanes[l]->stream, fork, 0));
  }
  // the scans' fallback counts add up over the call's segments
  VDBG_RETURN_IF_ERROR(ResetFallbacks(c, s));
  struct Accumulate {
    Ctx* c;
    ~Accumulate() { c->fb_accumulate = false; }
  } acc{c};
  c->fb_accumulate = true;
  // each lane's segments, issued by the lane's own host thread (lane 0: this thread) when the
  // context runs lanes threaded: one thread alone spends more time issuing a segment's
  // launches than the GPU spends running them
  std::vector<std::vector<size_t>> lane_jobs(size_t(std::max(nlanes, 1)));
  int next_lane = 0;
  std::vector<uint32_t> hr, xr;
  std::vector<float> hd, xd;
  // host-searched segments: each hit's external id, resident for the merge, which reads it
  // as row q * k + i of the segment
  std::vector<DevBuf> host_ext(nseg);
  std::vector<std::vector<uint32_t>> host_pos(nseg);  // (kept until the copies complete)
  for (size_t p = 0; p < nseg; ++p) {
    SegPlan& sp = plan[p];
    uint32_t* ids = static_cast<uint32_t*>(hits_r.p) + p * slice;
    float* dd = static_cast<float*>(hits_d.p) + p * slice;
    const uint64_t* allow = sp.allow.empty() ? nullptr : static_cast<const uint64_t*>(allow_dev.p) + allow_at[p];
    if (nlanes > 0 && on_lane(p)) {
      lane_jobs[size_t(next_lane)].push_back(p);
      next_lane = (next_lane + 1) % nlanes;
      if (dist_comps != nullptr) {
        const size_t n = sp.plan == VDBG_PLAN_INDEX ? segs[p].rows->d.n : sp.matches;  // flat_index.cc:75-76
        for (size_t i = 0; i < nq; ++i) dist_comps[i] += n;
      }
      continue;
    }
    switch (sp.plan) {
      case VDBG_PLAN_SCAN:
      case VDBG_PLAN_SCAN_FILTER:
        VDBG_RETURN_IF_ERROR(vdbg_flat_search_device(segs[p].rows, q, nq, k, allow, ids, dd, s));
        if (dist_comps != nullptr)
          for (size_t i = 0; i < nq; ++i) dist_comps[i] += sp.matches;
        break;
      case VDBG_PLAN_INDEX:
        VDBG_RETURN_IF_ERROR(index_search(p, k, sp.nprobe, allow, ids, dd, P.ef));
        break;
      case VDBG_PLAN_HOST: {
        const vdbg_segment& g = segs[p];
        std::vector<uint32_t>& pos = host_pos[p];
        pos.resize(slice);
        for (size_t i = 0; i < slice; ++i) pos[i] = g.host_rows[i] == kNoId ? kNoId : uint32_t(i);
        VDBG_RETURN_IF_ERROR(Alloc(&host_ext[p], slice * 8, s));
        VDBG_HIP(hipMemcpyAsync(ids, pos.data(), slice * 4, hipMemcpyHostToDevice, s));
        VDBG_HIP(hipMemcpyAsync(dd, g.host_dists, slice * 4, hipMemcpyHostToDevice, s));
        VDBG_HIP(hipMemcpyAsync(host_ext[p].p, g.host_ext, slice * 8, hipMemcpyHostToDevice, s));
        if (dist_comps != nullptr && g.host_dist_comps != nullptr)
          for (size_t i = 0; i < nq; ++i) dist_comps[i] += g.host_dist_comps[i];
        break;
      }
      case VDBG_PLAN_EMPTY:
        VDBG_HIP(hipMemsetAsync(ids, 0xff, slice * 4, s));
        VDBG_HIP(hipMemsetAsync(dd, 0, slice * 4, s));
        break;
      case VDBG_PLAN_PREFILTER_EXACT:
        VDBG_RETURN_IF_ERROR(exact(p, allow, ids, dd));
        break;
      case VDBG_PLAN_FILTERED_INDEX: {
        VDBG_RETURN_IF_ERROR(index_search(p, k, sp.nprobe, allow, ids, dd, P.ef));
        if (P.strategy != VDBG_STRATEGY_AUTO) break;
        // :103-108: never fewer than min(k, matches) hits; the short queries take the exact
        // scan of the allowed rows
        hr.resize(slice);
        VDBG_HIP(hipMemcpyAsync(hr.data(), ids, slice * 4, hipMemcpyDeviceToHost, s));
        VDBG_HIP(hipStreamSynchronize(s));
        const size_t want = std::min(k, sp.matches);
        std::vector<size_t> shortq;
        for (size_t i = 0; i < nq; ++i) {
          size_t h = 0;
          while (h < k && hr[i * k + h] != kNoId) ++h;
          if (h < want) shortq.push_back(i);
        }
        if (shortq.empty()) break;
        sp.plan = VDBG_PLAN_FILTERED_INDEX_EXACT_FALLBACK;
        DevBuf xi, xdd;
        VDBG_RETURN_IF_ERROR(Alloc(&xi, slice * 4, s));
        VDBG_RETURN_IF_ERROR(Alloc(&xdd, slice * 4, s));
        VDBG_RETURN_IF_ERROR(vdbg_flat_search_device(segs[p].rows, q, nq, k, allow,
                                                     static_cast<uint32_t*>(xi.p),
                                                     static_cast<float*>(xdd.p), s));
        for (size_t i : shortq) {
          VDBG_HIP(hipMemcpyAsync(ids + i * k, static_cast<uint32_t*>(xi.p) + i * k, k * 4,
                                  hipMemcpyDeviceToDevice, s));
          VDBG_HIP(hipMemcpyAsync(dd + i * k, static_cast<float*>(xdd.p) + i * k, k * 4,
                                  hipMemcpyDeviceToDevice, s));
          if (dist_comps != nullptr) dist_comps[i] += sp.matches;
        }
        VDBG_HIP(hipStreamSynchronize(s));  // xi / xdd are released on return
        break;
      }
      case VDBG_PLAN_POST_FILTER: {
        // :110-127: search k * alpha under the delete filter, keep the hits the filter allows
        const vdbg_segment& g = segs[p];
        const size_t rows = g.rows->d.n;
        const size_t deleted = g.deleted_words ? CountRows(g.deleted_words, rows) : 0;
        const size_t live = rows - std::min(rows, deleted);
        const size_t kk = std::min(std::max<size_t>(live, 1), k * std::max<size_t>(1, P.post_filter_alpha));
        std::vector<uint64_t> del_allow;
        DevBuf da, wi, wd;
        const uint64_t* dallow = nullptr;
        if (deleted > 0) {
          const size_t nw = (rows + 63) / 64;
          del_allow.resize(nw);
          for (size_t i = 0; i < nw; ++i) del_allow[i] = ~g.deleted_words[i];
          VDBG_RETURN_IF_ERROR(Alloc(&da, nw * 8, s));
          VDBG_HIP(hipMemcpyAsync(da.p, del_allow.data(), nw * 8, hipMemcpyHostToDevice, s));
          dallow = static_cast<const uint64_t*>(da.p);
        }
        VDBG_RETURN_IF_ERROR(Alloc(&wi, nq * kk * 4, s));
        VDBG_RETURN_IF_ERROR(Alloc(&wd, nq * kk * 4, s));
        // ef raised to kk (:113-114)
        VDBG_RETURN_IF_ERROR(index_search(p, kk, sp.nprobe, dallow, static_cast<uint32_t*>(wi.p),
                                          static_cast<float*>(wd.p), std::max(P.ef, kk)));
        hr.resize(nq * kk);
        hd.resize(nq * kk);
        VDBG_HIP(hipMemcpyAsync(hr.data(), wi.p, nq * kk * 4, hipMemcpyDeviceToHost, s));
        VDBG_HIP(hipMemcpyAsync(hd.data(), wd.p, nq * kk * 4, hipMemcpyDeviceToHost, s));
        VDBG_HIP(hipStreamSynchronize(s));
        xr.assign(slice, kNoId);
        xd.assign(slice, __builtin_inff());
        for (size_t i = 0; i < nq; ++i) {
          size_t out = 0;
          for (size_t j = 0; j < kk && out < k; ++j) {
            const uint32_t r = hr[i * kk + j];
            if (r == kNoId) break;
            if ((sp.allow[r >> 6] >> (r & 63)) & 1u) {
              xr[i * k + out] = r;
              xd[i * k + out] = hd[i * kk + j];
              ++out;
            }
          }
        }
        VDBG_HIP(hipMemcpyAsync(ids, xr.data(), slice * 4, hipMemcpyHostToDevice, s));
        VDBG_HIP(hipMemcpyAsync(dd, xd.data(), slice * 4, hipMemcpyHostToDevice, s));
        VDBG_HIP(hipStreamSynchronize(s));
        break;
      }
      default:
        return SetError(kInternal, "bad plan");
    }
  }

  if (nlanes > 0) {
    // the lanes' flat scans: ScanMasked with the count of allowed rows the host words give
    auto run_lane = [&](int l) -> int {
      ScanScratch* lane = c->lanes[size_t(l)];
      for (size_t p : lane_jobs[size_t(l)]) {
        const SegPlan& sp = plan[p];
        const uint64_t* allow =
            sp.allow.empty() ? nullptr : static_cast<const uint64_t*>(allow_dev.p) + allow_at[p];
        VDBG_RETURN_IF_ERROR(ScanMasked(c, &segs[p].rows->d.src, q, nq, k, allow,
                                        static_cast<uint32_t*>(hits_r.p) + p * slice,
                                        static_cast<float*>(hits_d.p) + p * slice, lane->stream,
                                        allow != nullptr ? sp.allowed : -1, lane));
      }
      return kOk;
    };
    int rc = kOk;
    if (c->lane_threads && nlanes > 1) {
      std::vector<int> rcs(size_t(nlanes), kOk);
      std::vector<std::string> errs{size_t(nlanes), std::string()};
      std::vector<std::thread> th;
      th.reserve(size_t(nlanes - 1));
      for (int l = 1; l < nlanes; ++l)
        th.emplace_back([&, l]() {
          if (hipSetDevice(c->device) != hipSuccess) {
            rcs[size_t(l)] = kInternal;
            errs[size_t(l)] = "lane thread: hipSetDevice";
            return;
          }
          rcs[size_t(l)] = run_lane(l);
          if (rcs[size_t(l)] != kOk) errs[size_t(l)] = vdbg_last_error();
        });
      rcs[0] = run_lane(0);
      if (rcs[0] != kOk) errs[0] = vdbg_last_error();
      for (auto& t : th) t.join();
      for (int l = 0; l < nlanes && rc == kOk; ++l)
        if (rcs[size_t(l)] != kOk) rc = SetError(rcs[size_t(l)], errs[size_t(l)]);
    } else {
      for (int l = 0; l < nlanes && rc == kOk; ++l) rc = run_lane(l);
    }
    // the merge waits for every lane (also after an error: nothing may still be queued on a
    // lane when this call's buffers are released)
    for (int l = 0; l < nlanes; ++l) {
      VDBG_HIP(hipEventRecord(c->lanes[l]->done, c->lanes[l]->stream));
      VDBG_HIP(hipStreamWaitEvent(s, c->lanes[l]->done, 0));
    }
    (void)hipEventDestroy(fork);
    if (rc != kOk) {
      (void)hipStreamSynchronize(s);
      return rc;
    }
  }

  // ---- the merge (collection_impl.cc:1076-1112) and the copy back
  std::vector<const uint64_t*> ext(np, nullptr);
  for (size_t p = 0; p < nseg; ++p)
    ext[p] = plan[p].plan == VDBG_PLAN_HOST ? static_cast<const uint64_t*>(host_ext[p].p)
                                            : segs[p].rows->d.ext_ids;
  VDBG_RETURN_IF_ERROR(Alloc(&extp, np * sizeof(void*), s));
  if (!device_io) {
    VDBG_RETURN_IF_ERROR(Alloc(&oe, slice * 8, s));
    VDBG_RETURN_IF_ERROR(Alloc(&od, slice * 4, s));
  }
  uint64_t* merge_ext = device_io ? out_ids : static_cast<uint64_t*>(oe.p);
  float* merge_d = device_io ? out_dists : static_cast<float*>(od.p);
  VDBG_HIP(hipMemcpyAsync(extp.p, ext.data(), np * sizeof(void*), hipMemcpyHostToDevice, s));
  if (nseg == 0) {
    VDBG_HIP(hipMemsetAsync(hits_r.p, 0xff, slice * 4, s));
    VDBG_HIP(hipMemsetAsync(hits_d.p, 0, slice * 4, s));
  }
  MergeArgs a{int(nq), int(np), int(k), static_cast<const float*>(hits_d.p),
              static_cast<const uint32_t*>(hits_r.p), nullptr, nullptr, merge_ext, merge_d};
  a.ext_parts = static_cast<const uint64_t* const*>(extp.p);
  VDBG_RETURN_IF_ERROR(MergeParts(c, a, s));
  if (!device_io) {
    VDBG_HIP(hipMemcpyAsync(out_ids, oe.p, slice * 8, hipMemcpyDeviceToHost, s));
    VDBG_HIP(hipMemcpyAsync(out_dists, od.p, slice * 4, hipMemcpyDeviceToHost, s));
  }
  // (the host arrays handed to asynchronous copies above live until here)
  VDBG_HIP(hipStreamSynchronize(s));
  if (seg_plans != nullptr)
    for (size_t p = 0; p < nseg; ++p) seg_plans[p] = plan[p].plan;
  return kOk;
}

}  // namespace

extern "C" {

int vdbg_collection_search_host(vdbg_ctx* ctx, const vdbg_segment* segs, size_t nseg,
                                size_t dim, int metric, const float* queries, size_t nq,
                                size_t k, const vdbg_search_params* params, uint64_t* out_ids,
                                float* out_dists, uint64_t* dist_comps, int* seg_plans) {
  return CollectionSearch(ctx, segs, nseg, dim, metric, queries, nq, k, params, out_ids,
                          out_dists, dist_comps, seg_plans, false, nullptr);
}

int vdbg_collection_search_device(vdbg_ctx* ctx, const vdbg_segment* segs, size_t nseg,
                                  size_t dim, int metric, const float* queries, size_t nq,
                                  size_t k, const vdbg_search_params* params,
                                  uint64_t* out_ids, float* out_dists, uint64_t* dist_comps,
                                  int* seg_plans, void* stream) {
  return CollectionSearch(ctx, segs, nseg, dim, metric, queries, nq, k, params, out_ids,
                          out_dists, dist_comps, seg_plans, true, stream);
}

}  // extern "C"
