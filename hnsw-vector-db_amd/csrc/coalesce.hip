// coalesce.hip -- concurrent one-query searches of one index gathered into device batches.
//
// vdb answers a request by calling Index::search once per query: CollectionImpl::SearchBatch
// hands each query to a pool worker (src/engine/collection_impl.cc:1120-1130) and Search fans
// a query out over the segments (:1069-1073), so every call reaching an index is a batch of
// one.  A coalescer queues concurrent calls that share (k, parameters, allow words) into one
// batch.  The first caller of a batch leads it: the batch stops taking queries when it holds
// max_batch of them, or once max_wait has passed since it opened and no earlier batch of this
// coalescer is still on the device (a batch keeps filling while an earlier one runs).  The
// leader runs the index's host entry point over the whole batch and every caller copies out
// its own row.  Queries of a batch are searched independently, so each caller gets what the
// one-query call returns.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "vdbg_internal.h"

using namespace vdbg;

namespace {

enum Kind { kFlat = 0, kSq8 = 1, kIvfPq = 2, kPqFlat = 3, kHnswSq8 = 4 };

using Clock = std::chrono::steady_clock;

struct Batch {
  // the key every query of the batch shares (written under the coalescer's mutex)
  size_t k = 0, param = 0;
  int rerank = 0;
  const uint64_t* allow = nullptr;
  Clock::time_point opened;
  std::vector<float> q;         // [n][pd], rows written under the mutex
  std::atomic<size_t> n{0};     // queries joined
  std::atomic<uint32_t> done{0};
  int rc = kOk;
  std::string err;
  std::vector<uint32_t> ids;    // [n][k]
  std::vector<float> d;
  std::vector<uint64_t> dc;     // [n]
  std::atomic<size_t> readers{0};  // callers that have not yet taken their row
};

}  // namespace

struct vdbg_coalescer {
  Kind kind;
  void* index;
  size_t pd;
  size_t max_batch;
  std::chrono::microseconds wait;
  std::mutex mu;                  // guards open, spare, calls and the batches' keys and rows
  std::vector<Batch*> open;       // batches taking queries, at most one per key
  std::vector<Batch*> spare;      // finished batches kept for reuse
  size_t calls = 0;               // calls inside vdbg_coalescer_search
  uint64_t batches = 0, queries = 0;  // batches run and the queries they held
  std::condition_variable filled;  // a leader waits here for its batch to fill
  std::mutex exec;                // held while a batch of this coalescer is on the device
};

namespace {

int Create(Kind kind, void* index, size_t pd, size_t max_batch, uint32_t max_wait_us,
           vdbg_coalescer** out) {
  if (out == nullptr) return SetError(kInvalidArgument, "null out");
  *out = nullptr;
  if (index == nullptr) return SetError(kInvalidArgument, "null index");
  if (max_batch < 1 || max_batch > 4096)
    return SetError(kInvalidArgument, "max_batch must be in 1..4096");
  if (max_wait_us > 1000000) return SetError(kInvalidArgument, "max_wait_us must be at most 1 s");
  auto* co = new (std::nothrow) vdbg_coalescer;
  if (co == nullptr) return SetError(kResourceExhausted, "out of host memory");
  co->kind = kind;
  co->index = index;
  co->pd = pd;
  co->max_batch = max_batch;
  co->wait = std::chrono::microseconds(max_wait_us);
  *out = co;
  return kOk;
}

// The index's host entry point over a closed batch; per-query distance counts in b->dc.
int RunBatch(vdbg_coalescer* co, Batch* b) {
  const size_t n = b->n, k = b->k;
  b->ids.resize(n * k);
  b->d.resize(n * k);
  b->dc.assign(n, 0);
  uint64_t total = 0;
  int rc = kOk;
  switch (co->kind) {
    case kFlat:
      rc = vdbg_flat_search_host(static_cast<vdbg_dataset*>(co->index), b->q.data(), n, k,
                                 b->allow, b->ids.data(), b->d.data(), &total);
      break;
    case kSq8:
      rc = vdbg_sq8_search_host(static_cast<vdbg_sq8*>(co->index), b->q.data(), n, k, b->param,
                                b->allow, b->ids.data(), b->d.data(), &total);
      break;
    case kIvfPq:
      rc = vdbg_ivfpq_search_host(static_cast<vdbg_ivfpq*>(co->index), b->q.data(), n, k,
                                  b->param, b->rerank, b->allow, b->ids.data(), b->d.data(),
                                  b->dc.data());
      break;
    case kPqFlat:
      rc = vdbg_pqflat_search_host(static_cast<vdbg_pqflat*>(co->index), b->q.data(), n, k,
                                   b->rerank, b->allow, b->ids.data(), b->d.data(),
                                   b->dc.data());
      break;
    case kHnswSq8:
      rc = vdbg_sq8_hnsw_search_host(static_cast<vdbg_sq8*>(co->index), b->q.data(), n, k,
                                     b->param, b->rerank, b->allow, b->ids.data(), b->d.data(),
                                     b->dc.data());
      break;
  }
  // the flat and SQ8 scans count the same work for every query of the batch
  if (rc == kOk && (co->kind == kFlat || co->kind == kSq8))
    std::fill(b->dc.begin(), b->dc.end(), total / n);
  return rc;
}

}  // namespace

extern "C" {

int vdbg_coalescer_create_flat(vdbg_dataset* ds, size_t max_batch, uint32_t max_wait_us,
                               vdbg_coalescer** out) {
  return Create(kFlat, ds, ds ? ds->d.pd : 0, max_batch, max_wait_us, out);
}

int vdbg_coalescer_create_sq8(vdbg_sq8* sq, size_t max_batch, uint32_t max_wait_us,
                              vdbg_coalescer** out) {
  return Create(kSq8, sq, sq ? sq->q.ds->pd : 0, max_batch, max_wait_us, out);
}

int vdbg_coalescer_create_sq8_hnsw(vdbg_sq8* sq, size_t max_batch, uint32_t max_wait_us,
                                   vdbg_coalescer** out) {
  return Create(kHnswSq8, sq, sq ? sq->q.ds->pd : 0, max_batch, max_wait_us, out);
}

int vdbg_coalescer_create_ivfpq(vdbg_ivfpq* ix, size_t max_batch, uint32_t max_wait_us,
                                vdbg_coalescer** out) {
  return Create(kIvfPq, ix, ix ? size_t(ix->x.pd) : 0, max_batch, max_wait_us, out);
}

int vdbg_coalescer_create_pqflat(vdbg_pqflat* ix, size_t max_batch, uint32_t max_wait_us,
                                 vdbg_coalescer** out) {
  return Create(kPqFlat, ix, ix ? ix->p.ds->pd : 0, max_batch, max_wait_us, out);
}

int vdbg_coalescer_search(vdbg_coalescer* co, const float* query, size_t k, size_t param,
                          int rerank, const uint64_t* allow_words, uint32_t* out_ids,
                          float* out_dists, uint64_t* dist_comps) {
  if (co == nullptr) return SetError(kInvalidArgument, "null coalescer");
  if (dist_comps != nullptr) *dist_comps = 0;
  if (k == 0) return kOk;
  if (query == nullptr || out_ids == nullptr || out_dists == nullptr)
    return SetError(kInvalidArgument, "null pointer");
  if (k > 10000) return SetError(kInvalidArgument, "k must be in 1..10000");
  // parameters the index does not read do not split batches
  if (co->kind == kFlat || co->kind == kSq8) rerank = 0;
  if (co->kind == kFlat || co->kind == kPqFlat) param = 0;
  std::unique_lock<std::mutex> lk(co->mu);
  ++co->calls;
  Batch* b = nullptr;
  for (Batch* o : co->open)
    if (o->k == k && o->param == param && o->rerank == rerank && o->allow == allow_words) {
      b = o;
      break;
    }
  const bool lead = b == nullptr;
  if (lead) {
    if (!co->spare.empty()) {
      b = co->spare.back();
      co->spare.pop_back();
    } else {
      b = new (std::nothrow) Batch;
      if (b == nullptr) {
        --co->calls;
        return SetError(kResourceExhausted, "out of host memory");
      }
    }
    b->k = k;
    b->param = param;
    b->rerank = rerank;
    b->allow = allow_words;
    b->opened = Clock::now();
    b->n.store(0, std::memory_order_relaxed);
    b->done.store(0, std::memory_order_relaxed);
    b->rc = kOk;
    b->err.clear();
    b->readers.store(0, std::memory_order_relaxed);
    b->q.resize(co->max_batch * co->pd);
    co->open.push_back(b);
  }
  auto close = [&]() {  // no more joins (under the mutex)
    auto it = std::find(co->open.begin(), co->open.end(), b);
    if (it != co->open.end()) co->open.erase(it);
  };
  const size_t slot = b->n.load(std::memory_order_relaxed);
  std::memcpy(b->q.data() + slot * co->pd, query, co->pd * sizeof(float));
  b->readers.fetch_add(1, std::memory_order_relaxed);
  b->n.store(slot + 1, std::memory_order_release);
  if (slot + 1 == co->max_batch) {
    close();
    co->filled.notify_all();
  }
  if (lead) {
    // until the batch is full or its time is up, then until the device is free (joins go on
    // meanwhile); the batch closes under the mutex, so every row joined is in place
    co->filled.wait_until(lk, b->opened + co->wait, [&] {
      return b->n.load(std::memory_order_relaxed) >= co->max_batch;
    });
    lk.unlock();
    {
      std::lock_guard<std::mutex> ex(co->exec);
      lk.lock();
      close();
      ++co->batches;
      co->queries += b->n.load(std::memory_order_relaxed);
      lk.unlock();
      b->rc = RunBatch(co, b);
      if (b->rc != kOk) b->err = vdbg_last_error();
    }
    b->done.store(1, std::memory_order_release);
    b->done.notify_all();  // (C++20 atomic wait: each follower sleeps on this word)
  } else {
    lk.unlock();
    b->done.wait(0, std::memory_order_acquire);
  }
  const int rc = b->rc;
  if (rc == kOk) {
    std::memcpy(out_ids, b->ids.data() + slot * k, k * sizeof(uint32_t));
    std::memcpy(out_dists, b->d.data() + slot * k, k * sizeof(float));
    if (dist_comps != nullptr) *dist_comps = b->dc[slot];
  } else if (!lead) {
    SetError(rc, b->err);  // the leader's message, on this thread too
  }
  const bool last = b->readers.fetch_sub(1, std::memory_order_acq_rel) == 1;
  lk.lock();
  if (last) co->spare.push_back(b);
  --co->calls;
  return rc;
}

int vdbg_coalescer_stats(vdbg_coalescer* co, uint64_t* batches, uint64_t* queries) {
  if (co == nullptr || batches == nullptr || queries == nullptr)
    return SetError(kInvalidArgument, "null argument");
  std::lock_guard<std::mutex> lk(co->mu);
  *batches = co->batches;
  *queries = co->queries;
  return kOk;
}

int vdbg_coalescer_destroy(vdbg_coalescer* co) {
  if (co == nullptr) return kOk;
  {
    std::lock_guard<std::mutex> lk(co->mu);
    if (co->calls != 0) return SetError(kFailedPrecondition, "coalescer has calls in flight");
  }
  for (Batch* b : co->spare) delete b;
  delete co;
  return kOk;
}

}  // extern "C"
