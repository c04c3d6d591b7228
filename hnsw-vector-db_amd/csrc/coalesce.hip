// coalesce.hip -- concurrent one-query searches of one index gathered into device batches.
//
// vdb answers a request by calling Index::search once per query: CollectionImpl::SearchBatch
// hands each query to a pool worker (src/engine/collection_impl.cc:1120-1130) and Search fans
// a query out over the segments (:1069-1073), so every call reaching an index is a batch of
// one.  A coalescer queues concurrent calls that share (k, parameters, allow words) into one
// batch.  The first caller of a batch leads it: the batch takes queries while an earlier batch
// of this coalescer is on the device, and then, until every caller of the batch that just left
// the device has called again or max_wait has passed since it left (those callers can join
// again); it closes sooner once it holds max_batch queries.  A lone caller never waits.  The
// leader runs the index's host entry point over the whole batch and every caller copies out
// its own row.  Queries of a batch are searched independently, so each caller gets what the
// one-query call returns.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include <sys/prctl.h>

#include "vdbg_internal.h"

using namespace vdbg;

namespace {

enum Kind { kFlat = 0, kSq8 = 1, kIvfPq = 2, kPqFlat = 3, kHnswSq8 = 4 };

using Clock = std::chrono::steady_clock;

// The calling thread's timer slack cut to 1 us for a scope (PR_SET_TIMERSLACK), then restored.
struct TightTimers {
  int old = prctl(PR_GET_TIMERSLACK, 0, 0, 0, 0);
  TightTimers() { prctl(PR_SET_TIMERSLACK, 1000, 0, 0, 0); }
  ~TightTimers() {
    if (old > 0) prctl(PR_SET_TIMERSLACK, old, 0, 0, 0);
  }
};

struct Batch {
  uint64_t seq = 0;             // a number no other batch of the process has
  // the key every query of the batch shares (written under the coalescer's mutex)
  size_t k = 0, param = 0;
  int rerank = 0;
  const uint64_t* allow = nullptr;
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

std::atomic<uint64_t> g_batch_seq{0};

// The last batch this thread took part in, per coalescer (a small direct-mapped table): a
// call tells its coalescer that a caller of its last batch is back.
struct Recent {
  const void* co = nullptr;
  uint64_t seq = 0;
};
thread_local Recent t_recent[8];

Recent& RecentFor(const void* co) { return t_recent[(reinterpret_cast<uintptr_t>(co) >> 6) & 7]; }

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
  // the batch that last left the device (under mu): its number, its callers, when it left,
  // and how many of its callers have called again since
  uint64_t last_seq = 0;
  size_t last_n = 0, back = 0;
  Clock::time_point freed{};
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
  Recent& mine = RecentFor(co);
  if (mine.co == co && mine.seq != 0 && mine.seq == co->last_seq) {
    mine.seq = 0;
    if (++co->back >= co->last_n) co->filled.notify_all();
  }
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
    b->seq = g_batch_seq.fetch_add(1, std::memory_order_relaxed) + 1;
    b->k = k;
    b->param = param;
    b->rerank = rerank;
    b->allow = allow_words;
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
    // The batch takes joins until the device is free, and then, while callers of the batch
    // that just left the device have not all called again, until max_wait has passed since it
    // left (or until full): those callers return just then and may join.  A lone caller, or
    // one after an idle spell, does not wait.  A timed wait can sleep for the thread's timer
    // slack (50 us by default) past its deadline, so the slack is cut to 1 us meanwhile.
    auto ready = [&] {
      return b->n.load(std::memory_order_relaxed) >= co->max_batch || co->back >= co->last_n;
    };
    {
      std::unique_lock<std::mutex> ex(co->exec, std::try_to_lock);
      if (!ex.owns_lock()) {
        lk.unlock();
        ex.lock();
        lk.lock();
      }
      const Clock::time_point deadline = co->freed + co->wait;
      if (!ready() && Clock::now() < deadline) {
        TightTimers tight;
        co->filled.wait_until(lk, deadline, ready);
      }
      close();
      ++co->batches;
      const size_t n = b->n.load(std::memory_order_relaxed);
      co->queries += n;
      lk.unlock();
      b->rc = RunBatch(co, b);
      if (b->rc != kOk) b->err = vdbg_last_error();
      lk.lock();
      co->last_seq = b->seq;
      co->last_n = n;
      co->back = 0;
      co->freed = Clock::now();
      lk.unlock();
    }
    b->done.store(1, std::memory_order_release);
    b->done.notify_all();  // (C++20 atomic wait: each follower sleeps on this word)
  } else {
    lk.unlock();
    b->done.wait(0, std::memory_order_acquire);
  }
  mine.co = co;
  mine.seq = b->seq;
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
