// segment_kernels.hip -- the collection-level pieces around the scans: dense row masks
// (counting and compaction), query preparation, and the cross-segment merge.
//
//  * A filter reaches the scans as a dense bitmask (bit r of word r/64 = row r allowed):
//    DeleteBits words complemented (src/util/delete_bits.h:50-55) or the roaring filter
//    result minus deletes (src/engine/planner.cc:64-65) expanded to words.  When few rows
//    are allowed the scan runs on a compacted copy of the allowed rows, kept in ascending
//    row order so that ExactOverBitmap's tie rule (planner.cc:31-38) is unchanged.
//  * PrepareQuery (src/engine/collection_impl.cc:1023-1034): pad, reject non-finite values,
//    normalise for cosine with NormalizeVector (src/util/dataset.cc:33-41).
//  * The merge of CollectionImpl::Search (collection_impl.cc:1076-1112): every part's hits
//    sorted by (dist, part, row), the first hit of each external id kept, k returned.
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <cstring>
#include <vector>

#include "vdbg_device.h"
#include "gemm.h"
#include "vdbg_internal.h"

namespace vdbg {

// ---------------------------------------------------------------- masks

__global__ void k_word_counts(const uint64_t* __restrict__ w, size_t nwords, uint32_t N,
                              uint32_t* __restrict__ cnt) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i >= nwords) return;
  uint64_t v = w[i];
  const size_t lo = i * 64;
  if (lo + 64 > N) v &= (N - lo >= 64) ? ~0ull : ((1ull << (N - lo)) - 1ull);
  cnt[i] = uint32_t(__popcll(v));
}

__global__ void k_compact_ids(const uint64_t* __restrict__ w, size_t nwords, uint32_t N,
                              const uint32_t* __restrict__ pre, uint32_t* __restrict__ ids) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i >= nwords) return;
  uint64_t v = w[i];
  const size_t lo = i * 64;
  if (lo + 64 > N) v &= (N - lo >= 64) ? ~0ull : ((1ull << (N - lo)) - 1ull);
  uint32_t p = pre[i];
  while (v != 0) {
    const int b = __ffsll(static_cast<long long>(v)) - 1;
    ids[p++] = uint32_t(lo + b);
    v &= v - 1;
  }
}

// The ascending ids of the allowed rows of a mask of at most kCompactBlockWords words and
// kCompactBlockIds allowed rows, in one block: each thread takes a run of consecutive words,
// the block scans the runs' counts in LDS, and each thread writes its run's ids from its
// offset.  (One launch instead of the count / scan / write sequence, for sparse masks.)
__device__ __forceinline__ void compact_block(const uint64_t* __restrict__ w, uint32_t nwords,
                                              uint32_t N, uint32_t* __restrict__ ids,
                                              uint32_t (&wave_tot)[16]) {
  const uint32_t t = threadIdx.x;
  const uint32_t per = (nwords + 1023) / 1024;
  const uint32_t lo = min(nwords, t * per), hi = min(nwords, lo + per);
  auto word = [&](uint32_t i) {
    uint64_t v = w[i];
    const size_t b0 = size_t(i) * 64;
    if (b0 + 64 > N) v &= (N - b0 >= 64) ? ~0ull : ((1ull << (N - b0)) - 1ull);
    return v;
  };
  uint32_t cnt = 0;
  for (uint32_t i = lo; i < hi; ++i) cnt += uint32_t(__popcll(word(i)));
  // block exclusive scan of cnt: within each wave, then over the 16 wave totals
  const int lane = lane_id(), wv = int(t) >> 6;
  uint32_t incl = cnt;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t x = __shfl_up(incl, o);
    if (lane >= o) incl += x;
  }
  if (lane == kWave - 1) wave_tot[wv] = incl;
  __syncthreads();
  uint32_t base = 0;
  for (int i = 0; i < wv; ++i) base += wave_tot[i];
  uint32_t p = base + incl - cnt;
  for (uint32_t i = lo; i < hi; ++i) {
    uint64_t v = word(i);
    while (v != 0) {
      const int b = __ffsll(static_cast<long long>(v)) - 1;
      ids[p++] = i * 64 + uint32_t(b);
      v &= v - 1;
    }
  }
}
__global__ __launch_bounds__(1024) void k_compact_block(const uint64_t* __restrict__ w,
                                                        uint32_t nwords, uint32_t N,
                                                        uint32_t* __restrict__ ids) {
  __shared__ uint32_t wave_tot[16];
  compact_block(w, nwords, N, ids, wave_tot);
}
// Several masks, one block each (CompactMulti).
__global__ __launch_bounds__(1024) void k_compact_multi(CompactMulti m) {
  __shared__ uint32_t wave_tot[16];
  const int b = blockIdx.x;
  compact_block(m.w[b], m.nwords[b], m.N[b], m.ids[b], wave_tot);
}

// Thread t of a gather: row t / W, 16-byte column t % W of the parts (GatherParts).
__device__ __forceinline__ void gather_one(const GatherParts& g, size_t t) {
  const uint32_t W = g.wa + g.wb + g.wc + 1;
  if (t >= size_t(g.n) * W) return;
  const uint32_t r = uint32_t(t / W), col = uint32_t(t - size_t(r) * W);
  const size_t src = g.ids != nullptr ? g.ids[r] : r;
  if (col < g.wa) {
    g.ao[size_t(r) * g.wa + col] = g.a[src * g.wa + col];
  } else if (col < g.wa + g.wb) {
    const uint32_t c = col - g.wa;
    g.bo[size_t(r) * g.wb + c] = g.b[src * g.wb + c];
  } else if (col < g.wa + g.wb + g.wc) {
    const uint32_t c = col - g.wa - g.wb;
    g.co[size_t(r) * g.wc + c] = g.c8[src * g.wc + c];
  } else {
    g.rno[r] = g.rn[src];
    if (g.i8 != nullptr) g.i8o[r] = g.i8[src];
    if (g.ext != nullptr) g.exto[r] = g.ext[src];
  }
}

// The compacted rows' parts in one launch (GatherParts, vdbg_internal.h).
__global__ __launch_bounds__(256) void k_gather_compact(GatherParts g) {
  gather_one(g, blockIdx.x * size_t(blockDim.x) + threadIdx.x);
}
// Several row sets' gathers in one launch: part p takes threads [start[p], start[p + 1]).
__global__ __launch_bounds__(256) void k_gather_multi(GatherMulti m) {
  const uint64_t t = blockIdx.x * uint64_t(blockDim.x) + threadIdx.x;
  if (t >= m.start[m.n]) return;
  int p = 0;
  while (t >= m.start[p + 1]) ++p;
  gather_one(m.g[p], t - m.start[p]);
}

int CompactGatherMulti(const CompactMulti& cm, const GatherMulti& gm, hipStream_t s) {
  if (cm.n > 0) {
    k_compact_multi<<<dim3(unsigned(cm.n)), 1024, 0, s>>>(cm);
    VDBG_HIP(hipGetLastError());
  }
  if (gm.n > 0 && gm.start[gm.n] > 0) {
    k_gather_multi<<<dim3(unsigned((gm.start[gm.n] + 255) / 256)), 256, 0, s>>>(gm);
    VDBG_HIP(hipGetLastError());
  }
  return kOk;
}

__global__ void k_map_ids(uint32_t* __restrict__ out, size_t n, const uint32_t* __restrict__ ids) {
  const size_t t = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (t < n && out[t] != kNoId) out[t] = ids[out[t]];
}

int CountAllowed(Ctx* c, const uint64_t* allow, uint32_t N, uint32_t* count, hipStream_t s,
                 ScanScratch* lane) {
  const size_t nwords = (size_t(N) + 63) / 64;
  size_t tmp_bytes = 0;
  VDBG_HIP(hipcub::DeviceReduce::Sum(nullptr, tmp_bytes, static_cast<uint32_t*>(nullptr),
                                     static_cast<uint32_t*>(nullptr), int(nwords), s));
  // the compaction scratch, kept across calls (reallocation would cost more than the scan at
  // low selectivity); its contents are dead once the count is read back
  Workspace& w = lane != nullptr ? lane->wsc : c->wsc;
  hipEvent_t done = lane != nullptr ? lane->wsc_done : c->wsc_done;
  w.used = 0;
  // a call on another stream may still read the scratch: wait for its last reader
  if (done != nullptr) VDBG_HIP(hipStreamWaitEvent(s, done, 0));
  VDBG_RETURN_IF_ERROR(w.reserve((nwords + 1) * 4 + tmp_bytes + 1024));
  uint32_t* cnt = w.take<uint32_t>(nwords + 1);
  void* tmp = w.take<char>(tmp_bytes + 16);
  k_word_counts<<<dim3(unsigned((nwords + 255) / 256)), 256, 0, s>>>(allow, nwords, N, cnt);
  VDBG_HIP(hipGetLastError());
  VDBG_HIP(hipcub::DeviceReduce::Sum(tmp, tmp_bytes, cnt, cnt + nwords, int(nwords), s));
  VDBG_RETURN_IF_ERROR(ReadWords(c, cnt + nwords, 1, s, count));
  return kOk;
}

// The scan over the allowed rows only: compact rows (ascending), scan without a mask, map
// the compact indexes back to row ids.
constexpr uint32_t kCompactOneBlock = 16384;

int CompactScan(Ctx* c, ScanSource* src, const float* Q, size_t nq, size_t kk,
                const uint64_t* allow, uint32_t count, uint32_t* out_ids, float* out_d,
                hipStream_t s, ScanScratch* lane) {
  const uint32_t N = src->N;
  const size_t pd = src->pd;
  const size_t nwords = (size_t(N) + 63) / 64;
  const size_t row_bytes = src->kind == 0 ? pd * sizeof(float) : pd;
  void* buf = nullptr;
  // Float rows in two parts: a batch large enough for the int8 two-part GEMM ranks on it, so
  // their fp16 pairs are not gathered (a batch failing the int8 check then takes the fp32
  // GEMM); smaller batches keep the fp16 pairs and skip the int8 copy.  (Float rows held as
  // fp16 h halves alone have no int8 copy.)
  bool keep16 = src->X16 != nullptr, keep8 = src->X8 != nullptr;
  if (src->kind == 0 && src->x16_parts == 2 && src->x8_parts == 2 && keep8) {
    const bool int8 = c->fp16_gemm && c->int8_gemm && Gemm8Supported(pd) &&
                      double(count) * double(nq) * double(pd) >= c->int8_float_min_work;
    (int8 ? keep16 : keep8) = false;
  }
  const size_t row16_bytes = keep16 ? src->x16_parts * pd * sizeof(uint16_t) : 0;
  const size_t row8_bytes = keep8 ? pd * src->x8_parts : 0;  // the int8 copy
  // Float rows held as high fp16 halves rank on that copy alone, so the fp32 rows are not
  // gathered: the exact re-scoring reads the parent's rows through the id map.
  const bool map32 = src->kind == 0 && src->x16_approx && keep16 && c->fp16_gemm;
  // the compacted source's sample lives in the same stream-ordered allocation
  ScanSource cs = *src;
  cs.N = count;
  const size_t sample_bytes = SampleBytes(cs, SampleRows(count));
  size_t tmp_bytes = 0;
  VDBG_HIP(hipcub::DeviceScan::ExclusiveSum(nullptr, tmp_bytes, static_cast<uint32_t*>(nullptr),
                                            static_cast<uint32_t*>(nullptr), int(nwords), s));
  const size_t bytes = (nwords + 1) * 4 * 2 +
                       size_t(count) * (4 + 4 + (map32 ? 0 : row_bytes) + row16_bytes + row8_bytes +
                                        (src->init8 != nullptr ? 4 : 0)) +
                       sample_bytes + tmp_bytes + 4096 + 512 + 16 * 256;
  // the compaction scratch (the context's or the lane's): reused in stream order by the next
  // call, whose stream waits for the event recorded below
  Workspace& w = lane != nullptr ? lane->wsc : c->wsc;
  hipEvent_t& wsc_done = lane != nullptr ? lane->wsc_done : c->wsc_done;
  if (wsc_done != nullptr) VDBG_HIP(hipStreamWaitEvent(s, wsc_done, 0));
  w.used = 0;
  VDBG_RETURN_IF_ERROR(w.reserve(bytes));
  buf = w.base;
  auto take = [&](size_t b) { return w.take<char>(b); };
  uint32_t* cnt = reinterpret_cast<uint32_t*>(take((nwords + 1) * 4));
  uint32_t* pre = reinterpret_cast<uint32_t*>(take((nwords + 1) * 4));
  uint32_t* ids = reinterpret_cast<uint32_t*>(take(size_t(count) * 4 + 4));
  float* rn = reinterpret_cast<float*>(take(size_t(count) * 4 + 4));
  void* rows = map32 ? nullptr : take(size_t(count) * row_bytes + 16);
  void* rows16 = row16_bytes != 0 ? take(size_t(count) * row16_bytes + 16) : nullptr;
  void* rows8 = row8_bytes != 0 ? take(size_t(count) * row8_bytes + 16) : nullptr;
  int* init8 = src->init8 != nullptr ? reinterpret_cast<int*>(take(size_t(count) * 4 + 4)) : nullptr;
  void* sample = take(sample_bytes);
  void* tmp = nullptr;
  {
    ProfScope ps(c, "compact", s);
    // one block for sparse masks; the device-wide count, scan and write past kCompactOneBlock
    // ids (one block writing 61k ids took 41-55 us)
    if (nwords <= size_t(kCompactBlockWords) && count <= kCompactOneBlock) {
      k_compact_block<<<1, 1024, 0, s>>>(allow, uint32_t(nwords), N, ids);
    } else {
      k_word_counts<<<dim3(unsigned((nwords + 255) / 256)), 256, 0, s>>>(allow, nwords, N, cnt);
      tmp = take(tmp_bytes + 16);
      VDBG_HIP(hipcub::DeviceScan::ExclusiveSum(tmp, tmp_bytes, cnt, pre, int(nwords), s));
      k_compact_ids<<<dim3(unsigned((nwords + 255) / 256)), 256, 0, s>>>(allow, nwords, N, pre,
                                                                          ids);
    }
    // every part of the rows in one launch (padded dims are multiples of 16, so each part is
    // whole 16-byte columns); float rows held as high fp16 halves gather no fp32 rows (the
    // compacted source reads its parent's through the id map, cs.Xmap below)
    GatherParts g{};
    if (!map32) {
      g.a = reinterpret_cast<const uint4*>(src->kind == 0 ? static_cast<const void*>(src->X)
                                                          : static_cast<const void*>(src->C));
      g.ao = static_cast<uint4*>(rows);
      g.wa = uint32_t(row_bytes / 16);
    }
    if (rows16 != nullptr) {
      g.b = reinterpret_cast<const uint4*>(src->X16);
      g.bo = static_cast<uint4*>(rows16);
      g.wb = uint32_t(row16_bytes / 16);
    }
    if (rows8 != nullptr) {
      g.c8 = reinterpret_cast<const uint4*>(src->X8);
      g.co = static_cast<uint4*>(rows8);
      g.wc = uint32_t(row8_bytes / 16);
      g.i8 = init8 != nullptr ? src->init8 : nullptr;
      g.i8o = init8;
    }
    g.rn = src->rn;
    g.rno = rn;
    g.ids = ids;
    g.n = count;
    const size_t total = size_t(count) * (g.wa + g.wb + g.wc + 1);
    k_gather_compact<<<dim3(unsigned((total + 255) / 256)), 256, 0, s>>>(g);
    VDBG_HIP(hipGetLastError());
  }
  cs.X = src->kind == 0 ? (map32 ? src->X : static_cast<const float*>(rows)) : nullptr;
  cs.Xmap = map32 ? ids : nullptr;
  cs.X16 = static_cast<const uint16_t*>(rows16);
  cs.X8 = static_cast<const int8_t*>(rows8);
  cs.init8 = init8;
  cs.C = src->kind == 1 ? static_cast<const uint8_t*>(rows) : nullptr;
  cs.rn = rn;
  cs.Sbuf = nullptr;
  // only as many sample rows as this one scan uses
  int rc = GatherSample(c, &cs, s, sample, SampleWant(c, cs, nq, kk));
  if (rc == kOk)
    rc = RunScan(c, &cs, Q, nq, kk, nullptr, out_ids, out_d, s,
                 lane != nullptr ? &lane->ws : nullptr, lane != nullptr ? &lane->ws2 : nullptr);
  if (rc == kOk) {
    k_map_ids<<<dim3(unsigned((nq * kk + 255) / 256)), 256, 0, s>>>(out_ids, nq * kk, ids);
    if (hipGetLastError() != hipSuccess) rc = SetError(kInternal, "map ids launch");
  }
  if (wsc_done == nullptr &&
      hipEventCreateWithFlags(&wsc_done, hipEventDisableTiming) != hipSuccess)
    wsc_done = nullptr;
  if (wsc_done == nullptr || hipEventRecord(wsc_done, s) != hipSuccess) {
    (void)hipStreamSynchronize(s);  // no event: drain before the scratch is reused
  }
  FreeSample(&cs);  // the sample lives in the scratch (cs.Sbuf is null): nothing to free
  (void)buf;
  return rc;
}

// The scans' entry for an optional filter: unfiltered and all-allowed filters scan every
// row; when at most half the rows are allowed the allowed rows are compacted first;
// otherwise the scan tests the mask per row.
int ScanMasked(Ctx* c, ScanSource* src, const float* Q, size_t nq, size_t kk,
               const uint64_t* allow, uint32_t* out_ids, float* out_d, hipStream_t s,
               int64_t allowed, ScanScratch* lane) {
  Workspace* ws = lane != nullptr ? &lane->ws : nullptr;
  Workspace* ws2 = lane != nullptr ? &lane->ws2 : nullptr;
  if (allow == nullptr || nq == 0 || kk == 0 || src->N == 0)
    return RunScan(c, src, Q, nq, kk, allow, out_ids, out_d, s, ws, ws2);
  uint32_t count = 0;
  if (allowed >= 0)
    count = uint32_t(std::min<int64_t>(allowed, src->N));
  else
    VDBG_RETURN_IF_ERROR(CountAllowed(c, allow, src->N, &count, s, lane));
  if (count == src->N) return RunScan(c, src, Q, nq, kk, nullptr, out_ids, out_d, s, ws, ws2);
  if (count == 0) {  // nothing allowed: every slot is padding
    ScanSource none = *src;
    none.N = 0;
    return RunScan(c, &none, Q, nq, kk, nullptr, out_ids, out_d, s, ws, ws2);
  }
  if (2ull * count <= src->N)
    return CompactScan(c, src, Q, nq, kk, allow, count, out_ids, out_d, s, lane);
  return RunScan(c, src, Q, nq, kk, allow, out_ids, out_d, s, ws, ws2);
}

ScanScratch::~ScanScratch() {
  ws.release();
  ws2.release();
  wsc.release();
  if (wsc_done != nullptr) (void)hipEventDestroy(wsc_done);
  if (done != nullptr) (void)hipEventDestroy(done);
  if (stream != nullptr) (void)hipStreamDestroy(stream);
}

// ---------------------------------------------------------------- query preparation

// PrepareQuery (collection_impl.cc:1023-1034): one wave per query copies dim values into a
// zero-padded row and flags a non-finite value; for cosine, NormalizeVector
// (dataset.cc:33-41): fp64 sum of squares in index order, inv = float(1 / sqrt(sum)), fp32
// multiply.  status: 0 ok, 1 non-finite, 2 zero vector under cosine.  The sum is one chain
// of adds in index order, so one lane runs it, over the query staged in LDS by the whole wave
// (kPrepChunk values at a time), not over its own global loads.
constexpr int kPrepChunk = 512;
__global__ __launch_bounds__(256) void k_prepare(const float* __restrict__ raw, int nq, int dim,
                                                 int pd, int cosine, float* __restrict__ out,
                                                 int* __restrict__ status) {
  __shared__ float stage_all[4][kPrepChunk];
  const int q = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= nq) return;
  float* stage = stage_all[threadIdx.x >> 6];
  const int lane = lane_id();
  const float* v = raw + size_t(q) * dim;
  float* o = out + size_t(q) * pd;
  int bad = 0;
  for (int i = lane; i < pd; i += kWave) {
    const float x = i < dim ? v[i] : 0.f;
    if (i < dim && !isfinite(x)) bad = 1;
    o[i] = x;
  }
  bad = __ballot(bad != 0) != 0;
  int st = bad ? 1 : 0;
  float inv = 1.f;
  if (!bad && cosine) {
    double norm = 0;
    for (int c0 = 0; c0 < dim; c0 += kPrepChunk) {
      const int n = min(kPrepChunk, dim - c0);
      for (int i = lane; i < n; i += kWave) stage[i] = v[c0 + i];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (lane == 0)
        for (int i = 0; i < n; ++i)
          norm += static_cast<double>(stage[i]) * static_cast<double>(stage[i]);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (lane == 0) {
      if (!(norm > 0) || !isfinite(norm))
        st = 2;
      else
        inv = static_cast<float>(1.0 / sqrt(norm));
    }
    st = __shfl(st, 0);
    inv = __shfl(inv, 0);
    if (st == 0)
      for (int i = lane; i < dim; i += kWave) o[i] = v[i] * inv;
  }
  if (lane == 0) status[q] = st;
}

PrepPending::~PrepPending() {
  if (st != nullptr) (void)hipFreeAsync(st, s);
}

int PrepareQueriesLaunch(Ctx* c, const float* raw, size_t nq, size_t dim, size_t pd, int metric,
                         float* out, hipStream_t s, PrepPending* pp) {
  pp->nq = nq;
  pp->s = s;
  if (nq == 0) return kOk;
  VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&pp->st), nq * sizeof(int), s));
  ProfScope ps(c, "prepare_queries", s);
  k_prepare<<<dim3(unsigned((nq + 3) / 4)), 256, 0, s>>>(raw, int(nq), int(dim), int(pd),
                                                         metric == 2 ? 1 : 0, out, pp->st);
  VDBG_HIP(hipGetLastError());
  return kOk;
}

int PrepareQueriesCheck(PrepPending* pp) {
  if (pp->nq == 0 || pp->st == nullptr) return kOk;
  std::vector<int> h(pp->nq);
  VDBG_HIP(hipMemcpyAsync(h.data(), pp->st, pp->nq * sizeof(int), hipMemcpyDeviceToHost, pp->s));
  VDBG_HIP(hipStreamSynchronize(pp->s));
  (void)hipFreeAsync(pp->st, pp->s);
  pp->st = nullptr;
  for (size_t i = 0; i < pp->nq; ++i) {
    if (h[i] == 1) return SetError(kInvalidArgument, "query has a NaN or infinite value");
    if (h[i] == 2) return SetError(kInvalidArgument, "a zero query cannot be normalized for cosine");
  }
  return kOk;
}

int PrepareQueries(Ctx* c, const float* raw, size_t nq, size_t dim, size_t pd, int metric,
                   float* out, hipStream_t s) {
  PrepPending pp;
  VDBG_RETURN_IF_ERROR(PrepareQueriesLaunch(c, raw, nq, dim, pd, metric, out, s, &pp));
  return PrepareQueriesCheck(&pp);
}

// ---------------------------------------------------------------- merge

// External id of row `row` of part p: from the per-part device tables when given, else from
// the concatenated table.
__device__ __forceinline__ uint64_t ext_of(const MergeArgs& a, uint32_t p, uint32_t row) {
  return a.ext_parts != nullptr ? a.ext_parts[p][row]
                                : a.ext[(a.part_off != nullptr ? a.part_off[p] : 0) + row];
}

// One wave per query.  Candidate c = p * k + i (part p, i-th hit) keeps (dist, part, row)
// order as the key (dist, c): a part's hits arrive sorted by (dist, row).
template <int E>
__global__ __launch_bounds__(256) void k_merge(MergeArgs a) {
  __shared__ uint64_t ext_s[4][kWave * E];
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int q = blockIdx.x * 4 + wave;
  if (q >= a.nq) return;
  const int total = a.nparts * a.k;
  const int ko = a.kout > 0 ? a.kout : a.k;  // results written per query
  WaveKeys<E> r;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int c = e * kWave + lane;
    r.d[e] = __builtin_inff();
    r.id[e] = kNoId;
    if (c < total) {
      const int p = c / a.k, i = c - p * a.k;
      const size_t at = (size_t(p) * a.nq + q) * a.k + i;
      if (a.part_rows[at] != kNoId) {
        r.d[e] = a.part_d[at];
        r.id[e] = uint32_t(c);
      }
    }
  }
  bitonic_sort<E>(r);
  uint64_t* ex = ext_s[wave];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    uint64_t v = ~0ull;
    if (r.id[e] != kNoId) {
      const int c = int(r.id[e]), p = c / a.k, i = c - p * a.k;
      const uint32_t row = a.part_rows[(size_t(p) * a.nq + q) * a.k + i];
      v = ext_of(a, uint32_t(p), row);
    }
    ex[e * kWave + lane] = v;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // keep the first occurrence of each external id
  int written = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int g = e * kWave + lane;
    const uint64_t v = ex[g];
    bool keep = r.id[e] != kNoId;
    for (int t = 0; keep && t < g; ++t)
      if (ex[t] == v) keep = false;
    const uint64_t bal = __ballot(keep);
    const int pos = written + __popcll(bal & ((1ull << lane) - 1ull));
    if (keep && pos < ko) {
      a.out_ext[size_t(q) * ko + pos] = v;
      a.out_d[size_t(q) * ko + pos] = r.d[e];
    }
    written += __popcll(bal);
  }
  for (int i = written + lane; i < ko; i += kWave) {
    a.out_ext[size_t(q) * ko + i] = ~0ull;
    a.out_d[size_t(q) * ko + i] = __builtin_inff();
  }
}

// ---- the merge for more than 1024 hits per query, by sorting
//  1. per query, keys (dist, part * k + i) sorted: the (dist, part, row) order, rank r;
//  2. (external id, r) pairs sorted stably by external id: the first of each id group is
//     that id's first hit in the (dist, part, row) order;
//  3. kept[q][r] marks those; one wave per query emits the first k kept in rank order.
// Queries run in chunks [q0, q0 + nc); the inputs keep the batch's [part][nq][k] layout.

struct MergeChunk {
  MergeArgs a;
  int q0, nc;
  uint32_t per;  // nparts * k
  __device__ __forceinline__ size_t at(int q, uint32_t cidx) const {
    const uint32_t p = cidx / uint32_t(a.k), i = cidx - p * uint32_t(a.k);
    return (size_t(p) * a.nq + (q0 + q)) * a.k + i;
  }
  __device__ __forceinline__ uint32_t part(uint32_t cidx) const { return cidx / uint32_t(a.k); }
};

__global__ void k_mkeys(MergeChunk m, uint64_t* __restrict__ keys) {
  const size_t t = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (t >= size_t(m.nc) * m.per) return;
  const int q = int(t / m.per);
  const uint32_t cidx = uint32_t(t - size_t(q) * m.per);
  const size_t at = m.at(q, cidx);
  keys[t] = m.a.part_rows[at] == kNoId ? kNoKey : dist_key(m.a.part_d[at], cidx);
}

__global__ void k_mext(MergeChunk m, const uint64_t* __restrict__ sorted,
                       uint64_t* __restrict__ ext, uint32_t* __restrict__ rank) {
  const size_t t = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (t >= size_t(m.nc) * m.per) return;
  const int q = int(t / m.per);
  const uint64_t key = sorted[t];
  rank[t] = uint32_t(t - size_t(q) * m.per);
  if (key == kNoKey) {  // padding sorts last in step 1, so it follows every real id here
    ext[t] = ~0ull;
    return;
  }
  const uint32_t cidx = uint32_t(key);
  ext[t] = ext_of(m.a, m.part(cidx), m.a.part_rows[m.at(q, cidx)]);
}

__global__ void k_mfirst(MergeChunk m, const uint64_t* __restrict__ sorted,
                         const uint64_t* __restrict__ ext, const uint32_t* __restrict__ rank,
                         uint8_t* __restrict__ kept) {
  const size_t t = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (t >= size_t(m.nc) * m.per) return;
  const size_t q = t / m.per, j = t - q * m.per;
  const uint32_t r = rank[t];
  const bool real = sorted[q * m.per + r] != kNoKey;
  kept[q * m.per + r] = (real && (j == 0 || ext[t - 1] != ext[t])) ? 1 : 0;
}

__global__ __launch_bounds__(256) void k_memit(MergeChunk m, const uint64_t* __restrict__ sorted,
                                               const uint8_t* __restrict__ kept) {
  const int q = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= m.nc) return;
  const int lane = lane_id();
  const int k = m.a.kout > 0 ? m.a.kout : m.a.k;  // results written per query
  const size_t gq = size_t(m.q0 + q);
  int written = 0;
  for (uint32_t r0 = 0; r0 < m.per && written < k; r0 += kWave) {
    const uint32_t r = r0 + lane;
    const bool keep = r < m.per && kept[size_t(q) * m.per + r];
    const uint64_t bal = __ballot(keep);
    const int pos = written + __popcll(bal & ((1ull << lane) - 1ull));
    if (keep && pos < k) {
      const uint64_t key = sorted[size_t(q) * m.per + r];
      const uint32_t cidx = uint32_t(key);
      m.a.out_ext[gq * k + pos] = ext_of(m.a, m.part(cidx), m.a.part_rows[m.at(q, cidx)]);
      m.a.out_d[gq * k + pos] = key_dist(key);
    }
    written += __popcll(bal);
  }
  for (int i = written + lane; i < k; i += kWave) {
    m.a.out_ext[gq * k + i] = ~0ull;
    m.a.out_d[gq * k + i] = __builtin_inff();
  }
}

__global__ void k_seg_off(int* off, int nseg, int len) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i <= nseg) off[i] = i * len;
}

static int MergePartsLarge(Ctx* c, const MergeArgs& a, hipStream_t s) {
  const size_t per = size_t(a.nparts) * a.k;
  if (per > (size_t(1) << 30)) return SetError(kInvalidArgument, "merge: too many hits per query");
  const size_t chunk = std::max<size_t>(1, std::min<size_t>(a.nq, (size_t(1) << 24) / per));
  const size_t n = chunk * per;
  char* buf = nullptr;
  const size_t bytes = n * (8 * 4 + 4 * 2 + 1) + (chunk + 1) * 4 + 8 * 256;
  VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&buf), bytes, s));
  char* p = buf;
  auto take = [&](size_t b) {
    char* r = p;
    p += (b + 255) & ~size_t(255);
    return r;
  };
  uint64_t* k1 = reinterpret_cast<uint64_t*>(take(n * 8));
  uint64_t* k2 = reinterpret_cast<uint64_t*>(take(n * 8));
  uint64_t* e1 = reinterpret_cast<uint64_t*>(take(n * 8));
  uint64_t* e2 = reinterpret_cast<uint64_t*>(take(n * 8));
  uint32_t* r1 = reinterpret_cast<uint32_t*>(take(n * 4));
  uint32_t* r2 = reinterpret_cast<uint32_t*>(take(n * 4));
  uint8_t* kept = reinterpret_cast<uint8_t*>(take(n));
  int* off = reinterpret_cast<int*>(take((chunk + 1) * 4));
  void* tmp = nullptr;
  size_t tmp_cap = 0;
  int rc = kOk;
  auto sort_temp = [&](size_t b) -> bool {
    if (b <= tmp_cap) return true;
    if (tmp != nullptr) (void)hipFreeAsync(tmp, s);
    tmp = nullptr;
    tmp_cap = b;
    return hipMallocAsync(&tmp, b + 16, s) == hipSuccess;
  };
  ProfScope ps(c, "merge_parts", s);
  for (size_t q0 = 0; q0 < size_t(a.nq) && rc == kOk; q0 += chunk) {
    MergeChunk m{a, int(q0), int(std::min(chunk, size_t(a.nq) - q0)), uint32_t(per)};
    const int total = int(size_t(m.nc) * per);
    const unsigned g = unsigned((size_t(total) + 255) / 256);
    k_mkeys<<<dim3(g), 256, 0, s>>>(m, k1);
    k_seg_off<<<dim3(unsigned((m.nc + 256) / 256)), 256, 0, s>>>(off, m.nc, int(per));
    size_t tb = 0;
    if (hipcub::DeviceSegmentedRadixSort::SortKeys(nullptr, tb, k1, k2, total, m.nc, off, off + 1,
                                                   0, 64, s) != hipSuccess ||
        !sort_temp(tb) ||
        hipcub::DeviceSegmentedRadixSort::SortKeys(tmp, tb, k1, k2, total, m.nc, off, off + 1, 0,
                                                   64, s) != hipSuccess) {
      rc = SetError(kInternal, "merge: sort by distance");
      break;
    }
    k_mext<<<dim3(g), 256, 0, s>>>(m, k2, e1, r1);
    tb = 0;
    if (hipcub::DeviceSegmentedRadixSort::SortPairs(nullptr, tb, e1, e2, r1, r2, total, m.nc, off,
                                                    off + 1, 0, 64, s) != hipSuccess ||
        !sort_temp(tb) ||
        hipcub::DeviceSegmentedRadixSort::SortPairs(tmp, tb, e1, e2, r1, r2, total, m.nc, off,
                                                    off + 1, 0, 64, s) != hipSuccess) {
      rc = SetError(kInternal, "merge: sort by external id");
      break;
    }
    k_mfirst<<<dim3(g), 256, 0, s>>>(m, k2, e2, r2, kept);
    k_memit<<<dim3(unsigned((m.nc + 3) / 4)), 256, 0, s>>>(m, k2, kept);
    if (hipGetLastError() != hipSuccess) rc = SetError(kInternal, "merge launch");
    // the chunk's buffers are reused by the next chunk: the stream orders that
  }
  (void)hipStreamSynchronize(s);
  if (tmp != nullptr) (void)hipFreeAsync(tmp, s);
  (void)hipFreeAsync(buf, s);
  return rc;
}

int MergeParts(Ctx* c, const MergeArgs& a, hipStream_t s) {
  if (a.nq == 0 || a.k == 0) return kOk;
  const int total = a.nparts * a.k;
  if (total > 16 * kWave) return MergePartsLarge(c, a, s);
  int e = 1;
  while (kWave * e < total) e <<= 1;
  ProfScope ps(c, "merge_parts", s);
  const dim3 grid((a.nq + 3) / 4);
  switch (e) {
    case 1: k_merge<1><<<grid, 256, 0, s>>>(a); break;
    case 2: k_merge<2><<<grid, 256, 0, s>>>(a); break;
    case 4: k_merge<4><<<grid, 256, 0, s>>>(a); break;
    case 8: k_merge<8><<<grid, 256, 0, s>>>(a); break;
    case 16: k_merge<16><<<grid, 256, 0, s>>>(a); break;
    default: return MergePartsLarge(c, a, s);
  }
  VDBG_HIP(hipGetLastError());
  return kOk;
}

}  // namespace vdbg

using namespace vdbg;

extern "C" {

int vdbg_prepare_queries_device(vdbg_ctx* ctx, const float* raw, size_t nq, size_t dim,
                                size_t padded_dim, int metric, float* out, void* stream) {
  if (ctx == nullptr || (nq > 0 && (raw == nullptr || out == nullptr)) || dim == 0 ||
      padded_dim < dim || padded_dim % 16 != 0 || metric < 0 || metric > 2)
    return SetError(kInvalidArgument, "bad argument");
  Ctx* c = &ctx->c;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  return PrepareQueries(c, raw, nq, dim, padded_dim, metric,
                        out, stream ? static_cast<hipStream_t>(stream) : c->stream);
}

int vdbg_prepare_queries_host(vdbg_ctx* ctx, const float* raw, size_t nq, size_t dim,
                              size_t padded_dim, int metric, float* out) {
  if (ctx == nullptr || (nq > 0 && (raw == nullptr || out == nullptr)))
    return SetError(kInvalidArgument, "bad argument");
  Ctx* c = &ctx->c;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  if (nq == 0) return kOk;
  float *dr = nullptr, *dout = nullptr;
  VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&dr), nq * dim * 4, s));
  VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&dout), nq * padded_dim * 4, s));
  VDBG_HIP(hipMemcpyAsync(dr, raw, nq * dim * 4, hipMemcpyHostToDevice, s));
  int rc = vdbg_prepare_queries_device(ctx, dr, nq, dim, padded_dim, metric, dout, s);
  if (rc == kOk) {
    VDBG_HIP(hipMemcpyAsync(out, dout, nq * padded_dim * 4, hipMemcpyDeviceToHost, s));
    VDBG_HIP(hipStreamSynchronize(s));
  }
  (void)hipFreeAsync(dr, s);
  (void)hipFreeAsync(dout, s);
  return rc;
}

int vdbg_merge_parts_device(vdbg_ctx* ctx, size_t nq, size_t nparts, size_t k,
                            const float* part_dists, const uint32_t* part_rows,
                            const uint64_t* ext_ids, const uint64_t* part_offsets,
                            uint64_t* out_ext, float* out_dists, void* stream) {
  if (ctx == nullptr || (nq > 0 && k > 0 && nparts > 0 &&
                         (part_dists == nullptr || part_rows == nullptr || ext_ids == nullptr ||
                          part_offsets == nullptr || out_ext == nullptr || out_dists == nullptr)))
    return SetError(kInvalidArgument, "bad argument");
  Ctx* c = &ctx->c;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  MergeArgs a{int(nq), int(nparts), int(k), part_dists, part_rows, ext_ids, part_offsets,
              out_ext, out_dists};
  return MergeParts(c, a, stream ? static_cast<hipStream_t>(stream) : c->stream);
}

int vdbg_merge_parts_host(vdbg_ctx* ctx, size_t nq, size_t nparts, size_t k,
                          const float* part_dists, const uint32_t* part_rows,
                          const uint64_t* ext_ids, size_t n_ext, const uint64_t* part_offsets,
                          uint64_t* out_ext, float* out_dists) {
  if (ctx == nullptr) return SetError(kInvalidArgument, "null ctx");
  Ctx* c = &ctx->c;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  if (nq == 0 || k == 0) return kOk;
  const size_t nc = nparts * nq * k;
  char* buf = nullptr;
  const size_t bytes = nc * 8 + n_ext * 8 + nparts * 8 + nq * k * 12 + 4096;
  VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&buf), bytes, s));
  float* pd_ = reinterpret_cast<float*>(buf);
  uint32_t* pr = reinterpret_cast<uint32_t*>(buf + nc * 4);
  uint64_t* ex = reinterpret_cast<uint64_t*>(buf + ((nc * 8 + 255) & ~size_t(255)));
  uint64_t* po = ex + n_ext;
  uint64_t* oe = po + nparts;
  float* od = reinterpret_cast<float*>(oe + nq * k);
  VDBG_HIP(hipMemcpyAsync(pd_, part_dists, nc * 4, hipMemcpyHostToDevice, s));
  VDBG_HIP(hipMemcpyAsync(pr, part_rows, nc * 4, hipMemcpyHostToDevice, s));
  VDBG_HIP(hipMemcpyAsync(ex, ext_ids, n_ext * 8, hipMemcpyHostToDevice, s));
  VDBG_HIP(hipMemcpyAsync(po, part_offsets, nparts * 8, hipMemcpyHostToDevice, s));
  int rc = vdbg_merge_parts_device(ctx, nq, nparts, k, pd_, pr, ex, po, oe, od, s);
  if (rc == kOk) {
    VDBG_HIP(hipMemcpyAsync(out_ext, oe, nq * k * 8, hipMemcpyDeviceToHost, s));
    VDBG_HIP(hipMemcpyAsync(out_dists, od, nq * k * 4, hipMemcpyDeviceToHost, s));
    VDBG_HIP(hipStreamSynchronize(s));
  }
  (void)hipFreeAsync(buf, s);
  return rc;
}

}  // extern "C"
