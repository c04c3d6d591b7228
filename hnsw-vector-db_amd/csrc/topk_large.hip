// topk_large.hip -- top-k beyond what one wavefront keeps in registers.
//
// The wave top-k of the scans holds up to 256 keys.  vdb allows k up to 10,000
// (src/engine/collection_impl.cc:26, 1038-1039), IVF-PQ's default rerank depth is
// max(10 k, 100) (src/index/quant/ivf_pq.cc:16-19) and nprobe may reach nlist.  For those
// sizes every candidate is scored into a per-query array of 64-bit keys
//   key = order-preserving bits of the distance << 32 | row id
// (-0 folded into +0, so equal distances tie on the id as Neighbor::operator< does,
// include/vdb/types.h:23-25), the arrays are sorted by a segmented radix sort, and the first
// k keys of each query are the reference's TopK(k).sorted().
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <vector>

#include "vdbg_device.h"
#include "vdbg_internal.h"

namespace vdbg {

__global__ void k_unpack_keys(const uint64_t* __restrict__ keys, const int* __restrict__ off,
                              int nseg, int K, uint32_t* __restrict__ out_ids,
                              float* __restrict__ out_d) {
  const size_t t = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (t >= size_t(nseg) * K) return;
  const int q = int(t / K), i = int(t - size_t(q) * K);
  const int at = off[q] + i;
  const uint64_t key = at < off[q + 1] ? keys[at] : kNoKey;
  if (key == kNoKey) {
    out_ids[t] = kNoId;
    out_d[t] = __builtin_inff();
  } else {
    out_ids[t] = uint32_t(key);
    out_d[t] = key_dist(key);
  }
}

int SortSegmentsTopK(Ctx* c, uint64_t* keys, uint64_t* keys_alt, const int* off_dev, int nseg,
                     int total, int K, uint32_t* out_ids, float* out_d, hipStream_t s) {
  if (nseg == 0) return kOk;
  if (total > 0) {
    size_t tmp_bytes = 0;
    VDBG_HIP(hipcub::DeviceSegmentedRadixSort::SortKeys(nullptr, tmp_bytes, keys, keys_alt, total,
                                                        nseg, off_dev, off_dev + 1, 0, 64, s));
    void* tmp = nullptr;
    VDBG_HIP(hipMallocAsync(&tmp, tmp_bytes + 16, s));
    {
      ProfScope ps(c, "segmented_sort", s);
      VDBG_HIP(hipcub::DeviceSegmentedRadixSort::SortKeys(tmp, tmp_bytes, keys, keys_alt, total,
                                                          nseg, off_dev, off_dev + 1, 0, 64, s));
    }
    (void)hipFreeAsync(tmp, s);
  }
  const size_t n = size_t(nseg) * K;
  k_unpack_keys<<<dim3(unsigned((n + 255) / 256)), 256, 0, s>>>(keys_alt, off_dev, nseg, K,
                                                                  out_ids, out_d);
  VDBG_HIP(hipGetLastError());
  return kOk;
}

// Exact distance of every (query, row) pair of a chunk of queries; disallowed rows get kNoKey.
template <class Scorer>
__global__ __launch_bounds__(256) void k_score_all(const float* __restrict__ Q, int pd,
                                                   uint32_t N, const uint64_t* __restrict__ allow,
                                                   Scorer sc, uint64_t* __restrict__ keys) {
  const uint32_t r = blockIdx.x * 256 + threadIdx.x;
  const int qi = blockIdx.y;
  if (r >= N) return;
  uint64_t key = kNoKey;
  if (row_allowed(allow, r)) key = dist_key(sc(Q + size_t(qi) * pd, r), r);
  keys[size_t(qi) * N + r] = key;
}

__global__ void k_seg_offsets(int* off, int nseg, int len) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i <= nseg) off[i] = i * len;
}

template <class Scorer>
static int ExactAllT(Ctx* c, const ScanSource& src, const Scorer& sc, const float* Q, size_t nq,
                     size_t kk, const uint64_t* allow, uint32_t* out_ids, float* out_d,
                     hipStream_t s) {
  const uint32_t N = src.N;
  // queries per chunk: at most 256 MiB of keys and fewer than 2^31 keys
  size_t chunk = std::max<size_t>(1, (size_t(256) << 20) / (size_t(N) * 8));
  chunk = std::min({chunk, nq, size_t(65535)});  // queries run on grid.y
  uint64_t* keys = nullptr;
  int* off = nullptr;
  const size_t nk = chunk * N;
  VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&keys), nk * 16 + 16, s));
  VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&off), (chunk + 1) * sizeof(int), s));
  int rc = kOk;
  for (size_t q0 = 0; q0 < nq && rc == kOk; q0 += chunk) {
    const int nc = int(std::min(chunk, nq - q0));
    {
      ProfScope ps(c, "exact_all", s);
      k_score_all<Scorer><<<dim3((N + 255) / 256, nc), 256, 0, s>>>(Q + q0 * src.pd, src.pd, N,
                                                                       allow, sc, keys);
    }
    k_seg_offsets<<<dim3(unsigned((nc + 256) / 256)), 256, 0, s>>>(off, nc, int(N));
    if (hipGetLastError() != hipSuccess) {
      rc = SetError(kInternal, "exact-all launch");
      break;
    }
    rc = SortSegmentsTopK(c, keys, keys + nk, off, nc, int(size_t(nc) * N), int(kk),
                          out_ids + q0 * kk, out_d + q0 * kk, s);
  }
  (void)hipStreamSynchronize(s);
  (void)hipFreeAsync(keys, s);
  (void)hipFreeAsync(off, s);
  return rc;
}

int ExactScanAll(Ctx* c, const ScanSource& src, const float* Q, size_t nq, size_t kk,
                 const uint64_t* allow, uint32_t* out_ids, float* out_d, hipStream_t s) {
  if (nq == 0 || kk == 0) return kOk;
  if (kk > (size_t(1) << 30)) return SetError(kInvalidArgument, "too many results per query");
  if (src.kind == 0)
    return ExactAllT(c, src, FlatScorer{src.X, src.pd, src.metric, c->kset, src.Xmap}, Q, nq, kk, allow,
                     out_ids, out_d, s);
  if (src.kind == 2)
    return ExactAllT(c, src, PqScorer{src.C, src.pq_m}, Q, nq, kk, allow, out_ids, out_d, s);
  return ExactAllT(c, src, Sq8Scorer{src.C, src.vmin, src.scale, src.pd, src.metric, c->kset}, Q,
                   nq, kk, allow, out_ids, out_d, s);
}

// Rerank (src/index/index.cc:89-95) for depths beyond the wave kernel: exact distances of
// the depth candidates per query, sorted, the first k.
__global__ void k_rerank_keys(const float* __restrict__ X, const float* __restrict__ Q, int pd,
                              int metric, int kset, const uint32_t* __restrict__ cand, int depth,
                              int nq, uint64_t* __restrict__ keys) {
  const size_t t = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (t >= size_t(nq) * depth) return;
  const size_t q = t / depth;
  const uint32_t id = cand[t];
  keys[t] = id == kNoId ? kNoKey
                        : dist_key(metric_exact_k(kset, metric, Q + q * pd, X + size_t(id) * pd, pd),
                                   id);
}

int RerankLarge(Ctx* c, const float* X, int pd, int metric, const float* Q, size_t nq,
                const uint32_t* cand, size_t depth, size_t k, uint32_t* out_ids, float* out_d,
                hipStream_t s) {
  if (nq == 0 || k == 0) return kOk;
  size_t chunk = std::max<size_t>(1, (size_t(256) << 20) / (depth * 8));
  chunk = std::min(chunk, nq);
  uint64_t* keys = nullptr;
  int* off = nullptr;
  const size_t nk = chunk * depth;
  VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&keys), nk * 16 + 16, s));
  VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&off), (chunk + 1) * sizeof(int), s));
  int rc = kOk;
  for (size_t q0 = 0; q0 < nq && rc == kOk; q0 += chunk) {
    const int nc = int(std::min(chunk, nq - q0));
    const size_t n = size_t(nc) * depth;
    {
      ProfScope ps(c, "rerank", s);
      k_rerank_keys<<<dim3(unsigned((n + 255) / 256)), 256, 0, s>>>(
          X, Q + q0 * pd, pd, metric, c->kset, cand + q0 * depth, int(depth), nc, keys);
    }
    k_seg_offsets<<<dim3(unsigned((nc + 256) / 256)), 256, 0, s>>>(off, nc, int(depth));
    if (hipGetLastError() != hipSuccess) {
      rc = SetError(kInternal, "rerank launch");
      break;
    }
    rc = SortSegmentsTopK(c, keys, keys + nk, off, nc, int(n), int(k), out_ids + q0 * k,
                          out_d + q0 * k, s);
  }
  (void)hipStreamSynchronize(s);
  (void)hipFreeAsync(keys, s);
  (void)hipFreeAsync(off, s);
  return rc;
}

}  // namespace vdbg
