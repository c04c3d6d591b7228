// ivf_kernels.hip -- IVF-PQ on gfx950: per-list precomputed tables, per-query tables, the
// ADC list scan with a top-R, and the PQ encoder.
//
// IvfPqIndex::search (src/index/quant/ivf_pq.cc:169-222) per query: coarse distances to
// every centroid, the nprobe nearest by (dist, list id); for L2 with precomputed tables
// table[i] = term2[l][i] + qtab[i] with qtab = 2 * (-<q_j, C_j[c]>) and offset = the coarse
// distance; the list's codes scored as offset + adc(table, code) into TopK(max(R, k)); then
// FinishSearch (:28-36).  Every float operation below follows that order, so scores match
// the reference bit for bit:
//   DotAny / L2SqAny  (src/distance/scalar.cc:43-73) four accumulators over i mod 4,
//                     (s0 + s1) + (s2 + s3), products rounded before the add;
//   adc               (src/index/quant/pq.h:36-46) four accumulators over j mod 4.
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <cstring>
#include <vector>

#include "vdbg_device.h"
#include "vdbg_internal.h"

namespace vdbg {

constexpr int kKsub = 256;

__device__ __forceinline__ bool row_ok(const uint64_t* w, uint32_t r) {
  return w == nullptr || ((w[r >> 6] >> (r & 63)) & 1ull);
}

// precompute_tables (ivf_pq.cc:152-167): term2[l][j][c] = DotAny(C, C) + 2 * DotAny(c_l,j, C).
// grid (nlist, m), one thread per centroid c.
__global__ void k_ivf_term2(const float* __restrict__ coarse, int pd,
                            const float* __restrict__ cen, int m, int dsub,
                            float* __restrict__ term2) {
  const int l = blockIdx.x, j = blockIdx.y, c = threadIdx.x;
  const float* cc = cen + (size_t(j) * kKsub + c) * dsub;
  const float* cl = coarse + size_t(l) * pd + size_t(j) * dsub;
  const float norm = dot_any(cc, cc, dsub);
  term2[(size_t(l) * m + j) * kKsub + c] = norm + 2.f * dot_any(cl, cc, dsub);
}

// Per-query tables (ProductQuantizer::compute_table, src/index/quant/pq.cc:63-73): with
// precomputed L2 tables, 2 * (-DotAny(q_j, C_j[c])) (ivf_pq.cc:192-196); for inner product
// and cosine -DotAny(q_j, C_j[c]), shared by every list (:191).  One thread per entry.
__global__ void k_ivf_qtab(const float* __restrict__ Q, int pd, int nq,
                           const float* __restrict__ cen, int m, int dsub, int twice,
                           float* __restrict__ qtab) {
  const size_t e = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  const size_t per = size_t(m) * kKsub;
  if (e >= per * nq) return;
  const int q = int(e / per);
  const int jc = int(e - size_t(q) * per);
  const int j = jc / kKsub;
  const float v = -dot_any(Q + size_t(q) * pd + size_t(j) * dsub, cen + size_t(jc) * dsub, dsub);
  qtab[e] = twice ? v * 2.f : v;
}



// table[j * 256 + c] of probed list l for query q, computed where it is needed: the same
// float operations as the table the reference builds per list (ivf_pq.cc:203-209).
__device__ __forceinline__ float ivf_entry(const IvfScanArgs& a, const float* qv,
                                           const float* qt, uint32_t l, int j, int c) {
  const int e = j * 256 + c;
  if (a.metric != 0) return qt[e];
  if (a.term2 != nullptr) return a.term2[size_t(l) * a.m * 256 + e] + qt[e];
  return l2sq_res_any(qv + size_t(j) * a.dsub, a.coarse + size_t(l) * a.pd + size_t(j) * a.dsub,
                      a.cen + size_t(e) * a.dsub, a.dsub);
}

constexpr int kIvfWaves = 4;
constexpr int kMaxTable = 32 * kKsub;  // m <= 32

// One wave per query.  For each probed list the wave builds the list's table in LDS (one
// fl(term2 + qtab) per entry, exactly table[i] of the reference), then each lane scores one
// code per step with the reference's ADC order and stages the ones below the running
// threshold; full stages of 64 enter the wave top-k.
template <int E>
__global__ __launch_bounds__(kIvfWaves * 64) void k_ivf_scan(IvfScanArgs a) {
  extern __shared__ float lds[];
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int q = blockIdx.x * kIvfWaves + wave;
  if (q >= a.nq) return;
  const int ts = a.m * kKsub;
  const int tl = a.ondemand ? 0 : ts;  // table floats held in LDS
  float* table = lds + size_t(wave) * (tl + 2 * 2 * kWave);
  float* st_d = table + tl;                                   // staging: 128 keys
  uint32_t* st_i = reinterpret_cast<uint32_t*>(st_d + 2 * kWave);
  const float* qv = a.Q + size_t(q) * a.pd;
  const float* qt = a.qtab + size_t(q) * ts;
  const bool l2 = a.metric == 0;
  const bool pre = l2 && a.term2 != nullptr;

  WaveTopK<E> top;
  top.init();
  int staged = 0;
  uint64_t scanned = 0;

  if (!l2 && !a.ondemand) {  // the shared IP table
    for (int e = lane; e < ts; e += kWave) table[e] = qt[e];
  }
  for (int pi = 0; pi < a.nprobe; ++pi) {
    // a probe at or past nlist (a query whose coarse distances are all NaN leaves no-id
    // slots) scans as an empty list
    uint32_t l = a.probe[size_t(q) * a.nprobe + pi];
    const bool lv = l < a.nlist;
    if (!lv) l = 0;
    const float* cl = a.coarse + size_t(l) * a.pd;
    float offset = 0.f;
    __builtin_amdgcn_wave_barrier();
    if (pre) {
      offset = a.probe_d[size_t(q) * a.nprobe + pi];
      const float* t2 = a.term2 + size_t(l) * ts;
      if (!a.ondemand)
        for (int e = lane * 4; e < ts; e += kWave * 4) {
          const float4 x = *reinterpret_cast<const float4*>(t2 + e);
          const float4 y = *reinterpret_cast<const float4*>(qt + e);
          *reinterpret_cast<float4*>(table + e) = make_float4(x.x + y.x, x.y + y.y, x.z + y.z,
                                                              x.w + y.w);
        }
    } else if (l2) {
      // residual table: L2SqAny(q_j - c_l,j, C_j[c]) with the residual rounded per dim
      if (!a.ondemand)
        for (int e = lane; e < ts; e += kWave) {
          const int j = e / kKsub;
          table[e] = l2sq_res_any(qv + j * a.dsub, cl + j * a.dsub, a.cen + size_t(e) * a.dsub,
                                  a.dsub);
        }
    } else {
      offset = -dot_any(qv, cl, a.dim);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    const uint32_t b = lv ? a.off[l] : 0u, e_ = lv ? a.off[l + 1] : 0u;
    scanned += e_ - b;
    for (uint32_t i0 = b; i0 < e_; i0 += kWave) {
      const uint32_t i = i0 + lane;
      float d = __builtin_inff();
      uint32_t id = kNoId;
      if (i < e_) {
        id = a.ids[i];
        if (row_ok(a.allow, id)) {
          const uint8_t* cd = a.codes + size_t(i) * a.m;
          auto T = [&](int j) {
            return a.ondemand ? ivf_entry(a, qv, qt, l, j, cd[j]) : table[j * kKsub + cd[j]];
          };
          float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
          int j = 0;
          for (; j + 4 <= a.m; j += 4) {
            s0 += T(j + 0);
            s1 += T(j + 1);
            s2 += T(j + 2);
            s3 += T(j + 3);
          }
          for (; j < a.m; ++j) s0 += T(j);
          d = offset + ((s0 + s1) + (s2 + s3));
        } else {
          id = kNoId;
        }
      }
      // stage the keys below the running threshold
      float td;
      uint32_t ti;
      top.threshold(td, ti);
      const bool want = id != kNoId && nb_less(d, id, td, ti);
      const uint64_t bal = __ballot(want);
      if (bal != 0) {
        const int pos = staged + __popcll(bal & ((1ull << lane) - 1ull));
        if (want) {
          st_d[pos] = d;
          st_i[pos] = id;
        }
        staged += __popcll(bal);
        if (staged >= kWave) {
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
          const float sd = st_d[lane];
          const uint32_t si = st_i[lane];
          const float rd = lane + kWave < staged ? st_d[lane + kWave] : 0.f;
          const uint32_t ri = lane + kWave < staged ? st_i[lane + kWave] : 0u;
          __builtin_amdgcn_wave_barrier();
          if (lane + kWave < staged) {
            st_d[lane] = rd;
            st_i[lane] = ri;
          }
          staged -= kWave;
          top.insert(sd, si);
        }
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (staged > 0) {
    const bool have = lane < staged;
    top.insert(have ? st_d[lane] : __builtin_inff(), have ? st_i[lane] : kNoId);
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int gi = e * kWave + lane;
    if (gi < a.R) {
      a.out_ids[size_t(q) * a.R + gi] = top.k.id[e];
      a.out_d[size_t(q) * a.R + gi] = top.k.d[e];
    }
  }
  if (a.dc != nullptr) {
    uint64_t valid = 0;
#pragma unroll
    for (int e = 0; e < E; ++e)
      valid += __popcll(__ballot(top.k.id[e] != kNoId && e * kWave + lane < a.R));
    if (lane == 0) a.dc[q] = a.dc_base + scanned + (a.count_top ? valid : 0);
  }
}

// Per-(query, list) offsets for inner product and cosine: -DotAny(q, c_l, d) over the real
// dims (ivf_pq.cc:209).  One thread per (query, probe).
__global__ void k_ivf_offsets(const float* __restrict__ Q, int pd, int dim,
                              const float* __restrict__ coarse, const uint32_t* __restrict__ probe,
                              int nprobe, int nq, uint32_t nlist, float* __restrict__ offs) {
  const size_t t = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (t >= size_t(nq) * nprobe) return;
  const size_t q = t / nprobe;
  const uint32_t l = probe[t];  // past nlist: an empty list (the scans skip it)
  offs[t] = l < nlist ? -dot_any(Q + q * pd, coarse + size_t(l) * pd, dim) : 0.f;
}

__global__ void k_first_probe(const uint32_t* __restrict__ probe, int nprobe, int nq,
                              uint32_t* __restrict__ key, uint32_t* __restrict__ val) {
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= nq) return;
  key[q] = probe[size_t(q) * nprobe];
  val[q] = uint32_t(q);
}

// The queries grouped by their nearest list (first[q], k_first_probe's keys, masked to their
// low bits, bins = 2^bits <= kOrderBins), lists ascending: one block counts the queries of
// each list in LDS, scans the counts and places every query at its list's next slot.  Within
// a list the order is that of the atomics; only the scan's scheduling depends on it, not any
// result.  (One launch where a device radix sort of the same keys takes five.)
constexpr int kOrderBins = 16384;
__global__ __launch_bounds__(1024) void k_order_first(const uint32_t* __restrict__ first,
                                                      int nq, uint32_t mask,
                                                      uint32_t* __restrict__ order) {
  __shared__ uint32_t cnt[kOrderBins];
  __shared__ uint32_t part[1024 / kWave];
  const int t = threadIdx.x, lane = lane_id(), wave = t >> 6;
  const int nbins = int(mask) + 1;
  for (int b = t; b < nbins; b += 1024) cnt[b] = 0u;
  __syncthreads();
  // each thread's keys load kBatch at a time, all in flight together
  constexpr int kBatch = 8;
  auto keys = [&](int q0, uint32_t (&kv)[kBatch]) {
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int q = q0 + i * 1024 + t;
      kv[i] = q < nq ? first[q] & mask : ~0u;
    }
  };
  for (int q0 = 0; q0 < nq; q0 += 1024 * kBatch) {
    uint32_t kv[kBatch];
    keys(q0, kv);
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      if (kv[i] != ~0u) atomicAdd(&cnt[kv[i]], 1u);
  }
  __syncthreads();
  // exclusive scan: thread t owns bins [t * per, (t + 1) * per)
  const int per = (nbins + 1023) / 1024;
  uint32_t own = 0;
  for (int i = 0; i < per; ++i) {
    const int b = t * per + i;
    if (b < nbins) own += cnt[b];
  }
  uint32_t incl = own;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t v = __shfl_up(incl, o);
    if (lane >= o) incl += v;
  }
  if (lane == kWave - 1) part[wave] = incl;
  __syncthreads();
  uint32_t base = 0;
  for (int w = 0; w < wave; ++w) base += part[w];
  uint32_t run = base + incl - own;
  for (int i = 0; i < per; ++i) {
    const int b = t * per + i;
    if (b < nbins) {
      const uint32_t c = cnt[b];
      cnt[b] = run;
      run += c;
    }
  }
  __syncthreads();
  for (int q0 = 0; q0 < nq; q0 += 1024 * kBatch) {
    uint32_t kv[kBatch];
    keys(q0, kv);
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      if (kv[i] != ~0u) order[atomicAdd(&cnt[kv[i]], 1u)] = uint32_t(q0 + i * 1024 + t);
  }
}

// Each query's probed lists with their coarse distances, reordered: the nearest list stays
// first (it tightens the top-R threshold early), the others follow in ascending list id.
// Queries that run together probe mostly the same lists, and walking them in one global
// order makes them touch a shared list's tables at about the same time, while the list is
// still in L2.  The scan's result does not depend on the order (TopK keeps the smallest
// (dist, id) of all).  One wave per query; key = list id (exact in fp32, -1 for the nearest),
// payload = position in the probe list.
template <int E>
__global__ __launch_bounds__(256) void k_sort_probes(const uint32_t* __restrict__ probe,
                                                     const float* __restrict__ probe_d, int nprobe,
                                                     int nq, uint32_t* __restrict__ sprobe,
                                                     float* __restrict__ sprobe_d) {
  const int q = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= nq) return;
  const int lane = lane_id();
  WaveKeys<E> k;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = e * kWave + lane;
    k.d[e] = i == 0 ? -1.f : i < nprobe ? float(probe[size_t(q) * nprobe + i]) : __builtin_inff();
    k.id[e] = i < nprobe ? uint32_t(i) : kNoId;
  }
  bitonic_sort<E>(k);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = e * kWave + lane;
    if (i < nprobe) {
      sprobe[size_t(q) * nprobe + i] = probe[size_t(q) * nprobe + k.id[e]];
      if (probe_d != nullptr) sprobe_d[size_t(q) * nprobe + i] = probe_d[size_t(q) * nprobe + k.id[e]];
    }
  }
}

struct IvfFastArgs {
  const uint32_t* qorder;  // queries sorted by nearest list (nullable)
  const float* offs;       // [nq][nprobe] offsets when there are no precomputed tables
  int items, per_xcd;
};

template <int M>
__device__ __forceinline__ void load_code(const uint8_t* codes, uint32_t i, uint32_t (&w)[(M + 3) / 4]) {
  if constexpr (M == 16) {
    const uint4 v = reinterpret_cast<const uint4*>(codes)[i];
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (M == 8) {
    const uint2 v = reinterpret_cast<const uint2*>(codes)[i];
    w[0] = v.x; w[1] = v.y;
  } else if constexpr (M == 4) {
    w[0] = reinterpret_cast<const uint32_t*>(codes)[i];
  } else {
#pragma unroll
    for (int t = 0; t < (M + 3) / 4; ++t) w[t] = 0;
#pragma unroll
    for (int j = 0; j < M; ++j) w[j >> 2] |= uint32_t(codes[size_t(i) * M + j]) << (8 * (j & 3));
  }
}

// The list scan for tables that fit in registers (m <= 16, precomputed L2 tables or the
// shared inner-product table).  One wave per query; queries run in nearest-list order and
// consecutive ones land on one XCD, so the per-list tables they share stay in that XCD's
// L2.  The query's 2 * (-<q_j, C>) table lives in VGPRs for the whole query; while list p
// is scanned, list p+1's term2 slice is already in flight into VGPRs, and the list table
// fl(term2 + qtab) (the reference's table[i]) is written to LDS per list.  Codes are read
// CH per lane at a time; ADC follows pq.h:36-46.
template <int E, int M>
__global__ __launch_bounds__(kIvfWaves * 64, 2) void k_ivf_scan_fast(IvfScanArgs a, IvfFastArgs f) {
  constexpr int TS = M * kKsub;
  constexpr int V = M;  // float4 per lane: TS / 4 / 64
  constexpr int CH = 4;
  constexpr int W = (M + 3) / 4;
  extern __shared__ float lds[];
  const int b = blockIdx.x;
  const int item = (b & 7) * f.per_xcd + (b >> 3);
  if (item >= f.items) return;
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int slot = item * kIvfWaves + wave;
  if (slot >= a.nq) return;
  const uint32_t q = f.qorder ? f.qorder[slot] : uint32_t(slot);
  float* table = lds + size_t(wave) * (TS + 4 * kWave);
  float* st_d = table + TS;
  uint32_t* st_i = reinterpret_cast<uint32_t*>(st_d + 2 * kWave);
  float4* table4 = reinterpret_cast<float4*>(table);
  const bool pre = a.term2 != nullptr;
  const uint32_t* probe = a.probe + size_t(q) * a.nprobe;

  float4 QT[V], T2[V];
  {
    const float4* qt4 = reinterpret_cast<const float4*>(a.qtab + size_t(q) * TS);
#pragma unroll
    for (int i = 0; i < V; ++i) QT[i] = qt4[i * kWave + lane];
  }
  if (pre) {
    const uint32_t l0 = probe[0] < a.nlist ? probe[0] : 0u;  // (a no-id probe scans nothing)
    const float4* t4 = reinterpret_cast<const float4*>(a.term2 + size_t(l0) * TS);
#pragma unroll
    for (int i = 0; i < V; ++i) T2[i] = t4[i * kWave + lane];
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) table4[i * kWave + lane] = QT[i];
  }

  WaveTopK<E> top;
  top.init();
  int staged = 0;
  uint64_t scanned = 0;
  auto push = [&](float d, uint32_t id, bool valid) {
    float td;
    uint32_t ti;
    top.threshold(td, ti);
    const bool want = valid && nb_less(d, id, td, ti);
    const uint64_t bal = __ballot(want);
    if (bal == 0) return;
    const int pos = staged + __popcll(bal & ((1ull << lane) - 1ull));
    if (want) {
      st_d[pos] = d;
      st_i[pos] = id;
    }
    staged += __popcll(bal);
    if (staged >= kWave) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const float sd = st_d[lane];
      const uint32_t si = st_i[lane];
      const bool more = lane + kWave < staged;
      const float rd = more ? st_d[lane + kWave] : 0.f;
      const uint32_t ri = more ? st_i[lane + kWave] : 0u;
      __builtin_amdgcn_wave_barrier();
      if (more) {
        st_d[lane] = rd;
        st_i[lane] = ri;
      }
      staged -= kWave;
      top.insert(sd, si);
    }
  };

  for (int pi = 0; pi < a.nprobe; ++pi) {
    const uint32_t l = probe[pi];
    const bool lv = l < a.nlist;  // past nlist: an empty list
    const float offset = pre ? a.probe_d[size_t(q) * a.nprobe + pi] : f.offs[size_t(q) * a.nprobe + pi];
    if (pre) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i = 0; i < V; ++i)
        table4[i * kWave + lane] = make_float4(T2[i].x + QT[i].x, T2[i].y + QT[i].y,
                                               T2[i].z + QT[i].z, T2[i].w + QT[i].w);
      if (pi + 1 < a.nprobe) {
        const uint32_t ln = probe[pi + 1] < a.nlist ? probe[pi + 1] : 0u;
        const float4* t4 = reinterpret_cast<const float4*>(a.term2 + size_t(ln) * TS);
#pragma unroll
        for (int i = 0; i < V; ++i) T2[i] = t4[i * kWave + lane];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    const uint32_t b0 = lv ? a.off[l] : 0u, e0 = lv ? a.off[l + 1] : 0u;
    scanned += e0 - b0;
    for (uint32_t c0 = b0; c0 < e0; c0 += CH * kWave) {
      uint32_t w[CH][W];
      uint32_t id[CH];
#pragma unroll
      for (int t = 0; t < CH; ++t) {
        const uint32_t i = c0 + t * kWave + lane;
        id[t] = kNoId;
        if (i < e0) {
          load_code<M>(a.codes, i, w[t]);
          id[t] = a.ids[i];
        }
      }
#pragma unroll
      for (int t = 0; t < CH; ++t) {
        const bool valid = id[t] != kNoId && row_ok(a.allow, id[t]);
        float d = __builtin_inff();
        if (valid) {
          float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
          for (int j = 0; j + 4 <= M; j += 4) {
            const uint32_t x = w[t][j >> 2];
            s0 += table[(j + 0) * kKsub + (x & 0xffu)];
            s1 += table[(j + 1) * kKsub + ((x >> 8) & 0xffu)];
            s2 += table[(j + 2) * kKsub + ((x >> 16) & 0xffu)];
            s3 += table[(j + 3) * kKsub + (x >> 24)];
          }
#pragma unroll
          for (int j = (M / 4) * 4; j < M; ++j)
            s0 += table[j * kKsub + ((w[t][j >> 2] >> (8 * (j & 3))) & 0xffu)];
          d = offset + ((s0 + s1) + (s2 + s3));
        }
        if (__ballot(id[t] != kNoId) == 0) break;
        push(d, id[t], valid);
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (staged > 0) {
    const bool have = lane < staged;
    top.insert(have ? st_d[lane] : __builtin_inff(), have ? st_i[lane] : kNoId);
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int gi = e * kWave + lane;
    if (gi < a.R) {
      a.out_ids[size_t(q) * a.R + gi] = top.k.id[e];
      a.out_d[size_t(q) * a.R + gi] = top.k.d[e];
    }
  }
  if (a.dc != nullptr) {
    uint64_t valid = 0;
#pragma unroll
    for (int e = 0; e < E; ++e)
      valid += __popcll(__ballot(top.k.id[e] != kNoId && e * kWave + lane < a.R));
    if (lane == 0) a.dc[q] = a.dc_base + scanned + (a.count_top ? valid : 0);
  }
}

// ---------------------------------------------------------------- row sums of the term-2 tables
//
// The reference scores a code of list l as offset + adc(table) with table[j][c] =
// fl(term2[l][j][c] + qtab[j][c]) (ivf_pq.cc:203-214).  The term-2 half of that sum depends on
// the row alone, so it is summed once per row when the index is installed:
//   rowsum[i] = sum_j term2[l][j][code_j(i)]   (CSR row i of list l, j ascending, fp32)
//   t2abs[l]  = sum_j max_c |term2[l][j][c]|   (bounds sum_j |term2| of any row of l)
// k_ivf_scan_rs ranks a row by offset + rowsum[i] + sum_j qtab[j][code_j], which reads only the
// query's table, and computes the reference's exact score for the rows ranking near the
// running threshold.

// One block per list, one thread per row.
__global__ __launch_bounds__(256) void k_ivf_rowsum(const uint32_t* __restrict__ off,
                                                     const uint8_t* __restrict__ codes, int m,
                                                     const float* __restrict__ term2,
                                                     float* __restrict__ rowsum) {
  const uint32_t l = blockIdx.x;
  const uint32_t b = off[l], e = off[l + 1];
  const float* t2 = term2 + size_t(l) * m * kKsub;
  for (uint32_t i = b + threadIdx.x; i < e; i += blockDim.x) {
    const uint8_t* cd = codes + size_t(i) * m;
    float s = 0.f;
    for (int j = 0; j < m; ++j) s += t2[j * kKsub + cd[j]];
    rowsum[i] = s;
  }
}

// One wave per list.  The fp32 sum of m non-negative maxima is raised by 2^-16 relative, more
// than its own rounding (m <= 256 additions of relative error 2^-24 each).
__global__ __launch_bounds__(64) void k_ivf_t2abs(const float* __restrict__ term2, int m,
                                                  float* __restrict__ t2abs) {
  const uint32_t l = blockIdx.x;
  const float* t2 = term2 + size_t(l) * m * kKsub;
  float tot = 0.f;
  for (int j = 0; j < m; ++j) {
    float mx = 0.f;
    for (int c = lane_id(); c < kKsub; c += kWave) mx = fmaxf(mx, fabsf(t2[j * kKsub + c]));
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    tot += mx;
  }
  if (lane_id() == 0) t2abs[l] = tot * (1.f + 0x1p-16f);
}

constexpr int kRsWaves = 4;
constexpr int kRsChunk = kWave;  // probed lists whose metadata sits in LDS at a time
constexpr int kQtabQueries = 32; // queries per block of k_ivf_qtab_rs

// One level of a max over the lanes of many values at once: lanes l and l ^ O exchange the
// halves of ax[0, 2N) that the other keeps (bit O of the lane picks the upper half), and each
// keeps the max of the pair in ax[0, N).
template <int O, int N>
__device__ __forceinline__ void halve_max(float (&ax)[32], int lane) {
  static_assert(2 * N <= 32, "the halves lie in the 32 values");
  const bool hi = (lane & O) != 0;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float keep = hi ? ax[i + N] : ax[i];
    const float give = hi ? ax[i] : ax[i + N];
    ax[i] = fmaxf(keep, lane_xor(give, O));
  }
}

// The per-query tables of the row-sum scan: qtab[q][j][c] = 2 * (-DotAny(q_j, C_j[c])), the
// same operations as k_ivf_qtab (ivf_pq.cc:192-196), and qmax[q][j] = max_c |qtab[q][j][c]|.
// grid (m, query groups of 32), one thread per centroid c: with DS = dsub known at compile
// time the centroid stays in registers and each query's sub-vector is read once per block
// (a uniform address); DS = 0 takes dsub at run time.
template <int DS>
__global__ __launch_bounds__(256) void k_ivf_qtab_rs(const float* __restrict__ Q, int pd, int nq,
                                                     const float* __restrict__ cen, int m,
                                                     int dsub_rt, float* __restrict__ qtab,
                                                     float* __restrict__ qmax) {
  __shared__ float wmax[4][kQtabQueries];
  const int dsub = DS > 0 ? DS : dsub_rt;
  const int j = blockIdx.x, c = threadIdx.x, wave = c >> 6, lane = lane_id();
  const int q0 = blockIdx.y * kQtabQueries;
  const int nqb = min(kQtabQueries, nq - q0);
  const float* cc = cen + (size_t(j) * kKsub + c) * dsub;
  float cr[DS > 0 ? DS : 1];
  if constexpr (DS > 0) {
#pragma unroll
    for (int i = 0; i < DS; ++i) cr[i] = cc[i];
  }
  static_assert(kQtabQueries == 32, "the max reduction below halves 32 values five times");
  float ax[kQtabQueries];  // |qtab| of this thread's centroid for each query of the block
#pragma unroll
  for (int t = 0; t < kQtabQueries; ++t) {
    ax[t] = 0.f;
    if (t >= nqb) continue;
    const int q = q0 + t;
    const float* qv = Q + size_t(q) * pd + size_t(j) * dsub;
    float v;
    if constexpr (DS > 0) {
      // DotAny (scalar.cc:43-73): four accumulators over i mod 4, (s0 + s1) + (s2 + s3)
      static_assert(DS % 4 == 0, "whole groups of four");
      float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
      for (int i = 0; i < DS; i += 4) {
        s0 += qv[i] * cr[i];
        s1 += qv[i + 1] * cr[i + 1];
        s2 += qv[i + 2] * cr[i + 2];
        s3 += qv[i + 3] * cr[i + 3];
      }
      v = -((s0 + s1) + (s2 + s3));
    } else {
      v = -dot_any(qv, cc, dsub);
    }
    const float x = v * 2.f;
    qtab[(size_t(q) * m + j) * kKsub + c] = x;
    ax[t] = fabsf(x);
  }
  // The wave's maxima of all 32 queries at once: each exchange of lanes xor o (o = 32, 16,
  // 8, 4, 2) keeps half of the values, the half the lane's bit o selects, at the max of the
  // pair; then xor 1 completes the max over the 64 lanes.  Lane L ends with query
  // (L >> 1) & 31's maximum (bit 5 of the lane selects the upper 16 queries, ..., bit 1 the
  // odd one).
  halve_max<32, 16>(ax, lane);
  halve_max<16, 8>(ax, lane);
  halve_max<8, 4>(ax, lane);
  halve_max<4, 2>(ax, lane);
  halve_max<2, 1>(ax, lane);
  {
    const float mx = fmaxf(ax[0], lane_xor(ax[0], 1));
    if ((lane & 1) == 0) wmax[wave][(lane >> 1) & 31] = mx;
  }
  __syncthreads();
  if (c < nqb)
    qmax[size_t(q0 + c) * m + j] =
        fmaxf(fmaxf(wmax[0][c], wmax[1][c]), fmaxf(wmax[2][c], wmax[3][c]));
}

// The precomputed-table L2 scan on row sums.  One block (four waves) per query; the query's
// table 2 * (-<q_j, C_j[c]>) sits in LDS for the whole query.  The rows of a chunk of 64 probed
// lists (nearest first) are numbered consecutively and dealt to the block's 256 threads CH at a
// time, so every thread streams contiguous code rows whatever the list sizes; the next CH rows
// are in flight while these are ranked.
//
// Ranking value of row i in probed list s: A = offset_s + (rowsum[i] + sum_j qtab[j][c_j]).
// The reference's score E = fl(offset_s + adc) with adc summing fl(term2 + qtab) entries in
// four accumulators (pq.h:36-46) differs from the real value V = offset + sum_j (term2_j +
// qtab_j) by at most gamma_7 * S, and A by at most gamma_17 * S, where S = |offset| +
// sum_j |term2_j| + sum_j |qtab_j| <= |offset| + t2abs[l] + Bq (Bq = sum_j max_c |qtab[j][c]|)
// and gamma_n = n u / (1 - n u), u = 2^-24.  So |A - E| <= gamma_24 * S < 2^-19 * S, and
// U = A + 2^-17 * S_bound >= E.  A row is skipped only when A > tau + 2^-17 * (S_bound + |tau|)
// for a tau no smaller than the d of the answer's R-th key, tested as rowsum + table sum >
// fl(tau + 2^-17 |tau|) + fl(2^-17 S_bound - offset): the margin (128 u of S + |tau|) covers
// |A - E| (24 u of S) with room for the few roundings of these terms (each at most u of
// |tau| + 2 S), so a skipped row has E > tau and cannot be in the answer.  tau is the smallest of
//   - the seed: the first 256 CH rows (the nearest lists) give U bounds; each wave sorts its
//     64 CH and the largest of the four waves' ceil(R/4)-th bounds has at least R rows at or
//     below;
//   - every wave's current R-th key (published by LDS atomic min after each flush).
// Rows not skipped (NaN included) are staged and scored exactly, as the reference scores them,
// and those below the wave's R-th key enter its top-R; the filter is tested on those alone,
// which skips nothing the reference would keep.  The four waves' tops merge at the end.
template <int E, int M, int CH>
__global__ __launch_bounds__(kRsWaves * 64, 6) void k_ivf_scan_rs(IvfScanArgs a, IvfFastArgs f) {
  constexpr int TS = M * kKsub;
  constexpr int W = (M + 3) / 4;
  constexpr int NT = kRsWaves * kWave;
  constexpr int MG = 2 * (kRsWaves - 1) * E * kWave;  // floats of the final merge
  constexpr float kRel = 0x1p-17f;
  __shared__ float smem[TS > MG ? TS : MG];  // the query's table, then the merge
  __shared__ uint32_t p_end[kRsChunk + 1];   // consecutive numbering of the chunk's rows
  __shared__ uint32_t p_beg[kRsChunk], p_list[kRsChunk];
  __shared__ float p_off[kRsChunk], p_bnd[kRsChunk], p_c[kRsChunk];
  __shared__ float seedv[kRsWaves];
  __shared__ float tau_blk;
  __shared__ uint32_t st_row[kRsWaves][2 * kWave];
  __shared__ uint32_t st_slot[kRsWaves][2 * kWave];

  const int b = blockIdx.x;
  const int item = (b & 7) * f.per_xcd + (b >> 3);
  if (item >= f.items) return;  // uniform over the block
  const uint32_t q = f.qorder ? f.qorder[item] : uint32_t(item);
  const int tid = threadIdx.x, wave = tid >> 6, lane = lane_id();
  float* qt = smem;
  {
    const float4* g = reinterpret_cast<const float4*>(a.qtab + size_t(q) * TS);
    for (int e = tid; e < TS / 4; e += NT) reinterpret_cast<float4*>(qt)[e] = g[e];
  }
  if (tid == 0) tau_blk = __builtin_inff();
  float bq = 0.f;
#pragma unroll
  for (int j = 0; j < M; ++j) bq += a.qmax[size_t(q) * M + j];
  bq *= 1.f + 0x1p-16f;
  __syncthreads();

  const int eR = (a.R - 1) / kWave, lR = (a.R - 1) % kWave;  // the R-th key of a top
  const int r4 = (a.R + kRsWaves - 1) / kRsWaves - 1;         // each wave's share of the seed
  WaveTopK<E> top;
  top.init();
  int staged = 0;
  uint64_t scanned = 0;
  float tau0 = __builtin_inff();
  const uint32_t* probe = a.probe + size_t(q) * a.nprobe;
  const float* probe_d = a.probe_d + size_t(q) * a.nprobe;

  // Scores the first min(staged, 64) staged rows exactly and inserts them (wave-uniform).
  auto flush = [&]() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float d = __builtin_inff();
    uint32_t id = kNoId;
    if (lane < staged) {
      // id and code are loaded together, the filter tested last: two round trips
      const uint32_t i = st_row[wave][lane];
      const int s = int(st_slot[wave][lane]);
      const uint32_t rid = a.ids[i];
      uint32_t w[W];
      load_code<M>(a.codes, i, w);
      const float* t2 = a.term2 + size_t(p_list[s]) * TS;
      float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
      for (int j = 0; j + 4 <= M; j += 4) {
        const uint32_t x = w[j >> 2];
        const int e0 = (j + 0) * kKsub + int(x & 0xffu);
        const int e1 = (j + 1) * kKsub + int((x >> 8) & 0xffu);
        const int e2 = (j + 2) * kKsub + int((x >> 16) & 0xffu);
        const int e3 = (j + 3) * kKsub + int((x >> 24) & 0xffu);
        s0 += t2[e0] + qt[e0];
        s1 += t2[e1] + qt[e1];
        s2 += t2[e2] + qt[e2];
        s3 += t2[e3] + qt[e3];
      }
      if (row_ok(a.allow, rid)) {
        d = p_off[s] + ((s0 + s1) + (s2 + s3));
        id = rid;
      }
    }
    const bool more = lane + kWave < staged;
    const uint32_t rr = more ? st_row[wave][lane + kWave] : 0u;
    const uint32_t rs = more ? st_slot[wave][lane + kWave] : 0u;
    __builtin_amdgcn_wave_barrier();
    if (more) {
      st_row[wave][lane] = rr;
      st_slot[wave][lane] = rs;
    }
    staged = staged > kWave ? staged - kWave : 0;
    // only keys below the R-th key can reach the answer (slots past R are never read)
    float rd = __builtin_inff();
    uint32_t ri = kNoId;
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (e == eR) {
        rd = top.k.d[e];
        ri = top.k.id[e];
      }
    rd = __shfl(rd, lR);
    ri = __shfl(ri, lR);
    if (!nb_less(d, id, rd, ri)) {
      d = __builtin_inff();
      id = kNoId;
    }
    top.insert(d, id);
    rd = __builtin_inff();
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (e == eR) rd = top.k.d[e];
    rd = __shfl(rd, lR);
    if (lane == 0)
      __hip_atomic_fetch_min(&tau_blk, rd, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  };

  for (int p0 = 0; p0 < a.nprobe; p0 += kRsChunk) {
    const int np = min(kRsChunk, a.nprobe - p0);
    __syncthreads();  // the previous chunk's metadata is no longer read
    if (wave == 0) {
      uint32_t n = 0;
      if (lane < np) {
        const uint32_t lp = probe[p0 + lane];
        const bool lv = lp < a.nlist;  // past nlist: an empty list
        const uint32_t l = lv ? lp : 0u;
        const uint32_t beg = lv ? a.off[l] : 0u;
        n = lv ? a.off[l + 1] - beg : 0u;
        const float off = probe_d[p0 + lane];
        p_list[lane] = l;
        p_beg[lane] = beg;
        p_off[lane] = off;
        p_bnd[lane] = fabsf(off) + a.t2abs[l] + bq;
        p_c[lane] = kRel * p_bnd[lane] - off;
      }
      uint32_t incl = n;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
      }
      p_end[lane + 1] = incl;
      if (lane == 0) p_end[0] = 0;
    }
    __syncthreads();
    const uint32_t total = p_end[np];
    scanned += total;
    int s = 0;  // this thread's probe slot; its rows only move forward
    struct Rows {
      uint32_t w[CH][W], row[CH];
      float rs[CH];
      int sl[CH];
      bool ok[CH];
    };
    auto fetch = [&](uint32_t v0, Rows& r) {
#pragma unroll
      for (int t = 0; t < CH; ++t) {
        const uint32_t v = v0 + uint32_t(t * NT + tid);
        r.ok[t] = v < total;
        r.sl[t] = 0;
        r.row[t] = 0;
        r.rs[t] = 0.f;
        if (r.ok[t]) {
          while (v >= p_end[s + 1]) ++s;
          r.sl[t] = s;
          r.row[t] = p_beg[s] + (v - p_end[s]);
          load_code<M>(a.codes, r.row[t], r.w[t]);
          r.rs[t] = a.rowsum[r.row[t]];
        }
      }
    };
    Rows cur, nxt;
    if (total > 0) fetch(0, cur);
    for (uint32_t v0 = 0; v0 < total; v0 += NT * CH) {
      if (v0 + NT * CH < total) fetch(v0 + NT * CH, nxt);
      float rq[CH];  // rowsum + table sum: the ranking value less the list's offset
#pragma unroll
      for (int t = 0; t < CH; ++t) {
        rq[t] = __builtin_nanf("");
        if (cur.ok[t]) {
          // any summation order: the bound covers it
          const uint32_t x0 = cur.w[t][0];
          float q0 = qt[0 * kKsub + int(x0 & 0xffu)];
          float q1 = qt[1 * kKsub + int((x0 >> 8) & 0xffu)];
          float q2 = qt[2 * kKsub + int((x0 >> 16) & 0xffu)];
          float q3 = qt[3 * kKsub + int((x0 >> 24) & 0xffu)];
#pragma unroll
          for (int j = 4; j + 4 <= M; j += 4) {
            const uint32_t x = cur.w[t][j >> 2];
            q0 += qt[(j + 0) * kKsub + int(x & 0xffu)];
            q1 += qt[(j + 1) * kKsub + int((x >> 8) & 0xffu)];
            q2 += qt[(j + 2) * kKsub + int((x >> 16) & 0xffu)];
            q3 += qt[(j + 3) * kKsub + int((x >> 24) & 0xffu)];
          }
          rq[t] = cur.rs[t] + ((q0 + q1) + (q2 + q3));
        }
      }
      if (p0 == 0 && v0 == 0) {  // the seed, from the first NT * CH rows (uniform branch)
        WaveKeys<CH> kk;
#pragma unroll
        for (int t = 0; t < CH; ++t) {
          float U = __builtin_inff();
          if (cur.ok[t] && (a.allow == nullptr || row_ok(a.allow, a.ids[cur.row[t]])))
            U = (p_off[cur.sl[t]] + rq[t]) + kRel * p_bnd[cur.sl[t]];
          if (!(U < __builtin_inff())) U = __builtin_inff();  // NaN bounds nothing
          kk.d[t] = U;
          kk.id[t] = uint32_t(t * kWave + lane);
        }
        bitonic_sort<CH>(kk);
        const float mine = __shfl(kk.d[0], r4);
        if (lane == 0) seedv[wave] = mine;
        __syncthreads();
        tau0 = fmaxf(fmaxf(seedv[0], seedv[1]), fmaxf(seedv[2], seedv[3]));
      }
      const float tau = fminf(tau0, __hip_atomic_load(&tau_blk, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_WORKGROUP));
      const float T0 = tau + kRel * fabsf(tau);
#pragma unroll
      for (int t = 0; t < CH; ++t) {
        // A > tau + 2^-17 (S_bound + |tau|) rearranged: rq > T0 + (2^-17 S_bound - offset)
        const bool cand = cur.ok[t] && !(rq[t] > T0 + p_c[cur.sl[t]]);
        const uint64_t bal = __ballot(cand);
        if (bal != 0) {
          const int pos = staged + __popcll(bal & ((1ull << lane) - 1ull));
          if (cand) {
            st_row[wave][pos] = cur.row[t];
            st_slot[wave][pos] = uint32_t(cur.sl[t]);
          }
          staged += __popcll(bal);
          if (staged >= kWave) flush();
        }
      }
      cur = nxt;
    }
    while (staged > 0) flush();  // staged rows name this chunk's slots
  }

  // merge the four waves' tops into wave 0's
  __syncthreads();
  float* mg_d = smem;
  uint32_t* mg_i = reinterpret_cast<uint32_t*>(smem + (kRsWaves - 1) * E * kWave);
  if (wave > 0) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      mg_d[((wave - 1) * E + e) * kWave + lane] = top.k.d[e];
      mg_i[((wave - 1) * E + e) * kWave + lane] = top.k.id[e];
    }
  }
  __syncthreads();
  if (wave != 0) return;
  for (int v = 0; v < kRsWaves - 1; ++v) {
#pragma unroll
    for (int e = 0; e < E; ++e)
      top.insert(mg_d[(v * E + e) * kWave + lane], mg_i[(v * E + e) * kWave + lane]);
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int gi = e * kWave + lane;
    if (gi < a.R) {
      a.out_ids[size_t(q) * a.R + gi] = top.k.id[e];
      a.out_d[size_t(q) * a.R + gi] = top.k.d[e];
    }
  }
  if (a.dc != nullptr) {
    uint64_t valid = 0;
#pragma unroll
    for (int e = 0; e < E; ++e)
      valid += __popcll(__ballot(top.k.id[e] != kNoId && e * kWave + lane < a.R));
    if (lane == 0) a.dc[q] = a.dc_base + scanned + (a.count_top ? valid : 0);
  }
}

// ProductQuantizer::encode (pq.cc:43-57) of the residual x - coarse[assign] (ivf_pq.cc:
// 128-139): per subspace the first centroid with the smallest L2SqAny.  One thread per
// (row, subspace).
__global__ void k_pq_encode(const float* __restrict__ X, uint32_t n, int pd, int dim,
                            const float* __restrict__ coarse, const uint32_t* __restrict__ assign,
                            const float* __restrict__ cen, int m, int dsub,
                            uint8_t* __restrict__ codes) {
  const size_t t = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (t >= size_t(n) * m) return;
  const uint32_t r = uint32_t(t / m);
  const int j = int(t - size_t(r) * m);
  const float* x = X + size_t(r) * pd + size_t(j) * dsub;
  const float* c = coarse != nullptr ? coarse + size_t(assign[r]) * pd + size_t(j) * dsub : nullptr;
  float best = __builtin_inff();
  int arg = 0;
  for (int k = 0; k < kKsub; ++k) {
    const float d = l2sq_res_any(x, c, cen + (size_t(j) * kKsub + k) * dsub, dsub);
    if (d < best) {
      best = d;
      arg = k;
    }
  }
  codes[size_t(r) * m + j] = uint8_t(arg);
}

// ---------------------------------------------------------------- launchers

int IvfTerm2(Ctx* c, const float* coarse, int nlist, int pd, const float* cen, int m, int dsub,
             float* term2, hipStream_t s) {
  if (nlist == 0) return kOk;
  ProfScope ps(c, "ivf_term2", s);
  k_ivf_term2<<<dim3(nlist, m), kKsub, 0, s>>>(coarse, pd, cen, m, dsub, term2);
  VDBG_HIP(hipGetLastError());
  return kOk;
}

int IvfQtab(Ctx* c, const float* Q, int pd, int nq, const float* cen, int m, int dsub,
            int twice, float* qtab, hipStream_t s) {
  const size_t total = size_t(nq) * m * kKsub;
  if (total == 0) return kOk;
  ProfScope ps(c, "ivf_qtab", s);
  k_ivf_qtab<<<dim3(unsigned((total + 255) / 256)), 256, 0, s>>>(Q, pd, nq, cen, m, dsub, twice,
                                                                qtab);
  VDBG_HIP(hipGetLastError());
  return kOk;
}

template <int E>
static void launch_ivf(hipStream_t s, const IvfScanArgs& a, size_t lds) {
  k_ivf_scan<E><<<dim3((a.nq + kIvfWaves - 1) / kIvfWaves), kIvfWaves * 64, lds, s>>>(a);
}

template <int E, int M>
static void launch_fast(hipStream_t s, const IvfScanArgs& a, const IvfFastArgs& f, size_t lds) {
  k_ivf_scan_fast<E, M><<<dim3(f.per_xcd * 8), kIvfWaves * 64, lds, s>>>(a, f);
}

template <int M>
static int launch_fast_m(int e, hipStream_t s, const IvfScanArgs& a, const IvfFastArgs& f) {
  const size_t lds = size_t(kIvfWaves) * (M * kKsub + 4 * kWave) * sizeof(float);
  switch (e) {
    case 1: launch_fast<1, M>(s, a, f, lds); break;
    case 2: launch_fast<2, M>(s, a, f, lds); break;
    case 4: launch_fast<4, M>(s, a, f, lds); break;
    default: return SetError(kNotSupported, "IVF-PQ: max(rerank, k) > 256 on the GPU path");
  }
  return kOk;
}

template <int M>
static int launch_rs_m(int e, hipStream_t s, const IvfScanArgs& a, const IvfFastArgs& f) {
  constexpr int CH = 2;
  const dim3 g(unsigned(f.per_xcd * 8)), blk(kRsWaves * 64);
  switch (e) {
    case 1: k_ivf_scan_rs<1, M, CH><<<g, blk, 0, s>>>(a, f); break;
    case 2: k_ivf_scan_rs<2, M, CH><<<g, blk, 0, s>>>(a, f); break;
    case 4: k_ivf_scan_rs<4, M, CH><<<g, blk, 0, s>>>(a, f); break;
    default: return SetError(kNotSupported, "IVF-PQ: max(rerank, k) > 256 on the GPU path");
  }
  return kOk;
}

// The row-sum scan's per-query tables and their per-subspace maxima (k_ivf_qtab_rs).
int IvfQtabRs(Ctx* c, const float* Q, int pd, int nq, const float* cen, int m, int dsub,
              float* qtab, float* qmax, hipStream_t s) {
  if (nq == 0) return kOk;
  ProfScope ps(c, "ivf_qtab", s);
  const dim3 g(unsigned(m), unsigned((nq + kQtabQueries - 1) / kQtabQueries));
  switch (dsub) {
    case 4: k_ivf_qtab_rs<4><<<g, kKsub, 0, s>>>(Q, pd, nq, cen, m, dsub, qtab, qmax); break;
    case 8: k_ivf_qtab_rs<8><<<g, kKsub, 0, s>>>(Q, pd, nq, cen, m, dsub, qtab, qmax); break;
    case 16: k_ivf_qtab_rs<16><<<g, kKsub, 0, s>>>(Q, pd, nq, cen, m, dsub, qtab, qmax); break;
    case 32: k_ivf_qtab_rs<32><<<g, kKsub, 0, s>>>(Q, pd, nq, cen, m, dsub, qtab, qmax); break;
    default: k_ivf_qtab_rs<0><<<g, kKsub, 0, s>>>(Q, pd, nq, cen, m, dsub, qtab, qmax); break;
  }
  VDBG_HIP(hipGetLastError());
  return kOk;
}

// rowsum / t2abs of an index with precomputed tables (k_ivf_rowsum, k_ivf_t2abs).
int IvfRowSums(Ctx* c, const uint32_t* off, int nlist, const uint8_t* codes, int m,
               const float* term2, float* rowsum, float* t2abs, hipStream_t s) {
  if (nlist == 0) return kOk;
  ProfScope ps(c, "ivf_rowsum", s);
  k_ivf_rowsum<<<dim3(unsigned(nlist)), 256, 0, s>>>(off, codes, m, term2, rowsum);
  VDBG_HIP(hipGetLastError());
  k_ivf_t2abs<<<dim3(unsigned(nlist)), 64, 0, s>>>(term2, m, t2abs);
  VDBG_HIP(hipGetLastError());
  return kOk;
}

// scratch: null, or at least IvfScanScratchBytes(nq, nprobe) bytes the caller owns (no
// allocation of its own then)
size_t IvfScanScratchBytes(size_t nq, size_t nprobe) { return nq * 16 + nq * nprobe * 12 + 4096; }

int IvfScan(Ctx* c, const IvfScanArgs& a_in, hipStream_t s, void* scratch) {
  if (a_in.nq == 0) return kOk;
  IvfScanArgs a = a_in;
  a.ondemand = a.m * kKsub > kMaxTable ? 1 : 0;  // tables above 32 KB: entries per lookup
  int e = 1;
  while (kWave * e < a.R) e <<= 1;
  const bool l2 = a.metric == 0;
  const bool fast_ok = (a.m == 4 || a.m == 8 || a.m == 16) && (!l2 || a.term2 != nullptr);
  if (fast_ok) {
    // queries in nearest-list order; offsets for the inner-product table
    void* buf = scratch;
    const size_t nq = size_t(a.nq);
    if (buf == nullptr) VDBG_HIP(hipMallocAsync(&buf, IvfScanScratchBytes(nq, size_t(a.nprobe)), s));
    uint32_t* key = static_cast<uint32_t*>(buf);
    uint32_t* val = key + nq;
    uint32_t* key2 = val + nq;
    uint32_t* order = key2 + nq;
    float* offs = reinterpret_cast<float*>(order + nq);
    uint32_t* sprobe = reinterpret_cast<uint32_t*>(offs + nq * a.nprobe);
    float* sprobe_d = reinterpret_cast<float*>(sprobe + nq * a.nprobe);
    // with row sums: one block per query (k_ivf_scan_rs) walking its lists nearest first, so
    // the threshold falls early; otherwise one wave per query
    const bool rs = l2 && a.rowsum != nullptr && a.t2abs != nullptr && a.qmax != nullptr &&
                    a.qtab != nullptr && a.probe_d != nullptr;
    IvfScanArgs as = a;  // the per-list table scan's view: probes in ascending list id
    if (!rs && a.nprobe > 1 && a.nprobe <= 4 * kWave) {
      const dim3 g(unsigned((nq + 3) / 4));
      if (a.nprobe <= kWave)
        k_sort_probes<1><<<g, 256, 0, s>>>(a.probe, a.probe_d, a.nprobe, a.nq, sprobe, sprobe_d);
      else if (a.nprobe <= 2 * kWave)
        k_sort_probes<2><<<g, 256, 0, s>>>(a.probe, a.probe_d, a.nprobe, a.nq, sprobe, sprobe_d);
      else
        k_sort_probes<4><<<g, 256, 0, s>>>(a.probe, a.probe_d, a.nprobe, a.nq, sprobe, sprobe_d);
      VDBG_HIP(hipGetLastError());
      as.probe = sprobe;
      as.probe_d = a.probe_d != nullptr ? sprobe_d : nullptr;
    }
    // the keys are list ids below nlist (dc_base): only their low bits take sort passes
    int end_bit = 1;
    while (end_bit < 32 && (uint64_t(1) << end_bit) < a.dc_base) ++end_bit;
    void* tmp = nullptr;
    k_first_probe<<<dim3(unsigned((nq + 255) / 256)), 256, 0, s>>>(a.probe, a.nprobe, a.nq, key, val);
    VDBG_HIP(hipGetLastError());
    if ((uint64_t(1) << end_bit) <= uint64_t(kOrderBins)) {
      k_order_first<<<dim3(1), 1024, 0, s>>>(key, a.nq, uint32_t((uint64_t(1) << end_bit) - 1),
                                             order);
      VDBG_HIP(hipGetLastError());
    } else {
      size_t tmp_bytes = 0;
      VDBG_HIP(hipcub::DeviceRadixSort::SortPairs(nullptr, tmp_bytes, key, key2, val, order, a.nq,
                                                  0, end_bit, s));
      VDBG_HIP(hipMallocAsync(&tmp, tmp_bytes + 16, s));
      VDBG_HIP(hipcub::DeviceRadixSort::SortPairs(tmp, tmp_bytes, key, key2, val, order, a.nq, 0,
                                                  end_bit, s));
    }
    if (!l2) {
      k_ivf_offsets<<<dim3(unsigned((nq * a.nprobe + 255) / 256)), 256, 0, s>>>(
          a.Q, a.pd, a.dim, a.coarse, as.probe, a.nprobe, a.nq, a.nlist, offs);
      VDBG_HIP(hipGetLastError());
    }
    IvfFastArgs f{order, l2 ? nullptr : offs, 0, 0};
    f.items = rs ? a.nq : (a.nq + kIvfWaves - 1) / kIvfWaves;
    f.per_xcd = (f.items + 7) / 8;
    int rc = kOk;
    {
      ProfScope ps(c, "ivf_scan", s);
      if (rs) {
        switch (a.m) {
          case 4: rc = launch_rs_m<4>(e, s, as, f); break;
          case 8: rc = launch_rs_m<8>(e, s, as, f); break;
          default: rc = launch_rs_m<16>(e, s, as, f); break;
        }
      } else {
        switch (a.m) {
          case 4: rc = launch_fast_m<4>(e, s, as, f); break;
          case 8: rc = launch_fast_m<8>(e, s, as, f); break;
          default: rc = launch_fast_m<16>(e, s, as, f); break;
        }
      }
      if (rc == kOk && hipGetLastError() != hipSuccess) rc = SetError(kInternal, "ivf scan launch");
    }
    if (tmp != nullptr) (void)hipFreeAsync(tmp, s);
    if (scratch == nullptr) (void)hipFreeAsync(buf, s);
    return rc;
  }
  const size_t lds = size_t(kIvfWaves) * ((a.ondemand ? 0 : a.m * kKsub) + 4 * kWave) * sizeof(float);
  ProfScope ps(c, "ivf_scan", s);
  switch (e) {
    case 1: launch_ivf<1>(s, a, lds); break;
    case 2: launch_ivf<2>(s, a, lds); break;
    case 4: launch_ivf<4>(s, a, lds); break;
    default: return SetError(kNotSupported, "IVF-PQ: max(rerank, k) > 256 on the GPU path");
  }
  VDBG_HIP(hipGetLastError());
  return kOk;
}

// ---------------------------------------------------------------- deep top-R

// Candidates per query: the sizes of its probed lists (every code is scored once).
__global__ void k_probe_counts(const uint32_t* __restrict__ probe, int nprobe, int nq,
                               uint32_t nlist, const uint32_t* __restrict__ off,
                               uint64_t* __restrict__ cnt) {
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= nq) return;
  uint64_t n = 0;
  for (int i = 0; i < nprobe; ++i) {
    const uint32_t l = probe[size_t(q) * nprobe + i];
    if (l < nlist) n += off[l + 1] - off[l];
  }
  cnt[q] = n;
}

// One wave per query of the chunk [q0, q0 + nc): the tables and ADC of k_ivf_scan, with
// every scored code written as a (dist, id) key into the query's segment (disallowed rows
// get kNoKey), for a segmented sort that keeps TopK(R) when R exceeds the wave top-k.
__global__ __launch_bounds__(kIvfWaves * 64) void k_ivf_score_all(IvfScanArgs a, int q0, int nc,
                                                                 const int* __restrict__ seg,
                                                                 uint64_t* __restrict__ keys) {
  extern __shared__ float lds[];
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int qi = blockIdx.x * kIvfWaves + wave;
  if (qi >= nc) return;
  const int q = q0 + qi;
  const int ts = a.m * kKsub;
  float* table = lds + size_t(wave) * (a.ondemand ? 0 : ts);
  const float* qv = a.Q + size_t(q) * a.pd;
  const float* qt = a.qtab + size_t(q) * ts;
  const bool l2 = a.metric == 0;
  const bool pre = l2 && a.term2 != nullptr;
  if (!l2 && !a.ondemand)
    for (int e = lane; e < ts; e += kWave) table[e] = qt[e];
  int pos = seg[qi];
  for (int pi = 0; pi < a.nprobe; ++pi) {
    // a probe at or past nlist (a query whose coarse distances are all NaN leaves no-id
    // slots) scans as an empty list
    uint32_t l = a.probe[size_t(q) * a.nprobe + pi];
    const bool lv = l < a.nlist;
    if (!lv) l = 0;
    const float* cl = a.coarse + size_t(l) * a.pd;
    float offset = 0.f;
    __builtin_amdgcn_wave_barrier();
    if (pre) {
      offset = a.probe_d[size_t(q) * a.nprobe + pi];
      const float* t2 = a.term2 + size_t(l) * ts;
      if (!a.ondemand)
        for (int e = lane; e < ts; e += kWave) table[e] = t2[e] + qt[e];
    } else if (l2) {
      if (!a.ondemand)
        for (int e = lane; e < ts; e += kWave) {
          const int j = e / kKsub;
          table[e] = l2sq_res_any(qv + j * a.dsub, cl + j * a.dsub, a.cen + size_t(e) * a.dsub,
                                  a.dsub);
        }
    } else {
      offset = -dot_any(qv, cl, a.dim);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t b = lv ? a.off[l] : 0u, e_ = lv ? a.off[l + 1] : 0u;
    for (uint32_t i0 = b; i0 < e_; i0 += kWave) {
      const uint32_t i = i0 + lane;
      if (i < e_) {
        const uint32_t id = a.ids[i];
        uint64_t key = kNoKey;
        if (row_ok(a.allow, id)) {
          const uint8_t* cd = a.codes + size_t(i) * a.m;
          auto T = [&](int j) {
            return a.ondemand ? ivf_entry(a, qv, qt, l, j, cd[j]) : table[j * kKsub + cd[j]];
          };
          float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
          int j = 0;
          for (; j + 4 <= a.m; j += 4) {
            s0 += T(j + 0);
            s1 += T(j + 1);
            s2 += T(j + 2);
            s3 += T(j + 3);
          }
          for (; j < a.m; ++j) s0 += T(j);
          key = dist_key(offset + ((s0 + s1) + (s2 + s3)), id);
        }
        keys[pos + int(i - b)] = key;
      }
    }
    pos += int(e_ - b);
  }
}

__global__ void k_ivf_dc(const uint32_t* __restrict__ top_ids, int R, int nq,
                         const uint64_t* __restrict__ cnt, uint64_t base, int count_top,
                         uint64_t* __restrict__ dc) {
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= nq) return;
  uint64_t v = 0;
  if (count_top)
    for (int i = 0; i < R; ++i) v += top_ids[size_t(q) * R + i] != kNoId ? 1 : 0;
  dc[q] = base + cnt[q] + v;
}

// The ADC scan for R > 256: every code scored into per-query key segments (chunks of at
// most 2^25 keys), sorted, the first R kept in out_ids / out_d as the scan's TopK(R).
int IvfScanDeep(Ctx* c, const IvfScanArgs& a_in, hipStream_t s) {
  if (a_in.nq == 0) return kOk;
  IvfScanArgs a = a_in;
  a.ondemand = a.m * kKsub > kMaxTable ? 1 : 0;
  const size_t nq = size_t(a.nq);
  uint64_t* cnt = nullptr;
  VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&cnt), nq * 8, s));
  k_probe_counts<<<dim3(unsigned((nq + 255) / 256)), 256, 0, s>>>(a.probe, a.nprobe, a.nq, a.nlist,
                                                                  a.off, cnt);
  VDBG_HIP(hipGetLastError());
  std::vector<uint64_t> h(nq);
  VDBG_HIP(hipMemcpyAsync(h.data(), cnt, nq * 8, hipMemcpyDeviceToHost, s));
  VDBG_HIP(hipStreamSynchronize(s));
  constexpr uint64_t kChunkKeys = uint64_t(1) << 25;
  uint64_t maxc = 0;
  for (uint64_t v : h) maxc = std::max(maxc, v);
  const uint64_t cap = std::max(kChunkKeys, maxc);
  uint64_t* keys = nullptr;
  int* seg = nullptr;
  VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&keys), cap * 16 + 16, s));
  VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&seg), (nq + 1) * sizeof(int), s));
  const size_t lds = size_t(kIvfWaves) * (a.ondemand ? 0 : a.m * kKsub) * sizeof(float);
  int rc = kOk;
  std::vector<int> off;
  for (size_t q0 = 0; q0 < nq && rc == kOk;) {
    off.assign(1, 0);
    size_t q1 = q0;
    uint64_t total = 0;
    while (q1 < nq && (q1 == q0 || total + h[q1] <= cap)) {
      total += h[q1];
      off.push_back(int(total));
      ++q1;
    }
    const int nc = int(q1 - q0);
    if (hipMemcpyAsync(seg, off.data(), off.size() * sizeof(int), hipMemcpyHostToDevice, s) !=
        hipSuccess) {
      rc = SetError(kInternal, "segment offsets upload");
      break;
    }
    {
      ProfScope ps(c, "ivf_scan", s);
      k_ivf_score_all<<<dim3(unsigned((nc + kIvfWaves - 1) / kIvfWaves)), kIvfWaves * 64, lds, s>>>(
          a, int(q0), nc, seg, keys);
    }
    if (hipGetLastError() != hipSuccess) {
      rc = SetError(kInternal, "ivf score launch");
      break;
    }
    rc = SortSegmentsTopK(c, keys, keys + cap, seg, nc, int(total), a.R,
                          a.out_ids + q0 * size_t(a.R), a.out_d + q0 * size_t(a.R), s);
    // the offsets buffer is rewritten for the next chunk: finish this one first
    if (rc == kOk && hipStreamSynchronize(s) != hipSuccess) rc = SetError(kInternal, "sync");
    q0 = q1;
  }
  if (rc == kOk && a.dc != nullptr) {
    k_ivf_dc<<<dim3(unsigned((nq + 255) / 256)), 256, 0, s>>>(a.out_ids, a.R, a.nq, cnt, a.dc_base,
                                                             a.count_top, a.dc);
    if (hipGetLastError() != hipSuccess) rc = SetError(kInternal, "dist count launch");
  }
  (void)hipStreamSynchronize(s);
  (void)hipFreeAsync(keys, s);
  (void)hipFreeAsync(seg, s);
  (void)hipFreeAsync(cnt, s);
  return rc;
}

int PqEncode(Ctx* c, const float* X, uint32_t n, int pd, int dim, const float* coarse,
             const uint32_t* assign, const float* cen, int m, int dsub, uint8_t* codes,
             hipStream_t s) {
  const size_t total = size_t(n) * m;
  if (total == 0) return kOk;
  ProfScope ps(c, "pq_encode", s);
  k_pq_encode<<<dim3(unsigned((total + 255) / 256)), 256, 0, s>>>(X, n, pd, dim, coarse, assign,
                                                                 cen, m, dsub, codes);
  VDBG_HIP(hipGetLastError());
  return kOk;
}

}  // namespace vdbg

