// flat_kernels.hip -- exact flat search on gfx950.
//
// vdb's FlatIndex scans every row with an AVX-512 distance kernel and keeps a top-k heap
// per query (src/index/flat_index.cc:11-39, 73-77).  Here a batch of queries runs as:
//
//   1. k_query_prep   ||q||^2 and the rounding bound of the GEMM form for each query; a
//                     query is "exact" when integer-valued data keeps every partial sum of
//                     the GEMM form exactly representable (then the bound is zero).
//   2. k_prepass      the exact k-th smallest distance over a strided sample of rows, an
//                     upper bound on the k-th smallest over all rows, which turns into a
//                     per-query admission threshold for the GEMM.
//   3. k_flat_gemm    Q.X^T on fp32 MFMA (v_mfma_f32_32x32x2f32), X streamed through LDS,
//                     epilogue ||x||^2 - 2 q.x compared with the threshold; the few rows
//                     that pass are appended to per-(query, chunk, half-wave) buffers.
//   4. k_select       per query: the K' smallest candidates by GEMM value (wave bitonic
//                     top-k), exact re-scoring in the reference's AVX-512 order, sort by
//                     (dist, id), and a certificate that no unselected row can enter the
//                     top k.  Queries that fail it (or overflowed a buffer) are re-scanned
//                     exactly by k_exact_scan and merged by k_select.
//
// Distances returned are always the exact AVX-512-order values; the GEMM only ranks.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "vdbg_device.h"
#include "vdbg_internal.h"

namespace vdbg {

typedef float v16f __attribute__((ext_vector_type(16)));

// ================================================================ small helpers

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ int wave_and(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v &= __shfl_xor(v, o);
  return v;
}

// Order-preserving float <-> uint32 map for atomicMin/atomicMax.
__device__ __forceinline__ uint32_t ord_enc(float f) {
  uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
static inline float ord_dec(uint32_t e) {
  uint32_t b = (e & 0x80000000u) ? (e & 0x7fffffffu) : ~e;
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}

__device__ __forceinline__ bool row_allowed(const uint64_t* w, uint32_t r) {
  return w == nullptr || ((w[r >> 6] >> (r & 63)) & 1ull);
}

// ================================================================ row statistics

struct RowStatsDev {
  uint32_t lo, hi, max_abs, xn_max;
  int all_int;
};

// One thread per row: ||x||^2 (sequential fmaf over the padded row), plus min, max,
// max |x| and integrality, reduced per wave and folded in with atomics.
__global__ __launch_bounds__(256) void k_row_stats(const float* __restrict__ X, size_t n,
                                                   int pd, float* __restrict__ norms,
                                                   RowStatsDev* __restrict__ st) {
  size_t r = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  float lo = __builtin_inff(), hi = -__builtin_inff(), ma = 0.f, nn = 0.f;
  int ai = 1;
  if (r < n) {
    const float* x = X + r * size_t(pd);
    float s = 0.f;
    for (int i = 0; i < pd; i += 4) {
      float4 v = *reinterpret_cast<const float4*>(x + i);
      float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        s = fmaf(e[t], e[t], s);
        lo = fminf(lo, e[t]);
        hi = fmaxf(hi, e[t]);
        ma = fmaxf(ma, fabsf(e[t]));
        ai &= (e[t] == rintf(e[t])) ? 1 : 0;
      }
    }
    norms[r] = s;
    nn = s;
  }
  lo = wave_min(lo);
  hi = wave_max(hi);
  ma = wave_max(ma);
  nn = wave_max(nn);
  ai = wave_and(ai);
  if (lane_id() == 0) {
    atomicMin(&st->lo, ord_enc(lo));
    atomicMax(&st->hi, ord_enc(hi));
    atomicMax(&st->max_abs, __float_as_uint(ma));
    atomicMax(&st->xn_max, __float_as_uint(nn));
    if (!ai) atomicAnd(&st->all_int, 0);
  }
}

int LaunchRowStats(Ctx* c, hipStream_t s, const float* rows, size_t n, size_t pd, float* norms,
                   RowStats* out) {
  RowStatsDev init{0xffffffffu, 0u, 0u, 0u, 1};
  RowStatsDev* d = nullptr;
  VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&d), sizeof(RowStatsDev), s));
  VDBG_HIP(hipMemcpyAsync(d, &init, sizeof(init), hipMemcpyHostToDevice, s));
  if (n > 0) {
    ProfScope ps(c, "row_stats", s);
    dim3 grid(static_cast<unsigned>((n + 255) / 256));
    k_row_stats<<<grid, 256, 0, s>>>(rows, n, static_cast<int>(pd), norms, d);
    VDBG_HIP(hipGetLastError());
  }
  RowStatsDev h;
  VDBG_HIP(hipMemcpyAsync(&h, d, sizeof(h), hipMemcpyDeviceToHost, s));
  VDBG_HIP(hipStreamSynchronize(s));
  VDBG_HIP(hipFreeAsync(d, s));
  if (n == 0) {
    *out = RowStats{};
    return kOk;
  }
  out->lo = ord_dec(h.lo);
  out->hi = ord_dec(h.hi);
  std::memcpy(&out->max_abs, &h.max_abs, 4);
  std::memcpy(&out->xn_max, &h.xn_max, 4);
  out->all_int = h.all_int;
  return kOk;
}

// ================================================================ query preparation

struct PrepArgs {
  const float* Q;
  int nq, pd;
  RowStats xs;
  float* qn;     // ||q||^2 in fp32
  float* eb;     // bound on |GEMM-form value + ||q||^2 - exact distance|
  int* exact;    // 1 when that bound is zero
};

// One wave per query.  The GEMM form is exact when every value is an integer and every
// partial sum that any summation order can form stays below 2^24:
//   pd*max|x|^2, pd*max|q|^2, pd*max|x|*max|q| (norms and dot products) and pd*R^2 with R
//   the value range (distances, and ||x||^2 - 2q.x = dist - ||q||^2).
// Otherwise the bound is (4*pd + 16) * 2^-24 * (||q||^2 + max ||x||^2): the MFMA dot and the
// fp32 norms carry at most pd roundings each on sums bounded by ||q||^2 + ||x||^2, the
// AVX-512-order exact value at most pd/16 + 6, and the factor two covers the fp32 arithmetic
// that forms thresholds from the bound.
__global__ __launch_bounds__(256) void k_query_prep(PrepArgs a) {
  const int q = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= a.nq) return;
  const float* v = a.Q + size_t(q) * a.pd;
  float s = 0.f, lo = __builtin_inff(), hi = -__builtin_inff(), ma = 0.f;
  int ai = 1;
  for (int i = lane_id(); i < a.pd; i += kWave) {
    float e = v[i];
    s = fmaf(e, e, s);
    lo = fminf(lo, e);
    hi = fmaxf(hi, e);
    ma = fmaxf(ma, fabsf(e));
    ai &= (e == rintf(e)) ? 1 : 0;
  }
  s = wave_sum(s);
  lo = wave_min(lo);
  hi = wave_max(hi);
  ma = wave_max(ma);
  ai = wave_and(ai);
  if (lane_id() == 0) {
    const double pd = a.pd, lim = 16777216.0;
    const double mx = a.xs.max_abs, mq = ma;
    const double range = double(fmaxf(hi, a.xs.hi)) - double(fminf(lo, a.xs.lo));
    const bool ex = a.xs.all_int && ai && pd * mx * mx < lim && pd * mq * mq < lim &&
                    pd * mx * mq < lim && pd * range * range < lim;
    a.qn[q] = s;
    a.exact[q] = ex ? 1 : 0;
    a.eb[q] = ex ? 0.f
                 : float((4.0 * pd + 16.0) * (1.0 / 16777216.0) *
                         (double(s) + double(a.xs.xn_max)) * 1.001);
  }
}

// ================================================================ sample pre-pass

struct PrepassArgs {
  const float* X;
  const float* Q;
  const uint64_t* allow;
  int nq, pd, metric, k;
  uint32_t N, S;  // sample row s is s * N / S
  const float* qn;
  const float* eb;
  float* T;       // admission threshold on the GEMM value
};

// One wave per query: exact distances to the sample rows into a wave top-k; the k-th
// smallest bounds the k-th smallest over all rows from above.
template <int E>
__global__ __launch_bounds__(256) void k_prepass(PrepassArgs a) {
  const int q = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= a.nq) return;
  const float* qv = a.Q + size_t(q) * a.pd;
  WaveTopK<E> top;
  top.init();
  for (uint32_t s0 = 0; s0 < a.S; s0 += kWave) {
    const uint32_t s = s0 + lane_id();
    float d = __builtin_inff();
    uint32_t id = kNoId;
    if (s < a.S) {
      const uint32_t r = uint32_t((uint64_t(s) * a.N) / a.S);
      if (row_allowed(a.allow, r)) {
        d = metric_exact(a.metric, qv, a.X + size_t(r) * a.pd, a.pd);
        id = r;
      }
    }
    top.insert(d, id);
  }
  const int g = a.k - 1;
  float kth = __builtin_inff();
#pragma unroll
  for (int e = 0; e < E; ++e) {
    float v = __shfl(top.k.d[e], g & (kWave - 1));
    if (e == g / kWave) kth = v;
  }
  if (lane_id() == 0) {
    float t = __builtin_inff();
    if (kth < __builtin_inff()) t = a.metric == 0 ? (kth - a.qn[q]) + a.eb[q] : kth + a.eb[q];
    a.T[q] = t;
  }
}

// ================================================================ MFMA GEMM + filter

struct GemmArgs {
  const float* X;
  const float* xn;
  const float* Q;
  const float* T;
  const uint64_t* allow;
  uint2* cand;        // [(q * nchunks + chunk) * 2 + half][caph] (GEMM value bits, row)
  uint32_t* counts;   // [(q * nchunks + chunk) * 2 + half]
  int* ovf;           // [q] set when a buffer overflowed
  uint32_t N;
  int nq;
  uint32_t chunk_rows;
  int nchunks;
  int caph;
};

constexpr int kGemmRows = 64;  // rows per LDS tile (two 32-row MFMA blocks)

// Block = 4 waves = 128 queries (32 per wave) x one chunk of rows.  Each wave keeps its 32
// queries in VGPRs as the MFMA B operand: lane l holds query (l % 32), dims
// [h*PD/2, (h+1)*PD/2) with h = l / 32, so MFMA step t contracts dims t and PD/2 + t (the
// summation order is irrelevant: the GEMM value only ranks, exact distances are recomputed).
// 64-row X tiles are double-buffered in LDS and feed the A operand.  The 32x32 accumulator
// of v_mfma_f32_32x32x2f32 gives lane l the values of query (l % 32) for rows
// 8*(r/4) + 4*h + (r%4), r = 0..15.
template <int PD, int METRIC>
__global__ __launch_bounds__(256, 2) void k_flat_gemm(GemmArgs a) {
  constexpr int STR = PD + 4;  // padded LDS row stride (floats)
  constexpr int HALF = PD / 2;
  constexpr int F4_PER_TILE = kGemmRows * PD / 4;
  constexpr int F4_PER_THREAD = (F4_PER_TILE + 255) / 256;
  __shared__ __attribute__((aligned(16))) float xs[2][kGemmRows * STR];
  __shared__ float xns[2][kGemmRows];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int j = lane & 31;
  const int h = lane >> 5;
  const int q = blockIdx.x * 128 + wave * 32 + j;
  const int chunk = blockIdx.y;
  const uint32_t r_begin = uint32_t(chunk) * a.chunk_rows;
  const uint32_t r_end = min(a.N, r_begin + a.chunk_rows);

  // query fragment
  float qv[HALF];
  if (q < a.nq) {
    const float* src = a.Q + size_t(q) * PD + h * HALF;
#pragma unroll
    for (int t = 0; t < HALF; t += 4) {
      float4 v = *reinterpret_cast<const float4*>(src + t);
      qv[t] = v.x;
      qv[t + 1] = v.y;
      qv[t + 2] = v.z;
      qv[t + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int t = 0; t < HALF; ++t) qv[t] = 0.f;
  }
  const float T = q < a.nq ? a.T[q] : -__builtin_inff();
  const size_t seg = (size_t(q) * a.nchunks + chunk) * 2 + h;
  uint2* out = a.cand + seg * size_t(a.caph);
  uint32_t cnt = 0;

  float4 pre[F4_PER_THREAD];
  float pre_n = 0.f;
  auto load_tile = [&](uint32_t base) {
    const float4* src = reinterpret_cast<const float4*>(a.X + size_t(base) * PD);
    const uint32_t valid = r_end > base ? min(uint32_t(kGemmRows), r_end - base) : 0u;
#pragma unroll
    for (int i = 0; i < F4_PER_THREAD; ++i) {
      const int f = tid + 256 * i;
      const int row = f / (PD / 4);
      if (f < F4_PER_TILE && uint32_t(row) < valid)
        pre[i] = src[f];
      else
        pre[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    pre_n = (tid < kGemmRows && uint32_t(tid) < valid) ? a.xn[base + tid] : 0.f;
  };
  auto store_tile = [&](int b) {
#pragma unroll
    for (int i = 0; i < F4_PER_THREAD; ++i) {
      const int f = tid + 256 * i;
      if (f < F4_PER_TILE) {
        const int row = f / (PD / 4), c4 = f % (PD / 4);
        *reinterpret_cast<float4*>(&xs[b][row * STR + c4 * 4]) = pre[i];
      }
    }
    if (tid < kGemmRows) xns[b][tid] = pre_n;
  };

  if (r_begin < r_end) {
    load_tile(r_begin);
    store_tile(0);
  }
  __syncthreads();

  int buf = 0;
  for (uint32_t base = r_begin; base < r_end; base += kGemmRows) {
    const uint32_t next = base + kGemmRows;
    if (next < r_end) load_tile(next);

    v16f acc0, acc1;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc0[r] = acc1[r] = 0.f;
    const float* xa0 = &xs[buf][j * STR + h * HALF];
    const float* xa1 = xa0 + 32 * STR;
#pragma unroll
    for (int t = 0; t < HALF; t += 4) {
      const float4 x0 = *reinterpret_cast<const float4*>(xa0 + t);
      const float4 x1 = *reinterpret_cast<const float4*>(xa1 + t);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.x, qv[t + 0], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.x, qv[t + 0], acc1, 0, 0, 0);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.y, qv[t + 1], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.y, qv[t + 1], acc1, 0, 0, 0);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.z, qv[t + 2], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.z, qv[t + 2], acc1, 0, 0, 0);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.w, qv[t + 3], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.w, qv[t + 3], acc1, 0, 0, 0);
    }

    // epilogue: GEMM value vs the query's threshold; rare passes go to the buffer
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rl = blk * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        const float g = blk == 0 ? acc0[r] : acc1[r];
        const float v = METRIC == 0 ? fmaf(-2.f, g, xns[buf][rl]) : -g;
        if (v <= T) {
          const uint32_t row = base + rl;
          if (q < a.nq && row < r_end && row_allowed(a.allow, row)) {
            if (cnt < uint32_t(a.caph)) out[cnt] = make_uint2(__float_as_uint(v), row);
            ++cnt;
          }
        }
      }
    }

    if (next < r_end) store_tile(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }

  if (q < a.nq) {
    a.counts[seg] = min(cnt, uint32_t(a.caph));
    if (cnt > uint32_t(a.caph)) a.ovf[q] = 1;
  }
}

// ================================================================ selection / merge

struct SelectArgs {
  const float* X;
  const float* Q;
  int pd, metric;
  const uint2* cand;
  const uint32_t* counts;
  int nseg, cap;
  const int* ovf;          // nullable
  const float* qn;         // rescore mode
  const float* eb;
  const int* exact;
  const uint32_t* qlist;   // nullable: slot i answers query qlist[i]
  int nslots, k;
  int rescore;             // 1: candidates hold GEMM values; 0: exact distances
  uint32_t* out_ids;
  float* out_d;
  uint32_t* fb_list;       // rescore mode: queries that need the exact re-scan
  uint32_t* fb_count;
};

constexpr int kMaxSeg = 1024;

// One wave per slot.  Candidates of the slot's segments are streamed (a prefix sum over the
// segment counts maps a flat index to its segment) into a wave top-k of capacity 64*E.
template <int E>
__global__ __launch_bounds__(256) void k_select(SelectArgs a) {
  __shared__ uint32_t pre_all[4][kMaxSeg + 1];
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const int slot = blockIdx.x * 4 + wave;
  if (slot >= a.nslots) return;
  const uint32_t q = a.qlist ? a.qlist[slot] : uint32_t(slot);
  uint32_t* pre = pre_all[wave];

  if (a.ovf != nullptr && a.ovf[q]) {
    if (lane == 0) {
      uint32_t p = atomicAdd(a.fb_count, 1u);
      a.fb_list[p] = q;
    }
    return;
  }

  // prefix sum of segment counts
  uint32_t run = 0;
  const uint32_t* cnts = a.counts + size_t(slot) * a.nseg;
  for (int b = 0; b < a.nseg; b += kWave) {
    const int s = b + lane;
    uint32_t c = s < a.nseg ? cnts[s] : 0u;
    uint32_t incl = c;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      uint32_t t = __shfl_up(incl, o);
      if (lane >= o) incl += t;
    }
    if (s < a.nseg) pre[s + 1] = run + incl;
    run += __shfl(incl, kWave - 1);
  }
  if (lane == 0) pre[0] = 0;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  const uint32_t total = run;

  WaveTopK<E> top;
  top.init();
  const uint2* cbase = a.cand + size_t(slot) * a.nseg * size_t(a.cap);
  for (uint32_t g0 = 0; g0 < total; g0 += kWave) {
    const uint32_t g = g0 + lane;
    float d = __builtin_inff();
    uint32_t id = kNoId;
    if (g < total) {
      int lo = 0, hi = a.nseg;  // largest s with pre[s] <= g
      while (hi - lo > 1) {
        int mid = (lo + hi) >> 1;
        if (pre[mid] <= g) lo = mid; else hi = mid;
      }
      const uint2 c = cbase[size_t(lo) * a.cap + (g - pre[lo])];
      d = __uint_as_float(c.x);
      id = c.y;
    }
    top.insert(d, id);
  }

  constexpr int N = kWave * E;
  uint32_t* oi = a.out_ids + size_t(q) * a.k;
  float* od = a.out_d + size_t(q) * a.k;
  if (!a.rescore) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int gi = e * kWave + lane;
      if (gi < a.k) {
        oi[gi] = top.k.id[e];
        od[gi] = top.k.d[e];
      }
    }
    return;
  }

  // rescore the K' = N-1 best by GEMM value with exact distances
  const float* qv = a.Q + size_t(q) * a.pd;
  const uint32_t nsel = min(total, uint32_t(N - 1));
  float a_next = __shfl(top.k.d[E - 1], kWave - 1);  // (K'+1)-th GEMM value
  WaveKeys<E> r;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint32_t gi = e * kWave + lane;
    if (gi < nsel) {
      r.d[e] = metric_exact(a.metric, qv, a.X + size_t(top.k.id[e]) * a.pd, a.pd);
      r.id[e] = top.k.id[e];
    } else {
      r.d[e] = __builtin_inff();
      r.id[e] = kNoId;
    }
  }
  bitonic_sort<E>(r);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int gi = e * kWave + lane;
    if (gi < a.k) {
      oi[gi] = r.id[e];
      od[gi] = r.d[e];
    }
  }
  // certificate: every unselected candidate's exact distance is >= its GEMM value (+qn)
  // minus the bound; it must exceed the k-th exact distance.
  if (total > nsel && !a.exact[q]) {
    const int g = a.k - 1;
    float dk = __builtin_inff();
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float v = __shfl(r.d[e], g & (kWave - 1));
      if (e == g / kWave) dk = v;
    }
    const float lower = a.metric == 0 ? (a_next + a.qn[q]) - a.eb[q] : a_next - a.eb[q];
    if (!(dk < lower) && lane == 0) {
      uint32_t p = atomicAdd(a.fb_count, 1u);
      a.fb_list[p] = q;
    }
  }
}

// ================================================================ exact scan

struct ScanArgs {
  const float* X;
  const float* Q;
  const uint64_t* allow;
  int pd, metric;
  uint32_t N;
  const uint32_t* qlist;  // nullable
  int nslots;
  uint32_t split_rows;
  int nsplit;
  uint2* part;            // [slot][split][64*E]
  uint32_t* part_counts;  // [slot][split]
};

// Block = 4 waves on one (query, row split); each wave keeps a top-64E of its rows with
// exact distances, then wave 0 merges the other three through LDS.
template <int E>
__global__ __launch_bounds__(256) void k_exact_scan(ScanArgs a) {
  constexpr int N = kWave * E;
  __shared__ float md[3][N];
  __shared__ uint32_t mi[3][N];
  const int slot = blockIdx.x, split = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const uint32_t q = a.qlist ? a.qlist[slot] : uint32_t(slot);
  const float* qv = a.Q + size_t(q) * a.pd;
  const uint32_t r0 = uint32_t(split) * a.split_rows;
  const uint32_t r1 = min(a.N, r0 + a.split_rows);
  WaveTopK<E> top;
  top.init();
  for (uint32_t base = r0 + wave * kWave; base < r1; base += 4 * kWave) {
    const uint32_t r = base + lane;
    float d = __builtin_inff();
    uint32_t id = kNoId;
    if (r < r1 && row_allowed(a.allow, r)) {
      d = metric_exact(a.metric, qv, a.X + size_t(r) * a.pd, a.pd);
      id = r;
    }
    top.insert(d, id);
  }
  if (wave > 0) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      md[wave - 1][e * kWave + lane] = top.k.d[e];
      mi[wave - 1][e * kWave + lane] = top.k.id[e];
    }
  }
  __syncthreads();
  if (wave != 0) return;
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int e = 0; e < E; ++e) top.insert(md[w][e * kWave + lane], mi[w][e * kWave + lane]);
  const size_t ps = size_t(slot) * a.nsplit + split;
  uint2* out = a.part + ps * N;
  uint32_t valid = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    out[e * kWave + lane] = make_uint2(__float_as_uint(top.k.d[e]), top.k.id[e]);
    valid += __popcll(__ballot(top.k.id[e] != kNoId));
  }
  if (lane == 0) a.part_counts[ps] = valid;
}

// ================================================================ orchestration

__global__ void k_fill_empty(uint32_t* ids, float* d, size_t n) {
  size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i < n) {
    ids[i] = kNoId;
    d[i] = __builtin_inff();
  }
}

template <int E>
static void launch_select(hipStream_t s, const SelectArgs& a) {
  dim3 grid((a.nslots + 3) / 4);
  k_select<E><<<grid, 256, 0, s>>>(a);
}
template <int E>
static void launch_scan(hipStream_t s, const ScanArgs& a) {
  dim3 grid(a.nslots, a.nsplit);
  k_exact_scan<E><<<grid, 256, 0, s>>>(a);
}
template <int E>
static void launch_prepass(hipStream_t s, const PrepassArgs& a) {
  dim3 grid((a.nq + 3) / 4);
  k_prepass<E><<<grid, 256, 0, s>>>(a);
}

static int pow2_e(size_t n) {  // smallest E in {1,2,4,8} with 64*E >= n
  int e = 1;
  while (size_t(kWave) * e < n) e <<= 1;
  return e;
}

#define VDBG_DISPATCH_E(E, FN, ...)                       \
  switch (E) {                                            \
    case 1: FN<1>(__VA_ARGS__); break;                    \
    case 2: FN<2>(__VA_ARGS__); break;                    \
    case 4: FN<4>(__VA_ARGS__); break;                    \
    default: return SetError(kNotSupported, "k too large"); \
  }

// Exact top-k of the given slots (all queries, or a list) by brute force: row splits
// scanned with exact distances, then merged.
static int ExactScan(Ctx* c, Workspace& w, Dataset* ds, const float* Q,
                     const uint32_t* qlist, int nslots, size_t k, const uint64_t* allow,
                     uint32_t* out_ids, float* out_d, hipStream_t s) {
  if (nslots == 0) return kOk;
  const int E = pow2_e(k);
  if (E > 4) return SetError(kNotSupported, "k > 256 is not supported on the GPU path");
  const uint32_t N = static_cast<uint32_t>(ds->n);
  int nsplit = static_cast<int>(std::min<size_t>((2048 + nslots - 1) / nslots,
                                                 std::max<size_t>(1, (N + 1023) / 1024)));
  nsplit = std::max(1, std::min(nsplit, kMaxSeg));
  uint32_t split_rows = (N + nsplit - 1) / nsplit;
  split_rows = (split_rows + 63) / 64 * 64;
  nsplit = static_cast<int>((N + split_rows - 1) / split_rows);
  const int cap = kWave * E;
  size_t need = size_t(nslots) * nsplit * cap * sizeof(uint2) +
                size_t(nslots) * nsplit * sizeof(uint32_t) + 4096;
  w.used = 0;
  VDBG_RETURN_IF_ERROR(w.reserve(need));
  uint2* part = w.take<uint2>(size_t(nslots) * nsplit * cap);
  uint32_t* pc = w.take<uint32_t>(size_t(nslots) * nsplit);
  ScanArgs sa{ds->rows, Q, allow, int(ds->pd), ds->metric, N, qlist, nslots, split_rows, nsplit,
              part, pc};
  {
    ProfScope ps(c, "exact_scan", s);
    VDBG_DISPATCH_E(E, launch_scan, s, sa);
    VDBG_HIP(hipGetLastError());
  }
  SelectArgs se{};
  se.X = ds->rows;
  se.Q = Q;
  se.pd = int(ds->pd);
  se.metric = ds->metric;
  se.cand = part;
  se.counts = pc;
  se.nseg = nsplit;
  se.cap = cap;
  se.qlist = qlist;
  se.nslots = nslots;
  se.k = int(k);
  se.rescore = 0;
  se.out_ids = out_ids;
  se.out_d = out_d;
  {
    ProfScope ps(c, "merge", s);
    VDBG_DISPATCH_E(E, launch_select, s, se);
    VDBG_HIP(hipGetLastError());
  }
  return kOk;
}

static bool GemmSupported(size_t pd) { return pd % 16 == 0 && pd >= 16 && pd <= 128; }

template <int PD, int METRIC>
static void launch_gemm_pd(hipStream_t s, dim3 grid, const GemmArgs& a) {
  k_flat_gemm<PD, METRIC><<<grid, 256, 0, s>>>(a);
}

static int LaunchGemm(size_t pd, int metric, hipStream_t s, dim3 grid, const GemmArgs& a) {
#define VDBG_GEMM_CASE(P)                                   \
  case P:                                                   \
    if (metric == 0)                                        \
      launch_gemm_pd<P, 0>(s, grid, a);                     \
    else                                                    \
      launch_gemm_pd<P, 1>(s, grid, a);                     \
    break;
  switch (pd) {
    VDBG_GEMM_CASE(16)
    VDBG_GEMM_CASE(32)
    VDBG_GEMM_CASE(48)
    VDBG_GEMM_CASE(64)
    VDBG_GEMM_CASE(80)
    VDBG_GEMM_CASE(96)
    VDBG_GEMM_CASE(112)
    VDBG_GEMM_CASE(128)
    default:
      return SetError(kNotSupported, "GEMM path: unsupported padded_dim");
  }
#undef VDBG_GEMM_CASE
  return kOk;
}

int FlatSearch(Dataset* ds, const float* Q, size_t nq, size_t k, const uint64_t* allow,
               uint32_t* out_ids, float* out_d, hipStream_t s) {
  Ctx* c = ds->ctx;
  c->last_fallbacks = 0;
  if (nq == 0 || k == 0) return kOk;
  if (k > 256) return SetError(kNotSupported, "k > 256 is not supported on the GPU path");
  if (ds->n == 0) {
    k_fill_empty<<<dim3(unsigned((nq * k + 255) / 256)), 256, 0, s>>>(out_ids, out_d, nq * k);
    VDBG_HIP(hipGetLastError());
    return kOk;
  }
  const uint32_t N = static_cast<uint32_t>(ds->n);
  const size_t pd = ds->pd;
  const bool gemm = GemmSupported(pd) && N >= 4096 && nq >= 32;
  Workspace& w = c->ws;
  w.used = 0;
  if (!gemm) return ExactScan(c, c->ws, ds, Q, nullptr, int(nq), k, allow, out_ids, out_d, s);

  // ---- plan
  const int nqt = int((nq + 127) / 128);
  int nchunks = std::max(1, std::min({(2048 + nqt - 1) / nqt, int((N + 63) / 64), 256}));
  uint32_t chunk_rows = (N + nchunks - 1) / nchunks;
  chunk_rows = (chunk_rows + 63) / 64 * 64;
  nchunks = int((N + chunk_rows - 1) / chunk_rows);
  const uint64_t target_cands = 4096;
  uint32_t S = uint32_t(std::min<uint64_t>(
      N, std::max<uint64_t>(2048, (uint64_t(k) * N + target_cands - 1) / target_cands)));
  const double expect_seg = double(k) * N / S / (2.0 * nchunks);
  int caph = 32;
  while (caph < 3.0 * expect_seg + 32) caph <<= 1;
  const int nseg = 2 * nchunks;
  const int Ek = pow2_e(k);
  const int Esel = pow2_e(k + 16);
  if (Esel > 4) return SetError(kNotSupported, "k too large for the GEMM path");

  size_t need = nq * (4 * sizeof(float) + 2 * sizeof(int) + sizeof(uint32_t)) +
                size_t(nq) * nseg * (sizeof(uint32_t) + size_t(caph) * sizeof(uint2)) + 16 * 256;
  VDBG_RETURN_IF_ERROR(w.reserve(need));
  float* qn = w.take<float>(nq);
  float* eb = w.take<float>(nq);
  float* T = w.take<float>(nq);
  int* exact = w.take<int>(nq);
  int* ovf = w.take<int>(nq);
  uint32_t* fb_list = w.take<uint32_t>(nq);
  uint32_t* fb_count = w.take<uint32_t>(1);
  uint32_t* counts = w.take<uint32_t>(size_t(nq) * nseg);
  uint2* cand = w.take<uint2>(size_t(nq) * nseg * caph);
  VDBG_HIP(hipMemsetAsync(ovf, 0, nq * sizeof(int), s));
  VDBG_HIP(hipMemsetAsync(fb_count, 0, sizeof(uint32_t), s));

  PrepArgs pa{Q, int(nq), int(pd), ds->stats, qn, eb, exact};
  {
    ProfScope ps(c, "query_prep", s);
    k_query_prep<<<dim3(unsigned((nq + 3) / 4)), 256, 0, s>>>(pa);
    VDBG_HIP(hipGetLastError());
  }
  PrepassArgs pp{ds->rows, Q, allow, int(nq), int(pd), ds->metric, int(k), N, S, qn, eb, T};
  {
    ProfScope ps(c, "prepass", s);
    VDBG_DISPATCH_E(Ek, launch_prepass, s, pp);
    VDBG_HIP(hipGetLastError());
  }
  GemmArgs ga{ds->rows, ds->norms, Q, T, allow, cand, counts, ovf, N, int(nq), chunk_rows,
              nchunks, caph};
  {
    ProfScope ps(c, "flat_gemm", s);
    VDBG_RETURN_IF_ERROR(LaunchGemm(pd, ds->metric == 0 ? 0 : 1, s, dim3(nqt, nchunks), ga));
    VDBG_HIP(hipGetLastError());
  }
  SelectArgs se{};
  se.X = ds->rows;
  se.Q = Q;
  se.pd = int(pd);
  se.metric = ds->metric;
  se.cand = cand;
  se.counts = counts;
  se.nseg = nseg;
  se.cap = caph;
  se.ovf = ovf;
  se.qn = qn;
  se.eb = eb;
  se.exact = exact;
  se.nslots = int(nq);
  se.k = int(k);
  se.rescore = 1;
  se.out_ids = out_ids;
  se.out_d = out_d;
  se.fb_list = fb_list;
  se.fb_count = fb_count;
  {
    ProfScope ps(c, "select", s);
    VDBG_DISPATCH_E(Esel, launch_select, s, se);
    VDBG_HIP(hipGetLastError());
  }
  VDBG_HIP(hipMemcpyAsync(c->host_pinned, fb_count, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  VDBG_HIP(hipStreamSynchronize(s));
  const uint32_t nfb = c->host_pinned[0];
  c->last_fallbacks = nfb;
  if (nfb > 0)
    VDBG_RETURN_IF_ERROR(
        ExactScan(c, c->ws2, ds, Q, fb_list, int(nfb), k, allow, out_ids, out_d, s));
  return kOk;
}

}  // namespace vdbg
