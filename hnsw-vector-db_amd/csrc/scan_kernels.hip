// scan_kernels.hip -- exhaustive scans on gfx950: flat exact search and the SQ8 scan.
//
// vdb's FlatIndex scans every row with an AVX-512 distance kernel into a top-k heap
// (src/index/flat_index.cc:11-39, 73-77); its SQ8 path scores uint8 codes with the
// asymmetric SQ8 kernel into a top-R heap and re-ranks with float rows
// (src/index/hnsw/hnsw_index.cc:82-100, src/index/index.cc:89-95).  Both run here as one
// pipeline over a batch of queries:
//
//   k_query_prep   per query: the GEMM B operand, the shift between the GEMM value and the
//                  exact distance, and a bound on their difference (zero when integer data
//                  makes every partial sum exact).
//   k_gemm (MODE 1) on a strided sample of rows: per lane the minimum GEMM value of each
//                  16-row group.  k_kth turns the r-th smallest group minimum into an
//                  admission threshold: r = kk provably keeps the top kk; a smaller r
//                  (ThresholdRank) keeps them except with probability below 1e-6, and
//                  k_select's certificate checks that they were kept.
//   k_gemm (MODE 0) Q.X^T (or Q''.C^T over codes) on fp32 MFMA (v_mfma_f32_32x32x2f32),
//                  rows streamed through LDS; the epilogue compares with the threshold and
//                  appends the few passing rows to per-(query, chunk, half) buffers.
//   k_select       per query: the K' smallest candidates by GEMM value (wave bitonic
//                  top-k), exact re-scoring in the reference's AVX-512 order, sort by
//                  (dist, id), and a certificate that no unselected row can enter the top
//                  kk; failures and overflows are re-scanned exactly (k_exact_scan).
//   k_rerank       (SQ8) exact fp32 distances of the top-R codes' rows, top k.
//
// Distances returned are always the reference's exact AVX-512-order values.
#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>
#include <type_traits>

#include "gemm.h"
#include "vdbg_device.h"
#include "vdbg_internal.h"

namespace vdbg {

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

// ================================================================ integer rows on int8

// Integer rows held in int8 as x8 = x - c8, and an integer query y whose every partial sum
// of any order stays below 2^24 (so the reference's fp32 distance is the exact integer): the
// query goes to LDS as int8 y8 = y - c8, four dims a word, and each distance takes four dims
// per packed dot product:
//   L2:  sum (x - y)^2 = sum x8^2 - 2 sum x8 y8 + sum y8^2
//   IP:  sum x y = sum x8 y8 + c8 sum x8 + c8 sum y8 + pd c8^2    (the distance is -sum x y)
struct Int8Query {
  int on;                // the query qualifies
  int ysum;              // sum y8^2 (L2) or sum y8 (IP)
  const uint32_t* ys;    // [pd / 4] packed y8
};

// Wave-level: decides and packs (ys: pd / 4 words of the wave's LDS, pd <= 1024).  The query
// is read in rounds of 256 dims, each round's loads issued before any is used (a single
// round trip up to 256 dims, whose values the packing reuses): dim i is lane i % 64's value
// (i / 64) % 4 of round i / 256, written to byte i of ys.
__device__ Int8Query int8_query(const int8_t* X8, int c8, float xlo, float xhi, float xmax,
                                int xint, int metric, int pd, const float* qv, uint32_t* ys) {
  Int8Query r{0, 0, ys};
  if (X8 == nullptr || !xint || metric == 2 || pd % 16 != 0 || pd > 1024) return r;
  constexpr int kRound = 4 * kWave;
  const int lane = lane_id();
  float v[4];
  auto load = [&](int base) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = base + lane + j * kWave;
      v[j] = i < pd ? qv[i] : 0.f;
    }
  };
  float mq = 0.f, lo = __builtin_inff(), hi = -__builtin_inff();
  int ai = 1;
  for (int base = 0; base < pd; base += kRound) {
    load(base);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (base + lane + j * kWave < pd) {
        mq = fmaxf(mq, fabsf(v[j]));
        lo = fminf(lo, v[j]);
        hi = fmaxf(hi, v[j]);
        ai &= v[j] == rintf(v[j]) ? 1 : 0;
      }
    }
  }
  mq = wave_max(mq);
  lo = wave_min(lo);
  hi = wave_max(hi);
  ai = wave_and(ai);
  const double dpd = pd, lim = 16777216.0, mx = xmax, m = mq;
  const double range = double(fmaxf(hi, xhi)) - double(fminf(lo, xlo));
  if (!(ai && dpd * mx * mx < lim && dpd * m * m < lim && dpd * mx * m < lim &&
        dpd * range * range < lim && lo - float(c8) >= -128.f && hi - float(c8) <= 127.f))
    return r;
  int ysum = 0;
  int8_t* yb = reinterpret_cast<int8_t*>(ys);
  for (int base = 0; base < pd; base += kRound) {
    if (pd > kRound) load(base);  // one round: its values are still in v
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = base + lane + j * kWave;
      if (i < pd) {
        const int y8 = int(v[j]) - c8;
        ysum += metric == 0 ? y8 * y8 : y8;
        yb[i] = int8_t(y8);
      }
    }
  }
  for (int o = kWave / 2; o > 0; o >>= 1) ysum += __shfl_xor(ysum, o);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  r.on = 1;
  r.ysum = ysum;
  return r;
}

// The row's 16-byte vectors load G at a time, all G in flight together (G = 8 covers a
// 128-dim row in one round trip; kernels short of registers take fewer).
template <int G = 8>
__device__ __forceinline__ float int8_distance(const int8_t* X8, int c8, int metric, int pd,
                                               const Int8Query& p, uint32_t row) {
  const int4* xr = reinterpret_cast<const int4*>(X8 + size_t(row) * pd);
  const int4* yr = reinterpret_cast<const int4*>(p.ys);
  const int one = 0x01010101;
  const int nv = pd / 16;
  int xy = 0, xx = 0;
  for (int i0 = 0; i0 < nv; i0 += G) {
    int4 x[G];
#pragma unroll
    for (int j = 0; j < G; ++j) x[j] = i0 + j < nv ? xr[i0 + j] : make_int4(0, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if (i0 + j >= nv) break;
      const int4 y = yr[i0 + j];
      xy = __builtin_amdgcn_sdot4(x[j].x, y.x, xy, false);
      xy = __builtin_amdgcn_sdot4(x[j].y, y.y, xy, false);
      xy = __builtin_amdgcn_sdot4(x[j].z, y.z, xy, false);
      xy = __builtin_amdgcn_sdot4(x[j].w, y.w, xy, false);
      // L2: sum x8^2; IP: sum x8 (against bytes of ones)
      xx = __builtin_amdgcn_sdot4(x[j].x, metric == 0 ? x[j].x : one, xx, false);
      xx = __builtin_amdgcn_sdot4(x[j].y, metric == 0 ? x[j].y : one, xx, false);
      xx = __builtin_amdgcn_sdot4(x[j].z, metric == 0 ? x[j].z : one, xx, false);
      xx = __builtin_amdgcn_sdot4(x[j].w, metric == 0 ? x[j].w : one, xx, false);
    }
  }
  if (metric == 0) return float(xx - 2 * xy + p.ysum);
  return -float(xy + c8 * xx + c8 * p.ysum + pd * c8 * c8);  // -0 for a zero dot, as -dot
}

// int8_distance of R rows per 8-lane group: lane j of the group takes each row's 16-byte
// vectors j, j + 8, ... (128 contiguous bytes per group load, every row's loads in flight
// together), and the integer partial sums add up in any order.  Every lane of a group returns
// its rows' distances in d; all 64 lanes must be active.
template <int R>
__device__ __forceinline__ void int8_distance_g8n(const int8_t* X8, int c8, int metric, int pd,
                                                  const Int8Query& p, const uint32_t (&rows)[R],
                                                  float (&d)[R]) {
  const int j = lane_id() & 7;
  const int4* yr = reinterpret_cast<const int4*>(p.ys);
  const int one = 0x01010101;
  const int nv = pd / 16;
  int xy[R], xx[R];
#pragma unroll
  for (int r = 0; r < R; ++r) xy[r] = xx[r] = 0;
  for (int i = j; i < nv; i += 8) {
    int4 x[R];
#pragma unroll
    for (int r = 0; r < R; ++r) x[r] = reinterpret_cast<const int4*>(X8 + size_t(rows[r]) * pd)[i];
    const int4 y = yr[i];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      xy[r] = __builtin_amdgcn_sdot4(x[r].x, y.x, xy[r], false);
      xy[r] = __builtin_amdgcn_sdot4(x[r].y, y.y, xy[r], false);
      xy[r] = __builtin_amdgcn_sdot4(x[r].z, y.z, xy[r], false);
      xy[r] = __builtin_amdgcn_sdot4(x[r].w, y.w, xy[r], false);
      xx[r] = __builtin_amdgcn_sdot4(x[r].x, metric == 0 ? x[r].x : one, xx[r], false);
      xx[r] = __builtin_amdgcn_sdot4(x[r].y, metric == 0 ? x[r].y : one, xx[r], false);
      xx[r] = __builtin_amdgcn_sdot4(x[r].z, metric == 0 ? x[r].z : one, xx[r], false);
      xx[r] = __builtin_amdgcn_sdot4(x[r].w, metric == 0 ? x[r].w : one, xx[r], false);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    int s = xy[r], t = xx[r];
    s += int(lane_mirror8(uint32_t(s)));
    t += int(lane_mirror8(uint32_t(t)));
    s += int(lane_xor(uint32_t(s), 2));
    t += int(lane_xor(uint32_t(t), 2));
    s += int(lane_xor(uint32_t(s), 1));
    t += int(lane_xor(uint32_t(t), 1));
    d[r] = metric == 0 ? float(t - 2 * s + p.ysum)
                       : -float(s + c8 * t + c8 * p.ysum + pd * c8 * c8);
  }
}

// Scores the keys that lanes [b0, b1) of a 64-key pass hold (own: the lane's key id) eight
// lanes a key, two keys per group a round while more than 8 remain: score(ids, d) fills d[r]
// with the distance of row ids[r] for the lane's group (row 0 stands in where the group has no
// key), and each lane in [b0, b1) receives its own key's distance in out (+inf for kNoId).
// Wave-uniform b0, b1; all 64 lanes active.
template <class F>
__device__ __forceinline__ void group_pass(uint32_t own, int b0, int b1, float& out, F&& score) {
  const int lane = lane_id();
  auto key = [&](int m) {
    const uint32_t id = __shfl(own, m & (kWave - 1));
    return m < b1 && id != kNoId ? id : 0u;
  };
  auto take = [&](float d, int c0) {  // key c0 + g's distance sits in lane 8g
    const float got = __shfl(d, ((lane - c0) & 7) << 3);
    if (lane >= c0 && lane < c0 + 8 && lane < b1) out = own != kNoId ? got : __builtin_inff();
  };
  int c0 = b0;
  for (; c0 + 8 < b1; c0 += 16) {
    const uint32_t ids[2] = {key(c0 + (lane >> 3)), key(c0 + 8 + (lane >> 3))};
    float d[2];
    score(ids, d);
    take(d[0], c0);
    take(d[1], c0 + 8);
  }
  if (c0 < b1) {
    const uint32_t ids[1] = {key(c0 + (lane >> 3))};
    float d[1];
    score(ids, d);
    take(d[0], c0);
  }
}

// Order-preserving float <-> uint32 map for atomicMin/atomicMax.
__device__ __forceinline__ uint32_t ord_enc(float f) {
  uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float ord_dec_dev(uint32_t e) {
  return __uint_as_float((e & 0x80000000u) ? (e & 0x7fffffffu) : ~e);
}
static inline float ord_dec(uint32_t e) {
  uint32_t b = (e & 0x80000000u) ? (e & 0x7fffffffu) : ~e;
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}


__host__ __device__ __forceinline__ uint32_t bitrev(uint32_t v, int bits) {
  uint32_t r = 0;
  for (int i = 0; i < bits; ++i) r |= ((v >> i) & 1u) << (bits - 1 - i);
  return r;
}

static int pow2_e(size_t n) {  // smallest E in {1,2,4,8,...} with 64*E >= n
  int e = 1;
  while (size_t(kWave) * e < n) e <<= 1;
  return e;
}

// ================================================================ row statistics

struct RowStatsDev {
  uint32_t lo, hi, max_abs, xn_max;
  int all_int;
};

// Rows are spread over the waves of the grid: per row ||x||^2 (lane-strided fmaf, wave sum);
// min, max, max |x|, the largest norm and integrality are kept per wave, reduced per block
// in LDS and folded into the result with one set of atomics per block.
__global__ __launch_bounds__(256) void k_row_stats(const float* __restrict__ X, size_t n,
                                                   int pd, float* __restrict__ norms,
                                                   RowStatsDev* __restrict__ st) {
  __shared__ float red[4][4];
  __shared__ int red_i[4];
  const int wave = threadIdx.x >> 6;
  const size_t nwaves = size_t(gridDim.x) * 4;
  float lo = __builtin_inff(), hi = -__builtin_inff(), ma = 0.f, xn = 0.f;
  int ai = 1;
  for (size_t r = blockIdx.x * size_t(4) + wave; r < n; r += nwaves) {
    const float* x = X + r * size_t(pd);
    float s = 0.f;
    for (int i = lane_id(); i < pd; i += kWave) {
      const float e = x[i];
      s = fmaf(e, e, s);
      lo = fminf(lo, e);
      hi = fmaxf(hi, e);
      ma = fmaxf(ma, fabsf(e));
      ai &= (e == rintf(e)) ? 1 : 0;
    }
    s = wave_sum(s);
    if (lane_id() == 0) norms[r] = s;
    xn = fmaxf(xn, s);
  }
  lo = wave_min(lo);
  hi = wave_max(hi);
  ma = wave_max(ma);
  ai = wave_and(ai);
  if (lane_id() == 0) {
    red[wave][0] = lo;
    red[wave][1] = hi;
    red[wave][2] = ma;
    red[wave][3] = xn;
    red_i[wave] = ai;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) {
      lo = fminf(lo, red[w][0]);
      hi = fmaxf(hi, red[w][1]);
      ma = fmaxf(ma, red[w][2]);
      xn = fmaxf(xn, red[w][3]);
      ai &= red_i[w];
    }
    atomicMin(&st->lo, ord_enc(lo));
    atomicMax(&st->hi, ord_enc(hi));
    atomicMax(&st->max_abs, __float_as_uint(ma));
    atomicMax(&st->xn_max, __float_as_uint(xn));
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
    const size_t blocks = std::min<size_t>((n + 3) / 4, size_t(c->cu_count) * 8);
    k_row_stats<<<dim3(unsigned(blocks)), 256, 0, s>>>(rows, n, int(pd), norms, d);
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

// ================================================================ SQ8 train / encode

// Sq8Quantizer::train (src/index/quant/sq8.cc:9-26) keeps the first of equal values
// (std::min / std::max); the partial reductions carry the row index so that equal values
// (which can differ only in the sign of zero) resolve to the earliest row as well.
struct MinMax {
  float mn;
  uint32_t mn_row;
  float mx;
  uint32_t mx_row;
};

__device__ __forceinline__ void mm_take(MinMax& a, float v, uint32_t row) {
  if (v < a.mn || (v == a.mn && row < a.mn_row)) {
    a.mn = v;
    a.mn_row = row;
  }
  if (v > a.mx || (v == a.mx && row < a.mx_row)) {
    a.mx = v;
    a.mx_row = row;
  }
}

__device__ __forceinline__ void mm_merge(MinMax& a, const MinMax& b) {
  if (b.mn < a.mn || (b.mn == a.mn && b.mn_row < a.mn_row)) {
    a.mn = b.mn;
    a.mn_row = b.mn_row;
  }
  if (b.mx > a.mx || (b.mx == a.mx && b.mx_row < a.mx_row)) {
    a.mx = b.mx;
    a.mx_row = b.mx_row;
  }
}

// grid.x = row blocks.  Thread t covers dims t % pd, t % pd + 256, ... (pd > 256) and rows
// r0 + t / pd, stepping max(1, 256 / pd) rows: each row is read contiguously.
__global__ __launch_bounds__(256) void k_sq8_minmax(const float* __restrict__ X, uint32_t n,
                                                    int pd, uint32_t rows_per_block,
                                                    MinMax* __restrict__ part) {
  __shared__ MinMax red[256];
  const int lanes_per_row = pd < 256 ? pd : 256;
  const int rsteps = 256 / lanes_per_row;
  const int t = threadIdx.x;
  const int roff = t / lanes_per_row;
  const int d0 = t % lanes_per_row;
  const uint32_t r0 = blockIdx.x * rows_per_block;
  const uint32_t r1 = min(n, r0 + rows_per_block);
  // uniform trip count: every thread reaches every barrier
  for (int dbase = 0; dbase < pd; dbase += lanes_per_row) {
    const int d = dbase + d0;
    MinMax a{__builtin_inff(), 0xffffffffu, -__builtin_inff(), 0xffffffffu};
    if (roff < rsteps && d < pd)
      for (uint32_t r = r0 + roff; r < r1; r += rsteps) mm_take(a, X[size_t(r) * pd + d], r);
    red[t] = a;
    __syncthreads();
    if (roff == 0 && d < pd) {
      for (int o = 1; o < rsteps; ++o) mm_merge(a, red[t + o * lanes_per_row]);
      part[size_t(blockIdx.x) * pd + d] = a;
    }
    __syncthreads();
  }
}

// One thread per dimension: fold the block partials; scale = (max - min) / 255.f.
__global__ void k_sq8_finish(const MinMax* __restrict__ part, int nblocks, int dim, int pd,
                             float* __restrict__ vmin, float* __restrict__ scale) {
  const int d = blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= pd) return;
  if (d >= dim || nblocks == 0) {
    vmin[d] = 0.f;
    scale[d] = 0.f;
    return;
  }
  MinMax a{__builtin_inff(), 0xffffffffu, -__builtin_inff(), 0xffffffffu};
  for (int b = 0; b < nblocks; ++b) mm_merge(a, part[size_t(b) * pd + d]);
  vmin[d] = a.mn;
  scale[d] = (a.mx - a.mn) / 255.f;
}

// Sq8Quantizer::encode (sq8.cc:28-37), one wave per row: IEEE divide, rintf (round half to
// even = std::nearbyint in the default mode), clamp to [0, 255]; padding dims and
// scale <= 0 give 0.  Also ||c * scale||^2, the row norm of the GEMM form.  With X null the
// codes are given (an index file's) and only their norms are computed.
__global__ __launch_bounds__(256) void k_sq8_encode(const float* __restrict__ X, uint32_t n,
                                                    int dim, int pd,
                                                    const float* __restrict__ vmin,
                                                    const float* __restrict__ scale,
                                                    uint8_t* __restrict__ codes,
                                                    float* __restrict__ yn) {
  const uint32_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= n) return;
  const float* x = X == nullptr ? nullptr : X + size_t(r) * pd;
  uint8_t* c = codes + size_t(r) * pd;
  float s = 0.f;
  for (int i = lane_id(); i < pd; i += kWave) {
    uint8_t code = 0;
    if (X == nullptr) {
      code = c[i];  // codes read from an index file: only their norms are computed
    } else {
      if (i < dim && scale[i] > 0.f) {
        const float v = rintf((x[i] - vmin[i]) / scale[i]);
        const float cl = v < 0.f ? 0.f : (255.f < v ? 255.f : v);
        code = uint8_t(cl);
      }
      c[i] = code;
    }
    const float y = float(code) * scale[i];
    s = fmaf(y, y, s);
  }
  s = wave_sum(s);
  if (lane_id() == 0) yn[r] = s;
}

int Sq8Train(Ctx* c, const Dataset* ds, float* vmin_dev, float* scale_dev, hipStream_t s) {
  const uint32_t n = uint32_t(ds->n);
  const int pd = int(ds->pd), dim = int(ds->dim);
  const uint32_t rpb = 8192;
  const int nb = int((n + rpb - 1) / rpb);
  MinMax* part = nullptr;
  if (nb > 0) {
    VDBG_HIP(hipMallocAsync(reinterpret_cast<void**>(&part), sizeof(MinMax) * nb * pd, s));
    ProfScope ps(c, "sq8_minmax", s);
    k_sq8_minmax<<<dim3(nb), 256, 0, s>>>(ds->rows, n, pd, rpb, part);
    VDBG_HIP(hipGetLastError());
  }
  k_sq8_finish<<<dim3((pd + 127) / 128), 128, 0, s>>>(part, nb, dim, pd, vmin_dev, scale_dev);
  VDBG_HIP(hipGetLastError());
  if (part) VDBG_HIP(hipFreeAsync(part, s));
  return kOk;
}

int Sq8Encode(Ctx* c, const Dataset* ds, const float* vmin_dev, const float* scale_dev,
              uint8_t* codes, float* yn, hipStream_t s, bool codes_given) {
  const uint32_t n = uint32_t(ds->n);
  if (n == 0) return kOk;
  ProfScope ps(c, "sq8_encode", s);
  k_sq8_encode<<<dim3((n + 3) / 4), 256, 0, s>>>(codes_given ? nullptr : ds->rows, n,
                                                 int(ds->dim), int(ds->pd),
                                                 vmin_dev, scale_dev, codes, yn);
  VDBG_HIP(hipGetLastError());
  return kOk;
}

// ================================================================ sample matrix

// Sample position p holds row floor(bitrev(p) * N / Smax): every power-of-two prefix of the
// sample is an evenly strided subset of the rows.
__global__ void k_gather_sample(const float* __restrict__ X, const uint32_t* __restrict__ Xmap,
                                const uint16_t* __restrict__ X16,
                                int pd16, const uint8_t* __restrict__ C,
                                const int8_t* __restrict__ X8, int pd8,
                                const int* __restrict__ init8,
                                const float* __restrict__ rn, uint32_t N, int pd, int bits,
                                uint32_t smax,
                                float* __restrict__ SX, uint16_t* __restrict__ SX16,
                                uint8_t* __restrict__ SC, int8_t* __restrict__ SX8,
                                int* __restrict__ Sinit8, float* __restrict__ Srn,
                                uint32_t* __restrict__ Sid) {
  const uint32_t p = blockIdx.x;
  if (p >= smax) return;
  const uint32_t row = uint32_t((uint64_t(bitrev(p, bits)) * N) / smax);
  const size_t xrow = Xmap != nullptr ? Xmap[row] : row;
  for (int i = threadIdx.x; i < pd; i += blockDim.x) {
    if (X) SX[size_t(p) * pd + i] = X[xrow * pd + i];
    if (C) SC[size_t(p) * pd + i] = C[size_t(row) * pd + i];
  }
  for (int i = threadIdx.x; X8 != nullptr && i < pd8; i += blockDim.x)
    SX8[size_t(p) * pd8 + i] = X8[size_t(row) * pd8 + i];
  for (int i = threadIdx.x; X16 != nullptr && i < pd16; i += blockDim.x)
    SX16[size_t(p) * pd16 + i] = X16[size_t(row) * pd16 + i];
  if (threadIdx.x == 0) {
    Srn[p] = rn[row];
    Sid[p] = row;
    if (init8) Sinit8[p] = init8[row];
  }
}

uint32_t SampleRows(uint32_t N) {
  uint32_t smax = 1;
  while (smax * 2 <= std::min<uint32_t>(N, 65536u)) smax *= 2;
  return smax;
}

size_t SampleBytes(const ScanSource& src, uint32_t smax) {
  auto al = [](size_t b) { return (b + 255) & ~size_t(255); };
  const size_t pd = src.pd;
  // (a source reading its parent's rows through Xmap ranks on its fp16 copy: no fp32 sample)
  return al(src.kind == 0 && src.Xmap == nullptr ? size_t(smax) * pd * sizeof(float) : 0) +
         al(src.X16 != nullptr ? size_t(smax) * pd * src.x16_parts * sizeof(uint16_t) : 0) +
         al(src.kind == 1 ? size_t(smax) * pd : 0) + al(size_t(smax) * sizeof(float)) +
         al(size_t(smax) * sizeof(uint32_t)) +
         (src.X8 != nullptr ? al(size_t(smax) * pd * src.x8_parts) + al(size_t(smax) * sizeof(int))
                            : 0) + 256;
}

int GatherSample(Ctx* c, ScanSource* src, hipStream_t s, void* buf, uint32_t cap) {
  // (a power-of-two prefix of a larger sample holds the same rows in the same positions, so
  // a sample gathered only as large as its one scan uses is that scan's sample exactly)
  const uint32_t smax = std::min(SampleRows(src->N), std::max<uint32_t>(cap, 1));
  int bits = 0;
  while ((1u << bits) < smax) ++bits;
  const size_t pd = src->pd;
  char* p = reinterpret_cast<char*>((reinterpret_cast<uintptr_t>(buf) + 255) & ~uintptr_t(255));
  auto take = [&](size_t b) {
    char* r = b != 0 ? p : nullptr;
    p += (b + 255) & ~size_t(255);
    return r;
  };
  const bool fp32 = src->kind == 0 && src->Xmap == nullptr;
  src->SX = reinterpret_cast<float*>(take(fp32 ? size_t(smax) * pd * sizeof(float) : 0));
  src->SX16 = reinterpret_cast<uint16_t*>(
      take(src->X16 != nullptr ? size_t(smax) * pd * src->x16_parts * sizeof(uint16_t) : 0));
  src->SC = reinterpret_cast<uint8_t*>(take(src->kind == 1 ? size_t(smax) * pd : 0));
  src->Srn = reinterpret_cast<float*>(take(size_t(smax) * sizeof(float)));
  src->Sid = reinterpret_cast<uint32_t*>(take(size_t(smax) * sizeof(uint32_t)));
  src->SX8 = reinterpret_cast<int8_t*>(
      take(src->X8 != nullptr ? size_t(smax) * pd * src->x8_parts : 0));
  src->Sinit8 = reinterpret_cast<int*>(take(src->X8 != nullptr ? size_t(smax) * sizeof(int) : 0));
  k_gather_sample<<<dim3(smax), 128, 0, s>>>(fp32 ? src->X : nullptr, src->Xmap,
                                             src->X16, int(pd) * src->x16_parts,
                                             src->kind == 1 ? src->C : nullptr, src->X8,
                                             int(pd) * src->x8_parts, src->init8, src->rn,
                                             src->N, int(pd), bits, smax,
                                             src->SX, src->SX16, src->SC, src->SX8,
                                             src->Sinit8, src->Srn, src->Sid);
  VDBG_HIP(hipGetLastError());
  src->Smax = smax;
  src->SN = src->N;
  return kOk;
}

// A persistent source's sample: one allocation, kept until FreeSample.
int BuildSample(Ctx* c, ScanSource* src, hipStream_t s) {
  if (src->Smax != 0) return kOk;
  void* buf = nullptr;
  VDBG_HIP(hipMalloc(&buf, SampleBytes(*src, SampleRows(src->N))));
  const int rc = GatherSample(c, src, s, buf, ~0u);
  if (rc != kOk) {
    (void)hipFree(buf);
    return rc;
  }
  src->Sbuf = buf;
  return kOk;
}

// Frees a sample BuildSample allocated (a sample gathered into caller memory is only
// forgotten).
void FreeSample(ScanSource* src) {
  if (src->Sbuf != nullptr) (void)hipFree(src->Sbuf);
  src->Sbuf = nullptr;
  src->SX = nullptr;
  src->SX16 = nullptr;
  src->SX8 = nullptr;
  src->Sinit8 = nullptr;
  src->SC = nullptr;
  src->Srn = nullptr;
  src->Sid = nullptr;
  src->Smax = 0;
  src->SN = 0;
}

// ================================================================ query preparation

struct PrepArgs {
  const float* Q;
  float* Qb;  // GEMM B operand (SQ8 only; the flat scan uses Q itself)
  int nq, pd, kind, metric;
  RowStats xs;
  float rmag;
  const float* vmin;
  const float* scale;
  float* shift;  // exact distance ~= GEMM value + shift
  float* eb;     // bound on |GEMM value + shift - exact distance|
  int* exact;    // the bound is zero
  uint16_t* Q16;  // nullable: the fp16 GEMM's B operand (gemm16.hip)
  int* all16;     // nullable: cleared when a query is outside the fp16 GEMM's bounds
  float* Qf;      // split operands: per-query factor taking the split GEMM back to GEMM units
  int x16_parts;  // flat rows: 2 when they are held as scaled fp16 h + l pairs
  int x16_exp;    // their scale exponent (two parts, or the h halves alone: single16)
  int8_t* Q8;     // nullable: the int8 GEMM's B operand, q - c8 (gemm8.hip)
  int* Qd;        // its per-query constant M c8 sum(q) - c8^2 pd
  int* all8;      // cleared when a query is outside the int8 GEMM's bounds
  int* fit8q;     // nullable: per query, 1 when it is inside the int8 GEMM's bounds
  int c8;
  uint32_t* mb8;  // nullable: SQ8 on the int8 GEMM, the batch's max |B| (float bits, atomicMax)
  int single16;   // float rows held as their scaled h halves alone (gemm16.hip SPLIT 3)
};

// One wave per query.
//  flat L2:  GEMM value ||x||^2 - 2 q.x, shift ||q||^2.   flat IP: -q.x, shift 0.
//  SQ8 L2:   B = (q - vmin) * scale, value ||c*scale||^2 - 2 c.B, shift ||q - vmin||^2.
//  SQ8 IP:   B = q * scale, value -c.B, shift -q.vmin.
// The flat GEMM form is exact when every value is an integer and every partial sum any
// summation order can form stays below 2^24: pd*max|x|^2, pd*max|q|^2, pd*max|x|*max|q|
// and pd*R^2 with R the value range.  Otherwise the bound is
// (4*pd + 16) * 2^-24 * (query magnitude + row magnitude): the MFMA dot and the fp32 norms
// carry at most pd roundings each on sums bounded by those magnitudes, the exact
// AVX-512-order value at most pd/16 + 6, and the factor two covers forming thresholds and
// the SQ8 decode roundings.
// Returns the query's contribution to the batch maximum *a.mb8 (float bits, 0 without one);
// the caller folds it in.
__device__ uint32_t query_prep_wave(const PrepArgs& a, int q) {
  uint32_t mbq = 0;
  const float* v = a.Q + size_t(q) * a.pd;
  float s = 0.f, s2 = 0.f, lo = __builtin_inff(), hi = -__builtin_inff(), ma = 0.f;
  float sq = 0.f;  // sum(q) (exact: integers of magnitude < 2^24 when the int8 GEMM applies)
  int ai = 1, in8 = 1;
  for (int i = lane_id(); i < a.pd; i += kWave) {
    const float e = v[i];
    s = fmaf(e, e, s);
    lo = fminf(lo, e);
    hi = fmaxf(hi, e);
    ma = fmaxf(ma, fabsf(e));
    ai &= (e == rintf(e)) ? 1 : 0;
    if (a.Q8 != nullptr) {  // q - c8, in range when the batch takes the int8 GEMM
      const float d = e - float(a.c8);
      in8 &= (d >= -128.f && d <= 127.f) ? 1 : 0;
      a.Q8[size_t(q) * a.pd + i] = int8_t(int(fminf(fmaxf(d, -128.f), 127.f)));
      sq += e;
    }
    if (a.Q16 != nullptr && a.kind == 0 && a.x16_parts == 1 && !a.single16)  // -2 q or -q
      a.Q16[size_t(q) * a.pd + i] =
          __builtin_bit_cast(uint16_t, _Float16(a.metric == 0 ? -2.f * e : -e));
    if (a.kind == 1) {
      if (a.metric == 0) {
        const float qp = e - a.vmin[i];
        a.Qb[size_t(q) * a.pd + i] = qp * a.scale[i];
        s2 = fmaf(qp, qp, s2);
      } else {
        a.Qb[size_t(q) * a.pd + i] = e * a.scale[i];
        s2 = fmaf(e, a.vmin[i], s2);
      }
    }
  }
  s = wave_sum(s);
  s2 = wave_sum(s2);
  // float rows on the int8 GEMM: the batch is scaled by its largest ||q||
  if (a.kind == 0 && a.mb8 != nullptr) mbq = __float_as_uint(sqrtf(s) * (1.f + 1e-6f));
  lo = wave_min(lo);
  hi = wave_max(hi);
  ma = wave_max(ma);
  ai = wave_and(ai);
  if (a.Q8 != nullptr) {
    sq = wave_sum(sq);
    in8 = wave_and(in8);
  }
  // SQ8 on the fp16 GEMM: B scaled by 2^sc (max |B| 2^sc in [2^14, 2^15)) and split into
  // fp16 h + l, |B 2^sc - h - l| <= 2^-22 |B 2^sc| (+ subnormal terms); codes are exact in
  // fp16, so the GEMM runs as c.h + c.l and Qf = -2 (L2) or -1 (IP) times 2^-sc takes it back
  int sc = 0;
  bool split_ok = true;
  if (a.kind == 0 && (a.x16_parts == 2 || a.single16) && a.Q16 != nullptr) {
    // float rows held as h + l (or h alone): q 2^sc split the same way (max |q| 2^sc in
    // [2^14, 2^15))
    split_ok = ma <= 3.0e38f;
    if (split_ok && ma > 0.f) {
      int ex = 0;
      (void)frexpf(ma, &ex);
      sc = 15 - ex;
    }
    uint16_t* hq = a.Q16 + size_t(q) * 2 * a.pd;
    for (int i = lane_id(); i < a.pd; i += kWave) {
      const float vs = ldexpf(v[i], sc);
      const _Float16 hh = _Float16(vs);
      const _Float16 ll = _Float16(vs - float(hh));
      hq[i] = __builtin_bit_cast(uint16_t, hh);
      hq[a.pd + i] = __builtin_bit_cast(uint16_t, ll);
    }
  } else if (a.kind == 1 && a.Q16 != nullptr) {
    float mb = 0.f;
    for (int i = lane_id(); i < a.pd; i += kWave) mb = fmaxf(mb, fabsf(a.Qb[size_t(q) * a.pd + i]));
    mb = wave_max(mb);
    // non-negative floats order as their bits; a NaN ends above +inf and stops the int8 GEMM
    if (a.mb8 != nullptr) mbq = max(mbq, __float_as_uint(mb));
    split_ok = mb <= 3.0e38f;  // finite
    if (split_ok && mb > 0.f) {
      int ex = 0;
      (void)frexpf(mb, &ex);  // mb = f 2^ex, f in [0.5, 1)
      sc = 15 - ex;
    }
    uint16_t* hq = a.Q16 + size_t(q) * 2 * a.pd;
    for (int i = lane_id(); i < a.pd; i += kWave) {
      const float bs = ldexpf(a.Qb[size_t(q) * a.pd + i], sc);
      const _Float16 hh = _Float16(bs);
      const _Float16 ll = _Float16(bs - float(hh));
      hq[i] = __builtin_bit_cast(uint16_t, hh);
      hq[a.pd + i] = __builtin_bit_cast(uint16_t, ll);
    }
  }
  if (lane_id() == 0) {
    const double pd = a.pd, lim = 16777216.0;
    bool ex = false;
    float shift, qmag;
    if (a.kind == 0) {
      const double mx = a.xs.max_abs, mq = ma;
      const double range = double(fmaxf(hi, a.xs.hi)) - double(fminf(lo, a.xs.lo));
      ex = a.xs.all_int && ai && pd * mx * mx < lim && pd * mq * mq < lim &&
           pd * mx * mq < lim && pd * range * range < lim;
      shift = a.metric == 0 ? s : 0.f;
      qmag = s;
    } else {
      shift = a.metric == 0 ? s2 : -s2;
      qmag = a.metric == 0 ? s + s2 : s;
    }
    a.shift[q] = shift;
    bool half_norm = false;  // L2 on the int8 GEMM: values up to 1 above the GEMM value
    // fp16 holds every integer of magnitude <= 2048 exactly (and -2 q, an even integer of
    // magnitude <= 4096); the fp16 GEMM accumulates ||x||^2 - 2 q.x (or -q.x) from the row
    // norm, every partial sum bounded by (|q| + R)^2 with R the largest row norm.  Below 2^24
    // its values are the fp32 GEMM's bit for bit.
    if (a.Qf != nullptr && (a.kind == 1 || a.x16_parts == 2 || a.single16)) {
      a.Qf[q] = ldexpf(a.metric == 0 ? -2.f : -1.f, -sc - (a.kind == 0 ? a.x16_exp : 0));
      if (!split_ok) atomicAnd(a.all16, 0);
    } else if (a.all16 != nullptr || a.fit8q != nullptr) {
      const double rq = sqrt(double(s)), rx = sqrt(double(a.xs.xn_max));
      const bool fits = ex && ma <= 2048.f && a.xs.max_abs <= 2048.f &&
                        (rq + rx) * (rq + rx) * 1.001 < lim;
      if (!fits && a.all16 != nullptr) atomicAnd(a.all16, 0);
      if (a.Q8 != nullptr) {
        // the int8 GEMM: the same bounds, every q - c8 an int8, and its constant in int32
        const double c = a.c8;
        const double d = (a.metric == 0 ? 2.0 : 1.0) * c * double(sq) - c * c * pd;
        const bool fits8 = fits && in8 && fabs(d) < 268435456.0;
        a.Qd[q] = fits8 ? int(d) : 0;
        if (!fits8 && a.all8 != nullptr) atomicAnd(a.all8, 0);
        if (a.fit8q != nullptr) a.fit8q[q] = fits8 ? 1 : 0;
        // L2 values on the int8 GEMM may exceed the GEMM value by 1 (the rounded half
        // norm): such a query carries that bound whichever GEMM the batch takes
        half_norm = fits8 && a.metric == 0;
      }
    }
    // Rounding bound of |GEMM value + shift - exact distance|.  Any fp32 summation order of
    // n products errs by at most ~n u sum|q_i x_i| (u = 2^-24), and sum|q_i x_i| <= |q||x|.
    // Inner product of fp32 rows: the MFMA dot and the exact dot each err by that, so
    // (2 pd + 16) u |q||x|.  Otherwise (L2 form, or SQ8 codes) the row norm, the shift and
    // the exact distance add their own terms: (4 pd + 16) u (|q|^2 + |x|^2).
    const double u = 1.0 / 16777216.0;
    const double bound =
        (a.kind == 0 && a.metric != 0)
            ? (2.0 * pd + 16.0) * u * sqrt(double(qmag) * double(a.rmag))
            : (4.0 * pd + 16.0) * u * (double(qmag) + double(a.rmag));
    // SQ8 on the split fp16 GEMM: the two fp32 accumulations, their sum, the split residual
    // (2^-22 relative) and the fma add at most (2 pd + 12) u sum c|B| <= (pd + 6) u (|q|^2 +
    // |x|^2); the bound below triples it, and adds 1020 pd 2^-14 2^-sc for fp16 values
    // below the normal range (each of h, l off by at most 2^-14 2^-sc, times c <= 255 and 2)
    const double bound16 = (6.0 * pd + 48.0) * u * (double(qmag) + double(a.rmag)) +
                           1020.0 * pd * ldexp(1.0, -14 - sc);
    // Float rows on the split fp16 GEMM (x_h q_h + x_h q_l + x_l q_h): per product the
    // parts miss at most 3 x 2^-22 relative (the dropped x_l q_l and the two split
    // residuals), the fp32 accumulations of 3 pd exact products (and their sum and fma) add
    // (3 pd + 4) u sum|q_i x_i|; doubled for margin, plus fp16 values below the normal range
    // (each part of x off by at most 2^-14 2^-x16_exp, of q by 2^-14 2^-sc).
    const double fsub = 4.0 * pd * ldexp(1.0, -14) *
                        (ldexp(double(ma), -a.x16_exp) + ldexp(double(a.xs.max_abs), -sc));
    const double bound16f =
        a.metric != 0 ? (2.0 * pd + 16.0 + 6.0 * pd + 48.0) * u * sqrt(double(qmag) * double(a.rmag)) + fsub
                      : (4.0 * pd + 16.0 + 6.0 * pd + 48.0) * u * (double(qmag) + double(a.rmag)) +
                            2.0 * fsub;
    // Float rows on the h halves alone (x_h q_h): the dropped x_h q_l + x_l q_h + x_l q_l is
    // at most (2^-10 + 2^-22) |x_i q_i| per product (each h within 2^-11 of its value), so
    // (2^-10 + 2^-21) |q||x| on the dot, twice that on the L2 form's 2 q.x.
    const double drop = ldexp(1.0, -10) + ldexp(1.0, -21);
    const double bound16h =
        bound16f + (a.metric != 0 ? drop * sqrt(double(qmag) * double(a.rmag))
                                  : drop * (double(qmag) + double(a.rmag)));
    const bool split = a.Q16 != nullptr && (a.kind == 1 || a.x16_parts == 2 || a.single16);
    const double bsplit = a.kind == 1 ? bound16 : (a.single16 ? bound16h : bound16f);
    a.exact[q] = ex && !half_norm ? 1 : 0;
    a.eb[q] = half_norm ? 1.f : ex ? 0.f : float((split ? bsplit : bound) * 1.001);
  }
  return mbq;
}

// Four queries per block; the batch maximum takes one atomic per block (one per query would
// serialise thousands of atomics on one word).
__global__ __launch_bounds__(256) void k_query_prep(PrepArgs a) {
  __shared__ uint32_t s_mb[4];
  const int wave = threadIdx.x >> 6;
  const int q = blockIdx.x * 4 + wave;
  const uint32_t mbq = q < a.nq ? query_prep_wave(a, q) : 0u;
  if (a.mb8 == nullptr) return;
  if (lane_id() == 0) s_mb[wave] = mbq;
  __syncthreads();
  if (threadIdx.x == 0)
    atomicMax(a.mb8, max(max(s_mb[0], s_mb[1]), max(s_mb[2], s_mb[3])));
}

// The scan's per-call words in one launch: overflow flags, fallback counts, the batch's GEMM
// eligibility flags, the all-ones filter word and the int8 operand exponent words.
struct ScanInit {
  int* ovf;              // [nq] 0
  int nq;
  uint32_t* fb_count;    // [2] 0
  int* all16;            // nullable, [2] 1
  uint32_t* ones;        // nullable, [1] all ones
  int* e8;               // nullable, [2] 0
  uint32_t* fb_zero;     // nullable: the context's count of device-gated re-scans, 0
};
__global__ void k_scan_init(ScanInit a) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < a.nq) a.ovf[i] = 0;
  if (i == 0 && a.fb_zero != nullptr) *a.fb_zero = 0;
  if (i < 2) {
    a.fb_count[i] = 0;
    if (a.all16 != nullptr) a.all16[i] = 1;
    if (a.e8 != nullptr) a.e8[i] = 0;
  }
  if (i == 0 && a.ones != nullptr) a.ones[0] = 0xffffffffu;
}

// SQ8 on the int8 GEMM (gemm8.hip, SQ = 1): the B operand of every query of the batch scaled
// by one 2^e, with 2^L <= 2^20 / pd (L <= 14) the bound on |B 2^e|, and rounded to integers
// v = 256 hi + lo (hi, lo int8).  So |sum c' v| < 2^27 for codes c' = c - 128, and the L2 row
// start rint(||c scale||^2 2^(e-1)) must stay below 2^27 too, or the batch takes the fp16 GEMM.
// The value (-M (sum c' v - start) - M 128 sum v) 2^-e misses the fp32 GEMM value by at most
// 2^-e (M 255 sum|B_i 2^e - v_i| + [L2] 1): that term is added to the query's bound (eb8).
//
// Float rows (fr = 1, gemm8.hip SQ = 2): B = q itself scaled by 2^eq (||v|| <= 2^13.9 for the
// batch's largest ||q||, mb8), the rows already held as v_x = rint(x 2^ex); e = ex + eq.
// Every (row, query) must keep |sum v_x v_q| + row start below 2^29 (checked with the rows'
// largest ||v_x||), and the value misses the fp32 GEMM value by at most
// M 2^-e (sum|v_x| / 2 + sum|v_q| / 2 + pd / 4) (+ 2^-e for the L2 row start).
struct Sq8Op8Args {
  const float* Qb;
  int nq, pd, metric;
  const uint32_t* mb8;
  float rn_max;       // max ||code * scale||^2 (SQ8) or ||x||^2 (float rows) over the rows
  const float* eb;    // the fp32-side bound of k_query_prep
  int8_t* Q8;         // [q][2][pd]: hi, lo
  int* Qd;            // M 128 sum(v) (SQ8), 0 (float rows)
  float* eb8;
  int* e8;
  int* all8;
  int fr;             // float rows
  int ex;             // their scale exponent
  float l1max, l2max; // their largest sum |v_x| and ||v_x||
};

__global__ __launch_bounds__(256) void k_sq8_operand8(Sq8Op8Args a) {
  const int q = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= a.nq) return;
  const float mb = __uint_as_float(*a.mb8);
  int L = 14;
  if (!a.fr) {
    L = 0;
    while (L < 14 && (int64_t(2) << L) * a.pd <= (int64_t(1) << 20)) ++L;
  }
  int e = 0;
  bool ok = mb <= 3.0e38f;
  if (ok && mb > 0.f) {
    if (a.fr) {
      e = int(floor(13.9 - log2(double(mb))));  // ||q 2^e|| <= 2^13.9
    } else {
      int ex = 0;
      (void)frexpf(mb, &ex);  // mb <= 2^ex
      e = L - ex;
    }
  }
  const int et = a.fr ? e + a.ex : e;  // the exponent of the values
  const double start_lim = a.fr ? 536870912.0 : 134217728.0;  // 2^29 or 2^27
  const double start = a.metric == 0 ? ldexp(double(a.rn_max), et - 1) : 0.0;
  if (!(start < start_lim)) ok = false;
  const float* b = a.Qb + size_t(q) * a.pd;
  int8_t* o = a.Q8 + size_t(q) * 2 * a.pd;
  int sv = 0, sa = 0;
  float sd = 0.f, s2 = 0.f;
  for (int i = lane_id(); i < a.pd; i += kWave) {
    const float x = ok ? ldexpf(b[i], e) : 0.f;  // |x| <= 2^L
    const float v = rintf(x);
    const int vi = int(v);
    const int hi = (vi + 128) >> 8;
    o[i] = int8_t(hi);
    o[a.pd + i] = int8_t(vi - 256 * hi);
    sv += vi;
    sa += vi < 0 ? -vi : vi;
    s2 = fmaf(v, v, s2);
    sd += fabsf(x - v);  // exact: x and its nearest integer share the exponent range
  }
  for (int off = kWave / 2; off > 0; off >>= 1) {
    sv += __shfl_xor(sv, off);
    sa += __shfl_xor(sa, off);
  }
  sd = wave_sum(sd);
  s2 = wave_sum(s2);
  if (lane_id() == 0) {
    const int M = a.metric == 0 ? 2 : 1;
    double quant;
    if (a.fr) {
      // |sum v_x v_q| <= ||v_x|| ||v_q||: with the row start it must stay below 2^29
      if (!(double(a.l2max) * sqrt(double(s2) * (1.0 + 1e-6 * a.pd)) + start <
            536870912.0 * (1.0 - 1e-3)))
        atomicAnd(a.all8, 0);
      a.Qd[q] = 0;
      quant = ldexp(M * (0.5 * double(a.l1max) + 0.5 * double(sa) + 0.25 * a.pd) +
                        (a.metric == 0 ? 1.0 : 0.0), -et);
    } else {
      a.Qd[q] = M * 128 * sv;
      quant = ldexp(M * 255.0 * double(sd) * (1.0 + 1e-6 * a.pd) + (a.metric == 0 ? 1.0 : 0.0),
                    -e);
    }
    a.eb8[q] = float((double(a.eb[q]) + quant) * 1.001);
    if (q == 0) *a.e8 = et;
    if (!ok) atomicAnd(a.all8, 0);
  }
}

// ================================================================ MFMA GEMM

// Block = 4 waves = 128 queries (32 per wave) x one chunk of rows.  Blocks are dispatched
// round-robin over the 8 XCDs, so block b takes work item (b % 8) * per_xcd + b / 8: the
// items of one XCD are consecutive and share row chunks in that XCD's L2.
//
// Each wave keeps its 32 queries in VGPRs as the MFMA B operand: for a K chunk of KC dims,
// lane l holds query l % 32, dims [h*KC/2, (h+1)*KC/2) of the chunk with h = l / 32, so MFMA
// step t contracts dims t and KC/2 + t (the order is irrelevant: the GEMM value only ranks;
// exact distances are recomputed).  Rows wider than 128 dims are streamed as (tile, chunk)
// stages and the query fragment is reloaded per chunk.  Stages are double-buffered in LDS
// and feed the A operand; code rows are widened to fp32 on the way in.  The 32x32
// accumulator gives lane l the values of query l % 32 for rows 8*(r/4) + 4*h + (r%4).
// The epilogue of tile t reads that tile's row norms after the tile's last barrier, while
// faster waves already stage tile t + 1 (norms of tile t + 2 are written only after the
// barrier that follows), so the norms rotate through three slots.
template <int PD, int METRIC, int KIND, int MODE>
__global__ __launch_bounds__(256, 2) void k_gemm(GemmArgs a) {
  constexpr int KC = GemmKc(PD);
  constexpr int NKC = PD / KC;
  constexpr int STR = KC + 4;  // padded LDS row stride (floats)
  constexpr int HALF = KC / 2;
  constexpr int VEC_PER_ROW = KIND == 0 ? KC / 4 : KC / 16;
  constexpr int VEC_PER_TILE = kGemmRows * VEC_PER_ROW;
  constexpr int VEC_PER_THREAD = (VEC_PER_TILE + 255) / 256;
  static_assert(PD % KC == 0 && KC % 16 == 0, "K chunking");
  __shared__ __attribute__((aligned(16))) float xs[2][kGemmRows * STR];
  __shared__ float xns[3][kGemmRows];
  if (gemm_gated_off(a)) return;

  const int b = blockIdx.x;
  const int item = (b & 7) * a.per_xcd + (b >> 3);
  if (item >= a.items) return;
  const int chunk = item / a.nqt;
  const int qt = item - chunk * a.nqt;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int j = lane & 31;
  const int h = lane >> 5;
  const int q = qt * 128 + wave * 32 + j;
  const bool wave_live = qt * 128 + wave * 32 < a.nq;
  const uint32_t r_begin = uint32_t(chunk) * a.chunk_rows;
  const uint32_t r_end = min(a.N, r_begin + a.chunk_rows);

  float qv[HALF];
  auto load_q = [&](int kc) {
    if (q < a.nq) {
      const float* src = a.Qb + size_t(q) * PD + kc * KC + h * HALF;
#pragma unroll
      for (int t = 0; t < HALF; t += 4) {
        const float4 v = *reinterpret_cast<const float4*>(src + t);
        qv[t] = v.x;
        qv[t + 1] = v.y;
        qv[t + 2] = v.z;
        qv[t + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int t = 0; t < HALF; ++t) qv[t] = 0.f;
    }
  };
  if (NKC == 1) load_q(0);
  const float T = (MODE == 0 && q < a.nq) ? a.T[q] : -__builtin_inff();
  const size_t seg = (size_t(q) * a.nchunks + chunk) * 2 + h;
  uint2* out = MODE == 0 ? a.cand + seg * size_t(a.caph) : nullptr;
  uint32_t cnt = 0;

  uint4 pre[VEC_PER_THREAD];
  float pre_n = 0.f;
  // stage (base, kc): rows base..base+63, dims kc*KC..kc*KC+KC-1
  auto load_stage = [&](uint32_t base, int kc) {
    const uint32_t valid = r_end > base ? min(uint32_t(kGemmRows), r_end - base) : 0u;
    if constexpr (VEC_PER_TILE % 256 == 0) {
      if (valid == kGemmRows) {  // a full tile: no per-vector bounds tests
#pragma unroll
        for (int i = 0; i < VEC_PER_THREAD; ++i) {
          const int f = tid + 256 * i;
          const int row = f / VEC_PER_ROW, c = f % VEC_PER_ROW;
          if (KIND == 0)
            pre[i] = *reinterpret_cast<const uint4*>(a.X + size_t(base + row) * PD + kc * KC + c * 4);
          else
            pre[i] = *reinterpret_cast<const uint4*>(a.C + size_t(base + row) * PD + kc * KC + c * 16);
        }
        if (kc == 0) pre_n = tid < kGemmRows ? a.rn[base + tid] : 0.f;
        return;
      }
    }
#pragma unroll
    for (int i = 0; i < VEC_PER_THREAD; ++i) {
      const int f = tid + 256 * i;
      const int row = f / VEC_PER_ROW, c = f % VEC_PER_ROW;
      if (f < VEC_PER_TILE && uint32_t(row) < valid) {
        if (KIND == 0)
          pre[i] = *reinterpret_cast<const uint4*>(a.X + size_t(base + row) * PD + kc * KC + c * 4);
        else
          pre[i] = *reinterpret_cast<const uint4*>(a.C + size_t(base + row) * PD + kc * KC + c * 16);
      } else {
        pre[i] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
    if (kc == 0) pre_n = (tid < kGemmRows && uint32_t(tid) < valid) ? a.rn[base + tid] : 0.f;
  };
  auto store_stage = [&](int buf, int kc, int nslot) {
#pragma unroll
    for (int i = 0; i < VEC_PER_THREAD; ++i) {
      const int f = tid + 256 * i;
      if (f < VEC_PER_TILE) {
        const int row = f / VEC_PER_ROW, c = f % VEC_PER_ROW;
        if (KIND == 0) {
          *reinterpret_cast<uint4*>(&xs[buf][row * STR + c * 4]) = pre[i];
        } else {
          float* dst = &xs[buf][row * STR + c * 16];
          const uint32_t w[4] = {pre[i].x, pre[i].y, pre[i].z, pre[i].w};
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            float4 v;
            v.x = float(w[g] & 0xffu);
            v.y = float((w[g] >> 8) & 0xffu);
            v.z = float((w[g] >> 16) & 0xffu);
            v.w = float(w[g] >> 24);
            *reinterpret_cast<float4*>(dst + 4 * g) = v;
          }
        }
      }
    }
    if (kc == 0 && tid < kGemmRows) xns[nslot][tid] = pre_n;
  };

  if (r_begin < r_end) {
    load_stage(r_begin, 0);
    store_stage(0, 0, 0);
  }
  __syncthreads();

  int buf = 0;
  int slot = 0;  // norm slot of the current tile
  for (uint32_t base = r_begin; base < r_end; base += kGemmRows) {
    v16f acc0, acc1;
    const v16f zero = {};
    if constexpr (NKC > 1) {
      acc0 = zero;
      acc1 = zero;
    }
#pragma unroll 1
    for (int kc = 0; kc < NKC; ++kc) {
      // prefetch the next stage: the next K chunk of this tile, or chunk 0 of the next tile
      const bool last_kc = kc + 1 == NKC;
      const uint32_t nbase = last_kc ? base + kGemmRows : base;
      const int nkc = last_kc ? 0 : kc + 1;
      const bool have_next = nbase < r_end;
      if (have_next) load_stage(nbase, nkc);
      if (NKC > 1 && wave_live) load_q(kc);

      if (wave_live) {
        const float* xa0 = &xs[buf][j * STR + h * HALF];
        const float* xa1 = xa0 + 32 * STR;
#pragma unroll
        for (int t = 0; t < HALF; t += 4) {
          const float4 x0 = *reinterpret_cast<const float4*>(xa0 + t);
          const float4 x1 = *reinterpret_cast<const float4*>(xa1 + t);
          // a single K chunk starts each tile from a zero accumulator operand
          const bool first = NKC == 1 && t == 0;
          acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.x, qv[t + 0], first ? zero : acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.x, qv[t + 0], first ? zero : acc1, 0, 0, 0);
          acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.y, qv[t + 1], acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.y, qv[t + 1], acc1, 0, 0, 0);
          acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.z, qv[t + 2], acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.z, qv[t + 2], acc1, 0, 0, 0);
          acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.w, qv[t + 3], acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.w, qv[t + 3], acc1, 0, 0, 0);
        }
      }

      if (have_next) store_stage(buf ^ 1, nkc, last_kc ? (slot == 2 ? 0 : slot + 1) : slot);
      __syncthreads();
      buf ^= 1;
    }
    if (wave_live && MODE == 0) {
      // threshold test on all 32 values; the rare passes go to the lane's buffer
      uint32_t pass = 0;
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rl = blk * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          const float g = blk == 0 ? acc0[r] : acc1[r];
          const float v = METRIC == 0 ? fmaf(-2.f, g, xns[slot][rl]) : -g;
          pass |= (v <= T ? 1u : 0u) << (blk * 16 + r);
        }
      if (__ballot(pass != 0) != 0) {
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            if (pass & (1u << (blk * 16 + r))) {
              const int rl = blk * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
              const float g = blk == 0 ? acc0[r] : acc1[r];
              const float v = METRIC == 0 ? fmaf(-2.f, g, xns[slot][rl]) : -g;
              const uint32_t row = base + rl;
              if (q < a.nq && row < r_end && row_allowed(a.allow, row)) {
                if (cnt < uint32_t(a.caph)) out[cnt] = make_uint2(__float_as_uint(v), row);
                ++cnt;
              }
            }
          }
      }
    } else if (wave_live) {
      // group minima over each lane's 16 rows of each 32-row block
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        float m = __builtin_inff();
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rl = blk * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          const float g = blk == 0 ? acc0[r] : acc1[r];
          const float v = METRIC == 0 ? fmaf(-2.f, g, xns[slot][rl]) : -g;
          const uint32_t row = base + rl;
          if (row < r_end && row_allowed(a.allow, a.rid[row])) m = fminf(m, v);
        }
        if (q < a.nq) {
          const uint32_t grp = ((base >> 5) + blk) * 2 + h;
          if (grp < uint32_t(a.ngroups)) a.gm[size_t(q) * a.ngroups + grp] = m;
        }
      }
    }
    slot = slot == 2 ? 0 : slot + 1;
  }

  if (MODE == 0 && q < a.nq) {
    a.counts[seg] = min(cnt, uint32_t(a.caph));
    if (cnt > uint32_t(a.caph)) a.ovf[q] = 1;
  }
}

// ================================================================ threshold from groups

struct KthArgs {
  const float* gm;
  int ngroups, nq, rank;  // the rank of the group minimum taken (ThresholdRank)
  const float* eb;
  float* T;
};


// One wave per query: the rank-th smallest group minimum A.  At rank kk, the kk groups at
// or below A hold kk distinct rows with GEMM value <= A, so the kk-th smallest exact
// distance is at most A + shift + eb and every row of the true top kk has GEMM value
// <= A + 2 eb.  At a lower rank the same holds unless the sample took more than rank - 1
// of the top kk - 1 rows (ThresholdRank), which the certificate detects.
// A is found by a bitwise radix select over the order-preserving encodings, held V per lane:
// from the top bit down, the answer keeps a 0 bit when at least kk keys lie at or below the
// prefix with all lower bits set (ballot + popcount, no cross-lane data movement).
template <int V>
__global__ __launch_bounds__(256) void k_kth(KthArgs a) {
  const int q = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= a.nq) return;
  const int lane = lane_id();
  const float* g = a.gm + size_t(q) * a.ngroups;
  uint32_t key[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int i = v * kWave + lane;
    key[v] = i < a.ngroups ? ord_enc(g[i]) : 0xffffffffu;
  }
  float A = __builtin_inff();
  if (a.rank <= a.ngroups) {
    uint32_t ans = 0;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t t = ans | ((1u << bit) - 1u);
      int cnt = 0;
#pragma unroll
      for (int v = 0; v < V; ++v) cnt += __popcll(__ballot(key[v] <= t));
      if (cnt < a.rank) ans |= 1u << bit;
    }
    A = ord_dec_dev(ans);
  }
  if (lane == 0) a.T[q] = A < __builtin_inff() ? A + 2.f * a.eb[q] : __builtin_inff();
}

// The same radix select with a block of 16 waves per query (small batches): V keys per
// thread, the per-bit counts summed across the waves through LDS, one barrier per bit.
template <int V>
__global__ __launch_bounds__(1024) void k_kth_block(KthArgs a) {
  __shared__ int s_cnt[2][16];
  const int q = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const float* g = a.gm + size_t(q) * a.ngroups;
  uint32_t key[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int i = v * 1024 + int(threadIdx.x);
    key[v] = i < a.ngroups ? ord_enc(g[i]) : 0xffffffffu;
  }
  float A = __builtin_inff();
  if (a.rank <= a.ngroups) {
    uint32_t ans = 0;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t t = ans | ((1u << bit) - 1u);
      int cnt = 0;
#pragma unroll
      for (int v = 0; v < V; ++v) cnt += __popcll(__ballot(key[v] <= t));
      if (lane == 0) s_cnt[bit & 1][wave] = cnt;
      __syncthreads();
      int total = 0;
#pragma unroll
      for (int w = 0; w < 16; ++w) total += s_cnt[bit & 1][w];
      if (total < a.rank) ans |= 1u << bit;
    }
    A = ord_dec_dev(ans);
  }
  if (threadIdx.x == 0) a.T[q] = A < __builtin_inff() ? A + 2.f * a.eb[q] : __builtin_inff();
}

// ================================================================ selection / merge

struct SelectArgs {
  const float* Q;
  const uint2* cand;
  const uint32_t* counts;
  int nseg, cap;
  const int* ovf;          // nullable
  const float* shift;      // rescore mode
  const float* eb;
  const int* exact;
  const uint32_t* qlist;   // nullable: slot i answers query qlist[i]
  int nslots, k, pd;
  int rescore;             // 0: candidates hold exact distances; 1: GEMM values, rescore
                           // the best K'; 2: GEMM values, rescore every candidate
  int by_query;            // candidate buffers are indexed by query (else by slot)
  const float* T;          // rescore 1 and 2: the admission threshold of the GEMM pass
  int force_fallback;      // testing: 1 fails every rescore-1 certificate, 2 also rescore 2
  uint32_t* out_ids;
  float* out_d;
  uint32_t* fb_list;       // rescore mode: queries that need the exact re-scan
  uint32_t* fb_count;
  const uint32_t* nslots_dev;  // nullable: slots at or past *nslots_dev exit (a pass queued
                               // for every slot whose count an earlier kernel decides)
  uint32_t* fb_acc;            // nullable: *nslots_dev is added here once (the context's count
                               // of exact re-scans queued without a host read)
};

constexpr int kMaxSeg = 1024;

// One wave per slot (WPS = 1, four slots per block), or WPS waves per slot for small
// batches: each wave streams the candidates of its share of the slot's segments (a prefix
// sum over the segment counts maps a flat index to its segment) into a wave top-k of
// capacity 64*E, and wave 0 merges the others' lists before the re-scoring.  Queries that
// fail a certificate (or whose buffers overflowed) are appended to fb_list.
template <int E, class Scorer, int WPS, bool STRIDE = false>
__global__ __launch_bounds__(WPS == 1 ? 256 : 64 * WPS) void k_select(SelectArgs a, Scorer sc) {
  static_assert(!STRIDE || WPS == 1, "striding waves share no barrier only with one wave a slot");
  constexpr int WAVES = WPS == 1 ? 4 : WPS;
  constexpr int PRE = WPS == 1 ? kMaxSeg : kMaxSeg / WPS;  // segments per wave
  __shared__ uint32_t pre_all[WAVES][PRE + 1];
  __shared__ float stage_d[WAVES][2 * kWave];
  __shared__ uint32_t stage_i[WAVES][2 * kWave];
  __shared__ float md[WPS == 1 ? 1 : WPS - 1][WPS == 1 ? 1 : kWave * E];
  __shared__ uint32_t mi[WPS == 1 ? 1 : WPS - 1][WPS == 1 ? 1 : kWave * E];
  __shared__ uint32_t mtot[WAVES];
  // flat rows with an int8 copy (FlatScorer8): the query packed into int8 when its
  // distances are exact integers (Int8Query)
  constexpr bool kI8 = std::is_same<Scorer, FlatScorer8>::value;
  __shared__ uint32_t ys_all[kI8 ? WAVES : 1][kI8 ? 256 : 1];
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const int sub = WPS == 1 ? 0 : wave;  // the wave's share of the slot's segments
  if (a.fb_acc != nullptr && blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(a.fb_acc, *a.nslots_dev);
  auto run = [&](const int slot) __attribute__((always_inline)) {
  if (slot >= a.nslots) return;
  if (a.nslots_dev != nullptr && uint32_t(slot) >= *a.nslots_dev) return;
  const uint32_t q = a.qlist ? a.qlist[slot] : uint32_t(slot);
  const uint32_t src = a.by_query ? q : uint32_t(slot);
  uint32_t* pre = pre_all[wave];

  if (a.ovf != nullptr && a.ovf[q]) {
    if (lane == 0 && sub == 0) {
      const uint32_t p = atomicAdd(a.fb_count, 1u);
      a.fb_list[p] = q;
    }
    return;
  }

  const int per = (a.nseg + WPS - 1) / WPS;
  const int s_lo = min(a.nseg, sub * per), nseg_w = min(a.nseg, s_lo + per) - s_lo;
  uint32_t run = 0;
  const uint32_t* cnts = a.counts + size_t(src) * a.nseg + s_lo;
  for (int b = 0; b < nseg_w; b += kWave) {
    const int s = b + lane;
    const uint32_t c = s < nseg_w ? cnts[s] : 0u;
    uint32_t incl = c;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const uint32_t t = __shfl_up(incl, o);
      if (lane >= o) incl += t;
    }
    if (s < nseg_w) pre[s + 1] = run + incl;
    run += __shfl(incl, kWave - 1);
  }
  if (lane == 0) pre[0] = 0;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint32_t total_w = run;

  WaveTopK<E> top;
  top.init();
  const float* qv = a.Q + size_t(q) * a.pd;
  Int8Query p8{0, 0, nullptr};
  if constexpr (kI8)
    p8 = int8_query(sc.X8, sc.c8, sc.xlo, sc.xhi, sc.xmax, sc.xint, sc.metric, sc.pd, qv,
                    ys_all[wave]);
  auto score = [&](uint32_t id) -> float {
    if constexpr (kI8) {
      if (p8.on) return int8_distance<1>(sc.X8, sc.c8, sc.metric, sc.pd, p8, id);
    }
    return sc(qv, id);
  };
  const uint2* cbase = a.cand + (size_t(src) * a.nseg + s_lo) * size_t(a.cap);
  // candidate g of the wave's flat order: the segment is the largest s with pre[s] <= g
  auto fetch = [&](uint32_t g) -> uint2 {
    if (g >= total_w) return make_uint2(__float_as_uint(__builtin_inff()), kNoId);
    int lo = 0, hi = nseg_w;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (pre[mid] <= g) lo = mid; else hi = mid;
    }
    return cbase[size_t(lo) * a.cap + (g - pre[lo])];
  };
  // Candidates that beat the current n-th key are packed into a per-wave staging area and
  // inserted 64 at a time, so the sort-and-merge runs once per 64 wanted keys rather than
  // once per 64 streamed ones (the key to beat only tightens, so filtering against an older
  // one keeps every key the final list needs).
  float* sd = stage_d[wave];
  uint32_t* si = stage_i[wave];
  int staged = 0;
  auto push = [&](float d, uint32_t id) {
    float td;
    uint32_t ti;
    top.threshold(td, ti);
    const bool want = id != kNoId && nb_less(d, id, td, ti);
    const uint64_t bal = __ballot(want);
    if (bal == 0) return;
    const int pos = staged + __popcll(bal & ((1ull << lane) - 1ull));
    if (want) {
      sd[pos] = d;
      si[pos] = id;
    }
    staged += __popcll(bal);
    if (staged >= kWave) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const float d0 = sd[lane];
      const uint32_t i0 = si[lane];
      const bool more = lane + kWave < staged;
      const float d1 = more ? sd[lane + kWave] : 0.f;
      const uint32_t i1 = more ? si[lane + kWave] : 0u;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (more) {
        sd[lane] = d1;
        si[lane] = i1;
      }
      staged -= kWave;
      top.insert(d0, i0);
    }
  };
  // the next batch is loaded before the current one is pushed (hides the load latency)
  uint2 cur = fetch(lane);
  for (uint32_t g0 = 0; g0 < total_w; g0 += kWave) {
    const uint2 nxt = fetch(g0 + kWave + lane);
    const uint32_t id = cur.y;
    float d = __uint_as_float(cur.x);
    if (a.rescore == 2 && id != kNoId) d = score(id);
    push(d, id);
    cur = nxt;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (staged > 0) {
    const bool have = lane < staged;
    top.insert(have ? sd[lane] : __builtin_inff(), have ? si[lane] : kNoId);
  }
  uint32_t total = total_w;
  if constexpr (WPS > 1) {
    // the other waves' lists and candidate counts into wave 0
    if (wave > 0) {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        md[wave - 1][e * kWave + lane] = top.k.d[e];
        mi[wave - 1][e * kWave + lane] = top.k.id[e];
      }
    }
    if (lane == 0) mtot[wave] = total_w;
    __syncthreads();
    if (wave > 0) return;
    for (int w = 1; w < WPS; ++w) {
      total += mtot[w];
#pragma unroll
      for (int e = 0; e < E; ++e) top.insert(md[w - 1][e * kWave + lane], mi[w - 1][e * kWave + lane]);
    }
  }

  constexpr int N = kWave * E;
  uint32_t* oi = a.out_ids + size_t(q) * a.k;
  float* od = a.out_d + size_t(q) * a.k;
  if (a.rescore == 2) {
    // every row outside the buffers has GEMM value > T, so exact distance
    // > T + shift - eb: certified when the k-th exact distance is at most that
    float dk = __builtin_inff();
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int gi = e * kWave + lane;
      if (gi < a.k) {
        oi[gi] = top.k.id[e];
        od[gi] = top.k.d[e];
      }
      const float v = __shfl(top.k.d[e], (a.k - 1) & (kWave - 1));
      if (e == (a.k - 1) / kWave) dk = v;
    }
    {
      const double lower = (double(a.T[q]) + double(a.shift[q])) - double(a.eb[q]);
      if ((!(double(dk) <= lower) || a.force_fallback >= 2) && lane == 0) {
        const uint32_t p = atomicAdd(a.fb_count, 1u);
        a.fb_list[p] = q;
      }
    }
    return;
  }
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

  // Flat rows score eight lanes a row (metric_exact_g8n, int8_distance_g8n: whole 128-byte runs
  // of a row per group load) where the scorer's order has that form; eight keys a round, each
  // key's distance then handed to its own lane.
  constexpr bool kGroup = std::is_same<Scorer, FlatScorer>::value || kI8;
  bool group = false;
  if constexpr (kGroup) group = (kI8 && p8.on) || sc.kset == kKsetAvx512;

  // exact re-scoring of the K' = N-1 best by GEMM value, in two stages.  Stage 1 re-scores
  // the best n1 = min(K', k + 8), rounded up to whole 64-lane passes when k + 8 takes more
  // than one (at k = 64 a stage of k + 8 keys fails the certificate often enough that its
  // second stage costs more than scoring the extra keys at once); its answer stands when
  // every later candidate provably lies behind it: the (n1+1)-th GEMM value plus the shift
  // minus the bound exceeds the k-th exact distance.  Rows outside the buffers have GEMM
  // value > T, at least that (n1+1)-th value, so they lie behind it too.  When no later
  // candidate exists, or in exact mode (the GEMM order is the distance order), the outside
  // rows are checked against T itself:
  // the k-th exact distance is at most T + shift - eb (always so when T came from the kk-th
  // group minimum; a threshold of lower rank fails it when it kept fewer than the top k).
  // Otherwise stage 2 scores the rest of the K' and checks the same certificate at K'+1.
  const uint32_t nsel = min(total, uint32_t(N - 1));
  const uint32_t want = uint32_t(a.k) + 8u;
  const uint32_t n1 = min(nsel, want > uint32_t(kWave) ? (want + kWave - 1) / kWave * kWave : want);
  const float shift = a.shift[q], ebq = a.eb[q];
  const bool exact = a.exact[q] != 0;
  WaveKeys<E> r;
  float ud[E];  // exact distances of the scored keys, in top.k's order
  // R keys per group (rows ids[0..R)), every row's loads in flight together
  auto score_g8 = [&](const auto& ids, auto& d) {
    if constexpr (kI8) {
      if (p8.on) {
        int8_distance_g8n(sc.X8, sc.c8, sc.metric, sc.pd, p8, ids, d);
        return;
      }
    }
    if constexpr (kGroup) {
      constexpr int R = sizeof(d) / sizeof(float);
      const float* xs[R];
#pragma unroll
      for (int i = 0; i < R; ++i)
        xs[i] = sc.X + size_t(sc.map != nullptr ? sc.map[ids[i]] : ids[i]) * sc.pd;
      metric_exact_g8n<R>(sc.metric, qv, xs, sc.pd, d);
    }
  };
  // scores keys [lo, hi) of top.k (passes with no key in range are skipped), then sorts the
  // first hi scored keys into r
  auto rescore_first = [&](uint32_t lo, uint32_t hi) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (uint32_t(e + 1) * kWave <= lo || uint32_t(e) * kWave >= hi) continue;
      const uint32_t gi = e * kWave + lane;
      if constexpr (kGroup) {
        if (group) {
          // lanes [b0, b1) of this pass hold the keys to score
          const int b0 = int(max(lo, uint32_t(e) * kWave) - uint32_t(e) * kWave);
          const int b1 = int(min(hi, uint32_t(e + 1) * kWave) - uint32_t(e) * kWave);
          group_pass(top.k.id[e], b0, b1, ud[e], score_g8);
          continue;
        }
      }
      if (gi >= lo && gi < hi) ud[e] = score(top.k.id[e]);
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const uint32_t gi = e * kWave + lane;
      r.d[e] = gi < hi ? ud[e] : __builtin_inff();
      r.id[e] = gi < hi ? top.k.id[e] : kNoId;
    }
    bitonic_sort<E>(r);
  };
  // element g of a wave-sorted list (wave-uniform g)
  auto at = [&](const float (&v)[E], uint32_t g) {
    float x = __builtin_inff();
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float t = __shfl(v[e], int(g & (kWave - 1)));
      if (uint32_t(e) == g / kWave) x = t;
    }
    return x;
  };
  const double lower = (double(a.T[q]) + double(shift)) - double(ebq);
  auto certify = [&](uint32_t n) {
    const float dk = at(r.d, uint32_t(a.k) - 1);
    if ((n >= total || exact) && double(dk) <= lower) return true;
    return n < total && dk < (at(top.k.d, n) + shift) - ebq;
  };
  rescore_first(0, n1);
  bool certified = certify(n1);
  if (!certified && n1 < nsel) {
    rescore_first(n1, nsel);
    certified = certify(nsel);
  }
  if (a.force_fallback >= 1) certified = false;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int gi = e * kWave + lane;
    if (gi < a.k) {
      oi[gi] = r.id[e];
      od[gi] = r.d[e];
    }
  }
  if (!certified && lane == 0) {
    const uint32_t p = atomicAdd(a.fb_count, 1u);
    a.fb_list[p] = q;
  }
  };
  if constexpr (STRIDE) {
    // a gated pass on a bounded grid: each wave strides over the slots the device count
    // allows (the waves of one slot share nothing, so no barrier is involved)
    const int n = int(min(*a.nslots_dev, uint32_t(a.nslots)));
    for (int slot = int(blockIdx.x) * 4 + wave; slot < n; slot += int(gridDim.x) * 4) run(slot);
  } else {
    run(WPS == 1 ? int(blockIdx.x) * 4 + wave : int(blockIdx.x));
  }
}

// ================================================================ exact scan

struct ScanArgs {
  const float* Q;
  const uint64_t* allow;
  int pd;
  uint32_t N;
  const uint32_t* qlist;  // nullable
  int nslots;
  uint32_t split_rows;
  int nsplit;
  uint2* part;            // [slot][split][64*E]
  uint32_t* part_counts;  // [slot][split]
  const uint32_t* nslots_dev;  // nullable: slots at or past *nslots_dev are not scanned
};

// Grid of a gated exact re-scan pass (two blocks per CU of a 256-CU part).
constexpr size_t kGatedScanBlocks = 512;

// Block = 4 waves on one (query, row split) item at a time; each wave keeps a top-64E of its
// rows with exact distances, then wave 0 merges the other three through LDS.  Items are
// slot * nsplit + split.  With nslots_dev the grid is bounded (a pass queued for every query
// but run for the few the pass before listed) and the blocks stride over the items the
// device count allows, so a pass with nothing to do costs a small grid, not one block per
// item.
template <int E, class Scorer>
__device__ __forceinline__ void exact_scan_item(const ScanArgs& a, const Scorer& sc, int slot,
                                                int split, float (*md)[kWave * E],
                                                uint32_t (*mi)[kWave * E]) {
  constexpr int N = kWave * E;
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
      d = sc(qv, r);
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

template <int E, class Scorer, bool GATED>
__global__ __launch_bounds__(256) void k_exact_scan(ScanArgs a, Scorer sc) {
  __shared__ float md[3][kWave * E];
  __shared__ uint32_t mi[3][kWave * E];
  if constexpr (!GATED) {  // one item per block: (slot, split) = (blockIdx.x, blockIdx.y)
    exact_scan_item<E, Scorer>(a, sc, int(blockIdx.x), int(blockIdx.y), md, mi);
  } else {
    const uint32_t nslots = min(*a.nslots_dev, uint32_t(a.nslots));
    const uint32_t items = nslots * uint32_t(a.nsplit);
    for (uint32_t item = blockIdx.x; item < items; item += gridDim.x) {
      exact_scan_item<E, Scorer>(a, sc, int(item / uint32_t(a.nsplit)),
                                 int(item % uint32_t(a.nsplit)), md, mi);
      __syncthreads();  // wave 0 has read md / mi before the next item writes them
    }
  }
}

// ================================================================ rerank

struct RerankArgs {
  const float* X;
  const float* Q;
  int pd, metric, kset;
  const uint32_t* cand;  // [nq][depth] ascending by SQ8 distance, kNoId padded
  int depth, nq, k;
  uint32_t* out_ids;
  float* out_d;
  const int8_t* X8;      // nullable: the rows' int8 copy (integer rows, x = x8 + c8)
  int c8;
  RowStats xs;           // the rows' value statistics
};

// Rerank (src/index/index.cc:89-95): exact fp32 distances of the candidates' rows, the k
// smallest by (dist, id).  One wave per query, up to 64*E candidates.
template <int E>
__global__ __launch_bounds__(256) void k_rerank(RerankArgs a) {
  __shared__ uint32_t ys_all[4][256];  // the query as int8 y - c8, four dims a word
  const int q = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= a.nq) return;
  const int lane = lane_id();
  const float* qv = a.Q + size_t(q) * a.pd;
  // Integer rows and an integer query whose every partial sum stays below 2^24: every fp32
  // summation order, the reference's included, gives the exact integer, so the distance is
  // computed from the rows' int8 copy (a quarter of the bytes) in int32: on packed dot
  // products when the shifted query fits int8 (Int8Query), else value by value.
  const Int8Query p8 = int8_query(a.X8, a.c8, a.xs.lo, a.xs.hi, a.xs.max_abs, a.xs.all_int,
                                  a.metric, a.pd, qv, ys_all[threadIdx.x >> 6]);
  bool ex8 = false;
  if (!p8.on && a.X8 != nullptr && a.metric != 2) {
    float mq = 0.f, lo = __builtin_inff(), hi = -__builtin_inff();
    int ai = 1;
    for (int i = lane; i < a.pd; i += kWave) {
      const float v = qv[i];
      mq = fmaxf(mq, fabsf(v));
      lo = fminf(lo, v);
      hi = fmaxf(hi, v);
      ai &= v == rintf(v) ? 1 : 0;
    }
    mq = wave_max(mq);
    lo = wave_min(lo);
    hi = wave_max(hi);
    ai = wave_and(ai);
    const double pd = a.pd, lim = 16777216.0, mx = a.xs.max_abs, m = mq;
    const double range = double(fmaxf(hi, a.xs.hi)) - double(fminf(lo, a.xs.lo));
    ex8 = a.xs.all_int && ai && pd * mx * mx < lim && pd * m * m < lim && pd * mx * m < lim &&
          pd * range * range < lim;
  }
  auto exact8 = [&](uint32_t id) {
    const int8_t* xr = a.X8 + size_t(id) * a.pd;
    int acc = 0;
    for (int i = 0; i < a.pd; i += 16) {
      const int4 w = *reinterpret_cast<const int4*>(xr + i);
      const int8_t* b = reinterpret_cast<const int8_t*>(&w);
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int x = int(b[t]) + a.c8, y = int(qv[i + t]);
        acc += a.metric == 0 ? (x - y) * (x - y) : x * y;
      }
    }
    return a.metric == 0 ? float(acc) : -float(acc);  // -0 for a zero dot, as -dot gives
  };
  WaveKeys<E> r;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = e * kWave + lane;
    const uint32_t id = i < a.depth ? a.cand[size_t(q) * a.depth + i] : kNoId;
    if (id != kNoId) {
      r.d[e] = p8.on ? int8_distance(a.X8, a.c8, a.metric, a.pd, p8, id)
               : ex8  ? exact8(id)
                      : metric_exact_k(a.kset, a.metric, qv, a.X + size_t(id) * a.pd, a.pd);
      r.id[e] = id;
    } else {
      r.d[e] = __builtin_inff();
      r.id[e] = kNoId;
    }
  }
  bitonic_sort<E>(r);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = e * kWave + lane;
    if (i < a.k) {
      a.out_ids[size_t(q) * a.k + i] = r.id[e];
      a.out_d[size_t(q) * a.k + i] = r.d[e];
    }
  }
}

// ================================================================ orchestration

__global__ void k_fill_empty(uint32_t* ids, float* d, size_t n) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i < n) {
    ids[i] = kNoId;
    d[i] = __builtin_inff();
  }
}

// Small batches split each slot's segments over 16 (up to 64 slots, k <= 112: 128 registers
// per lane hold that list) or 4 waves (up to 256) so the slot's candidates stream in
// parallel; larger ones run one wave per slot.
template <int E, class Scorer>
static void launch_select(hipStream_t s, const SelectArgs& a, const Scorer& sc) {
  if (a.nslots <= 256 && a.nseg >= 16)
    k_select<E, Scorer, 4><<<dim3(a.nslots), 256, 0, s>>>(a, sc);
  else if (a.nslots_dev != nullptr)  // gated: a bounded grid of striding waves
    k_select<E, Scorer, 1, true><<<dim3(unsigned(std::min<size_t>((size_t(a.nslots) + 3) / 4,
                                                                   kGatedScanBlocks))),
                                   256, 0, s>>>(a, sc);
  else
    k_select<E, Scorer, 1><<<dim3((a.nslots + 3) / 4), 256, 0, s>>>(a, sc);
}
template <int E, class Scorer>
static void launch_scan(hipStream_t s, const ScanArgs& a, const Scorer& sc) {
  if (a.nslots_dev == nullptr) {
    k_exact_scan<E, Scorer, false><<<dim3(a.nslots, a.nsplit), 256, 0, s>>>(a, sc);
  } else {  // a gated pass: a bounded grid striding over the items the device count allows
    const size_t items = size_t(a.nslots) * size_t(a.nsplit);
    const unsigned blocks = unsigned(std::max<size_t>(1, std::min<size_t>(items, kGatedScanBlocks)));
    k_exact_scan<E, Scorer, true><<<dim3(blocks), 256, 0, s>>>(a, sc);
  }
}
template <int V>
static void launch_kth_v(hipStream_t s, const KthArgs& a) {
  k_kth<V><<<dim3((a.nq + 3) / 4), 256, 0, s>>>(a);
}
static int LaunchKth(hipStream_t s, const KthArgs& a) {
  // a block per query for many groups; up to 256 (a small sample, small N) a wave per
  // query costs less (100k x 128 rows, 1,000 queries, 128 groups: 7.05 -> 8.27M q/s)
  if (a.nq <= 1024 && a.ngroups > 256 && a.ngroups <= 4096) {
    if (a.ngroups <= 1024) k_kth_block<1><<<dim3(a.nq), 1024, 0, s>>>(a);
    else if (a.ngroups <= 2048) k_kth_block<2><<<dim3(a.nq), 1024, 0, s>>>(a);
    else k_kth_block<4><<<dim3(a.nq), 1024, 0, s>>>(a);
    return kOk;
  }
  int v = 1;
  while (v * kWave < a.ngroups) v <<= 1;
  switch (v) {
    case 1: launch_kth_v<1>(s, a); break;
    case 2: launch_kth_v<2>(s, a); break;
    case 4: launch_kth_v<4>(s, a); break;
    case 8: launch_kth_v<8>(s, a); break;
    case 16: launch_kth_v<16>(s, a); break;
    case 32: launch_kth_v<32>(s, a); break;
    case 64: launch_kth_v<64>(s, a); break;
    default: return SetError(kInternal, "threshold: more than 4096 sample groups");
  }
  return kOk;
}
template <int E>
static void launch_rerank(hipStream_t s, const RerankArgs& a) {
  k_rerank<E><<<dim3((a.nq + 3) / 4), 256, 0, s>>>(a);
}

#define VDBG_DISPATCH_E(E, FN, ...)                          \
  switch (E) {                                               \
    case 1: FN<1>(__VA_ARGS__); break;                       \
    case 2: FN<2>(__VA_ARGS__); break;                       \
    case 4: FN<4>(__VA_ARGS__); break;                       \
    default: return SetError(kNotSupported, "k too large"); \
  }
#define VDBG_DISPATCH_ES(E, FN, SC, ...)                     \
  switch (E) {                                               \
    case 1: FN<1, SC>(__VA_ARGS__); break;                   \
    case 2: FN<2, SC>(__VA_ARGS__); break;                   \
    case 4: FN<4, SC>(__VA_ARGS__); break;                   \
    default: return SetError(kNotSupported, "k too large"); \
  }

static FlatScorer FlatOf(const ScanSource& src, int kset) {
  return FlatScorer{src.X, src.pd, src.metric, kset, src.Xmap};
}
// Whether a selection takes FlatScorer8: rows with a one-part int8 copy, and more keys to
// re-score than one 64-lane pass, every buffered candidate (the second chance), or a small
// batch (latency-bound: the fp32 rows' loads form a chain of dependent rounds per lane, the
// int8 rows' loads issue together).  For one pass over many queries the query packing costs
// more than it saves.
static bool UseFlat8(const ScanSource& src, size_t nq, size_t kk, int rescore) {
  return src.kind == 0 && src.X8 != nullptr && src.x8_parts == 1 &&
         (rescore == 2 || kk + 8 > size_t(kWave) || nq <= 256);
}
static FlatScorer8 Flat8Of(const ScanSource& src, int kset) {
  FlatScorer8 f;
  static_cast<FlatScorer&>(f) = FlatOf(src, kset);
  f.X8 = src.X8;
  f.c8 = src.c8;
  f.xlo = src.stats.lo;
  f.xhi = src.stats.hi;
  f.xmax = src.stats.max_abs;
  f.xint = src.stats.all_int;
  return f;
}
static Sq8Scorer Sq8Of(const ScanSource& src, int kset) {
  return Sq8Scorer{src.C, src.vmin, src.scale, src.pd, src.metric, kset};
}

__global__ void k_fb_reset(uint32_t* __restrict__ acc) {
  if (threadIdx.x == 0) *acc = 0;
}

// A new call's count of exact re-scans starts from zero: the host's, and the device's when
// an earlier call left one there (a call spanning several scans, the collection search,
// clears it once and sets fb_accumulate for its scans).
int ResetFallbacks(Ctx* c, hipStream_t s) {
  if (c->fb_accumulate) return kOk;
  c->last_fallbacks = 0;
  if (c->fb_dev_used) {
    k_fb_reset<<<1, 64, 0, s>>>(c->fb_dev);
    VDBG_HIP(hipGetLastError());
  }
  return kOk;
}

// Largest worst-case exact re-scan scratch (every query of the batch re-scanned) for which
// the fallback passes are queued without reading their counts on the host.
constexpr size_t kGatedExactBytes = size_t(64) << 20;

// The exact scan's row splits for nslots queries over N rows, and its scratch bytes.
struct ExactPlan {
  int nsplit;
  uint32_t split_rows;
  size_t need;
};
static ExactPlan PlanExact(uint32_t N, int nslots, size_t k) {
  ExactPlan p{};
  int nsplit = int(std::min<size_t>((2048 + nslots - 1) / nslots,
                                    std::max<size_t>(1, (N + 1023) / 1024)));
  nsplit = std::max(1, std::min(nsplit, kMaxSeg));
  p.split_rows = (N + nsplit - 1) / nsplit;
  p.split_rows = (p.split_rows + 63) / 64 * 64;
  p.nsplit = int((N + p.split_rows - 1) / p.split_rows);
  const int cap = kWave * pow2_e(k);
  p.need = size_t(nslots) * p.nsplit * cap * sizeof(uint2) +
           size_t(nslots) * p.nsplit * sizeof(uint32_t) + 4096;
  return p;
}

template <class Scorer>
static int ExactScanT(Ctx* c, Workspace& w, const ScanSource& src, const Scorer& sc,
                      const float* Q, const uint32_t* qlist, int nslots, size_t k,
                      const uint64_t* allow, uint32_t* out_ids, float* out_d, hipStream_t s,
                      const uint32_t* nslots_dev = nullptr, uint32_t* fb_acc = nullptr) {
  const int E = pow2_e(k);
  const uint32_t N = src.N;
  const ExactPlan ep = PlanExact(N, nslots, k);
  const int nsplit = ep.nsplit;
  const uint32_t split_rows = ep.split_rows;
  const int cap = kWave * E;
  const size_t need = ep.need;
  WsUse wuse(&w, s);
  VDBG_RETURN_IF_ERROR(wuse.status());
  w.used = 0;
  VDBG_RETURN_IF_ERROR(w.reserve(need));
  uint2* part = w.take<uint2>(size_t(nslots) * nsplit * cap);
  uint32_t* pc = w.take<uint32_t>(size_t(nslots) * nsplit);
  ScanArgs sa{Q, allow, src.pd, N, qlist, nslots, split_rows, nsplit, part, pc, nslots_dev};
  {
    ProfScope ps(c, "exact_scan", s);
    VDBG_DISPATCH_ES(E, launch_scan, Scorer, s, sa, sc);
    VDBG_HIP(hipGetLastError());
  }
  SelectArgs se{};
  se.Q = Q;
  se.cand = part;
  se.counts = pc;
  se.nseg = nsplit;
  se.cap = cap;
  se.qlist = qlist;
  se.nslots = nslots;
  se.k = int(k);
  se.pd = src.pd;
  se.rescore = 0;
  se.out_ids = out_ids;
  se.out_d = out_d;
  se.nslots_dev = nslots_dev;
  se.fb_acc = fb_acc;
  {
    ProfScope ps(c, "merge", s);
    VDBG_DISPATCH_ES(E, launch_select, Scorer, s, se, sc);
    VDBG_HIP(hipGetLastError());
  }
  return kOk;
}

static int ExactScan(Ctx* c, Workspace& w, const ScanSource& src, const float* Q,
                     const uint32_t* qlist, int nslots, size_t k, const uint64_t* allow,
                     uint32_t* out_ids, float* out_d, hipStream_t s,
                     const uint32_t* nslots_dev = nullptr, uint32_t* fb_acc = nullptr) {
  if (nslots == 0) return kOk;
  if (pow2_e(k) > 4) return SetError(kNotSupported, "k > 256 is not supported on the GPU path");
  if (src.kind == 0)
    return ExactScanT(c, w, src, FlatOf(src, c->kset), Q, qlist, nslots, k, allow, out_ids, out_d,
                      s, nslots_dev, fb_acc);
  if (src.kind == 2)
    return ExactScanT(c, w, src, PqScorer{src.C, src.pq_m}, Q, qlist, nslots, k, allow, out_ids,
                      out_d, s, nslots_dev, fb_acc);
  return ExactScanT(c, w, src, Sq8Of(src, c->kset), Q, qlist, nslots, k, allow, out_ids, out_d,
                    s, nslots_dev, fb_acc);
}

template <int PD, int METRIC, int KIND, int MODE>
static void launch_gemm(hipStream_t s, int blocks, const GemmArgs& a) {
  k_gemm<PD, METRIC, KIND, MODE><<<dim3(blocks), 256, 0, s>>>(a);
}

template <int PD>
static void launch_gemm_pd(int metric, int kind, int mode, hipStream_t s, int blocks,
                           const GemmArgs& a) {
  if (kind == 0) {
    if (metric == 0) {
      if (mode == 0) launch_gemm<PD, 0, 0, 0>(s, blocks, a);
      else launch_gemm<PD, 0, 0, 1>(s, blocks, a);
    } else {
      if (mode == 0) launch_gemm<PD, 1, 0, 0>(s, blocks, a);
      else launch_gemm<PD, 1, 0, 1>(s, blocks, a);
    }
  } else {
    if (metric == 0) {
      if (mode == 0) launch_gemm<PD, 0, 1, 0>(s, blocks, a);
      else launch_gemm<PD, 0, 1, 1>(s, blocks, a);
    } else {
      if (mode == 0) launch_gemm<PD, 1, 1, 0>(s, blocks, a);
      else launch_gemm<PD, 1, 1, 1>(s, blocks, a);
    }
  }
}

static int LaunchGemm(size_t pd, int metric, int kind, int mode, hipStream_t s, int blocks,
                      const GemmArgs& a) {
  switch (pd) {
    case 16: launch_gemm_pd<16>(metric, kind, mode, s, blocks, a); break;
    case 32: launch_gemm_pd<32>(metric, kind, mode, s, blocks, a); break;
    case 48: launch_gemm_pd<48>(metric, kind, mode, s, blocks, a); break;
    case 64: launch_gemm_pd<64>(metric, kind, mode, s, blocks, a); break;
    case 80: launch_gemm_pd<80>(metric, kind, mode, s, blocks, a); break;
    case 96: launch_gemm_pd<96>(metric, kind, mode, s, blocks, a); break;
    case 112: launch_gemm_pd<112>(metric, kind, mode, s, blocks, a); break;
    case 128: launch_gemm_pd<128>(metric, kind, mode, s, blocks, a); break;
    case 192: launch_gemm_pd<192>(metric, kind, mode, s, blocks, a); break;
    case 256: launch_gemm_pd<256>(metric, kind, mode, s, blocks, a); break;
    case 384: launch_gemm_pd<384>(metric, kind, mode, s, blocks, a); break;
    case 512: launch_gemm_pd<512>(metric, kind, mode, s, blocks, a); break;
    case 768: launch_gemm_pd<768>(metric, kind, mode, s, blocks, a); break;
    case 960: launch_gemm_pd<960>(metric, kind, mode, s, blocks, a); break;
    case 1024: launch_gemm_pd<1024>(metric, kind, mode, s, blocks, a); break;
    default: return SetError(kNotSupported, "GEMM path: unsupported padded_dim");
  }
  return kOk;
}

// Chunk count for nqt query tiles over N rows: the fewest chunks whose last round of blocks
// fills the resident slots (2 blocks per CU) within 3% of the best balance on offer.
static int PlanChunks(int nqt, uint32_t N, int slots, int max_chunks) {
  const int limit = std::max(1, std::min<int>(max_chunks, int((N + 63) / 64)));
  std::vector<std::pair<int, double>> opts;
  double best = 0;
  for (int nc = 1; nc <= limit; ++nc) {
    uint32_t rows = (N + nc - 1) / nc;
    rows = (rows + 63) / 64 * 64;
    if (int((N + rows - 1) / rows) != nc) continue;
    const double items = double(nqt) * nc;
    const double util = items / (std::ceil(items / slots) * slots);
    opts.emplace_back(nc, util);
    best = std::max(best, util);
  }
  for (const auto& o : opts)
    if (o.second >= best - 0.03) return o.first;
  return 1;
}

static void GemmGrid(GemmArgs& ga, int nqt, int nchunks, int* blocks) {
  ga.nqt = nqt;
  ga.nchunks = nchunks;
  ga.items = nqt * nchunks;
  ga.per_xcd = (ga.items + 7) / 8;
  *blocks = ga.per_xcd * 8;
}

int ScoreScan(Ctx* c, const ScanSource& src, const float* Q, size_t nq, size_t kk,
              const uint64_t* allow, uint32_t* out_ids, float* out_d, hipStream_t s) {
  VDBG_RETURN_IF_ERROR(ResetFallbacks(c, s));
  c->last_gemm_bits = 0;
  c->last_gemm_gate = nullptr;
  if (nq == 0 || kk == 0) return kOk;
  if (src.N == 0) {
    k_fill_empty<<<dim3(unsigned((nq * kk + 255) / 256)), 256, 0, s>>>(out_ids, out_d, nq * kk);
    VDBG_HIP(hipGetLastError());
    return kOk;
  }
  if (kk > 240) return ExactScanAll(c, src, Q, nq, kk, allow, out_ids, out_d, s);
  return ExactScan(c, c->ws, src, Q, nullptr, int(nq), kk, allow, out_ids, out_d, s);
}

// ================================================================ tiny batches
//
// At most kTinyQ queries over integer rows with an int8 copy: two launches and no threshold
// pre-pass.  k_tiny_scan: each block streams a contiguous chunk of rows once, scores every
// row against every query as the int8 GEMM does (u = row start + sum x8 q8, exact in int32;
// key = -M u, the GEMM value plus the query's constant Qd) and keeps, per query, the kp
// smallest keys of its chunk with their rows, plus the chunk's kp-th key (+inf when the
// chunk holds fewer rows).  k_tiny_merge: one block per query prepares the query's operands
// and bound (query_prep_wave) beside merging the best keys of all chunks, re-scores the best n1 = min(K', k +
// 8) exactly (the reference's distance) and certifies the answer when the k-th exact
// distance lies strictly below every unscored row's lower bound: the (n1+1)-th key, and each
// full chunk's kp-th key (a row outside a chunk's list has a key at least that), taken back
// to distances by -Qd + shift - eb.  Queries that are outside the int8 bounds or fail the
// certificate go to the exact re-scan.  The last block publishes the fallback count to the
// host (as ReadWords does), so the call makes no other launch.

constexpr int kTinyQ = 2;       // queries
constexpr int kTinyK = 48;      // k (kp = k + 16 <= 64 keys per chunk)
constexpr int kTinyMaxPd = 256; // |key| < 2^23 stays exact in fp32
constexpr int kTinyWaves = 4;   // waves per scan block

struct TinyArgs {
  const float* Q;
  int nq, pd, metric, c8, k, kp;
  const int8_t* X8;
  const int* init8;
  const uint64_t* allow;
  uint32_t N, chunk_rows;
  uint2* part;            // [q][chunk][kp] (key bits, row)
  float* bound;           // [q][chunk] the chunk's kp-th key, +inf when not full
  uint32_t* fb_count;     // [2] zeroed by the scan's block 0; [1] counts finished merges
  int nchunks;            // the scan's blocks
  uint32_t* fb_zero;      // nullable: the call's device fallback count, zeroed by block 0
};

// Rows reach the lanes through a per-wave LDS tile: the wave reads 64 consecutive rows with
// coalesced 16-byte loads (consecutive lanes, consecutive bytes), then each lane reads its
// own row from the tile (row stride padded by 16 bytes against bank conflicts).
template <int NQ, int VPR>
__global__ __launch_bounds__(kTinyWaves * 64) void k_tiny_scan(TinyArgs a) {
  __shared__ int s_q8[NQ][kTinyMaxPd / 4];
  __shared__ float sd[kTinyWaves][NQ][2 * kWave];
  __shared__ uint32_t si[kTinyWaves][NQ][2 * kWave];
  __shared__ float md[kTinyWaves - 1][NQ][kWave];
  __shared__ uint32_t mi[kTinyWaves - 1][NQ][kWave];
  extern __shared__ int4 tile_all[];  // [4][64][pd / 16 + 1]
  const int tid = threadIdx.x, wave = tid >> 6, lane = lane_id();
  constexpr int vpr = VPR;             // 16-byte vectors per row (pd / 16)
  int4* tile = tile_all + size_t(wave) * kWave * (vpr + 1);
  if (blockIdx.x == 0 && tid < 2) a.fb_count[tid] = 0;
  if (blockIdx.x == 0 && tid == 0 && a.fb_zero != nullptr) *a.fb_zero = 0;
  const int pw = a.pd / 4;
  for (int e = tid; e < NQ * pw; e += kTinyWaves * 64) {
    const int q = e / pw, w = e - q * pw;
    uint32_t packed = 0;
    if (q < a.nq) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        // q - c8 clamped into int8 (queries outside the window are re-scanned exactly)
        const float d = a.Q[size_t(q) * a.pd + 4 * w + t] - float(a.c8);
        packed |= uint32_t(uint8_t(int8_t(int(fminf(fmaxf(d, -128.f), 127.f))))) << (8 * t);
      }
    }
    s_q8[q][w] = int(packed);
  }
  __syncthreads();
  const uint32_t r0 = blockIdx.x * a.chunk_rows, r1 = min(a.N, r0 + a.chunk_rows);
  const int M = a.metric == 0 ? 2 : 1;
  WaveTopK<1> top[NQ];
  int staged[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    top[q].init();
    staged[q] = 0;
  }
  const int rl = (a.kp - 1) & (kWave - 1);
  // the 64 rows of a step, coalesced (vector e of the 64-row block: consecutive lanes read
  // consecutive bytes); the next step's rows load while this one is scored
  auto load_step = [&](uint32_t base, int4 (&v)[VPR]) {
    const uint32_t nrow = base < r1 ? min(uint32_t(kWave), r1 - base) : 0u;
    const int4* src = reinterpret_cast<const int4*>(a.X8 + size_t(base) * a.pd);
#pragma unroll
    for (int t = 0; t < VPR; ++t) {
      const int e = t * kWave + lane;
      v[t] = e < int(nrow) * vpr ? src[e] : make_int4(0, 0, 0, 0);
    }
  };
  int4 vn[VPR];
  load_step(r0 + wave * kWave, vn);
  for (uint32_t base = r0 + wave * kWave; base < r1; base += kTinyWaves * kWave) {
    const uint32_t r = base + lane;
    const bool live = r < r1 && row_allowed(a.allow, r);
    {
      const uint32_t nrow = min(uint32_t(kWave), r1 - base);
      int4 v[VPR];
#pragma unroll
      for (int t = 0; t < VPR; ++t) v[t] = vn[t];
      load_step(base + kTinyWaves * kWave, vn);
#pragma unroll
      for (int t = 0; t < VPR; ++t) {
        const int e = t * kWave + lane;
        if (e < int(nrow) * vpr) tile[(e / vpr) * (vpr + 1) + e % vpr] = v[t];
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    int u[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) u[q] = live ? a.init8[r] : 0;
    if (live) {
      const int4* xr = tile + lane * (vpr + 1);
      int4 xw[VPR];
#pragma unroll
      for (int i = 0; i < VPR; ++i) xw[i] = xr[i];
#pragma unroll
      for (int i = 0; i < VPR; ++i) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          u[q] = __builtin_amdgcn_sdot4(xw[i].x, s_q8[q][4 * i + 0], u[q], false);
          u[q] = __builtin_amdgcn_sdot4(xw[i].y, s_q8[q][4 * i + 1], u[q], false);
          u[q] = __builtin_amdgcn_sdot4(xw[i].z, s_q8[q][4 * i + 2], u[q], false);
          u[q] = __builtin_amdgcn_sdot4(xw[i].w, s_q8[q][4 * i + 3], u[q], false);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();  // every lane has read its row before the next tile
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if (q >= a.nq) break;
      // stage the keys below the wave's current kp-th key; insert 64 at a time
      const float key = float(-M * u[q]);
      const float td = __shfl(top[q].k.d[0], rl);
      const uint32_t ti = __shfl(top[q].k.id[0], rl);
      const bool want = live && nb_less(key, r, td, ti);
      const uint64_t bal = __ballot(want);
      if (bal == 0) continue;
      const int pos = staged[q] + __popcll(bal & ((1ull << lane) - 1ull));
      if (want) {
        sd[wave][q][pos] = key;
        si[wave][q][pos] = r;
      }
      staged[q] += __popcll(bal);
      if (staged[q] >= kWave) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const float d0 = sd[wave][q][lane];
        const uint32_t i0 = si[wave][q][lane];
        const bool more = lane + kWave < staged[q];
        const float d1 = more ? sd[wave][q][lane + kWave] : 0.f;
        const uint32_t i1 = more ? si[wave][q][lane + kWave] : 0u;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (more) {
          sd[wave][q][lane] = d1;
          si[wave][q][lane] = i1;
        }
        staged[q] -= kWave;
        top[q].insert(d0, i0);
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    if (q >= a.nq) break;
    if (staged[q] > 0) {
      const bool have = lane < staged[q];
      top[q].insert(have ? sd[wave][q][lane] : __builtin_inff(), have ? si[wave][q][lane] : kNoId);
    }
    if (wave > 0) {
      md[wave - 1][q][lane] = top[q].k.d[0];
      mi[wave - 1][q][lane] = top[q].k.id[0];
    }
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    if (q >= a.nq) break;
    for (int w = 0; w < kTinyWaves - 1; ++w) top[q].insert(md[w][q][lane], mi[w][q][lane]);
    const size_t o = size_t(q) * a.nchunks + blockIdx.x;
    if (lane < a.kp) a.part[o * a.kp + lane] = make_uint2(__float_as_uint(top[q].k.d[0]), top[q].k.id[0]);
    const float kth = __shfl(top[q].k.d[0], rl);
    const uint32_t kid = __shfl(top[q].k.id[0], rl);
    if (lane == 0) a.bound[o] = kid == kNoId ? __builtin_inff() : kth;
  }
}

// ================================================================ small batches
//
// More than kTinyQ and at most kSmallQ queries over the same rows: k_small_scan replaces
// k_tiny_scan ahead of the same merge.  Each wave walks its own range of rows in 32-row
// blocks and scores them against every query at once on int8 MFMA
// (v_mfma_i32_32x32x32_i8, k_gemm8's operand layout: lane l holds 16 bytes of row l % 32 and
// of query l % 32, dims 16 (l / 32) + 32 kb onward; its 16 outputs are rows 8 (r / 4) +
// 4 (l / 32) + r % 4 of the block against query l % 32).  The row bytes load straight from
// memory in that layout, two blocks ahead of the one multiplied, and the accumulators start
// from the rows' init8, so u and the key -M u are k_tiny_scan's.  Every lane keeps the
// kSmallKp smallest (key, row) of the rows it scores for its query, sorted.  The two lanes
// of a query in a wave merge their lists into one of kSmallKp (a row either dropped is at
// least its own list's last key, which is at least the merged list's last), and the block's
// four waves' lists merge into the block's chunk of kSmallBlockKp keys, whose bound is the
// smaller of that list's last key and every full wave list's last: every row the block
// left out has a key at least its chunk's bound, so k_tiny_merge's certificate holds as it
// does over k_tiny_scan's chunks.
constexpr int kSmallQ = 32;
constexpr int kSmallKp = 4;      // keys a lane keeps
constexpr int kSmallBlockKp = 8; // keys a block's chunk keeps
constexpr int kSmallWaves = 4;

// Inserts (key, row) into a sorted list of L whose last entry it beats: into the last slot,
// then up to its place.
template <int L>
__device__ __forceinline__ void small_push(float (&kd)[L], uint32_t (&ki)[L], float key,
                                           uint32_t row) {
  kd[L - 1] = key;
  ki[L - 1] = row;
#pragma unroll
  for (int s = L - 1; s > 0; --s) {
    const bool sw = nb_less(kd[s], ki[s], kd[s - 1], ki[s - 1]);
    const float td = kd[s];
    const uint32_t ti = ki[s];
    kd[s] = sw ? kd[s - 1] : kd[s];
    ki[s] = sw ? ki[s - 1] : ki[s];
    kd[s - 1] = sw ? td : kd[s - 1];
    ki[s - 1] = sw ? ti : ki[s - 1];
  }
}

// A scored 32-row block into the lane's list: value r is row rb + 8 (r / 4) + 4 h + r % 4,
// its key -M u.  Every lane publishes its list's last key in LDS (thr[query][list], one
// list per half-wave of each of the block's waves) and a value is a candidate only when its
// key is at most the smallest of the query's eight published keys T: a row above a full
// list's last key is above that wave's merged list's last key, hence above the chunk's
// bound, so dropping it keeps the certificate (a stale published key is larger, so it
// drops less).  In u, key <= T is u >= ceil(-T / M), one integer compare per value.  The
// candidates form a 16-bit mask and only its set bits are pushed (their value picked by a
// select tree), each checked again against the lane's own list as it tightens.
template <class V16>
__device__ __forceinline__ void small_take(const TinyArgs& a, const V16& acc, uint32_t rb,
                                           uint32_t r1, int h, int M, bool qlive,
                                           float (&kd)[kSmallKp], uint32_t (&ki)[kSmallKp],
                                           float* thr, int j, int slot) {
  thr[slot] = kd[kSmallKp - 1];
  const float4 t0 = *reinterpret_cast<const float4*>(thr + 8 * j);
  const float4 t1 = *reinterpret_cast<const float4*>(thr + 8 * j + 4);
  const float T = fminf(fminf(fminf(t0.x, t0.y), fminf(t0.z, t0.w)),
                        fminf(fminf(t1.x, t1.y), fminf(t1.z, t1.w)));
  // keys are -M u for integers u (|u| < 2^24), so -T / M is exact when T is finite
  const int tu = T == __builtin_inff() ? INT_MIN : int(ceilf(-T / float(M)));
  int m = acc[0];
#pragma unroll
  for (int r = 1; r < 16; ++r) m = max(m, acc[r]);
  if (__ballot(qlive && m >= tu) == 0) return;
  const bool whole = rb + 32u <= r1 && a.allow == nullptr;  // every row in range and allowed
  const uint32_t hb = rb + uint32_t(4 * h);
  uint32_t mask = 0;
  if (qlive) {
#pragma unroll
    for (int r = 0; r < 16; ++r) mask |= acc[r] >= tu ? 1u << r : 0u;
    if (!whole) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t row = hb + uint32_t(8 * (r >> 2) + (r & 3));
        if (!(row < r1 && row_allowed(a.allow, row))) mask &= ~(1u << r);
      }
    }
  }
  while (mask != 0) {
    const int r = __builtin_ctz(mask);
    mask &= mask - 1u;
    // acc[r] by the bits of r: a tree of register selects, each result pinned so that the
    // tree is not folded into a dynamic index (which would go through scratch memory)
    auto pick = [](bool c, int x1, int x0) __attribute__((always_inline)) {
      int v = c ? x1 : x0;
      asm volatile("" : "+v"(v));
      return v;
    };
    const bool b0 = r & 1, b1 = r & 2, b2 = r & 4, b3 = r & 8;
    const int p0 = pick(b0, acc[1], acc[0]), p1 = pick(b0, acc[3], acc[2]);
    const int p2 = pick(b0, acc[5], acc[4]), p3 = pick(b0, acc[7], acc[6]);
    const int p4 = pick(b0, acc[9], acc[8]), p5 = pick(b0, acc[11], acc[10]);
    const int p6 = pick(b0, acc[13], acc[12]), p7 = pick(b0, acc[15], acc[14]);
    const int q0 = pick(b1, p1, p0), q1 = pick(b1, p3, p2), q2 = pick(b1, p5, p4),
              q3 = pick(b1, p7, p6);
    const int s0 = pick(b2, q1, q0), s1 = pick(b2, q3, q2);
    const int u = pick(b3, s1, s0);
    const float key = float(-M * u);
    const uint32_t row = hb + uint32_t(8 * (r >> 2) + (r & 3));
    if (nb_less(key, row, kd[kSmallKp - 1], ki[kSmallKp - 1])) small_push(kd, ki, key, row);
  }
}

// The two half-wave lists of a query into one (a row either half dropped is at least that
// half's last key, hence at least the merged list's last), then the block's four waves'
// lists into the block's list of kSmallBlockKp, written as the block's chunk.  A row a
// wave dropped is at least that wave's last key and a key the block dropped at least the
// block list's last, so the chunk's bound is the smaller of the block list's last key and
// every full wave list's last (+inf when neither holds).  bk / bi: LDS for
// kSmallWaves x 32 lists, free of other use.
__device__ __forceinline__ void small_finish(const TinyArgs& a, float (&kd)[kSmallKp],
                                             uint32_t (&ki)[kSmallKp], int j, int h, int wave,
                                             bool qlive, float* bk, uint32_t* bi) {
  float od[kSmallKp];
  uint32_t oi[kSmallKp];
#pragma unroll
  for (int s = 0; s < kSmallKp; ++s) {
    od[s] = __shfl_xor(kd[s], 32);
    oi[s] = __shfl_xor(ki[s], 32);
  }
  if (h == 0) {
#pragma unroll
    for (int s = 0; s < kSmallKp; ++s)
      if (oi[s] != kNoId && nb_less(od[s], oi[s], kd[kSmallKp - 1], ki[kSmallKp - 1]))
        small_push(kd, ki, od[s], oi[s]);
#pragma unroll
    for (int s = 0; s < kSmallKp; ++s) {
      bk[(wave * 32 + j) * kSmallKp + s] = kd[s];
      bi[(wave * 32 + j) * kSmallKp + s] = ki[s];
    }
  }
  __syncthreads();
  if (wave != 0 || h != 0 || !qlive) return;
  float md[kSmallBlockKp];
  uint32_t mi[kSmallBlockKp];
#pragma unroll
  for (int s = 0; s < kSmallBlockKp; ++s) {
    md[s] = s < kSmallKp ? kd[s] : __builtin_inff();
    mi[s] = s < kSmallKp ? ki[s] : kNoId;
  }
  float wb = ki[kSmallKp - 1] == kNoId ? __builtin_inff() : kd[kSmallKp - 1];
  for (int w = 1; w < kSmallWaves; ++w) {
    const int o = (w * 32 + j) * kSmallKp;
    if (bi[o + kSmallKp - 1] != kNoId) wb = fminf(wb, bk[o + kSmallKp - 1]);
#pragma unroll
    for (int t = 0; t < kSmallKp; ++t) {
      const float key = bk[o + t];
      const uint32_t row = bi[o + t];
      if (row != kNoId && nb_less(key, row, md[kSmallBlockKp - 1], mi[kSmallBlockKp - 1]))
        small_push(md, mi, key, row);
    }
  }
  const size_t o = size_t(j) * a.nchunks + blockIdx.x;  // the block's chunk of this query
#pragma unroll
  for (int s = 0; s < kSmallBlockKp; ++s)
    a.part[o * kSmallBlockKp + s] = make_uint2(__float_as_uint(md[s]), mi[s]);
  a.bound[o] = fminf(wb, mi[kSmallBlockKp - 1] == kNoId ? __builtin_inff()
                                                        : md[kSmallBlockKp - 1]);
}

// The query's int8 bytes in the MFMA B layout (q - c8 clamped: a query outside the window
// fails the merge's fitness test and is re-scanned exactly).
template <int NKB, class V4>
__device__ __forceinline__ void small_query(const TinyArgs& a, int j, int h, V4 (&qv)[NKB]) {
  const float* qr = a.Q + size_t(min(j, a.nq - 1)) * a.pd + 16 * h;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint32_t packed = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const float d = qr[32 * kb + 4 * t + b] - float(a.c8);
        packed |= uint32_t(uint8_t(int8_t(int(fminf(fmaxf(d, -128.f), 127.f))))) << (8 * b);
      }
      qv[kb][t] = int(packed);
    }
}

// Each wave's blocks load into registers two blocks ahead of the one multiplied (three
// block buffers with fixed roles in a three-way unrolled loop: no copies between them).
// Blocks per CU of k_small_scan (its launch bounds): three up to 128 dims, two at 256.
constexpr int SmallOccupancy(int pd) { return pd <= 128 ? 3 : 2; }

template <int NKB>
__global__ __launch_bounds__(kSmallWaves * 64, SmallOccupancy(NKB * 32)) void k_small_scan(
    TinyArgs a) {
  typedef int v4i __attribute__((ext_vector_type(4)));
  typedef int v16i __attribute__((ext_vector_type(16)));
  const int tid = threadIdx.x, wave = tid >> 6, lane = lane_id();
  if (blockIdx.x == 0 && tid < 2) a.fb_count[tid] = 0;
  if (blockIdx.x == 0 && tid == 0 && a.fb_zero != nullptr) *a.fb_zero = 0;
  const int j = lane & 31, h = lane >> 5;
  const int M = a.metric == 0 ? 2 : 1;
  const bool qlive = j < a.nq;
  constexpr int PD = NKB * 32;
  // each list's last key, published for the block's threshold per query (see small_take)
  __shared__ __align__(16) float s_thr[32 * 2 * kSmallWaves];
  if (tid < 32 * 2 * kSmallWaves) s_thr[tid] = __builtin_inff();
  __syncthreads();
  const uint32_t gw = blockIdx.x * kSmallWaves + wave;  // the wave's range of rows
  const uint32_t r0 = min(a.N, gw * a.chunk_rows), r1 = min(a.N, r0 + a.chunk_rows);
  v4i qv[NKB];  // the queries, packed once the first rows are on their way
  float kd[kSmallKp];
  uint32_t ki[kSmallKp];
#pragma unroll
  for (int s = 0; s < kSmallKp; ++s) {
    kd[s] = __builtin_inff();
    ki[s] = kNoId;
  }
  // one block's row fragments and accumulator starts (rows past the end read the last row;
  // they are not live)
  struct Blk {
    v4i x[NKB];
    int4 n[4];
  };
  auto load = [&](Blk& B, uint32_t rb) {
    const uint32_t ra = min(rb + uint32_t(j), a.N - 1);
    const int8_t* xr = a.X8 + size_t(ra) * PD + 16 * h;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) B.x[kb] = *reinterpret_cast<const v4i*>(xr + 32 * kb);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t rg = rb + uint32_t(8 * g + 4 * h);
      if (rg + 3 < a.N) {
        B.n[g] = *reinterpret_cast<const int4*>(a.init8 + rg);
      } else {
        B.n[g] = make_int4(a.init8[min(rg, a.N - 1)], a.init8[min(rg + 1, a.N - 1)],
                           a.init8[min(rg + 2, a.N - 1)], a.init8[min(rg + 3, a.N - 1)]);
      }
    }
  };
  const int nblk = int((r1 - r0 + 31) / 32);
  auto compute = [&](const Blk& B, int b) __attribute__((always_inline)) {
    const uint32_t rb = r0 + uint32_t(b) * 32;
    v16i acc;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      acc[4 * g + 0] = B.n[g].x;
      acc[4 * g + 1] = B.n[g].y;
      acc[4 * g + 2] = B.n[g].z;
      acc[4 * g + 3] = B.n[g].w;
    }
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
      acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(B.x[kb], qv[kb], acc, 0, 0, 0);
    small_take(a, acc, rb, r1, h, M, qlive, kd, ki, s_thr, j, 8 * j + 2 * wave + h);
  };
  Blk B0, B1, B2;
  if (nblk > 0) load(B0, r0);
  if (nblk > 1) load(B1, r0 + 32);
  // the queries pack while the first rows load
  small_query<NKB>(a, j, h, qv);
  for (int b = 0; b < nblk; b += 3) {
    if (b + 2 < nblk) load(B2, r0 + uint32_t(b + 2) * 32);
    compute(B0, b);
    if (b + 1 >= nblk) break;
    if (b + 3 < nblk) load(B0, r0 + uint32_t(b + 3) * 32);
    compute(B1, b + 1);
    if (b + 2 >= nblk) break;
    if (b + 4 < nblk) load(B1, r0 + uint32_t(b + 4) * 32);
    compute(B2, b + 2);
  }
  __shared__ float bk[kSmallWaves * 32 * kSmallKp];
  __shared__ uint32_t bi[kSmallWaves * 32 * kSmallKp];
  small_finish(a, kd, ki, j, h, wave, qlive, bk, bi);
}

constexpr int kMergeWaves = 8;  // key-merging waves of k_tiny_merge (plus one preparing)

struct TinyMergeArgs {
  PrepArgs pa;            // the query's operands and bound (fit8q set)
  const uint2* part;
  const float* bound;
  int nchunks, kp, k;
  FlatScorer8 sc;         // the rows and their int8 copy (the re-scoring reads the copy)
  uint32_t* out_ids;
  float* out_d;
  uint32_t* fb_list;
  uint32_t* fb_count;     // [0] fallbacks, [1] finished merges
  uint32_t* host_flag;    // nullable: pinned host words ([0] sequence, [1] fallback count)
                          // the last merge publishes the count into
  uint32_t seq;
  int force_fallback;
};

// One block of 8 + 1 waves per query.  Each of 8 waves loads its share of the chunks' keys
// with all loads in flight (up to 32 per lane at a time) and keeps the 64 best (staged, then
// inserted 64 at a time); the ninth prepares the query's operands and bound meanwhile.  The
// 8 sorted lists merge in a three-level tree of bitonic merges into wave 0, which then
// re-scores and certifies.
__global__ __launch_bounds__(kMergeWaves * 64 + 64) void k_tiny_merge(TinyMergeArgs a) {
  constexpr int W = kMergeWaves;  // waves that merge keys; wave W prepares the query
  constexpr int B = 8;   // keys per lane of a group
  constexpr int G = 4;   // groups in flight: 32 keys per lane (all of them, for k up to ~30)
  __shared__ float md[W][kWave];      // the waves' sorted lists, handed down the merge tree
  __shared__ uint32_t mi[W][kWave];
  __shared__ float s_lb[W];
  __shared__ float sd[W][(B + 1) * kWave];  // staged keys: below 64 left over + a group's
  __shared__ uint32_t si[W][(B + 1) * kWave];
  __shared__ uint32_t ys[256];  // the query packed into int8 (Int8Query)
  const int q = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = lane_id();
  WaveTopK<1> top;
  top.init();
  float lb = __builtin_inff();
  const bool keys = wave < W;
  const int per = (a.nchunks + W - 1) / W;
  const int c0 = keys ? min(a.nchunks, wave * per) : a.nchunks, c1 = min(a.nchunks, c0 + per);
  const size_t total = size_t(c1 - c0) * a.kp;
  const uint2* src = a.part + (size_t(q) * a.nchunks + c0) * a.kp;
  constexpr size_t kGroup = size_t(B) * kWave;
  auto load_keys = [&](size_t g0, uint2 (&v)[B]) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const size_t g = g0 + size_t(b) * kWave + lane;
      v[b] = g < total ? src[g] : make_uint2(__float_as_uint(__builtin_inff()), kNoId);
    }
  };
  // every key of the first round in flight before any is used
  uint2 v0[B], v1[B], v2[B], v3[B];
  load_keys(0, v0);
  load_keys(kGroup, v1);
  load_keys(2 * kGroup, v2);
  load_keys(3 * kGroup, v3);
  // Wave W prepares the query's operands and bound (shift, eb, Qd, fit8q, and the exact
  // fallback's inputs) while the others merge keys; wave 0 reads them after the merge's
  // barriers.  Wave 0 also packs the query for the re-scoring now: its loads go out behind
  // the keys, so the round trip overlaps theirs.
  if (wave == W) (void)query_prep_wave(a.pa, q);
  const float* qv = a.pa.Q + size_t(q) * a.pa.pd;
  Int8Query p8{0, 0, ys};
  if (wave == 0)
    p8 = int8_query(a.sc.X8, a.sc.c8, a.sc.xlo, a.sc.xhi, a.sc.xmax, a.sc.xint, a.sc.metric,
                    a.sc.pd, qv, ys);
  // Every chunk holds kp keys at or below its bound, so the best kp keys of all lie at or
  // below the smallest bound LB: keys above it are skipped.
#pragma unroll 4
  for (int ch = c0 + lane; ch < c1; ch += kWave) lb = fminf(lb, a.bound[size_t(q) * a.nchunks + ch]);
  lb = wave_min(lb);
  if (lane == 0 && keys) s_lb[wave] = lb;
  __syncthreads();
  float LB = s_lb[0];
  for (int w = 1; w < W; ++w) LB = fminf(LB, s_lb[w]);
  // the key to beat: the (k + 9)-th (the certificate reads the key after the k + 8 scored).
  // A group stages its keys below LB and below the list's current (k + 9)-th key (read once
  // per group: it only tightens, so a stale one admits more keys, never fewer); the staged
  // keys then go into the list 64 at a time and fewer than 64 stay staged.
  const int rl = (a.k + 9 - 1) & (kWave - 1);
  int staged = 0;
  auto group = [&](const uint2 (&v)[B]) __attribute__((always_inline)) {
    const float td = __shfl(top.k.d[0], rl);
    const uint32_t ti = __shfl(top.k.id[0], rl);
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const bool want = v[b].y != kNoId && __uint_as_float(v[b].x) <= LB &&
                        nb_less(__uint_as_float(v[b].x), v[b].y, td, ti);
      const uint64_t bal = __ballot(want);
      if (want) {
        const int pos = staged + __popcll(bal & ((1ull << lane) - 1ull));
        sd[wave][pos] = __uint_as_float(v[b].x);
        si[wave][pos] = v[b].y;
      }
      staged += __popcll(bal);
    }
    if (staged < kWave) return;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int base = 0;
    for (; base + kWave <= staged; base += kWave) top.insert(sd[wave][base + lane], si[wave][base + lane]);
    const int rest = staged - base;
    const float dr = lane < rest ? sd[wave][base + lane] : 0.f;
    const uint32_t ir = lane < rest ? si[wave][base + lane] : 0u;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < rest) {
      sd[wave][lane] = dr;
      si[wave][lane] = ir;
    }
    staged = rest;
  };
  for (size_t g0 = 0; g0 < total; g0 += G * kGroup) {
    if (g0 > 0) {
      load_keys(g0, v0);
      load_keys(g0 + kGroup, v1);
      load_keys(g0 + 2 * kGroup, v2);
      load_keys(g0 + 3 * kGroup, v3);
    }
    group(v0);
    group(v1);
    group(v2);
    group(v3);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (staged > 0) {
    const bool have = lane < staged;
    top.insert(have ? sd[wave][lane] : __builtin_inff(), have ? si[wave][lane] : kNoId);
  }
  // Tree merge: at level L the waves w with w % 2L == L hand their lists to waves w - L,
  // which keep the 64 smallest of both (the partner's list reversed against their own is
  // a bitonic sequence holding them), so wave 0 ends with the best 64 of all, sorted.  A
  // wave hands its list down once, to a slot no wave reads at any other level.
#pragma unroll
  for (int L = 1; L < W; L <<= 1) {
    if (keys && (wave & (2 * L - 1)) == L) {
      md[wave][lane] = top.k.d[0];
      mi[wave][lane] = top.k.id[0];
    }
    __syncthreads();
    if (keys && (wave & (2 * L - 1)) == 0) {
      const float pd = md[wave + L][kWave - 1 - lane];
      const uint32_t pi = mi[wave + L][kWave - 1 - lane];
      if (nb_less(pd, pi, top.k.d[0], top.k.id[0])) {
        top.k.d[0] = pd;
        top.k.id[0] = pi;
      }
      bitonic_merge<1>(top.k);
    }
  }
  if (wave != 0) return;
  const float shift = a.pa.shift[q], eb = a.pa.eb[q];
  const float Qd = float(a.pa.Qd[q]);
  const bool fits = a.pa.fit8q[q] != 0;
  lb = __builtin_inff();
  for (int w = 0; w < W; ++w) lb = fminf(lb, s_lb[w]);
  // exact re-scoring of the best n1 keys, certificate against every unscored row
  // (rows of 128 bytes from the int8 copy: their loads issue together, where the fp32
  // rows' 512 bytes per lane form a chain of dependent load rounds)
  const int n1 = min(kWave - 1, a.k + 8);
  float d = __builtin_inff();
  uint32_t id = kNoId;
  if (lane < n1 && top.k.id[0] != kNoId) {
    id = top.k.id[0];
    d = p8.on ? int8_distance(a.sc.X8, a.sc.c8, a.sc.metric, a.sc.pd, p8, id) : a.sc(qv, id);
  }
  WaveKeys<1> r;
  r.d[0] = d;
  r.id[0] = id;
  bitonic_sort<1>(r);
  const float dk = __shfl(r.d[0], a.k - 1);
  const float next = __shfl(top.k.d[0], n1);   // the (n1+1)-th key (+inf when none)
  const float lower = (fminf(next, lb) - Qd + shift) - eb;
  // every row scored (fewer keys than n1 + 1 and no full chunk): the answer is complete
  const bool all_scored = next == __builtin_inff() && lb == __builtin_inff();
  const bool certified = fits && a.force_fallback == 0 && (dk < lower || all_scored);
  if (lane < a.k) {
    a.out_ids[size_t(q) * a.k + lane] = r.id[0];
    a.out_d[size_t(q) * a.k + lane] = r.d[0];
  }
  if (lane == 0) {
    if (!certified) a.fb_list[atomicAdd(a.fb_count, 1u)] = uint32_t(q);
    if (a.host_flag == nullptr) return;  // the re-scan is gated on the device count
    __threadfence();
    if (atomicAdd(a.fb_count + 1, 1u) == uint32_t(gridDim.x - 1)) {
      // the last merge: publish the fallback count (seq written last, with release)
      a.host_flag[1] = __hip_atomic_load(a.fb_count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __threadfence_system();
      __hip_atomic_store(a.host_flag, a.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

// The rank r of the sample's group minimum that becomes the admission threshold.  The sample
// holds a fraction f = S / N of the rows, spread evenly; the r-th smallest group minimum
// lies below the kk-th smallest GEMM value of all rows only when the sample holds at least
// r of the kk - 1 rows before it, which for rows taken independently with probability f is
// the binomial tail P(Bin(kk - 1, f) >= r).  r is the smallest rank with that tail below
// 1e-6 (at most kk, which keeps the top kk with certainty).  About r / f rows then pass the
// threshold per query instead of kk / f; k_select's certificate catches the rare query
// whose threshold fell short, and the second chance and the exact re-scan answer it.
static int ThresholdRank(size_t kk, uint32_t S, uint32_t N) {
  if (kk <= 1 || S >= N) return int(kk);
  const double f = double(S) / double(N), n = double(kk - 1);
  const double lf = std::log(f), lg = std::log1p(-f);
  double cdf = 0.0;  // P(Bin(n, f) < r)
  for (size_t r = 1; r < kk; ++r) {
    const double j = double(r - 1);
    cdf += std::exp(std::lgamma(n + 1.0) - std::lgamma(j + 1.0) - std::lgamma(n - j + 1.0) +
                    j * lf + (n - j) * lg);
    if (1.0 - cdf <= 1e-6) return int(r);
  }
  return int(kk);
}

// Whether a batch takes the tiny-batch path: integer rows with their int8 copy, the int8
// GEMM on, at most kSmallQ queries (k_tiny_scan up to kTinyQ, k_small_scan above),
// k <= kTinyK, rows of 64, 128 or 256 dims.
static bool TinyEligible(const Ctx* c, const ScanSource& src, size_t nq, size_t kk,
                         const Workspace& w) {
  return nq >= 1 && nq <= size_t(kSmallQ) && kk <= size_t(kTinyK) && src.kind == 0 &&
         src.metric <= 1 && src.X8 != nullptr && src.x8_parts == 1 && src.init8 != nullptr &&
         c->fp16_gemm && c->int8_gemm && src.x16_parts == 1 && !src.x16_approx &&
         (src.pd == 64 || src.pd == 128 || src.pd == 256) && src.N >= 1024 && !w.fixed;
}

template <int NQ>
static void launch_tiny(hipStream_t s, int blocks, const TinyArgs& a) {
  const size_t tile = size_t(kTinyWaves) * kWave * (a.pd / 16 + 1) * sizeof(int4);
  const int threads = kTinyWaves * 64;
  switch (a.pd) {
    case 64: k_tiny_scan<NQ, 4><<<dim3(blocks), threads, tile, s>>>(a); break;
    case 128: k_tiny_scan<NQ, 8><<<dim3(blocks), threads, tile, s>>>(a); break;
    default: k_tiny_scan<NQ, 16><<<dim3(blocks), threads, tile, s>>>(a); break;
  }
}

static void launch_small(hipStream_t s, int blocks, const TinyArgs& a) {
  switch (a.pd) {
    case 64: k_small_scan<2><<<dim3(blocks), kSmallWaves * 64, 0, s>>>(a); break;
    case 128: k_small_scan<4><<<dim3(blocks), kSmallWaves * 64, 0, s>>>(a); break;
    default: k_small_scan<8><<<dim3(blocks), kSmallWaves * 64, 0, s>>>(a); break;
  }
}

static int TinyScan(Ctx* c, ScanSource* src, const float* Q, size_t nq, size_t kk,
                    const uint64_t* allow, uint32_t* out_ids, float* out_d, hipStream_t s,
                    Workspace& W, Workspace& W2) {
  const uint32_t N = src->N;
  const int pd = int(src->pd);
  // Uncertified queries go to the exact re-scan.  When its scratch for every query of the
  // batch is small (always, at these batch sizes) it is queued for every query and runs for
  // those the merge listed, their count staying on the device (added to the call's count,
  // which the scan's first block clears unless several scans of one call accumulate into
  // it): nothing waits on the host.  Otherwise the merge publishes the count to the host.
  const bool gated = c->gate_fallbacks && PlanExact(N, int(nq), kk).need <= kGatedExactBytes;
  if (!gated) VDBG_RETURN_IF_ERROR(ResetFallbacks(c, s));
  uint32_t* fb_zero = nullptr;
  if (gated && !c->fb_accumulate) {
    c->last_fallbacks = 0;
    fb_zero = c->fb_dev;
  }
  // k_tiny_scan: a chunk of rows per block, kk + 9 keys each.  k_small_scan: a range of
  // rows per wave, each block one chunk of kSmallBlockKp keys per query
  const bool small = nq > size_t(kTinyQ);
  const int kp = small ? kSmallBlockKp : int(kk) + 9;
  // k_small_scan: as many blocks as fit the device at once (one round)
  const int blocks = small ? c->cu_count * SmallOccupancy(pd) : 2 * c->cu_count;
  const uint32_t units = small ? uint32_t(blocks) * kSmallWaves : uint32_t(blocks);
  uint32_t chunk = (N + units - 1) / units;
  chunk = small ? (chunk + 31) / 32 * 32 : (chunk + 255) / 256 * 256;
  const int nchunks = small ? blocks : int((N + chunk - 1) / chunk);
  WsUse wuse(&W, s);
  VDBG_RETURN_IF_ERROR(wuse.status());
  W.used = 0;
  const size_t need = nq * size_t(nchunks) * (size_t(kp) * sizeof(uint2) + sizeof(float)) +
                      nq * (3 * sizeof(float) + 3 * sizeof(int) + 2 * sizeof(uint32_t) + pd) +
                      16 * 256;
  VDBG_RETURN_IF_ERROR(W.reserve(need));
  uint2* part = W.take<uint2>(nq * size_t(nchunks) * kp);
  float* bound = W.take<float>(nq * size_t(nchunks));
  float* shift = W.take<float>(nq);
  float* eb = W.take<float>(nq);
  int* exact = W.take<int>(nq);
  int* Qd = W.take<int>(nq);
  int* fit8q = W.take<int>(nq);
  int8_t* Q8 = W.take<int8_t>(nq * size_t(pd));
  uint32_t* fb_list = W.take<uint32_t>(nq);
  uint32_t* fb_count = W.take<uint32_t>(2);
  c->last_gemm_bits = 8;
  PrepArgs pa{Q, nullptr, int(nq), pd, src->kind, src->metric, src->stats, src->rmag,
              src->vmin, src->scale, shift, eb, exact, nullptr, nullptr, nullptr,
              src->x16_parts, src->x16_exp, Q8, Qd, nullptr, fit8q, src->c8, nullptr};
  TinyArgs ta{Q, int(nq), pd, src->metric, src->c8, int(kk), kp, src->X8, src->init8, allow, N,
              chunk, part, bound, fb_count, nchunks, fb_zero};
  {
    ProfScope ps(c, "flat_gemm", s);
    if (small) launch_small(s, blocks, ta);
    else if (nq == 1) launch_tiny<1>(s, nchunks, ta);
    else launch_tiny<2>(s, nchunks, ta);
    VDBG_HIP(hipGetLastError());
  }
  if (gated) {
    TinyMergeArgs ma{pa, part, bound, nchunks, kp, int(kk), Flat8Of(*src, c->kset), out_ids,
                     out_d, fb_list, fb_count, nullptr, 0u, c->test_fallbacks};
    {
      ProfScope ps(c, "select", s);
      k_tiny_merge<<<dim3(unsigned(nq)), kMergeWaves * 64 + 64, 0, s>>>(ma);
      VDBG_HIP(hipGetLastError());
    }
    VDBG_RETURN_IF_ERROR(ExactScan(c, W2, *src, Q, fb_list, int(nq), kk, allow, out_ids, out_d,
                                   s, fb_count, c->fb_dev));
    c->fb_dev_used = true;
    return kOk;
  }
  uint32_t nfb = 0;
  {  // the merge publishes the fallback count through the context's host flag
    std::lock_guard<std::mutex> g(c->flag_mu);
    const uint32_t seq = NextFlagSeq(c);
    TinyMergeArgs ma{pa, part, bound, nchunks, kp, int(kk), Flat8Of(*src, c->kset), out_ids,
                     out_d, fb_list, fb_count, c->host_flag_dev, seq, c->test_fallbacks};
    {
      ProfScope ps(c, "select", s);
      k_tiny_merge<<<dim3(unsigned(nq)), kMergeWaves * 64 + 64, 0, s>>>(ma);
      VDBG_HIP(hipGetLastError());
    }
    VDBG_RETURN_IF_ERROR(WaitWords(c, seq, fb_count, 1, s));
    nfb = c->host_pinned[0];
  }
  c->last_fallbacks += nfb;
  if (nfb > 0)
    VDBG_RETURN_IF_ERROR(ExactScan(c, W2, *src, Q, fb_list, int(nfb), kk, allow, out_ids, out_d, s));
  return kOk;
}

// The sample size RunScan plans for a batch (before the cap of the source's sample): S >=
// kk * N / P, P = 160 for large batches on the exact GEMMs, 640 otherwise, and at least
// 16 * max(128, 4 kk) rows and N / 64, rounded up to a power of two.
uint32_t SampleWant(const Ctx* c, const ScanSource& src, size_t nq, size_t kk) {
  const uint32_t N = src.N;
  const bool try16 = c->fp16_gemm && src.X16 != nullptr;
  const int split = src.kind == 1 ? 1 : (src.x16_parts == 2 ? 2 : (src.x16_approx ? 3 : 0));
  const uint64_t passes = try16 && split == 0 && nq >= 1024 ? 160 : 640;  // (int8 too)
  const uint64_t s_want = std::max<uint64_t>({16ull * std::max<uint64_t>(128, 4 * kk), N / 64,
                                              uint64_t(N) * kk / passes});
  uint32_t S = 1;
  while (S < s_want && S < (1u << 30)) S *= 2;
  return S;
}

int RunScan(Ctx* c, ScanSource* src, const float* Q, size_t nq, size_t kk,
            const uint64_t* allow, uint32_t* out_ids, float* out_d, hipStream_t s,
            Workspace* ws, Workspace* ws2) {
  Workspace& W = ws != nullptr ? *ws : c->ws;
  Workspace& W2 = ws2 != nullptr ? *ws2 : c->ws2;
  // (the tiny path clears the call's fallback count itself, in its scan kernel)
  const bool tiny = nq > 0 && kk > 0 && kk <= 10000 && src->N > 0 &&
                    GemmSupported(src->pd) && TinyEligible(c, *src, nq, kk, W);
  // the GEMM path clears the device count in its init kernel (no launch of its own)
  const bool main_path = !tiny && nq > 0 && kk > 0 && kk <= 240 && src->N >= 1024 &&
                         GemmSupported(src->pd);
  uint32_t* fb_zero = nullptr;
  if (main_path && !c->fb_accumulate) {
    c->last_fallbacks = 0;
    if (c->fb_dev_used) fb_zero = c->fb_dev;
  } else if (!tiny) {
    VDBG_RETURN_IF_ERROR(ResetFallbacks(c, s));
  }
  c->last_gemm_bits = 0;
  c->last_gemm_gate = nullptr;
  if (nq == 0 || kk == 0) return kOk;
  if (kk > 10000) return SetError(kInvalidArgument, "k must be in 1..10000");
  if (src->N == 0) {
    k_fill_empty<<<dim3(unsigned((nq * kk + 255) / 256)), 256, 0, s>>>(out_ids, out_d, nq * kk);
    VDBG_HIP(hipGetLastError());
    return kOk;
  }
  // the select keeps K' >= kk + 16 keys in one wavefront (at most 256)
  if (kk > 240) return ExactScanAll(c, *src, Q, nq, kk, allow, out_ids, out_d, s);
  const uint32_t N = src->N;
  const size_t pd = src->pd;
  const bool gemm = GemmSupported(pd) && N >= 1024;
  if (!gemm) return ExactScan(c, W, *src, Q, nullptr, int(nq), kk, allow, out_ids, out_d, s);
  if (tiny) return TinyScan(c, src, Q, nq, kk, allow, out_ids, out_d, s, W, W2);
  // A re-scan workspace that cannot grow must hold the re-scan of every query, checked
  // before anything is queued (which queries fall back is known only on the device).
  if (W2.fixed && PlanExact(N, int(nq), kk).need > W2.cap)
    return SetError(kResourceExhausted,
                    std::string(W2.name) + ": the batch's exact re-scan could need " +
                        std::to_string(PlanExact(N, int(nq), kk).need) +
                        " bytes of scratch, more than the " + std::to_string(W2.cap) +
                        " this path holds");
  VDBG_RETURN_IF_ERROR(BuildSample(c, src, s));

  // ---- plan: the fp32 GEMM runs 128 queries per block; the fp16 GEMM 256 (64 per wave,
  // each LDS row fragment feeding two MFMAs), or 128 for batches of at most 128 queries
  const int slots = 2 * c->cu_count;
  const bool try16 = c->fp16_gemm && src->X16 != nullptr;
  // the fp16 GEMM's operand mode (gemm16.hip): exact rows 0, SQ8 codes 1, float rows in two
  // parts 2, float rows as their h halves alone 3 (one fp16 MFMA per product, ranked under
  // the wider bound, replacing both the split and the int8 pass)
  const int split = src->kind == 1 ? 1 : (src->x16_parts == 2 ? 2 : (src->x16_approx ? 3 : 0));
  // integer rows spanning at most 256 values may rank on the int8 GEMM (gemm8.hip)
  const bool try8 = try16 && c->int8_gemm && split == 0 && src->X8 != nullptr;
  // SQ8 codes may rank on the int8 GEMM with the query operand in two int8 parts, float rows
  // with both operands in two parts
  const bool try8s = try16 && c->int8_gemm && src->kind == 1 && Gemm8Supported(pd);
  // (float rows only for GEMMs large enough to repay the batch's operand pass and flag
  // readback: the fp16 split GEMM costs about 2 N nq pd / 2e14 s, the int8 one 0.6 of that)
  const bool single = split == 3 && try16;
  // rows wider than one K chunk keep each wave's query fragments resident (one 32-query
  // block per wave, gemm16.hip QRES); the sample pass keeps two blocks per wave
  const bool wide16 = single && Gemm16ResQueries(pd);
  const bool try8f = c->fp16_gemm && c->int8_gemm && split == 2 &&
                     src->X8 != nullptr && src->x8_parts == 2 && Gemm8Supported(pd) &&
                     double(N) * double(nq) * double(pd) >= c->int8_float_min_work;
  const bool try8op = try8s || try8f;  // the two-part query operand (k_sq8_operand8)
  const bool try8any = try8 || try8op;
  const int sq8 = try8s ? 1 : (try8f ? 2 : 0);
  // Sample size: every row passing the threshold costs a scattered buffer write and a select
  // insertion (and on the exact fp16 and int8 GEMMs every 32-row block holding one takes the
  // per-value test), while the pre-pass costs S / N of the main GEMM.  S >= kk * N / P until
  // the sample cap: P = 160 for large batches on the exact GEMMs, whose MFMA work per row is
  // smallest, 640 otherwise (N / 64 at k = 10).  (Measured at 1M x 128, k = 10, on the int8
  // GEMM: a 16,384-row sample saved 0.07 ms of pre-pass but its threshold admitted ~300 rows
  // per query instead of ~110, and the main pass and select lost 0.17 ms.)
  uint32_t S = SampleWant(c, *src, nq, kk);
  // Small batches of integer rows (at most 128 queries) choose between the int8 and the
  // fp32 main pass on the device (no host round trip before the main pass).
  const bool gated = nq <= 128 && split == 0 && try8 && !try8op;
  S = std::min(S, src->Smax);
  // the sample's positions spread over its first SN rows (an appendable dataset's sample
  // may trail its rows): a top row there is sampled with probability S / SN, one past
  // them never, so the tail bound takes f = S / SN
  const int rank = ThresholdRank(kk, S, std::min(N, src->SN != 0 ? src->SN : N));
  const int ngroups = int((S + 31) / 32) * 2;
  struct Plan {
    int qb, nqt, nchunks, caph, nseg, schunks;
    int snqt;  // query tiles of the sample pass
    uint32_t chunk_rows, schunk_rows;
  };
  auto make_plan = [&](int qb, int tile_queries, int slots, int max_chunks = kMaxSeg / 2,
                       int sample_tile = 0) {
    Plan p{};
    p.qb = qb;
    p.nqt = int((nq + tile_queries - 1) / tile_queries);
    p.snqt = sample_tile ? int((nq + sample_tile - 1) / sample_tile) : p.nqt;
    p.nchunks = PlanChunks(p.nqt, N, slots, max_chunks);
    p.chunk_rows = (N + p.nchunks - 1) / p.nchunks;
    p.chunk_rows = (p.chunk_rows + 63) / 64 * 64;
    p.nchunks = int((N + p.chunk_rows - 1) / p.chunk_rows);
    p.schunks = PlanChunks(p.snqt, S, slots, int((S + 63) / 64));
    p.schunk_rows = (S + p.schunks - 1) / p.schunks;
    p.schunk_rows = (p.schunk_rows + 63) / 64 * 64;
    p.schunks = int((S + p.schunk_rows - 1) / p.schunk_rows);
    const double expect_seg = double(rank) * N / S * 2.0 / (2.0 * p.nchunks);
    p.caph = 32;
    while (p.caph < 3.0 * expect_seg + 32) p.caph <<= 1;
    p.nseg = 2 * p.nchunks;
    return p;
  };
  // Rows with an fp16 copy may rank on the fp16 GEMM: integer-valued flat rows exactly
  // (64 queries per wave, or 32 for batches of at most 128), SQ8 codes with the query operand
  // split in two fp16 parts (both register sets hold the same 32 queries).  The int8 GEMM
  // tiles as the exact fp16 one, its large-batch kernel with Gemm8Occupancy blocks per CU.
  const int slots8 = (try8op ? (try8f ? 2 : Gemm8Occupancy(pd)) : Gemm8Occupancy(pd)) * c->cu_count;
  auto plan_all = [&](Plan* p32, Plan* p16, Plan* p8, int max_chunks) {
    *p32 = make_plan(1, 128, slots, max_chunks);
    *p16 = wide16  ? make_plan(1, 128, slots, max_chunks, 256)
           : single ? make_plan(2, 256, slots, max_chunks)
           : split ? make_plan(2, 128, slots, max_chunks)
                   : (nq > 128 ? make_plan(2, 256, slots, max_chunks)
                               : make_plan(1, 128, slots, max_chunks));
    *p8 = try8op ? make_plan(2, 128, slots8, max_chunks)
                 : (nq > 128 ? make_plan(2, 256, slots8, max_chunks) : *p16);
  };
  Plan p32, p16, p8;
  plan_all(&p32, &p16, &p8, kMaxSeg / 2);
  auto cand_bytes = [&](const Plan& p) {
    return size_t(nq) * p.nseg * (sizeof(uint32_t) + size_t(p.caph) * sizeof(uint2));
  };
  // counts then candidates, the candidates 256-byte aligned
  auto cand_total = [&]() {
    return std::max({cand_bytes(p32), try16 ? cand_bytes(p16) : 0,
                     try8any ? cand_bytes(p8) : 0}) + 256;
  };
  size_t cand_need = cand_total();
  const int Esel = pow2_e(kk + 16);
  // The int8 sample pass keeps the kTop8 smallest group minima per lane and chunk half when
  // the lists hold three times kk in all (more than kTop8 of the top kk groups meet in one
  // lane's list only by rare chance, and then the threshold is merely looser); otherwise
  // it keeps every group minimum.
  const int ngroups8 = p8.schunks * 2 * kTop8;
  const bool compact8 = try8any && ngroups8 <= 4096 && uint64_t(ngroups8) >= 3 * kk;
  const int gm_groups = std::max(ngroups, compact8 ? ngroups8 : 0);

  Workspace& w = W;
  // launches of an earlier call on another stream may still read this workspace
  WsUse wuse(&w, s);
  VDBG_RETURN_IF_ERROR(wuse.status());
  w.used = 0;
  const size_t other_need =
      nq * (4 * sizeof(float) + 2 * sizeof(int) + 2 * sizeof(uint32_t)) +
      (src->kind == 1 ? nq * pd * sizeof(float) : 0) + size_t(nq) * gm_groups * sizeof(float) +
      (try16 ? (split ? 2 : 1) * nq * pd * sizeof(uint16_t) + nq * sizeof(float) : 0) +
      (try8 ? nq * pd + nq * sizeof(int) : 0) +
      (try8op ? 2 * nq * pd + nq * (sizeof(int) + sizeof(float)) : 0) + 26 * 256;
  // A workspace that cannot grow caps the candidate buffers instead: fewer, longer row
  // chunks (fewer blocks, so a less filled GPU) until they fit in what the rest leaves.
  // The sample pass and everything else are planned as before.
  if (w.fixed && other_need < w.cap && other_need + cand_need > w.cap) {
    int limit = std::max({p32.nchunks, p16.nchunks, p8.nchunks});
    while (limit > 1 && other_need + cand_need > w.cap) {
      limit = std::max(1, limit / 2);
      plan_all(&p32, &p16, &p8, limit);
      cand_need = cand_total();
    }
  }
  const size_t need = other_need + cand_need;
  VDBG_RETURN_IF_ERROR(w.reserve(need));
  float* shift = w.take<float>(nq);
  float* eb = w.take<float>(nq);
  float* T = w.take<float>(nq);
  int* exact = w.take<int>(nq);
  int* ovf = w.take<int>(nq);
  uint32_t* fb_list = w.take<uint32_t>(nq);
  uint32_t* fb_count = w.take<uint32_t>(2);  // [0] first pass, [1] second chance
  uint32_t* fb2_list = w.take<uint32_t>(nq);
  float* Qb = src->kind == 1 ? w.take<float>(nq * pd) : nullptr;
  float* gm = w.take<float>(size_t(nq) * gm_groups);
  char* cand_base = w.take<char>(cand_need);
  uint16_t* Q16 = try16 ? w.take<uint16_t>((split ? 2 : 1) * nq * pd) : nullptr;
  float* Qf = try16 && split ? w.take<float>(nq) : nullptr;
  int* all16 = try16 || try8any ? w.take<int>(2) : nullptr;  // [0] fp16, [1] int8 bounds
  int* all8 = try8any ? all16 + 1 : nullptr;
  int8_t* Q8 = try8any ? w.take<int8_t>((try8op ? 2 : 1) * nq * pd) : nullptr;
  int* Qd = try8any ? w.take<int>(nq) : nullptr;
  float* eb8 = try8op ? w.take<float>(nq) : nullptr;
  int* e8 = try8op ? w.take<int>(2) : nullptr;  // [0] exponent, [1] max |B| bits
  uint32_t* mb8 = try8op ? reinterpret_cast<uint32_t*>(e8 + 1) : nullptr;
  // the no-filter word of the fp16 and int8 GEMMs
  uint32_t* ones = try16 || try8any ? w.take<uint32_t>(1) : nullptr;
  int* fit8q = gated ? w.take<int>(nq) : nullptr;  // per query: inside the int8 bounds
  {
    const ScanInit si{ovf, int(nq), fb_count, all16, ones, try8op ? e8 : nullptr, fb_zero};
    k_scan_init<<<dim3(unsigned((std::max<size_t>(nq, 2) + 255) / 256)), 256, 0, s>>>(si);
    VDBG_HIP(hipGetLastError());
  }

  PrepArgs pa{Q, Qb, int(nq), int(pd), src->kind, src->metric, src->stats, src->rmag,
              src->vmin, src->scale, shift, eb, exact, Q16, all16, Qf, src->x16_parts,
              src->x16_exp, try8 ? Q8 : nullptr, try8 ? Qd : nullptr, try8 ? all8 : nullptr,
              fit8q, src->c8, mb8, single ? 1 : 0};
  {
    ProfScope ps(c, "query_prep", s);
    k_query_prep<<<dim3(unsigned((nq + 3) / 4)), 256, 0, s>>>(pa);
    VDBG_HIP(hipGetLastError());
    if (try8op) {
      Sq8Op8Args oa{try8s ? Qb : Q, int(nq), int(pd), src->metric, mb8,
                    try8s ? src->rn_max : src->stats.xn_max, eb, Q8, Qd, eb8, e8, all8,
                    try8f ? 1 : 0, src->x8_exp, src->x8_l1max, src->x8_l2max};
      k_sq8_operand8<<<dim3(unsigned((nq + 3) / 4)), 256, 0, s>>>(oa);
      VDBG_HIP(hipGetLastError());
    }
  }
  // The exact-integer GEMM needs every query of the batch inside its bounds, so the host
  // reads the flag.  The split operands need no such check: a non-finite query only yields
  // NaN or infinite GEMM values and bound, its certificate fails and it is re-scanned
  // exactly, as on the fp32 GEMM.  Small batches of integer rows make no round trip: the
  // int8 and the fp32 main pass are both queued, gated on the per-query flags (their plans,
  // candidate layout and bound coincide at nq <= 128), and the one they rule out exits.
  bool use16 = try16 && split != 0, use8 = false;
  if (((try16 && split == 0) || try8op) && !gated) {
    uint32_t fl[2];
    VDBG_RETURN_IF_ERROR(ReadWords(c, reinterpret_cast<const uint32_t*>(all16), 2, s, fl));
    use8 = try8any && fl[1] != 0;
    use16 = try16 && !use8 && (split != 0 || fl[0] != 0);
  }
  // a source reading its parent's rows through Xmap ranks on its fp16 copy (no fp32 GEMM)
  if (src->Xmap != nullptr && !use8 && !use16)
    return SetError(kInternal, "scan: remapped fp32 rows on the fp32 GEMM");
  // the bound of the GEMM the batch ranks on
  const float* ebx = use8 && try8op ? eb8 : eb;
  c->last_gemm_bits = use8 ? 8 : (use16 ? 16 : 32);
  c->last_gemm_gate = gated ? fit8q : nullptr;
  c->last_gemm_gate_n = int(nq);
  const Plan& P = use8 ? p8 : (use16 ? p16 : p32);
  const int nchunks = P.nchunks;
  const int caph = P.caph;
  const int nseg = P.nseg;
  uint32_t* counts = reinterpret_cast<uint32_t*>(cand_base);
  uint2* cand = reinterpret_cast<uint2*>(
      cand_base + ((size_t(nq) * nseg * sizeof(uint32_t) + 255) & ~size_t(255)));
  const float* B = src->kind == 1 ? Qb : Q;
  const int metric = src->metric == 0 ? 0 : 1;

  // sample pre-pass -> thresholds
  GemmArgs sg{};
  sg.X = src->SX;
  sg.C = src->SC;
  sg.rn = src->Srn;
  sg.rid = src->Sid;
  sg.Qb = B;
  sg.allow = allow;
  sg.gm = gm;
  sg.ngroups = ngroups;
  const bool top8 = use8 && P.qb == 2 && compact8;
  sg.N = S;
  sg.nq = int(nq);
  sg.chunk_rows = P.schunk_rows;
  int sblocks = 0;
  {
    ProfScope ps(c, "sample_gemm", s);
    if (use8 && P.qb == 2) {
      sg.X8 = try8s ? reinterpret_cast<const int8_t*>(src->SC) : src->SX8;
      sg.rn8 = src->Sinit8;
      sg.Q8 = Q8;
      sg.Qd = Qd;
      sg.e8 = e8;
      GemmGrid(sg, P.snqt, P.schunks, &sblocks);
      if (top8) sg.ngroups = ngroups8;
      VDBG_RETURN_IF_ERROR(LaunchGemm8(pd, metric, 2, top8 ? 2 : 1, sq8, s, sblocks, sg));
    } else if (use16 && (P.qb == 2 || wide16)) {
      sg.X16 = src->SX16;
      sg.Q16 = Q16;
      sg.Qf = Qf;
      GemmGrid(sg, P.snqt, P.schunks, &sblocks);
      VDBG_RETURN_IF_ERROR(LaunchGemm16(pd, metric, 2, 1, split, s, sblocks, sg));
    } else {
      // the fp32 sample pass runs 128-query tiles
      GemmGrid(sg, p32.nqt, p32.schunks, &sblocks);
      sg.chunk_rows = p32.schunk_rows;
      if (gated) {
        // the int8 sample pass when every query fits the int8 GEMM (one 256-query tile
        // covers the batch, so the fp32 plan's sample chunks serve it), else the fp32 one;
        // both write every group minimum (MODE 1)
        GemmArgs s8 = sg;
        s8.X8 = src->SX8;
        s8.rn8 = src->Sinit8;
        s8.Q8 = Q8;
        s8.Qd = Qd;
        s8.gate = fit8q;
        s8.gate_n = int(nq);
        s8.gate_on = 1;
        VDBG_RETURN_IF_ERROR(LaunchGemm8(pd, metric, 2, 1, 0, s, sblocks, s8));
        sg.gate = fit8q;
        sg.gate_n = int(nq);
        sg.gate_on = 0;
      }
      VDBG_RETURN_IF_ERROR(LaunchGemm(pd, metric, src->kind, 1, s, sblocks, sg));
    }
    VDBG_HIP(hipGetLastError());
  }
  KthArgs ka{gm, sg.ngroups, int(nq), rank, ebx, T};
  {
    ProfScope ps(c, "kth", s);
    VDBG_RETURN_IF_ERROR(LaunchKth(s, ka));
    VDBG_HIP(hipGetLastError());
  }

  // main pass
  GemmArgs ga{};
  ga.X = src->X;
  ga.C = src->C;
  ga.rn = src->rn;
  ga.Qb = B;
  ga.T = T;
  ga.allow = allow;
  ga.cand = cand;
  ga.counts = counts;
  ga.ovf = ovf;
  ga.N = N;
  ga.nq = int(nq);
  ga.chunk_rows = P.chunk_rows;
  ga.caph = caph;
  int blocks = 0;
  GemmGrid(ga, P.nqt, nchunks, &blocks);
  {
    ProfScope ps(c, src->kind == 0 ? "flat_gemm" : "sq8_gemm", s);
    if (gated) {
      // the int8 pass when every query fits it, else the fp32 pass (one grid, one plan)
      GemmArgs g8 = ga;
      g8.X8 = src->X8;
      g8.rn8 = src->init8;
      g8.Q8 = Q8;
      g8.Qd = Qd;
      g8.e8 = e8;
      g8.aw = allow != nullptr ? reinterpret_cast<const uint32_t*>(allow) : ones;
      g8.aw_mask = allow != nullptr ? ~0u : 0u;
      g8.gate = fit8q;
      g8.gate_n = int(nq);
      g8.gate_on = 1;
      VDBG_RETURN_IF_ERROR(LaunchGemm8(pd, metric, P.qb, 0, 0, s, blocks, g8));
      ga.gate = fit8q;
      ga.gate_n = int(nq);
      ga.gate_on = 0;
      VDBG_RETURN_IF_ERROR(LaunchGemm(pd, metric, src->kind, 0, s, blocks, ga));
    } else if (use8) {
      ga.X8 = try8s ? reinterpret_cast<const int8_t*>(src->C) : src->X8;
      ga.rn8 = src->init8;
      ga.Q8 = Q8;
      ga.Qd = Qd;
      ga.e8 = e8;
      ga.aw = allow != nullptr ? reinterpret_cast<const uint32_t*>(allow) : ones;
      ga.aw_mask = allow != nullptr ? ~0u : 0u;
      VDBG_RETURN_IF_ERROR(LaunchGemm8(pd, metric, P.qb, 0, sq8, s, blocks, ga));
    } else if (use16) {
      ga.X16 = src->X16;
      ga.Q16 = Q16;
      ga.Qf = Qf;
      ga.aw = allow != nullptr ? reinterpret_cast<const uint32_t*>(allow) : ones;
      ga.aw_mask = allow != nullptr ? ~0u : 0u;
      VDBG_RETURN_IF_ERROR(LaunchGemm16(pd, metric, P.qb, 0, split, s, blocks, ga));
    } else {
      VDBG_RETURN_IF_ERROR(LaunchGemm(pd, metric, src->kind, 0, s, blocks, ga));
    }
    VDBG_HIP(hipGetLastError());
  }
  SelectArgs se{};
  se.Q = Q;
  se.cand = cand;
  se.counts = counts;
  se.nseg = nseg;
  se.cap = caph;
  se.ovf = ovf;
  se.shift = shift;
  se.eb = ebx;
  se.exact = exact;
  se.nslots = int(nq);
  se.k = int(kk);
  se.pd = int(pd);
  se.rescore = 1;
  se.T = T;
  se.out_ids = out_ids;
  se.out_d = out_d;
  se.fb_list = fb_list;
  se.fb_count = fb_count;
  se.force_fallback = c->test_fallbacks;
  {
    ProfScope ps(c, "select", s);
    if (UseFlat8(*src, nq, kk, 1)) {
      VDBG_DISPATCH_ES(Esel, launch_select, FlatScorer8, s, se, Flat8Of(*src, c->kset));
    } else if (src->kind == 0) {
      VDBG_DISPATCH_ES(Esel, launch_select, FlatScorer, s, se, FlatOf(*src, c->kset));
    } else {
      VDBG_DISPATCH_ES(Esel, launch_select, Sq8Scorer, s, se, Sq8Of(*src, c->kset));
    }
    VDBG_HIP(hipGetLastError());
  }
  // Uncertified queries take a second chance (every buffered candidate re-scored) and, if it
  // fails too, the exact re-scan.  When the re-scan's scratch for every query of the batch is
  // small, both passes are queued for every slot and run only for the slots the pass before
  // listed (its count stays on the device): nothing waits on the host.  Otherwise the host
  // reads each count and sizes the pass to it.
  if (c->gate_fallbacks && PlanExact(N, int(nq), kk).need <= kGatedExactBytes) {
    SelectArgs s2 = se;
    s2.qlist = fb_list;
    s2.nslots = int(nq);
    s2.nslots_dev = fb_count;
    s2.by_query = 1;
    s2.rescore = 2;
    s2.T = T;
    s2.fb_list = fb2_list;
    s2.fb_count = fb_count + 1;
    {
      ProfScope ps(c, "rescore", s);
      if (UseFlat8(*src, nq, kk, 2)) {
        VDBG_DISPATCH_ES(Esel, launch_select, FlatScorer8, s, s2, Flat8Of(*src, c->kset));
      } else if (src->kind == 0) {
        VDBG_DISPATCH_ES(Esel, launch_select, FlatScorer, s, s2, FlatOf(*src, c->kset));
      } else {
        VDBG_DISPATCH_ES(Esel, launch_select, Sq8Scorer, s, s2, Sq8Of(*src, c->kset));
      }
      VDBG_HIP(hipGetLastError());
    }
    VDBG_RETURN_IF_ERROR(ExactScan(c, W2, *src, Q, fb2_list, int(nq), kk, allow, out_ids, out_d,
                                   s, fb_count + 1, c->fb_dev));
    c->fb_dev_used = true;
    return kOk;
  }
  uint32_t nfb = 0;
  VDBG_RETURN_IF_ERROR(ReadWords(c, fb_count, 1, s, &nfb));
  if (nfb == 0) return kOk;
  // second chance: rescore every buffered candidate of the uncertified queries
  SelectArgs s2 = se;
  s2.qlist = fb_list;
  s2.nslots = int(nfb);
  s2.by_query = 1;
  s2.rescore = 2;
  s2.T = T;
  s2.fb_list = fb2_list;
  s2.fb_count = fb_count + 1;
  {
    ProfScope ps(c, "rescore", s);
    if (UseFlat8(*src, nq, kk, 2)) {
      VDBG_DISPATCH_ES(Esel, launch_select, FlatScorer8, s, s2, Flat8Of(*src, c->kset));
    } else if (src->kind == 0) {
      VDBG_DISPATCH_ES(Esel, launch_select, FlatScorer, s, s2, FlatOf(*src, c->kset));
    } else {
      VDBG_DISPATCH_ES(Esel, launch_select, Sq8Scorer, s, s2, Sq8Of(*src, c->kset));
    }
    VDBG_HIP(hipGetLastError());
  }
  uint32_t nfb2 = 0;
  VDBG_RETURN_IF_ERROR(ReadWords(c, fb_count + 1, 1, s, &nfb2));
  c->last_fallbacks += nfb2;
  if (nfb2 > 0)
    VDBG_RETURN_IF_ERROR(
        ExactScan(c, W2, *src, Q, fb2_list, int(nfb2), kk, allow, out_ids, out_d, s));
  return kOk;
}

int Rerank(Ctx* c, const float* X, int pd, int metric, const float* Q, size_t nq,
           const uint32_t* cand, size_t depth, size_t k, uint32_t* out_ids, float* out_d,
           hipStream_t s, const ScanSource* rows) {
  if (nq == 0 || k == 0) return kOk;
  if (std::max(depth, k) > 256)
    return RerankLarge(c, X, pd, metric, Q, nq, cand, depth, k, out_ids, out_d, s);
  const int E = pow2_e(std::max(depth, k));
  const bool int8 = rows != nullptr && rows->X8 != nullptr && rows->x8_parts == 1 && pd % 16 == 0;
  RerankArgs ra{X, Q, pd, metric, c->kset, cand, int(depth), int(nq), int(k), out_ids, out_d,
                int8 ? rows->X8 : nullptr, int8 ? rows->c8 : 0,
                rows != nullptr ? rows->stats : RowStats{}};
  ProfScope ps(c, "rerank", s);
  VDBG_DISPATCH_E(E, launch_rerank, s, ra);
  VDBG_HIP(hipGetLastError());
  return kOk;
}

}  // namespace vdbg
