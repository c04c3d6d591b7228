// vdbg_device.h -- device-side building blocks shared by every vdbg kernel (gfx950).
//
//  * exact distance functions that reproduce vdb's AVX-512 kernels bit for bit
//    (src/distance/avx512.cc:19-64): 16-lane FMA accumulators and GCC's horizontal
//    reduction tree.  The library is compiled with -ffp-contract=off, so the only fused
//    operations are the explicit fmaf() calls standing for _mm512_fmadd_ps.
//  * (dist, id) ordering with vdb's tie rule (include/vdb/types.h:23-25).
//  * wave64 bitonic sorting and a streaming "WaveTopK" that keeps the n smallest keys of
//    a stream in registers spread over the 64 lanes of one wavefront.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vdbg {

constexpr int kWave = 64;
constexpr uint32_t kNoId = 0xffffffffu;

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// Neighbor::operator< (include/vdb/types.h:23-25): distance first, then id.  Float
// comparison keeps -0.0 == +0.0, as the reference does.
__device__ __forceinline__ bool nb_less(float ad, uint32_t ai, float bd, uint32_t bi) {
  // bitwise, not short-circuit: the comparisons combine as lane masks with no branch
  return (ad < bd) | ((ad == bd) & (ai < bi));
}

// A dense row mask (bit r of word r / 64 set = row r allowed); null allows every row.
__device__ __forceinline__ bool row_allowed(const uint64_t* w, uint32_t r) {
  return w == nullptr || ((w[r >> 6] >> (r & 63)) & 1ull);
}

// 64-bit sort key of a (dist, id) pair ordered as Neighbor::operator<: the distance's
// order-preserving bits (-0 folded into +0, which compares equal to it) above the id.
constexpr uint64_t kNoKey = ~0ull;
__device__ __forceinline__ uint64_t dist_key(float d, uint32_t id) {
  const uint32_t b = __float_as_uint(d == 0.f ? 0.f : d);
  const uint32_t e = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (uint64_t(e) << 32) | id;
}
__device__ __forceinline__ float key_dist(uint64_t key) {
  const uint32_t e = uint32_t(key >> 32);
  return __uint_as_float((e & 0x80000000u) ? (e & 0x7fffffffu) : ~e);
}

// ----------------------------------------------------------------- exact distances

// _mm512_reduce_add_ps as GCC expands it: upper 256 bits + lower, upper 128 + lower,
// lanes {0,1} + {2,3}, then lane 0 + lane 1.
__device__ __forceinline__ float reduce16(const float (&v)[16]) {
  float t3[8], t6[4];
#pragma unroll
  for (int i = 0; i < 8; ++i) t3[i] = v[8 + i] + v[i];
#pragma unroll
  for (int i = 0; i < 4; ++i) t6[i] = t3[4 + i] + t3[i];
  return (t6[0] + t6[2]) + (t6[1] + t6[3]);
}

// l2_sq_avx512 (avx512.cc:19-33) for one (query, row) pair.  q and x are pd floats
// (pd % 16 == 0), 16-byte aligned.
__device__ __forceinline__ float l2_exact(const float* __restrict__ q,
                                          const float* __restrict__ x, int pd) {
  float acc0[16], acc1[16];
#pragma unroll
  for (int l = 0; l < 16; ++l) acc0[l] = acc1[l] = 0.f;
  int i = 0;
  for (; i + 32 <= pd; i += 32) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float4 a = *reinterpret_cast<const float4*>(q + i + 4 * v);
      float4 b = *reinterpret_cast<const float4*>(x + i + 4 * v);
      float d0 = a.x - b.x, d1 = a.y - b.y, d2 = a.z - b.z, d3 = a.w - b.w;
      acc0[4 * v + 0] = fmaf(d0, d0, acc0[4 * v + 0]);
      acc0[4 * v + 1] = fmaf(d1, d1, acc0[4 * v + 1]);
      acc0[4 * v + 2] = fmaf(d2, d2, acc0[4 * v + 2]);
      acc0[4 * v + 3] = fmaf(d3, d3, acc0[4 * v + 3]);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float4 a = *reinterpret_cast<const float4*>(q + i + 16 + 4 * v);
      float4 b = *reinterpret_cast<const float4*>(x + i + 16 + 4 * v);
      float d0 = a.x - b.x, d1 = a.y - b.y, d2 = a.z - b.z, d3 = a.w - b.w;
      acc1[4 * v + 0] = fmaf(d0, d0, acc1[4 * v + 0]);
      acc1[4 * v + 1] = fmaf(d1, d1, acc1[4 * v + 1]);
      acc1[4 * v + 2] = fmaf(d2, d2, acc1[4 * v + 2]);
      acc1[4 * v + 3] = fmaf(d3, d3, acc1[4 * v + 3]);
    }
  }
  if (i < pd) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float4 a = *reinterpret_cast<const float4*>(q + i + 4 * v);
      float4 b = *reinterpret_cast<const float4*>(x + i + 4 * v);
      float d0 = a.x - b.x, d1 = a.y - b.y, d2 = a.z - b.z, d3 = a.w - b.w;
      acc0[4 * v + 0] = fmaf(d0, d0, acc0[4 * v + 0]);
      acc0[4 * v + 1] = fmaf(d1, d1, acc0[4 * v + 1]);
      acc0[4 * v + 2] = fmaf(d2, d2, acc0[4 * v + 2]);
      acc0[4 * v + 3] = fmaf(d3, d3, acc0[4 * v + 3]);
    }
  }
  float s[16];
#pragma unroll
  for (int l = 0; l < 16; ++l) s[l] = acc0[l] + acc1[l];
  return reduce16(s);
}

// dot_avx512 (avx512.cc:35-44); the IP/cosine distance is its negation (:46).
__device__ __forceinline__ float dot_exact(const float* __restrict__ q,
                                           const float* __restrict__ x, int pd) {
  float acc0[16], acc1[16];
#pragma unroll
  for (int l = 0; l < 16; ++l) acc0[l] = acc1[l] = 0.f;
  int i = 0;
  for (; i + 32 <= pd; i += 32) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float4 a = *reinterpret_cast<const float4*>(q + i + 4 * v);
      float4 b = *reinterpret_cast<const float4*>(x + i + 4 * v);
      acc0[4 * v + 0] = fmaf(a.x, b.x, acc0[4 * v + 0]);
      acc0[4 * v + 1] = fmaf(a.y, b.y, acc0[4 * v + 1]);
      acc0[4 * v + 2] = fmaf(a.z, b.z, acc0[4 * v + 2]);
      acc0[4 * v + 3] = fmaf(a.w, b.w, acc0[4 * v + 3]);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float4 a = *reinterpret_cast<const float4*>(q + i + 16 + 4 * v);
      float4 b = *reinterpret_cast<const float4*>(x + i + 16 + 4 * v);
      acc1[4 * v + 0] = fmaf(a.x, b.x, acc1[4 * v + 0]);
      acc1[4 * v + 1] = fmaf(a.y, b.y, acc1[4 * v + 1]);
      acc1[4 * v + 2] = fmaf(a.z, b.z, acc1[4 * v + 2]);
      acc1[4 * v + 3] = fmaf(a.w, b.w, acc1[4 * v + 3]);
    }
  }
  if (i < pd) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float4 a = *reinterpret_cast<const float4*>(q + i + 4 * v);
      float4 b = *reinterpret_cast<const float4*>(x + i + 4 * v);
      acc0[4 * v + 0] = fmaf(a.x, b.x, acc0[4 * v + 0]);
      acc0[4 * v + 1] = fmaf(a.y, b.y, acc0[4 * v + 1]);
      acc0[4 * v + 2] = fmaf(a.z, b.z, acc0[4 * v + 2]);
      acc0[4 * v + 3] = fmaf(a.w, b.w, acc0[4 * v + 3]);
    }
  }
  float s[16];
#pragma unroll
  for (int l = 0; l < 16; ++l) s[l] = acc0[l] + acc1[l];
  return reduce16(s);
}

// The kernel sets vdb picks from (src/distance/cpu_features.cc:33-58): the scalar kernels,
// AVX2 and AVX-512.  Each restates its own summation order; the -ffp-contract=off build
// keeps the scalar kernels' products and sums as separate roundings.
enum KernelSet : int { kKsetScalar = 0, kKsetAvx2 = 1, kKsetAvx512 = 2 };

// HorizontalSum of an 8-lane register (src/distance/avx2.cc:11-16): low 128 + high 128,
// then two hadds: (s0 + s1) + (s2 + s3).
__device__ __forceinline__ float hsum8(const float (&v)[8]) {
  float s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = v[i] + v[4 + i];
  return (s[0] + s[1]) + (s[2] + s[3]);
}

// l2_sq_scalar / dot_scalar (src/distance/scalar.cc:8-21): one accumulator, in order.
__device__ __forceinline__ float l2_scalar_k(const float* __restrict__ q,
                                             const float* __restrict__ x, int pd) {
  float s = 0.f;
  for (int i = 0; i < pd; ++i) {
    const float t = q[i] - x[i];
    s += t * t;
  }
  return s;
}
__device__ __forceinline__ float dot_scalar_k(const float* __restrict__ q,
                                              const float* __restrict__ x, int pd) {
  float s = 0.f;
  for (int i = 0; i < pd; ++i) s += q[i] * x[i];
  return s;
}

// l2_sq_avx2 / dot_avx2 (src/distance/avx2.cc:26-44): per 16 floats, lanes 0-7 into one
// 8-lane FMA accumulator and 8-15 into another; their sum, HorizontalSum.
__device__ __forceinline__ float l2_avx2_k(const float* __restrict__ q,
                                           const float* __restrict__ x, int pd) {
  float acc0[8], acc1[8];
#pragma unroll
  for (int l = 0; l < 8; ++l) acc0[l] = acc1[l] = 0.f;
  for (int i = 0; i < pd; i += 16) {
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const float d0 = q[i + l] - x[i + l];
      acc0[l] = fmaf(d0, d0, acc0[l]);
      const float d1 = q[i + 8 + l] - x[i + 8 + l];
      acc1[l] = fmaf(d1, d1, acc1[l]);
    }
  }
  float s[8];
#pragma unroll
  for (int l = 0; l < 8; ++l) s[l] = acc0[l] + acc1[l];
  return hsum8(s);
}
__device__ __forceinline__ float dot_avx2_k(const float* __restrict__ q,
                                            const float* __restrict__ x, int pd) {
  float acc0[8], acc1[8];
#pragma unroll
  for (int l = 0; l < 8; ++l) acc0[l] = acc1[l] = 0.f;
  for (int i = 0; i < pd; i += 16) {
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      acc0[l] = fmaf(q[i + l], x[i + l], acc0[l]);
      acc1[l] = fmaf(q[i + 8 + l], x[i + 8 + l], acc1[l]);
    }
  }
  float s[8];
#pragma unroll
  for (int l = 0; l < 8; ++l) s[l] = acc0[l] + acc1[l];
  return hsum8(s);
}

// MetricDistance (src/distance/cpu_features.cc:71-73) of a kernel set: 0 = L2, else minus
// the dot product.
__device__ __forceinline__ float metric_exact_k(int kset, int metric, const float* q,
                                                const float* x, int pd) {
  if (kset == kKsetAvx512) return metric == 0 ? l2_exact(q, x, pd) : -dot_exact(q, x, pd);
  if (kset == kKsetAvx2) return metric == 0 ? l2_avx2_k(q, x, pd) : -dot_avx2_k(q, x, pd);
  return metric == 0 ? l2_scalar_k(q, x, pd) : -dot_scalar_k(q, x, pd);
}
// The AVX-512 set (the one vdb selects on AVX-512 hosts).
__device__ __forceinline__ float metric_exact(int metric, const float* q, const float* x,
                                              int pd) {
  return metric == 0 ? l2_exact(q, x, pd) : -dot_exact(q, x, pd);
}

// sq8_l2_avx512 / sq8_ip_avx512 (avx512.cc:48-64): each code byte decodes as
// fma(code, scale, vmin) (Decode16, :11-15); one 16-lane accumulator; GCC reduce tree.
__device__ __forceinline__ float sq8_exact(int metric, const float* __restrict__ q,
                                           const uint8_t* __restrict__ c,
                                           const float* __restrict__ vmin,
                                           const float* __restrict__ scale, int pd) {
  float acc[16];
#pragma unroll
  for (int l = 0; l < 16; ++l) acc[l] = 0.f;
  for (int i = 0; i < pd; i += 16) {
    const uint4 cb = *reinterpret_cast<const uint4*>(c + i);
    const uint32_t w[4] = {cb.x, cb.y, cb.z, cb.w};
#pragma unroll
    for (int l = 0; l < 16; ++l) {
      const float code = float((w[l >> 2] >> (8 * (l & 3))) & 0xffu);
      const float x = fmaf(code, scale[i + l], vmin[i + l]);
      if (metric == 0) {
        const float diff = q[i + l] - x;
        acc[l] = fmaf(diff, diff, acc[l]);
      } else {
        acc[l] = fmaf(q[i + l], x, acc[l]);
      }
    }
  }
  const float s = reduce16(acc);
  return metric == 0 ? s : -s;
}

// sq8_l2_scalar / sq8_ip_scalar (src/distance/scalar.cc:25-41): vmin + code * scale in two
// roundings, one accumulator.
__device__ __forceinline__ float sq8_scalar_k(int metric, const float* __restrict__ q,
                                              const uint8_t* __restrict__ c,
                                              const float* __restrict__ vmin,
                                              const float* __restrict__ scale, int pd) {
  float s = 0.f;
  for (int i = 0; i < pd; ++i) {
    const float x = vmin[i] + float(c[i]) * scale[i];
    if (metric == 0) {
      const float t = q[i] - x;
      s += t * t;
    } else {
      s += q[i] * x;
    }
  }
  return metric == 0 ? s : -s;
}

// sq8_l2_avx2 / sq8_ip_avx2 (src/distance/avx2.cc:48-74): Decode8 = fma(code, scale, vmin)
// on each half of 16 code bytes, two 8-lane accumulators, HorizontalSum.
__device__ __forceinline__ float sq8_avx2_k(int metric, const float* __restrict__ q,
                                            const uint8_t* __restrict__ c,
                                            const float* __restrict__ vmin,
                                            const float* __restrict__ scale, int pd) {
  float acc0[8], acc1[8];
#pragma unroll
  for (int l = 0; l < 8; ++l) acc0[l] = acc1[l] = 0.f;
  for (int i = 0; i < pd; i += 16) {
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const float x0 = fmaf(float(c[i + l]), scale[i + l], vmin[i + l]);
      const float x1 = fmaf(float(c[i + 8 + l]), scale[i + 8 + l], vmin[i + 8 + l]);
      if (metric == 0) {
        const float d0 = q[i + l] - x0, d1 = q[i + 8 + l] - x1;
        acc0[l] = fmaf(d0, d0, acc0[l]);
        acc1[l] = fmaf(d1, d1, acc1[l]);
      } else {
        acc0[l] = fmaf(q[i + l], x0, acc0[l]);
        acc1[l] = fmaf(q[i + 8 + l], x1, acc1[l]);
      }
    }
  }
  float s[8];
#pragma unroll
  for (int l = 0; l < 8; ++l) s[l] = acc0[l] + acc1[l];
  const float r = hsum8(s);
  return metric == 0 ? r : -r;
}

// MetricSq8Distance (cpu_features.cc:75-78) of a kernel set.
__device__ __forceinline__ float sq8_exact_k(int kset, int metric, const float* q,
                                             const uint8_t* c, const float* vmin,
                                             const float* scale, int pd) {
  if (kset == kKsetAvx512) return sq8_exact(metric, q, c, vmin, scale, pd);
  if (kset == kKsetAvx2) return sq8_avx2_k(metric, q, c, vmin, scale, pd);
  return sq8_scalar_k(metric, q, c, vmin, scale, pd);
}

// Exact scorers: the reference's distance of query q to row `row` under kernel set kset.
// DotAny / L2SqAny (src/distance/scalar.cc:43-73): four accumulators over i mod 4,
// (s0 + s1) + (s2 + s3), products rounded before the add.
__device__ __forceinline__ float dot_any(const float* a, const float* b, int d) {
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  int i = 0;
  for (; i + 4 <= d; i += 4) {
    s0 += a[i] * b[i];
    s1 += a[i + 1] * b[i + 1];
    s2 += a[i + 2] * b[i + 2];
    s3 += a[i + 3] * b[i + 3];
  }
  for (; i < d; ++i) s0 += a[i] * b[i];
  return (s0 + s1) + (s2 + s3);
}

__device__ __forceinline__ float l2sq_any(const float* a, const float* b, int d) {
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  int i = 0;
  for (; i + 4 <= d; i += 4) {
    const float t0 = a[i] - b[i], t1 = a[i + 1] - b[i + 1];
    const float t2 = a[i + 2] - b[i + 2], t3 = a[i + 3] - b[i + 3];
    s0 += t0 * t0;
    s1 += t1 * t1;
    s2 += t2 * t2;
    s3 += t3 * t3;
  }
  for (; i < d; ++i) {
    const float t = a[i] - b[i];
    s0 += t * t;
  }
  return (s0 + s1) + (s2 + s3);
}

// L2SqAny(r, b, d) of the residual r = q - c, each r_i rounded to fp32 as the reference
// stores it before the call (ivf_pq.cc:207-208, 128-139); c null means r = q.
__device__ __forceinline__ float l2sq_res_any(const float* q, const float* c, const float* b,
                                              int d) {
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  int i = 0;
  for (; i + 4 <= d; i += 4) {
    const float r0 = c ? q[i] - c[i] : q[i], r1 = c ? q[i + 1] - c[i + 1] : q[i + 1];
    const float r2 = c ? q[i + 2] - c[i + 2] : q[i + 2], r3 = c ? q[i + 3] - c[i + 3] : q[i + 3];
    const float t0 = r0 - b[i], t1 = r1 - b[i + 1];
    const float t2 = r2 - b[i + 2], t3 = r3 - b[i + 3];
    s0 += t0 * t0;
    s1 += t1 * t1;
    s2 += t2 * t2;
    s3 += t3 * t3;
  }
  for (; i < d; ++i) {
    const float r = c ? q[i] - c[i] : q[i];
    const float t = r - b[i];
    s0 += t * t;
  }
  return (s0 + s1) + (s2 + s3);
}

// ProductQuantizer::adc (src/index/quant/pq.h:36-46) of row `row`'s code against a query's
// table (m x 256 floats, the "query" pointer the scans hand the scorer): four accumulators
// over j mod 4.
struct PqScorer {
  const uint8_t* codes;  // n x m
  int m;
  __device__ __forceinline__ float operator()(const float* table, uint32_t row) const {
    const uint8_t* cd = codes + size_t(row) * m;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    int j = 0;
    for (; j + 4 <= m; j += 4) {
      s0 += table[(j + 0) * 256 + cd[j + 0]];
      s1 += table[(j + 1) * 256 + cd[j + 1]];
      s2 += table[(j + 2) * 256 + cd[j + 2]];
      s3 += table[(j + 3) * 256 + cd[j + 3]];
    }
    for (; j < m; ++j) s0 += table[j * 256 + cd[j]];
    return (s0 + s1) + (s2 + s3);
  }
};

struct FlatScorer {
  const float* X;
  int pd, metric, kset;
  const uint32_t* map = nullptr;  // nullable: row r is row map[r] of X
  __device__ __forceinline__ float operator()(const float* q, uint32_t row) const {
    const size_t r = map != nullptr ? map[row] : row;
    return metric_exact_k(kset, metric, q, X + r * pd, pd);
  }
};

// The same, with the rows' int8 copy x8 = x - c8 (integer rows) and their value range: a
// selection re-scoring many keys takes them from the int8 copy for queries whose distances
// are exact integers (scan_kernels.hip, Int8Query).
struct FlatScorer8 : FlatScorer {
  const int8_t* X8;
  int c8;
  float xlo, xhi, xmax;
  int xint;
};

struct Sq8Scorer {
  const uint8_t* C;
  const float* vmin;
  const float* scale;
  int pd, metric, kset;
  __device__ __forceinline__ float operator()(const float* q, uint32_t row) const {
    return sq8_exact_k(kset, metric, q, C + size_t(row) * pd, vmin, scale, pd);
  }
};

// ----------------------------------------------------------------- wave bitonic

// Keys live in registers: element g = e * 64 + lane for e in [0, E).  All loops unroll
// at compile time, so every shuffle distance is a constant.
template <int E>
struct WaveKeys {
  float d[E];
  uint32_t id[E];
};

// v of lane (lane ^ j), j a power of two below 64, in the VALU (no trip through the LDS
// unit): a DPP quad permutation for j = 1, 2; DPP row rotates for j = 4, 8 (row_ror:n gives
// lane i the value of lane (i - n) mod 16 of its 16-lane row: lane ^ 8 is ror 8, lane ^ 4 is
// ror 12 where bit 2 of the lane is clear and ror 4 where it is set); v_permlane16_swap and
// v_permlane32_swap for j = 16, 32 (each returns the even and the odd row, or half, of the
// lane's pair: the partner's is the one the lane is not in).
__device__ __forceinline__ uint32_t lane_xor(uint32_t v, int j) {
  if (j == 1) return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0xB1, 0xF, 0xF, true));
  if (j == 2) return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x4E, 0xF, 0xF, true));
  const uint32_t lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  if (j == 4) {
    const uint32_t up = uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x12C, 0xF, 0xF, false));
    const uint32_t down = uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x124, 0xF, 0xF, false));
    return (lane & 4u) ? down : up;
  }
  if (j == 8) return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x128, 0xF, 0xF, false));
  if (j == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane & 16u) ? p[0] : p[1];
  }
  const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (lane & 32u) ? p[0] : p[1];
}
__device__ __forceinline__ float lane_xor(float v, int j) {
  return __uint_as_float(lane_xor(__float_as_uint(v), j));
}
// v of lane 7 - (lane & 7) of the lane's group of eight (DPP row_half_mirror).
__device__ __forceinline__ uint32_t lane_mirror8(uint32_t v) {
  return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x141, 0xF, 0xF, true));
}
__device__ __forceinline__ float lane_mirror8(float v) {
  return __uint_as_float(lane_mirror8(__float_as_uint(v)));
}

// l2_exact / dot_exact (the AVX-512 set) of R rows per 8-lane group: lanes 8g..8g+7 score
// the rows x[0..R) their group passes, every row's loads in flight together.  The 32
// accumulators of l2_exact (acc0 is 0..15, acc1 16..31) come in 8 runs of four, run k being
// accumulators 4k..4k+3; lane j of a group keeps run k = j for j < 4 and k = 11 - j above, so
// run k and run k + 4 sit in lanes j and 7 - j.  Accumulator a sums dims a, a + 32, a + 64,
// ... in that order, and the tail of a row with pd % 32 == 16 goes to acc0 (runs 0..3), as
// there.  The reduction pairs the same operands through lane exchanges: the mirror j <-> 7 - j
// forms acc0[m] + acc1[m], xor 2 and xor 1 the first two levels of reduce16 (runs k <-> k + 2,
// then 0 <-> 1), and the lane the last two; each exchange is one DPP operand of the add.  A
// group reads a row in 128-byte runs (one lane scoring a row alone reads 16 bytes of it per
// load, 64 rows per wave load).  Every lane of a group returns its rows' distances in d; all
// 64 lanes must be active.
template <int R>
__device__ __forceinline__ void metric_exact_g8n(int metric, const float* __restrict__ q,
                                                 const float* const (&x)[R], int pd,
                                                 float (&d)[R]) {
  const int j = lane_id() & 7;
  const int run = j < 4 ? j : 11 - j;
  float a[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r) a[r][0] = a[r][1] = a[r][2] = a[r][3] = 0.f;
  auto add = [&](float (&acc)[4], const float4& u, const float4& v) {
    if (metric == 0) {
      const float d0 = u.x - v.x, d1 = u.y - v.y, d2 = u.z - v.z, d3 = u.w - v.w;
      acc[0] = fmaf(d0, d0, acc[0]);
      acc[1] = fmaf(d1, d1, acc[1]);
      acc[2] = fmaf(d2, d2, acc[2]);
      acc[3] = fmaf(d3, d3, acc[3]);
    } else {
      acc[0] = fmaf(u.x, v.x, acc[0]);
      acc[1] = fmaf(u.y, v.y, acc[1]);
      acc[2] = fmaf(u.z, v.z, acc[2]);
      acc[3] = fmaf(u.w, v.w, acc[3]);
    }
  };
  auto ld = [&](const float* p, int i) { return *reinterpret_cast<const float4*>(p + i + 4 * run); };
  // 128 dims a round: the round's loads are all issued before the first is used
  int i = 0;
  for (; i + 128 <= pd; i += 128) {
    float4 u[4], v[R][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      u[t] = ld(q, i + 32 * t);
#pragma unroll
      for (int r = 0; r < R; ++r) v[r][t] = ld(x[r], i + 32 * t);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int r = 0; r < R; ++r) add(a[r], u[t], v[r][t]);
    }
  }
  for (; i + 32 <= pd; i += 32) {
    const float4 u = ld(q, i);
#pragma unroll
    for (int r = 0; r < R; ++r) add(a[r], u, ld(x[r], i));
  }
  if (i < pd && run < 4) {
    const float4 u = ld(q, i);
#pragma unroll
    for (int r = 0; r < R; ++r) add(a[r], u, ld(x[r], i));
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int c = 0; c < 4; ++c) a[r][c] = a[r][c] + lane_mirror8(a[r][c]);
#pragma unroll
    for (int c = 0; c < 4; ++c) a[r][c] = a[r][c] + lane_xor(a[r][c], 2);
#pragma unroll
    for (int c = 0; c < 4; ++c) a[r][c] = a[r][c] + lane_xor(a[r][c], 1);
    const float s = (a[r][0] + a[r][2]) + (a[r][1] + a[r][3]);
    d[r] = metric == 0 ? s : -s;
  }
}

// One compare-exchange layer of a bitonic network over 64*E elements: partner g ^ j,
// ascending in blocks where (g & size) == 0.
template <int E>
__device__ __forceinline__ void bitonic_layer(WaveKeys<E>& k, int size, int j) {
  const int lane = lane_id();
  if (j >= kWave) {
    const int je = j / kWave;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int pe = e ^ je;
      if (pe > e) {
        const int g = e * kWave + lane;
        const bool up = (g & size) == 0;
        const bool lt = nb_less(k.d[pe], k.id[pe], k.d[e], k.id[e]);
        const bool gt = nb_less(k.d[e], k.id[e], k.d[pe], k.id[pe]);
        const bool sw = up ? lt : gt;
        const float d0 = k.d[e], d1 = k.d[pe];
        const uint32_t i0 = k.id[e], i1 = k.id[pe];
        k.d[e] = sw ? d1 : d0;
        k.d[pe] = sw ? d0 : d1;
        k.id[e] = sw ? i1 : i0;
        k.id[pe] = sw ? i0 : i1;
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int g = e * kWave + lane;
      const float pd = lane_xor(k.d[e], j);
      const uint32_t pi = lane_xor(k.id[e], j);
      const bool up = (g & size) == 0;
      const bool lower = (lane & j) == 0;
      const bool lt = nb_less(pd, pi, k.d[e], k.id[e]);
      const bool gt = nb_less(k.d[e], k.id[e], pd, pi);
      const bool take = (lower == up) ? lt : gt;
      k.d[e] = take ? pd : k.d[e];
      k.id[e] = take ? pi : k.id[e];
    }
  }
}

// Full ascending sort of 64*E keys.
template <int E>
__device__ __forceinline__ void bitonic_sort(WaveKeys<E>& k) {
  constexpr int N = kWave * E;
#pragma unroll
  for (int size = 2; size <= N; size <<= 1) {
#pragma unroll
    for (int j = size >> 1; j > 0; j >>= 1) bitonic_layer<E>(k, size, j);
  }
}

// Sorts a bitonic sequence of 64*E keys ascending.
template <int E>
__device__ __forceinline__ void bitonic_merge(WaveKeys<E>& k) {
  constexpr int N = kWave * E;
#pragma unroll
  for (int j = N >> 1; j > 0; j >>= 1) bitonic_layer<E>(k, N, j);
}

// The n = 64*E smallest keys of a stream, kept sorted ascending across the wave.  Insert
// a batch of up to 64 keys (one per lane, +inf/kNoId for none): the batch is sorted,
// reversed against the tail of the list (the minimum of an ascending and a descending
// sequence is bitonic and holds the n smallest), then merged.
template <int E>
struct WaveTopK {
  WaveKeys<E> k;

  __device__ __forceinline__ void init() {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      k.d[e] = __builtin_inff();
      k.id[e] = kNoId;
    }
  }

  // The current n-th smallest key (broadcast to every lane).
  __device__ __forceinline__ void threshold(float& td, uint32_t& ti) const {
    td = __shfl(k.d[E - 1], kWave - 1);
    ti = __shfl(k.id[E - 1], kWave - 1);
  }

  // Wave-uniform call.  Inserts the lanes' keys; lanes with nothing pass +inf/kNoId.
  __device__ __forceinline__ void insert(float cd, uint32_t ci) {
    float td;
    uint32_t ti;
    threshold(td, ti);
    const bool want = nb_less(cd, ci, td, ti);
    if (__ballot(want) == 0) return;
    WaveKeys<1> b;
    b.d[0] = want ? cd : __builtin_inff();
    b.id[0] = want ? ci : kNoId;
    bitonic_sort<1>(b);
    const int lane = lane_id();
    const float rd = __shfl(b.d[0], kWave - 1 - lane);
    const uint32_t ri = __shfl(b.id[0], kWave - 1 - lane);
    if (nb_less(rd, ri, k.d[E - 1], k.id[E - 1])) {
      k.d[E - 1] = rd;
      k.id[E - 1] = ri;
    }
    bitonic_merge<E>(k);
  }
};

}  // namespace vdbg
