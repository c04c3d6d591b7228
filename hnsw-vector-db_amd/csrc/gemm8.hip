// gemm8.hip -- the ranking GEMM of the flat scan for integer rows spanning at most 256
// consecutive values, on int8 MFMA (v_mfma_i32_32x32x32_i8: twice the fp16 rate, half the
// operand bytes).
//
// With a per-dataset integer shift c, every row value x and query value q becomes an int8
// x' = x - c, q' = q - c (rows: c centres their range; queries: the batch qualifies when every
// q' fits).  Over all padded dims
//     ||x'||^2 - 2 q'.x' = (||x||^2 - 2 q.x) + 2 c sum(q) - c^2 pd          (L2)
//     -q'.x' - c sum(x)  = -q.x + c sum(q) - c^2 pd                          (inner product)
// so the GEMM value of the fp32 form is, per query, the integer GEMM plus a constant
// delta_q = M c sum(q) - c^2 pd (M = 2 for L2, 1 for inner product).  The accumulator runs
//     u = init(x) + q'.x'      init = -ceil(||x'||^2 / 2) (L2)  or  c sum(x) (inner product)
// exactly in int32, and value = -M u - delta_q.  For inner product that is the GEMM value
// exactly; for L2 it is the GEMM value plus (||x'||^2 mod 2), so at most 1 above it: the
// batch carries a bound eb = 1 and the exact re-scoring decides, as on every inexact path.
// The threshold test value <= T becomes u >= ceil((-T - delta_q) / M): one integer compare
// per value, the same count as the fp16 GEMM's.  Rows that take no part start from -2^29,
// below any threshold and any group maximum of a live row.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <type_traits>

#include "gemm.h"
#include "vdbg_device.h"
#include "vdbg_internal.h"

namespace vdbg {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kDead8 = -(1 << 29);   // accumulator start of rows that take no part
constexpr int kLive8 = -(1 << 28);   // every live row's u is above this

// Block = 4 waves x (32 QB) queries each x one chunk of rows, blocks mapped to work items
// XCD by XCD; rows stream through double-buffered 64-row LDS stages (K chunks of KC dims for
// rows wider than 128), row starts through three slots.
//
// Operand layout of v_mfma_i32_32x32x32_i8: per 32-dim K block, lane l holds 16 bytes, dims
// 16 (l / 32) .. 16 (l / 32) + 15 of row l % 32 (A, from LDS) and of query l % 32 (B, in
// VGPRs); both operands use the same dim of a lane's byte, so the contraction covers every
// dim once whatever order the unit sums in (integer sums are exact in any order).  Lane l's
// 16 outputs are rows 8 (r / 4) + 4 (l / 32) + r % 4 of the 32-row block against query l % 32.
//
// MODE 0: every value at or below the query's threshold T goes to the lane's candidate
// buffer; MODE 1: the minimum value of each 16-row group (the sample pass); MODE 2: the
// sample pass keeping only the kTop8 smallest group minima each lane meets in its chunk (the
// minima of kTop8 distinct groups, so the kk-th smallest of all lanes' lists is still a
// value at least kk distinct rows reach), written once at the end: gm[q][(chunk * 2 + h) *
// kTop8 + t].  It replaces a scattered store per group with two vector stores per lane.
//
// SQ = 1: SQ8 codes against a query operand in two int8 parts.  Codes c (uint8) enter LDS as
// c' = c - 128; the scaled query operand B 2^e (one exponent e for the whole batch, *a.e8) is
// rounded to integers v = 256 hi + lo with hi, lo int8 ([q][2][pd] in Q8).  The two register
// sets hold the same 32 queries (QB = 2 parts), the hi accumulator starts at 0 and the lo one
// at the row start -rint(||c scale||^2 2^(e-1)) (L2) or 0 (inner product), and
// u = 256 acc_hi + acc_lo.  With dq = M 128 sum(v) (a.Qd) the value in GEMM units is
// (-M u - dq) 2^-e; its distance from the fp32 GEMM value is in the query's bound.
//
// SQ = 2: float rows, both operands in two int8 parts.  Rows x 2^ex and the batch's queries
// q 2^eq rounded to integers 256 h + l (rows stored per K chunk as [h | l], row bytes
// 2 pd), so sum v_x v_q = 2^16 (h.h) + 2^8 (h.l + l.h) + l.l: four MFMAs into three
// accumulators, u = (acc_hh << 16) + (acc_mid << 8) + acc_ll exactly in int32 (the batch is
// admitted only while |sum v_x v_q| + row start < 2^29).  e = ex + eq, dq = 0.
template <int PD, int METRIC, int QB, int MODE, int OCC = 2, int SQ = 0>
__global__ __launch_bounds__(256, OCC) void k_gemm8(GemmArgs a) {
  static_assert(SQ == 0 || QB == 2, "the two-part operands run two parts");
  constexpr int NQ = SQ ? 1 : QB;                  // queries per lane
  constexpr int NACC = SQ == 2 ? 3 : QB;           // accumulator sets
  constexpr int RP = SQ == 2 ? 2 : 1;              // row parts
  // accumulator start of rows that take no part, and the bound every live row's u exceeds
  constexpr int kDead = SQ == 2 ? -(1 << 30) : kDead8;
  constexpr int kLive = SQ == 2 ? -(1 << 29) : kLive8;
  constexpr int KC = SQ == 2 ? Gemm8KcSplit(PD) : Gemm8Kc(PD);
  constexpr int NKC = PD / KC;
  constexpr int NKB = KC / 32;                     // 32-dim MFMA K blocks per stage
  constexpr int STR = RP * KC + 16;                // LDS row stride in bytes (16 B padding)
  constexpr int VEC_PER_ROW = RP * KC / 16;        // 16-byte vectors per stage row
  constexpr int VEC_PER_TILE = kGemmRows * VEC_PER_ROW;
  constexpr int VEC_PER_THREAD = (VEC_PER_TILE + 255) / 256;
  constexpr int QT = 128 * NQ;                     // queries per block
  constexpr int M = METRIC == 0 ? 2 : 1;
  static_assert(PD % KC == 0 && KC % 32 == 0, "K chunking");
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][kGemmRows * STR];
  __shared__ __attribute__((aligned(16))) int xns[3][kGemmRows];
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
  const int q0 = qt * QT + wave * 32 * NQ;
  const bool wave_live = q0 < a.nq;
  const uint32_t r_begin = uint32_t(chunk) * a.chunk_rows;
  const uint32_t r_end = min(a.N, r_begin + a.chunk_rows);

  // SQ8: the batch exponent e; values leave the kernel as (-M u - dq) 2^-e
  const int e8 = SQ ? *a.e8 : 0;
  int q[NQ], ui[NQ], dq[NQ];
  uint2* out[NQ];
  uint32_t cnt[NQ];
  int top[MODE == 2 ? NQ : 1][kTop8];  // MODE 2: largest u of distinct groups, descending
  auto gemm_units = [&](int u, int d) {
    const float v = float(-M * u - d);
    return SQ ? ldexpf(v, -e8) : v;
  };
#pragma unroll
  for (int qb = 0; qb < NQ; ++qb) {
    q[qb] = q0 + qb * 32 + j;
    cnt[qb] = 0;
    if constexpr (MODE == 2) {
#pragma unroll
      for (int t = 0; t < kTop8; ++t) top[qb][t] = kDead;
    }
    dq[qb] = a.Qd[min(q[qb], a.nq - 1)];
    if constexpr (MODE == 0) {
      // value <= T  <=>  u >= ceil((-T - delta) / M); +inf admits every live row, -inf (a
      // lane past the batch) none
      const float T = q[qb] < a.nq ? a.T[q[qb]] : -__builtin_inff();
      const double t = ceil((-ldexp(double(T), e8) - double(dq[qb])) / M);
      ui[qb] = !(t <= double(1 << 30)) ? (1 << 30) : (t < double(kLive) ? kLive : int(t));
      out[qb] = a.cand + ((size_t(q[qb]) * a.nchunks + chunk) * 2 + h) * size_t(a.caph);
    }
  }

  // Loads are unconditional (addresses clamped), as in the fp16 GEMM, so the waits before
  // the LDS stores never drain the prefetch early.
  constexpr int QF = NKC > 1 ? 2 : 1;
  v4i qv[QF][QB][NKB];
  const int8_t* qrow[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
    qrow[qb] = SQ ? a.Q8 + (size_t(min(q[0], a.nq - 1)) * 2 + qb) * PD + h * 16
                  : a.Q8 + size_t(min(q[qb], a.nq - 1)) * PD + h * 16;
  auto load_q = [&](int f, int kc) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        qv[f][qb][kb] = *reinterpret_cast<const v4i*>(qrow[qb] + kc * KC + kb * 32);
  };
  load_q(0, 0);

  // byte offsets of the stage's 16-byte vectors: row f / VEC_PER_ROW, column f % VEC_PER_ROW
  int voff[VEC_PER_THREAD];
  int vrow[VEC_PER_THREAD];
#pragma unroll
  for (int i = 0; i < VEC_PER_THREAD; ++i) {
    const int f = min(tid + 256 * i, VEC_PER_TILE - 1);
    vrow[i] = f / VEC_PER_ROW;
    voff[i] = vrow[i] * RP * PD + (f % VEC_PER_ROW) * 16;
  }
  // Stages s = tile * NKC + kc (64 rows x KC dims), stage s + 2 loaded while stage s is
  // multiplied, two register sets swapping roles each step, as in the fp16 GEMM.
  struct Stage {
    u32x4 v[VEC_PER_THREAD];
    int n;
    uint32_t aw;  // filter bits of the lane's half of the tile
  };
  const int ntiles = int((r_end - r_begin + kGemmRows - 1) / kGemmRows);
  const int nstages = ntiles * NKC;
  auto load_stage = [&](Stage& st, int sidx) {
    sidx = min(sidx, nstages - 1);
    const int tile = sidx / NKC, kc = sidx - tile * NKC;
    const uint32_t base = r_begin + uint32_t(tile) * kGemmRows;
    const uint32_t valid = min(uint32_t(kGemmRows), r_end - base);  // >= 1
    const char* src = reinterpret_cast<const char*>(a.X8 + size_t(base) * RP * PD + kc * RP * KC);
    if (valid == kGemmRows) {
#pragma unroll
      for (int i = 0; i < VEC_PER_THREAD; ++i)
        st.v[i] = *reinterpret_cast<const u32x4*>(src + uint32_t(voff[i]));
    } else {  // rows past the end read row valid - 1
      const int over = int(valid) - 1;
#pragma unroll
      for (int i = 0; i < VEC_PER_THREAD; ++i) {
        const int o = voff[i] - max(0, vrow[i] - over) * RP * PD;
        st.v[i] = *reinterpret_cast<const u32x4*>(src + uint32_t(o));
      }
    }
    if constexpr (SQ)  // L2: -rint(||c scale||^2 2^(e - 1)), inner product: 0
      st.n = METRIC == 0
                 ? -int(rintf(ldexpf(a.rn[base + min(uint32_t(tid & 63), valid - 1)], e8 - 1)))
                 : 0;
    else
      st.n = a.rn8[base + min(uint32_t(tid & 63), valid - 1)];
    if constexpr (MODE == 0)
      st.aw = a.aw[((base >> 5) + (uint32_t(tid & 63) >> 5)) & a.aw_mask];
  };
  auto store_stage = [&](const Stage& st, int sidx) {
    const int tile = sidx / NKC, kc = sidx - tile * NKC;
    const int buf = sidx & 1;
#pragma unroll
    for (int i = 0; i < VEC_PER_THREAD; ++i) {
      const int f = tid + 256 * i;
      if (VEC_PER_TILE % 256 == 0 || f < VEC_PER_TILE)
        *reinterpret_cast<u32x4*>(&xs[buf][vrow[i] * STR + (voff[i] - vrow[i] * RP * PD)]) =
            SQ == 1 ? (st.v[i] ^ 0x80808080u) : st.v[i];  // SQ8: codes c to int8 c - 128
    }
    if (kc == 0 && tid < kGemmRows) {
      const uint32_t valid = min(uint32_t(kGemmRows), r_end - (r_begin + uint32_t(tile) * kGemmRows));
      const bool ok = uint32_t(tid) < valid && (MODE != 0 || ((st.aw >> (tid & 31)) & 1u));
      xns[tile % 3][tid] = ok ? st.n : kDead;
    }
  };

  v16i acc[NACC][2];
  auto step = [&](Stage& X, Stage& Y, int sidx, auto fcur) {
    constexpr int QS = decltype(fcur)::value;
    const int tile = sidx / NKC, kc = sidx - tile * NKC;
    const uint32_t base = r_begin + uint32_t(tile) * kGemmRows;
    if constexpr (QF == 2) load_q(QS ^ 1, (kc + 1 == NKC) ? 0 : kc + 1);
    load_stage(Y, sidx + 2);
    __builtin_amdgcn_sched_barrier(0);
    if (kc == 0) {
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        v16i init;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int4 n4 = *reinterpret_cast<const int4*>(&xns[tile % 3][blk * 32 + 8 * g + 4 * h]);
          init[4 * g + 0] = n4.x;
          init[4 * g + 1] = n4.y;
          init[4 * g + 2] = n4.z;
          init[4 * g + 3] = n4.w;
        }
#pragma unroll
        for (int s = 0; s < NACC; ++s) {
          if (SQ && s + 1 < NACC)
            acc[s][blk] = v16i{};  // the high parts start at 0, the lowest at the row start
          else
            acc[s][blk] = init;
        }
      }
    }
    const uint8_t* xa0 = &xs[sidx & 1][j * STR + h * 16];
    const uint8_t* xa1 = xa0 + 32 * STR;
    if constexpr (SQ != 2) {
      // row block 0 over every K block, then row block 1: block 0's accumulators are final
      // while block 1's MFMAs still run, so its threshold test starts a block earlier
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          const v4i x = *reinterpret_cast<const v4i*>((blk ? xa1 : xa0) + kb * 32);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb)
            acc[qb][blk] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, qv[QS][qb][kb], acc[qb][blk], 0, 0, 0);
        }
    } else {  // rows [h | l]: h.h, h.l + l.h, l.l
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const v4i x0 = *reinterpret_cast<const v4i*>(xa0 + kb * 32);
        const v4i x1 = *reinterpret_cast<const v4i*>(xa1 + kb * 32);
        const v4i y0 = *reinterpret_cast<const v4i*>(xa0 + KC + kb * 32);
        const v4i y1 = *reinterpret_cast<const v4i*>(xa1 + KC + kb * 32);
        const v4i qh = qv[QS][0][kb], ql = qv[QS][1][kb];
        acc[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x0, qh, acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x1, qh, acc[0][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x0, ql, acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x1, ql, acc[1][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(y0, qh, acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(y1, qh, acc[1][1], 0, 0, 0);
        acc[2][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(y0, ql, acc[2][0], 0, 0, 0);
        acc[2][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(y1, ql, acc[2][1], 0, 0, 0);
      }
    }
    if (sidx + 1 < nstages) store_stage(X, sidx + 1);
    __syncthreads();
    if (kc != NKC - 1) return;

    const uint32_t lane_base = base + 4 * h;  // row of output r = 0 of block 0
    if constexpr (SQ == 1) {  // u = 256 acc_hi + acc_lo, into the first set
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[0][blk][r] = (acc[0][blk][r] << 8) + acc[1][blk][r];
    } else if constexpr (SQ == 2) {  // u = 2^16 acc_hh + 2^8 acc_mid + acc_ll
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          acc[0][blk][r] = (acc[0][blk][r] << 16) + (acc[1][blk][r] << 8) + acc[2][blk][r];
    }
    if (wave_live && MODE == 0) {
      // per 32-row block: the lane's largest u against the bound, one wave-uniform branch;
      // a block passing on some lane tests its four groups of four values the same way, and
      // only a passing group its values one by one (row block 0 first)
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int qb = 0; qb < NQ; ++qb) {
          int m = acc[qb][blk][0];
#pragma unroll
          for (int r = 1; r < 16; ++r) m = max(m, acc[qb][blk][r]);
          if (__builtin_amdgcn_ballot_w64(m >= ui[qb]) == 0) continue;
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const int m4 = max(max(acc[qb][blk][4 * g4], acc[qb][blk][4 * g4 + 1]),
                               max(acc[qb][blk][4 * g4 + 2], acc[qb][blk][4 * g4 + 3]));
            if (__builtin_amdgcn_ballot_w64(m4 >= ui[qb]) == 0) continue;
#pragma unroll
            for (int r = 4 * g4; r < 4 * g4 + 4; ++r) {
              const int u = acc[qb][blk][r];
              if (__builtin_amdgcn_ballot_w64(u >= ui[qb]) != 0) {
                const uint32_t row = lane_base + (blk * 32 + 8 * (r >> 2) + (r & 3));
                if (u >= ui[qb]) {
                  if (cnt[qb] < uint32_t(a.caph))
                    out[qb][cnt[qb]] = make_uint2(__float_as_uint(gemm_units(u, dq[qb])), row);
                  ++cnt[qb];
                }
              }
            }
          }
        }
    } else if (wave_live) {
#pragma unroll
      for (int qb = 0; qb < NQ; ++qb)
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
          int m = kDead;
          if (a.allow == nullptr) {
#pragma unroll
            for (int r = 0; r < 16; ++r) m = max(m, acc[qb][blk][r]);
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const uint32_t row = lane_base + (blk * 32 + 8 * (r >> 2) + (r & 3));
              if (row < r_end && row_allowed(a.allow, a.rid[row])) m = max(m, acc[qb][blk][r]);
            }
          }
          if constexpr (MODE == 2) {
            // insert into the descending list: t' = clamp(m, top[t + 1], top[t]) from the
            // bottom up, each step reading the entry above before it changes
#pragma unroll
            for (int t = kTop8 - 1; t > 0; --t)
              top[qb][t] = max(top[qb][t], min(top[qb][t - 1], m));
            top[qb][0] = max(top[qb][0], m);
          } else if (q[qb] < a.nq) {
            const uint32_t grp = ((base >> 5) + blk) * 2 + h;
            if (grp < uint32_t(a.ngroups))
              a.gm[size_t(q[qb]) * a.ngroups + grp] =
                  m < kLive ? __builtin_inff() : gemm_units(m, dq[qb]);
          }
        }
    }
  };

  if (r_begin >= r_end) return;
  Stage A, B;
  load_stage(B, 0);
  load_stage(A, 1);
  store_stage(B, 0);
  __syncthreads();
  for (int sidx = 0; sidx < nstages; sidx += 2) {
    step(A, B, sidx, std::integral_constant<int, 0>{});
    if (sidx + 1 < nstages) step(B, A, sidx + 1, std::integral_constant<int, QF - 1>{});
  }

  if constexpr (MODE == 2) {
#pragma unroll
    for (int qb = 0; qb < NQ; ++qb) {
      if (q[qb] < a.nq) {
        float v[kTop8];
#pragma unroll
        for (int t = 0; t < kTop8; ++t)
          v[t] = top[qb][t] < kLive ? __builtin_inff() : gemm_units(top[qb][t], dq[qb]);
        float4* g = reinterpret_cast<float4*>(a.gm + size_t(q[qb]) * a.ngroups +
                                              (size_t(chunk) * 2 + h) * kTop8);
#pragma unroll
        for (int t = 0; t < kTop8 / 4; ++t)
          g[t] = make_float4(v[4 * t], v[4 * t + 1], v[4 * t + 2], v[4 * t + 3]);
      }
    }
  }
  if constexpr (MODE == 0) {
#pragma unroll
    for (int qb = 0; qb < NQ; ++qb) {
      if (q[qb] < a.nq) {
        const size_t seg = (size_t(q[qb]) * a.nchunks + chunk) * 2 + h;
        a.counts[seg] = min(cnt[qb], uint32_t(a.caph));
        if (cnt[qb] > uint32_t(a.caph)) a.ovf[q[qb]] = 1;
      }
    }
  }
}

template <int PD, int METRIC>
static void launch8_pm(int qb, int mode, int sq, hipStream_t s, int blocks, const GemmArgs& a) {
  const dim3 g(blocks), t(256);
  constexpr int OCC = PD <= 128 ? 3 : 2;  // Gemm8Occupancy
  if (sq == 2) {
    if (mode == 1)
      k_gemm8<PD, METRIC, 2, 1, 2, 2><<<g, t, 0, s>>>(a);
    else if (mode == 2)
      k_gemm8<PD, METRIC, 2, 2, 2, 2><<<g, t, 0, s>>>(a);
    else
      k_gemm8<PD, METRIC, 2, 0, 2, 2><<<g, t, 0, s>>>(a);
  } else if (sq) {
    if (mode == 1)
      k_gemm8<PD, METRIC, 2, 1, 2, 1><<<g, t, 0, s>>>(a);
    else if (mode == 2)
      k_gemm8<PD, METRIC, 2, 2, OCC, 1><<<g, t, 0, s>>>(a);
    else
      k_gemm8<PD, METRIC, 2, 0, OCC, 1><<<g, t, 0, s>>>(a);
  } else if (mode == 1) {
    k_gemm8<PD, METRIC, 2, 1><<<g, t, 0, s>>>(a);
  } else if (mode == 2) {
    k_gemm8<PD, METRIC, 2, 2, OCC><<<g, t, 0, s>>>(a);
  } else if (qb == 1) {
    k_gemm8<PD, METRIC, 1, 0><<<g, t, 0, s>>>(a);
  } else {
    k_gemm8<PD, METRIC, 2, 0, OCC><<<g, t, 0, s>>>(a);
  }
}

template <int PD>
static void launch8_pd(int metric, int qb, int mode, int sq, hipStream_t s, int blocks,
                       const GemmArgs& a) {
  if (metric == 0)
    launch8_pm<PD, 0>(qb, mode, sq, s, blocks, a);
  else
    launch8_pm<PD, 1>(qb, mode, sq, s, blocks, a);
}

int Gemm8Occupancy(size_t pd) { return pd <= 128 ? 3 : 2; }

int LaunchGemm8(size_t pd, int metric, int qb, int mode, int sq, hipStream_t s, int blocks,
                const GemmArgs& a) {
  if (qb != 1 && qb != 2) return SetError(kInternal, "GEMM8: query blocks per wave");
  if ((mode != 0 || sq) && qb != 2)
    return SetError(kInternal, "GEMM8: the sample pass and the SQ8 operand run 2 blocks");
  switch (pd) {
#define VDBG_PD8(P) \
  case P: launch8_pd<P>(metric, qb, mode, sq, s, blocks, a); break;
    VDBG_PD8(32) VDBG_PD8(64) VDBG_PD8(96) VDBG_PD8(128) VDBG_PD8(192) VDBG_PD8(256)
    VDBG_PD8(384) VDBG_PD8(512) VDBG_PD8(768) VDBG_PD8(960) VDBG_PD8(1024)
#undef VDBG_PD8
    default: return SetError(kNotSupported, "GEMM8: unsupported padded_dim");
  }
  return kOk;
}

// One wave per row: x' = x - c as int8 and the accumulator start, -ceil(||x'||^2 / 2) (L2)
// or c sum(x) (inner product).
__global__ __launch_bounds__(256) void k_to_i8(const float* __restrict__ X, uint32_t n, int pd,
                                               int c, int metric, int8_t* __restrict__ y,
                                               int* __restrict__ init) {
  const uint32_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= n) return;
  int sq = 0, sx = 0;
  for (int i = lane_id(); i < pd; i += kWave) {
    const int x = int(X[size_t(r) * pd + i]);
    const int xp = x - c;
    y[size_t(r) * pd + i] = int8_t(xp);
    sq += xp * xp;
    sx += x;
  }
  for (int o = kWave / 2; o > 0; o >>= 1) {
    sq += __shfl_xor(sq, o);
    sx += __shfl_xor(sx, o);
  }
  if (lane_id() == 0) init[r] = metric == 0 ? -((sq + 1) >> 1) : c * sx;
}

int MakeRows8(Ctx* c, hipStream_t s, const float* rows, size_t n, size_t pd, int metric,
              const RowStats& st, int8_t** out, int** init, int* shift) {
  *out = nullptr;
  *init = nullptr;
  *shift = 0;
  if (n == 0 || !Gemm8Supported(pd) || !st.all_int || !(st.max_abs <= 2048.f)) return kOk;
  const double lo = st.lo, hi = st.hi;
  if (hi - lo > 255.0) return kOk;
  // centre the rows' range in [-128, 127], leaving queries equal room on both sides
  const int cs = int(lo) + 128 - int((255.0 - (hi - lo)) / 2);
  // every accumulator start stays inside (-2^27, 2^27): live rows' u inside (-2^28, 2^28)
  if (double(pd) * 2048.0 * (std::abs(cs) + 1.0) >= 134217728.0) return kOk;
  int8_t* y = nullptr;
  int* in = nullptr;
  VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&y), n * pd));
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&in), n * sizeof(int));
  if (e != hipSuccess) {
    (void)hipFree(y);
    return SetError(kResourceExhausted, std::string("int8 rows: ") + hipGetErrorString(e));
  }
  k_to_i8<<<dim3(unsigned((n + 3) / 4)), 256, 0, s>>>(rows, uint32_t(n), int(pd), cs, metric, y, in);
  e = hipGetLastError();
  if (e != hipSuccess) {
    (void)hipFree(y);
    (void)hipFree(in);
    return SetError(kInternal, std::string("int8 rows: ") + hipGetErrorString(e));
  }
  *out = y;
  *init = in;
  *shift = cs;
  return kOk;
}

// Float rows to v = rint(x 2^ex), v = 256 h + l, stored [h | l] per K chunk of kc dims; each
// wave walks rows with a grid stride and raises the dataset's largest sum |v| and sum v^2
// once at the end (one atomic per wave, not per row).
__global__ __launch_bounds__(256) void k_to_i8_split(const float* __restrict__ X, uint32_t n,
                                                     int pd, int kc, int ex,
                                                     int8_t* __restrict__ y,
                                                     uint32_t* __restrict__ l1max,
                                                     unsigned long long* __restrict__ l2max) {
  const uint32_t waves = gridDim.x * 4;
  int m1 = 0;
  unsigned long long m2 = 0;
  for (uint32_t r = blockIdx.x * 4 + (threadIdx.x >> 6); r < n; r += waves) {
    int s1 = 0;
    unsigned long long s2 = 0;
    int8_t* out = y + size_t(r) * 2 * pd;
    for (int i = lane_id(); i < pd; i += kWave) {
      const int v = int(rintf(ldexpf(X[size_t(r) * pd + i], ex)));
      const int hi = (v + 128) >> 8;
      const int c = i / kc, o = i - c * kc;
      out[c * 2 * kc + o] = int8_t(hi);
      out[c * 2 * kc + kc + o] = int8_t(v - 256 * hi);
      s1 += v < 0 ? -v : v;
      s2 += (unsigned long long)(int64_t(v) * v);
    }
    for (int off = kWave / 2; off > 0; off >>= 1) {
      s1 += __shfl_xor(s1, off);
      s2 += __shfl_xor(s2, off);
    }
    m1 = max(m1, s1);
    m2 = s2 > m2 ? s2 : m2;
  }
  if (lane_id() == 0) {
    atomicMax(l1max, uint32_t(m1));
    atomicMax(l2max, m2);
  }
}

int MakeRows8Split(Ctx* c, hipStream_t s, const float* rows, size_t n, size_t pd,
                   const RowStats& st, int8_t** out, int* exp, float* l1max, float* l2max) {
  *out = nullptr;
  *exp = 0;
  *l1max = *l2max = 0.f;
  if (n == 0 || !Gemm8Supported(pd) || !(st.max_abs > 0.f) || !(st.max_abs <= 3.0e38f) ||
      !(st.xn_max > 0.f) || !(st.xn_max <= 3.0e38f))
    return kOk;
  // the largest ||x 2^ex|| at most 2^13.9, so every |v| < 2^14 and, with a query scaled the
  // same way, |sum v_x v_q| < 2^28
  const int ex = int(std::floor(13.9 - 0.5 * std::log2(double(st.xn_max))));
  int8_t* y = nullptr;
  uint32_t* m1 = nullptr;
  VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&y), n * pd * 2));
  hipError_t err = hipMalloc(reinterpret_cast<void**>(&m1), 16);
  if (err == hipSuccess) err = hipMemsetAsync(m1, 0, 16, s);
  if (err == hipSuccess) {
    const unsigned blocks = unsigned(std::min<size_t>((n + 3) / 4, size_t(c->cu_count) * 8));
    k_to_i8_split<<<dim3(blocks), 256, 0, s>>>(
        rows, uint32_t(n), int(pd), Gemm8KcSplit(int(pd)), ex, y, m1,
        reinterpret_cast<unsigned long long*>(m1 + 2));
    err = hipGetLastError();
  }
  uint32_t h[4] = {0, 0, 0, 0};
  if (err == hipSuccess) err = hipMemcpyAsync(h, m1, 16, hipMemcpyDeviceToHost, s);
  if (err == hipSuccess) err = hipStreamSynchronize(s);
  (void)hipFree(m1);
  if (err != hipSuccess) {
    (void)hipFree(y);
    return SetError(kInternal, std::string("int8 split rows: ") + hipGetErrorString(err));
  }
  unsigned long long q2 = 0;
  std::memcpy(&q2, h + 2, 8);
  *out = y;
  *exp = ex;
  *l1max = float(h[0]);
  *l2max = float(std::sqrt(double(q2)) * (1.0 + 1e-6));
  return kOk;
}

}  // namespace vdbg
