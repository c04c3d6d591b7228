// gemm16.hip -- the ranking GEMM of the flat scan for integer-valued data, on fp16 MFMA.
//
// When every row and query value is an integer of magnitude <= 2048, fp16 holds each value
// exactly, and so it holds -2 q (an even integer of magnitude <= 4096) and -q.  Every product
// of two such values is an integer below 2^23 and exact in fp32.  With R the largest row norm
// and |q| the query norm, every partial sum of
//     ||x||^2 + sum_i (-2 q_i) x_i        (L2)        or        sum_i (-q_i) x_i     (IP)
// is bounded by R^2 + 2 |q| R <= (|q| + R)^2 (Cauchy-Schwarz), so when (|q| + R)^2 < 2^24
// every partial sum is an integer that fp32 represents and the accumulation is exact in any
// order.  v_mfma_f32_32x32x16_f16 started from the row norms then yields exactly the value the
// fp32 GEMM forms as fma(-2, q.x, ||x||^2) (or -q.x), at 16 times the fp32 MFMA rate, with the
// threshold test reduced to one compare per value.  k_query_prep writes the fp16 B operand
// and clears a flag when a query of the batch falls outside these bounds; the batch then takes
// the fp32 GEMM.
#include <algorithm>
#include <string>
#include <type_traits>
#include <utility>

#include "gemm.h"
#include "vdbg_device.h"
#include "vdbg_internal.h"

namespace vdbg {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16-byte vector (plain loads)

// Block = 4 waves x (32 QB) queries each x one chunk of rows; block b takes work item
// (b % 8) * per_xcd + b / 8 so the items of one XCD are consecutive and share row chunks in
// its L2.  Rows stream through double-buffered 64-row LDS stages (K chunks of KC dims for
// wide rows), row norms through three slots.
//
// Operand layout of v_mfma_f32_32x32x16_f16: per 16-dim K block, lane l holds dims
// 8 (l / 32) .. 8 (l / 32) + 7 of row l % 32 (A, from LDS) and of query l % 32 (B, kept in
// VGPRs for the whole launch); lane l's 16 outputs are rows 8 (r / 4) + 4 (l / 32) + r % 4 of
// the 32-row block against query l % 32.  Each A fragment read from LDS feeds QB MFMAs.
//
// MODE 0: every value at or below the query's threshold T goes to the lane's candidate
// buffer (per query, chunk and lane half).  The test is one compare per value; only a value
// that passes on some lane of the wave (a wave-uniform branch) pays for the write.  Rows the
// filter excludes start their accumulators from NaN, which fails every compare.
// MODE 1: minimum value of each 16-row group (the rows one lane holds of a 32-row block).
//
// SPLIT (SQ8): rows are uint8 codes held as fp16 (exact), and the query operand B (fp32) is
// scaled by 2^sc and split into fp16 parts h + l (k_query_prep).  Both register sets hold the
// same 32 queries, one per part; every product is exact in fp32, the accumulators start from
// zero, and the epilogue forms fma(Qf, acc_h + acc_l, ||c scale||^2) (NaN for excluded rows)
// with Qf = -2 (L2) or -1 (IP) times 2^-sc: the GEMM value of the fp32 SQ8 GEMM up to the
// rounding bound k_query_prep accounts for.
//
// SPLIT 2 (float rows): rows scaled by 2^sx and split into fp16 h + l as well, stored per K
// chunk as [h | l]; per 16-dim block the wave runs x_h q_h into one accumulator and x_h q_l,
// x_l q_h into the other (x_l q_l, of relative size 2^-22, is left out), then the same
// epilogue.
//
// SPLIT 3 (float rows, one product): rows held as their h halves alone (fp16(x 2^sx), one
// part, whole rows as in the exact path) against the h part of the split query operand:
// x_h q_h, one MFMA per product, two distinct 32-query blocks per wave, and the epilogue
// fma(Qf, acc, norm).  The dropped x_h q_l + x_l q_h + x_l q_l is at most
// (2^-10 + 2^-22) |x_i q_i| per product; k_query_prep widens the query's bound by it.
//
// QRES (rows wider than one K chunk, SPLIT 3, one 32-query block per wave): the wave's query
// fragments for every K chunk stay in registers for the whole launch, so each stage loads
// only its rows.  Otherwise they are reloaded for every stage of every tile: at 384 dims
// with 64 queries per wave that was four times the row bytes through the vector cache, which
// then bounds the kernel.
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  [&]<int... I>(std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
  }(std::make_integer_sequence<int, N>{});
}

template <int PD, int METRIC, int QB, int MODE, int SPLIT, int QRES = 0>
__global__ __launch_bounds__(256, 2) void k_gemm16(GemmArgs a) {
  constexpr int KC = Gemm16Kc(PD, SPLIT);
  constexpr int NKC = PD / KC;
  constexpr int NKB = KC / 16;                     // 16-dim MFMA K blocks per stage
  constexpr int XP = SPLIT == 2 ? 2 : 1;           // fp16 parts per staged row value
  constexpr int XS = SPLIT == 2 ? 2 : 1;           // fp16 parts per stored row value
  constexpr int ROWW = XS * PD;                    // fp16 row width in halfs
  constexpr int SKC = XP * KC;                     // stage width in halfs
  constexpr int CSTR = XS * KC;                    // stored K chunk width in halfs
  constexpr int STR = SKC + 8;                     // LDS row stride in halfs (16 B padding)
  constexpr int VEC_PER_ROW = SKC / 8;             // uint4 = 8 halfs
  constexpr int VEC_PER_TILE = kGemmRows * VEC_PER_ROW;
  constexpr int VEC_PER_THREAD = (VEC_PER_TILE + 255) / 256;
  constexpr int NQB = (SPLIT == 1 || SPLIT == 2) ? 1 : QB;  // distinct 32-query blocks per wave
  constexpr int QT = 128 * NQB;                    // queries per block
  static_assert(PD % KC == 0 && KC % 16 == 0, "K chunking");
  static_assert(!SPLIT || QB == 2 || (SPLIT == 3 && QRES), "the split operand takes both register sets");
  static_assert(!QRES || (SPLIT == 3 && QB == 1 && NKC > 1), "resident queries: SPLIT 3, one block");
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][kGemmRows * STR];
  __shared__ __attribute__((aligned(16))) float xns[3][kGemmRows];

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
  const int q0 = qt * QT + wave * 32 * NQB;  // first query of the wave
  const bool wave_live = q0 < a.nq;
  const uint32_t r_begin = uint32_t(chunk) * a.chunk_rows;
  const uint32_t r_end = min(a.N, r_begin + a.chunk_rows);

  int q[NQB];
  float T[NQB];
  uint2* out[NQB];
  uint32_t cnt[NQB];
  float qf[NQB];  // split operands: the GEMM-unit factor of the lane's query
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    q[qb] = q0 + qb * 32 + j;
    qf[qb] = SPLIT ? a.Qf[min(q[qb], a.nq - 1)] : 1.f;
    cnt[qb] = 0;
    if constexpr (MODE == 0) {
      T[qb] = q[qb] < a.nq ? a.T[q[qb]] : -__builtin_inff();
      out[qb] = a.cand + ((size_t(q[qb]) * a.nchunks + chunk) * 2 + h) * size_t(a.caph);
    }
  }

  // Every load below is unconditional (addresses clamped into the rows, queries and norms
  // that exist), so each wave has a fixed count of loads in flight and the waits before the
  // LDS stores do not drain the prefetch early.  Lanes of queries past the batch read query
  // nq - 1; their values are never emitted.
  // Query fragments of a stage's K chunk.  With one chunk they load once; with several, the
  // next stage's fragments load a step ahead into the other set (QF sets in all).
  constexpr int QF = QRES ? NKC : (NKC > 1 ? 2 : 1);
  half8 qv[QF][QB][NKB];
  const uint16_t* qrow[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
    qrow[qb] = SPLIT == 3 ? a.Q16 + size_t(min(q[qb], a.nq - 1)) * 2 * PD + h * 8
               : SPLIT    ? a.Q16 + (size_t(min(q[0], a.nq - 1)) * 2 + qb) * PD + h * 8
                          : a.Q16 + size_t(min(q[qb], a.nq - 1)) * PD + h * 8;
  auto load_q = [&](int f, int kc) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        qv[f][qb][kb] = *reinterpret_cast<const half8*>(qrow[qb] + kc * KC + kb * 16);
  };
  if constexpr (QRES)
    static_for<NKC>([&](auto I) { load_q(decltype(I)::value, decltype(I)::value); });
  else
    load_q(0, 0);

  // lane offsets (in halfs) of the stage's 16-byte vectors: row f / VEC_PER_ROW, column
  // f % VEC_PER_ROW of the 64 x KC stage
  int voff[VEC_PER_THREAD];
  int vrow[VEC_PER_THREAD];
#pragma unroll
  for (int i = 0; i < VEC_PER_THREAD; ++i) {
    const int f = min(tid + 256 * i, VEC_PER_TILE - 1);
    vrow[i] = f / VEC_PER_ROW;
    voff[i] = vrow[i] * ROWW + (f % VEC_PER_ROW) * 8;
  }
  // The chunk's rows run as stages s = tile * NKC + kc (64 rows x KC dims each), staged
  // through registers into two LDS buffers.  Stage s + 2 is loaded while stage s is
  // multiplied, so each load has two stages of MFMA work to land:
  //   step s:  load stage s + 2 -> set Y;  MFMA on LDS buffer s % 2;
  //            store set X (stage s + 1, loaded during step s - 1) -> buffer (s + 1) % 2;
  //            barrier;  after a tile's last K chunk, its threshold test.
  // The sets swap roles each step (the loop body is unrolled twice).  Rows past r_end repeat
  // the last valid row and get a NaN accumulator start (SPLIT: a NaN norm), so no compare
  // passes them and no group minimum takes them.  Norms rotate through three slots per tile.
  struct Stage {
    u32x4 v[VEC_PER_THREAD];
    float n;
    uint32_t aw;  // filter bits of the lane's half of the tile (tiles start on multiples of 64)
  };
  const int ntiles = int((r_end - r_begin + kGemmRows - 1) / kGemmRows);
  const int nstages = ntiles * NKC;
  auto load_stage = [&](Stage& st, int sidx) {
    sidx = min(sidx, nstages - 1);  // past the end: a harmless repeat, so the count is fixed
    const int tile = sidx / NKC, kc = sidx - tile * NKC;
    const uint32_t base = r_begin + uint32_t(tile) * kGemmRows;
    const uint32_t valid = min(uint32_t(kGemmRows), r_end - base);  // >= 1
    const char* src = reinterpret_cast<const char*>(a.X16 + size_t(base) * ROWW + kc * CSTR);
    if (valid == kGemmRows) {  // a full tile: the precomputed lane offsets
#pragma unroll
      for (int i = 0; i < VEC_PER_THREAD; ++i)
        st.v[i] = *reinterpret_cast<const u32x4*>(src + uint32_t(voff[i]) * 2u);
    } else {  // rows past it read row valid - 1 (the same count of loads)
      const int over = int(valid) - 1;
#pragma unroll
      for (int i = 0; i < VEC_PER_THREAD; ++i) {
        const int o = voff[i] - max(0, vrow[i] - over) * ROWW;
        st.v[i] = *reinterpret_cast<const u32x4*>(src + uint32_t(o) * 2u);
      }
    }
    st.n = a.rn[base + min(uint32_t(tid & 63), valid - 1)];  // (the store applies validity)
    if constexpr (MODE == 0)  // a scan without a filter reads one all-ones word (mask 0)
      st.aw = a.aw[((base >> 5) + (uint32_t(tid & 63) >> 5)) & a.aw_mask];
  };
  auto store_stage = [&](const Stage& st, int sidx) {
    const int tile = sidx / NKC, kc = sidx - tile * NKC;
    const int buf = sidx & 1;
#pragma unroll
    for (int i = 0; i < VEC_PER_THREAD; ++i) {
      const int f = tid + 256 * i;
      if (VEC_PER_TILE % 256 == 0 || f < VEC_PER_TILE)
        *reinterpret_cast<u32x4*>(&xs[buf][vrow[i] * STR + (voff[i] - vrow[i] * ROWW)]) = st.v[i];
    }
    if (kc == 0 && tid < kGemmRows) {
      const uint32_t valid = min(uint32_t(kGemmRows), r_end - (r_begin + uint32_t(tile) * kGemmRows));
      // rows past r_end, and in MODE 0 rows the filter excludes, start from NaN
      const bool ok = uint32_t(tid) < valid && (MODE != 0 || ((st.aw >> (tid & 31)) & 1u));
      xns[tile % 3][tid] = ok ? (METRIC == 0 ? st.n : 0.f) : __builtin_nanf("");
    }
  };

  v16f acc[QB][2];
  // step s multiplies with query set s % 2 (QF = 2) and loads set (s + 1) % 2 for stage s + 1
  auto step = [&](Stage& X, Stage& Y, int sidx, auto fcur) {
    constexpr int QS = decltype(fcur)::value;  // the query fragment set of this step
    const int tile = sidx / NKC, kc = sidx - tile * NKC;
    const uint32_t base = r_begin + uint32_t(tile) * kGemmRows;
    if constexpr (QF == 2 && !QRES)  // the next stage's K chunk (a harmless repeat past the end)
      load_q(QS ^ 1, (kc + 1 == NKC) ? 0 : kc + 1);
    load_stage(Y, sidx + 2);
    // keep the scheduler from sinking Y's loads below the MFMAs (which would shorten the
    // time they have to land to a single step)
    __builtin_amdgcn_sched_barrier(0);
    if (kc == 0) {
      // accumulators start from the row norms (L2) or zero (inner product), NaN past r_end;
      // SPLIT: from zero (the epilogue adds the norms)
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        v16f init = {};
        if constexpr (!SPLIT) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float4 n4 =
                *reinterpret_cast<const float4*>(&xns[tile % 3][blk * 32 + 8 * g + 4 * h]);
            init[4 * g + 0] = n4.x;
            init[4 * g + 1] = n4.y;
            init[4 * g + 2] = n4.z;
            init[4 * g + 3] = n4.w;
          }
        }
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) acc[qb][blk] = init;
      }
    }
    // waves past the batch run the MFMAs too (on query nq - 1): no branch splits the
    // accumulator chains; their values are never emitted
    const uint16_t* xa0 = &xs[sidx & 1][j * STR + h * 8];
    const uint16_t* xa1 = xa0 + 32 * STR;
    auto mfma_stage = [&](auto qsel) {  // with query fragment set QI
      constexpr int QI = decltype(qsel)::value;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const half8 x0 = *reinterpret_cast<const half8*>(xa0 + kb * 16);
        const half8 x1 = *reinterpret_cast<const half8*>(xa1 + kb * 16);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          acc[qb][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x0, qv[QI][qb][kb], acc[qb][0], 0, 0, 0);
          acc[qb][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x1, qv[QI][qb][kb], acc[qb][1], 0, 0, 0);
        }
        if constexpr (SPLIT == 2) {  // x_l q_h into the cross-term accumulator
          const half8 y0 = *reinterpret_cast<const half8*>(xa0 + KC + kb * 16);
          const half8 y1 = *reinterpret_cast<const half8*>(xa1 + KC + kb * 16);
          acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(y0, qv[QI][0][kb], acc[1][0], 0, 0, 0);
          acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(y1, qv[QI][0][kb], acc[1][1], 0, 0, 0);
        }
      }
    };
    if constexpr (QRES)  // the stage's K chunk selects the resident set (one branch per set)
      static_for<NKC>([&](auto I) { if (kc == decltype(I)::value) mfma_stage(I); });
    else
      mfma_stage(std::integral_constant<int, QS>{});
    if (sidx + 1 < nstages) store_stage(X, sidx + 1);
    __syncthreads();
    if (kc != NKC - 1) return;

    // the value of output r of block blk for query block qb (in GEMM units)
    float xn[SPLIT ? 2 : 1][SPLIT ? 16 : 1];
    if constexpr (SPLIT) {
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 n4 = *reinterpret_cast<const float4*>(&xns[tile % 3][blk * 32 + 8 * g + 4 * h]);
          xn[blk][4 * g + 0] = n4.x;
          xn[blk][4 * g + 1] = n4.y;
          xn[blk][4 * g + 2] = n4.z;
          xn[blk][4 * g + 3] = n4.w;
        }
    }
    auto value = [&](int qb, int blk, int r) {
      if constexpr (SPLIT == 3)
        return fmaf(qf[qb], acc[qb][blk][r], xn[blk][r]);
      else if constexpr (SPLIT)
        return fmaf(qf[0], acc[0][blk][r] + acc[1][blk][r], xn[blk][r]);
      else
        return acc[qb][blk][r];
    };
    const uint32_t lane_base = base + 4 * h;  // row of output r = 0 of block 0
    if (wave_live && MODE == 0) {
      // Per 32-row block: the minimum of the lane's 16 values (NaN skipped) against the
      // threshold, one wave-uniform branch; a block passing on some lane tests its four groups
      // of four values the same way, and only a passing group its values one by one, a value
      // passing on some lane branching to the write.
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
          float m = value(qb, blk, 0);
#pragma unroll
          for (int r = 1; r < 16; ++r) m = fminf(m, value(qb, blk, r));
          if (__builtin_amdgcn_ballot_w64(m <= T[qb]) == 0) continue;
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const float m4 = fminf(fminf(value(qb, blk, 4 * g4), value(qb, blk, 4 * g4 + 1)),
                                   fminf(value(qb, blk, 4 * g4 + 2), value(qb, blk, 4 * g4 + 3)));
            if (__builtin_amdgcn_ballot_w64(m4 <= T[qb]) == 0) continue;
#pragma unroll
            for (int r = 4 * g4; r < 4 * g4 + 4; ++r) {
              const float v = value(qb, blk, r);
              if (__builtin_amdgcn_ballot_w64(v <= T[qb]) != 0) {
                const uint32_t row = lane_base + (blk * 32 + 8 * (r >> 2) + (r & 3));
                if (v <= T[qb]) {
                  if (cnt[qb] < uint32_t(a.caph))
                    out[qb][cnt[qb]] = make_uint2(__float_as_uint(v), row);
                  ++cnt[qb];
                }
              }
            }
          }
        }
    } else if (wave_live) {
      // fminf skips the NaN values of rows past r_end
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
          float m = __builtin_inff();
          if (a.allow == nullptr) {
#pragma unroll
            for (int r = 0; r < 16; ++r) m = fminf(m, value(qb, blk, r));
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const uint32_t row = lane_base + (blk * 32 + 8 * (r >> 2) + (r & 3));
              if (row < r_end && row_allowed(a.allow, a.rid[row])) m = fminf(m, value(qb, blk, r));
            }
          }
          if (q[qb] < a.nq) {
            const uint32_t grp = ((base >> 5) + blk) * 2 + h;
            if (grp < uint32_t(a.ngroups)) a.gm[size_t(q[qb]) * a.ngroups + grp] = m;
          }
        }
    }
  };

  if (r_begin >= r_end) return;  // (every planned chunk holds rows)
  Stage A, B;
  load_stage(B, 0);
  load_stage(A, 1);
  store_stage(B, 0);
  __syncthreads();
  for (int sidx = 0; sidx < nstages; sidx += 2) {
    step(A, B, sidx, std::integral_constant<int, 0>{});
    if (sidx + 1 < nstages) step(B, A, sidx + 1, std::integral_constant<int, QF - 1>{});
  }

  if constexpr (MODE == 0) {
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
      if (q[qb] < a.nq) {
        const size_t seg = (size_t(q[qb]) * a.nchunks + chunk) * 2 + h;
        a.counts[seg] = min(cnt[qb], uint32_t(a.caph));
        if (cnt[qb] > uint32_t(a.caph)) a.ovf[q[qb]] = 1;
      }
    }
  }
}

template <int PD, int METRIC>
static void launch16_pm(int qb, int mode, int split, hipStream_t s, int blocks,
                        const GemmArgs& a) {
  const dim3 g(blocks), t(256);
  if (split == 1) {
    if (mode == 0) k_gemm16<PD, METRIC, 2, 0, 1><<<g, t, 0, s>>>(a);
    else k_gemm16<PD, METRIC, 2, 1, 1><<<g, t, 0, s>>>(a);
  } else if (split == 2) {
    if (mode == 0) k_gemm16<PD, METRIC, 2, 0, 2><<<g, t, 0, s>>>(a);
    else k_gemm16<PD, METRIC, 2, 1, 2><<<g, t, 0, s>>>(a);
  } else if (split == 3) {
    if constexpr (Gemm16Kc(PD, 3) < PD && PD <= kGemm16ResMaxPd) {
      if (mode == 0 && qb == 1) {  // resident query fragments
        k_gemm16<PD, METRIC, 1, 0, 3, 1><<<g, t, 0, s>>>(a);
        return;
      }
    }
    if (mode == 0) k_gemm16<PD, METRIC, 2, 0, 3><<<g, t, 0, s>>>(a);
    else k_gemm16<PD, METRIC, 2, 1, 3><<<g, t, 0, s>>>(a);
  } else if (mode == 0) {
    if (qb == 1) k_gemm16<PD, METRIC, 1, 0, 0><<<g, t, 0, s>>>(a);
    else k_gemm16<PD, METRIC, 2, 0, 0><<<g, t, 0, s>>>(a);
  } else {
    k_gemm16<PD, METRIC, 2, 1, 0><<<g, t, 0, s>>>(a);
  }
}

template <int PD>
static void launch16_pd(int metric, int qb, int mode, int split, hipStream_t s, int blocks,
                        const GemmArgs& a) {
  if (metric == 0)
    launch16_pm<PD, 0>(qb, mode, split, s, blocks, a);
  else
    launch16_pm<PD, 1>(qb, mode, split, s, blocks, a);
}

int LaunchGemm16(size_t pd, int metric, int qb, int mode, int split, hipStream_t s, int blocks,
                 const GemmArgs& a) {
  if (qb != 1 && qb != 2) return SetError(kInternal, "GEMM16: query blocks per wave");
  if ((mode == 1 || split) && qb != 2 && !(split == 3 && mode == 0 && Gemm16ResQueries(pd)))
    return SetError(kInternal, "GEMM16: the sample pass and the split operand run 2 blocks");
  switch (pd) {
#define VDBG_PD16(P) \
  case P: launch16_pd<P>(metric, qb, mode, split, s, blocks, a); break;
    VDBG_PD16(16) VDBG_PD16(32) VDBG_PD16(48) VDBG_PD16(64) VDBG_PD16(80) VDBG_PD16(96)
    VDBG_PD16(112) VDBG_PD16(128) VDBG_PD16(192) VDBG_PD16(256) VDBG_PD16(384) VDBG_PD16(512)
    VDBG_PD16(768) VDBG_PD16(960) VDBG_PD16(1024)
#undef VDBG_PD16
    default: return SetError(kNotSupported, "GEMM path: unsupported padded_dim");
  }
  return kOk;
}

__global__ void k_to_f16(const float* __restrict__ x, size_t n, uint16_t* __restrict__ y) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i < n) y[i] = __builtin_bit_cast(uint16_t, _Float16(x[i]));
}

// Rows as their h halves alone: fp16(x 2^e).
__global__ void k_to_f16_scaled(const float* __restrict__ x, size_t n, int e,
                                uint16_t* __restrict__ y) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i < n) y[i] = __builtin_bit_cast(uint16_t, _Float16(ldexpf(x[i], e)));
}

// Two-part fp16 rows: x 2^e = h + l (h = fp16(x 2^e), l = fp16(x 2^e - h)), stored per
// K chunk of kc dims as [h | l].
__global__ void k_to_f16_split(const float* __restrict__ x, size_t n, int pd, int kc, int e,
                               uint16_t* __restrict__ y) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i >= n) return;
  const size_t r = i / pd;
  const int col = int(i - r * pd);
  const int c = col / kc, w = col - c * kc;
  const float v = ldexpf(x[i], e);
  const _Float16 hh = _Float16(v);
  const _Float16 ll = _Float16(v - float(hh));
  uint16_t* dst = y + r * 2 * pd + size_t(c) * 2 * kc + w;
  dst[0] = __builtin_bit_cast(uint16_t, hh);
  dst[kc] = __builtin_bit_cast(uint16_t, ll);
}

int MakeRows16(Ctx* c, hipStream_t s, const float* rows, size_t n, size_t pd, int* parts, int* exp,
               int* approx, const RowStats& st, uint16_t** out) {
  *out = nullptr;
  *parts = 1;
  *exp = 0;
  *approx = 0;
  if (n == 0 || !GemmSupported(pd) || !(st.max_abs <= 3.0e38f)) return kOk;
  const bool exact = st.all_int && st.max_abs <= 2048.f;
  if (!exact) {
    // scale so the largest magnitude lands in [2^14, 2^15)
    int ex = 0;
    if (st.max_abs > 0.f) (void)frexpf(st.max_abs, &ex);
    *exp = st.max_abs > 0.f ? 15 - ex : 0;
    if (c->fp16_single) *approx = 1; else *parts = 2;
  }
  uint16_t* y = nullptr;
  VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&y), n * pd * *parts * sizeof(uint16_t)));
  if (exact)
    k_to_f16<<<dim3(unsigned((n * pd + 255) / 256)), 256, 0, s>>>(rows, n * pd, y);
  else if (*approx)
    k_to_f16_scaled<<<dim3(unsigned((n * pd + 255) / 256)), 256, 0, s>>>(rows, n * pd, *exp, y);
  else
    k_to_f16_split<<<dim3(unsigned((n * pd + 255) / 256)), 256, 0, s>>>(
        rows, n * pd, int(pd), Gemm16Kc(int(pd), 2), *exp, y);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    (void)hipFree(y);
    return SetError(kInternal, std::string("fp16 rows: ") + hipGetErrorString(e));
  }
  *out = y;
  return kOk;
}

__global__ void k_u8_to_f16(const uint8_t* __restrict__ x, size_t n, uint16_t* __restrict__ y) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i < n) y[i] = __builtin_bit_cast(uint16_t, _Float16(float(x[i])));
}

int MakeCodes16(Ctx* c, hipStream_t s, const uint8_t* codes, size_t n, size_t pd, uint16_t** out) {
  *out = nullptr;
  if (n == 0 || !GemmSupported(pd)) return kOk;
  uint16_t* y = nullptr;
  VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&y), n * pd * sizeof(uint16_t)));
  k_u8_to_f16<<<dim3(unsigned((n * pd + 255) / 256)), 256, 0, s>>>(codes, n * pd, y);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    (void)hipFree(y);
    return SetError(kInternal, std::string("fp16 codes: ") + hipGetErrorString(e));
  }
  *out = y;
  return kOk;
}

}  // namespace vdbg
