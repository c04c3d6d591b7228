// gemm.h -- what the ranking GEMMs of the flat/SQ8 scans share: the argument block, the row
// tile and K-chunk geometry, and the padded dimensions with compiled GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace vdbg {

typedef float v16f __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const float* X;      // fp32 rows (KIND 0)
  const uint16_t* X16; // fp16 rows (k_gemm16)
  const uint16_t* Q16; // fp16 B operand: -2 q (L2) or -q (inner product) (k_gemm16), or for
                       // SQ8 the scaled query operand as two fp16 parts [q][2][pd]
  const float* Qf;     // SQ8 split: per-query factor from split-GEMM to GEMM units
  const uint8_t* C;    // code rows (KIND 1)
  const float* rn;     // row norms of the GEMM form
  const uint32_t* rid; // MODE 1: original row id of each sample row
  const float* Qb;
  const float* T;
  const uint64_t* allow;
  const uint32_t* aw;  // k_gemm16 MODE 0: the filter as 32-bit words, or one all-ones word
  uint32_t aw_mask;    // ~0 with a filter, 0 without (every row then reads aw[0])
  uint2* cand;         // MODE 0: [(q * nchunks + chunk) * 2 + half][caph]
  uint32_t* counts;    // MODE 0: [(q * nchunks + chunk) * 2 + half]
  const int8_t* X8;    // k_gemm8: rows shifted to int8
  const int8_t* Q8;    // k_gemm8: queries shifted to int8
  const int* rn8;      // k_gemm8: accumulator start per row
  const int* Qd;       // k_gemm8: per-query constant between the integer GEMM and GEMM units
  const int* e8;       // k_gemm8 on SQ8 codes: the batch's query scale exponent (device)
  int* ovf;            // MODE 0: [q]
  float* gm;           // MODE 1: [q][ngroups] minimum GEMM value of each 16-row group
  int ngroups;
  uint32_t N;
  int nq, nqt;
  uint32_t chunk_rows;
  int nchunks, caph;
  int items;           // nqt * nchunks
  int per_xcd;         // items assigned to each of the 8 XCDs
  const int* gate;     // nullable: per-query int8 fitness [gate_n]; the launch runs only
  int gate_n, gate_on; // when (every query fits) == gate_on
};

// A gated launch: the batch's GEMM is chosen on the device (every query inside the int8
// GEMM's bounds, or not), the other launch exits at once.  Block-uniform; call it before
// any other barrier.
__device__ __forceinline__ bool gemm_gated_off(const GemmArgs& a) {
  if (a.gate == nullptr) return false;
  __shared__ int s_fit;
  if (threadIdx.x == 0) s_fit = 1;
  __syncthreads();
  for (int i = threadIdx.x; i < a.gate_n; i += blockDim.x)
    if (a.gate[i] == 0) s_fit = 0;
  __syncthreads();
  return (s_fit != 0) != (a.gate_on != 0);
}

constexpr int kGemmRows = 64;  // rows per LDS tile (two 32-row MFMA blocks)

// The int8 GEMM's compact sample pass keeps this many group minima per lane (a multiple of 4).
constexpr int kTop8 = 8;

// Dimensions staged per LDS pass: the whole row up to 128 dims, else the largest of
// 128/64/32/16 that divides it.
__host__ __device__ constexpr int GemmKc(int pd) {
  return pd <= 128 ? pd : (pd % 128 == 0 ? 128 : (pd % 64 == 0 ? 64 : (pd % 32 == 0 ? 32 : 16)));
}

// K chunk of the fp16 GEMM.  Rows up to 128 dims stage whole (the query fragments then load
// once); wider rows, and two-part float rows (split 2, staged as [h | l] per chunk), stage
// chunks of at most 64 dims (the largest multiple of 16 dividing pd), which keeps two
// staging register sets and two sets of query fragments (the next chunk's load a step
// ahead) within the wave's registers.
__host__ __device__ constexpr int Gemm16Kc(int pd, int split) {
  if (split != 2 && pd <= 128) return pd;
  if (split == 2 && pd <= 64) return pd;
  for (int kc = 64; kc > 16; kc -= 16)
    if (pd % kc == 0) return kc;
  return 16;
}

// The fp16 GEMM on float rows held as high halves (split 3) keeps each wave's query fragments
// for every K chunk in registers (one 32-query block per wave) when the rows span several
// chunks and the fragments fit: up to 512 dims (128 VGPRs of fragments).
constexpr int kGemm16ResMaxPd = 512;
inline bool Gemm16ResQueries(size_t pd) {
  return Gemm16Kc(int(pd), 3) < int(pd) && pd <= size_t(kGemm16ResMaxPd);
}

// K chunk of the int8 GEMM: the whole row up to 128 dims, else the largest of 128/64/32
// dividing it.
__host__ __device__ constexpr int Gemm8Kc(int pd) {
  return pd <= 128 ? pd : (pd % 128 == 0 ? 128 : (pd % 64 == 0 ? 64 : 32));
}

// K chunk of the int8 GEMM on float rows held in two int8 parts (stored per chunk as
// [h | l]): the whole row up to 64 dims, else 64 or 32 dims, which keeps both register sets
// of the two-part stage and query fragments within two blocks per CU.
__host__ __device__ constexpr int Gemm8KcSplit(int pd) {
  return pd <= 64 ? pd : (pd % 64 == 0 ? 64 : 32);
}

// Padded dimensions with compiled GEMM kernels; others scan exactly.
inline bool GemmSupported(size_t pd) {
  switch (pd) {
    case 16: case 32: case 48: case 64: case 80: case 96: case 112: case 128:
    case 192: case 256: case 384: case 512: case 768: case 960: case 1024:
      return true;
    default:
      return false;
  }
}

// Padded dimensions with int8 GEMM kernels (multiples of 32).
inline bool Gemm8Supported(size_t pd) { return pd % 32 == 0 && GemmSupported(pd); }

// int8 GEMM (gemm8.hip): qb query blocks of 32 per wave, mode 0 = threshold pass, 1 = group
// minima of the sample (qb 2).
// Blocks per CU of the int8 main pass with two query blocks per wave (its launch bounds):
// three for rows of at most 128 dims, whose kernel fits 168 registers, else two.
int Gemm8Occupancy(size_t pd);
// sq = 1: SQ8 codes against the two-part query operand (k_gemm8 SQ = 1, qb must be 2).
int LaunchGemm8(size_t pd, int metric, int qb, int mode, int sq, hipStream_t s, int blocks,
                const GemmArgs& a);

// fp16 GEMM (gemm16.hip): qb query blocks of 32 per wave (1 or 2), mode 0 = threshold pass
// into candidate buffers, 1 = group minima of the sample; split 1 = SQ8 codes against the
// two-part query operand (qb 2, both register sets on the same 32 queries), 2 = two-part
// float rows against the two-part query operand, 3 = float rows as high halves (qb 2, or
// qb 1 with resident query fragments where Gemm16ResQueries).
int LaunchGemm16(size_t pd, int metric, int qb, int mode, int split, hipStream_t s, int blocks,
                 const GemmArgs& a);

}  // namespace vdbg
