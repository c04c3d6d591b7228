// vdbg_internal.h -- host-side structures shared by the C ABI and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <mutex>
#include <string>
#include <atomic>
#include <vector>

#include "../../include/vdbg.h"

namespace vdbg {

// Status codes, numbered as vdb::Status::Code (include/vdb/status.h:14-26).
enum Code : int {
  kOk = VDBG_OK,
  kInvalidArgument = VDBG_INVALID_ARGUMENT,
  kNotFound = VDBG_NOT_FOUND,
  kFailedPrecondition = VDBG_FAILED_PRECONDITION,
  kResourceExhausted = VDBG_RESOURCE_EXHAUSTED,
  kNotSupported = VDBG_NOT_SUPPORTED,
  kInternal = VDBG_INTERNAL,
};

int SetError(int code, const std::string& msg);  // records the thread's message, returns code
int BestHostKernelSet();  // the host CPU's best distance kernel set (host_cpu.cc)

// File formats (files.cc): CRC32C of every vdb file, and Segment::Open's vectors.f32 checks
// (src/storage/segment_reader.cc:37-55); *data is the first row, *rows the header's count.
uint32_t Crc32c(const void* data, size_t n);
int CheckSegmentVectors(const void* file, size_t len, size_t dim, int metric,
                        uint64_t expect_rows, int verify_crc, const float** data,
                        uint64_t* rows);

#define VDBG_HIP(expr)                                                                  \
  do {                                                                                  \
    hipError_t e_ = (expr);                                                             \
    if (e_ != hipSuccess)                                                               \
      return ::vdbg::SetError(e_ == hipErrorOutOfMemory ? ::vdbg::kResourceExhausted    \
                                                        : ::vdbg::kInternal,            \
                              std::string(#expr) + ": " + hipGetErrorString(e_));      \
  } while (0)

#define VDBG_RETURN_IF_ERROR(expr) \
  do {                             \
    int rc_ = (expr);              \
    if (rc_ != 0) return rc_;      \
  } while (0)

// Value statistics of a resident row set, used to decide when the GEMM formulation is
// exact (integer-valued data with bounded sums) and to bound its rounding otherwise.
struct RowStats {
  float lo = 0.f, hi = 0.f;  // min and max over all stored values (padding included)
  float max_abs = 0.f;
  float xn_max = 0.f;        // largest row norm ||x||^2
  int all_int = 1;           // every value is an integer
};

// Grow-only device scratch, carved into aligned slices per call.  A fixed workspace wraps
// memory it does not own (the allocation-free entry point's static array) and never grows:
// reserve() beyond its capacity is ResourceExhausted.
struct Workspace {
  void* base = nullptr;
  size_t cap = 0;
  size_t used = 0;
  bool fixed = false;
  const char* name = "workspace";  // for the fixed workspace's capacity error
  hipEvent_t done = nullptr;  // recorded after the last launch of the last call that used it
  hipStream_t last = nullptr;  // the stream that call ran on (compared, never used)
  bool used_once = false;      // `last` is set
  int reserve(size_t bytes);  // makes `bytes` available (may reallocate; call before carving)
  template <class T>
  T* take(size_t count) {
    size_t off = (used + 255) & ~size_t(255);
    used = off + count * sizeof(T);
    return reinterpret_cast<T*>(static_cast<char*>(base) + off);
  }
  void release();
};

// Orders one call's use of a workspace after every earlier call's, whatever stream each
// ran on: the constructor makes stream s wait (on the device) for the event the previous
// user recorded, unless that user ran on s itself (the stream orders them); the destructor
// records it on s, after every launch the call queued that reads the workspace.  The
// host-side order comes from the owner's mutex.
class WsUse {
 public:
  WsUse(Workspace* w, hipStream_t s);
  ~WsUse();
  int status() const { return rc_; }

 private:
  Workspace* w_;
  hipStream_t s_;
  int rc_ = 0;
};

struct ProfEntry {
  std::string name;
  hipEvent_t start, stop;
};

struct ScanScratch;  // below

struct Ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::recursive_mutex mu;
  Workspace ws;   // per-call scratch
  Workspace ws2;  // scratch of the exact re-scan that runs while ws is live
  Workspace wsc;  // scratch of the filtered scan's row compaction (kept across calls)
  hipEvent_t wsc_done = nullptr;  // recorded after the last launch reading wsc
  uint32_t* host_pinned = nullptr;  // small pinned staging for counters
  // ReadWords: coherent pinned words the device publishes into ([0] sequence, then data),
  // their device address, and the last sequence number used
  uint32_t* host_flag = nullptr;
  uint32_t* host_flag_dev = nullptr;
  uint32_t flag_seq = 0;
  // StageHost's blocks: pinned host memory mapped into the device (coherent: the device's
  // writes reach the host without a copy engine), outgrown host blocks (freed with the
  // context), and the device block ([256-byte completion counter][inputs][outputs])
  uint8_t* stage_h = nullptr;
  uint8_t* stage_h_dev = nullptr;
  size_t stage_h_cap = 0;
  std::vector<uint8_t*> stage_h_retired;
  uint8_t* stage_d = nullptr;
  size_t stage_d_cap = 0;
  std::mutex flag_mu;  // one readback through host_flag at a time (scan lanes may run on
                       // worker threads of one call)
  std::mutex prof_mu;  // guards pending / free_events against those threads
  bool profiling = false;
  std::vector<ProfEntry> pending;
  std::vector<hipEvent_t> free_events;
  std::map<std::string, std::pair<double, uint64_t>> prof;  // name -> (ms, launches)
  std::atomic<uint64_t> last_fallbacks{0};
  // exact re-scans of fallback passes queued without a host read (RunScan), accumulated on
  // the device until vdbg_last_fallbacks reads them
  bool gate_fallbacks = true;
  uint32_t* fb_dev = nullptr;
  std::atomic<bool> fb_dev_used{false};
  bool fb_accumulate = false;  // set while one call runs several scans (ResetFallbacks)
  std::vector<ScanScratch*> lanes;  // the collection search's side-by-side scan lanes
  Workspace wcomb;                  // the collection search's combined rows (kept across calls)
  hipEvent_t wcomb_done = nullptr;  // recorded after the last launch reading wcomb
  bool combine_segments = true;     // small flat segments scanned as one (collection.hip)
  int collection_lanes = 2;         // lanes a collection search may use (0: none)
  bool lane_threads = true;         // each lane issued by its own host thread
  std::atomic<int> last_gemm_bits{0};  // input width of the last scan's main GEMM: 32, 16, 8, 0
  std::atomic<const int*> last_gemm_gate{nullptr};  // when the batch chose its GEMM on the
  std::atomic<int> last_gemm_gate_n{0};  // device: the per-query int8 flags (all 1: int8)
  int cu_count = 256;
  int live_datasets = 0;       // datasets created on this context and not yet destroyed
  int kset = 2;                // distance kernel set: 0 scalar, 1 avx2, 2 avx512 (KernelSet)
  int test_fallbacks = 0;      // testing: 1 fails every first certificate (second chance),
                               // 2 also every second one (exact re-scan)
  bool fp16_gemm = true;       // flat and SQ8 scans may rank on the fp16 GEMM (gemm16.hip)
  bool fp16_single = true;     // new float datasets hold their fp16 h halves alone
                               // (x16_approx, gemm16.hip SPLIT 3) instead of h + l pairs
  bool int8_gemm = true;       // integer flat rows may rank on the int8 GEMM (gemm8.hip)
  bool ivf_row_sums = true;    // IVF-PQ L2 scans rank on per-row term-2 sums (k_ivf_scan_rs)
  double int8_float_min_work = 2e10;  // float rows: smallest N nq pd for the int8 GEMM
  int host_threads = 0;        // host threads of the HNSW walk; 0 = DefaultHostThreads()
  vdbg_ctx* handle = nullptr;  // the C-ABI handle that owns this context
};

// What an exhaustive scan reads: fp32 rows (kind 0, flat) or SQ8 codes (kind 1), the
// GEMM-form row norms, and a bit-reversed strided sample of rows built on first use; or PQ
// codes (kind 2, scored by ADC against per-query tables of pd = m x 256 floats, ScoreScan
// only).
struct ScanSource {
  int kind = 0;
  int pq_m = 0;                 // kind 2: bytes per code
  const float* X = nullptr;     // kind 0: n x pd rows
  const uint32_t* Xmap = nullptr;  // kind 0, nullable: row r of this source is row Xmap[r] of
                                   // X (a compacted source reading its parent's fp32 rows)
  const uint16_t* X16 = nullptr;  // rows as fp16 for the fp16 GEMM (gemm16.hip), or null:
                                  // kind 0 integer rows exactly (x16_parts 1), kind 0 float
                                  // rows as 2^x16_exp-scaled h + l pairs (x16_parts 2, [h|l]
                                  // per K chunk), kind 1 codes exactly (x16_parts 1)
  int x16_parts = 1;
  int x16_exp = 0;
  int x16_approx = 0;           // kind 0 float rows held as fp16(x 2^x16_exp) alone (one part,
                                // ranked under a widened bound, gemm16.hip SPLIT 3)
  const int8_t* X8 = nullptr;   // kind 0 rows for the int8 GEMM (gemm8.hip), or null: integer
                                // rows - c8 (x8_parts 1), or float rows 2^x8_exp-scaled and
                                // rounded, as int8 h + l pairs ([h | l] per K chunk, x8_parts 2)
  const int* init8 = nullptr;   // x8_parts 1: its accumulator start per row
  int c8 = 0;
  int x8_parts = 1;
  int x8_exp = 0;
  float x8_l1max = 0.f;         // x8_parts 2: the largest sum |v| and |v| of a row's integers
  float x8_l2max = 0.f;
  const uint8_t* C = nullptr;   // kind 1: n x pd codes
  const float* rn = nullptr;    // ||x||^2 (flat) or ||code * scale||^2 (SQ8)
  const float* vmin = nullptr;  // SQ8 quantizer (device)
  const float* scale = nullptr;
  uint32_t N = 0;
  int pd = 0, metric = 0;
  float rmag = 0.f;             // row magnitude term of the rounding bound
  float rn_max = 0.f;           // SQ8: max ||code * scale||^2 (the int8 GEMM's row-start bound)
  RowStats stats;               // flat: value statistics for the exactness test
  float* SX = nullptr;          // sample rows (kind 0)
  uint16_t* SX16 = nullptr;     // sample rows of X16 (same layout)
  int8_t* SX8 = nullptr;        // sample rows of X8
  int* Sinit8 = nullptr;
  uint8_t* SC = nullptr;        // sample codes (kind 1)
  float* Srn = nullptr;
  uint32_t* Sid = nullptr;
  uint32_t Smax = 0;
  uint32_t SN = 0;              // rows the sample's positions spread over (N when gathered;
                                // an appendable dataset's sample may trail its rows)
  void* Sbuf = nullptr;         // the sample's allocation when the source owns it
};

struct Dataset {
  Ctx* ctx = nullptr;
  float* rows = nullptr;   // n x pd
  float* norms = nullptr;  // n row norms (fp32, ||x||^2)
  uint16_t* rows16 = nullptr;  // fp16 copy of the rows (see ScanSource::X16)
  int rows16_parts = 1, rows16_exp = 0, rows16_approx = 0;
  int8_t* rows8 = nullptr;     // int8 copy of the rows (see ScanSource::X8)
  int* init8 = nullptr;
  int c8 = 0;
  int rows8_parts = 1, rows8_exp = 0;
  float rows8_l1max = 0.f, rows8_l2max = 0.f;
  size_t n = 0, dim = 0, pd = 0;
  int metric = 0;
  RowStats stats;
  ScanSource src;          // the flat scan's view of these rows
  int live_indexes = 0;    // SQ8 / IVF-PQ indexes over these rows not yet destroyed (ctx mu)
  uint64_t* ext_ids = nullptr;  // n external ids (device) for the collection merge, or null
  bool ext_unique = false;      // no two rows share an external id (checked when they are set)
  // appendable datasets (vdb's MutableSegment): rows, norms and external ids are reserved
  // for cap rows and grow in place; no fp16 / int8 copies are kept
  bool appendable = false;
  size_t cap = 0;
  std::vector<void*> retired;  // replaced samples, freed once the device is idle (growth,
                               // destroy): searches queued earlier may still read them
};

// SQ8 codes of a dataset's rows (HnswSq8Index's codes_ and Sq8Quantizer,
// src/index/hnsw/hnsw_index.h:89-95, without the graph).
struct HnswGraph;  // hnsw_host.h

struct Sq8Index {
  Dataset* ds = nullptr;
  HnswGraph* graph = nullptr;     // the VDBHSQ81 file's graph (host), or null
  std::vector<uint8_t> codes_h;   // host copy of the codes for the graph walk (with a graph)
  uint8_t* codes = nullptr;  // n x pd
  uint16_t* codes16 = nullptr;  // n x pd, the codes as fp16 (ScanSource::X16 of the scan)
  float* yn = nullptr;       // ||code * scale||^2 per row
  float* vmin = nullptr;     // pd (device)
  float* scale = nullptr;
  std::vector<float> vmin_h, scale_h;
  ScanSource src;
};

// Brackets a launch with events when the context is profiling.
class ProfScope {
 public:
  ProfScope(Ctx* c, const char* name, hipStream_t s);
  ~ProfScope();

 private:
  Ctx* c_;
  hipStream_t s_;
  ProfEntry e_;
  bool on_;
};

// IvfPqIndex (src/index/quant/ivf_pq.h:42-81) made resident: coarse centroids (also a
// dataset, so the coarse probe reuses the exhaustive scan), the PQ codebook, the inverted
// lists in CSR form (ids ascending inside a list, codes contiguous) and, for L2, the
// precomputed per-list tables.
struct IvfIndex {
  Dataset* ds = nullptr;             // the segment's rows (Rerank reads them)
  vdbg_dataset* coarse_ds = nullptr; // nlist x pd coarse centroids
  int nlist = 0, m = 0, dsub = 0, dim = 0, pd = 0, metric = 0;
  float* cen = nullptr;              // m x 256 x dsub
  uint32_t* off = nullptr;           // nlist + 1
  uint32_t* ids = nullptr;           // n
  uint8_t* codes = nullptr;          // n x m
  float* term2 = nullptr;            // nlist x m x 256, or null
  float* rowsum = nullptr;           // n: sum_j term2[l][j][code_j] per CSR row (with term2)
  float* t2abs = nullptr;            // nlist: sum_j max_c |term2[l][j][c]| (with term2)
  std::vector<float> coarse_h, cen_h;
  std::vector<uint32_t> off_h;
};

// The IVF-PQ list scan of a batch (ivf_kernels.hip), as IvfSearch (ivf_api.hip) hands it over.
struct IvfScanArgs {
  const float* Q;
  int pd, dim, m, dsub, metric;
  const float* coarse;
  const float* cen;
  const uint32_t* off;     // nlist + 1
  const uint32_t* ids;     // CSR row ids
  const uint8_t* codes;    // CSR codes, m bytes per row
  const float* term2;      // nullable
  const float* qtab;       // [nq][m*256]: 2*(-<q_j,C>) (L2 with term2) or -<q_j,C> (IP)
  const uint32_t* probe;   // [nq][nprobe] list ids, nearest first
  const float* probe_d;    // [nq][nprobe] coarse distances
  int nprobe, nq;
  const uint64_t* allow;
  int R;                   // TopK capacity max(depth, k)
  uint32_t* out_ids;       // [nq][R]
  float* out_d;
  uint64_t* dc;            // [nq] distance computations (nullable)
  uint64_t dc_base;        // nlist: the coarse distances
  int count_top;           // add the candidates handed to Rerank
  int ondemand;            // the table does not fit LDS (m > 32): entries computed per lookup
  const float* rowsum;     // per CSR row term-2 sums (nullable: the per-list table scan)
  const float* t2abs;      // per list bound of sum_j |term2| (with rowsum)
  const float* qmax;       // [nq][m] max_c |qtab[q][j][c]| (with rowsum)
  uint32_t nlist;          // probes at or past it (no-id slots) scan as empty lists
};

// PqFlatIndex (src/index/quant/ivf_pq.h:12-36) made resident: the PQ codebook and every
// row's code, scanned in full by ADC against per-query tables.
struct PqFlatIndex {
  Dataset* ds = nullptr;   // the segment's rows (Rerank reads them)
  int m = 0, dsub = 0;
  float* cen = nullptr;    // m x 256 x dsub (device)
  uint8_t* codes = nullptr;  // n x m
  std::vector<float> cen_h;
  bool trained = false;    // false for an index built over no rows (no codebook)
};

// ---------------------------------------------------------------- launchers

// ProductQuantizer::train (pq.cc:14-41) of n device rows at `stride` on the GPU's k-means,
// with IndexOptions' seed and sample cap and `iters` Lloyd iterations.
int PqTrainRows(Ctx* c, const float* data, size_t n, size_t stride, size_t dim, size_t m,
                uint64_t seed, size_t max_points, size_t iters, std::vector<float>* centroids,
                hipStream_t s);
// ProductQuantizer::encode (pq.cc:43-57) of n rows, of their residuals against
// coarse[assign] when coarse is not null.
int PqEncode(Ctx* c, const float* X, uint32_t n, int pd, int dim, const float* coarse,
             const uint32_t* assign, const float* cen, int m, int dsub, uint8_t* codes,
             hipStream_t s);

int LaunchRowStats(Ctx* c, hipStream_t s, const float* rows, size_t n, size_t pd,
                   float* norms, RowStats* out);
// The fp16 copy of rows whose values are all integers of magnitude <= 2048 (each exactly
// representable), used by the exact-integer GEMM; *out stays null when not applicable.
// SQ8 codes as fp16 (exact) for the split fp16 GEMM; null when pd has no GEMM kernel.
int MakeCodes16(Ctx* c, hipStream_t s, const uint8_t* codes, size_t n, size_t pd, uint16_t** out);
// fp16 copy of flat rows for the fp16 GEMM: integer rows of magnitude <= 2048 exactly
// (*parts 1), other finite rows as h + l parts of x 2^*exp (*parts 2); null when pd has no
// GEMM kernel.
int MakeRows16(Ctx* c, hipStream_t s, const float* rows, size_t n, size_t pd, int* parts, int* exp,
               int* approx,
               const RowStats& st, uint16_t** out);
// int8 copy of integer rows spanning at most 256 values, shifted by *shift, with each row's
// accumulator start (gemm8.hip); *out stays null when not applicable.
int MakeRows8(Ctx* c, hipStream_t s, const float* rows, size_t n, size_t pd, int metric,
              const RowStats& st, int8_t** out, int** init, int* shift);
// Float rows as two int8 parts for the int8 GEMM (gemm8.hip, SQ = 2): v = rint(x 2^*exp) with
// ||v|| < 2^14, v = 256 h + l, stored [h | l] per Gemm8KcSplit chunk; *l1max / *l2max the
// largest sum |v| / ||v|| of a row.  *out stays null when not applicable.
int MakeRows8Split(Ctx* c, hipStream_t s, const float* rows, size_t n, size_t pd,
                   const RowStats& st, int8_t** out, int* exp, float* l1max, float* l2max);

// Top-kk rows by the source's exact distance for nq queries (device pointers).  Scratch comes
// from ws (the pipeline) and ws2 (the exact re-scan of uncertified queries), by default the
// context's own; with fixed workspaces and a source whose sample is built, nothing is
// allocated (kk <= 240).
int RunScan(Ctx* c, ScanSource* src, const float* Q, size_t nq, size_t kk,
            const uint64_t* allow, uint32_t* out_ids, float* out_d, hipStream_t s,
            Workspace* ws = nullptr, Workspace* ws2 = nullptr);
// Top-kk by the source's exact score without a ranking GEMM: every allowed row scored, wave
// top-k per row split then a merge (kk <= 240), or a segmented sort (kk up to 10,000).
int ScoreScan(Ctx* c, const ScanSource& src, const float* Q, size_t nq, size_t kk,
              const uint64_t* allow, uint32_t* out_ids, float* out_d, hipStream_t s);
// Sets up the allocation-free flat search's scratch on `device` (its address there), once per
// device; called by vdbg_ctx_create with the device current (noalloc.hip).
int InitNoAllocScratch(int device);
// Fills n 32-bit words with v on stream s (a kernel, so a captured graph holds no memset).
int Fill32(void* p, uint32_t v, size_t n, hipStream_t s);
// Exact fp32 distances of `depth` candidate rows per query, the k smallest.
// rows (nullable): the dataset's scan source, whose int8 copy of integer rows serves
// exact-integer queries.
int Rerank(Ctx* c, const float* X, int pd, int metric, const float* Q, size_t nq,
           const uint32_t* cand, size_t depth, size_t k, uint32_t* out_ids, float* out_d,
           hipStream_t s, const ScanSource* rows = nullptr);
int Sq8Train(Ctx* c, const Dataset* ds, float* vmin_dev, float* scale_dev, hipStream_t s);
int Sq8Encode(Ctx* c, const Dataset* ds, const float* vmin_dev, const float* scale_dev,
              uint8_t* codes, float* yn, hipStream_t s, bool codes_given = false);
// Top-kk for kk beyond the wave kernels (up to 10,000): exact distance of every allowed row
// per query, segmented sort.
int ExactScanAll(Ctx* c, const ScanSource& src, const float* Q, size_t nq, size_t kk,
                 const uint64_t* allow, uint32_t* out_ids, float* out_d, hipStream_t s);
// Rerank for depths beyond 256 candidates per query.
int RerankLarge(Ctx* c, const float* X, int pd, int metric, const float* Q, size_t nq,
                const uint32_t* cand, size_t depth, size_t k, uint32_t* out_ids, float* out_d,
                hipStream_t s);
// Sorts nseg key segments (int offsets off_dev[0..nseg]) from keys into keys_alt and writes
// the first K of each as (id, dist), padded with (UINT32_MAX, +inf).
int SortSegmentsTopK(Ctx* c, uint64_t* keys, uint64_t* keys_alt, const int* off_dev, int nseg,
                     int total, int K, uint32_t* out_ids, float* out_d, hipStream_t s);
// RunScan under an optional filter; compacts the allowed rows when they are few.
// CollectionImpl::Search's merge (segment_kernels.hip): hits of every part ordered by
// (dist, part, row), first hit of each external id kept.
struct MergeArgs {
  int nq, nparts, k;
  const float* part_d;        // [nparts][nq][k]
  const uint32_t* part_rows;  // [nparts][nq][k], UINT32_MAX padded
  const uint64_t* ext;        // external ids, part p row r at ext[part_off[p] + r]
  const uint64_t* part_off;   // (null: ext[r], one part)
  uint64_t* out_ext;          // [nq][k], UINT64_MAX padded
  float* out_d;
  const uint64_t* const* ext_parts = nullptr;  // or row r of part p at ext_parts[p][r]
  int kout = 0;  // results per query written to out_ext / out_d ([nq][kout]); 0: k
};
int MergeParts(Ctx* c, const MergeArgs& a, hipStream_t s);
// PrepareQuery + NormalizeVector for nq raw queries into padded rows; waits for the result
// (a query with a non-finite value, or a zero query under cosine, is InvalidArgument).
int PrepareQueries(Ctx* c, const float* raw, size_t nq, size_t dim, size_t pd, int metric,
                   float* out, hipStream_t s);
// The same in two halves, so that host work can run between the launch and the wait: the
// launch queues the preparation and its per-query status, the check waits for the status and
// turns it into the error (the pending status is freed on the stream either way).
struct PrepPending {
  int* st = nullptr;
  size_t nq = 0;
  hipStream_t s = nullptr;
  PrepPending() = default;
  PrepPending(const PrepPending&) = delete;
  PrepPending& operator=(const PrepPending&) = delete;
  ~PrepPending();
};
int PrepareQueriesLaunch(Ctx* c, const float* raw, size_t nq, size_t dim, size_t pd, int metric,
                         float* out, hipStream_t s, PrepPending* pp);
int PrepareQueriesCheck(PrepPending* pp);
// The scratch of one scan pipeline other than the context's own (a lane of a collection
// search running several segments' scans side by side on their own streams).
struct ScanScratch {
  Workspace ws, ws2, wsc;          // as Ctx::ws, ws2, wsc
  hipEvent_t wsc_done = nullptr;   // as Ctx::wsc_done
  hipStream_t stream = nullptr;
  hipEvent_t done = nullptr;       // recorded after the lane's last launch of a call
  ~ScanScratch();
};
// Rows gathered by id into compact arrays, every part in one launch: per row, 16-byte columns
// of up to three row arrays (fp32 rows or codes, the fp16 copy, the int8 copy) and one column
// for the row's scalars (norm, int8 accumulator start, external id).
struct GatherParts {
  const uint4* a;  uint4* ao;  uint32_t wa;   // fp32 rows or codes (wa columns per row)
  const uint4* b;  uint4* bo;  uint32_t wb;   // fp16 copy
  const uint4* c8; uint4* co;  uint32_t wc;   // int8 copy
  const float* rn; float* rno;
  const int* i8;   int* i8o;                  // nullable
  const uint64_t* ext; uint64_t* exto;        // nullable
  const uint32_t* ids;                        // null: rows 0..n-1
  uint32_t n;
};
// Masks of at most kCompactBlockWords words allowing at most kCompactBlockIds rows compact
// in one block each (k_compact_block, k_compact_multi): up to kMultiParts masks in one launch,
// and up to kMultiParts row sets gathered in another.
constexpr int kCompactBlockWords = 32 * 1024;
constexpr uint32_t kCompactBlockIds = 65536;
constexpr int kMultiParts = 16;
struct CompactMulti {
  const uint64_t* w[kMultiParts];
  uint32_t* ids[kMultiParts];
  uint32_t nwords[kMultiParts], N[kMultiParts];
  int n;
};
struct GatherMulti {
  GatherParts g[kMultiParts];
  uint64_t start[kMultiParts + 1];  // part p's threads: [start[p], start[p + 1])
  int n;
};
int CompactGatherMulti(const CompactMulti& cm, const GatherMulti& gm, hipStream_t s);

// The exhaustive scan under dense allow words (null: every row): rows compacted when at most
// half are allowed.  allowed: the number of allowed rows when the caller knows it (read on the
// device otherwise, one host round trip); lane: scratch other than the context's.
int ScanMasked(Ctx* c, ScanSource* src, const float* Q, size_t nq, size_t kk,
               const uint64_t* allow, uint32_t* out_ids, float* out_d, hipStream_t s,
               int64_t allowed = -1, ScanScratch* lane = nullptr);
int BuildSample(Ctx* c, ScanSource* src, hipStream_t s);
// Starts a call's count of exact re-scans at zero (host and, when needed, device).
int ResetFallbacks(Ctx* c, hipStream_t s);
// The sample rows of an N-row source, its buffer size, and the gather into caller memory
// (at least SampleBytes, any alignment) for sources that live one call, of at most cap rows
// (SampleWant: the rows that call's scan uses).  SampleWant is the sample size RunScan plans.
uint32_t SampleRows(uint32_t N);
size_t SampleBytes(const ScanSource& src, uint32_t smax);
int GatherSample(Ctx* c, ScanSource* src, hipStream_t s, void* buf, uint32_t cap);
uint32_t SampleWant(const Ctx* c, const ScanSource& src, size_t nq, size_t kk);
void FreeSample(ScanSource* src);

// Host-pointer staging shared by the _host entry points.  The host writes the queries (and
// the filter words) into the context's pinned, mapped, coherent block; one kernel copies them
// to the device block; `fn` runs on device pointers; one kernel writes the results back into
// the pinned block and then raises host_flag, which the host polls (no allocation, no
// pageable copy and no stream synchronisation per call).  Regions start on 256-byte bounds.
constexpr size_t kStageAlign = 256;
inline size_t StageRound(size_t b) { return (b + kStageAlign - 1) & ~(kStageAlign - 1); }
// The bytes an input region of b bytes takes: at least one zero word past its end.
inline size_t StageSpan(size_t b) { return StageRound(b + 8); }
// Copies the nin host regions src[i] (bytes[i] each, zero-padded to StageSpan) into the
// device block back to back from its base, after reserving `out` more bytes for results;
// *dev receives the device block's base.
int StageIn(Ctx* c, const void* const* src, const size_t* bytes, int nin, size_t out,
            hipStream_t s, uint8_t** dev);
// Copies the nout <= 3 device regions src[i] (inside the device block) to the host pointers
// dst[i] after the work queued on s, through the pinned block.
int StageOut(Ctx* c, const uint8_t* const* src, const size_t* bytes, void* const* dst, int nout,
             hipStream_t s);

// The general form: nq queries of qb bytes in all, an optional second input region (extra,
// eb bytes: filter words or candidate lists), nq x k results, and per-query counts when
// dist_comps is non-null; fn(dq, dextra, di, dd, ddc, s) runs on the device copies (dextra,
// ddc null when absent).
template <class Fn>
inline int StageRegions(Ctx* c, const float* queries, size_t qb, const void* extra, size_t eb,
                        size_t nq, size_t k, uint32_t* out_ids, float* out_dists,
                        uint64_t* dist_comps, Fn fn) {
  hipStream_t s = c->stream;
  const size_t ob = nq * k * 4;
  const size_t cb = dist_comps ? nq * sizeof(uint64_t) : 0;
  const void* src[2] = {queries, extra};
  const size_t bytes[2] = {qb, eb};
  uint8_t* base = nullptr;
  VDBG_RETURN_IF_ERROR(StageIn(c, src, bytes, extra ? 2 : 1,
                               2 * StageRound(ob) + StageRound(cb), s, &base));
  const size_t in_end = StageSpan(qb) + (extra ? StageSpan(eb) : 0);
  const float* dq = reinterpret_cast<const float*>(base);
  const void* dx = extra ? static_cast<const void*>(base + StageSpan(qb)) : nullptr;
  uint32_t* di = reinterpret_cast<uint32_t*>(base + in_end);
  float* dd = reinterpret_cast<float*>(base + in_end + StageRound(ob));
  uint64_t* ddc = dist_comps ? reinterpret_cast<uint64_t*>(base + in_end + 2 * StageRound(ob))
                             : nullptr;
  VDBG_RETURN_IF_ERROR(fn(dq, dx, di, dd, ddc, s));
  const uint8_t* osrc[3] = {reinterpret_cast<const uint8_t*>(di),
                            reinterpret_cast<const uint8_t*>(dd),
                            reinterpret_cast<const uint8_t*>(ddc)};
  const size_t obytes[3] = {ob, ob, cb};
  void* const odst[3] = {out_ids, out_dists, dist_comps};
  return StageOut(c, osrc, obytes, odst, dist_comps ? 3 : 2, s);
}

// Queries of pd floats over an n_rows source with optional dense allow words (ceil(n/64)
// words, one zero word past them on the device); fn(dq, dm, di, dd, ddc, s).
template <class Fn>
inline int StageHost(Ctx* c, size_t n_rows, size_t pd, const float* queries, size_t nq,
                     size_t k, const uint64_t* allow_words, uint32_t* out_ids,
                     float* out_dists, uint64_t* dist_comps, Fn fn) {
  const size_t wb = allow_words ? ((n_rows + 63) / 64) * sizeof(uint64_t) : 0;
  return StageRegions(c, queries, nq * pd * sizeof(float), allow_words, wb, nq, k, out_ids,
                      out_dists, dist_comps,
                      [&](const float* dq, const void* dx, uint32_t* di, float* dd,
                          uint64_t* ddc, hipStream_t s) {
                        return fn(dq, static_cast<const uint64_t*>(dx), di, dd, ddc, s);
                      });
}

// Copies n <= 64 32-bit counters from device memory to c->host_pinned[0..n) after the work
// queued on s: a one-wave kernel publishes them into coherent pinned memory with a sequence
// number that the host polls (far less latency than a stream synchronisation); the host
// falls back to synchronising when the stream ends without the number showing.
int ReadWords(Ctx* c, const uint32_t* dev, int n, hipStream_t s, uint32_t* out);
// The host side of ReadWords for a kernel that publishes the words itself: waits until the
// flag carries seq (NextFlagSeq), then copies the n words to host_pinned (or, should the
// stream end without the number showing, copies them from dev).
uint32_t NextFlagSeq(Ctx* c);
int WaitWords(Ctx* c, uint32_t seq, const uint32_t* dev, int n, hipStream_t s);

}  // namespace vdbg

struct vdbg_ctx {
  vdbg::Ctx c;
};
struct vdbg_dataset {
  vdbg::Dataset d;
};
struct vdbg_sq8 {
  vdbg::Sq8Index q;
};
struct vdbg_ivfpq {
  vdbg::IvfIndex x;
};
struct vdbg_pqflat {
  vdbg::PqFlatIndex p;
};
