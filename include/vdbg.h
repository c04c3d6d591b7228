/*
 * vdbg.h -- C ABI of the MI355X (gfx950) search backend for vdb's nearest-neighbour path.
 *
 * This is the drop-in boundary: plain pointers and sizes, no C++ or framework types.  vdb's
 * C++ Index implementations (or any FFI) bind these entry points; the header-only C++20
 * classes in include/vdbg.hpp (GpuFlatIndex, GpuSq8Index, GpuIvfPqIndex) are such a binding.
 *
 * Conventions
 *  - Every call returns an int equal to vdb::Status::Code (include/vdb/status.h:14-26):
 *    0 ok, 1 invalid argument, 2 not found, 3 already exists, 4 I/O error, 5 corruption,
 *    6 failed precondition, 7 resource exhausted, 8 unavailable, 9 not supported,
 *    10 internal.  vdbg_last_error() gives the calling thread's last message.
 *  - Metrics: 0 = L2 (squared), 1 = inner product (minus dot), 2 = cosine (minus dot over
 *    vectors normalised at insert and at query), as include/vdb/types.h:13-17.
 *  - Rows and queries are padded_dim floats, zero padded (padded_dim % 16 == 0,
 *    include/vdb/types.h:30-32).  Results are row-major [nq][k], ascending by (dist, id)
 *    with ties broken by id (include/vdb/types.h:23-25), padded with
 *    (UINT32_MAX, +inf) when fewer than k rows are allowed (python/bindings.cc:131-136).
 *  - Distances are the reference's AVX-512 kernels' values bit for bit
 *    (src/distance/avx512.cc:19-64).
 *  - Filters are dense bitmasks: bit r of word r/64 set = row r allowed.  They replace
 *    RowFilter::allowed (src/index/index.h:23-27): a DeleteFilter (src/engine/planner.cc:12-19)
 *    is the complement of the DeleteBits words (src/util/delete_bits.h:50-55); a BitmapFilter
 *    (:21-29) is the roaring result minus deletes, expanded to words.
 *  - "_host" entry points take host pointers and block until results are on the host.
 *    "_device" entry points take device pointers, run on the given HIP stream (NULL = the
 *    context's stream) and return once the work is queued; inputs must stay valid until the
 *    stream reaches that point.  The flat, SQ8 and IVF-PQ searches are not fully
 *    asynchronous: they read a few device-side words on the host (whether a batch of more
 *    than 128 queries fits the integer GEMM, how many queries need the exact re-scan), so
 *    such a call returns only after the stream has reached its last ranking kernel.  Flat
 *    batches of at most 128 queries over integer rows make no read before that point.
 *  - All entry points on one context are serialised by the context (host threads may share
 *    it).  Calls on different streams of one context are ordered on the device where they
 *    share scratch: a call's launches wait for the previous call's last launch that reads
 *    it.
 */
#ifndef VDBG_H_
#define VDBG_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct vdbg_ctx vdbg_ctx;
typedef struct vdbg_dataset vdbg_dataset;

enum {
  VDBG_OK = 0,
  VDBG_INVALID_ARGUMENT = 1,
  VDBG_NOT_FOUND = 2,
  VDBG_ALREADY_EXISTS = 3,
  VDBG_IO_ERROR = 4,
  VDBG_CORRUPTION = 5,
  VDBG_FAILED_PRECONDITION = 6,
  VDBG_RESOURCE_EXHAUSTED = 7,
  VDBG_UNAVAILABLE = 8,
  VDBG_NOT_SUPPORTED = 9,
  VDBG_INTERNAL = 10
};

enum { VDBG_METRIC_L2 = 0, VDBG_METRIC_IP = 1, VDBG_METRIC_COSINE = 2 };

/* Library version, (major << 16) | minor. */
int vdbg_version(void);

/* The calling thread's last error message ("" when none). */
const char* vdbg_last_error(void);

/* ---------------------------------------------------------------- context */

/* A device, its stream and reusable device workspace.  Replaces nothing in the reference
 * (vdb's CPU indexes need no device state); owned by the GPU Index adapters. */
int vdbg_ctx_create(int device, vdbg_ctx** out);
/* Fails (VDBG_INVALID_ARGUMENT, nothing released) while datasets of the context remain:
 * destroy indexes, then datasets, then the context. */
int vdbg_ctx_destroy(vdbg_ctx* ctx);
/* The context's HIP stream (a hipStream_t), for callers that order their own work with it. */
void* vdbg_ctx_stream(vdbg_ctx* ctx);
/* Waits for all work queued on the context's stream. */
int vdbg_ctx_synchronize(vdbg_ctx* ctx);
/* The distance kernel set whose arithmetic order exact distances follow: "scalar", "avx2"
 * or "avx512" (KernelSet, src/distance/distance.h:26-33).  A new context takes what
 * Kernels() takes in a vdb process on this host (src/distance/cpu_features.cc:27-58): the
 * VDB_KERNELS environment variable when it names a set this CPU offers, else the best set
 * of this CPU.  Setting an unknown or unavailable set is InvalidArgument. */
int vdbg_ctx_set_kernels(vdbg_ctx* ctx, const char* name);
const char* vdbg_ctx_kernels(vdbg_ctx* ctx);
/* Whether flat and SQ8 scans may rank rows on fp16 MFMA (default 1): integer-valued rows
 * exactly when a batch fits the exact bounds, SQ8 codes and float rows with the operands
 * split into two fp16 parts under a widened rounding bound.  Datasets created while it is
 * on keep an fp16 copy of their rows (2 bytes per value for integer rows, 4 for float rows;
 * SQ8 indexes 2 bytes per code).  Returned results are identical either way; 0 ranks on the
 * fp32 GEMM.  No counterpart in the reference. */
int vdbg_ctx_set_fp16_gemm(vdbg_ctx* ctx, int enable);
/* Whether scans may rank on int8 MFMA (default 1; it also needs fp16 ranking on):
 * integer-valued flat rows spanning at most 256 consecutive values shifted into int8 (exact);
 * SQ8 codes against the query operand rounded to integers in two int8 parts; float rows and
 * queries scaled by powers of two, rounded and split into two int8 parts each (under a
 * widened rounding bound).  Datasets created while it is on keep an int8 copy of their rows
 * (1 byte per value and 4 per row for integer rows, 2 bytes per value for float rows).
 * Returned results are identical either way.  No counterpart in the reference. */
int vdbg_ctx_set_int8_gemm(vdbg_ctx* ctx, int enable);
/* How float datasets created from now on hold their fp16 copy (default 1): on, as the high
 * fp16 halves fp16(x 2^e) alone (2 bytes per value, no int8 copy), ranked with one fp16 MFMA
 * per product under a bound widened by (2^-10 + 2^-21) |q||x|; off, as two-part h + l pairs
 * (4 bytes per value, plus the int8 copy while the int8 GEMM is on), ranked with three fp16
 * or four int8 MFMAs per product.  A dataset keeps the form it was created with.  Returned
 * results are identical either way.  No counterpart in the reference. */
int vdbg_ctx_set_fp16_single(vdbg_ctx* ctx, int enable);
/* The smallest rows x queries x padded_dim product of a float-row batch that ranks on the
 * int8 GEMM (default 2e10; smaller batches keep the fp16 split GEMM, whose extra operand pass
 * and flag readback the int8 GEMM would not repay).  Results are identical either way.  No
 * counterpart in the reference. */
int vdbg_ctx_set_int8_float_min_work(vdbg_ctx* ctx, double work);
/* How IVF-PQ L2 indexes with precomputed tables (ivf_pq.cc:152-167) are scanned (default 1):
 * on, each row is ranked by its term-2 sum, kept per row (4 bytes per row, made when the index
 * is loaded or built), plus the query's table, and the rows near the running threshold are
 * scored exactly as the reference scores them; off, each probed list's table
 * fl(term2 + qtab) is built per query and every code scored on it.  Results are identical
 * either way.  No counterpart in the reference. */
int vdbg_ctx_set_ivf_row_sums(vdbg_ctx* ctx, int enable);

/* Host threads for the CPU side of a search (the HNSW walk); n <= 0 restores the default:
 * the cores this process may run on, capped by OMP_NUM_THREADS when set. */
int vdbg_ctx_set_host_threads(vdbg_ctx* ctx, int n);
/* The SQ8 distance the HNSW walk computes on the host for a kernel set ("scalar", "avx2",
 * "avx512") and metric: vdb's sq8_l2_* / sq8_ip_* (src/distance/scalar.cc:25-41,
 * avx2.cc:48-74, avx512.cc:48-64) bit for bit; portable != 0 takes the lane-by-lane form used
 * on hosts without the instructions.  Pure host code (no device work), so it can be checked
 * on any machine.  Returns NaN for an unknown set. */
float vdbg_host_sq8_distance(const char* kernels, int metric, const float* q, const uint8_t* c,
                             const float* vmin, const float* scale, size_t d, int portable);

/* Testing: forces the fallbacks of the flat and SQ8 scans' certificates so that tests can
 * check them.  1 fails every first certificate, so every query takes the second chance
 * (exact re-scoring of all its buffered candidates); 2 also fails the second one, so every
 * query is re-scanned exactly.  Results are identical at every level; 0 (the default) is
 * the normal path.  No counterpart in the reference. */
int vdbg_ctx_set_test_fallbacks(vdbg_ctx* ctx, int level);
/* How the flat and SQ8 scans run their fallback passes (the second chance and the exact
 * re-scan of uncertified queries).  On (the default), when the re-scan's scratch for every
 * query of the batch is at most 64 MiB, both passes are queued for every query and run only
 * for those the pass before listed, with no host wait; the fallback count then stays on the
 * device until vdbg_last_fallbacks reads it (which waits for the device).  Off, the host reads
 * each count and sizes the passes to it.  Results are identical either way.  No counterpart
 * in the reference. */
int vdbg_ctx_set_gated_fallbacks(vdbg_ctx* ctx, int enable);
/* How vdbg_collection_search_* schedules its segments' flat scans.  combine != 0 (the
 * default): when every segment is a flat scan (in-memory parts, flat indexes, prefilter
 * plans) whose external ids are unique within it (checked by vdbg_dataset_set_external_ids),
 * with k x segments <= 240 and at most 262,144 allowed rows in all, the allowed rows of every
 * segment are gathered into one row set and scanned once for the top k x segments, then
 * merged (the same results as vdb's merge of per-segment lists).  Otherwise each segment is
 * scanned on its own, side by side on `lanes` streams (0..16; 0 or 1: in turn on the call's
 * stream; default 2) with their own scratch, each lane issued by its own host thread when
 * threaded != 0 (the default).  Results are identical under every schedule.  No counterpart
 * in the reference. */
int vdbg_ctx_set_collection_schedule(vdbg_ctx* ctx, int combine, int lanes, int threaded);

/* Per-kernel timing with HIP events on the stream each kernel runs on.  When enabled, every
 * launch is bracketed by events; vdbg_profile_get returns the summed milliseconds and launch
 * count of kernel `name` since the last reset (after synchronising). */
int vdbg_profile_enable(vdbg_ctx* ctx, int enable);
int vdbg_profile_reset(vdbg_ctx* ctx);
int vdbg_profile_get(vdbg_ctx* ctx, const char* name, double* total_ms, uint64_t* launches);

/* ---------------------------------------------------------------- datasets */

/* Makes a segment's rows resident in HBM: the device copy of the VectorView an Index reads
 * (src/util/aligned_buffer.h:56-63, filled from the segment mmap at
 * src/storage/segment_reader.cc:56-59).  rows is n x padded_dim floats on the host.  Row
 * norms and value statistics used by the GEMM formulation are computed once here. */
int vdbg_dataset_create(vdbg_ctx* ctx, const float* rows, size_t n, size_t dim,
                        size_t padded_dim, int metric, vdbg_dataset** out);
/* The same from rows already in device memory (copied; the caller keeps ownership).  Work
 * queued on any stream of the device is waited for before the copy, and the copy has
 * completed when the call returns. */
int vdbg_dataset_create_device(vdbg_ctx* ctx, const float* rows_dev, size_t n, size_t dim,
                               size_t padded_dim, int metric, vdbg_dataset** out);
/* Fails (VDBG_INVALID_ARGUMENT, nothing released) while SQ8 or IVF-PQ indexes over the
 * dataset remain. */
int vdbg_dataset_destroy(vdbg_dataset* ds);
/* Device pointer to the resident rows (n x padded_dim floats). */
const float* vdbg_dataset_rows(vdbg_dataset* ds);

/* ---------------------------------------------------------------- segment files */

/* Segment::Open's read of vectors.f32 (src/storage/segment_reader.cc:37-59): the 4 KiB header
 * (magic VDBSEG01, CRC32C of bytes 0..4091 at 4092, version 1, metric, rows, dim, padded
 * dim, data offset 4096, data length rows x padded_dim x 4; src/storage/segment.h:9-12,
 * segment_writer.cc:58-75) is checked as :41-52 checks it, the data CRC32C when verify_crc
 * (:53-55), and the rows become a resident dataset, as vdbg_dataset_create.  file/len: the
 * file's bytes (e.g. its mmap).  rows: the manifest's row count, or UINT64_MAX to take the
 * header's.  Errors: 5 (corruption) with the reference's messages. */
int vdbg_dataset_open_vectors(vdbg_ctx* ctx, const void* file, size_t len, size_t dim,
                              int metric, uint64_t rows, int verify_crc, vdbg_dataset** out);
/* crc32c::Extend (src/util/crc32c.h:9-13): CRC32C (Castagnoli) of n bytes continuing crc
 * (0 to start).  Host-only. */
uint32_t vdbg_crc32c_extend(uint32_t crc, const void* data, size_t n);
/* DecodeBlob (src/storage/file_format.cc:21-33): checks a blob file ([magic 8][u32 version 1]
 * [u32 CRC32C of the payload][u64 payload length][payload], file_format.h:3-4), e.g. ids.u64
 * (magic "VDBIDS01") or a delete set ("VDBDEL01"); the payload is file[*payload_offset ..
 * + *payload_len).  Errors: 5 with the reference's messages.  Host-only. */
int vdbg_blob_decode(const void* file, size_t len, const char* magic, size_t* payload_offset,
                     size_t* payload_len);
/* The delete-set read of Segment::Open (segment_reader.cc:102-117): a deletes-<n>.roar blob
 * file whose payload is a roaring bitmap in the portable serialization
 * (segment_writer.cc:29-39), expanded into deleted_words[ceil(rows/64)] (bit r of word r/64
 * set = row r deleted, the DeleteBits layout of src/util/delete_bits.h:50-55); *count
 * (nullable) receives the number of deleted rows.  A row >= rows is corruption ("delete set
 * out of range", :111).  The complement of the words is the DeleteFilter the searches take.
 * Host-only. */
int vdbg_deletes_decode(const void* file, size_t len, size_t rows, uint64_t* deleted_words,
                        uint64_t* count);

/* ---------------------------------------------------------------- flat exact search */

/* Exact top-k for nq queries: FlatIndex::search (src/index/flat_index.cc:73-77, which is
 * FlatSearch :11-39 without a pool) for every query, and FlatSearchBatch (:41-68), which
 * returns the same results.  allow_words (nullable) has ceil(n/64) words.  dist_comps
 * (nullable) receives IndexSearchStats::distance_computations for the batch (rows per
 * query, as :75-76 adds).  Host pointers. */
int vdbg_flat_search_host(vdbg_dataset* ds, const float* queries, size_t nq, size_t k,
                          const uint64_t* allow_words, uint32_t* out_ids, float* out_dists,
                          uint64_t* dist_comps);
/* Device-pointer variant of vdbg_flat_search_host, queued on `stream`. */
int vdbg_flat_search_device(vdbg_dataset* ds, const float* queries, size_t nq, size_t k,
                            const uint64_t* allow_words, uint32_t* out_ids, float* out_dists,
                            void* stream);

/* vdbg_flat_search_device without any device allocation, for callers that cannot allocate
 * (tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * It cannot be captured into a HIP graph: it reads the count of uncertified queries back on
 * the host (as vdbg_flat_search_device does) before it queues their exact re-scan.  Same arguments, results and stream semantics as
 * vdbg_flat_search_device, with these limits:
 *  - k <= 240 (InvalidArgument otherwise);
 *  - the scratch is one static device array of 32 MiB per GPU (24 MiB for the scan
 *    pipeline, 8 MiB for the exact re-scan of uncertified queries), held by every GPU the
 *    library runs on until the process ends.  Batches that would need more scan into fewer,
 *    longer row chunks; a batch that still does not fit fails with ResourceExhausted before
 *    anything is queued: at 1M x 128 rows and k = 10 about 500 queries fit per call;
 *  - under a filter the rows are tested in place rather than compacted (same results).
 * All calls on one GPU share its array, and its contents persist between calls (everything
 * that must start cleared is cleared by each call with a fill kernel).  Calls that overlap
 * on one GPU would race for it, so the library orders them: a call's launches wait, on the
 * device, for the previous call's last launch that reads the array. */
int vdbg_flat_search_device_noalloc(vdbg_dataset* ds, const float* queries, size_t nq,
                                    size_t k, const uint64_t* allow_words, uint32_t* out_ids,
                                    float* out_dists, void* stream);

/* ---------------------------------------------------------------- SQ8 */

typedef struct vdbg_sq8 vdbg_sq8;

/* Sq8Quantizer::train (src/index/quant/sq8.cc:9-26) over the dataset's rows: per real
 * dimension min and max, scale = (max - min) / 255; padding dimensions get 0.  vmin_out and
 * scale_out receive padded_dim floats (host). */
int vdbg_sq8_train(vdbg_dataset* ds, float* vmin_out, float* scale_out);
/* Encodes every row with Sq8Quantizer::encode (sq8.cc:28-37), byte-identical to the CPU
 * encoder, and keeps the codes resident: HnswSq8Index::build (src/index/hnsw/hnsw_index.cc:
 * 66-79) without the graph.  vmin/scale are padded_dim floats (host), e.g. from
 * vdbg_sq8_train or a deserialised quantizer (sq8.cc:43-63). */
int vdbg_sq8_create(vdbg_dataset* ds, const float* vmin, const float* scale, vdbg_sq8** out);
/* LoadIndex (src/index/index.cc:38-87) of a VDBHSQ81 file, the HNSW-SQ8 index of a segment
 * (hnsw_index.cc:108-129): CRC32C footer, then rows, the Sq8Quantizer and the codes are read
 * and made resident as they are (no re-encoding), and the graph that follows is read with
 * HnswGraph::Deserialize's checks (src/index/hnsw/hnsw_graph.h:368-413) into host memory,
 * together with a host copy of the codes, for vdbg_sq8_hnsw_search_*.  `ds` is the segment
 * the index belongs to (rows and padded_dim must match).  Errors: 5 (corruption) for a bad
 * file, with the reference's messages. */
int vdbg_sq8_load(vdbg_dataset* ds, const void* file, size_t len, vdbg_sq8** out);
/* The loaded graph: out[0] nodes, [1] M, [2] ef_construction, [3] top layer (-1 when empty),
 * [4] entry point.  FailedPrecondition for an index made by vdbg_sq8_create (no graph). */
int vdbg_sq8_graph_info(vdbg_sq8* sq, int64_t out[5]);
/* HnswSq8Index::search (src/index/hnsw/hnsw_index.cc:82-100) for a batch of queries, over a
 * graph loaded by vdbg_sq8_load.  The graph walk stays on the CPU, as in vdb: greedy descent
 * through the upper layers and the layer-0 beam of HnswGraph::search (hnsw_graph.h:301-324,
 * 467-548) on the SQ8 distance of the context's kernel set, with ef = max(ef, k, depth) and
 * depth = rerank < 0 ? max(ef, k) : rerank; queries run on the context's host threads
 * (vdbg_ctx_set_host_threads).  The float Rerank of each query's beam (index.cc:89-95) runs
 * on the GPU over the resident rows; depth 0 returns the beam's k best by SQ8 distance.
 * allow_words (nullable) is the RowFilter: rejected rows are walked through but never
 * returned.  dist_comps (nullable, nq) receives IndexSearchStats::distance_computations.
 * The _device form takes device queries, words and outputs and synchronises the stream
 * twice (queries to the host for the walk, candidates back). */
int vdbg_sq8_hnsw_search_host(vdbg_sq8* sq, const float* queries, size_t nq, size_t k,
                              size_t ef, int rerank, const uint64_t* allow_words,
                              uint32_t* out_ids, float* out_dists, uint64_t* dist_comps);
int vdbg_sq8_hnsw_search_device(vdbg_sq8* sq, const float* queries, size_t nq, size_t k,
                                size_t ef, int rerank, const uint64_t* allow_words,
                                uint32_t* out_ids, float* out_dists, uint64_t* dist_comps,
                                void* stream);
int vdbg_sq8_destroy(vdbg_sq8* sq);
/* Copies the n x padded_dim code bytes to the host. */
int vdbg_sq8_codes(vdbg_sq8* sq, uint8_t* codes_out);
/* Exhaustive SQ8 search: the max(depth, k) smallest asymmetric SQ8 distances
 * (MetricSq8Distance, src/distance/cpu_features.cc:75-78) by (dist, id), then, when
 * depth > 0, Rerank (src/index/index.cc:89-95) with the fp32 rows to k; depth 0 returns the
 * top k by SQ8 distance.  This is HnswSq8Index::search (hnsw_index.cc:82-100) with the
 * graph beam replaced by a full scan. */
int vdbg_sq8_search_host(vdbg_sq8* sq, const float* queries, size_t nq, size_t k, size_t depth,
                         const uint64_t* allow_words, uint32_t* out_ids, float* out_dists,
                         uint64_t* dist_comps);
int vdbg_sq8_search_device(vdbg_sq8* sq, const float* queries, size_t nq, size_t k,
                           size_t depth, const uint64_t* allow_words, uint32_t* out_ids,
                           float* out_dists, void* stream);

/* ---------------------------------------------------------------- IVF-PQ */

typedef struct vdbg_ivfpq vdbg_ivfpq;

/* LoadIndex for a VDBIVFP1 file (src/index/index.cc:38-87: magic and CRC32C footer) followed
 * by IvfPqIndex::load (src/index/quant/ivf_pq.cc:251-278): coarse centroids, PQ codebook and
 * inverted lists become resident, and the per-list tables of precompute_tables (:152-167) are
 * derived on the GPU (L2, at most 1 GiB).  `ds` is the segment the index belongs to (rows
 * must match).  Errors: 5 (corruption) for a bad file, as the reference returns. */
int vdbg_ivfpq_load(vdbg_dataset* ds, const void* file, size_t len, vdbg_ivfpq** out);
/* Index::save for the resident index (ivf_pq.cc:236-249 + index.cc:110-117): writes the
 * VDBIVFP1 file into buf (cap bytes); *len receives its size (buf may be NULL to ask). */
int vdbg_ivfpq_save(vdbg_ivfpq* ix, void* buf, size_t cap, size_t* len);
int vdbg_ivfpq_destroy(vdbg_ivfpq* ix);
/* IvfPqIndex::build (src/index/quant/ivf_pq.cc:102-149) on the GPU over the dataset's rows:
 * nlist clamped to [1, n/39], KMeans of the padded rows (kmeans_iters Lloyd steps; the
 * reference uses 25), AssignNearest, PQ training on residuals of a strided <= 65,536-row
 * sample (seed + j * 7919 per subspace, pq.cc:14-41), residual encoding, lists with ids
 * ascending, precomputed tables.  The seeded draws follow the reference's
 * std::mt19937_64 sequence, so the index equals the reference's (with kmeans_iters = 25). */
int vdbg_ivfpq_build(vdbg_dataset* ds, size_t nlist, size_t pq_m, uint64_t seed,
                     size_t max_train_points_per_centroid, size_t kmeans_iters, vdbg_ivfpq** out);
/* nlist, m and whether precomputed tables are in use (IvfPqIndex::nlist,
 * precomputed_tables, ivf_pq.h:55-57). */
int vdbg_ivfpq_info(vdbg_ivfpq* ix, size_t* nlist, size_t* m, int* precomputed_tables);
/* IvfPqIndex::list_size for every list (ivf_pq.h:56); sizes has nlist entries. */
int vdbg_ivfpq_list_sizes(vdbg_ivfpq* ix, uint64_t* sizes);
/* IvfPqIndex::search (ivf_pq.cc:169-222) for nq queries: nprobe (SearchParams::nprobe,
 * clamped to [1, nlist]) nearest lists by (dist, list id), ADC scores into
 * TopK(max(R, k)) with R = RerankDepth(rerank) (:16-19: rerank < 0 -> max(10k, 100)), then
 * FinishSearch (:28-36): R = 0 truncates, otherwise Rerank with the fp32 rows.  dist_comps
 * (nullable, nq entries) receives IndexSearchStats::distance_computations per query. */
int vdbg_ivfpq_search_host(vdbg_ivfpq* ix, const float* queries, size_t nq, size_t k,
                           size_t nprobe, int rerank, const uint64_t* allow_words,
                           uint32_t* out_ids, float* out_dists, uint64_t* dist_comps);
/* Device-pointer variant; dist_comps (nullable) is a device array of nq entries. */
int vdbg_ivfpq_search_device(vdbg_ivfpq* ix, const float* queries, size_t nq, size_t k,
                             size_t nprobe, int rerank, const uint64_t* allow_words,
                             uint32_t* out_ids, float* out_dists, uint64_t* dist_comps,
                             void* stream);

/* ---------------------------------------------------------------- k-means */

/* KMeans (src/index/quant/kmeans.cc:57-174, options kmeans.h:13-20) with the assignment
 * steps on the GPU: n rows of d floats at `stride` (host), k centroids written to
 * centroids_out (k x d, host).  inertia / empty_reseeds (nullable) as KMeansStats. */
int vdbg_kmeans(vdbg_ctx* ctx, const float* data, size_t n, size_t d, size_t stride, size_t k,
                size_t iters, uint64_t seed, size_t max_points_per_centroid, int kmeanspp,
                float* centroids_out, double* inertia, size_t* empty_reseeds);
/* AssignNearest (kmeans.cc:23-55): the first nearest centroid of every row (padded rows use
 * the AVX-512-order kernel, others L2SqAny), and its distance (dist nullable). */
int vdbg_assign_nearest(vdbg_ctx* ctx, const float* data, size_t n, size_t d, size_t stride,
                        const float* centroids, size_t k, uint32_t* assign, float* dist);

/* ---------------------------------------------------------------- rerank */

/* Rerank (src/index/index.cc:89-95) against the resident rows, for nq queries at once: the
 * exact fp32 distances (MetricDistance, AVX-512 order) of each query's `depth` candidate rows
 * (cand is [nq][depth], UINT32_MAX = no candidate), the k smallest by (dist, id).  This is the
 * float rerank of HnswSq8Index::search (src/index/hnsw/hnsw_index.cc:82-100) and of
 * IvfPqIndex's FinishSearch (src/index/quant/ivf_pq.cc:28-36) for candidates found by vdb's
 * CPU graph.  A row id beyond the dataset is InvalidArgument.  dist_comps (nullable, nq
 * entries) receives each query's candidate count, as Rerank adds it. */
int vdbg_rerank_host(vdbg_dataset* ds, const float* queries, size_t nq, const uint32_t* cand,
                     size_t depth, size_t k, uint32_t* out_ids, float* out_dists,
                     uint64_t* dist_comps);
/* Device-pointer variant (dist_comps a device array); waits for the row check. */
int vdbg_rerank_device(vdbg_dataset* ds, const float* queries, size_t nq, const uint32_t* cand,
                       size_t depth, size_t k, uint32_t* out_ids, float* out_dists,
                       uint64_t* dist_comps, void* stream);

/* ---------------------------------------------------------------- collection read path */

/* CollectionImpl::PrepareQuery (src/engine/collection_impl.cc:1023-1034) for nq raw queries
 * of dim floats: each becomes a zero-padded row of padded_dim floats in `out`; a NaN or
 * infinite value is InvalidArgument (1); under cosine (metric 2) NormalizeVector
 * (src/util/dataset.cc:33-41: fp64 sum of squares in index order, fp32 scale by
 * float(1 / sqrt(sum))) and a zero vector is InvalidArgument.  Device pointers. */
int vdbg_prepare_queries_device(vdbg_ctx* ctx, const float* raw, size_t nq, size_t dim,
                                size_t padded_dim, int metric, float* out, void* stream);
/* Host-pointer variant. */
int vdbg_prepare_queries_host(vdbg_ctx* ctx, const float* raw, size_t nq, size_t dim,
                              size_t padded_dim, int metric, float* out);

/* The merge of CollectionImpl::Search (collection_impl.cc:1076-1112) for nq queries over
 * nparts per-segment results: part_dists / part_rows are [nparts][nq][k], each part's list
 * sorted by (dist, row) and padded with UINT32_MAX rows, as the per-segment searches return
 * them.  Row r of part p has external id ext_ids[part_offsets[p] + r].  All hits are ordered
 * by (dist, part, row), the first hit of each external id is kept and k are written per
 * query to out_ext / out_dists (padded with UINT64_MAX / +inf).  Up to 1024 hits per query
 * merge in one wavefront; more are merged by segmented sorts. */
int vdbg_merge_parts_device(vdbg_ctx* ctx, size_t nq, size_t nparts, size_t k,
                            const float* part_dists, const uint32_t* part_rows,
                            const uint64_t* ext_ids, const uint64_t* part_offsets,
                            uint64_t* out_ext, float* out_dists, void* stream);
/* Host-pointer variant; ext_ids holds n_ext entries. */
int vdbg_merge_parts_host(vdbg_ctx* ctx, size_t nq, size_t nparts, size_t k,
                          const float* part_dists, const uint32_t* part_rows,
                          const uint64_t* ext_ids, size_t n_ext, const uint64_t* part_offsets,
                          uint64_t* out_ext, float* out_dists);

/* Diagnostics of the last flat/SQ8 search on this context (all segments of the last
 * collection search): queries whose GEMM-ranked candidates could not be certified and were
 * re-scanned exactly.  Waits for the device when the count is still there. */
int vdbg_last_fallbacks(vdbg_ctx* ctx, uint64_t* fallback_queries);
/* Input width of the last flat/SQ8 scan's ranking GEMM on this context: 32 (fp32 MFMA), 16
 * (fp16 MFMA: integer rows and queries of magnitude <= 2048 with every partial sum below
 * 2^24, exactly; SQ8 codes and float rows on split operands), 8 (int8 MFMA: such integer
 * rows spanning at most 256 values, with every query value inside the same int8 window), or
 * 0 (no GEMM: the exact scan ran).  Batches of at most 128 queries over such integer rows
 * choose between the int8 and the fp32 GEMM on the device (no host round trip); for them
 * this call waits for the device and reads the choice. */
int vdbg_last_gemm_bits(vdbg_ctx* ctx);

/* ---------------------------------------------------------------- mutable segments */

/* MutableSegment (src/engine/mutable_segment.cc:10-64): an empty dataset that takes rows by
 * vdbg_dataset_append, with room reserved for `capacity` rows (doubling when exceeded).  It
 * is searched like any dataset (vdbg_flat_search_*: the exact top k over the allowed rows, as
 * MutableSegment::Search) and joins a collection search as an in-memory part.  It keeps no
 * fp16 / int8 copies, and takes no index. */
int vdbg_dataset_create_appendable(vdbg_ctx* ctx, size_t dim, size_t padded_dim, int metric,
                                   size_t capacity, vdbg_dataset** out);
/* MutableSegment::Append (mutable_segment.cc:24-44) of n rows (n x padded_dim floats, host)
 * and their external ids (host, nullable: NULL gives each new row its row number as external
 * id), published together when the call returns (later searches see them; rows never move
 * for readers of earlier calls).  *first_row (nullable) receives the first new row's number.
 * The call waits for its own copies on the context's stream; only growth past the reserved
 * capacity (capacity doubles) waits for the whole device.  FailedPrecondition for a dataset
 * not made appendable or one with an index. */
int vdbg_dataset_append(vdbg_dataset* ds, const float* rows, size_t n, const uint64_t* ext_ids,
                        uint64_t* first_row);
/* The dataset's row count. */
int vdbg_dataset_size(vdbg_dataset* ds, uint64_t* rows);

/* ---------------------------------------------------------------- PQ-flat */

typedef struct vdbg_pqflat vdbg_pqflat;

/* PqFlatIndex::build (src/index/quant/ivf_pq.cc:45-57): ProductQuantizer::train over every row
 * (pq.cc:14-41: per subspace a strided sample of at most 256 x max_points_per_centroid rows,
 * k-means seeded with seed + 7919 j) and every row encoded, on the GPU.  pq_m must divide the
 * dimension (InvalidArgument otherwise, index.cc:27-29).  vdb builds with kmeans_iters 25. */
int vdbg_pqflat_build(vdbg_dataset* ds, size_t pq_m, uint64_t seed,
                      size_t max_points_per_centroid, size_t kmeans_iters, vdbg_pqflat** out);
/* LoadIndex of a VDBPQFL1 file (index.cc:38-87) and PqFlatIndex::load (ivf_pq.cc:89-98):
 * the codebook and the codes made resident as they are.  Errors: 5 (corruption) for a bad
 * file, with the reference's messages. */
int vdbg_pqflat_load(vdbg_dataset* ds, const void* file, size_t len, vdbg_pqflat** out);
/* PqFlatIndex::save (ivf_pq.cc:81-87): the VDBPQFL1 file; *len its size, written to buf
 * when cap allows (ResourceExhausted otherwise; buf NULL asks for the size). */
int vdbg_pqflat_save(vdbg_pqflat* ix, void* buf, size_t cap, size_t* len);
int vdbg_pqflat_destroy(vdbg_pqflat* ix);
/* *m, and the m x 256 x (dim / m) codebook floats when centroids_out is not NULL. */
int vdbg_pqflat_info(vdbg_pqflat* ix, size_t* m, float* centroids_out);
/* Copies the n x m code bytes to the host. */
int vdbg_pqflat_codes(vdbg_pqflat* ix, uint8_t* codes_out);
/* PqFlatIndex::search (ivf_pq.cc:59-79): every allowed row's code scored by ADC against the
 * query's table (compute_table, pq.cc:63-73; adc, pq.h:36-46), the max(depth, k) best by
 * (ADC, id), then FinishSearch (:28-36) with depth = rerank < 0 ? max(10 k, 100) : rerank:
 * the float Rerank to k, or with depth 0 the k best by ADC.  dist_comps (nullable, nq):
 * rows + the candidates reranked. */
int vdbg_pqflat_search_host(vdbg_pqflat* ix, const float* queries, size_t nq, size_t k,
                            int rerank, const uint64_t* allow_words, uint32_t* out_ids,
                            float* out_dists, uint64_t* dist_comps);
int vdbg_pqflat_search_device(vdbg_pqflat* ix, const float* queries, size_t nq, size_t k,
                              int rerank, const uint64_t* allow_words, uint32_t* out_ids,
                              float* out_dists, uint64_t* dist_comps, void* stream);

/* ---------------------------------------------------------------- collection search */

/* One disk segment of a collection snapshot as CollectionImpl::Search reads it
 * (src/engine/collection_impl.cc:1050-1064, src/storage/segment.h:56-79). */
typedef struct vdbg_segment {
  vdbg_dataset* rows;             /* the segment's rows, external ids set with
                                     vdbg_dataset_set_external_ids */
  vdbg_sq8* sq8;                  /* the segment's index: HNSW-SQ8 (vdbg_sq8_load: the
                                     graph walk with GPU rerank) or this library's SQ8 scan
                                     index (vdbg_sq8_create: every code scanned), */
  vdbg_ivfpq* ivfpq;              /* or IVF-PQ lists; both NULL = a flat index */
  const uint64_t* deleted_words;  /* host, nullable: DeleteBits words, ceil(rows/64) */
  const uint64_t* filter_words;   /* host, nullable: the request's filter evaluated on this
                                     segment (SegmentColumns::Evaluate, planner.cc:64) as
                                     words; NULL = the request has no filter */
  vdbg_pqflat* pqflat;            /* or a PQ-flat index (at most one of sq8, ivfpq, pqflat) */
  int memory_part;                /* 1: an in-memory part (the active or a frozen mutable
                                     segment, MutableSegment::Search through SearchMutable,
                                     planner.cc:131-151): every row not deleted and matching
                                     the filter is scored exactly, no planner, no index.
                                     In-memory parts come first in the array, as in vdb's
                                     snapshot order (active, frozen, then disk). */
  /* A disk segment searched on the host: vdb's own SearchDiskSegment (planner.cc:42-129)
   * over an index this library does not hold, such as HnswIndex over a VDBHNSW1 file
   * (vdb's default IndexType::Hnsw, options.h:22).  When host_rows is set, rows and the
   * index pointers are ignored (rows may be NULL) and the segment's hits join the merge in
   * its place of the array: */
  const float* host_dists;        /* host [nq][k]: each query's hits, ascending (dist, row) */
  const uint32_t* host_rows;      /* host [nq][k]: their rows; UINT32_MAX after the last hit */
  const uint64_t* host_ext;       /* host [nq][k]: their external ids (Segment::external_id) */
  const uint64_t* host_dist_comps;/* host [nq], nullable: SegmentExplain distance_computations */
} vdbg_segment;

/* FilterStrategy (include/vdb/options.h:57). */
enum {
  VDBG_STRATEGY_AUTO = 0,
  VDBG_STRATEGY_PREFILTER = 1,
  VDBG_STRATEGY_GRAPH = 2,
  VDBG_STRATEGY_POST_FILTER = 3
};

/* SearchParams (include/vdb/options.h:59-67). */
typedef struct vdbg_search_params {
  size_t ef;                   /* 64 */
  size_t nprobe;               /* 16 */
  int rerank;                  /* -1 = auto, 0 = none */
  int strategy;                /* VDBG_STRATEGY_*, AUTO */
  size_t prefilter_threshold;  /* 10000 */
  size_t post_filter_alpha;    /* 10 */
} vdbg_search_params;

/* The per-segment plans of SearchDiskSegment (planner.cc:53-128), its SegmentExplain
 * strategies "index", "empty", "prefilter_exact", "filtered_index",
 * "filtered_index+exact_fallback" (some query of the batch fell back) and "post_filter". */
enum {
  VDBG_PLAN_INDEX = 0,
  VDBG_PLAN_EMPTY = 1,
  VDBG_PLAN_PREFILTER_EXACT = 2,
  VDBG_PLAN_FILTERED_INDEX = 3,
  VDBG_PLAN_FILTERED_INDEX_EXACT_FALLBACK = 4,
  VDBG_PLAN_POST_FILTER = 5,
  VDBG_PLAN_SCAN = 6,        /* an in-memory part without a filter (SearchMutable "scan") */
  VDBG_PLAN_SCAN_FILTER = 7, /* an in-memory part under a filter ("scan_filter") */
  VDBG_PLAN_HOST = 8         /* a disk segment whose hits the caller searched on the host */
};

/* Makes the segment's external ids (ids.u64, n entries, host) resident for the collection
 * merge; replaces earlier ones. */
int vdbg_dataset_set_external_ids(vdbg_dataset* ds, const uint64_t* ids);

/* CollectionImpl::SearchBatch (collection_impl.cc:1121-1135) over the disk segments of a
 * snapshot, in the snapshot's order: PrepareQuery for each raw query (nq x dim, host;
 * :1023-1034; a non-finite value or a zero cosine query fails the batch with 1), each
 * segment searched with SearchDiskSegment's plan (planner.cc:42-129: no filter -> the index
 * under the delete filter; a filter -> matches = filter minus deletes, then empty,
 * prefilter_exact, filtered_index with nprobe / selectivity and the exact fallback for
 * queries short of min(k, matches), or post_filter), and the merge by (dist, part, row)
 * keeping the first hit of each external id (:1076-1112).  Outputs [nq][k]: external ids
 * (UINT64_MAX padded) and distances (+inf padded; the score is the distance for L2 and its
 * negation otherwise).  dist_comps (nullable, nq) receives each query's distance
 * computations; seg_plans (nullable, nseg) each segment's VDBG_PLAN_*.  k must be in
 * 1..10000 (:1038-1039).  A segment with host_rows set is taken as searched: its hits (which
 * must be in ascending (dist, row) order per query, InvalidArgument otherwise) merge in its
 * place with the others, and its plan reads VDBG_PLAN_HOST.  Host pointers; blocks until the
 * results are on the host. */
int vdbg_collection_search_host(vdbg_ctx* ctx, const vdbg_segment* segs, size_t nseg,
                                size_t dim, int metric, const float* queries, size_t nq,
                                size_t k, const vdbg_search_params* params, uint64_t* out_ids,
                                float* out_dists, uint64_t* dist_comps, int* seg_plans);
/* vdbg_collection_search_host with the raw queries (nq x dim) and the outputs in device
 * memory, queued on `stream` (NULL = the context's): the same plans, results and counts
 * without the query upload and the result download.  Segment words, host parts, dist_comps
 * and seg_plans stay host memory.  Returns once the results are written (the call reads a
 * few device words on the host on the way: the queries' status, and the counts some plans
 * need). */
int vdbg_collection_search_device(vdbg_ctx* ctx, const vdbg_segment* segs, size_t nseg,
                                  size_t dim, int metric, const float* queries, size_t nq,
                                  size_t k, const vdbg_search_params* params,
                                  uint64_t* out_ids, float* out_dists, uint64_t* dist_comps,
                                  int* seg_plans, void* stream);

/* ---------------------------------------------------------------- coalesced one-query calls */

/* vdb searches an index with one query per call: CollectionImpl::SearchBatch gives each query
 * to a pool worker (src/engine/collection_impl.cc:1120-1130) and CollectionImpl::Search runs
 * Index::search (src/index/index.h:36-55) on every segment for it (:1060-1073), so these
 * calls arrive concurrently from many host threads.  A coalescer gathers concurrent calls on
 * one index that share k, the index parameters and the allow-words pointer into one device
 * batch of that index's *_host entry point.  The first call of a batch leads it; the batch
 * takes calls while the coalescer's previous batch is on the device, then until every caller
 * of that batch has called again or max_wait_us has passed since it left the device (so those
 * callers can join again; 0 = no such wait), and closes sooner once it holds max_batch
 * queries.  A lone caller never waits.  Every query of a batch is searched independently:
 * each call returns exactly what the one-query *_host call returns (ids, distances, and its
 * IndexSearchStats::distance_computations in dist_comps).  Thread-safe; a call blocks until
 * its batch is done.  max_batch in 1..4096, max_wait_us at most 1,000,000.  The coalescer
 * holds the index pointer: destroy it before the index.  No counterpart in vdb (its indexes
 * are called directly); for the Index adapters of GPU-resident indexes. */
typedef struct vdbg_coalescer vdbg_coalescer;
int vdbg_coalescer_create_flat(vdbg_dataset* ds, size_t max_batch, uint32_t max_wait_us,
                               vdbg_coalescer** out);
/* SQ8 scan (vdbg_sq8_search_host; param = rerank depth). */
int vdbg_coalescer_create_sq8(vdbg_sq8* sq, size_t max_batch, uint32_t max_wait_us,
                              vdbg_coalescer** out);
/* HNSW-SQ8 walk + GPU rerank (vdbg_sq8_hnsw_search_host; param = ef, rerank as there). */
int vdbg_coalescer_create_sq8_hnsw(vdbg_sq8* sq, size_t max_batch, uint32_t max_wait_us,
                                   vdbg_coalescer** out);
/* IVF-PQ (vdbg_ivfpq_search_host; param = nprobe, rerank as there). */
int vdbg_coalescer_create_ivfpq(vdbg_ivfpq* ix, size_t max_batch, uint32_t max_wait_us,
                                vdbg_coalescer** out);
/* PQ-flat (vdbg_pqflat_search_host; rerank as there). */
int vdbg_coalescer_create_pqflat(vdbg_pqflat* ix, size_t max_batch, uint32_t max_wait_us,
                                 vdbg_coalescer** out);
/* One query (padded_dim floats, host) through the coalescer: k nearest ids and distances
 * (host, k each, UINT32_MAX / +inf padded as the *_host call pads), dist_comps (nullable) the
 * query's distance computations.  param and rerank as the index's create call names them
 * (ignored where the index has none); allow_words as the *_host call takes them, and calls
 * passing the same pointer share batches (the words must not change while calls use them). */
int vdbg_coalescer_search(vdbg_coalescer* co, const float* query, size_t k, size_t param,
                          int rerank, const uint64_t* allow_words, uint32_t* out_ids,
                          float* out_dists, uint64_t* dist_comps);
/* Batches run so far and the queries they held (their mean size is queries / batches). */
int vdbg_coalescer_stats(vdbg_coalescer* co, uint64_t* batches, uint64_t* queries);
/* FailedPrecondition while calls are inside vdbg_coalescer_search. */
int vdbg_coalescer_destroy(vdbg_coalescer* co);

#ifdef __cplusplus
}
#endif

#endif /* VDBG_H_ */
