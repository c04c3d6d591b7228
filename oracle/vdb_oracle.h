/*
 * vdb_oracle.h -- CPU restatement of vdb's nearest-neighbour hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle that the HIP backend is
 * compared against: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product (libvdbg.so and the vdbg package) never links,
 * loads or calls it, and has no CPU fallback that routes through it.
 *
 * Every function restates one routine of the reference (KoduruChandrasekhar/
 * HNSW-Vector-DB, cited as path:line relative to the reference root) in plain C.
 * Floating-point operations are written out in the reference's order, and the file
 * is compiled with -ffp-contract=off, so every explicit fmaf() is a fused
 * multiply-add and nothing else is.
 *
 * Kernel sets ("kset"): the reference picks one kernel set at start-up
 * (src/distance/cpu_features.cc:33-58).  0 = scalar (scalar.cc), 1 = avx2
 * (avx2.cc), 2 = avx512 (avx512.cc).  The SIMD sets are emulated lane by lane,
 * including GCC's horizontal-reduction trees, so results are bit-identical to the
 * reference's intrinsics on any host.
 *
 * Metrics follow include/vdb/types.h:13-17: 0 = L2 (squared), 1 = InnerProduct
 * (minus dot), 2 = Cosine (minus dot over normalised vectors).
 *
 * Parity pinning, per function (tests/test_oracle.py):
 *   distances      golden bit patterns from the compiled reference + closed forms
 *   topk           closed form (full sort by (dist, id)) + reference golden vectors
 *   flat search    compiled reference + brute force closed form
 *   sq8            compiled reference (byte-identical codes) + half-step invariant
 *   pq             compiled reference (byte-identical codes) + ADC == decoded dist
 *   assign         compiled reference + brute force
 *   ivf-pq search  compiled reference on an index it built and saved (VDBIVFP1)
 *   rerank         compiled reference + brute force
 *   normalize      compiled reference + closed form
 *   merge          closed form (sort by (dist, part, row), dedupe external id)
 *   crc32c         known answer 0xE3069283 for "123456789" (tests/distance_test.cc:94)
 *   pq-flat        compiled reference (PqFlatIndex::search on files it built and saved)
 *                  + closed form (rerank over every row equals exact flat search)
 *   hnsw-sq8       compiled reference (HnswSq8Index::search on files it built and saved)
 *                  + closed form (ef >= rows walks every node: equals exact flat search)
 */
#ifndef VDB_ORACLE_H_
#define VDB_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_KSET_SCALAR = 0, OR_KSET_AVX2 = 1, OR_KSET_AVX512 = 2 };
enum { OR_METRIC_L2 = 0, OR_METRIC_IP = 1, OR_METRIC_COSINE = 2 };

/* ---- distance kernels (src/distance/scalar.cc, avx2.cc, avx512.cc) ---- */
float or_l2(int kset, const float* a, const float* b, size_t d);
float or_dot(int kset, const float* a, const float* b, size_t d);
float or_metric_dist(int kset, int metric, const float* a, const float* b, size_t d);
float or_sq8_l2(int kset, const float* q, const uint8_t* c, const float* vmin,
                const float* scale, size_t d);
float or_sq8_ip(int kset, const float* q, const uint8_t* c, const float* vmin,
                const float* scale, size_t d);
float or_metric_sq8(int kset, int metric, const float* q, const uint8_t* c,
                    const float* vmin, const float* scale, size_t d);
float or_l2sq_any(const float* a, const float* b, size_t d);
float or_dot_any(const float* a, const float* b, size_t d);

/* ---- top-k (src/util/topk.h:13-62) ----
 * k smallest (dist, id) of n pairs, ascending; returns the count written (min(n, k)). */
size_t or_topk(const float* dist, const uint32_t* id, size_t n, size_t k, float* out_d,
               uint32_t* out_id);

/* ---- flat exact search (src/index/flat_index.cc:11-39, 41-68) ----
 * Rows are `rows` x `pd` floats.  allow_words (nullable) is a dense bitmask, bit r of
 * word r/64 set = row r allowed.  Outputs are [nq][k], padded with (+inf, UINT32_MAX).
 * nthreads <= 1 runs inline. */
void or_flat_search_batch(int kset, int metric, const float* base, size_t rows, size_t pd,
                          const float* queries, size_t nq, size_t k,
                          const uint64_t* allow_words, float* out_d, uint32_t* out_id,
                          int nthreads);

/* ---- rerank (src/index/index.cc:89-95) ---- */
size_t or_rerank(int kset, int metric, const float* base, size_t pd, const float* q,
                 const uint32_t* cand_ids, size_t ncand, size_t k, float* out_d,
                 uint32_t* out_id);

/* ---- SQ8 (src/index/quant/sq8.cc:9-41) ---- */
void or_sq8_train(const float* base, size_t rows, size_t dim, size_t pd, float* vmin,
                  float* scale);
void or_sq8_encode(const float* x, size_t dim, size_t pd, const float* vmin,
                   const float* scale, uint8_t* code);
void or_sq8_encode_rows(const float* base, size_t rows, size_t dim, size_t pd,
                        const float* vmin, const float* scale, uint8_t* codes);
void or_sq8_decode(const uint8_t* code, size_t pd, const float* vmin, const float* scale,
                   float* x);
/* Full SQ8 scan into TopK(max(depth, k)), then fp32 Rerank to k (depth 0: truncate).
 * Composed from sq8.cc, cpu_features.cc:69-72, topk.h and index.cc:89-95 the way
 * HnswSq8Index::search composes them (src/index/hnsw/hnsw_index.cc:82-100). */
void or_sq8_search_batch(int kset, int metric, const float* base, const uint8_t* codes,
                         size_t rows, size_t pd, const float* vmin, const float* scale,
                         const float* queries, size_t nq, size_t k, size_t depth,
                         const uint64_t* allow_words, float* out_d, uint32_t* out_id,
                         int nthreads);

/* ---- product quantizer (src/index/quant/pq.h:36-46, pq.cc:43-73) ----
 * centroids: m x 256 x dsub floats. */
void or_pq_encode(const float* centroids, size_t m, size_t dsub, const float* x,
                  uint8_t* code);
void or_pq_compute_table(const float* centroids, size_t m, size_t dsub, const float* q,
                         int metric, float* table);
float or_pq_adc(const float* table, size_t m, const uint8_t* code);

/* ---- k-means assignment (src/index/quant/kmeans.cc:16-55) ---- */
void or_assign_nearest(int kset, const float* data, size_t n, size_t d, size_t stride,
                       const float* centroids, size_t k, uint32_t* assign, float* dist,
                       int nthreads);

/* ---- IVF-PQ (src/index/quant/ivf_pq.cc:152-222) ----
 * Lists in CSR form: list l holds rows list_ids[off[l] .. off[l+1]) and codes
 * list_codes[off[l]*m ..].  term2 (nullable) is nlist x m x 256. */
void or_ivfpq_term2(const float* coarse, size_t nlist, size_t pd, const float* pq_centroids,
                    size_t m, size_t dsub, float* term2);
void or_ivfpq_search_batch(int kset, int metric, const float* base, size_t dim, size_t pd,
                           const float* coarse, size_t nlist, const float* pq_centroids,
                           size_t m, const uint64_t* list_off, const uint32_t* list_ids,
                           const uint8_t* list_codes, const float* term2,
                           const float* queries, size_t nq, size_t k, size_t nprobe,
                           int rerank, const uint64_t* allow_words, float* out_d,
                           uint32_t* out_id, uint64_t* dist_comps, int nthreads);

/* ---- query preparation (src/util/dataset.cc:33-41) ---- */
int or_normalize(float* v, size_t dim);

/* ---- cross-segment merge (src/engine/collection_impl.cc:1076-1112) ----
 * nparts lists of up to k hits each ([part][k], padded with UINT32_MAX ids), external
 * ids per part via ext[part_off[p] + row].  Writes up to k external ids and dists. */
size_t or_merge_parts(size_t nparts, size_t k, const float* part_d, const uint32_t* part_row,
                      const uint64_t* ext, const uint64_t* part_off, float* out_d,
                      uint64_t* out_ext);

/* ---- the per-segment plan of SearchDiskSegment (src/engine/planner.cc:53-108) ----
 * Returns 0 index, 1 empty, 2 prefilter_exact, 3 filtered_index, 5 post_filter;
 * *nprobe_out is the probe count of the index search. */
int or_plan_segment(int has_filter, size_t rows, size_t deleted, size_t matches, int index_flat,
                    int strategy, size_t ef, size_t k, size_t nprobe,
                    size_t prefilter_threshold, size_t* nprobe_out);

/* ---- PQ-flat search (src/index/quant/ivf_pq.cc:59-79) ----
 * PqFlatIndex::search per query: ADC of every allowed row's code (rows x m bytes) against
 * compute_table(q), TopK(max(depth, k)) with depth = rerank < 0 ? max(10 k, 100) : rerank,
 * then Rerank (or the k best by ADC at depth 0).  dist_comps (nullable): rows + reranked. */
void or_pqflat_search_batch(int kset, int metric, const float* base, size_t rows, size_t pd,
                            const float* pq_centroids, size_t m, size_t dsub,
                            const uint8_t* codes, const float* queries, size_t nq, size_t k,
                            int rerank, const uint64_t* allow_words, float* out_d,
                            uint32_t* out_id, uint64_t* dist_comps, int nthreads);

/* ---- HNSW-SQ8 search (src/index/hnsw/hnsw_index.cc:82-100) ----
 * HnswSq8Index::search per query over a VDBHSQ81 file (quantizer, codes and graph read from
 * it): HnswGraph::search's greedy descent and layer-0 beam (hnsw_graph.h:301-324, 467-548)
 * on SQ8 distances, then Rerank on the float rows.  ef and rerank are SearchParams' (rerank
 * -1 = auto).  dist_comps (nullable) receives IndexSearchStats::distance_computations.
 * Returns 0, or -1 when the file does not parse. */
int or_hnsw_sq8_search_file(int kset, int metric, const uint8_t* file, size_t len,
                            const float* base, size_t rows, size_t pd, const float* queries,
                            size_t nq, size_t k, size_t ef, int rerank,
                            const uint64_t* allow_words, float* out_d, uint32_t* out_id,
                            uint64_t* dist_comps, int nthreads);

/* ---- CRC32C (src/util/crc32c.cc) ---- */
uint32_t or_crc32c(uint32_t crc, const void* data, size_t n);

#ifdef __cplusplus
}
#endif

#endif /* VDB_ORACLE_H_ */
