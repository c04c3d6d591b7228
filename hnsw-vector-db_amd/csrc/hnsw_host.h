// hnsw_host.h -- vdb's HNSW graph on the host: parsing a saved graph and walking it.
//
// vdb keeps HNSW graph traversal on the CPU (src/index/hnsw/hnsw_graph.h); so does this
// library.  An HnswSq8Index segment's walk runs here, over a host copy of its SQ8 codes,
// with the SQ8 distance of the process's kernel set, and hands each query's beam to the
// GPU rerank.  Plain types only: this interface is shared by g++- and hipcc-built objects.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace vdbg {

struct HnswGraph;  // opaque: levels, layer-0 lists, upper-layer lists, entry point

// HnswGraph::Deserialize (hnsw_graph.h:368-413) of the graph that ends an HnswSq8Index file,
// with its checks and Corruption messages; `rows` is the segment's row count (the graph's
// expected capacity).  On success *out owns the graph and *used is the bytes read.  Returns
// 0, or VDBG_CORRUPTION with *err set to the reference's message.
int HnswParse(const uint8_t* p, size_t len, uint64_t rows, HnswGraph** out, size_t* used,
              const char** err);
void HnswFree(HnswGraph* g);
// size, M, ef_construction, max level (-1 for an empty graph), entry point
void HnswInfo(const HnswGraph* g, int64_t out[5]);

// SQ8 asymmetric distance of a kernel set (0 scalar, 1 avx2, 2 avx512) and metric (0 L2,
// 1 inner product, 2 cosine): vdb's sq8_l2_* / sq8_ip_* (src/distance/scalar.cc:25-41,
// avx2.cc:48-74, avx512.cc:48-64), bit for bit on any host.  The SIMD sets use the host's
// instructions when it has them, else (or with `portable`) a lane-by-lane form of the same
// arithmetic.
using Sq8HostFn = float (*)(const float* q, const uint8_t* c, const float* vmin,
                            const float* scale, size_t d);
Sq8HostFn HostSq8Kernel(int kset, int metric, bool portable = false);

struct HnswWalkArgs {
  const HnswGraph* g;
  const uint8_t* codes;  // rows x pd, host
  const float* vmin;
  const float* scale;
  size_t pd;
  Sq8HostFn dist;
  const float* Q;        // nq x pd, host
  size_t nq;
  size_t kk;             // results kept per query
  size_t ef;             // beam width (raised to kk)
  const uint64_t* allow; // nullable dense words: the RowFilter
  uint32_t* out_ids;     // nq x kk, ascending (dist, id), padded with UINT32_MAX
  float* out_d;          // nq x kk SQ8 distances, padded with +inf
  uint32_t* out_n;       // nq: results found
  uint64_t* dc;          // nq: distance computations of the walk
  int threads;           // host threads (<= 1: the calling thread only)
};

// HnswGraph::search (hnsw_graph.h:301-324) for every query: greedy descent through the
// upper layers, then the layer-0 beam (filtered: rejected nodes are walked through but never
// enter the results).  Queries are spread over `threads` host threads.
void HnswWalk(const HnswWalkArgs& a);

// Host threads for CPU-side work: the cores this process may run on, capped by
// OMP_NUM_THREADS when set.
int DefaultHostThreads();

}  // namespace vdbg
