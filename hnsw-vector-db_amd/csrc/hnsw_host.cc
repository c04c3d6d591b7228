// hnsw_host.cc -- vdb's HNSW graph on the host (see hnsw_host.h).
//
// Host-only code, built with -ffp-contract=off: the only fused multiply-adds are the explicit
// FMA intrinsics and std::fma calls that stand for the reference's _mm256/_mm512_fmadd_ps.
#include "hnsw_host.h"

#include <immintrin.h>
#include <sched.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "../../include/vdbg.h"

namespace vdbg {

// ---------------------------------------------------------------- the graph

// A walk's visited set: one epoch tag per node; a query bumps the epoch instead of clearing
// the array (cleared once when the epoch wraps).
struct Visited {
  std::vector<uint32_t> mark;
  uint32_t epoch = 0;
};

struct HnswGraph {
  uint64_t cap = 0, size = 0;
  uint32_t M = 0, M0 = 0, efc = 0;
  uint64_t seed = 0;
  int max_level = -1;
  uint32_t entry = 0;
  std::vector<uint8_t> level;    // per node
  std::vector<uint32_t> links0;  // cap x (1 + M0): [count][links...]
  std::vector<uint64_t> up_at;   // per node: where its layer-1 list starts in up
  std::vector<uint32_t> up;      // level x (1 + M) words per node above layer 0

  const uint32_t* links(uint32_t id, int layer) const {
    if (layer == 0) return links0.data() + size_t(id) * (1 + M0);
    return up.data() + up_at[id] + size_t(layer - 1) * (1 + M);
  }

  // Visited sets kept between walks (a fresh one costs a cap-sized allocation and clear,
  // more than a whole one-query walk), as vdb's VisitedPool keeps its SearchContexts.
  mutable std::mutex pool_mu;
  mutable std::vector<std::unique_ptr<Visited>> pool;
  std::unique_ptr<Visited> take() const {
    {
      std::lock_guard<std::mutex> g(pool_mu);
      if (!pool.empty()) {
        std::unique_ptr<Visited> v = std::move(pool.back());
        pool.pop_back();
        return v;
      }
    }
    auto v = std::make_unique<Visited>();
    v->mark.assign(cap, 0);
    return v;
  }
  void give(std::unique_ptr<Visited> v) const {
    std::lock_guard<std::mutex> g(pool_mu);
    pool.push_back(std::move(v));
  }
};

namespace {

constexpr int kMaxLevel = 15;  // hnsw_graph.h:46

struct Reader {
  const uint8_t* p;
  size_t left;
  template <class T>
  bool get(T* v) {
    if (left < sizeof(T)) return false;
    std::memcpy(v, p, sizeof(T));
    p += sizeof(T);
    left -= sizeof(T);
    return true;
  }
  bool bytes(void* dst, size_t n) {
    if (left < n) return false;
    if (n > 0) std::memcpy(dst, p, n);
    p += n;
    left -= n;
    return true;
  }
};

}  // namespace

int HnswParse(const uint8_t* p, size_t len, uint64_t rows, HnswGraph** out, size_t* used,
              const char** err) {
  auto bad = [&](const char* m) {
    *err = m;
    return int(VDBG_CORRUPTION);
  };
  Reader r{p, len};
  uint64_t cap = 0, sz = 0, seed = 0;
  uint32_t m = 0, efc = 0, maxl = 0, ep = 0;
  if (!r.get(&cap) || !r.get(&sz) || !r.get(&m) || !r.get(&efc) || !r.get(&seed) ||
      !r.get(&maxl) || !r.get(&ep))
    return bad("truncated hnsw header");
  if (cap != rows || sz > cap || m < 2 || m > 4096)
    return bad("hnsw header does not match the segment");
  const int max_level = static_cast<int>(maxl);
  if (max_level > kMaxLevel || (cap > 0 && ep >= cap)) return bad("bad hnsw entry point");
  auto g = new (std::nothrow) HnswGraph;
  if (g == nullptr) return bad("out of host memory for the hnsw graph");
  auto fail = [&](const char* msg) {
    delete g;
    return bad(msg);
  };
  g->cap = cap;
  g->size = sz;
  g->M = m;
  g->M0 = 2 * m;
  g->efc = std::max(efc, m);
  g->seed = seed;
  g->max_level = max_level;
  g->entry = ep;
  try {
    g->level.resize(cap);
    g->links0.resize(cap * (1 + size_t(g->M0)));
    g->up_at.resize(cap);
  } catch (...) {
    return fail("out of host memory for the hnsw graph");
  }
  if (!r.bytes(g->level.data(), cap)) return fail("truncated hnsw levels");
  if (!r.bytes(g->links0.data(), g->links0.size() * 4)) return fail("truncated hnsw layer 0");
  uint64_t total = 0;  // node by node, in the reference's order of checks
  for (uint64_t i = 0; i < cap; ++i) {
    const int lvl = g->level[i];
    if (sz > 0 && lvl > max_level) return fail("node above the top layer");
    g->up_at[i] = total;
    total += uint64_t(lvl) * (1 + m);
    if (total * 4 > r.left) return fail("truncated hnsw upper layers");
  }
  g->up.resize(total);
  r.bytes(g->up.data(), total * 4);
  // every link, so a bad file can never send a walk out of bounds
  for (uint64_t i = 0; i < cap; ++i) {
    for (int l = 0; l <= g->level[i]; ++l) {
      const uint32_t* ll = g->links(uint32_t(i), l);
      if (ll[0] > (l == 0 ? g->M0 : g->M)) return fail("bad link count");
      for (uint32_t j = 0; j < ll[0]; ++j)
        if (ll[1 + j] >= cap) return fail("bad link target");
    }
  }
  *out = g;
  *used = len - r.left;
  return 0;
}

void HnswFree(HnswGraph* g) { delete g; }

void HnswInfo(const HnswGraph* g, int64_t out[5]) {
  out[0] = int64_t(g->size);
  out[1] = g->M;
  out[2] = g->efc;
  out[3] = g->max_level;
  out[4] = g->entry;
}

// ---------------------------------------------------------------- SQ8 distances

namespace {

// scalar.cc:25-41: decode with a multiply and an add, then a sequential sum.
float Sq8L2Scalar(const float* q, const uint8_t* c, const float* vmin, const float* scale,
                  size_t d) {
  float s = 0.f;
  for (size_t i = 0; i < d; ++i) {
    const float x = vmin[i] + static_cast<float>(c[i]) * scale[i];
    const float t = q[i] - x;
    s += t * t;
  }
  return s;
}
float Sq8IpScalar(const float* q, const uint8_t* c, const float* vmin, const float* scale,
                  size_t d) {
  float s = 0.f;
  for (size_t i = 0; i < d; ++i) s += q[i] * (vmin[i] + static_cast<float>(c[i]) * scale[i]);
  return -s;
}

// The AVX2 set's order (avx2.cc:48-74): two 8-lane accumulators over each 16 values, decode
// fma(code, scale, vmin), then (lo128 + hi128) of their sum reduced by two horizontal adds.
// The AVX-512 set's (avx512.cc:48-64): one 16-lane accumulator, then GCC's
// _mm512_reduce_add_ps tree (halves of 8, of 4, then pairs at distance 2 and 1).  Portable
// lane-by-lane forms for hosts without the instructions:
template <bool L2>
float Sq8Avx2Portable(const float* q, const uint8_t* c, const float* vmin, const float* scale,
                      size_t d) {
  float acc[16] = {};
  for (size_t i = 0; i < d; i += 16)
    for (int l = 0; l < 16; ++l) {
      const float x = std::fma(static_cast<float>(c[i + l]), scale[i + l], vmin[i + l]);
      if (L2) {
        const float t = q[i + l] - x;
        acc[l] = std::fma(t, t, acc[l]);
      } else {
        acc[l] = std::fma(q[i + l], x, acc[l]);
      }
    }
  float v[8], s[4];
  for (int l = 0; l < 8; ++l) v[l] = acc[l] + acc[l + 8];
  for (int l = 0; l < 4; ++l) s[l] = v[l] + v[l + 4];
  const float r = (s[0] + s[1]) + (s[2] + s[3]);
  return L2 ? r : -r;
}
template <bool L2>
float Sq8Avx512Portable(const float* q, const uint8_t* c, const float* vmin,
                        const float* scale, size_t d) {
  float acc[16] = {};
  for (size_t i = 0; i < d; i += 16)
    for (int l = 0; l < 16; ++l) {
      const float x = std::fma(static_cast<float>(c[i + l]), scale[i + l], vmin[i + l]);
      if (L2) {
        const float t = q[i + l] - x;
        acc[l] = std::fma(t, t, acc[l]);
      } else {
        acc[l] = std::fma(q[i + l], x, acc[l]);
      }
    }
  float h[8], f[4];
  for (int l = 0; l < 8; ++l) h[l] = acc[8 + l] + acc[l];
  for (int l = 0; l < 4; ++l) f[l] = h[4 + l] + h[l];
  const float r = (f[0] + f[2]) + (f[1] + f[3]);
  return L2 ? r : -r;
}

// The same with the instructions themselves.
__attribute__((target("avx2,fma"))) inline float HSum8(__m256 v) {
  __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  s = _mm_hadd_ps(s, s);
  s = _mm_hadd_ps(s, s);
  return _mm_cvtss_f32(s);
}
template <bool L2>
__attribute__((target("avx2,fma"))) float Sq8Avx2(const float* q, const uint8_t* c,
                                                   const float* vmin, const float* scale,
                                                   size_t d) {
  __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
  for (size_t i = 0; i < d; i += 16) {
    const __m128i b = _mm_loadu_si128(reinterpret_cast<const __m128i*>(c + i));
    const __m256 x0 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(b)),
                                      _mm256_loadu_ps(scale + i), _mm256_loadu_ps(vmin + i));
    const __m256 x1 =
        _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(b, 8))),
                        _mm256_loadu_ps(scale + i + 8), _mm256_loadu_ps(vmin + i + 8));
    const __m256 q0 = _mm256_loadu_ps(q + i), q1 = _mm256_loadu_ps(q + i + 8);
    if (L2) {
      const __m256 t0 = _mm256_sub_ps(q0, x0), t1 = _mm256_sub_ps(q1, x1);
      a0 = _mm256_fmadd_ps(t0, t0, a0);
      a1 = _mm256_fmadd_ps(t1, t1, a1);
    } else {
      a0 = _mm256_fmadd_ps(q0, x0, a0);
      a1 = _mm256_fmadd_ps(q1, x1, a1);
    }
  }
  const float r = HSum8(_mm256_add_ps(a0, a1));
  return L2 ? r : -r;
}
template <bool L2>
__attribute__((target("avx512f,avx2,fma"))) float Sq8Avx512(const float* q, const uint8_t* c,
                                                            const float* vmin,
                                                            const float* scale, size_t d) {
  __m512 acc = _mm512_setzero_ps();
  for (size_t i = 0; i < d; i += 16) {
    const __m128i b = _mm_loadu_si128(reinterpret_cast<const __m128i*>(c + i));
    const __m512 x = _mm512_fmadd_ps(_mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(b)),
                                     _mm512_loadu_ps(scale + i), _mm512_loadu_ps(vmin + i));
    const __m512 qv = _mm512_loadu_ps(q + i);
    if (L2) {
      const __m512 t = _mm512_sub_ps(qv, x);
      acc = _mm512_fmadd_ps(t, t, acc);
    } else {
      acc = _mm512_fmadd_ps(qv, x, acc);
    }
  }
  const float r = _mm512_reduce_add_ps(acc);
  return L2 ? r : -r;
}

bool HostHasAvx2() {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}
bool HostHasAvx512() { return HostHasAvx2() && __builtin_cpu_supports("avx512f"); }

}  // namespace

Sq8HostFn HostSq8Kernel(int kset, int metric, bool portable) {
  const bool l2 = metric == 0;
  if (kset == 2) {
    if (!portable && HostHasAvx512()) return l2 ? Sq8Avx512<true> : Sq8Avx512<false>;
    return l2 ? Sq8Avx512Portable<true> : Sq8Avx512Portable<false>;
  }
  if (kset == 1) {
    if (!portable && HostHasAvx2()) return l2 ? Sq8Avx2<true> : Sq8Avx2<false>;
    return l2 ? Sq8Avx2Portable<true> : Sq8Avx2Portable<false>;
  }
  return l2 ? Sq8L2Scalar : Sq8IpScalar;
}

// ---------------------------------------------------------------- the walk

namespace {

struct Nb {
  float d;
  uint32_t id;
};
// Neighbor's order (include/vdb/types.h:23-26): distance, then id.
inline bool NbLess(const Nb& a, const Nb& b) { return a.d < b.d || (a.d == b.d && a.id < b.id); }
inline bool NbGreater(const Nb& a, const Nb& b) { return NbLess(b, a); }

// Per-thread state of the walk: an epoch-tagged visited set and the two heaps.
struct Walker {
  const HnswWalkArgs& a;
  std::unique_ptr<Visited> vis;  // from the graph's pool, returned when the walker ends
  std::vector<uint32_t>& mark;
  uint32_t& epoch;
  std::vector<Nb> res, cand;

  explicit Walker(const HnswWalkArgs& args)
      : a(args), vis(args.g->take()), mark(vis->mark), epoch(vis->epoch) {}
  ~Walker() { a.g->give(std::move(vis)); }

  float dist(const float* q, uint32_t id) const {
    return a.dist(q, a.codes + size_t(id) * a.pd, a.vmin, a.scale, a.pd);
  }
  bool allowed(uint32_t id) const {
    return a.allow == nullptr || ((a.allow[id >> 6] >> (id & 63)) & 1u);
  }
  void next_epoch() {
    if (++epoch == 0) {
      std::fill(mark.begin(), mark.end(), 0);
      epoch = 1;
    }
  }

  // One query: hnsw_graph.h:301-324 (descent :467-496, beam :501-548).
  void run(size_t qi) {
    const HnswGraph& g = *a.g;
    const float* q = a.Q + qi * a.pd;
    uint32_t* oi = a.out_ids + qi * a.kk;
    float* od = a.out_d + qi * a.kk;
    size_t found = 0;
    uint64_t dc = 0;
    if (g.max_level >= 0 && a.kk > 0) {
      dc = 1;
      uint32_t cur = g.entry;
      float curd = dist(q, cur);
      for (int l = g.max_level; l > 0; --l) {
        for (bool changed = true; changed;) {
          changed = false;
          const uint32_t* ll = g.links(cur, l);
          const uint32_t cnt = ll[0];
          for (uint32_t j = 0; j < cnt; ++j) {  // the whole list of the node entered with
            const float d = dist(q, ll[1 + j]);
            ++dc;
            if (d < curd) {
              curd = d;
              cur = ll[1 + j];
              changed = true;
            }
          }
        }
      }
      const size_t ef = std::max(a.ef, a.kk);
      const bool filtered = a.allow != nullptr;
      next_epoch();
      res.clear();
      cand.clear();
      mark[cur] = epoch;
      float lower = std::numeric_limits<float>::infinity();
      if (!filtered || allowed(cur)) {
        res.push_back({curd, cur});
        lower = curd;
      }
      cand.push_back({curd, cur});
      while (!cand.empty()) {
        const Nb c = cand.front();
        if (c.d > lower && (!filtered || res.size() >= ef)) break;
        std::pop_heap(cand.begin(), cand.end(), NbGreater);
        cand.pop_back();
        const uint32_t* ll = g.links(c.id, 0);
        const uint32_t cnt = ll[0];
        for (uint32_t j = 0; j < cnt; ++j) {
          const uint32_t e = ll[1 + j];
          if (mark[e] == epoch) continue;
          mark[e] = epoch;
          const float de = dist(q, e);
          ++dc;
          if (res.size() < ef || de < lower) {
            cand.push_back({de, e});
            std::push_heap(cand.begin(), cand.end(), NbGreater);
            if (!filtered || allowed(e)) {
              res.push_back({de, e});
              std::push_heap(res.begin(), res.end(), NbLess);
              if (res.size() > ef) {
                std::pop_heap(res.begin(), res.end(), NbLess);
                res.pop_back();
              }
              lower = res.front().d;
            }
          }
        }
      }
      while (res.size() > a.kk) {
        std::pop_heap(res.begin(), res.end(), NbLess);
        res.pop_back();
      }
      std::sort(res.begin(), res.end(), NbLess);
      found = res.size();
      for (size_t i = 0; i < found; ++i) {
        oi[i] = res[i].id;
        od[i] = res[i].d;
      }
    }
    for (size_t i = found; i < a.kk; ++i) {
      oi[i] = UINT32_MAX;
      od[i] = std::numeric_limits<float>::infinity();
    }
    a.out_n[qi] = uint32_t(found);
    a.dc[qi] = dc;
  }
};

}  // namespace

void HnswWalk(const HnswWalkArgs& a) {
  const size_t nthreads = std::min<size_t>(a.threads > 1 ? size_t(a.threads) : 1, a.nq);
  if (nthreads <= 1) {
    Walker w(a);
    for (size_t i = 0; i < a.nq; ++i) w.run(i);
    return;
  }
  std::atomic<size_t> next{0};
  constexpr size_t kChunk = 4;
  auto work = [&]() {
    Walker w(a);
    for (;;) {
      const size_t b = next.fetch_add(kChunk);
      if (b >= a.nq) break;
      const size_t e = std::min(a.nq, b + kChunk);
      for (size_t i = b; i < e; ++i) w.run(i);
    }
  };
  std::vector<std::thread> pool;
  pool.reserve(nthreads - 1);
  for (size_t t = 1; t < nthreads; ++t) pool.emplace_back(work);
  work();
  for (auto& t : pool) t.join();
}

int DefaultHostThreads() {
  int n = 1;
  cpu_set_t set;
  if (sched_getaffinity(0, sizeof(set), &set) == 0) n = CPU_COUNT(&set);
  if (n < 1) n = int(std::max(1u, std::thread::hardware_concurrency()));
  if (const char* env = std::getenv("OMP_NUM_THREADS")) {
    const int cap = std::atoi(env);
    if (cap > 0) n = std::min(n, cap);
  }
  return std::max(1, n);
}

}  // namespace vdbg

extern "C" float vdbg_host_sq8_distance(const char* kernels, int metric, const float* q,
                                        const uint8_t* c, const float* vmin, const float* scale,
                                        size_t d, int portable) {
  if (kernels == nullptr || q == nullptr || c == nullptr || vmin == nullptr || scale == nullptr)
    return std::numeric_limits<float>::quiet_NaN();
  int kset = -1;
  if (std::strcmp(kernels, "scalar") == 0) kset = 0;
  if (std::strcmp(kernels, "avx2") == 0) kset = 1;
  if (std::strcmp(kernels, "avx512") == 0) kset = 2;
  if (kset < 0 || d % 16 != 0) return std::numeric_limits<float>::quiet_NaN();
  return vdbg::HostSq8Kernel(kset, metric, portable != 0)(q, c, vmin, scale, d);
}
