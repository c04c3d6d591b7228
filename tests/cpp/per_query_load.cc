// per_query_load.cc -- concurrent one-query flat searches, as vdb's pool workers issue
// Index::search (src/engine/collection_impl.cc:1120-1130): T host threads each call with one
// query at a time, through a coalescer (vdbg_coalescer_search) or the one-query host call
// directly (--direct).
//
//   per_query_load [--rows N] [--dim D] [--queries Q] [--threads T] [--k K]
//                  [--max-batch B] [--wait-us W] [--seconds S] [--direct]
//                  [--data FILE] [--out FILE]
//
// Rows and queries come from FILE (raw float32: N x D rows, then Q x D queries) or are
// generated (integer values 0..255 around 1,000 centres, SplitMix64).  A first pass sends
// every query once and keeps its result; a timed pass then keeps the threads busy for S
// seconds.  The first pass's results are compared with one batched vdbg_flat_search_host
// call over all Q queries (ids and distance bits) and, with --out, written to FILE
// (Q x K uint32 ids, then Q x K float distances).  Prints one JSON line.
#include <atomic>
#include <cmath>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "../../include/vdbg.h"

namespace {

uint64_t SplitMix(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

double U01(uint64_t x) { return double(SplitMix(x) >> 11) * 0x1.0p-53; }

void Generate(size_t n, size_t dim, uint64_t seed, float* out) {
  const size_t centres = 1000;
  for (size_t r = 0; r < n; ++r) {
    const size_t c = SplitMix(seed ^ (r * 0x2545F4914F6CDD1Dull)) % centres;
    for (size_t j = 0; j < dim; ++j) {
      const double base = 64.0 * U01(0xC0FFEEull + c * dim + j) + 96.0;
      const double noise = 48.0 * (U01(seed + r * dim + j + 1) - 0.5);
      double v = std::nearbyint(base + noise);
      out[r * dim + j] = float(v < 0 ? 0 : (v > 255 ? 255 : v));
    }
  }
}

int Fail(const char* what, int rc) {
  std::fprintf(stderr, "per_query_load: %s: %d %s\n", what, rc, vdbg_last_error());
  return 1;
}

}  // namespace

int main(int argc, char** argv) {
  size_t rows = 1000000, dim = 128, nq = 4096, threads = 16, k = 10, max_batch = 16;
  uint32_t wait_us = 50;
  double seconds = 3.0;
  bool direct = false;
  std::string data, out;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto next = [&]() -> const char* {
      if (i + 1 >= argc) {
        std::fprintf(stderr, "per_query_load: %s needs a value\n", a.c_str());
        std::exit(2);
      }
      return argv[++i];
    };
    if (a == "--rows") rows = std::strtoull(next(), nullptr, 10);
    else if (a == "--dim") dim = std::strtoull(next(), nullptr, 10);
    else if (a == "--queries") nq = std::strtoull(next(), nullptr, 10);
    else if (a == "--threads") threads = std::strtoull(next(), nullptr, 10);
    else if (a == "--k") k = std::strtoull(next(), nullptr, 10);
    else if (a == "--max-batch") max_batch = std::strtoull(next(), nullptr, 10);
    else if (a == "--wait-us") wait_us = uint32_t(std::strtoul(next(), nullptr, 10));
    else if (a == "--seconds") seconds = std::strtod(next(), nullptr);
    else if (a == "--direct") direct = true;
    else if (a == "--data") data = next();
    else if (a == "--out") out = next();
    else {
      std::fprintf(stderr, "per_query_load: unknown argument %s\n", a.c_str());
      return 2;
    }
  }
  if (rows == 0 || nq == 0 || threads == 0 || k == 0 || dim == 0) {
    std::fprintf(stderr, "per_query_load: sizes must be positive\n");
    return 2;
  }
  const size_t pd = (dim + 15) / 16 * 16;
  std::vector<float> base(rows * dim), queries(nq * dim);
  if (!data.empty()) {
    FILE* f = std::fopen(data.c_str(), "rb");
    if (f == nullptr) {
      std::fprintf(stderr, "per_query_load: cannot open %s\n", data.c_str());
      return 2;
    }
    const bool ok = std::fread(base.data(), 4, base.size(), f) == base.size() &&
                    std::fread(queries.data(), 4, queries.size(), f) == queries.size();
    std::fclose(f);
    if (!ok) {
      std::fprintf(stderr, "per_query_load: %s is shorter than the sizes given\n", data.c_str());
      return 2;
    }
  } else {
    Generate(rows, dim, 2002, base.data());
    Generate(nq, dim, 2003, queries.data());
  }
  // rows and queries padded to pd floats
  std::vector<float> rows_p(rows * pd, 0.f), q_p(nq * pd, 0.f);
  for (size_t r = 0; r < rows; ++r) std::memcpy(&rows_p[r * pd], &base[r * dim], dim * 4);
  for (size_t r = 0; r < nq; ++r) std::memcpy(&q_p[r * pd], &queries[r * dim], dim * 4);
  std::vector<float>().swap(base);

  vdbg_ctx* ctx = nullptr;
  vdbg_dataset* ds = nullptr;
  vdbg_coalescer* co = nullptr;
  int rc = vdbg_ctx_create(0, &ctx);
  if (rc != 0) return Fail("context", rc);
  rc = vdbg_dataset_create(ctx, rows_p.data(), rows, dim, pd, VDBG_METRIC_L2, &ds);
  if (rc != 0) return Fail("dataset", rc);
  std::vector<float>().swap(rows_p);
  if (!direct) {
    rc = vdbg_coalescer_create_flat(ds, max_batch, wait_us, &co);
    if (rc != 0) return Fail("coalescer", rc);
  }
  auto one = [&](size_t i, uint32_t* ids, float* d) {
    return direct ? vdbg_flat_search_host(ds, &q_p[i * pd], 1, k, nullptr, ids, d, nullptr)
                  : vdbg_coalescer_search(co, &q_p[i * pd], k, 0, 0, nullptr, ids, d, nullptr);
  };

  // pass 1: every query once, results kept
  std::vector<uint32_t> ids(nq * k);
  std::vector<float> dists(nq * k);
  std::atomic<size_t> next{0};
  std::atomic<int> failed{0};
  auto pass1 = [&]() {
    for (size_t i; (i = next.fetch_add(1)) < nq;)
      if (one(i, &ids[i * k], &dists[i * k]) != 0) {
        std::fprintf(stderr, "per_query_load: query %zu: %s\n", i, vdbg_last_error());
        failed = 1;
        return;
      }
  };
  {
    std::vector<std::thread> pool;
    for (size_t t = 0; t < threads; ++t) pool.emplace_back(pass1);
    for (auto& t : pool) t.join();
  }
  if (failed) return 1;

  // pass 2: timed
  uint64_t b0 = 0, q0 = 0, b1 = 0, q1 = 0;
  if (co != nullptr) vdbg_coalescer_stats(co, &b0, &q0);
  std::atomic<uint64_t> done{0};
  std::atomic<bool> stop{false};
  auto pass2 = [&](size_t t) {
    std::vector<uint32_t> ti(k);
    std::vector<float> td(k);
    uint64_t n = 0;
    for (size_t i = t; !stop.load(std::memory_order_relaxed); i = (i + threads) % nq) {
      if (one(i, ti.data(), td.data()) != 0) {
        failed = 1;
        break;
      }
      ++n;
    }
    done += n;
  };
  const auto t0 = std::chrono::steady_clock::now();
  {
    std::vector<std::thread> pool;
    for (size_t t = 0; t < threads; ++t) pool.emplace_back(pass2, t);
    std::this_thread::sleep_for(std::chrono::duration<double>(seconds));
    stop = true;
    for (auto& t : pool) t.join();
  }
  const double el = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  if (failed) return Fail("timed pass", 1);
  if (co != nullptr) vdbg_coalescer_stats(co, &b1, &q1);

  // the same queries as one batch
  std::vector<uint32_t> bi(nq * k);
  std::vector<float> bd(nq * k);
  rc = vdbg_flat_search_host(ds, q_p.data(), nq, k, nullptr, bi.data(), bd.data(), nullptr);
  if (rc != 0) return Fail("batch", rc);
  size_t differ = 0;
  for (size_t i = 0; i < nq; ++i)
    if (std::memcmp(&ids[i * k], &bi[i * k], k * 4) != 0 ||
        std::memcmp(&dists[i * k], &bd[i * k], k * 4) != 0)
      ++differ;
  if (!out.empty()) {
    FILE* f = std::fopen(out.c_str(), "wb");
    if (f == nullptr || std::fwrite(ids.data(), 4, ids.size(), f) != ids.size() ||
        std::fwrite(dists.data(), 4, dists.size(), f) != dists.size()) {
      std::fprintf(stderr, "per_query_load: cannot write %s\n", out.c_str());
      return 2;
    }
    std::fclose(f);
  }
  const double mean_batch = (b1 > b0) ? double(q1 - q0) / double(b1 - b0) : 1.0;
  std::printf("{\"mode\": \"%s\", \"rows\": %zu, \"dim\": %zu, \"k\": %zu, \"threads\": %zu, "
              "\"max_batch\": %zu, \"wait_us\": %u, \"queries_done\": %llu, \"seconds\": %.3f, "
              "\"qps\": %.1f, \"mean_batch\": %.2f, \"queries_checked\": %zu, "
              "\"differ_from_batch\": %zu}\n",
              direct ? "direct" : "coalesced", rows, dim, k, threads, max_batch, wait_us,
              static_cast<unsigned long long>(done.load()), el, double(done.load()) / el,
              mean_batch, nq, differ);
  if (co != nullptr) vdbg_coalescer_destroy(co);
  vdbg_dataset_destroy(ds);
  vdbg_ctx_destroy(ctx);
  return differ == 0 ? 0 : 3;
}
