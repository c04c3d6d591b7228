// ivf_build.hip -- index construction on the GPU: AssignNearest, Lloyd's k-means, the
// product quantizer's training and the IVF-PQ build.
//
// The reference's construction (src/index/quant/kmeans.cc, pq.cc:14-41, ivf_pq.cc:102-149)
// is reproduced exactly: the seeded std::mt19937_64 draws (subsample, initialisation, empty
// cluster noise) stay on the host with the same standard-library distributions; every
// distance and assignment runs on the GPU with the reference's arithmetic (AVX-512 order for
// padded rows, L2SqAny otherwise, first minimum wins); centroid sums are fp64 over each
// cluster's members in row order (a stable radix sort by cluster, then one thread per
// (cluster, dim)), which is the order of the reference's single loop.
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <numeric>
#include <random>
#include <vector>

#include "vdbg_device.h"
#include "vdbg_internal.h"

namespace vdbg {

int InstallIvf(Ctx* c, IvfIndex* x, hipStream_t s);
void FreeIvf(IvfIndex* x);
int PqEncode(Ctx* c, const float* X, uint32_t n, int pd, int dim, const float* coarse,
             const uint32_t* assign, const float* cen, int m, int dsub, uint8_t* codes,
             hipStream_t s);

namespace {

// ---------------------------------------------------------------- host distances

// l2_sq_avx512 (src/distance/avx512.cc:19-33) lane by lane, for the k-means++ pass.
float HostL2Avx512(const float* a, const float* b, size_t d) {
  float acc0[16] = {0}, acc1[16] = {0};
  size_t i = 0;
  for (; i + 32 <= d; i += 32) {
    for (int l = 0; l < 16; ++l) {
      const float d0 = a[i + l] - b[i + l];
      acc0[l] = std::fma(d0, d0, acc0[l]);
    }
    for (int l = 0; l < 16; ++l) {
      const float d1 = a[i + 16 + l] - b[i + 16 + l];
      acc1[l] = std::fma(d1, d1, acc1[l]);
    }
  }
  if (i < d)
    for (int l = 0; l < 16; ++l) {
      const float d0 = a[i + l] - b[i + l];
      acc0[l] = std::fma(d0, d0, acc0[l]);
    }
  float v[16], t3[8], t6[4];
  for (int l = 0; l < 16; ++l) v[l] = acc0[l] + acc1[l];
  for (int l = 0; l < 8; ++l) t3[l] = v[8 + l] + v[l];
  for (int l = 0; l < 4; ++l) t6[l] = t3[4 + l] + t3[l];
  return (t6[0] + t6[2]) + (t6[1] + t6[3]);
}

// L2SqAny (src/distance/scalar.cc:43-60).
float HostL2Any(const float* a, const float* b, size_t d) {
  float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
  size_t i = 0;
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

// l2_sq_avx2 (src/distance/avx2.cc:26-35) and l2_sq_scalar (scalar.cc:8-15).
float HostL2Avx2(const float* a, const float* b, size_t d) {
  float acc0[8] = {0}, acc1[8] = {0};
  for (size_t i = 0; i < d; i += 16)
    for (int l = 0; l < 8; ++l) {
      const float d0 = a[i + l] - b[i + l];
      acc0[l] = std::fma(d0, d0, acc0[l]);
      const float d1 = a[i + 8 + l] - b[i + 8 + l];
      acc1[l] = std::fma(d1, d1, acc1[l]);
    }
  float v[8], h[4];
  for (int l = 0; l < 8; ++l) v[l] = acc0[l] + acc1[l];
  for (int l = 0; l < 4; ++l) h[l] = v[l] + v[4 + l];
  return (h[0] + h[1]) + (h[2] + h[3]);
}
float HostL2Scalar(const float* a, const float* b, size_t d) {
  float s = 0.f;
  for (size_t i = 0; i < d; ++i) {
    const float t = a[i] - b[i];
    s += t * t;
  }
  return s;
}
float HostL2Kset(int kset, const float* a, const float* b, size_t d) {
  return kset == 2 ? HostL2Avx512(a, b, d) : kset == 1 ? HostL2Avx2(a, b, d) : HostL2Scalar(a, b, d);
}

// PickL2 (src/index/quant/kmeans.cc:16-19): the kernel set's L2 when rows are padded.
bool SimdL2(size_t d, size_t stride) { return d % 16 == 0 && stride % 16 == 0; }

}  // namespace

// ---------------------------------------------------------------- device kernels

template <int D>
__device__ __forceinline__ float l2any_fixed(const float* a, const float* b, int d) {
  const int dd = D > 0 ? D : d;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  int i = 0;
#pragma unroll
  for (; i + 4 <= dd; i += 4) {
    const float t0 = a[i] - b[i], t1 = a[i + 1] - b[i + 1];
    const float t2 = a[i + 2] - b[i + 2], t3 = a[i + 3] - b[i + 3];
    s0 += t0 * t0;
    s1 += t1 * t1;
    s2 += t2 * t2;
    s3 += t3 * t3;
  }
  for (; i < dd; ++i) {
    const float t = a[i] - b[i];
    s0 += t * t;
  }
  return (s0 + s1) + (s2 + s3);
}

// AssignNearest with L2SqAny (kmeans.cc:23-55 when rows are not padded): one thread per
// point, the first centroid with the smallest distance.  Centroids staged in LDS.
template <int D>
__global__ __launch_bounds__(256) void k_assign_any(const float* __restrict__ x, uint32_t n, int d,
                                                    int stride, const float* __restrict__ cen,
                                                    int k, uint32_t* __restrict__ assign,
                                                    float* __restrict__ dist) {
  extern __shared__ float cs[];
  for (int i = threadIdx.x; i < k * d; i += blockDim.x) cs[i] = cen[i];
  __syncthreads();
  const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n) return;
  float xr[D > 0 ? D : 64];
  const int dd = D > 0 ? D : d;
  for (int i = 0; i < dd; ++i) xr[i] = x[size_t(p) * stride + i];
  float best = __builtin_inff();
  uint32_t arg = 0;
  for (int c = 0; c < k; ++c) {
    const float v = l2any_fixed<D>(xr, cs + c * dd, dd);
    if (v < best) {
      best = v;
      arg = uint32_t(c);
    }
  }
  assign[p] = arg;
  if (dist != nullptr) dist[p] = best;
}

// The same for rows too wide to stage (d > 64): rows and centroids read where they lie.
__global__ __launch_bounds__(256) void k_assign_wide(const float* __restrict__ x, uint32_t n,
                                                     int d, int stride,
                                                     const float* __restrict__ cen, int k,
                                                     uint32_t* __restrict__ assign,
                                                     float* __restrict__ dist) {
  const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n) return;
  const float* xr = x + size_t(p) * stride;
  float best = __builtin_inff();
  uint32_t arg = 0;
  for (int c = 0; c < k; ++c) {
    const float v = l2sq_any(xr, cen + size_t(c) * d, d);
    if (v < best) {
      best = v;
      arg = uint32_t(c);
    }
  }
  assign[p] = arg;
  if (dist != nullptr) dist[p] = best;
}

__global__ void k_iota(uint32_t* v, uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) v[i] = i;
}

__global__ void k_histogram(const uint32_t* __restrict__ a, uint32_t n, uint32_t* __restrict__ counts) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) atomicAdd(&counts[a[i]], 1u);
}

// Centroid update (kmeans.cc:146-158): fp64 sums of each cluster's members in row order,
// float(sum * (1.0 / count)) for non-empty clusters.  grid = clusters, threads over dims.
__global__ void k_centroid_update(const float* __restrict__ x, int d, int stride,
                                  const uint32_t* __restrict__ order, const uint32_t* __restrict__ off,
                                  float* __restrict__ cen) {
  const int c = blockIdx.x;
  const uint32_t b = off[c], e = off[c + 1];
  if (b == e) return;
  const double inv = 1.0 / double(e - b);
  for (int j = threadIdx.x; j < d; j += blockDim.x) {
    double s = 0.0;
    for (uint32_t t = b; t < e; ++t) s += double(x[size_t(order[t]) * stride + j]);
    cen[size_t(c) * d + j] = float(s * inv);
  }
}

__global__ void k_gather_rows(const float* __restrict__ x, int stride, const uint32_t* __restrict__ idx,
                              uint32_t n, int d, int xo, float* __restrict__ out) {
  const size_t t = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (t >= size_t(n) * d) return;
  const size_t r = t / d, j = t - r * d;
  out[t] = x[size_t(idx[r]) * stride + xo + j];
}

// Residuals x - coarse[assign] over the real dims (ivf_pq.cc:116-124, 128-139).
__global__ void k_residuals(const float* __restrict__ X, int pd, int dim,
                            const float* __restrict__ coarse, const uint32_t* __restrict__ assign,
                            const uint32_t* __restrict__ rows, uint32_t nrows, float* __restrict__ out) {
  const size_t t = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (t >= size_t(nrows) * dim) return;
  const size_t r = t / dim, j = t - r * dim;
  const uint32_t i = rows[r];
  out[t] = X[size_t(i) * pd + j] - coarse[size_t(assign[i]) * pd + j];
}

__global__ void k_gather_codes(const uint8_t* __restrict__ all, const uint32_t* __restrict__ order,
                               uint32_t n, int m, uint8_t* __restrict__ out) {
  const size_t t = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (t >= size_t(n) * m) return;
  const size_t r = t / m, j = t - r * m;
  out[t] = all[size_t(order[r]) * m + j];
}

// ---------------------------------------------------------------- host orchestration

struct DevBuf {
  void* p = nullptr;
  hipStream_t s = nullptr;
  ~DevBuf() {
    if (p) (void)hipFreeAsync(p, s);
  }
  template <class T>
  T* get() const {
    return static_cast<T*>(p);
  }
};

static int Alloc(DevBuf* b, size_t bytes, hipStream_t s) {
  b->s = s;
  VDBG_HIP(hipMallocAsync(&b->p, std::max<size_t>(bytes, 16), s));
  return kOk;
}

// AssignNearest (kmeans.cc:23-55): x is n rows of d floats at `stride`, centroids k x d
// (device).  Padded rows go through the exact scan with k = 1 (AVX-512 order, ties to the
// lowest index); other shapes through L2SqAny.
int AssignNearestGpu(Ctx* c, const float* x, size_t n, size_t d, size_t stride, const float* cen,
                     size_t k, uint32_t* assign, float* dist, hipStream_t s) {
  if (n == 0) return kOk;
  if (SimdL2(d, stride)) {
    if (stride != d) return SetError(kNotSupported, "AssignNearest: padded rows need stride == d");
    vdbg_dataset* cds = nullptr;
    VDBG_RETURN_IF_ERROR(vdbg_dataset_create_device(c->handle, cen, k, d, d, 0, &cds));
    DevBuf dd;
    int rc = dist ? kOk : Alloc(&dd, n * sizeof(float), s);
    if (rc == kOk) rc = RunScan(c, &cds->d.src, x, n, 1, nullptr, assign, dist ? dist : dd.get<float>(), s);
    if (rc == kOk) rc = hipStreamSynchronize(s) == hipSuccess ? kOk : SetError(kInternal, "sync");
    vdbg_dataset_destroy(cds);
    return rc;
  }
  const size_t lds = k * d * sizeof(float);
  ProfScope ps(c, "assign_any", s);
  const dim3 grid(unsigned((n + 255) / 256));
  if (d > 64 || lds > 64 * 1024) {
    k_assign_wide<<<grid, 256, 0, s>>>(x, uint32_t(n), int(d), int(stride), cen, int(k), assign,
                                       dist);
    VDBG_HIP(hipGetLastError());
    return kOk;
  }
#define VDBG_ASSIGN(DD) k_assign_any<DD><<<grid, 256, lds, s>>>(x, uint32_t(n), int(d), int(stride), cen, int(k), assign, dist)
  switch (d) {
    case 4: VDBG_ASSIGN(4); break;
    case 8: VDBG_ASSIGN(8); break;
    case 12: VDBG_ASSIGN(12); break;
    case 24: VDBG_ASSIGN(24); break;
    default: VDBG_ASSIGN(0); break;
  }
#undef VDBG_ASSIGN
  VDBG_HIP(hipGetLastError());
  return kOk;
}

struct KMeansOpts {
  size_t iters = 25;
  uint64_t seed = 1234;
  size_t max_points = 256;
  bool kmeanspp = true;
};

struct KMeansInfo {
  double inertia = 0;
  size_t train_points = 0, empty_reseeds = 0, iterations = 0;
};

// KMeans (kmeans.cc:57-174) over n device rows of d floats at `stride`.
int KMeansGpu(Ctx* c, const float* data, size_t n, size_t d, size_t stride, size_t k,
              const KMeansOpts& o, std::vector<float>* centroids, KMeansInfo* info, hipStream_t s) {
  if (k == 0 || d == 0) return SetError(kInvalidArgument, "k-means needs k > 0 and d > 0");
  if (n == 0) return SetError(kInvalidArgument, "k-means needs training points");
  centroids->assign(k * d, 0.f);
  std::mt19937_64 rng(o.seed);
  KMeansInfo st;

  // Fewer points than centroids: the points themselves, with duplicates.
  if (n <= k) {
    std::vector<float> rows(n * stride);
    VDBG_HIP(hipMemcpyAsync(rows.data(), data, n * stride * sizeof(float), hipMemcpyDeviceToHost, s));
    VDBG_HIP(hipStreamSynchronize(s));
    for (size_t q = 0; q < k; ++q)
      std::memcpy(centroids->data() + q * d, rows.data() + (q % n) * stride, d * sizeof(float));
    st.train_points = n;
    if (info) *info = st;
    return kOk;
  }

  // Subsample to k * max_points rows: partial Fisher-Yates, then sorted.
  const size_t m = std::min(n, k * std::max<size_t>(1, o.max_points));
  DevBuf sample;
  const float* x = data;
  size_t xs = stride;
  if (m < n) {
    std::vector<size_t> idx(n);
    std::iota(idx.begin(), idx.end(), 0);
    for (size_t i = 0; i < m; ++i) {
      std::uniform_int_distribution<size_t> u(i, n - 1);
      std::swap(idx[i], idx[u(rng)]);
    }
    std::sort(idx.begin(), idx.begin() + static_cast<std::ptrdiff_t>(m));
    std::vector<uint32_t> idx32(idx.begin(), idx.begin() + static_cast<std::ptrdiff_t>(m));
    DevBuf di;
    VDBG_RETURN_IF_ERROR(Alloc(&di, m * 4, s));
    VDBG_RETURN_IF_ERROR(Alloc(&sample, m * d * sizeof(float), s));
    VDBG_HIP(hipMemcpyAsync(di.p, idx32.data(), m * 4, hipMemcpyHostToDevice, s));
    k_gather_rows<<<dim3(unsigned((m * d + 255) / 256)), 256, 0, s>>>(
        data, int(stride), di.get<uint32_t>(), uint32_t(m), int(d), 0, sample.get<float>());
    VDBG_HIP(hipGetLastError());
    VDBG_HIP(hipStreamSynchronize(s));
    x = sample.get<float>();
    xs = d;
  }
  const bool simd = SimdL2(d, xs);
  auto fn = [&](const float* a, const float* b) {
    return simd ? HostL2Kset(c->kset, a, b, d) : HostL2Any(a, b, d);
  };

  // Initialisation.
  float* cen = centroids->data();
  const bool use_pp = o.kmeanspp && static_cast<double>(k) * static_cast<double>(m) <= 2.0e7;
  if (use_pp) {
    std::vector<float> xh(m * xs);
    VDBG_HIP(hipMemcpyAsync(xh.data(), x, m * xs * sizeof(float), hipMemcpyDeviceToHost, s));
    VDBG_HIP(hipStreamSynchronize(s));
    std::vector<float> mind(m, std::numeric_limits<float>::infinity());
    std::uniform_int_distribution<size_t> u0(0, m - 1);
    const size_t first = u0(rng);
    std::memcpy(cen, xh.data() + first * xs, d * sizeof(float));
    for (size_t q = 1; q < k; ++q) {
      const float* last = cen + (q - 1) * d;
      double total = 0;
      for (size_t i = 0; i < m; ++i) {
        mind[i] = std::min(mind[i], fn(xh.data() + i * xs, last));
        total += mind[i];
      }
      size_t pick = 0;
      if (total > 0) {
        std::uniform_real_distribution<double> ur(0.0, total);
        const double t = ur(rng);
        double acc = 0;
        for (pick = 0; pick + 1 < m; ++pick) {
          acc += mind[pick];
          if (acc >= t) break;
        }
      } else {
        pick = u0(rng);
      }
      std::memcpy(cen + q * d, xh.data() + pick * xs, d * sizeof(float));
    }
  } else {
    std::vector<size_t> idx(m);
    std::iota(idx.begin(), idx.end(), 0);
    std::vector<uint32_t> rows(k);
    for (size_t q = 0; q < k; ++q) {
      std::uniform_int_distribution<size_t> u(q, m - 1);
      std::swap(idx[q], idx[u(rng)]);
      rows[q] = uint32_t(idx[q]);
    }
    DevBuf dr, dc;
    VDBG_RETURN_IF_ERROR(Alloc(&dr, k * 4, s));
    VDBG_RETURN_IF_ERROR(Alloc(&dc, k * d * sizeof(float), s));
    VDBG_HIP(hipMemcpyAsync(dr.p, rows.data(), k * 4, hipMemcpyHostToDevice, s));
    k_gather_rows<<<dim3(unsigned((k * d + 255) / 256)), 256, 0, s>>>(
        x, int(xs), dr.get<uint32_t>(), uint32_t(k), int(d), 0, dc.get<float>());
    VDBG_HIP(hipGetLastError());
    VDBG_HIP(hipMemcpyAsync(cen, dc.p, k * d * sizeof(float), hipMemcpyDeviceToHost, s));
    VDBG_HIP(hipStreamSynchronize(s));
  }

  // Lloyd iterations.
  DevBuf dcen, assign, dist, keys_out, vals_in, vals_out, counts, off, tmp;
  VDBG_RETURN_IF_ERROR(Alloc(&dcen, k * d * sizeof(float), s));
  VDBG_RETURN_IF_ERROR(Alloc(&assign, m * 4, s));
  VDBG_RETURN_IF_ERROR(Alloc(&dist, m * 4, s));
  VDBG_RETURN_IF_ERROR(Alloc(&keys_out, m * 4, s));
  VDBG_RETURN_IF_ERROR(Alloc(&vals_in, m * 4, s));
  VDBG_RETURN_IF_ERROR(Alloc(&vals_out, m * 4, s));
  VDBG_RETURN_IF_ERROR(Alloc(&counts, k * 4, s));
  VDBG_RETURN_IF_ERROR(Alloc(&off, (k + 1) * 4, s));
  int end_bit = 1;
  while ((size_t(1) << end_bit) < k) ++end_bit;
  size_t tmp_bytes = 0;
  VDBG_HIP(hipcub::DeviceRadixSort::SortPairs(nullptr, tmp_bytes, assign.get<uint32_t>(),
                                              keys_out.get<uint32_t>(), vals_in.get<uint32_t>(),
                                              vals_out.get<uint32_t>(), int(m), 0, end_bit, s));
  VDBG_RETURN_IF_ERROR(Alloc(&tmp, tmp_bytes, s));
  k_iota<<<dim3(unsigned((m + 255) / 256)), 256, 0, s>>>(vals_in.get<uint32_t>(), uint32_t(m));
  VDBG_HIP(hipGetLastError());
  std::vector<uint32_t> cnt(k), offh(k + 1);
  std::vector<float> disth(m);
  st.train_points = m;
  constexpr float kEps = 1.0f / 1024.0f;
  for (size_t it = 0; it < o.iters; ++it) {
    VDBG_HIP(hipMemcpyAsync(dcen.p, cen, k * d * sizeof(float), hipMemcpyHostToDevice, s));
    VDBG_RETURN_IF_ERROR(AssignNearestGpu(c, x, m, d, xs, dcen.get<float>(), k,
                                          assign.get<uint32_t>(), dist.get<float>(), s));
    VDBG_HIP(hipMemsetAsync(counts.p, 0, k * 4, s));
    k_histogram<<<dim3(unsigned((m + 255) / 256)), 256, 0, s>>>(assign.get<uint32_t>(), uint32_t(m),
                                                                counts.get<uint32_t>());
    VDBG_HIP(hipGetLastError());
    VDBG_HIP(hipcub::DeviceRadixSort::SortPairs(tmp.p, tmp_bytes, assign.get<uint32_t>(),
                                                keys_out.get<uint32_t>(), vals_in.get<uint32_t>(),
                                                vals_out.get<uint32_t>(), int(m), 0, end_bit, s));
    VDBG_HIP(hipMemcpyAsync(cnt.data(), counts.p, k * 4, hipMemcpyDeviceToHost, s));
    VDBG_HIP(hipMemcpyAsync(disth.data(), dist.p, m * 4, hipMemcpyDeviceToHost, s));
    VDBG_HIP(hipStreamSynchronize(s));
    st.inertia = 0;
    for (size_t i = 0; i < m; ++i) st.inertia += disth[i];
    offh[0] = 0;
    for (size_t q = 0; q < k; ++q) offh[q + 1] = offh[q] + cnt[q];
    VDBG_HIP(hipMemcpyAsync(off.p, offh.data(), (k + 1) * 4, hipMemcpyHostToDevice, s));
    k_centroid_update<<<dim3(unsigned(k)), unsigned(std::min<size_t>(256, (d + 63) / 64 * 64)), 0, s>>>(
        x, int(d), int(xs), vals_out.get<uint32_t>(), off.get<uint32_t>(), dcen.get<float>());
    VDBG_HIP(hipGetLastError());
    VDBG_HIP(hipMemcpyAsync(cen, dcen.p, k * d * sizeof(float), hipMemcpyDeviceToHost, s));
    VDBG_HIP(hipStreamSynchronize(s));
    // Empty clusters: split the largest in two with a symmetric perturbation (:159-172).
    std::vector<size_t> counts_sz(cnt.begin(), cnt.end());
    for (size_t q = 0; q < k; ++q) {
      if (counts_sz[q] != 0) continue;
      const size_t big = static_cast<size_t>(
          std::max_element(counts_sz.begin(), counts_sz.end()) - counts_sz.begin());
      std::uniform_real_distribution<float> noise(-1.f, 1.f);
      for (size_t j = 0; j < d; ++j) {
        const float v = cen[big * d + j];
        const float delta = kEps * (std::fabs(v) + 1e-3f) * noise(rng);
        cen[q * d + j] = v + delta;
        cen[big * d + j] = v - delta;
      }
      counts_sz[q] = counts_sz[big] / 2;
      counts_sz[big] -= counts_sz[q];
      ++st.empty_reseeds;
    }
    st.iterations = it + 1;
  }
  if (info) *info = st;
  return kOk;
}

// ProductQuantizer::train (src/index/quant/pq.cc:14-41) on n device rows at `stride`.
int PqTrainGpu(Ctx* c, const float* data, size_t n, size_t stride, size_t dim, size_t m,
               const KMeansOpts& opts, std::vector<float>* centroids, hipStream_t s) {
  if (m == 0 || dim % m != 0)
    return SetError(kInvalidArgument, "pq_m must divide the dimension (dim " + std::to_string(dim) +
                                          ", m " + std::to_string(m) + ")");
  const size_t dsub = dim / m;
  centroids->assign(m * 256 * dsub, 0.f);
  const size_t cap = std::min(n, size_t(256) * std::max<size_t>(1, opts.max_points));
  const size_t step = std::max<size_t>(1, n / std::max<size_t>(1, cap));
  std::vector<uint32_t> rows;
  for (size_t i = 0, taken = 0; i < n && taken < cap; i += step, ++taken) rows.push_back(uint32_t(i));
  DevBuf dr, sub;
  VDBG_RETURN_IF_ERROR(Alloc(&dr, rows.size() * 4, s));
  VDBG_RETURN_IF_ERROR(Alloc(&sub, rows.size() * dsub * sizeof(float), s));
  VDBG_HIP(hipMemcpyAsync(dr.p, rows.data(), rows.size() * 4, hipMemcpyHostToDevice, s));
  std::vector<float> cen;
  for (size_t j = 0; j < m; ++j) {
    k_gather_rows<<<dim3(unsigned((rows.size() * dsub + 255) / 256)), 256, 0, s>>>(
        data, int(stride), dr.get<uint32_t>(), uint32_t(rows.size()), int(dsub), int(j * dsub),
        sub.get<float>());
    VDBG_HIP(hipGetLastError());
    KMeansOpts o = opts;
    o.seed = opts.seed + j * 7919;
    VDBG_RETURN_IF_ERROR(KMeansGpu(c, sub.get<float>(), rows.size(), dsub, dsub, 256, o, &cen,
                                   nullptr, s));
    std::memcpy(centroids->data() + j * 256 * dsub, cen.data(), 256 * dsub * sizeof(float));
  }
  return kOk;
}

// ProductQuantizer::train with IndexOptions' k-means settings (MakeKMeansOptions,
// ivf_pq.cc:21-26), for callers outside this file (PqFlatIndex::build).
int PqTrainRows(Ctx* c, const float* data, size_t n, size_t stride, size_t dim, size_t m,
                uint64_t seed, size_t max_points, size_t iters, std::vector<float>* centroids,
                hipStream_t s) {
  KMeansOpts ko;
  ko.seed = seed;
  ko.max_points = max_points;
  ko.iters = iters;
  return PqTrainGpu(c, data, n, stride, dim, m, ko, centroids, s);
}

// IvfPqIndex::build (ivf_pq.cc:102-149).
int IvfBuildGpu(Ctx* c, IvfIndex* x, size_t nlist_req, size_t m, uint64_t seed, size_t max_points,
                size_t iters, hipStream_t s) {
  Dataset* ds = x->ds;
  const size_t n = ds->n, pd = ds->pd, d = ds->dim;
  if (m == 0 || d % m != 0) return SetError(kInvalidArgument, "pq_m must divide the dimension");
  x->pd = int(pd);
  x->dim = int(d);
  x->m = int(m);
  x->dsub = int(d / m);
  x->metric = ds->metric;
  if (n == 0) {
    x->nlist = 0;
    x->off_h.assign(1, 0);
    return kOk;
  }
  // Small segments get fewer lists (FAISS warns below 39 training points per centroid).
  const size_t nlist = std::clamp<size_t>(nlist_req, 1, std::max<size_t>(1, n / 39));
  x->nlist = int(nlist);
  KMeansOpts ko;
  ko.seed = seed;
  ko.max_points = max_points;
  ko.iters = iters;
  VDBG_RETURN_IF_ERROR(KMeansGpu(c, ds->rows, n, pd, pd, nlist, ko, &x->coarse_h, nullptr, s));

  DevBuf dcoarse, assign;
  VDBG_RETURN_IF_ERROR(Alloc(&dcoarse, nlist * pd * sizeof(float), s));
  VDBG_RETURN_IF_ERROR(Alloc(&assign, n * 4, s));
  VDBG_HIP(hipMemcpyAsync(dcoarse.p, x->coarse_h.data(), nlist * pd * sizeof(float),
                          hipMemcpyHostToDevice, s));
  VDBG_RETURN_IF_ERROR(AssignNearestGpu(c, ds->rows, n, pd, pd, dcoarse.get<float>(), nlist,
                                        assign.get<uint32_t>(), nullptr, s));

  // Train PQ on residuals of a strided sample (<= 65,536 rows).
  constexpr size_t kMaxPqTrainRows = 65536;
  const size_t step = std::max<size_t>(1, n / kMaxPqTrainRows);
  std::vector<uint32_t> rows;
  for (size_t i = 0; i < n; i += step) rows.push_back(uint32_t(i));
  DevBuf drows, res;
  VDBG_RETURN_IF_ERROR(Alloc(&drows, rows.size() * 4, s));
  VDBG_RETURN_IF_ERROR(Alloc(&res, rows.size() * d * sizeof(float), s));
  VDBG_HIP(hipMemcpyAsync(drows.p, rows.data(), rows.size() * 4, hipMemcpyHostToDevice, s));
  k_residuals<<<dim3(unsigned((rows.size() * d + 255) / 256)), 256, 0, s>>>(
      ds->rows, int(pd), int(d), dcoarse.get<float>(), assign.get<uint32_t>(),
      drows.get<uint32_t>(), uint32_t(rows.size()), res.get<float>());
  VDBG_HIP(hipGetLastError());
  VDBG_RETURN_IF_ERROR(PqTrainGpu(c, res.get<float>(), rows.size(), d, d, m, ko, &x->cen_h, s));

  // Encode every row's residual, then the lists: ids ascending within a list.
  DevBuf dcen, all, order_in, order_out, keys_out, counts, tmp;
  VDBG_RETURN_IF_ERROR(Alloc(&dcen, x->cen_h.size() * sizeof(float), s));
  VDBG_RETURN_IF_ERROR(Alloc(&all, n * m, s));
  VDBG_HIP(hipMemcpyAsync(dcen.p, x->cen_h.data(), x->cen_h.size() * sizeof(float),
                          hipMemcpyHostToDevice, s));
  VDBG_RETURN_IF_ERROR(PqEncode(c, ds->rows, uint32_t(n), int(pd), int(d), dcoarse.get<float>(),
                                assign.get<uint32_t>(), dcen.get<float>(), int(m), int(d / m),
                                all.get<uint8_t>(), s));
  VDBG_RETURN_IF_ERROR(Alloc(&order_in, n * 4, s));
  VDBG_RETURN_IF_ERROR(Alloc(&keys_out, n * 4, s));
  VDBG_RETURN_IF_ERROR(Alloc(&counts, nlist * 4, s));
  VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&x->ids), n * 4));
  VDBG_HIP(hipMalloc(reinterpret_cast<void**>(&x->codes), n * m));
  k_iota<<<dim3(unsigned((n + 255) / 256)), 256, 0, s>>>(order_in.get<uint32_t>(), uint32_t(n));
  VDBG_HIP(hipMemsetAsync(counts.p, 0, nlist * 4, s));
  k_histogram<<<dim3(unsigned((n + 255) / 256)), 256, 0, s>>>(assign.get<uint32_t>(), uint32_t(n),
                                                              counts.get<uint32_t>());
  int end_bit = 1;
  while ((size_t(1) << end_bit) < nlist) ++end_bit;
  size_t tmp_bytes = 0;
  VDBG_HIP(hipcub::DeviceRadixSort::SortPairs(nullptr, tmp_bytes, assign.get<uint32_t>(),
                                              keys_out.get<uint32_t>(), order_in.get<uint32_t>(),
                                              x->ids, int(n), 0, end_bit, s));
  VDBG_RETURN_IF_ERROR(Alloc(&tmp, tmp_bytes, s));
  VDBG_HIP(hipcub::DeviceRadixSort::SortPairs(tmp.p, tmp_bytes, assign.get<uint32_t>(),
                                              keys_out.get<uint32_t>(), order_in.get<uint32_t>(),
                                              x->ids, int(n), 0, end_bit, s));
  k_gather_codes<<<dim3(unsigned((n * m + 255) / 256)), 256, 0, s>>>(all.get<uint8_t>(), x->ids,
                                                                     uint32_t(n), int(m), x->codes);
  VDBG_HIP(hipGetLastError());
  std::vector<uint32_t> cnt(nlist);
  VDBG_HIP(hipMemcpyAsync(cnt.data(), counts.p, nlist * 4, hipMemcpyDeviceToHost, s));
  VDBG_HIP(hipStreamSynchronize(s));
  x->off_h.assign(nlist + 1, 0);
  for (size_t l = 0; l < nlist; ++l) x->off_h[l + 1] = x->off_h[l] + cnt[l];
  return InstallIvf(c, x, s);
}

}  // namespace vdbg

using namespace vdbg;

extern "C" {

int vdbg_kmeans(vdbg_ctx* ctx, const float* data, size_t n, size_t d, size_t stride, size_t k,
                size_t iters, uint64_t seed, size_t max_points_per_centroid, int kmeanspp,
                float* centroids_out, double* inertia, size_t* empty_reseeds) {
  if (ctx == nullptr || (n > 0 && data == nullptr) || centroids_out == nullptr || stride < d)
    return SetError(kInvalidArgument, "bad argument");
  Ctx* c = &ctx->c;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  DevBuf dd;
  VDBG_RETURN_IF_ERROR(Alloc(&dd, std::max<size_t>(1, n * stride) * sizeof(float), s));
  if (n > 0)
    VDBG_HIP(hipMemcpyAsync(dd.p, data, n * stride * sizeof(float), hipMemcpyHostToDevice, s));
  KMeansOpts o;
  o.iters = iters;
  o.seed = seed;
  o.max_points = max_points_per_centroid;
  o.kmeanspp = kmeanspp != 0;
  std::vector<float> cen;
  KMeansInfo info;
  VDBG_RETURN_IF_ERROR(KMeansGpu(c, dd.get<float>(), n, d, stride, k, o, &cen, &info, s));
  std::memcpy(centroids_out, cen.data(), cen.size() * sizeof(float));
  if (inertia) *inertia = info.inertia;
  if (empty_reseeds) *empty_reseeds = info.empty_reseeds;
  return kOk;
}

int vdbg_assign_nearest(vdbg_ctx* ctx, const float* data, size_t n, size_t d, size_t stride,
                        const float* centroids, size_t k, uint32_t* assign, float* dist) {
  if (ctx == nullptr || (n > 0 && (data == nullptr || assign == nullptr)) || centroids == nullptr ||
      stride < d || k == 0)
    return SetError(kInvalidArgument, "bad argument");
  Ctx* c = &ctx->c;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  if (n == 0) return kOk;
  DevBuf dd, dc, da, dist_d;
  VDBG_RETURN_IF_ERROR(Alloc(&dd, n * stride * sizeof(float), s));
  VDBG_RETURN_IF_ERROR(Alloc(&dc, k * d * sizeof(float), s));
  VDBG_RETURN_IF_ERROR(Alloc(&da, n * 4, s));
  VDBG_RETURN_IF_ERROR(Alloc(&dist_d, n * 4, s));
  VDBG_HIP(hipMemcpyAsync(dd.p, data, n * stride * sizeof(float), hipMemcpyHostToDevice, s));
  VDBG_HIP(hipMemcpyAsync(dc.p, centroids, k * d * sizeof(float), hipMemcpyHostToDevice, s));
  VDBG_RETURN_IF_ERROR(AssignNearestGpu(c, dd.get<float>(), n, d, stride, dc.get<float>(), k,
                                        da.get<uint32_t>(), dist_d.get<float>(), s));
  VDBG_HIP(hipMemcpyAsync(assign, da.p, n * 4, hipMemcpyDeviceToHost, s));
  if (dist) VDBG_HIP(hipMemcpyAsync(dist, dist_d.p, n * 4, hipMemcpyDeviceToHost, s));
  VDBG_HIP(hipStreamSynchronize(s));
  return kOk;
}

int vdbg_ivfpq_build(vdbg_dataset* ds, size_t nlist, size_t pq_m, uint64_t seed,
                     size_t max_train_points_per_centroid, size_t kmeans_iters, vdbg_ivfpq** out) {
  if (ds == nullptr || out == nullptr) return SetError(kInvalidArgument, "null argument");
  Ctx* c = ds->d.ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  VDBG_HIP(hipSetDevice(c->device));
  auto* h = new (std::nothrow) vdbg_ivfpq;
  if (h == nullptr) return SetError(kResourceExhausted, "out of host memory");
  h->x.ds = &ds->d;
  int rc = IvfBuildGpu(c, &h->x, nlist, pq_m, seed, max_train_points_per_centroid, kmeans_iters,
                       c->stream);
  if (rc != kOk) {
    FreeIvf(&h->x);
    delete h;
    return rc;
  }
  ++ds->d.live_indexes;
  *out = h;
  return kOk;
}

}  // extern "C"
