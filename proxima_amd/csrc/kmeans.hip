// k-means and product-quantizer training on MI355X
// (crates/proxima-quantize/src/kmeans.rs, product.rs:198-380).
//
// Assignment (kmeans.rs:90-97, nearest 200-212): one thread per point, the
// point's coordinates in registers when dim is a compiled width, centroids
// staged through LDS and read as wave-wide broadcasts; each distance is the
// reference's own sequential `squared` (or the 8-lane unrolled kernel for the
// IVF coarse quantizer), scanned in centroid order with strict `<`, so the
// assignment and the best distance are the reference's bit for bit.
//
// Update (kmeans.rs:104-135): points are grouped by cluster with a stable
// radix sort (so each cluster's members stay in point order), then one thread
// per (cluster, coordinate) sums the members' coordinates in f64 in that
// order and writes (float)(sum * (1.0 / count)) -- the reference's rounding
// sequence. Empty clusters are re-seeded in ascending order onto
// farthest_point (kmeans.rs:215-226) evaluated against the partially updated
// centroid array, exactly as the sequential loop sees it.
//
// Inertia and k-means++ totals are f64 sums over points in point order. Up to
// SEQ_SUM_LIMIT points they are evaluated sequentially on the device (the
// reference's rounding); above it, in a fixed tree order (deterministic; the
// last bits can differ from the sequential sum, which can change a k-means++
// pick only when the drawn target falls within that difference of a
// cumulative boundary).
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>

#include "common.hpp"
#include "device.hpp"
#include "train.hpp"

namespace pxg {

constexpr int KM_LDS_FLOATS = 8192;  // 32 KiB of staged centroids
constexpr size_t SEQ_SUM_LIMIT = 1u << 17;

// ---------------------------------------------------------------------------
// assignment
// ---------------------------------------------------------------------------
template <int D, bool UNR>
__device__ inline float point_dist(const float* x, const float* __restrict__ c, int dim) {
  constexpr int DD = D > 0 ? D : 1;
  (void)DD;
  if constexpr (!UNR) {
    float sum = 0.0f;  // squared(), kmeans.rs:234-241
    if constexpr (D > 0) {
#pragma unroll
      for (int j = 0; j < D; ++j) {
        const float d = x[j] - c[j];
        sum += d * d;
      }
    } else {
      for (int j = 0; j < dim; ++j) {
        const float d = x[j] - c[j];
        sum += d * d;
      }
    }
    return sum;
  } else {
    // squared_euclidean_unrolled, distance.rs:267-283
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int n = D > 0 ? D : dim;
    const int chunks = n >> 3;
    if constexpr (D > 0) {
#pragma unroll
      for (int cc = 0; cc < D / 8; ++cc)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float d = x[cc * 8 + j] - c[cc * 8 + j];
          acc[j] += d * d;
        }
    } else {
      for (int cc = 0; cc < chunks; ++cc)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float d = x[cc * 8 + j] - c[cc * 8 + j];
          acc[j] += d * d;
        }
    }
    float tail = 0.0f;
    for (int i = chunks * 8; i < n; ++i) {
      const float d = x[i] - c[i];
      tail += d * d;
    }
    return (((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]))) + tail;
  }
}

template <int D, bool UNR>
__global__ __launch_bounds__(256) void km_assign(const float* __restrict__ P, int ldp, const uint32_t* __restrict__ rows,
                                                 int n, int dim, const float* __restrict__ C, int ldc, int k,
                                                 uint32_t* __restrict__ assign, float* __restrict__ dist) {
  __shared__ float cs[KM_LDS_FLOATS];
  const int i = blockIdx.x * 256 + threadIdx.x;
  const bool valid = i < n;
  const size_t row = valid ? (rows ? rows[i] : (uint32_t)i) : 0;
  const float* pr = P + row * ldp;
  constexpr int DR = D > 0 ? D : 1;
  float x[DR];
  if constexpr (D > 0) {
#pragma unroll
    for (int j = 0; j < D; ++j) x[j] = valid ? pr[j] : 0.0f;
  }
  float bd = INFINITY;
  int bi = 0;
  const bool staged = dim <= KM_LDS_FLOATS;
  const int per = staged ? KM_LDS_FLOATS / dim : 1;
  for (int c0 = 0; c0 < k; c0 += per) {
    const int r = min(per, k - c0);
    if (staged) {
      __syncthreads();
      for (int t = threadIdx.x; t < r * dim; t += 256) cs[t] = C[(size_t)(c0 + t / dim) * ldc + (t % dim)];
      __syncthreads();
    }
    if (valid) {
      for (int c = 0; c < r; ++c) {
        const float* cc = staged ? cs + c * dim : C + (size_t)(c0 + c) * ldc;
        float d;
        if constexpr (D > 0)
          d = point_dist<D, UNR>(x, cc, dim);
        else
          d = point_dist<0, UNR>(pr, cc, dim);
        if (d < bd) {
          bd = d;
          bi = c0 + c;
        }
      }
    }
  }
  if (valid) {
    assign[i] = (uint32_t)bi;
    if (dist) dist[i] = bd;
  }
}

template <bool UNR>
static void launch_assign(const float* P, int ldp, const uint32_t* rows, size_t n, int dim, const float* C, int ldc,
                          size_t k, uint32_t* assign, float* dist, hipStream_t s) {
  const dim3 g((unsigned)((n + 255) / 256)), b(256);
#define PXG_ASSIGN(DD) \
  hipLaunchKernelGGL((km_assign<DD, UNR>), g, b, 0, s, P, ldp, rows, (int)n, dim, C, ldc, (int)k, assign, dist)
  switch (dim) {
    case 1: PXG_ASSIGN(1); break;
    case 2: PXG_ASSIGN(2); break;
    case 4: PXG_ASSIGN(4); break;
    case 8: PXG_ASSIGN(8); break;
    case 16: PXG_ASSIGN(16); break;
    case 32: PXG_ASSIGN(32); break;
    case 64: PXG_ASSIGN(64); break;
    case 96: PXG_ASSIGN(96); break;
    case 128: PXG_ASSIGN(128); break;
    default: PXG_ASSIGN(0); break;
  }
#undef PXG_ASSIGN
  PXG_HIP(hipGetLastError());
}

void nearest_device(const float* P, int ldp, const uint32_t* rows, size_t n, int dim, const float* C, int ldc,
                    size_t k, bool unrolled, uint32_t* assign, float* dist, hipStream_t s) {
  if (n == 0) return;
  if (unrolled)
    launch_assign<true>(P, ldp, rows, n, dim, C, ldc, k, assign, dist, s);
  else
    launch_assign<false>(P, ldp, rows, n, dim, C, ldc, k, assign, dist, s);
}

// ---------------------------------------------------------------------------
// f64 sums in point order
// ---------------------------------------------------------------------------
// Sequential f64 prefix sums of v[0..n) in index order: prefix[i] =
// (((0 + v0) + v1) + ... + vi), total = prefix[n-1]. One wave: all lanes
// stage the next 1024 values through LDS while lane 0 runs the dependent
// chain on the current ones. The running sums are non-decreasing for
// non-negative inputs, so "first index whose cumulative sum reaches target"
// is a binary search over prefix (seq_find_prefix).
__global__ __launch_bounds__(64) void seq_prefix_f64(const float* __restrict__ v, int n, double* __restrict__ prefix,
                                                     double* __restrict__ total) {
  __shared__ float buf[2][1024];
  const int lane = threadIdx.x;
  const int nchunks = (n + 1023) / 1024;
  auto stage = [&](int c, int b) {
    for (int t = lane; t < 1024; t += 64) {
      const int i = c * 1024 + t;
      buf[b][t] = i < n ? v[i] : 0.0f;
    }
  };
  double s = 0.0;
  if (nchunks > 0) stage(0, 0);
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    const int b = c & 1;
    // issue the next chunk's loads before the chain
    float nx[16];
    const bool more = c + 1 < nchunks;
    if (more)
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int i = (c + 1) * 1024 + u * 64 + lane;
        nx[u] = i < n ? v[i] : 0.0f;
      }
    if (lane == 0) {
      const int m = min(1024, n - c * 1024);
      double* pf = prefix + (size_t)c * 1024;
      for (int t = 0; t < m; ++t) {
        s += (double)buf[b][t];
        pf[t] = s;
      }
    }
    if (more)
#pragma unroll
      for (int u = 0; u < 16; ++u) buf[b ^ 1][u * 64 + lane] = nx[u];
    __syncthreads();
  }
  if (lane == 0) *total = s;
}

__global__ void seq_find_prefix(const double* __restrict__ prefix, int n, double target, long long* __restrict__ out) {
  if (threadIdx.x != 0) return;
  // first i with prefix[i] >= target; n - 1 if none (kmeans.rs:171-180)
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (prefix[mid] >= target)
      hi = mid;
    else
      lo = mid + 1;
  }
  *out = lo < n ? lo : n - 1;
}

// Fixed-order tree sums: block b sums v[b*1024 ..) pairwise; partials summed in order.
constexpr int TREE_SEG = 1024;
__global__ __launch_bounds__(256) void tree_partials(const float* __restrict__ v, int n, double* __restrict__ part) {
  __shared__ double sh[256];
  const int b = blockIdx.x, t = threadIdx.x;
  double acc = 0.0;
  for (int j = 0; j < TREE_SEG / 256; ++j) {
    const int i = b * TREE_SEG + j * 256 + t;
    acc += i < n ? (double)v[i] : 0.0;
  }
  sh[t] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (t < o) sh[t] = sh[t] + sh[t + o];
    __syncthreads();
  }
  if (t == 0) part[b] = sh[0];
}

__global__ __launch_bounds__(64) void tree_total(const double* __restrict__ part, int nb, double* __restrict__ out) {
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int b = 0; b < nb; ++b) s += part[b];
    *out = s;
  }
}

__global__ __launch_bounds__(64) void tree_find_cum(const float* __restrict__ v, int n, const double* __restrict__ part,
                                                    int nb, double target, long long* __restrict__ out) {
  if (threadIdx.x != 0) return;
  double s = 0.0;
  int b = 0;
  for (; b < nb; ++b) {
    if (s + part[b] >= target) break;
    s += part[b];
  }
  long long found = n - 1;
  if (b < nb) {
    for (int i = b * TREE_SEG; i < min(n, (b + 1) * TREE_SEG); ++i) {
      s += (double)v[i];
      if (s >= target) {
        found = i;
        break;
      }
    }
  }
  *out = found;
}

struct F64Sum {
  DevBuf<double> part, tot, prefix;
  DevBuf<long long> idx;
  double total(const float* v, size_t n, hipStream_t s) {
    tot.reserve(1);
    if (n <= SEQ_SUM_LIMIT) {
      prefix.reserve(std::max<size_t>(n, 1));
      hipLaunchKernelGGL(seq_prefix_f64, dim3(1), dim3(64), 0, s, v, (int)n, prefix.p, tot.p);
    } else {
      const int nb = (int)((n + TREE_SEG - 1) / TREE_SEG);
      part.reserve(nb);
      hipLaunchKernelGGL(tree_partials, dim3(nb), dim3(256), 0, s, v, (int)n, part.p);
      hipLaunchKernelGGL(tree_total, dim3(1), dim3(64), 0, s, part.p, nb, tot.p);
    }
    PXG_HIP(hipGetLastError());
    double h = 0;
    PXG_HIP(hipMemcpyAsync(&h, tot.p, 8, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    return h;
  }
  // uses the prefix (or partials) of the last total() over the same values
  size_t find(const float* v, size_t n, double target, hipStream_t s) {
    idx.reserve(1);
    if (n <= SEQ_SUM_LIMIT)
      hipLaunchKernelGGL(seq_find_prefix, dim3(1), dim3(64), 0, s, prefix.p, (int)n, target, idx.p);
    else
      hipLaunchKernelGGL(tree_find_cum, dim3(1), dim3(64), 0, s, v, (int)n, part.p,
                         (int)((n + TREE_SEG - 1) / TREE_SEG), target, idx.p);
    PXG_HIP(hipGetLastError());
    long long h = 0;
    PXG_HIP(hipMemcpyAsync(&h, idx.p, 8, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    return (size_t)h;
  }
};

// ---------------------------------------------------------------------------
// k-means++ (kmeans.rs:146-194)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void km_pp_update(const float* __restrict__ P, int ldp, int n, int dim,
                                                    const float* __restrict__ c, float* __restrict__ ns, int init) {
  __shared__ float cs[KM_LDS_FLOATS];
  const bool staged = dim <= KM_LDS_FLOATS;
  if (staged) {
    for (int t = threadIdx.x; t < dim; t += 256) cs[t] = c[t];
    __syncthreads();
  }
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float* cc = staged ? cs : c;
  const float* pr = P + (size_t)i * ldp;
  float sum = 0.0f;
  for (int j = 0; j < dim; ++j) {
    const float d = pr[j] - cc[j];
    sum += d * d;
  }
  if (init || sum < ns[i]) ns[i] = sum;
}

__global__ void copy_row(const float* __restrict__ src, int ld_src, size_t row, int dim, float* __restrict__ dst) {
  for (int j = threadIdx.x; j < dim; j += blockDim.x) dst[j] = src[row * ld_src + j];
}

void kmeans_pp_device(const float* P, size_t n, int dim, int ldp, size_t k, ChaCha8& rng, float* cents,
                      hipStream_t s) {
  DevBuf<float> ns(n);
  F64Sum sums;
  const size_t first = rng.gen_range_usize(n);
  hipLaunchKernelGGL(copy_row, dim3(1), dim3(256), 0, s, P, ldp, first, dim, cents);
  const dim3 g((unsigned)((n + 255) / 256));
  hipLaunchKernelGGL(km_pp_update, g, dim3(256), 0, s, P, ldp, (int)n, dim, cents, ns.p, 1);
  PXG_HIP(hipGetLastError());
  for (size_t chosen = 1; chosen < k; ++chosen) {
    const double total = sums.total(ns.p, n, s);
    if (!std::isfinite(total))
      internal_error("kmeans++", "the sum of squared distances is not finite; coordinates are too large to square");
    size_t picked;
    if (total <= 0.0) {
      picked = rng.gen_range_usize(n);
    } else {
      const double target = rng.gen_range_f64(0.0, total);
      picked = sums.find(ns.p, n, target, s);
    }
    float* c = cents + chosen * dim;
    hipLaunchKernelGGL(copy_row, dim3(1), dim3(256), 0, s, P, ldp, picked, dim, c);
    hipLaunchKernelGGL(km_pp_update, g, dim3(256), 0, s, P, ldp, (int)n, dim, c, ns.p, 0);
    PXG_HIP(hipGetLastError());
  }
  PXG_HIP(hipStreamSynchronize(s));
}

// ---------------------------------------------------------------------------
// update step
// ---------------------------------------------------------------------------
__global__ void km_changed_counts(const uint32_t* __restrict__ a, uint32_t* __restrict__ prev, int n,
                                  uint32_t* __restrict__ counts, int* __restrict__ changed, uint32_t* __restrict__ idx) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t c = a[i];
  if (prev[i] != c) {
    *changed = 1;
    prev[i] = c;
  }
  atomicAdd(&counts[c], 1u);
  idx[i] = (uint32_t)i;
}

// One thread per (cluster, coordinate): f64 sum of the members in point order.
__global__ void km_sums(const float* __restrict__ P, int ldp, int dim, const uint32_t* __restrict__ members,
                        const uint32_t* __restrict__ offsets, const uint32_t* __restrict__ counts, int k,
                        float* __restrict__ newc) {
  const int c = blockIdx.x;
  const int j = blockIdx.y * blockDim.x + threadIdx.x;
  if (c >= k || j >= dim) return;
  const uint32_t cnt = counts[c];
  if (cnt == 0) return;
  const uint32_t off = offsets[c];
  double sum = 0.0;
  for (uint32_t m = 0; m < cnt; ++m) sum += (double)P[(size_t)members[off + m] * ldp + j];
  const double inv = 1.0 / (double)cnt;
  newc[(size_t)c * dim + j] = (float)(sum * inv);
}

// farthest_point (kmeans.rs:215-226): first point with the largest distance
// (strict >, starting from -1.0).
__global__ __launch_bounds__(1024) void km_farthest(const float* __restrict__ dist, int n, long long* __restrict__ out) {
  __shared__ float sd[1024];
  __shared__ int si[1024];
  float bd = -1.0f;
  int bi = 0;
  const int t = threadIdx.x;
  // contiguous ranges keep the "first" rule with a per-thread strict >
  const int per = (n + 1023) / 1024;
  for (int i = t * per; i < min(n, (t + 1) * per); ++i) {
    if (dist[i] > bd) {
      bd = dist[i];
      bi = i;
    }
  }
  sd[t] = bd;
  si[t] = bi;
  __syncthreads();
  if (t == 0) {
    float b = -1.0f;
    int best = 0;
    for (int u = 0; u < 1024; ++u)
      if (sd[u] > b) {
        b = sd[u];
        best = si[u];
      }
    *out = best;
  }
}

// Optional phase timings on stderr (PXG_TRAIN_VERBOSE=1), for tuning.
static bool train_verbose() {
  static const bool v = [] {
    const char* e = std::getenv("PXG_TRAIN_VERBOSE");
    return e && *e && *e != '0';
  }();
  return v;
}
static double now_s() {
  return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

KmeansOut kmeans_device(const float* P, size_t n, int dim, int ldp, size_t k_req, size_t max_iter, ChaCha8* rng,
                        const float* init, DevBuf<float>& cents, DevBuf<uint32_t>* assign_out, hipStream_t s) {
  KmeansOut out;
  if (dim == 0) n = 0;
  const size_t k = std::max<size_t>(std::min(k_req, n), 1);
  out.k = k;
  cents.reserve(k * dim);
  if (n == 0) {
    PXG_HIP(hipMemsetAsync(cents.p, 0, k * dim * 4, s));
    PXG_HIP(hipStreamSynchronize(s));
    return out;
  }
  const double t_start = now_s();
  if (init)
    PXG_HIP(hipMemcpyAsync(cents.p, init, k * dim * 4, hipMemcpyDeviceToDevice, s));
  else
    kmeans_pp_device(P, n, dim, ldp, k, *rng, cents.p, s);
  const double t_seeded = now_s();
  size_t empties = 0;

  DevBuf<uint32_t> assign(n), prev(n), counts(k), offsets(k), idx(n), keys_sorted(n), members(n);
  DevBuf<float> dist(n), newc(k * dim), work(k * dim);
  DevBuf<int> changed(1);
  DevBuf<long long> far(1);
  PXG_HIP(hipMemsetAsync(prev.p, 0, n * 4, s));
  F64Sum sums;
  size_t tmp_bytes = 0;
  PXG_HIP(hipcub::DeviceRadixSort::SortPairs(nullptr, tmp_bytes, assign.p, keys_sorted.p, idx.p, members.p, (int)n, 0, 32, s));
  DevBuf<unsigned char> tmp(tmp_bytes + 16);
  int bits = 1;
  while ((1ull << bits) < k) ++bits;
  std::vector<uint32_t> h_counts(k), h_off(k);
  const dim3 gn((unsigned)((n + 255) / 256));
  for (size_t it = 0; it < max_iter; ++it) {
    out.iterations = it + 1;
    nearest_device(P, ldp, nullptr, n, dim, cents.p, dim, k, false, assign.p, dist.p, s);
    out.inertia = sums.total(dist.p, n, s);
    PXG_HIP(hipMemsetAsync(changed.p, 0, 4, s));
    PXG_HIP(hipMemsetAsync(counts.p, 0, k * 4, s));
    hipLaunchKernelGGL(km_changed_counts, gn, dim3(256), 0, s, assign.p, prev.p, (int)n, counts.p, changed.p, idx.p);
    PXG_HIP(hipGetLastError());
    int h_changed = 0;
    PXG_HIP(hipMemcpyAsync(&h_changed, changed.p, 4, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipMemcpyAsync(h_counts.data(), counts.p, k * 4, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    if (!h_changed && it > 0) break;  // kmeans.rs:99-102
    // group points by cluster, point order kept (stable radix sort)
    PXG_HIP(hipcub::DeviceRadixSort::SortPairs(tmp.p, tmp_bytes, assign.p, keys_sorted.p, idx.p, members.p, (int)n,
                                               0, bits, s));
    uint32_t acc = 0;
    for (size_t c = 0; c < k; ++c) {
      h_off[c] = acc;
      acc += h_counts[c];
    }
    PXG_HIP(hipMemcpyAsync(offsets.p, h_off.data(), k * 4, hipMemcpyHostToDevice, s));
    PXG_HIP(hipMemcpyAsync(newc.p, cents.p, k * dim * 4, hipMemcpyDeviceToDevice, s));
    hipLaunchKernelGGL(km_sums, dim3((unsigned)k, (unsigned)((dim + 63) / 64)), dim3(64), 0, s, P, ldp, dim,
                       members.p, offsets.p, counts.p, (int)k, newc.p);
    PXG_HIP(hipGetLastError());
    // empty clusters, ascending, against the partially updated array
    for (size_t c = 0; c < k; ++c) {
      if (h_counts[c] != 0) continue;
      ++empties;
      PXG_HIP(hipMemcpyAsync(work.p, newc.p, c * dim * 4, hipMemcpyDeviceToDevice, s));
      PXG_HIP(hipMemcpyAsync(work.p + c * dim, cents.p + c * dim, (k - c) * dim * 4, hipMemcpyDeviceToDevice, s));
      nearest_device(P, ldp, nullptr, n, dim, work.p, dim, k, false, keys_sorted.p, dist.p, s);
      hipLaunchKernelGGL(km_farthest, dim3(1), dim3(1024), 0, s, dist.p, (int)n, far.p);
      long long victim = 0;
      PXG_HIP(hipMemcpyAsync(&victim, far.p, 8, hipMemcpyDeviceToHost, s));
      PXG_HIP(hipStreamSynchronize(s));
      hipLaunchKernelGGL(copy_row, dim3(1), dim3(256), 0, s, P, ldp, (size_t)victim, dim, newc.p + c * dim);
    }
    PXG_HIP(hipMemcpyAsync(cents.p, newc.p, k * dim * 4, hipMemcpyDeviceToDevice, s));
  }
  if (assign_out) {
    assign_out->reserve(n);
    PXG_HIP(hipMemcpyAsync(assign_out->p, prev.p, n * 4, hipMemcpyDeviceToDevice, s));
  }
  PXG_HIP(hipStreamSynchronize(s));
  if (train_verbose())
    std::fprintf(stderr, "[pxg kmeans] n=%zu dim=%d k=%zu: seeding %.3fs, lloyd %zu it %.3fs, %zu empty reseeds\n", n,
                 dim, k, t_seeded - t_start, out.iterations, now_s() - t_seeded, empties);
  return out;
}

// ---------------------------------------------------------------------------
// product quantizer
// ---------------------------------------------------------------------------
__global__ void gather_cols(const float* __restrict__ R, int ldr, int n, int off, int w, float* __restrict__ out) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (size_t)n * w) return;
  const size_t i = t / w, j = t % w;
  out[t] = R[i * ldr + off + j];
}

__global__ void pad_book(float* __restrict__ book, int produced, int w) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  const int r = produced + t / w;
  if (r >= 256 || t >= (256 - produced) * w) return;
  book[r * w + (t % w)] = book[(produced - 1) * w + (t % w)];
}

void pq_train_device(const float* R, size_t n, int dim, int ldr, const PqLayout& L, size_t max_iter, uint64_t seed,
                     float* d_books, double* inertia, size_t* iterations, hipStream_t s) {
  ChaCha8 rng(seed);  // one generator advanced across subspaces (product.rs:244-247)
  double in = 0.0;
  size_t its = 0;
  DevBuf<float> proj(std::max<size_t>(n * (size_t)(L.width.empty() ? 1 : *std::max_element(L.width.begin(), L.width.end())), 1));
  DevBuf<float> cents;
  for (int sidx = 0; sidx < L.M; ++sidx) {
    const int w = L.width[sidx], off = L.off[sidx];
    const size_t tot = n * (size_t)w;
    if (tot) hipLaunchKernelGGL(gather_cols, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, R, ldr, (int)n, off, w, proj.p);
    PXG_HIP(hipGetLastError());
    KmeansOut r = kmeans_device(proj.p, n, w, w, 256, max_iter, &rng, nullptr, cents, nullptr, s);
    in += r.inertia;
    its += r.iterations;
    float* book = d_books + L.book_off[sidx];
    PXG_HIP(hipMemcpyAsync(book, cents.p, r.k * w * 4, hipMemcpyDeviceToDevice, s));
    if (r.k < 256) {
      const int t = (int)(256 - r.k) * w;
      hipLaunchKernelGGL(pad_book, dim3((t + 255) / 256), dim3(256), 0, s, book, (int)r.k, w);
      PXG_HIP(hipGetLastError());
    }
  }
  PXG_HIP(hipStreamSynchronize(s));
  *inertia = in;
  *iterations = its;
}

// One thread per vector; the subspace's 256-row codebook staged in LDS.
__global__ __launch_bounds__(256) void pq_encode_kernel(const float* __restrict__ P, int ldp,
                                                        const uint32_t* __restrict__ rows, int n,
                                                        const float* __restrict__ C, int ldc,
                                                        const uint32_t* __restrict__ assign,
                                                        const float* __restrict__ books, int off, int w, int book_off,
                                                        int s_idx, int M, uint8_t* __restrict__ out) {
  __shared__ float bs[KM_LDS_FLOATS];
  const bool staged = 256 * w <= KM_LDS_FLOATS;
  if (staged) {
    for (int t = threadIdx.x; t < 256 * w; t += 256) bs[t] = books[book_off + t];
    __syncthreads();
  }
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const size_t row = rows ? rows[i] : (uint32_t)i;
  const float* pr = P + row * ldp + off;
  const float* cr = C ? C + (size_t)assign[i] * ldc + off : nullptr;
  const float* b = staged ? bs : books + book_off;
  // nearest_centroid (product.rs:529-547): sequential sum over the residual slice
  float r[16];
  const bool small = w <= 16;
  if (small)
    for (int j = 0; j < w; ++j) r[j] = cr ? pr[j] - cr[j] : pr[j];
  float bd = INFINITY;
  int bi = 0;
  for (int c = 0; c < 256; ++c) {
    float sum = 0.0f;
    for (int j = 0; j < w; ++j) {
      const float rj = small ? r[j] : (cr ? pr[j] - cr[j] : pr[j]);
      const float d = rj - b[c * w + j];
      sum += d * d;
    }
    if (sum < bd) {
      bd = sum;
      bi = c;
    }
  }
  out[row * M + s_idx] = (uint8_t)bi;
}

void pq_encode_device(const float* P, int ldp, const uint32_t* rows, size_t n, int dim, const float* C, int ldc,
                      const uint32_t* assign, const float* books, const PqLayout& L, uint8_t* out, hipStream_t s) {
  (void)dim;
  if (n == 0) return;
  for (int sidx = 0; sidx < L.M; ++sidx) {
    hipLaunchKernelGGL(pq_encode_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, P, ldp, rows, (int)n, C,
                       ldc, assign, books, L.off[sidx], L.width[sidx], L.book_off[sidx], sidx, L.M, out);
    PXG_HIP(hipGetLastError());
  }
}

}  // namespace pxg

// ===========================================================================
// C ABI: k-means and the product quantizer
// ===========================================================================
extern "C" {

static void kmeans_common(const float* points, uint64_t n, uint32_t dim, uint64_t k, uint64_t max_iter, uint64_t seed,
                          const float* init, float* centroids_out, uint32_t* assign_out, double* inertia,
                          uint64_t* iterations, uint64_t* k_out, bool device_points) {
  hipStream_t s;
  PXG_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  struct SG {
    hipStream_t s;
    ~SG() { (void)hipStreamDestroy(s); }
  } sg{s};
  const float* P = points;
  pxg::DevBuf<float> dP;
  if (!device_points && n) {
    dP.alloc(n * dim);
    PXG_HIP(hipMemcpyAsync(dP.p, points, n * dim * 4, hipMemcpyHostToDevice, s));
    P = dP.p;
  }
  pxg::DevBuf<float> dinit;
  const size_t kk = std::max<size_t>(std::min<size_t>(k, n), 1);
  if (init) {
    dinit.alloc(kk * dim);
    PXG_HIP(hipMemcpyAsync(dinit.p, init, kk * dim * 4, device_points ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, s));
  }
  pxg::ChaCha8 rng(seed);
  pxg::DevBuf<float> cents;
  pxg::DevBuf<uint32_t> assign;
  pxg::KmeansOut r = pxg::kmeans_device(P, n, (int)dim, (int)dim, k, max_iter, &rng, init ? dinit.p : nullptr, cents,
                                        assign_out ? &assign : nullptr, s);
  const hipMemcpyKind d2x = device_points ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost;
  PXG_HIP(hipMemcpyAsync(centroids_out, cents.p, r.k * dim * 4, d2x, s));
  if (assign_out && n) PXG_HIP(hipMemcpyAsync(assign_out, assign.p, n * 4, d2x, s));
  PXG_HIP(hipStreamSynchronize(s));
  if (inertia) *inertia = r.inertia;
  if (iterations) *iterations = r.iterations;
  if (k_out) *k_out = r.k;
}

int pxg_kmeans(const float* points, uint64_t n, uint32_t dim, uint64_t k, uint64_t max_iterations, uint64_t seed,
               float* centroids_out, double* inertia, uint64_t* iterations, uint64_t* k_out) {
  return pxg::guard([&] {
    kmeans_common(points, n, dim, k, max_iterations, seed, nullptr, centroids_out, nullptr, inertia, iterations,
                  k_out, false);
  });
}

int pxg_kmeans_lloyd(const float* points, uint64_t n, uint32_t dim, uint64_t k, uint64_t max_iterations,
                     const float* init, float* centroids_out, uint32_t* assign_out, double* inertia,
                     uint64_t* iterations) {
  return pxg::guard([&] {
    if (k == 0 || k > n) pxg::config_error("k", k, "initial centroids must number between 1 and n");
    kmeans_common(points, n, dim, k, max_iterations, 0, init, centroids_out, assign_out, inertia, iterations, nullptr,
                  false);
  });
}

int pxg_kmeans_device(const float* d_points, uint64_t n, uint32_t dim, uint64_t k, uint64_t max_iterations,
                      uint64_t seed, const float* d_init, float* d_centroids_out, uint32_t* d_assign_out,
                      double* inertia, uint64_t* iterations) {
  return pxg::guard([&] {
    kmeans_common(d_points, n, dim, k, max_iterations, seed, d_init, d_centroids_out, d_assign_out, inertia,
                  iterations, nullptr, true);
  });
}

int pxg_kmeans_pp(const float* points, uint64_t n, uint32_t dim, uint64_t k, uint64_t seed, float* centroids_out) {
  return pxg::guard([&] {
    if (n == 0 || k == 0 || k > n) pxg::config_error("k", k, "must be between 1 and n");
    hipStream_t s;
    PXG_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    pxg::DevBuf<float> dP(n * dim), c(k * dim);
    PXG_HIP(hipMemcpyAsync(dP.p, points, n * dim * 4, hipMemcpyHostToDevice, s));
    pxg::ChaCha8 rng(seed);
    pxg::kmeans_pp_device(dP.p, n, (int)dim, (int)dim, k, rng, c.p, s);
    PXG_HIP(hipMemcpyAsync(centroids_out, c.p, k * dim * 4, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    (void)hipStreamDestroy(s);
  });
}

int pxg_kmeans_assign(const float* points, uint64_t n, uint32_t dim, const float* centroids, uint64_t k,
                      uint32_t* assign_out, float* dist_out) {
  return pxg::guard([&] {
    if (n == 0) return;
    hipStream_t s;
    PXG_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    pxg::DevBuf<float> dP(n * dim), dC(k * dim), dd(n);
    pxg::DevBuf<uint32_t> da(n);
    PXG_HIP(hipMemcpyAsync(dP.p, points, n * dim * 4, hipMemcpyHostToDevice, s));
    PXG_HIP(hipMemcpyAsync(dC.p, centroids, k * dim * 4, hipMemcpyHostToDevice, s));
    pxg::nearest_device(dP.p, (int)dim, nullptr, n, (int)dim, dC.p, (int)dim, k, false, da.p, dd.p, s);
    PXG_HIP(hipMemcpyAsync(assign_out, da.p, n * 4, hipMemcpyDeviceToHost, s));
    if (dist_out) PXG_HIP(hipMemcpyAsync(dist_out, dd.p, n * 4, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    (void)hipStreamDestroy(s);
  });
}

int pxg_pq_train_device(const float* d_training, uint64_t n, uint32_t dim, uint64_t subspaces,
                        uint64_t max_iterations, uint64_t seed, float* d_codebooks_out, double* inertia,
                        uint64_t* iterations) {
  return pxg::guard([&] {
    // ProductQuantizer::train validation (product.rs:200-223); the values
    // are not scanned for non-finite entries here (device data)
    if (subspaces == 0 || subspaces > dim) pxg::config_error("subspaces", subspaces, "must be between 1 and the space dimension");
    if (max_iterations == 0) pxg::config_error("max_iterations", max_iterations, "must be at least 1");
    if (n == 0) pxg::config_error("training", 0, "must be a non-empty multiple of the space dimension");
    pxg::PqLayout L;
    L.build((int)dim, (int)subspaces);
    hipStream_t s;
    PXG_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    struct SG {
      hipStream_t s;
      ~SG() { (void)hipStreamDestroy(s); }
    } sg{s};
    size_t its = 0;
    pxg::pq_train_device(d_training, n, (int)dim, (int)dim, L, max_iterations, seed, d_codebooks_out, inertia, &its,
                         s);
    PXG_HIP(hipStreamSynchronize(s));
    if (iterations) *iterations = its;
  });
}

int pxg_pq_train(const float* training, uint64_t n, uint32_t dim, uint64_t subspaces, uint64_t max_iterations,
                 uint64_t seed, float* codebooks_out, double* inertia, uint64_t* iterations) {
  return pxg::guard([&] {
    // ProductQuantizer::train validation (product.rs:200-223)
    if (subspaces == 0 || subspaces > dim) pxg::config_error("subspaces", subspaces, "must be between 1 and the space dimension");
    if (max_iterations == 0) pxg::config_error("max_iterations", max_iterations, "must be at least 1");
    if (n == 0) pxg::config_error("training", 0, "must be a non-empty multiple of the space dimension");
    for (uint64_t i = 0; i < n * dim; ++i)
      if (!std::isfinite(training[i]))
        pxg::raise(PXG_ERR_NON_FINITE, "vector component " + std::to_string(i % dim) + " is not finite", i % dim,
                   i / dim, training[i]);
    pxg::PqLayout L;
    L.build((int)dim, (int)subspaces);
    hipStream_t s;
    PXG_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    pxg::DevBuf<float> R(n * dim), B(L.book_floats());
    PXG_HIP(hipMemcpyAsync(R.p, training, n * dim * 4, hipMemcpyHostToDevice, s));
    size_t its = 0;
    pxg::pq_train_device(R.p, n, (int)dim, (int)dim, L, max_iterations, seed, B.p, inertia, &its, s);
    PXG_HIP(hipMemcpyAsync(codebooks_out, B.p, L.book_floats() * 4, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    (void)hipStreamDestroy(s);
    if (iterations) *iterations = its;
  });
}

int pxg_pq_encode(const float* codebooks, uint32_t dim, uint64_t subspaces, const float* vectors, uint64_t n,
                  uint8_t* codes_out) {
  return pxg::guard([&] {
    if (subspaces == 0 || subspaces > dim) pxg::config_error("subspaces", subspaces, "must be between 1 and the space dimension");
    if (n == 0) return;
    pxg::PqLayout L;
    L.build((int)dim, (int)subspaces);
    hipStream_t s;
    PXG_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    pxg::DevBuf<float> V(n * dim), B(L.book_floats());
    pxg::DevBuf<uint8_t> O(n * subspaces);
    PXG_HIP(hipMemcpyAsync(V.p, vectors, n * dim * 4, hipMemcpyHostToDevice, s));
    PXG_HIP(hipMemcpyAsync(B.p, codebooks, L.book_floats() * 4, hipMemcpyHostToDevice, s));
    pxg::pq_encode_device(V.p, (int)dim, nullptr, n, (int)dim, nullptr, 0, nullptr, B.p, L, O.p, s);
    PXG_HIP(hipMemcpyAsync(codes_out, O.p, n * subspaces, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    (void)hipStreamDestroy(s);
  });
}

}  // extern "C"
