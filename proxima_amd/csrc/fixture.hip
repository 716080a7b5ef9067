// The benchmark fixture generator on MI355X: fixture::generate
// (crates/proxima-cli/src/fixture.rs:71-123).
//
// ChaCha8Rng::seed_from_u64(seed) is a counter-mode stream: word w of its
// output is word w % 16 of the block with counter w / 16, and every
// gen::<f32>() draw consumes exactly one word, so draw t of the generator is
// known without running the draws before it. gaussian() takes two draws, so
// Gaussian number g uses words 2g and 2g+1. The reference draws, in order:
// clusters*dim centre Gaussians, count*dim point Gaussians and queries*dim
// query Gaussians. One thread here produces one 64-byte block, that is, 8
// consecutive Gaussians.
//
// gaussian(): u1 = max(gen_f32, f32::MIN_POSITIVE), u2 = gen_f32,
// sqrt(-2 ln u1) * cos(TAU * u2), every step in f32 as the reference writes
// it. ln and cos are the platform's f32 libm functions in the reference; here
// they are evaluated in f64 and rounded to f32 (correctly rounded results),
// so a value can differ from another libm's in the last bit of ln or cos.
#include <cmath>

#include "common.hpp"
#include "rng.hpp"

namespace pxg {

__device__ inline float fx_u01(uint32_t w) { return (float)(w >> 8) * (1.0f / 16777216.0f); }

__device__ inline float fx_gaussian(uint32_t w1, uint32_t w2) {
  const float u1 = fmaxf(fx_u01(w1), 1.17549435e-38f);
  const float u2 = fx_u01(w2);
  const float l = (float)log((double)u1);
  const float a = 6.28318530717958647692f * u2;
  const float c = (float)cos((double)a);
  return sqrtf(-2.0f * l) * c;
}

// This thread's block of the stream: Gaussians first .. first+7 into v.
// False when the block starts at or past g1.
__device__ inline bool fx_values(const uint32_t* key, uint64_t g0, uint64_t g1, uint64_t& first, float (&v)[8]) {
  const uint64_t blk = (g0 / 8) + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  first = blk * 8;
  if (first >= g1) return false;
  uint32_t k[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) k[i] = key[i];
  uint32_t w[16];
  ChaCha8::block(k, blk, w);
#pragma unroll
  for (int u = 0; u < 8; ++u) v[u] = fx_gaussian(w[2 * u], w[2 * u + 1]);
  return true;
}

__global__ void fx_centres(const uint32_t* __restrict__ key, uint64_t total, float* __restrict__ centres) {
  uint64_t first;
  float v[8];
  if (!fx_values(key, 0, total, first, v)) return;
#pragma unroll
  for (int u = 0; u < 8; ++u)
    if (first + u < total) centres[first + u] = v[u] * 4.0f;
}

// Point t = i * dim + d (Gaussian base + t) is centre (i % clusters) plus the
// Gaussian. A thread's Gaussians are consecutive, so (i, d, i % clusters) is
// divided out once for its first one and then stepped.
__global__ void fx_points(const uint32_t* __restrict__ key, uint64_t base, uint64_t total, uint32_t dim,
                          uint64_t clusters, const float* __restrict__ centres, float* __restrict__ vectors) {
  uint64_t first;
  float v[8];
  if (!fx_values(key, base, base + total, first, v)) return;
  const uint64_t t0 = (first > base ? first : base) - base, i0 = t0 / dim;
  uint32_t d = (uint32_t)(t0 - i0 * dim);
  uint64_t ci = i0 % clusters;
  const float* crow = centres + ci * dim;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const uint64_t g = first + u;
    if (g >= base && g < base + total) {
      vectors[g - base] = crow[d] + v[u];
      if (++d == dim) {
        d = 0;
        if (++ci == clusters) ci = 0;
        crow = centres + ci * dim;
      }
    }
  }
}

// Query t = q * dim + d is corpus point (q * stride) % count plus a quarter
// of the Gaussian; the source row changes only when q does.
__global__ void fx_queries(const uint32_t* __restrict__ key, uint64_t base, uint64_t total, uint32_t dim,
                           uint64_t count, uint64_t stride, const float* __restrict__ vectors,
                           float* __restrict__ queries) {
  uint64_t first;
  float v[8];
  if (!fx_values(key, base, base + total, first, v)) return;
  const uint64_t t0 = (first > base ? first : base) - base;
  uint64_t q = t0 / dim;
  uint32_t d = (uint32_t)(t0 - q * dim);
  const float* srow = vectors + ((q * stride) % count) * dim;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const uint64_t g = first + u;
    if (g >= base && g < base + total) {
      queries[g - base] = srow[d] + v[u] * 0.25f;
      if (++d == dim) {
        d = 0;
        ++q;
        srow = vectors + ((q * stride) % count) * dim;
      }
    }
  }
}

static void launch_blocks(uint64_t g0, uint64_t g1, dim3& grid) {
  const uint64_t blocks = (g1 + 7) / 8 - g0 / 8;
  grid = dim3((unsigned)((blocks + 255) / 256));
}

void fixture_generate_device(uint64_t count, uint32_t dim, uint64_t clusters, uint64_t queries, uint64_t seed,
                             float* d_vectors, float* d_queries, hipStream_t s) {
  const ChaCha8 rng(seed);
  DevBuf<uint32_t> key(8);
  const uint64_t cd = clusters * dim, nd = count * dim, qd = queries * dim;
  DevBuf<float> centres(std::max<uint64_t>(cd, 1));
  PXG_HIP(hipMemcpyAsync(key.p, rng.key, 32, hipMemcpyHostToDevice, s));
  dim3 g;
  if (cd) {
    launch_blocks(0, cd, g);
    hipLaunchKernelGGL(fx_centres, g, dim3(256), 0, s, key.p, cd, centres.p);
  }
  if (nd) {
    launch_blocks(cd, cd + nd, g);
    hipLaunchKernelGGL(fx_points, g, dim3(256), 0, s, key.p, cd, nd, dim, clusters, centres.p, d_vectors);
  }
  if (qd) {
    const uint64_t stride = std::max<uint64_t>(count / std::max<uint64_t>(queries, 1), 1);
    launch_blocks(cd + nd, cd + nd + qd, g);
    hipLaunchKernelGGL(fx_queries, g, dim3(256), 0, s, key.p, cd + nd, qd, dim, count, stride, d_vectors,
                       d_queries);
  }
  PXG_HIP(hipGetLastError());
  PXG_HIP(hipStreamSynchronize(s));
}

// ---------------------------------------------------------------------------
// Synthetic inputs of the benchmark configurations (no reference
// counterpart; the reference's own generator is fixture::generate above).
// The same counter-mode ChaCha8Rng::seed_from_u64(seed) stream and the same
// Box-Muller step, in this order of Gaussian slots (slot g = words 2g, 2g+1):
//   [0, C*dim)                  centres, centre_scale * gaussian
//   [gB, gB + ceil(items / 2))  cluster choices, when drawn: item t (points
//                               first, then queries) takes word 2 gB + t as
//                               c = (word * C) >> 32
//   [gC, gC + count*dim)        points:  centre[cluster(i)] + sigma * gaussian
//   [gD, gD + queries*dim)      queries: centre[cluster(q)] + sigma * gaussian
// with cluster(i) = i % C (points) and q % C (queries) when not drawn.
// ---------------------------------------------------------------------------
__global__ void mx_centres(const uint32_t* __restrict__ key, uint64_t total, float scale, float* __restrict__ centres) {
  uint64_t first;
  float v[8];
  if (!fx_values(key, 0, total, first, v)) return;
#pragma unroll
  for (int u = 0; u < 8; ++u)
    if (first + u < total) centres[first + u] = v[u] * scale;
}

// cluster choices of `items` items from word 2 gB on: one 16-word block per thread
__global__ void mx_choices(const uint32_t* __restrict__ key, uint64_t w0, uint64_t items, uint64_t clusters,
                           uint32_t* __restrict__ cl) {
  const uint64_t blk = w0 / 16 + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (blk * 16 >= w0 + items) return;
  uint32_t k[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) k[i] = key[i];
  uint32_t w[16];
  ChaCha8::block(k, blk, w);
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const uint64_t pos = blk * 16 + u;
    if (pos >= w0 && pos < w0 + items) cl[pos - w0] = (uint32_t)(((uint64_t)w[u] * clusters) >> 32);
  }
}

// Item t = i * dim + d of a region at Gaussian slot `base`: centre row of
// cluster(i) plus sigma times the Gaussian; cl (cluster per item) or i % C.
__global__ void mx_rows(const uint32_t* __restrict__ key, uint64_t base, uint64_t total, uint32_t dim,
                        uint64_t clusters, const uint32_t* __restrict__ cl, float sigma,
                        const float* __restrict__ centres, float* __restrict__ out) {
  uint64_t first;
  float v[8];
  if (!fx_values(key, base, base + total, first, v)) return;
  const uint64_t t0 = (first > base ? first : base) - base;
  uint64_t i = t0 / dim;
  uint32_t d = (uint32_t)(t0 - i * dim);
  const float* crow = centres + (cl ? (uint64_t)cl[i] : i % clusters) * dim;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const uint64_t g = first + u;
    if (g >= base && g < base + total) {
      out[g - base] = crow[d] + sigma * v[u];
      if (++d == dim) {
        d = 0;
        ++i;
        if (g + 1 < base + total) crow = centres + (cl ? (uint64_t)cl[i] : i % clusters) * dim;
      }
    }
  }
}

// value t = lo + (hi - lo) * gen::<f32>() of word t: one 16-word block per thread
__global__ void mx_uniform(const uint32_t* __restrict__ key, uint64_t total, float lo, float hi,
                           float* __restrict__ out) {
  const uint64_t blk = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (blk * 16 >= total) return;
  uint32_t k[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) k[i] = key[i];
  uint32_t w[16];
  ChaCha8::block(k, blk, w);
  const float span = hi - lo;
#pragma unroll
  for (int u = 0; u < 16; ++u)
    if (blk * 16 + u < total) out[blk * 16 + u] = lo + span * fx_u01(w[u]);
}

void mixture_generate_device(uint64_t count, uint32_t dim, uint64_t clusters, float centre_scale, float sigma,
                             uint64_t queries, int drawn, uint64_t seed, float* d_vectors, float* d_queries,
                             hipStream_t s) {
  const ChaCha8 rng(seed);
  DevBuf<uint32_t> key(8);
  const uint64_t cd = clusters * dim, nd = count * dim, qd = queries * dim, items = count + queries;
  DevBuf<float> centres(std::max<uint64_t>(cd, 1));
  DevBuf<uint32_t> cl(drawn ? std::max<uint64_t>(items, 1) : 0);
  PXG_HIP(hipMemcpyAsync(key.p, rng.key, 32, hipMemcpyHostToDevice, s));
  const uint64_t gB = cd, gC = gB + (drawn ? (items + 1) / 2 : 0), gD = gC + nd;
  dim3 g;
  if (cd) {
    launch_blocks(0, cd, g);
    hipLaunchKernelGGL(mx_centres, g, dim3(256), 0, s, key.p, cd, centre_scale, centres.p);
  }
  if (drawn && items) {
    const uint64_t blocks = (2 * gB + items + 15) / 16 - (2 * gB) / 16;
    hipLaunchKernelGGL(mx_choices, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, s, key.p, 2 * gB, items,
                       clusters, cl.p);
  }
  if (nd) {
    launch_blocks(gC, gC + nd, g);
    hipLaunchKernelGGL(mx_rows, g, dim3(256), 0, s, key.p, gC, nd, dim, clusters, drawn ? cl.p : nullptr, sigma,
                       centres.p, d_vectors);
  }
  if (qd) {
    launch_blocks(gD, gD + qd, g);
    hipLaunchKernelGGL(mx_rows, g, dim3(256), 0, s, key.p, gD, qd, dim, clusters,
                       drawn ? cl.p + count : nullptr, sigma, centres.p, d_queries);
  }
  PXG_HIP(hipGetLastError());
  PXG_HIP(hipStreamSynchronize(s));
}

void uniform_generate_device(uint64_t count, uint32_t dim, float lo, float hi, uint64_t seed, float* d_out,
                             hipStream_t s) {
  const ChaCha8 rng(seed);
  DevBuf<uint32_t> key(8);
  const uint64_t total = count * dim;
  PXG_HIP(hipMemcpyAsync(key.p, rng.key, 32, hipMemcpyHostToDevice, s));
  if (total) {
    const uint64_t blocks = (total + 15) / 16;
    hipLaunchKernelGGL(mx_uniform, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, s, key.p, total, lo, hi,
                       d_out);
  }
  PXG_HIP(hipGetLastError());
  PXG_HIP(hipStreamSynchronize(s));
}

}  // namespace pxg

extern "C" {

static void fixture_check(uint64_t count, uint64_t clusters, uint64_t queries) {
  if (count > 0 && clusters == 0) pxg::config_error("clusters", 0, "points are assigned to cluster index % clusters");
  if (queries > 0 && count == 0) pxg::config_error("count", 0, "queries are drawn from corpus points");
}

struct FxStream {
  hipStream_t s = nullptr;
  FxStream() { PXG_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking)); }
  ~FxStream() {
    if (s) (void)hipStreamDestroy(s);
  }
};

int pxg_fixture_generate_device(uint64_t count, uint32_t dim, uint64_t clusters, uint64_t queries, uint64_t seed,
                                float* d_vectors, float* d_queries) {
  return pxg::guard([&] {
    fixture_check(count, clusters, queries);
    FxStream st;
    pxg::fixture_generate_device(count, dim, clusters, queries, seed, d_vectors, d_queries, st.s);
  });
}

int pxg_mixture_generate_device(uint64_t count, uint32_t dim, uint64_t clusters, float centre_scale, float sigma,
                                uint64_t queries, int drawn_clusters, uint64_t seed, float* d_vectors,
                                float* d_queries) {
  return pxg::guard([&] {
    if (count + queries > 0 && clusters == 0)
      pxg::config_error("clusters", 0, "every point and query belongs to a cluster");
    if (clusters > 0xFFFFFFFFull) pxg::config_error("clusters", clusters, "at most 2^32 - 1 clusters");
    if (!std::isfinite(centre_scale) || !std::isfinite(sigma))
      pxg::config_error("sigma", 0, "centre_scale and sigma must be finite");
    FxStream st;
    pxg::mixture_generate_device(count, dim, clusters, centre_scale, sigma, queries, drawn_clusters ? 1 : 0, seed,
                                 d_vectors, d_queries, st.s);
  });
}

int pxg_uniform_generate_device(uint64_t count, uint32_t dim, float lo, float hi, uint64_t seed, float* d_out) {
  return pxg::guard([&] {
    if (!std::isfinite(lo) || !std::isfinite(hi) || !(lo < hi)) pxg::config_error("hi", 0, "need finite lo < hi");
    FxStream st;
    pxg::uniform_generate_device(count, dim, lo, hi, seed, d_out, st.s);
  });
}

int pxg_fixture_generate(uint64_t count, uint32_t dim, uint64_t clusters, uint64_t queries, uint64_t seed,
                         float* vectors, float* query_vectors) {
  return pxg::guard([&] {
    fixture_check(count, clusters, queries);
    FxStream st;
    pxg::DevBuf<float> v(std::max<uint64_t>(count * dim, 1)), q(std::max<uint64_t>(queries * dim, 1));
    pxg::fixture_generate_device(count, dim, clusters, queries, seed, v.p, q.p, st.s);
    if (count * dim) PXG_HIP(hipMemcpyAsync(vectors, v.p, count * dim * 4, hipMemcpyDeviceToHost, st.s));
    if (queries * dim) PXG_HIP(hipMemcpyAsync(query_vectors, q.p, queries * dim * 4, hipMemcpyDeviceToHost, st.s));
    PXG_HIP(hipStreamSynchronize(st.s));
  });
}

}  // extern "C"
