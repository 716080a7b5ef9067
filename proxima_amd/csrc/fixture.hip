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

// Gaussians g in [g0, g1) of the stream, written through `emit(g, value)`.
template <class Emit>
__device__ inline void fx_block(const uint32_t* key, uint64_t g0, uint64_t g1, Emit emit) {
  const uint64_t blk = (g0 / 8) + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t first = blk * 8;
  if (first >= g1) return;
  uint32_t k[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) k[i] = key[i];
  uint32_t w[16];
  ChaCha8::block(k, blk, w);
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const uint64_t g = first + u;
    if (g >= g0 && g < g1) emit(g, fx_gaussian(w[2 * u], w[2 * u + 1]));
  }
}

__global__ void fx_centres(const uint32_t* __restrict__ key, uint64_t total, float* __restrict__ centres) {
  fx_block(key, 0, total, [&](uint64_t g, float v) { centres[g] = v * 4.0f; });
}

__global__ void fx_points(const uint32_t* __restrict__ key, uint64_t base, uint64_t total, uint32_t dim,
                          uint64_t clusters, const float* __restrict__ centres, float* __restrict__ vectors) {
  fx_block(key, base, base + total, [&](uint64_t g, float v) {
    const uint64_t t = g - base, i = t / dim, d = t % dim;
    vectors[t] = centres[(i % clusters) * dim + d] + v;
  });
}

__global__ void fx_queries(const uint32_t* __restrict__ key, uint64_t base, uint64_t total, uint32_t dim,
                           uint64_t count, uint64_t stride, const float* __restrict__ vectors,
                           float* __restrict__ queries) {
  fx_block(key, base, base + total, [&](uint64_t g, float v) {
    const uint64_t t = g - base, q = t / dim, d = t % dim;
    const uint64_t src = (q * stride) % count;
    queries[t] = vectors[src * dim + d] + v * 0.25f;
  });
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
