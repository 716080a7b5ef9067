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
// Inertia, cluster sums and k-means++ totals are f64 sums of f32 values in
// point order. They are summed in parallel with an exactness certificate
// (every nonzero term a multiple of 2^e and sum |x| < 2^(e+53) makes every
// partial sum exact, so any order gives the sequential bits); where the
// certificate fails, sequentially on the device, except k-means++ and inertia
// totals above SEQ_SUM_LIMIT points, which then keep a fixed parallel order
// (deterministic; a k-means++ pick can differ from the reference only when
// the drawn target falls within the last-bit difference of a cumulative
// boundary). k-means++ runs all rounds on the device, with the generator's
// state copied there and back.
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <exception>
#include <type_traits>
#include <vector>

#include "common.hpp"
#include "device.hpp"
#include "train.hpp"

namespace pxg {

constexpr int KM_LDS_FLOATS = 8192;  // 32 KiB of staged centroids
typedef float f16v __attribute__((ext_vector_type(16)));
// points of the last nearest_device call that the MFMA pass could not certify
thread_local size_t g_last_redo = 0;
// counters of this thread's last k-means run (measurement only)
struct KmStats {
  double mfma_ms = 0.0, mfma_flops = 0.0;
  uint64_t passes = 0, rescanned = 0, inexact_sums = 0;
  uint64_t reseeds = 0, pool_reseeds = 0, pool_fallbacks = 0;
};
thread_local KmStats g_km;
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
__device__ __forceinline__ void km_assign_body(const float* __restrict__ P, int ldp, const uint32_t* __restrict__ rows,
                                                 int n, int dim, const float* __restrict__ C, int ldc, int k,
                                                 uint32_t* __restrict__ assign, float* __restrict__ dist, int vec4, int bx) {
  __shared__ float cs[KM_LDS_FLOATS];
  const int i = bx * 256 + threadIdx.x;
  const bool valid = i < n;
  const size_t row = valid ? (rows ? rows[i] : (uint32_t)i) : 0;
  const float* pr = P + row * ldp;
  constexpr int DR = D > 0 ? D : 1;
  float x[DR];
  if constexpr (D > 0) {
    bool loaded = false;
    if constexpr (D % 4 == 0) {
      if (vec4) {  // rows 16-byte aligned: a quarter of the load instructions
#pragma unroll
        for (int j = 0; j < D; j += 4) {
          const float4 v = *reinterpret_cast<const float4*>(pr + j);
          x[j] = valid ? v.x : 0.0f;
          x[j + 1] = valid ? v.y : 0.0f;
          x[j + 2] = valid ? v.z : 0.0f;
          x[j + 3] = valid ? v.w : 0.0f;
        }
        loaded = true;
      }
    }
    if (!loaded) {
#pragma unroll
      for (int j = 0; j < D; ++j) x[j] = valid ? pr[j] : 0.0f;
    }
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

template <int D, bool UNR>
__global__ __launch_bounds__(256) void km_assign(const float* __restrict__ P, int ldp, const uint32_t* __restrict__ rows,
                                                 int n, int dim, const float* __restrict__ C, int ldc, int k,
                                                 uint32_t* __restrict__ assign, float* __restrict__ dist, int vec4) {
  km_assign_body<D, UNR>(P, ldp, rows, n, dim, C, ldc, k, assign, dist, vec4, blockIdx.x);
}

template <bool UNR>
static void launch_assign(const float* P, int ldp, const uint32_t* rows, size_t n, int dim, const float* C, int ldc,
                          size_t k, uint32_t* assign, float* dist, hipStream_t s) {
  const dim3 g((unsigned)((n + 255) / 256)), b(256);
  const int vec4 = (ldp % 4 == 0 && ((uintptr_t)P & 15) == 0) ? 1 : 0;
#define PXG_ASSIGN(DD)                                                                                             \
  hipLaunchKernelGGL((km_assign<DD, UNR>), g, b, 0, s, P, ldp, rows, (int)n, dim, C, ldc, (int)k, assign, dist, \
                     vec4)
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

// ---------------------------------------------------------------------------
// assignment on FP32 MFMA with exact verification
// ---------------------------------------------------------------------------
// km_mfma_top: for a block of 128 points, approximate squared distances to
// every centroid less the point's own |p|^2, a = |c|^2 - 2 p.c (one fma),
// with the dot product on v_mfma_f32_32x32x2f32 (128x128 tiles, 32-wide k
// slices double-buffered in LDS). Each lane keeps, per row it owns, the
// smallest and second-smallest approximation (and the smallest's centroid)
// over the columns it sees; the lanes and waves are merged at the end.
//
// km_mfma_verify: with eps a bound on |approx - exact| for every centroid of
// the point, every centroid whose exact distance could tie or beat the
// approximate winner's has approx <= best + 2 eps. If the second-smallest
// approximation is above best + 2 eps, the winner is the exact argmin
// (including the lower-index tie rule, since a tied centroid would be within
// 2 eps too); its exact distance is recomputed with the reference's own
// arithmetic. Other points are listed and take the exact VALU scan.
//
// A point's approximations all omit the same |p|^2, so their differences are
// those of the exact distances up to the errors below, and the certificate
// only compares differences.
//
// eps: the fp32 dot product and norms over d terms, the final rounding and
// the exact sequential (or 8-lane) sum of squares each stay within
// (2d + 6) * 2^-24 * (|p| + max|c|)^2; twice that is used.
//
// Non-finite values: with finite coordinates every partial sum of the
// approximation is at most (|p| + |c|)^2 in magnitude, which is below s^2 in
// km_mfma_verify's bound, so the approximations are finite whenever eps is.
// A NaN or infinite coordinate makes that row's norm non-finite (km_max_of
// propagates a centroid's), eps is then not finite, and the point takes the
// exact scan.
constexpr int KA_M = 128, KA_N = 128, KA_K = 32;

// |row|^2 in fp32 (any order; it only feeds the approximation): eight lanes
// per row, float4 loads (rows 16-byte aligned, dim a multiple of 4).
__device__ __forceinline__ void km_row_norms_body(const float* __restrict__ P, int ldp,
                                                  const uint32_t* __restrict__ rows, int n, int dim,
                                                  float* __restrict__ out, int bx) {
  const int i = bx * 32 + (threadIdx.x >> 3), sub = threadIdx.x & 7;
  float s = 0.0f;
  if (i < n) {
    const float* pr = P + (size_t)(rows ? rows[i] : (uint32_t)i) * ldp;
    for (int j = sub * 4; j < dim; j += 32) {
      const float4 x = *reinterpret_cast<const float4*>(pr + j);
      s += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
    }
  }
  s += __shfl_xor(s, 4, WAVE);
  s += __shfl_xor(s, 2, WAVE);
  s += __shfl_xor(s, 1, WAVE);
  if (i < n && sub == 0) out[i] = s;
}
__global__ __launch_bounds__(256) void km_row_norms(const float* __restrict__ P, int ldp,
                                                    const uint32_t* __restrict__ rows, int n, int dim,
                                                    float* __restrict__ out) {
  km_row_norms_body(P, ldp, rows, n, dim, out, blockIdx.x);
}

// The largest of v[0..n), or NaN if any is NaN.
__global__ __launch_bounds__(1024) void km_max_of(const float* __restrict__ v, int n, float* __restrict__ out) {
  __shared__ float sh[1024];
  float m = 0.0f;
  for (int i = threadIdx.x; i < n; i += 1024) {
    const float x = v[i];
    m = x > m || x != x ? x : m;  // a NaN, once taken, stays
  }
  sh[threadIdx.x] = m;
  __syncthreads();
  for (int o = 512; o > 0; o >>= 1) {
    if (threadIdx.x < o) {
      const float x = sh[threadIdx.x + o];
      if (x > sh[threadIdx.x] || x != x) sh[threadIdx.x] = x;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = sh[0];
}

// 16 zero bytes: the source of slice chunks past the end of a row.
__device__ const float4 km_zero16 = {0.0f, 0.0f, 0.0f, 0.0f};

// Global -> LDS copy of 16 bytes per lane (lane i's bytes land at m0 + 16 i),
// 64-bit address per lane. Inline asm, so that the compiler does not count
// it under vmcnt; km_mfma_top waits for it with km_vm_wait0 before each
// slice's barrier and uses m0 for nothing else.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void km_lds_copy16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g) : "memory", "m0");
}
#pragma clang diagnostic pop
__device__ __forceinline__ void km_vm_wait0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__global__ __launch_bounds__(256, 2) void km_mfma_top(const float* __restrict__ P, int ldp,
                                                      const uint32_t* __restrict__ rows, int n, int dim,
                                                      const float* __restrict__ C, int ldc, int k,
                                                      const float* __restrict__ cn,
                                                      uint32_t* __restrict__ best_idx, float* __restrict__ best,
                                                      float* __restrict__ second) {
  // k slices of the points (A) and of the centroids (B), double-buffered,
  // and after each tile's k loop the tile's dot products (dt), share one LDS
  // buffer. The slices are unpadded 128 x 32 floats: 16-byte chunk c of row
  // r sits at position c ^ (r & 7), so the MFMA operand reads are
  // conflict-free. A dt row holds columns 0-63, a 4-float gap, then columns
  // 64-127, so that the two threads of a row read their halves as float4
  // without bank conflicts.
  constexpr int SLICE = KA_M * KA_K, DT_LD = KA_N + 8;
  static_assert(KA_M == KA_N && 4 * SLICE <= KA_M * DT_LD, "slices fit the dot-product tile");
  static_assert(KA_N == 128 && KA_K == 32, "two 64-column halves per row; 8 chunks per slice row");
  __shared__ __align__(16) float smem[KA_M * DT_LD];
  __shared__ __align__(16) float scn[KA_N];
  float* dt = smem;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int h = lane >> 5, r = lane & 31;
  const int wm = (wid >> 1) * 64, wn = (wid & 1) * 64;
  const int p0 = blockIdx.x * KA_M;
  // DMA lanes: instruction u of wave wid fills rows 32 wid + 8 u .. +7 of a
  // slice, lane l landing at chunk position l & 7 of row 8 u + l / 8, so it
  // fetches that row's chunk (l & 7) ^ (row & 7). Rows past n (points) or k
  // (centroids) read a valid row: their products only reach outputs that are
  // never used.
  const int crow0 = 32 * wid + (lane >> 3), cchunk = (lane & 7) ^ ((lane >> 3) & 7);
  const float* prow[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int p = min(p0 + crow0 + 8 * u, n - 1);
    prow[u] = P + (size_t)(rows ? rows[p] : (uint32_t)p) * ldp;
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float*)smem;
  const int wid_s = __builtin_amdgcn_readfirstlane(wid);
  // slice k0 of centroid tile n0 into buffer buf
  auto gload = [&](int n0, int k0, int buf) __attribute__((always_inline)) {
    const int kc = k0 + cchunk * 4;
    const bool kin = kc < dim;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = min(n0 + crow0 + 8 * u, k - 1);
      const float* pa = kin ? prow[u] + kc : reinterpret_cast<const float*>(&km_zero16);
      const float* pb = kin ? C + (size_t)c * ldc + kc : reinterpret_cast<const float*>(&km_zero16);
      const uint32_t grp = (uint32_t)((32 * wid_s + 8 * u) * KA_K * 4);
      km_lds_copy16(pa, lds0 + (uint32_t)(buf * SLICE * 4) + grp);
      km_lds_copy16(pb, lds0 + (uint32_t)((2 + buf) * SLICE * 4) + grp);
    }
  };
  const int nK = (dim + KA_K - 1) / KA_K;
  // this thread scans row tid/2, columns 64 (tid&1) .. +63 of every tile
  const int my_row = tid >> 1, my_par = tid & 1;
  float b1 = INFINITY, b2 = INFINITY;
  int i1 = 0, t1 = 0;  // the smallest's column in its tile, and that tile
  for (int n0 = 0; n0 < k; n0 += KA_N) {
    f16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    __syncthreads();  // the previous tile's scan of dt is done
    if (tid < KA_N) scn[tid] = n0 + tid < k ? cn[n0 + tid] : 0.0f;
    gload(n0, 0, 0);
    km_vm_wait0();
    __syncthreads();
    for (int kt = 0; kt < nK; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nK) gload(n0, (kt + 1) * KA_K, cur ^ 1);
      // lane (h, r) feeds k = h*16 + 4 k4 + t of row r: chunk 4h + k4,
      // stored at position (4h + k4) ^ (r & 7); A and B agree on that map
      const float* a0p = &smem[cur * SLICE + (wm + r) * KA_K];
      const float* a1p = &smem[cur * SLICE + (wm + 32 + r) * KA_K];
      const float* b0p = &smem[(2 + cur) * SLICE + (wn + r) * KA_K];
      const float* b1p = &smem[(2 + cur) * SLICE + (wn + 32 + r) * KA_K];
      const int r7 = r & 7;
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4) {
        const int co = ((4 * h + k4) ^ r7) * 4;
        const float4 a0 = *reinterpret_cast<const float4*>(a0p + co);
        const float4 a1 = *reinterpret_cast<const float4*>(a1p + co);
        const float4 q0 = *reinterpret_cast<const float4*>(b0p + co);
        const float4 q1 = *reinterpret_cast<const float4*>(b1p + co);
        const float av0[4] = {a0.x, a0.y, a0.z, a0.w}, av1[4] = {a1.x, a1.y, a1.z, a1.w};
        const float bv0[4] = {q0.x, q0.y, q0.z, q0.w}, bv1[4] = {q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(av0[t], bv0[t], acc[0][0], 0, 0, 0);
          acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(av0[t], bv1[t], acc[0][1], 0, 0, 0);
          acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(av1[t], bv0[t], acc[1][0], 0, 0, 0);
          acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(av1[t], bv1[t], acc[1][1], 0, 0, 0);
        }
      }
      km_vm_wait0();  // this wave's copies of the next slice have landed
      __syncthreads();
    }
    // the tile's dot products to LDS, then each thread scans its row's
    // columns in ascending order (strict < keeps the first of equal values)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          dt[(wm + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3)) * DT_LD + wn + (wn >> 4) + j * 32 + r] = acc[i][j][v];
    __syncthreads();
    const float* drow = dt + my_row * DT_LD + my_par * 68;
    const int c0 = my_par * 64, cols = min(KA_N, k - n0);
    // Smallest, its first column (strict <) and second-smallest, in column
    // order. With b1 <= b2 the new second-smallest is the median of (b1, b2,
    // x) and the new smallest min(b1, x): one med3 and one min per value.
    // The column is kept within this thread's half-tile (a constant per
    // value); the tile is recorded once, after the tile, if b1 went down.
    const float b1_in = b1;
    auto take = [&](float x, int m) {
      i1 = x < b1 ? m : i1;
      b2 = __builtin_amdgcn_fmed3f(b1, b2, x);
      b1 = fminf(b1, x);
    };
    if (cols == KA_N) {
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const float4 d4 = *reinterpret_cast<const float4*>(drow + 4 * q);
        const float4 s4 = *reinterpret_cast<const float4*>(scn + c0 + 4 * q);
        take(__builtin_fmaf(-2.0f, d4.x, s4.x), 4 * q);
        take(__builtin_fmaf(-2.0f, d4.y, s4.y), 4 * q + 1);
        take(__builtin_fmaf(-2.0f, d4.z, s4.z), 4 * q + 2);
        take(__builtin_fmaf(-2.0f, d4.w, s4.w), 4 * q + 3);
      }
    } else {
      for (int m = c0; m < min(cols, c0 + 64); ++m) take(__builtin_fmaf(-2.0f, drow[m - c0], scn[m]), m - c0);
    }
    t1 = b1 < b1_in ? n0 : t1;
  }
  i1 += t1 + my_par * 64;
  // merge the two threads of each row
  const float y1 = __shfl_xor(b1, 1, WAVE), y2 = __shfl_xor(b2, 1, WAVE);
  const int yi = __shfl_xor(i1, 1, WAVE);
  if (my_par == 0 && p0 + my_row < n) {
    const bool take = y1 < b1 || (y1 == b1 && yi < i1);
    best[p0 + my_row] = take ? y1 : b1;
    best_idx[p0 + my_row] = (uint32_t)(take ? yi : i1);
    second[p0 + my_row] = fminf(take ? b1 : y1, fminf(b2, y2));
  }
}

// km_mfma_small: the same certified approximation for narrow rows (dim 8,
// 16 or 24: product-quantizer subspaces), with the centroids (k * dim <=
// KS_MAXF floats) and their norms staged in LDS once per workgroup. One wave
// takes 32 points at a time. With the centroids as the MFMA's A operand and
// the points as B, lane (h, r) ends each 32-centroid block holding point r's
// values for centroids 8 (v / 4) + 4 h + v % 4 of the block (v < 16), so the
// running top-2 stays in registers, as in km_mfma_top's scan (one fma, one
// compare and select, one med3, one min per value, the index as the value's
// position v with the block recorded once per block); the two half-waves
// merge at the end. Lane half h supplies dims [h dim/2, (h+1) dim/2) of both
// operands over the dim/2 MFMA steps: any order of the dot product's terms
// that both operands share is a valid one, and this one makes every operand
// load a float4. Rows 16-byte aligned.
constexpr int KS_MAXF = 8192;  // centroid floats staged in LDS (32 KB)
constexpr int KS_PW = 4;       // 32-point groups per wave
template <int DS>  // dim = 8 DS
__device__ __forceinline__ void km_mfma_small_body(const float* __restrict__ P, int ldp,
                                                   const uint32_t* __restrict__ rows, int n,
                                                   const float* __restrict__ C, int ldc, int k,
                                                   const float* __restrict__ cn, uint32_t* __restrict__ best_idx,
                                                   float* __restrict__ best, float* __restrict__ second,
                                                   float* __restrict__ sc, int bx) {
  constexpr int D = 8 * DS, HD = D / 2;
  // sc: [k][D] centroids, then their norms [k rounded up to 32]
  float* scn = sc + k * D;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, r = lane & 31;
  for (int f = tid; f < k * 2 * DS; f += 256) {
    const int row = f / (2 * DS), c4 = (f - row * 2 * DS) * 4;
    *reinterpret_cast<float4*>(&sc[row * D + c4]) = *reinterpret_cast<const float4*>(C + (size_t)row * ldc + c4);
  }
  const int kr = (k + 31) & ~31;
  for (int i = tid; i < kr; i += 256) scn[i] = i < k ? cn[i] : 0.0f;
  __syncthreads();
  const int nblk = kr / 32;
  for (int g = 0; g < KS_PW; ++g) {
    const int p0 = ((bx * 4 + w) * KS_PW + g) * 32;
    if (p0 >= n) break;  // wave-uniform
    const int pi = min(p0 + r, n - 1);
    const float* prow = P + (size_t)(rows ? rows[pi] : (uint32_t)pi) * ldp + h * HD;
    float bq[HD];
#pragma unroll
    for (int q = 0; q < HD / 4; ++q) {
      const float4 x = *reinterpret_cast<const float4*>(prow + 4 * q);
      bq[4 * q] = x.x;
      bq[4 * q + 1] = x.y;
      bq[4 * q + 2] = x.z;
      bq[4 * q + 3] = x.w;
    }
    float b1 = INFINITY, b2 = INFINITY;
    int i1 = 0, t1 = 0;
    auto take = [&](float x, int v) {
      i1 = x < b1 ? v : i1;
      b2 = __builtin_amdgcn_fmed3f(b1, b2, x);
      b1 = fminf(b1, x);
    };
    // one 32-centroid block; PART masks the centroids past k (last block)
    auto block = [&](int blk, auto part) __attribute__((always_inline)) {
      const float* ca = &sc[min(blk * 32 + r, k - 1) * D + h * HD];
      f16v acc;
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
#pragma unroll
      for (int q = 0; q < HD / 4; ++q) {
        const float4 a = *reinterpret_cast<const float4*>(ca + 4 * q);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, bq[4 * q], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, bq[4 * q + 1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, bq[4 * q + 2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, bq[4 * q + 3], acc, 0, 0, 0);
      }
      const float b1_in = b1;
#pragma unroll
      for (int vb = 0; vb < 4; ++vb) {
        const float4 c4 = *reinterpret_cast<const float4*>(&scn[blk * 32 + 8 * vb + 4 * h]);
        const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float x = __builtin_fmaf(-2.0f, acc[4 * vb + e], cv[e]);
          if constexpr (decltype(part)::value) x = blk * 32 + 8 * vb + 4 * h + e < k ? x : INFINITY;
          take(x, 4 * vb + e);
        }
      }
      t1 = b1 < b1_in ? blk : t1;
    };
    const int nfull = k / 32;
    for (int blk = 0; blk < nfull; ++blk) block(blk, std::false_type{});
    if (nfull < nblk) block(nfull, std::true_type{});
    int ix = t1 * 32 + 8 * (i1 >> 2) + 4 * h + (i1 & 3);
    // merge the two halves of the wave (lanes r and r + 32 hold point r)
    const float y1 = __shfl_xor(b1, 32, WAVE), y2 = __shfl_xor(b2, 32, WAVE);
    const int yi = __shfl_xor(ix, 32, WAVE);
    if (h == 0 && p0 + r < n) {
      const bool tk = y1 < b1 || (y1 == b1 && yi < ix);
      best[p0 + r] = tk ? y1 : b1;
      best_idx[p0 + r] = (uint32_t)(tk ? yi : ix);
      second[p0 + r] = fminf(tk ? b1 : y1, fminf(b2, y2));
    }
  }
}
template <int DS>
__global__ __launch_bounds__(256, 2) void km_mfma_small(const float* __restrict__ P, int ldp,
                                                     const uint32_t* __restrict__ rows, int n,
                                                     const float* __restrict__ C, int ldc, int k,
                                                     const float* __restrict__ cn, uint32_t* __restrict__ best_idx,
                                                     float* __restrict__ best, float* __restrict__ second) {
  extern __shared__ float4 ks_sm[];
  km_mfma_small_body<DS>(P, ldp, rows, n, C, ldc, k, cn, best_idx, best, second, reinterpret_cast<float*>(ks_sm),
                         blockIdx.x);
}

// km_mfma_reg: km_mfma_small's form for rows of 32 to 128 floats (dim a
// multiple of 32): each wave holds its 32 points' rows in VGPRs (lane half h
// the dims [h dim/2, (h+1) dim/2)) for the whole pass, and the centroids
// stream through LDS 32 rows at a time (a block of the MFMA), copied
// straight from memory (km_lds_copy16), double-buffered, one barrier per
// block. Rows are stored unpadded with 16-byte chunk c of row r at position
// c ^ (r & 7), so the lanes' float4 operand reads of 32 rows spread over the
// banks. The top-2 scan is km_mfma_small's; no dot-product tile goes
// through LDS. 128 points per 256-thread workgroup.
template <int HD>  // dim / 2
__global__ __launch_bounds__(256, 3) void km_mfma_reg(const float* __restrict__ P, int ldp,
                                                   const uint32_t* __restrict__ rows, int n,
                                                   const float* __restrict__ C, int ldc, int k,
                                                   const float* __restrict__ cn, uint32_t* __restrict__ best_idx,
                                                   float* __restrict__ best, float* __restrict__ second) {
  constexpr int D = 2 * HD, CPR = D / 4;  // 16-byte chunks per row
  static_assert(D % 32 == 0 && D <= 128, "whole groups of eight chunks per row");
  constexpr int TILE = 32 * D;             // floats per centroid block
  constexpr int NI = CPR / 8;              // copy instructions per wave per block (4 waves, 64 lanes)
  __shared__ __align__(16) float sc[2 * TILE];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, r = lane & 31;
  const int wid_s = __builtin_amdgcn_readfirstlane(w);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float*)sc;
  // the copy of block b into buffer buf: instruction u of wave w covers
  // chunk positions 64 (w NI + u) + lane of the block
  // (a full block's rows are the lane's fixed offsets plus the block's
  // uniform first row; the last block clamps its rows to k - 1)
  auto gload = [&](int b, int buf) __attribute__((always_inline)) {
    const bool full = b * 32 + 32 <= k;
    const float* cb = C + (size_t)(b * 32) * ldc;
#pragma unroll
    for (int u = 0; u < NI; ++u) {
      const int g = wid_s * NI + u;
      const int idx = 64 * g + lane, row = idx / CPR, pos = idx - row * CPR;
      const int c = pos ^ (row & 7);
      const float* src = full ? cb + (row * ldc + 4 * c) : C + (size_t)min(b * 32 + row, k - 1) * ldc + 4 * c;
      km_lds_copy16(src, lds0 + (uint32_t)((buf * TILE + 64 * 4 * g) * 4));
    }
  };
  const int p0 = (blockIdx.x * 4 + w) * 32;
  const int pi = min(p0 + r, n - 1);
  const float* prow = P + (size_t)(rows ? rows[pi] : (uint32_t)pi) * ldp + h * HD;
  float bq[HD];
#pragma unroll
  for (int q = 0; q < HD / 4; ++q) {
    const float4 x = *reinterpret_cast<const float4*>(prow + 4 * q);
    bq[4 * q] = x.x;
    bq[4 * q + 1] = x.y;
    bq[4 * q + 2] = x.z;
    bq[4 * q + 3] = x.w;
  }
  const int nblk = (k + 31) / 32;
  gload(0, 0);
  float b1 = INFINITY, b2 = INFINITY;
  int i1 = 0, t1 = 0;
  auto take = [&](float x, int v) {
    i1 = x < b1 ? v : i1;
    b2 = __builtin_amdgcn_fmed3f(b1, b2, x);
    b1 = fminf(b1, x);
  };
  const int r7 = r & 7;
  for (int blk = 0; blk < nblk; ++blk) {
    const int cur = blk & 1;
    // this block's norms (rows 8 (v/4) + 4 h + v%4), loaded before the wait:
    // four rows at a time in a full block (cn is 16-byte aligned)
    float cv[16];
    if (blk * 32 + 32 <= k) {
      const float* cr = cn + blk * 32 + 4 * h;
#pragma unroll
      for (int vb = 0; vb < 4; ++vb) {
        const float4 c4 = *reinterpret_cast<const float4*>(cr + 8 * vb);
        cv[4 * vb] = c4.x;
        cv[4 * vb + 1] = c4.y;
        cv[4 * vb + 2] = c4.z;
        cv[4 * vb + 3] = c4.w;
      }
    } else {
#pragma unroll
      for (int vb = 0; vb < 4; ++vb) {
#pragma unroll
        for (int e = 0; e < 4; ++e) cv[4 * vb + e] = cn[min(blk * 32 + 8 * vb + 4 * h + e, k - 1)];
      }
    }
    km_vm_wait0();  // this wave's copies of block blk (and the norms) have landed
    __syncthreads();  // everyone's copies of blk are in; everyone is done with blk - 1
    if (blk + 1 < nblk) gload(blk + 1, cur ^ 1);
    const float* ca = &sc[cur * TILE + r * D];
    f16v acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
#pragma unroll
    for (int q = 0; q < HD / 4; ++q) {
      const float4 a = *reinterpret_cast<const float4*>(ca + 4 * ((h * (HD / 4) + q) ^ r7));
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, bq[4 * q], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, bq[4 * q + 1], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, bq[4 * q + 2], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, bq[4 * q + 3], acc, 0, 0, 0);
    }
    const float b1_in = b1;
    if (blk * 32 + 32 <= k) {
#pragma unroll
      for (int v = 0; v < 16; ++v) take(__builtin_fmaf(-2.0f, acc[v], cv[v]), v);
    } else {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float x = __builtin_fmaf(-2.0f, acc[v], cv[v]);
        take(blk * 32 + 8 * (v >> 2) + 4 * h + (v & 3) < k ? x : INFINITY, v);
      }
    }
    t1 = b1 < b1_in ? blk : t1;
  }
  const int ix = t1 * 32 + 8 * (i1 >> 2) + 4 * h + (i1 & 3);
  const float y1 = __shfl_xor(b1, 32, WAVE), y2 = __shfl_xor(b2, 32, WAVE);
  const int yi = __shfl_xor(ix, 32, WAVE);
  if (h == 0 && p0 + r < n) {
    const bool tk = y1 < b1 || (y1 == b1 && yi < ix);
    best[p0 + r] = tk ? y1 : b1;
    best_idx[p0 + r] = (uint32_t)(tk ? yi : ix);
    second[p0 + r] = fminf(tk ? b1 : y1, fminf(b2, y2));
  }
}

constexpr int KV_PB = 128;  // points per km_mfma_verify block (256 threads)
template <bool UNR>
__device__ __forceinline__ void km_mfma_verify_body(const float* __restrict__ P, int ldp,
                                                    const uint32_t* __restrict__ rows, int n, int dim,
                                                    const float* __restrict__ C, int ldc,
                                                    const float* __restrict__ pn, const float* __restrict__ cmax,
                                                    const uint32_t* __restrict__ best_idx,
                                                    const float* __restrict__ best, const float* __restrict__ second,
                                                    uint32_t* __restrict__ assign, float* __restrict__ dist,
                                                    uint32_t* __restrict__ redo, int* __restrict__ nredo, int bx) {
  // the block's KV_PB points and their winning centroids, staged through LDS
  // 32 coordinates at a time (eight lanes per 128-byte row slice); 34 KB of
  // LDS, so four blocks per CU keep the row loads in flight
  __shared__ float tp[KV_PB * 33], tc[KV_PB * 33];
  __shared__ uint32_t sr[KV_PB], sc[KV_PB];
  const int t = threadIdx.x, i0 = bx * KV_PB, i = i0 + t;
  bool ok = false;
  if (t < KV_PB) {  // threads KV_PB.. only help with the loads
    if (i < n) {
      const float s = (sqrtf(pn[i]) + sqrtf(cmax[0])) * 1.0001f;
      const float eps = 2.0f * (2.0f * (float)dim + 6.0f) * 5.9604645e-08f * s * s;
      ok = second[i] > best[i] + 2.0f * eps;
      if (!ok) redo[atomicAdd(nredo, 1)] = (uint32_t)i;
      sr[t] = rows ? rows[i] : (uint32_t)i;
      sc[t] = best_idx[i];
    } else {
      sr[t] = 0;
      sc[t] = 0;
    }
  }
  float sum = 0.0f, acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const int ch8 = (dim >> 3) << 3;
  for (int j0 = 0; j0 < dim; j0 += 32) {
    const int w = min(32, dim - j0);
    __syncthreads();
    for (int f = t; f < KV_PB * 8; f += 256) {
      const int r = f >> 3, c4 = (f & 7) * 4;
      if (c4 < w && i0 + r < n) {
        const float4 x = *reinterpret_cast<const float4*>(P + (size_t)sr[r] * ldp + j0 + c4);
        const float4 y = *reinterpret_cast<const float4*>(C + (size_t)sc[r] * ldc + j0 + c4);
        float* dp = tp + r * 33 + c4;
        float* dc = tc + r * 33 + c4;
        dp[0] = x.x; dp[1] = x.y; dp[2] = x.z; dp[3] = x.w;
        dc[0] = y.x; dc[1] = y.y; dc[2] = y.z; dc[3] = y.w;
      }
    }
    __syncthreads();
    if (ok) {
      const float* a = tp + t * 33;
      const float* b = tc + t * 33;
      int jj = 0;
      if constexpr (UNR) {
        // squared_euclidean_unrolled: lane j & 7 for the 8-wide chunks
        // (j0 and ch8 are multiples of 8), then the sequential tail
        for (; jj + 8 <= w && j0 + jj < ch8; jj += 8)
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const float d = a[jj + u] - b[jj + u];
            acc[u] += d * d;
          }
      }
      for (; jj < w; ++jj) {
        const float d = a[jj] - b[jj];
        sum += d * d;  // squared(), kmeans.rs:234-241 (or the unrolled tail)
      }
    }
  }
  if (ok) {
    assign[i] = sc[t];
    if (dist) {
      if constexpr (UNR)
        dist[i] = (((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]))) + sum;
      else
        dist[i] = sum;
    }
  }
}
template <bool UNR>
__global__ __launch_bounds__(256) void km_mfma_verify(const float* __restrict__ P, int ldp,
                                                      const uint32_t* __restrict__ rows, int n, int dim,
                                                      const float* __restrict__ C, int ldc,
                                                      const float* __restrict__ pn, const float* __restrict__ cmax,
                                                      const uint32_t* __restrict__ best_idx,
                                                      const float* __restrict__ best, const float* __restrict__ second,
                                                      uint32_t* __restrict__ assign, float* __restrict__ dist,
                                                      uint32_t* __restrict__ redo, int* __restrict__ nredo) {
  km_mfma_verify_body<UNR>(P, ldp, rows, n, dim, C, ldc, pn, cmax, best_idx, best, second, assign, dist, redo, nredo,
                           blockIdx.x);
}

constexpr int KW_DMAX = 2048;  // largest dim of the MFMA assignment path

// Exact nearest centroid for the listed points, KX_PB points per workgroup
// staged in LDS: each lane takes centroids c, c+256, ... in order (strict <)
// and applies the values it loads to all KX_PB points, so the centroids
// stream once per KX_PB points. Per point the distance is the reference's
// sequential `squared` (or, UNR, the 8-lane kernel); the lanes' and waves'
// bests merge lexicographically in (distance, centroid), which keeps the
// lowest index among equal distances. Centroid rows are read as float4 (rows
// 16-byte aligned, dim a multiple of 4, dim <= KW_DMAX).
constexpr int KX_PB = 8;
template <bool UNR>
__global__ __launch_bounds__(256) void km_exact_multi(const float* __restrict__ P, int ldp,
                                                      const uint32_t* __restrict__ rows, int m, int dim,
                                                      const float* __restrict__ C, int ldc, int k,
                                                      uint32_t* __restrict__ assign, float* __restrict__ dist) {
  extern __shared__ float4 kx_sm[];
  float* sp = reinterpret_cast<float*>(kx_sm);  // [KX_PB][dim]
  __shared__ float sbd[4][KX_PB];
  __shared__ int sbi[4][KX_PB];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int p0 = blockIdx.x * KX_PB, np = min(KX_PB, m - p0);
  for (int t = tid; t < KX_PB * dim; t += 256) {
    const int i = t / dim, j = t - i * dim;
    sp[t] = i < np ? P[(size_t)rows[p0 + i] * ldp + j] : 0.0f;
  }
  __syncthreads();
  float bd[KX_PB];
  int bi[KX_PB];
#pragma unroll
  for (int i = 0; i < KX_PB; ++i) {
    bd[i] = INFINITY;
    bi[i] = 0;
  }
  const int ch8 = (dim >> 3) << 3;
  for (int c = w * 64 + lane; c < k; c += 256) {
    const float* cr = C + (size_t)c * ldc;
    float sum[KX_PB];
    if constexpr (UNR) {
      float acc[KX_PB][8];
#pragma unroll
      for (int i = 0; i < KX_PB; ++i)
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[i][u] = 0.0f;
      for (int j = 0; j < ch8; j += 8) {
        const float4 c0 = *reinterpret_cast<const float4*>(cr + j);
        const float4 c1 = *reinterpret_cast<const float4*>(cr + j + 4);
        const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
        for (int i = 0; i < KX_PB; ++i) {
          const float4 x0 = *reinterpret_cast<const float4*>(sp + i * dim + j);
          const float4 x1 = *reinterpret_cast<const float4*>(sp + i * dim + j + 4);
          const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const float d = xv[u] - cv[u];
            acc[i][u] += d * d;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < KX_PB; ++i) {
        float t = 0.0f;
        for (int j = ch8; j < dim; ++j) {
          const float d = sp[i * dim + j] - cr[j];
          t += d * d;
        }
        const float* a = acc[i];
        sum[i] = (((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]))) + t;
      }
    } else {
#pragma unroll
      for (int i = 0; i < KX_PB; ++i) sum[i] = 0.0f;
      for (int j = 0; j < dim; j += 4) {
        const float4 cv = *reinterpret_cast<const float4*>(cr + j);
#pragma unroll
        for (int i = 0; i < KX_PB; ++i) {
          const float4 x = *reinterpret_cast<const float4*>(sp + i * dim + j);
          float d = x.x - cv.x;
          sum[i] += d * d;
          d = x.y - cv.y;
          sum[i] += d * d;
          d = x.z - cv.z;
          sum[i] += d * d;
          d = x.w - cv.w;
          sum[i] += d * d;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < KX_PB; ++i)
      if (sum[i] < bd[i]) {
        bd[i] = sum[i];
        bi[i] = c;
      }
  }
#pragma unroll
  for (int i = 0; i < KX_PB; ++i) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float od = __shfl_xor(bd[i], o, WAVE);
      const int oi = __shfl_xor(bi[i], o, WAVE);
      if (od < bd[i] || (od == bd[i] && oi < bi[i])) {
        bd[i] = od;
        bi[i] = oi;
      }
    }
    if (lane == 0) {
      sbd[w][i] = bd[i];
      sbi[w][i] = bi[i];
    }
  }
  __syncthreads();
  if (tid < np) {
    float b = sbd[0][tid];
    int x = sbi[0][tid];
    for (int v = 1; v < 4; ++v)
      if (sbd[v][tid] < b || (sbd[v][tid] == b && sbi[v][tid] < x)) {
        b = sbd[v][tid];
        x = sbi[v][tid];
      }
    assign[p0 + tid] = (uint32_t)x;
    dist[p0 + tid] = b;
  }
}

__global__ void km_scatter_redo(const uint32_t* __restrict__ redo, int m, const uint32_t* __restrict__ a,
                                const float* __restrict__ d, uint32_t* __restrict__ assign, float* __restrict__ dist) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= m) return;
  assign[redo[t]] = a[t];
  if (dist) dist[redo[t]] = d[t];
}

__global__ void km_compose_rows(const uint32_t* __restrict__ redo, int m, const uint32_t* __restrict__ rows,
                                uint32_t* __restrict__ out) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t < m) out[t] = rows ? rows[redo[t]] : redo[t];
}

// Points with enough work for the matrix cores (and float4-aligned rows)
// take the MFMA pass; the exact VALU scan serves the rest and the points the
// MFMA pass cannot certify.
void nearest_device(const float* P, int ldp, const uint32_t* rows, size_t n, int dim, const float* C, int ldc,
                    size_t k, bool unrolled, uint32_t* assign, float* dist, hipStream_t s) {
  nearest_device(P, ldp, rows, n, dim, C, ldc, k, unrolled, assign, dist, s, nullptr);
}

void nearest_device(const float* P, int ldp, const uint32_t* rows, size_t n, int dim, const float* C, int ldc,
                    size_t k, bool unrolled, uint32_t* assign, float* dist, hipStream_t s, NearestWork* ws) {
  g_last_redo = 0;
  if (n == 0) return;
  const bool aligned = ldp % 4 == 0 && ldc % 4 == 0 && dim % 4 == 0 && ((uintptr_t)P & 15) == 0 &&
                       ((uintptr_t)C & 15) == 0;
  // narrow rows (product-quantizer subspaces) with their centroids in LDS
  const bool small = aligned && (dim == 8 || dim == 16 || dim == 24) && k >= 64 && k * dim <= KS_MAXF && n >= 4096;
  if (!small && !(aligned && dim >= 32 && dim <= KW_DMAX && k >= 64 && n >= 4096)) {
    if (unrolled)
      launch_assign<true>(P, ldp, rows, n, dim, C, ldc, k, assign, dist, s);
    else
      launch_assign<false>(P, ldp, rows, n, dim, C, ldc, k, assign, dist, s);
    return;
  }
  NearestWork local;
  NearestWork& w = ws ? *ws : local;
  w.pn.reserve(n);
  w.cn.reserve(k);
  w.cmax.reserve(1);
  w.best.reserve(n);
  w.second.reserve(n);
  w.bidx.reserve(n);
  w.redo.reserve(n);
  w.nredo.reserve(1);
  float *const pn = w.pn.p, *const cn = w.cn.p, *const cmax = w.cmax.p, *const best = w.best.p,
               *const second = w.second.p;
  uint32_t *const bidx = w.bidx.p, *const redo = w.redo.p;
  int* const nredo = w.nredo.p;
  const bool keyed = rows == nullptr;
  if (!(keyed && w.pn_of == P && w.pn_ld == ldp && w.pn_dim == dim && w.pn_n == n)) {
    hipLaunchKernelGGL(km_row_norms, dim3((unsigned)((n + 31) / 32)), dim3(256), 0, s, P, ldp, rows, (int)n, dim,
                       pn);
    w.pn_of = keyed ? P : nullptr;
    w.pn_ld = ldp;
    w.pn_dim = dim;
    w.pn_n = n;
  }
  hipLaunchKernelGGL(km_row_norms, dim3((unsigned)((k + 31) / 32)), dim3(256), 0, s, C, ldc,
                     (const uint32_t*)nullptr, (int)k, dim, cn);
  hipLaunchKernelGGL(km_max_of, dim3(1), dim3(1024), 0, s, cn, (int)k, cmax);
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (small) {
    const dim3 gs((unsigned)((n + 4 * KS_PW * 32 - 1) / (4 * KS_PW * 32)));
    const size_t lds = (k * dim + ((k + 31) & ~(size_t)31)) * 4;
    if (dim == 8)
      hipLaunchKernelGGL(km_mfma_small<1>, gs, dim3(256), lds, s, P, ldp, rows, (int)n, C, ldc, (int)k,
                         (const float*)cn, bidx, best, second);
    else if (dim == 16)
      hipLaunchKernelGGL(km_mfma_small<2>, gs, dim3(256), lds, s, P, ldp, rows, (int)n, C, ldc, (int)k,
                         (const float*)cn, bidx, best, second);
    else
      hipLaunchKernelGGL(km_mfma_small<3>, gs, dim3(256), lds, s, P, ldp, rows, (int)n, C, ldc, (int)k,
                         (const float*)cn, bidx, best, second);
  } else {
    PXG_HIP(hipEventCreate(&e0));
    PXG_HIP(hipEventCreate(&e1));
    PXG_HIP(hipEventRecord(e0, s));
    const dim3 g128((unsigned)((n + 127) / 128));
    if (dim == 128)
      hipLaunchKernelGGL(km_mfma_reg<64>, g128, dim3(256), 0, s, P, ldp, rows, (int)n, C, ldc, (int)k,
                         (const float*)cn, bidx, best, second);
    else if (dim == 96)
      hipLaunchKernelGGL(km_mfma_reg<48>, g128, dim3(256), 0, s, P, ldp, rows, (int)n, C, ldc, (int)k,
                         (const float*)cn, bidx, best, second);
    else if (dim == 64)
      hipLaunchKernelGGL(km_mfma_reg<32>, g128, dim3(256), 0, s, P, ldp, rows, (int)n, C, ldc, (int)k,
                         (const float*)cn, bidx, best, second);
    else if (dim == 32)
      hipLaunchKernelGGL(km_mfma_reg<16>, g128, dim3(256), 0, s, P, ldp, rows, (int)n, C, ldc, (int)k,
                         (const float*)cn, bidx, best, second);
    else
      hipLaunchKernelGGL(km_mfma_top, dim3((unsigned)((n + KA_M - 1) / KA_M)), dim3(256), 0, s, P, ldp, rows,
                         (int)n, dim, C, ldc, (int)k, (const float*)cn, bidx, best, second);
    PXG_HIP(hipEventRecord(e1, s));
  }
  PXG_HIP(hipMemsetAsync(nredo, 0, 4, s));
  const dim3 g((unsigned)((n + KV_PB - 1) / KV_PB));
  if (unrolled)
    hipLaunchKernelGGL(km_mfma_verify<true>, g, dim3(256), 0, s, P, ldp, rows, (int)n, dim, C, ldc, (const float*)pn,
                       (const float*)cmax, (const uint32_t*)bidx, (const float*)best, (const float*)second, assign,
                       dist, redo, nredo);
  else
    hipLaunchKernelGGL(km_mfma_verify<false>, g, dim3(256), 0, s, P, ldp, rows, (int)n, dim, C, ldc, (const float*)pn,
                       (const float*)cmax, (const uint32_t*)bidx, (const float*)best, (const float*)second, assign,
                       dist, redo, nredo);
  PXG_HIP(hipGetLastError());
  int m = 0;
  PXG_HIP(hipMemcpyAsync(&m, nredo, 4, hipMemcpyDeviceToHost, s));
  PXG_HIP(hipStreamSynchronize(s));
  if (!small) {  // the counters cover km_mfma_top
    float ms = 0.0f;
    PXG_HIP(hipEventElapsedTime(&ms, e0, e1));
    PXG_HIP(hipEventDestroy(e0));
    PXG_HIP(hipEventDestroy(e1));
    g_km.mfma_ms += ms;
    g_km.mfma_flops += 2.0 * (double)n * (double)k * (double)dim;
    g_km.passes += 1;
  }
  g_km.rescanned += (uint64_t)m;
  g_last_redo = (size_t)m;
  if (m == 0) return;
  // the uncertified points: exact scan over their rows, results scattered back
  w.rrows.reserve(m);
  w.ra.reserve(m);
  w.rd.reserve(m);
  uint32_t *const rrows = w.rrows.p, *const ra = w.ra.p;
  float* const rd = w.rd.p;
  hipLaunchKernelGGL(km_compose_rows, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s, (const uint32_t*)redo, m,
                     rows, rrows);
  const dim3 gx((unsigned)((m + KX_PB - 1) / KX_PB));
  const size_t lx = (size_t)KX_PB * dim * 4;
  if (unrolled)
    hipLaunchKernelGGL(km_exact_multi<true>, gx, dim3(256), lx, s, P, ldp, (const uint32_t*)rrows, m, dim, C, ldc,
                       (int)k, ra, rd);
  else
    hipLaunchKernelGGL(km_exact_multi<false>, gx, dim3(256), lx, s, P, ldp, (const uint32_t*)rrows, m, dim, C, ldc,
                       (int)k, ra, rd);
  hipLaunchKernelGGL(km_scatter_redo, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s, (const uint32_t*)redo, m,
                     (const uint32_t*)ra, (const float*)rd, assign, dist);
  PXG_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// f64 sums of f32 values in point order
// ---------------------------------------------------------------------------
// The reference adds f32 values into an f64 accumulator in point order
// (kmeans.rs:94, 107-112, 161, 171-176). If every nonzero term is a multiple
// of 2^e (e = the smallest ulp exponent among them) and sum |x| < 2^(e+53),
// every partial sum of any subset is a multiple of 2^e below 2^(e+53), hence
// an exact f64: a parallel sum then has the sequential sum's bits. The
// kernels below carry that certificate (f64 sum, f64 sum of |x|, smallest ulp
// exponent) per block; where it fails the sum is redone sequentially up to
// SEQ_SUM_LIMIT terms, and kept in the fixed parallel order above that.
constexpr int NO_TERMS = 1 << 20;  // ulp exponent of a set with no nonzero term

__device__ inline int ulp_exp(float x) {  // nonzero finite x
  const int e = (int)((__float_as_uint(x) >> 23) & 0xFFu);
  return (e > 0 ? e : 1) - 150;
}

__host__ __device__ inline bool sums_exact(double abs_sum, int emin) {
  if (emin >= NO_TERMS) return true;
  // the margin covers rounding in abs_sum itself (n < 2^30 terms)
  return abs_sum < ldexp(1.0 - 0x1p-20, emin + 53);
}

struct SumCert {
  double s, a;
  int e;
};

__device__ inline double shfl_xor_f64(double v, int m) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)b, m, WAVE);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(b >> 32), m, WAVE);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Fixed-order reduction over a 256-thread block (xor butterflies, then the
// four wave results in wave order); every thread gets the result.
__device__ inline SumCert block_cert_256(SumCert v, SumCert* sh) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    v.s += shfl_xor_f64(v.s, o);
    v.a += shfl_xor_f64(v.a, o);
    v.e = min(v.e, __shfl_xor(v.e, o, WAVE));
  }
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  SumCert r = sh[0];
  for (int i = 1; i < 4; ++i) {
    r.s += sh[i].s;
    r.a += sh[i].a;
    r.e = min(r.e, sh[i].e);
  }
  return r;
}

__device__ inline SumCert cert_of(float x) {
  return SumCert{(double)x, (double)fabsf(x), x != 0.0f ? ulp_exp(x) : NO_TERMS};
}

// per-256-value block certificates of v[0..n)
__device__ __forceinline__ void f64_partials_body(const float* __restrict__ v, int n, double* __restrict__ ps,
                                                    double* __restrict__ pa, int* __restrict__ pe, int bx) {
  __shared__ SumCert sh[4];
  const int i = bx * 256 + threadIdx.x;
  const SumCert r = block_cert_256(cert_of(i < n ? v[i] : 0.0f), sh);
  if (threadIdx.x == 0) {
    ps[bx] = r.s;
    pa[bx] = r.a;
    pe[bx] = r.e;
  }
}

__global__ __launch_bounds__(256) void f64_partials(const float* __restrict__ v, int n, double* __restrict__ ps,
                                                    double* __restrict__ pa, int* __restrict__ pe) {
  f64_partials_body(v, n, ps, pa, pe, blockIdx.x);
}

// Sequential sum of v[0..n) by one block: all threads stage 4096 values in
// LDS, thread 0 runs the dependent chain.
__device__ inline double seq_sum_block(const float* __restrict__ v, int n, float* stage) {
  double s = 0.0;
  for (int c0 = 0; c0 < n; c0 += 4096) {
    const int m = min(4096, n - c0);
    __syncthreads();
    for (int t = threadIdx.x; t < m; t += blockDim.x) stage[t] = v[c0 + t];
    __syncthreads();
    if (threadIdx.x == 0)
      for (int t = 0; t < m; ++t) s += (double)stage[t];
  }
  return s;
}

// Total of v from its block certificates (one 1024-thread block): exact when
// the certificate holds, else sequential (n <= SEQ_SUM_LIMIT) or the fixed
// order. out[0] = total, out[1] = 1.0 if it equals the sequential sum.
__device__ __forceinline__ void f64_total_body(const float* __restrict__ v, int n, const double* __restrict__ ps,
                                                  const double* __restrict__ pa, const int* __restrict__ pe, int nb,
                                                  double* __restrict__ out) {
  __shared__ double ss[1024], sa[1024];
  __shared__ int se[1024];
  __shared__ float stage[4096];
  const int t = threadIdx.x, per = (nb + 1023) / 1024;
  double s = 0.0, a = 0.0;
  int e = NO_TERMS;
  for (int b = t * per; b < min(nb, (t + 1) * per); ++b) {
    s += ps[b];
    a += pa[b];
    e = min(e, pe[b]);
  }
  ss[t] = s;
  sa[t] = a;
  se[t] = e;
  __syncthreads();
  for (int o = 512; o > 0; o >>= 1) {
    if (t < o) {
      ss[t] += ss[t + o];
      sa[t] += sa[t + o];
      se[t] = min(se[t], se[t + o]);
    }
    __syncthreads();
  }
  const bool exact = sums_exact(sa[0], se[0]);
  double total = ss[0];
  if (!exact && n <= (int)SEQ_SUM_LIMIT) total = seq_sum_block(v, n, stage);
  if (t == 0) {
    out[0] = total;
    out[1] = (exact || n <= (int)SEQ_SUM_LIMIT) ? 1.0 : 0.0;
  }
}

__global__ __launch_bounds__(1024) void f64_total(const float* __restrict__ v, int n, const double* __restrict__ ps,
                                                  const double* __restrict__ pa, const int* __restrict__ pe, int nb,
                                                  double* __restrict__ out) {
  f64_total_body(v, n, ps, pa, pe, nb, out);
}

struct F64Sum {
  DevBuf<double> ps, pa, out;
  DevBuf<int> pe;
  bool last_exact = true;  // the last total equals the sequential sum
  // f64 sum of v[0..n) in point order (see above); synchronises the stream
  double total(const float* v, size_t n, hipStream_t s) {
    const int nb = (int)std::max<size_t>((n + 255) / 256, 1);
    ps.reserve(nb);
    pa.reserve(nb);
    pe.reserve(nb);
    out.reserve(2);
    hipLaunchKernelGGL(f64_partials, dim3(nb), dim3(256), 0, s, v, (int)n, ps.p, pa.p, pe.p);
    hipLaunchKernelGGL(f64_total, dim3(1), dim3(1024), 0, s, v, (int)n, ps.p, pa.p, pe.p, nb, out.p);
    PXG_HIP(hipGetLastError());
    double h[2] = {0, 0};
    PXG_HIP(hipMemcpyAsync(h, out.p, 16, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    last_exact = h[1] != 0.0;
    return h[0];
  }
};

// ---------------------------------------------------------------------------
// k-means++ (kmeans.rs:146-194), all rounds on the device
// ---------------------------------------------------------------------------
// Round r: km_pp_pick draws the next centre from the distances left by round
// r-1 (total, target = gen_range(0.0..total) from the device copy of the
// generator, first point whose cumulative sum reaches it) and copies its row;
// km_pp_round then lowers every point's distance to that centre (strict <)
// and leaves per-block sum certificates for the next pick. No host round trip.
constexpr int PP_ROWS = 256;  // points per km_pp_round block

// Sequential squared (kmeans.rs:234-241) of each of the block's 256 points to
// centre c: the block's rows are staged through LDS 32 coordinates at a time
// (coalesced loads), each thread then runs its point's chain.
__device__ __forceinline__ void km_pp_round_body(const float* __restrict__ P, int ldp, int n, int dim,
                                                   const float* __restrict__ c, float* __restrict__ ns, int init,
                                                   double* __restrict__ ps, int* __restrict__ pe, int vec4, int bx) {
  constexpr int CS = 2048;  // centre coordinates staged in LDS
  __shared__ float tile[PP_ROWS * 33];
  __shared__ float cs[CS];
  __shared__ SumCert sh[4];
  const int t = threadIdx.x;
  const int r0 = bx * PP_ROWS;
  const bool staged_c = dim <= CS;
  if (staged_c)
    for (int j = t; j < dim; j += 256) cs[j] = c[j];
  const float* cc = staged_c ? cs : c;
  float sum = 0.0f;
  // vec4: 8 threads per 32-coordinate row slice, 16 bytes each (w is a
  // multiple of 4); the next slice is loaded into registers while this one
  // is scored
  constexpr int PF = PP_ROWS * 8 / 256;
  float4 nx[PF];
  auto gload = [&](int j0) {
    const int w = min(32, dim - j0);
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int f = t + 256 * u, r = f >> 3, c4 = (f & 7) * 4;
      nx[u] = (c4 < w && r0 + r < n) ? *reinterpret_cast<const float4*>(P + (size_t)(r0 + r) * ldp + j0 + c4)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  if (vec4) gload(0);
  for (int j0 = 0; j0 < dim; j0 += 32) {
    const int w = min(32, dim - j0);
    __syncthreads();
    if (vec4) {
#pragma unroll
      for (int u = 0; u < PF; ++u) {
        const int f = t + 256 * u, r = f >> 3, c4 = (f & 7) * 4;
        float* d = tile + r * 33 + c4;
        d[0] = nx[u].x;
        d[1] = nx[u].y;
        d[2] = nx[u].z;
        d[3] = nx[u].w;
      }
      if (j0 + 32 < dim) gload(j0 + 32);
    } else {
      for (int f = t; f < PP_ROWS * 32; f += 256) {
        const int r = f >> 5, cidx = f & 31;
        if (cidx < w) tile[r * 33 + cidx] = r0 + r < n ? P[(size_t)(r0 + r) * ldp + j0 + cidx] : 0.0f;
      }
    }
    __syncthreads();
    const float* row = tile + t * 33;
    for (int jj = 0; jj < w; ++jj) {
      const float d = row[jj] - cc[j0 + jj];
      sum += d * d;
    }
  }
  const int i = r0 + t;
  float nv = 0.0f;
  if (i < n) {
    nv = sum;
    if (!init) {
      const float cur = ns[i];
      if (!(sum < cur)) nv = cur;
    }
    ns[i] = nv;
  }
  const SumCert r = block_cert_256(cert_of(nv), sh);
  if (t == 0) {
    ps[bx] = r.s;
    pe[bx] = r.e;
  }
}

__global__ __launch_bounds__(256) void km_pp_round(const float* __restrict__ P, int ldp, int n, int dim,
                                                   const float* __restrict__ c, float* __restrict__ ns, int init,
                                                   double* __restrict__ ps, int* __restrict__ pe, int vec4) {
  km_pp_round_body(P, ldp, n, dim, c, ns, init, ps, pe, vec4, blockIdx.x);
}

// ---------------------------------------------------------------------------
// k-means++ rounds over an int8 copy of the points, certified
// ---------------------------------------------------------------------------
// A round only lowers ns[i] when the new centre c is strictly nearer than the
// current one. Each point also has an int8 copy q_i (scale s_i = max|p_i| /
// 127, q = rint(p / s_i)) and the exact distance delta_i = |p_i - s_i q_i|.
// The centre is itself a point (kmeans.rs:169-186 picks rows), so it has q_c,
// s_c and delta_c. With e = |s_i q_i - s_c q_c| from the exact integer dot
// product, the triangle inequality gives |p_i - c| >= e - delta_i - delta_c
// = L. The reference's sequential f32 sum (kmeans.rs:234-241) of dim
// squares is >= |p_i - c|^2 (1 - (dim + 2) 2^-24) for non-negative terms, so
// when L^2 (1 - gamma) >= ns[i] (with margins for the f64 rounding of e and
// for subnormal terms) the exact distance cannot be below ns[i] and the
// point keeps its value without its f32 row being read. The other points
// (those the centre may capture) are scored exactly as km_pp_round does.
// Per point the round then reads 4 + 16 bytes plus dim bytes, not 4 dim.
constexpr int Q8_ROWS = 256;  // points per km_pp_round_q8 block

// int8 copy, scale, delta and squared norm of the copy: one wave per point.
__global__ __launch_bounds__(256) void km_q8_prep(const float* __restrict__ P, int ldp, int n, int dim, int kq,
                                                  int8_t* __restrict__ Q, float* __restrict__ scale,
                                                  float* __restrict__ delta, int* __restrict__ qnorm) {
  const int lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= n) return;
  const float* p = P + (size_t)i * ldp;
  float mx = 0.0f;
  for (int j = lane; j < dim; j += 64) mx = fmaxf(mx, fabsf(p[j]));
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  const float sc = mx / 127.0f;
  double d2 = 0.0;
  int qn = 0;
  for (int j = lane; j < kq; j += 64) {
    int q = 0;
    if (j < dim && sc > 0.0f) q = max(-127, min(127, (int)rintf(p[j] / sc)));
    if (j < dim) {
      const double r = (double)p[j] - (double)q * (double)sc;
      d2 += r * r;
    }
    qn += q * q;
    Q[(size_t)i * kq + j] = (int8_t)q;
  }
  for (int o = 32; o > 0; o >>= 1) {
    d2 += __shfl_xor(d2, o, 64);
    qn += __shfl_xor(qn, o, 64);
  }
  if (lane == 0) {
    scale[i] = sc;
    // an upper bound in f32 (the f64 sum's own rounding is far below one ulp)
    const double d = sqrt(d2) * (1.0 + 1e-12);
    float df = (float)d;
    if ((double)df < d) df = nextafterf(df, INFINITY);
    delta[i] = isfinite(mx) ? df : INFINITY;
    qnorm[i] = qn;
  }
}

// Lower bounds on the distances from the chosen centres 0 .. chosen-1 to
// centre `chosen` (all rows of the points): f64 sums of the f32 coordinates'
// squared differences, four lanes per centre, rounded down to f32 after a
// relative margin far above the f64 rounding.
__global__ __launch_bounds__(256) void km_pp_cdist(const float* __restrict__ cents, int dim, int chosen,
                                                   float* __restrict__ dcc) {
  const int j = blockIdx.x * 64 + (threadIdx.x >> 2), part = threadIdx.x & 3;
  const bool on = j < chosen;
  const float* a = cents + (size_t)(on ? j : 0) * dim;
  const float* b = cents + (size_t)chosen * dim;
  double d = 0.0;
  for (int u = part; u < dim; u += 4) {
    const double x = (double)a[u] - (double)b[u];
    d += x * x;
  }
  d += __shfl_xor(d, 1, 64);
  d += __shfl_xor(d, 2, 64);
  if (on && part == 0) dcc[j] = __double2float_rd(sqrt(d) * (1.0 - 1e-12));
}

// near[i] is the chosen centre whose distance ns[i] holds. Before the
// int8 test, a point whose nearest centre a lies far from the new centre c
// keeps its distance without reading its codes: |p - c| >= |a - c| - |p - a|,
// with |p - a|^2 <= (ns + 1e-35) / (1 - gamma) from ns being the reference's
// sequential sum for a, and dcc[a] a lower bound on |a - c|; the same
// L^2 (1 - gamma) >= ns + 1e-35 test as the int8 bound then follows.
__global__ __launch_bounds__(256) void km_pp_round_q8(const float* __restrict__ P, int ldp, int n, int dim,
                                                      const int8_t* __restrict__ Q, int kq,
                                                      const float* __restrict__ scale,
                                                      const float* __restrict__ delta, const int* __restrict__ qnorm,
                                                      const int* __restrict__ picked, float* __restrict__ ns,
                                                      double* __restrict__ ps, int* __restrict__ pe,
                                                      double gamma, uint32_t* __restrict__ near,
                                                      const float* __restrict__ dcc, int chosen) {
  __shared__ int qc[KW_DMAX / 4];
  __shared__ float cs[KW_DMAX];
  __shared__ int list[Q8_ROWS];
  __shared__ int nlist;
  __shared__ SumCert sh[4];
  const int t = threadIdx.x;
  const int c = *picked;
  const int words = kq / 4;
  for (int j = t; j < words; j += 256) qc[j] = reinterpret_cast<const int*>(Q + (size_t)c * kq)[j];
  for (int j = t; j < dim; j += 256) cs[j] = P[(size_t)c * ldp + j];
  if (t == 0) nlist = 0;
  __syncthreads();
  const double sc = scale[c], dc = delta[c], qnc = (double)qnorm[c];
  const int i = blockIdx.x * Q8_ROWS + t;
  float cur = 0.0f;
  bool exact = false;
  bool far = false;
  if (i < n) {
    cur = ns[i];
    const double r = sqrt(((double)cur + 1e-35) / (1.0 - gamma)) * (1.0 + 1e-12);
    const double L0 = (double)dcc[near[i]] - r;
    far = isfinite(cur) && L0 > 0.0 && L0 * L0 * (1.0 - gamma) >= (double)cur + 1e-35;
  }
  if (i < n && !far) {
    int dot = 0;  // exact in any order: |dot| < 2^31 for kq <= KW_DMAX
    if ((kq & 15) == 0) {
      // 16-byte loads: the row's bytes in kq/16 loads instead of kq/4
      const int4* qv = reinterpret_cast<const int4*>(Q + (size_t)i * kq);
      for (int j = 0; j < words / 4; ++j) {
        const int4 v = qv[j];
        dot = __builtin_amdgcn_sdot4(v.x, qc[4 * j], dot, false);
        dot = __builtin_amdgcn_sdot4(v.y, qc[4 * j + 1], dot, false);
        dot = __builtin_amdgcn_sdot4(v.z, qc[4 * j + 2], dot, false);
        dot = __builtin_amdgcn_sdot4(v.w, qc[4 * j + 3], dot, false);
      }
    } else {
      const int* qv = reinterpret_cast<const int*>(Q + (size_t)i * kq);
      for (int j = 0; j < words; ++j) dot = __builtin_amdgcn_sdot4(qv[j], qc[j], dot, false);
    }
    const double sp = scale[i];
    const double A = sp * sp * (double)qnorm[i], B = sc * sc * qnc, C = sp * sc * (double)dot;
    const double e2 = A + B - 2.0 * C;
    const double err = 1e-13 * (A + B + 2.0 * fabs(C));
    const double e = sqrt(fmax(e2 - err, 0.0)) * (1.0 - 1e-13);
    const double L = e - (double)delta[i] - dc;
    const bool keep = isfinite(cur) && L > 0.0 && L * L * (1.0 - gamma) >= (double)cur + 1e-35;
    exact = !keep;
  }
  if (exact) list[atomicAdd(&nlist, 1)] = t;
  __syncthreads();
  __shared__ float nv_s[Q8_ROWS];
  nv_s[t] = cur;
  __syncthreads();
  const int m = nlist;
  for (int u = t; u < m; u += 256) {
    const int tt = list[u];
    const int ii = blockIdx.x * Q8_ROWS + tt;
    const float* row = P + (size_t)ii * ldp;
    float sum = 0.0f;
    for (int j = 0; j < dim; ++j) {
      const float d = row[j] - cs[j];
      sum += d * d;
    }
    if (sum < nv_s[tt]) nv_s[tt] = sum;
  }
  __syncthreads();
  const float nv = i < n ? nv_s[t] : 0.0f;
  if (i < n && nv != cur) {
    ns[i] = nv;
    near[i] = (uint32_t)chosen;
  }
  const SumCert r = block_cert_256(cert_of(nv), sh);
  if (t == 0) {
    ps[blockIdx.x] = r.s;
    pe[blockIdx.x] = r.e;
  }
}

// Inclusive prefix sum over a wave (shuffles, no LDS).
__device__ inline double wave_incl_scan_f64(double v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  return v;
}

// One 1024-thread block: the pick of one round and the copy of its row.
// status: 0 ok, 1 non-finite total (the round and all later ones stop).
// The prefix sums are wave scans joined through the 16 (or 4) wave totals:
// under the certificate every order gives the exact sums, and otherwise this
// is the fixed parallel order.
__device__ __forceinline__ void km_pp_pick_body(const float* __restrict__ P, int ldp, int n, int dim,
                                                   const float* __restrict__ ns, const double* __restrict__ ps,
                                                   const int* __restrict__ pe, int nb, ChaCha8* __restrict__ grng,
                                                   float* __restrict__ row_out, int* __restrict__ status,
                                                   int* __restrict__ inexact, int* __restrict__ picked_out) {
  __shared__ double wtot[16];
  __shared__ int wemin[16];
  __shared__ double s_pre;
  __shared__ float stage[4096];
  __shared__ __align__(8) unsigned char rng_mem[sizeof(ChaCha8)];
  ChaCha8& rng = *reinterpret_cast<ChaCha8*>(rng_mem);
  __shared__ double s_target;
  __shared__ int s_mode, s_pick, s_block;
  const int t = threadIdx.x;
  if (*status != 0) return;
  if (t == 0) rng = *grng;
  // each thread sums a contiguous run of block partials
  const int per = (nb + 1023) / 1024;
  const int b0 = min(nb, t * per), b1 = min(nb, (t + 1) * per);
  double ls = 0.0;
  int le = NO_TERMS;
  for (int b = b0; b < b1; ++b) {
    ls += ps[b];
    le = min(le, pe[b]);
  }
  // inclusive scan over the threads: wave scans, then the earlier waves'
  // totals in wave order
  const int lane = t & 63, wv = t >> 6;
  double incl = wave_incl_scan_f64(ls, lane);
  int wm = le;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) wm = min(wm, __shfl_xor(wm, o, 64));
  if (lane == 63) wtot[wv] = incl;
  if (lane == 0) wemin[wv] = wm;
  __syncthreads();
  double total = 0.0, wpre = 0.0;
  int emin = NO_TERMS;
  for (int q = 0; q < 16; ++q) {
    if (q == wv) wpre = total;
    total += wtot[q];
    emin = min(emin, wemin[q]);
  }
  incl += wpre;
  const double before = incl - ls;  // exact when the certificate holds
  // distances are >= 0, so the sum of |x| is the total itself
  const bool exact = sums_exact(total, emin);
  const bool sequential = !exact && n <= (int)SEQ_SUM_LIMIT;
  if (sequential) total = seq_sum_block(ns, n, stage);
  if (t == 0) {
    if (!(total <= 1.79769313486231570e308 && total >= 0.0)) {
      *status = 1;
      s_mode = -1;
    } else if (total <= 0.0) {
      s_pick = (int)rng.gen_range_usize((uint64_t)n);  // kmeans.rs:162-166
      s_mode = 0;
    } else {
      s_target = rng.gen_range_f64(0.0, total);
      s_mode = sequential ? 2 : 1;
      s_pick = n - 1;
      s_block = nb;
    }
    if (!exact && !sequential) atomicAdd(inexact, 1);
  }
  __syncthreads();
  const int mode = s_mode;
  if (mode < 0) return;
  const double target = s_target;
  if (mode == 2) {
    // the reference's cumulative scan, sequentially (kmeans.rs:169-176)
    double cum = 0.0;
    bool found = false;
    for (int c0 = 0; c0 < n; c0 += 4096) {
      const int m = min(4096, n - c0);
      __syncthreads();
      for (int u = t; u < m; u += 1024) stage[u] = ns[c0 + u];
      __syncthreads();
      if (t == 0 && !found)
        for (int u = 0; u < m; ++u) {
          cum += (double)stage[u];
          if (cum >= target) {
            s_pick = c0 + u;
            found = true;
            break;
          }
        }
    }
  } else if (mode == 1) {
    // first block whose inclusive prefix reaches the target, then the first
    // point inside it
    double run = before;
    for (int b = b0; b < b1; ++b) {
      if (run + ps[b] >= target) {
        atomicMin(&s_block, b);
        break;
      }
      run += ps[b];
    }
    __syncthreads();
    const int bb = s_block;
    if (bb < nb) {
      // prefix before block bb: recomputed by the owning thread's run
      if (b0 <= bb && bb < b1) {
        double pre = before;
        for (int b = b0; b < bb; ++b) pre += ps[b];
        s_pre = pre;
      }
      // the block's PP_ROWS points (the first PP_ROWS / 64 waves): wave
      // scans, then the earlier waves' totals; wtot is free after the scan
      // above (every thread read it before s_block was settled)
      static_assert(PP_ROWS % 64 == 0 && PP_ROWS <= 1024, "whole waves of points");
      const int i = bb * PP_ROWS + t;
      double inc2 = wave_incl_scan_f64((t < PP_ROWS && i < n) ? (double)ns[i] : 0.0, lane);
      if (lane == 63 && t < PP_ROWS) wtot[wv] = inc2;
      __syncthreads();
      const double pre = s_pre;
      for (int q = 0; q < wv && t < PP_ROWS; ++q) inc2 += wtot[q];
      if (t < PP_ROWS && i < n && pre + inc2 >= target) atomicMin(&s_pick, i);
    }
  }
  __syncthreads();
  const int picked = s_pick;
  for (int j = t; j < dim; j += 1024) row_out[j] = P[(size_t)picked * ldp + j];
  if (t == 0) {
    *grng = rng;
    if (picked_out) *picked_out = picked;
  }
}

__global__ __launch_bounds__(1024) void km_pp_pick(const float* __restrict__ P, int ldp, int n, int dim,
                                                   const float* __restrict__ ns, const double* __restrict__ ps,
                                                   const int* __restrict__ pe, int nb, ChaCha8* __restrict__ grng,
                                                   float* __restrict__ row_out, int* __restrict__ status,
                                                   int* __restrict__ inexact, int* __restrict__ picked_out) {
  km_pp_pick_body(P, ldp, n, dim, ns, ps, pe, nb, grng, row_out, status, inexact, picked_out);
}

__global__ void copy_row(const float* __restrict__ src, int ld_src, size_t row, int dim, float* __restrict__ dst) {
  for (int j = threadIdx.x; j < dim; j += blockDim.x) dst[j] = src[row * ld_src + j];
}

// copy_row with the row index read from device memory
__global__ void copy_row_at(const float* __restrict__ src, int ld_src, const long long* __restrict__ row, int dim,
                            float* __restrict__ dst) {
  const size_t r = (size_t)*row;
  for (int j = threadIdx.x; j < dim; j += blockDim.x) dst[j] = src[r * ld_src + j];
}

// a[i] = min(a[i], b[i]); out (if given) receives the result instead of a
__global__ void km_min_into(float* __restrict__ a, const float* __restrict__ b, int n, float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = fminf(a[i], b[i]);
  if (out)
    out[i] = v;
  else
    a[i] = v;
}

__global__ void km_fill(float* __restrict__ a, int n, float v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) a[i] = v;
}

// Returns the number of rounds whose pick used the fixed parallel order
// instead of the reference's sequential sums (0 whenever the certificate
// holds or n <= SEQ_SUM_LIMIT).
size_t kmeans_pp_device(const float* P, size_t n, int dim, int ldp, size_t k, ChaCha8& rng, float* cents,
                        hipStream_t s) {
  const int nb = (int)((n + PP_ROWS - 1) / PP_ROWS);
  DevBuf<float> ns(n);
  DevBuf<double> ps(nb);
  DevBuf<int> pe(nb), flags(2);
  DevBuf<ChaCha8> drng(1);
  const size_t first = rng.gen_range_usize(n);
  hipLaunchKernelGGL(copy_row, dim3(1), dim3(256), 0, s, P, ldp, first, dim, cents);
  PXG_HIP(hipMemcpyAsync(drng.p, &rng, sizeof(ChaCha8), hipMemcpyHostToDevice, s));
  PXG_HIP(hipMemsetAsync(flags.p, 0, 8, s));
  const int vec4 = (ldp % 4 == 0 && dim % 4 == 0 && ((uintptr_t)P & 15) == 0) ? 1 : 0;
  hipLaunchKernelGGL(km_pp_round, dim3(nb), dim3(256), 0, s, P, ldp, (int)n, dim, cents, ns.p, 1, ps.p, pe.p, vec4);
  PXG_HIP(hipGetLastError());
  // rounds after the first over the certified int8 copy (dim >= 32; for
  // narrower points the copy saves little of each row's bytes)
  const bool q8 = dim >= 32 && dim <= KW_DMAX && k > 1 && Q8_ROWS == PP_ROWS;
  const int kq = (dim + 3) / 4 * 4;
  DevBuf<int8_t> Q(q8 ? n * kq : 0);
  DevBuf<float> qscale(q8 ? n : 0), qdelta(q8 ? n : 0);
  DevBuf<int> qnorm(q8 ? n : 0), picked(1);
  DevBuf<uint32_t> near(q8 ? n : 0);  // every distance is to centre 0 so far
  DevBuf<float> dcc(q8 ? k : 0);
  if (q8) {
    PXG_HIP(hipMemsetAsync(near.p, 0, n * 4, s));
    hipLaunchKernelGGL(km_q8_prep, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, P, ldp, (int)n, dim, kq, Q.p,
                       qscale.p, qdelta.p, qnorm.p);
    PXG_HIP(hipGetLastError());
  }
  const double gamma = (double)(dim + 4) * 0x1p-24 * 1.01;
  for (size_t chosen = 1; chosen < k; ++chosen) {
    float* c = cents + chosen * dim;
    hipLaunchKernelGGL(km_pp_pick, dim3(1), dim3(1024), 0, s, P, ldp, (int)n, dim, ns.p, ps.p, pe.p, nb, drng.p, c,
                       flags.p, flags.p + 1, picked.p);
    if (chosen + 1 < k) {
      if (q8) {
        hipLaunchKernelGGL(km_pp_cdist, dim3((unsigned)((chosen + 63) / 64)), dim3(256), 0, s, (const float*)cents,
                           dim, (int)chosen, dcc.p);
        hipLaunchKernelGGL(km_pp_round_q8, dim3(nb), dim3(256), 0, s, P, ldp, (int)n, dim, (const int8_t*)Q.p, kq,
                           (const float*)qscale.p, (const float*)qdelta.p, (const int*)qnorm.p, (const int*)picked.p,
                           ns.p, ps.p, pe.p, gamma, near.p, (const float*)dcc.p, (int)chosen);
      } else
        hipLaunchKernelGGL(km_pp_round, dim3(nb), dim3(256), 0, s, P, ldp, (int)n, dim, c, ns.p, 0, ps.p, pe.p,
                           vec4);
    }
    PXG_HIP(hipGetLastError());
  }
  int h[2] = {0, 0};
  PXG_HIP(hipMemcpyAsync(&rng, drng.p, sizeof(ChaCha8), hipMemcpyDeviceToHost, s));
  PXG_HIP(hipMemcpyAsync(h, flags.p, 8, hipMemcpyDeviceToHost, s));
  PXG_HIP(hipStreamSynchronize(s));
  if (h[0] != 0)
    internal_error("kmeans++", "the sum of squared distances is not finite; coordinates are too large to square");
  return (size_t)h[1];
}

// ---------------------------------------------------------------------------
// update step
// ---------------------------------------------------------------------------
// Records changed assignments (kmeans.rs:93-96), counts members per cluster
// (a block histogram in LDS when k fits) and writes the identity permutation
// the radix sort carries along. 2048 points per block.
constexpr int KM_HIST = 8192;
__global__ __launch_bounds__(256) void km_changed_counts(const uint32_t* __restrict__ a, uint32_t* __restrict__ prev,
                                                         int n, int k, uint32_t* __restrict__ counts,
                                                         int* __restrict__ changed, uint32_t* __restrict__ idx) {
  __shared__ uint32_t hist[KM_HIST];
  __shared__ int any;
  const bool local = k <= KM_HIST;
  if (local)
    for (int c = threadIdx.x; c < k; c += 256) hist[c] = 0;
  if (threadIdx.x == 0) any = 0;
  __syncthreads();
  const int end = min(n, (int)(blockIdx.x + 1) * 2048);
  for (int i = blockIdx.x * 2048 + threadIdx.x; i < end; i += 256) {
    const uint32_t c = a[i];
    if (prev[i] != c) {
      any = 1;
      prev[i] = c;
    }
    if (local)
      atomicAdd(&hist[c], 1u);
    else
      atomicAdd(&counts[c], 1u);
    idx[i] = (uint32_t)i;
  }
  __syncthreads();
  if (local)
    for (int c = threadIdx.x; c < k; c += 256)
      if (hist[c]) atomicAdd(&counts[c], hist[c]);
  if (threadIdx.x == 0 && any) *changed = 1;
}

// Cluster means (kmeans.rs:104-135): one block per (cluster, JW-coordinate
// slice), 256/JW member groups. Each (cluster, coordinate) f64 sum carries
// the exactness certificate; where it fails for any coordinate of the slice,
// the block stages the members' values through LDS in point order and one
// thread per coordinate redoes the sum sequentially. The mean is
// (float)(sum * (1.0 / count)).
template <int JW, int NT>
__device__ __forceinline__ void km_sums_body(const float* __restrict__ P, int ldp, int dim,
                                               const uint32_t* __restrict__ members,
                                               const uint32_t* __restrict__ offsets,
                                               const uint32_t* __restrict__ counts, int k, float* __restrict__ newc, int bx, int by) {
  constexpr int G = NT / JW, ROWS = 2048 / JW;  // 8 KiB of staged values (the sequential redo)
  __shared__ double ss[G][JW], sa[G][JW];
  __shared__ int se[G][JW];
  __shared__ float stage[ROWS][JW];
  __shared__ int redo;
  const int c = bx;
  const int jl = threadIdx.x % JW, g = threadIdx.x / JW;
  const int j = by * JW + jl;
  const uint32_t cnt = counts[c];
  if (cnt == 0) return;
  const uint32_t off = offsets[c];
  double s = 0.0, a = 0.0;
  int e = NO_TERMS;
  // Under the certificate every order gives the same bits, so four members
  // are loaded at a time (four index loads, then four row loads in flight).
  auto add = [&](float x) {
    s += (double)x;
    a += (double)fabsf(x);
    if (x != 0.0f) e = min(e, ulp_exp(x));
  };
  if (j < dim) {
    uint32_t m = g;
    for (; m + 3 * G < cnt; m += 4 * G) {
      const uint32_t r0 = members[off + m], r1 = members[off + m + G], r2 = members[off + m + 2 * G],
                     r3 = members[off + m + 3 * G];
      const float x0 = P[(size_t)r0 * ldp + j], x1 = P[(size_t)r1 * ldp + j], x2 = P[(size_t)r2 * ldp + j],
                  x3 = P[(size_t)r3 * ldp + j];
      add(x0);
      add(x1);
      add(x2);
      add(x3);
    }
    for (; m < cnt; m += G) add(P[(size_t)members[off + m] * ldp + j]);
  }
  ss[g][jl] = s;
  sa[g][jl] = a;
  se[g][jl] = e;
  if (threadIdx.x == 0) redo = 0;
  __syncthreads();
  bool exact = true;
  if (g == 0 && j < dim) {
    for (int q = 1; q < G; ++q) {
      s += ss[q][jl];
      a += sa[q][jl];
      e = min(e, se[q][jl]);
    }
    exact = sums_exact(a, e);
    if (!exact) redo = 1;
  }
  __syncthreads();
  if (redo) {
    double q = 0.0;
    for (uint32_t m0 = 0; m0 < cnt; m0 += ROWS) {
      const uint32_t rows = min((uint32_t)ROWS, cnt - m0);
      __syncthreads();
      for (uint32_t r = g; r < rows; r += G) stage[r][jl] = j < dim ? P[(size_t)members[off + m0 + r] * ldp + j] : 0.0f;
      __syncthreads();
      if (g == 0 && !exact)
        for (uint32_t r = 0; r < rows; ++r) q += (double)stage[r][jl];
    }
    if (g == 0 && !exact) s = q;
  }
  if (g == 0 && j < dim) {
    const double inv = 1.0 / (double)cnt;
    newc[(size_t)c * dim + j] = (float)(s * inv);
  }
}

template <int JW, int NT>
__global__ __launch_bounds__(NT) void km_sums(const float* __restrict__ P, int ldp, int dim,
                                               const uint32_t* __restrict__ members,
                                               const uint32_t* __restrict__ offsets,
                                               const uint32_t* __restrict__ counts, int k, float* __restrict__ newc) {
  km_sums_body<JW, NT>(P, ldp, dim, members, offsets, counts, k, newc, blockIdx.x, blockIdx.y);
}

// farthest_point (kmeans.rs:215-226): the first point with the largest
// distance (strict >, starting from -1.0). Distances are >= 0 (sums of
// squares and minima of them; + 0.0 folds a -0.0 into +0.0, which compares
// equal), so that is the largest value and, among equal values, the smallest
// index: the largest key (value bits << 32 | ~index). Stage 1 gives one key
// per block over a contiguous range read coalesced, stage 2 the largest.
constexpr int KF_BLOCKS = 512;

__device__ inline unsigned long long block_max_u64_256(unsigned long long v, unsigned long long* sh) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long p = shfl_xor64(v, o);
    v = p > v ? p : v;
  }
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  unsigned long long r = sh[0];
  for (int i = 1; i < 4; ++i) r = sh[i] > r ? sh[i] : r;
  return r;
}

__global__ __launch_bounds__(256) void km_farthest_part(const float* __restrict__ dist, int n,
                                                        unsigned long long* __restrict__ part) {
  __shared__ unsigned long long sh[4];
  const int per = (n + KF_BLOCKS - 1) / KF_BLOCKS;
  const int lo = blockIdx.x * per, hi = min(n, lo + per);
  unsigned long long best = 0;  // below every point's key (~index is never 0)
  for (int i = lo + (int)threadIdx.x; i < hi; i += 256) {
    const unsigned long long key =
        ((unsigned long long)__float_as_uint(dist[i] + 0.0f) << 32) | (0xFFFFFFFFu - (uint32_t)i);
    best = key > best ? key : best;
  }
  best = block_max_u64_256(best, sh);
  if (threadIdx.x == 0) part[blockIdx.x] = best;
}

__global__ __launch_bounds__(256) void km_farthest_pick(const unsigned long long* __restrict__ part,
                                                        long long* __restrict__ out) {
  __shared__ unsigned long long sh[4];
  unsigned long long best = 0;
  for (int i = threadIdx.x; i < KF_BLOCKS; i += 256) best = part[i] > best ? part[i] : best;
  best = block_max_u64_256(best, sh);
  if (threadIdx.x == 0) *out = (long long)(0xFFFFFFFFu - (uint32_t)best);
}

static void launch_farthest(const float* dist, size_t n, unsigned long long* part, long long* out, hipStream_t s) {
  hipLaunchKernelGGL(km_farthest_part, dim3(KF_BLOCKS), dim3(256), 0, s, dist, (int)n, part);
  hipLaunchKernelGGL(km_farthest_pick, dim3(1), dim3(256), 0, s, (const unsigned long long*)part, out);
}

// ---------------------------------------------------------------------------
// Empty-cluster reseeds from a candidate pool
// ---------------------------------------------------------------------------
// At empty cluster E[i] the reference takes farthest_point over the array
// holding the new means (and the victims so far) below E[i] and the old rows
// from E[i] on (kmeans.rs:115-124). A point's own cluster w is not empty (the
// point is in it), so that array's row w is its old centroid if w > E[i] and
// its new mean if w < E[i], and the point's nearest distance there is at
// most ub_i = d_old or squared(p, new_w) accordingly; a NaN distance
// (overflow) counts as +inf, and a nearest distance is never NaN. Take as
// the pool the points of the largest ub_i and let theta be the largest ub_i
// outside it: every point outside has distance <= theta. So if the largest
// exact distance over the pool is above theta, the farthest point (the
// first index among equal distances) is in the pool, and is the pool's. Each
// empty cluster then costs a sort of the bounds and an exact scan of the
// pool instead of passes over every point; if the test fails at any empty
// cluster, the segment passes redo them all.
constexpr size_t RESEED_POOL = 8192;

// squared(p, new_w) per point (NaN as +inf): the reference's sequential sum,
// staged through LDS as in km_mfma_verify (rows 16-byte aligned, dim a
// multiple of 4).
__global__ __launch_bounds__(256) void km_reseed_bound(const float* __restrict__ P, int ldp, int n, int dim,
                                                       const float* __restrict__ newc,
                                                       const uint32_t* __restrict__ assign,
                                                       float* __restrict__ dnew) {
  __shared__ float tp[KV_PB * 33], tc[KV_PB * 33];
  __shared__ uint32_t sc[KV_PB];
  const int t = threadIdx.x, i0 = blockIdx.x * KV_PB, i = i0 + t;
  if (t < KV_PB) sc[t] = i < n ? assign[i] : 0u;
  float sum = 0.0f;
  for (int j0 = 0; j0 < dim; j0 += 32) {
    const int w = min(32, dim - j0);
    __syncthreads();
    for (int f = t; f < KV_PB * 8; f += 256) {
      const int r = f >> 3, c4 = (f & 7) * 4;
      if (c4 < w && i0 + r < n) {
        const float4 x = *reinterpret_cast<const float4*>(P + (size_t)(i0 + r) * ldp + j0 + c4);
        const float4 y = *reinterpret_cast<const float4*>(newc + (size_t)sc[r] * dim + j0 + c4);
        float* dp = tp + r * 33 + c4;
        float* dc = tc + r * 33 + c4;
        dp[0] = x.x; dp[1] = x.y; dp[2] = x.z; dp[3] = x.w;
        dc[0] = y.x; dc[1] = y.y; dc[2] = y.z; dc[3] = y.w;
      }
    }
    __syncthreads();
    if (t < KV_PB && i < n) {
      const float* a = tp + t * 33;
      const float* b = tc + t * 33;
      for (int jj = 0; jj < w; ++jj) {
        const float d = a[jj] - b[jj];
        sum += d * d;  // squared(), kmeans.rs:234-241
      }
    }
  }
  if (t < KV_PB && i < n) dnew[i] = sum == sum ? sum : INFINITY;
}

// ub_i per point as a descending sort key (~ its bits; ub_i >= 0), with the
// point's index as the value, for the empty cluster e.
__global__ __launch_bounds__(256) void km_reseed_keys(const uint32_t* __restrict__ assign,
                                                      const float* __restrict__ dold, const float* __restrict__ dnew,
                                                      int n, uint32_t e, uint32_t* __restrict__ key,
                                                      uint32_t* __restrict__ idx) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float ub = assign[i] > e ? dold[i] : dnew[i];
  key[i] = ~__float_as_uint(ub + 0.0f);
  idx[i] = (uint32_t)i;
}

// The pool's farthest point: the largest distance, then the smallest index
// (the largest key, as in km_farthest_part). *fail is set unless that
// distance is above theta = the largest ub outside the pool (theta_key holds
// its sort key; none when the pool holds every point).
__global__ __launch_bounds__(256) void km_pool_farthest(const uint32_t* __restrict__ rows,
                                                        const float* __restrict__ d, int m,
                                                        const uint32_t* __restrict__ theta_key, int force_fail,
                                                        long long* __restrict__ out, int* __restrict__ fail) {
  __shared__ unsigned long long sh[4];
  unsigned long long best = 0;
  for (int j = threadIdx.x; j < m; j += 256) {
    const unsigned long long key =
        ((unsigned long long)__float_as_uint(d[j] + 0.0f) << 32) | (0xFFFFFFFFu - rows[j]);
    best = key > best ? key : best;
  }
  best = block_max_u64_256(best, sh);
  if (threadIdx.x == 0) {
    *out = (long long)(0xFFFFFFFFu - (uint32_t)best);
    const float dmax = __uint_as_float((uint32_t)(best >> 32));
    if (force_fail || (theta_key && !(dmax > __uint_as_float(~*theta_key)))) *fail = 1;
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
  g_km = KmStats();
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
    out.inexact_sums += kmeans_pp_device(P, n, dim, ldp, k, *rng, cents.p, s);
  const double t_seeded = now_s();
  size_t empties = 0;
  std::string empties_per_it;

  DevBuf<uint32_t> assign(n), prev(n), counts(k), offsets(k), idx(n), keys_sorted(n), members(n);
  DevBuf<float> dist(n), newc(k * dim), work(k * dim);
  DevBuf<int> changed(1), pool_fail(1);
  DevBuf<long long> far(1);
  // the reseed pool's bounds, their sorted order, and the pool's exact scan
  DevBuf<uint32_t> rs_key, rs_skey, rs_idx, rs_rows, pool_a;
  DevBuf<float> rs_dnew, pool_d;
  size_t pool_reseeds = 0, pool_fallbacks = 0;
  // PXG_RESEED_POOL=size sets the pool size (0: no pool), so that small
  // inputs can take the pool path; PXG_RESEED_FAIL_AT=i fails the pool's test
  // at empty cluster i, so that the fallback runs after victims were placed
  // (test hooks; the results are the same either way)
  size_t pool = RESEED_POOL;
  if (const char* e = std::getenv("PXG_RESEED_POOL")) pool = (size_t)std::strtoull(e, nullptr, 10);
  const char* fail_env = std::getenv("PXG_RESEED_FAIL_AT");
  const long long fail_at = fail_env ? std::atoll(fail_env) : -1;
  const bool pool_fits = pool > 0 && n > 4 * pool && dim % 4 == 0 && dim <= KW_DMAX && ldp % 4 == 0 &&
                         ((uintptr_t)P & 15) == 0;
  DevBuf<unsigned long long> far_part(KF_BLOCKS);
  NearestWork nw;  // the points do not change during the run
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
    nearest_device(P, ldp, nullptr, n, dim, cents.p, dim, k, false, assign.p, dist.p, s, &nw);
    out.inertia = sums.total(dist.p, n, s);
    if (!sums.last_exact) ++out.inexact_sums;
    PXG_HIP(hipMemsetAsync(changed.p, 0, 4, s));
    PXG_HIP(hipMemsetAsync(counts.p, 0, k * 4, s));
    hipLaunchKernelGGL(km_changed_counts, dim3((unsigned)((n + 2047) / 2048)), dim3(256), 0, s, assign.p, prev.p,
                       (int)n, (int)k, counts.p, changed.p, idx.p);
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
    // more member groups per block when the clusters are few and large
    const bool wide = n >= 64 * k;
    if (dim <= 8 && wide)
      hipLaunchKernelGGL((km_sums<8, 1024>), dim3((unsigned)k, 1), dim3(1024), 0, s, P, ldp, dim, members.p,
                         offsets.p, counts.p, (int)k, newc.p);
    else if (dim <= 8)
      hipLaunchKernelGGL((km_sums<8, 256>), dim3((unsigned)k, 1), dim3(256), 0, s, P, ldp, dim, members.p, offsets.p,
                         counts.p, (int)k, newc.p);
    else if (dim <= 16)
      hipLaunchKernelGGL((km_sums<16, 256>), dim3((unsigned)k, 1), dim3(256), 0, s, P, ldp, dim, members.p,
                         offsets.p, counts.p, (int)k, newc.p);
    else
      hipLaunchKernelGGL((km_sums<32, 256>), dim3((unsigned)k, (unsigned)((dim + 31) / 32)), dim3(256), 0, s, P, ldp,
                         dim, members.p, offsets.p, counts.p, (int)k, newc.p);
    PXG_HIP(hipGetLastError());
    // empty clusters, ascending, against the partially updated array
    if (train_verbose()) {
      size_t e = 0;
      for (size_t c = 0; c < k; ++c) e += h_counts[c] == 0;
      empties_per_it += " " + std::to_string(e);
    }
    std::vector<size_t> E;
    for (size_t c = 0; c < k; ++c)
      if (h_counts[c] == 0) E.push_back(c);
    const size_t m = E.size();
    if (m >= 1 && pool_fits) {
      rs_key.reserve(n);
      rs_skey.reserve(n);
      rs_idx.reserve(n);
      rs_rows.reserve(n);
      rs_dnew.reserve(n);
      pool_a.reserve(pool);
      pool_d.reserve(pool);
      hipLaunchKernelGGL(km_reseed_bound, dim3((unsigned)((n + KV_PB - 1) / KV_PB)), dim3(256), 0, s, P, ldp, (int)n,
                         dim, (const float*)newc.p, (const uint32_t*)assign.p, rs_dnew.p);
      PXG_HIP(hipMemsetAsync(pool_fail.p, 0, 4, s));
      for (size_t ii = 0; ii < m; ++ii) {
        const size_t c = E[ii];
        hipLaunchKernelGGL(km_reseed_keys, gn, dim3(256), 0, s, (const uint32_t*)assign.p, (const float*)dist.p,
                           (const float*)rs_dnew.p, (int)n, (uint32_t)c, rs_key.p, rs_idx.p);
        PXG_HIP(hipcub::DeviceRadixSort::SortPairs(tmp.p, tmp_bytes, rs_key.p, rs_skey.p, rs_idx.p, rs_rows.p, (int)n,
                                                   0, 32, s));
        PXG_HIP(hipMemcpyAsync(work.p, newc.p, c * dim * 4, hipMemcpyDeviceToDevice, s));
        PXG_HIP(hipMemcpyAsync(work.p + c * dim, cents.p + c * dim, (k - c) * dim * 4, hipMemcpyDeviceToDevice, s));
        hipLaunchKernelGGL(km_exact_multi<false>, dim3((unsigned)((pool + KX_PB - 1) / KX_PB)), dim3(256),
                           (size_t)KX_PB * dim * 4, s, P, ldp, (const uint32_t*)rs_rows.p, (int)pool, dim,
                           (const float*)work.p, dim, (int)k, pool_a.p, pool_d.p);
        hipLaunchKernelGGL(km_pool_farthest, dim3(1), dim3(256), 0, s, (const uint32_t*)rs_rows.p,
                           (const float*)pool_d.p, (int)pool, (const uint32_t*)(rs_skey.p + pool),
                           (int)((long long)ii == fail_at), far.p, pool_fail.p);
        hipLaunchKernelGGL(copy_row_at, dim3(1), dim3(256), 0, s, P, ldp, (const long long*)far.p, dim,
                           newc.p + c * dim);
        PXG_HIP(hipGetLastError());
      }
      int h_fail = 0;
      PXG_HIP(hipMemcpyAsync(&h_fail, pool_fail.p, 4, hipMemcpyDeviceToHost, s));
      PXG_HIP(hipStreamSynchronize(s));
      if (h_fail) {
        ++pool_fallbacks;  // the passes below redo every empty cluster, victims included
      } else {
        empties += m;
        pool_reseeds += m;
        E.clear();
      }
    }
    if (E.size() >= 2 && m * n <= ((size_t)1 << 29)) {
      // Several empty clusters: the nearest distance of a point against the
      // array seen at empty cluster E[i] is min(L_i, R_i), L_i over the rows
      // below E[i] (new means and the victims chosen so far), R_i over the
      // old rows from E[i] on. R_i are suffix minima of exact per-segment
      // minima over the old rows; L_i grows by the new means between
      // consecutive empties and by each victim. Minima of exact distances
      // are exact, so each farthest point is the reference's.
      empties += m;
      const int nb = (int)((n + PP_ROWS - 1) / PP_ROWS);
      DevBuf<float> R(m * n), L(n), tmp(n);
      DevBuf<double> rps(nb);
      DevBuf<int> rpe(nb);
      const dim3 gm((unsigned)((n + 255) / 256));
      for (size_t ii = m; ii-- > 0;) {
        const size_t lo = E[ii], hi = ii + 1 < m ? E[ii + 1] : k;
        nearest_device(P, ldp, nullptr, n, dim, cents.p + lo * dim, dim, hi - lo, false, keys_sorted.p,
                       R.p + ii * n, s, &nw);
        if (ii + 1 < m)
          hipLaunchKernelGGL(km_min_into, gm, dim3(256), 0, s, R.p + ii * n, R.p + (ii + 1) * n, (int)n,
                             (float*)nullptr);
      }
      hipLaunchKernelGGL(km_fill, gm, dim3(256), 0, s, L.p, (int)n, INFINITY);
      const int vec4 = (ldp % 4 == 0 && dim % 4 == 0 && ((uintptr_t)P & 15) == 0) ? 1 : 0;
      for (size_t ii = 0; ii < m; ++ii) {
        const size_t lo = ii == 0 ? 0 : E[ii - 1] + 1, hi = E[ii];
        if (hi > lo) {
          nearest_device(P, ldp, nullptr, n, dim, newc.p + lo * dim, dim, hi - lo, false, keys_sorted.p, tmp.p, s,
                         &nw);
          hipLaunchKernelGGL(km_min_into, gm, dim3(256), 0, s, L.p, tmp.p, (int)n, (float*)nullptr);
        }
        hipLaunchKernelGGL(km_min_into, gm, dim3(256), 0, s, L.p, R.p + ii * n, (int)n, tmp.p);
        launch_farthest(tmp.p, n, far_part.p, far.p, s);
        hipLaunchKernelGGL(copy_row_at, dim3(1), dim3(256), 0, s, P, ldp, far.p, dim, newc.p + E[ii] * dim);
        if (ii + 1 < m)
          hipLaunchKernelGGL(km_pp_round, dim3(nb), dim3(256), 0, s, P, ldp, (int)n, dim, newc.p + E[ii] * dim, L.p,
                             0, rps.p, rpe.p, vec4);
        PXG_HIP(hipGetLastError());
      }
      E.clear();
    }
    for (size_t c : E) {
      ++empties;
      PXG_HIP(hipMemcpyAsync(work.p, newc.p, c * dim * 4, hipMemcpyDeviceToDevice, s));
      PXG_HIP(hipMemcpyAsync(work.p + c * dim, cents.p + c * dim, (k - c) * dim * 4, hipMemcpyDeviceToDevice, s));
      nearest_device(P, ldp, nullptr, n, dim, work.p, dim, k, false, keys_sorted.p, dist.p, s, &nw);
      launch_farthest(dist.p, n, far_part.p, far.p, s);
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
  g_km.inexact_sums = out.inexact_sums;
  g_km.reseeds = empties;
  g_km.pool_reseeds = pool_reseeds;
  g_km.pool_fallbacks = pool_fallbacks;
  if (train_verbose())
    std::fprintf(stderr,
                 "[pxg kmeans] n=%zu dim=%d k=%zu: seeding %.3fs, lloyd %zu it %.3fs, %zu empty reseeds (%zu from the "
                 "pool, %zu pool fallbacks), %zu points rescanned exactly in the last assignment; empties per "
                 "iteration:%s\n",
                 n, dim, k, t_seeded - t_start, out.iterations, now_s() - t_seeded, empties, pool_reseeds,
                 pool_fallbacks, g_last_redo,
                 empties_per_it.c_str());
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

// ---------------------------------------------------------------------------
// Product-quantizer training, every subspace in one launch per step
// ---------------------------------------------------------------------------
// ProductQuantizer::train (product.rs:198-296) runs kmeans on each subspace
// in turn with one generator advanced across them. Only the k-means++
// seedings draw from it (kmeans.rs:146-194; Lloyd and the farthest-point
// reseeds draw nothing), and in the common case a seeding's draws do not
// depend on the data: one gen_range over the points, then one 64-bit word
// per further centroid (gen_range_f64 accepts its first word unless the
// product rounds up to the total; only a zero total takes a gen_range
// instead). So the host predicts each subspace's starting state, and every
// step below covers all subspaces in one launch from one host thread:
// blockIdx.y (blockIdx.x for the one-block kernels) names the subspace, and
// each subspace's kernels are the single-run kernels' bodies over its own
// arrays. After the seedings each subspace's final generator state is
// compared with the next one's predicted start; from the first that differs,
// the later subspaces are trained again in order from the true state by the
// single-run path, so every codebook is the sequential run's. Empty clusters
// (rare) are reseeded per subspace with the single-run farthest-point pass.

// One subspace of a batched training: its projected points (n x w, row
// stride w) and its working arrays.
struct PqSub {
  const float* P;
  float* cents;       // k x w, the centroid array (updated in place per iteration)
  float* newc;        // k x w, the next iteration's array while it is built
  float* ns;          // n: k-means++ nearest squared distances
  double* ps;         // k-means++ per-block sums and exponents
  int* pe;
  ChaCha8* rng;       // the subspace's generator
  uint32_t* assign;   // n
  uint32_t* prev;     // n: the previous assignment (kmeans.rs:93-96)
  float* dist;        // n: the assignment's distances
  uint32_t* counts;   // k
  uint32_t* offsets;  // k: each cluster's first member in the shared member array
  double* fps;        // per-256-point certificates of dist (the inertia)
  double* fpa;
  int* fpe;
  double* total;      // [2]: inertia, 1.0 when it equals the sequential sum
  int* flags;         // [0] non-finite k-means++ total, [1] inexact picks, [2] assignment changed
  // the certified matrix-core assignment (narrow equal widths)
  float* pn;          // n: the points' squared norms
  float* cn;          // k: the centroids' squared norms
  float* cmax;        // [1]: the largest of them
  uint32_t* bidx;     // n: the approximate pass's best centroid
  float* best;        // n: its approximate score
  float* second;      // n: the second-best approximate score
  uint32_t* redo;     // n: the points the certificate leaves to the exact scan
  int* nredo;         // [1]
  int w;
  int active;         // still iterating
};

__global__ void pqb_first(const PqSub* __restrict__ S, const uint64_t* __restrict__ first) {
  const PqSub& q = S[blockIdx.x];
  for (int j = threadIdx.x; j < q.w; j += blockDim.x) q.cents[j] = q.P[first[blockIdx.x] * q.w + j];
}

__global__ __launch_bounds__(256) void pqb_pp_round(const PqSub* __restrict__ S, int n, int chosen, int init,
                                                    int vec4) {
  const PqSub& q = S[blockIdx.y];
  km_pp_round_body(q.P, q.w, n, q.w, q.cents + (size_t)chosen * q.w, q.ns, init, q.ps, q.pe, vec4, blockIdx.x);
}

// The same round for narrow equal-width subspaces (W a multiple of 4, rows
// 16-byte aligned): one thread per point reads its row straight into
// registers (the centre row is uniform over the block), so a wave's loads
// cover 64 consecutive rows.
template <int W>
__global__ __launch_bounds__(256) void pqb_pp_round_w(const PqSub* __restrict__ S, int n, int chosen, int init) {
  __shared__ SumCert sh[4];
  const PqSub& q = S[blockIdx.y];
  const int i = blockIdx.x * PP_ROWS + threadIdx.x;
  const float* c = q.cents + (size_t)chosen * W;
  float nv = 0.0f;
  if (i < n) {
    const float4* pr = reinterpret_cast<const float4*>(q.P + (size_t)i * W);
    float x[W];
#pragma unroll
    for (int u = 0; u < W / 4; ++u) {
      const float4 v = pr[u];
      x[4 * u] = v.x;
      x[4 * u + 1] = v.y;
      x[4 * u + 2] = v.z;
      x[4 * u + 3] = v.w;
    }
    float sum = 0.0f;  // squared(), kmeans.rs:234-241
#pragma unroll
    for (int j = 0; j < W; ++j) {
      const float d = x[j] - c[j];
      sum += d * d;
    }
    nv = sum;
    if (!init) {
      const float cur = q.ns[i];
      if (!(sum < cur)) nv = cur;
    }
    q.ns[i] = nv;
  }
  const SumCert r = block_cert_256(cert_of(nv), sh);
  if (threadIdx.x == 0) {
    q.ps[blockIdx.x] = r.s;
    q.pe[blockIdx.x] = r.e;
  }
}

__global__ __launch_bounds__(1024) void pqb_pp_pick(const PqSub* __restrict__ S, int n, int nb, int chosen) {
  const PqSub& q = S[blockIdx.x];
  km_pp_pick_body(q.P, q.w, n, q.w, q.ns, q.ps, q.pe, nb, q.rng, q.cents + (size_t)chosen * q.w, q.flags,
                  q.flags + 1, nullptr);
}

// The certified matrix-core assignment of every subspace at once: the
// single-run pass's kernels (km_row_norms, the centroid norms and their
// largest, km_mfma_small, km_mfma_verify) over each subspace's arrays. The
// points the certificate leaves go to the exact scan per subspace.
__global__ __launch_bounds__(256) void pqb_point_norms(const PqSub* __restrict__ S, int n) {
  const PqSub& q = S[blockIdx.y];
  km_row_norms_body(q.P, q.w, nullptr, n, q.w, q.pn, blockIdx.x);
}

// cn[c] = |c|^2 and cmax = the largest (NaN if any is NaN), per active subspace
__global__ __launch_bounds__(256) void pqb_cent_norms(const PqSub* __restrict__ S, int k) {
  __shared__ float sh[256];
  const PqSub& q = S[blockIdx.x];
  if (!q.active) return;  // uniform over the block
  float m = 0.0f;
  for (int c = threadIdx.x; c < k; c += 256) {
    const float* cr = q.cents + (size_t)c * q.w;
    float v = 0.0f;
    for (int j = 0; j < q.w; ++j) v += cr[j] * cr[j];
    q.cn[c] = v;
    m = v > m || v != v ? v : m;  // a NaN, once taken, stays
  }
  sh[threadIdx.x] = m;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) {
      const float x = sh[threadIdx.x + o];
      if (x > sh[threadIdx.x] || x != x) sh[threadIdx.x] = x;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) q.cmax[0] = sh[0];
}

template <int DS>
__global__ __launch_bounds__(256, 2) void pqb_mfma_small(const PqSub* __restrict__ S, int n, int k) {
  extern __shared__ float4 ks_sm[];
  const PqSub& q = S[blockIdx.y];
  if (!q.active) return;
  km_mfma_small_body<DS>(q.P, q.w, nullptr, n, q.cents, q.w, k, q.cn, q.bidx, q.best, q.second,
                         reinterpret_cast<float*>(ks_sm), blockIdx.x);
}

__global__ __launch_bounds__(256) void pqb_verify(const PqSub* __restrict__ S, int n) {
  const PqSub& q = S[blockIdx.y];
  if (!q.active) return;
  km_mfma_verify_body<false>(q.P, q.w, nullptr, n, q.w, q.cents, q.w, q.pn, q.cmax, q.bidx, q.best, q.second,
                             q.assign, q.dist, q.redo, q.nredo, blockIdx.x);
}

template <int D>
__global__ __launch_bounds__(256) void pqb_assign(const PqSub* __restrict__ S, int n, int k, int vec4) {
  const PqSub& q = S[blockIdx.y];
  if (!q.active) return;  // uniform over the block
  km_assign_body<D, false>(q.P, q.w, nullptr, n, q.w, q.cents, q.w, k, q.assign, q.dist, vec4, blockIdx.x);
}

__global__ __launch_bounds__(256) void pqb_partials(const PqSub* __restrict__ S, int n) {
  const PqSub& q = S[blockIdx.y];
  if (!q.active) return;
  f64_partials_body(q.dist, n, q.fps, q.fpa, q.fpe, blockIdx.x);
}

__global__ __launch_bounds__(1024) void pqb_total(const PqSub* __restrict__ S, int n, int nb) {
  const PqSub& q = S[blockIdx.x];
  if (!q.active) return;
  f64_total_body(q.dist, n, q.fps, q.fpa, q.fpe, nb, q.total);
}

// km_changed_counts per subspace, plus the sort keys (subspace, cluster) and
// point indices of the shared member sort: 2048 points per block.
__global__ __launch_bounds__(256) void pqb_changed_counts(const PqSub* __restrict__ S, int n, int k,
                                                          uint32_t* __restrict__ keys, uint32_t* __restrict__ vals) {
  __shared__ uint32_t hist[256];
  __shared__ int any;
  const int sub = blockIdx.y;
  const PqSub& q = S[sub];
  const size_t base = (size_t)sub * n;
  const bool active = q.active;
  for (int c = threadIdx.x; c < k; c += 256) hist[c] = 0;
  if (threadIdx.x == 0) any = 0;
  __syncthreads();
  const int end = min(n, (int)(blockIdx.x + 1) * 2048);
  for (int i = blockIdx.x * 2048 + threadIdx.x; i < end; i += 256) {
    const uint32_t c = active ? q.assign[i] : 0u;
    if (active) {
      if (q.prev[i] != c) {
        any = 1;
        q.prev[i] = c;
      }
      atomicAdd(&hist[c], 1u);
    }
    keys[base + i] = (uint32_t)sub * (uint32_t)k + c;
    vals[base + i] = (uint32_t)i;
  }
  __syncthreads();
  if (!active) return;
  for (int c = threadIdx.x; c < k; c += 256)
    if (hist[c]) atomicAdd(&q.counts[c], hist[c]);
  if (threadIdx.x == 0 && any) q.flags[2] = 1;
}

template <int JW, int NT>
__global__ __launch_bounds__(NT) void pqb_sums(const PqSub* __restrict__ S, int k,
                                               const uint32_t* __restrict__ members) {
  const PqSub& q = S[blockIdx.y];
  if (!q.active) return;
  km_sums_body<JW, NT>(q.P, q.w, q.w, members, q.offsets, q.counts, k, q.newc, blockIdx.x, 0);
}

__global__ void pqb_reset_changed(const PqSub* __restrict__ S, int M) {
  for (int q = threadIdx.x; q < M; q += blockDim.x) S[q].flags[2] = 0;
}

// newc = cents before the means are written: the rows of empty clusters are
// replaced by the reseeds
__global__ void pqb_stage(const PqSub* __restrict__ S, int k) {
  const PqSub& q = S[blockIdx.x];
  if (!q.active) return;
  for (int t = threadIdx.x; t < k * q.w; t += blockDim.x) q.newc[t] = q.cents[t];
}

__global__ void pqb_commit(const PqSub* __restrict__ S, int k) {
  const PqSub& q = S[blockIdx.x];
  if (!q.active) return;
  for (int t = threadIdx.x; t < k * q.w; t += blockDim.x) q.cents[t] = q.newc[t];
}

// Every subspace at once; widths up to 32. Writes each subspace's k x w
// centroids to cents[sidx] and its result to res[sidx]; returns the index of
// the first subspace whose seeding's draws differed from the prediction (M
// when none did): that subspace's results stand, the later ones must be
// trained again from `next` (its final generator state).
static int pq_train_batched(const std::vector<DevBuf<float>>& proj, size_t n, const PqLayout& L, size_t k,
                            size_t max_iter, const std::vector<ChaCha8>& start, std::vector<DevBuf<float>>& cents,
                            std::vector<KmeansOut>& res, ChaCha8* next, hipStream_t s) {
  const int M = L.M;
  const int nb = (int)((n + PP_ROWS - 1) / PP_ROWS), nb256 = (int)((n + 255) / 256);
  std::vector<PqSub> h(M);
  DevBuf<float> ns((size_t)M * n), dist((size_t)M * n), newc_all;
  DevBuf<uint32_t> assign((size_t)M * n), prev((size_t)M * n), counts((size_t)M * k), offsets((size_t)M * k);
  DevBuf<uint32_t> keys((size_t)M * n), keys_sorted((size_t)M * n), vals((size_t)M * n), members((size_t)M * n);
  DevBuf<double> ps((size_t)M * nb), fps((size_t)M * nb256), fpa((size_t)M * nb256), total((size_t)M * 2);
  DevBuf<int> pe((size_t)M * nb), fpe((size_t)M * nb256), flags((size_t)M * 4);
  DevBuf<ChaCha8> drng(M);
  DevBuf<uint64_t> dfirst(M);
  DevBuf<PqSub> dS(M);
  // the matrix-core assignment: narrow equal widths with enough points
  const int w0 = L.width[0];
  size_t cofs_total = 0;
  std::vector<size_t> cofs(M);
  for (int q = 0; q < M; ++q) {
    cofs[q] = cofs_total;
    cofs_total += k * L.width[q];
  }
  newc_all.reserve(cofs_total);
  std::vector<ChaCha8> rng(start);
  std::vector<uint64_t> first(M);
  bool vec4 = true, equal = true;
  for (int q = 0; q < M; ++q) {
    const int w = L.width[q];
    cents[q].reserve(k * w);
    first[q] = rng[q].gen_range_usize(n);  // kmeans.rs:150
    PqSub& t = h[q];
    t.P = proj[q].p;
    t.cents = cents[q].p;
    t.newc = newc_all.p + cofs[q];
    t.ns = ns.p + (size_t)q * n;
    t.ps = ps.p + (size_t)q * nb;
    t.pe = pe.p + (size_t)q * nb;
    t.rng = drng.p + q;
    t.assign = assign.p + (size_t)q * n;
    t.prev = prev.p + (size_t)q * n;
    t.dist = dist.p + (size_t)q * n;
    t.counts = counts.p + (size_t)q * k;
    t.offsets = offsets.p + (size_t)q * k;
    t.fps = fps.p + (size_t)q * nb256;
    t.fpa = fpa.p + (size_t)q * nb256;
    t.fpe = fpe.p + (size_t)q * nb256;
    t.total = total.p + (size_t)q * 2;
    t.flags = flags.p + (size_t)q * 4;
    t.w = w;
    t.active = 1;
    vec4 = vec4 && w % 4 == 0 && ((uintptr_t)proj[q].p & 15) == 0;
    equal = equal && w == L.width[0];
  }
  const bool mfma = vec4 && equal && (w0 == 8 || w0 == 16 || w0 == 24) && k >= 64 && k * (size_t)w0 <= KS_MAXF &&
                    n >= 4096;
  DevBuf<float> pn, cn, cmax, best, second;
  DevBuf<uint32_t> bidx, redo, ra;
  DevBuf<float> rd;
  DevBuf<int> nredo;
  if (mfma) {
    pn.reserve((size_t)M * n);
    cn.reserve((size_t)M * k);
    cmax.reserve(M);
    bidx.reserve((size_t)M * n);
    best.reserve((size_t)M * n);
    second.reserve((size_t)M * n);
    redo.reserve((size_t)M * n);
    nredo.reserve(M);
    for (int q = 0; q < M; ++q) {
      PqSub& t = h[q];
      t.pn = pn.p + (size_t)q * n;
      t.cn = cn.p + (size_t)q * k;
      t.cmax = cmax.p + q;
      t.bidx = bidx.p + (size_t)q * n;
      t.best = best.p + (size_t)q * n;
      t.second = second.p + (size_t)q * n;
      t.redo = redo.p + (size_t)q * n;
      t.nredo = nredo.p + q;
    }
  }
  PXG_HIP(hipMemcpyAsync(dS.p, h.data(), M * sizeof(PqSub), hipMemcpyHostToDevice, s));
  PXG_HIP(hipMemcpyAsync(drng.p, rng.data(), M * sizeof(ChaCha8), hipMemcpyHostToDevice, s));
  PXG_HIP(hipMemcpyAsync(dfirst.p, first.data(), M * 8, hipMemcpyHostToDevice, s));
  PXG_HIP(hipMemsetAsync(flags.p, 0, (size_t)M * 16, s));
  PXG_HIP(hipMemsetAsync(prev.p, 0, (size_t)M * n * 4, s));  // kmeans.rs:88: every point starts in cluster 0
  // k-means++, all subspaces a round at a time
  auto round = [&](int chosen, int init) {
    const dim3 g(nb, M);
    if (vec4 && equal && w0 == 8)
      hipLaunchKernelGGL(pqb_pp_round_w<8>, g, dim3(256), 0, s, (const PqSub*)dS.p, (int)n, chosen, init);
    else if (vec4 && equal && w0 == 4)
      hipLaunchKernelGGL(pqb_pp_round_w<4>, g, dim3(256), 0, s, (const PqSub*)dS.p, (int)n, chosen, init);
    else if (vec4 && equal && w0 == 16)
      hipLaunchKernelGGL(pqb_pp_round_w<16>, g, dim3(256), 0, s, (const PqSub*)dS.p, (int)n, chosen, init);
    else
      hipLaunchKernelGGL(pqb_pp_round, g, dim3(256), 0, s, (const PqSub*)dS.p, (int)n, chosen, init, vec4 ? 1 : 0);
  };
  hipLaunchKernelGGL(pqb_first, dim3(M), dim3(64), 0, s, (const PqSub*)dS.p, (const uint64_t*)dfirst.p);
  round(0, 1);
  for (size_t chosen = 1; chosen < k; ++chosen) {
    hipLaunchKernelGGL(pqb_pp_pick, dim3(M), dim3(1024), 0, s, (const PqSub*)dS.p, (int)n, nb, (int)chosen);
    if (chosen + 1 < k) round((int)chosen, 0);
  }
  PXG_HIP(hipGetLastError());
  std::vector<int> hf((size_t)M * 4);
  PXG_HIP(hipMemcpyAsync(rng.data(), drng.p, M * sizeof(ChaCha8), hipMemcpyDeviceToHost, s));
  PXG_HIP(hipMemcpyAsync(hf.data(), flags.p, (size_t)M * 16, hipMemcpyDeviceToHost, s));
  PXG_HIP(hipStreamSynchronize(s));
  for (int q = 0; q < M; ++q)
    if (hf[(size_t)q * 4] != 0)
      internal_error("kmeans++", "the sum of squared distances is not finite; coordinates are too large to square");
  // the stream position (32-bit words drawn) of a generator state
  auto pos = [](const ChaCha8& r) { return r.counter * 16 - (uint64_t)(64 - r.index); };
  // PXG_PQ_REDO_AFTER=i takes the in-order path after subspace i as if its
  // draws had differed (a test of that path; the results are the same)
  const char* force = std::getenv("PXG_PQ_REDO_AFTER");
  const int forced = force ? std::atoi(force) : -1;
  int redo_from = M;
  for (int q = 0; q + 1 < M; ++q)
    if (q == forced || pos(rng[q]) != pos(start[q + 1])) {
      redo_from = q + 1;
      *next = rng[q];
      break;
    }
  const int Mb = redo_from;  // subspaces whose seeding stands
  for (int q = Mb; q < M; ++q) h[q].active = 0;
  for (int q = 0; q < Mb; ++q) {
    res[q] = KmeansOut();
    res[q].k = k;
    res[q].inexact_sums = (size_t)hf[(size_t)q * 4 + 1];
  }
  // Lloyd (kmeans.rs:85-136), the active subspaces a step at a time
  int bits = 1;
  while ((1ull << bits) < (uint64_t)M * k) ++bits;
  size_t tmp_bytes = 0;
  PXG_HIP(hipcub::DeviceRadixSort::SortPairs(nullptr, tmp_bytes, keys.p, keys_sorted.p, vals.p, members.p,
                                             (int)((size_t)M * n), 0, bits, s));
  DevBuf<unsigned char> tmp(tmp_bytes + 16);
  std::vector<uint32_t> hc((size_t)M * k), ho((size_t)M * k);
  std::vector<double> ht((size_t)M * 2);
  // the single-run reseed pass's buffers (empty clusters)
  DevBuf<float> work, rdist;
  DevBuf<uint32_t> rassign;
  DevBuf<unsigned long long> far_part(KF_BLOCKS);
  DevBuf<long long> far(1);
  const dim3 gn((unsigned)((n + 255) / 256), (unsigned)M);
  if (mfma)
    hipLaunchKernelGGL(pqb_point_norms, dim3((unsigned)((n + 31) / 32), (unsigned)M), dim3(256), 0, s,
                       (const PqSub*)dS.p, (int)n);
  std::vector<int> hredo(M);
  for (size_t it = 0; it < max_iter; ++it) {
    int live = 0;
    for (int q = 0; q < Mb; ++q) live += h[q].active;
    if (!live) break;
    PXG_HIP(hipMemcpyAsync(dS.p, h.data(), M * sizeof(PqSub), hipMemcpyHostToDevice, s));
    for (int q = 0; q < Mb; ++q)
      if (h[q].active) res[q].iterations = it + 1;
    // assignment: the sequential squared, strict < (kmeans.rs:200-212)
    const int v4 = vec4 ? 1 : 0;
    if (mfma) {
      // the certified approximation, then the exact scan of the points it
      // leaves (nearest_device's steps, every subspace at once)
      hipLaunchKernelGGL(pqb_cent_norms, dim3(M), dim3(256), 0, s, (const PqSub*)dS.p, (int)k);
      PXG_HIP(hipMemsetAsync(nredo.p, 0, (size_t)M * 4, s));
      const dim3 gs((unsigned)((n + 4 * KS_PW * 32 - 1) / (4 * KS_PW * 32)), (unsigned)M);
      const size_t lds = (k * w0 + ((k + 31) & ~(size_t)31)) * 4;
      if (w0 == 8)
        hipLaunchKernelGGL(pqb_mfma_small<1>, gs, dim3(256), lds, s, (const PqSub*)dS.p, (int)n, (int)k);
      else if (w0 == 16)
        hipLaunchKernelGGL(pqb_mfma_small<2>, gs, dim3(256), lds, s, (const PqSub*)dS.p, (int)n, (int)k);
      else
        hipLaunchKernelGGL(pqb_mfma_small<3>, gs, dim3(256), lds, s, (const PqSub*)dS.p, (int)n, (int)k);
      hipLaunchKernelGGL(pqb_verify, dim3((unsigned)((n + KV_PB - 1) / KV_PB), (unsigned)M), dim3(256), 0, s,
                         (const PqSub*)dS.p, (int)n);
      PXG_HIP(hipGetLastError());
      PXG_HIP(hipMemcpyAsync(hredo.data(), nredo.p, (size_t)M * 4, hipMemcpyDeviceToHost, s));
      PXG_HIP(hipStreamSynchronize(s));
      int mmax = 0;
      for (int q = 0; q < Mb; ++q)
        if (h[q].active) mmax = std::max(mmax, hredo[q]);
      ra.reserve(mmax);  // the stream is idle here (synchronized above)
      rd.reserve(mmax);
      for (int q = 0; q < Mb; ++q) {
        const int m = hredo[q];
        if (!h[q].active || m == 0) continue;
        const dim3 gx((unsigned)((m + KX_PB - 1) / KX_PB));
        hipLaunchKernelGGL(km_exact_multi<false>, gx, dim3(256), (size_t)KX_PB * w0 * 4, s, h[q].P, w0,
                           (const uint32_t*)h[q].redo, m, w0, (const float*)h[q].cents, w0, (int)k, ra.p, rd.p);
        hipLaunchKernelGGL(km_scatter_redo, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s,
                           (const uint32_t*)h[q].redo, m, (const uint32_t*)ra.p, (const float*)rd.p, h[q].assign,
                           h[q].dist);
        PXG_HIP(hipGetLastError());
      }
    } else if (equal && L.width[0] == 8)
      hipLaunchKernelGGL(pqb_assign<8>, gn, dim3(256), 0, s, (const PqSub*)dS.p, (int)n, (int)k, v4);
    else if (equal && L.width[0] == 16)
      hipLaunchKernelGGL(pqb_assign<16>, gn, dim3(256), 0, s, (const PqSub*)dS.p, (int)n, (int)k, v4);
    else if (equal && L.width[0] == 4)
      hipLaunchKernelGGL(pqb_assign<4>, gn, dim3(256), 0, s, (const PqSub*)dS.p, (int)n, (int)k, v4);
    else if (equal && L.width[0] == 2)
      hipLaunchKernelGGL(pqb_assign<2>, gn, dim3(256), 0, s, (const PqSub*)dS.p, (int)n, (int)k, v4);
    else if (equal && L.width[0] == 1)
      hipLaunchKernelGGL(pqb_assign<1>, gn, dim3(256), 0, s, (const PqSub*)dS.p, (int)n, (int)k, v4);
    else if (equal && L.width[0] == 32)
      hipLaunchKernelGGL(pqb_assign<32>, gn, dim3(256), 0, s, (const PqSub*)dS.p, (int)n, (int)k, v4);
    else
      hipLaunchKernelGGL(pqb_assign<0>, gn, dim3(256), 0, s, (const PqSub*)dS.p, (int)n, (int)k, 0);
    // inertia: the f64 sum of the distances in point order (certified)
    hipLaunchKernelGGL(pqb_partials, dim3(nb256, M), dim3(256), 0, s, (const PqSub*)dS.p, (int)n);
    hipLaunchKernelGGL(pqb_total, dim3(M), dim3(1024), 0, s, (const PqSub*)dS.p, (int)n, nb256);
    PXG_HIP(hipMemsetAsync(counts.p, 0, (size_t)M * k * 4, s));
    hipLaunchKernelGGL(pqb_reset_changed, dim3(1), dim3(256), 0, s, (const PqSub*)dS.p, M);
    hipLaunchKernelGGL(pqb_changed_counts, dim3((unsigned)((n + 2047) / 2048), M), dim3(256), 0, s,
                       (const PqSub*)dS.p, (int)n, (int)k, keys.p, vals.p);
    PXG_HIP(hipGetLastError());
    PXG_HIP(hipMemcpyAsync(hc.data(), counts.p, (size_t)M * k * 4, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipMemcpyAsync(ht.data(), total.p, (size_t)M * 16, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipMemcpyAsync(hf.data(), flags.p, (size_t)M * 16, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    for (int q = 0; q < Mb; ++q) {
      if (!h[q].active) continue;
      res[q].inertia = ht[(size_t)q * 2];
      if (ht[(size_t)q * 2 + 1] == 0.0) ++res[q].inexact_sums;
      if (hf[(size_t)q * 4 + 2] == 0 && it > 0) h[q].active = 0;  // kmeans.rs:99-102
    }
    live = 0;
    for (int q = 0; q < Mb; ++q) live += h[q].active;
    if (!live) break;
    PXG_HIP(hipMemcpyAsync(dS.p, h.data(), M * sizeof(PqSub), hipMemcpyHostToDevice, s));
    // members of each (subspace, cluster) in point order: a stable sort
    PXG_HIP(hipcub::DeviceRadixSort::SortPairs(tmp.p, tmp_bytes, keys.p, keys_sorted.p, vals.p, members.p,
                                               (int)((size_t)M * n), 0, bits, s));
    for (int q = 0; q < M; ++q) {
      uint32_t acc = (uint32_t)((size_t)q * n);
      for (size_t c = 0; c < k; ++c) {
        ho[(size_t)q * k + c] = acc;
        acc += hc[(size_t)q * k + c];
      }
    }
    PXG_HIP(hipMemcpyAsync(offsets.p, ho.data(), (size_t)M * k * 4, hipMemcpyHostToDevice, s));
    hipLaunchKernelGGL(pqb_stage, dim3(M), dim3(256), 0, s, (const PqSub*)dS.p, (int)k);
    const int wmax = *std::max_element(L.width.begin(), L.width.end());
    const bool wide = n >= 64 * k;
    if (wmax <= 8 && wide)
      hipLaunchKernelGGL((pqb_sums<8, 1024>), dim3((unsigned)k, M), dim3(1024), 0, s, (const PqSub*)dS.p, (int)k,
                         (const uint32_t*)members.p);
    else if (wmax <= 8)
      hipLaunchKernelGGL((pqb_sums<8, 256>), dim3((unsigned)k, M), dim3(256), 0, s, (const PqSub*)dS.p, (int)k,
                         (const uint32_t*)members.p);
    else if (wmax <= 16)
      hipLaunchKernelGGL((pqb_sums<16, 256>), dim3((unsigned)k, M), dim3(256), 0, s, (const PqSub*)dS.p, (int)k,
                         (const uint32_t*)members.p);
    else
      hipLaunchKernelGGL((pqb_sums<32, 256>), dim3((unsigned)k, M), dim3(256), 0, s, (const PqSub*)dS.p, (int)k,
                         (const uint32_t*)members.p);
    PXG_HIP(hipGetLastError());
    // empty clusters, ascending, against the partially updated array
    // (kmeans.rs:119-123): the farthest point of [new rows < c, old rows >= c]
    for (int q = 0; q < Mb; ++q) {
      if (!h[q].active) continue;
      const int w = h[q].w;
      for (size_t c = 0; c < k; ++c) {
        if (hc[(size_t)q * k + c] != 0) continue;
        work.reserve(k * w);
        rdist.reserve(n);
        rassign.reserve(n);
        PXG_HIP(hipMemcpyAsync(work.p, h[q].newc, c * w * 4, hipMemcpyDeviceToDevice, s));
        PXG_HIP(hipMemcpyAsync(work.p + c * w, h[q].cents + c * w, (k - c) * w * 4, hipMemcpyDeviceToDevice, s));
        nearest_device(h[q].P, w, nullptr, n, w, work.p, w, k, false, rassign.p, rdist.p, s);
        launch_farthest(rdist.p, n, far_part.p, far.p, s);
        hipLaunchKernelGGL(copy_row_at, dim3(1), dim3(256), 0, s, h[q].P, w, (const long long*)far.p, w,
                           h[q].newc + c * w);
        PXG_HIP(hipGetLastError());
      }
    }
    hipLaunchKernelGGL(pqb_commit, dim3(M), dim3(256), 0, s, (const PqSub*)dS.p, (int)k);
    PXG_HIP(hipGetLastError());
  }
  PXG_HIP(hipStreamSynchronize(s));
  return redo_from;
}

void pq_train_device(const float* R, size_t n, int dim, int ldr, const PqLayout& L, size_t max_iter, uint64_t seed,
                     float* d_books, double* inertia, size_t* iterations, hipStream_t s) {
  (void)dim;
  const int M = L.M;
  const size_t k = std::max<size_t>(std::min<size_t>(256, n), 1);
  std::vector<DevBuf<float>> proj(M), seeds(M), cents(M);
  std::vector<KmeansOut> res(M);
  std::vector<ChaCha8> start(M);
  {
    ChaCha8 r(seed);
    for (int sidx = 0; sidx < M; ++sidx) {
      start[sidx] = r;
      if (n) {
        (void)r.gen_range_usize(n);
        for (size_t c = 1; c < k; ++c) (void)r.next_u64();
      }
    }
  }
  for (int sidx = 0; sidx < M; ++sidx) {
    const int w = L.width[sidx], off = L.off[sidx];
    const size_t tot = n * (size_t)w;
    proj[sidx].reserve(std::max<size_t>(tot, 1));
    if (tot)
      hipLaunchKernelGGL(gather_cols, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, R, ldr, (int)n, off, w,
                         proj[sidx].p);
    PXG_HIP(hipGetLastError());
  }
  // seeding from `rng` (advanced by it) and the Lloyd loop of one subspace:
  // the single-run path
  auto train_one = [&](int sidx, ChaCha8& rng) {
    const int w = L.width[sidx];
    seeds[sidx].reserve(k * w);
    size_t inexact = 0;
    if (n) inexact = kmeans_pp_device(proj[sidx].p, n, w, w, k, rng, seeds[sidx].p, s);
    res[sidx] = kmeans_device(proj[sidx].p, n, w, w, 256, max_iter, nullptr, n ? seeds[sidx].p : nullptr, cents[sidx],
                              nullptr, s);
    res[sidx].inexact_sums += inexact;
  };
  const int wmax = *std::max_element(L.width.begin(), L.width.end());
  int done = 0;
  ChaCha8 next(seed);
  // the shared member sort indexes M * n entries with an int
  if (n && wmax <= 32 && (uint64_t)M * n < (1ull << 31)) {
    done = pq_train_batched(proj, n, L, k, max_iter, start, cents, res, &next, s);
  } else {
    next = start[0];
  }
  for (int t = done; t < M; ++t) train_one(t, next);
  double in = 0.0;
  size_t its = 0;
  for (int sidx = 0; sidx < M; ++sidx) {
    const int w = L.width[sidx];
    const KmeansOut& r = res[sidx];
    in += r.inertia;
    its += r.iterations;
    float* book = d_books + L.book_off[sidx];
    PXG_HIP(hipMemcpyAsync(book, cents[sidx].p, r.k * w * 4, hipMemcpyDeviceToDevice, s));
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

int pxg_kmeans_last_stats(double* mfma_ms, double* mfma_flops, uint64_t* mfma_passes, uint64_t* rescanned,
                          uint64_t* inexact_sums) {
  return pxg::guard([&] {
    if (mfma_ms) *mfma_ms = pxg::g_km.mfma_ms;
    if (mfma_flops) *mfma_flops = pxg::g_km.mfma_flops;
    if (mfma_passes) *mfma_passes = pxg::g_km.passes;
    if (rescanned) *rescanned = pxg::g_km.rescanned;
    if (inexact_sums) *inexact_sums = pxg::g_km.inexact_sums;
  });
}

int pxg_kmeans_last_reseeds(uint64_t* reseeds, uint64_t* pool_reseeds, uint64_t* pool_fallbacks) {
  return pxg::guard([&] {
    if (reseeds) *reseeds = pxg::g_km.reseeds;
    if (pool_reseeds) *pool_reseeds = pxg::g_km.pool_reseeds;
    if (pool_fallbacks) *pool_fallbacks = pxg::g_km.pool_fallbacks;
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
