// Device helpers shared by the kernels: the total order on f32 scores, the
// reference's exact 8-lane distance arithmetic, a register bitonic sort across
// one 64-wide wavefront, and a block radix select over 64-bit keys.
//
// Everything that must match the reference bit for bit is built with
// -ffp-contract=off (no FMA contraction), so `acc += d * d` rounds twice
// exactly as the Rust source does.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace pxg {

constexpr int WAVE = 64;
constexpr uint64_t KEY_MAX = ~0ull;

// f32::total_cmp order as an unsigned key (topk.rs:63-67 orders by it).
__host__ __device__ inline uint32_t ord_key(float f) {
  uint32_t b = __builtin_bit_cast(uint32_t, f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__host__ __device__ inline float key_float(uint32_t k) {
  uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __builtin_bit_cast(float, b);
}

// The value held by lane (lane ^ M), M a power of two below 64, by VALU lane
// exchanges rather than the LDS crossbar: DPP quad permutes for 1 and 2, row
// shifts for 4 (left for lanes with bit 2 clear, right for the others), a
// half-row rotate for 8, and the gfx950 permlane swaps for 16 and 32 (which,
// given the same register twice, return a wave with the upper and one with
// the lower half of each 32- or 16-lane pair).
template <int M>
__device__ __forceinline__ uint32_t xor_lane(uint32_t x) {
  const int lane = __lane_id();
  if constexpr (M == 1) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  } else if constexpr (M == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else if constexpr (M == 4) {
    const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x104, 0xF, 0xF, false);  // row_shl:4
    const uint32_t dn = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF, false);  // row_shr:4
    return (lane & 4) ? dn : up;
  } else if constexpr (M == 8) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (M == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (lane & 16) ? p[0] : p[1];
  } else {
    static_assert(M == 32, "xor distance");
    const auto p = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (lane & 32) ? p[0] : p[1];
  }
}

__device__ __forceinline__ uint32_t xor_lane_rt(uint32_t x, int mask) {
  switch (mask) {  // folds wherever the mask is a constant (unrolled networks)
    case 1: return xor_lane<1>(x);
    case 2: return xor_lane<2>(x);
    case 4: return xor_lane<4>(x);
    case 8: return xor_lane<8>(x);
    case 16: return xor_lane<16>(x);
    case 32: return xor_lane<32>(x);
    default: return (uint32_t)__shfl_xor((int)x, mask, WAVE);
  }
}

// Lane (lane - 1)'s value (DPP wave_shr:1; lane 0 gets 0).
__device__ __forceinline__ uint32_t lane_up1(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x138, 0xF, 0xF, false);
}

// Lane (63 - lane)'s value: a row mirror (lane ^ 15 within each 16-lane row),
// then the xor 16 and xor 32 exchanges.
__device__ __forceinline__ uint32_t lane_reverse(uint32_t x) {
  const uint32_t m = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x140, 0xF, 0xF, false);  // row_mirror
  return xor_lane<32>(xor_lane<16>(m));
}

// 64-bit shuffle across the wave: lane (lane ^ mask)'s value.
__device__ inline uint64_t shfl_xor64(uint64_t v, int mask) {
  const uint32_t lo = xor_lane_rt((uint32_t)v, mask), hi = xor_lane_rt((uint32_t)(v >> 32), mask);
  return ((uint64_t)hi << 32) | lo;
}

// NaN results, as on the reference's aarch64 platform: an invalid operation
// (inf + -inf) yields the default NaN 0x7FC00000 with its sign clear, and a
// NaN operand propagates. Inputs are finite, so every NaN inside a dot-type
// sum is that default NaN, and only a later negation (inner product, the IP
// ADC) flips its sign, which decides where total_cmp ranks it. The sums are
// mapped to 0x7FC00000 before any negation so that no result depends on the
// sign this GPU gives a generated NaN.
__host__ __device__ inline float arm_nan(float x) { return x != x ? __builtin_bit_cast(float, 0x7FC00000u) : x; }

// The IVF cosine score (1 - q.c) + inner_product(code) (ivfpq.rs:1068-1074)
// under the same rule: omq = arm_nan(1 - q.c) is +NaN when NaN, a NaN ADC sum
// negates to -NaN, the addition returns its first NaN operand, and
// inf + (-inf) gives +NaN.
__device__ inline float ivf_cos_score(float omq, float sum) {
  const float s = omq + (-sum);
  if (s == s) return s;
  return (omq != omq || sum == sum) ? __builtin_bit_cast(float, 0x7FC00000u) : __builtin_bit_cast(float, 0xFFC00000u);
}

// ----------------------------------------------------------------------------
// Exact distances in the reference's arithmetic.
//
// squared_euclidean_unrolled / dot_unrolled / manhattan_unrolled
// (distance.rs:267-372): eight lane accumulators over chunks_exact(8), the
// pairwise reduce of distance.rs:534-538, then + a sequential tail.
//
// dist_group8: eight consecutive threads (group lane g = 0..7) cooperate on
// one pair; thread g owns accumulator g. Every thread of the group returns
// the same value.
// ----------------------------------------------------------------------------
template <int METRIC>
__device__ inline float lane_term(float a, float b) {
  if constexpr (METRIC == 0) {
    float d = a - b;
    return d * d;
  } else if constexpr (METRIC == 3) {
    return fabsf(a - b);
  } else {
    return a * b;
  }
}

template <int METRIC>
__device__ inline float dist_group8(const float* __restrict__ a, const float* __restrict__ b, int dim, int g) {
  float acc = 0.0f;
  const int chunks = dim >> 3;
  // unrolled so that 16 chunks' loads are in flight together; the adds stay
  // in chunk order
#pragma unroll 16
  for (int c = 0; c < chunks; ++c) acc += lane_term<METRIC>(a[c * 8 + g], b[c * 8 + g]);
  // ((0+1)+(2+3))+((4+5)+(6+7)): f32 addition is commutative, so the xor
  // partner order gives the same bits on every lane of the group.
  acc = acc + __shfl_xor(acc, 1, WAVE);
  acc = acc + __shfl_xor(acc, 2, WAVE);
  acc = acc + __shfl_xor(acc, 4, WAVE);
  float tail = 0.0f;
  for (int i = chunks * 8; i < dim; ++i) tail += lane_term<METRIC>(a[i], b[i]);
  float r = acc + tail;
  if constexpr (METRIC == 1) return arm_nan(1.0f - arm_nan(r));  // cosine_normalized, distance.rs:400-402
  if constexpr (METRIC == 2) return -arm_nan(r);                 // inner_product, distance.rs:291-293
  return r;
}

// dist_group8's arithmetic with two lanes per row: lane h (of an adjacent
// pair) owns the reference's accumulators 4h .. 4h+3, i.e. elements 8c + 4h
// .. 8c + 4h + 3 of every chunk c, loaded as one float4 per chunk and added
// in chunk order; its half (a0 + a1) + (a2 + a3) and the partner's combine
// as ((0+1)+(2+3)) + ((4+5)+(6+7)), dist_group8's reduce (the last add is
// commutative, so both lanes get the same bits). Rows start 16-byte aligned.
template <int METRIC>
__device__ inline float dist_pair4(const float* __restrict__ a, const float* __restrict__ b, int dim, int h) {
  float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
  const int chunks = dim >> 3;
  const float* ap = a + 4 * h;
  const float* bp = b + 4 * h;
#pragma unroll 8
  for (int c = 0; c < chunks; ++c) {
    const float4 x = *reinterpret_cast<const float4*>(ap + 8 * c);
    const float4 y = *reinterpret_cast<const float4*>(bp + 8 * c);
    s0 += lane_term<METRIC>(x.x, y.x);
    s1 += lane_term<METRIC>(x.y, y.y);
    s2 += lane_term<METRIC>(x.z, y.z);
    s3 += lane_term<METRIC>(x.w, y.w);
  }
  const float half = (s0 + s1) + (s2 + s3);
  const float acc = half + __shfl_xor(half, 1, WAVE);
  float tail = 0.0f;
  for (int i = chunks * 8; i < dim; ++i) tail += lane_term<METRIC>(a[i], b[i]);
  const float r = acc + tail;
  if constexpr (METRIC == 1) return arm_nan(1.0f - arm_nan(r));
  if constexpr (METRIC == 2) return -arm_nan(r);
  return r;
}

// dist_pair4 for QG queries a[0..QG) against one row b: the row's float4 of
// each chunk is loaded once and used by every query, and each query keeps its
// own four accumulators and operand order, so out[j] has the bits of
// dist_pair4(a[j], b, dim, h).
template <int METRIC, int QG>
__device__ inline void dist_pair4_multi(const float* const (&a)[QG], const float* __restrict__ b, int dim, int h,
                                        float (&out)[QG], int nv = QG) {
  float s[QG][4];
#pragma unroll
  for (int j = 0; j < QG; ++j) s[j][0] = s[j][1] = s[j][2] = s[j][3] = 0.0f;
  const int chunks = dim >> 3;
  const float* bp = b + 4 * h;
#pragma unroll 4
  for (int c = 0; c < chunks; ++c) {
    const float4 y = *reinterpret_cast<const float4*>(bp + 8 * c);
#pragma unroll
    for (int j = 0; j < QG; ++j) {
      if (j >= nv) break;  // uniform: queries past the group's end
      const float4 x = *reinterpret_cast<const float4*>(a[j] + 4 * h + 8 * c);
      s[j][0] += lane_term<METRIC>(x.x, y.x);
      s[j][1] += lane_term<METRIC>(x.y, y.y);
      s[j][2] += lane_term<METRIC>(x.z, y.z);
      s[j][3] += lane_term<METRIC>(x.w, y.w);
    }
  }
#pragma unroll
  for (int j = 0; j < QG; ++j) {
    const float half = (s[j][0] + s[j][1]) + (s[j][2] + s[j][3]);
    const float acc = half + __shfl_xor(half, 1, WAVE);
    float tail = 0.0f;
    for (int i = chunks * 8; i < dim; ++i) tail += lane_term<METRIC>(a[j][i], b[i]);
    const float r = acc + tail;
    if constexpr (METRIC == 1) out[j] = arm_nan(1.0f - arm_nan(r));
    else if constexpr (METRIC == 2) out[j] = -arm_nan(r);
    else out[j] = r;
  }
}

template <int QG>
__device__ inline void dist_pair4_multi_rt(int metric, const float* const (&a)[QG], const float* b, int dim, int h,
                                           float (&out)[QG], int nv = QG) {
  switch (metric) {
    case 0: dist_pair4_multi<0, QG>(a, b, dim, h, out, nv); break;
    case 1: dist_pair4_multi<1, QG>(a, b, dim, h, out, nv); break;
    case 2: dist_pair4_multi<2, QG>(a, b, dim, h, out, nv); break;
    default: dist_pair4_multi<3, QG>(a, b, dim, h, out, nv); break;
  }
}

__device__ inline float dist_pair4_rt(int metric, const float* a, const float* b, int dim, int h) {
  switch (metric) {
    case 0: return dist_pair4<0>(a, b, dim, h);
    case 1: return dist_pair4<1>(a, b, dim, h);
    case 2: return dist_pair4<2>(a, b, dim, h);
    default: return dist_pair4<3>(a, b, dim, h);
  }
}

// One thread computes the whole distance (same arithmetic as dist_group8).
template <int METRIC>
__device__ inline float dist_thread(const float* __restrict__ a, const float* __restrict__ b, int dim) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const int chunks = dim >> 3;
  for (int c = 0; c < chunks; ++c) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += lane_term<METRIC>(a[c * 8 + j], b[c * 8 + j]);
  }
  float tail = 0.0f;
  for (int i = chunks * 8; i < dim; ++i) tail += lane_term<METRIC>(a[i], b[i]);
  float r = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  r = r + tail;
  if constexpr (METRIC == 1) return arm_nan(1.0f - arm_nan(r));
  if constexpr (METRIC == 2) return -arm_nan(r);
  return r;
}

__device__ inline float dist_group8_rt(int metric, const float* a, const float* b, int dim, int g) {
  switch (metric) {
    case 0: return dist_group8<0>(a, b, dim, g);
    case 1: return dist_group8<1>(a, b, dim, g);
    case 2: return dist_group8<2>(a, b, dim, g);
    default: return dist_group8<3>(a, b, dim, g);
  }
}

// ----------------------------------------------------------------------------
// Bitonic sort (ascending) of 64*E unsigned 64-bit keys held in registers by
// one wavefront; lane L holds elements L*E .. L*E+E-1.
// ----------------------------------------------------------------------------
template <int E>
__device__ inline void wave_bitonic_sort(uint64_t (&k)[E], int lane) {
  constexpr int N = WAVE * E;
#pragma unroll
  for (int size = 2; size <= N; size <<= 1) {
#pragma unroll
    for (int j = size >> 1; j > 0; j >>= 1) {
      if (j >= E) {
        const int lm = j / E;
        const bool lower = (lane & lm) == 0;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int i = lane * E + e;
          const bool asc = (i & size) == 0;
          uint64_t p = shfl_xor64(k[e], lm);
          uint64_t mn = k[e] < p ? k[e] : p;
          uint64_t mx = k[e] < p ? p : k[e];
          k[e] = (lower == asc) ? mn : mx;
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          if ((e & j) == 0) {
            const int i = lane * E + e;
            const bool asc = (i & size) == 0;
            uint64_t x = k[e], y = k[e | j];
            bool sw = asc ? (y < x) : (x < y);
            k[e] = sw ? y : x;
            k[e | j] = sw ? x : y;
          }
        }
      }
    }
  }
}

// Ascending bitonic sort of 64 (key, value) pairs across one wavefront, one
// pair per lane: afterwards lane L holds the L-th smallest key and its value.
__device__ inline void wave_sort_kv64(uint64_t& key, uint32_t& val, int lane) {
#pragma unroll
  for (int size = 2; size <= WAVE; size <<= 1) {
#pragma unroll
    for (int j = size >> 1; j > 0; j >>= 1) {
      const uint64_t pk = shfl_xor64(key, j);
      const uint32_t pv = xor_lane_rt(val, j);
      // the lower lane of a pair keeps the smaller key in an ascending run
      const bool take_min = ((lane & j) == 0) == ((lane & size) == 0);
      const bool take = take_min ? pk < key : key < pk;
      key = take ? pk : key;
      val = take ? pv : val;
    }
  }
}

// ----------------------------------------------------------------------------
// Block radix select: the K-th smallest (1-based, counting repeats) of n
// BITS-bit keys read through `get(i)`. All threads of the block call it;
// returns the pivot in every thread. `hist` is 256 ints of shared memory,
// `sh` 4 u64 of shared. Keys equal to KEY_MAX are padding and never
// selected; the caller clamps K to the number of real keys.
//
// PER > 0 reads each key once into registers (key i of thread t is
// i = t + j * blockDim.x, j < PER; requires n <= PER * blockDim.x); PER = 0
// reads the keys through `get` on every pass. The digit passes stop early
// once the chosen digit's bin holds exactly the keys still needed: all of
// them are then among the K smallest, and the K-th smallest is their
// largest, found by a block maximum.
// ----------------------------------------------------------------------------
// block_radix_select over keys the calling threads already hold: each(f)
// calls f(x) once for every key of the calling thread, in a fixed order (the
// keys of all threads together are the n keys).
template <int BITS, class Each>
__device__ inline uint64_t block_radix_select_each(Each each, int K, int* hist, uint64_t* sh) {
  static_assert(BITS % 8 == 0 && BITS <= 64, "whole-byte digits");
  if (threadIdx.x == 0) sh[3] = 0;
  uint64_t prefix = 0, mask = 0;
  int remaining = K;
  for (int pass = 0; pass < BITS / 8; ++pass) {
    const int shift = BITS - 8 - 8 * pass;
    for (int i = threadIdx.x; i < 256; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    // runs of one digit in a thread's keys go in as one add (the leading
    // digits are often shared by most keys, which would otherwise serialise
    // every add on one bin)
    int run_d = -1, run_n = 0;
    each([&](uint64_t x) {
      if ((x & mask) == prefix) {
        const int dg = (int)((x >> shift) & 255);
        if (dg != run_d) {
          if (run_n) atomicAdd(&hist[run_d], run_n);
          run_d = dg;
          run_n = 0;
        }
        ++run_n;
      }
    });
    if (run_n) atomicAdd(&hist[run_d], run_n);
    __syncthreads();
    if (threadIdx.x < WAVE) {
      // exclusive scan over 256 bins by one wave: 4 bins per lane
      const int lane = threadIdx.x;
      int c0 = hist[lane * 4], c1 = hist[lane * 4 + 1], c2 = hist[lane * 4 + 2], c3 = hist[lane * 4 + 3];
      int s = c0 + c1 + c2 + c3;
      int incl = s;
      for (int o = 1; o < WAVE; o <<= 1) {
        int t = __shfl_up(incl, o, WAVE);
        if (lane >= o) incl += t;
      }
      int excl = incl - s;
      // the digit d with excl(d) < remaining <= excl(d) + count(d)
      int e0 = excl, e1 = e0 + c0, e2 = e1 + c1, e3 = e2 + c2;
      int d = -1, before = 0, cnt = 0;
      if (remaining > e0 && remaining <= e1) { d = lane * 4; before = e0; cnt = c0; }
      else if (remaining > e1 && remaining <= e2) { d = lane * 4 + 1; before = e1; cnt = c1; }
      else if (remaining > e2 && remaining <= e3) { d = lane * 4 + 2; before = e2; cnt = c2; }
      else if (remaining > e3 && remaining <= e3 + c3) { d = lane * 4 + 3; before = e3; cnt = c3; }
      if (d >= 0) {
        sh[0] = (uint64_t)d;
        sh[1] = (uint64_t)before;
        sh[2] = (uint64_t)cnt;
      }
    }
    __syncthreads();
    const uint64_t d = sh[0];
    remaining -= (int)sh[1];
    const int cnt = (int)sh[2];
    prefix |= d << shift;
    mask |= 255ull << shift;
    __syncthreads();
    if (cnt == remaining && pass + 1 < BITS / 8) {
      uint64_t m = 0;
      each([&](uint64_t x) {
        if ((x & mask) == prefix && x > m) m = x;
      });
      if (m) atomicMax((unsigned long long*)&sh[3], (unsigned long long)m);
      __syncthreads();
      const uint64_t r = sh[3];
      __syncthreads();  // sh may be reused by the caller's next select
      return r;
    }
  }
  return prefix;
}

template <class Get, int BITS = 64, int PER = 0>
__device__ inline uint64_t block_radix_select(Get get, int n, int K, int* hist, uint64_t* sh) {
  static_assert(BITS % 8 == 0 && BITS <= 64, "whole-byte digits");
  constexpr int C = PER > 0 ? PER : 1;
  uint64_t v[C];
  if constexpr (PER > 0) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = threadIdx.x + j * blockDim.x;
      v[j] = i < n ? (uint64_t)get(i) : 0;
    }
  }
  // every key of this thread, in order: f(x)
  auto each = [&](auto f) {
    if constexpr (PER > 0) {
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (threadIdx.x + j * blockDim.x < n) f(v[j]);
    } else {
      for (int i = threadIdx.x; i < n; i += blockDim.x) f((uint64_t)get(i));
    }
  };
  return block_radix_select_each<BITS>(each, K, hist, sh);
}

}  // namespace pxg
