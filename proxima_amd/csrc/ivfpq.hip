// IVF-PQ on MI355X: IvfPqIndex (crates/proxima-index/src/ivfpq.rs) with the
// product quantizer's distance table and ADC (crates/proxima-quantize/src/
// product.rs:407-616).
//
// HBM layout of a trained index:
//   cents      [produced][ld] f32   coarse centroids (zero padded rows)
//   books      [sum_s 256*width_s] f32, subspace s at book_off[s], row c of
//              width_s floats (product.rs:226-238 layout)
//   codes      [cap][M] u8           slot-major PQ codes (product.rs:361-380)
//   list_of    [cap] u32             coarse list per slot, UINT32_MAX if none
//   list view, one entry per live slot (ivfpq.rs:891-896): list l's entries
//   at positions [list_beg[l], list_end[l]) of a pool with slack per list,
//   kept current by every insert (append) and removal (the list's last entry
//   fills the hole), laid out again only after train, load, compact or when
//   the pool fills:
//     list_beg, list_end [produced] u32, list_slot [pool] u32 (slot),
//     list_codes [pool][M] u8 -> M bytes per scanned vector streamed by
//     ivf_scan16 (slots, and through them id ranks and filters, read only
//     for entries that pass its screen), M + 4 by the other scans.
//   X          [cap][ld] f32 prepared vectors when retained (rerank, training,
//              the untrained exhaustive path).
//
// Search (ivfpq.rs:998-1110), per batch:
//   coarse      the nprobe smallest (exact squared_euclidean_unrolled, list)
//               over every centroid (bit-exact, so the probed list set is the
//               reference's): for nprobe <= 64, ivf_coarse_mfma (FP32 matrix
//               core distances with a stated error bound) + ivf_coarse_pick_approx
//               (exact rescoring of every list the bound cannot exclude) when
//               dim >= 32, else ivf_coarse_dist (all exact keys, over the
//               transposed centroids) + ivf_coarse_pick; beyond 64 the exact
//               flat index over the centroids, else ivf_coarse_keys +
//               ivf_coarse_select.
//   scan        build each probe's distance table exactly as distance_table
//               does (per subspace, per centroid, sequential d = q - c;
//               l2 += d*d; ip += q*c), stream the list's codes coalesced,
//               ADC-sum the table in subspace order (bit-exact), keep a
//               per-wave top-kk by (score, id): ivf_scan16 (16 subspaces,
//               dim <= 128, kk <= 128: codebook rows in VGPRs, one workgroup
//               per query and up to 32 probes, codes staged through LDS by
//               asynchronous copies, id ranks fetched only for entries whose
//               score passes the wave's current k-th distance),
//               ivf_scan_reg (other equal-width layouts, same work split),
//               else ivf_scan (table in LDS, one workgroup per query and
//               probe).
//   ivf_merge   per query: select the shortlist over all probes, optionally
//               rescore it exactly against the stored vectors (rerank), keep k;
//               skipped when one probe group covers each query and there is
//               no rerank (the scan merges its waves and writes the results).
#include <algorithm>
#include <cmath>
#include <mutex>
#include <shared_mutex>

#include "common.hpp"
#include "device.hpp"
#include "exact_scan.hpp"
#include "flat.hpp"
#include "wide.hpp"
#include "train.hpp"
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <memory>

namespace pxg {

constexpr uint32_t UNASSIGNED = 0xFFFFFFFFu;
constexpr int IVF_MAX_M = 128;
thread_local uint64_t g_last_scanned = 0;

// ---------------------------------------------------------------------------
// coarse stage
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ivf_coarse_keys(const float* __restrict__ Qp, int ld, int dim,
                                                       const float* __restrict__ cents, int produced,
                                                       uint64_t* __restrict__ ck) {
  const int q = blockIdx.x;
  const int g = threadIdx.x & 7, grp = threadIdx.x >> 3;
  const float* qv = Qp + (size_t)q * ld;
  for (int l = grp; l < produced; l += 32) {
    const float d = dist_group8<0>(qv, cents + (size_t)l * ld, dim, g);  // squared_l2, ivfpq.rs:1247-1249
    if (g == 0) ck[(size_t)q * produced + l] = ((uint64_t)ord_key(d) << 32) | (uint32_t)l;
  }
}

__global__ __launch_bounds__(256) void ivf_coarse_select(const uint64_t* __restrict__ ck, int produced, int nprobe,
                                                         int* __restrict__ probes) {
  const int q = blockIdx.x;
  __shared__ int hist[256];
  __shared__ uint64_t sh[4];
  __shared__ int n_sel;
  const uint64_t* base = ck + (size_t)q * produced;
  auto get = [&](int i) -> uint64_t { return base[i]; };
  if (threadIdx.x == 0) n_sel = 0;
  __syncthreads();
  // (distance total_cmp, list) order: ivfpq.rs:1025
  const uint64_t pivot = block_radix_select(get, produced, nprobe, hist, sh);
  for (int i = threadIdx.x; i < produced; i += blockDim.x) {
    const uint64_t x = base[i];
    if (x <= pivot) probes[(size_t)q * nprobe + atomicAdd(&n_sel, 1)] = (int)(uint32_t)x;
  }
}

// ---------------------------------------------------------------------------
// ADC scan of one probed list per workgroup
// ---------------------------------------------------------------------------
template <int CAPW>
__device__ inline void wave_compact(uint64_t* wb, int cnt, int kk, int lane) {
  constexpr int E = CAPW / WAVE;
  uint64_t kv[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int idx = lane * E + e;
    kv[e] = idx < cnt ? wb[idx] : KEY_MAX;
  }
  wave_bitonic_sort<E>(kv, lane);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int idx = lane * E + e;
    if (idx < kk) wb[idx] = kv[e];
  }
}

template <int CAPW, int METRIC>
__global__ __launch_bounds__(256) void ivf_scan(const float* __restrict__ Qp, int ld, int dim, int M,
                                                const int* __restrict__ probes, int nprobe,
                                                const float* __restrict__ cents, const float* __restrict__ books,
                                                const int* __restrict__ sub_off, const int* __restrict__ book_off,
                                                const uint32_t* __restrict__ list_beg,
                                                const uint32_t* __restrict__ list_end,
                                                const uint32_t* __restrict__ list_slot,
                                                const uint8_t* __restrict__ list_codes,
                                                const uint32_t* __restrict__ rank_slot,
                                                const uint32_t* __restrict__ slot_rank,
                                                const uint8_t* __restrict__ accept, int kk,
                                                uint64_t* __restrict__ out) {
  extern __shared__ float lut[];  // M * 256 floats
  __shared__ uint64_t wbuf[4][CAPW];
  __shared__ float s_qdc;
  const int q = blockIdx.x / nprobe, p = blockIdx.x % nprobe;
  const int l = probes[(size_t)q * nprobe + p];
  const float* qv = Qp + (size_t)q * ld;
  const float* cv = cents + (size_t)l * ld;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

  if constexpr (METRIC == 1) {
    // q . c for the cosine decomposition (ivfpq.rs:1068-1072, dot_unrolled)
    if (tid < 8) {
      const float d = -dist_group8<2>(qv, cv, dim, tid);
      if (tid == 0) s_qdc = d;
    }
  }
  // Distance table (product.rs:416-433). L2: on the residual q - c
  // (ivfpq.rs:1052-1054); cosine: on the query itself (shared table).
  for (int e = tid; e < M * 256; e += 256) {
    const int s = e >> 8, c = e & 255;
    const int w_s = sub_off[s + 1] - sub_off[s];
    const float* b = books + book_off[s] + c * w_s;
    const int o = sub_off[s];
    float acc = 0.0f;
    for (int j = 0; j < w_s; ++j) {
      if constexpr (METRIC == 0) {
        const float r = qv[o + j] - cv[o + j];
        const float d = r - b[j];
        acc += d * d;
      } else {
        acc += qv[o + j] * b[j];
      }
    }
    lut[e] = acc;
  }
  __syncthreads();
  const float one_minus_qdc = METRIC == 1 ? arm_nan(1.0f - s_qdc) : 0.0f;

  uint64_t* wb = wbuf[w];
  uint64_t thr = KEY_MAX;
  int cnt = 0;
  const uint32_t begin = list_beg[l], end = list_end[l];
  for (uint32_t e0 = begin + w * 64; e0 < end; e0 += 256) {
    const uint32_t e = e0 + lane;
    uint64_t key = KEY_MAX;
    if (e < end) {
      const uint32_t sl = list_slot[e];
      if (accept == nullptr || accept[sl]) {
        const uint32_t rk = slot_rank[sl];
        const uint8_t* code = list_codes + (size_t)e * M;
        float sum = 0.0f;  // DistanceTable::squared_l2 / inner_product, product.rs:580-603
        if (M == 16) {
          const uint4 cw = *reinterpret_cast<const uint4*>(code);
          const uint32_t wv[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
          for (int s = 0; s < 16; ++s) sum += lut[s * 256 + ((wv[s >> 2] >> (8 * (s & 3))) & 255)];
        } else {
          for (int s = 0; s < M; ++s) sum += lut[s * 256 + code[s]];
        }
        const float score = METRIC == 0 ? sum : ivf_cos_score(one_minus_qdc, sum);
        key = ((uint64_t)ord_key(score) << 32) | rk;
      }
    }
    const bool pass = key < thr;
    const uint64_t mask = __ballot(pass);
    const int pos = cnt + __popcll(mask & ((1ull << lane) - 1));
    if (pass) wb[pos] = key;
    cnt += __popcll(mask);
    if (cnt > CAPW - 64) {
      wave_compact<CAPW>(wb, cnt, kk, lane);
      cnt = kk;
      thr = wb[kk - 1];
    }
  }
  wave_compact<CAPW>(wb, cnt, kk, lane);
  uint64_t* o = out + (((size_t)q * nprobe + p) * 4 + w) * kk;
  for (int i = lane; i < kk; i += 64) o[i] = i < cnt ? wb[i] : KEY_MAX;
}

// ---------------------------------------------------------------------------
// ADC scan, register-resident codebooks (uniform subspace width W, M*W = dim
// <= 128, shortlist <= 64). One workgroup per (query, group of probes); thread
// t holds row t of every subspace codebook in VGPRs, so building a probe's
// distance table is VALU work on LDS-broadcast residuals; each wave keeps its
// best keys one per lane, sorted, across the whole probe group.
// ---------------------------------------------------------------------------
__device__ inline uint64_t readlane64(uint64_t v, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}

// Insert the passing keys of this batch (one candidate key per lane) into
// the wave's sorted list `kept` (lane i = i-th smallest, KEY_MAX when empty).
__device__ inline void wave_topk_insert(uint64_t key, uint64_t& kept, uint64_t& thr, int kk, int lane) {
  uint64_t mask = __ballot(key < thr);
  while (mask) {
    const int src = __builtin_ctzll(mask);
    mask &= mask - 1;
    const uint64_t x = readlane64(key, src);
    if (x < thr) {
      const int pos = __popcll(__ballot(kept < x));
      const uint32_t up_lo = lane_up1((uint32_t)kept);
      const uint32_t up_hi = lane_up1((uint32_t)(kept >> 32));
      const uint64_t up = ((uint64_t)up_hi << 32) | up_lo;
      if (lane > pos) kept = up;
      else if (lane == pos) kept = x;
      thr = readlane64(kept, kk - 1);
    }
  }
}

// `kept` (ascending over the lanes) becomes the 64 smallest of kept and
// `other` (also ascending): min against the reversed list is bitonic and
// holds those 64, and a half-cleaner cascade sorts it.
__device__ inline void wave_merge_sorted(uint64_t& kept, uint64_t other, int lane) {
  const uint64_t r = ((uint64_t)lane_reverse((uint32_t)(other >> 32)) << 32) | lane_reverse((uint32_t)other);
  uint64_t v = kept < r ? kept : r;
#pragma unroll
  for (int st = 32; st > 0; st >>= 1) {
    const uint64_t p = shfl_xor64(v, st);
    v = (lane & st) ? (v < p ? p : v) : (v < p ? v : p);
  }
  kept = v;
}

// The 128 keys of two ascending lists (one key per lane each) as two
// ascending lists: lo the 64 smallest, hi the other 64. Min and max against
// the reversed b are the two bitonic halves; a half-cleaner cascade sorts each.
__device__ inline void wave_merge_split(uint64_t a, uint64_t b, int lane, uint64_t& lo, uint64_t& hi) {
  const uint64_t r = ((uint64_t)lane_reverse((uint32_t)(b >> 32)) << 32) | lane_reverse((uint32_t)b);
  uint64_t l = a < r ? a : r, h = a < r ? r : a;
#pragma unroll
  for (int st = 32; st > 0; st >>= 1) {
    const uint64_t pl = shfl_xor64(l, st), ph = shfl_xor64(h, st);
    l = (lane & st) ? (l < pl ? pl : l) : (l < pl ? l : pl);
    h = (lane & st) ? (h < ph ? ph : h) : (h < ph ? h : ph);
  }
  lo = l;
  hi = h;
}

// Add one candidate key per lane to the sorted list: a batch with many
// passing keys is sorted and merged, a sparse one inserted key by key.
__device__ inline void wave_topk_add(uint64_t key, uint64_t& kept, uint64_t& thr, int kk, int lane) {
  const uint64_t mask = __ballot(key < thr);
  if (mask == 0) return;
  if (__popcll(mask) > 6) {
    uint64_t b[1] = {key < thr ? key : KEY_MAX};
    wave_bitonic_sort<1>(b, lane);
    wave_merge_sorted(kept, b[0], lane);
    thr = readlane64(kept, kk - 1);
  } else {
    wave_topk_insert(key, kept, thr, kk, lane);
  }
}

// Coarse top-nprobe for nprobe <= 64 over the transposed centroid matrix
// cT[dim][cst] (cst = list count rounded up to 64, zero padded), in two
// phases: keys of IVF_CQ queries against slices of IVF_CW * 64 lists, then a
// selection per query.
constexpr int IVF_CQ = 4, IVF_CW = 8;

// Two-phase coarse stage (np <= 64, dim <= 2048). Phase one: the (distance,
// list) keys of IVF_CQ queries against one slice of IVF_CW * 64 lists per
// workgroup (grid: query groups x list slices), with the arithmetic of
// squared_euclidean_unrolled (distance.rs:267-283): lane l of a wave takes
// list c0 + l, the queries broadcast from LDS as one
// float4 per dimension, the transposed centroids loaded coalesced. A wave
// keeping its own top-np lists instead (one workgroup per 4 queries over all
// lists) took 0.12 ms at 1024 x 4096 x 128: nearly every tile passed its
// threshold and took the sort-and-merge path.
__global__ __launch_bounds__(IVF_CW * 64) void ivf_coarse_dist(const float* __restrict__ Qp, int ld, int dim, int nq,
                                                               const float* __restrict__ cT, int cst, int produced,
                                                               uint64_t* __restrict__ ck) {
  extern __shared__ float4 sm4[];
  float* sq = (float*)sm4;  // [dim][IVF_CQ]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int q0 = blockIdx.x * IVF_CQ;
  const int c0 = blockIdx.y * (IVF_CW * 64) + w * 64;
  for (int t = tid; t < dim * IVF_CQ; t += IVF_CW * 64) {
    const int i = t / IVF_CQ, j = t % IVF_CQ;
    sq[t] = q0 + j < nq ? Qp[(size_t)(q0 + j) * ld + i] : 0.0f;
  }
  __syncthreads();
  if (c0 >= produced) return;
  const int chunks = dim >> 3;
  const float* col = cT + c0 + lane;
  float acc[IVF_CQ][8];
#pragma unroll
  for (int j = 0; j < IVF_CQ; ++j)
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[j][u] = 0.0f;
  for (int cc = 0; cc < chunks; ++cc) {
    float cv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) cv[u] = col[(size_t)(cc * 8 + u) * cst];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float4 qv = sm4[cc * 8 + u];
      float d;
      d = qv.x - cv[u]; acc[0][u] += d * d;
      d = qv.y - cv[u]; acc[1][u] += d * d;
      d = qv.z - cv[u]; acc[2][u] += d * d;
      d = qv.w - cv[u]; acc[3][u] += d * d;
    }
  }
  float tail[IVF_CQ] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int i = chunks * 8; i < dim; ++i) {
    const float c = col[(size_t)i * cst];
    const float4 qv = sm4[i];
    float d;
    d = qv.x - c; tail[0] += d * d;
    d = qv.y - c; tail[1] += d * d;
    d = qv.z - c; tail[2] += d * d;
    d = qv.w - c; tail[3] += d * d;
  }
  if (c0 + lane >= produced) return;
#pragma unroll
  for (int j = 0; j < IVF_CQ; ++j) {
    const float* a = acc[j];
    const float dd = (((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]))) + tail[j];
    if (q0 + j < nq) ck[(size_t)(q0 + j) * cst + c0 + lane] = ((uint64_t)ord_key(dd) << 32) | (uint32_t)(c0 + lane);
  }
}

// Phase two, one workgroup per query: the np smallest keys, sorted, give the
// probes in (distance, list) order (ivfpq.rs:1025), and the probed list
// lengths go to *scanned. The keys are cut into ng = min(64, produced)
// groups; the np-th smallest group minimum T bounds the np-th smallest key
// from above (np distinct keys are <= T), so the keys <= T hold the answer:
// they are gathered in LDS and sorted. Should they exceed IVF_PICK_CAP, a
// radix select of the np-th key takes over.
constexpr int IVF_PICK_CAP = 1024;
// The scanned-entry count is spread over this many counters (query q adds to
// counter q % IVF_SCAN_SLOTS), so that a batch's workgroups do not all
// update one address; the host adds them up.
constexpr int IVF_SCAN_SLOTS = 64;
__global__ __launch_bounds__(256) void ivf_coarse_pick(const uint64_t* __restrict__ ck, int cst, int produced, int np,
                                                       int* __restrict__ probes, const uint32_t* __restrict__ list_beg,
                                                       const uint32_t* __restrict__ list_end,
                                                       unsigned long long* __restrict__ scanned,
                                                       uint32_t* __restrict__ qwork) {
  const int q = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  __shared__ uint64_t cand[IVF_PICK_CAP];
  __shared__ uint64_t gmin[64];
  __shared__ int hist[256];
  __shared__ uint64_t sh[4];
  __shared__ int ncand;
  __shared__ uint64_t s_t;
  const uint64_t* base = ck + (size_t)q * cst;
  const int ng = min(64, produced), gs = (produced + ng - 1) / ng;
  if (tid == 0) ncand = 0;
  for (int g = w; g < 64; g += 4) {
    uint64_t m = KEY_MAX;
    if (g < ng) {
      const int b = g * gs, e = min(produced, b + gs);
      for (int i = b + lane; i < e; i += 64) m = base[i] < m ? base[i] : m;
    }
#pragma unroll
    for (int st = 32; st > 0; st >>= 1) {
      const uint64_t o = shfl_xor64(m, st);
      m = o < m ? o : m;
    }
    if (lane == 0) gmin[g] = m;
  }
  __syncthreads();
  if (w == 0) {
    uint64_t v[1] = {gmin[lane]};
    wave_bitonic_sort<1>(v, lane);
    const uint64_t t = readlane64(v[0], np - 1);
    if (lane == 0) s_t = t;
  }
  __syncthreads();
  const uint64_t t = s_t;
  for (int i = tid; i < produced; i += 256) {
    const uint64_t x = base[i];
    if (x <= t) {
      const int at = atomicAdd(&ncand, 1);
      if (at < IVF_PICK_CAP) cand[at] = x;
    }
  }
  __syncthreads();
  const int nc = ncand;
  if (nc <= 64) {  // the usual case: one wave sorts them
    if (w == 0) {
      uint64_t v[1] = {lane < nc ? cand[lane] : KEY_MAX};
      wave_bitonic_sort<1>(v, lane);
      cand[lane] = v[0];
    }
    __syncthreads();
  } else if (nc <= IVF_PICK_CAP) {
    int P = 128;
    while (P < nc) P <<= 1;
    for (int i = nc + tid; i < P; i += 256) cand[i] = KEY_MAX;
    __syncthreads();
    block_bitonic_sort(cand, P);
  } else {
    auto get = [&](int i) -> uint64_t { return base[i]; };
    const uint64_t pivot = block_radix_select(get, produced, np, hist, sh);
    if (tid == 0) ncand = 0;
    __syncthreads();
    for (int i = tid; i < produced; i += 256) {
      const uint64_t x = base[i];
      if (x <= pivot) cand[atomicAdd(&ncand, 1)] = x;  // np <= 64 of them
    }
    __syncthreads();
    if (w == 0) {
      uint64_t v[1] = {lane < np ? cand[lane] : KEY_MAX};
      wave_bitonic_sort<1>(v, lane);
      cand[lane] = v[0];
    }
    __syncthreads();
  }
  if (w == 0) {
    const int l = (int)(uint32_t)cand[lane];
    if (lane < np) probes[(size_t)q * np + lane] = l;
    uint32_t len = lane < np ? list_end[l] - list_beg[l] : 0u;
#pragma unroll
    for (int st = 32; st > 0; st >>= 1) len += xor_lane_rt(len, st);
    if (lane == 0) atomicAdd(scanned + (q & (IVF_SCAN_SLOTS - 1)), (unsigned long long)len);
    if (lane == 0 && qwork) qwork[q] = len;
  }
}

// ---------------------------------------------------------------------------
// Coarse stage on matrix cores, certified
// ---------------------------------------------------------------------------
// The probe set is the np smallest (squared_euclidean_unrolled, list) keys
// (ivfpq.rs:1019-1026), so it must come from the exact arithmetic. Phase one
// computes a[q][l] = |q|^2 + |c_l|^2 - 2 q.c_l with FP32 MFMA; the exact
// D = squared_euclidean_unrolled(q, c_l) satisfies |a - D| <= eps_ql =
// 4 dim 2^-24 (|q| + |c_l|)^2 (the f32 errors of both computations, each at
// most about dim ulps of (|q| + |c_l|)^2). Phase two per query: T = the np-th
// smallest of the 64 group minima of a + eps bounds the np-th smallest D
// from above, so every list with D below it has a - eps <= T; those lists
// are rescored exactly and sorted by (D, list). More than IVF_PICK_CAP of
// them falls back to exact keys over every list.
typedef float fv16 __attribute__((ext_vector_type(16)));

// 64 queries x 64 lists per 256-thread block, a 32 x 32 block per wave. The
// k index is permuted alike for both operands (lane half h feeds k-block
// [8j + 4h, 8j + 4h + 4) of step group j), so each lane loads float4 rows
// and the dot product covers every k once.
__global__ __launch_bounds__(256) void ivf_coarse_mfma(const float* __restrict__ Qp, int ld, int nq,
                                                       const float* __restrict__ qn,
                                                       const float* __restrict__ C, int produced,
                                                       const float* __restrict__ cn, int cst,
                                                       float* __restrict__ A) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int qrow = blockIdx.x * 64 + (w & 1) * 32 + r;
  const int crow = blockIdx.y * 64 + (w >> 1) * 32 + r;
  const float* qp = Qp + (size_t)min(qrow, nq - 1) * ld + 4 * h;
  const float* cp = C + (size_t)min(crow, produced - 1) * ld + 4 * h;
  fv16 acc;
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
  for (int k = 0; k < ld; k += 8) {
    const float4 a4 = *reinterpret_cast<const float4*>(qp + k);
    const float4 b4 = *reinterpret_cast<const float4*>(cp + k);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.x, b4.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.y, b4.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.z, b4.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.w, b4.w, acc, 0, 0, 0);
  }
  // lane holds rows 8 (v/4) + 4 h + v%4 (queries) of column r (list)
  const int l = blockIdx.y * 64 + (w >> 1) * 32 + r;
  if (l >= produced) return;
  const float c2 = cn[l] * cn[l];
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int q = blockIdx.x * 64 + (w & 1) * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
    if (q < nq) {
      const float q2 = qn[q] * qn[q];
      A[(size_t)q * cst + l] = (q2 + c2) - 2.0f * acc[v];
    }
  }
}

// Phase two, one workgroup per query (see above); writes the probes in (D,
// list) order and adds their list lengths to *scanned.
__global__ __launch_bounds__(256) void ivf_coarse_pick_approx(const float* __restrict__ A, int cst, int produced,
                                                              int np, const float* __restrict__ Qp, int ld, int dim,
                                                              const float* __restrict__ qn,
                                                              const float* __restrict__ C,
                                                              const float* __restrict__ cn,
                                                              int* __restrict__ probes,
                                                              const uint32_t* __restrict__ list_beg,
                                                              const uint32_t* __restrict__ list_end,
                                                              unsigned long long* __restrict__ scanned,
                                                              uint32_t* __restrict__ qwork) {
  const int q = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  __shared__ uint64_t cand[IVF_PICK_CAP];
  __shared__ int cl[IVF_PICK_CAP];
  __shared__ float gmin[64];
  __shared__ int hist[256];
  __shared__ uint64_t sh[4];
  __shared__ int ncand;
  __shared__ float s_t;
  const float* a = A + (size_t)q * cst;
  const float qv = qn[q];
  const float ef = 4.0f * (float)dim * 5.9604645e-08f;
  const float* qrow = Qp + (size_t)q * ld;
  auto eps = [&](int l) {
    const float s = qv + cn[l];
    return ef * s * s * 1.0001f + 1e-30f;
  };
  const int ng = min(64, produced), gs = (produced + ng - 1) / ng;
  if (tid == 0) ncand = 0;
  // Groups of up to 64 lists (up to 4096 lists): thread 4 g + u holds lists
  // g gs + u + 4 j of group g, all loaded at once, and keeps a - eps of each
  // for the candidate test, so the lists are read once.
  const bool held = gs <= 64;
  float lo[16];
  if (held) {
    const int g = tid >> 2, u = tid & 3;
    const int b = g * gs, e = g < ng ? min(produced, b + gs) : b;
    float av[16], cv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int i = min(b + u + 4 * j, produced - 1);
      av[j] = a[i];
      cv[j] = cn[i];
    }
    float m = INFINITY;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float sv = qv + cv[j];
      const float ev = ef * sv * sv * 1.0001f + 1e-30f;
      const bool in = b + u + 4 * j < e;
      m = in ? fminf(m, av[j] + ev) : m;
      lo[j] = in ? av[j] - ev : INFINITY;
    }
    m = fminf(m, __shfl_xor(m, 1, 64));
    m = fminf(m, __shfl_xor(m, 2, 64));
    if (u == 0) gmin[g] = m;
  } else {
    for (int g = w; g < 64; g += 4) {
      float m = INFINITY;
      if (g < ng) {
        const int b = g * gs, e = min(produced, b + gs);
        for (int i = b + lane; i < e; i += 64) m = fminf(m, a[i] + eps(i));
      }
#pragma unroll
      for (int st = 32; st > 0; st >>= 1) m = fminf(m, __shfl_xor(m, st, 64));
      if (lane == 0) gmin[g] = m;
    }
  }
  __syncthreads();
  if (w == 0) {
    // the np-th smallest group minimum (np <= ng <= 64); NaN (from overflow)
    // sorts last under the ordered key
    uint64_t v[1] = {lane < ng ? (uint64_t)ord_key(gmin[lane]) : KEY_MAX};
    wave_bitonic_sort<1>(v, lane);
    const uint64_t t = readlane64(v[0], np - 1);
    if (lane == 0) s_t = key_float((uint32_t)t);
  }
  __syncthreads();
  const float t = s_t;
  const bool finite_t = t == t && t < INFINITY;
  if (held && finite_t) {
    const int g = tid >> 2, u = tid & 3, b = g * gs;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (!(lo[j] > t)) {  // NaN a (overflow) is kept and rescored
        const int at = atomicAdd(&ncand, 1);
        if (at < IVF_PICK_CAP) cl[at] = b + u + 4 * j;
      }
    }
  } else {
    for (int i = tid; i < produced && finite_t; i += 256) {
      const float av = a[i];
      if (!(av - eps(i) > t)) {  // NaN a (overflow) is kept and rescored
        const int at = atomicAdd(&ncand, 1);
        if (at < IVF_PICK_CAP) cl[at] = i;
      }
    }
  }
  __syncthreads();
  const int nc = finite_t ? ncand : IVF_PICK_CAP + 1;
  if (nc <= IVF_PICK_CAP) {
    // exact keys of the candidates: 8 threads per list (dist_group8)
    const int g8 = tid & 7;
    for (int c = tid >> 3; c < nc; c += 32) {
      const int l = cl[c];
      const float d = dist_group8<0>(qrow, C + (size_t)l * ld, dim, g8);
      if (g8 == 0) cand[c] = ((uint64_t)ord_key(d) << 32) | (uint32_t)l;
    }
    __syncthreads();
    if (nc <= 64) {
      if (w == 0) {
        uint64_t v[1] = {lane < nc ? cand[lane] : KEY_MAX};
        wave_bitonic_sort<1>(v, lane);
        cand[lane] = v[0];
      }
      __syncthreads();
    } else {
      int P = 128;
      while (P < nc) P <<= 1;
      for (int i = nc + tid; i < P; i += 256) cand[i] = KEY_MAX;
      __syncthreads();
      block_bitonic_sort(cand, P);
    }
  } else {
    // exact keys of every list, radix select of the np-th, then sort
    auto key = [&](int i) -> uint64_t {
      return ((uint64_t)ord_key(dist_thread<0>(qrow, C + (size_t)i * ld, dim)) << 32) | (uint32_t)i;
    };
    const uint64_t pivot = block_radix_select(key, produced, np, hist, sh);
    if (tid == 0) ncand = 0;
    __syncthreads();
    for (int i = tid; i < produced; i += 256) {
      const uint64_t x = key(i);
      if (x <= pivot) cand[atomicAdd(&ncand, 1)] = x;  // np <= 64 of them
    }
    __syncthreads();
    if (w == 0) {
      uint64_t v[1] = {lane < np ? cand[lane] : KEY_MAX};
      wave_bitonic_sort<1>(v, lane);
      cand[lane] = v[0];
    }
    __syncthreads();
  }
  if (w == 0) {
    const int l = (int)(uint32_t)cand[lane];
    if (lane < np) probes[(size_t)q * np + lane] = l;
    uint32_t len = lane < np ? list_end[l] - list_beg[l] : 0u;
#pragma unroll
    for (int st = 32; st > 0; st >>= 1) len += xor_lane_rt(len, st);
    if (lane == 0) atomicAdd(scanned + (q & (IVF_SCAN_SLOTS - 1)), (unsigned long long)len);
    if (lane == 0 && qwork) qwork[q] = len;
  }
}

// |c_l| rounded to f32 (the bound above only needs it within a few ulps)
__global__ void ivf_cent_norms(const float* __restrict__ C, int ld, int dim, int produced, float* __restrict__ cn) {
  const int l = blockIdx.x * blockDim.x + threadIdx.x;
  if (l >= produced) return;
  double s = 0.0;
  for (int j = 0; j < dim; ++j) s += (double)C[(size_t)l * ld + j] * (double)C[(size_t)l * ld + j];
  cn[l] = (float)sqrt(s);
}

__global__ void ivf_transpose_cents(const float* __restrict__ C, int ld, int dim, int produced, int cst,
                                    float* __restrict__ cT) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (size_t)dim * cst) return;
  const int i = (int)(t / cst), c = (int)(t % cst);
  cT[t] = c < produced ? C[(size_t)c * ld + i] : 0.0f;
}

constexpr int IVF_PGMAX = 32;   // probes per scan workgroup, at most
constexpr int IVF_SW = 8;       // waves per scan workgroup

// ADC scan, register-resident codebooks (uniform subspace width W, M*W = dim
// <= 128, shortlist <= 64). One workgroup of 512 threads per (query, group of
// up to IVF_PGMAX probes); thread t holds row t%256 of the codebooks of half
// of the subspaces (t/256 picks the half) in VGPRs. The group's residuals
// are computed up front (one round of global-load latency); then per probe
// the threads build their rows of the distance table (VALU work on
// LDS-broadcast residual vectors) and the 8 waves stream the list: coalesced
// 16-byte codes and 4-byte ranks, ADC sums in subspace order, and a per-wave
// top-kk (sorted keys, one per lane) kept across the whole group.
template <int W, int METRIC>
__global__ __launch_bounds__(IVF_SW * 64) void ivf_scan_reg(const float* __restrict__ Qp, int ld, int dim, int M,
                                                         const int* __restrict__ probes, int nprobe, int pg,
                                                         int groups, const float* __restrict__ cents,
                                                         const float* __restrict__ books,
                                                         const uint32_t* __restrict__ list_beg,
                                                         const uint32_t* __restrict__ list_end,
                                                         const uint32_t* __restrict__ list_slot,
                                                         const uint8_t* __restrict__ list_codes,
                                                         const uint32_t* __restrict__ rank_slot,
                                                         const uint32_t* __restrict__ slot_rank,
                                                         const uint8_t* __restrict__ accept, int kk,
                                                         uint64_t* __restrict__ out, int k,
                                                         const uint64_t* __restrict__ ids,
                                                         uint64_t* __restrict__ out_ids, float* __restrict__ out_d,
                                                         uint32_t* __restrict__ out_count,
                                                         const int* __restrict__ qorder) {
  constexpr int MMAX = 128 / W, MH = (MMAX + 1) / 2;
  extern __shared__ float lut[];  // 2 x M * 256 floats (cosine: one table)
  __shared__ uint64_t s_kept[IVF_SW][64];
  __shared__ __align__(16) float srs[IVF_PGMAX][128];
  __shared__ float s_qdc[IVF_PGMAX];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c = tid & 255, half = tid >> 8;
  const int qi = blockIdx.x / groups, grp = blockIdx.x % groups;
  const int q = qorder ? qorder[qi] : qi;
  const int p0 = grp * pg, np = min(nprobe, p0 + pg) - p0;
  const int mh = (M + 1) / 2;           // subspaces per half
  const int sb = half * mh;             // this thread's first subspace
  const int ns = min(mh, M - sb);       // and how many
  // codebook row c of subspaces sb .. sb+ns-1 (book_off[s] = s*256*W)
  float breg[MH][W];
#pragma unroll
  for (int si = 0; si < MH; ++si)
#pragma unroll
    for (int j = 0; j < W; ++j) breg[si][j] = si < ns ? books[(size_t)(sb + si) * 256 * W + c * W + j] : 0.0f;
  const float* qv = Qp + (size_t)q * ld;
  // residuals of every probe of the group (ivfpq.rs:1052-1054); cosine: the
  // query once and q.c per probe (ivfpq.rs:1042-1045)
  const int nres = METRIC == 0 ? np : 1;
  for (int i = tid; i < nres * dim; i += IVF_SW * 64) {
    const int pi = i / dim, j = i % dim;
    srs[pi][j] = METRIC == 0 ? qv[j] - cents[(size_t)probes[(size_t)q * nprobe + p0 + pi] * ld + j] : qv[j];
  }
  if (METRIC == 1) {
    for (int pi = w; pi < np; pi += IVF_SW) {
      if (lane < 8) {
        const int l = probes[(size_t)q * nprobe + p0 + pi];
        const float d = -dist_group8<2>(qv, cents + (size_t)l * ld, dim, lane);
        if (lane == 0) s_qdc[pi] = d;
      }
    }
  }
  auto build = [&](const float* sr, float* tab) {  // distance_table, product.rs:416-433
#pragma unroll
    for (int si = 0; si < MH; ++si) {
      if (si < ns) {
        const int s2 = sb + si;
        float rv[W];
        if constexpr (W % 4 == 0) {
#pragma unroll
          for (int j = 0; j < W; j += 4) {
            const float4 r4 = *reinterpret_cast<const float4*>(&sr[s2 * W + j]);
            rv[j] = r4.x;
            rv[j + 1] = r4.y;
            rv[j + 2] = r4.z;
            rv[j + 3] = r4.w;
          }
        } else {
#pragma unroll
          for (int j = 0; j < W; ++j) rv[j] = sr[s2 * W + j];
        }
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < W; ++j) {
          if constexpr (METRIC == 0) {
            const float d = rv[j] - breg[si][j];
            acc += d * d;
          } else {
            acc += rv[j] * breg[si][j];
          }
        }
        tab[s2 * 256 + c] = acc;
      }
    }
  };
  // Tables are double-buffered (L2): each wave builds its rows of probe
  // pi+1's table before scanning its share of probe pi, so building and
  // scanning overlap across waves and one barrier per probe suffices.
  const int tsz = M * 256;
  __syncthreads();
  build(srs[0], lut);
  __syncthreads();
  uint64_t kept = KEY_MAX, thr = KEY_MAX;
  for (int pi = 0; pi < np; ++pi) {
    const int l = probes[(size_t)q * nprobe + p0 + pi];
    if (METRIC == 0 && pi + 1 < np) build(srs[pi + 1], lut + ((pi + 1) & 1) * tsz);
    const float* tab = lut + (METRIC == 0 ? (pi & 1) * tsz : 0);
    const float one_minus_qdc = METRIC == 1 ? arm_nan(1.0f - s_qdc[pi]) : 0.0f;
    const uint32_t begin = list_beg[l], end = list_end[l];
    for (uint32_t e0 = begin + w * 64; e0 < end; e0 += IVF_SW * 64) {
      const uint32_t e = e0 + lane;
      uint64_t key = KEY_MAX;
      if (e < end) {
        const uint32_t sl = list_slot[e];
        if (accept == nullptr || accept[sl]) {
          const uint32_t rk = slot_rank[sl];
          float sum = 0.0f;  // DistanceTable::squared_l2 / inner_product, product.rs:580-603
          if (M == 16) {
            const uint4 cw = *reinterpret_cast<const uint4*>(list_codes + (size_t)e * 16);
            const uint32_t wv[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
            for (int s2 = 0; s2 < 16; ++s2) sum += tab[s2 * 256 + ((wv[s2 >> 2] >> (8 * (s2 & 3))) & 255)];
          } else {
            const uint8_t* code = list_codes + (size_t)e * M;
            for (int s2 = 0; s2 < M; ++s2) sum += tab[s2 * 256 + code[s2]];
          }
          const float score = METRIC == 0 ? sum : ivf_cos_score(one_minus_qdc, sum);
          key = ((uint64_t)ord_key(score) << 32) | rk;
        }
      }
      wave_topk_add(key, kept, thr, kk, lane);
    }
    __syncthreads();  // table pi+1 complete; table pi free for pi+2
  }
  if (out_ids == nullptr) {
    uint64_t* o = out + (((size_t)q * groups + grp) * IVF_SW + w) * kk;
    if (lane < kk) o[lane] = kept;
    return;
  }
  // One group per query and no rerank: merge the waves' sorted lists here
  // (bitonic half-cleaners) and write the query's results.
  s_kept[w][lane] = kept;
  __syncthreads();
  if (w == 0) {
    uint64_t v = s_kept[0][lane];
    for (int ww = 1; ww < IVF_SW; ++ww) wave_merge_sorted(v, s_kept[ww][lane], lane);
    const int n = min(k, (int)__popcll(__ballot(v != KEY_MAX)));
    if (lane < n) {
      out_ids[(size_t)q * k + lane] = ids[rank_slot[(uint32_t)v]];
      out_d[(size_t)q * k + lane] = key_float((uint32_t)(v >> 32));
    }
    if (lane == 0) out_count[q] = (uint32_t)n;
  }
}

// ---------------------------------------------------------------------------
// ADC scan for 16 subspaces (16-byte codes), the common IVF-PQ shape: the
// same work split as ivf_scan_reg, with the list stream staged through LDS
// by the waves' own asynchronous loads so that HBM latency is hidden without
// holding the data in VGPRs.
//
// Each wave owns a ring of IVF_NS chunk slots (64 entries: 1 KiB of codes)
// and walks the group's (probe, 64-entry chunk) sequence
// twice: a producer cursor issues global->LDS copies (global_load_lds,
// vmcnt-tracked) up to IVF_NS chunks ahead, refilling each slot as soon as it
// has been read, and the consumer cursor waits for its chunk with s_waitcnt
// vmcnt and scores it. The copies cross probe boundaries (they
// need no table), so the stream does not drain at the per-probe barrier.
// Tables live at fixed LDS offsets (the probe loop is unrolled by two for the
// double buffer), so every lookup is one SDWA byte-select shift plus one
// ds_read_b32 with an immediate offset.
// ---------------------------------------------------------------------------
constexpr int IVF_NS = 3;                       // staged chunks per wave (all in flight)
constexpr int IVF_CHUNK = 64 * 16;              // codes of 64 entries

typedef __attribute__((address_space(3))) uint8_t lds_byte;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_byte*)p;
}

// Global -> LDS copy; lane i's 16 bytes land at m0 + 16*i; lanes off in exec
// copy nothing. Written as inline asm so that the
// compiler neither sees LDS writes pending behind vmcnt (it would drain them
// with vmcnt(0) at every barrier) nor schedules around them: the consumer
// waits with an explicit vmcnt. The asm sets m0 itself; the kernels that use
// these copies keep no value of their own in m0 (no dynamic register
// indexing, no LDS-DMA builtins, no messages), so the clobber of the
// reserved register is harmless there.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_copy16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g) : "memory", "m0");
}
#pragma clang diagnostic pop
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N <= 15, "immediate vmcnt");
  if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if constexpr (N == 1) asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
  else if constexpr (N == 2) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
  else if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else if constexpr (N == 6) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  else static_assert(N == 0, "unsupported count");
}

// Byte B of x times 4 (the byte offset of a table entry): one SDWA shift.
template <int B>
__device__ __forceinline__ uint32_t byte_x4(uint32_t x) {
  uint32_t r;
  if constexpr (B == 0)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
        : "=v"(r) : "v"(x));
  else if constexpr (B == 1)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
        : "=v"(r) : "v"(x));
  else if constexpr (B == 2)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
        : "=v"(r) : "v"(x));
  else
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
        : "=v"(r) : "v"(x));
  return r;
}

template <int S>
__device__ __forceinline__ float lut_at(const float* tab, const uint32_t (&wv)[4]) {
  return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(tab) + S * 1024 +
                                         byte_x4<S & 3>(wv[S >> 2]));
}

// DistanceTable::squared_l2 / inner_product (product.rs:580-603) over one
// 16-byte code: sum = 0.0 + t0 + t1 + ... + t15 in subspace order. Table
// entries are never -0.0 (each starts from +0.0), so starting the sum at t0
// gives the same bits as adding t0 to 0.0.
__device__ __forceinline__ float adc16(const float* tab, const uint4& cw) {
  const uint32_t wv[4] = {cw.x, cw.y, cw.z, cw.w};
  float s = lut_at<0>(tab, wv);
  s += lut_at<1>(tab, wv);
  s += lut_at<2>(tab, wv);
  s += lut_at<3>(tab, wv);
  s += lut_at<4>(tab, wv);
  s += lut_at<5>(tab, wv);
  s += lut_at<6>(tab, wv);
  s += lut_at<7>(tab, wv);
  s += lut_at<8>(tab, wv);
  s += lut_at<9>(tab, wv);
  s += lut_at<10>(tab, wv);
  s += lut_at<11>(tab, wv);
  s += lut_at<12>(tab, wv);
  s += lut_at<13>(tab, wv);
  s += lut_at<14>(tab, wv);
  s += lut_at<15>(tab, wv);
  return s;
}

template <int W, int METRIC>
__global__ __launch_bounds__(IVF_SW * 64) void ivf_scan16(const float* __restrict__ Qp, int ld,
                                                          const int* __restrict__ probes, int nprobe, int pg,
                                                          int groups, const float* __restrict__ cents,
                                                          const float* __restrict__ books,
                                                          const uint32_t* __restrict__ list_beg,
                                                          const uint32_t* __restrict__ list_end,
                                                          const uint32_t* __restrict__ list_slot,
                                                          const uint8_t* __restrict__ list_codes,
                                                          const uint32_t* __restrict__ rank_slot,
                                                          const uint32_t* __restrict__ slot_rank,
                                                          const uint8_t* __restrict__ accept, int kk,
                                                          uint64_t* __restrict__ out, int k,
                                                          const uint64_t* __restrict__ ids,
                                                          uint64_t* __restrict__ out_ids, float* __restrict__ out_d,
                                                          uint32_t* __restrict__ out_count,
                                                          const int* __restrict__ qorder) {
  constexpr int M = 16, DIM = 16 * W, MH = 8, NT = METRIC == 0 ? 2 : 1;
  __shared__ __align__(16) float tabs[NT][M * 256];
  __shared__ __align__(16) float srs[IVF_PGMAX][DIM];
  __shared__ float s_qdc[IVF_PGMAX];
  __shared__ uint32_t s_lb[IVF_PGMAX], s_le[IVF_PGMAX];  // the group's list ranges
  __shared__ __align__(16) uint8_t ring[IVF_SW][IVF_NS][IVF_CHUNK];
  __shared__ uint2 cbuf[IVF_SW][64];  // each wave's pending candidates: (distance key, list entry)
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  // thread t builds subspace ts = t/32 of every table, centroid rows
  // t%32 + 32*(i ^ (ts&1)), i < 8: one residual slice per table, and the two
  // half-waves (even and odd subspace) write distinct banks at every store
  const int ts = tid >> 5, g = tid & 31, flip = ts & 1;
  const int qi = blockIdx.x / groups, grp = blockIdx.x % groups;
  const int q = qorder ? qorder[qi] : qi;
  const int p0 = grp * pg, np = min(nprobe, p0 + pg) - p0;
  const int* pq = probes + (size_t)q * nprobe + p0;
  float breg[MH][W];
#pragma unroll
  for (int i = 0; i < MH; ++i)
#pragma unroll
    for (int j = 0; j < W; ++j) breg[i][j] = books[((size_t)ts * 256 + g + 32 * (i ^ flip)) * W + j];
  const float* qv = Qp + (size_t)q * ld;
  // residuals of the group's probes (ivfpq.rs:1052-1054); cosine: the query
  // once and q.c per probe (ivfpq.rs:1042-1045)
  const int nres = METRIC == 0 ? np : 1;
  for (int i = tid; i < nres * DIM; i += IVF_SW * 64) {
    const int pi = i / DIM, j = i % DIM;
    srs[pi][j] = METRIC == 0 ? qv[j] - cents[(size_t)pq[pi] * ld + j] : qv[j];
  }
  if (tid < np) {
    s_lb[tid] = list_beg[pq[tid]];
    s_le[tid] = list_end[pq[tid]];
  }
  if (METRIC == 1) {
    for (int pi = w; pi < np; pi += IVF_SW) {
      if (lane < 8) {
        const float d = -dist_group8<2>(qv, cents + (size_t)pq[pi] * ld, DIM, lane);
        if (lane == 0) s_qdc[pi] = d;
      }
    }
  }
  // distance_table (product.rs:416-433): per entry, in dimension order,
  // d = r - c; l2 += d*d (ip += r*c). The L2 sum starts at d0*d0, which is
  // what 0.0 + d0*d0 gives (a square is never -0.0); the inner product keeps
  // the 0.0 start, which turns a -0.0 first product into +0.0.
  auto load_slice = [&](const float* sr, float (&rv)[W]) {
    if constexpr (W % 4 == 0) {
#pragma unroll
      for (int j = 0; j < W; j += 4) {
        const float4 r4 = *reinterpret_cast<const float4*>(&sr[ts * W + j]);
        rv[j] = r4.x;
        rv[j + 1] = r4.y;
        rv[j + 2] = r4.z;
        rv[j + 3] = r4.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < W; ++j) rv[j] = sr[ts * W + j];
    }
  };
  // entries I .. I+N-1 of this thread's share of a table
  auto build_part = [&](auto ic, auto nc, const float (&rv)[W], float* tab) {
    constexpr int I = decltype(ic)::value, N = decltype(nc)::value;
#pragma unroll
    for (int i = I; i < I + N; ++i) {
      float acc;
      if constexpr (METRIC == 0) {
        const float d0 = rv[0] - breg[i][0];
        acc = d0 * d0;
#pragma unroll
        for (int j = 1; j < W; ++j) {
          const float d = rv[j] - breg[i][j];
          acc += d * d;
        }
      } else {
        acc = 0.0f;
#pragma unroll
        for (int j = 0; j < W; ++j) acc += rv[j] * breg[i][j];
      }
      tab[ts * 256 + g + 32 * (i ^ flip)] = acc;
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I2 = std::integral_constant<int, 2>;
  using I4 = std::integral_constant<int, 4>;
  using I6 = std::integral_constant<int, 6>;
  using I8 = std::integral_constant<int, 8>;

  // Cursors over this wave's chunks of the group: chunk (p, e) covers
  // entries e .. e+63 of probe p's list (e advances by 512, the group's
  // stride); seek moves past exhausted lists.
  auto open = [&](int p, uint32_t& e, uint32_t& end) {
    e = __builtin_amdgcn_readfirstlane(s_lb[p]) + (uint32_t)w * 64;
    end = __builtin_amdgcn_readfirstlane(s_le[p]);
  };
  auto seek = [&](int& p, uint32_t& e, uint32_t& end) {
    while (p < np && e >= end)
      if (++p < np) open(p, e, end);
  };
  __syncthreads();
  int pp = 0, cp;
  uint32_t pe, pend, ce, cend;
  open(0, pe, pend);
  seek(pp, pe, pend);
  cp = pp;
  ce = pe;
  cend = pend;
  int issued = 0, consumed = 0;
  uint8_t* myring = &ring[w][0][0];
  auto issue = [&]() __attribute__((always_inline)) {
    uint8_t* slot = myring + (issued % IVF_NS) * IVF_CHUNK;
    const uint32_t e = pe + lane;
    const uint32_t a = __builtin_amdgcn_readfirstlane(lds_addr(slot));
    if (e < pend) lds_copy16(list_codes + (size_t)e * 16, a);
    ++issued;
    pe += IVF_SW * 64;
    seek(pp, pe, pend);
  };
  for (int i = 0; i < IVF_NS - 1 && pp < np; ++i) issue();
  {
    float rv[W];
    load_slice(srs[0], rv);
    build_part(I0{}, I8{}, rv, tabs[0]);
  }
  __syncthreads();
  // the wave's best keys, ascending, one per lane: kept the first 64 and,
  // for a shortlist above 64, kept2 the next 64
  uint64_t kept = KEY_MAX, kept2 = KEY_MAX, thr = KEY_MAX;
  // Candidates are screened on the distance key alone: an entry whose key
  // exceeds the distance of the wave's kk-th kept key cannot enter the wave's
  // top kk, whatever its id rank. The rest (ties included) wait in cbuf as
  // (distance key, list entry); a flush fetches their id ranks (and applies
  // the filter), sorts the full keys and merges them into `kept`. The list
  // stream therefore carries codes only: ranks are read for the few entries
  // that pass, and the screen threshold only tightens, at flushes.
  uint32_t thr_d = 0xFFFFFFFFu;  // distance part of thr
  int ncand = 0;                 // pending candidates (wave-uniform)
  auto flush = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    uint64_t b[1] = {KEY_MAX};
    if (lane < ncand) {
      const uint2 c = cbuf[w][lane];
      const uint32_t sl = list_slot[c.y];
      if (accept == nullptr || accept[sl]) b[0] = ((uint64_t)c.x << 32) | slot_rank[sl];
    }
    wave_bitonic_sort<1>(b, lane);
    if (kk > 64) {
      // the 64 smallest of kept and the batch stay first; the rest competes
      // with kept2 for the next 64 (no key of kept2 is below any of kept)
      uint64_t lo, hi;
      wave_merge_split(kept, b[0], lane, lo, hi);
      kept = lo;
      wave_merge_sorted(kept2, hi, lane);
      thr = readlane64(kept2, kk - 65);
    } else {
      wave_merge_sorted(kept, b[0], lane);
      thr = readlane64(kept, kk - 1);
    }
    thr_d = (uint32_t)(thr >> 32);
    ncand = 0;
    // The rank and filter loads above were waited with vmcnt(0) before use.
    // Say so to the compiler with a wait it can see, or its wait bookkeeping
    // carries them as possibly pending into every chunk and drains the ring
    // copies (vmcnt(0)) before each chunk's lookups.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt and lgkmcnt unconstrained
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  // One consumer iteration: refill the slot read in the previous iteration
  // (its reads are done), wait for this chunk (the chunks issued after it
  // stay in flight), score it and queue the entries that pass the screen.
  auto chunk = [&](const float* tab, float one_minus_qdc) __attribute__((always_inline)) {
    if (pp < np) issue();
    static_assert(IVF_NS <= 3, "the waits below cover up to two later chunks");
    const int later = issued - consumed - 1;
    if (later >= 2) vm_wait<2>();
    else if (later == 1) vm_wait<1>();
    else vm_wait<0>();
    const uint8_t* slot = myring + (consumed % IVF_NS) * IVF_CHUNK;
    const uint4 cw = *reinterpret_cast<const uint4*>(slot + lane * 16);
    const uint32_t e = ce + lane;
    const bool valid = e < cend;
    ++consumed;
    ce += IVF_SW * 64;
    seek(cp, ce, cend);
    uint32_t dk = 0xFFFFFFFFu;
    if (valid) {
      const float sum = adc16(tab, cw);
      // L2: sums of squares are in [+0, +inf], so the order key is the bits
      // with the sign bit set
      dk = METRIC == 0 ? (__float_as_uint(sum) | 0x80000000u) : ord_key(ivf_cos_score(one_minus_qdc, sum));
    }
    bool pass = valid && dk <= thr_d;
    uint64_t m = __ballot(pass);
    if (m == 0) return;
    if (ncand + __popcll(m) > 64) {
      flush();
      pass = pass && dk <= thr_d;
      m = __ballot(pass);
    }
    if (pass) {
      const int pos = ncand + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                            __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
      cbuf[w][pos] = make_uint2(dk, e);
    }
    ncand += __popcll(m);
  };
  // Probe pi scans table B while building table B^1 for probe pi+1 (L2),
  // two entries per thread between the first chunks so that the build's VALU
  // work overlaps the lookups' LDS latency.
  auto probe_step = [&](auto bc, int pi) __attribute__((always_inline)) {
    constexpr int B = decltype(bc)::value;
    const float* tab = tabs[METRIC == 0 ? B : 0];
    const float one_minus_qdc = METRIC == 1 ? arm_nan(1.0f - s_qdc[pi]) : 0.0f;
    if (METRIC == 0 && pi + 1 < np) {
      float* nt = tabs[METRIC == 0 ? (B ^ 1) : 0];
      float rv[W];
      load_slice(srs[pi + 1], rv);
      build_part(I0{}, I2{}, rv, nt);
      if (cp == pi) chunk(tab, one_minus_qdc);
      build_part(I2{}, I2{}, rv, nt);
      if (cp == pi) chunk(tab, one_minus_qdc);
      build_part(I4{}, I2{}, rv, nt);
      if (cp == pi) chunk(tab, one_minus_qdc);
      build_part(I6{}, I2{}, rv, nt);
    }
    while (cp == pi) chunk(tab, one_minus_qdc);
    __syncthreads();  // table pi+1 complete; table pi free for pi+2
  };
  for (int pi = 0; pi < np; pi += 2) {
    probe_step(std::integral_constant<int, 0>{}, pi);
    if (pi + 1 < np) probe_step(std::integral_constant<int, 1>{}, pi + 1);
  }
  if (ncand) flush();
  if (out_ids == nullptr) {
    uint64_t* o = out + (((size_t)q * groups + grp) * IVF_SW + w) * kk;
    if (lane < kk) o[lane] = kept;
    if (64 + lane < kk) o[64 + lane] = kept2;
    return;
  }
  // One group per query and no rerank: merge the waves' sorted lists here
  // and write the query's results. Every copy has landed (the last chunk was
  // waited with vmcnt(0)), so the rings are free.
  uint64_t* s_kept = reinterpret_cast<uint64_t*>(&ring[0][0][0]);
  s_kept[w * 64 + lane] = kept;
  __syncthreads();
  if (w == 0) {
    uint64_t v = s_kept[lane];
    for (int ww = 1; ww < IVF_SW; ++ww) wave_merge_sorted(v, s_kept[ww * 64 + lane], lane);
    const int n = min(k, (int)__popcll(__ballot(v != KEY_MAX)));
    if (lane < n) {
      out_ids[(size_t)q * k + lane] = ids[rank_slot[(uint32_t)v]];
      out_d[(size_t)q * k + lane] = key_float((uint32_t)(v >> 32));
    }
    if (lane == 0) out_count[q] = (uint32_t)n;
  }
}

// ---------------------------------------------------------------------------
// merge over probes (+ optional exact rerank)
// ---------------------------------------------------------------------------
constexpr int IVF_MAX_SHORT = 960;

__global__ __launch_bounds__(256) void ivf_merge(const uint64_t* __restrict__ cand, int n_per_q, int kk, int k,
                                                 int rerank, const float* __restrict__ Qp, int ld, int dim,
                                                 int metric, const float* __restrict__ X,
                                                 const uint32_t* __restrict__ rank_slot,
                                                 const uint64_t* __restrict__ ids, uint64_t* __restrict__ out_ids,
                                                 float* __restrict__ out_d, uint32_t* __restrict__ out_count) {
  const int q = blockIdx.x;
  __shared__ int hist[256];
  __shared__ uint64_t sh[4];
  __shared__ uint64_t sel[1024];
  __shared__ int n_sel, n_valid;
  const uint64_t* base = cand + (size_t)q * n_per_q;
  auto get = [&](int i) -> uint64_t { return base[i]; };
  if (threadIdx.x == 0) {
    n_sel = 0;
    n_valid = 0;
  }
  __syncthreads();
  int local = 0;
  // four keys per thread per step, loaded together before any is used
  for (int i0 = threadIdx.x; i0 < n_per_q; i0 += 4 * blockDim.x) {
    uint64_t x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = base[min(i0 + u * (int)blockDim.x, n_per_q - 1)];
#pragma unroll
    for (int u = 0; u < 4; ++u) local += (i0 + u * (int)blockDim.x < n_per_q && x[u] != KEY_MAX) ? 1 : 0;
  }
  atomicAdd(&n_valid, local);
  __syncthreads();
  const int ksel = min(kk, n_valid);
  if (ksel == 0) {
    if (threadIdx.x == 0) out_count[q] = 0;
    return;
  }
  const uint64_t pivot = n_per_q <= 16 * (int)blockDim.x
                             ? block_radix_select<decltype(get), 64, 16>(get, n_per_q, ksel, hist, sh)
                             : block_radix_select(get, n_per_q, ksel, hist, sh);
  for (int i0 = threadIdx.x; i0 < n_per_q; i0 += 4 * blockDim.x) {
    uint64_t x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = base[min(i0 + u * (int)blockDim.x, n_per_q - 1)];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (i0 + u * (int)blockDim.x < n_per_q && x[u] <= pivot && x[u] != KEY_MAX) sel[atomicAdd(&n_sel, 1)] = x[u];
  }
  __syncthreads();
  int P = 1;
  while (P < ksel) P <<= 1;
  for (int i = ksel + threadIdx.x; i < P; i += blockDim.x) sel[i] = KEY_MAX;
  __syncthreads();
  block_bitonic_sort(sel, P);
  int kout = min(k, ksel);
  if (rerank) {
    // exact rescoring of the shortlist (ivfpq.rs:1098-1109): two lanes per
    // candidate (dist_pair4, the same bits as dist_group8), eight for rows
    // narrower than one 8-wide chunk
    const float* qv = Qp + (size_t)q * ld;
    if (dim >= 8) {
      const int h = threadIdx.x & 1;
      for (int c = threadIdx.x >> 1; c < ksel; c += (int)blockDim.x / 2) {
        const uint32_t rk = (uint32_t)sel[c];
        const float d = dist_pair4_rt(metric, qv, X + (size_t)rank_slot[rk] * ld, dim, h);
        if (h == 0) sel[c] = ((uint64_t)ord_key(d) << 32) | rk;
      }
    } else {
      const int g = threadIdx.x & 7, grp = threadIdx.x >> 3;
      for (int c = grp; c < ksel; c += 32) {
        const uint32_t rk = (uint32_t)sel[c];
        const float d = dist_group8_rt(metric, qv, X + (size_t)rank_slot[rk] * ld, dim, g);
        if (g == 0) sel[c] = ((uint64_t)ord_key(d) << 32) | rk;
      }
    }
    __syncthreads();
    block_bitonic_sort(sel, P);
  }
  for (int i = threadIdx.x; i < kout; i += blockDim.x) {
    const uint64_t key = sel[i];
    out_ids[(size_t)q * k + i] = ids[rank_slot[(uint32_t)key]];
    out_d[(size_t)q * k + i] = key_float((uint32_t)(key >> 32));
  }
  if (threadIdx.x == 0) out_count[q] = kout;
}

__global__ void ivf_probes_from_ids(const uint64_t* __restrict__ ids, int n, int* __restrict__ probes) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) probes[i] = (int)ids[i];
}

// Longest first: the scan's workgroups take queries in descending order of
// the entries their probes hold (buckets of 256 entries), so the last
// workgroups of a batch are short ones and the tail of the launch is short.
// Each query's results come from its own workgroup whatever the order.
constexpr int LPT_BUCKETS = 1024, LPT_MAXQ = 8192;
__global__ __launch_bounds__(1024) void ivf_lpt_order(const uint32_t* __restrict__ qwork, int nq,
                                                      int* __restrict__ qorder) {
  __shared__ uint32_t cnt[LPT_BUCKETS];
  __shared__ uint16_t key[LPT_MAXQ];
  __shared__ uint32_t wsum[16];
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  cnt[t] = 0;
  __syncthreads();
  for (int q = t; q < nq; q += 1024) {
    const uint32_t b = (uint32_t)(LPT_BUCKETS - 1) - min(qwork[q] >> 8, (uint32_t)(LPT_BUCKETS - 1));
    key[q] = (uint16_t)b;
    atomicAdd(&cnt[b], 1u);
  }
  __syncthreads();
  // exclusive prefix over the buckets: wave scans joined through the wave totals
  const uint32_t v = cnt[t];
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[wid] = x;
  __syncthreads();
  uint32_t before = 0;
  for (int i = 0; i < wid; ++i) before += wsum[i];
  __syncthreads();
  cnt[t] = before + x - v;
  __syncthreads();
  for (int q = t; q < nq; q += 1024) qorder[atomicAdd(&cnt[key[q]], 1u)] = q;
}

__global__ void ivf_count_scanned(const int* __restrict__ probes, int n, const uint32_t* __restrict__ list_beg,
                                  const uint32_t* __restrict__ list_end,
                                  unsigned long long* __restrict__ total) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int l = probes[i];
  atomicAdd(total + (i & (IVF_SCAN_SLOTS - 1)), (unsigned long long)(list_end[l] - list_beg[l]));
}

__global__ void ivf_gather_rows(const float* __restrict__ X, int ld, const uint32_t* __restrict__ rows, int n,
                                int dim, float* __restrict__ out) {
  const int i = blockIdx.x;
  if (i >= n) return;
  for (int j = threadIdx.x; j < dim; j += blockDim.x) out[(size_t)i * dim + j] = X[(size_t)rows[i] * ld + j];
}

// First non-finite value of n rows (row-major order): the vector and
// component `space.validate` reports first (space.rs:104-121).
__global__ void ivf_first_nonfinite(const float* __restrict__ R, size_t n, int dim, unsigned long long* bad) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * (size_t)dim) return;
  if (!isfinite(R[i])) atomicMin(bad, ((unsigned long long)(i / dim) << 32) | (unsigned)(i % dim));
}

__global__ void ivf_residuals(const float* __restrict__ S, const float* __restrict__ C, const uint32_t* __restrict__ a,
                              int dim, float* __restrict__ R) {
  const int i = blockIdx.x;
  for (int j = threadIdx.x; j < dim; j += blockDim.x)
    R[(size_t)i * dim + j] = S[(size_t)i * dim + j] - C[(size_t)a[i] * dim + j];
}

__global__ void ivf_scatter_u32(const uint32_t* __restrict__ idx, const uint32_t* __restrict__ val, int n,
                                uint32_t* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[idx[i]] = val[i];
}

// Codes and list assignments of n compactly encoded rows, to their slots.
__global__ void ivf_scatter_codes(const uint8_t* __restrict__ tmp, const uint32_t* __restrict__ sl,
                                  const uint32_t* __restrict__ as, int n, int M, uint8_t* __restrict__ codes,
                                  uint32_t* __restrict__ list_of) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const size_t s = sl[i];
  for (int j = 0; j < M; ++j) codes[s * M + j] = tmp[(size_t)i * M + j];
  list_of[s] = as[i];
}

// ---------------------------------------------------------------------------
// Wide path (shortlist beyond the block selections, or tables beyond the
// LDS): per (query, probe) item, a distance table in device memory, the ADC
// keys of every entry of the probed list into the query's segment, then the
// segmented sort and optional rerank of wide.hpp.
// ---------------------------------------------------------------------------
// Table of item i = q * np + p (grid: items of queries q0 .. q0 + G - 1), the
// loop of product.rs:416-433 per (subspace, centroid): L2 on the residual
// q - c_list (ivfpq.rs:1052-1054), cosine on the query; for cosine also
// omq = 1 - q.c_list (ivfpq.rs:1068-1072).
__global__ __launch_bounds__(256) void ivf_wide_tables(const float* __restrict__ Qp, int ld, int dim, int M,
                                                       int metric, const int* __restrict__ probes, int np, int q0,
                                                       const float* __restrict__ cents,
                                                       const float* __restrict__ books,
                                                       const int* __restrict__ sub_off,
                                                       const int* __restrict__ book_off, float* __restrict__ tables,
                                                       float* __restrict__ omq) {
  const int item = blockIdx.x;
  const int q = q0 + item / np;
  const int l = probes[(size_t)q0 * np + item];
  const float* qv = Qp + (size_t)q * ld;
  const float* cv = cents + (size_t)l * ld;
  float* tab = tables + (size_t)item * M * 256;
  for (int e = threadIdx.x; e < M * 256; e += blockDim.x) {
    const int sidx = e >> 8, c = e & 255;
    const int o = sub_off[sidx], w = sub_off[sidx + 1] - o;
    const float* b = books + book_off[sidx] + c * w;
    float acc = 0.0f;
    for (int j = 0; j < w; ++j) {
      if (metric == 0) {
        const float r = qv[o + j] - cv[o + j];
        const float d = r - b[j];
        acc += d * d;
      } else {
        acc += qv[o + j] * b[j];
      }
    }
    tab[e] = acc;
  }
  if (metric == 1 && threadIdx.x < 8) {
    const float d = -dist_group8<2>(qv, cv, dim, threadIdx.x);
    if (threadIdx.x == 0) omq[item] = arm_nan(1.0f - d);
  }
}

// ADC keys of every entry of item i's list, at pofs[i] onwards (same sums and
// scores as the scans: DistanceTable::squared_l2 / inner_product,
// product.rs:580-603, in subspace order).
__global__ __launch_bounds__(256) void ivf_wide_keys(const int* __restrict__ probes, int np, int q0, int M,
                                                     int metric, const float* __restrict__ tables,
                                                     const float* __restrict__ omq,
                                                     const uint32_t* __restrict__ list_beg,
                                                     const uint32_t* __restrict__ list_end,
                                                     const uint32_t* __restrict__ list_slot,
                                                     const uint8_t* __restrict__ list_codes,
                                                     const uint32_t* __restrict__ rank_slot,
                                                     const uint32_t* __restrict__ slot_rank,
                                                     const uint8_t* __restrict__ accept,
                                                     const uint32_t* __restrict__ pofs, uint64_t* __restrict__ keys) {
  const int item = blockIdx.x;
  const int l = probes[(size_t)q0 * np + item];
  const float* tab = tables + (size_t)item * M * 256;
  const uint32_t begin = list_beg[l], end = list_end[l];
  uint64_t* out = keys + pofs[item];
  const float om = metric == 1 ? omq[item] : 0.0f;
  for (uint32_t e = begin + threadIdx.x; e < end; e += blockDim.x) {
    const uint32_t sl = list_slot[e];
    uint64_t key = KEY_MAX;
    if (accept == nullptr || accept[sl]) {
      const uint32_t rk = slot_rank[sl];
      const uint8_t* code = list_codes + (size_t)e * M;
      float sum = 0.0f;
      for (int sidx = 0; sidx < M; ++sidx) sum += tab[sidx * 256 + code[sidx]];
      const float score = metric == 0 ? sum : ivf_cos_score(om, sum);
      key = ((uint64_t)ord_key(score) << 32) | rk;
    }
    out[e - begin] = key;
  }
}

// Exact rescoring of the first min(t, len) keys of each segment (the rerank
// of ivfpq.rs:1094-1109), from `sorted` into the same positions of `keys`.
// Grid (ceil(t / 32), G), 8 threads per candidate.
__global__ __launch_bounds__(256) void ivf_wide_rerank(const uint64_t* __restrict__ sorted,
                                                       const uint32_t* __restrict__ begins,
                                                       const uint32_t* __restrict__ ends, uint64_t t, int q0,
                                                       const float* __restrict__ Qp, int ld, int dim, int metric,
                                                       const float* __restrict__ X,
                                                       const uint32_t* __restrict__ rank_slot,
                                                       uint64_t* __restrict__ keys) {
  const int gq = blockIdx.y;
  const uint64_t len = ends[gq] - begins[gq];
  const uint64_t take = t < len ? t : len;
  const uint64_t i = (uint64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  const int g = threadIdx.x & 7;
  if (i >= take) return;
  const uint64_t key = sorted[begins[gq] + i];
  uint64_t nk = KEY_MAX;
  if (key != KEY_MAX) {
    const uint32_t rk = (uint32_t)key;
    const float d = dist_group8_rt(metric, Qp + (size_t)(q0 + gq) * ld, X + (size_t)rank_slot[rk] * ld, dim, g);
    nk = ((uint64_t)ord_key(d) << 32) | rk;
  }
  if (g == 0) keys[begins[gq] + i] = nk;
}

// Compaction (ivfpq.rs:907-975): new slot i takes old slot keep[i].
__global__ void ivf_compact_rows(const uint32_t* __restrict__ keep, int n, int ld, int M, const float* __restrict__ X0,
                                 float* __restrict__ X1, const uint8_t* __restrict__ c0, uint8_t* __restrict__ c1,
                                 const uint32_t* __restrict__ l0, uint32_t* __restrict__ l1,
                                 const uint64_t* __restrict__ i0, uint64_t* __restrict__ i1,
                                 const uint32_t* __restrict__ r0, uint32_t* __restrict__ r1,
                                 uint8_t* __restrict__ live1) {
  const int i = blockIdx.x;
  if (i >= n) return;
  const size_t o = keep[i];
  if (X0 != nullptr)
    for (int c = threadIdx.x; c < ld; c += blockDim.x) X1[(size_t)i * ld + c] = X0[o * ld + c];
  for (int j = threadIdx.x; j < M; j += blockDim.x) c1[(size_t)i * M + j] = c0[o * M + j];
  if (threadIdx.x == 0) {
    l1[i] = l0[o];
    i1[i] = i0[o];
    r1[i] = r0[o];
    live1[i] = 1;
  }
}

// rank_slot[r] = new_of_old[rank_slot[r]]
__global__ void ivf_remap_slots(uint32_t* __restrict__ rank_slot, uint32_t len,
                                const uint32_t* __restrict__ new_of_old) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r < len) rank_slot[r] = new_of_old[rank_slot[r]];
}

// The list view's entry at `from` moves to `to` (a removal's hole).
__global__ void ivf_move_entry(uint32_t* __restrict__ list_slot, uint8_t* __restrict__ list_codes, int M,
                               uint32_t from, uint32_t to) {
  if (threadIdx.x == 0) list_slot[to] = list_slot[from];
  for (int j = threadIdx.x; j < M; j += blockDim.x) list_codes[(size_t)to * M + j] = list_codes[(size_t)from * M + j];
}

__global__ void ivf_gather_csr(const uint32_t* __restrict__ entry_slot, int n, const uint32_t* __restrict__ pos,
                               const uint8_t* __restrict__ codes, int M, uint32_t* __restrict__ list_slot,
                               uint8_t* __restrict__ list_codes) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t s = entry_slot[i], e = pos[i];
  list_slot[e] = s;
  for (int j = 0; j < M; ++j) list_codes[(size_t)e * M + j] = codes[(size_t)s * M + j];
}

// Entry order within each list of a 16-subspace index, chosen for the scan's
// table gathers. A scan wave reads one table entry per lane per subspace, lane
// l taking entry (list start + 64j + l). The LDS serves a ds_read_b32 one
// half-wave (32 lanes) at a time over 32 four-byte banks, and a half-wave
// takes as many passes as its most loaded bank holds distinct addresses
// (lanes on the same code share one broadcast). Every table starts on a bank
// boundary, so code c of any subspace falls in bank c mod 32.
//
// The entries of a list are dealt into 32-entry groups, aligned to the list
// start. Each place of a group takes, among the BO_WIN oldest entries not yet
// placed, the one that adds the least sum over subspaces of load^3, where
// load is the number of distinct codes the group already has on that entry's
// bank (a code already present adds nothing); ties go to the lowest window
// position, so the order is deterministic. On uniform random codes this
// lowers the mean passes per half-wave gather from ~3.1 to ~2.0.
//
// A wave orders one segment {first entry, entries} of at most BO_SEG entries
// (lists are cut at multiples of BO_SEG from their start, so the groups stay
// aligned), which keeps long lists from serialising the pass.
//
// Scan keys are (distance, id rank), so no result depends on this order.
constexpr int BO_PER_LANE = 2, BO_WIN = 64 * BO_PER_LANE;
constexpr uint32_t BO_SEG = 2048;
static_assert(BO_SEG % 32 == 0, "segments hold whole groups");

__device__ __forceinline__ uint32_t bo_byte(const uint4& w, int s) {
  const uint32_t v = s < 4 ? w.x : s < 8 ? w.y : s < 12 ? w.z : w.w;
  return (v >> (8 * (s & 3))) & 0xFFu;
}

__global__ __launch_bounds__(64) void ivf_bank_order(const uint2* __restrict__ segs,
                                                     const uint32_t* __restrict__ entry_in,
                                                     const uint8_t* __restrict__ codes,
                                                     uint32_t* __restrict__ entry_out) {
  // per (subspace, bank): distinct codes placed (bits 0-7) and which of the
  // bank's 8 codes are present (bit 8 + (c >> 5))
  __shared__ uint32_t st[16 * 32];
  const int lane = threadIdx.x;
  const uint32_t b = segs[blockIdx.x].x, n = segs[blockIdx.x].y;
  if (n <= 32) {  // one group: every order costs the same
    if ((uint32_t)lane < n) entry_out[b + lane] = entry_in[b + lane];
    return;
  }
  uint32_t slot[BO_PER_LANE];
  uint4 cw[BO_PER_LANE];
  bool ok[BO_PER_LANE];
#pragma unroll
  for (int j = 0; j < BO_PER_LANE; ++j) {
    const uint32_t i = (uint32_t)(j * 64 + lane);
    ok[j] = i < n;
    slot[j] = ok[j] ? entry_in[b + i] : 0u;
    cw[j] = ok[j] ? *reinterpret_cast<const uint4*>(codes + (size_t)slot[j] * 16) : make_uint4(0, 0, 0, 0);
  }
  uint32_t next = n < (uint32_t)BO_WIN ? n : (uint32_t)BO_WIN;
  for (uint32_t g0 = 0; g0 < n; g0 += 32) {
    for (int i = lane; i < 16 * 32; i += 64) st[i] = 0;
    __syncthreads();
    const uint32_t gs = n - g0 < 32 ? n - g0 : 32;
    for (uint32_t k = 0; k < gs; ++k) {
      uint32_t key = 0xFFFFFFFFu;
#pragma unroll
      for (int j = 0; j < BO_PER_LANE; ++j) {
        uint32_t cost = 0;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
          const uint32_t c = bo_byte(cw[j], s);
          const uint32_t w = st[s * 32 + (c & 31)];
          const uint32_t l = w & 0xFFu;
          cost += ((w >> (8 + (c >> 5))) & 1u) ? 0u : l * l * l;
        }
        // cost <= 16 * 32^3 < 2^20; position j*64 + lane < 2^7
        const uint32_t kj = (cost << 7) | (uint32_t)(j * 64 + lane);
        if (ok[j] && kj < key) key = kj;
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)key, off);
        key = o < key ? o : key;
      }
      const int pos = (int)(key & 127u), wl = pos & 63, wj = pos >> 6;
      const uint32_t mine = wj == 0 ? slot[0] : slot[1];
      const uint4 mc = wj == 0 ? cw[0] : cw[1];
      const uint32_t wslot = (uint32_t)__builtin_amdgcn_readlane((int)mine, wl);
      const uint4 wc = make_uint4((uint32_t)__builtin_amdgcn_readlane((int)mc.x, wl),
                                  (uint32_t)__builtin_amdgcn_readlane((int)mc.y, wl),
                                  (uint32_t)__builtin_amdgcn_readlane((int)mc.z, wl),
                                  (uint32_t)__builtin_amdgcn_readlane((int)mc.w, wl));
      if (lane == 0) entry_out[b + g0 + k] = wslot;
      __syncthreads();  // every lane has read st for this place
      if (lane < 16) {
        uint32_t c = 0;
#pragma unroll
        for (int s = 0; s < 16; ++s)
          if (lane == s) c = bo_byte(wc, s);
        const int i = lane * 32 + (int)(c & 31);
        const uint32_t bit = 1u << (8 + (c >> 5)), w = st[i];
        if (!(w & bit)) st[i] = (w + 1) | bit;
      }
      __syncthreads();
      if (lane == wl) {  // refill the winner's window place from the list
        const bool more = next < n;
        const uint32_t ns = more ? entry_in[b + next] : 0u;
        const uint4 nc = more ? *reinterpret_cast<const uint4*>(codes + (size_t)ns * 16) : make_uint4(0, 0, 0, 0);
        if (wj == 0) {
          slot[0] = ns;
          cw[0] = nc;
          ok[0] = more;
        } else {
          slot[1] = ns;
          cw[1] = nc;
          ok[1] = more;
        }
      }
      if (next < n) ++next;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
struct IvfPqIndex {
  uint32_t dim = 0, ld = 0;
  int metric = 0;
  pxg_ivfpq_config cfg{};
  PqLayout pq;

  // slot table (ivfpq.rs:452-479)
  std::vector<uint64_t> ids;
  std::vector<uint8_t> live;
  std::vector<uint32_t> list_of_h;
  std::unordered_map<uint64_t, uint32_t> by_id;
  SlotAllocator slots;
  bool vectors_kept = true;  // false once trained with retain_vectors = false

  // trained state
  bool trained = false;
  int produced = 0;
  pxg_training_report report{};
  bool has_report = false;

  size_t cap = 0;
  DevBuf<float> X;
  DevBuf<uint8_t> d_live;
  DevBuf<uint64_t> d_ids;
  DevBuf<uint8_t> codes;
  DevBuf<uint32_t> d_list_of;
  DevBuf<float> cents, books;
  DevBuf<float> cents_t;  // [dim][cst] transposed centroids for the coarse scan
  DevBuf<float> cent_norm;  // |c_l| (slightly rounded up), for the certified MFMA coarse stage
  int cst = 0;
  DevBuf<int> d_sub_off, d_book_off;
  RankTable ranks;  // id ranks of the live slots, current after every mutation
  // The scan view (ivfpq.rs:891-896): list l's entries, each a slot and its
  // M code bytes, at pool positions [lbeg[l], lend[l]) of a region of
  // lcap[l] positions. An insert appends to its list (a full region moves to
  // the pool's end with twice the room, O(|list|)); a removal moves the
  // list's last entry into its hole; so a mutation costs O(1) amortised, as
  // the reference's Vec pushes and retains do (ivfpq.rs:893-896, 1172). Scan
  // keys are (distance, id rank), so the order within a list changes no
  // result. A full rebuild (train, load, compact, or a pool half made of
  // regions left behind by moves) lays the lists out again with slack.
  DevBuf<uint32_t> list_beg, list_end, list_slot;
  DevBuf<uint8_t> list_codes;
  std::vector<uint32_t> list_len_h, lbeg_h, lend_h, lcap_h;
  std::vector<uint32_t> ent_slot_h;  // pool position -> slot
  std::vector<uint32_t> pos_h;       // slot -> pool position (NO_POS when not in the view)
  size_t pool_cap = 0, pool_used = 0, pool_abandoned = 0;
  uint64_t view_rebuilds = 0, view_moves = 0;  // full rebuilds; regions moved by appends
  static constexpr uint32_t NO_POS = 0xFFFFFFFFu;
  // the coarse quantizer as an exact flat index over the centroids (ids =
  // list numbers): MFMA candidates + exact unrolled rescoring give the
  // reference's (distance, list) order for the probe selection
  std::unique_ptr<FlatIndex> coarse;
  bool csr_dirty = true;
  std::mutex lazy_mu;

  mutable std::shared_mutex mu;
  CtxPool pool;
  hipStream_t stream = nullptr;

  ~IvfPqIndex() {
    if (stream) (void)hipStreamDestroy(stream);
  }

  size_t M() const { return (size_t)cfg.subspaces; }

  // Grow the device arrays to hold `need` slots, keeping the first `keep`
  // (the high-water mark before the current allocation, never above cap).
  void ensure_capacity(size_t need, size_t keep) {
    if (need <= cap) return;
    size_t nc = std::max<size_t>(need, std::max<size_t>(cap * 2, 1024));
    const size_t hw = std::min(keep, cap);
    if (vectors_kept) X.grow(nc * ld, hw * ld, stream);
    d_live.grow(nc, hw, stream);
    d_ids.grow(nc, hw, stream);
    codes.grow(nc * M(), hw * M(), stream);
    d_list_of.grow(nc, hw, stream);
    ranks.grow(nc, hw, stream);
    PXG_HIP(hipMemsetAsync(d_live.p + hw, 0, nc - hw, stream));
    PXG_HIP(hipStreamSynchronize(stream));
    cap = nc;
  }

  // room of a list region holding `len` entries: slack for appends, whole
  // 32-entry groups (the bank order's unit)
  static uint32_t region_for(uint64_t len) {
    const uint64_t c = len + std::max<uint64_t>(32, len / 16);
    return (uint32_t)((c + 31) & ~(uint64_t)31);
  }

  // The full rebuild of the scan view, on first use after train, load,
  // compact or too many abandoned regions.
  void refresh(hipStream_t s) {
    std::lock_guard<std::mutex> lk(lazy_mu);
    const size_t hw = slots.high_water();
    if (trained && csr_dirty) {
      std::vector<uint64_t> count(produced + 1, 0);
      for (size_t i = 0; i < hw; ++i)
        if (live[i] && list_of_h[i] != UNASSIGNED) count[list_of_h[i] + 1]++;
      for (int l = 0; l < produced; ++l) count[l + 1] += count[l];
      const uint64_t total = count[produced];
      std::vector<uint32_t> entry(std::max<uint64_t>(total, 1));
      std::vector<uint64_t> cur(count.begin(), count.end() - 1);
      for (size_t i = 0; i < hw; ++i)
        if (live[i] && list_of_h[i] != UNASSIGNED) entry[cur[list_of_h[i]]++] = (uint32_t)i;
      list_len_h.assign(produced, 0);
      lbeg_h.assign(produced, 0);
      lend_h.assign(produced, 0);
      lcap_h.assign(produced, 0);
      uint64_t at = 0;
      for (int l = 0; l < produced; ++l) {
        list_len_h[l] = (uint32_t)(count[l + 1] - count[l]);
        lcap_h[l] = region_for(list_len_h[l]);
        lbeg_h[l] = (uint32_t)at;
        lend_h[l] = (uint32_t)(at + list_len_h[l]);
        at += lcap_h[l];
      }
      pool_used = at;
      pool_cap = at + at / 8 + 1024;  // room for moved regions
      if (pool_cap >= NO_POS) capacity_error("ivf-pq list view", NO_POS, "capacity exceeded: the IVF-PQ list view holds fewer than 2^32 entries");
      pool_abandoned = 0;
      list_beg.reserve(std::max(produced, 1));
      list_end.reserve(std::max(produced, 1));
      list_slot.alloc(pool_cap);
      list_codes.alloc(pool_cap * M() + 16);
      PXG_HIP(hipMemcpyAsync(list_beg.p, lbeg_h.data(), produced * 4, hipMemcpyHostToDevice, s));
      PXG_HIP(hipMemcpyAsync(list_end.p, lend_h.data(), produced * 4, hipMemcpyHostToDevice, s));
      ent_slot_h.assign(pool_cap, NO_POS);
      pos_h.assign(std::max<size_t>(cap, hw), NO_POS);
      if (total) {
        DevBuf<uint32_t> d_entry(total), d_banked, d_pos(total);
        DevBuf<uint2> d_segs;
        std::vector<uint2> segs;  // read by an async copy: lives to the sync below
        PXG_HIP(hipMemcpyAsync(d_entry.p, entry.data(), total * 4, hipMemcpyHostToDevice, s));
        const uint32_t* order = d_entry.p;
        if (M() == 16) {  // the staged 16-subspace scan gathers by half-wave
          for (int l = 0; l < produced; ++l)
            for (uint32_t s0 = 0; s0 < list_len_h[l]; s0 += BO_SEG)
              segs.push_back(make_uint2((uint32_t)count[l] + s0, std::min(BO_SEG, list_len_h[l] - s0)));
          d_banked.reserve(total);
          d_segs.reserve(segs.size());
          PXG_HIP(hipMemcpyAsync(d_segs.p, segs.data(), segs.size() * sizeof(uint2), hipMemcpyHostToDevice, s));
          hipLaunchKernelGGL(ivf_bank_order, dim3((unsigned)segs.size()), dim3(64), 0, s, d_segs.p, d_entry.p,
                             codes.p, d_banked.p);
          PXG_HIP(hipGetLastError());
          order = d_banked.p;
          PXG_HIP(hipMemcpyAsync(entry.data(), d_banked.p, total * 4, hipMemcpyDeviceToHost, s));
        }
        // dense entry i of list l goes to position lbeg[l] + (i - count[l])
        std::vector<uint32_t> pos(total);
        for (int l = 0; l < produced; ++l)
          for (uint64_t i = count[l]; i < count[l + 1]; ++i) pos[i] = lbeg_h[l] + (uint32_t)(i - count[l]);
        PXG_HIP(hipMemcpyAsync(d_pos.p, pos.data(), total * 4, hipMemcpyHostToDevice, s));
        hipLaunchKernelGGL(ivf_gather_csr, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, order, (int)total,
                           (const uint32_t*)d_pos.p, codes.p, (int)M(), list_slot.p, list_codes.p);
        PXG_HIP(hipGetLastError());
        PXG_HIP(hipStreamSynchronize(s));  // entry holds the banked order now
        for (uint64_t i = 0; i < total; ++i) {
          ent_slot_h[pos[i]] = entry[i];
          pos_h[entry[i]] = pos[i];
        }
      }
      PXG_HIP(hipStreamSynchronize(s));
      csr_dirty = false;
      ++view_rebuilds;
    }
  }

  // Move list l's region to the pool's end with room for `room` entries; a
  // full pool doubles first (one copy of the used part, amortised over the
  // appends that filled it). False when the pool would pass 2^32 entries
  // (the caller lays the view out again instead).
  bool view_move(int l, uint64_t room) {
    const uint32_t nc = region_for(room);
    if (pool_used + nc > pool_cap) {
      const size_t grown = std::max<size_t>(2 * pool_cap, pool_used + nc);
      if (grown >= NO_POS) return false;
      list_slot.grow(grown, pool_used, stream);
      list_codes.grow(grown * M() + 16, pool_used * M(), stream);
      ent_slot_h.resize(grown, NO_POS);
      pool_cap = grown;
    }
    const uint32_t nb = (uint32_t)pool_used, len = lend_h[l] - lbeg_h[l];
    if (len) {
      PXG_HIP(hipMemcpyAsync(list_slot.p + nb, list_slot.p + lbeg_h[l], (size_t)len * 4, hipMemcpyDeviceToDevice,
                             stream));
      PXG_HIP(hipMemcpyAsync(list_codes.p + (size_t)nb * M(), list_codes.p + (size_t)lbeg_h[l] * M(),
                             (size_t)len * M(), hipMemcpyDeviceToDevice, stream));
    }
    for (uint32_t i = 0; i < len; ++i) {
      const uint32_t sl = ent_slot_h[lbeg_h[l] + i];
      ent_slot_h[nb + i] = sl;
      ent_slot_h[lbeg_h[l] + i] = NO_POS;
      pos_h[sl] = nb + i;
    }
    pool_abandoned += lcap_h[l];
    pool_used += nc;
    lbeg_h[l] = nb;
    lend_h[l] = nb + len;
    lcap_h[l] = nc;
    ++view_moves;
    return true;
  }

  // Append newly encoded slots (list_of_h and codes set) to their lists.
  void view_append(const std::vector<uint32_t>& sl) {
    if (!trained || csr_dirty || sl.empty()) return;
    if (pos_h.size() < cap) pos_h.resize(cap, NO_POS);
    // room first, so that no region moves after an entry was placed in it
    std::unordered_map<uint32_t, uint64_t> add;
    for (uint32_t s0 : sl) add[list_of_h[s0]]++;
    for (auto& kv : add) {
      const int l = (int)kv.first;
      const uint64_t need = (uint64_t)(lend_h[l] - lbeg_h[l]) + kv.second;
      if (need > lcap_h[l] && !view_move(l, std::max<uint64_t>(need, 2ull * lcap_h[l]))) {
        csr_dirty = true;  // the next search lays the lists out again
        return;
      }
    }
    std::vector<uint32_t> pos(sl.size());
    for (size_t i = 0; i < sl.size(); ++i) {
      const uint32_t l = list_of_h[sl[i]], p = lend_h[l]++;
      ++list_len_h[l];
      ent_slot_h[p] = sl[i];
      pos_h[sl[i]] = p;
      pos[i] = p;
    }
    DevBuf<uint32_t> d_sl(sl.size()), d_pos(sl.size());
    PXG_HIP(hipMemcpyAsync(d_sl.p, sl.data(), sl.size() * 4, hipMemcpyHostToDevice, stream));
    PXG_HIP(hipMemcpyAsync(d_pos.p, pos.data(), pos.size() * 4, hipMemcpyHostToDevice, stream));
    hipLaunchKernelGGL(ivf_gather_csr, dim3((unsigned)((sl.size() + 255) / 256)), dim3(256), 0, stream,
                       (const uint32_t*)d_sl.p, (int)sl.size(), (const uint32_t*)d_pos.p, codes.p, (int)M(),
                       list_slot.p, list_codes.p);
    PXG_HIP(hipGetLastError());
    PXG_HIP(hipMemcpyAsync(list_beg.p, lbeg_h.data(), produced * 4, hipMemcpyHostToDevice, stream));
    PXG_HIP(hipMemcpyAsync(list_end.p, lend_h.data(), produced * 4, hipMemcpyHostToDevice, stream));
    PXG_HIP(hipStreamSynchronize(stream));
    // regions left behind by moves: lay the view out again once they are half the pool
    if (pool_abandoned > pool_used / 2) csr_dirty = true;
  }

  // Drop slot s (in list l) from the view: the list's last entry fills its place.
  void view_remove(uint32_t s0, uint32_t l) {
    if (!trained || csr_dirty || l == UNASSIGNED || s0 >= pos_h.size() || pos_h[s0] == NO_POS) return;
    const uint32_t p = pos_h[s0], last = lend_h[l] - 1;
    if (p != last) {
      const uint32_t t = ent_slot_h[last];
      hipLaunchKernelGGL(ivf_move_entry, dim3(1), dim3(64), 0, stream, list_slot.p, list_codes.p, (int)M(), last, p);
      PXG_HIP(hipGetLastError());
      ent_slot_h[p] = t;
      pos_h[t] = p;
    }
    ent_slot_h[last] = NO_POS;
    pos_h[s0] = NO_POS;
    lend_h[l] = last;
    --list_len_h[l];
    PXG_HIP(hipMemcpyAsync(list_end.p + l, &lend_h[l], 4, hipMemcpyHostToDevice, stream));
  }

  void build_coarse() {
    coarse.reset(new FlatIndex());
    FlatIndex& c = *coarse;
    c.dim = dim;
    c.ld = ld;
    c.metric = PXG_EUCLIDEAN;
    PXG_HIP(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking));
    c.ensure_capacity((size_t)produced, 0);
    DevBuf<float> dense((size_t)produced * dim);
    PXG_HIP(hipMemcpy2DAsync(dense.p, dim * 4, cents.p, ld * 4, dim * 4, produced, hipMemcpyDeviceToDevice, stream));
    PXG_HIP(hipStreamSynchronize(stream));
    std::vector<uint64_t> lid(produced);
    for (int l = 0; l < produced; ++l) lid[l] = (uint64_t)l;
    c.insert_device(lid.data(), dense.p, (uint64_t)produced, nullptr);
    cst = (produced + 63) / 64 * 64;
    cent_norm.alloc(std::max(produced, 1));
    hipLaunchKernelGGL(ivf_cent_norms, dim3((unsigned)((produced + 255) / 256)), dim3(256), 0, stream, cents.p,
                       (int)ld, (int)dim, produced, cent_norm.p);
    cents_t.alloc((size_t)dim * cst);
    const size_t tot = (size_t)dim * cst;
    hipLaunchKernelGGL(ivf_transpose_cents, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, stream, cents.p,
                       (int)ld, (int)dim, produced, cst, cents_t.p);
    PXG_HIP(hipGetLastError());
    PXG_HIP(hipStreamSynchronize(stream));
  }

  void upload_books(const float* h_cents, int nprod, const float* h_books) {
    produced = nprod;
    cents.alloc((size_t)std::max(nprod, 1) * ld);
    PXG_HIP(hipMemsetAsync(cents.p, 0, (size_t)std::max(nprod, 1) * ld * 4, stream));
    PXG_HIP(hipMemcpy2DAsync(cents.p, ld * 4, h_cents, dim * 4, dim * 4, nprod, hipMemcpyHostToDevice, stream));
    books.alloc(pq.book_off[pq.M]);
    PXG_HIP(hipMemcpyAsync(books.p, h_books, pq.book_off[pq.M] * 4, hipMemcpyHostToDevice, stream));
    PXG_HIP(hipStreamSynchronize(stream));
    trained = true;
    csr_dirty = true;
    build_coarse();
  }

  // encode the given slots (vectors must be in X) on the device: nearest
  // coarse centroid with the unrolled kernel (ivfpq.rs:1231-1243), residual,
  // PQ code (product.rs:361-380)
  void encode_slots(const std::vector<uint32_t>& sl) {
    if (sl.empty()) return;
    DevBuf<uint32_t> d_sl(sl.size()), d_as(sl.size());
    PXG_HIP(hipMemcpyAsync(d_sl.p, sl.data(), sl.size() * 4, hipMemcpyHostToDevice, stream));
    nearest_device(X.p, (int)ld, d_sl.p, sl.size(), (int)dim, cents.p, (int)ld, produced, true, d_as.p, nullptr,
                   stream);
    pq_encode_device(X.p, (int)ld, d_sl.p, sl.size(), (int)dim, cents.p, (int)ld, d_as.p, books.p, pq, codes.p,
                     stream);
    std::vector<uint32_t> as(sl.size());
    PXG_HIP(hipMemcpyAsync(as.data(), d_as.p, as.size() * 4, hipMemcpyDeviceToHost, stream));
    PXG_HIP(hipStreamSynchronize(stream));
    for (size_t i = 0; i < sl.size(); ++i) list_of_h[sl[i]] = as[i];
    // device copy of the assignment, slot-indexed: only the encoded slots
    hipLaunchKernelGGL(ivf_scatter_u32, dim3((unsigned)((sl.size() + 255) / 256)), dim3(256), 0, stream, d_sl.p,
                       d_as.p, (int)sl.size(), d_list_of.p);
    PXG_HIP(hipGetLastError());
    PXG_HIP(hipStreamSynchronize(stream));
    view_append(sl);
  }

  // Encode n prepared rows staged compactly on the device (st[n][ld]) into
  // their slots: the same nearest-centroid and PQ arithmetic as encode_slots,
  // without a slot-indexed copy of the rows.
  void encode_staged(const float* st, const std::vector<uint32_t>& sl) {
    const size_t n = sl.size();
    if (n == 0) return;
    DevBuf<uint32_t> d_sl(n), d_as(n);
    DevBuf<uint8_t> tmp(n * M());
    PXG_HIP(hipMemcpyAsync(d_sl.p, sl.data(), n * 4, hipMemcpyHostToDevice, stream));
    if (n < 4096 && coarse) {
      // Few rows (inserts into a trained index): nearest_centroid
      // (ivfpq.rs:1231-1243, unrolled kernel, first minimum) as the exact
      // flat search of k = 1 over the centroids, whose (distance, list)
      // order gives the same list; it spreads the centroids over the GPU
      // instead of one thread per row scanning them all.
      const float* q = st;
      DevBuf<float> dense;
      if (ld != dim) {
        dense.alloc(n * dim);
        PXG_HIP(hipMemcpy2DAsync(dense.p, dim * 4, st, ld * 4, dim * 4, n, hipMemcpyDeviceToDevice, stream));
        q = dense.p;
      }
      DevBuf<uint64_t> cid(n);
      DevBuf<float> cd(n);
      DevBuf<uint32_t> cc(n);
      CtxLease cl(coarse->pool);
      CtxScratch csc(cl.c);
      uint64_t fb = 0;
      coarse->search_device(q, false, n, 1, nullptr, cid.p, cd.p, cc.p, csc, stream, &fb, 1);
      hipLaunchKernelGGL(ivf_probes_from_ids, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                         (const uint64_t*)cid.p, (int)n, (int*)d_as.p);
      PXG_HIP(hipGetLastError());
    } else {
      nearest_device(st, (int)ld, nullptr, n, (int)dim, cents.p, (int)ld, produced, true, d_as.p, nullptr, stream);
    }
    pq_encode_device(st, (int)ld, nullptr, n, (int)dim, cents.p, (int)ld, d_as.p, books.p, pq, tmp.p, stream);
    hipLaunchKernelGGL(ivf_scatter_codes, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, tmp.p, d_sl.p,
                       d_as.p, (int)n, (int)M(), codes.p, d_list_of.p);
    PXG_HIP(hipGetLastError());
    std::vector<uint32_t> as(n);
    PXG_HIP(hipMemcpyAsync(as.data(), d_as.p, n * 4, hipMemcpyDeviceToHost, stream));
    PXG_HIP(hipStreamSynchronize(stream));
    for (size_t i = 0; i < n; ++i) list_of_h[sl[i]] = as[i];
    view_append(sl);
  }

  // IvfPqIndex::train (ivfpq.rs:735-825)
  pxg_training_report train() {
    if (!vectors_kept && !by_id.empty())
      config_error("retain_vectors", 0, "training needs the full-precision vectors, which were dropped");
    std::vector<uint32_t> live_slots;
    for (size_t i = 0; i < slots.high_water(); ++i)
      if (live[i]) live_slots.push_back((uint32_t)i);
    if (live_slots.empty()) config_error("len", 0, "an empty index has nothing to fit centroids to");
    // deterministic stride sample (ivfpq.rs:758-768)
    const size_t L = live_slots.size();
    const size_t stride = std::max<size_t>((L + cfg.training_sample - 1) / cfg.training_sample, 1);
    std::vector<uint32_t> sample;
    for (size_t i = 0; i < L; i += stride) sample.push_back(live_slots[i]);
    const size_t ns = sample.size();
    DevBuf<uint32_t> d_sample(ns);
    PXG_HIP(hipMemcpyAsync(d_sample.p, sample.data(), ns * 4, hipMemcpyHostToDevice, stream));
    DevBuf<float> S(ns * dim);
    hipLaunchKernelGGL(ivf_gather_rows, dim3((unsigned)ns), dim3(256), 0, stream, X.p, (int)ld, d_sample.p, (int)ns,
                       (int)dim, S.p);
    PXG_HIP(hipGetLastError());
    // coarse quantizer: kmeans with ChaCha8Rng::seed_from_u64(seed) (ivfpq.rs:770-777)
    ChaCha8 rng(cfg.seed);
    DevBuf<float> coarse;
    KmeansOut kc = kmeans_device(S.p, ns, (int)dim, (int)dim, cfg.nlist, cfg.max_iterations, &rng, nullptr, coarse,
                                 nullptr, stream);
    // residuals of the sample against their nearest centroid (ivfpq.rs:787-792)
    DevBuf<uint32_t> as(ns);
    nearest_device(S.p, (int)dim, nullptr, ns, (int)dim, coarse.p, (int)dim, kc.k, true, as.p, nullptr, stream);
    DevBuf<float> R(ns * dim);
    hipLaunchKernelGGL(ivf_residuals, dim3((unsigned)ns), dim3(256), 0, stream, S.p, coarse.p, as.p, (int)dim, R.p);
    PXG_HIP(hipGetLastError());
    {
      // ProductQuantizer::train validates every residual (product.rs:221-223):
      // x - c can overflow even though x and c are finite
      DevBuf<unsigned long long> bad(1);
      PXG_HIP(hipMemsetAsync(bad.p, 0xFF, 8, stream));
      const size_t tot = ns * dim;
      hipLaunchKernelGGL(ivf_first_nonfinite, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, stream, R.p, ns,
                         (int)dim, bad.p);
      PXG_HIP(hipGetLastError());
      unsigned long long bv = 0;
      PXG_HIP(hipMemcpyAsync(&bv, bad.p, 8, hipMemcpyDeviceToHost, stream));
      PXG_HIP(hipStreamSynchronize(stream));
      if (bv != ~0ull) {
        const uint64_t row = bv >> 32, comp = (uint32_t)bv;
        float v = NAN;
        PXG_HIP(hipMemcpy(&v, R.p + row * dim + comp, 4, hipMemcpyDeviceToHost));
        raise(PXG_ERR_NON_FINITE,
              "vector component " + std::to_string(comp) + " is not finite (" + std::to_string(v) + ")", comp, row, v);
      }
    }
    // PQ with a fresh generator from the same seed (ivfpq.rs:794-801)
    DevBuf<float> B(pq.book_floats());
    double rin = 0.0;
    size_t rit = 0;
    pq_train_device(R.p, ns, (int)dim, (int)dim, pq, cfg.max_iterations, cfg.seed, B.p, &rin, &rit, stream);
    // install (padded centroid rows) and encode every live vector
    produced = (int)kc.k;
    cents.alloc((size_t)produced * ld);
    PXG_HIP(hipMemsetAsync(cents.p, 0, (size_t)produced * ld * 4, stream));
    PXG_HIP(hipMemcpy2DAsync(cents.p, ld * 4, coarse.p, dim * 4, dim * 4, produced, hipMemcpyDeviceToDevice, stream));
    books = std::move(B);
    PXG_HIP(hipStreamSynchronize(stream));
    trained = true;
    csr_dirty = true;  // new lists: the view is laid out again
    build_coarse();
    const double t_enc = std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
    encode_slots(live_slots);
    if (std::getenv("PXG_TRAIN_VERBOSE"))
      std::fprintf(stderr, "[pxg ivfpq] encode %zu vectors %.3fs\n", live_slots.size(),
                   std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count() - t_enc);
    if (!cfg.retain_vectors) {
      X.release();
      vectors_kept = false;
    }
    pxg_training_report rep{};
    rep.sampled = ns;
    rep.coarse_inertia = kc.inertia;
    rep.coarse_iterations = kc.iterations;
    rep.residual_inertia = rin;
    std::vector<uint64_t> cnt(produced, 0);
    for (uint32_t s : live_slots) cnt[list_of_h[s]]++;
    rep.populated_lists = (uint64_t)std::count_if(cnt.begin(), cnt.end(), [](uint64_t c) { return c > 0; });
    rep.largest_list = cnt.empty() ? 0 : *std::max_element(cnt.begin(), cnt.end());
    report = rep;
    has_report = true;
    return rep;
  }

  // Validate + prepare a batch into a device staging buffer [n][ld]:
  // from host vectors (space.rs:130-138 on the host) or device vectors
  // (the same arithmetic on the device). Nothing is mutated on failure.
  void stage_host(const float* vecs, uint64_t n, DevBuf<float>& st) {
    std::vector<float> prepared((size_t)n * ld, 0.0f);
    for (uint64_t i = 0; i < n; ++i) {
      long long bad = validate_prepare(metric, vecs + i * dim, dim, prepared.data() + i * ld);
      if (bad >= 0)
        raise(PXG_ERR_NON_FINITE,
              "vector component " + std::to_string(bad) + " is not finite (" + std::to_string(vecs[i * dim + bad]) + ")",
              (uint64_t)bad, i, vecs[i * dim + bad]);
    }
    st.alloc(n * ld);
    PXG_HIP(hipMemcpyAsync(st.p, prepared.data(), n * ld * 4, hipMemcpyHostToDevice, stream));
    PXG_HIP(hipStreamSynchronize(stream));
  }
  void stage_device(const float* d_vecs, uint64_t n, DevBuf<float>& st) {
    st.alloc(n * ld);
    DevBuf<float> b(n), nn(n);
    DevBuf<unsigned long long> bad(1);
    PXG_HIP(hipMemsetAsync(bad.p, 0xFF, 8, stream));
    hipLaunchKernelGGL(flat_prep_queries, dim3((unsigned)n), dim3(64), 0, stream, d_vecs, (int)dim, (int)ld, metric,
                       1, st.p, b.p, nn.p, bad.p);
    PXG_HIP(hipGetLastError());
    unsigned long long bv = 0;
    PXG_HIP(hipMemcpyAsync(&bv, bad.p, 8, hipMemcpyDeviceToHost, stream));
    PXG_HIP(hipStreamSynchronize(stream));
    if (bv != ~0ull) {
      const uint64_t row = bv >> 32, comp = (uint32_t)bv;
      raise(PXG_ERR_NON_FINITE,
            "vector component " + std::to_string(comp) + " is not finite (vector " + std::to_string(row) + ")", comp,
            row, NAN);
    }
  }

  // Insert prepared rows staged on the device (ivfpq.rs:1129-1158).
  void insert_rows(const uint64_t* in_ids, const DevBuf<float>& st, uint64_t n, uint32_t* out_slots) {
    {
      std::unordered_map<uint64_t, int> seen;
      for (uint64_t i = 0; i < n; ++i)
        if (by_id.count(in_ids[i]) || !seen.emplace(in_ids[i], 1).second)
          raise(PXG_ERR_DUPLICATE_ID, "duplicate vector id " + std::to_string(in_ids[i]), in_ids[i]);
    }
    std::vector<uint32_t> sl(n);
    const size_t old_hw = slots.high_water();
    for (uint64_t i = 0; i < n; ++i) sl[i] = slots.allocate();
    const size_t hw = slots.high_water();
    ensure_capacity(hw, old_hw);
    if (ids.size() < hw) {
      ids.resize(hw, 0);
      live.resize(hw, 0);
      list_of_h.resize(hw, UNASSIGNED);
    }
    // vectors go to X when kept; an index that drops them encodes from the
    // staged rows and keeps only the codes (ivfpq.rs:1134-1141)
    DevBuf<uint32_t> st_sl(n);
    DevBuf<uint64_t> st_ids(n);
    PXG_HIP(hipMemcpyAsync(st_sl.p, sl.data(), n * 4, hipMemcpyHostToDevice, stream));
    PXG_HIP(hipMemcpyAsync(st_ids.p, in_ids, n * 8, hipMemcpyHostToDevice, stream));
    hipLaunchKernelGGL(flat_scatter_rows, dim3((unsigned)n), dim3(256), 0, stream, st.p, st_sl.p, (const float*)nullptr,
                       st_ids.p, (int)n, (int)ld, vectors_kept ? X.p : (float*)nullptr, (float*)nullptr, d_live.p,
                       d_ids.p);
    PXG_HIP(hipGetLastError());
    PXG_HIP(hipStreamSynchronize(stream));
    for (uint64_t i = 0; i < n; ++i) {
      ids[sl[i]] = in_ids[i];
      live[sl[i]] = 1;
      list_of_h[sl[i]] = UNASSIGNED;
      by_id[in_ids[i]] = sl[i];
      if (out_slots) out_slots[i] = sl[i];
    }
    ranks.insert(in_ids, sl.data(), n, d_ids.p, stream);
    if (trained) encode_staged(st.p, sl);
  }

  // IvfPqIndex::compact (ivfpq.rs:907-975): drop the free slots, renumber
  // the live ones in slot order, shrink every array. Codebooks, centroids,
  // codes and ids are unchanged, so searches return the same results.
  uint64_t compact() {
    const size_t hw = slots.high_water();
    const uint64_t reclaimed = hw - by_id.size();
    if (reclaimed == 0) return 0;
    std::vector<uint32_t> keep, new_of_old(std::max<size_t>(hw, 1), UINT32_MAX);
    keep.reserve(by_id.size());
    for (size_t i = 0; i < hw; ++i)
      if (live[i]) {
        new_of_old[i] = (uint32_t)keep.size();
        keep.push_back((uint32_t)i);
      }
    const size_t n = keep.size();
    const size_t nc = std::max<size_t>(n, 1024);
    DevBuf<float> X1;
    if (vectors_kept) X1.alloc(nc * ld);
    DevBuf<uint8_t> c1(nc * M()), live1(nc);
    DevBuf<uint32_t> l1(nc), r1(nc), d_keep(std::max<size_t>(n, 1)), d_map(std::max<size_t>(hw, 1));
    DevBuf<uint64_t> i1(nc);
    PXG_HIP(hipMemsetAsync(live1.p, 0, nc, stream));
    if (n) {
      PXG_HIP(hipMemcpyAsync(d_keep.p, keep.data(), n * 4, hipMemcpyHostToDevice, stream));
      hipLaunchKernelGGL(ivf_compact_rows, dim3((unsigned)n), dim3(128), 0, stream, d_keep.p, (int)n, (int)ld,
                         (int)M(), vectors_kept ? X.p : (const float*)nullptr, X1.p, codes.p, c1.p, d_list_of.p, l1.p,
                         d_ids.p, i1.p, ranks.rank.p, r1.p, live1.p);
      PXG_HIP(hipMemcpyAsync(d_map.p, new_of_old.data(), hw * 4, hipMemcpyHostToDevice, stream));
      hipLaunchKernelGGL(ivf_remap_slots, dim3((ranks.len + 255) / 256), dim3(256), 0, stream, ranks.rank_slot.p,
                         ranks.len, d_map.p);
      PXG_HIP(hipGetLastError());
    }
    PXG_HIP(hipStreamSynchronize(stream));
    if (vectors_kept) std::swap(X, X1);
    std::swap(codes, c1);
    std::swap(d_live, live1);
    std::swap(d_list_of, l1);
    std::swap(d_ids, i1);
    std::swap(ranks.rank, r1);
    cap = nc;
    std::vector<uint64_t> ids1(n);
    std::vector<uint8_t> live_h(n, 1);
    std::vector<uint32_t> lo1(n);
    by_id.clear();
    for (size_t i = 0; i < n; ++i) {
      ids1[i] = ids[keep[i]];
      lo1[i] = list_of_h[keep[i]];
      by_id[ids1[i]] = (uint32_t)i;
    }
    ids.swap(ids1);
    live.swap(live_h);
    list_of_h.swap(lo1);
    slots.clear();
    for (size_t i = 0; i < n; ++i) slots.allocate();
    csr_dirty = true;
    return reclaimed;
  }

  void remove(uint64_t id) {
    auto it = by_id.find(id);
    if (it == by_id.end()) raise(PXG_ERR_UNKNOWN_ID, "unknown vector id " + std::to_string(id), id);
    const uint32_t s = it->second;
    by_id.erase(it);
    live[s] = 0;
    view_remove(s, list_of_h[s]);
    list_of_h[s] = UNASSIGNED;
    slots.release(s);
    const uint32_t un = UNASSIGNED;
    PXG_HIP(hipMemsetAsync(d_live.p + s, 0, 1, stream));
    PXG_HIP(hipMemcpyAsync(d_list_of.p + s, &un, 4, hipMemcpyHostToDevice, stream));
    ranks.remove(s, stream);
    PXG_HIP(hipStreamSynchronize(stream));
  }

  // The wide search of a trained index over the probes already chosen: all
  // entries of the probed lists keyed, each query's segment sorted, the
  // shortlist optionally reranked and sorted again, the first kq emitted.
  // Returns the number of entries scanned.
  uint64_t search_wide_trained(const float* Qp, uint64_t nq, const int* probes, int np, uint64_t kq,
                               uint64_t shortlist, bool rerank, const uint8_t* d_accept, uint64_t* d_oid, float* d_od,
                               uint32_t* d_oc, Scratch& sc, hipStream_t s, size_t ldo) {
    std::vector<int> hp((size_t)nq * np);
    PXG_HIP(hipMemcpyAsync(hp.data(), probes, hp.size() * 4, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    std::vector<uint64_t> tot(nq, 0);
    uint64_t scanned = 0;
    for (uint64_t q = 0; q < nq; ++q) {
      for (int p = 0; p < np; ++p) tot[q] += list_len_h[hp[q * np + p]];
      scanned += tot[q];
    }
    // query groups: keys + sorted keys within 1 GiB, tables within 512 MiB,
    // sizes within 32 bits (a single query is always taken)
    const size_t table_bytes = (size_t)np * M() * 256 * 4;
    const uint64_t key_cap = std::min<uint64_t>((1ull << 30) / 16, (1ull << 32) - 1);
    const uint64_t qmax = std::max<uint64_t>(1, (512ull << 20) / table_bytes);
    std::vector<std::pair<uint64_t, uint64_t>> groups;  // [q0, q1)
    for (uint64_t q0 = 0; q0 < nq;) {
      uint64_t q1 = q0, keys = 0;
      while (q1 < nq && q1 - q0 < qmax && (q1 == q0 || keys + tot[q1] <= key_cap)) keys += tot[q1++];
      if (keys >= (1ull << 32)) config_error("nprobe", (uint64_t)np, "a query's probed lists hold 2^32 entries or more");
      groups.emplace_back(q0, q1);
      q0 = q1;
    }
    uint64_t max_keys = 0, max_q = 0;
    for (auto& g : groups) {
      uint64_t kk = 0;
      for (uint64_t q = g.first; q < g.second; ++q) kk += tot[q];
      max_keys = std::max(max_keys, kk);
      max_q = std::max(max_q, g.second - g.first);
    }
    const size_t nk = std::max<uint64_t>(max_keys, 1);
    uint64_t* keys = (uint64_t*)sc.get(30, nk * 8);
    uint64_t* sorted = (uint64_t*)sc.get(31, nk * 8);
    uint32_t* d_be = (uint32_t*)sc.get(32, (3 * max_q + max_q * np) * 4);  // begins, ends, ends2, pofs
    float* tables = (float*)sc.get(33, max_q * table_bytes);
    float* omq = (float*)sc.get(34, max_q * np * 4);
    const size_t temp_bytes = wide_sort_temp_bytes((uint32_t)nk, (uint32_t)max_q);
    void* temp = sc.get(35, std::max<size_t>(temp_bytes, 1));
    std::vector<uint32_t> hb(3 * max_q + max_q * np);
    for (auto& g : groups) {
      const int gn = (int)(g.second - g.first);
      uint32_t* begins = hb.data();
      uint32_t* ends = begins + max_q;
      uint32_t* pofs = ends + 2 * max_q;
      uint32_t at = 0;
      for (int i = 0; i < gn; ++i) {
        const uint64_t q = g.first + i;
        begins[i] = at;
        for (int p = 0; p < np; ++p) {
          pofs[i * np + p] = at;
          at += list_len_h[hp[q * np + p]];
        }
        ends[i] = at;
      }
      PXG_HIP(hipMemcpyAsync(d_be, hb.data(), hb.size() * 4, hipMemcpyHostToDevice, s));
      const uint32_t* dbeg = d_be;
      const uint32_t* dend = d_be + max_q;
      uint32_t* dend2 = d_be + 2 * max_q;
      const uint32_t* dpofs = d_be + 3 * max_q;
      const int items = gn * np;
      hipLaunchKernelGGL(ivf_wide_tables, dim3((unsigned)items), dim3(256), 0, s, Qp, (int)ld, (int)dim, (int)M(),
                         metric, probes, np, (int)g.first, cents.p, books.p, d_sub_off.p, d_book_off.p, tables, omq);
      hipLaunchKernelGGL(ivf_wide_keys, dim3((unsigned)items), dim3(256), 0, s, probes, np, (int)g.first, (int)M(),
                         metric, tables, omq, list_beg.p, list_end.p, list_slot.p, list_codes.p, ranks.rank_slot.p, ranks.rank.p, d_accept,
                         dpofs, keys);
      PXG_HIP(hipGetLastError());
      wide_sort(temp, temp_bytes, keys, sorted, at, (uint32_t)gn, dbeg, dend, s);
      const uint32_t* emit_end = dend;
      if (rerank) {
        const uint64_t t = shortlist;
        hipLaunchKernelGGL(ivf_wide_rerank, dim3((unsigned)((t + 31) / 32), (unsigned)gn), dim3(256), 0, s, sorted,
                           dbeg, dend, t, (int)g.first, Qp, (int)ld, (int)dim, metric, X.p, ranks.rank_slot.p, keys);
        hipLaunchKernelGGL(wide_truncate, dim3((unsigned)((gn + 255) / 256)), dim3(256), 0, s, dbeg, dend, gn, t,
                           dend2);
        PXG_HIP(hipGetLastError());
        wide_sort(temp, temp_bytes, keys, sorted, at, (uint32_t)gn, dbeg, dend2, s);
        emit_end = dend2;
      } else if (shortlist < kq) {
        internal_error("IvfPqIndex::search_wide_trained", "shortlist below k");
      }
      hipLaunchKernelGGL(wide_emit, dim3((unsigned)((kq + 255) / 256), (unsigned)gn), dim3(256), 0, s, sorted, dbeg,
                         emit_end, (int)g.first, kq, ranks.rank_slot.p, d_ids.p, d_oid, d_od, d_oc, ldo);
      PXG_HIP(hipGetLastError());
      PXG_HIP(hipStreamSynchronize(s));  // the host offsets are rewritten for the next group
    }
    return scanned;
  }

  void search_device(const float* d_raw, bool do_prepare, uint64_t nq, uint64_t k, uint64_t nprobe_in,
                     const uint8_t* d_accept, uint64_t* d_oid, float* d_od, uint32_t* d_oc, Scratch& sc,
                     hipStream_t s, size_t ldo) {
    check_k(k);
    if (nq == 0) return;
    // at most the live count per query (the probed lists hold no more)
    const uint64_t kq = std::min<uint64_t>(k, by_id.size());
    refresh(s);
    Timer tm(s);
    tm.on = tm.on && sc.timing();
    tm.mark(0);
    float* Qp = (float*)sc.get(1, nq * ld * 4);
    float* qb = (float*)sc.get(2, nq * 4);
    float* qn = (float*)sc.get(3, nq * 4);
    // flag word, flag count, then the IVF_SCAN_SLOTS scanned-entry counters
    static_assert(2 + IVF_SCAN_SLOTS <= TAIL_WORDS, "one readback holds the flags and the counters");
    unsigned long long* bad = (unsigned long long*)sc.get(4, 8 * (2 + IVF_SCAN_SLOTS));
    int* flag_count = (int*)(bad + 1);
    unsigned long long* scanned_dev = nullptr;
    uint64_t scanned_host = 0;
    // the flags, and the scanned-entry counters after them (used by the
    // trained path's scan)
    hipLaunchKernelGGL(init_search_flags_zero, dim3(1), dim3(64), 0, s, bad, flag_count,
                       (unsigned long long*)(flag_count + 2), IVF_SCAN_SLOTS);
    hipLaunchKernelGGL(flat_prep_queries, dim3((unsigned)nq), dim3(64), 0, s, d_raw, (int)dim, (int)ld, metric,
                       do_prepare ? 1 : 0, Qp, qb, qn, bad);
    PXG_HIP(hipGetLastError());
    const size_t N = slots.high_water();
    if (kq == 0) {
      hipLaunchKernelGGL(fill_u32, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, d_oc, (size_t)nq, 0u);
      PXG_HIP(hipGetLastError());
    } else if (!trained && kq > EXACT_MERGE_MAXK) {
      exact_wide_search(Qp, (int)ld, (int)dim, metric, nq, kq, X.p, N, d_live.p, d_accept, ranks.rank.p,
                        ranks.rank_slot.p, d_ids.p, d_oid, d_od, d_oc, ldo, sc, s);
    } else if (!trained) {
      // untrained: exact exhaustive scan (ivfpq.rs:1008-1012, 1113-1125)
      int* qlist = (int*)sc.get(5, nq * 4);
      hipLaunchKernelGGL(iota_kernel, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, qlist, (int)nq,
                         flag_count);
      const int QG = exact_query_group((size_t)nq, dim, N);
      const int CH = exact_chunk_rows(((size_t)nq + QG - 1) / QG, N);
      const int nchunks = (int)((N + CH - 1) / CH);
      const int kk = (int)std::min<uint64_t>(kq, (uint64_t)CH);
      uint64_t* ecand = (uint64_t*)sc.get(7, (size_t)nq * nchunks * kk * 8);
      tm.mark(1);
#define PXG_EXACT_SCAN(CHV, QGV)                                                                                  \
  hipLaunchKernelGGL((flat_exact_candidates<CHV, QGV>),                                                           \
                     dim3((std::min<int>(((int)nq + QGV - 1) / QGV * nchunks, 4096) + 7) / 8 * 8), dim3(256), 0, s, \
                     qlist, flag_count, nchunks, Qp, (int)ld, (int)dim, metric, X.p, (int)N, d_live.p, d_accept,  \
                     ranks.rank.p, (int)kq, ecand)
#define PXG_EXACT_MERGE(CHV)                                                                                      \
  hipLaunchKernelGGL(flat_merge_exact<CHV>, dim3((unsigned)nq), dim3(256), 0, s, qlist, flag_count, ecand, nchunks, \
                     (int)kq, ranks.rank_slot.p, d_ids.p, d_oid, d_od, d_oc, (uint64_t*)nullptr, ldo)
      if (CH == 256) {
        if (QG == 4) PXG_EXACT_SCAN(256, 4); else PXG_EXACT_SCAN(256, 1);
      } else {
        if (QG == 4) PXG_EXACT_SCAN(EXACT_CH, 4); else PXG_EXACT_SCAN(EXACT_CH, 1);
      }
      PXG_HIP(hipGetLastError());
      tm.mark(2);
      if (CH == 256) PXG_EXACT_MERGE(256); else PXG_EXACT_MERGE(EXACT_CH);
#undef PXG_EXACT_SCAN
#undef PXG_EXACT_MERGE
      PXG_HIP(hipGetLastError());
    } else {
      const int np = (int)std::min<uint64_t>(std::max<uint64_t>(nprobe_in, 1), (uint64_t)std::max(produced, 1));
      const bool rerank = cfg.rerank > 0 && vectors_kept;
      // TopK(max(rerank, k)) of the ADC scores (ivfpq.rs:1060-1064), never
      // more than the live count
      const uint64_t shortlist =
          std::min<uint64_t>(cfg.rerank > 0 ? std::max<uint64_t>(cfg.rerank, kq) : kq, by_id.size());
      // beyond the block selections, or tables beyond the LDS: sorted segments
      const bool wide = shortlist > IVF_MAX_SHORT || M() > IVF_MAX_M;
      const int kk = (int)std::min<uint64_t>(shortlist, IVF_MAX_SHORT);
      uint64_t* ck = (uint64_t*)sc.get(8, (size_t)nq * produced * 8);
      int* probes = (int*)sc.get(9, (size_t)nq * np * 4);
      tm.mark(0);
      scanned_dev = (unsigned long long*)(flag_count + 2);  // cleared by init_search_flags_zero
      const bool fused_count = np <= 64 && dim <= 2048;
      // entries per query (written by the fused pick), for the longest-first order
      uint32_t* qwork = fused_count && nq <= (uint64_t)LPT_MAXQ ? (uint32_t*)sc.get(16, nq * 4) : nullptr;
      // matrix-core distances with exact rescoring near the cut, for widths
      // where the GEMM outweighs the rescoring
      const bool coarse_mfma = fused_count && dim >= 32 && ld % 8 == 0 && np <= produced;
      if (coarse_mfma) {
        float* A = (float*)sc.get(13, (size_t)nq * cst * 4);
        const dim3 gd((unsigned)((nq + 63) / 64), (unsigned)((produced + 63) / 64));
        hipLaunchKernelGGL(ivf_coarse_mfma, gd, dim3(256), 0, s, Qp, (int)ld, (int)nq, qn, cents.p, produced,
                           cent_norm.p, cst, A);
        hipLaunchKernelGGL(ivf_coarse_pick_approx, dim3((unsigned)nq), dim3(256), 0, s, (const float*)A, cst,
                           produced, np, Qp, (int)ld, (int)dim, qn, cents.p, cent_norm.p, probes, list_beg.p,
                           list_end.p, scanned_dev, qwork);
      } else if (fused_count) {
        uint64_t* keys = (uint64_t*)sc.get(13, (size_t)nq * cst * 8);
        const dim3 gd((unsigned)((nq + IVF_CQ - 1) / IVF_CQ), (unsigned)((produced + IVF_CW * 64 - 1) / (IVF_CW * 64)));
        hipLaunchKernelGGL(ivf_coarse_dist, gd, dim3(IVF_CW * 64), (size_t)dim * IVF_CQ * 4, s, Qp, (int)ld, (int)dim,
                           (int)nq, cents_t.p, cst, produced, keys);
        hipLaunchKernelGGL(ivf_coarse_pick, dim3((unsigned)nq), dim3(256), 0, s, (const uint64_t*)keys, cst, produced,
                           np, probes, list_beg.p, list_end.p, scanned_dev, qwork);
      } else if (np <= 1024 && coarse) {
        // exact top-nprobe by (squared_l2, list) through the flat pipeline
        const float* Qd = Qp;
        if (ld != dim) {
          float* dq = (float*)sc.get(11, nq * dim * 4);
          PXG_HIP(hipMemcpy2DAsync(dq, dim * 4, Qp, ld * 4, dim * 4, nq, hipMemcpyDeviceToDevice, s));
          Qd = dq;
        }
        uint64_t* cid = (uint64_t*)sc.get(12, nq * np * 8);
        float* cdist = (float*)sc.get(13, nq * np * 4);
        uint32_t* ccnt = (uint32_t*)sc.get(14, nq * 4);
        CtxLease cl(coarse->pool);
        uint64_t fb = 0;
        CtxScratch csc(cl.c);
        coarse->search_device(Qd, false, nq, (uint64_t)np, nullptr, cid, cdist, ccnt, csc, s, &fb, (size_t)np);
        hipLaunchKernelGGL(ivf_probes_from_ids, dim3((unsigned)((nq * np + 255) / 256)), dim3(256), 0, s, cid,
                           (int)(nq * np), probes);
      } else {
        hipLaunchKernelGGL(ivf_coarse_keys, dim3((unsigned)nq), dim3(256), 0, s, Qp, (int)ld, (int)dim, cents.p,
                           produced, ck);
        hipLaunchKernelGGL(ivf_coarse_select, dim3((unsigned)nq), dim3(256), 0, s, ck, produced, np, probes);
      }
      PXG_HIP(hipGetLastError());
      if (!fused_count)
        hipLaunchKernelGGL(ivf_count_scanned, dim3((unsigned)((nq * np + 255) / 256)), dim3(256), 0, s, probes,
                           (int)(nq * np), list_beg.p, list_end.p, scanned_dev);
      const int W = (int)(dim / M());
      // the register-codebook scans keep two distance tables in LDS (one for
      // cosine): an L2 index with 128 subspaces takes the general scan
      // (the 16-subspace scan keeps shortlists up to 128 per wave, the
      // other register-codebook scan up to 64)
      const bool reg_shape = !wide && dim <= 128 && dim % M() == 0 &&
                             (W == 1 || W == 2 || W == 4 || W == 8 || W == 16 || W == 32) &&
                             (metric == PXG_COSINE || M() <= 64);
      const bool staged16 = reg_shape && M() == 16 && kk <= 128;
      const bool reg_path = reg_shape && (kk <= 64 || staged16);
      if (reg_path) {
        const size_t lds = (size_t)(metric == PXG_COSINE ? 1 : 2) * M() * 256 * 4;
        // probes per workgroup: up to IVF_PGMAX, fewer when that would leave
        // the GPU with under ~2 workgroups per CU
        int pg = IVF_PGMAX;
        while (pg > 1 && (int64_t)nq * ((np + pg - 1) / pg) < 512) pg >>= 1;
        const int groups = (np + pg - 1) / pg;
        uint64_t* cand = (uint64_t*)sc.get(10, (size_t)nq * groups * IVF_SW * kk * 8);
        const int grid = (int)(nq * groups);
        // queries longest first (two or more rounds of workgroups)
        int* qorder = nullptr;
        if (qwork && grid > 512) {
          qorder = (int*)sc.get(15, nq * 4);
          hipLaunchKernelGGL(ivf_lpt_order, dim3(1), dim3(1024), 0, s, (const uint32_t*)qwork, (int)nq, qorder);
          PXG_HIP(hipGetLastError());
        }
        tm.mark(1);
        // one group per query, no rerank and a shortlist within one key per
        // lane: the scan writes the results
        const bool fused = groups == 1 && !rerank && kk <= 64;
#define PXG_SCANR(WW, MET)                                                                                          \
  hipLaunchKernelGGL((ivf_scan_reg<WW, MET>), dim3(grid), dim3(IVF_SW * 64), lds, s, Qp, (int)ld, (int)dim,        \
                     (int)M(), probes, np, pg, groups, cents.p, books.p, list_beg.p, list_end.p, list_slot.p, list_codes.p,      \
                     ranks.rank_slot.p, ranks.rank.p, d_accept, kk, cand, (int)ldo, d_ids.p, fused ? d_oid : nullptr, d_od, d_oc, \
                     (const int*)qorder)
#define PXG_SCANR_W(MET)                  \
  switch (W) {                            \
    case 1: PXG_SCANR(1, MET); break;     \
    case 2: PXG_SCANR(2, MET); break;     \
    case 4: PXG_SCANR(4, MET); break;     \
    case 8: PXG_SCANR(8, MET); break;     \
    case 16: PXG_SCANR(16, MET); break;   \
    default: PXG_SCANR(32, MET); break;   \
  }
#define PXG_SCAN16(WW, MET)                                                                                         \
  hipLaunchKernelGGL((ivf_scan16<WW, MET>), dim3(grid), dim3(IVF_SW * 64), 0, s, Qp, (int)ld, probes, np, pg, groups, \
                     cents.p, books.p, list_beg.p, list_end.p, list_slot.p, list_codes.p, ranks.rank_slot.p, ranks.rank.p, d_accept, kk, cand,     \
                     (int)ldo, d_ids.p, fused ? d_oid : nullptr, d_od, d_oc, (const int*)qorder)
#define PXG_SCAN16_W(MET)                 \
  switch (W) {                            \
    case 1: PXG_SCAN16(1, MET); break;    \
    case 2: PXG_SCAN16(2, MET); break;    \
    case 4: PXG_SCAN16(4, MET); break;    \
    default: PXG_SCAN16(8, MET); break;   \
  }
        if (staged16) {
          if (metric == PXG_COSINE) {
            PXG_SCAN16_W(1)
          } else {
            PXG_SCAN16_W(0)
          }
        } else if (metric == PXG_COSINE) {
          PXG_SCANR_W(1)
        } else {
          PXG_SCANR_W(0)
        }
#undef PXG_SCAN16_W
#undef PXG_SCAN16
#undef PXG_SCANR_W
#undef PXG_SCANR
        PXG_HIP(hipGetLastError());
        tm.mark(2);
        if (!fused) {
          hipLaunchKernelGGL(ivf_merge, dim3((unsigned)nq), dim3(256), 0, s, cand, groups * IVF_SW * kk, kk, (int)ldo,
                             rerank ? 1 : 0, Qp, (int)ld, (int)dim, metric, X.p, ranks.rank_slot.p, d_ids.p, d_oid, d_od,
                             d_oc);
          PXG_HIP(hipGetLastError());
        }
      } else if (wide) {
        tm.mark(1);
        scanned_host = search_wide_trained(Qp, nq, probes, np, kq, shortlist, rerank, d_accept, d_oid, d_od, d_oc, sc,
                                           s, ldo);
        scanned_dev = nullptr;
      } else {
      const size_t lds = (size_t)M() * 256 * 4;
      uint64_t* cand = (uint64_t*)sc.get(10, (size_t)nq * np * 4 * kk * 8);
      const int grid = (int)(nq * np);
      tm.mark(1);
#define PXG_SCAN(CAPW, MET)                                                                                       \
  hipLaunchKernelGGL((ivf_scan<CAPW, MET>), dim3(grid), dim3(256), lds, s, Qp, (int)ld, (int)dim, (int)M(), probes, \
                     np, cents.p, books.p, d_sub_off.p, d_book_off.p, list_beg.p, list_end.p, list_slot.p, list_codes.p,       \
                     ranks.rank_slot.p, ranks.rank.p, d_accept, kk, cand)
      if (kk <= 192) {
        if (metric == PXG_COSINE) PXG_SCAN(256, 1); else PXG_SCAN(256, 0);
      } else if (kk <= 448) {
        if (metric == PXG_COSINE) PXG_SCAN(512, 1); else PXG_SCAN(512, 0);
      } else {
        if (metric == PXG_COSINE) PXG_SCAN(1024, 1); else PXG_SCAN(1024, 0);
      }
#undef PXG_SCAN
      PXG_HIP(hipGetLastError());
      tm.mark(2);
      hipLaunchKernelGGL(ivf_merge, dim3((unsigned)nq), dim3(256), 0, s, cand, np * 4 * kk, kk, (int)ldo,
                         rerank ? 1 : 0, Qp, (int)ld, (int)dim, metric, X.p, ranks.rank_slot.p, d_ids.p, d_oid, d_od,
                         d_oc);
      PXG_HIP(hipGetLastError());
      }
    }
    // one copy brings back the validation flag (word 0) and the scanned-entry
    // counters (words 2 ..) of the same scratch block
    unsigned long long* tail = sc.host_words();
    tail[0] = 0;
    PXG_HIP(hipMemcpyAsync(tail, bad, scanned_dev ? 8 * (2 + IVF_SCAN_SLOTS) : 8, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    tm.finish();
    uint64_t scanned = scanned_host;
    if (scanned_dev) {
      scanned = 0;
      for (int i = 0; i < IVF_SCAN_SLOTS; ++i) scanned += tail[2 + i];
    }
    const unsigned long long badv = tail[0];
    g_last_scanned = scanned;
    if (badv != ~0ull) {
      const uint32_t qi = (uint32_t)(badv >> 32), comp = (uint32_t)badv;
      raise(PXG_ERR_NON_FINITE,
            "vector component " + std::to_string(comp) + " is not finite (query " + std::to_string(qi) + ")", comp,
            qi, NAN);
    }
  }
};

// IvfPqConfig::validate (ivfpq.rs:259-304)
void validate_config(const pxg_ivfpq_config& c, uint32_t dim) {
  if (c.nlist == 0) config_error("nlist", c.nlist, "must be at least 1");
  if (c.subspaces == 0 || c.subspaces > dim) config_error("subspaces", c.subspaces, "must be between 1 and the space dimension");
  if (c.nprobe == 0 || c.nprobe > c.nlist) config_error("nprobe", c.nprobe, "must be between 1 and nlist");
  if (c.max_iterations == 0) config_error("max_iterations", c.max_iterations, "must be at least 1");
  if (c.training_sample == 0) config_error("training_sample", c.training_sample, "must be at least 1");
  if (c.rerank > 0 && !c.retain_vectors)
    config_error("rerank", c.rerank, "requires retain_vectors, because reranking is against the exact vectors");
}

}  // namespace pxg

using pxg::IvfPqIndex;

struct pxg_ivfpq {
  IvfPqIndex impl;
};

extern "C" {

int pxg_ivfpq_config_default(uint64_t nlist, uint64_t subspaces, pxg_ivfpq_config* out) {
  return pxg::guard([&] {
    // IvfPqConfig::new (ivfpq.rs:124-150)
    out->nlist = nlist;
    out->subspaces = subspaces;
    out->nprobe = std::max<uint64_t>(nlist / 16, 1);
    out->rerank = 0;
    out->seed = 0x1FF9C0D;
    out->max_iterations = 25;
    out->training_sample = 100000;
    out->train_threshold = nlist > UINT64_MAX / 100 ? UINT64_MAX : nlist * 100;
    out->retain_vectors = 1;
  });
}

int pxg_ivfpq_create(uint32_t dim, int metric, const pxg_ivfpq_config* cfg, pxg_ivfpq** out) {
  return pxg::guard([&] {
    if (dim < 1) pxg::config_error("dim", dim, "must be at least 1; a 0-dimensional space makes all distances equal");
    if (dim > (1u << 20)) pxg::config_error("dim", dim, "exceeds the 1048576 dimension ceiling");
    if (metric != PXG_EUCLIDEAN && metric != PXG_COSINE)
      pxg::config_error("metric", (uint64_t)metric, "IVF-PQ supports euclidean and cosine only; see the module docs");
    pxg::validate_config(*cfg, dim);
    auto* h = new pxg_ivfpq();
    IvfPqIndex& f = h->impl;
    f.dim = dim;
    f.ld = (dim + 3) & ~3u;
    f.metric = metric;
    f.cfg = *cfg;
    f.pq.build((int)dim, (int)cfg->subspaces);
    try {
      PXG_HIP(hipStreamCreateWithFlags(&f.stream, hipStreamNonBlocking));
      f.d_sub_off.alloc(f.pq.M + 1);
      f.d_book_off.alloc(f.pq.M + 1);
      PXG_HIP(hipMemcpy(f.d_sub_off.p, f.pq.off.data(), (f.pq.M + 1) * 4, hipMemcpyHostToDevice));
      PXG_HIP(hipMemcpy(f.d_book_off.p, f.pq.book_off.data(), (f.pq.M + 1) * 4, hipMemcpyHostToDevice));
    } catch (...) {
      delete h;
      throw;
    }
    *out = h;
  });
}

void pxg_ivfpq_destroy(pxg_ivfpq* index) { delete index; }

static void ivfpq_insert_impl(pxg_ivfpq* index, const uint64_t* ids, const float* vectors, uint64_t n,
                              uint32_t* out_slots, bool device) {
  std::unique_lock<std::shared_mutex> lk(index->impl.mu);
  IvfPqIndex& f = index->impl;
  // validate and prepare the whole batch first (all-or-nothing)
  pxg::DevBuf<float> st;
  if (device)
    f.stage_device(vectors, n, st);
  else
    f.stage_host(vectors, n, st);
  {
    std::unordered_map<uint64_t, int> seen;
    for (uint64_t i = 0; i < n; ++i)
      if (f.by_id.count(ids[i]) || !seen.emplace(ids[i], 1).second)
        pxg::raise(PXG_ERR_DUPLICATE_ID, "duplicate vector id " + std::to_string(ids[i]), ids[i]);
  }
  // Auto-training fires when the live count reaches train_threshold
  // (ivfpq.rs:1154-1156): split the batch at that insert.
  uint64_t done = 0;
  while (done < n) {
    uint64_t take = n - done;
    if (!f.trained && f.cfg.train_threshold > f.by_id.size() && f.cfg.train_threshold - f.by_id.size() < take)
      take = f.cfg.train_threshold - f.by_id.size();
    if (done == 0 && take == n) {
      f.insert_rows(ids, st, n, out_slots);
    } else {
      pxg::DevBuf<float> part(take * f.ld);
      PXG_HIP(hipMemcpyAsync(part.p, st.p + done * f.ld, take * f.ld * 4, hipMemcpyDeviceToDevice, f.stream));
      f.insert_rows(ids + done, part, take, out_slots ? out_slots + done : nullptr);
    }
    done += take;
    if (!f.trained && f.by_id.size() >= f.cfg.train_threshold) f.train();
  }
}

int pxg_ivfpq_insert(pxg_ivfpq* index, const uint64_t* ids, const float* vectors, uint64_t n, uint32_t* out_slots) {
  return pxg::guard([&] {
    if (n) ivfpq_insert_impl(index, ids, vectors, n, out_slots, false);
  });
}

int pxg_ivfpq_insert_device(pxg_ivfpq* index, const uint64_t* ids, const float* d_vectors, uint64_t n,
                            uint32_t* out_slots) {
  return pxg::guard([&] {
    if (n) ivfpq_insert_impl(index, ids, d_vectors, n, out_slots, true);
  });
}

int pxg_ivfpq_train(pxg_ivfpq* index, pxg_training_report* report) {
  return pxg::guard([&] {
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    pxg_training_report r = index->impl.train();
    if (report) *report = r;
  });
}

int pxg_ivfpq_training_report(const pxg_ivfpq* index, pxg_training_report* report) {
  return pxg::guard([&] {
    std::shared_lock<std::shared_mutex> lk(index->impl.mu);
    if (!index->impl.has_report) pxg::config_error("trained", 0, "the index has not been trained");
    *report = index->impl.report;
  });
}

int pxg_ivfpq_remove(pxg_ivfpq* index, uint64_t id) {
  return pxg::guard([&] {
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    index->impl.remove(id);
  });
}

int pxg_ivfpq_compact(pxg_ivfpq* index, uint64_t* reclaimed) {
  return pxg::guard([&] {
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    const uint64_t r = index->impl.compact();
    if (reclaimed) *reclaimed = r;
  });
}

int pxg_ivfpq_contains(const pxg_ivfpq* index, uint64_t id) {
  std::shared_lock<std::shared_mutex> lk(index->impl.mu);
  return index->impl.by_id.count(id) ? 1 : 0;
}

uint64_t pxg_ivfpq_len(const pxg_ivfpq* index) {
  std::shared_lock<std::shared_mutex> lk(index->impl.mu);
  return index->impl.by_id.size();
}

int pxg_ivfpq_is_trained(const pxg_ivfpq* index) {
  std::shared_lock<std::shared_mutex> lk(index->impl.mu);
  return index->impl.trained ? 1 : 0;
}

int pxg_ivfpq_stats(const pxg_ivfpq* index, pxg_index_stats* out) {
  return pxg::guard([&] {
    std::shared_lock<std::shared_mutex> lk(index->impl.mu);
    const IvfPqIndex& f = index->impl;
    out->len = f.by_id.size();
    out->deleted = 0;
    out->dim = f.dim;
    out->metric = f.metric;
    out->layers = 1;
    out->edges = 0;
    out->vector_bytes = f.vectors_kept ? f.X.bytes() : 0;
    // codes, lists and codebooks (ivfpq.rs:575-588, 1207-1212)
    out->graph_bytes = f.codes.bytes() + f.d_list_of.bytes() + f.list_slot.bytes() + f.list_beg.bytes() +
                       f.list_end.bytes() +
                       f.list_codes.bytes() + f.cents.bytes() + f.cents_t.bytes() + f.books.bytes();
  });
}

int pxg_ivfpq_get_vector(const pxg_ivfpq* index, uint64_t id, float* out) {
  return pxg::guard([&] {
    std::shared_lock<std::shared_mutex> lk(index->impl.mu);
    const IvfPqIndex& f = index->impl;
    auto it = f.by_id.find(id);
    if (it == f.by_id.end()) pxg::raise(PXG_ERR_UNKNOWN_ID, "unknown vector id " + std::to_string(id), id);
    if (!f.vectors_kept)
      pxg::config_error("retain_vectors", 0, "the full-precision vectors were dropped after training");
    PXG_HIP(hipMemcpy(out, f.X.p + (size_t)it->second * f.ld, f.dim * 4, hipMemcpyDeviceToHost));
  });
}

uint64_t pxg_ivfpq_slot_count(const pxg_ivfpq* index) {
  std::shared_lock<std::shared_mutex> lk(index->impl.mu);
  return index->impl.slots.high_water();
}

int pxg_ivfpq_slots(const pxg_ivfpq* index, uint64_t* ids, uint8_t* live) {
  return pxg::guard([&] {
    std::shared_lock<std::shared_mutex> lk(index->impl.mu);
    const IvfPqIndex& f = index->impl;
    for (size_t s = 0; s < f.slots.high_water(); ++s) {
      if (ids) ids[s] = f.live[s] ? f.ids[s] : 0;
      if (live) live[s] = f.live[s];
    }
  });
}

uint64_t pxg_ivfpq_list_count(const pxg_ivfpq* index) {
  std::shared_lock<std::shared_mutex> lk(index->impl.mu);
  return index->impl.trained ? (uint64_t)index->impl.produced : (uint64_t)index->impl.cfg.nlist;
}

int pxg_ivfpq_list_lengths(const pxg_ivfpq* index, uint64_t* out) {
  return pxg::guard([&] {
    std::shared_lock<std::shared_mutex> lk(index->impl.mu);
    const IvfPqIndex& f = index->impl;
    const size_t nl = f.trained ? (size_t)f.produced : (size_t)f.cfg.nlist;
    std::vector<uint64_t> cnt(nl, 0);
    for (size_t s = 0; s < f.slots.high_water(); ++s)
      if (f.live[s] && f.list_of_h[s] != pxg::UNASSIGNED) cnt[f.list_of_h[s]]++;
    for (size_t l = 0; l < nl; ++l) out[l] = cnt[l];
  });
}

// Download the trained parts (IvfPqIndex::parts, ivfpq.rs:606-617).
int pxg_ivfpq_parts(const pxg_ivfpq* index, float* centroids, float* codebooks, uint8_t* codes, uint32_t* list_of) {
  return pxg::guard([&] {
    std::shared_lock<std::shared_mutex> lk(index->impl.mu);
    const IvfPqIndex& f = index->impl;
    if (!f.trained) pxg::config_error("trained", 0, "the index has no codebooks yet");
    const size_t hw = f.slots.high_water();
    if (centroids)
      PXG_HIP(hipMemcpy2D(centroids, f.dim * 4, f.cents.p, f.ld * 4, f.dim * 4, f.produced, hipMemcpyDeviceToHost));
    if (codebooks) PXG_HIP(hipMemcpy(codebooks, f.books.p, f.pq.book_off[f.pq.M] * 4, hipMemcpyDeviceToHost));
    if (codes && hw) PXG_HIP(hipMemcpy(codes, f.codes.p, hw * f.M(), hipMemcpyDeviceToHost));
    if (list_of)
      for (size_t s = 0; s < hw; ++s) list_of[s] = f.list_of_h[s];
  });
}

// IvfPqIndex::from_parts (ivfpq.rs:624-717): install a trained state on an
// index whose vectors are already inserted (slot table from inserts). codes
// and list_of cover slot_count() slots; NULL codes means "encode on device".
int pxg_ivfpq_load_trained(pxg_ivfpq* index, const float* centroids, uint64_t produced, const float* codebooks,
                           const uint8_t* codes, const uint32_t* list_of) {
  return pxg::guard([&] {
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    IvfPqIndex& f = index->impl;
    if (produced == 0 || produced > f.cfg.nlist) pxg::config_error("produced", produced, "must be between 1 and nlist");
    // every check before any state changes (IvfPqIndex::from_parts builds
    // nothing when it returns an error, ivfpq.rs:624-717)
    const size_t hw = f.slots.high_water();
    if ((codes == nullptr) != (list_of == nullptr))
      pxg::raise(PXG_ERR_CORRUPTION, "corrupt ivfpq index: codes and list assignments come together");
    if (codes) {
      for (size_t s = 0; s < hw; ++s)
        if (f.live[s] && list_of[s] != pxg::UNASSIGNED && list_of[s] >= produced)
          pxg::raise(PXG_ERR_CORRUPTION, "corrupt ivfpq index: slot " + std::to_string(s) + " names list " +
                                             std::to_string(list_of[s]) + " of " + std::to_string(produced));
    } else if (!f.vectors_kept && !f.by_id.empty()) {
      pxg::config_error("codes", 0, "the index keeps no vectors to encode: codes and list assignments are required");
    }
    f.upload_books(centroids, (int)produced, codebooks);
    if (codes) {
      for (size_t s = 0; s < hw; ++s) f.list_of_h[s] = f.live[s] ? list_of[s] : pxg::UNASSIGNED;
      if (hw) {
        PXG_HIP(hipMemcpy(f.codes.p, codes, hw * f.M(), hipMemcpyHostToDevice));
        PXG_HIP(hipMemcpy(f.d_list_of.p, f.list_of_h.data(), hw * 4, hipMemcpyHostToDevice));
      }
      f.csr_dirty = true;
    } else {
      std::vector<uint32_t> sl;
      for (size_t s = 0; s < hw; ++s)
        if (f.live[s]) sl.push_back((uint32_t)s);
      f.encode_slots(sl);
    }
  });
}

int pxg_ivfpq_search(const pxg_ivfpq* index, const float* queries, uint64_t nq, uint64_t k, uint64_t nprobe,
                     const uint8_t* accept, uint64_t* out_ids, float* out_dist, uint32_t* out_count) {
  return pxg::guard([&] {
    pxg::check_k(k);
    IvfPqIndex& f = const_cast<IvfPqIndex&>(index->impl);
    std::shared_lock<std::shared_mutex> lk(f.mu);
    if (nq == 0) return;
    std::vector<float> prep((size_t)nq * f.dim);
    for (uint64_t i = 0; i < nq; ++i) {
      long long bad = pxg::validate_prepare(f.metric, queries + i * f.dim, f.dim, prep.data() + i * f.dim);
      if (bad >= 0)
        pxg::raise(PXG_ERR_NON_FINITE,
                   "vector component " + std::to_string(bad) + " is not finite (" +
                       std::to_string(queries[i * f.dim + bad]) + ")",
                   (uint64_t)bad, i, queries[i * f.dim + bad]);
    }
    // at most the live count per query: device rows of kq, copied into the
    // caller's rows of k
    const uint64_t kq = std::min<uint64_t>(k, f.by_id.size());
    if (kq == 0) {
      for (uint64_t i = 0; i < nq; ++i) out_count[i] = 0;
      return;
    }
    pxg::CtxLease ctx(f.pool);
    pxg::CtxScratch sc(ctx.c);
    hipStream_t s = ctx->stream;
    const size_t N = f.slots.high_water();
    float* d_q = (float*)ctx->get(20, prep.size() * 4);
    uint8_t* d_acc = nullptr;
    if (accept) {
      d_acc = ctx->get(21, N);
      PXG_HIP(hipMemcpyAsync(d_acc, accept, N, hipMemcpyHostToDevice, s));
    }
    uint64_t* d_oid = (uint64_t*)ctx->get(22, nq * kq * 8);
    float* d_od = (float*)ctx->get(23, nq * kq * 4);
    uint32_t* d_oc = (uint32_t*)ctx->get(24, nq * 4);
    PXG_HIP(hipMemcpyAsync(d_q, prep.data(), prep.size() * 4, hipMemcpyHostToDevice, s));
    f.search_device(d_q, false, nq, kq, nprobe ? nprobe : f.cfg.nprobe, d_acc, d_oid, d_od, d_oc, sc, s, kq);
    pxg::results_to_host(*ctx.c, s, nq, k, kq, kq, d_oid, d_od, d_oc, out_ids, out_dist, out_count, [] {});
  });
}

int pxg_ivfpq_search_device(const pxg_ivfpq* index, const float* d_queries, uint64_t nq, uint64_t k, uint64_t nprobe,
                            const uint8_t* d_accept, uint64_t* d_out_ids, float* d_out_dist, uint32_t* d_out_count,
                            void* stream) {
  return pxg::guard([&] {
    pxg::check_k(k);  // first, as ivfpq.rs:988
    IvfPqIndex& f = const_cast<IvfPqIndex&>(index->impl);
    std::shared_lock<std::shared_mutex> lk(f.mu);
    pxg::CtxLease ctx(f.pool);
    pxg::CtxScratch sc(ctx.c);
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    pxg::DrainOnUnwind drain{s};
    f.search_device(d_queries, true, nq, k, nprobe ? nprobe : f.cfg.nprobe, d_accept, d_out_ids, d_out_dist,
                    d_out_count, sc, s, k);
    PXG_HIP(hipStreamSynchronize(s));
  });
}

uint64_t pxg_ivfpq_last_scanned(void) { return pxg::g_last_scanned; }

int pxg_ivfpq_view_stats(const pxg_ivfpq* index, uint64_t* rebuilds, uint64_t* moves) {
  return pxg::guard([&] {
    std::shared_lock<std::shared_mutex> lk(index->impl.mu);
    if (rebuilds) *rebuilds = index->impl.view_rebuilds;
    if (moves) *moves = index->impl.view_moves;
  });
}

}  // extern "C"
