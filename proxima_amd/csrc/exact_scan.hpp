// Kernels shared by every index: query/vector preparation on the device, the
// exact VALU scan (the reference's 8-lane arithmetic, exact (distance, id)
// ordering) used for Manhattan, small problems, unproven MFMA queries and
// untrained IVF-PQ indexes, and a shared-memory bitonic sort. Kernels are
// `static` so each translation unit that includes this header owns a copy.
#pragma once

#include "device.hpp"

namespace pxg {

constexpr int EXACT_CH = 1024;

// Rows per chunk of the exact scan: EXACT_CH, or 256 when EXACT_CH-row
// chunks would give the launch fewer workgroups than there are CUs (a single
// query over a small store), so that more of the GPU scans at once.
inline int exact_chunk_rows(size_t nq, size_t N) {
  return nq * ((N + EXACT_CH - 1) / EXACT_CH) < 256 ? 256 : EXACT_CH;
}

// Small fills done by kernels rather than memsets (so that a caller's stream
// holds only kernel work): the query flag word ~0, the flagged-query count 0.
[[maybe_unused]] static __global__ void init_search_flags(unsigned long long* bad, int* flag_count) {
  if (threadIdx.x == 0) {
    *bad = ~0ull;
    *flag_count = 0;
  }
}
// init_search_flags that also clears the n 64-bit words at `words` (a
// search's counters beside its flags), saving a fill launch.
[[maybe_unused]] static __global__ void init_search_flags_zero(unsigned long long* bad, int* flag_count,
                                                               unsigned long long* words, int n) {
  if (threadIdx.x == 0) {
    *bad = ~0ull;
    *flag_count = 0;
  }
  for (int i = threadIdx.x; i < n; i += blockDim.x) words[i] = 0;
}
[[maybe_unused]] static __global__ void fill_u32(uint32_t* p, size_t n, uint32_t v) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}
[[maybe_unused]] static __global__ void set_int(int* p, int v) {
  if (threadIdx.x == 0) *p = v;
}

// ---------------------------------------------------------------------------
// 1. query preparation
// ---------------------------------------------------------------------------
// One 64-thread workgroup per row: validate, (cosine) normalise, pad to ld.
__device__ inline void prep_query_row(const float* __restrict__ raw, int dim, int ld, int metric, int do_prepare,
                                      float* __restrict__ Qp, float* __restrict__ qb, float* __restrict__ qn,
                                      unsigned long long* __restrict__ bad) {
  const int q = blockIdx.x;
  const int lane = threadIdx.x;
  const float* v = raw + (size_t)q * dim;
  float* out = Qp + (size_t)q * ld;
  __shared__ float s_inv;
  // validate: first non-finite component (space.rs:104-121)
  for (int i = lane; i < dim; i += 64) {
    if (!isfinite(v[i])) atomicMin(bad, ((unsigned long long)q << 32) | (unsigned)i);
  }
  if (lane < 8) {
    float d = dist_group8<2>(v, v, dim, lane);  // = -dot_unrolled(v, v)
    if (lane == 0) {
      float dot = -d;
      float inv = 1.0f;
      if (do_prepare && metric == 1) {
        float n = sqrtf(dot);
        inv = (n > 0.0f && isfinite(n)) ? 1.0f / n : 1.0f;
        s_inv = (n > 0.0f && isfinite(n)) ? inv : 0.0f;  // 0 marks "leave untouched"
      } else {
        s_inv = 0.0f;
      }
    }
  }
  __syncthreads();
  const float inv = s_inv;
  for (int i = lane; i < ld; i += 64) {
    float x = i < dim ? v[i] : 0.0f;
    if (inv != 0.0f) x = x * inv;
    out[i] = x;
  }
  __syncthreads();
  if (lane < 8) {
    float d = -dist_group8<2>(out, out, dim, lane);
    if (lane == 0) {
      qn[q] = sqrtf(d);
      qb[q] = metric == 0 ? d : (metric == 1 ? 1.0f : 0.0f);
    }
  }
}

[[maybe_unused]] static __global__ __launch_bounds__(64) void flat_prep_queries(const float* __restrict__ raw, int dim,
                                                                                int ld, int metric, int do_prepare,
                                                                                float* __restrict__ Qp,
                                                                                float* __restrict__ qb,
                                                                                float* __restrict__ qn,
                                                                                unsigned long long* __restrict__ bad) {
  prep_query_row(raw, dim, ld, metric, do_prepare, Qp, qb, qn, bad);
}

// flat_prep_queries for a flat search, which also sets each query's shared
// candidate threshold to its initial "none" (~0), saving the search a fill
// launch ahead of its candidate passes.
[[maybe_unused]] static __global__ __launch_bounds__(64) void flat_prep_search_queries(
    const float* __restrict__ raw, int dim, int ld, int metric, int do_prepare, float* __restrict__ Qp,
    float* __restrict__ qb, float* __restrict__ qn, unsigned long long* __restrict__ bad,
    unsigned long long* __restrict__ gthr) {
  if (threadIdx.x == 0) gthr[blockIdx.x] = ~0ull;
  prep_query_row(raw, dim, ld, metric, do_prepare, Qp, qb, qn, bad);
}

// ---------------------------------------------------------------------------
// shared-memory bitonic sort (ascending) of n = power-of-two keys
// ---------------------------------------------------------------------------
__device__ inline void block_bitonic_sort(uint64_t* keys, int n) {
  for (int size = 2; size <= n; size <<= 1) {
    for (int j = size >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < (n >> 1); i += blockDim.x) {
        const int idx = ((i / j) * 2 * j) + (i % j);
        const bool asc = (idx & size) == 0;
        const uint64_t a = keys[idx], b = keys[idx + j];
        if ((a > b) == asc) {
          keys[idx] = b;
          keys[idx + j] = a;
        }
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------
// 4. exact VALU scan for a list of queries
// ---------------------------------------------------------------------------
// Work item (chunk c, query group): the CH rows of chunk c against QG of the
// listed queries (the last group may hold fewer). With QG > 1 the group's
// queries are staged in LDS and each lane pair loads a row chunk once for the
// whole group (dist_pair4_multi), so the store streams through L2 once per
// group instead of once per query (exact_query_group decides when). Each query's keys are sorted on their own,
// and its kk smallest go to ecand[(f * nchunks + c) * kk], as with QG = 1.
constexpr int EXACT_QG_MAXD = 1024;
template <int CH, int QG = 1>
[[maybe_unused]] static __global__ __launch_bounds__(256) void flat_exact_candidates(
    const int* __restrict__ qlist, const int* __restrict__ qcount, int nchunks, const float* __restrict__ Qp, int ld,
    int dim, int metric, const float* __restrict__ X, int N, const uint8_t* __restrict__ live,
    const uint8_t* __restrict__ accept, const uint32_t* __restrict__ rank, int k, uint64_t* __restrict__ ecand) {
  __shared__ uint64_t keys[QG][CH];
  __shared__ __align__(16) float sq[QG > 1 ? QG : 1][QG > 1 ? EXACT_QG_MAXD : 4];
  const int nf = *qcount;
  const int ng = (nf + QG - 1) / QG;
  const int total = ng * nchunks;
  const int g = threadIdx.x & 7, grp = threadIdx.x >> 3;
  const int kk = min(k, CH);
  // Chunk-major work order, dealt to the XCDs in contiguous ranges: the
  // query groups of one chunk run on one XCD at about the same time and share
  // its L2 copy of the chunk's rows. Workgroup ids go round-robin over the 8
  // XCDs and the grid is a multiple of 8, so w & 7 keeps naming the same XCD
  // on every pass of the grid-stride loop.
  const int per_xcd = (total + 7) / 8;
  for (int w = blockIdx.x; w < 8 * per_xcd; w += gridDim.x) {
    const int item = (w & 7) * per_xcd + (w >> 3);
    if (item >= total) continue;  // uniform over the workgroup
    const int c = item / ng, f0 = (item % ng) * QG;
    const int nv = min(QG, nf - f0);
    const float* qv[QG];
    if constexpr (QG > 1) {
      // the group's queries in LDS (the previous item's last barrier has
      // passed, so nothing still reads them)
      for (int i = threadIdx.x; i < nv * dim; i += blockDim.x) {
        const int j = i / dim;
        sq[j][i - j * dim] = Qp[(size_t)qlist[f0 + j] * ld + (i - j * dim)];
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < QG; ++j) qv[j] = &sq[j][0];
    } else {
      qv[0] = Qp + (size_t)qlist[f0] * ld;
    }
    const int base = c * CH;
    if (QG > 1 || dim >= 8) {
      // two lanes per row (dist_pair4): 128 rows per pass of the workgroup,
      // one float4 per lane per 8-wide chunk; rows past N or not usable are
      // scored from a clamped row (both lanes of a pair take part in its
      // shuffle) and keep KEY_MAX
      const int h = threadIdx.x & 1;
      for (int s = threadIdx.x >> 1; s < CH; s += 128) {
        const int slot = base + s;
        const bool u = slot < N && live[slot] && (accept == nullptr || accept[slot]);
        uint64_t key[QG];
#pragma unroll
        for (int j = 0; j < QG; ++j) key[j] = KEY_MAX;
        if (__any(u)) {
          const float* row = X + (size_t)max(min(slot, N - 1), 0) * ld;
          float d[QG];
          if constexpr (QG == 1) d[0] = dist_pair4_rt(metric, qv[0], row, dim, h);
          else dist_pair4_multi_rt<QG>(metric, qv, row, dim, h, d, nv);
          if (u) {
            const uint32_t rk = rank[slot];
#pragma unroll
            for (int j = 0; j < QG; ++j) key[j] = ((uint64_t)ord_key(d[j]) << 32) | rk;
          }
        }
        if (h == 0) {
#pragma unroll
          for (int j = 0; j < QG; ++j) keys[j][s] = key[j];
        }
      }
    } else {
      // rows narrower than one 8-wide chunk: eight lanes per row
      for (int s = grp; s < CH; s += 32) {
        const int slot = base + s;
        uint64_t key = KEY_MAX;
        if (slot < N && live[slot] && (accept == nullptr || accept[slot])) {
          const float d = dist_group8_rt(metric, qv[0], X + (size_t)slot * ld, dim, g);
          key = ((uint64_t)ord_key(d) << 32) | rank[slot];
        }
        if (g == 0) keys[0][s] = key;
      }
    }
    __syncthreads();
    for (int j = 0; j < nv; ++j) {
      block_bitonic_sort(keys[j], CH);
      uint64_t* out = ecand + ((size_t)(f0 + j) * nchunks + c) * kk;
      for (int i = threadIdx.x; i < kk; i += blockDim.x) out[i] = keys[j][i];
    }
    __syncthreads();
  }
}

// Query group size of the exact scan for nq queries of dim floats over N
// rows: four queries share each row load for rows of 256 to EXACT_QG_MAXD
// floats, at least four queries, and at least 512 grouped work items of
// EXACT_CH rows. Measured against one query per item (mode 2, k = 10):
// 1M x 768 with 4/8/128 queries 1.45/2.53/36.0 -> 1.29/1.62/16.3 ms,
// 300k x 256 with 8/16/128 queries 0.31/0.50/3.45 -> 0.30/0.44/2.25 ms; where
// the groups leave fewer items the GPU idles (300k x 256 with 4 queries, 293
// items: 0.21 -> 0.26 ms), and with narrower rows or two queries they lost
// too (1M x 768 with 2 queries 0.89 -> 1.06 ms, 100k x 128 with 32 queries
// 0.21 -> 0.29 ms): the per-query sorts stay, and four times fewer items
// keep fewer workgroups busy.
inline int exact_query_group(size_t nq, size_t dim, size_t N) {
  const size_t items = (nq + 3) / 4 * ((N + EXACT_CH - 1) / EXACT_CH);
  return (nq >= 4 && dim >= 256 && dim <= EXACT_QG_MAXD && items >= 512) ? 4 : 1;
}

constexpr int EXACT_MERGE_MAXK = 1024;

template <int CH>
[[maybe_unused]] static __global__ __launch_bounds__(256) void flat_merge_exact(const int* __restrict__ qlist, const int* __restrict__ qcount,
                                                        const uint64_t* __restrict__ ecand, int nchunks, int k,
                                                        const uint32_t* __restrict__ rank_slot,
                                                        const uint64_t* __restrict__ ids,
                                                        uint64_t* __restrict__ out_ids, float* __restrict__ out_d,
                                                        uint32_t* __restrict__ out_count,
                                                        uint64_t* __restrict__ out_keys, size_t ldo) {
  const int f = blockIdx.x;
  if (f >= *qcount) return;
  const int q = qlist[f];
  __shared__ int hist[256];
  __shared__ uint64_t sh[4];
  __shared__ uint64_t sel[EXACT_MERGE_MAXK];
  __shared__ int n_sel, n_valid;
  const int kk = min(k, CH);
  const uint64_t* base = ecand + (size_t)f * nchunks * kk;
  const int n = nchunks * kk;
  auto get = [&](int i) -> uint64_t { return base[i]; };
  if (threadIdx.x == 0) {
    n_sel = 0;
    n_valid = 0;
  }
  __syncthreads();
  int local = 0;
  // four keys per thread per step, loaded together before any is used
  for (int i0 = threadIdx.x; i0 < n; i0 += 4 * blockDim.x) {
    uint64_t x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = base[min(i0 + u * (int)blockDim.x, n - 1)];
#pragma unroll
    for (int u = 0; u < 4; ++u) local += (i0 + u * (int)blockDim.x < n && x[u] != KEY_MAX) ? 1 : 0;
  }
  atomicAdd(&n_valid, local);
  __syncthreads();
  const int ksel = min(k, n_valid);
  if (ksel == 0) {
    if (threadIdx.x == 0) out_count[q] = 0;
    return;
  }
  const uint64_t pivot = n <= 16 * (int)blockDim.x   ? block_radix_select<decltype(get), 64, 16>(get, n, ksel, hist, sh)
                         : n <= 40 * (int)blockDim.x ? block_radix_select<decltype(get), 64, 40>(get, n, ksel, hist, sh)
                                                     : block_radix_select(get, n, ksel, hist, sh);
  for (int i0 = threadIdx.x; i0 < n; i0 += 4 * blockDim.x) {
    uint64_t x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = base[min(i0 + u * (int)blockDim.x, n - 1)];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (i0 + u * (int)blockDim.x < n && x[u] <= pivot && x[u] != KEY_MAX) sel[atomicAdd(&n_sel, 1)] = x[u];
  }
  __syncthreads();
  int P = 1;
  while (P < ksel) P <<= 1;
  for (int i = ksel + threadIdx.x; i < P; i += blockDim.x) sel[i] = KEY_MAX;
  __syncthreads();
  block_bitonic_sort(sel, P);
  for (int i = threadIdx.x; i < ksel; i += blockDim.x) {
    const uint64_t key = sel[i];
    if (out_keys) {
      out_keys[(size_t)q * ldo + i] = key;  // (distance, id rank) keys for a later stage
    } else {
      out_ids[(size_t)q * ldo + i] = ids[rank_slot[(uint32_t)key]];
      out_d[(size_t)q * ldo + i] = key_float((uint32_t)(key >> 32));
    }
  }
  if (threadIdx.x == 0) out_count[q] = ksel;
}

[[maybe_unused]] static __global__ void iota_kernel(int* a, int n, int* count) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) a[i] = i;
  if (i == 0) *count = n;
}

// Scatter staged rows into their slots (insert path); X and xb may be null
// (an index that keeps no full-precision rows).
[[maybe_unused]] static __global__ void flat_scatter_rows(const float* __restrict__ staged, const uint32_t* __restrict__ slots,
                                  const float* __restrict__ bias, const uint64_t* __restrict__ sid, int n, int ld,
                                  float* __restrict__ X, float* __restrict__ xb, uint8_t* __restrict__ live,
                                  uint64_t* __restrict__ ids) {
  const int i = blockIdx.x;
  if (i >= n) return;
  const uint32_t s = slots[i];
  if (X != nullptr)
    for (int c = threadIdx.x; c < ld; c += blockDim.x) X[(size_t)s * ld + c] = staged[(size_t)i * ld + c];
  if (threadIdx.x == 0) {
    if (xb != nullptr) xb[s] = bias[i];
    live[s] = 1;
    ids[s] = sid[i];
  }
}


}  // namespace pxg
