// Searches whose k (or shortlist) exceeds what the block-level selections
// hold: every candidate of a query gets its (ord_key(distance) << 32 | id
// rank) key in a per-query segment of device memory, the segments are radix
// sorted (rocPRIM, widesort.hip), optionally the first t keys of each are
// rescored and sorted again (IVF-PQ rerank, SQ8 rescoring), and the first
// min(k, valid) keys of each are emitted. Slower than the selection paths,
// but bounded by no k up to check_k's 2^24 (index.rs:212-224).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"
#include "device.hpp"

namespace pxg {

// Temporary bytes the segmented sort of `total` keys in `segments` segments needs.
size_t wide_sort_temp_bytes(uint32_t total, uint32_t segments);
// Sort each segment [begins[i], ends[i]) of `in` ascending into the same
// positions of `out`.
void wide_sort(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, uint32_t total, uint32_t segments,
               const uint32_t* begins, const uint32_t* ends, hipStream_t s);

// Exact search over a slot-major store for kq beyond the block selections
// (the flat index and the untrained IVF-PQ index): keys of every slot,
// segmented sort, first kq. Results go to rows of ldo entries.
void exact_wide_search(const float* Qp, int ld, int dim, int metric, uint64_t nq, uint64_t kq, const float* X,
                       size_t N, const uint8_t* live, const uint8_t* accept, const uint32_t* rank,
                       const uint32_t* rank_slot, const uint64_t* ids, uint64_t* d_oid, float* d_od, uint32_t* d_oc,
                       size_t ldo, Scratch& sc, hipStream_t s);

// offsets[i] = i * seg for i <= n
[[maybe_unused]] static __global__ void wide_offsets(uint32_t* offsets, int n, uint32_t seg) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i <= n) offsets[i] = (uint32_t)i * seg;
}

// ends[g] = begins[g] + min(t, ends_in[g] - begins[g])
[[maybe_unused]] static __global__ void wide_truncate(const uint32_t* __restrict__ begins, const uint32_t* __restrict__ ends_in,
                                     int n, uint64_t t, uint32_t* __restrict__ ends) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= n) return;
  const uint64_t len = ends_in[g] - begins[g];
  ends[g] = begins[g] + (uint32_t)(len < t ? len : t);
}

// Results of queries q0 .. q0 + G - 1 from their sorted segments: the first
// min(kq, valid) keys (KEY_MAX marks no candidate; valid keys sort first).
// Grid (ceil(kq / 256), G).
[[maybe_unused]] static __global__ void wide_emit(const uint64_t* __restrict__ sorted, const uint32_t* __restrict__ begins,
                                 const uint32_t* __restrict__ ends, int q0, uint64_t kq,
                                 const uint32_t* __restrict__ rank_slot, const uint64_t* __restrict__ ids,
                                 uint64_t* __restrict__ out_ids, float* __restrict__ out_d,
                                 uint32_t* __restrict__ out_count, size_t ldo) {
  const int g = blockIdx.y, q = q0 + g;
  const uint64_t len = ends[g] - begins[g];
  const uint64_t take = kq < len ? kq : len;
  const uint64_t* seg = sorted + begins[g];
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (take == 0) {
    if (i == 0) out_count[q] = 0;
    return;
  }
  if (i >= take) return;
  const uint64_t key = seg[i];
  const bool valid = key != KEY_MAX;
  if (valid) {
    out_ids[(size_t)q * ldo + i] = ids[rank_slot[(uint32_t)key]];
    out_d[(size_t)q * ldo + i] = key_float((uint32_t)(key >> 32));
  }
  // the last valid key of the first `take` writes the count
  const bool next_invalid = i + 1 == take || seg[i + 1] == KEY_MAX;
  if (valid && next_invalid) out_count[q] = (uint32_t)(i + 1);
  if (i == 0 && !valid) out_count[q] = 0;
}

// Exact (distance, id rank) keys of every slot for queries q0 .. q0 + G - 1
// (grid (ceil(N / 32), G), 8 threads per slot), KEY_MAX for free or
// filtered slots; segment g starts at g * seg.
[[maybe_unused]] static __global__ __launch_bounds__(256) void wide_exact_keys(const float* __restrict__ Qp, int ld, int dim,
                                                              int metric, const float* __restrict__ X, int N,
                                                              const uint8_t* __restrict__ live,
                                                              const uint8_t* __restrict__ accept,
                                                              const uint32_t* __restrict__ rank, int q0, size_t seg,
                                                              uint64_t* __restrict__ keys) {
  const int g = threadIdx.x & 7;
  const int slot = blockIdx.x * 32 + (threadIdx.x >> 3);
  const float* qv = Qp + (size_t)(q0 + blockIdx.y) * ld;
  if (slot >= N) return;
  uint64_t key = KEY_MAX;
  if (live[slot] && (accept == nullptr || accept[slot])) {
    const float d = dist_group8_rt(metric, qv, X + (size_t)slot * ld, dim, g);
    key = ((uint64_t)ord_key(d) << 32) | rank[slot];
  }
  if (g == 0) keys[(size_t)blockIdx.y * seg + slot] = key;
}

}  // namespace pxg
