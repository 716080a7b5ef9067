// Searches whose k exceeds what the block-level selections hold (k > 1024
// after clamping k to the live count): every candidate of a query gets its
// (ord_key(distance) << 32 | id rank) key in a per-query segment of device
// memory, the segments are radix sorted (rocPRIM, widesort.hip), and the
// first min(k, valid) keys of each are emitted. Slower than the selection
// paths, but bounded by no k up to check_k's 2^24 (index.rs:212-224).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "device.hpp"

namespace pxg {

// Temporary bytes the segmented sort of `total` keys in `segments` segments needs.
size_t wide_sort_temp_bytes(uint32_t total, uint32_t segments);
// Sort each segment [offsets[i], offsets[i + 1]) of `in` ascending into `out`.
void wide_sort(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, uint32_t total, uint32_t segments,
               const uint32_t* offsets, hipStream_t s);

// offsets[i] = i * seg for i <= n
static __global__ void wide_offsets(uint32_t* offsets, int n, uint32_t seg) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i <= n) offsets[i] = (uint32_t)i * seg;
}

// Results of queries q0 .. q0 + G - 1 from their sorted segments: the first
// min(kq, valid) keys (KEY_MAX marks no candidate; valid keys sort first).
// Grid (ceil(kq / 256), G).
static __global__ void wide_emit(const uint64_t* __restrict__ sorted, const uint32_t* __restrict__ offsets, int q0,
                                 uint64_t kq, const uint32_t* __restrict__ rank_slot,
                                 const uint64_t* __restrict__ ids, uint64_t* __restrict__ out_ids,
                                 float* __restrict__ out_d, uint32_t* __restrict__ out_count, size_t ldo) {
  const int g = blockIdx.y, q = q0 + g;
  const uint64_t len = offsets[g + 1] - offsets[g];
  const uint64_t take = kq < len ? kq : len;
  const uint64_t* seg = sorted + offsets[g];
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

}  // namespace pxg
