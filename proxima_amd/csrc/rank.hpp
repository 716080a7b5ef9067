// The id-rank table of an index, kept current on the device at every
// mutation.
//
// Every search orders candidates by (total_cmp(distance), id), which is
// SearchResult's order (topk.rs:63-67). The kernels carry, instead of the
// 64-bit id, its rank among the live ids in a 32-bit field of each 64-bit
// key, so a key sorts exactly as (distance, id). The table holds
//   rank[slot]       the rank of the slot's id (live slots only),
//   rank_slot[r]     the slot of the id of rank r, r < len,
// and is updated in O(len) device work per insert batch or removal (no host
// sort, no rebuild at search time):
//   insert: the batch's (id, slot) pairs are sorted by id on the host, then an
//           old rank r moves to r + #(new ids below its id) and a new pair j
//           lands at j + #(old ids below its id), both by binary search;
//   remove: ranks above the removed one move down by one.
// Both write a second rank_slot buffer and swap, so no kernel reads what
// another thread of it writes.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <numeric>
#include <vector>

#include "common.hpp"

namespace pxg {

static __global__ void rank_merge_old(const uint32_t* __restrict__ rank_slot, uint32_t len,
                                      const uint64_t* __restrict__ ids, const uint64_t* __restrict__ new_ids,
                                      uint32_t n, uint32_t* __restrict__ out_rank_slot, uint32_t* __restrict__ rank) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= len) return;
  const uint32_t s = rank_slot[r];
  const uint64_t id = ids[s];
  uint32_t lo = 0, hi = n;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (new_ids[mid] < id) lo = mid + 1;
    else hi = mid;
  }
  out_rank_slot[r + lo] = s;
  rank[s] = r + lo;
}

static __global__ void rank_merge_new(const uint32_t* __restrict__ rank_slot, uint32_t len,
                                      const uint64_t* __restrict__ ids, const uint64_t* __restrict__ new_ids,
                                      const uint32_t* __restrict__ new_slots, uint32_t n,
                                      uint32_t* __restrict__ out_rank_slot, uint32_t* __restrict__ rank) {
  const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const uint64_t id = new_ids[j];
  uint32_t lo = 0, hi = len;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (ids[rank_slot[mid]] < id) lo = mid + 1;
    else hi = mid;
  }
  out_rank_slot[j + lo] = new_slots[j];
  rank[new_slots[j]] = j + lo;
}

// Drop the removed slot's entry. No thread writes rank[removed_slot], so
// every thread may read it.
static __global__ void rank_drop(const uint32_t* __restrict__ rank_slot, uint32_t len, uint32_t removed_slot,
                                 uint32_t* __restrict__ out_rank_slot, uint32_t* __restrict__ rank) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= len) return;
  const uint32_t removed = rank[removed_slot];
  const uint32_t s = rank_slot[r];
  if (r < removed) {
    out_rank_slot[r] = s;
  } else if (r > removed) {
    out_rank_slot[r - 1] = s;
    rank[s] = r - 1;
  }
}

struct RankTable {
  DevBuf<uint32_t> rank;       // per slot
  DevBuf<uint32_t> rank_slot;  // per rank
  DevBuf<uint32_t> spare;      // the other rank_slot buffer
  uint32_t len = 0;

  // Slot capacity grew to `cap` (the first `keep` slots are kept).
  void grow(size_t cap, size_t keep, hipStream_t s) { rank.grow(cap, keep, s); }

  // After a batch of n new live (id, slot) pairs was written to d_ids (ids
  // unique and absent before). h_ids / h_slots are host arrays.
  void insert(const uint64_t* h_ids, const uint32_t* h_slots, uint64_t n, const uint64_t* d_ids, hipStream_t s) {
    if (n == 0) return;
    std::vector<uint64_t> sid(n);
    std::vector<uint32_t> sslot(n);
    bool sorted = true;
    for (uint64_t i = 1; i < n && sorted; ++i) sorted = h_ids[i - 1] < h_ids[i];
    if (sorted) {
      std::copy(h_ids, h_ids + n, sid.begin());
      std::copy(h_slots, h_slots + n, sslot.begin());
    } else {
      std::vector<uint32_t> ord(n);
      std::iota(ord.begin(), ord.end(), 0u);
      std::sort(ord.begin(), ord.end(), [&](uint32_t a, uint32_t b) { return h_ids[a] < h_ids[b]; });
      for (uint64_t i = 0; i < n; ++i) {
        sid[i] = h_ids[ord[i]];
        sslot[i] = h_slots[ord[i]];
      }
    }
    const size_t total = (size_t)len + n;
    if (rank_slot.n < total) {
      const size_t c = std::max<size_t>(total, rank_slot.n * 2);
      rank_slot.grow(c, len, s);
      spare.alloc(c);
    }
    DevBuf<uint64_t> d_new(n);
    DevBuf<uint32_t> d_slots(n);
    PXG_HIP(hipMemcpyAsync(d_new.p, sid.data(), n * 8, hipMemcpyHostToDevice, s));
    PXG_HIP(hipMemcpyAsync(d_slots.p, sslot.data(), n * 4, hipMemcpyHostToDevice, s));
    if (len)
      hipLaunchKernelGGL(rank_merge_old, dim3((len + 255) / 256), dim3(256), 0, s, rank_slot.p, len, d_ids, d_new.p,
                         (uint32_t)n, spare.p, rank.p);
    hipLaunchKernelGGL(rank_merge_new, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, rank_slot.p, len, d_ids,
                       d_new.p, d_slots.p, (uint32_t)n, spare.p, rank.p);
    PXG_HIP(hipGetLastError());
    PXG_HIP(hipStreamSynchronize(s));  // the staged pairs are freed on return
    std::swap(rank_slot, spare);
    len = (uint32_t)total;
  }

  // After the live slot `slot` was removed (its rank entry still current).
  void remove(uint32_t slot, hipStream_t s) {
    hipLaunchKernelGGL(rank_drop, dim3((len + 255) / 256), dim3(256), 0, s, rank_slot.p, len, slot, spare.p, rank.p);
    PXG_HIP(hipGetLastError());
    std::swap(rank_slot, spare);
    --len;
  }

  void clear() { len = 0; }
};

}  // namespace pxg
