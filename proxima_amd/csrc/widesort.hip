// The segmented radix sort of the large-k search paths (wide.hpp): rocPRIM's
// device segmented radix sort over 64-bit keys, kept in a translation unit of
// its own so that its templates are compiled once; and the exact wide search
// shared by the flat and the untrained IVF-PQ index.
#include <rocprim/device/device_segmented_radix_sort.hpp>

#include <algorithm>

#include "common.hpp"
#include "wide.hpp"

namespace pxg {

size_t wide_sort_temp_bytes(uint32_t total, uint32_t segments) {
  size_t bytes = 0;
  PXG_HIP(rocprim::segmented_radix_sort_keys((void*)nullptr, bytes, (const uint64_t*)nullptr, (uint64_t*)nullptr,
                                             total, segments, (const uint32_t*)nullptr, (const uint32_t*)nullptr, 0,
                                             64, (hipStream_t)0));
  return bytes;
}

void wide_sort(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, uint32_t total, uint32_t segments,
               const uint32_t* begins, const uint32_t* ends, hipStream_t s) {
  if (wide_sort_temp_bytes(total, segments) > temp_bytes)
    internal_error("wide_sort", "sort scratch smaller than the sort asks for");
  size_t bytes = temp_bytes;
  PXG_HIP(rocprim::segmented_radix_sort_keys(temp, bytes, in, out, total, segments, begins, ends, 0, 64, s));
}

void exact_wide_search(const float* Qp, int ld, int dim, int metric, uint64_t nq, uint64_t kq, const float* X,
                       size_t N, const uint8_t* live, const uint8_t* accept, const uint32_t* rank,
                       const uint32_t* rank_slot, const uint64_t* ids, uint64_t* d_oid, float* d_od, uint32_t* d_oc,
                       size_t ldo, Scratch& sc, hipStream_t s) {
  // queries per group: two key buffers of N each, within 1 GiB (or what a
  // fixed scratch holds) and within the sort's 32-bit sizes
  const size_t per_query = 2 * N * 8 + 8;
  size_t G = std::max<size_t>(1, std::min<size_t>((1ull << 30) / per_query, ((1ull << 32) - 1) / N));
  G = std::min<size_t>(G, nq);
  for (;;) {
    const size_t need = G * per_query + 256 * 4 + wide_sort_temp_bytes((uint32_t)(G * N), (uint32_t)G) + 1024;
    if (need <= sc.room() || G == 1) break;
    G = std::max<size_t>(1, G / 2);
  }
  uint64_t* keys = (uint64_t*)sc.get(8, G * N * 8);
  uint64_t* sorted = (uint64_t*)sc.get(9, G * N * 8);
  uint32_t* offs = (uint32_t*)sc.get(10, (G + 1) * 4);
  const size_t temp_bytes = wide_sort_temp_bytes((uint32_t)(G * N), (uint32_t)G);
  void* temp = sc.get(11, std::max<size_t>(temp_bytes, 1));
  for (size_t q0 = 0; q0 < nq; q0 += G) {
    const int gn = (int)std::min<size_t>(G, nq - q0);
    hipLaunchKernelGGL(wide_exact_keys, dim3((unsigned)((N + 31) / 32), (unsigned)gn), dim3(256), 0, s, Qp, ld, dim,
                       metric, X, (int)N, live, accept, rank, (int)q0, N, keys);
    hipLaunchKernelGGL(wide_offsets, dim3((unsigned)((gn + 256) / 256)), dim3(256), 0, s, offs, gn, (uint32_t)N);
    PXG_HIP(hipGetLastError());
    wide_sort(temp, temp_bytes, keys, sorted, (uint32_t)(gn * N), (uint32_t)gn, offs, offs + 1, s);
    hipLaunchKernelGGL(wide_emit, dim3((unsigned)((kq + 255) / 256), (unsigned)gn), dim3(256), 0, s, sorted, offs,
                       offs + 1, (int)q0, kq, rank_slot, ids, d_oid, d_od, d_oc, ldo);
    PXG_HIP(hipGetLastError());
  }
}

}  // namespace pxg
