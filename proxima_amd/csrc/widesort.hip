// The segmented radix sort of the large-k search paths (wide.hpp): rocPRIM's
// device segmented radix sort over 64-bit keys, kept in a translation unit of
// its own so that its templates are compiled once.
#include <rocprim/device/device_segmented_radix_sort.hpp>

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
               const uint32_t* offsets, hipStream_t s) {
  size_t bytes = temp_bytes;
  PXG_HIP(rocprim::segmented_radix_sort_keys(temp, bytes, in, out, total, segments, offsets, offsets + 1, 0, 64, s));
}

}  // namespace pxg
