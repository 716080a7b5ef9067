// pxg_flat_search_device_noalloc: the exact flat search of flat.hip that
// allocates nothing (no hipMalloc, hipFree, pinned host memory, stream or
// event), for callers that cannot allocate. The search pipeline is
// FlatIndex::search_device with its scratch carved from a fixed block.
#include <mutex>
#include <shared_mutex>
#include <string>

#include "common.hpp"
#include "flat.hpp"

namespace pxg {

void set_last_fallbacks(uint64_t v);

// Scratch of pxg_flat_search_device_noalloc: a fixed block per GPU, held
// until the process ends. Its name is a host-side stand-in; host code uses
// the device address from hipGetSymbolAddress.
constexpr size_t NOALLOC_SCRATCH_BYTES = 128ull << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];
constexpr int NOALLOC_MAX_DEVICES = 64;
static std::mutex g_noalloc_mu[NOALLOC_MAX_DEVICES];
static void* g_noalloc_ptr[NOALLOC_MAX_DEVICES];

}  // namespace pxg

using pxg::FlatIndex;

extern "C" {

// The search that allocates nothing: its scratch is `scratch`, one static
// device array per GPU (each GPU holds its own copy at its own address, which
// hipGetSymbolAddress gives once per device with that device current; host
// code uses only that address). Calls on one GPU share the array, so a
// per-GPU lock serializes them, and each call has finished on the GPU when it
// returns, also when it fails: a request too large for the array fails with
// Capacity when it reaches the first region that does not fit, possibly after
// earlier stages were queued, and those are waited for before the lock is
// released.
int pxg_flat_search_device_noalloc(const pxg_flat* index, const float* d_queries, uint64_t nq, uint64_t k,
                                   const uint8_t* d_accept, uint64_t* d_out_ids, float* d_out_dist,
                                   uint32_t* d_out_count, void* stream) {
  return pxg::guard([&] {
    pxg::check_k(k);
    int dev = 0;
    PXG_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= pxg::NOALLOC_MAX_DEVICES)
      pxg::raise(PXG_ERR_CONFIGURATION, "device index beyond the no-allocation search's table", (uint64_t)dev);
    std::lock_guard<std::mutex> g(pxg::g_noalloc_mu[dev]);
    if (pxg::g_noalloc_ptr[dev] == nullptr) {
      void* p = nullptr;
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(pxg::scratch));
      if (e != hipSuccess || p == nullptr)
        pxg::internal_error("pxg_flat_search_device_noalloc",
                            std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
      pxg::g_noalloc_ptr[dev] = p;
    }
    FlatIndex& f = const_cast<FlatIndex&>(index->impl);
    std::shared_lock<std::shared_mutex> lk(f.mu);
    pxg::Arena arena(pxg::g_noalloc_ptr[dev], pxg::NOALLOC_SCRATCH_BYTES);
    hipStream_t s = (hipStream_t)stream;
    pxg::DrainOnUnwind drain{s};  // after the lock: an error waits for queued work before the lock is released
    uint64_t fb = 0;
    f.search_device(d_queries, true, nq, k, d_accept, d_out_ids, d_out_dist, d_out_count, arena, s, &fb, k);
    PXG_HIP(hipStreamSynchronize(s));
    pxg::set_last_fallbacks(fb);
  });
}

}  // extern "C"
