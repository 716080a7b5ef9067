// FlatIndex: the device-resident exact index (crates/proxima-index/src/
// flat.rs:68-236). Defined in flat.hip; the IVF-PQ coarse quantizer reuses it.
#pragma once

#include <mutex>
#include <shared_mutex>
#include <unordered_map>
#include <vector>

#include "common.hpp"
#include "rank.hpp"

namespace pxg {

struct FlatIndex {
  uint32_t dim = 0, ld = 0;
  int metric = 0;
  int mode = 0;  // 0 auto, 1 force MFMA candidates, 2 force exact scan

  // host mirror of the slot table (storage.rs:100-115)
  std::vector<uint64_t> ids;
  std::vector<uint8_t> live;
  std::unordered_map<uint64_t, uint32_t> by_id;
  SlotAllocator slots;
  float maxnorm = 0.0f;

  // device state
  size_t cap = 0;
  DevBuf<float> X;         // cap * ld, prepared vectors, zero padded
  DevBuf<float> xb;        // cap: |x|^2 for L2, 0 otherwise
  DevBuf<uint8_t> d_live;  // cap
  DevBuf<uint64_t> d_ids;  // cap
  RankTable ranks;         // id ranks of the live slots, current after every mutation

  mutable std::shared_mutex mu;
  CtxPool pool;
  hipStream_t stream = nullptr;

  ~FlatIndex();
  void ensure_capacity(size_t need, size_t keep);
  void insert(const uint64_t* in_ids, const float* vecs, uint64_t n, uint32_t* out_slots);
  void remove(uint64_t id);
  // Search nq device queries (raw when do_prepare, else already prepared
  // rows of ld floats); results go to rows of ldo entries. Scratch comes from
  // `sc`; the call returns after the results are complete. With `deferred`
  // given, a search that ends on the exact scan may instead return with its
  // work queued on `s` and the copy of its flag words into sc.host_words()
  // queued after it (*deferred = true): the caller then waits on `s` and
  // calls check_query_flags(sc.host_words()) before using the results.
  void search_device(const float* d_raw, bool do_prepare, uint64_t nq, uint64_t k, const uint8_t* d_accept,
                     uint64_t* d_oid, float* d_od, uint32_t* d_oc, Scratch& sc, hipStream_t s, uint64_t* fallbacks,
                     size_t ldo, bool* deferred = nullptr);
  void search_wide(const float* Qp, uint64_t nq, uint64_t kq, const uint8_t* d_accept, uint64_t* d_oid, float* d_od,
                   uint32_t* d_oc, Scratch& sc, hipStream_t s, size_t ldo);
  void insert_device(const uint64_t* in_ids, const float* d_vecs, uint64_t n, uint32_t* out_slots);
};

// Raises NonFinite when a search's flag words, read back from the device,
// name a non-finite query (word 0: query << 32 | component, all ones when
// every query is finite).
void check_query_flags(const unsigned long long* words);

}  // namespace pxg

// The C ABI handle (include/proxima_hip.h).
struct pxg_flat {
  pxg::FlatIndex impl;
};
