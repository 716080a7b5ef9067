// Host-side plumbing shared by every index in libproxima_hip: status codes,
// the thread-local last-error record, HIP error checks and RAII device
// buffers. No C++ exception crosses the C ABI: every entry point runs its
// body through pxg::guard(), which maps exceptions to status codes.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <exception>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/proxima_hip.h"

namespace pxg {

// The error the C ABI reports, with the fields ProximaError carries
// (error.rs:37-160) so the caller can rebuild the variant exactly.
struct Error {
  int status;
  std::string message;
  uint64_t a = 0, b = 0;  // expected/actual, index, id or limit, per variant
  float value = 0.0f;
  // Configuration: the parameter's name and the constraint it broke;
  // Capacity: the structure that ran out of room. Always string literals
  // (static storage), so the C ABI can hand the pointers out as they are.
  const char* parameter = "";
  const char* reason = "";
};

struct Raise {
  Error e;
};

void set_last_error(const Error& e);
void clear_last_error();

[[noreturn]] inline void raise(int status, std::string msg, uint64_t a = 0, uint64_t b = 0, float v = 0.0f) {
  throw Raise{Error{status, std::move(msg), a, b, v}};
}
// `parameter` and `reason` must be string literals.
[[noreturn]] inline void config_error(const char* parameter, uint64_t value, const char* reason) {
  Error e{PXG_ERR_CONFIGURATION,
          std::string("invalid configuration: ") + parameter + " = " + std::to_string(value) + " (" + reason + ")",
          value};
  e.parameter = parameter;
  e.reason = reason;
  throw Raise{std::move(e)};
}
// Capacity{what, limit} (error.rs:80-85); `what` must be a string literal.
[[noreturn]] inline void capacity_error(const char* what, uint64_t limit, std::string msg) {
  Error e{PXG_ERR_CAPACITY, std::move(msg), limit};
  e.parameter = what;
  throw Raise{std::move(e)};
}
[[noreturn]] inline void internal_error(const char* location, const std::string& detail) {
  raise(PXG_ERR_INTERNAL, std::string("internal invariant violated in ") + location + ": " + detail);
}

#define PXG_HIP(call)                                                                         \
  do {                                                                                        \
    hipError_t e_ = (call);                                                                   \
    if (e_ != hipSuccess) {                                                                   \
      if (e_ == hipErrorOutOfMemory || e_ == hipErrorMemoryAllocation)                        \
        ::pxg::capacity_error("device memory", 0,                                              \
                              std::string("capacity exceeded: device memory limit (") +        \
                                  hipGetErrorString(e_) + ")");                                \
      ::pxg::internal_error(#call, hipGetErrorString(e_));                                    \
    }                                                                                         \
  } while (0)

template <class F>
int guard(F&& f) {
  try {
    f();
    clear_last_error();
    return PXG_OK;
  } catch (const Raise& r) {
    set_last_error(r.e);
    return r.e.status;
  } catch (const std::bad_alloc&) {
    Error e{PXG_ERR_CAPACITY, "capacity exceeded: host memory"};
    e.parameter = "host memory";
    set_last_error(e);
    return PXG_ERR_CAPACITY;
  } catch (const std::exception& ex) {
    set_last_error(Error{PXG_ERR_INTERNAL, std::string("internal invariant violated: ") + ex.what()});
    return PXG_ERR_INTERNAL;
  } catch (...) {
    set_last_error(Error{PXG_ERR_INTERNAL, "internal invariant violated: unknown exception"});
    return PXG_ERR_INTERNAL;
  }
}

// Owning device allocation.
template <class T>
struct DevBuf {
  T* p = nullptr;
  size_t n = 0;
  DevBuf() = default;
  explicit DevBuf(size_t count) { alloc(count); }
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  DevBuf(DevBuf&& o) noexcept : p(o.p), n(o.n) { o.p = nullptr; o.n = 0; }
  DevBuf& operator=(DevBuf&& o) noexcept {
    if (this != &o) { release(); p = o.p; n = o.n; o.p = nullptr; o.n = 0; }
    return *this;
  }
  ~DevBuf() { release(); }
  void alloc(size_t count) {
    release();
    if (count) PXG_HIP(hipMalloc(&p, count * sizeof(T)));
    n = count;
  }
  // Grow to at least `count`, keeping the first `keep` elements.
  void grow(size_t count, size_t keep, hipStream_t s) {
    if (count <= n) return;
    T* q = nullptr;
    PXG_HIP(hipMalloc(&q, count * sizeof(T)));
    if (keep && p) PXG_HIP(hipMemcpyAsync(q, p, keep * sizeof(T), hipMemcpyDeviceToDevice, s));
    PXG_HIP(hipStreamSynchronize(s));
    release();
    p = q;
    n = count;
  }
  // Ensure capacity without preserving contents.
  void reserve(size_t count) {
    if (count > n) alloc(count);
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
  }
  size_t bytes() const { return n * sizeof(T); }
};

// Copy `rows` rows of `width` bytes from device rows `spitch` bytes apart to
// host rows `dpitch` bytes apart. A strided copy into pageable memory goes
// row by row, so the rows come over in one contiguous copy and are spread on
// the host; equal pitches take one direct copy. Returns after the copy.
inline void rows_to_host(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width, size_t rows,
                         hipStream_t s) {
  if (rows == 0 || width == 0) return;
  if (dpitch == spitch && width == spitch) {
    PXG_HIP(hipMemcpyAsync(dst, src, rows * width, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    return;
  }
  std::vector<unsigned char> tmp(rows * spitch);
  PXG_HIP(hipMemcpyAsync(tmp.data(), src, rows * spitch, hipMemcpyDeviceToHost, s));
  PXG_HIP(hipStreamSynchronize(s));
  for (size_t r = 0; r < rows; ++r) std::memcpy((unsigned char*)dst + r * dpitch, tmp.data() + r * spitch, width);
}

// LIFO slot allocator: id.rs:137-229 (most recently released slot first).
struct SlotAllocator {
  uint32_t next = 0;
  std::vector<uint32_t> free;
  uint32_t allocate() {
    if (!free.empty()) {
      uint32_t s = free.back();
      free.pop_back();
      return s;
    }
    if (next == UINT32_MAX)
      capacity_error("slot allocator", UINT32_MAX, "capacity exceeded: slot allocator limit is 4294967295");
    return next++;
  }
  void release(uint32_t s) { free.push_back(s); }
  size_t high_water() const { return next; }
  void clear() { next = 0; free.clear(); }
};

// Pinned host words a search reads its device flags and counts back into.
constexpr int TAIL_WORDS = 128;

// Per-call execution context: a stream plus scratch memory. Searches on one
// handle may run concurrently from many host threads; each takes its own
// context from the pool, so no two calls share a stream or scratch.
struct Ctx {
  hipStream_t stream = nullptr;
  std::unordered_map<int, DevBuf<unsigned char>> scratch;  // keyed by purpose
  std::vector<unsigned char> host;                         // pinned-free host staging
  unsigned long long* pinned = nullptr;                    // 64 pinned host bytes for a search's flags
  unsigned char* stage = nullptr;                          // pinned host staging for a search's results
  size_t stage_n = 0;
  unsigned char* get(int key, size_t bytes) {
    auto& b = scratch[key];
    if (b.n < bytes) b.alloc(bytes + bytes / 8 + 256);
    return b.p;
  }
  // TAIL_WORDS pinned host words: a search copies its device flags and
  // counts here, so the copy is one direct DMA rather than a staged copy
  // into pageable memory.
  unsigned long long* tail_host() {
    if (!pinned) PXG_HIP(hipHostMalloc((void**)&pinned, TAIL_WORDS * 8, hipHostMallocDefault));
    return pinned;
  }
  // Pinned host bytes a host-pointer search copies its results into (one
  // direct DMA per array instead of staged copies into pageable memory);
  // grown on demand, only between calls (no copy is in flight then).
  unsigned char* host_stage(size_t bytes) {
    if (stage_n < bytes) {
      if (stage) PXG_HIP(hipHostFree(stage));
      stage = nullptr;
      stage_n = 0;
      const size_t n = bytes + bytes / 8 + 256;
      PXG_HIP(hipHostMalloc((void**)&stage, n, hipHostMallocDefault));
      stage_n = n;
    }
    return stage;
  }
  ~Ctx() {
    scratch.clear();
    if (pinned) (void)hipHostFree(pinned);
    if (stage) (void)hipHostFree(stage);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

// A search's results, from device rows of `sp` entries (the first `n` used)
// to the caller's host rows of `k`: nq rows of ids and of distances, and nq
// counts. They come through the context's pinned staging with one wait when
// they fit in 64 MiB, else through staged copies. `check` runs after the
// wait and before anything reaches the caller's arrays (it may raise).
template <class F>
inline void results_to_host(Ctx& c, hipStream_t s, uint64_t nq, uint64_t k, uint64_t n, uint64_t sp,
                            const uint64_t* d_oid, const float* d_od, const uint32_t* d_oc, uint64_t* out_ids,
                            float* out_dist, uint32_t* out_count, F check) {
  const size_t bi = (size_t)nq * sp * 8, bd = (size_t)nq * sp * 4, bc = (size_t)nq * 4;
  if (bi + bd + bc <= ((size_t)64 << 20)) {
    unsigned char* st = c.host_stage(bi + bd + bc);
    if (n) {
      PXG_HIP(hipMemcpyAsync(st, d_oid, bi, hipMemcpyDeviceToHost, s));
      PXG_HIP(hipMemcpyAsync(st + bi, d_od, bd, hipMemcpyDeviceToHost, s));
    }
    PXG_HIP(hipMemcpyAsync(st + bi + bd, d_oc, bc, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    check();
    if (n)
      for (uint64_t i = 0; i < nq; ++i) {
        std::memcpy(out_ids + i * k, st + i * sp * 8, n * 8);
        std::memcpy(out_dist + i * k, st + bi + i * sp * 4, n * 4);
      }
    std::memcpy(out_count, st + bi + bd, bc);
  } else {
    PXG_HIP(hipStreamSynchronize(s));
    check();
    if (n) {
      rows_to_host(out_ids, k * 8, d_oid, sp * 8, n * 8, nq, s);
      rows_to_host(out_dist, k * 4, d_od, sp * 4, n * 4, nq, s);
    }
    PXG_HIP(hipMemcpyAsync(out_count, d_oc, bc, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
  }
}

// Device scratch of one search, by purpose, plus host words for the flag
// readback at its end. A Ctx allocates on demand; an Arena hands out regions
// of a fixed block and never allocates.
struct Scratch {
  virtual ~Scratch() = default;
  virtual unsigned char* get(int key, size_t bytes) = 0;
  // bytes an arena can still hand out (an allocating scratch has no limit)
  virtual size_t room() const { return SIZE_MAX; }
  // an arena takes back the region of `key` and everything carved after it
  virtual void release_from(int key) { (void)key; }
  virtual unsigned long long* host_words() = 0;  // TAIL_WORDS words
  virtual bool timing() const { return true; }   // stage timers may create events
};

struct CtxScratch : Scratch {
  Ctx* c;
  explicit CtxScratch(Ctx* ctx) : c(ctx) {}
  unsigned char* get(int key, size_t bytes) override { return c->get(key, bytes); }
  unsigned long long* host_words() override { return c->tail_host(); }
};

struct Arena : Scratch {
  static constexpr int KEYS = 64;
  unsigned char* base;
  size_t cap, off = 0;
  size_t start[KEYS];
  unsigned long long words[TAIL_WORDS] = {};
  Arena(void* p, size_t bytes) : base((unsigned char*)p), cap(bytes) {
    for (size_t& x : start) x = SIZE_MAX;
  }
  unsigned char* get(int key, size_t bytes) override {
    const size_t at = (off + 255) & ~(size_t)255;
    if (key < 0 || key >= KEYS || at > cap || bytes > cap - at)
      capacity_error("no-allocation scratch", cap,
                     "this search needs more than the " + std::to_string(cap >> 20) +
                         " MiB of the no-allocation scratch (region " + std::to_string(key) + " of " +
                         std::to_string(bytes) + " bytes at offset " + std::to_string(at) + ")");
    start[key] = at;
    off = at + bytes;
    return base + at;
  }
  size_t room() const override {
    const size_t at = (off + 255) & ~(size_t)255;
    return at >= cap ? 0 : cap - at;
  }
  void release_from(int key) override {
    if (key >= 0 && key < KEYS && start[key] != SIZE_MAX) off = start[key];
  }
  unsigned long long* host_words() override { return words; }
  bool timing() const override { return false; }
};

struct CtxPool {
  std::mutex mu;
  std::vector<Ctx*> idle;
  std::vector<Ctx*> all;
  Ctx* acquire() {
    std::lock_guard<std::mutex> lk(mu);
    if (!idle.empty()) {
      Ctx* c = idle.back();
      idle.pop_back();
      return c;
    }
    Ctx* c = new Ctx();
    PXG_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    all.push_back(c);
    return c;
  }
  void release(Ctx* c) {
    std::lock_guard<std::mutex> lk(mu);
    idle.push_back(c);
  }
  ~CtxPool() {
    for (Ctx* c : all) delete c;
  }
};

struct CtxLease {
  CtxPool& pool;
  Ctx* c;
  explicit CtxLease(CtxPool& p) : pool(p), c(p.acquire()) {}
  ~CtxLease() { pool.release(c); }
  Ctx* operator->() { return c; }
};

// A search that fails part-way (a capacity error in a later scratch region,
// a non-finite query found at the flag readback) may already have kernels
// queued that read its scratch and write the caller's outputs. Declared after
// the scratch's owner (a CtxLease, or the lock of the fixed no-allocation
// block), this waits for that work as the error unwinds, so no kernel still
// touches the scratch once another call may take it, and none writes the
// outputs after the call has returned.
struct DrainOnUnwind {
  hipStream_t s;
  ~DrainOnUnwind() {
    if (std::uncaught_exceptions() > 0) (void)hipStreamSynchronize(s);
  }
};

// VectorSpace::validate / prepare on the host (space.rs:104-138). Returns -1
// or the index of the first non-finite component. Cosine normalisation is the
// reference's: n = sqrt(8-lane dot(v, v)); if n > 0 and finite, v *= 1/n.
long long validate_prepare(int metric, const float* in, uint32_t dim, float* out);
float host_dot_unrolled(const float* a, const float* b, uint32_t n);

void check_k(uint64_t k);  // index.rs:212-224

// Stage timings (pxg_set_profiling / pxg_last_timings). A Timer records
// hipEvents on one stream; read() runs after the stream has synchronised.
bool profiling_enabled();
void set_last_timings(const pxg_timings& t);

struct Timer {
  bool on;
  hipStream_t s;
  hipEvent_t ev[8] = {};
  int n = 0;
  int stage_of[8] = {};
  Timer(hipStream_t stream) : on(profiling_enabled()), s(stream) {}
  // mark the start of `stage` (0 prep, 1 candidates, 2 merge, 3 fallback, 4 end)
  void mark(int stage) {
    if (!on || n >= 8) return;
    if (hipEventCreate(&ev[n]) != hipSuccess) { on = false; return; }
    (void)hipEventRecord(ev[n], s);
    stage_of[n++] = stage;
  }
  void finish() {
    if (!on) return;
    mark(4);
    (void)hipEventSynchronize(ev[n - 1]);
    pxg_timings t{0, 0, 0, 0, 0};
    float* slot[4] = {&t.prep_ms, &t.candidates_ms, &t.merge_ms, &t.fallback_ms};
    for (int i = 0; i + 1 < n; ++i) {
      float ms = 0;
      (void)hipEventElapsedTime(&ms, ev[i], ev[i + 1]);
      if (stage_of[i] < 4) *slot[stage_of[i]] += ms;
    }
    (void)hipEventElapsedTime(&t.total_ms, ev[0], ev[n - 1]);
    set_last_timings(t);
  }
  ~Timer() {
    for (int i = 0; i < n; ++i) (void)hipEventDestroy(ev[i]);
  }
};

}  // namespace pxg
