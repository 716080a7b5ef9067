// Error plumbing and host-side preparation shared by every index.
#include <atomic>
#include <cmath>

#include "common.hpp"

namespace pxg {

namespace {
thread_local Error g_last{PXG_OK, ""};
}

std::atomic<int> g_profiling{0};
thread_local pxg_timings g_timings{0, 0, 0, 0, 0};
bool profiling_enabled() { return g_profiling.load(std::memory_order_relaxed) != 0; }
void set_last_timings(const pxg_timings& t) { g_timings = t; }

void set_last_error(const Error& e) { g_last = e; }
void clear_last_error() { g_last = Error{PXG_OK, ""}; }

// dot_unrolled (distance.rs:317-331) on the host, for the cosine prepare step.
float host_dot_unrolled(const float* a, const float* b, uint32_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  uint32_t chunks = n / 8;
  for (uint32_t c = 0; c < chunks; ++c)
    for (uint32_t j = 0; j < 8; ++j) acc[j] += a[c * 8 + j] * b[c * 8 + j];
  float tail = 0.0f;
  for (uint32_t i = chunks * 8; i < n; ++i) tail += a[i] * b[i];
  return (((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]))) + tail;
}

// VectorSpace::validate + prepare (space.rs:104-138; normalize_in_place
// distance.rs:508-517: multiply by the reciprocal of the norm).
long long validate_prepare(int metric, const float* in, uint32_t dim, float* out) {
  for (uint32_t i = 0; i < dim; ++i)
    if (!std::isfinite(in[i])) return (long long)i;
  if (out != in) std::memcpy(out, in, dim * sizeof(float));
  if (metric == PXG_COSINE) {
    float n = std::sqrt(host_dot_unrolled(out, out, dim));
    if (n > 0.0f && std::isfinite(n)) {
      float inv = 1.0f / n;
      for (uint32_t i = 0; i < dim; ++i) out[i] *= inv;
    }
  }
  return -1;
}

// check_k: index.rs:212-224 (k above 2^24 is a configuration error).
void check_k(uint64_t k) {
  if (k > (1ull << 24)) config_error("k", k, "exceeds the 16777216 result ceiling");
}

}  // namespace pxg

extern "C" {

const char* pxg_last_error_message(void) { return pxg::g_last.message.c_str(); }

int pxg_last_error_detail(uint64_t* a, uint64_t* b, float* value) {
  if (a) *a = pxg::g_last.a;
  if (b) *b = pxg::g_last.b;
  if (value) *value = pxg::g_last.value;
  return pxg::g_last.status;
}

const char* pxg_last_error_parameter(void) { return pxg::g_last.parameter; }

const char* pxg_last_error_reason(void) { return pxg::g_last.reason; }

const char* pxg_version(void) { return "proxima-hip 0.1.0 (gfx950)"; }

void pxg_set_profiling(int enabled) { pxg::g_profiling.store(enabled ? 1 : 0); }

int pxg_last_timings(pxg_timings* out) {
  if (out) *out = pxg::g_timings;
  return PXG_OK;
}

int pxg_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

}  // extern "C"
