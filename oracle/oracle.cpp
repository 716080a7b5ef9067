// Oracle: a CPU restatement of the reference's nearest-neighbour hot path.
//
// TEST INFRASTRUCTURE ONLY. Nothing in the shipped library (proxima_amd/)
// links, loads or calls this file. Only tests/, __graft_entry__.smoke() and
// the CPU-baseline leg of bench.py use it, and only as the checker.
//
// Every function restates one piece of the Rust reference (Liona-orph/proxima)
// from its source text, keeping its exact arithmetic: IEEE binary32/binary64
// round-to-nearest, no FMA contraction (build with -ffp-contract=off), the
// same summation orders, the same strict/non-strict comparisons and the same
// tie rules. Citations are file:line into the reference tree.
//
// Parity pinning (what checks each part; see tests/test_oracle_*.py):
//   distance kernels   KATs of distance.rs:551-614, the lane-order overflow
//                      KAT metric_properties.rs:307-333, brute float64 bounds
//   normalise/prepare  space.rs:41-42 doc test, flat.rs:329-340
//   TopK               topk.rs:216-296, flat.rs:294-308, flat.rs:343-355
//   flat search        brute-force sort on tiny inputs + flat.rs tests
//   scalar quantizer   scalar.rs:366-451 tests, properties.rs:108-114
//   PQ table / ADC     ADC == |q - decode(code)|^2 identity (product.rs:681-706),
//                      uneven split (product.rs:667-678)
//   k-means            kmeans.rs:271-336 tests; Lloyd closed form on 1-D data
//   ChaCha core        RFC 8439 / RFC 7539 A.1 keystream at 20 rounds
//   ChaCha8 stream, rand 0.8 samplers, seed_from_u64, fixture bytes:
//                      parity unpinned vs the Rust crates (no reference test
//                      pins their values; only same-seed-same-output).
#include <cmath>
#include <cstdint>
#include <cstring>
#include <cstdlib>
#include <algorithm>
#include <vector>
#include <thread>
#include <unordered_map>
#include <limits>

namespace {

constexpr size_t LANES = 8;  // distance.rs:72

// NaN results. Rust, like IEEE 754, leaves the sign of a NaN produced by
// arithmetic to the hardware. On the reference's benchmark platform, aarch64
// (BENCHMARKS.md:13-21; FPCR.DN clear), an invalid operation such as
// inf + (-inf) or inf * 0 yields the default NaN 0x7FC00000 (sign clear), and
// an operation with one NaN operand returns that NaN. Inputs are finite
// (space.rs:104-128), so every NaN inside a sum is that default NaN and only a
// later negation (inner_product, the IP ADC, the SQ inner product) flips its
// sign, which decides where total_cmp ranks it (topk.rs:63-67). x86 yields
// 0xFFC00000 instead, so the oracle maps a NaN result to 0x7FC00000 before any
// negation.
inline float arm_nan(float x) { return std::isnan(x) ? std::numeric_limits<float>::quiet_NaN() : x; }
// a + b where both may be NaN: aarch64 FADD returns its first NaN operand,
// else the default NaN for inf + (-inf).
inline float arm_add(float a, float b) {
  if (std::isnan(a)) return a;
  if (std::isnan(b)) return b;
  return arm_nan(a + b);
}

// reduce(): distance.rs:534-538. Pairwise over the eight lane accumulators.
inline float reduce8(const float acc[LANES]) {
  float a = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  float b = (acc[4] + acc[5]) + (acc[6] + acc[7]);
  return a + b;
}

// squared_euclidean_unrolled: distance.rs:267-283.
float sq_l2_unrolled(const float* a, const float* b, size_t n) {
  float acc[LANES] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t chunks = n / LANES;
  for (size_t c = 0; c < chunks; ++c) {
    for (size_t j = 0; j < LANES; ++j) {
      float d = a[c * LANES + j] - b[c * LANES + j];
      acc[j] += d * d;
    }
  }
  float tail = 0.0f;
  for (size_t i = chunks * LANES; i < n; ++i) {
    float d = a[i] - b[i];
    tail += d * d;
  }
  return reduce8(acc) + tail;
}

// squared_euclidean_scalar: distance.rs:251-258.
float sq_l2_scalar(const float* a, const float* b, size_t n) {
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    float d = a[i] - b[i];
    sum += d * d;
  }
  return sum;
}

// dot_unrolled: distance.rs:317-331.
float dot_unrolled(const float* a, const float* b, size_t n) {
  float acc[LANES] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t chunks = n / LANES;
  for (size_t c = 0; c < chunks; ++c)
    for (size_t j = 0; j < LANES; ++j) acc[j] += a[c * LANES + j] * b[c * LANES + j];
  float tail = 0.0f;
  for (size_t i = chunks * LANES; i < n; ++i) tail += a[i] * b[i];
  return arm_nan(reduce8(acc) + tail);
}

// dot_scalar: distance.rs:307-313.
float dot_scalar(const float* a, const float* b, size_t n) {
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) sum += a[i] * b[i];
  return arm_nan(sum);
}

// manhattan_unrolled: distance.rs:358-372; scalar 345-351.
float l1_unrolled(const float* a, const float* b, size_t n) {
  float acc[LANES] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t chunks = n / LANES;
  for (size_t c = 0; c < chunks; ++c)
    for (size_t j = 0; j < LANES; ++j) acc[j] += std::fabs(a[c * LANES + j] - b[c * LANES + j]);
  float tail = 0.0f;
  for (size_t i = chunks * LANES; i < n; ++i) tail += std::fabs(a[i] - b[i]);
  return reduce8(acc) + tail;
}
float l1_scalar(const float* a, const float* b, size_t n) {
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) sum += std::fabs(a[i] - b[i]);
  return sum;
}

// cosine_unrolled + cosine_terms_unrolled: distance.rs:424-471.
float cosine_unrolled(const float* a, const float* b, size_t n) {
  float ad[LANES] = {0}, aa[LANES] = {0}, ab[LANES] = {0};
  size_t chunks = n / LANES;
  for (size_t c = 0; c < chunks; ++c)
    for (size_t j = 0; j < LANES; ++j) {
      float x = a[c * LANES + j], y = b[c * LANES + j];
      ad[j] += x * y;
      aa[j] += x * x;
      ab[j] += y * y;
    }
  float d = 0, na = 0, nb = 0;
  for (size_t i = chunks * LANES; i < n; ++i) {
    d += a[i] * b[i];
    na += a[i] * a[i];
    nb += b[i] * b[i];
  }
  float dot = reduce8(ad) + d, norm_a = reduce8(aa) + na, norm_b = reduce8(ab) + nb;
  float denom = std::sqrt(norm_a * norm_b);
  if (denom <= 0.0f) return 1.0f;
  return arm_nan(1.0f - dot / denom);
}

// cosine_scalar: distance.rs:406-421.
float cosine_scalar(const float* a, const float* b, size_t n) {
  float dot = 0, na = 0, nb = 0;
  for (size_t i = 0; i < n; ++i) {
    dot += a[i] * b[i];
    na += a[i] * a[i];
    nb += b[i] * b[i];
  }
  float denom = std::sqrt(na * nb);
  if (denom <= 0.0f) return 1.0f;
  return arm_nan(1.0f - dot / denom);
}

enum Metric { EUCLIDEAN = 0, COSINE = 1, INNER_PRODUCT = 2, MANHATTAN = 3 };  // distance.rs:90-118

// VectorSpace::distance on prepared operands: space.rs:148-156.
float space_distance(int metric, const float* a, const float* b, size_t n) {
  switch (metric) {
    case EUCLIDEAN: return sq_l2_unrolled(a, b, n);
    case COSINE: return arm_nan(1.0f - dot_unrolled(a, b, n));  // cosine_normalized distance.rs:400-402
    case INNER_PRODUCT: return -dot_unrolled(a, b, n);        // inner_product distance.rs:291-293
    default: return l1_unrolled(a, b, n);
  }
}

// normalize_in_place: distance.rs:508-517 (multiply by the reciprocal).
float normalize_in_place(float* v, size_t n) {
  float nrm = std::sqrt(dot_unrolled(v, v, n));
  if (nrm > 0.0f && std::isfinite(nrm)) {
    float inv = 1.0f / nrm;
    for (size_t i = 0; i < n; ++i) v[i] *= inv;
  }
  return nrm;
}

// f32::total_cmp key: topk.rs:63-67 orders by this, then by id.
inline uint32_t total_key(float f) {
  uint32_t b;
  std::memcpy(&b, &f, 4);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

struct Hit {
  uint64_t id;
  float d;
};
// SearchResult::cmp: topk.rs:63-67.
inline bool hit_less(const Hit& a, const Hit& b) {
  uint32_t ka = total_key(a.d), kb = total_key(b.d);
  if (ka != kb) return ka < kb;
  return a.id < b.id;
}

// Bounded max-heap of the k best: topk.rs:93-199. push keeps a candidate when
// the heap is under-full, else only when it is strictly below the current
// worst under the (total_cmp, id) order.
struct TopK {
  size_t k;
  std::vector<Hit> heap;
  explicit TopK(size_t k_) : k(k_) { heap.reserve(k_ + 1); }
  static bool heap_cmp(const Hit& a, const Hit& b) { return hit_less(a, b); }  // max-heap by order
  bool push(uint64_t id, float d) {
    if (k == 0) return false;
    Hit c{id, d};
    if (heap.size() < k) {
      heap.push_back(c);
      std::push_heap(heap.begin(), heap.end(), heap_cmp);
      return true;
    }
    if (hit_less(c, heap.front())) {
      std::pop_heap(heap.begin(), heap.end(), heap_cmp);
      heap.back() = c;
      std::push_heap(heap.begin(), heap.end(), heap_cmp);
      return true;
    }
    return false;
  }
  // into_sorted_vec: ascending, topk.rs:189-191.
  std::vector<Hit> sorted() const {
    std::vector<Hit> out = heap;
    std::sort(out.begin(), out.end(), hit_less);
    return out;
  }
};

size_t emit(const TopK& top, uint64_t* out_ids, float* out_d) {
  auto v = top.sorted();
  for (size_t i = 0; i < v.size(); ++i) {
    out_ids[i] = v[i].id;
    out_d[i] = v[i].d;
  }
  return v.size();
}

inline bool accepted(const uint8_t* accept, size_t slot) { return accept == nullptr || accept[slot] != 0; }

// ---------------------------------------------------------------------------
// ChaCha8 + rand 0.8 samplers (third-party: rand_chacha 0.3.1, rand 0.8.x,
// rand_core 0.6.4; pinned versions per Cargo.lock:397-421). Restated from the
// published algorithms. The ChaCha core is pinned against RFC 7539 A.1 at 20
// rounds; the 8-round stream and samplers are parity unpinned vs Rust.
// ---------------------------------------------------------------------------
inline uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

void chacha_block(const uint32_t key[8], uint64_t counter, uint64_t stream, int rounds, uint32_t out[16]) {
  uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u,
                    key[0], key[1], key[2], key[3], key[4], key[5], key[6], key[7],
                    (uint32_t)counter, (uint32_t)(counter >> 32), (uint32_t)stream, (uint32_t)(stream >> 32)};
  uint32_t x[16];
  std::memcpy(x, s, sizeof x);
#define QR(a, b, c, d)          \
  x[a] += x[b]; x[d] ^= x[a]; x[d] = rotl32(x[d], 16); \
  x[c] += x[d]; x[b] ^= x[c]; x[b] = rotl32(x[b], 12); \
  x[a] += x[b]; x[d] ^= x[a]; x[d] = rotl32(x[d], 8);  \
  x[c] += x[d]; x[b] ^= x[c]; x[b] = rotl32(x[b], 7);
  for (int r = 0; r < rounds; r += 2) {
    QR(0, 4, 8, 12) QR(1, 5, 9, 13) QR(2, 6, 10, 14) QR(3, 7, 11, 15)
    QR(0, 5, 10, 15) QR(1, 6, 11, 12) QR(2, 7, 8, 13) QR(3, 4, 9, 14)
  }
#undef QR
  for (int i = 0; i < 16; ++i) out[i] = x[i] + s[i];
}

// rand_chacha's block RNG: a 64-word buffer refilled four blocks at a time,
// counter from 0, stream 0. next_u64 follows rand_core 0.6 BlockRng::next_u64.
struct Rng {
  uint32_t key[8];
  int rounds = 8;
  uint64_t counter = 0;
  uint32_t buf[64];
  size_t index = 64;

  void refill() {
    for (int b = 0; b < 4; ++b) chacha_block(key, counter + b, 0, rounds, buf + 16 * b);
    counter += 4;
    index = 0;
  }
  uint32_t next_u32() {
    if (index >= 64) refill();
    return buf[index++];
  }
  uint64_t next_u64() {
    if (index < 63) {
      uint64_t lo = buf[index], hi = buf[index + 1];
      index += 2;
      return (hi << 32) | lo;
    }
    if (index >= 64) {
      refill();
      index = 2;
      return ((uint64_t)buf[1] << 32) | buf[0];
    }
    uint64_t lo = buf[63];
    refill();
    index = 1;
    return ((uint64_t)buf[0] << 32) | lo;
  }
  // rand 0.8 UniformInt<usize>::sample_single(0, n): widening multiply with
  // the "conservative" zone, rejecting lo > zone.
  uint64_t gen_range_usize(uint64_t n) {
    uint64_t range = n;  // high - low for low = 0
    int lz = __builtin_clzll(range);
    uint64_t zone = (range << lz) - 1;
    for (;;) {
      uint64_t v = next_u64();
      unsigned __int128 m = (unsigned __int128)v * range;
      uint64_t hi = (uint64_t)(m >> 64), lo = (uint64_t)m;
      if (lo <= zone) return hi;
    }
  }
  // rand 0.8 UniformFloat<f64>::sample_single(low, high).
  double gen_range_f64(double low, double high) {
    double scale = high - low;
    for (;;) {
      uint64_t bits = (next_u64() >> 12) | (uint64_t(1023) << 52);
      double v12;
      std::memcpy(&v12, &bits, 8);
      double v01 = v12 - 1.0;
      double res = v01 * scale + low;
      if (res < high) return res;
    }
  }
  // rand 0.8 Standard for f32: 24 high bits times 2^-24.
  float gen_f32() { return (float)(next_u32() >> 8) * (1.0f / 16777216.0f); }
};

// rand_core 0.6 SeedableRng::seed_from_u64: PCG32 expansion into the key.
void seed_from_u64(Rng& r, uint64_t state) {
  const uint64_t MUL = 6364136223846793005ull, INC = 11634580027462260723ull;
  for (int i = 0; i < 8; ++i) {
    state = state * MUL + INC;
    uint32_t xorshifted = (uint32_t)(((state >> 18) ^ state) >> 27);
    uint32_t rot = (uint32_t)(state >> 59);
    r.key[i] = (xorshifted >> rot) | (xorshifted << ((32 - rot) & 31));
  }
  r.counter = 0;
  r.index = 64;
}

// ---------------------------------------------------------------------------
// k-means: kmeans.rs:59-241
// ---------------------------------------------------------------------------
// squared(): kmeans.rs:234-241 -- sequential, NOT the unrolled kernel.
inline float km_squared(const float* a, const float* b, size_t n) { return sq_l2_scalar(a, b, n); }

// nearest(): kmeans.rs:200-212 (best=0, +inf, strict <).
inline void km_nearest(const float* p, const float* cents, size_t dim, size_t k, size_t* best_out, float* bd_out) {
  size_t best = 0;
  float bd = INFINITY;
  for (size_t c = 0; c < k; ++c) {
    float d = km_squared(p, cents + c * dim, dim);
    if (d < bd) {
      bd = d;
      best = c;
    }
  }
  *best_out = best;
  *bd_out = bd;
}

// farthest_point(): kmeans.rs:215-226 (init -1, strict >).
size_t km_farthest(const float* pts, size_t n, size_t dim, const float* cents, size_t k) {
  size_t best = 0;
  float bd = -1.0f;
  for (size_t i = 0; i < n; ++i) {
    size_t c;
    float d;
    km_nearest(pts + i * dim, cents, dim, k, &c, &d);
    if (d > bd) {
      bd = d;
      best = i;
    }
  }
  return best;
}

// The D^2 pick of one k-means++ round (kmeans.rs:167-178): the first index
// whose f64 cumulative sum of the nearest-squared distances reaches `target`,
// n-1 if none does.
size_t pp_pick(const float* ns, size_t n, double target) {
  double cum = 0.0;
  size_t index = n - 1;
  for (size_t i = 0; i < n; ++i) {
    cum += (double)ns[i];
    if (cum >= target) {
      index = i;
      break;
    }
  }
  return index;
}

// kmeans_plus_plus: kmeans.rs:146-194.
void kmeans_pp(const float* pts, size_t n, size_t dim, size_t k, Rng& rng, float* cents) {
  size_t first = rng.gen_range_usize(n);
  std::memcpy(cents, pts + first * dim, dim * sizeof(float));
  std::vector<float> ns(n);
  for (size_t i = 0; i < n; ++i) ns[i] = km_squared(pts + i * dim, cents, dim);
  for (size_t chosen = 1; chosen < k; ++chosen) {
    double total = 0.0;
    for (size_t i = 0; i < n; ++i) total += (double)ns[i];
    size_t picked;
    if (total <= 0.0) {
      picked = rng.gen_range_usize(n);
    } else {
      double target = rng.gen_range_f64(0.0, total);
      picked = pp_pick(ns.data(), n, target);
    }
    float* c = cents + chosen * dim;
    std::memcpy(c, pts + picked * dim, dim * sizeof(float));
    for (size_t i = 0; i < n; ++i) {
      float d = km_squared(pts + i * dim, c, dim);
      if (d < ns[i]) ns[i] = d;
    }
  }
}

// The Lloyd loop of kmeans(): kmeans.rs:85-136, starting from given centroids.
void lloyd(const float* pts, size_t n, size_t dim, size_t k, size_t max_iter, float* cents, uint32_t* assign,
           double* inertia_out, size_t* iters_out) {
  std::vector<uint32_t> counts(k);
  std::vector<double> sums(k * dim);
  for (size_t i = 0; i < n; ++i) assign[i] = 0;
  double inertia = 0.0;
  size_t iterations = 0;
  for (size_t it = 0; it < max_iter; ++it) {
    iterations = it + 1;
    bool changed = false;
    inertia = 0.0;
    for (size_t i = 0; i < n; ++i) {
      size_t best;
      float bd;
      km_nearest(pts + i * dim, cents, dim, k, &best, &bd);
      inertia += (double)bd;
      if (assign[i] != (uint32_t)best) {
        assign[i] = (uint32_t)best;
        changed = true;
      }
    }
    if (!changed && it > 0) break;
    std::fill(counts.begin(), counts.end(), 0u);
    std::fill(sums.begin(), sums.end(), 0.0);
    for (size_t i = 0; i < n; ++i) {
      size_t c = assign[i];
      counts[c] += 1;
      for (size_t j = 0; j < dim; ++j) sums[c * dim + j] += (double)pts[i * dim + j];
    }
    for (size_t c = 0; c < k; ++c) {
      if (counts[c] == 0) {
        size_t victim = km_farthest(pts, n, dim, cents, k);
        std::vector<float> v(pts + victim * dim, pts + (victim + 1) * dim);
        std::memcpy(cents + c * dim, v.data(), dim * sizeof(float));
        continue;
      }
      double inv = 1.0 / (double)counts[c];
      for (size_t j = 0; j < dim; ++j) cents[c * dim + j] = (float)(sums[c * dim + j] * inv);
    }
  }
  *inertia_out = inertia;
  *iters_out = iterations;
}

// kmeans(): kmeans.rs:59-143. Returns the clamped k.
size_t kmeans_full(const float* pts, size_t n, size_t dim, size_t k, size_t max_iter, Rng& rng,
                   std::vector<float>& cents, double* inertia, size_t* iters) {
  if (dim == 0) n = 0;
  k = std::max<size_t>(std::min(k, n), 1);
  cents.assign(k * dim, 0.0f);
  if (n == 0) {
    *inertia = 0.0;
    *iters = 0;
    return k;
  }
  kmeans_pp(pts, n, dim, k, rng, cents.data());
  std::vector<uint32_t> assign(n);
  lloyd(pts, n, dim, k, max_iter, cents.data(), assign.data(), inertia, iters);
  return k;
}

// ---------------------------------------------------------------------------
// Product quantizer: product.rs:198-616
// ---------------------------------------------------------------------------
struct PqLayout {
  std::vector<size_t> widths, offsets, book_offsets;
};
// Subspace widths d/M with the remainder spread over the leading subspaces:
// product.rs:226-238 (train) and 478-495 (from_parts).
PqLayout pq_layout(size_t dim, size_t m) {
  PqLayout L;
  size_t base = dim / m, rem = dim % m, cur = 0, bcur = 0;
  for (size_t s = 0; s < m; ++s) {
    size_t w = base + (s < rem ? 1 : 0);
    L.widths.push_back(w);
    L.offsets.push_back(cur);
    L.book_offsets.push_back(bcur);
    cur += w;
    bcur += w * 256;
  }
  L.offsets.push_back(cur);
  L.book_offsets.push_back(bcur);
  return L;
}

// nearest_centroid: product.rs:529-547 (sequential sum, strict <).
uint8_t pq_nearest(const PqLayout& L, const float* books, size_t s, const float* slice) {
  size_t w = L.widths[s];
  const float* book = books + L.book_offsets[s];
  size_t best = 0;
  float bd = INFINITY;
  for (size_t c = 0; c < 256; ++c) {
    float sum = 0.0f;
    for (size_t j = 0; j < w; ++j) {
      float d = slice[j] - book[c * w + j];
      sum += d * d;
    }
    if (sum < bd) {
      bd = sum;
      best = c;
    }
  }
  return (uint8_t)best;
}

// encode_into: product.rs:361-380.
void pq_encode(const PqLayout& L, const float* books, size_t m, const float* v, uint8_t* out) {
  for (size_t s = 0; s < m; ++s) out[s] = pq_nearest(L, books, s, v + L.offsets[s]);
}

// distance_table: product.rs:407-439.
void pq_table(const PqLayout& L, const float* books, size_t m, const float* q, float* squared, float* dotv) {
  for (size_t s = 0; s < m; ++s) {
    const float* slice = q + L.offsets[s];
    size_t w = L.widths[s];
    const float* book = books + L.book_offsets[s];
    for (size_t c = 0; c < 256; ++c) {
      float l2 = 0.0f, ip = 0.0f;
      for (size_t j = 0; j < w; ++j) {
        float qq = slice[j], cc = book[c * w + j];
        float d = qq - cc;
        l2 += d * d;
        ip += qq * cc;
      }
      squared[s * 256 + c] = l2;
      dotv[s * 256 + c] = arm_nan(ip);
    }
  }
}

// DistanceTable::squared_l2 / inner_product: product.rs:580-603.
inline float adc_l2(const float* squared, size_t m, const uint8_t* code) {
  float sum = 0.0f;
  for (size_t s = 0; s < m; ++s) sum += squared[s * 256 + code[s]];
  return sum;
}
inline float adc_ip(const float* dotv, size_t m, const uint8_t* code) {
  float sum = 0.0f;
  for (size_t s = 0; s < m; ++s) sum += dotv[s * 256 + code[s]];
  return -arm_nan(sum);
}

// ProductQuantizer::train: product.rs:198-296 (one RNG advanced across
// subspaces; codebook padded by repeating the last centroid).
void pq_train(const float* training, size_t n, size_t dim, size_t m, size_t max_iter, uint64_t seed,
              float* books_out, double* inertia_out, size_t* iters_out) {
  PqLayout L = pq_layout(dim, m);
  Rng rng;
  seed_from_u64(rng, seed);
  double inertia = 0.0;
  size_t iters = 0;
  std::vector<float> proj;
  for (size_t s = 0; s < m; ++s) {
    size_t w = L.widths[s], off = L.offsets[s];
    proj.resize(n * w);
    for (size_t i = 0; i < n; ++i) std::memcpy(&proj[i * w], training + i * dim + off, w * sizeof(float));
    std::vector<float> cents;
    double in;
    size_t it;
    size_t produced = kmeans_full(proj.data(), n, w, 256, max_iter, rng, cents, &in, &it);
    inertia += in;
    iters += it;
    float* book = books_out + L.book_offsets[s];
    std::memcpy(book, cents.data(), produced * w * sizeof(float));
    for (size_t c = produced; c < 256; ++c) std::memcpy(book + c * w, cents.data() + (produced - 1) * w, w * sizeof(float));
  }
  *inertia_out = inertia;
  *iters_out = iters;
}

}  // namespace

// ===========================================================================
// extern "C" surface for tests (ctypes)
// ===========================================================================
extern "C" {

float orc_squared_euclidean_unrolled(const float* a, const float* b, size_t n) { return sq_l2_unrolled(a, b, n); }
float orc_squared_euclidean_scalar(const float* a, const float* b, size_t n) { return sq_l2_scalar(a, b, n); }
float orc_dot_unrolled(const float* a, const float* b, size_t n) { return dot_unrolled(a, b, n); }
float orc_dot_scalar(const float* a, const float* b, size_t n) { return dot_scalar(a, b, n); }
float orc_manhattan_unrolled(const float* a, const float* b, size_t n) { return l1_unrolled(a, b, n); }
float orc_manhattan_scalar(const float* a, const float* b, size_t n) { return l1_scalar(a, b, n); }
float orc_cosine_unrolled(const float* a, const float* b, size_t n) { return cosine_unrolled(a, b, n); }
float orc_cosine_scalar(const float* a, const float* b, size_t n) { return cosine_scalar(a, b, n); }
float orc_space_distance(int metric, const float* a, const float* b, size_t n) { return space_distance(metric, a, b, n); }
// Metric::distance (raw operands): distance.rs:134-141.
float orc_metric_distance(int metric, const float* a, const float* b, size_t n) {
  switch (metric) {
    case EUCLIDEAN: return sq_l2_unrolled(a, b, n);
    case COSINE: return cosine_unrolled(a, b, n);
    case INNER_PRODUCT: return -dot_unrolled(a, b, n);
    default: return l1_unrolled(a, b, n);
  }
}
float orc_normalize_in_place(float* v, size_t n) { return normalize_in_place(v, n); }

// VectorSpace::validate + prepare: space.rs:104-138. Returns -1 when valid
// (out holds the prepared vector), else the index of the first non-finite.
long long orc_prepare(int metric, const float* in, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i)
    if (!std::isfinite(in[i])) return (long long)i;
  std::memcpy(out, in, n * sizeof(float));
  if (metric == COSINE) normalize_in_place(out, n);
  return -1;
}

// prepare() over n rows with `threads` host threads. Returns -1, or the
// first row holding a non-finite component.
long long orc_prepare_batch(int metric, const float* in, size_t n, size_t dim, float* out, int threads) {
  std::vector<long long> bad(std::max(threads, 1), -1);
  auto work = [&](int t, size_t a, size_t b) {
    for (size_t i = a; i < b; ++i) {
      long long r = orc_prepare(metric, in + i * dim, dim, out + i * dim);
      if (r >= 0 && bad[t] < 0) bad[t] = (long long)i;
    }
  };
  threads = std::max(threads, 1);
  std::vector<std::thread> pool;
  size_t per = (n + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    size_t a = t * per, b = std::min(n, a + per);
    if (a >= b) break;
    pool.emplace_back(work, t, a, b);
  }
  for (auto& th : pool) th.join();
  for (long long b : bad)
    if (b >= 0) return b;
  return -1;
}

// Push (ids[i], d[i]) in order through a TopK(k); write into_sorted_vec.
size_t orc_topk(const uint64_t* ids, const float* d, size_t n, size_t k, uint64_t* out_ids, float* out_d) {
  TopK top(k);
  for (size_t i = 0; i < n; ++i) top.push(ids[i], d[i]);
  return emit(top, out_ids, out_d);
}

// FlatIndex::search over a slot-major store: flat.rs:153-169 (slots in
// ascending order, free slots skipped: storage.rs:332-337; filter before
// scoring). `query` must be prepared. Batched over queries with `threads`
// host threads (results are independent of the split).
void orc_flat_search(const float* data, const uint8_t* live, const uint64_t* ids, size_t slots, size_t dim,
                     int metric, const float* queries, size_t nq, size_t k, const uint8_t* accept, int threads,
                     uint64_t* out_ids, float* out_d, uint32_t* out_count) {
  auto work = [&](size_t q0, size_t q1) {
    for (size_t q = q0; q < q1; ++q) {
      TopK top(k);
      const float* qv = queries + q * dim;
      for (size_t s = 0; s < slots; ++s) {
        if (!live[s] || !accepted(accept, s)) continue;
        top.push(ids[s], space_distance(metric, qv, data + s * dim, dim));
      }
      out_count[q] = (uint32_t)emit(top, out_ids + q * k, out_d + q * k);
    }
  };
  if (threads <= 1 || nq <= 1) {
    work(0, nq);
    return;
  }
  std::vector<std::thread> pool;
  size_t per = (nq + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    size_t a = t * per, b = std::min(nq, a + per);
    if (a >= b) break;
    pool.emplace_back(work, a, b);
  }
  for (auto& th : pool) th.join();
}

// --- scalar quantizer: scalar.rs:141-337 -----------------------------------
// train: per-dimension (groups = dim) or global (groups = 1) min/max, scale =
// (max-min)/255, inverse = scale>0 ? 1/scale : 0. Returns -1, or the
// component index of a non-finite training value.
long long orc_sq_train(const float* training, size_t n, size_t dim, int per_dim, float* mn, float* scale, float* inv) {
  size_t groups = per_dim ? dim : 1;
  for (size_t g = 0; g < groups; ++g) {
    mn[g] = INFINITY;
    scale[g] = -INFINITY;  // holds max until the end
  }
  for (size_t i = 0; i < n; ++i)
    for (size_t c = 0; c < dim; ++c) {
      float v = training[i * dim + c];
      if (!std::isfinite(v)) return (long long)c;
      size_t g = groups == 1 ? 0 : c;
      mn[g] = std::fmin(mn[g], v);
      scale[g] = std::fmax(scale[g], v);
    }
  for (size_t g = 0; g < groups; ++g) {
    float hi = scale[g];
    scale[g] = (hi - mn[g]) / 255.0f;
    inv[g] = scale[g] > 0.0f ? 1.0f / scale[g] : 0.0f;
  }
  return -1;
}

// encode_into: scalar.rs:246-268. code_type 0 = U8, 1 = I8 (level - 128).
void orc_sq_encode(const float* v, size_t dim, int per_dim, int code_type, const float* mn, const float* inv,
                   uint8_t* out) {
  for (size_t c = 0; c < dim; ++c) {
    size_t g = per_dim ? c : 0;
    float r = std::round((v[c] - mn[g]) * inv[g]);
    r = std::fmin(std::fmax(r, 0.0f), 255.0f);  // f32::clamp; NaN cannot occur (finite inputs)
    uint8_t level = (uint8_t)r;
    out[c] = code_type == 1 ? (uint8_t)(level - 128) : level;
  }
}

// encode_into over n rows, rows split across threads (each row as above).
void orc_sq_encode_rows(const float* v, size_t n, size_t dim, int per_dim, int code_type, const float* mn,
                        const float* inv, int threads, uint8_t* out) {
  auto work = [&](size_t a, size_t b) {
    for (size_t i = a; i < b; ++i) orc_sq_encode(v + i * dim, dim, per_dim, code_type, mn, inv, out + i * dim);
  };
  if (threads <= 1 || n < 2) {
    work(0, n);
    return;
  }
  std::vector<std::thread> pool;
  size_t per = (n + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    size_t a = t * per, b = std::min(n, a + per);
    if (a >= b) break;
    pool.emplace_back(work, a, b);
  }
  for (auto& th : pool) th.join();
}

// reconstruct: scalar.rs:323-327.
void orc_sq_decode(const uint8_t* code, size_t dim, int per_dim, int code_type, const float* mn, const float* scale,
                   float* out) {
  for (size_t c = 0; c < dim; ++c) {
    size_t g = per_dim ? c : 0;
    uint8_t level = code_type == 1 ? (uint8_t)(code[c] + 128) : code[c];
    out[c] = mn[g] + (float)level * scale[g];
  }
}

// asymmetric_squared_l2 / asymmetric_inner_product: scalar.rs:298-319.
float orc_sq_asym(int ip, const float* q, const uint8_t* code, size_t dim, int per_dim, int code_type, const float* mn,
                  const float* scale) {
  float sum = 0.0f;
  for (size_t c = 0; c < dim; ++c) {
    size_t g = per_dim ? c : 0;
    uint8_t level = code_type == 1 ? (uint8_t)(code[c] + 128) : code[c];
    float rec = mn[g] + (float)level * scale[g];
    if (ip) {
      sum += q[c] * rec;
    } else {
      float d = q[c] - rec;
      sum += d * d;
    }
  }
  return ip ? -arm_nan(sum) : sum;
}

// SQ8 inner-product search over I8 codes (CodeType::I8 bytes). The reference
// has no integer-domain distance (scalar.rs:298-319 is asymmetric f32); the
// defined score is -(float)(sum_i q_i * x_i) with the sum an exact int32 over
// the signed code bytes, slots filtered by `accept` (flat.rs:162-167), ties
// and order as TopK. With rescore > 0 the best max(rescore, k) by that score
// are rescored with asymmetric_inner_product (scalar.rs:313-319) of the
// prepared f32 query `qf` against the decoded code (ranges mn / scale,
// per-dimension or global), and the best k by (distance, id) are kept.
void orc_sq8_search(const int8_t* codes, const uint8_t* live, const uint64_t* ids, size_t slots, size_t dim,
                    const int8_t* qcodes, size_t nq, size_t k, const uint8_t* accept, size_t rescore, const float* qf,
                    int per_dim, const float* mn, const float* scale, int threads, uint64_t* out_ids, float* out_d,
                    uint32_t* out_count) {
  auto work = [&](size_t q0, size_t q1) {
    const size_t kk = rescore ? std::max(rescore, k) : k;
    std::unordered_map<uint64_t, size_t> slot_of;
    for (size_t q = q0; q < q1; ++q) {
      TopK top(kk);
      const int8_t* qc = qcodes + q * dim;
      for (size_t s = 0; s < slots; ++s) {
        if (!live[s] || !accepted(accept, s)) continue;
        const int8_t* xc = codes + s * dim;
        int32_t acc = 0;
        for (size_t j = 0; j < dim; ++j) acc += (int32_t)qc[j] * (int32_t)xc[j];
        top.push(ids[s], -(float)acc);
      }
      if (!rescore) {
        out_count[q] = (uint32_t)emit(top, out_ids + q * k, out_d + q * k);
        continue;
      }
      if (slot_of.empty())
        for (size_t s = 0; s < slots; ++s)
          if (live[s]) slot_of[ids[s]] = s;
      TopK fin(k);
      for (const Hit& h : top.sorted()) {
        const uint8_t* code = reinterpret_cast<const uint8_t*>(codes + slot_of[h.id] * dim);
        float sum = 0.0f;
        for (size_t c = 0; c < dim; ++c) {
          const size_t g = per_dim ? c : 0;
          const uint8_t level = (uint8_t)(code[c] + 128);
          const float rec = mn[g] + (float)level * scale[g];
          sum += qf[q * dim + c] * rec;
        }
        fin.push(h.id, -arm_nan(sum));
      }
      out_count[q] = (uint32_t)emit(fin, out_ids + q * k, out_d + q * k);
    }
  };
  if (threads <= 1 || nq <= 1) {
    work(0, nq);
    return;
  }
  std::vector<std::thread> pool;
  size_t per = (nq + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    size_t a = t * per, b = std::min(nq, a + per);
    if (a >= b) break;
    pool.emplace_back(work, a, b);
  }
  for (auto& th : pool) th.join();
}

// --- product quantizer -----------------------------------------------------
void orc_pq_layout(size_t dim, size_t m, size_t* widths, size_t* offsets) {
  PqLayout L = pq_layout(dim, m);
  for (size_t s = 0; s < m; ++s) widths[s] = L.widths[s];
  for (size_t s = 0; s <= m; ++s) offsets[s] = L.offsets[s];
}
void orc_pq_table(const float* books, size_t dim, size_t m, const float* q, float* squared, float* dotv) {
  PqLayout L = pq_layout(dim, m);
  pq_table(L, books, m, q, squared, dotv);
}
float orc_pq_adc_l2(const float* squared, size_t m, const uint8_t* code) { return adc_l2(squared, m, code); }
float orc_pq_adc_ip(const float* dotv, size_t m, const uint8_t* code) { return adc_ip(dotv, m, code); }
void orc_pq_encode(const float* books, size_t dim, size_t m, const float* v, size_t n, uint8_t* out) {
  PqLayout L = pq_layout(dim, m);
  for (size_t i = 0; i < n; ++i) pq_encode(L, books, m, v + i * dim, out + i * m);
}
// decode: product.rs:387-404.
void orc_pq_decode(const float* books, size_t dim, size_t m, const uint8_t* code, float* out) {
  PqLayout L = pq_layout(dim, m);
  for (size_t s = 0; s < m; ++s)
    std::memcpy(out + L.offsets[s], books + L.book_offsets[s] + (size_t)code[s] * L.widths[s], L.widths[s] * sizeof(float));
}
void orc_pq_train(const float* training, size_t n, size_t dim, size_t m, size_t max_iter, uint64_t seed,
                  float* books_out, double* inertia, size_t* iters) {
  pq_train(training, n, dim, m, max_iter, seed, books_out, inertia, iters);
}

// --- k-means -----------------------------------------------------------------
// Lloyd from given initial centroids (kmeans.rs:85-136); centroids updated in place.
void orc_kmeans_lloyd(const float* pts, size_t n, size_t dim, size_t k, size_t max_iter, float* cents,
                      uint32_t* assign, double* inertia, size_t* iters) {
  lloyd(pts, n, dim, k, max_iter, cents, assign, inertia, iters);
}
// kmeans_plus_plus with ChaCha8Rng::seed_from_u64(seed): kmeans.rs:146-194.
void orc_kmeans_pp(const float* pts, size_t n, size_t dim, size_t k, uint64_t seed, float* cents) {
  Rng rng;
  seed_from_u64(rng, seed);
  kmeans_pp(pts, n, dim, k, rng, cents);
}
// kmeans() with a fresh ChaCha8Rng::seed_from_u64(seed). Returns clamped k.
size_t orc_kmeans_pp_pick(const float* ns, size_t n, double target) { return pp_pick(ns, n, target); }
// kmeans() driven by a caller's generator (left advanced, as the reference's
// `&mut rng` is): the composition product.rs:247-270 repeats per subspace.
size_t orc_kmeans_rng(const float* pts, size_t n, size_t dim, size_t k, size_t max_iter, void* rng, float* cents_out,
                      double* inertia, size_t* iters) {
  std::vector<float> cents;
  size_t kk = kmeans_full(pts, n, dim, k, max_iter, *(Rng*)rng, cents, inertia, iters);
  std::memcpy(cents_out, cents.data(), cents.size() * sizeof(float));
  return kk;
}
size_t orc_kmeans(const float* pts, size_t n, size_t dim, size_t k, size_t max_iter, uint64_t seed, float* cents_out,
                  double* inertia, size_t* iters) {
  Rng rng;
  seed_from_u64(rng, seed);
  std::vector<float> cents;
  size_t kk = kmeans_full(pts, n, dim, k, max_iter, rng, cents, inertia, iters);
  std::memcpy(cents_out, cents.data(), cents.size() * sizeof(float));
  return kk;
}
// Assignment pass only (kmeans.rs:90-97): nearest centroid + its distance.
void orc_kmeans_assign(const float* pts, size_t n, size_t dim, const float* cents, size_t k, uint32_t* assign,
                       float* dist) {
  for (size_t i = 0; i < n; ++i) {
    size_t b;
    float d;
    km_nearest(pts + i * dim, cents, dim, k, &b, &d);
    assign[i] = (uint32_t)b;
    dist[i] = d;
  }
}

// The same assignment pass with the points split across host threads (each
// point's nearest() is independent, so the results are identical).
void orc_kmeans_assign_mt(const float* pts, size_t n, size_t dim, const float* cents, size_t k, uint32_t* assign,
                          float* dist, int threads) {
  if (threads < 1) threads = 1;
  std::vector<std::thread> pool;
  const size_t per = (n + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    const size_t a = t * per, b = std::min(n, a + per);
    if (a >= b) break;
    pool.emplace_back([=] { orc_kmeans_assign(pts + a * dim, b - a, dim, cents, k, assign + a, dist + a); });
  }
  for (auto& th : pool) th.join();
}

// --- RNG surface -------------------------------------------------------------
void* orc_rng_new(uint64_t seed, int rounds) {
  Rng* r = new Rng();
  seed_from_u64(*r, seed);
  r->rounds = rounds;
  return r;
}
void orc_rng_set_key(void* h, const uint32_t* key) {
  Rng* r = (Rng*)h;
  std::memcpy(r->key, key, 32);
  r->counter = 0;
  r->index = 64;
}
void orc_rng_key(void* h, uint32_t* key) { std::memcpy(key, ((Rng*)h)->key, 32); }
uint32_t orc_rng_next_u32(void* h) { return ((Rng*)h)->next_u32(); }
uint64_t orc_rng_next_u64(void* h) { return ((Rng*)h)->next_u64(); }
uint64_t orc_rng_gen_range_usize(void* h, uint64_t n) { return ((Rng*)h)->gen_range_usize(n); }
double orc_rng_gen_range_f64(void* h, double lo, double hi) { return ((Rng*)h)->gen_range_f64(lo, hi); }
float orc_rng_gen_f32(void* h) { return ((Rng*)h)->gen_f32(); }
void orc_rng_free(void* h) { delete (Rng*)h; }
void orc_chacha_block(const uint32_t* key, uint64_t counter, uint64_t stream, int rounds, uint32_t* out) {
  chacha_block(key, counter, stream, rounds, out);
}

// --- fixture: proxima-cli/src/fixture.rs:71-123 --------------------------------
// gaussian(): Box-Muller on two gen::<f32>() draws, u1 clamped to MIN_POSITIVE.
// ln/cos are the platform libm's (not Rust-defined): parity unpinned.
static float fixture_gaussian(Rng& rng) {
  float u1 = std::fmax(rng.gen_f32(), 1.17549435e-38f);
  float u2 = rng.gen_f32();
  return std::sqrt(-2.0f * std::log(u1)) * std::cos(6.28318530717958647692f * u2);
}
void orc_fixture_generate(size_t count, size_t dim, size_t clusters, size_t queries, uint64_t seed, float* vectors,
                          float* query_vectors) {
  Rng rng;
  seed_from_u64(rng, seed);
  std::vector<float> centres(clusters * dim);
  for (auto& c : centres) c = fixture_gaussian(rng) * 4.0f;
  for (size_t i = 0; i < count; ++i) {
    size_t cl = i % clusters;
    for (size_t d = 0; d < dim; ++d) vectors[i * dim + d] = centres[cl * dim + d] + fixture_gaussian(rng);
  }
  size_t stride = std::max<size_t>(count / std::max<size_t>(queries, 1), 1);
  for (size_t q = 0; q < queries; ++q) {
    size_t src = (q * stride) % count;
    for (size_t d = 0; d < dim; ++d)
      query_vectors[q * dim + d] = vectors[src * dim + d] + fixture_gaussian(rng) * 0.25f;
  }
}

// --- IVF-PQ: ivfpq.rs:735-1125 ---------------------------------------------------
// nearest_centroid: ivfpq.rs:1231-1243 (UNROLLED kernel, best=0, strict <).
static size_t ivf_nearest(const float* v, const float* cents, size_t dim, size_t count) {
  size_t best = 0;
  float bd = INFINITY;
  for (size_t l = 0; l < count; ++l) {
    float d = sq_l2_unrolled(v, cents + l * dim, dim);
    if (d < bd) {
      bd = d;
      best = l;
    }
  }
  return best;
}

// IvfPqIndex::train (ivfpq.rs:735-825) over a slot-major store with a live
// mask: stride sample of live slots (ceil(live/sample)), coarse kmeans with
// its own ChaCha8Rng(seed), residuals of the sample, PQ train with a fresh
// RNG from the same seed. Writes centroids (produced*dim) and codebooks.
// Returns `produced` (k-means clamps nlist to the sample size).
size_t orc_ivf_train(const float* vectors, const uint8_t* live, size_t slots, size_t dim, size_t nlist, size_t m,
                     size_t max_iter, size_t training_sample, uint64_t seed, float* cents_out, float* books_out,
                     double* report /* [coarse_inertia, coarse_iterations, residual_inertia, sampled] */) {
  std::vector<size_t> live_slots;
  for (size_t s = 0; s < slots; ++s)
    if (live[s]) live_slots.push_back(s);
  size_t L = live_slots.size();
  if (L == 0) return 0;
  size_t stride = std::max<size_t>((L + training_sample - 1) / training_sample, 1);
  std::vector<float> sample;
  for (size_t i = 0; i < L; i += stride)
    sample.insert(sample.end(), vectors + live_slots[i] * dim, vectors + (live_slots[i] + 1) * dim);
  size_t sampled = sample.size() / dim;
  Rng rng;
  seed_from_u64(rng, seed);
  std::vector<float> cents;
  double cin;
  size_t cit;
  size_t produced = kmeans_full(sample.data(), sampled, dim, nlist, max_iter, rng, cents, &cin, &cit);
  std::vector<float> resid(sample.size());
  for (size_t i = 0; i < sampled; ++i) {
    size_t l = ivf_nearest(&sample[i * dim], cents.data(), dim, produced);
    for (size_t j = 0; j < dim; ++j) resid[i * dim + j] = sample[i * dim + j] - cents[l * dim + j];
  }
  // ProductQuantizer::train validates every residual first (product.rs:221-223):
  // the first non-finite one is reported as (component, vector, value)
  for (size_t i = 0; i < resid.size(); ++i)
    if (!std::isfinite(resid[i])) {
      report[0] = (double)(i % dim);
      report[1] = (double)(i / dim);
      report[2] = (double)resid[i];
      return SIZE_MAX;
    }
  double rin;
  size_t rit;
  pq_train(resid.data(), sampled, dim, m, max_iter, seed, books_out, &rin, &rit);
  std::memcpy(cents_out, cents.data(), cents.size() * sizeof(float));
  report[0] = cin;
  report[1] = (double)cit;
  report[2] = rin;
  report[3] = (double)sampled;
  return produced;
}

// encode_all / encode_slot: ivfpq.rs:828-898. list_of = UINT32_MAX for free slots.
void orc_ivf_encode(const float* vectors, const uint8_t* live, size_t slots, size_t dim, const float* cents,
                    size_t produced, const float* books, size_t m, uint8_t* codes, uint32_t* list_of) {
  PqLayout L = pq_layout(dim, m);
  std::vector<float> r(dim);
  for (size_t s = 0; s < slots; ++s) {
    if (!live[s]) {
      list_of[s] = 0xFFFFFFFFu;
      std::memset(codes + s * m, 0, m);
      continue;
    }
    const float* v = vectors + s * dim;
    size_t l = ivf_nearest(v, cents, dim, produced);
    for (size_t j = 0; j < dim; ++j) r[j] = v[j] - cents[l * dim + j];
    pq_encode(L, books, m, r.data(), codes + s * m);
    list_of[s] = (uint32_t)l;
  }
}

// search_prepared: ivfpq.rs:998-1110 (+ exhaustive 1113-1125 when untrained,
// i.e. produced == 0). metric 0 = Euclidean, 1 = Cosine. `vectors` may be
// NULL (vectors dropped: no rerank). Batched over queries.
void orc_ivf_search(int metric, const float* cents, size_t produced, const float* books, size_t dim, size_t m,
                    const uint8_t* codes, const uint32_t* list_of, const uint8_t* live, const uint64_t* ids,
                    size_t slots, const float* vectors, size_t rerank, const float* queries, size_t nq, size_t k,
                    size_t nprobe, const uint8_t* accept, int threads, uint64_t* out_ids, float* out_d,
                    uint32_t* out_count) {
  PqLayout L = pq_layout(dim, m);
  // lists[l] = slots with list_of == l in ascending slot order (ivfpq.rs:891-896).
  std::vector<std::vector<uint32_t>> lists(produced);
  if (produced)
    for (size_t s = 0; s < slots; ++s)
      if (live[s] && list_of[s] != 0xFFFFFFFFu) lists[list_of[s]].push_back((uint32_t)s);
  size_t np = std::min(std::max<size_t>(nprobe, 1), std::max<size_t>(produced, 1));  // clamp, ivfpq.rs:993
  std::unordered_map<uint64_t, size_t> slot_of;  // by_id
  for (size_t s = 0; s < slots; ++s)
    if (live[s]) slot_of[ids[s]] = s;
  auto work = [&](size_t q0, size_t q1) {
    std::vector<float> sq(m * 256), dt(m * 256), resid(dim);
    std::vector<std::pair<float, size_t>> coarse(produced);
    for (size_t q = q0; q < q1; ++q) {
      const float* qv = queries + q * dim;
      uint64_t* oi = out_ids + q * k;
      float* od = out_d + q * k;
      size_t nlive = 0;
      for (size_t s = 0; s < slots; ++s) nlive += live[s];
      if (k == 0 || nlive == 0) {
        out_count[q] = 0;
        continue;
      }
      if (produced == 0) {  // exhaustive: ivfpq.rs:1113-1125
        TopK top(k);
        for (size_t s = 0; s < slots; ++s) {
          if (!live[s] || !accepted(accept, s)) continue;
          top.push(ids[s], space_distance(metric, qv, vectors + s * dim, dim));
        }
        out_count[q] = (uint32_t)emit(top, oi, od);
        continue;
      }
      for (size_t l = 0; l < produced; ++l) coarse[l] = {sq_l2_unrolled(qv, cents + l * dim, dim), l};
      std::sort(coarse.begin(), coarse.end(), [](const std::pair<float, size_t>& a, const std::pair<float, size_t>& b) {
        uint32_t ka = total_key(a.first), kb = total_key(b.first);
        if (ka != kb) return ka < kb;
        return a.second < b.second;
      });
      size_t shortlist = rerank > 0 ? std::max(rerank, k) : k;
      TopK top(shortlist);
      if (metric == COSINE) pq_table(L, books, m, qv, sq.data(), dt.data());
      for (size_t p = 0; p < np; ++p) {
        size_t l = coarse[p].second;
        const float* c = cents + l * dim;
        float qdc = 0.0f;
        if (metric != COSINE) {
          for (size_t j = 0; j < dim; ++j) resid[j] = qv[j] - c[j];
          pq_table(L, books, m, resid.data(), sq.data(), dt.data());
        } else {
          qdc = dot_unrolled(qv, c, dim);
        }
        for (uint32_t s : lists[l]) {
          if (!accepted(accept, s)) continue;
          const uint8_t* code = codes + (size_t)s * m;
          float score = metric == COSINE ? arm_add(arm_nan(1.0f - qdc), adc_ip(dt.data(), m, code))
                                         : adc_l2(sq.data(), m, code);
          top.push(ids[s], score);
        }
      }
      std::vector<Hit> cand = top.sorted();
      if (rerank == 0 || vectors == nullptr) {
        size_t n = std::min(cand.size(), k);
        for (size_t i = 0; i < n; ++i) {
          oi[i] = cand[i].id;
          od[i] = cand[i].d;
        }
        out_count[q] = (uint32_t)n;
        continue;
      }
      TopK exact(k);  // exact rescoring of the shortlist, ivfpq.rs:1098-1109
      for (auto& h : cand) {
        size_t s = slot_of.at(h.id);
        exact.push(h.id, space_distance(metric, qv, vectors + s * dim, dim));
      }
      out_count[q] = (uint32_t)emit(exact, oi, od);
    }
  };
  if (threads <= 1 || nq <= 1) {
    work(0, nq);
    return;
  }
  std::vector<std::thread> pool;
  size_t per = (nq + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    size_t a = t * per, b = std::min(nq, a + per);
    if (a >= b) break;
    pool.emplace_back(work, a, b);
  }
  for (auto& th : pool) th.join();
}

}  // extern "C"
