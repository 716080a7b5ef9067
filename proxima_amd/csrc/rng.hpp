// The seeded generator the reference's trainers use: rand_chacha 0.3.1
// ChaCha8Rng (8 rounds, 64-bit block counter from 0, stream 0, a 64-word
// buffer refilled four blocks at a time), rand_core 0.6.4 seed_from_u64 (PCG32
// expansion into the 32-byte key), and the rand 0.8 samplers used at the call
// sites kmeans.rs:150,167-169 (usize gen_range: widening multiply with zone
// rejection; f64 gen_range: 52 random bits as [1,2) - 1, scaled, rejected if
// >= high). Restated from those crates' published algorithms. The state is
// plain data: the host seeds it, a device kernel can continue the stream from
// a copy in device memory, and the host picks it up again afterwards.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace pxg {

struct ChaCha8 {
  uint32_t key[8];
  uint64_t counter = 0;
  uint32_t buf[64];
  int index = 64;

  __host__ __device__ static inline uint32_t rotl(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

  __host__ __device__ static void block(const uint32_t k[8], uint64_t ctr, uint32_t out[16]) {
    const uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u, k[0], k[1], k[2], k[3],
                            k[4],        k[5],        k[6],        k[7],        (uint32_t)ctr, (uint32_t)(ctr >> 32),
                            0,           0};
    uint32_t x[16];
    for (int i = 0; i < 16; ++i) x[i] = s[i];
    auto qr = [&](int a, int b, int c, int d) {
      x[a] += x[b]; x[d] = rotl(x[d] ^ x[a], 16);
      x[c] += x[d]; x[b] = rotl(x[b] ^ x[c], 12);
      x[a] += x[b]; x[d] = rotl(x[d] ^ x[a], 8);
      x[c] += x[d]; x[b] = rotl(x[b] ^ x[c], 7);
    };
    for (int r = 0; r < 8; r += 2) {
      qr(0, 4, 8, 12); qr(1, 5, 9, 13); qr(2, 6, 10, 14); qr(3, 7, 11, 15);
      qr(0, 5, 10, 15); qr(1, 6, 11, 12); qr(2, 7, 8, 13); qr(3, 4, 9, 14);
    }
    for (int i = 0; i < 16; ++i) out[i] = x[i] + s[i];
  }

  ChaCha8() = default;
  __host__ __device__ explicit ChaCha8(uint64_t seed) {
    const uint64_t MUL = 6364136223846793005ull, INC = 11634580027462260723ull;
    uint64_t st = seed;
    for (int i = 0; i < 8; ++i) {
      st = st * MUL + INC;
      const uint32_t xs = (uint32_t)(((st >> 18) ^ st) >> 27);
      const uint32_t rot = (uint32_t)(st >> 59);
      key[i] = (xs >> rot) | (xs << ((32 - rot) & 31));
    }
  }

  __host__ __device__ void refill() {
    for (int b = 0; b < 4; ++b) block(key, counter + b, buf + 16 * b);
    counter += 4;
    index = 0;
  }
  __host__ __device__ uint32_t next_u32() {
    if (index >= 64) refill();
    return buf[index++];
  }
  __host__ __device__ uint64_t next_u64() {
    if (index < 63) {
      const uint64_t lo = buf[index], hi = buf[index + 1];
      index += 2;
      return (hi << 32) | lo;
    }
    if (index >= 64) {
      refill();
      index = 2;
      return ((uint64_t)buf[1] << 32) | buf[0];
    }
    const uint64_t lo = buf[63];
    refill();
    index = 1;
    return ((uint64_t)buf[0] << 32) | lo;
  }
  // high and low 64 bits of a * b
  __host__ __device__ static void mul_wide(uint64_t a, uint64_t b, uint64_t& hi, uint64_t& lo) {
    const uint64_t a0 = (uint32_t)a, a1 = a >> 32, b0 = (uint32_t)b, b1 = b >> 32;
    const uint64_t p00 = a0 * b0, p01 = a0 * b1, p10 = a1 * b0, p11 = a1 * b1;
    const uint64_t mid = (p00 >> 32) + (uint32_t)p01 + (uint32_t)p10;
    lo = (mid << 32) | (uint32_t)p00;
    hi = p11 + (p01 >> 32) + (p10 >> 32) + (mid >> 32);
  }
  __host__ __device__ uint64_t gen_range_usize(uint64_t n) {  // 0..n
    const uint64_t zone = (n << __builtin_clzll(n)) - 1;
    for (;;) {
      const uint64_t v = next_u64();
      uint64_t hi, lo;
      mul_wide(v, n, hi, lo);
      if (lo <= zone) return hi;
    }
  }
  __host__ __device__ double gen_range_f64(double low, double high) {
    const double scale = high - low;
    for (;;) {
      const uint64_t bits = (next_u64() >> 12) | (uint64_t(1023) << 52);
      const double v = __builtin_bit_cast(double, bits);
      const double res = (v - 1.0) * scale + low;
      if (res < high) return res;
    }
  }
};

}  // namespace pxg
