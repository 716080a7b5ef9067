// Scalar quantizer (crates/proxima-quantize/src/scalar.rs) and the SQ8 flat
// index on gfx950.
//
// The reference has a ScalarQuantizer but no SQ index and no integer-domain
// distance: its distance is the asymmetric f32 one (scalar.rs:298-319). The
// SQ8 index defines, for I8 codes (level - 128) of the query and of every
// stored vector, the score
//
//     distance = -(float) S,   S = sum_i q_i * x_i   (exact int32)
//
// ordered as TopK orders search results (topk.rs:63-67: distance, then id).
// Optionally the best max(rescore, k) by that score are rescored with
// asymmetric_inner_product (scalar.rs:313-319) on the prepared f32 query.
//
// Kernels
//   sq_minmax / sq_encode_rows          range training and encoding
//   sq8_mfma_scan<KB,STAGE1>            i8 x i8 -> i32 on v_mfma_i32_32x32x32_i8
//       stage 1: every SQ_SAMPLE-th row tile, per-lane maxima over usable rows
//       stage 2: every tile; a v_max3 chain and one compare per 16 scores,
//                rows scoring >= the query's threshold are appended
//   sq8_thresholds                      k-th largest stage-1 maximum per query
//   sq8_finish                          exact sort of each query's candidates
//   sq8_exact_candidates                v_dot4 exact scan (overflowed queries,
//                                       small or wide indexes)
//   sq8_rescore / sq8_emit              f32 rescoring or id/distance output
//
// Why the threshold is safe: stage-1 maxima are scores of distinct usable
// rows (each (chunk, lane half) covers its own rows), so the k-th largest of
// them is <= the k-th best score of the whole index. Every row of the true
// top k, ties at the boundary included, scores >= it and is appended; the
// candidates are then ordered exactly. A query with more than `cap`
// candidates takes the exact scan instead.
#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>
#include <mutex>
#include <shared_mutex>
#include <unordered_map>
#include <vector>

#include "common.hpp"
#include "device.hpp"
#include "rank.hpp"
#include "wide.hpp"
#include "exact_scan.hpp"

namespace pxg {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i16v __attribute__((ext_vector_type(16)));

constexpr int SQ_NW = 8;              // waves per scan workgroup
constexpr int SQ_SAMPLE = 12;         // stage 1 visits at most one row tile in 12
constexpr int SQ_MAX_CHUNKS = 1024;   // stage-1 entries per query <= 2 * this
constexpr int SQ_MAX_KB = 8;          // MFMA path: code rows up to 256 bytes
constexpr uint32_t SQ_MAX_DIM = 65536;  // |S| < 2^31
// Buffer resource word 3 for raw (untyped, stride 0) gfx9 buffer accesses.
[[maybe_unused]] constexpr int SQ_RSRC_WORD3 = 0x00020000;
constexpr int SQ_LCAP = 1024;         // per-workgroup candidate list in LDS

__host__ __device__ constexpr int sq_rows(int kb) { return kb <= 4 ? 256 : 128; }

// s_waitcnt with vmcnt <= N (expcnt and lgkmcnt left unconstrained); gfx9
// encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8.
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__host__ __device__ constexpr int sq_qt(int kb) { return kb <= 4 ? 4 : 2; }

__device__ inline uint32_t f2ord(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
static float ord2f(uint32_t u) {
  const uint32_t b = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}

// ---------------------------------------------------------------------------
// Range training (scalar.rs:141-199): per-dimension or global min / max of a
// training set, plus the first non-finite value in row-major order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void sq_minmax(const float* __restrict__ X, int ld, uint64_t n, int dim,
                                                 int per_dim, uint64_t row0, uint32_t* __restrict__ omin,
                                                 uint32_t* __restrict__ omax, unsigned long long* __restrict__ bad) {
  const uint64_t per = (n + gridDim.x - 1) / gridDim.x;
  const uint64_t r0 = (uint64_t)blockIdx.x * per, r1 = r0 + per < n ? r0 + per : n;
  if (r0 >= r1) return;
  if (per_dim) {
    for (int c = threadIdx.x; c < dim; c += blockDim.x) {
      uint32_t mn = 0xFFFFFFFFu, mx = 0u;
      for (uint64_t r = r0; r < r1; ++r) {
        const float v = X[r * ld + c];
        if (!isfinite(v)) {
          atomicMin(bad, ((unsigned long long)(row0 + r) << 32) | (unsigned)c);
          continue;
        }
        const uint32_t o = f2ord(v);
        mn = min(mn, o);
        mx = max(mx, o);
      }
      atomicMin(&omin[c], mn);
      atomicMax(&omax[c], mx);
    }
  } else {
    __shared__ uint32_t smn[256], smx[256];
    uint32_t mn = 0xFFFFFFFFu, mx = 0u;
    const uint64_t total = (r1 - r0) * (uint64_t)dim;
    for (uint64_t e = threadIdx.x; e < total; e += blockDim.x) {
      const float v = X[(r0 + e / dim) * ld + e % dim];
      if (!isfinite(v)) {
        atomicMin(bad, ((unsigned long long)(row0 + r0 + e / dim) << 32) | (unsigned)(e % dim));
        continue;
      }
      const uint32_t o = f2ord(v);
      mn = min(mn, o);
      mx = max(mx, o);
    }
    smn[threadIdx.x] = mn;
    smx[threadIdx.x] = mx;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
      if ((int)threadIdx.x < s) {
        smn[threadIdx.x] = min(smn[threadIdx.x], smn[threadIdx.x + s]);
        smx[threadIdx.x] = max(smx[threadIdx.x], smx[threadIdx.x + s]);
      }
      __syncthreads();
    }
    if (threadIdx.x == 0) {
      atomicMin(&omin[0], smn[0]);
      atomicMax(&omax[0], smx[0]);
    }
  }
}

// encode_into (scalar.rs:246-268): level = clamp(round((v - min) * inv),
// 0, 255) with round half away from zero; I8 stores level - 128. Row i of P
// (stride ld) goes to row dst[i] (or i) of `out` (stride ostride), zero padded.
__global__ __launch_bounds__(64) void sq_encode_rows(const float* __restrict__ P, int ld, int n, int dim, int per_dim,
                                                     int code_type, const float* __restrict__ mn,
                                                     const float* __restrict__ inv, const uint32_t* __restrict__ dst,
                                                     uint8_t* __restrict__ out, int ostride) {
  const int i = blockIdx.x;
  if (i >= n) return;
  uint8_t* o = out + (size_t)(dst ? dst[i] : (uint32_t)i) * ostride;
  const float* v = P + (size_t)i * ld;
  for (int c = threadIdx.x; c < ostride; c += blockDim.x) {
    uint8_t b = 0;
    if (c < dim) {
      const int g = per_dim ? c : 0;
      float r = roundf((v[c] - mn[g]) * inv[g]);
      r = fminf(fmaxf(r, 0.0f), 255.0f);
      const uint8_t level = (uint8_t)r;
      b = code_type == 1 ? (uint8_t)(level - 128u) : level;
    }
    o[c] = b;
  }
}

// reconstruct (scalar.rs:323-327) and the asymmetric distances (298-319),
// one code row per thread, components in order.
__device__ inline float sq_reconstruct(uint8_t byte, int code_type, float mn, float scale) {
  const uint8_t level = code_type == 1 ? (uint8_t)(byte + 128u) : byte;
  return mn + (float)level * scale;
}

__global__ void sq_decode_rows(const uint8_t* __restrict__ codes, uint64_t n, int dim, int per_dim, int code_type,
                               const float* __restrict__ mn, const float* __restrict__ scale, float* __restrict__ out) {
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * (uint64_t)dim) return;
  const int c = (int)(t % dim), g = per_dim ? c : 0;
  out[t] = sq_reconstruct(codes[t], code_type, mn[g], scale[g]);
}

__global__ void sq_asym_rows(int ip, const float* __restrict__ q, const uint8_t* __restrict__ codes, uint64_t n,
                             int dim, int per_dim, int code_type, const float* __restrict__ mn,
                             const float* __restrict__ scale, float* __restrict__ out) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint8_t* code = codes + i * dim;
  float sum = 0.0f;
  for (int c = 0; c < dim; ++c) {
    const int g = per_dim ? c : 0;
    const float rec = sq_reconstruct(code[c], code_type, mn[g], scale[g]);
    if (ip) {
      sum += q[c] * rec;
    } else {
      const float d = q[c] - rec;
      sum += d * d;
    }
  }
  out[i] = ip ? -arm_nan(sum) : sum;
}

// Copy caller codes (stride dim) into index rows (stride KP, zero padded).
__global__ void sq8_place_codes(const int8_t* __restrict__ src, int n, int dim, int KP,
                                const uint32_t* __restrict__ dst, int8_t* __restrict__ C) {
  const int i = blockIdx.x;
  if (i >= n) return;
  int8_t* o = C + (size_t)(dst ? dst[i] : (uint32_t)i) * KP;
  for (int c = threadIdx.x; c < KP; c += blockDim.x) o[c] = c < dim ? src[(size_t)i * dim + c] : (int8_t)0;
}

__global__ void sq8_mark(const uint32_t* __restrict__ slots, const uint64_t* __restrict__ sid, int n,
                         uint8_t* __restrict__ live, uint64_t* __restrict__ ids) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  live[slots[i]] = 1;
  ids[slots[i]] = sid[i];
}

#if defined(__HIP_DEVICE_COMPILE__)
// A raw buffer resource over [p, p + bytes), from wave-uniform values.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t sq_rsrc(const void* p, int bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)(((uint64_t)hi << 32) | lo), 0,
                                           __builtin_amdgcn_readfirstlane(bytes), SQ_RSRC_WORD3);
}

// Buffer loads straight into LDS: lane i's 16 (4) bytes land at m0 + 16 i
// (m0 + 4 i); an offset outside the resource lands as zeros. Inline asm, so
// that the compiler does not count these loads under vmcnt (it would wait
// for every one in flight before each LDS read of the tile); the scan waits
// for them itself (wait_vm_upto) before the tile barrier. The scan kernel
// has no other use of m0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void sq_dma16(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(voff), "s"(rs)
               : "memory", "m0");
}
__device__ __forceinline__ void sq_dma4(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(m0), "v"(voff), "s"(rs)
               : "memory", "m0");
}
#pragma clang diagnostic pop
#endif

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 15].
__device__ __forceinline__ void wait_vm_upto(int n) {
  switch (n) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<1>(); break;
    case 2: wait_vm<2>(); break;
    case 3: wait_vm<3>(); break;
    case 4: wait_vm<4>(); break;
    case 5: wait_vm<5>(); break;
    case 6: wait_vm<6>(); break;
    case 7: wait_vm<7>(); break;
    case 8: wait_vm<8>(); break;
    case 9: wait_vm<9>(); break;
    case 10: wait_vm<10>(); break;
    case 11: wait_vm<11>(); break;
    case 12: wait_vm<12>(); break;
    case 13: wait_vm<13>(); break;
    case 14: wait_vm<14>(); break;
    default: wait_vm<15>(); break;
  }
}

template <typename T>
__device__ __forceinline__ uint32_t lds_addr(const T* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) T*)p;
}

// ---------------------------------------------------------------------------
// Integer MFMA scan. Workgroup = SQ_NW waves, two per SIMD, each with up to
// 256 registers. Wave w holds QT tiles of 32 query codes in VGPRs (the MFMA
// B operand: lane l gives query l%32, bytes [kb*32 + 16*(l/32), +16) of K
// block kb); database rows stream through D LDS tiles of R rows (row stride
// KP+16 bytes: 16-byte reads of 16 consecutive rows hit distinct banks) and
// feed the A operand the same way. Output lane l, register v = row
// 8*(v/4) + 4*(l/32) + v%4 of the tile against query l%32, so every lane
// filters scores of one query.
//
// Every wave issues its share of the tile DMAs (buffer loads into LDS, D - 1
// tiles ahead) and waits only for its own share before the tile barrier, so
// no wave stalls on HBM inside a tile. Within a tile the row blocks are
// software-pipelined: the MFMAs of row block rt+1 are issued before the
// scores of block rt are filtered, from a second accumulator set and a
// second A operand, so the matrix core runs while the filter's VALU work and
// the next block's LDS reads proceed.
// ---------------------------------------------------------------------------
// QTT: query tiles per wave (0 = sq_qt(KB)). A smaller batch takes fewer,
// so that its queries spread over all the waves (and SIMDs) of a workgroup
// rather than a few waves multiplying code tiles of absent queries.
template <int KB, bool STAGE1, int QTT = 0>
__global__ __launch_bounds__(SQ_NW * 64) void sq8_mfma_scan(
    const int8_t* __restrict__ Qc, int nq, const int8_t* __restrict__ C, int N, const uint8_t* __restrict__ live,
    const uint8_t* __restrict__ accept, const uint32_t* __restrict__ rank, int nchunks, int qgroups,
    int tiles_per_chunk, int sample, const int* __restrict__ thr_in, int* __restrict__ tmax,
    int* __restrict__ ccount, uint64_t* __restrict__ cand, int cap) {
  constexpr int KP = KB * 32, SR = KP + 16, R = sq_rows(KB), RT = R / 32, QT = QTT > 0 ? QTT : sq_qt(KB);
  constexpr int PPR = KP / 16;         // 16-byte pieces per row
  constexpr int D = 3;                // LDS tiles: the next two tiles load during the current one
  __shared__ __align__(16) int8_t tile[D][R * SR];
  // stage 1: the tile's live and accept bytes (256 per tile; rows past the
  // tile or past N read zero)
  __shared__ __align__(16) uint8_t vlive[STAGE1 ? D : 1][256];
  __shared__ __align__(16) uint8_t vacc[STAGE1 ? D : 1][256];
  // stage 2: passing scores of recomputed tiles go to a workgroup list in
  // LDS, filtered and published after the scan
  __shared__ int lc_score[STAGE1 ? 1 : SQ_LCAP];
  __shared__ int lc_row[STAGE1 ? 1 : SQ_LCAP];
  __shared__ int lc_q[STAGE1 ? 1 : SQ_LCAP];
  __shared__ int lc_n;
  static_assert(R <= 256, "one 4-byte DMA per lane covers a tile's live bytes");

  // XCD-aware mapping: workgroup ids are dealt round-robin over the 8 XCDs;
  // consecutive logical ids (the query groups of one chunk) go to the same
  // XCD at about the same time and share its L2 copy of the chunk.
  const int total = nchunks * qgroups;
  const int per_xcd = (total + 7) / 8;
  const int lid = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (lid >= total) return;  // uniform over the workgroup, before any barrier
  const int chunk = lid / qgroups, qgroup = lid % qgroups;

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, r = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q0 = qgroup * (SQ_NW * QT * 32) + w * (QT * 32);
  const bool active = q0 < nq;

  i4v qa[QT][KB];
  int thr[QT], run[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int q = q0 + qt * 32 + r;
    const bool ok = active && q < nq;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
      qa[qt][kb] = ok ? *reinterpret_cast<const i4v*>(Qc + (size_t)q * KP + kb * 32 + h * 16) : i4v{0, 0, 0, 0};
    thr[qt] = STAGE1 ? INT_MIN : (ok ? thr_in[q] : INT_MAX);
    run[qt] = INT_MIN;
  }
  // The query loads land here, before any tile DMA: a compiler wait for them
  // inside the loop would also drain the DMAs in flight.
  wait_vm<0>();

  const int ntiles = (N + R - 1) / R;
  const int tb = chunk * tiles_per_chunk;
  const int te = min(ntiles, tb + tiles_per_chunk);
  const int step = STAGE1 ? sample : 1;
  const int t0 = STAGE1 ? (tb + sample - 1) / sample * sample : tb;
  const int niter = t0 < te ? (te - t0 + step - 1) / step : 0;

  // Tile DMA: instruction i writes 64 x 16 bytes at LDS offset 1024*i,
  // lane l to byte 16*l, i.e. the 16-byte slot 64*i + l of the padded tile
  // (PPR data slots + 1 padding slot per row). Wave w issues the
  // instructions i = w, w + SQ_NW, ...; the buffer resource is rebased on
  // each tile and covers its rows only, so rows past N and padding slots
  // (given an offset beyond the range) read zeros. Stage 1 adds one 4-byte
  // DMA each for the tile's live and accept bytes, on the last two waves
  // (the ones with the fewest tile instructions).
  constexpr int SPR = PPR + 1, NI = R * SPR / 64, NJ = (NI + SQ_NW - 1) / SQ_NW;
  static_assert(R * SPR % 64 == 0 && NI < 64, "tile must split into whole DMA instructions");
  const int nmine = w < NI % SQ_NW || NI % SQ_NW == 0 ? NJ : NJ - 1;
  const bool vdma = STAGE1 && w >= SQ_NW - 2;
  const int ndma = nmine + (vdma ? 1 : 0);  // vmcnt entries per issued tile
  uint32_t voff[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int sl = 64 * (w + j * SQ_NW) + lane, row = sl / SPR, part = sl % SPR;
    voff[j] = part < PPR ? row * KP + part * 16 : 0x7FFFFFF0u;  // padding: beyond the range, reads zeros
  }
  [[maybe_unused]] const uint8_t* vsrc = w == SQ_NW - 1 ? live : (accept ? accept : live);
  auto issue = [&](int t, int buf) __attribute__((always_inline)) {
#if defined(__HIP_DEVICE_COMPILE__)
    const int rows = min(R, N - t * R);
    const __amdgpu_buffer_rsrc_t rs = sq_rsrc(C + (size_t)t * R * KP, rows * KP);
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (j < nmine) sq_dma16(rs, voff[j], lds_addr(&tile[buf][(w + j * SQ_NW) * 1024]));
    if (vdma) {
      const __amdgpu_buffer_rsrc_t vs = sq_rsrc(vsrc + (size_t)t * R, rows);
      sq_dma4(vs, 4u * lane, lds_addr(w == SQ_NW - 1 ? &vlive[buf][0] : &vacc[buf][0]));
    }
#endif
  };

  // A operand of row block rt: lane l reads row rt*32 + l%32, bytes
  // kb*32 + 16*(l/32) .. +16 of every K block.
  auto load_a = [&](i4v(&a)[KB], const int8_t* tl, int rt) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) a[kb] = *reinterpret_cast<const i4v*>(&tl[(rt * 32 + r) * SR + kb * 32 + h * 16]);
  };
  auto mfmas = [&](i16v(&acc)[QT], const i4v(&a)[KB]) __attribute__((always_inline)) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[qt][v] = 0;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) acc[qt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[kb], qa[qt][kb], acc[qt], 0, 0, 0);
  };
  uint32_t passmask = 0;  // stage 2, bit rt*QT+qt: that 32 x 32 block has a score >= the threshold
  auto reduce = [&](const i16v(&acc)[QT], int rt, int buf) __attribute__((always_inline)) {
    if constexpr (STAGE1) {
      uint32_t vw[4];
#pragma unroll
      for (int g = 0; g < 4; ++g)
        vw[g] = *reinterpret_cast<const uint32_t*>(&vlive[buf][rt * 32 + 8 * g + 4 * h]) &
                *reinterpret_cast<const uint32_t*>(&vacc[buf][rt * 32 + 8 * g + 4 * h]);
      if (__all((vw[0] & vw[1] & vw[2] & vw[3]) == 0x01010101u)) {
        // every row of the 32 x 32 block is usable: a v_max3 chain
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const i16v x = acc[qt];
          int m = max(max(run[qt], x[0]), x[1]);
          m = max(max(m, x[2]), x[3]);
          m = max(max(m, x[4]), x[5]);
          m = max(max(m, x[6]), x[7]);
          m = max(max(m, x[8]), x[9]);
          m = max(max(m, x[10]), x[11]);
          m = max(max(m, x[12]), x[13]);
          run[qt] = max(max(m, x[14]), x[15]);
        }
      } else {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bool ok = (vw[g] >> (8 * j)) & 1u;
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) run[qt] = ok ? max(run[qt], acc[qt][4 * g + j]) : run[qt];
          }
        }
      }
    } else {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const i16v x = acc[qt];
        int m = max(max(x[0], x[1]), x[2]);  // a chain of v_max3
        m = max(max(m, x[3]), x[4]);
        m = max(max(m, x[5]), x[6]);
        m = max(max(m, x[7]), x[8]);
        m = max(max(m, x[9]), x[10]);
        m = max(max(m, x[11]), x[12]);
        m = max(max(m, x[13]), x[14]);
        m = max(m, x[15]);
        passmask |= (__ballot(m >= thr[qt]) != 0 ? 1u : 0u) << (rt * QT + qt);
      }
    }
  };

  // Tile j goes to buffer j % D, issued D - 1 iterations before it is used
  // (its buffer was last read in the iteration before the issue). Before
  // each barrier a wave waits until only its DMAs of the tile issued in
  // that iteration are outstanding, i.e. its share of the next tile landed.
  static_assert(D == 3, "the waits below keep exactly one later tile in flight");
  if (tid == 0) lc_n = 0;
  if (niter > 0) issue(t0, 0);
  if (niter > 1) issue(t0 + step, 1);
  wait_vm_upto(niter > 1 ? ndma : 0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  for (int it = 0; it < niter; ++it) {
    const int buf = it % D;
    const int t = t0 + it * step;
    const bool more = it + D - 1 < niter;
    if (more) issue(t0 + (it + D - 1) * step, (it + D - 1) % D);
    if (active) {
      const int8_t* tl = &tile[buf][0];
      passmask = 0;
      i4v a0[KB], a1[KB];
      i16v c0[QT], c1[QT];
      load_a(a0, tl, 0);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        if (rt % 2 == 0) {
          mfmas(c0, a0);
          if (rt + 1 < RT) load_a(a1, tl, rt + 1);
          if (rt > 0) reduce(c1, rt - 1, buf);
        } else {
          mfmas(c1, a1);
          if (rt + 1 < RT) load_a(a0, tl, rt + 1);
          reduce(c0, rt - 1, buf);
        }
        if constexpr (!STAGE1) {
          // the next A operand's reads first, then each MFMA followed by
          // four of the previous block's filter instructions; nothing of
          // this block's filter moves up
          __builtin_amdgcn_sched_group_barrier(0x100, KB, 0);
#pragma unroll
          for (int g = 0; g < KB * QT; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if ((RT - 1) % 2 == 0) reduce(c0, RT - 1, buf);
      else reduce(c1, RT - 1, buf);
      // Rare: some 32 x 32 blocks hold a score >= the threshold. Recompute
      // exactly those from the LDS tile (still valid until the barrier) and
      // append their passing scores to the workgroup list.
      if constexpr (!STAGE1) {
        if (passmask) {
#pragma unroll 1
          for (int rt = 0; rt < RT; ++rt) {
            const uint32_t bits = (passmask >> (rt * QT)) & ((1u << QT) - 1u);
            if (!bits) continue;
            i4v a[KB];
            load_a(a, tl, rt);
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
              if (!((bits >> qt) & 1u)) continue;
              i16v x;
#pragma unroll
              for (int v = 0; v < 16; ++v) x[v] = 0;
#pragma unroll
              for (int kb = 0; kb < KB; ++kb) x = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[kb], qa[qt][kb], x, 0, 0, 0);
              const int q = q0 + qt * 32 + r;
              const int tq = thr[qt];
              const int rowb = t * R + rt * 32 + 4 * h;
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                const int val = x[v];
                const int row = rowb + 8 * (v >> 2) + (v & 3);
                if (val >= tq && row < N && q < nq) {
                  const int pos = atomicAdd(&lc_n, 1);
                  if (pos < SQ_LCAP) {
                    lc_score[pos] = val;
                    lc_row[pos] = row;
                    lc_q[pos] = q;
                  } else if (live[row] && (accept == nullptr || accept[row])) {  // list full: publish directly
                    const int gp = atomicAdd(&ccount[q], 1);
                    if (gp < cap) cand[(size_t)q * cap + gp] = ((uint64_t)ord_key(-(float)val) << 32) | rank[row];
                  }
                }
              }
            }
          }
        }
      }
    }
    // This wave's share of the next tile has landed once only the DMAs
    // issued in this iteration remain. Tile barrier without the workgroup
    // fence of __syncthreads (that fence would drain every DMA in flight,
    // the later tile's included); the waves' LDS appends complete before it
    // (lgkmcnt(0)); tile reads were consumed by their MFMAs.
    wait_vm_upto(more ? ndma : 0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }
  if constexpr (STAGE1) {
    if (active) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const int q = q0 + qt * 32 + r;
        if (q < nq) tmax[(size_t)q * (nchunks * 2) + chunk * 2 + h] = run[qt];
      }
    }
  } else {
    // publish the workgroup's candidates (the loop's last barrier ordered
    // every append before this read)
    const int n = min(lc_n, SQ_LCAP);
    for (int i = tid; i < n; i += SQ_NW * 64) {
      const int row = lc_row[i], q = lc_q[i];
      if (live[row] && (accept == nullptr || accept[row])) {
        const int gp = atomicAdd(&ccount[q], 1);
        if (gp < cap) cand[(size_t)q * cap + gp] = ((uint64_t)ord_key(-(float)lc_score[i]) << 32) | rank[row];
      }
    }
  }
}

// Per query: the k-th largest of its E stage-1 maxima (INT_MIN when E < k).
__global__ __launch_bounds__(256) void sq8_thresholds(const int* __restrict__ tmax, int E, int k,
                                                      int* __restrict__ thr) {
  __shared__ int hist[256];
  __shared__ uint64_t sh[4];
  const int q = blockIdx.x;
  if (k > E) {
    if (threadIdx.x == 0) thr[q] = INT_MIN;
    return;
  }
  // the k-th largest maximum: the k-th smallest of INT_MAX - v (in [0, 2^32))
  const int* t = tmax + (size_t)q * E;
  auto get = [&](int i) { return (uint64_t)((int64_t)INT_MAX - (int64_t)t[i]); };
  const uint64_t v = E <= 8 * (int)blockDim.x ? block_radix_select<decltype(get), 32, 8>(get, E, k, hist, sh)
                                  : block_radix_select<decltype(get), 32>(get, E, k, hist, sh);
  if (threadIdx.x == 0) thr[q] = (int)((int64_t)INT_MAX - (int64_t)v);
}

// Per query: sort the appended candidates and keep the first kk; a query
// with more than `cap` candidates is listed for the exact scan.
__global__ __launch_bounds__(256) void sq8_finish(const int* __restrict__ ccount, const uint64_t* __restrict__ cand,
                                                  int cap, int kk, uint64_t* __restrict__ okeys,
                                                  uint32_t* __restrict__ ocount, int* __restrict__ flag_list,
                                                  int* __restrict__ flag_count) {
  extern __shared__ uint64_t sk[];
  const int q = blockIdx.x;
  const int c = ccount[q];
  if (c > cap) {
    // listed for the exact scan; no result until then
    if (threadIdx.x == 0) {
      flag_list[atomicAdd(flag_count, 1)] = q;
      ocount[q] = 0;
    }
    return;
  }
  int P = 1;
  while (P < c) P <<= 1;
  for (int i = threadIdx.x; i < P; i += blockDim.x) sk[i] = i < c ? cand[(size_t)q * cap + i] : KEY_MAX;
  __syncthreads();
  block_bitonic_sort(sk, P);
  const int kout = min(kk, c);
  for (int i = threadIdx.x; i < kout; i += blockDim.x) okeys[(size_t)q * kk + i] = sk[i];
  if (threadIdx.x == 0) ocount[q] = (uint32_t)kout;
}

// Exact scan of listed queries in EXACT_CH-row chunks (v_dot4_i32_i8 over
// the padded code rows; padding bytes are zero in both operands).
__global__ __launch_bounds__(256) void sq8_exact_candidates(const int* __restrict__ qlist,
                                                            const int* __restrict__ qcount, int nchunks,
                                                            const int8_t* __restrict__ Qc, int KP,
                                                            const int8_t* __restrict__ C, int N,
                                                            const uint8_t* __restrict__ live,
                                                            const uint8_t* __restrict__ accept,
                                                            const uint32_t* __restrict__ rank, int k,
                                                            uint64_t* __restrict__ ecand) {
  __shared__ uint64_t keys[EXACT_CH];
  const int total = (*qcount) * nchunks;
  const int kk = min(k, EXACT_CH);
  const int words = KP / 4;
  for (int w = blockIdx.x; w < total; w += gridDim.x) {
    const int f = w / nchunks, c = w % nchunks;
    const int* qv = reinterpret_cast<const int*>(Qc + (size_t)qlist[f] * KP);
    const int base = c * EXACT_CH;
    for (int s = threadIdx.x; s < EXACT_CH; s += blockDim.x) {
      const int slot = base + s;
      uint64_t key = KEY_MAX;
      if (slot < N && live[slot] && (accept == nullptr || accept[slot])) {
        const int* xv = reinterpret_cast<const int*>(C + (size_t)slot * KP);
        int acc = 0;
        for (int j = 0; j < words; ++j) acc = __builtin_amdgcn_sdot4(qv[j], xv[j], acc, false);
        key = ((uint64_t)ord_key(-(float)acc) << 32) | rank[slot];
      }
      keys[s] = key;
    }
    __syncthreads();
    block_bitonic_sort(keys, EXACT_CH);
    uint64_t* out = ecand + ((size_t)f * nchunks + c) * kk;
    for (int i = threadIdx.x; i < kk; i += blockDim.x) out[i] = keys[i];
    __syncthreads();
  }
}

// Integer-score keys (the exact int32 dot of the codes, as
// sq8_exact_candidates) of every slot for queries q0 .. q0 + G - 1: grid
// (ceil(N / 256), G), segment g at g * N.
__global__ __launch_bounds__(256) void sq8_wide_keys(const int8_t* __restrict__ Qc, int KP,
                                                     const int8_t* __restrict__ C, int N,
                                                     const uint8_t* __restrict__ live,
                                                     const uint8_t* __restrict__ accept,
                                                     const uint32_t* __restrict__ rank, int q0,
                                                     uint64_t* __restrict__ keys) {
  const int slot = blockIdx.x * blockDim.x + threadIdx.x;
  if (slot >= N) return;
  const int words = KP / 4;
  const int* qv = reinterpret_cast<const int*>(Qc + (size_t)(q0 + blockIdx.y) * KP);
  uint64_t key = KEY_MAX;
  if (live[slot] && (accept == nullptr || accept[slot])) {
    const int* xv = reinterpret_cast<const int*>(C + (size_t)slot * KP);
    int acc = 0;
    for (int j = 0; j < words; ++j) acc = __builtin_amdgcn_sdot4(qv[j], xv[j], acc, false);
    key = ((uint64_t)ord_key(-(float)acc) << 32) | rank[slot];
  }
  keys[(size_t)blockIdx.y * N + slot] = key;
}

// asymmetric_inner_product (scalar.rs:313-319) of the first min(t, len) keys
// of each sorted segment, into the same positions of `keys` (as sq8_rescore).
__global__ __launch_bounds__(256) void sq8_wide_rescore(const uint64_t* __restrict__ sorted,
                                                        const uint32_t* __restrict__ begins,
                                                        const uint32_t* __restrict__ ends, uint64_t t, int q0,
                                                        const float* __restrict__ Qp, int ld, int dim,
                                                        const int8_t* __restrict__ C, int KP, int per_dim,
                                                        const float* __restrict__ mn,
                                                        const float* __restrict__ scale,
                                                        const uint32_t* __restrict__ rank_slot,
                                                        uint64_t* __restrict__ keys) {
  const int gq = blockIdx.y;
  const uint64_t len = ends[gq] - begins[gq];
  const uint64_t take = t < len ? t : len;
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= take) return;
  const uint64_t key = sorted[begins[gq] + i];
  uint64_t nk = KEY_MAX;
  if (key != KEY_MAX) {
    const uint32_t rk = (uint32_t)key;
    const uint8_t* code = reinterpret_cast<const uint8_t*>(C + (size_t)rank_slot[rk] * KP);
    const float* qv = Qp + (size_t)(q0 + gq) * ld;
    float sum = 0.0f;
    for (int j = 0; j < dim; ++j) {
      const int g = per_dim ? j : 0;
      sum += qv[j] * sq_reconstruct(code[j], 1, mn[g], scale[g]);
    }
    nk = ((uint64_t)ord_key(-arm_nan(sum)) << 32) | rk;
  }
  keys[begins[gq] + i] = nk;
}

// Rescore a query's integer top kk with asymmetric_inner_product
// (scalar.rs:313-319) and keep the best k by (distance, id).
__global__ __launch_bounds__(256) void sq8_rescore(const uint64_t* __restrict__ okeys,
                                                   const uint32_t* __restrict__ ocount, int kk, int k,
                                                   const float* __restrict__ Qp, int ld, int dim,
                                                   const int8_t* __restrict__ C, int KP, int per_dim,
                                                   const float* __restrict__ mn, const float* __restrict__ scale,
                                                   const uint32_t* __restrict__ rank_slot,
                                                   const uint64_t* __restrict__ ids, uint64_t* __restrict__ out_ids,
                                                   float* __restrict__ out_d, uint32_t* __restrict__ out_count) {
  extern __shared__ uint64_t sk[];
  const int q = blockIdx.x;
  const int c = (int)ocount[q];
  int P = 1;
  while (P < c) P <<= 1;
  const float* qv = Qp + (size_t)q * ld;
  for (int i = threadIdx.x; i < P; i += blockDim.x) {
    uint64_t key = KEY_MAX;
    if (i < c) {
      const uint32_t rk = (uint32_t)okeys[(size_t)q * kk + i];
      const uint8_t* code = reinterpret_cast<const uint8_t*>(C + (size_t)rank_slot[rk] * KP);
      float sum = 0.0f;
      for (int j = 0; j < dim; ++j) {
        const int g = per_dim ? j : 0;
        sum += qv[j] * sq_reconstruct(code[j], 1, mn[g], scale[g]);
      }
      key = ((uint64_t)ord_key(-arm_nan(sum)) << 32) | rk;
    }
    sk[i] = key;
  }
  __syncthreads();
  block_bitonic_sort(sk, P);
  const int kout = min(k, c);
  for (int i = threadIdx.x; i < kout; i += blockDim.x) {
    const uint64_t key = sk[i];
    out_ids[(size_t)q * k + i] = ids[rank_slot[(uint32_t)key]];
    out_d[(size_t)q * k + i] = key_float((uint32_t)(key >> 32));
  }
  if (threadIdx.x == 0) out_count[q] = (uint32_t)kout;
}

__global__ void sq8_emit(const uint64_t* __restrict__ okeys, const uint32_t* __restrict__ ocount, int kk, int k,
                         const uint32_t* __restrict__ rank_slot, const uint64_t* __restrict__ ids,
                         uint64_t* __restrict__ out_ids, float* __restrict__ out_d, uint32_t* __restrict__ out_count) {
  const int q = blockIdx.x;
  const int c = min((int)ocount[q], k);
  for (int i = threadIdx.x; i < c; i += blockDim.x) {
    const uint64_t key = okeys[(size_t)q * kk + i];
    out_ids[(size_t)q * k + i] = ids[rank_slot[(uint32_t)key]];
    out_d[(size_t)q * k + i] = key_float((uint32_t)(key >> 32));
  }
  if (threadIdx.x == 0) out_count[q] = (uint32_t)c;
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
struct Ranges {
  std::vector<float> mn, scale, inv;
};

// Range training accumulator over device-resident rows (stride ld); rows may
// arrive in several batches (row0 = index of the batch's first row).
struct RangeTrainer {
  int groups;
  DevBuf<uint32_t> omin, omax;
  DevBuf<unsigned long long> bad;
  RangeTrainer(int g, hipStream_t s) : groups(g), omin(g), omax(g), bad(1) {
    PXG_HIP(hipMemsetAsync(omin.p, 0xFF, g * 4, s));
    PXG_HIP(hipMemsetAsync(omax.p, 0, g * 4, s));
    PXG_HIP(hipMemsetAsync(bad.p, 0xFF, 8, s));
  }
  void add(const float* d_x, int ld, uint64_t n, uint32_t dim, int per_dim, uint64_t row0, hipStream_t s) {
    if (!n) return;
    const unsigned grid = (unsigned)std::min<uint64_t>(1024, std::max<uint64_t>(1, n / 16));
    hipLaunchKernelGGL(sq_minmax, dim3(grid), dim3(256), 0, s, d_x, ld, n, (int)dim, per_dim, row0, omin.p, omax.p,
                       bad.p);
    PXG_HIP(hipGetLastError());
  }
  // first non-finite (row << 32 | component), or ~0
  unsigned long long first_bad(hipStream_t s) {
    unsigned long long hb = 0;
    PXG_HIP(hipMemcpyAsync(&hb, bad.p, 8, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    return hb;
  }
  // scale = (max - min) / 255, inverse = scale > 0 ? 1 / scale : 0 (scalar.rs:181-188)
  Ranges finish(hipStream_t s) {
    std::vector<uint32_t> hmn(groups), hmx(groups);
    PXG_HIP(hipMemcpyAsync(hmn.data(), omin.p, groups * 4, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipMemcpyAsync(hmx.data(), omax.p, groups * 4, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    Ranges rg;
    rg.mn.resize(groups);
    rg.scale.resize(groups);
    rg.inv.resize(groups);
    for (int g = 0; g < groups; ++g) {
      const float lo = ord2f(hmn[g]), hi = ord2f(hmx[g]);
      rg.mn[g] = lo;
      rg.scale[g] = (hi - lo) / 255.0f;
      rg.inv[g] = rg.scale[g] > 0.0f ? 1.0f / rg.scale[g] : 0.0f;
    }
    return rg;
  }
};

static void check_training_len(uint64_t n) {
  if (n == 0) config_error("training", 0, "must be a non-empty multiple of the space dimension");
}

// the first non-finite value in row-major order (scalar.rs:162-170)
static void check_finite_host(const float* x, uint64_t n, uint32_t dim) {
  for (uint64_t i = 0; i < n * dim; ++i)
    if (!std::isfinite(x[i]))
      raise(PXG_ERR_NON_FINITE,
            "vector component " + std::to_string(i % dim) + " is not finite (" + std::to_string(x[i]) + ")", i % dim,
            i / dim, x[i]);
}

// ScalarQuantizer::train over a host sample, streamed through the device.
static Ranges train_ranges_host(const float* x, uint64_t n, uint32_t dim, int per_dim, hipStream_t s) {
  check_training_len(n);
  check_finite_host(x, n, dim);
  RangeTrainer tr(per_dim ? (int)dim : 1, s);
  const uint64_t rows_per = std::max<uint64_t>(1, (64u << 20) / ((uint64_t)dim * 4));
  DevBuf<float> st(std::min<uint64_t>(rows_per, n) * dim);
  for (uint64_t a = 0; a < n; a += rows_per) {
    const uint64_t m = std::min<uint64_t>(rows_per, n - a);
    PXG_HIP(hipMemcpyAsync(st.p, x + a * dim, m * dim * 4, hipMemcpyHostToDevice, s));
    tr.add(st.p, (int)dim, m, dim, per_dim, a, s);
    PXG_HIP(hipStreamSynchronize(s));
  }
  return tr.finish(s);
}

struct Sq8Index {
  uint32_t dim = 0, ld = 0, KP = 0;
  int metric = PXG_INNER_PRODUCT;
  int per_dim = 1;
  int mode = 0;  // 0 auto, 1 MFMA candidates, 2 exact scan
  bool trained = false;
  Ranges rg;
  DevBuf<float> d_mn, d_scale, d_inv;

  std::vector<uint64_t> ids;
  std::vector<uint8_t> live;
  std::unordered_map<uint64_t, uint32_t> by_id;
  SlotAllocator slots;

  size_t cap = 0;
  DevBuf<int8_t> codes;  // cap * KP, I8 codes, zero padded
  DevBuf<uint8_t> d_live;
  DevBuf<uint64_t> d_ids;
  RankTable ranks;  // id ranks of the live slots, current after every mutation

  mutable std::shared_mutex mu;
  CtxPool pool;
  hipStream_t stream = nullptr;

  ~Sq8Index() {
    if (stream) (void)hipStreamDestroy(stream);
  }

  int groups() const { return per_dim ? (int)dim : 1; }

  void set_ranges(const Ranges& r) {
    rg = r;
    const int g = groups();
    d_mn.reserve(g);
    d_scale.reserve(g);
    d_inv.reserve(g);
    PXG_HIP(hipMemcpyAsync(d_mn.p, rg.mn.data(), g * 4, hipMemcpyHostToDevice, stream));
    PXG_HIP(hipMemcpyAsync(d_scale.p, rg.scale.data(), g * 4, hipMemcpyHostToDevice, stream));
    PXG_HIP(hipMemcpyAsync(d_inv.p, rg.inv.data(), g * 4, hipMemcpyHostToDevice, stream));
    PXG_HIP(hipStreamSynchronize(stream));
    trained = true;
  }

  // Fit the ranges to the prepared (space.rs:130-138) training vectors,
  // from host or device memory, in batches.
  void train(const float* x, bool on_device, uint64_t n) {
    check_training_len(n);
    if (!on_device) check_finite_host(x, n, dim);
    RangeTrainer tr(groups(), stream);
    const size_t chunk = std::min<size_t>(std::max<size_t>(1, (128u << 20) / ((size_t)ld * 4)), n);
    DevBuf<float> st(chunk * ld), sb(chunk), sn(chunk), raw(on_device ? 0 : chunk * dim);
    DevBuf<unsigned long long> bad(1);
    for (size_t a = 0; a < n; a += chunk) {
      const size_t m = std::min<size_t>(chunk, n - a);
      const float* src = x + a * dim;
      if (!on_device) {
        PXG_HIP(hipMemcpyAsync(raw.p, src, m * dim * 4, hipMemcpyHostToDevice, stream));
        src = raw.p;
      }
      PXG_HIP(hipMemsetAsync(bad.p, 0xFF, 8, stream));
      hipLaunchKernelGGL(flat_prep_queries, dim3((unsigned)m), dim3(64), 0, stream, src, (int)dim, (int)ld, metric, 1,
                         st.p, sb.p, sn.p, bad.p);
      PXG_HIP(hipGetLastError());
      unsigned long long bv = 0;
      PXG_HIP(hipMemcpyAsync(&bv, bad.p, 8, hipMemcpyDeviceToHost, stream));
      PXG_HIP(hipStreamSynchronize(stream));
      if (bv != ~0ull) {
        const uint64_t row = a + (bv >> 32), comp = (uint32_t)bv;
        float v = NAN;
        if (on_device) PXG_HIP(hipMemcpy(&v, x + row * dim + comp, 4, hipMemcpyDeviceToHost));
        raise(PXG_ERR_NON_FINITE, "vector component " + std::to_string(comp) + " is not finite (training vector " +
                                      std::to_string(row) + ")",
              comp, row, v);
      }
      tr.add(st.p, (int)ld, m, dim, per_dim, a, stream);
      PXG_HIP(hipStreamSynchronize(stream));
    }
    set_ranges(tr.finish(stream));
  }

  void require_trained() const {
    if (!trained)
      config_error("quantizer", 0, "the SQ8 index must be trained (or given ranges) before vectors are added");
  }

  void ensure_capacity(size_t need, size_t keep) {
    if (need <= cap) return;
    const size_t nc = std::max<size_t>(need, std::max<size_t>(cap * 2, 1024));
    const size_t hw = std::min(keep, cap);
    codes.grow(nc * KP, hw * KP, stream);
    d_live.grow(nc, hw, stream);
    d_ids.grow(nc, hw, stream);
    ranks.grow(nc, hw, stream);
    PXG_HIP(hipMemsetAsync(d_live.p + hw, 0, nc - hw, stream));
    PXG_HIP(hipMemsetAsync(codes.p + hw * KP, 0, (nc - hw) * KP, stream));
    PXG_HIP(hipStreamSynchronize(stream));
    cap = nc;
  }

  void check_new_ids(const uint64_t* in_ids, uint64_t n) {
    std::unordered_map<uint64_t, int> seen;
    for (uint64_t i = 0; i < n; ++i)
      if (by_id.count(in_ids[i]) || !seen.emplace(in_ids[i], 1).second)
        raise(PXG_ERR_DUPLICATE_ID, "duplicate vector id " + std::to_string(in_ids[i]), in_ids[i]);
    if (by_id.size() + n > (size_t)UINT32_MAX - 1)
      capacity_error("slot allocator", UINT32_MAX, "capacity exceeded: slot allocator limit is 4294967295");
  }

  std::vector<uint32_t> claim_slots(const uint64_t* in_ids, uint64_t n, uint32_t* out_slots) {
    std::vector<uint32_t> sl(n);
    const size_t old_hw = slots.high_water();
    for (uint64_t i = 0; i < n; ++i) sl[i] = slots.allocate();
    const size_t hw = slots.high_water();
    ensure_capacity(hw, old_hw);
    if (ids.size() < hw) {
      ids.resize(hw, 0);
      live.resize(hw, 0);
    }
    for (uint64_t i = 0; i < n; ++i) {
      ids[sl[i]] = in_ids[i];
      live[sl[i]] = 1;
      by_id[in_ids[i]] = sl[i];
      if (out_slots) out_slots[i] = sl[i];
    }
    return sl;
  }

  // prepare (space.rs:130-138) + validate every row of a device batch; raises
  // NonFinite before any state changes.
  void validate_device(const float* d_vecs, uint64_t n, size_t chunk, DevBuf<float>& st, DevBuf<float>& sb,
                       DevBuf<float>& sn, DevBuf<unsigned long long>& bad) {
    for (size_t a = 0; a < n; a += chunk) {
      const size_t m = std::min<size_t>(chunk, n - a);
      PXG_HIP(hipMemsetAsync(bad.p, 0xFF, 8, stream));
      hipLaunchKernelGGL(flat_prep_queries, dim3((unsigned)m), dim3(64), 0, stream, d_vecs + a * dim, (int)dim,
                         (int)ld, metric, 1, st.p, sb.p, sn.p, bad.p);
      PXG_HIP(hipGetLastError());
      unsigned long long bv = 0;
      PXG_HIP(hipMemcpyAsync(&bv, bad.p, 8, hipMemcpyDeviceToHost, stream));
      PXG_HIP(hipStreamSynchronize(stream));
      if (bv != ~0ull) {
        const uint64_t row = a + (bv >> 32), comp = (uint32_t)bv;
        raise(PXG_ERR_NON_FINITE, "vector component " + std::to_string(comp) + " is not finite (vector " +
                                      std::to_string(row) + ")",
              comp, row, NAN);
      }
    }
  }

  void insert_device(const uint64_t* in_ids, const float* d_vecs, uint64_t n, uint32_t* out_slots) {
    require_trained();
    check_new_ids(in_ids, n);
    const size_t chunk = std::min<size_t>(std::max<size_t>(1, (256u << 20) / ((size_t)ld * 4)), n);
    DevBuf<float> st(chunk * ld), sb(chunk), sn(chunk);
    DevBuf<unsigned long long> bad(1);
    validate_device(d_vecs, n, chunk, st, sb, sn, bad);
    std::vector<uint32_t> sl = claim_slots(in_ids, n, out_slots);
    DevBuf<uint32_t> st_slots(chunk);
    DevBuf<uint64_t> st_ids(chunk);
    for (size_t a = 0; a < n; a += chunk) {
      const size_t m = std::min<size_t>(chunk, n - a);
      hipLaunchKernelGGL(flat_prep_queries, dim3((unsigned)m), dim3(64), 0, stream, d_vecs + a * dim, (int)dim,
                         (int)ld, metric, 1, st.p, sb.p, sn.p, bad.p);
      PXG_HIP(hipMemcpyAsync(st_slots.p, sl.data() + a, m * 4, hipMemcpyHostToDevice, stream));
      PXG_HIP(hipMemcpyAsync(st_ids.p, in_ids + a, m * 8, hipMemcpyHostToDevice, stream));
      hipLaunchKernelGGL(sq_encode_rows, dim3((unsigned)m), dim3(64), 0, stream, st.p, (int)ld, (int)m, (int)dim,
                         per_dim, 1, d_mn.p, d_inv.p, st_slots.p, (uint8_t*)codes.p, (int)KP);
      hipLaunchKernelGGL(sq8_mark, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, stream, st_slots.p, st_ids.p,
                         (int)m, d_live.p, d_ids.p);
      PXG_HIP(hipGetLastError());
      PXG_HIP(hipStreamSynchronize(stream));
    }
    ranks.insert(in_ids, sl.data(), n, d_ids.p, stream);
  }

  void insert_host(const uint64_t* in_ids, const float* vecs, uint64_t n, uint32_t* out_slots) {
    require_trained();
    // validate on the host first: all-or-nothing (space.rs:104-121)
    for (uint64_t i = 0; i < n; ++i)
      for (uint32_t c = 0; c < dim; ++c)
        if (!std::isfinite(vecs[i * dim + c]))
          raise(PXG_ERR_NON_FINITE,
                "vector component " + std::to_string(c) + " is not finite (" + std::to_string(vecs[i * dim + c]) + ")",
                c, i, vecs[i * dim + c]);
    check_new_ids(in_ids, n);
    const size_t chunk = std::min<size_t>(std::max<size_t>(1, (64u << 20) / ((size_t)dim * 4)), n);
    DevBuf<float> raw(chunk * dim);
    // the device path re-validates (finite rows pass) and prepares
    for (size_t a = 0; a < n; a += chunk) {
      const size_t m = std::min<size_t>(chunk, n - a);
      PXG_HIP(hipMemcpyAsync(raw.p, vecs + a * dim, m * dim * 4, hipMemcpyHostToDevice, stream));
      PXG_HIP(hipStreamSynchronize(stream));
      std::vector<uint32_t> part(m);
      insert_device(in_ids + a, raw.p, m, part.data());
      if (out_slots) std::copy(part.begin(), part.end(), out_slots + a);
    }
  }

  void add_codes(const uint64_t* in_ids, const int8_t* h_codes, uint64_t n, uint32_t* out_slots) {
    check_new_ids(in_ids, n);
    std::vector<uint32_t> sl = claim_slots(in_ids, n, out_slots);
    const size_t chunk = std::min<size_t>(std::max<size_t>(1, (64u << 20) / (size_t)dim), n);
    DevBuf<int8_t> st(chunk * dim);
    DevBuf<uint32_t> st_slots(chunk);
    DevBuf<uint64_t> st_ids(chunk);
    for (size_t a = 0; a < n; a += chunk) {
      const size_t m = std::min<size_t>(chunk, n - a);
      PXG_HIP(hipMemcpyAsync(st.p, h_codes + a * dim, m * dim, hipMemcpyHostToDevice, stream));
      PXG_HIP(hipMemcpyAsync(st_slots.p, sl.data() + a, m * 4, hipMemcpyHostToDevice, stream));
      PXG_HIP(hipMemcpyAsync(st_ids.p, in_ids + a, m * 8, hipMemcpyHostToDevice, stream));
      hipLaunchKernelGGL(sq8_place_codes, dim3((unsigned)m), dim3(64), 0, stream, st.p, (int)m, (int)dim, (int)KP,
                         st_slots.p, codes.p);
      hipLaunchKernelGGL(sq8_mark, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, stream, st_slots.p, st_ids.p,
                         (int)m, d_live.p, d_ids.p);
      PXG_HIP(hipGetLastError());
      PXG_HIP(hipStreamSynchronize(stream));
    }
    ranks.insert(in_ids, sl.data(), n, d_ids.p, stream);
  }

  void remove(uint64_t id) {
    auto it = by_id.find(id);
    if (it == by_id.end()) raise(PXG_ERR_UNKNOWN_ID, "unknown vector id " + std::to_string(id), id);
    const uint32_t s = it->second;
    by_id.erase(it);
    live[s] = 0;
    ids[s] = 0;
    slots.release(s);
    PXG_HIP(hipMemsetAsync(d_live.p + s, 0, 1, stream));
    ranks.remove(s, stream);
    PXG_HIP(hipStreamSynchronize(stream));
  }

  // max(k, rescore) beyond the block selections: integer keys of every slot,
  // segmented sort, optional rescoring of the first t and a second sort, the
  // first kq emitted. t = 0: no rescoring.
  void search_wide(const int8_t* Qc, const float* Qp, uint64_t nq, uint64_t kq, uint64_t t, const uint8_t* d_accept,
                   uint64_t* d_oid, float* d_od, uint32_t* d_oc, Scratch& sc, hipStream_t s, size_t ldo) {
    const size_t N = slots.high_water();
    const size_t per_query = 2 * N * 8 + 16;
    size_t G = std::max<size_t>(1, std::min<size_t>((1ull << 30) / per_query, ((1ull << 32) - 1) / N));
    G = std::min<size_t>(G, nq);
    uint64_t* keys = (uint64_t*)sc.get(40, G * N * 8);
    uint64_t* sorted = (uint64_t*)sc.get(41, G * N * 8);
    uint32_t* offs = (uint32_t*)sc.get(42, (2 * G + 2) * 4);
    uint32_t* ends2 = offs + G + 1;
    const size_t temp_bytes = wide_sort_temp_bytes((uint32_t)(G * N), (uint32_t)G);
    void* temp = sc.get(43, std::max<size_t>(temp_bytes, 1));
    for (size_t q0 = 0; q0 < nq; q0 += G) {
      const int gn = (int)std::min<size_t>(G, nq - q0);
      hipLaunchKernelGGL(sq8_wide_keys, dim3((unsigned)((N + 255) / 256), (unsigned)gn), dim3(256), 0, s, Qc,
                         (int)KP, (const int8_t*)codes.p, (int)N, d_live.p, d_accept, ranks.rank.p, (int)q0, keys);
      hipLaunchKernelGGL(wide_offsets, dim3((unsigned)((gn + 256) / 256)), dim3(256), 0, s, offs, gn, (uint32_t)N);
      PXG_HIP(hipGetLastError());
      wide_sort(temp, temp_bytes, keys, sorted, (uint32_t)(gn * N), (uint32_t)gn, offs, offs + 1, s);
      const uint32_t* emit_end = offs + 1;
      if (t) {
        hipLaunchKernelGGL(sq8_wide_rescore, dim3((unsigned)((t + 255) / 256), (unsigned)gn), dim3(256), 0, s, sorted,
                           offs, offs + 1, t, (int)q0, Qp, (int)ld, (int)dim, (const int8_t*)codes.p, (int)KP,
                           per_dim, d_mn.p, d_scale.p, ranks.rank_slot.p, keys);
        hipLaunchKernelGGL(wide_truncate, dim3((unsigned)((gn + 255) / 256)), dim3(256), 0, s, offs, offs + 1, gn, t,
                           ends2);
        PXG_HIP(hipGetLastError());
        wide_sort(temp, temp_bytes, keys, sorted, (uint32_t)(gn * N), (uint32_t)gn, offs, ends2, s);
        emit_end = ends2;
      }
      hipLaunchKernelGGL(wide_emit, dim3((unsigned)((kq + 255) / 256), (unsigned)gn), dim3(256), 0, s, sorted, offs,
                         emit_end, (int)q0, kq, ranks.rank_slot.p, d_ids.p, d_oid, d_od, d_oc, ldo);
      PXG_HIP(hipGetLastError());
    }
  }

  // Queries: f32 (prepared + encoded here; rescoring possible) or I8 codes.
  void search_device(const float* d_raw, const int8_t* d_qcodes, uint64_t nq, uint64_t k, uint64_t rescore,
                     const uint8_t* d_accept, uint64_t* d_oid, float* d_od, uint32_t* d_oc, Scratch& sc,
                     hipStream_t s, uint64_t* fallbacks, size_t ldo) {
    check_k(k);
    *fallbacks = 0;
    if (nq == 0) return;
    if (!d_raw && rescore) config_error("rescore", rescore, "rescoring needs the f32 queries");
    if (d_raw) require_trained();
    // at most the live count per query; the integer candidates are the best
    // max(k, rescore), also clamped to the live count
    const uint64_t kq = std::min<uint64_t>(k, by_id.size());
    const uint64_t kk64 = std::min<uint64_t>(std::max<uint64_t>(kq, rescore), by_id.size());
    Timer tm(s);
    tm.on = tm.on && sc.timing();
    tm.mark(0);
    int8_t* Qc = (int8_t*)sc.get(1, nq * KP);
    float* Qp = nullptr;
    unsigned long long* bad = (unsigned long long*)sc.get(4, 64);
    int* flag_count = (int*)(bad + 1);
    hipLaunchKernelGGL(init_search_flags, dim3(1), dim3(64), 0, s, bad, flag_count);
    if (d_raw) {
      Qp = (float*)sc.get(2, nq * ld * 4);
      float* qb = (float*)sc.get(3, nq * 4);
      float* qn = (float*)sc.get(5, nq * 4);
      hipLaunchKernelGGL(flat_prep_queries, dim3((unsigned)nq), dim3(64), 0, s, d_raw, (int)dim, (int)ld, metric, 1,
                         Qp, qb, qn, bad);
      hipLaunchKernelGGL(sq_encode_rows, dim3((unsigned)nq), dim3(64), 0, s, Qp, (int)ld, (int)nq, (int)dim, per_dim,
                         1, d_mn.p, d_inv.p, (const uint32_t*)nullptr, (uint8_t*)Qc, (int)KP);
      PXG_HIP(hipGetLastError());
      // the non-finite flag is read with the search's next host sync (a
      // non-finite query only scores garbage until then)
    } else {
      hipLaunchKernelGGL(sq8_place_codes, dim3((unsigned)nq), dim3(64), 0, s, d_qcodes, (int)nq, (int)dim, (int)KP,
                         (const uint32_t*)nullptr, Qc);
      PXG_HIP(hipGetLastError());
    }
    const int N = (int)slots.high_water();
    if (kq == 0 || kk64 > 1024) {
      if (kq == 0) {
        hipLaunchKernelGGL(fill_u32, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, d_oc, (size_t)nq, 0u);
        PXG_HIP(hipGetLastError());
      } else {
        search_wide(Qc, Qp, nq, kq, rescore ? kk64 : 0, d_accept, d_oid, d_od, d_oc, sc, s, ldo);
      }
      unsigned long long* tail = sc.host_words();
      PXG_HIP(hipMemcpyAsync(tail, bad, 8, hipMemcpyDeviceToHost, s));
      PXG_HIP(hipStreamSynchronize(s));
      if (d_raw) check_non_finite(tail[0]);
      tm.finish();
      return;
    }
    const int kk = (int)kk64;
    const int KB = (int)(KP / 32);
    uint64_t* okeys = (uint64_t*)sc.get(6, nq * kk * 8);
    uint32_t* ocount = (uint32_t*)sc.get(7, nq * 4);
    int* flag_list = (int*)sc.get(8, nq * 4);
    // automatic: the MFMA path when stage 1 can give every query >= 4 * kk
    // maxima (two per sampled chunk); smaller indexes take the exact scan
    const int ntiles_all = KB <= SQ_MAX_KB ? (N + sq_rows(KB) - 1) / sq_rows(KB) : 0;
    const bool mfma = mode != 2 && KB <= SQ_MAX_KB && (mode == 1 || (N >= 4096 && 2 * ntiles_all >= 4 * kk));
    int nflag = 0;
    // ids and distances (or the f32 rescoring) of each query's kept keys
    auto emit = [&]() {
      if (rescore) {
        int P = 1;
        while (P < kk) P <<= 1;
        hipLaunchKernelGGL(sq8_rescore, dim3((unsigned)nq), dim3(256), (size_t)P * 8, s, (const uint64_t*)okeys,
                           (const uint32_t*)ocount, kk, (int)ldo, (const float*)Qp, (int)ld, (int)dim,
                           (const int8_t*)codes.p, (int)KP, per_dim, d_mn.p, d_scale.p, ranks.rank_slot.p, d_ids.p,
                           d_oid, d_od, d_oc);
      } else {
        hipLaunchKernelGGL(sq8_emit, dim3((unsigned)nq), dim3(64), 0, s, (const uint64_t*)okeys,
                           (const uint32_t*)ocount, kk, (int)ldo, ranks.rank_slot.p, d_ids.p, d_oid, d_od, d_oc);
      }
      PXG_HIP(hipGetLastError());
    };
    if (mfma) {
      // query tiles per wave: the fewest that hold the batch in one
      // workgroup's SQ_NW waves (1 up to 256 queries, 2 up to 512), at most
      // sq_qt(KB); qtt names the kernel variant (0 = sq_qt(KB))
      const int R = sq_rows(KB), QT = nq <= 256 ? 1 : (nq <= 512 ? std::min(2, sq_qt(KB)) : sq_qt(KB));
      const int qtt = QT == sq_qt(KB) ? 0 : QT;
      // Chunks: about 512 (two per CU), and at least 2 * kk so that every
      // query gets >= 4 * kk stage-1 maxima when the index has the tiles.
      // Stage 1 samples every `sample`-th tile (a divisor of the chunk
      // length, so every chunk contributes).
      const int ntiles = (N + R - 1) / R;
      // Stage 1 visits the tiles t % sample == 0; with chunks of >= sample
      // tiles every full chunk holds one (a chunk without one only adds
      // INT_MIN entries, which never raise the threshold).
      const int target = std::min(std::min(SQ_MAX_CHUNKS, ntiles), std::max(512, 2 * kk));
      int tpc = (ntiles + target - 1) / target;
      int sample = SQ_SAMPLE;
      if (tpc < SQ_SAMPLE) {
        sample = 1;
        while (sample * 2 <= tpc) sample *= 2;
        tpc = sample;
      }
      const int nchunks = (ntiles + tpc - 1) / tpc;
      if (nchunks > SQ_MAX_CHUNKS) internal_error("sq8", "chunk count above the stage-1 limit");
      const int qgroups = (int)((nq + SQ_NW * QT * 32 - 1) / (SQ_NW * QT * 32));
      const int E = nchunks * 2;
      const int cap_c = kk <= 32 ? 1024 : 4096;
      int* tmax = (int*)sc.get(9, nq * E * 4);
      int* thr = (int*)sc.get(10, nq * 4);
      int* ccount = (int*)sc.get(11, nq * 4);
      uint64_t* cand = (uint64_t*)sc.get(12, nq * cap_c * 8);
      const dim3 grid((unsigned)((nchunks * qgroups + 7) / 8 * 8));
#define PXG_SQ_SCAN_Q(KBV, ST, QTV)                                                                                 \
  hipLaunchKernelGGL((sq8_mfma_scan<KBV, ST, QTV>), grid, dim3(SQ_NW * 64), 0, s, (const int8_t*)Qc, (int)nq,      \
                     (const int8_t*)codes.p, N, d_live.p, d_accept, ranks.rank.p, nchunks, qgroups, tpc, sample,       \
                     (const int*)thr, tmax,                                                                        \
                     ccount, cand, cap_c)
#define PXG_SQ_SCAN(KBV, ST)             \
  if (qtt == 1)                          \
    PXG_SQ_SCAN_Q(KBV, ST, 1);           \
  else if (qtt == 2)                     \
    PXG_SQ_SCAN_Q(KBV, ST, 2);           \
  else                                   \
    PXG_SQ_SCAN_Q(KBV, ST, 0)
#define PXG_SQ_SWITCH(ST)                  \
  switch (KB) {                            \
    case 1: PXG_SQ_SCAN(1, ST); break;     \
    case 2: PXG_SQ_SCAN(2, ST); break;     \
    case 3: PXG_SQ_SCAN(3, ST); break;     \
    case 4: PXG_SQ_SCAN(4, ST); break;     \
    case 5: PXG_SQ_SCAN(5, ST); break;     \
    case 6: PXG_SQ_SCAN(6, ST); break;     \
    case 7: PXG_SQ_SCAN(7, ST); break;     \
    default: PXG_SQ_SCAN(8, ST); break;    \
  }
      // stage 1 and the thresholds count as preparation; the candidates
      // stage is the stage-2 scan alone
      PXG_SQ_SWITCH(true)
      PXG_HIP(hipGetLastError());
      hipLaunchKernelGGL(sq8_thresholds, dim3((unsigned)nq), dim3(256), 0, s, (const int*)tmax, E, kk, thr);
      hipLaunchKernelGGL(fill_u32, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, (uint32_t*)ccount, (size_t)nq,
                         0u);
      tm.mark(1);
      PXG_SQ_SWITCH(false)
#undef PXG_SQ_SWITCH
#undef PXG_SQ_SCAN
#undef PXG_SQ_SCAN_Q
      PXG_HIP(hipGetLastError());
      tm.mark(2);
      hipLaunchKernelGGL(sq8_finish, dim3((unsigned)nq), dim3(256), (size_t)cap_c * 8, s, (const int*)ccount,
                         (const uint64_t*)cand, cap_c, kk, okeys, ocount, flag_list, flag_count);
      PXG_HIP(hipGetLastError());
      // The results go out before the one host round trip; a query listed
      // for the exact scan has none yet, and its results are emitted again
      // after that scan.
      emit();
      // bad (8 bytes) and flag_count (the int after it) in one copy
      unsigned long long* tail = sc.host_words();
      PXG_HIP(hipMemcpyAsync(tail, bad, 16, hipMemcpyDeviceToHost, s));
      PXG_HIP(hipStreamSynchronize(s));
      if (d_raw) check_non_finite(tail[0]);
      std::memcpy(&nflag, &tail[1], sizeof nflag);
      *fallbacks = (uint64_t)nflag;
    } else {
      tm.mark(1);
      hipLaunchKernelGGL(iota_kernel, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, flag_list, (int)nq,
                         flag_count);
      PXG_HIP(hipGetLastError());
      nflag = (int)nq;
    }
    if (nflag > 0) {
      if (mfma) tm.mark(3);
      const int nchunks = (N + EXACT_CH - 1) / EXACT_CH;
      const int kke = std::min(kk, EXACT_CH);
      uint64_t* ecand = (uint64_t*)sc.get(13, (size_t)nflag * nchunks * kke * 8);
      hipLaunchKernelGGL(sq8_exact_candidates, dim3((unsigned)std::min<int64_t>((int64_t)nflag * nchunks, 4096)),
                         dim3(256), 0, s, (const int*)flag_list, (const int*)flag_count, nchunks, (const int8_t*)Qc,
                         (int)KP, (const int8_t*)codes.p, N, d_live.p, d_accept, ranks.rank.p, kk, ecand);
      PXG_HIP(hipGetLastError());
      if (!mfma) tm.mark(2);
      hipLaunchKernelGGL(flat_merge_exact<EXACT_CH>, dim3((unsigned)nflag), dim3(256), 0, s, (const int*)flag_list,
                         (const int*)flag_count, (const uint64_t*)ecand, nchunks, kk, ranks.rank_slot.p, d_ids.p,
                         (uint64_t*)nullptr, (float*)nullptr, ocount, okeys, (size_t)kk);
      PXG_HIP(hipGetLastError());
      emit();
      unsigned long long* tail = sc.host_words();
      if (d_raw && !mfma) PXG_HIP(hipMemcpyAsync(tail, bad, 8, hipMemcpyDeviceToHost, s));
      PXG_HIP(hipStreamSynchronize(s));
      if (d_raw && !mfma) check_non_finite(tail[0]);
    }
    tm.finish();
  }

  // flat_prep_queries' flag: ~0 or (query << 32 | component) of the first
  // non-finite component
  static void check_non_finite(unsigned long long bv) {
    if (bv == ~0ull) return;
    const uint64_t row = bv >> 32, comp = (uint32_t)bv;
    raise(PXG_ERR_NON_FINITE,
          "vector component " + std::to_string(comp) + " is not finite (query " + std::to_string(row) + ")", comp,
          row, NAN);
  }
};

thread_local uint64_t g_sq8_fallbacks = 0;

}  // namespace pxg

using pxg::Sq8Index;

struct pxg_sq8 {
  Sq8Index impl;
};

namespace {

void check_groups_args(uint32_t dim) {
  if (dim < 1) pxg::config_error("dim", dim, "must be at least 1; a 0-dimensional space makes all distances equal");
  if (dim > pxg::SQ_MAX_DIM) pxg::config_error("dim", dim, "the SQ8 path supports dimensions up to 65536");
}

}  // namespace

extern "C" {

int pxg_sq_train(const float* training, uint64_t n, uint32_t dim, int per_dim, float* min, float* scale,
                 float* inverse_scale) {
  return pxg::guard([&] {
    check_groups_args(dim);
    pxg::check_training_len(n);
    pxg::check_finite_host(training, n, dim);
    hipStream_t s = nullptr;
    PXG_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    struct Del {
      hipStream_t s;
      ~Del() { (void)hipStreamDestroy(s); }
    } del{s};
    pxg::Ranges r = pxg::train_ranges_host(training, n, dim, per_dim ? 1 : 0, s);
    std::copy(r.mn.begin(), r.mn.end(), min);
    std::copy(r.scale.begin(), r.scale.end(), scale);
    std::copy(r.inv.begin(), r.inv.end(), inverse_scale);
  });
}

int pxg_sq_encode(const float* vectors, uint64_t n, uint32_t dim, int per_dim, int code_type, const float* min,
                  const float* inverse_scale, uint8_t* out) {
  return pxg::guard([&] {
    check_groups_args(dim);
    if (code_type != 0 && code_type != 1) pxg::config_error("code_type", (uint64_t)code_type, "0 = U8, 1 = I8");
    if (n == 0) return;
    for (uint64_t i = 0; i < n; ++i)
      for (uint32_t c = 0; c < dim; ++c)
        if (!std::isfinite(vectors[i * dim + c]))
          pxg::raise(PXG_ERR_NON_FINITE,
                     "vector component " + std::to_string(c) + " is not finite (" +
                         std::to_string(vectors[i * dim + c]) + ")",
                     c, i, vectors[i * dim + c]);
    const int g = per_dim ? (int)dim : 1;
    pxg::DevBuf<float> dv(n * dim), dmn(g), dinv(g);
    pxg::DevBuf<uint8_t> dout(n * dim);
    PXG_HIP(hipMemcpy(dv.p, vectors, n * dim * 4, hipMemcpyHostToDevice));
    PXG_HIP(hipMemcpy(dmn.p, min, g * 4, hipMemcpyHostToDevice));
    PXG_HIP(hipMemcpy(dinv.p, inverse_scale, g * 4, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(pxg::sq_encode_rows, dim3((unsigned)n), dim3(64), 0, 0, dv.p, (int)dim, (int)n, (int)dim,
                       per_dim ? 1 : 0, code_type, dmn.p, dinv.p, (const uint32_t*)nullptr, dout.p, (int)dim);
    PXG_HIP(hipGetLastError());
    PXG_HIP(hipMemcpy(out, dout.p, n * dim, hipMemcpyDeviceToHost));
  });
}

int pxg_sq_decode(const uint8_t* codes, uint64_t n, uint32_t dim, int per_dim, int code_type, const float* min,
                  const float* scale, float* out) {
  return pxg::guard([&] {
    check_groups_args(dim);
    if (code_type != 0 && code_type != 1) pxg::config_error("code_type", (uint64_t)code_type, "0 = U8, 1 = I8");
    if (n == 0) return;
    const int g = per_dim ? (int)dim : 1;
    pxg::DevBuf<uint8_t> dc(n * dim);
    pxg::DevBuf<float> dmn(g), dsc(g), dout(n * dim);
    PXG_HIP(hipMemcpy(dc.p, codes, n * dim, hipMemcpyHostToDevice));
    PXG_HIP(hipMemcpy(dmn.p, min, g * 4, hipMemcpyHostToDevice));
    PXG_HIP(hipMemcpy(dsc.p, scale, g * 4, hipMemcpyHostToDevice));
    const uint64_t tot = n * dim;
    hipLaunchKernelGGL(pxg::sq_decode_rows, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, 0, dc.p, n, (int)dim,
                       per_dim ? 1 : 0, code_type, dmn.p, dsc.p, dout.p);
    PXG_HIP(hipGetLastError());
    PXG_HIP(hipMemcpy(out, dout.p, tot * 4, hipMemcpyDeviceToHost));
  });
}

int pxg_sq_asymmetric(int inner_product, const float* query, const uint8_t* codes, uint64_t n, uint32_t dim,
                      int per_dim, int code_type, const float* min, const float* scale, float* out) {
  return pxg::guard([&] {
    check_groups_args(dim);
    if (code_type != 0 && code_type != 1) pxg::config_error("code_type", (uint64_t)code_type, "0 = U8, 1 = I8");
    if (n == 0) return;
    const int g = per_dim ? (int)dim : 1;
    pxg::DevBuf<uint8_t> dc(n * dim);
    pxg::DevBuf<float> dq(dim), dmn(g), dsc(g), dout(n);
    PXG_HIP(hipMemcpy(dc.p, codes, n * dim, hipMemcpyHostToDevice));
    PXG_HIP(hipMemcpy(dq.p, query, dim * 4, hipMemcpyHostToDevice));
    PXG_HIP(hipMemcpy(dmn.p, min, g * 4, hipMemcpyHostToDevice));
    PXG_HIP(hipMemcpy(dsc.p, scale, g * 4, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(pxg::sq_asym_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, 0, inner_product ? 1 : 0,
                       dq.p, dc.p, n, (int)dim, per_dim ? 1 : 0, code_type, dmn.p, dsc.p, dout.p);
    PXG_HIP(hipGetLastError());
    PXG_HIP(hipMemcpy(out, dout.p, n * 4, hipMemcpyDeviceToHost));
  });
}

int pxg_sq8_create(uint32_t dim, int metric, int per_dim, uint64_t capacity, pxg_sq8** out) {
  return pxg::guard([&] {
    if (!out) pxg::config_error("out", 0, "must not be NULL");
    check_groups_args(dim);
    if (metric != PXG_INNER_PRODUCT && metric != PXG_COSINE)
      pxg::config_error("metric", (uint64_t)metric, "the SQ8 index scores inner product (or cosine on prepared vectors)");
    auto* h = new pxg_sq8();
    Sq8Index& f = h->impl;
    f.dim = dim;
    f.ld = (dim + 3) & ~3u;
    f.KP = (dim + 31) & ~31u;
    f.metric = metric;
    f.per_dim = per_dim ? 1 : 0;
    try {
      PXG_HIP(hipStreamCreateWithFlags(&f.stream, hipStreamNonBlocking));
      if (capacity) f.ensure_capacity(capacity, 0);
    } catch (...) {
      delete h;
      throw;
    }
    *out = h;
  });
}

void pxg_sq8_destroy(pxg_sq8* index) { delete index; }

int pxg_sq8_train(pxg_sq8* index, const float* training, uint64_t n) {
  return pxg::guard([&] {
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    index->impl.train(training, false, n);
  });
}

int pxg_sq8_train_device(pxg_sq8* index, const float* d_training, uint64_t n) {
  return pxg::guard([&] {
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    index->impl.train(d_training, true, n);
  });
}

int pxg_sq8_set_ranges(pxg_sq8* index, const float* min, const float* scale, const float* inverse_scale) {
  return pxg::guard([&] {
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    Sq8Index& f = index->impl;
    const int g = f.groups();
    pxg::Ranges r;
    r.mn.assign(min, min + g);
    r.scale.assign(scale, scale + g);
    r.inv.assign(inverse_scale, inverse_scale + g);
    f.set_ranges(r);
  });
}

int pxg_sq8_ranges(const pxg_sq8* index, float* min, float* scale, float* inverse_scale) {
  return pxg::guard([&] {
    std::shared_lock<std::shared_mutex> lk(index->impl.mu);
    const Sq8Index& f = index->impl;
    if (!f.trained) pxg::config_error("quantizer", 0, "the SQ8 index has not been trained");
    std::copy(f.rg.mn.begin(), f.rg.mn.end(), min);
    std::copy(f.rg.scale.begin(), f.rg.scale.end(), scale);
    std::copy(f.rg.inv.begin(), f.rg.inv.end(), inverse_scale);
  });
}

int pxg_sq8_is_trained(const pxg_sq8* index) {
  std::shared_lock<std::shared_mutex> lk(index->impl.mu);
  return index->impl.trained ? 1 : 0;
}

int pxg_sq8_insert(pxg_sq8* index, const uint64_t* ids, const float* vectors, uint64_t n, uint32_t* out_slots) {
  return pxg::guard([&] {
    if (n == 0) return;
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    index->impl.insert_host(ids, vectors, n, out_slots);
  });
}

int pxg_sq8_insert_device(pxg_sq8* index, const uint64_t* ids, const float* d_vectors, uint64_t n,
                          uint32_t* out_slots) {
  return pxg::guard([&] {
    if (n == 0) return;
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    index->impl.insert_device(ids, d_vectors, n, out_slots);
  });
}

int pxg_sq8_add_codes(pxg_sq8* index, const uint64_t* ids, const int8_t* codes, uint64_t n, uint32_t* out_slots) {
  return pxg::guard([&] {
    if (n == 0) return;
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    index->impl.add_codes(ids, codes, n, out_slots);
  });
}

int pxg_sq8_remove(pxg_sq8* index, uint64_t id) {
  return pxg::guard([&] {
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    index->impl.remove(id);
  });
}

int pxg_sq8_contains(const pxg_sq8* index, uint64_t id) {
  std::shared_lock<std::shared_mutex> lk(index->impl.mu);
  return index->impl.by_id.count(id) ? 1 : 0;
}

uint64_t pxg_sq8_len(const pxg_sq8* index) {
  std::shared_lock<std::shared_mutex> lk(index->impl.mu);
  return index->impl.by_id.size();
}

int pxg_sq8_stats(const pxg_sq8* index, pxg_index_stats* out) {
  return pxg::guard([&] {
    std::shared_lock<std::shared_mutex> lk(index->impl.mu);
    const Sq8Index& f = index->impl;
    out->len = f.by_id.size();
    out->deleted = 0;
    out->dim = f.dim;
    out->metric = f.metric;
    out->layers = 1;
    out->edges = 0;
    out->vector_bytes = f.codes.bytes();
    out->graph_bytes = (uint64_t)(f.rg.mn.size() + f.rg.scale.size() + f.rg.inv.size()) * 4;  // table_bytes
  });
}

int pxg_sq8_get_code(const pxg_sq8* index, uint64_t id, int8_t* out) {
  return pxg::guard([&] {
    std::shared_lock<std::shared_mutex> lk(index->impl.mu);
    const Sq8Index& f = index->impl;
    auto it = f.by_id.find(id);
    if (it == f.by_id.end()) pxg::raise(PXG_ERR_UNKNOWN_ID, "unknown vector id " + std::to_string(id), id);
    PXG_HIP(hipMemcpy(out, f.codes.p + (size_t)it->second * f.KP, f.dim, hipMemcpyDeviceToHost));
  });
}

uint64_t pxg_sq8_slot_count(const pxg_sq8* index) {
  std::shared_lock<std::shared_mutex> lk(index->impl.mu);
  return index->impl.slots.high_water();
}

int pxg_sq8_slots(const pxg_sq8* index, uint64_t* ids, uint8_t* live) {
  return pxg::guard([&] {
    std::shared_lock<std::shared_mutex> lk(index->impl.mu);
    const Sq8Index& f = index->impl;
    const size_t hw = f.slots.high_water();
    for (size_t s = 0; s < hw; ++s) {
      if (ids) ids[s] = f.live[s] ? f.ids[s] : 0;
      if (live) live[s] = f.live[s];
    }
  });
}

static int sq8_search_host(const pxg_sq8* index, const float* queries, const int8_t* qcodes, uint64_t nq, uint64_t k,
                           uint64_t rescore, const uint8_t* accept, uint64_t* out_ids, float* out_dist,
                           uint32_t* out_count) {
  return pxg::guard([&] {
    pxg::check_k(k);
    Sq8Index& f = const_cast<Sq8Index&>(index->impl);
    std::shared_lock<std::shared_mutex> lk(f.mu);
    if (nq == 0) return;
    pxg::CtxLease ctx(f.pool);
    pxg::CtxScratch sc(ctx.c);
    hipStream_t s = ctx->stream;
    const size_t N = f.slots.high_water();
    uint8_t* d_acc = nullptr;
    if (accept && N) {
      d_acc = ctx->get(21, N);
      PXG_HIP(hipMemcpyAsync(d_acc, accept, N, hipMemcpyHostToDevice, s));
    }
    // at most the live count per query: device rows of kq, copied into the
    // caller's rows of k
    const uint64_t kq = std::min<uint64_t>(k, f.by_id.size());
    const size_t kk = std::max<size_t>(kq, 1);
    uint64_t* d_oid = (uint64_t*)ctx->get(22, nq * kk * 8);
    float* d_od = (float*)ctx->get(23, nq * kk * 4);
    uint32_t* d_oc = (uint32_t*)ctx->get(24, nq * 4);
    float* d_q = nullptr;
    int8_t* d_qc = nullptr;
    if (queries) {
      d_q = (float*)ctx->get(20, nq * f.dim * 4);
      PXG_HIP(hipMemcpyAsync(d_q, queries, nq * f.dim * 4, hipMemcpyHostToDevice, s));
    } else {
      d_qc = (int8_t*)ctx->get(25, nq * f.dim);
      PXG_HIP(hipMemcpyAsync(d_qc, qcodes, nq * f.dim, hipMemcpyHostToDevice, s));
    }
    uint64_t fb = 0;
    f.search_device(d_q, d_qc, nq, kq, rescore, d_acc, d_oid, d_od, d_oc, sc, s, &fb, kk);
    pxg::results_to_host(*ctx.c, s, nq, k, kq, kk, d_oid, d_od, d_oc, out_ids, out_dist, out_count, [] {});
    pxg::g_sq8_fallbacks = fb;
  });
}

int pxg_sq8_search(const pxg_sq8* index, const float* queries, uint64_t nq, uint64_t k, uint64_t rescore,
                   const uint8_t* accept, uint64_t* out_ids, float* out_dist, uint32_t* out_count) {
  return sq8_search_host(index, queries, nullptr, nq, k, rescore, accept, out_ids, out_dist, out_count);
}

int pxg_sq8_search_codes(const pxg_sq8* index, const int8_t* query_codes, uint64_t nq, uint64_t k,
                         const uint8_t* accept, uint64_t* out_ids, float* out_dist, uint32_t* out_count) {
  return sq8_search_host(index, nullptr, query_codes, nq, k, 0, accept, out_ids, out_dist, out_count);
}

int pxg_sq8_search_device(const pxg_sq8* index, const float* d_queries, uint64_t nq, uint64_t k, uint64_t rescore,
                          const uint8_t* d_accept, uint64_t* d_out_ids, float* d_out_dist, uint32_t* d_out_count,
                          void* stream) {
  return pxg::guard([&] {
    pxg::check_k(k);
    Sq8Index& f = const_cast<Sq8Index&>(index->impl);
    std::shared_lock<std::shared_mutex> lk(f.mu);
    pxg::CtxLease ctx(f.pool);
    pxg::CtxScratch sc(ctx.c);
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    pxg::DrainOnUnwind drain{s};
    uint64_t fb = 0;
    f.search_device(d_queries, nullptr, nq, k, rescore, d_accept, d_out_ids, d_out_dist, d_out_count, sc, s, &fb, k);
    PXG_HIP(hipStreamSynchronize(s));
    pxg::g_sq8_fallbacks = fb;
  });
}

uint64_t pxg_sq8_last_fallbacks(void) { return pxg::g_sq8_fallbacks; }

int pxg_sq8_set_search_mode(pxg_sq8* index, int mode) {
  return pxg::guard([&] {
    if (mode < 0 || mode > 2) pxg::config_error("mode", (uint64_t)mode, "0 = auto, 1 = MFMA candidates, 2 = exact scan");
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    index->impl.mode = mode;
  });
}

}  // extern "C"
