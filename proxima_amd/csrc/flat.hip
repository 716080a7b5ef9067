// Exact flat search on MI355X: FlatIndex (crates/proxima-index/src/flat.rs).
//
// Search pipeline for a batch of nq prepared queries against N slots:
//
//  1. flat_prep_queries   validate + (cosine) normalise each query on the
//                         device, pad rows to `ld`, and compute the bias and
//                         norm terms of the MFMA epilogue.
//  2. flat_mfma_candidates  FP32-MFMA (v_mfma_f32_32x32x2f32) tiled GEMM of
//                         the query block against database tiles staged in
//                         LDS, fused with a per-query top-k' filter: scores
//                         below the running threshold are appended to a
//                         per-(query, split) buffer that a wave-level bitonic
//                         sort compacts back to k' whenever it fills. The
//                         N x nq score matrix never reaches HBM. A seeding
//                         pass scores the first tile of every split first:
//                         flat_seed_threshold2 (from each split's two
//                         smallest keys per row; _wave sorts them in one
//                         wavefront for up to 64 splits) or
//                         flat_seed_threshold (from all of them) turns those
//                         keys into each query's starting threshold, and the
//                         full pass filters them instead of recomputing
//                         that tile.
//  3. flat_merge_rescore  per query: radix-select the k' best approximate
//                         keys over all splits, rescore those k' exactly with
//                         the reference's 8-lane arithmetic, sort by
//                         (total_cmp(distance), id) and keep k. A query whose
//                         k-th exact distance is not below the k'-th
//                         approximate one minus the MFMA error bound is
//                         flagged. flat_merge_rescore_reg does the same
//                         when a query's keys fit eight per thread and k'
//                         one wavefront: its keys are read once into
//                         registers and one wavefront sorts the rescored
//                         ones.
//  4. flat_exact_candidates + flat_merge_exact   exact VALU scan for flagged
//                         queries (and the whole batch for Manhattan, small
//                         problems, or when forced). Distances are the
//                         reference's bit for bit and ordering is exact, so
//                         results equal the reference's FlatIndex::search.
//
// Ordering key everywhere: (ord_key(distance) << 32) | id_rank, where
// id_rank is the rank of the slot's id among live ids. Sorting that key is
// sorting by (total_cmp(distance), id), which is SearchResult's order
// (topk.rs:63-67).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <mutex>
#include <numeric>
#include <shared_mutex>

#include "common.hpp"
#include "device.hpp"
#include "exact_scan.hpp"
#include "flat.hpp"
#include "wide.hpp"

namespace pxg {

typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int FB_M = 128;   // queries per workgroup tile
constexpr int FB_N = 128;   // slots per workgroup tile
constexpr int FB_K = 32;    // k-slice staged in LDS
// A staged slice is [rows][FB_K] floats without padding; 16-byte chunk c of
// row r sits at chunk position c ^ (r & 7), so 8 lanes reading chunk c of 8
// consecutive rows touch 8 different groups of banks.
constexpr int MARGIN = 16;  // k' = k + MARGIN
constexpr int FAST_KMAX = 256;

// ---------------------------------------------------------------------------
// 2. MFMA distance GEMM fused with a per-query top-k' filter
// ---------------------------------------------------------------------------
#if defined(__HIP_DEVICE_COMPILE__)
// A raw buffer resource over [p, p + bytes), built from wave-uniform scalars.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void* p, int bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  const int n = __builtin_amdgcn_readfirstlane(bytes);
  return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)(((uint64_t)hi << 32) | lo), 0, n, 0x00020000);
}

// Buffer load of 16 bytes per lane straight into LDS: lane i's bytes land at
// m0 + 16 i, and an offset outside the resource lands as zeros. Inline asm,
// so that the compiler neither tracks these loads under vmcnt (it would wait
// for them before every LDS read) nor needs m0 elsewhere: this kernel has no
// other use of m0 (no LDS-DMA builtins, no indirect register indexing). The
// wait is vm_wait0().
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(m0), "v"(voff), "s"(rs),
               "s"(soff)
               : "memory", "m0");
}
#pragma clang diagnostic pop
#endif

// LDS byte address of a __shared__ location.
__device__ __forceinline__ uint32_t lds_u32(const float* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float*)p;
}
__device__ __forceinline__ void vm_wait0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <int CAP>
__device__ inline void compact_row_w(uint64_t* __restrict__ base, int c, int Kp, int lane, uint64_t* thr_row,
                                     float* thrf_row, int* cnt_row, unsigned long long* gthr_row, bool final_pass) {
  constexpr int E = CAP / WAVE;
  uint64_t kk[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int idx = lane * E + e;
    kk[e] = idx < c ? base[idx] : KEY_MAX;
  }
  wave_bitonic_sort<E>(kk, lane);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int idx = lane * E + e;
    if (idx < Kp) base[idx] = kk[e];
    if (idx == Kp - 1 && !final_pass) {
      *thr_row = kk[e];
      *thrf_row = key_float((uint32_t)(kk[e] >> 32));
      // this split keeps Kp candidates at or below kk[e] to the end, so no
      // key above it can be in the query's top Kp over all splits
      if (kk[e] != KEY_MAX) atomicMin(gthr_row, (unsigned long long)kk[e]);
    }
  }
  if (lane == 0 && !final_pass) *cnt_row = Kp;
}

// Keep the Kp smallest of a row's c buffered keys, sorted, KEY_MAX padded to
// Kp: sorted over the narrowest width (64 keys per lane-slot step) that
// holds max(c, Kp), up to the buffer's CAP.
template <int CAP>
__device__ __attribute__((noinline)) void compact_row(uint64_t* __restrict__ base, int c, int Kp, int lane, uint64_t* thr_row,
                                   float* thrf_row, int* cnt_row, unsigned long long* gthr_row, bool final_pass) {
  const int need = c > Kp ? c : Kp;
  if (need <= 64)
    compact_row_w<64>(base, c, Kp, lane, thr_row, thrf_row, cnt_row, gthr_row, final_pass);
  else if (need <= 128 && CAP >= 128)
    compact_row_w<(CAP >= 128 ? 128 : CAP)>(base, c, Kp, lane, thr_row, thrf_row, cnt_row, gthr_row, final_pass);
  else if (need <= 256 && CAP >= 256)
    compact_row_w<(CAP >= 256 ? 256 : CAP)>(base, c, Kp, lane, thr_row, thrf_row, cnt_row, gthr_row, final_pass);
  else
    compact_row_w<CAP>(base, c, Kp, lane, thr_row, thrf_row, cnt_row, gthr_row, final_pass);
}

// The first tile of a seeded split in the full pass: the keys the seeding
// pass left in the last FB_N / 2 entries of each row's buffer (FB_N 32-bit
// distance parts, slot n0 + c at word c), rebuilt as (distance part, slot)
// and tested against the row's threshold like computed ones. 32 threads per
// row, 16 bytes each (thread t takes chunk t & 31 of rows t / 32 + 8 u, the
// same four slots in every row), all loads in flight together, the slots'
// liveness and acceptance read once beside them; a word above the
// threshold's distance part is skipped before the exact key test. The
// appends (at most FB_N per row, the row's first) stay below the stored
// words. Out of line, so that the main loop's registers are not shaped by it.
template <int CAP>
__device__ __attribute__((noinline)) void flat_stored_tile(uint64_t* __restrict__ cand, int S, int split, int q0,
                                                           int nq, int n0, int s_end, const uint8_t* __restrict__ live,
                                                           const uint8_t* __restrict__ acc_src, const uint64_t* thr,
                                                           int* cnt, int tid) {
  constexpr int U = FB_M / 8;
  const int c = tid & 31;
  uint4 w[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int qr = min(q0 + (tid >> 5) + 8 * u, nq - 1);  // unconditional loads
    w[u] = reinterpret_cast<const uint4*>(cand + ((size_t)qr * S + split) * CAP + (CAP - FB_N / 2))[c];
  }
  bool usable[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int slot = n0 + 4 * c + e;
    const int sl = min(slot, s_end - 1);  // unconditional loads
    usable[e] = slot < s_end && (live[sl] & acc_src[sl]) != 0;
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int row = (tid >> 5) + 8 * u;
    if (q0 + row >= nq) continue;
    const uint64_t t = thr[row];
    const uint32_t th = (uint32_t)(t >> 32);
    const uint32_t kk[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (kk[e] <= th) {
        const int slot = n0 + 4 * c + e;
        const uint64_t key = ((uint64_t)kk[e] << 32) | (uint32_t)slot;
        if (key < t && usable[e]) {
          const int pos = atomicAdd(&cnt[row], 1);
          cand[((size_t)(q0 + row) * S + split) * CAP + pos] = key;
        }
      }
    }
  }
}

// SEED: the seeding pass (a separate instantiation, so that the full pass's
// code is not shaped by the seeding epilogue).
template <int CAP, bool SEED>
__global__ __launch_bounds__(256, 2) void flat_mfma_candidates(
    const float* __restrict__ Q, int nq, const float* __restrict__ X, int N, int ld,
    const float* __restrict__ qb, const float* __restrict__ xb, float scale, const uint8_t* __restrict__ live,
    const uint8_t* __restrict__ accept, int S, int QB, int per_split, int Kp,
    uint64_t* __restrict__ cand, unsigned long long* __restrict__ gthr, int seeded) {
  __shared__ __align__(16) float sQ[2][FB_M * FB_K];
  __shared__ __align__(16) float sX[2][FB_N * FB_K];
  __shared__ uint64_t thr[FB_M];
  __shared__ int cnt[FB_M];
  __shared__ __align__(16) float sqb[FB_M];
  // thr as a float, key_float(thr >> 32): NaN while thr is KEY_MAX
  __shared__ __align__(16) float thr_f[FB_M];

  // XCD-aware mapping: consecutive workgroup ids are dealt round-robin over
  // the 8 XCDs, so give each XCD a contiguous range of (split, query block)
  // work; the QB workgroups sharing one split's database tiles then run on
  // the same XCD at the same time and share its L2.
  const int total = QB * S;
  const int per_xcd = (total + 7) / 8;
  const int g = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (g >= total) return;
  const int qblk = g % QB, split = g / QB;
  const int q0 = qblk * FB_M;
  const int s_begin = split * per_split;
  // a seeding pass visits only the first tile of each split
  const int s_end = min(N, s_begin + (SEED ? FB_N : per_split));

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int h = lane >> 5, r = lane & 31;
  const int wm = (wid >> 1) * 64, wn = (wid & 1) * 64;

  for (int i = tid; i < FB_M; i += 256) {
    thr[i] = KEY_MAX;
    thr_f[i] = key_float((uint32_t)(KEY_MAX >> 32));
    cnt[i] = 0;
    sqb[i] = (q0 + i < nq) ? qb[q0 + i] : 0.0f;
  }
  __syncthreads();

  // global->LDS copy: instruction u of wave wid fills rows 32 wid + 8 u ..
  // +7 of a slice; lane l lands at chunk position l & 7 of row 8 u + l / 8,
  // so it fetches that row's chunk (l & 7) ^ (row & 7)
  [[maybe_unused]] const int crow = 32 * wid + (lane >> 3), cchunk = (lane & 7) ^ ((lane >> 3) & 7);
  [[maybe_unused]] const int wid_s = __builtin_amdgcn_readfirstlane(wid);
  const int nK = (ld + FB_K - 1) / FB_K;
  // The two slice buffers alternate over the whole run of tiles (gs counts
  // the slices consumed so far): the last slice of a tile prefetches the
  // first slice of the next, so only the first tile waits for its first
  // slice.
  int gs = 0;

  for (int n0 = s_begin; n0 < s_end; n0 += FB_N) {
    // the other splits' published thresholds for this tile's rows, read now
    // and applied after the k loop (an older value is only looser)
    const uint64_t g_thr = tid < FB_M && q0 + tid < nq
                               ? __hip_atomic_load(gthr + q0 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                               : KEY_MAX;
    // this lane's two slots of the tile (live, accepted, norm), also read
    // before the k loop so that the epilogue does not wait for them
    // (unconditional loads at a clamped slot, so that nothing waits for them
    // before the epilogue; slots past s_end are masked there)
    int slotj[2];
    uint32_t lvj[2], acj[2];
    float xbr[2];
    const uint8_t* acc_src = accept != nullptr ? accept : live;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      slotj[j] = n0 + wn + j * 32 + r;
      const int sl = min(slotj[j], N - 1);
      lvj[j] = live[sl];
      acj[j] = acc_src[sl];
      xbr[j] = xb[sl];
    }
    // A seeded full pass takes the first tile of its split from the keys
    // the seeding pass left at the tail of each row's buffer (the same
    // instructions on the same operands, so the same keys) instead of
    // computing it again.
    const bool stored = !SEED && seeded != 0 && n0 == s_begin;
    f16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

#if defined(__HIP_DEVICE_COMPILE__)
    // Buffer loads over a tile's query and slot rows, straight to LDS: rows
    // past the valid ones, and the chunks past a row's end in the last slice
    // of a stride that is not a multiple of FB_K, are given an offset outside
    // the resource and land as zeros.
    const float* q_rows = Q + (size_t)q0 * ld;
    const int q_bytes = max(min(nq - q0, FB_M), 0) * ld * 4;
#endif
    // slice k0 of the tile starting at slot t0, into buffer buf
    auto gload = [&](int t0, int k0, int buf) {
#if defined(__HIP_DEVICE_COMPILE__)
      const float* x_rows = X + (size_t)t0 * ld;
      const int x_bytes = max(min(s_end - t0, FB_N), 0) * ld * 4;
      // the resources are rebuilt per call from readfirstlane'd scalars (a
      // hoisted resource kept in VGPRs is not known to be uniform)
      const __amdgpu_buffer_rsrc_t rs_q = uniform_rsrc(q_rows, q_bytes);
      const __amdgpu_buffer_rsrc_t rs_x = uniform_rsrc(x_rows, x_bytes);
      // row group u adds 8 u rows through the scalar offset; a lane past the
      // row end stays outside the resource for every group
      const int kc = k0 + cchunk * 4;
      const uint32_t voff = kc < ld ? (uint32_t)((crow * ld + kc) * 4) : 0x7FFFFFF0u;
      const uint32_t q_lds = lds_u32(&sQ[buf][0]), x_lds = lds_u32(&sX[buf][0]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t soff = (uint32_t)(8 * u * ld * 4), grp = (uint32_t)((32 * wid_s + 8 * u) * FB_K * 4);
        lds_dma16(rs_q, voff, soff, q_lds + grp);
        lds_dma16(rs_x, voff, soff, x_lds + grp);
      }
#endif
    };

    if (stored) {
      // the next tile's first slice, which the k loop below would have
      // prefetched (no slice is consumed here, so gs is unchanged); waited
      // for after the stored keys' epilogue
      if (n0 + FB_N < s_end) gload(n0 + FB_N, 0, gs & 1);
    } else {
      if (n0 == s_begin) {
        gload(n0, 0, gs & 1);
        vm_wait0();
        __syncthreads();
      }
      for (int kt = 0; kt < nK; ++kt) {
        const int cur = (gs + kt) & 1;
        if (kt + 1 < nK) gload(n0, (kt + 1) * FB_K, cur ^ 1);
        else if (n0 + FB_N < s_end) gload(n0 + FB_N, 0, cur ^ 1);
        // Lane (h, r) feeds k = h*16 + kk of row r: the MFMA pairs A and B by
        // lane half, so any fixed permutation of k within the slice is a
        // valid dot product; this one lets each lane read 16 contiguous floats
        // (chunks 4h .. 4h+3 of its row, swizzled by r & 7; wm, wn and 32 are
        // multiples of 8).
        const float* a0p = &sQ[cur][(wm + r) * FB_K];
        const float* a1p = &sQ[cur][(wm + 32 + r) * FB_K];
        const float* b0p = &sX[cur][(wn + r) * FB_K];
        const float* b1p = &sX[cur][(wn + 32 + r) * FB_K];
        const int r7 = r & 7;
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) {
          const int co = ((4 * h + k4) ^ r7) * 4;
          const float4 a0 = *reinterpret_cast<const float4*>(a0p + co);
          const float4 a1 = *reinterpret_cast<const float4*>(a1p + co);
          const float4 b0 = *reinterpret_cast<const float4*>(b0p + co);
          const float4 b1 = *reinterpret_cast<const float4*>(b1p + co);
          const float av0[4] = {a0.x, a0.y, a0.z, a0.w}, av1[4] = {a1.x, a1.y, a1.z, a1.w};
          const float bv0[4] = {b0.x, b0.y, b0.z, b0.w}, bv1[4] = {b1.x, b1.y, b1.z, b1.w};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(av0[t], bv0[t], acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(av0[t], bv1[t], acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(av1[t], bv0[t], acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(av1[t], bv1[t], acc[1][1], 0, 0, 0);
          }
        }
        vm_wait0();  // this wave's copies of the next slice have landed
        __syncthreads();
      }
      gs += nK;
    }
    if (tid < FB_M && g_thr < thr[tid]) {
      thr[tid] = g_thr;
      thr_f[tid] = key_float((uint32_t)(g_thr >> 32));
    }
    __syncthreads();

    // Epilogue: approximate score, threshold filter, append. Lane (h, r)
    // holds rows wm + 32i + 8vb + 4h + e (e < 4) of slots n0 + wn + 32j + r.
    // The score (qb + xb) - scale * dot is one fma: scale is 2 or 1, so the
    // product is exact and the fma rounds once, as the subtraction would.
    // A branch-free pass marks the values a with !(a > thr_f[row]), reading
    // four rows' norms and thresholds per LDS read. That test passes every
    // key below thr[row] (key_float inverts ord_key; NaN and the sign of zero
    // pass), so only the marked values take the exact key test and append.
    if constexpr (SEED) {
      // Seeding pass: every usable value of its one tile is kept, as its
      // distance part (unusable slots: 0xFFFFFFFF), in the last FB_N / 2
      // entries of the row's buffer read as FB_N 32-bit words (no counters,
      // no atomics; the seed threshold needs only the distance parts, and
      // the full pass rebuilds each key from its slot). The full pass's
      // appends from this tile (at most FB_N) stay below that region.
      // The tile's words go through LDS first: both slice buffers are free
      // after a one-tile k loop, and hold the 128 x 128 words exactly (rows
      // 0..63 in sQ, 64..127 in sX, the wave's rows wm..wm+63 in one of
      // them). Row R's word c sits at c ^ (32 * bit 2 of R), so that the
      // two lane halves of a store (rows 4 apart) use different banks.
      uint32_t* wbase = reinterpret_cast<uint32_t*>(wm == 0 ? &sQ[0][0] : &sX[0][0]);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const bool ok = (slotj[j] < s_end) & ((lvj[j] & acj[j]) != 0u);
        const float xo = ok ? xbr[j] : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int lrow = i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);  // row - wm
            const float a = __builtin_fmaf(-scale, acc[i][j][v], sqb[wm + lrow] + xo);
            wbase[lrow * FB_N + ((wn + j * 32 + r) ^ (32 * h))] = ok ? ord_key(a) : 0xFFFFFFFFu;
          }
      }
      __syncthreads();
      const uint32_t* words = reinterpret_cast<const uint32_t*>(&sQ[0][0]);
      const uint32_t* words_hi = reinterpret_cast<const uint32_t*>(&sX[0][0]);
      // copy out: 32 threads per row, 16 bytes each (the row's 512 bytes)
#pragma unroll 4
      for (int u = 0; u < FB_M / 8; ++u) {
        const int row = (tid >> 5) + 8 * u, c = tid & 31;
        if (q0 + row < nq) {
          const uint32_t* rw = (row < 64 ? words + row * FB_N : words_hi + (row - 64) * FB_N);
          const uint4 w4 = *reinterpret_cast<const uint4*>(rw + ((4 * c) ^ (32 * ((row >> 2) & 1))));
          reinterpret_cast<uint4*>(cand + ((size_t)(q0 + row) * S + split) * CAP + (CAP - FB_N / 2))[c] = w4;
        }
      }
      // Each row's two smallest words, as two 32-bit words in the entry just
      // below them (smallest first): two threads per row, each over one half
      // of the row's positions (any order: it starts at chunk row & 15, so
      // that the rows of one read use different banks), keep a sorted pair
      // and merge with the neighbour lane's pair.
      {
        const int row = tid >> 1, half = tid & 1;
        const uint32_t* rw = (row < 64 ? words + row * FB_N : words_hi + (row - 64) * FB_N) + half * (FB_N / 2);
        uint32_t m1 = 0xFFFFFFFFu, m2 = 0xFFFFFFFFu;
#pragma unroll
        for (int u = 0; u < FB_N / 8; ++u) {
          const uint4 w = reinterpret_cast<const uint4*>(rw)[(u + row) & (FB_N / 8 - 1)];
          const uint32_t x4[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            m2 = min(m2, max(m1, x4[e]));
            m1 = min(m1, x4[e]);
          }
        }
        const uint32_t p1 = __shfl_xor(m1, 1), p2 = __shfl_xor(m2, 1);
        const uint32_t n1 = min(m1, p1), n2 = min(max(m1, p1), min(m2, p2));
        if (half == 0 && q0 + row < nq)
          cand[((size_t)(q0 + row) * S + split) * CAP + (CAP - FB_N / 2 - 1)] = ((uint64_t)n2 << 32) | n1;
      }
    } else if (stored) {
      flat_stored_tile<CAP>(cand, S, split, q0, nq, n0, s_end, live, acc_src, thr, cnt, tid);
      vm_wait0();  // the prefetched slice
    } else {
      // Validity as bit masks applied once per row group (usable slots: the
      // j halves; rows below nq: both halves), so that the per-value work is
      // straight-line code: one compare and one select into the mask.
      uint32_t okbits = 0u;
      float xbj[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const bool ok = (slotj[j] < s_end) & ((lvj[j] & acj[j]) != 0u);
        okbits |= ok ? 0xFFFFu << (16 * j) : 0u;
        xbj[j] = ok ? xbr[j] : 0.0f;
      }
      // Appends go through this wave's 8 KB of the slice buffer the k loop
      // has finished with (all waves are past its last read, and the next
      // tile's first write to it follows the epilogue's closing barrier):
      // each row group's eight approximate scores are stored there, and a
      // lane then visits only its own marked values, lowest bit first, so
      // the wave loops as often as its busiest lane has marks instead of
      // once per value with two LDS round trips each.
      const int fb = (gs - 1) & 1;
      float* slab = (wid < 2 ? &sQ[fb][0] : &sX[fb][0]) + (wid & 1) * (2 * 4 * WAVE * 4);
      // value (j, v) of this lane at slab[((j * 4 + (v >> 2)) * WAVE + lane) * 4 + (v & 3)]
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        uint32_t pass = 0u;  // bit j * 16 + v
        uint32_t rokbits = 0u;
#pragma unroll
        for (int v = 0; v < 16; ++v)
          rokbits |= q0 + wm + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3) < nq ? 0x10001u << v : 0u;
#pragma unroll
        for (int vb = 0; vb < 4; ++vb) {
          const int row0 = wm + i * 32 + 8 * vb + 4 * h;
          const float4 sq = *reinterpret_cast<const float4*>(&sqb[row0]);
          const float4 tf = *reinterpret_cast<const float4*>(&thr_f[row0]);
          const float sqv[4] = {sq.x, sq.y, sq.z, sq.w}, tfv[4] = {tf.x, tf.y, tf.z, tf.w};
          float av[2][4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              const float a = __builtin_fmaf(-scale, acc[i][j][vb * 4 + e], sqv[e] + xbj[j]);
              av[j][e] = a;
              pass |= !(a > tfv[e]) ? 1u << (j * 16 + vb * 4 + e) : 0u;
            }
          }
#pragma unroll
          for (int j = 0; j < 2; ++j)
            *reinterpret_cast<float4*>(&slab[((j * 4 + vb) * WAVE + lane) * 4]) =
                make_float4(av[j][0], av[j][1], av[j][2], av[j][3]);
          __builtin_amdgcn_sched_barrier(0);  // bounds the live rows (no spills)
        }
        pass &= okbits & rokbits;
        while (__ballot(pass != 0u)) {
          if (pass != 0u) {
            const int b = __builtin_ctz(pass);
            pass &= pass - 1u;
            const int j = b >> 4, v = b & 15;
            const int row = wm + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
            const float a = slab[((j * 4 + (v >> 2)) * WAVE + lane) * 4 + (v & 3)];
            const uint64_t key = ((uint64_t)ord_key(a) << 32) | (uint32_t)(n0 + wn + j * 32 + r);
            if (key < thr[row]) {
              const int pos = atomicAdd(&cnt[row], 1);
              cand[((size_t)(q0 + row) * S + split) * CAP + pos] = key;
            }
          }
        }
      }
    }
    __syncthreads();
    if constexpr (!SEED) {
      // this wave's rows wid, wid + 4, ...: one count per lane, then a
      // compaction for each row that might not take another tile's appends
      const int c_l = lane < FB_M / 4 ? cnt[wid + 4 * lane] : 0;
      uint64_t full = __ballot(c_l > CAP - FB_N);
      while (full) {
        const int l = __builtin_ctzll(full);
        full &= full - 1;
        const int row = wid + 4 * l;
        compact_row<CAP>(cand + ((size_t)(q0 + row) * S + split) * CAP, __builtin_amdgcn_readlane(c_l, l), Kp,
                         lane, &thr[row], &thr_f[row], &cnt[row], gthr + q0 + row, false);
      }
      __syncthreads();
    }
  }
  // Seeding pass: each row has left its one tile's FB_N distance parts.
  if constexpr (SEED) return;
  // Final: every row leaves Kp keys, its Kp smallest (KEY_MAX padded). The
  // merge reads them as a set, so a row with at most Kp keys is only padded;
  // a fuller one is sorted down to Kp.
  for (int row = wid; row < FB_M; row += 4) {
    if (q0 + row >= nq) continue;
    uint64_t* base = cand + ((size_t)(q0 + row) * S + split) * CAP;
    const int c = cnt[row];
    if (c <= Kp) {
      for (int i = c + lane; i < Kp; i += WAVE) base[i] = KEY_MAX;
    } else {
      compact_row<CAP>(base, c, Kp, lane, &thr[row], &thr_f[row], &cnt[row], gthr + q0 + row, true);
    }
  }
}

// ---------------------------------------------------------------------------
// 3. merge + exact rescore (approximate candidates)
// ---------------------------------------------------------------------------
// Per query: the Kp-th smallest distance part over the words a seeding pass
// left (the first tile of every split, FB_N 32-bit distance parts in the
// last FB_N / 2 entries of each split's buffer, 0xFFFFFFFF for unusable
// slots).
// The full pass meets all of those rows again, so a threshold above every
// key with that distance part (the strict key test passes them all) leaves
// at least Kp rows, the query's Kp best among them, in its lists.
__global__ __launch_bounds__(512) void flat_seed_threshold(const uint64_t* __restrict__ cand, int S, int CAP, int Kp,
                                                           unsigned long long* __restrict__ gthr) {
  __shared__ int hist[256];
  __shared__ uint64_t sh[4];
  const int q = blockIdx.x;
  const uint64_t* c = cand + (size_t)q * S * CAP;
  const uint32_t* c32 = reinterpret_cast<const uint32_t*>(c);
  auto get = [&](int i) { return (uint64_t)c32[(size_t)(i / FB_N) * (2 * CAP) + 2 * (CAP - FB_N / 2) + i % FB_N]; };
  const int n = S * FB_N;
  if (n < Kp) return;  // fewer words than Kp bound nothing (the host does not seed then)
  const uint64_t hi = n <= 16 * (int)blockDim.x ? block_radix_select<decltype(get), 32, 16>(get, n, Kp, hist, sh)
                                    : block_radix_select<decltype(get), 32>(get, n, Kp, hist, sh);
  if (threadIdx.x == 0 && hi != 0xFFFFFFFFull) atomicMin(gthr + q, (unsigned long long)((hi << 32) | 0xFFFFFFFFull));
}

// Per query: the Kp-th smallest of the splits' pairs of smallest distance
// parts (2 S >= Kp words, one entry below each split's stored words). The
// pairs come from distinct rows, so at least Kp rows have a distance part at
// or below it: the same kind of bound as flat_seed_threshold's, from 2 words
// per split instead of FB_N, and as tight unless a split holds three or more
// of the Kp best seeding rows.
__global__ __launch_bounds__(64) void flat_seed_threshold2(const uint64_t* __restrict__ cand, int S, int CAP, int Kp,
                                                           unsigned long long* __restrict__ gthr) {
  __shared__ int hist[256];
  __shared__ uint64_t sh[4];
  const int q = blockIdx.x;
  const uint32_t* c32 = reinterpret_cast<const uint32_t*>(cand + (size_t)q * S * CAP + (CAP - FB_N / 2 - 1));
  auto get = [&](int i) { return (uint64_t)c32[(size_t)(i >> 1) * (2 * CAP) + (i & 1)]; };
  if (2 * S < Kp) return;  // the host launches this with 2 S >= 4 Kp
  const uint64_t hi = block_radix_select<decltype(get), 32, 16>(get, 2 * S, Kp, hist, sh);
  if (threadIdx.x == 0 && hi != 0xFFFFFFFFull) atomicMin(gthr + q, (unsigned long long)((hi << 32) | 0xFFFFFFFFull));
}

// flat_seed_threshold2 for S <= 64 splits: lane L loads split L's pair of
// smallest words (0xFFFFFFFF past S) and one wavefront sorts the 128 words
// in registers; the Kp-th smallest (1-based) is sorted element Kp - 1. Same
// value as the radix select over the 2 S words (the padding words are the
// largest possible, and Kp <= 2 S).
__global__ __launch_bounds__(64) void flat_seed_threshold2_wave(const uint64_t* __restrict__ cand, int S, int CAP,
                                                                int Kp, unsigned long long* __restrict__ gthr) {
  const int q = blockIdx.x, lane = threadIdx.x;
  if (2 * S < Kp) return;  // the host launches this with 2 S >= 4 Kp
  uint64_t w[2] = {0xFFFFFFFFull, 0xFFFFFFFFull};
  if (lane < S) {
    const uint64_t pr = cand[((size_t)q * S + lane) * CAP + (CAP - FB_N / 2 - 1)];
    w[0] = pr & 0xFFFFFFFFull;
    w[1] = pr >> 32;
  }
  wave_bitonic_sort<2>(w, lane);
  const int src = (Kp - 1) >> 1;
  const uint64_t mine = ((Kp - 1) & 1) ? w[1] : w[0];
  const uint64_t hi = (uint64_t)(uint32_t)__shfl((int)(uint32_t)mine, src, WAVE);
  if (lane == 0 && hi != 0xFFFFFFFFull) atomicMin(gthr + q, (unsigned long long)((hi << 32) | 0xFFFFFFFFull));
}

constexpr int MERGE_MAXP = 512;

// The certificate of one query's merge. Every candidate outside the
// selection has approx >= approx(pivot), hence exact >= approx(pivot) - eps;
// the k-th exact distance (the high word of `kth`) must be strictly below
// that for the selection to contain the exact top-k.
__device__ inline bool merge_certified(uint64_t pivot, uint64_t kth, int metric, float qnv, float maxnorm, float eps_c,
                                       int dim) {
  const float ak = key_float((uint32_t)(pivot >> 32));
  const float dk = key_float((uint32_t)(kth >> 32));
  float eps;
  if (metric == 0) {
    const float s = qnv + maxnorm;
    eps = eps_c * (float)dim * 5.9604645e-08f * s * s;
  } else {
    eps = eps_c * (float)dim * 5.9604645e-08f * qnv * maxnorm + 2.4e-7f;
  }
  eps += 1e-30f;
  return dk < ak - eps;
}

__global__ __launch_bounds__(256) void flat_merge_rescore(
    const uint64_t* __restrict__ cand, int S, int CAP, int Kp, int k, const float* __restrict__ Qp, int ld, int dim,
    int metric, const float* __restrict__ X, const uint32_t* __restrict__ rank, const uint32_t* __restrict__ rank_slot,
    const uint64_t* __restrict__ ids, const float* __restrict__ qn, float maxnorm, float eps_c,
    uint64_t* __restrict__ out_ids, float* __restrict__ out_d, uint32_t* __restrict__ out_count,
    int* __restrict__ flag_list, int* __restrict__ flag_count, size_t ldo) {
  const int q = blockIdx.x;
  __shared__ int hist[256];
  __shared__ uint64_t sh[4];
  __shared__ uint64_t sel[MERGE_MAXP];
  __shared__ int n_sel;
  __shared__ int n_valid;
  const uint64_t* base = cand + (size_t)q * S * CAP;
  const int n = S * Kp;
  auto get = [&](int i) -> uint64_t { return base[(size_t)(i / Kp) * CAP + (i % Kp)]; };

  if (threadIdx.x == 0) {
    n_valid = 0;
    n_sel = 0;
  }
  __syncthreads();
  int local = 0;
  // eight keys per thread per step, loaded together before any is used
  for (int i0 = threadIdx.x; i0 < n; i0 += 8 * blockDim.x) {
    uint64_t x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = get(min(i0 + u * (int)blockDim.x, n - 1));  // unconditional loads
#pragma unroll
    for (int u = 0; u < 8; ++u) local += (i0 + u * (int)blockDim.x < n && x[u] != KEY_MAX) ? 1 : 0;
  }
  atomicAdd(&n_valid, local);
  __syncthreads();
  const int valid = n_valid;
  const int ksel = min(Kp, valid);
  if (ksel == 0) {
    if (threadIdx.x == 0) out_count[q] = 0;
    return;
  }
  const uint64_t pivot = n <= 16 * (int)blockDim.x ? block_radix_select<decltype(get), 64, 16>(get, n, ksel, hist, sh)
                         : n <= 40 * (int)blockDim.x ? block_radix_select<decltype(get), 64, 40>(get, n, ksel, hist, sh)
                                         : block_radix_select(get, n, ksel, hist, sh);
  for (int i0 = threadIdx.x; i0 < n; i0 += 8 * blockDim.x) {
    uint64_t x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = get(min(i0 + u * (int)blockDim.x, n - 1));  // unconditional loads
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (i0 + u * (int)blockDim.x < n && x[u] <= pivot && x[u] != KEY_MAX) {
        const int p = atomicAdd(&n_sel, 1);
        sel[p] = x[u];
      }
  }
  __syncthreads();
  // rescore: 8 threads per candidate
  const int g = threadIdx.x & 7, grp = threadIdx.x >> 3;
  const float* qv = Qp + (size_t)q * ld;
  for (int c = grp; c < ksel; c += 32) {
    const uint32_t slot = (uint32_t)sel[c];
    const float d = dist_group8_rt(metric, qv, X + (size_t)slot * ld, dim, g);
    if (g == 0) sel[c] = ((uint64_t)ord_key(d) << 32) | rank[slot];
  }
  __syncthreads();
  int P = 1;
  while (P < ksel) P <<= 1;
  for (int i = ksel + threadIdx.x; i < P; i += blockDim.x) sel[i] = KEY_MAX;
  __syncthreads();
  block_bitonic_sort(sel, P);
  const int kout = min(k, ksel);
  for (int i = threadIdx.x; i < kout; i += blockDim.x) {
    const uint64_t key = sel[i];
    const uint32_t slot = rank_slot[(uint32_t)key];
    out_ids[(size_t)q * ldo + i] = ids[slot];
    out_d[(size_t)q * ldo + i] = key_float((uint32_t)(key >> 32));
  }
  if (threadIdx.x == 0) {
    out_count[q] = kout;
    if (valid >= Kp && !merge_certified(pivot, sel[kout - 1], metric, qn[q], maxnorm, eps_c, dim)) {
      const int p = atomicAdd(flag_count, 1);
      flag_list[p] = q;
    }
  }
}

// flat_merge_rescore for a query whose S * Kp keys fit PER per thread of an
// NT-thread block and whose Kp fits one wavefront. Each key is read once into
// registers, and the count, the select and the gather use that copy; one
// wavefront sorts the rescored keys with their slots in registers. Same
// results as the general kernel: the same selection, rescore arithmetic and
// (distance, rank) order.
template <int NT, int PER>
__global__ __launch_bounds__(NT) void flat_merge_rescore_reg(
    const uint64_t* __restrict__ cand, int S, int CAP, int Kp, int k, const float* __restrict__ Qp, int ld, int dim,
    int metric, const float* __restrict__ X, const uint32_t* __restrict__ rank, const uint64_t* __restrict__ ids,
    const float* __restrict__ qn, float maxnorm, float eps_c, uint64_t* __restrict__ out_ids,
    float* __restrict__ out_d, uint32_t* __restrict__ out_count, int* __restrict__ flag_list,
    int* __restrict__ flag_count, size_t ldo) {
  const int q = blockIdx.x;
  const int lane = threadIdx.x & (WAVE - 1);
  __shared__ int hist[256];
  __shared__ uint64_t sh[4];
  __shared__ uint64_t sel[WAVE];
  __shared__ uint64_t rkey[WAVE];
  __shared__ uint32_t rslot[WAVE];
  __shared__ int n_sel;
  __shared__ int n_valid;
  const uint64_t* base = cand + (size_t)q * S * CAP;
  const int n = S * Kp;
  if (threadIdx.x == 0) {
    n_valid = 0;
    n_sel = 0;
  }
  uint64_t x[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = min((int)threadIdx.x + u * NT, n - 1);  // unconditional loads
    x[u] = base[(size_t)(i / Kp) * CAP + i % Kp];
  }
  int wcount = 0;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    if ((int)threadIdx.x + u * NT >= n) x[u] = KEY_MAX;
    wcount += __popcll(__ballot(x[u] != KEY_MAX));
  }
  __syncthreads();  // the counters are set
  if (lane == 0) atomicAdd(&n_valid, wcount);
  __syncthreads();
  const int valid = n_valid;
  const int ksel = min(Kp, valid);
  if (ksel == 0) {
    if (threadIdx.x == 0) out_count[q] = 0;
    return;
  }
  auto each = [&](auto f) {
#pragma unroll
    for (int u = 0; u < PER; ++u)
      if (x[u] != KEY_MAX) f(x[u]);
  };
  const uint64_t pivot = block_radix_select_each<64>(each, ksel, hist, sh);
  // keys are distinct (one per row), so exactly ksel <= WAVE of them are
  // <= pivot (the bound on the write only guards the array)
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (x[u] <= pivot && x[u] != KEY_MAX) {
      const int p = atomicAdd(&n_sel, 1);
      if (p < WAVE) sel[p] = x[u];
    }
  __syncthreads();
  // rescore: 8 threads per candidate
  const int g = threadIdx.x & 7, grp = threadIdx.x >> 3;
  const float* qv = Qp + (size_t)q * ld;
  for (int c = grp; c < ksel; c += NT / 8) {
    const uint32_t slot = (uint32_t)sel[c];
    const float d = dist_group8_rt(metric, qv, X + (size_t)slot * ld, dim, g);
    if (g == 0) {
      rkey[c] = ((uint64_t)ord_key(d) << 32) | rank[slot];
      rslot[c] = slot;
    }
  }
  __syncthreads();
  if (threadIdx.x >= WAVE) return;
  uint64_t key = lane < ksel ? rkey[lane] : KEY_MAX;
  uint32_t slot = lane < ksel ? rslot[lane] : 0;
  wave_sort_kv64(key, slot, lane);
  const int kout = min(k, ksel);
  if (lane < kout) {
    out_ids[(size_t)q * ldo + lane] = ids[slot];
    out_d[(size_t)q * ldo + lane] = key_float((uint32_t)(key >> 32));
  }
  const uint32_t kth_hi = (uint32_t)__shfl((int)(uint32_t)(key >> 32), kout - 1, WAVE);
  if (lane == 0) {
    out_count[q] = kout;
    if (valid >= Kp && !merge_certified(pivot, (uint64_t)kth_hi << 32, metric, qn[q], maxnorm, eps_c, dim)) {
      const int p = atomicAdd(flag_count, 1);
      flag_list[p] = q;
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
// Whether the exact scan is expected to finish nq queries over N rows of dim
// floats sooner than the MFMA candidate path. Both estimates are fitted to
// timings of the two paths at 20k x 128, 100k x 128, 300k x 256, 1M x 96 and
// 1M x 768 with 1 to 128 queries (the crossover, 4 to 50 queries over those
// stores, lands within one measured batch size): the MFMA path costs about
// 0.1 ms of fixed work plus its GEMM, whole 128-query blocks at about 80% of
// the FP32 MFMA peak; the exact scan reads the store from HBM once (about
// 5 TB/s) and streams it through L2 again for every further query (about
// 0.4 ns per 1000 floats).
static bool exact_scan_cheaper(size_t N, size_t dim, size_t nq) {
  const double nd = (double)N * (double)dim;
  const double t_mfma = 1.0e-4 + (double)((nq + 127) / 128) * nd * 256.0 / 1.25e14;
  const double t_exact = 5.0e-5 + nd * 4.0 / 5.0e12 + (double)(nq - 1) * nd * 4.0e-13;
  return t_exact < t_mfma;
}

FlatIndex::~FlatIndex() {
  if (stream) (void)hipStreamDestroy(stream);
}

// Grow the device arrays to hold `need` slots, keeping the first `keep`
// (the high-water mark before the current allocation, never above cap).
void FlatIndex::ensure_capacity(size_t need, size_t keep) {
  if (need <= cap) return;
  size_t nc = std::max<size_t>(need, std::max<size_t>(cap * 2, 1024));
  const size_t hw = std::min(keep, cap);
  X.grow(nc * ld, hw * ld, stream);
  xb.grow(nc, hw, stream);
  d_live.grow(nc, hw, stream);
  d_ids.grow(nc, hw, stream);
  ranks.grow(nc, hw, stream);
  // zero the new tail of the liveness map
  PXG_HIP(hipMemsetAsync(d_live.p + hw, 0, nc - hw, stream));
  PXG_HIP(hipStreamSynchronize(stream));
  cap = nc;
}

void FlatIndex::insert(const uint64_t* in_ids, const float* vecs, uint64_t n, uint32_t* out_slots) {
  // Validate everything first: all-or-nothing.
  std::vector<float> prepared((size_t)n * ld, 0.0f);
  std::vector<float> bias(n);
  float newmax = maxnorm;
  for (uint64_t i = 0; i < n; ++i) {
    long long bad = validate_prepare(metric, vecs + i * dim, dim, prepared.data() + i * ld);
    if (bad >= 0)
      raise(PXG_ERR_NON_FINITE,
            "vector component " + std::to_string(bad) + " is not finite (" + std::to_string(vecs[i * dim + bad]) + ")",
            (uint64_t)bad, i, vecs[i * dim + bad]);
    const float* p = prepared.data() + i * ld;
    float n2 = host_dot_unrolled(p, p, dim);
    bias[i] = metric == PXG_EUCLIDEAN ? n2 : 0.0f;
    float nr = std::sqrt(n2);
    if (!(nr <= newmax)) newmax = std::isnan(nr) ? INFINITY : nr;
  }
  {
    std::unordered_map<uint64_t, int> seen;
    for (uint64_t i = 0; i < n; ++i) {
      if (by_id.count(in_ids[i]) || !seen.emplace(in_ids[i], 1).second)
        raise(PXG_ERR_DUPLICATE_ID, "duplicate vector id " + std::to_string(in_ids[i]), in_ids[i]);
    }
  }
  if (by_id.size() + n > (size_t)UINT32_MAX - 1)
    capacity_error("slot allocator", UINT32_MAX, "capacity exceeded: slot allocator limit is 4294967295");
  std::vector<uint32_t> sl(n);
  const size_t old_hw = slots.high_water();
  // Allocate in order, exactly as repeated VectorStore::insert would.
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
  maxnorm = newmax;
  // stage and scatter in chunks of <= 64 MiB of rows
  const size_t rows_per = std::max<size_t>(1, (64u << 20) / ((size_t)ld * 4));
  DevBuf<float> st_rows(std::min<size_t>(rows_per, n) * ld);
  DevBuf<uint32_t> st_slots(std::min<size_t>(rows_per, n));
  DevBuf<float> st_bias(std::min<size_t>(rows_per, n));
  DevBuf<uint64_t> st_ids(std::min<size_t>(rows_per, n));
  for (size_t a = 0; a < n; a += rows_per) {
    const size_t m = std::min<size_t>(rows_per, n - a);
    PXG_HIP(hipMemcpyAsync(st_rows.p, prepared.data() + a * ld, m * ld * 4, hipMemcpyHostToDevice, stream));
    PXG_HIP(hipMemcpyAsync(st_slots.p, sl.data() + a, m * 4, hipMemcpyHostToDevice, stream));
    PXG_HIP(hipMemcpyAsync(st_bias.p, bias.data() + a, m * 4, hipMemcpyHostToDevice, stream));
    PXG_HIP(hipMemcpyAsync(st_ids.p, in_ids + a, m * 8, hipMemcpyHostToDevice, stream));
    hipLaunchKernelGGL(flat_scatter_rows, dim3((unsigned)m), dim3(256), 0, stream, st_rows.p, st_slots.p,
                       st_bias.p, st_ids.p, (int)m, (int)ld, X.p, xb.p, d_live.p, d_ids.p);
    PXG_HIP(hipGetLastError());
    PXG_HIP(hipStreamSynchronize(stream));
  }
  ranks.insert(in_ids, sl.data(), n, d_ids.p, stream);
}

void FlatIndex::remove(uint64_t id) {
  auto it = by_id.find(id);
  if (it == by_id.end()) raise(PXG_ERR_UNKNOWN_ID, "unknown vector id " + std::to_string(id), id);
  const uint32_t s = it->second;
  by_id.erase(it);
  live[s] = 0;
  slots.release(s);
  PXG_HIP(hipMemsetAsync(d_live.p + s, 0, 1, stream));
  ranks.remove(s, stream);
  PXG_HIP(hipStreamSynchronize(stream));
}

// Run the search pipeline on prepared-or-raw device queries.
void check_query_flags(const unsigned long long* words) {
  const unsigned long long badv = words[0];
  if (badv != ~0ull) {
    const uint32_t qi = (uint32_t)(badv >> 32), comp = (uint32_t)badv;
    raise(PXG_ERR_NON_FINITE,
          "vector component " + std::to_string(comp) + " is not finite (query " + std::to_string(qi) + ")", comp,
          qi, NAN);
  }
}

void FlatIndex::search_device(const float* d_raw, bool do_prepare, uint64_t nq, uint64_t k, const uint8_t* d_accept,
                              uint64_t* d_oid, float* d_od, uint32_t* d_oc, Scratch& sc, hipStream_t s,
                              uint64_t* fallbacks, size_t ldo, bool* deferred) {
  if (deferred) *deferred = false;
  check_k(k);
  *fallbacks = 0;
  if (nq == 0) return;
  const size_t N = slots.high_water();
  // A search returns at most the live count per query, so k is clamped to it
  // before any path is chosen.
  const uint64_t kq = std::min<uint64_t>(k, by_id.size());

  Timer tm(s);
  tm.on = tm.on && sc.timing();
  tm.mark(0);
  // 1. prepare queries; a non-finite query fails the call whatever k is
  // (space.rs:104-121 runs before the scan, flat.rs:153-155)
  float* Qp = (float*)sc.get(1, nq * ld * 4);
  float* qb = (float*)sc.get(2, nq * 4);
  float* qn = (float*)sc.get(3, nq * 4);
  unsigned long long* bad = (unsigned long long*)sc.get(4, 8 + 8);
  int* flag_count = (int*)(bad + 1);
  int* grp_count = flag_count + 1;
  // per query, the least threshold any split has published (MFMA path),
  // cleared by the preparation kernel
  unsigned long long* gthr = (unsigned long long*)sc.get(25, nq * 8);
  hipLaunchKernelGGL(init_search_flags, dim3(1), dim3(64), 0, s, bad, flag_count);
  hipLaunchKernelGGL(flat_prep_search_queries, dim3((unsigned)nq), dim3(64), 0, s, d_raw, (int)dim, (int)ld, metric,
                     do_prepare ? 1 : 0, Qp, qb, qn, bad, gthr);
  PXG_HIP(hipGetLastError());
  unsigned long long* tail = sc.host_words();
  auto read_flags = [&](int* nflag) {
    PXG_HIP(hipMemcpyAsync(tail, bad, 16, hipMemcpyDeviceToHost, s));
    PXG_HIP(hipStreamSynchronize(s));
    if (nflag) std::memcpy(nflag, &tail[1], sizeof(int));
    check_query_flags(tail);
  };
  if (kq == 0) {
    hipLaunchKernelGGL(fill_u32, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, d_oc, (size_t)nq, 0u);
    PXG_HIP(hipGetLastError());
    read_flags(nullptr);
    return;
  }
  if (kq > EXACT_MERGE_MAXK) {
    search_wide(Qp, nq, kq, d_accept, d_oid, d_od, d_oc, sc, s, ldo);
    read_flags(nullptr);
    tm.finish();
    return;
  }

  int* flag_list = (int*)sc.get(5, nq * 4);
  // Manhattan has no inner-product form and k beyond FAST_KMAX exceeds the
  // candidate buffers: both take the exact scan, as do stores under 4096
  // rows and batches the exact scan finishes sooner.
  const bool exact_all = mode == 2 || metric == PXG_MANHATTAN || kq > FAST_KMAX ||
                         (mode == 0 && (N < 4096 || exact_scan_cheaper(N, dim, nq)));
  if (!exact_all) {
    const int Kp = (int)std::min<uint64_t>(kq + MARGIN, (uint64_t)FAST_KMAX + MARGIN);
    // a row's buffer holds its Kp keys, one tile's appends (FB_N) and at
    // least 64 more before it must be compacted
    const int CAP = (Kp + FB_N + 64) <= 256 ? 256 : 512;
    const int QB = (int)((nq + FB_M - 1) / FB_M);
    const int tiles = (int)((N + FB_N - 1) / FB_N);
    int S = std::max(1, std::min(512 / QB, std::max(1, tiles / 4)));
    // a fixed scratch may hold fewer splits (the results do not depend on S)
    const size_t per_split_bytes = (size_t)nq * CAP * 8;
    const size_t fit = sc.room() / per_split_bytes;
    if (fit == 0) (void)sc.get(6, per_split_bytes);  // raises the capacity error
    S = (int)std::min<size_t>((size_t)S, fit);
    const int tiles_per = (tiles + S - 1) / S;
    const int per_split = tiles_per * FB_N;
    S = (int)((N + per_split - 1) / per_split);
    uint64_t* cand = (uint64_t*)sc.get(6, (size_t)nq * S * CAP * 8);
    const int total = QB * S;
    tm.mark(1);
    const int grid = ((total + 7) / 8) * 8;
    const float scale = metric == PXG_EUCLIDEAN ? 2.0f : 1.0f;
    // A first pass over the first tile of each split (spread over the whole
    // store) seeds each query's threshold with the Kp-th best of those rows,
    // so the full pass appends and compacts little from its first tile on
    // (unseeded, every row would append its split's first two tiles whole
    // and compact them); the full pass then filters that tile's stored keys
    // instead of computing it again. The seed needs at least Kp words per
    // query: S tiles of FB_N.
    const int seeded = (size_t)S * FB_N >= (size_t)Kp ? 1 : 0;
    auto candidates = [&](auto seed) {
      constexpr bool SD = decltype(seed)::value;
      if (CAP == 256)
        hipLaunchKernelGGL((flat_mfma_candidates<256, SD>), dim3(grid), dim3(256), 0, s, Qp, (int)nq, X.p, (int)N,
                           (int)ld, qb, xb.p, scale, d_live.p, d_accept, S, QB, per_split, Kp, cand, gthr, seeded);
      else
        hipLaunchKernelGGL((flat_mfma_candidates<512, SD>), dim3(grid), dim3(256), 0, s, Qp, (int)nq, X.p, (int)N,
                           (int)ld, qb, xb.p, scale, d_live.p, d_accept, S, QB, per_split, Kp, cand, gthr, seeded);
      PXG_HIP(hipGetLastError());
    };
    if (seeded) {
      candidates(std::true_type{});
      // the splits' pairs when they are many against Kp (and fit the
      // select's 16 words per thread), else every seeding word
      if (2 * S >= 4 * Kp && S <= WAVE)
        hipLaunchKernelGGL(flat_seed_threshold2_wave, dim3((unsigned)nq), dim3(64), 0, s, (const uint64_t*)cand, S,
                           CAP, Kp, gthr);
      else if (2 * S >= 4 * Kp && 2 * S <= 16 * 64)
        hipLaunchKernelGGL(flat_seed_threshold2, dim3((unsigned)nq), dim3(64), 0, s, (const uint64_t*)cand, S, CAP,
                           Kp, gthr);
      else
        hipLaunchKernelGGL(flat_seed_threshold, dim3((unsigned)nq), dim3(512), 0, s, (const uint64_t*)cand, S, CAP,
                           Kp, gthr);
      PXG_HIP(hipGetLastError());
    }
    candidates(std::false_type{});
    tm.mark(2);
    const size_t nkeys = (size_t)S * Kp;
    if (nkeys <= 8 * 256 && Kp <= WAVE)
      hipLaunchKernelGGL((flat_merge_rescore_reg<256, 8>), dim3((unsigned)nq), dim3(256), 0, s, cand, S, CAP, Kp,
                         (int)kq, Qp, (int)ld, (int)dim, metric, X.p, ranks.rank.p, d_ids.p, qn, maxnorm, 4.0f, d_oid,
                         d_od, d_oc, flag_list, flag_count, ldo);
    else if (nkeys <= 16 * 1024 && Kp <= WAVE)
      hipLaunchKernelGGL((flat_merge_rescore_reg<1024, 16>), dim3((unsigned)nq), dim3(1024), 0, s, cand, S, CAP, Kp,
                         (int)kq, Qp, (int)ld, (int)dim, metric, X.p, ranks.rank.p, d_ids.p, qn, maxnorm, 4.0f, d_oid,
                         d_od, d_oc, flag_list, flag_count, ldo);
    else
      hipLaunchKernelGGL(flat_merge_rescore, dim3((unsigned)nq), dim3(256), 0, s, cand, S, CAP, Kp, (int)kq, Qp,
                         (int)ld, (int)dim, metric, X.p, ranks.rank.p, ranks.rank_slot.p, d_ids.p, qn, maxnorm, 4.0f,
                         d_oid, d_od, d_oc, flag_list, flag_count, ldo);
    PXG_HIP(hipGetLastError());
  } else {
    hipLaunchKernelGGL(iota_kernel, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, flag_list, (int)nq,
                       flag_count);
    PXG_HIP(hipGetLastError());
  }
  // exact scan for flagged queries (all of them on the exact path, where the
  // count is known here and the flags are read once, with the results)
  int nflag = 0;
  if (exact_all)
    nflag = (int)nq;
  else
    read_flags(&nflag);
  if (nflag > 0) {
    sc.release_from(6);  // the candidate buffers are dead
    const int QG = exact_query_group((size_t)nflag, dim, N);
    const int CH = exact_chunk_rows(((size_t)nflag + QG - 1) / QG, N);
    const int nchunks = (int)((N + CH - 1) / CH);
    const int kk = (int)std::min<uint64_t>(kq, (uint64_t)CH);
    const size_t per_query = (size_t)nchunks * kk * 8;
    size_t fit = sc.room() / per_query;
    if (fit == 0) {
      if (exact_all) read_flags(nullptr);  // a non-finite query is reported first
      (void)sc.get(7, per_query);          // raises the capacity error
    }
    const int G = (int)std::min<size_t>((size_t)nflag, fit);
    uint64_t* ecand = (uint64_t*)sc.get(7, (size_t)G * per_query);
    tm.mark(exact_all ? 1 : 3);
    for (int g0 = 0; g0 < nflag; g0 += G) {
      const int gn = std::min(G, nflag - g0);
      const int* count = flag_count;
      if (gn != nflag) {  // a fixed scratch takes the flagged queries in groups
        hipLaunchKernelGGL(set_int, dim3(1), dim3(64), 0, s, grp_count, gn);
        count = grp_count;
      }
#define PXG_EXACT_SCAN(CHV, QGV)                                                                              \
  hipLaunchKernelGGL((flat_exact_candidates<CHV, QGV>), dim3((std::min((gn + QGV - 1) / QGV * nchunks, 4096) + 7) / 8 * 8), \
                     dim3(256), 0, s, flag_list + g0, count, nchunks, Qp, (int)ld, (int)dim, metric, X.p, (int)N,       \
                     d_live.p, d_accept, ranks.rank.p, (int)kq, ecand)
#define PXG_EXACT_MERGE(CHV)                                                                                  \
  hipLaunchKernelGGL(flat_merge_exact<CHV>, dim3((unsigned)gn), dim3(256), 0, s, flag_list + g0, count, ecand, \
                     nchunks, (int)kq, ranks.rank_slot.p, d_ids.p, d_oid, d_od, d_oc, (uint64_t*)nullptr, ldo)
      if (CH == 256) {
        if (QG == 4) PXG_EXACT_SCAN(256, 4); else PXG_EXACT_SCAN(256, 1);
      } else {
        if (QG == 4) PXG_EXACT_SCAN(EXACT_CH, 4); else PXG_EXACT_SCAN(EXACT_CH, 1);
      }
      PXG_HIP(hipGetLastError());
      if (exact_all && g0 == 0) tm.mark(2);
      if (CH == 256) PXG_EXACT_MERGE(256); else PXG_EXACT_MERGE(EXACT_CH);
#undef PXG_EXACT_SCAN
#undef PXG_EXACT_MERGE
      PXG_HIP(hipGetLastError());
    }
    if (exact_all && deferred) {
      // the caller waits once, for this copy and its own result copies
      PXG_HIP(hipMemcpyAsync(tail, bad, 16, hipMemcpyDeviceToHost, s));
      *deferred = true;
    } else if (exact_all) {
      read_flags(nullptr);  // waits for the results; a non-finite query fails the call
    } else {
      PXG_HIP(hipStreamSynchronize(s));
    }
    *fallbacks = exact_all ? 0 : (uint64_t)nflag;
  }
  tm.finish();
}

// k beyond the block selections: exact keys of every slot per query, a
// segmented radix sort, the first kq of each segment.
void FlatIndex::search_wide(const float* Qp, uint64_t nq, uint64_t kq, const uint8_t* d_accept, uint64_t* d_oid,
                            float* d_od, uint32_t* d_oc, Scratch& sc, hipStream_t s, size_t ldo) {
  exact_wide_search(Qp, (int)ld, (int)dim, metric, nq, kq, X.p, slots.high_water(), d_live.p, d_accept, ranks.rank.p,
                    ranks.rank_slot.p, d_ids.p, d_oid, d_od, d_oc, ldo, sc, s);
}

// Insert from device memory: validate + prepare on the device, then the
// same slot allocation and scatter as insert().
void FlatIndex::insert_device(const uint64_t* in_ids, const float* d_vecs, uint64_t n, uint32_t* out_slots) {
  {
    std::unordered_map<uint64_t, int> seen;
    for (uint64_t i = 0; i < n; ++i)
      if (by_id.count(in_ids[i]) || !seen.emplace(in_ids[i], 1).second)
        raise(PXG_ERR_DUPLICATE_ID, "duplicate vector id " + std::to_string(in_ids[i]), in_ids[i]);
  }
  if (by_id.size() + n > (size_t)UINT32_MAX - 1)
    capacity_error("slot allocator", UINT32_MAX, "capacity exceeded: slot allocator limit is 4294967295");
  const size_t rows_per = std::max<size_t>(1, (256u << 20) / ((size_t)ld * 4));
  const size_t chunk = std::min<size_t>(rows_per, n);
  DevBuf<float> st_rows(chunk * ld);
  DevBuf<float> st_b(chunk), st_n(chunk);
  DevBuf<unsigned long long> bad(1);
  // pass 1: validate every row before touching any state (all-or-nothing)
  std::vector<float> norms(n);
  for (size_t a = 0; a < n; a += chunk) {
    const size_t m = std::min<size_t>(chunk, n - a);
    PXG_HIP(hipMemsetAsync(bad.p, 0xFF, 8, stream));
    hipLaunchKernelGGL(flat_prep_queries, dim3((unsigned)m), dim3(64), 0, stream, d_vecs + a * dim, (int)dim,
                       (int)ld, metric, 1, st_rows.p, st_b.p, st_n.p, bad.p);
    PXG_HIP(hipGetLastError());
    unsigned long long bv = 0;
    PXG_HIP(hipMemcpyAsync(&bv, bad.p, 8, hipMemcpyDeviceToHost, stream));
    PXG_HIP(hipMemcpyAsync(norms.data() + a, st_n.p, m * 4, hipMemcpyDeviceToHost, stream));
    PXG_HIP(hipStreamSynchronize(stream));
    if (bv != ~0ull) {
      const uint64_t row = a + (bv >> 32), comp = (uint32_t)bv;
      raise(PXG_ERR_NON_FINITE, "vector component " + std::to_string(comp) + " is not finite (vector " +
                                    std::to_string(row) + ")",
            comp, row, NAN);
    }
  }
  float newmax = maxnorm;
  for (float nr : norms)
    if (!(nr <= newmax)) newmax = std::isnan(nr) ? INFINITY : nr;
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
  maxnorm = newmax;
  DevBuf<uint32_t> st_slots(chunk);
  DevBuf<uint64_t> st_ids(chunk);
  DevBuf<float> st_bias(chunk);
  for (size_t a = 0; a < n; a += chunk) {
    const size_t m = std::min<size_t>(chunk, n - a);
    hipLaunchKernelGGL(flat_prep_queries, dim3((unsigned)m), dim3(64), 0, stream, d_vecs + a * dim, (int)dim,
                       (int)ld, metric, 1, st_rows.p, st_b.p, st_n.p, bad.p);
    PXG_HIP(hipGetLastError());
    // bias: |x|^2 for Euclidean (st_b holds it), 0 otherwise
    if (metric == PXG_EUCLIDEAN)
      PXG_HIP(hipMemcpyAsync(st_bias.p, st_b.p, m * 4, hipMemcpyDeviceToDevice, stream));
    else
      PXG_HIP(hipMemsetAsync(st_bias.p, 0, m * 4, stream));
    PXG_HIP(hipMemcpyAsync(st_slots.p, sl.data() + a, m * 4, hipMemcpyHostToDevice, stream));
    PXG_HIP(hipMemcpyAsync(st_ids.p, in_ids + a, m * 8, hipMemcpyHostToDevice, stream));
    hipLaunchKernelGGL(flat_scatter_rows, dim3((unsigned)m), dim3(256), 0, stream, st_rows.p, st_slots.p,
                       st_bias.p, st_ids.p, (int)m, (int)ld, X.p, xb.p, d_live.p, d_ids.p);
    PXG_HIP(hipGetLastError());
    PXG_HIP(hipStreamSynchronize(stream));
  }
  ranks.insert(in_ids, sl.data(), n, d_ids.p, stream);
}

thread_local uint64_t g_last_fallbacks = 0;
void set_last_fallbacks(uint64_t v) { g_last_fallbacks = v; }


}  // namespace pxg

using pxg::FlatIndex;


extern "C" {

int pxg_flat_create(uint32_t dim, int metric, uint64_t capacity, pxg_flat** out) {
  return pxg::guard([&] {
    if (!out) pxg::config_error("out", 0, "must not be NULL");
    if (dim < 1) pxg::config_error("dim", dim, "must be at least 1; a 0-dimensional space makes all distances equal");
    if (dim > (1u << 20)) pxg::config_error("dim", dim, "exceeds the 1048576 dimension ceiling");
    if (metric < 0 || metric > 3) pxg::config_error("metric", (uint64_t)metric, "unknown metric");
    auto* h = new pxg_flat();
    FlatIndex& f = h->impl;
    f.dim = dim;
    f.ld = (dim + 3) & ~3u;
    f.metric = metric;
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

void pxg_flat_destroy(pxg_flat* index) { delete index; }

int pxg_flat_insert(pxg_flat* index, const uint64_t* ids, const float* vectors, uint64_t n, uint32_t* out_slots) {
  return pxg::guard([&] {
    if (n == 0) return;
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    index->impl.insert(ids, vectors, n, out_slots);
  });
}

int pxg_flat_insert_device(pxg_flat* index, const uint64_t* ids, const float* d_vectors, uint64_t n,
                           uint32_t* out_slots) {
  return pxg::guard([&] {
    if (n == 0) return;
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    index->impl.insert_device(ids, d_vectors, n, out_slots);
  });
}

int pxg_flat_remove(pxg_flat* index, uint64_t id) {
  return pxg::guard([&] {
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    index->impl.remove(id);
  });
}

int pxg_flat_contains(const pxg_flat* index, uint64_t id) {
  std::shared_lock<std::shared_mutex> lk(index->impl.mu);
  return index->impl.by_id.count(id) ? 1 : 0;
}

uint64_t pxg_flat_len(const pxg_flat* index) {
  std::shared_lock<std::shared_mutex> lk(index->impl.mu);
  return index->impl.by_id.size();
}

int pxg_flat_stats(const pxg_flat* index, pxg_index_stats* out) {
  return pxg::guard([&] {
    std::shared_lock<std::shared_mutex> lk(index->impl.mu);
    const FlatIndex& f = index->impl;
    out->len = f.by_id.size();
    out->deleted = 0;  // slots are freed on delete: no tombstones
    out->dim = f.dim;
    out->metric = f.metric;
    out->layers = 1;
    out->edges = 0;
    out->vector_bytes = f.X.bytes();
    out->graph_bytes = 0;
  });
}

int pxg_flat_get_vector(const pxg_flat* index, uint64_t id, float* out) {
  return pxg::guard([&] {
    std::shared_lock<std::shared_mutex> lk(index->impl.mu);
    const FlatIndex& f = index->impl;
    auto it = f.by_id.find(id);
    if (it == f.by_id.end()) pxg::raise(PXG_ERR_UNKNOWN_ID, "unknown vector id " + std::to_string(id), id);
    PXG_HIP(hipMemcpy(out, f.X.p + (size_t)it->second * f.ld, f.dim * 4, hipMemcpyDeviceToHost));
  });
}

uint64_t pxg_flat_slot_count(const pxg_flat* index) {
  std::shared_lock<std::shared_mutex> lk(index->impl.mu);
  return index->impl.slots.high_water();
}

int pxg_flat_slots(const pxg_flat* index, uint64_t* ids, uint8_t* live) {
  return pxg::guard([&] {
    std::shared_lock<std::shared_mutex> lk(index->impl.mu);
    const FlatIndex& f = index->impl;
    const size_t hw = f.slots.high_water();
    for (size_t s = 0; s < hw; ++s) {
      if (ids) ids[s] = f.live[s] ? f.ids[s] : 0;
      if (live) live[s] = f.live[s];
    }
  });
}

int pxg_flat_search(const pxg_flat* index, const float* queries, uint64_t nq, uint64_t k, const uint8_t* accept,
                    uint64_t* out_ids, float* out_dist, uint32_t* out_count) {
  return pxg::guard([&] {
    pxg::check_k(k);
    FlatIndex& f = const_cast<FlatIndex&>(index->impl);
    std::shared_lock<std::shared_mutex> lk(f.mu);
    if (nq == 0) return;
    // validate + prepare on the host (space.rs:130-138)
    std::vector<float> prep((size_t)nq * f.dim);
    for (uint64_t i = 0; i < nq; ++i) {
      long long bad = pxg::validate_prepare(f.metric, queries + i * f.dim, f.dim, prep.data() + i * f.dim);
      if (bad >= 0)
        pxg::raise(PXG_ERR_NON_FINITE,
                   "vector component " + std::to_string(bad) + " is not finite (" +
                       std::to_string(queries[i * f.dim + bad]) + ")",
                   (uint64_t)bad, i, queries[i * f.dim + bad]);
    }
    // at most the live count per query: device rows of kq, copied into the
    // caller's rows of k
    const uint64_t kq = std::min<uint64_t>(k, f.by_id.size());
    if (kq == 0) {
      for (uint64_t i = 0; i < nq; ++i) out_count[i] = 0;
      return;
    }
    pxg::CtxLease ctx(f.pool);
    pxg::CtxScratch sc(ctx.c);
    hipStream_t s = ctx->stream;
    const size_t N = f.slots.high_water();
    float* d_q = (float*)ctx->get(20, prep.size() * 4);
    uint8_t* d_acc = nullptr;
    if (accept) {
      d_acc = ctx->get(21, N);
      PXG_HIP(hipMemcpyAsync(d_acc, accept, N, hipMemcpyHostToDevice, s));
    }
    uint64_t* d_oid = (uint64_t*)ctx->get(22, nq * kq * 8);
    float* d_od = (float*)ctx->get(23, nq * kq * 4);
    uint32_t* d_oc = (uint32_t*)ctx->get(24, nq * 4);
    PXG_HIP(hipMemcpyAsync(d_q, prep.data(), prep.size() * 4, hipMemcpyHostToDevice, s));
    uint64_t fb = 0;
    bool deferred = false;
    f.search_device(d_q, false, nq, kq, d_acc, d_oid, d_od, d_oc, sc, s, &fb, kq, &deferred);
    pxg::results_to_host(*ctx.c, s, nq, k, kq, kq, d_oid, d_od, d_oc, out_ids, out_dist, out_count, [&] {
      if (deferred) pxg::check_query_flags(sc.host_words());
    });
    pxg::g_last_fallbacks = fb;
  });
}

int pxg_flat_search_device(const pxg_flat* index, const float* d_queries, uint64_t nq, uint64_t k,
                           const uint8_t* d_accept, uint64_t* d_out_ids, float* d_out_dist, uint32_t* d_out_count,
                           void* stream) {
  return pxg::guard([&] {
    pxg::check_k(k);  // first, as flat.rs:153-155
    FlatIndex& f = const_cast<FlatIndex&>(index->impl);
    std::shared_lock<std::shared_mutex> lk(f.mu);
    pxg::CtxLease ctx(f.pool);
    pxg::CtxScratch sc(ctx.c);
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    pxg::DrainOnUnwind drain{s};
    uint64_t fb = 0;
    f.search_device(d_queries, true, nq, k, d_accept, d_out_ids, d_out_dist, d_out_count, sc, s, &fb, k);
    PXG_HIP(hipStreamSynchronize(s));
    pxg::g_last_fallbacks = fb;
  });
}

uint64_t pxg_flat_last_fallbacks(void) { return pxg::g_last_fallbacks; }

int pxg_flat_set_search_mode(pxg_flat* index, int mode) {
  return pxg::guard([&] {
    if (mode < 0 || mode > 2) pxg::config_error("mode", (uint64_t)mode, "0 = auto, 1 = MFMA candidates, 2 = exact scan");
    std::unique_lock<std::shared_mutex> lk(index->impl.mu);
    index->impl.mode = mode;
  });
}

}  // extern "C"
