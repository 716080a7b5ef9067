// Device-side training and encoding used by the IVF-PQ index and the k-means /
// PQ entry points: Lloyd's k-means with k-means++ seeding
// (crates/proxima-quantize/src/kmeans.rs), product-quantizer training and
// encoding (product.rs:198-380), and nearest-centroid assignment with either
// of the reference's two L2 kernels (k-means' sequential `squared`,
// kmeans.rs:234-241; IVF's 8-lane unrolled one, ivfpq.rs:1231-1249).
#pragma once

#include <vector>

#include "common.hpp"
#include "rng.hpp"

namespace pxg {

// PQ layout (product.rs:226-238): widths d/M, remainder spread over the
// leading subspaces; codebook s holds 256 rows of width_s floats at book_off[s].
struct PqLayout {
  int M = 0;
  std::vector<int> width, off, book_off;
  void build(int dim, int m) {
    M = m;
    width.assign(m, 0);
    off.assign(m + 1, 0);
    book_off.assign(m + 1, 0);
    int base = dim / m, rem = dim % m, cur = 0, bcur = 0;
    for (int s = 0; s < m; ++s) {
      width[s] = base + (s < rem ? 1 : 0);
      off[s] = cur;
      book_off[s] = bcur;
      cur += width[s];
      bcur += width[s] * 256;
    }
    off[m] = cur;
    book_off[m] = bcur;
  }
  int book_floats() const { return book_off[M]; }
};

struct KmeansOut {
  size_t k = 0;
  double inertia = 0.0;
  size_t iterations = 0;
  size_t inexact_sums = 0;  // f64 sums kept in the fixed parallel order
};

// Nearest centroid for points P[rows ? rows[i] : i] (first dim columns of rows
// of stride ldp) among C[k][ldc]: best = 0, best_d = +inf, strict <, in
// centroid order. unrolled selects the 8-lane kernel, else the sequential one.
void nearest_device(const float* P, int ldp, const uint32_t* rows, size_t n, int dim, const float* C, int ldc,
                    size_t k, bool unrolled, uint32_t* assign, float* dist, hipStream_t s);

// Scratch of the MFMA assignment, kept across calls on one stream. Without a
// row list and with the same P, ldp, dim and n as the call that computed
// them, the point norms are reused: the caller promises the points did not
// change in between.
struct NearestWork {
  DevBuf<float> pn, cn, cmax, best, second, rd;
  DevBuf<uint32_t> bidx, redo, rrows, ra;
  DevBuf<int> nredo;
  const float* pn_of = nullptr;
  int pn_ld = 0, pn_dim = 0;
  size_t pn_n = 0;
};
void nearest_device(const float* P, int ldp, const uint32_t* rows, size_t n, int dim, const float* C, int ldc,
                    size_t k, bool unrolled, uint32_t* assign, float* dist, hipStream_t s, NearestWork* ws);

// kmeans(): Lloyd from k-means++ seeds drawn from `rng` (or from `init`, k*dim
// dense device floats), points P[n][ldp]. Writes k*dim dense centroids.
KmeansOut kmeans_device(const float* P, size_t n, int dim, int ldp, size_t k, size_t max_iter, ChaCha8* rng,
                        const float* init, DevBuf<float>& cents, DevBuf<uint32_t>* assign_out, hipStream_t s);

// k-means++ seeding alone (kmeans.rs:146-194): k*dim dense device centroids;
// `rng` continues from the state the device rounds left. Returns the number
// of rounds whose f64 sums could not be proven equal to the sequential ones
// (above 2^17 points only; 0 otherwise).
size_t kmeans_pp_device(const float* P, size_t n, int dim, int ldp, size_t k, ChaCha8& rng, float* cents,
                        hipStream_t s);

// ProductQuantizer::train on device rows R[n][ldr]: one ChaCha8(seed) advanced
// across subspaces, 256 centroids each, padded with the last centroid.
void pq_train_device(const float* R, size_t n, int dim, int ldr, const PqLayout& L, size_t max_iter, uint64_t seed,
                     float* d_books, double* inertia, size_t* iterations, hipStream_t s);

// PQ codes of the residual P[row] - C[assign[i]] (or of P[row] itself when C
// is NULL); codes written at out[row * M].
void pq_encode_device(const float* P, int ldp, const uint32_t* rows, size_t n, int dim, const float* C, int ldc,
                      const uint32_t* assign, const float* books, const PqLayout& L, uint8_t* out, hipStream_t s);

}  // namespace pxg
