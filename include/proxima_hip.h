/*
 * libproxima_hip: the MI355X (gfx950) data-parallel nearest-neighbour hot
 * path of Liona-orph/proxima behind a plain C ABI.
 *
 * The reference's drop-in boundary is the `VectorIndex` trait
 * (crates/proxima-index/src/index.rs:154-205): insert / remove / search /
 * contains / len / stats. Each index type below exports exactly that surface
 * as `pxg_<index>_*` functions on an opaque handle, plus a batched search
 * that the single-query trait method is a batch of one of, and a
 * device-pointer search for callers whose queries are already in HBM.
 *
 * Conventions
 *   - Every function returns a pxg_status (0 = ok). The message and the
 *     structured fields of the last error on the calling thread are available
 *     from pxg_last_error_message() / pxg_last_error_detail(). No C++
 *     exception crosses this boundary.
 *   - Host pointers unless the name ends in _device. Output buffers are
 *     caller-allocated: ids[nq*k], dist[nq*k], count[nq].
 *   - Vectors are validated (length implicit in dim; every component finite)
 *     and, for the cosine metric, normalised with the reference's
 *     normalize_in_place (distance.rs:508-517) before they reach the device.
 *   - Results are ranking scores (index.rs:136-149): squared L2, 1 - dot for
 *     prepared cosine, -dot for inner product; nearest first, ties broken by
 *     id, at most k per query; `count` says how many.
 *   - search on one handle is re-entrant from many host threads; insert,
 *     remove, train and load are exclusive (the trait takes &mut self).
 */
#ifndef PROXIMA_HIP_H
#define PROXIMA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: one per ProximaError variant (crates/proxima-core/src/error.rs:37-160). */
typedef enum pxg_status {
  PXG_OK = 0,
  PXG_ERR_DIMENSION_MISMATCH = 1, /* detail a = expected, b = actual */
  PXG_ERR_UNKNOWN_ID = 2,         /* detail a = id */
  PXG_ERR_DUPLICATE_ID = 3,       /* detail a = id */
  PXG_ERR_CAPACITY = 4,           /* detail a = limit */
  PXG_ERR_NON_FINITE = 5,         /* detail a = component index, b = vector index in the batch, value */
  PXG_ERR_CORRUPTION = 6,
  PXG_ERR_CONFIGURATION = 7,      /* detail a = offending value */
  PXG_ERR_INTERNAL = 8            /* device or runtime failure */
} pxg_status;

/* Metric: crates/proxima-core/src/distance.rs:90-118 (declaration order). */
typedef enum pxg_metric {
  PXG_EUCLIDEAN = 0,
  PXG_COSINE = 1,
  PXG_INNER_PRODUCT = 2,
  PXG_MANHATTAN = 3
} pxg_metric;

/* IndexStats: crates/proxima-index/src/index.rs:68-130 (nodes_per_layer is
 * [len] for every index here, so it is not a separate field). */
typedef struct pxg_index_stats {
  uint64_t len;
  uint64_t deleted;
  uint32_t dim;
  int32_t metric;
  uint64_t layers;
  uint64_t edges;
  uint64_t vector_bytes; /* device bytes of the full-precision store */
  uint64_t graph_bytes;  /* device bytes of codes, lists, codebooks */
} pxg_index_stats;

/* Thread-local description of the last error on this thread ("" if none). */
const char* pxg_last_error_message(void);
/* Structured fields of the last error; returns its status. Any pointer may be NULL. */
int pxg_last_error_detail(uint64_t* a, uint64_t* b, float* value);
/* PXG_ERR_CONFIGURATION: the parameter's name, as the reference's
 * Configuration{parameter} spells it ("k", "nprobe", "subspaces", ...);
 * PXG_ERR_CAPACITY: the structure that ran out of room, as Capacity{what}
 * ("slot allocator", "device memory", ...). "" for other errors. The pointer
 * is to static storage and stays valid for the life of the process. */
const char* pxg_last_error_parameter(void);
/* PXG_ERR_CONFIGURATION: the constraint that was broken, as the reference's
 * Configuration{reason}; "" otherwise. Static storage, as above. */
const char* pxg_last_error_reason(void);
/* Library version string. */
const char* pxg_version(void);
/* Number of visible devices (0 when none); never fails. */
int pxg_device_count(void);

/* Device timings of the last search/train call on the calling thread, in
 * milliseconds, measured with hipEvents on the stream the kernels ran on.
 * Recorded only while profiling is enabled (it adds event records, no
 * extra synchronisation). No reference counterpart: measurement hook. */
typedef struct pxg_timings {
  float prep_ms;       /* query validation / preparation */
  float candidates_ms; /* dominant kernel: MFMA candidate GEMM, ADC scan, ... */
  float merge_ms;      /* merge, exact rescoring, final ordering */
  float fallback_ms;   /* exact rescans of unproven queries (0 if none) */
  float total_ms;      /* first to last recorded event */
} pxg_timings;
void pxg_set_profiling(int enabled);
int pxg_last_timings(pxg_timings* out);

/* ------------------------------------------------------------------------ */
/* Flat (exact) index: replaces FlatIndex, crates/proxima-index/src/flat.rs:68-236. */
typedef struct pxg_flat pxg_flat;

/* FlatIndex::new / with_capacity (flat.rs:72-84) over VectorSpace::new (space.rs:71-92). */
int pxg_flat_create(uint32_t dim, int metric, uint64_t capacity, pxg_flat** out);
void pxg_flat_destroy(pxg_flat* index);
/* VectorIndex::insert (flat.rs:139-143) for a batch of n vectors, all-or-nothing:
 * nothing is inserted if any vector is non-finite or any id is a duplicate
 * (of a live id or of another id in the batch). out_slots may be NULL. */
int pxg_flat_insert(pxg_flat* index, const uint64_t* ids, const float* vectors, uint64_t n, uint32_t* out_slots);
/* Same, with the vectors already in device memory (row-major n x dim); ids
 * and out_slots stay on the host. Validation and preparation run on the
 * device with the same arithmetic; still all-or-nothing. */
int pxg_flat_insert_device(pxg_flat* index, const uint64_t* ids, const float* d_vectors, uint64_t n,
                           uint32_t* out_slots);
/* VectorIndex::remove (flat.rs:145-151): frees the slot for LIFO reuse. */
int pxg_flat_remove(pxg_flat* index, uint64_t id);
/* VectorIndex::contains / len / stats (flat.rs:171-193). */
int pxg_flat_contains(const pxg_flat* index, uint64_t id);
uint64_t pxg_flat_len(const pxg_flat* index);
int pxg_flat_stats(const pxg_flat* index, pxg_index_stats* out);
/* FlatIndex::vector (flat.rs:104-106): the stored, prepared vector. */
int pxg_flat_get_vector(const pxg_flat* index, uint64_t id, float* out);
/* Slot table for building per-slot accept masks: slot_count() slots; ids[s]
 * and live[s] (0 for a free slot). Either pointer may be NULL. */
uint64_t pxg_flat_slot_count(const pxg_flat* index);
int pxg_flat_slots(const pxg_flat* index, uint64_t* ids, uint8_t* live);
/* VectorIndex::search (flat.rs:153-169) over nq queries (row-major nq x dim).
 * accept: NULL (AcceptAll) or one byte per slot (nonzero = the filter accepts
 * that slot), evaluated by the caller exactly as Filter::accepts would be. */
int pxg_flat_search(const pxg_flat* index, const float* queries, uint64_t nq, uint64_t k, const uint8_t* accept,
                    uint64_t* out_ids, float* out_dist, uint32_t* out_count);
/* Same, with every pointer in device memory and work ordered on `stream`
 * (a hipStream_t; NULL = the library's own). Queries are validated and
 * prepared on the device; a non-finite query fails the call. Returns after
 * the results are complete. */
int pxg_flat_search_device(const pxg_flat* index, const float* d_queries, uint64_t nq, uint64_t k,
                           const uint8_t* d_accept, uint64_t* d_out_ids, float* d_out_dist, uint32_t* d_out_count,
                           void* stream);
/* pxg_flat_search_device that allocates nothing: no hipMalloc, hipFree,
 * pinned host memory, stream or event. No counterpart in the reference; it is
 * for callers that cannot allocate (serving loops with a fixed memory budget,
 * code that must not touch the allocator). Its scratch is one static device
 * array of 128 MiB per GPU, held until the process ends. A call that needs
 * more fails with PXG_ERR_CAPACITY (parameter "no-allocation scratch",
 * detail a = the array's size) at the first scratch region that does not fit:
 * prepared queries (nq x round_up(dim, 4) x 4 bytes), candidate buffers
 * (nq x CAP x 8 bytes per split, CAP = 256 for k <= 48, else 512, at least
 * one split), exact-scan keys, or the wide path's keys. Stages queued before
 * that point are waited for before the call returns, so no kernel still uses
 * the array or writes the outputs afterwards (the outputs are then undefined).
 * Calls on one GPU share that array: a per-GPU lock inside the library
 * serializes them, and each call has finished on the GPU when it returns.
 * stream: the caller's (NULL = the null stream). Results equal
 * pxg_flat_search_device's bit for bit. */
int pxg_flat_search_device_noalloc(const pxg_flat* index, const float* d_queries, uint64_t nq, uint64_t k,
                                   const uint8_t* d_accept, uint64_t* d_out_ids, float* d_out_dist,
                                   uint32_t* d_out_count, void* stream);
/* Search statistics of the last search on this thread: queries whose MFMA
 * candidate set could not be proven to contain the exact top-k and were
 * rescanned exactly. */
uint64_t pxg_flat_last_fallbacks(void);
/* Search path selection (no reference counterpart; for tests and tuning):
 * 0 = automatic (the exact scan for stores under 4096 rows and for batches
 * it is estimated to finish sooner, e.g. up to about 13 queries over
 * 100k x 128 or 4 over 1M x 768; otherwise the MFMA path), 1 = MFMA
 * candidates + exact rescoring whenever the metric and k allow it, 2 = exact
 * VALU scan only. Results are identical. */
int pxg_flat_set_search_mode(pxg_flat* index, int mode);

/* ------------------------------------------------------------------------ */
/* IVF-PQ: replaces IvfPqIndex, crates/proxima-index/src/ivfpq.rs:452-1228.  */
typedef struct pxg_ivfpq pxg_ivfpq;

/* IvfPqConfig (ivfpq.rs:106-304). */
typedef struct pxg_ivfpq_config {
  uint64_t nlist;
  uint64_t subspaces;
  uint64_t nprobe;
  uint64_t rerank;
  uint64_t seed;
  uint64_t max_iterations;
  uint64_t training_sample;
  uint64_t train_threshold;
  int32_t retain_vectors;
} pxg_ivfpq_config;

/* TrainingReport (ivfpq.rs:322-357). */
typedef struct pxg_training_report {
  uint64_t sampled;
  double coarse_inertia;
  uint64_t coarse_iterations;
  double residual_inertia;
  uint64_t populated_lists;
  uint64_t largest_list;
} pxg_training_report;

/* IvfPqConfig::new (ivfpq.rs:124-150): nprobe nlist/16, seed 0x1FF9C0D, 25
 * iterations, 100000-vector sample, threshold nlist*100, vectors retained. */
int pxg_ivfpq_config_default(uint64_t nlist, uint64_t subspaces, pxg_ivfpq_config* out);
/* IvfPqIndex::new (ivfpq.rs:481-509): Euclidean or Cosine only; config validated
 * (ivfpq.rs:259-304): 1 to dim subspaces. Above 128 subspaces the per-probe
 * tables do not fit in LDS and the search takes the wide path (tables and
 * keys in device memory, sorted). */
int pxg_ivfpq_create(uint32_t dim, int metric, const pxg_ivfpq_config* config, pxg_ivfpq** out);
void pxg_ivfpq_destroy(pxg_ivfpq* index);
/* VectorIndex::insert (ivfpq.rs:1129-1158), batched and all-or-nothing per
 * validation; encodes when trained, auto-trains when the live count reaches
 * train_threshold (splitting the batch at that insert). */
int pxg_ivfpq_insert(pxg_ivfpq* index, const uint64_t* ids, const float* vectors, uint64_t n, uint32_t* out_slots);
/* Same, vectors in device memory (ids and out_slots on the host). */
int pxg_ivfpq_insert_device(pxg_ivfpq* index, const uint64_t* ids, const float* d_vectors, uint64_t n,
                            uint32_t* out_slots);
/* VectorIndex::remove (ivfpq.rs:1160-1180). */
int pxg_ivfpq_remove(pxg_ivfpq* index, uint64_t id);
/* IvfPqIndex::compact (ivfpq.rs:907-975), reached through AnyIndex::compact
 * (proxima-store/src/index.rs:114-120): drop the free slots and renumber the
 * live ones in slot order; results are unchanged. reclaimed (may be NULL) =
 * slots given back (high-water mark minus the live count). */
int pxg_ivfpq_compact(pxg_ivfpq* index, uint64_t* reclaimed);
int pxg_ivfpq_contains(const pxg_ivfpq* index, uint64_t id);
uint64_t pxg_ivfpq_len(const pxg_ivfpq* index);
int pxg_ivfpq_is_trained(const pxg_ivfpq* index);
/* VectorIndex::stats (ivfpq.rs:1194-1214): graph_bytes = codes, lists, codebooks. */
int pxg_ivfpq_stats(const pxg_ivfpq* index, pxg_index_stats* out);
/* IvfPqIndex::vector (ivfpq.rs:544-552). */
int pxg_ivfpq_get_vector(const pxg_ivfpq* index, uint64_t id, float* out);
uint64_t pxg_ivfpq_slot_count(const pxg_ivfpq* index);
int pxg_ivfpq_slots(const pxg_ivfpq* index, uint64_t* ids, uint8_t* live);
/* IvfPqIndex::list_lengths (ivfpq.rs:567-569): list_count() entries. */
uint64_t pxg_ivfpq_list_count(const pxg_ivfpq* index);
int pxg_ivfpq_list_lengths(const pxg_ivfpq* index, uint64_t* out);
/* IvfPqIndex::train (ivfpq.rs:735-825) on the GPU: stride sample, k-means with
 * k-means++ (ChaCha8Rng(seed)), residual PQ training with a fresh generator
 * from the same seed, encode every live vector. report may be NULL. */
int pxg_ivfpq_train(pxg_ivfpq* index, pxg_training_report* report);
int pxg_ivfpq_training_report(const pxg_ivfpq* index, pxg_training_report* report);
/* IvfPqIndex::parts (ivfpq.rs:606-617): list_count() x dim centroids, the
 * codebooks (sum over subspaces of 256 x width floats), slot_count() x M
 * codes and slot_count() list assignments (UINT32_MAX when none). Any may be NULL. */
int pxg_ivfpq_parts(const pxg_ivfpq* index, float* centroids, float* codebooks, uint8_t* codes, uint32_t* list_of);
/* IvfPqIndex::from_parts (ivfpq.rs:624-717) for the trained state of an index
 * whose vectors are already inserted: `produced` centroids, codebooks, and
 * codes/list_of per slot (codes NULL = encode the live vectors on the GPU). */
int pxg_ivfpq_load_trained(pxg_ivfpq* index, const float* centroids, uint64_t produced, const float* codebooks,
                           const uint8_t* codes, const uint32_t* list_of);
/* IvfPqIndex::search_with_nprobe (ivfpq.rs:981-996); nprobe 0 = the configured one. */
int pxg_ivfpq_search(const pxg_ivfpq* index, const float* queries, uint64_t nq, uint64_t k, uint64_t nprobe,
                     const uint8_t* accept, uint64_t* out_ids, float* out_dist, uint32_t* out_count);
int pxg_ivfpq_search_device(const pxg_ivfpq* index, const float* d_queries, uint64_t nq, uint64_t k, uint64_t nprobe,
                            const uint8_t* d_accept, uint64_t* d_out_ids, float* d_out_dist, uint32_t* d_out_count,
                            void* stream);

/* Code entries (M bytes + a 4-byte id rank each) the last search on this
 * thread streamed: the scan's algorithmic traffic. No reference counterpart. */
uint64_t pxg_ivfpq_last_scanned(void);
/* Maintenance counters of the index's list view (no reference counterpart):
 * full rebuilds (after train, load, compact, or a full pool) and list regions
 * moved by appends. Inserts and removals otherwise update the view in place. */
int pxg_ivfpq_view_stats(const pxg_ivfpq* index, uint64_t* rebuilds, uint64_t* moves);

/* ------------------------------------------------------------------------ */
/* k-means and the product quantizer (crates/proxima-quantize).              */

/* kmeans() (kmeans.rs:59-143) with ChaCha8Rng::seed_from_u64(seed): k-means++
 * seeding then Lloyd; k is clamped to [1, n]; writes k_out x dim centroids. */
int pxg_kmeans(const float* points, uint64_t n, uint32_t dim, uint64_t k, uint64_t max_iterations, uint64_t seed,
               float* centroids_out, double* inertia, uint64_t* iterations, uint64_t* k_out);
/* The Lloyd loop of kmeans() (kmeans.rs:85-136) from given initial centroids;
 * assign_out (n, may be NULL) is the last assignment pass. */
int pxg_kmeans_lloyd(const float* points, uint64_t n, uint32_t dim, uint64_t k, uint64_t max_iterations,
                     const float* init, float* centroids_out, uint32_t* assign_out, double* inertia,
                     uint64_t* iterations);
/* pxg_kmeans / pxg_kmeans_lloyd with points, init, centroids and assignment in
 * device memory (d_init NULL = k-means++ from seed). */
int pxg_kmeans_device(const float* d_points, uint64_t n, uint32_t dim, uint64_t k, uint64_t max_iterations,
                      uint64_t seed, const float* d_init, float* d_centroids_out, uint32_t* d_assign_out,
                      double* inertia, uint64_t* iterations);
/* kmeans_plus_plus (kmeans.rs:146-194) alone, 1 <= k <= n. */
int pxg_kmeans_pp(const float* points, uint64_t n, uint32_t dim, uint64_t k, uint64_t seed, float* centroids_out);
/* The assignment pass (kmeans.rs:90-97, nearest 200-212). */
int pxg_kmeans_assign(const float* points, uint64_t n, uint32_t dim, const float* centroids, uint64_t k,
                      uint32_t* assign_out, float* dist_out);
/* Counters of the calling thread's last k-means run (the last one inside a
 * pxg_kmeans* or pxg_pq_train* call). No counterpart in the reference; it is
 * for measurement: time and algorithmic flops (2*n*k*dim per pass) of the
 * FP32-MFMA distance passes of its assignments, the number of those passes,
 * the points they could not certify (rescanned exactly), and the f64
 * point-order sums that had to keep the fixed parallel order. Any pointer may
 * be NULL. */
int pxg_kmeans_last_stats(double* mfma_ms, double* mfma_flops, uint64_t* mfma_passes, uint64_t* rescanned,
                          uint64_t* inexact_sums);
/* Empty-cluster reseeds (kmeans.rs:115-124) of the calling thread's last
 * k-means run. No counterpart in the reference; it is for measurement and
 * tests: the reseeds in all, those found in the candidate pool of the points
 * with the largest distance bounds, and the iterations whose pool test
 * failed (their reseeds went through the segment passes). Any pointer may be
 * NULL. */
int pxg_kmeans_last_reseeds(uint64_t* reseeds, uint64_t* pool_reseeds, uint64_t* pool_fallbacks);
/* ProductQuantizer::train (product.rs:198-296): codebooks_out holds, per
 * subspace, 256 rows of its width (dim floats x 256 in total). */
int pxg_pq_train(const float* training, uint64_t n, uint32_t dim, uint64_t subspaces, uint64_t max_iterations,
                 uint64_t seed, float* codebooks_out, double* inertia, uint64_t* iterations);
/* pxg_pq_train with the training vectors and the codebooks in device memory
 * (training values are taken as finite: device data is not scanned). */
int pxg_pq_train_device(const float* d_training, uint64_t n, uint32_t dim, uint64_t subspaces,
                        uint64_t max_iterations, uint64_t seed, float* d_codebooks_out, double* inertia,
                        uint64_t* iterations);
/* ProductQuantizer::encode_into (product.rs:361-380) for n vectors. */
int pxg_pq_encode(const float* codebooks, uint32_t dim, uint64_t subspaces, const float* vectors, uint64_t n,
                  uint8_t* codes_out);

/* ------------------------------------------------------------------------ */
/* Scalar quantizer (crates/proxima-quantize/src/scalar.rs:112-337), on the  */
/* device. per_dim: 1 = RangeMode::PerDimension (dim ranges), 0 = Global (1). */
/* code_type: 0 = CodeType::U8, 1 = CodeType::I8 (scalar.rs:25-52).          */

/* ScalarQuantizer::train (scalar.rs:141-199): min / scale / inverse_scale per
 * range group. A non-finite value fails with NonFinite (its component). */
int pxg_sq_train(const float* training, uint64_t n, uint32_t dim, int per_dim, float* min, float* scale,
                 float* inverse_scale);
/* ScalarQuantizer::encode_into (scalar.rs:246-268) for n vectors (n x dim bytes out). */
int pxg_sq_encode(const float* vectors, uint64_t n, uint32_t dim, int per_dim, int code_type, const float* min,
                  const float* inverse_scale, uint8_t* out);
/* ScalarQuantizer::decode (scalar.rs:271-281, reconstruct 323-327). */
int pxg_sq_decode(const uint8_t* codes, uint64_t n, uint32_t dim, int per_dim, int code_type, const float* min,
                  const float* scale, float* out);
/* asymmetric_inner_product (inner_product != 0, scalar.rs:313-319) or
 * asymmetric_squared_l2 (298-305) of one f32 query against n codes. */
int pxg_sq_asymmetric(int inner_product, const float* query, const uint8_t* codes, uint64_t n, uint32_t dim,
                      int per_dim, int code_type, const float* min, const float* scale, float* out);

/* SQ8 flat index: a VectorIndex over I8 codes with no reference counterpart
 * (the reference has the quantizer but no SQ index). The score of a stored
 * vector is -(float)S, S the exact int32 dot product of the query's and the
 * vector's I8 codes, ordered as TopK (topk.rs:63-67). Metric: inner product,
 * or cosine (vectors and queries prepared as space.rs:130-138 first). */
typedef struct pxg_sq8 pxg_sq8;
int pxg_sq8_create(uint32_t dim, int metric, int per_dim, uint64_t capacity, pxg_sq8** out);
void pxg_sq8_destroy(pxg_sq8* index);
/* Fit the ranges (pxg_sq_train semantics) to a host or device sample. */
int pxg_sq8_train(pxg_sq8* index, const float* training, uint64_t n);
int pxg_sq8_train_device(pxg_sq8* index, const float* d_training, uint64_t n);
/* Use ranges trained elsewhere (a ScalarQuantizer's min / scale / inverse_scale). */
int pxg_sq8_set_ranges(pxg_sq8* index, const float* min, const float* scale, const float* inverse_scale);
int pxg_sq8_ranges(const pxg_sq8* index, float* min, float* scale, float* inverse_scale);
int pxg_sq8_is_trained(const pxg_sq8* index);
/* VectorIndex::insert for n f32 vectors (encoded on the device; the index
 * must be trained), all-or-nothing as pxg_flat_insert. */
int pxg_sq8_insert(pxg_sq8* index, const uint64_t* ids, const float* vectors, uint64_t n, uint32_t* out_slots);
int pxg_sq8_insert_device(pxg_sq8* index, const uint64_t* ids, const float* d_vectors, uint64_t n,
                          uint32_t* out_slots);
/* Insert already encoded I8 codes (n x dim bytes). */
int pxg_sq8_add_codes(pxg_sq8* index, const uint64_t* ids, const int8_t* codes, uint64_t n, uint32_t* out_slots);
int pxg_sq8_remove(pxg_sq8* index, uint64_t id);
int pxg_sq8_contains(const pxg_sq8* index, uint64_t id);
uint64_t pxg_sq8_len(const pxg_sq8* index);
/* vector_bytes = device code bytes; graph_bytes = the range table (table_bytes). */
int pxg_sq8_stats(const pxg_sq8* index, pxg_index_stats* out);
int pxg_sq8_get_code(const pxg_sq8* index, uint64_t id, int8_t* out);
uint64_t pxg_sq8_slot_count(const pxg_sq8* index);
int pxg_sq8_slots(const pxg_sq8* index, uint64_t* ids, uint8_t* live);
/* Search nq f32 queries (encoded with the index's ranges). rescore > 0:
 * the best max(rescore, k) by integer score are rescored with
 * asymmetric_inner_product and the best k by (distance, id) returned.
 * accept as pxg_flat_search. k up to 2^24 (check_k); max(k, rescore) above
 * 1024 takes the sorted path. */
int pxg_sq8_search(const pxg_sq8* index, const float* queries, uint64_t nq, uint64_t k, uint64_t rescore,
                   const uint8_t* accept, uint64_t* out_ids, float* out_dist, uint32_t* out_count);
/* Search with queries given as I8 codes (nq x dim bytes); no rescoring. */
int pxg_sq8_search_codes(const pxg_sq8* index, const int8_t* query_codes, uint64_t nq, uint64_t k,
                         const uint8_t* accept, uint64_t* out_ids, float* out_dist, uint32_t* out_count);
/* pxg_sq8_search with every pointer in device memory, ordered on `stream`. */
int pxg_sq8_search_device(const pxg_sq8* index, const float* d_queries, uint64_t nq, uint64_t k, uint64_t rescore,
                          const uint8_t* d_accept, uint64_t* d_out_ids, float* d_out_dist, uint32_t* d_out_count,
                          void* stream);
/* Queries of the last search on this thread that took the exact scan
 * because their candidate set overflowed. No reference counterpart. */
uint64_t pxg_sq8_last_fallbacks(void);
/* 0 = automatic, 1 = integer MFMA whenever dim <= 256, 2 = exact scan. */
int pxg_sq8_set_search_mode(pxg_sq8* index, int mode);

/* ------------------------------------------------------------------------ */
/* The benchmark fixture (crates/proxima-cli/src/fixture.rs).               */

/* fixture::generate (fixture.rs:71-123) from ChaCha8Rng::seed_from_u64(seed):
 * vectors (count x dim) = centre[i % clusters] + gaussian, centres =
 * 4 * gaussian; queries (queries x dim) = vectors[(q * stride) % count] +
 * 0.25 * gaussian with stride = max(count / max(queries, 1), 1). ln and cos
 * of the Box-Muller step are correctly rounded f32 values (the reference
 * uses the platform libm). Configuration error when clusters = 0 with
 * count > 0, or queries > 0 with count = 0 (the reference would panic). */
int pxg_fixture_generate(uint64_t count, uint32_t dim, uint64_t clusters, uint64_t queries, uint64_t seed,
                         float* vectors, float* query_vectors);
/* pxg_fixture_generate writing to device memory. */
int pxg_fixture_generate_device(uint64_t count, uint32_t dim, uint64_t clusters, uint64_t queries, uint64_t seed,
                                float* d_vectors, float* d_queries);

/* Synthetic inputs of the benchmark configurations. No reference counterpart
 * (the reference's generator is fixture::generate above): the same
 * ChaCha8Rng::seed_from_u64(seed) stream and Box-Muller step, drawn in this
 * order of Gaussian slots (slot g = stream words 2g and 2g+1): clusters x dim
 * centres = centre_scale * gaussian; when drawn_clusters, one cluster choice
 * per point then per query, item t from word 2*clusters*dim + t as
 * (word * clusters) >> 32, the region rounded up to whole slots; count x dim
 * points = centre[cluster(i)] + sigma * gaussian; queries x dim queries the
 * same, cluster(q). Without drawn_clusters, cluster(i) = i % clusters and
 * cluster(q) = q % clusters. Device pointers; returns when written. */
int pxg_mixture_generate_device(uint64_t count, uint32_t dim, uint64_t clusters, float centre_scale, float sigma,
                                uint64_t queries, int drawn_clusters, uint64_t seed, float* d_vectors,
                                float* d_queries);
/* count x dim values lo + (hi - lo) * gen::<f32>() of stream word t (no
 * reference counterpart; the uniform configuration's inputs). */
int pxg_uniform_generate_device(uint64_t count, uint32_t dim, float lo, float hi, uint64_t seed, float* d_out);

#ifdef __cplusplus
}
#endif
#endif /* PROXIMA_HIP_H */
