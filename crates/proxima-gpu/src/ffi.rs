//! The C ABI of libproxima_hip (`include/proxima_hip.h`), one declaration per
//! header entry. Everything here is `pub(crate)`: the safe wrappers in
//! `lib.rs` are the crate's interface.

use std::os::raw::{c_char, c_int, c_void};

/// Opaque handle of a flat index.
#[repr(C)]
pub(crate) struct PxgFlat {
    _p: [u8; 0],
}

/// Opaque handle of an IVF-PQ index.
#[repr(C)]
pub(crate) struct PxgIvfPq {
    _p: [u8; 0],
}

/// Opaque handle of an SQ8 index.
#[repr(C)]
pub(crate) struct PxgSq8 {
    _p: [u8; 0],
}

/// `pxg_index_stats` (index.rs:68-130).
#[repr(C)]
#[derive(Default)]
pub(crate) struct PxgIndexStats {
    pub(crate) len: u64,
    pub(crate) deleted: u64,
    pub(crate) dim: u32,
    pub(crate) metric: i32,
    pub(crate) layers: u64,
    pub(crate) edges: u64,
    pub(crate) vector_bytes: u64,
    pub(crate) graph_bytes: u64,
}

/// `pxg_timings`: device stage timings of the last call (measurement only).
#[repr(C)]
#[derive(Default)]
pub(crate) struct PxgTimings {
    pub(crate) prep_ms: f32,
    pub(crate) candidates_ms: f32,
    pub(crate) merge_ms: f32,
    pub(crate) fallback_ms: f32,
    pub(crate) total_ms: f32,
}

/// `pxg_ivfpq_config` (IvfPqConfig, ivfpq.rs:106-304).
#[repr(C)]
#[derive(Default, Clone, Copy)]
pub(crate) struct PxgIvfPqConfig {
    pub(crate) nlist: u64,
    pub(crate) subspaces: u64,
    pub(crate) nprobe: u64,
    pub(crate) rerank: u64,
    pub(crate) seed: u64,
    pub(crate) max_iterations: u64,
    pub(crate) training_sample: u64,
    pub(crate) train_threshold: u64,
    pub(crate) retain_vectors: i32,
}

/// `pxg_training_report` (TrainingReport, ivfpq.rs:322-357).
#[repr(C)]
#[derive(Default)]
pub(crate) struct PxgTrainingReport {
    pub(crate) sampled: u64,
    pub(crate) coarse_inertia: f64,
    pub(crate) coarse_iterations: u64,
    pub(crate) residual_inertia: f64,
    pub(crate) populated_lists: u64,
    pub(crate) largest_list: u64,
}

extern "C" {
    pub(crate) fn pxg_last_error_message() -> *const c_char;
    pub(crate) fn pxg_last_error_detail(a: *mut u64, b: *mut u64, value: *mut f32) -> c_int;
    pub(crate) fn pxg_last_error_parameter() -> *const c_char;
    pub(crate) fn pxg_last_error_reason() -> *const c_char;
    pub(crate) fn pxg_version() -> *const c_char;
    pub(crate) fn pxg_device_count() -> c_int;
    pub(crate) fn pxg_set_profiling(enabled: c_int);
    pub(crate) fn pxg_last_timings(out: *mut PxgTimings) -> c_int;
    pub(crate) fn pxg_flat_create(dim: u32, metric: c_int, capacity: u64, out: *mut *mut PxgFlat) -> c_int;
    pub(crate) fn pxg_flat_destroy(index: *mut PxgFlat);
    pub(crate) fn pxg_flat_insert(index: *mut PxgFlat, ids: *const u64, vectors: *const f32, n: u64,
        out_slots: *mut u32) -> c_int;
    pub(crate) fn pxg_flat_insert_device(index: *mut PxgFlat, ids: *const u64, d_vectors: *const f32, n: u64,
        out_slots: *mut u32) -> c_int;
    pub(crate) fn pxg_flat_remove(index: *mut PxgFlat, id: u64) -> c_int;
    pub(crate) fn pxg_flat_contains(index: *const PxgFlat, id: u64) -> c_int;
    pub(crate) fn pxg_flat_len(index: *const PxgFlat) -> u64;
    pub(crate) fn pxg_flat_stats(index: *const PxgFlat, out: *mut PxgIndexStats) -> c_int;
    pub(crate) fn pxg_flat_get_vector(index: *const PxgFlat, id: u64, out: *mut f32) -> c_int;
    pub(crate) fn pxg_flat_slot_count(index: *const PxgFlat) -> u64;
    pub(crate) fn pxg_flat_slots(index: *const PxgFlat, ids: *mut u64, live: *mut u8) -> c_int;
    pub(crate) fn pxg_flat_search(index: *const PxgFlat, queries: *const f32, nq: u64, k: u64,
        accept: *const u8, out_ids: *mut u64, out_dist: *mut f32, out_count: *mut u32) -> c_int;
    pub(crate) fn pxg_flat_search_device(index: *const PxgFlat, d_queries: *const f32, nq: u64, k: u64,
        d_accept: *const u8, d_out_ids: *mut u64, d_out_dist: *mut f32, d_out_count: *mut u32,
        stream: *mut c_void) -> c_int;
    pub(crate) fn pxg_flat_search_device_noalloc(index: *const PxgFlat, d_queries: *const f32, nq: u64,
        k: u64, d_accept: *const u8, d_out_ids: *mut u64, d_out_dist: *mut f32, d_out_count: *mut u32,
        stream: *mut c_void) -> c_int;
    pub(crate) fn pxg_flat_last_fallbacks() -> u64;
    pub(crate) fn pxg_flat_set_search_mode(index: *mut PxgFlat, mode: c_int) -> c_int;
    pub(crate) fn pxg_ivfpq_config_default(nlist: u64, subspaces: u64, out: *mut PxgIvfPqConfig) -> c_int;
    pub(crate) fn pxg_ivfpq_create(dim: u32, metric: c_int, config: *const PxgIvfPqConfig,
        out: *mut *mut PxgIvfPq) -> c_int;
    pub(crate) fn pxg_ivfpq_destroy(index: *mut PxgIvfPq);
    pub(crate) fn pxg_ivfpq_insert(index: *mut PxgIvfPq, ids: *const u64, vectors: *const f32, n: u64,
        out_slots: *mut u32) -> c_int;
    pub(crate) fn pxg_ivfpq_insert_device(index: *mut PxgIvfPq, ids: *const u64, d_vectors: *const f32,
        n: u64, out_slots: *mut u32) -> c_int;
    pub(crate) fn pxg_ivfpq_remove(index: *mut PxgIvfPq, id: u64) -> c_int;
    pub(crate) fn pxg_ivfpq_compact(index: *mut PxgIvfPq, reclaimed: *mut u64) -> c_int;
    pub(crate) fn pxg_ivfpq_contains(index: *const PxgIvfPq, id: u64) -> c_int;
    pub(crate) fn pxg_ivfpq_len(index: *const PxgIvfPq) -> u64;
    pub(crate) fn pxg_ivfpq_is_trained(index: *const PxgIvfPq) -> c_int;
    pub(crate) fn pxg_ivfpq_stats(index: *const PxgIvfPq, out: *mut PxgIndexStats) -> c_int;
    pub(crate) fn pxg_ivfpq_get_vector(index: *const PxgIvfPq, id: u64, out: *mut f32) -> c_int;
    pub(crate) fn pxg_ivfpq_slot_count(index: *const PxgIvfPq) -> u64;
    pub(crate) fn pxg_ivfpq_slots(index: *const PxgIvfPq, ids: *mut u64, live: *mut u8) -> c_int;
    pub(crate) fn pxg_ivfpq_list_count(index: *const PxgIvfPq) -> u64;
    pub(crate) fn pxg_ivfpq_list_lengths(index: *const PxgIvfPq, out: *mut u64) -> c_int;
    pub(crate) fn pxg_ivfpq_train(index: *mut PxgIvfPq, report: *mut PxgTrainingReport) -> c_int;
    pub(crate) fn pxg_ivfpq_training_report(index: *const PxgIvfPq, report: *mut PxgTrainingReport) -> c_int;
    pub(crate) fn pxg_ivfpq_parts(index: *const PxgIvfPq, centroids: *mut f32, codebooks: *mut f32,
        codes: *mut u8, list_of: *mut u32) -> c_int;
    pub(crate) fn pxg_ivfpq_load_trained(index: *mut PxgIvfPq, centroids: *const f32, produced: u64,
        codebooks: *const f32, codes: *const u8, list_of: *const u32) -> c_int;
    pub(crate) fn pxg_ivfpq_search(index: *const PxgIvfPq, queries: *const f32, nq: u64, k: u64, nprobe: u64,
        accept: *const u8, out_ids: *mut u64, out_dist: *mut f32, out_count: *mut u32) -> c_int;
    pub(crate) fn pxg_ivfpq_search_device(index: *const PxgIvfPq, d_queries: *const f32, nq: u64, k: u64,
        nprobe: u64, d_accept: *const u8, d_out_ids: *mut u64, d_out_dist: *mut f32, d_out_count: *mut u32,
        stream: *mut c_void) -> c_int;
    pub(crate) fn pxg_ivfpq_last_scanned() -> u64;
    pub(crate) fn pxg_ivfpq_view_stats(index: *const PxgIvfPq, rebuilds: *mut u64, moves: *mut u64) -> c_int;
    pub(crate) fn pxg_kmeans(points: *const f32, n: u64, dim: u32, k: u64, max_iterations: u64, seed: u64,
        centroids_out: *mut f32, inertia: *mut f64, iterations: *mut u64, k_out: *mut u64) -> c_int;
    pub(crate) fn pxg_kmeans_lloyd(points: *const f32, n: u64, dim: u32, k: u64, max_iterations: u64,
        init: *const f32, centroids_out: *mut f32, assign_out: *mut u32, inertia: *mut f64,
        iterations: *mut u64) -> c_int;
    pub(crate) fn pxg_kmeans_device(d_points: *const f32, n: u64, dim: u32, k: u64, max_iterations: u64,
        seed: u64, d_init: *const f32, d_centroids_out: *mut f32, d_assign_out: *mut u32, inertia: *mut f64,
        iterations: *mut u64) -> c_int;
    pub(crate) fn pxg_kmeans_pp(points: *const f32, n: u64, dim: u32, k: u64, seed: u64,
        centroids_out: *mut f32) -> c_int;
    pub(crate) fn pxg_kmeans_assign(points: *const f32, n: u64, dim: u32, centroids: *const f32, k: u64,
        assign_out: *mut u32, dist_out: *mut f32) -> c_int;
    pub(crate) fn pxg_kmeans_last_stats(mfma_ms: *mut f64, mfma_flops: *mut f64, mfma_passes: *mut u64,
        rescanned: *mut u64, inexact_sums: *mut u64) -> c_int;
    pub(crate) fn pxg_kmeans_last_reseeds(reseeds: *mut u64, pool_reseeds: *mut u64,
        pool_fallbacks: *mut u64) -> c_int;
    pub(crate) fn pxg_pq_train(training: *const f32, n: u64, dim: u32, subspaces: u64, max_iterations: u64,
        seed: u64, codebooks_out: *mut f32, inertia: *mut f64, iterations: *mut u64) -> c_int;
    pub(crate) fn pxg_pq_train_device(d_training: *const f32, n: u64, dim: u32, subspaces: u64,
        max_iterations: u64, seed: u64, d_codebooks_out: *mut f32, inertia: *mut f64,
        iterations: *mut u64) -> c_int;
    pub(crate) fn pxg_pq_encode(codebooks: *const f32, dim: u32, subspaces: u64, vectors: *const f32, n: u64,
        codes_out: *mut u8) -> c_int;
    pub(crate) fn pxg_sq_train(training: *const f32, n: u64, dim: u32, per_dim: c_int, min: *mut f32,
        scale: *mut f32, inverse_scale: *mut f32) -> c_int;
    pub(crate) fn pxg_sq_encode(vectors: *const f32, n: u64, dim: u32, per_dim: c_int, code_type: c_int,
        min: *const f32, inverse_scale: *const f32, out: *mut u8) -> c_int;
    pub(crate) fn pxg_sq_decode(codes: *const u8, n: u64, dim: u32, per_dim: c_int, code_type: c_int,
        min: *const f32, scale: *const f32, out: *mut f32) -> c_int;
    pub(crate) fn pxg_sq_asymmetric(inner_product: c_int, query: *const f32, codes: *const u8, n: u64,
        dim: u32, per_dim: c_int, code_type: c_int, min: *const f32, scale: *const f32,
        out: *mut f32) -> c_int;
    pub(crate) fn pxg_sq8_create(dim: u32, metric: c_int, per_dim: c_int, capacity: u64,
        out: *mut *mut PxgSq8) -> c_int;
    pub(crate) fn pxg_sq8_destroy(index: *mut PxgSq8);
    pub(crate) fn pxg_sq8_train(index: *mut PxgSq8, training: *const f32, n: u64) -> c_int;
    pub(crate) fn pxg_sq8_train_device(index: *mut PxgSq8, d_training: *const f32, n: u64) -> c_int;
    pub(crate) fn pxg_sq8_set_ranges(index: *mut PxgSq8, min: *const f32, scale: *const f32,
        inverse_scale: *const f32) -> c_int;
    pub(crate) fn pxg_sq8_ranges(index: *const PxgSq8, min: *mut f32, scale: *mut f32,
        inverse_scale: *mut f32) -> c_int;
    pub(crate) fn pxg_sq8_is_trained(index: *const PxgSq8) -> c_int;
    pub(crate) fn pxg_sq8_insert(index: *mut PxgSq8, ids: *const u64, vectors: *const f32, n: u64,
        out_slots: *mut u32) -> c_int;
    pub(crate) fn pxg_sq8_insert_device(index: *mut PxgSq8, ids: *const u64, d_vectors: *const f32, n: u64,
        out_slots: *mut u32) -> c_int;
    pub(crate) fn pxg_sq8_add_codes(index: *mut PxgSq8, ids: *const u64, codes: *const i8, n: u64,
        out_slots: *mut u32) -> c_int;
    pub(crate) fn pxg_sq8_remove(index: *mut PxgSq8, id: u64) -> c_int;
    pub(crate) fn pxg_sq8_contains(index: *const PxgSq8, id: u64) -> c_int;
    pub(crate) fn pxg_sq8_len(index: *const PxgSq8) -> u64;
    pub(crate) fn pxg_sq8_stats(index: *const PxgSq8, out: *mut PxgIndexStats) -> c_int;
    pub(crate) fn pxg_sq8_get_code(index: *const PxgSq8, id: u64, out: *mut i8) -> c_int;
    pub(crate) fn pxg_sq8_slot_count(index: *const PxgSq8) -> u64;
    pub(crate) fn pxg_sq8_slots(index: *const PxgSq8, ids: *mut u64, live: *mut u8) -> c_int;
    pub(crate) fn pxg_sq8_search(index: *const PxgSq8, queries: *const f32, nq: u64, k: u64, rescore: u64,
        accept: *const u8, out_ids: *mut u64, out_dist: *mut f32, out_count: *mut u32) -> c_int;
    pub(crate) fn pxg_sq8_search_codes(index: *const PxgSq8, query_codes: *const i8, nq: u64, k: u64,
        accept: *const u8, out_ids: *mut u64, out_dist: *mut f32, out_count: *mut u32) -> c_int;
    pub(crate) fn pxg_sq8_search_device(index: *const PxgSq8, d_queries: *const f32, nq: u64, k: u64,
        rescore: u64, d_accept: *const u8, d_out_ids: *mut u64, d_out_dist: *mut f32, d_out_count: *mut u32,
        stream: *mut c_void) -> c_int;
    pub(crate) fn pxg_sq8_last_fallbacks() -> u64;
    pub(crate) fn pxg_sq8_set_search_mode(index: *mut PxgSq8, mode: c_int) -> c_int;
    pub(crate) fn pxg_fixture_generate(count: u64, dim: u32, clusters: u64, queries: u64, seed: u64,
        vectors: *mut f32, query_vectors: *mut f32) -> c_int;
    pub(crate) fn pxg_fixture_generate_device(count: u64, dim: u32, clusters: u64, queries: u64, seed: u64,
        d_vectors: *mut f32, d_queries: *mut f32) -> c_int;
    pub(crate) fn pxg_mixture_generate_device(count: u64, dim: u32, clusters: u64, centre_scale: f32, sigma: f32,
        queries: u64, drawn_clusters: c_int, seed: u64, d_vectors: *mut f32, d_queries: *mut f32) -> c_int;
    pub(crate) fn pxg_uniform_generate_device(count: u64, dim: u32, lo: f32, hi: f32, seed: u64, d_out: *mut f32) -> c_int;
}
