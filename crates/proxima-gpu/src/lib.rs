//! MI355X indexes behind proxima's [`VectorIndex`]: exact flat search, SQ8
//! int8 search and the IVF-PQ scan and trainer, computed by libproxima_hip's
//! hand-written gfx950 kernels.
//!
//! This is the workspace's one crate that may use `unsafe`: every call into
//! the C ABI (`include/proxima_hip.h`) is in this file, behind safe types.
//! Results equal the CPU indexes' bit for bit: the same ids in the same
//! order, the same ranking scores, ties broken by id (index.rs:136-149).
//!
//! * [`GpuFlatIndex`] replaces [`proxima_index::FlatIndex`];
//! * [`GpuIvfPqIndex`] replaces [`proxima_index::IvfPqIndex`], with `train`,
//!   `search_with_nprobe` and `compact`;
//! * [`GpuSq8Index`] is an index over I8 scalar codes (the reference has the
//!   quantizer but no SQ index): score `-(float)S`, `S` the exact int32 dot
//!   product of the query's and the vector's codes.
//!
//! A filter, a Rust closure, reaches the device as one accept byte per slot
//! built here; `search_all` passes none.
#![allow(unsafe_code)]

mod ffi;

use std::collections::HashMap;
use std::ffi::CStr;
use std::os::raw::c_int;
use std::ptr::{self, NonNull};

use proxima_core::{Metadata, Metric, ProximaError, Result, SearchResult, VectorId, VectorSpace};
use proxima_index::{Filter, IndexStats, IvfPqConfig, TrainingReport, VectorIndex};

/// Map a library status to the reference's error (error.rs:37-160).
fn check(status: c_int) -> Result<()> {
    if status == 0 {
        return Ok(());
    }
    let (mut a, mut b, mut value) = (0u64, 0u64, 0f32);
    // SAFETY: the detail accessor writes three plain values of this thread's last error.
    unsafe { ffi::pxg_last_error_detail(&mut a, &mut b, &mut value) };
    // SAFETY: the message is a NUL-terminated thread-local string that lives until the next call.
    let detail = unsafe { CStr::from_ptr(ffi::pxg_last_error_message()) }.to_string_lossy().into_owned();
    // SAFETY: both accessors return pointers to string literals inside the
    // library (static storage; the library is linked, never unloaded), so the
    // borrow may be 'static.
    let parameter = unsafe { static_str(ffi::pxg_last_error_parameter()) };
    let reason = unsafe { static_str(ffi::pxg_last_error_reason()) };
    Err(match status {
        1 => ProximaError::DimensionMismatch { expected: a as usize, actual: b as usize },
        2 => ProximaError::UnknownId { id: VectorId::new(a) },
        3 => ProximaError::DuplicateId { id: VectorId::new(a) },
        4 => ProximaError::Capacity { what: parameter.unwrap_or("device memory"), limit: a as usize },
        5 => ProximaError::NonFinite { index: a as usize, value },
        6 => ProximaError::Corruption { structure: "device index", detail },
        7 => ProximaError::Configuration {
            parameter: parameter.unwrap_or("proxima-gpu"),
            value: a.to_string(),
            reason: reason.unwrap_or("rejected by libproxima_hip"),
        },
        _ => ProximaError::Internal { location: "proxima-gpu", detail },
    })
}

/// A NUL-terminated string of static storage from the library, or `None`
/// when it is empty or not UTF-8.
///
/// # Safety
/// `p` is NULL or points to a NUL-terminated string that lives for the rest
/// of the process.
unsafe fn static_str(p: *const std::os::raw::c_char) -> Option<&'static str> {
    if p.is_null() {
        return None;
    }
    let s: &'static CStr = CStr::from_ptr(p);
    s.to_str().ok().filter(|s| !s.is_empty())
}

/// `Metric` in declaration order (distance.rs:90-118), as the C ABI numbers it.
fn metric_code(metric: Metric) -> c_int {
    match metric {
        Metric::Euclidean => 0,
        Metric::Cosine => 1,
        Metric::InnerProduct => 2,
        Metric::Manhattan => 3,
    }
}

/// One accept byte per slot: `Filter::accepts(id, &metadata)` for live slots,
/// 0 for free ones (index.rs:27-60).
fn accept_mask(
    ids: &[u64],
    live: &[u8],
    meta: &HashMap<VectorId, Metadata>,
    filter: &dyn Filter,
) -> Vec<u8> {
    let empty = Metadata::new();
    ids.iter()
        .zip(live)
        .map(|(&id, &l)| {
            let id = VectorId::new(id);
            u8::from(l != 0 && filter.accepts(id, meta.get(&id).unwrap_or(&empty)))
        })
        .collect()
}

/// Unpack `nq` rows of `kq` results written by a batched search.
fn unpack(ids: &[u64], dist: &[f32], count: &[u32], kq: usize) -> Vec<Vec<SearchResult>> {
    count
        .iter()
        .enumerate()
        .map(|(q, &c)| {
            (0..c as usize).map(|i| SearchResult::new(VectorId::new(ids[q * kq + i]), dist[q * kq + i])).collect()
        })
        .collect()
}

fn to_stats(s: &ffi::PxgIndexStats, metric: Metric) -> IndexStats {
    IndexStats {
        len: s.len as usize,
        deleted: s.deleted as usize,
        dim: s.dim as usize,
        metric,
        layers: s.layers as usize,
        nodes_per_layer: vec![s.len as usize],
        edges: s.edges as usize,
        vector_bytes: s.vector_bytes as usize,
        graph_bytes: s.graph_bytes as usize,
    }
}

/// The k accepted by `check_k` (index.rs:212-224).
fn check_k(k: usize) -> Result<()> {
    if k > 1 << 24 {
        return Err(ProximaError::config("k", k, "exceeds the 16777216 result ceiling"));
    }
    Ok(())
}

/// Queries of a batch, validated on the host as `VectorSpace::validate` does.
fn validate_batch(space: &VectorSpace, queries: &[f32]) -> Result<usize> {
    let dim = space.dim();
    if queries.len() % dim != 0 {
        return Err(ProximaError::DimensionMismatch { expected: dim, actual: queries.len() % dim });
    }
    for q in queries.chunks_exact(dim) {
        space.validate(q)?;
    }
    Ok(queries.len() / dim)
}

macro_rules! index_common {
    ($name:ident, $destroy:ident, $slot_count:ident, $slots:ident) => {
        impl Drop for $name {
            fn drop(&mut self) {
                // SAFETY: the handle came from the matching create call and is dropped once.
                unsafe { ffi::$destroy(self.raw.as_ptr()) };
            }
        }

        impl std::fmt::Debug for $name {
            fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
                f.debug_struct(stringify!($name)).field("space", &self.space).field("len", &self.len()).finish()
            }
        }

        // SAFETY: searches on one handle are re-entrant from many threads (the
        // library leases a stream and scratch per call and orders searches
        // against mutations with a shared lock); mutations take `&mut self`.
        unsafe impl Send for $name {}
        // SAFETY: as above.
        unsafe impl Sync for $name {}

        impl $name {
            /// The accept mask of `filter` over the current slot table.
            fn mask(&self, filter: &dyn Filter) -> Result<Vec<u8>> {
                // SAFETY: read-only calls on a live handle into buffers of the reported size.
                let n = unsafe { ffi::$slot_count(self.raw.as_ptr()) } as usize;
                let mut ids = vec![0u64; n];
                let mut live = vec![0u8; n];
                check(unsafe { ffi::$slots(self.raw.as_ptr(), ids.as_mut_ptr(), live.as_mut_ptr()) })?;
                Ok(accept_mask(&ids, &live, &self.meta, filter))
            }

            /// The vector space of this index.
            pub fn space(&self) -> &VectorSpace {
                &self.space
            }
        }
    };
}

// ---------------------------------------------------------------------------
// Flat
// ---------------------------------------------------------------------------

/// Exact search on the GPU: replaces `FlatIndex` (flat.rs:68-236).
pub struct GpuFlatIndex {
    raw: NonNull<ffi::PxgFlat>,
    space: VectorSpace,
    meta: HashMap<VectorId, Metadata>,
}

index_common!(GpuFlatIndex, pxg_flat_destroy, pxg_flat_slot_count, pxg_flat_slots);

impl GpuFlatIndex {
    /// An empty index over `space` (flat.rs:72-77).
    pub fn new(space: VectorSpace) -> Result<Self> {
        Self::with_capacity(space, 0)
    }

    /// An empty index with room for `capacity` vectors (flat.rs:79-84).
    pub fn with_capacity(space: VectorSpace, capacity: usize) -> Result<Self> {
        let mut raw = ptr::null_mut();
        // SAFETY: out-pointer to a handle the library allocates.
        check(unsafe { ffi::pxg_flat_create(space.dim() as u32, metric_code(space.metric()), capacity as u64, &mut raw) })?;
        let raw = NonNull::new(raw).ok_or(ProximaError::Internal { location: "GpuFlatIndex::new", detail: "null handle".into() })?;
        Ok(GpuFlatIndex { raw, space, meta: HashMap::new() })
    }

    /// Insert a batch, all or nothing: `vectors` holds `ids.len()` rows.
    pub fn insert_batch(&mut self, ids: &[VectorId], vectors: &[f32]) -> Result<()> {
        let n = validate_batch(&self.space, vectors)?;
        if n != ids.len() {
            return Err(ProximaError::DimensionMismatch { expected: ids.len() * self.space.dim(), actual: vectors.len() });
        }
        let raw: Vec<u64> = ids.iter().map(|id| id.get()).collect();
        // SAFETY: host arrays of n ids and n * dim floats.
        check(unsafe { ffi::pxg_flat_insert(self.raw.as_ptr(), raw.as_ptr(), vectors.as_ptr(), n as u64, ptr::null_mut()) })?;
        for id in ids {
            self.meta.insert(*id, Metadata::new());
        }
        Ok(())
    }

    /// The stored (prepared) vector of `id` (flat.rs:104-106).
    pub fn vector(&self, id: VectorId) -> Option<Vec<f32>> {
        let mut out = vec![0f32; self.space.dim()];
        // SAFETY: out holds dim floats.
        let st = unsafe { ffi::pxg_flat_get_vector(self.raw.as_ptr(), id.get(), out.as_mut_ptr()) };
        (st == 0).then_some(out)
    }

    /// Search many queries (rows of `queries`) in one call.
    pub fn search_batch(&self, queries: &[f32], k: usize, filter: Option<&dyn Filter>) -> Result<Vec<Vec<SearchResult>>> {
        check_k(k)?;
        let nq = validate_batch(&self.space, queries)?;
        let kq = k.min(self.len());
        let mask = filter.map(|f| self.mask(f)).transpose()?;
        let (mut ids, mut dist, mut count) = (vec![0u64; nq * kq], vec![0f32; nq * kq], vec![0u32; nq]);
        // SAFETY: queries hold nq rows; the outputs hold nq rows of kq; the mask one byte per slot.
        check(unsafe {
            ffi::pxg_flat_search(self.raw.as_ptr(), queries.as_ptr(), nq as u64, kq as u64,
                mask.as_ref().map_or(ptr::null(), |m| m.as_ptr()), ids.as_mut_ptr(), dist.as_mut_ptr(), count.as_mut_ptr())
        })?;
        Ok(unpack(&ids, &dist, &count, kq))
    }

    fn search_one(&self, query: &[f32], k: usize, filter: Option<&dyn Filter>) -> Result<Vec<SearchResult>> {
        check_k(k)?;  // first, as flat.rs:153-155 and ivfpq.rs:988
        self.space.validate(query)?;
        Ok(self.search_batch(query, k, filter)?.pop().unwrap_or_default())
    }
}

impl VectorIndex for GpuFlatIndex {
    fn insert(&mut self, id: VectorId, vector: &[f32], metadata: Metadata) -> Result<()> {
        self.space.validate(vector)?;
        let raw = id.get();
        // SAFETY: one id and one row of dim floats.
        check(unsafe { ffi::pxg_flat_insert(self.raw.as_ptr(), &raw, vector.as_ptr(), 1, ptr::null_mut()) })?;
        self.meta.insert(id, metadata);
        Ok(())
    }

    fn remove(&mut self, id: VectorId) -> Result<()> {
        // SAFETY: plain value call on a live handle.
        check(unsafe { ffi::pxg_flat_remove(self.raw.as_ptr(), id.get()) })?;
        self.meta.remove(&id);
        Ok(())
    }

    fn search(&self, query: &[f32], k: usize, filter: &dyn Filter) -> Result<Vec<SearchResult>> {
        self.search_one(query, k, Some(filter))
    }

    fn search_all(&self, query: &[f32], k: usize) -> Result<Vec<SearchResult>> {
        self.search_one(query, k, None)
    }

    fn contains(&self, id: VectorId) -> bool {
        // SAFETY: plain value call on a live handle.
        unsafe { ffi::pxg_flat_contains(self.raw.as_ptr(), id.get()) != 0 }
    }

    fn len(&self) -> usize {
        // SAFETY: plain value call on a live handle.
        unsafe { ffi::pxg_flat_len(self.raw.as_ptr()) as usize }
    }

    fn stats(&self) -> IndexStats {
        let mut s = ffi::PxgIndexStats::default();
        // SAFETY: out-pointer to a plain struct.
        let _ = unsafe { ffi::pxg_flat_stats(self.raw.as_ptr(), &mut s) };
        to_stats(&s, self.space.metric())
    }
}

// ---------------------------------------------------------------------------
// IVF-PQ
// ---------------------------------------------------------------------------

/// The IVF-PQ index on the GPU: replaces `IvfPqIndex` (ivfpq.rs:452-1228).
pub struct GpuIvfPqIndex {
    raw: NonNull<ffi::PxgIvfPq>,
    space: VectorSpace,
    config: IvfPqConfig,
    meta: HashMap<VectorId, Metadata>,
}

index_common!(GpuIvfPqIndex, pxg_ivfpq_destroy, pxg_ivfpq_slot_count, pxg_ivfpq_slots);

fn report_from(r: &ffi::PxgTrainingReport) -> TrainingReport {
    TrainingReport {
        sampled: r.sampled as usize,
        coarse_inertia: r.coarse_inertia,
        coarse_iterations: r.coarse_iterations as usize,
        residual_inertia: r.residual_inertia,
        populated_lists: r.populated_lists as usize,
        largest_list: r.largest_list as usize,
    }
}

impl GpuIvfPqIndex {
    /// `IvfPqIndex::new` (ivfpq.rs:481-509): Euclidean or cosine, the config
    /// validated as `IvfPqConfig::validate` (ivfpq.rs:259-304).
    pub fn new(space: VectorSpace, config: IvfPqConfig) -> Result<Self> {
        config.validate(space.dim())?;
        let c = ffi::PxgIvfPqConfig {
            nlist: config.nlist() as u64,
            subspaces: config.subspaces() as u64,
            nprobe: config.nprobe() as u64,
            rerank: config.rerank() as u64,
            seed: config.seed(),
            max_iterations: config.max_iterations() as u64,
            training_sample: config.training_sample() as u64,
            train_threshold: config.train_threshold() as u64,
            retain_vectors: i32::from(config.retain_vectors()),
        };
        let mut raw = ptr::null_mut();
        // SAFETY: a plain config struct in, a handle out.
        check(unsafe { ffi::pxg_ivfpq_create(space.dim() as u32, metric_code(space.metric()), &c, &mut raw) })?;
        let raw = NonNull::new(raw).ok_or(ProximaError::Internal { location: "GpuIvfPqIndex::new", detail: "null handle".into() })?;
        Ok(GpuIvfPqIndex { raw, space, config, meta: HashMap::new() })
    }

    /// The configuration this index was built with.
    pub fn config(&self) -> &IvfPqConfig {
        &self.config
    }

    /// `IvfPqIndex::train` (ivfpq.rs:735-825) on the GPU.
    pub fn train(&mut self) -> Result<TrainingReport> {
        let mut r = ffi::PxgTrainingReport::default();
        // SAFETY: out-pointer to a plain struct.
        check(unsafe { ffi::pxg_ivfpq_train(self.raw.as_ptr(), &mut r) })?;
        Ok(report_from(&r))
    }

    /// `true` once the codebooks exist.
    pub fn is_trained(&self) -> bool {
        // SAFETY: plain value call on a live handle.
        unsafe { ffi::pxg_ivfpq_is_trained(self.raw.as_ptr()) != 0 }
    }

    /// `IvfPqIndex::compact` (ivfpq.rs:907-975): slots reclaimed.
    pub fn compact(&mut self) -> Result<usize> {
        let mut reclaimed = 0u64;
        // SAFETY: out-pointer to a u64.
        check(unsafe { ffi::pxg_ivfpq_compact(self.raw.as_ptr(), &mut reclaimed) })?;
        Ok(reclaimed as usize)
    }

    /// Entries per inverted list (ivfpq.rs:567-569).
    pub fn list_lengths(&self) -> Vec<usize> {
        // SAFETY: the output holds list_count() entries.
        let n = unsafe { ffi::pxg_ivfpq_list_count(self.raw.as_ptr()) } as usize;
        let mut out = vec![0u64; n];
        let _ = unsafe { ffi::pxg_ivfpq_list_lengths(self.raw.as_ptr(), out.as_mut_ptr()) };
        out.into_iter().map(|x| x as usize).collect()
    }

    /// `search_with_nprobe` (ivfpq.rs:981-996) over many queries.
    pub fn search_batch(&self, queries: &[f32], k: usize, nprobe: usize, filter: Option<&dyn Filter>) -> Result<Vec<Vec<SearchResult>>> {
        check_k(k)?;
        let nq = validate_batch(&self.space, queries)?;
        let kq = k.min(self.len());
        let mask = filter.map(|f| self.mask(f)).transpose()?;
        let (mut ids, mut dist, mut count) = (vec![0u64; nq * kq], vec![0f32; nq * kq], vec![0u32; nq]);
        // SAFETY: as GpuFlatIndex::search_batch.
        check(unsafe {
            ffi::pxg_ivfpq_search(self.raw.as_ptr(), queries.as_ptr(), nq as u64, kq as u64, nprobe.max(1) as u64,
                mask.as_ref().map_or(ptr::null(), |m| m.as_ptr()), ids.as_mut_ptr(), dist.as_mut_ptr(), count.as_mut_ptr())
        })?;
        Ok(unpack(&ids, &dist, &count, kq))
    }

    /// `IvfPqIndex::search_with_nprobe` (ivfpq.rs:981-996).
    pub fn search_with_nprobe(&self, query: &[f32], k: usize, nprobe: usize, filter: &dyn Filter) -> Result<Vec<SearchResult>> {
        check_k(k)?;  // first, as flat.rs:153-155 and ivfpq.rs:988
        self.space.validate(query)?;
        Ok(self.search_batch(query, k, nprobe, Some(filter))?.pop().unwrap_or_default())
    }
}

impl VectorIndex for GpuIvfPqIndex {
    fn insert(&mut self, id: VectorId, vector: &[f32], metadata: Metadata) -> Result<()> {
        self.space.validate(vector)?;
        let raw = id.get();
        // SAFETY: one id and one row of dim floats.
        check(unsafe { ffi::pxg_ivfpq_insert(self.raw.as_ptr(), &raw, vector.as_ptr(), 1, ptr::null_mut()) })?;
        self.meta.insert(id, metadata);
        Ok(())
    }

    fn remove(&mut self, id: VectorId) -> Result<()> {
        // SAFETY: plain value call on a live handle.
        check(unsafe { ffi::pxg_ivfpq_remove(self.raw.as_ptr(), id.get()) })?;
        self.meta.remove(&id);
        Ok(())
    }

    fn search(&self, query: &[f32], k: usize, filter: &dyn Filter) -> Result<Vec<SearchResult>> {
        self.search_with_nprobe(query, k, self.config.nprobe(), filter)
    }

    fn search_all(&self, query: &[f32], k: usize) -> Result<Vec<SearchResult>> {
        check_k(k)?;  // first, as flat.rs:153-155 and ivfpq.rs:988
        self.space.validate(query)?;
        Ok(self.search_batch(query, k, self.config.nprobe(), None)?.pop().unwrap_or_default())
    }

    fn contains(&self, id: VectorId) -> bool {
        // SAFETY: plain value call on a live handle.
        unsafe { ffi::pxg_ivfpq_contains(self.raw.as_ptr(), id.get()) != 0 }
    }

    fn len(&self) -> usize {
        // SAFETY: plain value call on a live handle.
        unsafe { ffi::pxg_ivfpq_len(self.raw.as_ptr()) as usize }
    }

    fn stats(&self) -> IndexStats {
        let mut s = ffi::PxgIndexStats::default();
        // SAFETY: out-pointer to a plain struct.
        let _ = unsafe { ffi::pxg_ivfpq_stats(self.raw.as_ptr(), &mut s) };
        to_stats(&s, self.space.metric())
    }
}

// ---------------------------------------------------------------------------
// SQ8
// ---------------------------------------------------------------------------

/// Flat search over I8 scalar codes on integer matrix cores. Ranges are
/// fitted per dimension (`RangeMode::PerDimension`, scalar.rs:58-74) with
/// [`GpuSq8Index::train`] or taken from a `ScalarQuantizer` with
/// [`GpuSq8Index::set_ranges`].
pub struct GpuSq8Index {
    raw: NonNull<ffi::PxgSq8>,
    space: VectorSpace,
    meta: HashMap<VectorId, Metadata>,
    rescore: usize,
}

index_common!(GpuSq8Index, pxg_sq8_destroy, pxg_sq8_slot_count, pxg_sq8_slots);

impl GpuSq8Index {
    /// An empty index (inner product or cosine); `rescore` > 0 rescores the
    /// best `max(k, rescore)` by integer score with
    /// `asymmetric_inner_product` (scalar.rs:313-319).
    pub fn new(space: VectorSpace, rescore: usize) -> Result<Self> {
        let mut raw = ptr::null_mut();
        // SAFETY: a handle out.
        check(unsafe { ffi::pxg_sq8_create(space.dim() as u32, metric_code(space.metric()), 1, 0, &mut raw) })?;
        let raw = NonNull::new(raw).ok_or(ProximaError::Internal { location: "GpuSq8Index::new", detail: "null handle".into() })?;
        Ok(GpuSq8Index { raw, space, meta: HashMap::new(), rescore })
    }

    /// Fit the ranges to `training` (rows of dim floats), `ScalarQuantizer::train` (scalar.rs:141-199).
    pub fn train(&mut self, training: &[f32]) -> Result<()> {
        let n = validate_batch(&self.space, training)?;
        // SAFETY: n rows of dim floats.
        check(unsafe { ffi::pxg_sq8_train(self.raw.as_ptr(), training.as_ptr(), n as u64) })
    }

    /// Use a quantizer's per-dimension `min`, `scale` and `inverse_scale`.
    pub fn set_ranges(&mut self, min: &[f32], scale: &[f32], inverse_scale: &[f32]) -> Result<()> {
        let d = self.space.dim();
        if min.len() != d || scale.len() != d || inverse_scale.len() != d {
            return Err(ProximaError::DimensionMismatch { expected: d, actual: min.len() });
        }
        // SAFETY: three arrays of dim floats.
        check(unsafe { ffi::pxg_sq8_set_ranges(self.raw.as_ptr(), min.as_ptr(), scale.as_ptr(), inverse_scale.as_ptr()) })
    }

    /// Search many queries in one call.
    pub fn search_batch(&self, queries: &[f32], k: usize, filter: Option<&dyn Filter>) -> Result<Vec<Vec<SearchResult>>> {
        check_k(k)?;
        let nq = validate_batch(&self.space, queries)?;
        let kq = k.min(self.len());
        let mask = filter.map(|f| self.mask(f)).transpose()?;
        let (mut ids, mut dist, mut count) = (vec![0u64; nq * kq], vec![0f32; nq * kq], vec![0u32; nq]);
        // SAFETY: as GpuFlatIndex::search_batch.
        check(unsafe {
            ffi::pxg_sq8_search(self.raw.as_ptr(), queries.as_ptr(), nq as u64, kq as u64, self.rescore as u64,
                mask.as_ref().map_or(ptr::null(), |m| m.as_ptr()), ids.as_mut_ptr(), dist.as_mut_ptr(), count.as_mut_ptr())
        })?;
        Ok(unpack(&ids, &dist, &count, kq))
    }
}

impl VectorIndex for GpuSq8Index {
    fn insert(&mut self, id: VectorId, vector: &[f32], metadata: Metadata) -> Result<()> {
        self.space.validate(vector)?;
        let raw = id.get();
        // SAFETY: one id and one row of dim floats.
        check(unsafe { ffi::pxg_sq8_insert(self.raw.as_ptr(), &raw, vector.as_ptr(), 1, ptr::null_mut()) })?;
        self.meta.insert(id, metadata);
        Ok(())
    }

    fn remove(&mut self, id: VectorId) -> Result<()> {
        // SAFETY: plain value call on a live handle.
        check(unsafe { ffi::pxg_sq8_remove(self.raw.as_ptr(), id.get()) })?;
        self.meta.remove(&id);
        Ok(())
    }

    fn search(&self, query: &[f32], k: usize, filter: &dyn Filter) -> Result<Vec<SearchResult>> {
        check_k(k)?;  // first, as flat.rs:153-155 and ivfpq.rs:988
        self.space.validate(query)?;
        Ok(self.search_batch(query, k, Some(filter))?.pop().unwrap_or_default())
    }

    fn search_all(&self, query: &[f32], k: usize) -> Result<Vec<SearchResult>> {
        check_k(k)?;  // first, as flat.rs:153-155 and ivfpq.rs:988
        self.space.validate(query)?;
        Ok(self.search_batch(query, k, None)?.pop().unwrap_or_default())
    }

    fn contains(&self, id: VectorId) -> bool {
        // SAFETY: plain value call on a live handle.
        unsafe { ffi::pxg_sq8_contains(self.raw.as_ptr(), id.get()) != 0 }
    }

    fn len(&self) -> usize {
        // SAFETY: plain value call on a live handle.
        unsafe { ffi::pxg_sq8_len(self.raw.as_ptr()) as usize }
    }

    fn stats(&self) -> IndexStats {
        let mut s = ffi::PxgIndexStats::default();
        // SAFETY: out-pointer to a plain struct.
        let _ = unsafe { ffi::pxg_sq8_stats(self.raw.as_ptr(), &mut s) };
        to_stats(&s, self.space.metric())
    }
}

/// Visible GPUs (0 when none); never fails.
pub fn device_count() -> usize {
    // SAFETY: no arguments.
    usize::try_from(unsafe { ffi::pxg_device_count() }).unwrap_or(0)
}
