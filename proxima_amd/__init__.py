"""proxima_amd: the MI355X hot path of Liona-orph/proxima.

A host-side mirror of the reference's index API (crates/proxima-index:
`VectorIndex`, `FlatIndex`, `IvfPqIndex`, `recall_at_k`; crates/proxima-core:
`Metric`, `VectorSpace`, `SearchResult`, `ProximaError`) over the C ABI of
libproxima_hip.so. Every search, train and encode runs in the HIP library on
the GPU; this module only marshals arguments, evaluates filters into per-slot
accept masks, and keeps metadata (which never reaches the device).
"""
import ctypes as C
from collections import namedtuple

import numpy as np

from ._capi import IndexStats as _IndexStatsC
from ._capi import Timings as _TimingsC
from ._capi import lib as _lib

__all__ = [
    "Metric", "VectorSpace", "SearchResult", "IndexStats", "ProximaError", "DimensionMismatch", "UnknownId",
    "DuplicateId", "Capacity", "NonFinite", "Corruption", "Configuration", "Internal", "FlatIndex", "check_k",
    "set_profiling", "last_timings",
]


def set_profiling(enabled):
    """Record per-stage device timings (hipEvents) for subsequent calls."""
    _lib.pxg_set_profiling(1 if enabled else 0)


def last_timings():
    """Stage timings (ms) of the last search/train on this thread."""
    t = _TimingsC()
    _lib.pxg_last_timings(C.byref(t))
    return {f: getattr(t, f) for f, _ in t._fields_}


# --- Metric: distance.rs:90-118 ----------------------------------------------------
class Metric:
    EUCLIDEAN = 0
    COSINE = 1
    INNER_PRODUCT = 2
    MANHATTAN = 3
    ALL = (0, 1, 2, 3)
    _NAMES = {0: "euclidean", 1: "cosine", 2: "inner_product", 3: "manhattan"}

    @staticmethod
    def name(m):
        return Metric._NAMES[m]

    @staticmethod
    def from_name(name):  # distance.rs:193-201
        for k, v in Metric._NAMES.items():
            if v == name:
                return k
        return None

    @staticmethod
    def to_true_distance(m, score):  # distance.rs:167-173
        if m == Metric.EUCLIDEAN:
            return float(np.sqrt(np.float32(score)))
        if m == Metric.INNER_PRODUCT:
            return -score
        return score


# --- ProximaError: error.rs:37-160 --------------------------------------------------
class ProximaError(Exception):
    status = None

    def __init__(self, message, a=0, b=0, value=0.0):
        super().__init__(message)
        self.a, self.b, self.value = a, b, value


class DimensionMismatch(ProximaError):
    status = 1

    @property
    def expected(self):
        return self.a

    @property
    def actual(self):
        return self.b


class UnknownId(ProximaError):
    status = 2

    @property
    def id(self):
        return self.a


class DuplicateId(ProximaError):
    status = 3

    @property
    def id(self):
        return self.a


class Capacity(ProximaError):
    status = 4

    def __init__(self, message, a=0, b=0, value=0.0, what=None):
        super().__init__(message, a, b, value)
        self.what = what  # Capacity{what}: the structure that ran out of room

    @property
    def limit(self):
        return self.a


class NonFinite(ProximaError):
    status = 5

    @property
    def index(self):
        return self.a


class Corruption(ProximaError):
    status = 6


class Configuration(ProximaError):
    status = 7

    def __init__(self, message, a=0, b=0, value=0.0, parameter=None, reason=None):
        super().__init__(message, a, b, value)
        self.parameter = parameter  # Configuration{parameter}, e.g. "k", "nprobe"
        self.reason = reason        # Configuration{reason}: the constraint that was broken


class Internal(ProximaError):
    status = 8


_BY_STATUS = {c.status: c for c in (DimensionMismatch, UnknownId, DuplicateId, Capacity, NonFinite, Corruption,
                                    Configuration, Internal)}


def _check(status):
    if status == 0:
        return
    a, b, v = C.c_uint64(), C.c_uint64(), C.c_float()
    _lib.pxg_last_error_detail(C.byref(a), C.byref(b), C.byref(v))
    msg = _lib.pxg_last_error_message().decode()
    cls = _BY_STATUS.get(status, Internal)
    err = cls(msg, a.value, b.value, v.value)
    if cls is Configuration:
        err.parameter = _lib.pxg_last_error_parameter().decode() or None
        err.reason = _lib.pxg_last_error_reason().decode() or None
    elif cls is Capacity:
        err.what = _lib.pxg_last_error_parameter().decode() or None
    raise err


def _config(parameter, value, reason):
    e = Configuration(f"invalid configuration: {parameter} = {value} ({reason})", value if isinstance(value, int)
                      else 0, parameter=parameter, reason=reason)
    return e


def check_k(k):  # index.rs:212-224
    if k > (1 << 24):
        raise _config("k", k, "exceeds the 16777216 result ceiling")


# --- VectorSpace: space.rs:53-162 ----------------------------------------------------
class VectorSpace:
    MAX_DIM = 1 << 20

    def __init__(self, dim, metric):
        if dim < 1:
            raise _config("dim", dim, "must be at least 1; a 0-dimensional space makes all distances equal")
        if dim > self.MAX_DIM:
            raise _config("dim", dim, "exceeds the 1048576 dimension ceiling")
        if metric not in Metric.ALL:
            raise _config("metric", metric, "unknown metric")
        self.dim = dim
        self.metric = metric

    def validate(self, vector):  # space.rs:104-121
        v = np.asarray(vector, dtype=np.float32).reshape(-1)
        if v.size != self.dim:
            raise DimensionMismatch(
                f"dimension mismatch: index holds {self.dim}-dimensional vectors, got {v.size}", self.dim, v.size)
        bad = np.flatnonzero(~np.isfinite(v))
        if bad.size:
            i = int(bad[0])
            raise NonFinite(f"vector component {i} is not finite ({v[i]})", i, 0, float(v[i]))
        return v

    def __str__(self):
        return f"{self.dim}d/{Metric.name(self.metric)}"

    def __eq__(self, other):
        return isinstance(other, VectorSpace) and (self.dim, self.metric) == (other.dim, other.metric)


SearchResult = namedtuple("SearchResult", ["id", "distance"])  # topk.rs:33-40


class IndexStats(namedtuple("IndexStats", ["len", "deleted", "dim", "metric", "layers", "nodes_per_layer", "edges",
                                           "vector_bytes", "graph_bytes"])):
    """index.rs:68-130."""

    def mean_degree(self):
        return 0.0 if self.len + self.deleted == 0 else self.edges / (self.len + self.deleted)

    def total_bytes(self):
        return self.vector_bytes + self.graph_bytes

    def bytes_per_vector(self):
        return 0.0 if self.len == 0 else self.total_bytes() / self.len


def _stats_from_c(s):
    return IndexStats(s.len, s.deleted, s.dim, s.metric, s.layers, [s.len], s.edges, s.vector_bytes, s.graph_bytes)


def _ptr(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _rows(vectors, dim):
    v = np.ascontiguousarray(vectors, dtype=np.float32)
    if v.ndim == 1:
        if v.size % dim != 0 or (v.size != dim and v.size == 0):
            raise DimensionMismatch(
                f"dimension mismatch: index holds {dim}-dimensional vectors, got {v.size}", dim, v.size)
        v = v.reshape(-1, dim)
    if v.shape[-1] != dim:
        raise DimensionMismatch(
            f"dimension mismatch: index holds {dim}-dimensional vectors, got {v.shape[-1]}", dim, v.shape[-1])
    return np.ascontiguousarray(v.reshape(-1, dim))


def _device_ptr(t):
    """Device address of a torch CUDA/HIP tensor (must be contiguous)."""
    if not t.is_contiguous():
        raise ValueError("device tensors must be contiguous")
    return C.c_void_p(t.data_ptr())


# --- the VectorIndex trait surface shared by every index ------------------------------
class _IndexBase:
    """VectorIndex (index.rs:154-205): insert / remove / search / contains / len /
    stats, the provided upsert and search_all, plus search_batch."""

    def upsert(self, id, vector, metadata=None):  # index.rs:194-199
        if self.contains(id):
            self.remove(id)
        self.insert(id, vector, metadata)

    def search_all(self, query, k):  # index.rs:202-204
        return self.search(query, k, None)

    def is_empty(self):
        return len(self) == 0

    def search(self, query, k, filter=None):
        ids, dists, counts = self.search_batch(np.asarray(query, dtype=np.float32).reshape(1, -1), k, filter)
        return [SearchResult(int(ids[0, i]), float(dists[0, i])) for i in range(int(counts[0]))]

    # metadata stays on the host; filters see it
    def metadata(self, id):
        if not self.contains(id):
            return None
        return self._meta.get(id, {})

    def set_metadata(self, id, metadata):
        if not self.contains(id):
            raise UnknownId(f"unknown vector id {id}", id)
        self._meta[id] = dict(metadata or {})

    def _accept_mask(self, filter, slot_ids, live):
        """Evaluate Filter::accepts over live slots (index.rs:27-35) into one byte per slot."""
        if filter is None:
            return None
        acc = np.zeros(slot_ids.size, np.uint8)
        for s in np.flatnonzero(live):
            i = int(slot_ids[s])
            acc[s] = 1 if filter(i, self._meta.get(i, {})) else 0
        return acc


# --- FlatIndex: flat.rs:68-236 ------------------------------------------------------------
class FlatIndex(_IndexBase):
    """Exact search over a device-resident slot-major store (GPU FlatIndex)."""

    def __init__(self, space, capacity=0):
        self.space = space
        h = C.c_void_p()
        _check(_lib.pxg_flat_create(space.dim, space.metric, capacity, C.byref(h)))
        self._h = h
        self._meta = {}

    @classmethod
    def with_capacity(cls, space, capacity):
        return cls(space, capacity)

    @classmethod
    def from_array(cls, space, data):  # TryFrom<(&VectorSpace, &[f32])>, flat.rs:215-236
        data = np.asarray(data, dtype=np.float32).reshape(-1)
        if data.size % space.dim != 0:
            raise _config("data", data.size, "must be a multiple of the space dimension")
        n = data.size // space.dim
        idx = cls(space, n)
        if n:
            idx.insert_batch(np.arange(n, dtype=np.uint64), data.reshape(n, space.dim))
        return idx

    def __del__(self):
        h = getattr(self, "_h", None)
        # at interpreter exit the module's globals may already be cleared;
        # the process is ending and its device memory goes with it
        if h and _lib is not None:
            _lib.pxg_flat_destroy(h)
            self._h = None

    # -- mutation (exclusive) --
    def insert(self, id, vector, metadata=None):
        v = np.asarray(vector, dtype=np.float32).reshape(-1)
        if v.size != self.space.dim:
            raise DimensionMismatch(
                f"dimension mismatch: index holds {self.space.dim}-dimensional vectors, got {v.size}",
                self.space.dim, v.size)
        self.insert_batch(np.array([id], np.uint64), v.reshape(1, -1))
        if metadata:
            self._meta[int(id)] = dict(metadata)

    def insert_batch(self, ids, vectors):
        ids = np.ascontiguousarray(ids, dtype=np.uint64).reshape(-1)
        v = _rows(vectors, self.space.dim)
        if v.shape[0] != ids.size:
            raise ValueError("ids and vectors disagree on the batch size")
        slots = np.zeros(ids.size, np.uint32)
        _check(_lib.pxg_flat_insert(self._h, _ptr(ids), _ptr(v), ids.size, _ptr(slots)))
        return slots

    def insert_device(self, ids, vectors):
        """Bulk insert from a contiguous GPU tensor [n, dim] (ids on the host)."""
        ids = np.ascontiguousarray(ids, dtype=np.uint64).reshape(-1)
        if vectors.shape[-1] != self.space.dim or vectors.shape[0] != ids.size:
            raise DimensionMismatch("dimension mismatch: device batch does not match the index", self.space.dim,
                                    vectors.shape[-1])
        slots = np.zeros(ids.size, np.uint32)
        _check(_lib.pxg_flat_insert_device(self._h, _ptr(ids), _device_ptr(vectors), ids.size, _ptr(slots)))
        return slots

    def remove(self, id):
        _check(_lib.pxg_flat_remove(self._h, int(id)))
        self._meta.pop(int(id), None)

    # -- queries --
    def contains(self, id):
        return bool(_lib.pxg_flat_contains(self._h, int(id)))

    def __len__(self):
        return int(_lib.pxg_flat_len(self._h))

    def stats(self):
        s = _IndexStatsC()
        _check(_lib.pxg_flat_stats(self._h, C.byref(s)))
        return _stats_from_c(s)

    def vector(self, id):
        out = np.zeros(self.space.dim, np.float32)
        try:
            _check(_lib.pxg_flat_get_vector(self._h, int(id), _ptr(out)))
        except UnknownId:
            return None
        return out

    def slots(self):
        n = int(_lib.pxg_flat_slot_count(self._h))
        ids = np.zeros(max(n, 1), np.uint64)
        live = np.zeros(max(n, 1), np.uint8)
        _check(_lib.pxg_flat_slots(self._h, _ptr(ids), _ptr(live)))
        return ids[:n], live[:n]

    def ids(self):
        """Live ids in slot order (flat.rs:118-120)."""
        ids, live = self.slots()
        return [int(i) for i in ids[live.astype(bool)]]

    def set_search_mode(self, mode):
        _check(_lib.pxg_flat_set_search_mode(self._h, mode))

    def search_batch(self, queries, k, filter=None):
        """Batched VectorIndex::search: returns (ids[nq,k], dists[nq,k], counts[nq])."""
        check_k(k)
        q = _rows(queries, self.space.dim)
        nq = q.shape[0]
        acc = None
        if filter is not None:
            sid, live = self.slots()
            acc = self._accept_mask(filter, sid, live)
        kk = max(k, 1)
        oi = np.zeros((nq, kk), np.uint64)
        od = np.zeros((nq, kk), np.float32)
        oc = np.zeros(max(nq, 1), np.uint32)
        _check(_lib.pxg_flat_search(self._h, _ptr(q), nq, k, _ptr(acc), _ptr(oi), _ptr(od), _ptr(oc)))
        return oi[:, :k] if k else oi[:, :0], od[:, :k] if k else od[:, :0], oc[:nq]

    def search_device(self, queries, k, out_ids, out_dist, out_count, accept=None, stream=None):
        """Device-pointer search: torch tensors on the GPU (queries f32 [nq, dim],
        out_ids int64 [nq, k], out_dist f32 [nq, k], out_count int32 [nq])."""
        _check(_lib.pxg_flat_search_device(
            self._h, _device_ptr(queries), queries.shape[0], k, None if accept is None else _device_ptr(accept),
            _device_ptr(out_ids), _device_ptr(out_dist), _device_ptr(out_count),
            None if stream is None else C.c_void_p(stream)))

    @staticmethod
    def last_fallbacks():
        return int(_lib.pxg_flat_last_fallbacks())

    def exact_ids(self, query, k, filter=None):  # flat.rs:201-212
        return [r.id for r in self.search(query, k, filter)]


# --- IvfPqConfig / IvfPqIndex: ivfpq.rs:106-1228 -----------------------------------
from ._capi import IvfPqConfigC as _IvfPqConfigC  # noqa: E402
from ._capi import TrainingReportC as _TrainingReportC  # noqa: E402

TrainingReport = namedtuple("TrainingReport", ["sampled", "coarse_inertia", "coarse_iterations", "residual_inertia",
                                               "populated_lists", "largest_list"])  # ivfpq.rs:322-357


class IvfPqConfig:
    """Builder mirroring IvfPqConfig (ivfpq.rs:106-304)."""

    def __init__(self, nlist, subspaces):
        c = _IvfPqConfigC()
        _check(_lib.pxg_ivfpq_config_default(nlist, subspaces, C.byref(c)))
        self._c = c

    def _with(self, field, value):
        setattr(self._c, field, value)
        return self

    def with_nprobe(self, v):
        return self._with("nprobe", v)

    def with_rerank(self, v):
        return self._with("rerank", v)

    def with_seed(self, v):
        return self._with("seed", v)

    def with_max_iterations(self, v):
        return self._with("max_iterations", v)

    def with_training_sample(self, v):
        return self._with("training_sample", v)

    def with_train_threshold(self, v):
        return self._with("train_threshold", min(int(v), (1 << 64) - 1))

    def with_retain_vectors(self, v):
        return self._with("retain_vectors", 1 if v else 0)

    def __getattr__(self, name):
        if name.startswith("_"):
            raise AttributeError(name)
        v = getattr(self._c, name)
        return bool(v) if name == "retain_vectors" else v

    def clone(self):
        o = IvfPqConfig.__new__(IvfPqConfig)
        o._c = _IvfPqConfigC()
        C.memmove(C.byref(o._c), C.byref(self._c), C.sizeof(_IvfPqConfigC))
        return o


def _report(r):
    return TrainingReport(r.sampled, r.coarse_inertia, r.coarse_iterations, r.residual_inertia, r.populated_lists,
                          r.largest_list)


class IvfPqIndex(_IndexBase):
    """GPU IVF-PQ (ivfpq.rs:452-1228): coarse lists, residual PQ codes, ADC scan."""

    def __init__(self, space, config):
        self.space = space
        self.config = config
        h = C.c_void_p()
        _check(_lib.pxg_ivfpq_create(space.dim, space.metric, C.byref(config._c), C.byref(h)))
        self._h = h
        self._meta = {}

    def __del__(self):
        h = getattr(self, "_h", None)
        # at interpreter exit the module's globals may already be cleared;
        # the process is ending and its device memory goes with it
        if h and _lib is not None:
            _lib.pxg_ivfpq_destroy(h)
            self._h = None

    def insert(self, id, vector, metadata=None):
        v = np.asarray(vector, dtype=np.float32).reshape(-1)
        if v.size != self.space.dim:
            raise DimensionMismatch(
                f"dimension mismatch: index holds {self.space.dim}-dimensional vectors, got {v.size}",
                self.space.dim, v.size)
        self.insert_batch(np.array([id], np.uint64), v.reshape(1, -1))
        if metadata:
            self._meta[int(id)] = dict(metadata)

    def insert_batch(self, ids, vectors):
        ids = np.ascontiguousarray(ids, dtype=np.uint64).reshape(-1)
        v = _rows(vectors, self.space.dim)
        slots = np.zeros(ids.size, np.uint32)
        _check(_lib.pxg_ivfpq_insert(self._h, _ptr(ids), _ptr(v), ids.size, _ptr(slots)))
        return slots

    def insert_device(self, ids, vectors):
        """Bulk insert from a contiguous GPU tensor [n, dim] (ids on the host)."""
        ids = np.ascontiguousarray(ids, dtype=np.uint64).reshape(-1)
        if vectors.shape[-1] != self.space.dim or vectors.shape[0] != ids.size:
            raise DimensionMismatch("dimension mismatch: device batch does not match the index", self.space.dim,
                                    vectors.shape[-1])
        slots = np.zeros(ids.size, np.uint32)
        _check(_lib.pxg_ivfpq_insert_device(self._h, _ptr(ids), _device_ptr(vectors), ids.size, _ptr(slots)))
        return slots

    @staticmethod
    def last_scanned():
        """Code entries streamed by the last search on this thread."""
        return int(_lib.pxg_ivfpq_last_scanned())

    def compact(self):
        """IvfPqIndex::compact (ivfpq.rs:907-975): drop free slots, renumber the
        live ones in slot order; returns the number of slots reclaimed."""
        r = C.c_uint64()
        _check(_lib.pxg_ivfpq_compact(self._h, C.byref(r)))
        return int(r.value)

    def remove(self, id):
        _check(_lib.pxg_ivfpq_remove(self._h, int(id)))
        self._meta.pop(int(id), None)

    def contains(self, id):
        return bool(_lib.pxg_ivfpq_contains(self._h, int(id)))

    def __len__(self):
        return int(_lib.pxg_ivfpq_len(self._h))

    def is_trained(self):
        return bool(_lib.pxg_ivfpq_is_trained(self._h))

    def stats(self):
        s = _IndexStatsC()
        _check(_lib.pxg_ivfpq_stats(self._h, C.byref(s)))
        return _stats_from_c(s)

    def vector_bytes(self):
        return self.stats().vector_bytes

    def compressed_bytes(self):
        return self.stats().graph_bytes

    def code_bytes_per_vector(self):
        return self.config.subspaces

    def vector(self, id):
        out = np.zeros(self.space.dim, np.float32)
        try:
            _check(_lib.pxg_ivfpq_get_vector(self._h, int(id), _ptr(out)))
        except (UnknownId, Configuration):
            return None
        return out

    def slots(self):
        n = int(_lib.pxg_ivfpq_slot_count(self._h))
        ids = np.zeros(max(n, 1), np.uint64)
        live = np.zeros(max(n, 1), np.uint8)
        _check(_lib.pxg_ivfpq_slots(self._h, _ptr(ids), _ptr(live)))
        return ids[:n], live[:n]

    def view_stats(self):
        """(full rebuilds, regions moved) of the list view so far (no reference counterpart)."""
        r, m = C.c_uint64(), C.c_uint64()
        _check(_lib.pxg_ivfpq_view_stats(self._h, C.byref(r), C.byref(m)))
        return int(r.value), int(m.value)

    def list_lengths(self):
        n = int(_lib.pxg_ivfpq_list_count(self._h))
        out = np.zeros(max(n, 1), np.uint64)
        _check(_lib.pxg_ivfpq_list_lengths(self._h, _ptr(out)))
        return [int(x) for x in out[:n]]

    def train(self):
        r = _TrainingReportC()
        _check(_lib.pxg_ivfpq_train(self._h, C.byref(r)))
        return _report(r)

    def training_report(self):
        r = _TrainingReportC()
        try:
            _check(_lib.pxg_ivfpq_training_report(self._h, C.byref(r)))
        except Configuration:
            return None
        return _report(r)

    def parts(self):
        """(centroids, codebooks, codes, list_of) of a trained index (ivfpq.rs:606-617)."""
        nl = int(_lib.pxg_ivfpq_list_count(self._h))
        ns = int(_lib.pxg_ivfpq_slot_count(self._h))
        m = self.config.subspaces
        cents = np.zeros((nl, self.space.dim), np.float32)
        books = np.zeros(256 * self.space.dim, np.float32)
        codes = np.zeros((max(ns, 1), m), np.uint8)
        list_of = np.zeros(max(ns, 1), np.uint32)
        _check(_lib.pxg_ivfpq_parts(self._h, _ptr(cents), _ptr(books), _ptr(codes), _ptr(list_of)))
        return cents, books, codes[:ns], list_of[:ns]

    def load_trained(self, centroids, codebooks, codes=None, list_of=None):
        """IvfPqIndex::from_parts (ivfpq.rs:624-717) onto the inserted vectors."""
        cents = np.ascontiguousarray(centroids, dtype=np.float32)
        books = np.ascontiguousarray(codebooks, dtype=np.float32).reshape(-1)
        c = None if codes is None else np.ascontiguousarray(codes, dtype=np.uint8)
        lo = None if list_of is None else np.ascontiguousarray(list_of, dtype=np.uint32)
        _check(_lib.pxg_ivfpq_load_trained(self._h, _ptr(cents), cents.shape[0], _ptr(books), _ptr(c), _ptr(lo)))

    def search_batch(self, queries, k, filter=None, nprobe=None):
        check_k(k)
        q = _rows(queries, self.space.dim)
        nq = q.shape[0]
        acc = None
        if filter is not None:
            sid, live = self.slots()
            acc = self._accept_mask(filter, sid, live)
        kk = max(k, 1)
        oi = np.zeros((nq, kk), np.uint64)
        od = np.zeros((nq, kk), np.float32)
        oc = np.zeros(max(nq, 1), np.uint32)
        _check(_lib.pxg_ivfpq_search(self._h, _ptr(q), nq, k, 0 if nprobe is None else max(int(nprobe), 1),
                                     _ptr(acc), _ptr(oi), _ptr(od), _ptr(oc)))
        return oi[:, :k], od[:, :k], oc[:nq]

    def search_with_nprobe(self, query, k, nprobe, filter=None):  # ivfpq.rs:981-996
        ids, dists, counts = self.search_batch(np.asarray(query, dtype=np.float32).reshape(1, -1), k, filter,
                                               max(int(nprobe), 1))
        return [SearchResult(int(ids[0, i]), float(dists[0, i])) for i in range(int(counts[0]))]

    def search_device(self, queries, k, out_ids, out_dist, out_count, nprobe=None, accept=None, stream=None):
        _check(_lib.pxg_ivfpq_search_device(
            self._h, _device_ptr(queries), queries.shape[0], k, 0 if nprobe is None else int(nprobe),
            None if accept is None else _device_ptr(accept), _device_ptr(out_ids), _device_ptr(out_dist),
            _device_ptr(out_count), None if stream is None else C.c_void_p(stream)))


# --- k-means / product quantizer (crates/proxima-quantize) ----------------------------
Clustering = namedtuple("Clustering", ["centroids", "inertia", "iterations"])  # kmeans.rs:34-48


def kmeans(points, dim, k, max_iterations, seed):
    """kmeans() (kmeans.rs:59-143) with ChaCha8Rng::seed_from_u64(seed), on the GPU."""
    p = np.ascontiguousarray(points, dtype=np.float32).reshape(-1)
    n = p.size // dim if dim else 0
    kk = max(min(k, n), 1)
    cents = np.zeros(kk * dim, np.float32)
    inertia, iters, kout = C.c_double(), C.c_uint64(), C.c_uint64()
    _check(_lib.pxg_kmeans(_ptr(p), n, dim, k, max_iterations, seed, _ptr(cents), C.byref(inertia), C.byref(iters),
                           C.byref(kout)))
    return Clustering(cents[: int(kout.value) * dim], inertia.value, iters.value)


def kmeans_lloyd(points, init, max_iterations):
    """The Lloyd loop (kmeans.rs:85-136) from the given initial centroids."""
    p = np.ascontiguousarray(points, dtype=np.float32)
    n, dim = p.shape
    init = np.ascontiguousarray(init, dtype=np.float32)
    k = init.shape[0]
    cents = np.zeros((k, dim), np.float32)
    assign = np.zeros(n, np.uint32)
    inertia, iters = C.c_double(), C.c_uint64()
    _check(_lib.pxg_kmeans_lloyd(_ptr(p), n, dim, k, max_iterations, _ptr(init), _ptr(cents), _ptr(assign),
                                 C.byref(inertia), C.byref(iters)))
    return cents, assign, inertia.value, iters.value


def kmeans_device(points, k, max_iterations, seed, centroids_out, assign_out=None, init=None):
    """kmeans() on device-resident data: points a contiguous GPU tensor
    [n, dim] f32, centroids_out [min(k, n), dim] f32 and assign_out [n]
    (int32, may be None) GPU tensors, init None (k-means++ from seed) or a GPU
    tensor of initial centroids. max_iterations = 0 returns the k-means++
    seeds. Returns (inertia, iterations)."""
    n, dim = points.shape
    inertia, iters = C.c_double(), C.c_uint64()
    _check(_lib.pxg_kmeans_device(_device_ptr(points), n, dim, k, max_iterations, seed,
                                  None if init is None else _device_ptr(init), _device_ptr(centroids_out),
                                  None if assign_out is None else _device_ptr(assign_out), C.byref(inertia),
                                  C.byref(iters)))
    return inertia.value, iters.value


def kmeans_last_stats():
    """Counters of this thread's last k-means run (measurement only): MFMA
    distance-pass time (ms) and algorithmic flops, number of passes, points
    rescanned exactly, f64 sums kept in the fixed parallel order."""
    ms, fl = C.c_double(), C.c_double()
    passes, resc, inex = C.c_uint64(), C.c_uint64(), C.c_uint64()
    _check(_lib.pxg_kmeans_last_stats(C.byref(ms), C.byref(fl), C.byref(passes), C.byref(resc), C.byref(inex)))
    return {"mfma_ms": ms.value, "mfma_flops": fl.value, "mfma_passes": passes.value, "rescanned": resc.value,
            "inexact_sums": inex.value}


def kmeans_last_reseeds():
    """Empty-cluster reseeds of this thread's last k-means run: in all, found
    in the candidate pool, and iterations whose pool test failed."""
    r, p, f = C.c_uint64(), C.c_uint64(), C.c_uint64()
    _check(_lib.pxg_kmeans_last_reseeds(C.byref(r), C.byref(p), C.byref(f)))
    return {"reseeds": r.value, "pool": p.value, "pool_fallbacks": f.value}


def kmeans_pp(points, k, seed):
    p = np.ascontiguousarray(points, dtype=np.float32)
    n, dim = p.shape
    cents = np.zeros((k, dim), np.float32)
    _check(_lib.pxg_kmeans_pp(_ptr(p), n, dim, k, seed, _ptr(cents)))
    return cents


def kmeans_assign(points, centroids):
    p = np.ascontiguousarray(points, dtype=np.float32)
    c = np.ascontiguousarray(centroids, dtype=np.float32)
    n, dim = p.shape
    a = np.zeros(n, np.uint32)
    d = np.zeros(n, np.float32)
    _check(_lib.pxg_kmeans_assign(_ptr(p), n, dim, _ptr(c), c.shape[0], _ptr(a), _ptr(d)))
    return a, d


class PqConfig:
    """PqConfig (product.rs:83-132)."""

    def __init__(self, subspaces):
        self.subspaces, self.max_iterations, self.seed = subspaces, 25, 0x5EED1EAF

    def with_seed(self, seed):
        self.seed = seed
        return self

    def with_max_iterations(self, n):
        self.max_iterations = n
        return self


class ProductQuantizer:
    """ProductQuantizer::train / encode (product.rs:198-380) on the GPU."""

    def __init__(self, dim, subspaces, codebooks, training_inertia=0.0, training_iterations=0):
        self.dim, self.subspaces, self.codebooks = dim, subspaces, codebooks
        self.training_inertia, self.training_iterations = training_inertia, training_iterations

    @classmethod
    def train(cls, space, training, config):
        t = np.ascontiguousarray(training, dtype=np.float32).reshape(-1)
        if t.size == 0 or t.size % space.dim:
            raise _config("training", t.size, "must be a non-empty multiple of the space dimension")
        n = t.size // space.dim
        books = np.zeros(256 * space.dim, np.float32)
        inertia, iters = C.c_double(), C.c_uint64()
        _check(_lib.pxg_pq_train(_ptr(t), n, space.dim, config.subspaces, config.max_iterations, config.seed,
                                 _ptr(books), C.byref(inertia), C.byref(iters)))
        return cls(space.dim, config.subspaces, books, inertia.value, iters.value)

    @classmethod
    def train_device(cls, space, training, config, codebooks_out):
        """train() on a contiguous GPU tensor [n, dim]; the codebooks (dim * 256
        f32) are written to the GPU tensor codebooks_out and kept on the host too."""
        if training.shape[-1] != space.dim or training.shape[0] == 0:
            raise _config("training", int(training.numel()), "must be a non-empty multiple of the space dimension")
        inertia, iters = C.c_double(), C.c_uint64()
        _check(_lib.pxg_pq_train_device(_device_ptr(training), training.shape[0], space.dim, config.subspaces,
                                        config.max_iterations, config.seed, _device_ptr(codebooks_out),
                                        C.byref(inertia), C.byref(iters)))
        return cls(space.dim, config.subspaces, codebooks_out.cpu().numpy().reshape(-1), inertia.value, iters.value)

    def code_len(self):
        return self.subspaces

    def compression_ratio(self):
        return self.dim * 4 / self.code_len()

    def encode(self, vectors):
        v = np.ascontiguousarray(vectors, dtype=np.float32).reshape(-1, self.dim)
        out = np.zeros((v.shape[0], self.subspaces), np.uint8)
        _check(_lib.pxg_pq_encode(_ptr(self.codebooks), self.dim, self.subspaces, _ptr(v), v.shape[0], _ptr(out)))
        return out


__all__ += ["IvfPqConfig", "IvfPqIndex", "TrainingReport", "Clustering", "kmeans", "kmeans_device", "kmeans_lloyd", "kmeans_pp", "kmeans_last_stats", "kmeans_last_reseeds",
            "kmeans_assign", "PqConfig", "ProductQuantizer"]


# --- ScalarQuantizer: scalar.rs:25-337 ----------------------------------------------------
class CodeType:
    """CodeType (scalar.rs:25-52): U8 stores the level, I8 stores level - 128."""
    U8 = 0
    I8 = 1


class RangeMode:
    """RangeMode (scalar.rs:58-74)."""
    GLOBAL = 0
    PER_DIMENSION = 1


class ScalarQuantizer:
    """Affine f32 -> one-byte quantizer (scalar.rs:112-337); training, encoding,
    decoding and the asymmetric distances run on the GPU."""

    LEVELS = 256

    def __init__(self, dim, mode, code_type, min, scale, inverse_scale):
        self._dim, self._mode, self._code_type = dim, mode, code_type
        self.min = np.ascontiguousarray(min, dtype=np.float32)
        self.scale = np.ascontiguousarray(scale, dtype=np.float32)
        self.inverse_scale = np.ascontiguousarray(inverse_scale, dtype=np.float32)

    @classmethod
    def train(cls, space, training, mode=RangeMode.PER_DIMENSION, code_type=CodeType.U8):
        t = np.ascontiguousarray(training, dtype=np.float32).reshape(-1)
        if t.size == 0 or t.size % space.dim:
            raise _config("training", t.size, "must be a non-empty multiple of the space dimension")
        g = space.dim if mode == RangeMode.PER_DIMENSION else 1
        mn, sc, inv = (np.zeros(g, np.float32) for _ in range(3))
        _check(_lib.pxg_sq_train(_ptr(t), t.size // space.dim, space.dim, int(mode == RangeMode.PER_DIMENSION),
                                 _ptr(mn), _ptr(sc), _ptr(inv)))
        return cls(space.dim, mode, code_type, mn, sc, inv)

    def dim(self):
        return self._dim

    def code_len(self):
        return self._dim

    def range_mode(self):
        return self._mode

    def code_type(self):
        return self._code_type

    def compression_ratio(self):
        return 4.0

    def table_bytes(self):
        return (self.min.size + self.scale.size + self.inverse_scale.size) * 4

    def _per_dim(self):
        return int(self._mode == RangeMode.PER_DIMENSION)

    def encode(self, vector):
        v = np.asarray(vector, dtype=np.float32).reshape(-1)
        if v.size != self._dim:
            raise DimensionMismatch(f"dimension mismatch: quantizer holds {self._dim} dimensions, got {v.size}",
                                    self._dim, v.size)
        return self.encode_batch(v.reshape(1, -1))[0]

    def encode_batch(self, vectors):
        v = _rows(vectors, self._dim)
        out = np.zeros(v.shape, np.uint8)
        _check(_lib.pxg_sq_encode(_ptr(v), v.shape[0], self._dim, self._per_dim(), self._code_type,
                                  _ptr(self.min), _ptr(self.inverse_scale), _ptr(out)))
        return out

    def decode(self, code):
        c = np.ascontiguousarray(code, dtype=np.uint8).reshape(-1)
        if c.size % self._dim or c.size == 0:
            raise DimensionMismatch(f"dimension mismatch: quantizer holds {self._dim} dimensions, got {c.size}",
                                    self._dim, c.size)
        out = np.zeros(c.size, np.float32)
        _check(_lib.pxg_sq_decode(_ptr(c), c.size // self._dim, self._dim, self._per_dim(), self._code_type,
                                  _ptr(self.min), _ptr(self.scale), _ptr(out)))
        return out.reshape(np.shape(code)) if np.ndim(code) > 1 else out

    def _asym(self, ip, query, codes):
        q = np.ascontiguousarray(query, dtype=np.float32).reshape(-1)
        c = np.ascontiguousarray(codes, dtype=np.uint8).reshape(-1, self._dim)
        out = np.zeros(c.shape[0], np.float32)
        _check(_lib.pxg_sq_asymmetric(ip, _ptr(q), _ptr(c), c.shape[0], self._dim, self._per_dim(),
                                      self._code_type, _ptr(self.min), _ptr(self.scale), _ptr(out)))
        return out if np.ndim(codes) > 1 else float(out[0])

    def asymmetric_squared_l2(self, query, code):  # scalar.rs:298-305
        return self._asym(0, query, code)

    def asymmetric_inner_product(self, query, code):  # scalar.rs:313-319
        return self._asym(1, query, code)


class Sq8Index(_IndexBase):
    """SQ8 flat index over I8 codes on integer MFMA (no reference counterpart:
    the reference has the quantizer, not an SQ index). Score = -(float)S with S
    the exact int32 dot product of the query's and the vector's I8 codes,
    ordered as TopK; `rescore` rescores the best max(rescore, k) with
    asymmetric_inner_product. Ranges are fitted to prepared vectors."""

    def __init__(self, space, mode=RangeMode.PER_DIMENSION, capacity=0):
        self.space = space
        self._mode = mode
        h = C.c_void_p()
        _check(_lib.pxg_sq8_create(space.dim, space.metric, int(mode == RangeMode.PER_DIMENSION), capacity,
                                   C.byref(h)))
        self._h = h
        self._meta = {}

    def __del__(self):
        h = getattr(self, "_h", None)
        # at interpreter exit the module's globals may already be cleared;
        # the process is ending and its device memory goes with it
        if h and _lib is not None:
            _lib.pxg_sq8_destroy(h)
            self._h = None

    @classmethod
    def from_array(cls, space, data, training_sample=100_000, mode=RangeMode.PER_DIMENSION):
        """Train on the first `training_sample` vectors, then insert all with ids 0..n."""
        data = _rows(data, space.dim)
        idx = cls(space, mode, data.shape[0])
        if data.shape[0]:
            idx.train(data[:training_sample])
            idx.insert_batch(np.arange(data.shape[0], dtype=np.uint64), data)
        return idx

    # -- quantizer --
    def train(self, training):
        t = np.ascontiguousarray(training, dtype=np.float32).reshape(-1)
        if t.size == 0 or t.size % self.space.dim:
            raise _config("training", t.size, "must be a non-empty multiple of the space dimension")
        _check(_lib.pxg_sq8_train(self._h, _ptr(t), t.size // self.space.dim))

    def train_device(self, training):
        if training.shape[-1] != self.space.dim:
            raise DimensionMismatch("dimension mismatch: device sample does not match the index", self.space.dim,
                                    training.shape[-1])
        _check(_lib.pxg_sq8_train_device(self._h, _device_ptr(training), training.shape[0]))

    def _groups(self):
        return self.space.dim if self._mode == RangeMode.PER_DIMENSION else 1

    def set_quantizer(self, sq):
        if sq.dim() != self.space.dim or sq.range_mode() != self._mode:
            raise _config("quantizer", sq.dim(), "dimension or range mode differs from the index")
        _check(_lib.pxg_sq8_set_ranges(self._h, _ptr(sq.min), _ptr(sq.scale), _ptr(sq.inverse_scale)))

    def quantizer(self):
        g = self._groups()
        mn, sc, inv = (np.zeros(g, np.float32) for _ in range(3))
        _check(_lib.pxg_sq8_ranges(self._h, _ptr(mn), _ptr(sc), _ptr(inv)))
        return ScalarQuantizer(self.space.dim, self._mode, CodeType.I8, mn, sc, inv)

    def is_trained(self):
        return bool(_lib.pxg_sq8_is_trained(self._h))

    # -- mutation --
    def insert(self, id, vector, metadata=None):
        v = np.asarray(vector, dtype=np.float32).reshape(-1)
        if v.size != self.space.dim:
            raise DimensionMismatch(
                f"dimension mismatch: index holds {self.space.dim}-dimensional vectors, got {v.size}",
                self.space.dim, v.size)
        self.insert_batch(np.array([id], np.uint64), v.reshape(1, -1))
        if metadata:
            self._meta[int(id)] = dict(metadata)

    def insert_batch(self, ids, vectors):
        ids = np.ascontiguousarray(ids, dtype=np.uint64).reshape(-1)
        v = _rows(vectors, self.space.dim)
        if v.shape[0] != ids.size:
            raise ValueError("ids and vectors disagree on the batch size")
        slots = np.zeros(ids.size, np.uint32)
        _check(_lib.pxg_sq8_insert(self._h, _ptr(ids), _ptr(v), ids.size, _ptr(slots)))
        return slots

    def insert_device(self, ids, vectors):
        ids = np.ascontiguousarray(ids, dtype=np.uint64).reshape(-1)
        if vectors.shape[-1] != self.space.dim or vectors.shape[0] != ids.size:
            raise DimensionMismatch("dimension mismatch: device batch does not match the index", self.space.dim,
                                    vectors.shape[-1])
        slots = np.zeros(ids.size, np.uint32)
        _check(_lib.pxg_sq8_insert_device(self._h, _ptr(ids), _device_ptr(vectors), ids.size, _ptr(slots)))
        return slots

    def add_codes(self, ids, codes):
        ids = np.ascontiguousarray(ids, dtype=np.uint64).reshape(-1)
        c = np.ascontiguousarray(codes, dtype=np.int8).reshape(-1, self.space.dim)
        if c.shape[0] != ids.size:
            raise ValueError("ids and codes disagree on the batch size")
        slots = np.zeros(ids.size, np.uint32)
        _check(_lib.pxg_sq8_add_codes(self._h, _ptr(ids), _ptr(c), ids.size, _ptr(slots)))
        return slots

    def remove(self, id):
        _check(_lib.pxg_sq8_remove(self._h, int(id)))
        self._meta.pop(int(id), None)

    # -- queries --
    def contains(self, id):
        return bool(_lib.pxg_sq8_contains(self._h, int(id)))

    def __len__(self):
        return int(_lib.pxg_sq8_len(self._h))

    def stats(self):
        s = _IndexStatsC()
        _check(_lib.pxg_sq8_stats(self._h, C.byref(s)))
        return _stats_from_c(s)

    def code(self, id):
        out = np.zeros(self.space.dim, np.int8)
        try:
            _check(_lib.pxg_sq8_get_code(self._h, int(id), _ptr(out)))
        except UnknownId:
            return None
        return out

    def slots(self):
        n = int(_lib.pxg_sq8_slot_count(self._h))
        ids = np.zeros(max(n, 1), np.uint64)
        live = np.zeros(max(n, 1), np.uint8)
        _check(_lib.pxg_sq8_slots(self._h, _ptr(ids), _ptr(live)))
        return ids[:n], live[:n]

    def set_search_mode(self, mode):
        _check(_lib.pxg_sq8_set_search_mode(self._h, mode))

    def search(self, query, k, filter=None, rescore=0):
        ids, dists, counts = self.search_batch(np.asarray(query, dtype=np.float32).reshape(1, -1), k, filter,
                                               rescore)
        return [SearchResult(int(ids[0, i]), float(dists[0, i])) for i in range(int(counts[0]))]

    def _outputs(self, nq, k):
        kk = max(k, 1)
        return np.zeros((nq, kk), np.uint64), np.zeros((nq, kk), np.float32), np.zeros(max(nq, 1), np.uint32)

    def _mask(self, filter):
        if filter is None:
            return None
        sid, live = self.slots()
        return self._accept_mask(filter, sid, live)

    def search_batch(self, queries, k, filter=None, rescore=0):
        check_k(k)
        q = _rows(queries, self.space.dim)
        nq = q.shape[0]
        acc = self._mask(filter)
        oi, od, oc = self._outputs(nq, k)
        _check(_lib.pxg_sq8_search(self._h, _ptr(q), nq, k, rescore, _ptr(acc), _ptr(oi), _ptr(od), _ptr(oc)))
        return oi[:, :k], od[:, :k], oc[:nq]

    def search_codes(self, query_codes, k, filter=None):
        """Search with queries given as I8 codes [nq, dim]."""
        check_k(k)
        c = np.ascontiguousarray(query_codes, dtype=np.int8).reshape(-1, self.space.dim)
        nq = c.shape[0]
        acc = self._mask(filter)
        oi, od, oc = self._outputs(nq, k)
        _check(_lib.pxg_sq8_search_codes(self._h, _ptr(c), nq, k, _ptr(acc), _ptr(oi), _ptr(od), _ptr(oc)))
        return oi[:, :k], od[:, :k], oc[:nq]

    def search_device(self, queries, k, out_ids, out_dist, out_count, rescore=0, accept=None, stream=None):
        _check(_lib.pxg_sq8_search_device(
            self._h, _device_ptr(queries), queries.shape[0], k, rescore,
            None if accept is None else _device_ptr(accept), _device_ptr(out_ids), _device_ptr(out_dist),
            _device_ptr(out_count), None if stream is None else C.c_void_p(stream)))

    @staticmethod
    def last_fallbacks():
        return int(_lib.pxg_sq8_last_fallbacks())


__all__ += ["CodeType", "RangeMode", "ScalarQuantizer", "Sq8Index"]


# --- recall: crates/proxima-index/src/recall.rs:27-187 -----------------------------------
class RecallReport:
    """RecallReport (recall.rs:27-70): queries, k, mean, min, per_query, short_results."""

    def __init__(self, queries, k, mean, min, per_query, short_results):
        self.queries, self.k, self.mean, self.min = queries, k, mean, min
        self.per_query, self.short_results = per_query, short_results

    def below(self, threshold):  # recall.rs:49-55
        if not self.per_query:
            return 0.0
        t = np.float32(threshold)
        return float(np.float32(sum(1 for r in self.per_query if r < t)) / np.float32(len(self.per_query)))

    def __str__(self):  # recall.rs:58-70
        return (f"recall@{self.k}: mean {self.mean:.4f}, min {self.min:.4f}, below 0.9 "
                f"{self.below(0.9) * 100.0:.1f}% ({self.queries} queries)")

    __repr__ = __str__


def _overlap(exact, approx):  # recall.rs:172-184: |exact ∩ approx| / |exact|
    if len(exact) == 0:
        return np.float32(1.0)
    ex = set(int(i) for i in exact)
    hits = sum(1 for i in approx if int(i) in ex)
    return np.float32(hits) / np.float32(len(exact))


def recall_at_k(candidate, truth, queries, k):
    """recall_at_k (recall.rs:108-115): `candidate` is any index of this
    module, `truth` a FlatIndex over the same vectors and ids."""
    return recall_at_k_filtered(candidate, truth, queries, k, None)


def recall_at_k_filtered(candidate, truth, queries, k, filter):
    """recall_at_k_filtered (recall.rs:123-166). The exact side is one batched
    exhaustive GPU scan over all queries (the flat kernel), the approximate
    side one batched search; the statistics follow the reference's f32
    arithmetic (sum in query order, then divide)."""
    dim = truth.space.dim
    q = np.asarray(queries, dtype=np.float32).reshape(-1)
    if q.size % dim != 0:
        raise _config("queries", q.size, "must be a multiple of the index dimension")
    q = q.reshape(-1, dim)
    per_query, short = [], 0
    if q.shape[0]:
        ti, _, tc = truth.search_batch(q, k, filter)
        ai, _, ac = candidate.search_batch(q, k, filter)
        for i in range(q.shape[0]):
            if ac[i] < tc[i]:
                short += 1
            per_query.append(_overlap(ti[i, :tc[i]], ai[i, :ac[i]]))
    n = len(per_query)
    total = np.float32(0.0)
    for r in per_query:
        total = np.float32(total + r)
    mean = float(total / np.float32(n)) if n else 0.0
    mn = min(per_query) if per_query else np.float32(np.inf)
    return RecallReport(n, k, mean, float(mn) if np.isfinite(mn) else 0.0, [float(r) for r in per_query], short)


__all__ += ["RecallReport", "recall_at_k", "recall_at_k_filtered"]


# ---------------------------------------------------------------------------
# the benchmark fixture (crates/proxima-cli/src/fixture.rs)
# ---------------------------------------------------------------------------
def fixture_generate(count, dim, clusters, queries, seed):
    """fixture::generate (fixture.rs:71-123) on the GPU: returns (vectors
    [count, dim], queries [queries, dim]) as f32 arrays."""
    v = np.zeros((count, dim), np.float32)
    q = np.zeros((queries, dim), np.float32)
    _check(_lib.pxg_fixture_generate(count, dim, clusters, queries, seed, _ptr(v) if v.size else None,
                                     _ptr(q) if q.size else None))
    return v, q


def fixture_generate_device(count, dim, clusters, queries, seed, vectors_out, queries_out=None):
    """fixture_generate into contiguous f32 GPU tensors [count, dim] and
    [queries, dim] (queries_out may be None when queries == 0)."""
    for t, rows, name in ((vectors_out, count, "vectors_out"), (queries_out, queries, "queries_out")):
        if rows == 0 and t is None:
            continue
        if t is None or not t.is_cuda or str(t.dtype) != "torch.float32" or t.numel() < rows * dim:
            raise ValueError(f"{name} must be a float32 GPU tensor of at least {rows} x {dim} elements")
    _check(_lib.pxg_fixture_generate_device(count, dim, clusters, queries, seed, _device_ptr(vectors_out),
                                            None if queries_out is None else _device_ptr(queries_out)))


def _gen_outputs(outs, dim):
    for t, rows, name in outs:
        if rows == 0 and t is None:
            continue
        if (t is None or not t.is_cuda or str(t.dtype) != "torch.float32" or not t.is_contiguous()
                or t.numel() < rows * dim):
            raise ValueError(f"{name} must be a contiguous float32 GPU tensor of at least {rows} x {dim} elements")


def mixture_generate_device(count, dim, clusters, centre_scale, sigma, queries, drawn_clusters, seed, vectors_out,
                            queries_out=None):
    """The benchmark configurations' Gaussian mixtures (no reference
    counterpart): centres centre_scale * N(0,1), each point and query its
    cluster's centre plus sigma * N(0,1), clusters i % C or drawn, all from one
    seeded ChaCha8 stream with fixture.rs's Box-Muller step. Writes contiguous
    f32 GPU tensors [count, dim] and [queries, dim]."""
    _gen_outputs(((vectors_out, count, "vectors_out"), (queries_out, queries, "queries_out")), dim)
    _check(_lib.pxg_mixture_generate_device(count, dim, clusters, float(centre_scale), float(sigma), queries,
                                            1 if drawn_clusters else 0, seed, _device_ptr(vectors_out),
                                            _device_ptr(queries_out) if queries else None))


def uniform_generate_device(count, dim, lo, hi, seed, out):
    """count x dim values lo + (hi - lo) * gen::<f32>() from a seeded ChaCha8
    stream, into a contiguous f32 GPU tensor (no reference counterpart)."""
    _gen_outputs(((out, count, "out"),), dim)
    _check(_lib.pxg_uniform_generate_device(count, dim, float(lo), float(hi), seed, _device_ptr(out)))


__all__ += ["fixture_generate", "fixture_generate_device", "mixture_generate_device", "uniform_generate_device"]
