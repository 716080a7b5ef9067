"""ctypes view of the oracle (oracle.cpp): the CPU restatement of the
reference's hot path. Test infrastructure: imported only by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker.

Array arguments are numpy arrays; every wrapper checks dtype/contiguity and
returns numpy results.
"""
import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# PXG_ORACLE_LIB names another build of oracle.cpp (the mutation tests load
# deliberately broken copies through it to show that the pins catch them)
_LIB_PATH = os.environ.get("PXG_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")

EUCLIDEAN, COSINE, INNER_PRODUCT, MANHATTAN = 0, 1, 2, 3

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
_sz = C.c_size_t


def build():
    """Compile liboracle.so in place (make)."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B"], check=True)


def _load():
    if not os.path.exists(_LIB_PATH):
        build()
    lib = C.CDLL(_LIB_PATH)
    sig = {
        "orc_squared_euclidean_unrolled": (C.c_float, [_f32p, _f32p, _sz]),
        "orc_squared_euclidean_scalar": (C.c_float, [_f32p, _f32p, _sz]),
        "orc_dot_unrolled": (C.c_float, [_f32p, _f32p, _sz]),
        "orc_dot_scalar": (C.c_float, [_f32p, _f32p, _sz]),
        "orc_manhattan_unrolled": (C.c_float, [_f32p, _f32p, _sz]),
        "orc_manhattan_scalar": (C.c_float, [_f32p, _f32p, _sz]),
        "orc_cosine_unrolled": (C.c_float, [_f32p, _f32p, _sz]),
        "orc_cosine_scalar": (C.c_float, [_f32p, _f32p, _sz]),
        "orc_space_distance": (C.c_float, [C.c_int, _f32p, _f32p, _sz]),
        "orc_metric_distance": (C.c_float, [C.c_int, _f32p, _f32p, _sz]),
        "orc_normalize_in_place": (C.c_float, [_f32p, _sz]),
        "orc_prepare": (C.c_longlong, [C.c_int, _f32p, _sz, _f32p]),
        "orc_topk": (_sz, [_u64p, _f32p, _sz, _sz, _u64p, _f32p]),
        "orc_prepare_batch": (C.c_longlong, [C.c_int, _f32p, _sz, _sz, _f32p, C.c_int]),
        "orc_flat_search": (None, [_f32p, _u8p, _u64p, _sz, _sz, C.c_int, _f32p, _sz, _sz, C.c_void_p,
                                   C.c_int, _u64p, _f32p, _u32p]),
        "orc_sq_train": (C.c_longlong, [_f32p, _sz, _sz, C.c_int, _f32p, _f32p, _f32p]),
        "orc_sq_encode": (None, [_f32p, _sz, C.c_int, C.c_int, _f32p, _f32p, _u8p]),
        "orc_sq_encode_rows": (None, [_f32p, _sz, _sz, C.c_int, C.c_int, _f32p, _f32p, C.c_int, _u8p]),
        "orc_sq_decode": (None, [_u8p, _sz, C.c_int, C.c_int, _f32p, _f32p, _f32p]),
        "orc_sq_asym": (C.c_float, [C.c_int, _f32p, _u8p, _sz, C.c_int, C.c_int, _f32p, _f32p]),
        "orc_sq8_search": (None, [_i8p, _u8p, _u64p, _sz, _sz, _i8p, _sz, _sz, C.c_void_p, _sz, C.c_void_p,
                                  C.c_int, C.c_void_p, C.c_void_p, C.c_int, _u64p, _f32p, _u32p]),
        "orc_pq_layout": (None, [_sz, _sz, np.ctypeslib.ndpointer(np.uintp), np.ctypeslib.ndpointer(np.uintp)]),
        "orc_pq_table": (None, [_f32p, _sz, _sz, _f32p, _f32p, _f32p]),
        "orc_pq_adc_l2": (C.c_float, [_f32p, _sz, _u8p]),
        "orc_pq_adc_ip": (C.c_float, [_f32p, _sz, _u8p]),
        "orc_pq_encode": (None, [_f32p, _sz, _sz, _f32p, _sz, _u8p]),
        "orc_pq_decode": (None, [_f32p, _sz, _sz, _u8p, _f32p]),
        "orc_pq_train": (None, [_f32p, _sz, _sz, _sz, _sz, C.c_uint64, _f32p, C.POINTER(C.c_double),
                                C.POINTER(C.c_size_t)]),
        "orc_kmeans_lloyd": (None, [_f32p, _sz, _sz, _sz, _sz, _f32p, _u32p, C.POINTER(C.c_double),
                                    C.POINTER(C.c_size_t)]),
        "orc_kmeans_pp": (None, [_f32p, _sz, _sz, _sz, C.c_uint64, _f32p]),
        "orc_kmeans": (_sz, [_f32p, _sz, _sz, _sz, _sz, C.c_uint64, _f32p, C.POINTER(C.c_double),
                             C.POINTER(C.c_size_t)]),
        "orc_kmeans_pp_pick": (_sz, [_f32p, _sz, C.c_double]),
        "orc_kmeans_rng": (_sz, [_f32p, _sz, _sz, _sz, _sz, C.c_void_p, _f32p, C.POINTER(C.c_double),
                                 C.POINTER(C.c_size_t)]),
        "orc_kmeans_assign": (None, [_f32p, _sz, _sz, _f32p, _sz, _u32p, _f32p]),
        "orc_kmeans_assign_mt": (None, [_f32p, _sz, _sz, _f32p, _sz, _u32p, _f32p, C.c_int]),
        "orc_rng_new": (C.c_void_p, [C.c_uint64, C.c_int]),
        "orc_rng_set_key": (None, [C.c_void_p, _u32p]),
        "orc_rng_key": (None, [C.c_void_p, _u32p]),
        "orc_rng_next_u32": (C.c_uint32, [C.c_void_p]),
        "orc_rng_next_u64": (C.c_uint64, [C.c_void_p]),
        "orc_rng_gen_range_usize": (C.c_uint64, [C.c_void_p, C.c_uint64]),
        "orc_rng_gen_range_f64": (C.c_double, [C.c_void_p, C.c_double, C.c_double]),
        "orc_rng_gen_f32": (C.c_float, [C.c_void_p]),
        "orc_rng_free": (None, [C.c_void_p]),
        "orc_chacha_block": (None, [_u32p, C.c_uint64, C.c_uint64, C.c_int, _u32p]),
        "orc_fixture_generate": (None, [_sz, _sz, _sz, _sz, C.c_uint64, _f32p, _f32p]),
        "orc_ivf_train": (_sz, [_f32p, _u8p, _sz, _sz, _sz, _sz, _sz, _sz, C.c_uint64, _f32p, _f32p, _f64p]),
        "orc_ivf_encode": (None, [_f32p, _u8p, _sz, _sz, _f32p, _sz, _f32p, _sz, _u8p, _u32p]),
        "orc_ivf_search": (None, [C.c_int, _f32p, _sz, _f32p, _sz, _sz, _u8p, _u32p, _u8p, _u64p, _sz, C.c_void_p,
                                  _sz, _f32p, _sz, _sz, _sz, C.c_void_p, C.c_int, _u64p, _f32p, _u32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _vp(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# --- distance kernels (distance.rs) ----------------------------------------
def squared_euclidean(a, b):
    a, b = f32(a), f32(b)
    return lib.orc_squared_euclidean_unrolled(a, b, min(a.size, b.size))


def squared_euclidean_scalar(a, b):
    a, b = f32(a), f32(b)
    return lib.orc_squared_euclidean_scalar(a, b, min(a.size, b.size))


def dot(a, b):
    a, b = f32(a), f32(b)
    return lib.orc_dot_unrolled(a, b, min(a.size, b.size))


def dot_scalar(a, b):
    a, b = f32(a), f32(b)
    return lib.orc_dot_scalar(a, b, min(a.size, b.size))


def manhattan(a, b):
    a, b = f32(a), f32(b)
    return lib.orc_manhattan_unrolled(a, b, min(a.size, b.size))


def cosine(a, b):
    a, b = f32(a), f32(b)
    return lib.orc_cosine_unrolled(a, b, min(a.size, b.size))


def cosine_scalar(a, b):
    a, b = f32(a), f32(b)
    return lib.orc_cosine_scalar(a, b, min(a.size, b.size))


def space_distance(metric, a, b):
    a, b = f32(a), f32(b)
    return lib.orc_space_distance(metric, a, b, min(a.size, b.size))


def metric_distance(metric, a, b):
    a, b = f32(a), f32(b)
    return lib.orc_metric_distance(metric, a, b, min(a.size, b.size))


def normalized(v):
    out = f32(v).copy()
    lib.orc_normalize_in_place(out, out.size)
    return out


def prepare(metric, v):
    """VectorSpace::prepare; returns (prepared, bad_index or -1)."""
    v = f32(v)
    out = np.empty_like(v)
    bad = lib.orc_prepare(metric, v, v.size, out)
    return out, bad


def prepare_rows(metric, x, threads=8):
    x = f32(x)
    n, dim = x.shape
    out = np.empty_like(x)
    bad = lib.orc_prepare_batch(metric, x, n, dim, out, threads)
    assert bad < 0, f"row {bad} is not finite"
    return out


def topk(ids, d, k):
    ids = np.ascontiguousarray(ids, dtype=np.uint64)
    d = f32(d)
    oi = np.zeros(max(k, 1), np.uint64)
    od = np.zeros(max(k, 1), np.float32)
    n = lib.orc_topk(ids, d, ids.size, k, oi, od)
    return oi[:n], od[:n]


def flat_search(data, ids, metric, queries, k, live=None, accept=None, threads=1):
    """FlatIndex::search over prepared data/queries. Returns (ids, dists, counts)."""
    data = f32(data)
    slots, dim = data.shape
    queries = f32(queries).reshape(-1, dim)
    nq = queries.shape[0]
    live = np.ones(slots, np.uint8) if live is None else np.ascontiguousarray(live, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.uint64)
    acc = None if accept is None else np.ascontiguousarray(accept, dtype=np.uint8)
    kk = max(k, 1)
    oi = np.zeros((nq, kk), np.uint64)
    od = np.zeros((nq, kk), np.float32)
    oc = np.zeros(nq, np.uint32)
    lib.orc_flat_search(data, live, ids, slots, dim, metric, queries, nq, k, _vp(acc), threads, oi, od, oc)
    return oi, od, oc


# --- scalar quantizer (scalar.rs) --------------------------------------------
def sq_train(training, per_dim=True):
    training = f32(training)
    n, dim = training.shape
    g = dim if per_dim else 1
    mn, scale, inv = (np.zeros(g, np.float32) for _ in range(3))
    bad = lib.orc_sq_train(training, n, dim, int(per_dim), mn, scale, inv)
    return mn, scale, inv, bad


def sq_encode(v, mn, inv, per_dim=True, code_type=1, threads=1):
    v = f32(v)
    dim = v.shape[-1]
    rows = np.ascontiguousarray(v.reshape(-1, dim))
    out = np.zeros(rows.shape, np.uint8)
    lib.orc_sq_encode_rows(rows, rows.shape[0], dim, int(per_dim), code_type, f32(mn), f32(inv), threads, out)
    return out.reshape(v.shape)


def sq_decode(code, mn, scale, per_dim=True, code_type=1):
    """Decode one code (1-D) or a batch of codes (one row each)."""
    code = np.ascontiguousarray(code, dtype=np.uint8)
    rows = code.reshape(-1, code.shape[-1])
    out = np.zeros(rows.shape, np.float32)
    for i in range(rows.shape[0]):
        o = np.zeros(rows.shape[1], np.float32)
        lib.orc_sq_decode(np.ascontiguousarray(rows[i]), rows.shape[1], int(per_dim), code_type, mn, scale, o)
        out[i] = o
    return out.reshape(code.shape)


def sq_asym(ip, q, code, mn, scale, per_dim=True, code_type=1):
    q = f32(q)
    code = np.ascontiguousarray(code, dtype=np.uint8)
    return lib.orc_sq_asym(int(ip), q, code, q.size, int(per_dim), code_type, mn, scale)


def sq8_search(codes, ids, qcodes, k, live=None, threads=1, accept=None, rescore=0, qf=None, ranges=None,
               per_dim=True):
    """Integer-score SQ8 search over I8 codes; with rescore > 0 the best
    max(rescore, k) are rescored with asymmetric_inner_product of the
    prepared f32 queries `qf` against codes decoded with `ranges` = (min,
    scale)."""
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    slots, dim = codes.shape
    qcodes = np.ascontiguousarray(qcodes, dtype=np.int8).reshape(-1, dim)
    nq = qcodes.shape[0]
    live = np.ones(slots, np.uint8) if live is None else np.ascontiguousarray(live, dtype=np.uint8)
    kk = max(k, 1)
    oi = np.zeros((nq, kk), np.uint64)
    od = np.zeros((nq, kk), np.float32)
    oc = np.zeros(nq, np.uint32)
    keep = []

    def ptr(a, dt):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dtype=dt)
        keep.append(a)
        return a.ctypes.data

    mn, sc = (None, None) if ranges is None else ranges
    if rescore and (qf is None or ranges is None):
        raise ValueError("rescore needs the f32 queries and the ranges")
    lib.orc_sq8_search(codes, live, np.ascontiguousarray(ids, dtype=np.uint64), slots, dim, qcodes, nq, k,
                       ptr(accept, np.uint8), rescore, ptr(qf, np.float32), int(per_dim), ptr(mn, np.float32),
                       ptr(sc, np.float32), threads, oi, od, oc)
    return oi, od, oc


# --- product quantizer (product.rs) ------------------------------------------
def pq_layout(dim, m):
    w = np.zeros(m, np.uintp)
    o = np.zeros(m + 1, np.uintp)
    lib.orc_pq_layout(dim, m, w, o)
    return [int(x) for x in w], [int(x) for x in o]


def pq_table(books, dim, m, q):
    sq = np.zeros(m * 256, np.float32)
    dt = np.zeros(m * 256, np.float32)
    lib.orc_pq_table(f32(books), dim, m, f32(q), sq, dt)
    return sq, dt


def pq_adc_l2(table, code):
    code = np.ascontiguousarray(code, dtype=np.uint8)
    return lib.orc_pq_adc_l2(f32(table), code.size, code)


def pq_adc_ip(table, code):
    code = np.ascontiguousarray(code, dtype=np.uint8)
    return lib.orc_pq_adc_ip(f32(table), code.size, code)


def pq_encode(books, dim, m, v):
    v = f32(v).reshape(-1, dim)
    out = np.zeros((v.shape[0], m), np.uint8)
    lib.orc_pq_encode(f32(books), dim, m, v, v.shape[0], out)
    return out


def pq_decode(books, dim, m, code):
    out = np.zeros(dim, np.float32)
    lib.orc_pq_decode(f32(books), dim, m, np.ascontiguousarray(code, dtype=np.uint8), out)
    return out


def pq_train(training, m, max_iter=25, seed=0x5EED1EAF):
    training = f32(training)
    n, dim = training.shape
    _, off = pq_layout(dim, m)
    books = np.zeros(256 * dim, np.float32)
    inertia = C.c_double()
    iters = C.c_size_t()
    lib.orc_pq_train(training, n, dim, m, max_iter, seed, books, C.byref(inertia), C.byref(iters))
    return books, inertia.value, iters.value


# --- k-means (kmeans.rs) ---------------------------------------------------------
def kmeans_lloyd(points, init, max_iter):
    points = f32(points)
    n, dim = points.shape
    cents = f32(init).copy()
    k = cents.shape[0]
    assign = np.zeros(n, np.uint32)
    inertia = C.c_double()
    iters = C.c_size_t()
    lib.orc_kmeans_lloyd(points, n, dim, k, max_iter, cents, assign, C.byref(inertia), C.byref(iters))
    return cents, assign, inertia.value, iters.value


def kmeans_pp(points, k, seed):
    points = f32(points)
    n, dim = points.shape
    cents = np.zeros((k, dim), np.float32)
    lib.orc_kmeans_pp(points, n, dim, k, seed, cents)
    return cents


def kmeans(points, k, max_iter, seed):
    points = f32(points)
    n, dim = points.shape if points.ndim == 2 else (0, 1)
    kk = max(min(k, n), 1)
    cents = np.zeros(kk * dim, np.float32)
    inertia = C.c_double()
    iters = C.c_size_t()
    got = lib.orc_kmeans(points.reshape(-1), n, dim, k, max_iter, seed, cents, C.byref(inertia), C.byref(iters))
    return cents.reshape(got, dim), inertia.value, iters.value


def kmeans_pp_pick(ns, target):
    ns = f32(ns)
    return int(lib.orc_kmeans_pp_pick(ns, ns.size, float(target)))


def kmeans_with_rng(points, k, max_iter, rng):
    """kmeans() over `rng` (an Rng), which is left advanced."""
    points = f32(points)
    n, dim = points.shape
    kk = max(min(k, n), 1)
    cents = np.zeros(kk * dim, np.float32)
    inertia = C.c_double()
    iters = C.c_size_t()
    got = lib.orc_kmeans_rng(points.reshape(-1), n, dim, k, max_iter, rng.h, cents, C.byref(inertia), C.byref(iters))
    return cents.reshape(got, dim), inertia.value, iters.value


def kmeans_assign(points, cents, threads=1):
    points, cents = f32(points), f32(cents)
    n, dim = points.shape
    a = np.zeros(n, np.uint32)
    d = np.zeros(n, np.float32)
    if threads > 1:
        lib.orc_kmeans_assign_mt(points, n, dim, cents, cents.shape[0], a, d, threads)
    else:
        lib.orc_kmeans_assign(points, n, dim, cents, cents.shape[0], a, d)
    return a, d


# --- RNG -----------------------------------------------------------------------------
class Rng:
    """ChaCha (8 rounds by default) seeded with rand_core's seed_from_u64."""

    def __init__(self, seed, rounds=8, key=None):
        self.h = lib.orc_rng_new(seed, rounds)
        if key is not None:
            lib.orc_rng_set_key(self.h, np.ascontiguousarray(key, dtype=np.uint32))

    def key(self):
        k = np.zeros(8, np.uint32)
        lib.orc_rng_key(self.h, k)
        return k

    def next_u32(self):
        return lib.orc_rng_next_u32(self.h)

    def next_u64(self):
        return lib.orc_rng_next_u64(self.h)

    def gen_range_usize(self, n):
        return lib.orc_rng_gen_range_usize(self.h, n)

    def gen_range_f64(self, lo, hi):
        return lib.orc_rng_gen_range_f64(self.h, lo, hi)

    def gen_f32(self):
        return lib.orc_rng_gen_f32(self.h)

    def __del__(self):
        if getattr(self, "h", None):
            lib.orc_rng_free(self.h)
            self.h = None


def chacha_block(key, counter, stream, rounds):
    out = np.zeros(16, np.uint32)
    lib.orc_chacha_block(np.ascontiguousarray(key, dtype=np.uint32), counter, stream, rounds, out)
    return out


def fixture_generate(count, dim, clusters, queries, seed):
    v = np.zeros((count, dim), np.float32)
    q = np.zeros((max(queries, 0), dim), np.float32)
    lib.orc_fixture_generate(count, dim, clusters, queries, seed, v, q if queries else np.zeros(1, np.float32))
    return v, q


# --- IVF-PQ (ivfpq.rs) ---------------------------------------------------------------
def ivf_train(vectors, nlist, m, max_iter=25, training_sample=100_000, seed=0x1FF9C0D, live=None):
    vectors = f32(vectors)
    slots, dim = vectors.shape
    live = np.ones(slots, np.uint8) if live is None else np.ascontiguousarray(live, dtype=np.uint8)
    cents = np.zeros(nlist * dim, np.float32)
    books = np.zeros(256 * dim, np.float32)
    report = np.zeros(4, np.float64)
    produced = lib.orc_ivf_train(vectors, live, slots, dim, nlist, m, max_iter, training_sample, seed, cents, books,
                                 report)
    if produced == np.iinfo(np.uintp).max:
        raise ValueError(f"NonFinite residual: component {int(report[0])} of sample vector {int(report[1])} "
                         f"({report[2]})", int(report[0]), int(report[1]), float(report[2]))
    return cents[: produced * dim].reshape(produced, dim), books, report


def ivf_encode(vectors, cents, books, m, live=None):
    vectors = f32(vectors)
    slots, dim = vectors.shape
    live = np.ones(slots, np.uint8) if live is None else np.ascontiguousarray(live, dtype=np.uint8)
    codes = np.zeros((slots, m), np.uint8)
    list_of = np.zeros(slots, np.uint32)
    cents = f32(cents)
    lib.orc_ivf_encode(vectors, live, slots, dim, cents.reshape(-1) if cents.size else np.zeros(1, np.float32),
                       cents.shape[0], f32(books), m, codes, list_of)
    return codes, list_of


def ivf_search(metric, cents, books, codes, list_of, ids, queries, k, nprobe, m, vectors=None, rerank=0,
               live=None, accept=None, threads=1):
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    slots = codes.shape[0]
    cents = f32(cents)
    produced = cents.shape[0] if cents.ndim == 2 else 0
    dim = queries.shape[-1]
    queries = f32(queries).reshape(-1, dim)
    nq = queries.shape[0]
    live = np.ones(slots, np.uint8) if live is None else np.ascontiguousarray(live, dtype=np.uint8)
    vec = None if vectors is None else f32(vectors)
    acc = None if accept is None else np.ascontiguousarray(accept, dtype=np.uint8)
    kk = max(k, 1)
    oi = np.zeros((nq, kk), np.uint64)
    od = np.zeros((nq, kk), np.float32)
    oc = np.zeros(nq, np.uint32)
    lib.orc_ivf_search(metric, cents.reshape(-1) if cents.size else np.zeros(1, np.float32), produced, f32(books),
                       dim, m, codes, np.ascontiguousarray(list_of, dtype=np.uint32), live,
                       np.ascontiguousarray(ids, dtype=np.uint64), slots, _vp(vec), rerank, queries, nq, k, nprobe,
                       _vp(acc), threads, oi, od, oc)
    return oi, od, oc
