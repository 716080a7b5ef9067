"""ctypes binding of libproxima_hip.so (the C ABI in include/proxima_hip.h).

The shared library is the product: there is no fallback. If it is missing or
fails to load, importing proxima_amd raises.
"""
import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libproxima_hip.so")

_vp = C.c_void_p
_u64 = C.c_uint64
_u32 = C.c_uint32
_i32 = C.c_int
_f32 = C.c_float
_f64 = C.c_double
_P = C.POINTER


class IndexStats(C.Structure):
    _fields_ = [
        ("len", _u64),
        ("deleted", _u64),
        ("dim", _u32),
        ("metric", C.c_int32),
        ("layers", _u64),
        ("edges", _u64),
        ("vector_bytes", _u64),
        ("graph_bytes", _u64),
    ]


class Timings(C.Structure):
    _fields_ = [
        ("prep_ms", _f32),
        ("candidates_ms", _f32),
        ("merge_ms", _f32),
        ("fallback_ms", _f32),
        ("total_ms", _f32),
    ]


class IvfPqConfigC(C.Structure):
    _fields_ = [
        ("nlist", _u64),
        ("subspaces", _u64),
        ("nprobe", _u64),
        ("rerank", _u64),
        ("seed", _u64),
        ("max_iterations", _u64),
        ("training_sample", _u64),
        ("train_threshold", _u64),
        ("retain_vectors", _i32),
    ]


class TrainingReportC(C.Structure):
    _fields_ = [
        ("sampled", _u64),
        ("coarse_inertia", _f64),
        ("coarse_iterations", _u64),
        ("residual_inertia", _f64),
        ("populated_lists", _u64),
        ("largest_list", _u64),
    ]


# name -> (restype, argtypes); every entry must exist in the library.
SIGNATURES = {
    "pxg_last_error_message": (C.c_char_p, []),
    "pxg_last_error_detail": (_i32, [_P(_u64), _P(_u64), _P(_f32)]),
    "pxg_last_error_parameter": (C.c_char_p, []),
    "pxg_last_error_reason": (C.c_char_p, []),
    "pxg_version": (C.c_char_p, []),
    "pxg_device_count": (_i32, []),
    "pxg_set_profiling": (None, [_i32]),
    "pxg_last_timings": (_i32, [_P(Timings)]),
    # flat
    "pxg_flat_create": (_i32, [_u32, _i32, _u64, _P(_vp)]),
    "pxg_flat_destroy": (None, [_vp]),
    "pxg_flat_insert": (_i32, [_vp, _vp, _vp, _u64, _vp]),
    "pxg_flat_insert_device": (_i32, [_vp, _vp, _vp, _u64, _vp]),
    "pxg_flat_remove": (_i32, [_vp, _u64]),
    "pxg_flat_contains": (_i32, [_vp, _u64]),
    "pxg_flat_len": (_u64, [_vp]),
    "pxg_flat_stats": (_i32, [_vp, _P(IndexStats)]),
    "pxg_flat_get_vector": (_i32, [_vp, _u64, _vp]),
    "pxg_flat_slot_count": (_u64, [_vp]),
    "pxg_flat_slots": (_i32, [_vp, _vp, _vp]),
    "pxg_flat_search": (_i32, [_vp, _vp, _u64, _u64, _vp, _vp, _vp, _vp]),
    "pxg_flat_search_device": (_i32, [_vp, _vp, _u64, _u64, _vp, _vp, _vp, _vp, _vp]),
    "pxg_flat_search_device_noalloc": (_i32, [_vp, _vp, _u64, _u64, _vp, _vp, _vp, _vp, _vp]),
    "pxg_flat_last_fallbacks": (_u64, []),
    "pxg_flat_set_search_mode": (_i32, [_vp, _i32]),
    # ivf-pq
    "pxg_ivfpq_config_default": (_i32, [_u64, _u64, _P(IvfPqConfigC)]),
    "pxg_ivfpq_create": (_i32, [_u32, _i32, _P(IvfPqConfigC), _P(_vp)]),
    "pxg_ivfpq_destroy": (None, [_vp]),
    "pxg_ivfpq_insert": (_i32, [_vp, _vp, _vp, _u64, _vp]),
    "pxg_ivfpq_insert_device": (_i32, [_vp, _vp, _vp, _u64, _vp]),
    "pxg_ivfpq_remove": (_i32, [_vp, _u64]),
    "pxg_ivfpq_compact": (_i32, [_vp, _P(_u64)]),
    "pxg_ivfpq_contains": (_i32, [_vp, _u64]),
    "pxg_ivfpq_len": (_u64, [_vp]),
    "pxg_ivfpq_is_trained": (_i32, [_vp]),
    "pxg_ivfpq_stats": (_i32, [_vp, _P(IndexStats)]),
    "pxg_ivfpq_get_vector": (_i32, [_vp, _u64, _vp]),
    "pxg_ivfpq_slot_count": (_u64, [_vp]),
    "pxg_ivfpq_slots": (_i32, [_vp, _vp, _vp]),
    "pxg_ivfpq_list_count": (_u64, [_vp]),
    "pxg_ivfpq_list_lengths": (_i32, [_vp, _vp]),
    "pxg_ivfpq_train": (_i32, [_vp, _P(TrainingReportC)]),
    "pxg_ivfpq_training_report": (_i32, [_vp, _P(TrainingReportC)]),
    "pxg_ivfpq_parts": (_i32, [_vp, _vp, _vp, _vp, _vp]),
    "pxg_ivfpq_load_trained": (_i32, [_vp, _vp, _u64, _vp, _vp, _vp]),
    "pxg_ivfpq_search": (_i32, [_vp, _vp, _u64, _u64, _u64, _vp, _vp, _vp, _vp]),
    "pxg_ivfpq_search_device": (_i32, [_vp, _vp, _u64, _u64, _u64, _vp, _vp, _vp, _vp, _vp]),
    "pxg_ivfpq_last_scanned": (_u64, []),
    "pxg_ivfpq_view_stats": (_i32, [_vp, _P(_u64), _P(_u64)]),
    # k-means / PQ
    "pxg_kmeans": (_i32, [_vp, _u64, _u32, _u64, _u64, _u64, _vp, _P(_f64), _P(_u64), _P(_u64)]),
    "pxg_kmeans_lloyd": (_i32, [_vp, _u64, _u32, _u64, _u64, _vp, _vp, _vp, _P(_f64), _P(_u64)]),
    "pxg_kmeans_device": (_i32, [_vp, _u64, _u32, _u64, _u64, _u64, _vp, _vp, _vp, _P(_f64), _P(_u64)]),
    "pxg_kmeans_pp": (_i32, [_vp, _u64, _u32, _u64, _u64, _vp]),
    "pxg_kmeans_last_stats": (_i32, [_P(_f64), _P(_f64), _P(_u64), _P(_u64), _P(_u64)]),
    "pxg_kmeans_last_reseeds": (_i32, [_P(_u64), _P(_u64), _P(_u64)]),
    "pxg_kmeans_assign": (_i32, [_vp, _u64, _u32, _vp, _u64, _vp, _vp]),
    "pxg_pq_train": (_i32, [_vp, _u64, _u32, _u64, _u64, _u64, _vp, _P(_f64), _P(_u64)]),
    "pxg_pq_encode": (_i32, [_vp, _u32, _u64, _vp, _u64, _vp]),
    "pxg_pq_train_device": (_i32, [_vp, _u64, _u32, _u64, _u64, _u64, _vp, _P(_f64), _P(_u64)]),
    "pxg_fixture_generate": (_i32, [_u64, _u32, _u64, _u64, _u64, _vp, _vp]),
    "pxg_fixture_generate_device": (_i32, [_u64, _u32, _u64, _u64, _u64, _vp, _vp]),
    "pxg_mixture_generate_device": (_i32, [_u64, _u32, _u64, _f32, _f32, _u64, _i32, _u64, _vp, _vp]),
    "pxg_uniform_generate_device": (_i32, [_u64, _u32, _f32, _f32, _u64, _vp]),
    # scalar quantizer / SQ8 index
    "pxg_sq_train": (_i32, [_vp, _u64, _u32, _i32, _vp, _vp, _vp]),
    "pxg_sq_encode": (_i32, [_vp, _u64, _u32, _i32, _i32, _vp, _vp, _vp]),
    "pxg_sq_decode": (_i32, [_vp, _u64, _u32, _i32, _i32, _vp, _vp, _vp]),
    "pxg_sq_asymmetric": (_i32, [_i32, _vp, _vp, _u64, _u32, _i32, _i32, _vp, _vp, _vp]),
    "pxg_sq8_create": (_i32, [_u32, _i32, _i32, _u64, _P(_vp)]),
    "pxg_sq8_destroy": (None, [_vp]),
    "pxg_sq8_train": (_i32, [_vp, _vp, _u64]),
    "pxg_sq8_train_device": (_i32, [_vp, _vp, _u64]),
    "pxg_sq8_set_ranges": (_i32, [_vp, _vp, _vp, _vp]),
    "pxg_sq8_ranges": (_i32, [_vp, _vp, _vp, _vp]),
    "pxg_sq8_is_trained": (_i32, [_vp]),
    "pxg_sq8_insert": (_i32, [_vp, _vp, _vp, _u64, _vp]),
    "pxg_sq8_insert_device": (_i32, [_vp, _vp, _vp, _u64, _vp]),
    "pxg_sq8_add_codes": (_i32, [_vp, _vp, _vp, _u64, _vp]),
    "pxg_sq8_remove": (_i32, [_vp, _u64]),
    "pxg_sq8_contains": (_i32, [_vp, _u64]),
    "pxg_sq8_len": (_u64, [_vp]),
    "pxg_sq8_stats": (_i32, [_vp, _P(IndexStats)]),
    "pxg_sq8_get_code": (_i32, [_vp, _u64, _vp]),
    "pxg_sq8_slot_count": (_u64, [_vp]),
    "pxg_sq8_slots": (_i32, [_vp, _vp, _vp]),
    "pxg_sq8_search": (_i32, [_vp, _vp, _u64, _u64, _u64, _vp, _vp, _vp, _vp]),
    "pxg_sq8_search_codes": (_i32, [_vp, _vp, _u64, _u64, _vp, _vp, _vp, _vp]),
    "pxg_sq8_search_device": (_i32, [_vp, _vp, _u64, _u64, _u64, _vp, _vp, _vp, _vp, _vp]),
    "pxg_sq8_last_fallbacks": (_u64, []),
    "pxg_sq8_set_search_mode": (_i32, [_vp, _i32]),
}


def load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python proxima_amd/build.py` "
            "(hipcc, gfx950). There is no CPU fallback.")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = load()
