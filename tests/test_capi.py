"""CPU checks of the C ABI: the library builds/loads and exports every entry
point include/*.h declares, and the ctypes signatures cover exactly those
(no compute calls: there is no GPU here)."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "proxima_amd", "libproxima_hip.so")


def declared_functions():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(pxg_[a-z0-9_]+)\s*\(", text):
            names.append(m.group(1))
    return sorted(set(names))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "pxg_flat_search" in names and "pxg_last_error_message" in names
    assert len(names) >= 15


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.skip("library not built (run __graft_entry__.build())")
    return ctypes.CDLL(LIB)


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_signatures_match_header():
    from proxima_amd import _capi
    declared = set(declared_functions())
    bound = set(_capi.SIGNATURES)
    assert bound == declared, (sorted(declared - bound), sorted(bound - declared))


def test_error_plumbing_without_gpu(lib):
    lib.pxg_last_error_message.restype = ctypes.c_char_p
    lib.pxg_flat_create.restype = ctypes.c_int
    h = ctypes.c_void_p()
    # dim 0 is a configuration error raised before any device work (space.rs:71-78)
    st = lib.pxg_flat_create(0, 0, 0, ctypes.byref(h))
    assert st == 7
    assert b"dim" in lib.pxg_last_error_message()
    st = lib.pxg_flat_create(4, 9, 0, ctypes.byref(h))
    assert st == 7 and b"metric" in lib.pxg_last_error_message()


def test_python_mirror_validation_without_gpu():
    import proxima_amd as px
    with pytest.raises(px.Configuration):
        px.VectorSpace(0, px.Metric.EUCLIDEAN)
    with pytest.raises(px.Configuration):
        px.VectorSpace((1 << 20) + 1, px.Metric.EUCLIDEAN)
    s = px.VectorSpace(3, px.Metric.EUCLIDEAN)
    with pytest.raises(px.DimensionMismatch) as e:
        s.validate([1.0, 2.0])
    assert e.value.expected == 3 and e.value.actual == 2
    with pytest.raises(px.NonFinite) as e:
        s.validate([1.0, float("inf"), 3.0])
    assert e.value.index == 1
    assert str(px.VectorSpace(768, px.Metric.COSINE)) == "768d/cosine"
    px.check_k(1 << 24)
    with pytest.raises(px.Configuration):
        px.check_k((1 << 24) + 1)


def test_sq8_configuration_errors_without_gpu(lib):
    lib.pxg_last_error_message.restype = ctypes.c_char_p
    h = ctypes.c_void_p()
    assert lib.pxg_sq8_create(8, 0, 1, 0, ctypes.byref(h)) == 7  # Euclidean is not an SQ8 metric
    assert b"metric" in lib.pxg_last_error_message()
    assert lib.pxg_sq8_create(70000, 2, 1, 0, ctypes.byref(h)) == 7
    assert b"dim" in lib.pxg_last_error_message()
    three = (ctypes.c_float * 3)()
    assert lib.pxg_sq_train(None, 0, 3, 1, three, three, three) == 7  # empty training (scalar.rs:145-152)
    assert b"training" in lib.pxg_last_error_message()


def test_fixture_configuration_errors_without_gpu(lib):
    lib.pxg_last_error_message.restype = ctypes.c_char_p
    buf = (ctypes.c_float * 16)()
    # a point needs a cluster (fixture.rs:93, index % clusters)
    assert lib.pxg_fixture_generate(ctypes.c_uint64(4), ctypes.c_uint32(4), ctypes.c_uint64(0), ctypes.c_uint64(0),
                                    ctypes.c_uint64(1), buf, buf) == 7
    assert b"clusters" in lib.pxg_last_error_message()
    # a query needs a corpus point (fixture.rs:102-103, % count)
    assert lib.pxg_fixture_generate(ctypes.c_uint64(0), ctypes.c_uint32(4), ctypes.c_uint64(1), ctypes.c_uint64(2),
                                    ctypes.c_uint64(1), buf, buf) == 7
    assert b"count" in lib.pxg_last_error_message()


def test_configuration_errors_carry_parameter_and_reason(lib):
    # Configuration{parameter, value, reason} (error.rs:110-128) crosses the
    # ABI as static strings, with the reference's parameter names
    lib.pxg_last_error_parameter.restype = ctypes.c_char_p
    lib.pxg_last_error_reason.restype = ctypes.c_char_p
    a = ctypes.c_uint64()
    null = ctypes.c_void_p()
    big_k = (1 << 24) + 1
    # k is checked before anything else, as flat.rs:153-155 and ivfpq.rs:988 do,
    # so a search fails on it without an index or a device
    for fn in ("pxg_flat_search", "pxg_flat_search_device", "pxg_flat_search_device_noalloc",
               "pxg_ivfpq_search", "pxg_ivfpq_search_device", "pxg_sq8_search", "pxg_sq8_search_codes",
               "pxg_sq8_search_device"):
        f = getattr(lib, fn)
        nargs = len(__import__("proxima_amd._capi", fromlist=["SIGNATURES"]).SIGNATURES[fn][1])
        args = [null] * nargs
        args[3] = ctypes.c_uint64(big_k)  # (index, queries, nq, k, ...)
        args[2] = ctypes.c_uint64(1)
        assert f(*args) == 7, fn
        assert lib.pxg_last_error_parameter() == b"k", fn
        assert lib.pxg_last_error_reason() == b"exceeds the 16777216 result ceiling"
        assert lib.pxg_last_error_detail(ctypes.byref(a), None, None) == 7 and a.value == big_k
    # subspaces outside 1..=dim (product.rs:200-206, ivfpq.rs:268-274)
    books = (ctypes.c_float * 64)()
    pts = (ctypes.c_float * 64)()
    inertia, iters = ctypes.c_double(), ctypes.c_uint64()
    st = lib.pxg_pq_train(pts, ctypes.c_uint64(8), ctypes.c_uint32(8), ctypes.c_uint64(9), ctypes.c_uint64(5),
                          ctypes.c_uint64(1), books, ctypes.byref(inertia), ctypes.byref(iters))
    assert st == 7 and lib.pxg_last_error_parameter() == b"subspaces"
    assert lib.pxg_last_error_reason() == b"must be between 1 and the space dimension"
    from proxima_amd import _capi
    cfg = _capi.IvfPqConfigC()
    assert lib.pxg_ivfpq_config_default(ctypes.c_uint64(16), ctypes.c_uint64(9), ctypes.byref(cfg)) == 0
    h = ctypes.c_void_p()
    assert lib.pxg_ivfpq_create(ctypes.c_uint32(8), 0, ctypes.byref(cfg), ctypes.byref(h)) == 7
    assert lib.pxg_last_error_parameter() == b"subspaces"
    cfg.subspaces, cfg.nprobe = 4, 17
    assert lib.pxg_ivfpq_create(ctypes.c_uint32(8), 0, ctypes.byref(cfg), ctypes.byref(h)) == 7
    assert lib.pxg_last_error_parameter() == b"nprobe"
    # a later success clears the record
    assert lib.pxg_ivfpq_config_default(ctypes.c_uint64(16), ctypes.c_uint64(4), ctypes.byref(cfg)) == 0
    assert lib.pxg_last_error_parameter() == b"" and lib.pxg_last_error_reason() == b""


def test_python_mirror_reads_parameter_names():
    import proxima_amd as px
    with pytest.raises(px.Configuration) as e:
        px.ProductQuantizer.train(px.VectorSpace(8, px.Metric.EUCLIDEAN), np.zeros((4, 8), np.float32), px.PqConfig(9))
    assert e.value.parameter == "subspaces" and e.value.reason == "must be between 1 and the space dimension"


def test_rust_ffi_declares_the_header():
    # crates/proxima-gpu/src/ffi.rs binds exactly the entry points of the header
    text = open(os.path.join(ROOT, "crates", "proxima-gpu", "src", "ffi.rs")).read()
    bound = set(re.findall(r"pub\(crate\) fn (pxg_[a-z0-9_]+)\s*\(", text))
    declared = set(declared_functions())
    assert bound == declared, (sorted(declared - bound), sorted(bound - declared))
