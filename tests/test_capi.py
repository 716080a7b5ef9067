"""CPU checks of the C ABI: the library builds/loads and exports every entry
point include/*.h declares, and the ctypes signatures cover exactly those
(no compute calls: there is no GPU here)."""
import ctypes
import glob
import os
import re

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
