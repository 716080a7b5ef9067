"""pxg_flat_search_device_noalloc (the flat search that allocates nothing)
against pxg_flat_search_device: the same ids, distances and counts bit for
bit, on two calls in a row (the second with a smaller input), on the MFMA and
the exact paths, with a filter, with k beyond the block selections (the wide
path inside the fixed scratch), and with a request too large for the scratch
(a Capacity error before any work)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _noalloc(px):
    return px._lib.pxg_flat_search_device_noalloc


def _run(px, fn, idx, q, k, accept=None, stream=None):
    import torch
    nq = q.shape[0]
    ids = torch.full((nq, k), -7, dtype=torch.int64, device="cuda")
    dist = torch.full((nq, k), -7.0, dtype=torch.float32, device="cuda")
    cnt = torch.full((nq,), -7, dtype=torch.int32, device="cuda")
    st = fn(idx._h, C.c_void_p(q.data_ptr()), nq, k, None if accept is None else C.c_void_p(accept.data_ptr()),
            C.c_void_p(ids.data_ptr()), C.c_void_p(dist.data_ptr()), C.c_void_p(cnt.data_ptr()),
            None if stream is None else C.c_void_p(stream))
    return st, ids.cpu().numpy(), dist.cpu().numpy(), cnt.cpu().numpy()


def _same(a, b):
    sa, ia, da, ca = a
    sb, ib, db, cb = b
    assert sa == 0 and sb == 0
    assert np.array_equal(ca, cb)
    for q in range(ca.size):
        c = int(ca[q])
        assert np.array_equal(ia[q, :c], ib[q, :c]), q
        assert np.array_equal(da[q, :c].view(np.uint32), db[q, :c].view(np.uint32)), q


@pytest.mark.parametrize("metric,mode", [(0, 0), (1, 1), (2, 2), (3, 0)])
def test_noalloc_matches_the_allocating_search(gpu, metric, mode):
    import torch
    px = gpu
    na = _noalloc(px)
    rng = np.random.default_rng(31 + metric)
    n, dim = 60_000, 96
    data = (rng.standard_normal((n, dim)) + rng.standard_normal((40, dim))[np.arange(n) % 40]).astype(np.float32)
    idx = px.FlatIndex(px.VectorSpace(dim, metric), n)
    idx.insert_batch(rng.permutation(n).astype(np.uint64) * 3 + 1, data)
    idx.set_search_mode(mode)
    for r in (5, 17, 29):
        idx.remove(int(idx.slots()[0][r]))
    q1 = torch.from_numpy((data[rng.integers(0, n, 700)] + 0.1).astype(np.float32)).cuda()
    q2 = torch.from_numpy((data[rng.integers(0, n, 90)] - 0.1).astype(np.float32)).cuda()
    ref = px._lib.pxg_flat_search_device
    # two calls in a row, the second smaller; then the first again
    for q, k in ((q1, 40), (q2, 7), (q1, 40)):
        _same(_run(px, na, idx, q, k), _run(px, ref, idx, q, k))
    # a filter, and the caller's stream
    acc = torch.from_numpy((np.arange(idx.slots()[0].size) % 3 != 0).astype(np.uint8)).cuda()
    s = torch.cuda.Stream()
    _same(_run(px, na, idx, q2, 12, acc, s.cuda_stream), _run(px, ref, idx, q2, 12, acc))


def test_noalloc_wide_k_and_capacity(gpu):
    import torch
    px = gpu
    na = _noalloc(px)
    rng = np.random.default_rng(5)
    n, dim = 6000, 32
    data = rng.standard_normal((n, dim)).astype(np.float32)
    idx = px.FlatIndex(px.VectorSpace(dim, 0), n)
    idx.insert_batch(np.arange(n, dtype=np.uint64), data)
    ref = px._lib.pxg_flat_search_device
    q = torch.from_numpy(rng.standard_normal((50, dim)).astype(np.float32)).cuda()
    _same(_run(px, na, idx, q, 2500), _run(px, ref, idx, q, 2500))
    _same(_run(px, na, idx, q[:3], 1 << 20), _run(px, ref, idx, q[:3], 1 << 20))
    # prepared query rows alone would exceed the scratch: refused up front
    big = torch.zeros((400_000, dim * 4), dtype=torch.float32, device="cuda")
    idx4 = px.FlatIndex(px.VectorSpace(dim * 4, 0), 16)
    idx4.insert_batch(np.arange(16, dtype=np.uint64), rng.standard_normal((16, dim * 4)).astype(np.float32))
    st = _run(px, na, idx4, big, 1)[0]
    assert st == 4  # PXG_ERR_CAPACITY
    assert "no-allocation scratch" in px._lib.pxg_last_error_message().decode()
    # still serves afterwards
    _same(_run(px, na, idx, q, 10), _run(px, ref, idx, q, 10))


def test_noalloc_capacity_after_queued_stages(gpu):
    # the prepared queries (50000 x 128 x 4 bytes) and the per-query regions fit
    # the 128 MiB, but one split of candidate buffers (50000 x 512 x 8 bytes at
    # k = 100, whose k' = 116 takes the 512-key buffers) does not: the call
    # fails with Capacity after its first stages were queued, waits for them,
    # and the next calls are served correctly
    import torch
    px = gpu
    na = _noalloc(px)
    rng = np.random.default_rng(9)
    n, dim = 8192, 128
    data = rng.standard_normal((n, dim)).astype(np.float32)
    idx = px.FlatIndex(px.VectorSpace(dim, 0), n)
    idx.insert_batch(np.arange(n, dtype=np.uint64), data)
    idx.set_search_mode(1)
    big = torch.from_numpy(rng.standard_normal((50_000, dim)).astype(np.float32)).cuda()
    st = _run(px, na, idx, big, 100)[0]
    assert st == 4  # PXG_ERR_CAPACITY
    px._lib.pxg_last_error_parameter.restype = C.c_char_p
    assert px._lib.pxg_last_error_parameter() == b"no-allocation scratch"
    ref = px._lib.pxg_flat_search_device
    q = big[:3000].contiguous()
    _same(_run(px, na, idx, q, 100), _run(px, ref, idx, q, 100))
    _same(_run(px, na, idx, q[:64], 10), _run(px, ref, idx, q[:64], 10))
