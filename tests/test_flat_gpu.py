"""GPU FlatIndex: the reference's flat.rs tests, parity with the oracle (ids and
distances bit-exact) on both device paths (MFMA candidates + exact rescoring,
and the exact VALU scan), the benchmark workloads at parity-test sizes, the
device-pointer entry point, and concurrent searches on one handle."""
import threading

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

MODES = (1, 2)  # 1 = MFMA candidates + exact rescoring, 2 = exact scan


def oracle_search(px, data, ids, metric, queries, k, accept=None, live=None, threads=8):
    pd = orc.prepare_rows(metric, data)
    pq = orc.prepare_rows(metric, queries)
    return orc.flat_search(pd, ids, metric, pq, k, live=live, accept=accept, threads=threads)


def assert_same(got, want):
    gi, gd, gc = got
    wi, wd, wc = want
    assert np.array_equal(gc, wc), (gc, wc)
    for q in range(gc.size):
        c = int(gc[q])
        assert np.array_equal(gi[q, :c], wi[q, :c]), (q, gi[q, :c], wi[q, :c])
        # bit-exact distances (exact rescoring in the reference's arithmetic)
        assert np.array_equal(gd[q, :c].view(np.uint32), wd[q, :c].view(np.uint32)), (q, gd[q, :c], wd[q, :c])


def make_index(px, data, metric, ids=None, mode=0):
    space = px.VectorSpace(data.shape[1], metric)
    idx = px.FlatIndex(space, data.shape[0])
    ids = np.arange(data.shape[0], dtype=np.uint64) if ids is None else ids
    idx.insert_batch(ids, data)
    idx.set_search_mode(mode)
    return idx


# --- flat.rs:253-419 -------------------------------------------------------------
def test_round_trip(gpu):
    px = gpu
    idx = px.FlatIndex(px.VectorSpace(2, px.Metric.EUCLIDEAN))
    idx.insert(1, [3.0, 4.0])
    assert idx.contains(1)
    assert list(idx.vector(1)) == [3.0, 4.0]
    assert idx.search_all([3.0, 4.0], 1)[0].distance == 0.0
    idx.remove(1)
    assert not idx.contains(1) and idx.is_empty()


def test_empty_k_zero_and_k_larger(gpu):
    px = gpu
    idx = px.FlatIndex(px.VectorSpace(3, px.Metric.EUCLIDEAN))
    assert idx.search_all([1.0, 2.0, 3.0], 10) == []
    idx1 = px.FlatIndex(px.VectorSpace(1, px.Metric.EUCLIDEAN))
    for i in range(3):
        idx1.insert(i, [float(i)])
    assert len(idx1.search_all([0.0], 100)) == 3
    assert idx1.search_all([0.0], 0) == []


def test_identical_vectors_tie_break_on_id(gpu):
    px = gpu
    for mode in MODES:
        idx = px.FlatIndex(px.VectorSpace(2, px.Metric.EUCLIDEAN))
        idx.set_search_mode(mode)
        for i in [9, 4, 7, 1]:
            idx.insert(i, [1.0, 1.0])
        assert [h.id for h in idx.search_all([1.0, 1.0], 3)] == [1, 4, 7]


def test_duplicate_insert_and_upsert(gpu):
    px = gpu
    idx = px.FlatIndex(px.VectorSpace(1, px.Metric.EUCLIDEAN))
    idx.insert(1, [0.0])
    with pytest.raises(px.DuplicateId):
        idx.insert(1, [1.0])
    idx.upsert(1, [1.0])
    assert list(idx.vector(1)) == [1.0] and len(idx) == 1
    with pytest.raises(px.DuplicateId):
        idx.insert_batch(np.array([5, 5], np.uint64), np.zeros((2, 1), np.float32))
    assert len(idx) == 1  # all-or-nothing


def test_cosine_normalised_on_the_way_in(gpu):
    px = gpu
    idx = px.FlatIndex(px.VectorSpace(2, px.Metric.COSINE))
    idx.insert(1, [3.0, 4.0])
    v = idx.vector(1)
    assert abs(v[0] - 0.6) < 1e-6 and abs(v[1] - 0.8) < 1e-6
    a = idx.search_all([30.0, 40.0], 1)[0].distance
    b = idx.search_all([0.3, 0.4], 1)[0].distance
    assert abs(a - b) < 1e-6


def test_filter_runs_during_scan(gpu):
    px = gpu
    for mode in MODES:
        idx = px.FlatIndex(px.VectorSpace(1, px.Metric.EUCLIDEAN))
        idx.set_search_mode(mode)
        for i in range(100):
            idx.insert(i, [float(i)], {"keep": i % 10 == 0})
        hits = idx.search([0.0], 5, lambda _id, m: m.get("keep") is True)
        assert [h.id for h in hits] == [0, 10, 20, 30, 40]


def test_dimension_mismatch_and_non_finite(gpu):
    px = gpu
    idx = px.FlatIndex(px.VectorSpace(3, px.Metric.EUCLIDEAN))
    with pytest.raises(px.DimensionMismatch):
        idx.insert(1, [1.0])
    with pytest.raises(px.DimensionMismatch):
        idx.search_all([1.0, 2.0], 1)
    with pytest.raises(px.NonFinite) as e:
        idx.insert(2, [1.0, float("nan"), 0.0])
    assert e.value.index == 1
    idx.insert(3, [1.0, 2.0, 3.0])
    with pytest.raises(px.NonFinite):
        idx.search_all([float("inf"), 0.0, 0.0], 1)


def test_stats_and_slot_recycling(gpu):
    px = gpu
    idx = px.FlatIndex(px.VectorSpace(4, px.Metric.EUCLIDEAN))
    for i in range(8):
        idx.insert(i, [float(i)] * 4)
    idx.remove(3)
    st = idx.stats()
    assert st.len == 7 and st.deleted == 0 and st.graph_bytes == 0 and st.layers == 1
    assert st.vector_bytes >= 8 * 4 * 4
    idx2 = px.FlatIndex(px.VectorSpace(2, px.Metric.EUCLIDEAN))
    for i in range(4):
        idx2.insert(i, [float(i)] * 2)
    before = idx2.stats().vector_bytes
    for rnd in range(200):
        idx2.remove(rnd % 4)
        idx2.insert(rnd % 4, [float(rnd)] * 2)
    assert idx2.stats().vector_bytes == before
    with pytest.raises(px.UnknownId):
        idx2.remove(99)


def test_from_array(gpu):
    px = gpu
    space = px.VectorSpace(2, px.Metric.EUCLIDEAN)
    idx = px.FlatIndex.from_array(space, [0.0, 0.0, 1.0, 1.0, 2.0, 2.0])
    assert len(idx) == 3 and idx.search_all([2.0, 2.0], 1)[0].id == 2
    with pytest.raises(px.Configuration):
        px.FlatIndex.from_array(space, [0.0, 0.0, 1.0])


# --- parity with the oracle ---------------------------------------------------------
@pytest.mark.parametrize("metric", [0, 1, 2, 3])
@pytest.mark.parametrize("mode", MODES)
def test_parity_random_shapes(gpu, metric, mode):
    px = gpu
    rng = np.random.default_rng(100 + metric * 7 + mode)
    for (n, dim, nq, k) in [(1, 3, 1, 5), (37, 5, 3, 4), (300, 24, 17, 10), (1000, 131, 40, 33), (5000, 64, 130, 100),
                            (2500, 8, 3, 256)]:
        data = rng.standard_normal((n, dim)).astype(np.float32)
        q = rng.standard_normal((nq, dim)).astype(np.float32)
        ids = rng.permutation(n * 3)[:n].astype(np.uint64)
        idx = make_index(px, data, metric, ids, mode)
        assert_same(idx.search_batch(q, k), oracle_search(px, data, ids, metric, q, k))


@pytest.mark.parametrize("metric", [0, 1, 2, 3])
def test_exact_scan_wide_rows(gpu, metric):
    """The exact scan's two-rows-per-group form (rows of 256+ dims, a tail
    past the last multiple of 8) with removed rows, a filter and a store
    whose size is not a multiple of the row pairs; one query (256-row
    chunks) and 40 queries over 9000 rows (1024-row chunks)."""
    px = gpu
    rng = np.random.default_rng(31 + metric)
    for (n, dim, nq, k) in [(1500, 260, 1, 7), (9000, 264, 40, 25)]:
        data = rng.standard_normal((n, dim)).astype(np.float32)
        q = rng.standard_normal((nq, dim)).astype(np.float32)
        ids = rng.permutation(n * 2)[:n].astype(np.uint64)
        idx = make_index(px, data, metric, ids, 2)
        gone = rng.choice(n, n // 10, replace=False)
        for i in gone:
            idx.remove(int(ids[i]))
        live = np.ones(n, np.uint8)
        live[gone] = 0
        assert_same(idx.search_batch(q, k), oracle_search(px, data, ids, metric, q, k, live=live))
        keep = lambda i, _m: i % 4 != 1  # noqa: E731
        acc = np.array([int(ids[s]) % 4 != 1 for s in range(n)], np.uint8)
        assert_same(idx.search_batch(q, k, keep), oracle_search(px, data, ids, metric, q, k, live=live, accept=acc))


@pytest.mark.parametrize("mode", MODES)
def test_parity_with_holes_ties_and_filter(gpu, mode):
    px = gpu
    rng = np.random.default_rng(7)
    n, dim = 3000, 16
    data = rng.integers(-3, 4, (n, dim)).astype(np.float32)  # many exact ties
    ids = rng.permutation(n).astype(np.uint64)
    idx = make_index(px, data, 0, ids, mode)
    gone = rng.choice(n, 500, replace=False)
    for i in gone:
        idx.remove(int(ids[i]))
    live = np.ones(n, np.uint8)
    live[gone] = 0
    q = rng.integers(-3, 4, (50, dim)).astype(np.float32)
    assert_same(idx.search_batch(q, 20), oracle_search(px, data, ids, 0, q, 20, live=live))
    keep = lambda i, _m: i % 3 == 0  # noqa: E731
    acc = np.array([int(ids[s]) % 3 == 0 for s in range(n)], np.uint8)
    assert_same(idx.search_batch(q, 20, keep), oracle_search(px, data, ids, 0, q, 20, live=live, accept=acc))
    # reinsert into recycled slots (LIFO) and search again
    new_ids = np.arange(10_000, 10_200, dtype=np.uint64)
    new = rng.integers(-3, 4, (200, dim)).astype(np.float32)
    slots = idx.insert_batch(new_ids, new)
    data2, ids2, live2 = data.copy(), ids.copy(), live.copy()
    for s, i, v in zip(slots, new_ids, new):
        data2[s], ids2[s], live2[s] = v, i, 1
    assert_same(idx.search_batch(q, 20), oracle_search(px, data2, ids2, 0, q, 20, live=live2))


def _mixture(rng, n, dim, clusters, sigma, nq):
    centres = rng.standard_normal((clusters, dim)).astype(np.float32)
    data = centres[np.arange(n) % clusters] + sigma * rng.standard_normal((n, dim)).astype(np.float32)
    qc = rng.integers(0, clusters, nq)
    q = centres[qc] + sigma * rng.standard_normal((nq, dim)).astype(np.float32)
    return data.astype(np.float32), q.astype(np.float32)


def test_config1_l2_100k_x128_k10_full(gpu):
    """FlatIndex exact search, Euclidean, k=10: 100k x 128, 100 clusters
    sigma 0.15, 1000 queries in one batch; full parity with the oracle."""
    px = gpu
    rng = np.random.default_rng(0x9E3779B9)
    data, q = _mixture(rng, 100_000, 128, 100, 0.15, 1000)
    idx = make_index(px, data, px.Metric.EUCLIDEAN)
    got = idx.search_batch(q, 10)
    assert px.FlatIndex.last_fallbacks() == 0
    assert_same(got, oracle_search(px, data, np.arange(100_000), 0, q, 10, threads=16))


def test_config2_cosine_k100_subset(gpu):
    """FlatIndex cosine, k=100 (and k=10): 768-d unit vectors from 256 offsets;
    200k-row slice of the 1M corpus and 64 queries, full parity."""
    px = gpu
    rng = np.random.default_rng(2)
    n, dim = 200_000, 768
    offs = rng.standard_normal((256, dim)).astype(np.float32)
    data = rng.standard_normal((n, dim)).astype(np.float32) + offs[np.arange(n) % 256]
    q = rng.standard_normal((64, dim)).astype(np.float32) + offs[rng.integers(0, 256, 64)]
    idx = make_index(px, data, px.Metric.COSINE)
    for k in (100, 10):
        got = idx.search_batch(q, k)
        assert_same(got, oracle_search(px, data, np.arange(n), 1, q, k, threads=16))


def test_device_entry_point_matches_host_path(gpu):
    import torch
    px = gpu
    rng = np.random.default_rng(11)
    data = rng.standard_normal((20_000, 96)).astype(np.float32)
    q = (rng.standard_normal((300, 96)) * 3).astype(np.float32)
    for metric in (0, 1, 2):
        idx = make_index(px, data, metric)
        hi, hd, hc = idx.search_batch(q, 10)
        dq = torch.from_numpy(q).cuda()
        oi = torch.zeros((300, 10), dtype=torch.int64, device="cuda")
        od = torch.zeros((300, 10), dtype=torch.float32, device="cuda")
        oc = torch.zeros(300, dtype=torch.int32, device="cuda")
        idx.search_device(dq, 10, oi, od, oc)
        torch.cuda.synchronize()
        assert np.array_equal(oc.cpu().numpy().astype(np.uint32), hc)
        assert np.array_equal(oi.cpu().numpy().view(np.uint64), hi)
        assert np.array_equal(od.cpu().numpy().view(np.uint32), hd.view(np.uint32))
    bad = torch.from_numpy(q).cuda()
    bad[5, 7] = float("nan")
    with pytest.raises(px.NonFinite):
        idx.search_device(bad, 10, oi, od, oc)


def test_concurrent_searches_on_one_handle(gpu):
    px = gpu
    rng = np.random.default_rng(12)
    data = rng.standard_normal((30_000, 64)).astype(np.float32)
    idx = make_index(px, data, 0)
    qs = [rng.standard_normal((64, 64)).astype(np.float32) for _ in range(8)]
    want = [idx.search_batch(q, 10) for q in qs]
    got = [None] * 8
    errs = []

    def run(i):
        try:
            for _ in range(3):
                got[i] = idx.search_batch(qs[i], 10)
        except Exception as e:  # pragma: no cover
            errs.append(e)

    th = [threading.Thread(target=run, args=(i,)) for i in range(8)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errs
    for g, w in zip(got, want):
        for a, b in zip(g, w):
            assert np.array_equal(a, b)


def test_insert_device_matches_host_insert(gpu):
    import torch
    px = gpu
    rng = np.random.default_rng(13)
    data = (rng.standard_normal((5000, 77)) * 4).astype(np.float32)
    for metric in (0, 1, 2):
        a = make_index(px, data, metric)
        b = px.FlatIndex(px.VectorSpace(77, metric))
        b.insert_device(np.arange(5000, dtype=np.uint64), torch.from_numpy(data).cuda())
        for i in (0, 17, 4999):
            assert np.array_equal(a.vector(i).view(np.uint32), b.vector(i).view(np.uint32))
        q = rng.standard_normal((40, 77)).astype(np.float32)
        for x, y in zip(a.search_batch(q, 12), b.search_batch(q, 12)):
            assert np.array_equal(x, y)
    bad = torch.from_numpy(data[:10].copy()).cuda()
    bad[3, 5] = float("inf")
    with pytest.raises(px.NonFinite):
        b.insert_device(np.arange(100_000, 100_010, dtype=np.uint64), bad)
    assert len(b) == 5000


def test_growth_preserves_contents(gpu):
    px = gpu
    rng = np.random.default_rng(21)
    data = rng.standard_normal((5000, 24)).astype(np.float32)
    idx = px.FlatIndex(px.VectorSpace(24, 0))  # capacity 0: grows 1024 -> 2048 -> 4096 -> 8192
    for a in range(0, 5000, 700):
        idx.insert_batch(np.arange(a, min(a + 700, 5000), dtype=np.uint64), data[a:a + 700])
    for i in (0, 1023, 1024, 2047, 4999):
        assert np.array_equal(idx.vector(i), data[i])
    q = rng.standard_normal((20, 24)).astype(np.float32)
    assert_same(idx.search_batch(q, 15), oracle_search(px, data, np.arange(5000), 0, q, 15))


@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("n,nq", [(16384, 1000), (131072, 40)])
def test_merge_register_boundary(gpu, metric, n, nq):
    """The merges that hold a query's keys in registers, at their limits.
    1000 queries over 16,384 rows make 32 splits: k = 48 (k' = 64) puts
    exactly 2048 keys per query into the 256-thread merge. 40 queries over
    131,072 rows make 256 splits: k = 48 puts exactly 16,384 keys into the
    1024-thread merge. k = 49 (k' = 65) takes the general merge, and k = 1 is
    the smallest selection. Every vector is stored twice under unrelated ids,
    so equal distances are ordered by id, and a filter that accepts n / 500
    rows leaves every query fewer than k' candidates at the first shape."""
    px = gpu
    rng = np.random.default_rng(901 + metric + n)
    dim = 40 if n <= 16384 else 16
    half = rng.standard_normal((n // 2, dim)).astype(np.float32)
    data = np.concatenate([half, half])
    ids = rng.permutation(n).astype(np.uint64)
    idx = make_index(px, data, metric, ids, 1)
    q = rng.standard_normal((nq, dim)).astype(np.float32)
    for k in (1, 48, 49):
        assert_same(idx.search_batch(q, k), oracle_search(px, data, ids, metric, q, k))
    keep = lambda i, _m: i % 500 == 0  # noqa: E731
    acc = (ids % 500 == 0).astype(np.uint8)
    assert_same(idx.search_batch(q, 48, keep), oracle_search(px, data, ids, metric, q, 48, accept=acc))


@pytest.mark.parametrize("n,nq", [(16384, 1000), (131072, 40)])
def test_merge_register_no_or_one_candidate(gpu, n, nq):
    """Filters that accept no row and exactly one row on the MFMA path: the
    merges that hold a query's keys in registers (256 threads at 1000
    queries over 16,384 rows, 1024 threads at 40 queries over 131,072 rows)
    see zero or one usable key per query, and the seeding pass bounds
    nothing. Counts 0 and 1, the one id and its exact distance match the
    oracle."""
    px = gpu
    rng = np.random.default_rng(77 + n)
    dim = 32
    data = rng.standard_normal((n, dim)).astype(np.float32)
    ids = rng.permutation(2 * n)[:n].astype(np.uint64)
    idx = make_index(px, data, 0, ids, 1)
    q = rng.standard_normal((nq, dim)).astype(np.float32)
    none = idx.search_batch(q, 10, lambda i, _m: False)
    assert_same(none, oracle_search(px, data, ids, 0, q, 10, accept=np.zeros(n, np.uint8)))
    assert not none[2].any()
    one_id = int(ids[n // 3])
    got = idx.search_batch(q, 10, lambda i, _m: i == one_id)
    assert_same(got, oracle_search(px, data, ids, 0, q, 10, accept=(ids == one_id).astype(np.uint8)))
    assert (got[2] == 1).all() and (got[0][:, 0] == one_id).all()


@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("n,ks", [(300, (5, 112, 113, 200)), (1024, (240, 241, 250))])
def test_seed_word_count_boundary(gpu, metric, n, ks):
    """The seeding pass bounds k' = k + 16 only from at least k' words, one
    tile's 128 per split. 300 rows are one split of 3 tiles on the MFMA
    path: k = 112 (k' = 128) is seeded, k = 113 and 200 take the unseeded
    full pass. 1024 rows are two splits of 4 tiles: k = 240 (k' = 256) is
    seeded, k = 241 and 250 are not, and their rows append whole tiles and
    compact them (512-key buffers). A filter leaves some tiles partly
    usable."""
    px = gpu
    rng = np.random.default_rng(313 + metric + n)
    dim, nq = 24, 50
    data = rng.standard_normal((n, dim)).astype(np.float32)
    ids = rng.permutation(10 * n)[:n].astype(np.uint64)
    idx = make_index(px, data, metric, ids, 1)
    q = rng.standard_normal((nq, dim)).astype(np.float32)
    for k in ks:
        assert_same(idx.search_batch(q, k), oracle_search(px, data, ids, metric, q, k))
    keep = lambda i, _m: i % 3 != 0  # noqa: E731
    acc = (ids % 3 != 0).astype(np.uint8)
    for k in ks[1:3]:
        assert_same(idx.search_batch(q, k, keep), oracle_search(px, data, ids, metric, q, k, accept=acc))


@pytest.mark.parametrize("n,dim,nqs", [(100_000, 128, (13, 14)), (300_000, 256, (5, 6)), (20_000, 128, (52, 53))])
def test_default_mode_path_crossover(gpu, n, dim, nqs):
    """The default mode picks the exact scan or the MFMA path by estimated
    cost; batch sizes on either side of each store's crossover (100k x 128 at
    13/14 queries, 300k x 256 at 5/6, 20k x 128 at 52/53) take different
    paths and match the oracle bit for bit."""
    px = gpu
    rng = np.random.default_rng(n + dim)
    data = rng.standard_normal((n, dim)).astype(np.float32)
    ids = np.arange(n, dtype=np.uint64)
    idx = make_index(px, data, 0, ids, 0)
    q = rng.standard_normal((max(nqs), dim)).astype(np.float32)
    for nq in nqs:
        assert_same(idx.search_batch(q[:nq], 10), oracle_search(px, data, ids, 0, q[:nq], 10, threads=16))


def test_search_mode_range(gpu):
    """Search modes are 0 (automatic), 1 (MFMA path) and 2 (exact scan);
    others are refused as a configuration error naming the parameter, and
    the index keeps its mode."""
    px = gpu
    rng = np.random.default_rng(5)
    data = rng.standard_normal((5000, 16)).astype(np.float32)
    idx = make_index(px, data, 0, mode=1)
    for bad in (3, -1):
        with pytest.raises(px.ProximaError) as e:
            idx.set_search_mode(bad)
        assert "mode" in str(e.value)
    q = rng.standard_normal((40, 16)).astype(np.float32)
    assert_same(idx.search_batch(q, 7), oracle_search(px, data, np.arange(5000, dtype=np.uint64), 0, q, 7))


@pytest.mark.parametrize("metric", [0, 2])
def test_thresholds_shared_across_splits(gpu, metric):
    """The MFMA path splits the store over many workgroups per query block,
    which share each query's running k'-th key. Queries whose neighbours sit
    in the last split, queries spread over the store, k from 1 to 64 and a
    filter: ids and distances match the oracle bit for bit."""
    px = gpu
    rng = np.random.default_rng(77 + metric)
    n, dim = 200_000, 64
    data = rng.standard_normal((n, dim)).astype(np.float32)
    idx = make_index(px, data, metric, mode=1)
    near_end = data[n - 500 + rng.integers(0, 500, 128)] + np.float32(0.01) * rng.standard_normal(
        (128, dim)).astype(np.float32)
    spread = rng.standard_normal((128, dim)).astype(np.float32)
    q = np.concatenate([near_end, spread])
    ids = np.arange(n, dtype=np.uint64)
    for k in (1, 10, 64):
        assert_same(idx.search_batch(q, k), oracle_search(px, data, ids, metric, q, k))
    acc = (np.arange(n) % 3 == 1).astype(np.uint8)
    got = idx.search_batch(q, 10, lambda i, _m: i % 3 == 1)
    assert_same(got, oracle_search(px, data, ids, metric, q, 10, accept=acc))


@pytest.mark.parametrize("metric", [0, 1, 2])
@pytest.mark.parametrize("dim", [16, 32])
def test_seeded_thresholds(gpu, metric, dim):
    """With many tiles per split, a first pass over one tile of every split
    seeds each query's threshold before the full pass, which filters that
    tile's stored keys instead of computing them again (k = 1 and 10 select
    the seed from each split's two smallest keys, k = 100 from every key).
    Integer data (exact distance ties at the seed), removed rows, a filter,
    queries whose neighbours all sit past the sampled tiles, and k from 1 to
    100: ids and distances match the oracle bit for bit, for rows of 16 and
    32 floats."""
    px = gpu
    rng = np.random.default_rng(5 + metric + dim)
    n, nq = 140_000, 1024  # 8 query blocks x 61 splits of 18 tiles (2304 rows)
    data = rng.integers(-2, 3, (n, dim)).astype(np.float32)
    ids = rng.permutation(n).astype(np.uint64)
    idx = make_index(px, data, metric, ids, mode=1)
    gone = rng.choice(n, 3000, replace=False)
    for i in gone:
        idx.remove(int(ids[i]))
    live = np.ones(n, np.uint8)
    live[gone] = 0
    # rows 128..255 of every split are never sampled: aim half the queries
    # there, with a shift that no sampled row shares
    far = np.concatenate([np.arange(s + 128, s + 256) for s in range(0, n - 256, 2304)])
    q = np.concatenate([data[rng.choice(far, nq // 2)] + np.float32(0.25),
                        rng.integers(-2, 3, (nq // 2, dim)).astype(np.float32)])
    for k in (1, 10, 100):
        assert_same(idx.search_batch(q, k), oracle_search(px, data, ids, metric, q, k, live=live))
    acc = np.array([int(i) % 4 == 1 for i in ids], np.uint8)
    got = idx.search_batch(q, 10, lambda i, _m: i % 4 == 1)
    assert_same(got, oracle_search(px, data, ids, metric, q, 10, live=live, accept=acc))


@pytest.mark.parametrize("metric", [0, 2])
def test_seeded_short_last_split(gpu, metric):
    """A seeded search whose last split is shorter than a tile: 57,346 rows
    and 1024 queries split into 57 splits of 8 tiles (1024 rows), the last
    holding 2 rows, so its seeding tile is mostly unusable slots and the full
    pass's stored first tile is partial. Removed rows (two of them in the last
    split), a filter, and k of 1, 10 and 30."""
    px = gpu
    rng = np.random.default_rng(91 + metric)
    n, nq, dim = 57_346, 1024, 24
    data = rng.standard_normal((n, dim)).astype(np.float32)
    data[n - 2:] = data[7]  # the last split's rows tie with an early row
    ids = rng.permutation(n).astype(np.uint64)
    idx = make_index(px, data, metric, ids, mode=1)
    gone = np.concatenate([rng.choice(n - 2, 400, replace=False), [n - 1]])
    for i in gone:
        idx.remove(int(ids[i]))
    live = np.ones(n, np.uint8)
    live[gone] = 0
    q = np.concatenate([data[rng.choice(n, nq // 2)] + np.float32(0.01), rng.standard_normal((nq // 2, dim))])
    q = q.astype(np.float32)
    for k in (1, 10, 30):
        assert_same(idx.search_batch(q, k), oracle_search(px, data, ids, metric, q, k, live=live, threads=16))
    acc = np.array([int(i) % 3 != 0 for i in ids], np.uint8)
    got = idx.search_batch(q, 10, lambda i, _m: i % 3 != 0)
    assert_same(got, oracle_search(px, data, ids, metric, q, 10, live=live, accept=acc, threads=16))


# --- k beyond the block selections (check_k allows up to 2^24, index.rs:212-224) ----------
@pytest.mark.parametrize("metric", [0, 2, 3])
def test_large_k_matches_oracle(gpu, metric):
    px = gpu
    rng = np.random.default_rng(70 + metric)
    n, dim = 20_000, 24
    data = rng.standard_normal((n, dim)).astype(np.float32)
    data[100:140] = data[7]  # exact ties across the cut
    ids = rng.permutation(n).astype(np.uint64)
    idx = make_index(px, data, metric, ids=ids)
    for s in (3, 9, 11):
        idx.remove(int(ids[s]))
    live = np.ones(n, np.uint8)
    live[[3, 9, 11]] = 0
    q = rng.standard_normal((6, dim)).astype(np.float32)
    q[0] = data[7]
    for k in (1025, 5000, n + 5):
        got = idx.search_batch(q, k)
        want = oracle_search(px, data, ids, metric, q, k, live=live)
        assert_same(got, want)
    # a filter with the wide path
    keep = lambda i, _m: int(i) % 5 != 0  # noqa: E731
    acc = np.array([0 if not live[s] else (int(ids[s]) % 5 != 0) for s in range(n)], np.uint8)
    assert_same(idx.search_batch(q, 3000, keep), oracle_search(px, data, ids, metric, q, 3000, accept=acc, live=live))


def test_k_far_above_the_live_count(gpu):
    px = gpu
    rng = np.random.default_rng(3)
    data = rng.standard_normal((100, 16)).astype(np.float32)
    for mode in MODES:
        idx = make_index(px, data, 0, mode=mode)
        q = rng.standard_normal((4, 16)).astype(np.float32)
        got = idx.search_batch(q, 1 << 20)
        want = oracle_search(px, data, np.arange(100, dtype=np.uint64), 0, q, 100)
        gi, gd, gc = got
        assert list(gc) == [100] * 4
        assert_same((gi[:, :100], gd[:, :100], gc), want)
    with pytest.raises(px.Configuration):
        idx.search_batch(q, (1 << 24) + 1)
