"""The C ABI serves what the reference's VectorIndex serves: any k up to
check_k's 2^24 (index.rs:212-224) on IVF-PQ and SQ8 (flat: test_flat_gpu.py),
IVF-PQ shortlists (max(rerank, k)) beyond the block selections, IVF-PQ with
as many subspaces as dimensions (IvfPqConfig::validate, ivfpq.rs:268-274), and
IvfPqIndex::compact (ivfpq.rs:907-975) with the reference's invariance test
(ivfpq.rs:1519-1546). Every result is checked against the oracle bit for bit."""
import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_same(got, want):
    gi, gd, gc = got
    wi, wd, wc = want
    assert np.array_equal(gc, wc), (gc, wc)
    for q in range(gc.size):
        c = int(gc[q])
        assert np.array_equal(gi[q, :c], wi[q, :c]), (q, gi[q, :c], wi[q, :c], gd[q, :c], wd[q, :c])
        assert np.array_equal(bits(gd[q, :c]), bits(wd[q, :c])), (q, gd[q, :c], wd[q, :c])


def clustered(rng, n, dim, c=16):
    centres = rng.standard_normal((c, dim)).astype(np.float32) * 3
    return (centres[np.arange(n) % c] + rng.standard_normal((n, dim))).astype(np.float32)


def ivf_index(px, data, metric, nlist, m, rerank=0, seed=5):
    prep = orc.prepare_rows(metric, data)
    cents, books, _ = orc.ivf_train(prep, nlist, m, max_iter=6, seed=seed)
    codes, list_of = orc.ivf_encode(prep, cents, books, m)
    cfg = px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62).with_rerank(rerank).with_seed(seed)
    idx = px.IvfPqIndex(px.VectorSpace(data.shape[1], metric), cfg)
    idx.insert_batch(np.arange(data.shape[0], dtype=np.uint64), data)
    idx.load_trained(cents, books, codes, list_of)
    return idx, prep, cents, books, codes, list_of


@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("rerank,k", [(0, 1500), (2000, 10), (2000, 2500)])
def test_ivf_wide_shortlists(gpu, metric, rerank, k):
    px = gpu
    rng = np.random.default_rng(11 + metric)
    n, dim, nlist, m = 9000, 32, 16, 8
    data = clustered(rng, n, dim)
    idx, prep, cents, books, codes, list_of = ivf_index(px, data, metric, nlist, m, rerank)
    q = (data[rng.integers(0, n, 12)] + 0.05).astype(np.float32)
    qp = orc.prepare_rows(metric, q)
    for nprobe in (3, 16):
        got = idx.search_batch(q, k, nprobe=nprobe)
        want = orc.ivf_search(metric, cents, books, codes, list_of, np.arange(n), qp, k, nprobe, m,
                              vectors=prep if rerank else None, rerank=rerank, threads=8)
        assert_same(got, want)
    # with a filter
    keep = lambda i, _m: int(i) % 4 != 1  # noqa: E731
    acc = (np.arange(n) % 4 != 1).astype(np.uint8)
    got = idx.search_batch(q, k, keep, nprobe=8)
    want = orc.ivf_search(metric, cents, books, codes, list_of, np.arange(n), qp, k, 8, m,
                          vectors=prep if rerank else None, rerank=rerank, accept=acc, threads=8)
    assert_same(got, want)


def test_ivf_untrained_large_k(gpu):
    px = gpu
    rng = np.random.default_rng(2)
    n, dim = 3000, 16
    data = rng.standard_normal((n, dim)).astype(np.float32)
    cfg = px.IvfPqConfig(8, 4).with_train_threshold(1 << 62)
    idx = px.IvfPqIndex(px.VectorSpace(dim, 0), cfg)
    idx.insert_batch(np.arange(n, dtype=np.uint64), data)
    assert not idx.is_trained()
    q = rng.standard_normal((5, dim)).astype(np.float32)
    for k in (2000, 1 << 20):
        got = idx.search_batch(q, k)
        want = orc.flat_search(data, np.arange(n), 0, q, min(k, n), threads=8)
        assert_same((got[0][:, :n], got[1][:, :n], got[2]), want)


@pytest.mark.parametrize("metric", [0, 1])
def test_ivf_one_dimension_per_subspace(gpu, metric):
    """subspaces = dim = 200: tables beyond the LDS take the wide scan."""
    px = gpu
    rng = np.random.default_rng(21)
    n, dim, nlist = 2500, 200, 8
    data = clustered(rng, n, dim, 8)
    idx, prep, cents, books, codes, list_of = ivf_index(px, data, metric, nlist, dim, rerank=0)
    q = (data[::400] + 0.1).astype(np.float32)
    qp = orc.prepare_rows(metric, q)
    for k, nprobe in ((10, 2), (50, 8)):
        got = idx.search_batch(q, k, nprobe=nprobe)
        want = orc.ivf_search(metric, cents, books, codes, list_of, np.arange(n), qp, k, nprobe, dim, threads=8)
        assert_same(got, want)
    # GPU training with M = dim agrees with the oracle's
    cfg = px.IvfPqConfig(nlist, dim).with_train_threshold(1 << 62).with_seed(3).with_max_iterations(4)
    t = px.IvfPqIndex(px.VectorSpace(dim, metric), cfg)
    t.insert_batch(np.arange(n, dtype=np.uint64), data)
    t.train()
    gc, gb, gcodes, glist = t.parts()
    wc, wb, _ = orc.ivf_train(prep, nlist, dim, max_iter=4, seed=3)
    assert np.array_equal(bits(gc), bits(wc)) and np.array_equal(bits(gb), bits(wb))
    wcodes, wlist = orc.ivf_encode(prep, wc, wb, dim)
    assert np.array_equal(gcodes, wcodes) and np.array_equal(glist, wlist)


def test_ivf_compaction_does_not_change_results(gpu):  # ivfpq.rs:1519-1546
    px = gpu
    rng = np.random.default_rng(4)
    n, dim = 600, 16
    data = rng.standard_normal((n, dim)).astype(np.float32)
    for retain in (True, False):
        cfg = px.IvfPqConfig(8, 4).with_seed(4).with_train_threshold(1 << 62).with_retain_vectors(retain)
        idx = px.IvfPqIndex(px.VectorSpace(dim, 0), cfg)
        idx.insert_batch(np.arange(n, dtype=np.uint64), data)
        idx.train()
        for i in range(0, n, 3):
            idx.remove(i)
        q = data[::50]
        before = idx.search_batch(q, 10)
        assert idx.compact() == 200
        after = idx.search_batch(q, 10)
        assert_same(after, before)
        assert idx.compact() == 0
        assert len(idx) == 400 and idx.slots()[0].size == 400
        # inserts after a compaction take fresh slots and are found
        idx.insert(10_000, data[1] + 0.001)
        assert idx.contains(10_000)
        ids = idx.search_batch(data[1:2], 20)[0][0]
        assert 10_000 in ids.tolist()


def test_sq8_large_k_and_rescore(gpu):
    px = gpu
    rng = np.random.default_rng(8)
    n, dim = 8000, 48
    x = rng.uniform(-1, 1, (n, dim)).astype(np.float32)
    idx = px.Sq8Index(px.VectorSpace(dim, px.Metric.INNER_PRODUCT), capacity=n)
    idx.train(x[:3000])
    idx.insert_batch(np.arange(n, dtype=np.uint64), x)
    for s in (5, 77):
        idx.remove(s)
    live = np.ones(n, np.uint8)
    live[[5, 77]] = 0
    mn, sc, inv, _ = orc.sq_train(x[:3000], True)
    codes = orc.sq_encode(x, mn, inv, True, 1).view(np.int8)
    q = rng.uniform(-1, 1, (7, dim)).astype(np.float32)
    qc = orc.sq_encode(q, mn, inv, True, 1).view(np.int8)
    for k, rescore in ((3000, 0), (10, 2000), (2500, 2600), (1 << 20, 0)):
        kk = min(k, n)
        want = orc.sq8_search(codes, np.arange(n), qc, kk, live=live, threads=8, rescore=rescore, qf=q,
                              ranges=(mn, sc), per_dim=True)
        gi, gd, gc = idx.search_batch(q, k, rescore=rescore)
        assert_same((gi[:, :kk], gd[:, :kk], gc), want)
