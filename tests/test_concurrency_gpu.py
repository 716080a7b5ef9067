"""Searches on one handle from many host threads (the C ABI's re-entrancy
claim, the reference's Sync expectation of proxima-index/tests/hnsw.rs:266-315
and the server's thread-per-connection reads under the collection's read
lock): every thread gets exactly the single-threaded results, for IVF-PQ
(plain, reranked, filtered, and the wide shortlist path) and SQ8 (integer,
rescored, wide)."""
import threading

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def hammer(jobs, threads=12, reps=3):
    """Run each job (a no-argument callable) on its own thread `reps` times;
    return the results of the last repetition and any exception."""
    got = [None] * len(jobs)
    errs = []
    barrier = threading.Barrier(len(jobs))

    def run(i):
        try:
            barrier.wait()
            for _ in range(reps):
                got[i] = jobs[i]()
        except Exception as e:  # pragma: no cover - reported below
            errs.append(e)

    th = [threading.Thread(target=run, args=(i,)) for i in range(len(jobs))]
    for t in th:
        t.start()
    for t in th:
        t.join()
    return got, errs


def same(a, b):
    return all(np.array_equal(x, y) for x, y in zip(a, b))


def test_ivfpq_searches_on_one_handle(gpu):
    px = gpu
    rng = np.random.default_rng(17)
    n, dim, nlist, m = 20_000, 32, 32, 8
    data = (rng.standard_normal((40, dim))[np.arange(n) % 40] * 3 + rng.standard_normal((n, dim))).astype(np.float32)
    cents, books, _ = orc.ivf_train(data, nlist, m, max_iter=5, seed=9)
    codes, list_of = orc.ivf_encode(data, cents, books, m)
    idxs = []
    for rerank in (0, 40):
        cfg = px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62).with_rerank(rerank)
        idx = px.IvfPqIndex(px.VectorSpace(dim, 0), cfg)
        idx.insert_batch(np.arange(n, dtype=np.uint64), data)
        idx.load_trained(cents, books, codes, list_of)
        idxs.append(idx)
    keep = lambda i, _m: int(i) % 3 != 0  # noqa: E731
    qs = [(data[rng.integers(0, n, 50)] + 0.1).astype(np.float32) for _ in range(12)]
    specs = [(idxs[i % 2], qs[i], (10, 1200)[i % 4 == 3], (4, 16)[i % 3 == 0], keep if i % 5 == 0 else None)
             for i in range(12)]
    jobs = [lambda s=s: s[0].search_batch(s[1], s[2], s[4], nprobe=s[3]) for s in specs]
    want = [j() for j in jobs]
    got, errs = hammer(jobs)
    assert not errs, errs
    for g, w in zip(got, want):
        assert same(g, w)


def test_sq8_searches_on_one_handle(gpu):
    px = gpu
    rng = np.random.default_rng(19)
    n, dim = 60_000, 64
    x = rng.uniform(-1, 1, (n, dim)).astype(np.float32)
    idx = px.Sq8Index(px.VectorSpace(dim, px.Metric.INNER_PRODUCT), capacity=n)
    idx.train(x[:10_000])
    idx.insert_batch(np.arange(n, dtype=np.uint64), x)
    keep = lambda i, _m: int(i) % 4 != 1  # noqa: E731
    qs = [rng.uniform(-1, 1, (40, dim)).astype(np.float32) for _ in range(12)]
    specs = [(qs[i], (10, 2000)[i % 4 == 2], (0, 50)[i % 2], keep if i % 3 == 0 else None) for i in range(12)]
    jobs = [lambda s=s: idx.search_batch(s[0], s[1], s[3], rescore=s[2]) for s in specs]
    want = [j() for j in jobs]
    got, errs = hammer(jobs)
    assert not errs, errs
    for g, w in zip(got, want):
        assert same(g, w)
