"""recall_at_k over the GPU indexes: the reference's recall.rs tests
(recall.rs:191-264) plus recall of the approximate indexes."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def fixture(px, count):  # recall.rs:197-211
    flat = px.FlatIndex(px.VectorSpace(4, px.Metric.EUCLIDEAN))
    queries = []
    for i in range(count):
        t = np.float32(i) * np.float32(0.1)
        v = np.array([t, np.sin(t), -t, 1.0], np.float32)
        flat.insert(i, v)
        if i % 10 == 0:
            queries.append(v)
    return flat, np.array(queries, np.float32).reshape(-1, 4)


def test_self_recall_is_perfect(gpu):  # recall.rs:214-222
    px = gpu
    flat, q = fixture(px, 200)
    r = px.recall_at_k(flat, flat, q, 10)
    assert r.mean == 1.0 and r.min == 1.0 and r.short_results == 0 and r.below(1.0) == 0.0


def test_broken_index_scores_badly(gpu):  # recall.rs:225-241
    px = gpu
    flat, q = fixture(px, 200)
    half = px.FlatIndex(px.VectorSpace(4, px.Metric.EUCLIDEAN))
    for i, id_ in enumerate(flat.ids()):
        if i % 2 == 0:
            half.insert(id_, flat.vector(id_))
    r = px.recall_at_k(half, flat, q, 10)
    assert 0.25 < r.mean < 0.75, str(r)


def test_short_results_dimension_empty_and_display(gpu):  # recall.rs:244-272
    px = gpu
    flat, q = fixture(px, 5)
    r = px.recall_at_k(flat, flat, q, 10)
    assert r.mean == 1.0 and r.short_results == 0
    flat10, _ = fixture(px, 10)
    with pytest.raises(px.Configuration):
        px.recall_at_k(flat10, flat10, np.array([1.0, 2.0, 3.0], np.float32), 5)
    r = px.recall_at_k(flat10, flat10, np.zeros(0, np.float32), 5)
    assert r.queries == 0 and r.mean == 0.0
    flat50, q50 = fixture(px, 50)
    s = str(px.recall_at_k(flat50, flat50, q50, 5))
    assert s.startswith("recall@5: mean 1.0000") and "\n" not in s


def test_recall_of_approximate_indexes_and_filtered(gpu):
    px = gpu
    rng = np.random.default_rng(4)
    n, dim = 20000, 32
    centres = rng.standard_normal((50, dim)).astype(np.float32)
    x = (centres[rng.integers(0, 50, n)] + 0.3 * rng.standard_normal((n, dim))).astype(np.float32)
    q = (centres[rng.integers(0, 50, 64)] + 0.3 * rng.standard_normal((64, dim))).astype(np.float32)
    ids = np.arange(n, dtype=np.uint64)
    # SQ8 on a uniform U(-1,1) workload like the 10M x 96 benchmark (inner product)
    xu = rng.uniform(-1, 1, (n, 64)).astype(np.float32)
    qu = rng.uniform(-1, 1, (64, 64)).astype(np.float32)
    truth = px.FlatIndex(px.VectorSpace(64, px.Metric.INNER_PRODUCT))
    truth.insert_batch(ids, xu)
    sq = px.Sq8Index(px.VectorSpace(64, px.Metric.INNER_PRODUCT))
    sq.train(xu[:5000])
    sq.insert_batch(ids, xu)
    r = px.recall_at_k(sq, truth, qu, 10)
    assert r.queries == 64 and r.mean > 0.85 and r.short_results == 0, str(r)
    rr = px.recall_at_k(_Rescore(sq, 100), truth, qu, 10)
    assert rr.mean >= r.mean, (str(rr), str(r))
    keep = lambda i, m: i % 3 == 0  # noqa: E731
    rf = px.recall_at_k_filtered(sq, truth, qu, 10, keep)
    assert rf.queries == 64 and rf.mean > 0.85 and rf.short_results == 0, str(rf)
    l2 = px.FlatIndex(px.VectorSpace(dim, px.Metric.EUCLIDEAN))
    l2.insert_batch(ids, x)
    ivf = px.IvfPqIndex(px.VectorSpace(dim, px.Metric.EUCLIDEAN),
                        px.IvfPqConfig(64, 8).with_nprobe(8).with_rerank(100).with_train_threshold(1 << 62))
    ivf.insert_batch(ids, x)
    ivf.train()
    ri = px.recall_at_k(ivf, l2, q, 10)
    assert ri.mean > 0.8, str(ri)
    # monotone in nprobe through search_batch's nprobe (ivfpq.rs:1367-1404)
    lo = px.recall_at_k(_Nprobe(ivf, 1), l2, q, 10).mean
    hi = px.recall_at_k(_Nprobe(ivf, 32), l2, q, 10).mean
    assert lo <= hi


class _Nprobe:
    """search_with_nprobe adapter: a candidate whose search uses a fixed nprobe."""

    def __init__(self, idx, nprobe):
        self.idx, self.nprobe = idx, nprobe

    def search_batch(self, queries, k, filter=None):
        return self.idx.search_batch(queries, k, filter, nprobe=self.nprobe)


class _Rescore:
    """An Sq8Index candidate that rescores the best `rescore` asymmetrically."""

    def __init__(self, idx, rescore):
        self.idx, self.rescore = idx, rescore

    def search_batch(self, queries, k, filter=None):
        return self.idx.search_batch(queries, k, filter, rescore=self.rescore)
