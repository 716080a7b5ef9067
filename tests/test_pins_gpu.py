"""The oracle's order- and NaN-level pins (tests/test_oracle_pins.py) run
through the GPU paths: the same inputs, whose answers follow from IEEE
arithmetic and the reference's operation order, give the same bits on the
device as in the oracle and as the closed forms.

- V = [4096, 1, 1, 1, 0...]: |V|^2 is 2^24 + 2 under the unrolled kernel's
  pairwise reduce (distance.rs:534-538) and 2^24 under a sequential sum
  (k-means `squared`, kmeans.rs:234-241; the PQ table, product.rs:416-433).
- Overflowing magnitudes: an L2 distance of +inf; an inner product whose
  overflow cancels is the default NaN with its sign clear on the reference's
  aarch64 platform, so inner_product (-dot) ranks it first and cosine
  (1 - dot) last under total_cmp (topk.rs:63-67). The MFMA paths' error bound
  is infinite there, so those queries must take the exact path.
"""
import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F32_MAX = np.float32(3.4028235e38)
TWO24 = 16777216.0
V = np.array([4096, 1, 1, 1, 0, 0, 0, 0], np.float32)
B = np.array([0, -0.25, 1, 1, 0, 0, 0, 0], np.float32)  # |V - B|^2 = 2^24 + 2 in either order
A = np.zeros(8, np.float32)


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


def flat(px, data, ids, metric, mode):
    idx = px.FlatIndex(px.VectorSpace(data.shape[1], metric), data.shape[0])
    idx.insert_batch(ids, data)
    idx.set_search_mode(mode)
    return idx


def oracle_flat(data, ids, metric, q, k):
    return orc.flat_search(orc.prepare_rows(metric, data), ids, metric, orc.prepare_rows(metric, q), k, threads=8)


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("dim", [8, 16, 10, 768])
def test_flat_pairwise_reduce(gpu, mode, dim):
    px = gpu
    rng = np.random.default_rng(dim)
    n = 4000
    data = rng.standard_normal((n, dim)).astype(np.float32)
    data[:, 0] -= 100  # every other vector is farther from the queries than A and B
    data[7] = 0  # A: 2^24 + 2 under the reference's tree
    data[3] = 0
    data[3, :8] = B  # B: 2^24 + 2 in any order
    ids = np.arange(n, dtype=np.uint64)[::-1].copy()  # A carries the lower id
    q = np.zeros((3, dim), np.float32)
    q[0, :8] = V
    q[1, 0], q[1, 9 % dim], q[1, 10 % dim], q[1, 11 % dim] = 4096, 1, 1, 1  # lanes 1..3 of chunk 2 (dim 16)
    q[2] = rng.standard_normal(dim).astype(np.float32) * 50
    idx = flat(px, data, ids, px.Metric.EUCLIDEAN, mode)
    got = idx.search_batch(q, 10)
    assert_same(got, oracle_flat(data, ids, px.Metric.EUCLIDEAN, q, 10))
    gi, gd, _ = got
    # the tie at 2^24 + 2 goes to the lower id (A), then B
    assert list(gi[0, :2]) == [ids[7], ids[3]] and list(gd[0, :2]) == [TWO24 + 2] * 2
    if dim == 16:
        assert gd[1, 0] == TWO24 + 2
    for metric in (px.Metric.INNER_PRODUCT, px.Metric.MANHATTAN):
        idx = flat(px, data, ids, metric, mode)
        assert_same(idx.search_batch(q, 10), oracle_flat(data, ids, metric, q, 10))


@pytest.mark.parametrize("mode", [1, 2])
def test_flat_overflow_and_nan_scores(gpu, mode):
    px = gpu
    rng = np.random.default_rng(5)
    n, dim = 3000, 64
    data = rng.standard_normal((n, dim)).astype(np.float32)
    data[11] = F32_MAX  # lanes 0-3 overflow to +inf, lanes 4-7 to -inf: NaN
    data[12, :8] = F32_MAX  # L2 to a negative query: +inf
    data[13] = -F32_MAX / 2
    ids = np.arange(n, dtype=np.uint64)
    q = np.where(np.arange(dim) % 8 < 4, 1.0, -1.0).astype(np.float32)[None, :].repeat(4, 0)
    q[1] = -F32_MAX / 4
    q[2] = rng.standard_normal(dim).astype(np.float32)
    q[3, :] = 0
    for metric in (px.Metric.EUCLIDEAN, px.Metric.INNER_PRODUCT, px.Metric.COSINE, px.Metric.MANHATTAN):
        idx = flat(px, data, ids, metric, mode)
        for k in (5, 40):
            assert_same(idx.search_batch(q, k), oracle_flat(data, ids, metric, q, k))
    # inner product: the NaN score (-NaN) ranks first
    gi, gd, _ = flat(px, data, ids, px.Metric.INNER_PRODUCT, mode).search_batch(q[:1], 3)
    assert gi[0, 0] == 11 and bits(gd[0, :1])[0] == 0xFFC00000


def test_kmeans_sequential_squared(gpu):
    px = gpu
    a, d = px.kmeans_assign(V.reshape(1, 8), np.stack([B, A]))
    assert int(a[0]) == 1 and float(d[0]) == TWO24
    # the same point among many, with enough centroids for the matrix-core pass
    rng = np.random.default_rng(2)
    pts = (rng.standard_normal((20000, 8)) * 300).astype(np.float32)
    pts[123] = V
    cents = (rng.standard_normal((300, 8)) * 300 + 5000).astype(np.float32)
    cents[40], cents[41] = B, A
    a, d = px.kmeans_assign(pts, cents)
    wa, wd = orc.kmeans_assign(pts, cents)
    assert np.array_equal(a, wa) and np.array_equal(bits(d), bits(wd))
    assert int(a[123]) == 41 and float(d[123]) == TWO24
    c, asg, inertia, iters = px.kmeans_lloyd(pts, cents, 3)
    wc, wasg, winertia, witers = orc.kmeans_lloyd(pts, cents, 3)
    assert np.array_equal(bits(c), bits(wc)) and np.array_equal(asg, wasg)
    assert inertia == winertia and iters == witers


def _books(rows, dim=8):
    books = np.full((256, dim), 1e6, np.float32)
    books[: len(rows)] = rows
    return books


def test_pq_encode_sequential(gpu):
    px = gpu
    books = _books([B, A])
    pq = px.ProductQuantizer(8, 1, books.reshape(-1))
    assert int(pq.encode(V.reshape(1, 8))[0, 0]) == 1
    assert np.array_equal(pq.encode(V.reshape(1, 8)), orc.pq_encode(books.reshape(-1), 8, 1, V.reshape(1, 8)))


@pytest.mark.parametrize("dim,m", [(8, 1), (128, 16)])
def test_ivf_unrolled_coarse_and_sequential_tables(gpu, dim, m):
    """Coarse scoring and nearest_centroid use the unrolled kernel (both lists
    at 2^24 + 2: list 0 wins the tie); the L2 table is a sequential sum (an
    entry of list 1 with code 0 scores exactly 2^24)."""
    px = gpu
    rng = np.random.default_rng(dim)
    n = 600
    cents = np.zeros((2, dim), np.float32)
    cents[0, :8] = B
    w = dim // m
    books = np.zeros((256 * dim,), np.float32)
    off = 0
    for s in range(m):
        b = (rng.standard_normal((256, w)) * 0.01 + 3000).astype(np.float32)
        b[0] = 0
        books[off: off + 256 * w] = b.reshape(-1)
        off += 256 * w
    data = (rng.standard_normal((n, dim)) * 0.1).astype(np.float32)
    data[:8] += V[None, :] if dim == 8 else 0
    data[5, :] = 0
    data[5, :8] = V  # equidistant from both centroids: list 0
    ids = np.arange(n, dtype=np.uint64)
    codes, list_of = orc.ivf_encode(data, cents, books, m)
    assert int(list_of[5]) == 0
    codes[::3] = 0
    list_of[::2] = 1 - list_of[::2]  # populate both lists
    cfg = px.IvfPqConfig(2, m).with_train_threshold(1 << 62)
    idx = px.IvfPqIndex(px.VectorSpace(dim, px.Metric.EUCLIDEAN), cfg)
    idx.insert_batch(ids, data)
    idx.load_trained(cents, books, codes, list_of)
    q = np.zeros((4, dim), np.float32)
    q[0, :8] = V
    q[1, :8] = V + B  # residual to list 0 is V: its code-0 entries score 2^24
    q[2] = data[17]
    q[3] = rng.standard_normal(dim).astype(np.float32) * 2
    for nprobe in (1, 2):
        for k in (1, 10, 100):
            got = idx.search_batch(q, k, nprobe=nprobe)
            want = orc.ivf_search(0, cents, books, codes, list_of, ids, q, k, nprobe, m, threads=8)
            assert_same(got, want)
    gi, gd, gc = idx.search_batch(q[:1], 1, nprobe=2)
    # list 1's residual is V itself: 2^24 for a code-0 entry (2^24 + 2 pairwise)
    assert float(gd[0, 0]) == TWO24
    # the GPU encode picks list 0 for the equidistant vector, as the oracle
    idx2 = px.IvfPqIndex(px.VectorSpace(dim, px.Metric.EUCLIDEAN), cfg)
    idx2.insert_batch(ids, data)
    idx2.load_trained(cents, books)  # codes encoded on the GPU
    gcodes, glist = idx2.parts()[2:]
    wcodes, wlist = orc.ivf_encode(data, cents, books, m)
    assert np.array_equal(glist, wlist) and np.array_equal(gcodes, wcodes) and int(glist[5]) == 0


@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("rerank", [0, 30])
def test_ivf_overflowing_centroids_and_vectors(gpu, metric, rerank):
    """A list whose centroid overflows the distances: L2 scores of +inf (ties
    broken by id); cosine scores of NaN when q.c cancels an overflow (+NaN,
    last); rerank against stored vectors that cannot be normalised."""
    px = gpu
    rng = np.random.default_rng(7 + metric)
    n, dim, nlist, m = 2000, 16, 8, 2
    data = rng.standard_normal((n, dim)).astype(np.float32)
    data[::50] = F32_MAX / 2
    data[1::50, : dim // 2] = -F32_MAX
    prep = orc.prepare_rows(metric, data)
    cents = rng.standard_normal((nlist, dim)).astype(np.float32)
    cents[3] = F32_MAX
    books = rng.standard_normal(256 * dim).astype(np.float32)
    codes, list_of = orc.ivf_encode(prep, cents, books, m)
    list_of[::4] = 3
    cfg = px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62).with_rerank(rerank)
    idx = px.IvfPqIndex(px.VectorSpace(dim, metric), cfg)
    idx.insert_batch(np.arange(n, dtype=np.uint64), data)
    idx.load_trained(cents, books, codes, list_of)
    q = rng.standard_normal((6, dim)).astype(np.float32)
    q[0, dim // 2:] = -q[0, dim // 2:] - 1
    q[1] = -F32_MAX / 3
    qp = orc.prepare_rows(metric, q)
    for k in (5, 60):
        got = idx.search_batch(q, k, nprobe=nlist)
        want = orc.ivf_search(metric, cents, books, codes, list_of, np.arange(n), qp, k, nlist, m,
                              vectors=prep if rerank else None, rerank=rerank, threads=8)
        assert_same(got, want)


@pytest.mark.parametrize("mode", [1, 2])
def test_sq8_rescoring_with_an_overflowing_query(gpu, mode):
    px = gpu
    rng = np.random.default_rng(9)
    n, dim = 5000, 32
    x = rng.uniform(-1, 1, (n, dim)).astype(np.float32)
    idx = px.Sq8Index(px.VectorSpace(dim, px.Metric.INNER_PRODUCT), capacity=n)
    idx.train(x[:2000])
    idx.insert_batch(np.arange(n, dtype=np.uint64), x)
    idx.set_search_mode(mode)
    mn, sc, inv, _ = orc.sq_train(x[:2000], True)
    codes = orc.sq_encode(x, mn, inv, True, 1).view(np.int8)
    q = rng.uniform(-1, 1, (3, dim)).astype(np.float32)
    q[0] = F32_MAX
    q[0, ::2] = -F32_MAX
    q[1] = F32_MAX / 7
    qc = orc.sq_encode(q, mn, inv, True, 1).view(np.int8)
    for rescore in (0, 40):
        want = orc.sq8_search(codes, np.arange(n), qc, 10, threads=8, rescore=rescore, qf=q, ranges=(mn, sc),
                              per_dim=True)
        assert_same(idx.search_batch(q, 10, rescore=rescore), want)
