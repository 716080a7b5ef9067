"""GPU k-means and product-quantizer training/encoding against the oracle.

With the same seed the GPU trainer must reproduce the oracle bit for bit:
k-means++ picks (same ChaCha8 stream continued on the device; f64 sums that
are provably exact in parallel, else sequential below 2^17 points), Lloyd assignments, f64 centroid updates, empty-cluster reseeding,
inertia and iteration counts; PQ codebooks and codes. Plus the reference's own
kmeans.rs / product.rs tests."""
import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def blobs():  # kmeans.rs:259-268
    pts = []
    for cx, cy in [(0.0, 0.0), (100.0, 0.0), (0.0, 100.0)]:
        for i in range(30):
            j = np.float32(i) * np.float32(0.01)
            pts.append([np.float32(cx) + j, np.float32(cy) - j])
    return np.array(pts, np.float32)


def clustered(rng, n, dim, clusters, sigma):
    c = rng.standard_normal((clusters, dim)).astype(np.float32) * 3
    return (c[np.arange(n) % clusters] + sigma * rng.standard_normal((n, dim))).astype(np.float32)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("n,dim,k,iters,seed", [(90, 2, 3, 25, 0x00C0FFEE), (3000, 8, 16, 25, 7),
                                                (5000, 10, 40, 15, 3), (20000, 128, 64, 8, 11), (700, 5, 256, 25, 9)])
def test_kmeans_bit_exact_vs_oracle(gpu, n, dim, k, iters, seed):
    px = gpu
    rng = np.random.default_rng(seed)
    pts = blobs() if dim == 2 else clustered(rng, n, dim, max(k // 2, 2), 0.5)
    got = px.kmeans(pts, dim, k, iters, seed)
    want_c, want_in, want_it = orc.kmeans(pts, k, iters, seed)
    assert got.iterations == want_it
    assert np.array_equal(bits(got.centroids), bits(want_c.reshape(-1)))
    assert got.inertia == want_in


# How the empty-cluster reseeds of a run are searched: the segment passes
# (inputs below four pool sizes), the candidate pool (a small pool size set
# for these inputs), or the pool with its test failed at the second empty
# cluster of an iteration (victims already placed), so that the segment passes
# redo them all. Each must give the reference's results.
RESEED_PATHS = ["segments", "pool", "pool_fallback"]


def reseed_path(monkeypatch, path, pool):
    if path != "segments":
        monkeypatch.setenv("PXG_RESEED_POOL", str(pool))
    if path == "pool_fallback":
        monkeypatch.setenv("PXG_RESEED_FAIL_AT", "1")


def check_reseed_path(px, path, several):
    st = px.kmeans_last_reseeds()
    assert st["reseeds"] > 0
    if path == "segments":
        assert st["pool"] == 0 and st["pool_fallbacks"] == 0
    elif path == "pool" or not several:
        assert st["pool"] == st["reseeds"] and st["pool_fallbacks"] == 0
    else:
        assert st["pool_fallbacks"] >= 1


@pytest.mark.parametrize("path", RESEED_PATHS)
def test_lloyd_from_init_with_empty_clusters(gpu, monkeypatch, path):
    px = gpu
    reseed_path(monkeypatch, path, 900)
    rng = np.random.default_rng(5)
    pts = clustered(rng, 4000, 16, 8, 0.3)
    init = pts[:12].copy()
    init[3] += 1000.0  # attracts nothing -> farthest-point reseed
    init[7] -= 1000.0
    got = px.kmeans_lloyd(pts, init, 20)
    check_reseed_path(px, path, True)
    want = orc.kmeans_lloyd(pts, init, 20)
    assert np.array_equal(bits(got[0]), bits(want[0]))
    assert np.array_equal(got[1], want[1])
    assert got[2] == want[2] and got[3] == want[3]


@pytest.mark.parametrize("path", RESEED_PATHS)
def test_lloyd_several_empty_clusters_in_one_iteration(gpu, monkeypatch, path):
    """Five centroids that attract nothing, spread over 512: the reseeds of
    one iteration go through the segmented farthest-point search (exact
    segment minima over old and new rows, MFMA-sized segments) or the pool
    and must pick the reference's points in order."""
    px = gpu
    reseed_path(monkeypatch, path, 2000)
    rng = np.random.default_rng(15)
    pts = clustered(rng, 9000, 32, 300, 0.4)
    init = pts[rng.choice(9000, 512, replace=False)].copy()
    for c, off in ((40, 900.0), (170, -800.0), (171, 700.0), (333, 650.0), (500, -950.0)):
        init[c] += np.float32(off)
    got = px.kmeans_lloyd(pts, init, 6)
    check_reseed_path(px, path, True)
    want = orc.kmeans_lloyd(pts, init, 6)
    assert np.array_equal(bits(got[0]), bits(want[0]))
    assert np.array_equal(got[1], want[1])
    assert got[2] == want[2] and got[3] == want[3]


@pytest.mark.parametrize("path", RESEED_PATHS)
@pytest.mark.parametrize("empties", [(7,), (7, 60)])
def test_farthest_point_ties_take_the_first_index(gpu, monkeypatch, empties, path):
    """Two distinct outliers, m - 20 e0 (index 1000) and m + 20 e0 (index
    4000), are the farthest points at exactly equal distance 400 from their
    centroid m, whose 8-point group keeps the mean m exactly: the reseed takes
    index 1000 (strict > from -1.0), through the one-empty and the segmented
    several-empty searches, and through the pool."""
    px = gpu
    reseed_path(monkeypatch, path, 1400)
    rng = np.random.default_rng(21)
    dim = 32
    pts = clustered(rng, 6000, dim, 40, 0.3)
    m = np.zeros(dim, np.float32)
    m[0] = 100.0
    group = {1000: -20.0, 4000: 20.0}
    for j, idx in enumerate(range(2000, 2006)):
        group[idx] = None
        pts[idx] = m
        pts[idx][1 + j // 2] += np.float32(1.0 if j % 2 == 0 else -1.0)
    for idx in (1000, 4000):
        pts[idx] = m
        pts[idx][0] += np.float32(group[idx])
    pool = np.setdiff1d(np.arange(6000), list(group))
    init = pts[rng.choice(pool, 80, replace=False)].copy()
    init[30] = m
    for c in empties:
        init[c] += np.float32(5000.0)  # attracts nothing
    got = px.kmeans_lloyd(pts, init, 3)
    check_reseed_path(px, path, len(empties) > 1)
    want = orc.kmeans_lloyd(pts, init, 3)
    assert np.array_equal(bits(got[0]), bits(want[0]))
    assert np.array_equal(got[1], want[1])
    assert got[2] == want[2] and got[3] == want[3]
    one = px.kmeans_lloyd(pts, init, 1)[0].reshape(80, dim)
    assert np.array_equal(bits(one[empties[0]]), bits(pts[1000]))  # the first of the tied pair


def test_kmeans_pp_picks_match(gpu):
    px = gpu
    rng = np.random.default_rng(6)
    pts = clustered(rng, 6000, 24, 20, 0.4)
    assert np.array_equal(bits(px.kmeans_pp(pts, 50, 1234)), bits(orc.kmeans_pp(pts, 50, 1234)))


def test_kmeans_pp_parallel_sums_above_2_17_points(gpu):
    """300k points on a 1/4 grid: every distance is a multiple of 1/16 and the
    totals stay far below 2^53 such units, so the parallel f64 sums are exact
    and the picks are the reference's, across more block partials (1172)
    than the pick kernel has threads."""
    px = gpu
    rng = np.random.default_rng(21)
    pts = (rng.integers(0, 16, (300_000, 4)) / 4).astype(np.float32)
    assert np.array_equal(bits(px.kmeans_pp(pts, 24, 77)), bits(orc.kmeans_pp(pts, 24, 77)))


def test_kmeans_pp_sequential_sums_when_not_provably_exact(gpu):
    """Near-duplicate points at scale 1000: distances from ~1e-5 to ~1e7, so
    an f64 sum of them rounds and only the sequential order reproduces it."""
    px = gpu
    rng = np.random.default_rng(22)
    pts = clustered(rng, 5000, 6, 10, 0.5) * np.float32(1000)
    pts[1::9] = pts[0::9][: pts[1::9].shape[0]] + np.float32(1e-3)
    assert np.array_equal(bits(px.kmeans_pp(pts, 40, 5)), bits(orc.kmeans_pp(pts, 40, 5)))


def test_kmeans_cluster_sums_with_mixed_magnitudes(gpu):
    """Coordinates of 1e-20 next to O(1) ones in the same cluster: their f64
    sums round, so those cluster means are summed in point order."""
    px = gpu
    rng = np.random.default_rng(23)
    pts = clustered(rng, 4000, 8, 6, 0.5)
    pts[::7, 0] = np.float32(1e-20)
    pts[::11, 3] = np.float32(-3e-25)
    got = px.kmeans(pts, 8, 12, 10, 31)
    want_c, want_in, want_it = orc.kmeans(pts, 12, 10, 31)
    assert got.iterations == want_it
    assert np.array_equal(bits(got.centroids), bits(want_c.reshape(-1)))
    assert got.inertia == want_in


def test_assign_matches_oracle(gpu):
    px = gpu
    rng = np.random.default_rng(8)
    for dim in (3, 8, 13, 128, 200):
        p = rng.standard_normal((3000, dim)).astype(np.float32)
        c = rng.standard_normal((77, dim)).astype(np.float32)
        c[5] = c[9]  # duplicate centroid: ties go to the lower index
        a, d = px.kmeans_assign(p, c)
        wa, wd = orc.kmeans_assign(p, c)
        assert np.array_equal(a, wa)
        assert np.array_equal(bits(d), bits(wd))


def test_assign_matrix_core_path_matches_oracle(gpu):
    """Enough points and centroids for the MFMA pass: approximate winners are
    certified against the runner-up and rescored exactly; duplicated
    centroids (exact ties, lower index wins), points equidistant from two
    centroids and rows whose norms overflow take the exact scan. Widths 8, 16
    and 24 take the narrow-row kernel (centroids in LDS, top-2 per lane)."""
    px = gpu
    rng = np.random.default_rng(9)
    for dim in (8, 16, 24, 32, 96, 128):
        p = clustered(rng, 9000, dim, 40, 0.3)
        c = p[rng.choice(9000, 300, replace=False)] + rng.standard_normal((300, dim)).astype(np.float32) * 0.05
        c[5] = c[9]
        c[17] = c[250]
        p[:40] = c[5] + np.float32(0.01)                      # nearest: the tied pair 5/9
        p[40:80] = (c[20] + c[21]) * np.float32(0.5)          # on a bisector
        p[80, :4] = np.float32(3e18)                          # |p|^2 overflows
        a, d = px.kmeans_assign(p, c)
        wa, wd = orc.kmeans_assign(p, c)
        assert np.array_equal(a, wa), dim
        assert np.array_equal(bits(d), bits(wd)), dim


@pytest.mark.parametrize("dim", [64, 8])
@pytest.mark.parametrize("case", ["centroid_nan", "centroid_inf", "centroid_norm_overflow", "points"])
def test_assign_matrix_core_nonfinite(gpu, case, dim):
    """Non-finite values on the MFMA path: a NaN or infinite centroid
    coordinate, or a centroid whose squared norm overflows, makes every
    point's bound non-finite (all take the exact scan); NaN and infinite
    point coordinates send only those points there. The assignments and
    distances are the reference's (a NaN distance never wins: strict <)."""
    px = gpu
    rng = np.random.default_rng(21)
    p = clustered(rng, 6000, dim, 30, 0.3)
    c = p[rng.choice(6000, 200, replace=False)] + rng.standard_normal((200, dim)).astype(np.float32) * 0.05
    if case == "centroid_nan":
        c[7, 3] = np.nan
    elif case == "centroid_inf":
        c[150, 0] = np.inf
    elif case == "centroid_norm_overflow":
        c[33, :2] = np.float32(2e19)
    else:
        p[10, 5] = np.nan
        p[11, 0] = np.inf
        p[12, :] = -np.inf
        p[13, dim - 1] = np.float32(-3e38)
    a, d = px.kmeans_assign(p, c)
    wa, wd = orc.kmeans_assign(p, c)
    assert np.array_equal(a, wa), case
    assert np.array_equal(bits(d), bits(wd)), case


def test_reference_kmeans_properties(gpu):  # kmeans.rs:271-336
    px = gpu
    r = px.kmeans(blobs(), 2, 3, 25, 0x00C0FFEE)
    found = sorted((int(round(x)), int(round(y))) for x, y in r.centroids.reshape(-1, 2))
    assert found == [(0, 0), (0, 100), (100, 0)] and r.inertia < 1.4
    assert px.kmeans(np.array([1, 2, 3, 4], np.float32), 2, 16, 25, 1).centroids.size == 4
    ident = px.kmeans(np.full(64, 7.0, np.float32), 4, 8, 25, 1)
    assert ident.inertia == 0.0 and np.all(ident.centroids == 7.0)
    empty = px.kmeans(np.zeros(0, np.float32), 4, 8, 25, 1)
    assert empty.iterations == 0 and empty.centroids.size == 4
    prev = float("inf")
    for cap in range(1, 8):
        r = px.kmeans(blobs(), 2, 3, cap, 0x00C0FFEE)
        assert r.inertia <= prev + 1e-9
        prev = r.inertia


def _lcg_clustered(dim, count, seed):  # product.rs:635-654
    state = seed
    mask = (1 << 64) - 1
    out = np.zeros((count, dim), np.float32)
    centres = [[np.float32((c * 7 + d * 3) % 11) for d in range(dim)] for c in range(8)]
    for i in range(count):
        for d in range(dim):
            state = (state * 6_364_136_223_846_793_005 + 1) & mask
            v = np.float32(np.float32(state >> 33) / np.float32(1 << 31)) - np.float32(0.5)
            out[i, d] = centres[i % 8][d] + v * np.float32(0.4)
    return out


# the last three train 8-, 24- and 16-wide subspaces on enough vectors for
# the narrow-row matrix-core assignment (all subspaces in each launch)
@pytest.mark.parametrize("dim,m,count,seed", [(32, 8, 512, 3), (10, 4, 300, 2), (8, 2, 3, 6), (64, 16, 400, 1),
                                              (16, 2, 6000, 4), (48, 2, 5000, 5), (32, 2, 4500, 8)])
def test_pq_train_and_encode_bit_exact(gpu, dim, m, count, seed):
    px = gpu
    t = _lcg_clustered(dim, count, seed)
    space = px.VectorSpace(dim, px.Metric.EUCLIDEAN)
    pq = px.ProductQuantizer.train(space, t, px.PqConfig(m).with_seed(7))
    books, inertia, iters = orc.pq_train(t, m, 25, 7)
    assert np.array_equal(bits(pq.codebooks), bits(books))
    assert pq.training_inertia == inertia and pq.training_iterations == iters
    assert np.array_equal(pq.encode(t), orc.pq_encode(books, dim, m, t))


@pytest.mark.parametrize("after", [0, 5])
def test_pq_train_in_order_path(gpu, monkeypatch, after):
    """The subspaces seed at once from predicted generator states; the
    in-order path that redoes the later subspaces (taken when a seeding's
    draws differ from the prediction, forced here) gives the same codebooks."""
    px = gpu
    t = _lcg_clustered(32, 512, 3)
    monkeypatch.setenv("PXG_PQ_REDO_AFTER", str(after))
    pq = px.ProductQuantizer.train(px.VectorSpace(32, px.Metric.EUCLIDEAN), t, px.PqConfig(8).with_seed(7))
    books, inertia, iters = orc.pq_train(t, 8, 25, 7)
    assert np.array_equal(bits(pq.codebooks), bits(books))
    assert pq.training_inertia == inertia and pq.training_iterations == iters


@pytest.mark.parametrize("dim,m,count,distinct", [(16, 2, 300, 40), (12, 3, 2000, 150), (16, 2, 6000, 60)])
def test_pq_train_duplicates_reseed_empty_clusters(gpu, dim, m, count, distinct):
    """Few distinct rows: k-means++ falls back to uniform picks once the total
    is zero (kmeans.rs:162-166), duplicate seeds leave clusters empty, and the
    batched trainer reseeds them per subspace with the farthest point of the
    partially updated array (kmeans.rs:119-123). With 6000 rows the
    assignment takes the matrix-core pass, whose certificate fails on the
    duplicate centroids' exact ties: those points go to the exact scan, which
    keeps the lower index."""
    px = gpu
    rng = np.random.default_rng(count)
    rows = rng.standard_normal((distinct, dim)).astype(np.float32)
    t = rows[rng.integers(0, distinct, count)]
    pq = px.ProductQuantizer.train(px.VectorSpace(dim, px.Metric.EUCLIDEAN), t, px.PqConfig(m).with_seed(11))
    books, inertia, iters = orc.pq_train(t, m, 25, 11)
    assert np.array_equal(bits(pq.codebooks), bits(books))
    assert pq.training_inertia == inertia and pq.training_iterations == iters


def test_pq_train_many_points_uneven_convergence(gpu):
    """Enough points for the wide cluster sums (n >= 64 k) and subspaces that
    stop at different iterations: one subspace's columns are a few exact
    clusters (converges early), the other's noisy."""
    px = gpu
    rng = np.random.default_rng(17)
    n, dim = 20000, 16
    t = np.empty((n, dim), np.float32)
    t[:, :8] = rng.standard_normal((300, 8)).astype(np.float32)[rng.integers(0, 300, n)]
    t[:, 8:] = rng.standard_normal((n, 8)).astype(np.float32)
    pq = px.ProductQuantizer.train(px.VectorSpace(dim, px.Metric.EUCLIDEAN), t,
                                   px.PqConfig(2).with_seed(5).with_max_iterations(12))
    books, inertia, iters = orc.pq_train(t, 2, 12, 5)
    assert np.array_equal(bits(pq.codebooks), bits(books))
    assert pq.training_inertia == inertia and pq.training_iterations == iters
    assert iters < 24  # the clustered subspace stopped early


def test_pq_validation(gpu):  # product.rs:775-809
    px = gpu
    space = px.VectorSpace(8, px.Metric.EUCLIDEAN)
    t = _lcg_clustered(8, 32, 7)
    for bad in (px.PqConfig(0), px.PqConfig(9), px.PqConfig(2).with_max_iterations(0)):
        with pytest.raises(px.Configuration):
            px.ProductQuantizer.train(space, t, bad)
    with pytest.raises(px.Configuration):
        px.ProductQuantizer.train(space, np.array([1.0, 2.0], np.float32), px.PqConfig(2))


@pytest.mark.parametrize("case", ["wide_range", "duplicates", "far_outliers"])
def test_kmeans_pp_certified_int8_rounds(gpu, case):
    """k-means++ rounds after the first skip a point only when an int8 copy
    proves its exact distance cannot drop (kmeans.rs:180-186): data where
    that copy is coarse (coordinates spanning 10 orders of magnitude), exact
    ties and zero distances (duplicate points), and outliers far from
    everything. Seeds, then full runs, equal the oracle's bit for bit."""
    px = gpu
    rng = np.random.default_rng(5)
    n, dim, k = 6000, 64, 48
    if case == "wide_range":
        pts = (rng.standard_normal((n, dim)) * 1e-3).astype(np.float32)
        pts[:, 0] += rng.integers(0, 5, n).astype(np.float32) * np.float32(1e4)
        pts[::7, 5] += np.float32(1e-30)
    elif case == "duplicates":
        base = rng.standard_normal((30, dim)).astype(np.float32)
        pts = base[rng.integers(0, 30, n)].copy()
        pts[::11, 3] += np.float32(1e-7)
    else:
        pts = rng.standard_normal((n, dim)).astype(np.float32)
        pts[::500] *= np.float32(1e5)
    got = px.kmeans_pp(pts, k, 3)
    want = orc.kmeans_pp(pts, k, 3)
    assert np.array_equal(bits(got), bits(want))
    g = px.kmeans(pts, dim, k, 4, 3)
    w = orc.kmeans(pts, k, 4, 3)
    assert np.array_equal(bits(g.centroids.reshape(-1)), bits(w[0].reshape(-1)))
    assert g.inertia == w[1] and g.iterations == w[2]
