"""GPU scalar quantizer and SQ8 index against the oracle and the reference's
scalar.rs tests.

Parity bar: ranges (min, scale, inverse scale), codes, decoded values and
asymmetric distances bit-identical to the oracle; SQ8 search ids and
distances bit-identical to the oracle's integer-score search (and its
asymmetric rescoring), through the integer-MFMA path, the exact path, the
candidate-overflow fallback, filters and removals."""
import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def skewed():  # scalar.rs:356-364
    t = np.arange(256, dtype=np.float32) / np.float32(255.0)
    return np.stack([t, np.float32(1000.0) * t], axis=1).astype(np.float32)


def assert_same(got, want):
    gi, gd, gc = got
    wi, wd, wc = want
    assert np.array_equal(gc, wc), (gc, wc)
    for q in range(gc.size):
        c = int(gc[q])
        assert np.array_equal(gi[q, :c], wi[q, :c]), (q, gi[q, :c], wi[q, :c], gd[q, :c], wd[q, :c])
        assert np.array_equal(bits(gd[q, :c]), bits(wd[q, :c])), (q, gd[q, :c], wd[q, :c])


# --- ScalarQuantizer ----------------------------------------------------------------------
@pytest.mark.parametrize("per_dim", [True, False])
@pytest.mark.parametrize("code_type", [0, 1])
def test_quantizer_bit_exact_vs_oracle(gpu, per_dim, code_type):
    px = gpu
    rng = np.random.default_rng(3)
    t = (rng.standard_normal((5000, 24)) * rng.uniform(0.1, 30, 24)).astype(np.float32)
    mode = px.RangeMode.PER_DIMENSION if per_dim else px.RangeMode.GLOBAL
    sq = px.ScalarQuantizer.train(px.VectorSpace(24, px.Metric.EUCLIDEAN), t, mode, code_type)
    mn, sc, inv, bad = orc.sq_train(t, per_dim)
    assert bad == -1
    assert np.array_equal(bits(sq.min), bits(mn)) and np.array_equal(bits(sq.scale), bits(sc))
    assert np.array_equal(bits(sq.inverse_scale), bits(inv))
    probe = (rng.standard_normal((300, 24)) * 40).astype(np.float32)  # clamps included
    codes = sq.encode_batch(probe)
    assert np.array_equal(codes, orc.sq_encode(probe, mn, inv, per_dim, code_type))
    dec = sq.decode(codes)
    assert np.array_equal(bits(dec), bits(orc.sq_decode(codes, mn, sc, per_dim, code_type)))
    q = rng.standard_normal(24).astype(np.float32)
    for ip in (0, 1):
        got = sq._asym(ip, q, codes)
        want = np.array([orc.sq_asym(ip, q, codes[i], mn, sc, per_dim, code_type) for i in range(300)], np.float32)
        assert np.array_equal(bits(got), bits(want))


def test_reference_scalar_tests(gpu):  # scalar.rs:366-519
    px = gpu
    s2 = px.VectorSpace(2, px.Metric.EUCLIDEAN)
    sq = px.ScalarQuantizer.train(s2, skewed(), px.RangeMode.PER_DIMENSION, px.CodeType.U8)
    for row in skewed():
        dec = sq.decode(sq.encode(row))
        assert abs(row[0] - dec[0]) <= (1.0 / 255.0) / 2 + 1e-5
        assert abs(row[1] - dec[1]) <= (1000.0 / 255.0) / 2 + 1e-5
    glob = px.ScalarQuantizer.train(s2, skewed(), px.RangeMode.GLOBAL, px.CodeType.U8)
    probe = np.array([0.5, 500.0], np.float32)
    ge = abs(glob.decode(glob.encode(probe))[0] - 0.5)
    pe = abs(sq.decode(sq.encode(probe))[0] - 0.5)
    assert ge > 100.0 * pe
    i8q = px.ScalarQuantizer.train(s2, skewed(), px.RangeMode.PER_DIMENSION, px.CodeType.I8)
    for row in skewed():
        assert np.array_equal(sq.decode(sq.encode(row)), i8q.decode(i8q.encode(row)))
    one = px.ScalarQuantizer.train(px.VectorSpace(1, 0), np.array([0.0, 1.0], np.float32))
    assert list(one.decode(one.encode([-5.0]))) == [0.0] and list(one.decode(one.encode([9.0]))) == [1.0]
    const = px.ScalarQuantizer.train(s2, np.array([3.0, 0.0, 3.0, 1.0], np.float32))
    assert const.decode(const.encode([3.0, 0.5]))[0] == 3.0
    query = np.array([0.3, 700.0], np.float32)
    for row in skewed():
        approx = sq.asymmetric_squared_l2(query, sq.encode(row))
        exact = orc.squared_euclidean(query, row)
        assert abs(approx - exact) <= 0.02 * max(exact, 1.0)
    s3 = px.VectorSpace(3, px.Metric.EUCLIDEAN)
    for bad in (np.zeros(0, np.float32), np.array([1.0, 2.0], np.float32)):
        with pytest.raises(px.Configuration):
            px.ScalarQuantizer.train(s3, bad, px.RangeMode.GLOBAL)
    with pytest.raises(px.NonFinite) as e:
        px.ScalarQuantizer.train(s2, np.array([1.0, np.nan], np.float32), px.RangeMode.GLOBAL)
    assert e.value.index == 1
    g2 = px.ScalarQuantizer.train(s2, np.array([0.0, 1.0], np.float32), px.RangeMode.GLOBAL)
    with pytest.raises(px.DimensionMismatch) as e:
        g2.encode([1.0])
    assert (e.value.expected, e.value.actual) == (2, 1)


# --- SQ8 index ------------------------------------------------------------------------------
def uniform(rng, n, dim):
    return rng.uniform(-1, 1, (n, dim)).astype(np.float32)


def oracle_index(x, sample, metric=2, per_dim=True):
    prep = orc.prepare_rows(metric, x)
    mn, sc, inv, _ = orc.sq_train(orc.prepare_rows(metric, sample), per_dim)
    codes = orc.sq_encode(prep, mn, inv, per_dim, 1).view(np.int8)
    return codes, (mn, sc, inv)


def oracle_search(codes, ids, q, ranges, k, metric=2, per_dim=True, accept=None, live=None, rescore=0):
    mn, sc, inv = ranges
    qp = orc.prepare_rows(metric, q)
    qc = orc.sq_encode(qp, mn, inv, per_dim, 1).view(np.int8)
    return orc.sq8_search(codes, ids, qc, k, live=live, threads=8, accept=accept, rescore=rescore, qf=qp,
                          ranges=(mn, sc), per_dim=per_dim)


@pytest.mark.parametrize("dim", [8, 37, 96, 128, 200, 256])
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_search_parity_all_paths(gpu, dim, mode):
    px = gpu
    rng = np.random.default_rng(dim)
    n, nq = 12000, 70
    x = uniform(rng, n, dim)
    idx = px.Sq8Index(px.VectorSpace(dim, px.Metric.INNER_PRODUCT), capacity=n)
    idx.train(x[:5000])
    idx.insert_batch(np.arange(n, dtype=np.uint64), x)
    idx.set_search_mode(mode)
    codes, ranges = oracle_index(x, x[:5000])
    qa = uniform(rng, 300, dim)
    q = qa[:nq]
    for k in (1, 10, 100):
        assert_same(idx.search_batch(q, k), oracle_search(codes, np.arange(n), q, ranges, k))
    if mode == 0:  # automatic mode picks a path that needs no rescans
        assert px.Sq8Index.last_fallbacks() == 0
    # other batch sizes: the MFMA scan holds 1 query tile per wave up to 256
    # queries, 2 up to 512, then the full count
    for m in (1, 17, 32, 300):
        for k in (1, 10):
            assert_same(idx.search_batch(qa[:m], k), oracle_search(codes, np.arange(n), qa[:m], ranges, k))


def test_ranges_and_codes_match_oracle(gpu):
    px = gpu
    rng = np.random.default_rng(11)
    x = uniform(rng, 3000, 40)
    for per_dim in (True, False):
        mode = px.RangeMode.PER_DIMENSION if per_dim else px.RangeMode.GLOBAL
        idx = px.Sq8Index(px.VectorSpace(40, px.Metric.INNER_PRODUCT), mode)
        idx.train(x[:1000])
        idx.insert_batch(np.arange(3000, dtype=np.uint64) * 7, x)
        codes, (mn, sc, inv) = oracle_index(x, x[:1000], per_dim=per_dim)
        qz = idx.quantizer()
        assert np.array_equal(bits(qz.min), bits(mn)) and np.array_equal(bits(qz.inverse_scale), bits(inv))
        for i in (0, 17, 2999):
            assert np.array_equal(idx.code(i * 7), codes[i])


def test_rescore_filter_removals_and_reinsert(gpu):
    px = gpu
    rng = np.random.default_rng(5)
    n, dim = 20000, 96
    x = uniform(rng, n, dim)
    ids = (np.arange(n) * 5 + 3).astype(np.uint64)
    idx = px.Sq8Index(px.VectorSpace(dim, px.Metric.INNER_PRODUCT))
    idx.train(x[:4000])
    idx.insert_batch(ids, x)
    codes, ranges = oracle_index(x, x[:4000])
    live = np.ones(n, np.uint8)
    for s in range(0, n, 7):  # remove every 7th; their slots are reused by new ids below
        idx.remove(int(ids[s]))
        live[s] = 0
    q = uniform(rng, 50, dim)
    for rescore in (0, 60):
        want = oracle_search(codes, ids, q, ranges, 10, live=live, rescore=rescore)
        assert_same(idx.search_batch(q, 10, rescore=rescore), want)
    meta_ok = {int(i) for i in ids[::3]}
    got = idx.search_batch(q, 10, filter=lambda i, m: i in meta_ok)
    accept = np.array([1 if int(i) in meta_ok else 0 for i in ids], np.uint8)
    assert_same(got, oracle_search(codes, ids, q, ranges, 10, live=live, accept=accept))
    # reinsert into freed slots (LIFO), then compare with the oracle's slot table
    new = uniform(rng, 50, dim)
    idx.insert_batch(np.arange(10 ** 9, 10 ** 9 + 50, dtype=np.uint64), new)
    sid, slive = idx.slots()
    all_codes = np.zeros((sid.size, dim), np.int8)
    for s in np.flatnonzero(slive):
        all_codes[s] = idx.code(int(sid[s]))
    assert_same(idx.search_batch(q, 10), oracle_search(all_codes, sid, q, ranges, 10, live=slive))


def test_overflowing_candidates_take_the_exact_scan(gpu):
    """5000 identical rows tie at the threshold: the candidate list overflows
    and those queries are rescanned exactly, ties broken by id."""
    px = gpu
    rng = np.random.default_rng(9)
    n, dim = 16000, 64
    x = uniform(rng, n, dim)
    x[3000:8000] = x[123]
    ids = rng.permutation(n).astype(np.uint64)
    idx = px.Sq8Index(px.VectorSpace(dim, px.Metric.INNER_PRODUCT))
    idx.train(x)
    idx.insert_batch(ids, x)
    idx.set_search_mode(1)
    codes, ranges = oracle_index(x, x)
    q = np.concatenate([x[123:124], uniform(rng, 8, dim)])
    assert_same(idx.search_batch(q, 20), oracle_search(codes, ids, q, ranges, 20))
    assert px.Sq8Index.last_fallbacks() >= 1


def test_cosine_search_codes_device_paths(gpu):
    px = gpu
    import torch
    rng = np.random.default_rng(21)
    n, dim = 9000, 96
    x = rng.standard_normal((n, dim)).astype(np.float32)
    idx = px.Sq8Index(px.VectorSpace(dim, px.Metric.COSINE))
    idx.train_device(torch.from_numpy(x[:3000]).cuda())
    idx.insert_device(np.arange(n, dtype=np.uint64), torch.from_numpy(x).cuda())
    codes, ranges = oracle_index(x, x[:3000], metric=1)
    q = rng.standard_normal((33, dim)).astype(np.float32)
    want = oracle_search(codes, np.arange(n), q, ranges, 10, metric=1)
    assert_same(idx.search_batch(q, 10), want)
    qc = orc.sq_encode(orc.prepare_rows(1, q), ranges[0], ranges[2], True, 1).view(np.int8)
    assert_same(idx.search_codes(qc, 10), want)
    out_i = torch.zeros((33, 10), dtype=torch.int64, device="cuda")
    out_d = torch.zeros((33, 10), dtype=torch.float32, device="cuda")
    out_c = torch.zeros(33, dtype=torch.int32, device="cuda")
    idx.search_device(torch.from_numpy(q).cuda(), 10, out_i, out_d, out_c)
    torch.cuda.synchronize()
    assert_same((out_i.cpu().numpy().view(np.uint64), out_d.cpu().numpy(), out_c.cpu().numpy().view(np.uint32)), want)


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("rescore", [0, 20])
def test_non_finite_query_raises_and_the_index_still_searches(gpu, mode, rescore):
    px = gpu
    rng = np.random.default_rng(11 + mode)
    n, dim = 9000, 64
    x = uniform(rng, n, dim)
    idx = px.Sq8Index(px.VectorSpace(dim, px.Metric.INNER_PRODUCT), capacity=n)
    idx.train(x[:4000])
    idx.insert_batch(np.arange(n, dtype=np.uint64), x)
    idx.set_search_mode(mode)
    q = uniform(rng, 40, dim)
    for pos, val in ((0, np.nan), (39, np.inf), (17, -np.inf)):
        bad = q.copy()
        bad[pos, 5 + pos] = val
        with pytest.raises(px.NonFinite) as e:
            idx.search_batch(bad, 10, rescore=rescore)
        assert e.value.index == 5 + pos
    codes, ranges = oracle_index(x, x[:4000])
    assert_same(idx.search_batch(q, 10, rescore=rescore),
                oracle_search(codes, np.arange(n), q, ranges, 10, rescore=rescore))


def test_sq8_errors_and_edges(gpu):
    px = gpu
    sp = px.VectorSpace(16, px.Metric.INNER_PRODUCT)
    idx = px.Sq8Index(sp)
    with pytest.raises(px.Configuration):
        idx.insert(1, np.zeros(16, np.float32))  # untrained
    rng = np.random.default_rng(2)
    x = uniform(rng, 100, 16)
    idx.train(x)
    assert idx.search(x[0], 5) == []  # empty index
    idx.insert_batch(np.arange(100, dtype=np.uint64), x)
    with pytest.raises(px.DuplicateId):
        idx.insert(5, x[0])
    bad = x[:3].copy()
    bad[2, 4] = np.inf
    with pytest.raises(px.NonFinite) as e:
        idx.insert_batch(np.arange(500, 503, dtype=np.uint64), bad)
    assert e.value.index == 4 and len(idx) == 100  # all-or-nothing
    assert idx.search(x[0], 0) == []
    # max(k, rescore) beyond the index is clamped to its live count
    assert list(idx.search_batch(x[:2], 10, rescore=2000)[2]) == [10, 10]
    with pytest.raises(px.UnknownId):
        idx.remove(777)
    assert len(idx.search(x[0], 1000)) == 100  # k above len
    st = idx.stats()
    assert st.len == 100 and st.graph_bytes == 16 * 3 * 4
