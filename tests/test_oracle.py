"""Pins the oracle (oracle/oracle.cpp) before anything is checked against it.

Each test is a known-answer test or fixture carried over from the reference's
own tests (cited file:line), a closed form, or a brute-force / invariant
check chosen so that a plausible slip in the restatement (a dropped tail, a
different lane or reduce order, a wrong tie rule, a sign error, a transposed
operand) fails one of them.
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc

F32_MAX = np.float32(3.4028235e38)


# --- distance.rs:551-614 -----------------------------------------------------------
def test_known_values():  # distance.rs:551-559
    a, b = [1.0, 2.0, 3.0], [4.0, 6.0, 3.0]
    assert orc.squared_euclidean(a, b) == 25.0
    assert math.sqrt(orc.squared_euclidean(a, b)) == 5.0
    assert orc.manhattan(a, b) == 7.0
    assert orc.dot(a, b) == 25.0
    assert orc.space_distance(orc.INNER_PRODUCT, a, b) == -25.0


def test_cosine_orthogonal_parallel_opposite():  # distance.rs:562-566
    assert abs(orc.cosine([1, 0], [0, 5]) - 1.0) < 1e-6
    assert abs(orc.cosine([1, 1], [3, 3])) < 1e-6
    assert abs(orc.cosine([1, 0], [-2, 0]) - 2.0) < 1e-6


def test_cosine_zero_vector_is_one():  # distance.rs:569-574
    assert orc.cosine([0, 0], [1, 1]) == 1.0
    assert orc.cosine_scalar([0, 0], [1, 1]) == 1.0


def test_cosine_on_unit_vectors_is_inner_product():  # distance.rs:577-586
    a = orc.normalized([0.3, -1.7, 2.5, 0.01, 4.0, -3.0, 1.0, 2.0, 9.0])
    b = orc.normalized([1.0, 2.0, -0.5, 3.3, 0.0, 1.0, -1.0, 0.5, 0.25])
    assert abs(orc.cosine(a, b) - orc.space_distance(orc.COSINE, a, b)) < 1e-5


def test_tail_shorter_than_a_lane_is_not_dropped():  # distance.rs:589-603
    for dim in range(0, 3 * 8 + 5):
        a = np.array([i * 0.5 - 3.0 for i in range(dim)], np.float32)
        b = np.array([7.0 - i * 0.25 for i in range(dim)], np.float32)
        s = orc.squared_euclidean_scalar(a, b)
        u = orc.squared_euclidean(a, b)
        assert abs(s - u) <= 1e-3 * max(abs(s), 1.0), dim
        # the exact value in float64 is within float32 rounding of both
        exact = float(np.sum((a.astype(np.float64) - b.astype(np.float64)) ** 2))
        assert abs(u - exact) <= 1e-5 * max(exact, 1.0), dim


def test_nan_propagates():  # distance.rs:606-614
    a, b = [1.0, float("nan"), 3.0], [0.0, 0.0, 0.0]
    assert math.isnan(orc.squared_euclidean(a, b))
    assert math.isnan(orc.manhattan(a, b))
    assert math.isnan(orc.dot(a, b))


def test_overflow_is_order_dependent():  # metric_properties.rs:307-333 (lane-order KAT)
    a = np.zeros(33, np.float32)
    b = np.zeros(33, np.float32)
    a[14], b[14] = F32_MAX, np.float32(-0.914_645_55)
    a[17], b[17] = np.float32(-0.880_665_24), F32_MAX
    a[25], b[25] = np.float32(1e30), F32_MAX
    a[30] = F32_MAX
    assert math.isnan(orc.dot_scalar(a, b))
    assert math.isinf(orc.dot(a, b))


def test_symmetry_is_bit_exact():  # metric_properties.rs:111-117
    rng = np.random.default_rng(1)
    for dim in (1, 7, 8, 9, 96, 128, 131):
        a = rng.standard_normal(dim).astype(np.float32)
        b = rng.standard_normal(dim).astype(np.float32)
        for m in (orc.EUCLIDEAN, orc.COSINE, orc.INNER_PRODUCT, orc.MANHATTAN):
            assert orc.metric_distance(m, a, b) == orc.metric_distance(m, b, a)


def test_unrolled_agrees_with_float64_within_rounding():
    rng = np.random.default_rng(2)
    for dim in (3, 8, 96, 128, 768, 1001):
        a = rng.standard_normal(dim).astype(np.float32)
        b = rng.standard_normal(dim).astype(np.float32)
        a64, b64 = a.astype(np.float64), b.astype(np.float64)
        bound = dim * 2 ** -23
        assert abs(orc.dot(a, b) - a64 @ b64) <= bound * (np.abs(a64) @ np.abs(b64))
        assert abs(orc.squared_euclidean(a, b) - np.sum((a64 - b64) ** 2)) <= bound * np.sum((a64 - b64) ** 2)
        # a transposed/misaligned operand would not give this
        assert orc.squared_euclidean(a, a) == 0.0


# --- space.rs / normalisation ----------------------------------------------------
def test_prepare_normalises_cosine_only():  # space.rs:41-42, flat.rs:329-340
    p, bad = orc.prepare(orc.COSINE, [3.0, 0.0, 4.0])
    assert bad == -1 and abs(p[0] - 0.6) < 1e-6 and abs(p[2] - 0.8) < 1e-6
    p, bad = orc.prepare(orc.EUCLIDEAN, [3.0, 0.0, 4.0])
    assert list(p) == [3.0, 0.0, 4.0]
    _, bad = orc.prepare(orc.EUCLIDEAN, [1.0, float("inf"), 3.0])
    assert bad == 1  # space.rs:207-213
    _, bad = orc.prepare(orc.EUCLIDEAN, [1.0, 2.0, float("nan")])
    assert bad == 2


def test_normalize_zero_and_multiply_by_reciprocal():  # distance.rs:499-517 doc test
    v = orc.normalized([3.0, 4.0])
    assert abs(math.sqrt(orc.dot(v, v)) - 1.0) < 1e-6
    assert list(orc.normalized([0.0, 0.0])) == [0.0, 0.0]
    # multiply by 1/n (not divide): for n = 3, x * fl(1/3) differs from x / 3 for x = 1.5*... pick a witness
    x = np.array([0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9], np.float32)
    n = np.float32(np.sqrt(np.float32(orc.dot(x, x))))
    inv = np.float32(1.0) / n
    assert np.array_equal(orc.normalized(x), (x * inv).astype(np.float32))


# --- topk.rs:216-296 ---------------------------------------------------------------
def test_topk_keeps_best_k():
    ids, _ = orc.topk([1, 2, 3, 4, 5], [8.0, 2.0, 5.0, 1.0, 9.0], 3)
    assert list(ids) == [4, 2, 3]


def test_topk_ties_break_on_id():
    a, _ = orc.topk([7, 3, 5], [1.0, 1.0, 1.0], 2)
    b, _ = orc.topk([5, 7, 3], [1.0, 1.0, 1.0], 2)
    assert list(a) == list(b) == [3, 5]


def test_topk_nan_evicted_and_infinity_orders():
    ids, _ = orc.topk([1, 2, 3, 4], [float("nan"), float("nan"), 100.0, 100.0], 2)
    assert list(ids) == [3, 4]
    ids, _ = orc.topk([1, 2, 3], [float("inf"), 0.0, 1.0], 2)
    assert list(ids) == [2, 3]


def test_topk_k_zero_and_underfull():
    ids, _ = orc.topk([1], [0.0], 0)
    assert ids.size == 0
    ids, _ = orc.topk([1], [1.0], 10)
    assert list(ids) == [1]


def test_topk_matches_sort_on_random():
    rng = np.random.default_rng(3)
    for k in (1, 5, 17, 100):
        d = rng.integers(0, 20, 500).astype(np.float32)  # many ties
        ids = rng.permutation(500).astype(np.uint64) * 3 + 1
        got_ids, got_d = orc.topk(ids, d, k)
        order = sorted(range(500), key=lambda i: (d[i], ids[i]))[:k]
        assert list(got_ids) == [ids[i] for i in order]
        assert list(got_d) == [d[i] for i in order]


# --- flat.rs tests -------------------------------------------------------------------
def test_flat_identical_vectors_tie_break_on_id():  # flat.rs:294-308
    data = np.ones((4, 2), np.float32)
    ids, d, c = orc.flat_search(data, [9, 4, 7, 1], orc.EUCLIDEAN, [[1.0, 1.0]], 3)
    assert list(ids[0][: c[0]]) == [1, 4, 7]


def test_flat_filter_runs_during_scan():  # flat.rs:343-355
    data = np.arange(100, dtype=np.float32).reshape(100, 1)
    accept = np.array([i % 10 == 0 for i in range(100)], np.uint8)
    ids, d, c = orc.flat_search(data, np.arange(100), orc.EUCLIDEAN, [[0.0]], 5, accept=accept)
    assert list(ids[0][: c[0]]) == [0, 10, 20, 30, 40]


def test_flat_free_slots_are_skipped_and_k_larger_than_index():
    data = np.arange(6, dtype=np.float32).reshape(3, 2)
    ids, d, c = orc.flat_search(data, [0, 1, 2], orc.EUCLIDEAN, [[0.0, 0.0]], 100, live=[1, 0, 1])
    assert c[0] == 2 and list(ids[0][:2]) == [0, 2]


def test_flat_matches_float64_brute_force():
    rng = np.random.default_rng(4)
    for metric in (orc.EUCLIDEAN, orc.COSINE, orc.INNER_PRODUCT, orc.MANHATTAN):
        data = rng.standard_normal((300, 24)).astype(np.float32)
        q = rng.standard_normal((5, 24)).astype(np.float32)
        pd = orc.prepare_rows(metric, data)
        pq = orc.prepare_rows(metric, q)
        ids = np.arange(300, dtype=np.uint64)
        got, gd, c = orc.flat_search(pd, ids, metric, pq, 10)
        d64 = pd.astype(np.float64)
        for i in range(5):
            qq = pq[i].astype(np.float64)
            if metric == orc.EUCLIDEAN:
                s = np.sum((d64 - qq) ** 2, axis=1)
            elif metric == orc.COSINE:
                s = 1.0 - d64 @ qq
            elif metric == orc.INNER_PRODUCT:
                s = -(d64 @ qq)
            else:
                s = np.sum(np.abs(d64 - qq), axis=1)
            want = np.argsort(s, kind="stable")[:10]
            assert list(got[i]) == list(want)
            assert np.allclose(gd[i], s[want], rtol=1e-5, atol=1e-5)


def test_flat_threads_do_not_change_results():
    rng = np.random.default_rng(5)
    data = rng.standard_normal((500, 16)).astype(np.float32)
    q = rng.standard_normal((9, 16)).astype(np.float32)
    a = orc.flat_search(data, np.arange(500), orc.EUCLIDEAN, q, 7, threads=1)
    b = orc.flat_search(data, np.arange(500), orc.EUCLIDEAN, q, 7, threads=4)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


# --- scalar.rs tests ------------------------------------------------------------------
def _skewed():
    return np.array([[i / 255.0, 1000.0 * (i / 255.0)] for i in range(256)], np.float32)


def test_sq_half_step_bound():  # scalar.rs:366-388
    t = _skewed()
    mn, sc, inv, bad = orc.sq_train(t, per_dim=True)
    assert bad == -1
    for row in t:
        dec = orc.sq_decode(orc.sq_encode(row, mn, inv, True, 0), mn, sc, True, 0)
        for c, step in ((0, 1.0 / 255.0), (1, 1000.0 / 255.0)):
            assert abs(row[c] - dec[c]) <= step / 2 + 1e-5


def test_sq_i8_and_u8_same_lattice_and_i8_is_level_minus_128():  # scalar.rs:412-426
    t = _skewed()
    mn, sc, inv, _ = orc.sq_train(t)
    for row in t[::7]:
        cu = orc.sq_encode(row, mn, inv, True, 0)
        ci = orc.sq_encode(row, mn, inv, True, 1)
        assert np.array_equal((cu.astype(np.int32) - 128).astype(np.int8).view(np.uint8), ci)
        assert np.array_equal(orc.sq_decode(cu, mn, sc, True, 0), orc.sq_decode(ci, mn, sc, True, 1))


def test_sq_clamps_and_constant_dimension_exact():  # scalar.rs:429-451
    mn, sc, inv, _ = orc.sq_train(np.array([[0.0], [1.0]], np.float32))
    assert orc.sq_decode(orc.sq_encode([-5.0], mn, inv, True, 0), mn, sc, True, 0)[0] == 0.0
    assert orc.sq_decode(orc.sq_encode([9.0], mn, inv, True, 0), mn, sc, True, 0)[0] == 1.0
    mn, sc, inv, _ = orc.sq_train(np.array([[3.0, 0.0], [3.0, 1.0]], np.float32))
    assert orc.sq_decode(orc.sq_encode([3.0, 0.5], mn, inv, True, 0), mn, sc, True, 0)[0] == 3.0


def test_sq_round_half_away_from_zero():
    # min 0, max 255 -> scale 1, inv 1: level = round(v). 2.5 -> 3 (not banker's 2), 0.5 -> 1
    mn, sc, inv, _ = orc.sq_train(np.array([[0.0], [255.0]], np.float32))
    assert orc.sq_encode([2.5], mn, inv, True, 0)[0] == 3
    assert orc.sq_encode([0.5], mn, inv, True, 0)[0] == 1
    assert orc.sq_encode([254.5], mn, inv, True, 0)[0] == 255


def test_sq_idempotent_and_global_mode():  # properties.rs:108-114
    rng = np.random.default_rng(6)
    t = rng.uniform(-50, 50, (50, 12)).astype(np.float32)
    for per_dim in (True, False):
        mn, sc, inv, _ = orc.sq_train(t, per_dim)
        assert mn.size == (12 if per_dim else 1)
        for _ in range(20):
            p = rng.uniform(-80, 80, 12).astype(np.float32)
            once = orc.sq_encode(p, mn, inv, per_dim, 0)
            twice = orc.sq_encode(orc.sq_decode(once, mn, sc, per_dim, 0), mn, inv, per_dim, 0)
            assert np.array_equal(once, twice)


def test_sq_train_rejects_non_finite():  # scalar.rs:474-488
    _, _, _, bad = orc.sq_train(np.array([[1.0, float("nan")]], np.float32), False)
    assert bad == 1


def test_sq_asymmetric_matches_reconstruction():  # properties.rs:117-134
    rng = np.random.default_rng(7)
    t = rng.uniform(-50, 50, (50, 12)).astype(np.float32)
    mn, sc, inv, _ = orc.sq_train(t)
    for _ in range(20):
        q = rng.uniform(-80, 80, 12).astype(np.float32)
        p = rng.uniform(-80, 80, 12).astype(np.float32)
        code = orc.sq_encode(p, mn, inv, True, 0)
        rec = orc.sq_decode(code, mn, sc, True, 0)
        direct = orc.squared_euclidean(q, rec)
        assert abs(orc.sq_asym(False, q, code, mn, sc, True, 0) - direct) <= 1e-4 * max(direct, 1.0)
        ip = float(q.astype(np.float64) @ rec)
        assert abs(orc.sq_asym(True, q, code, mn, sc, True, 0) + ip) <= 1e-5 * max(abs(ip), 1.0)


def test_sq8_int_dot_search_exact():
    rng = np.random.default_rng(8)
    codes = rng.integers(-128, 128, (400, 96)).astype(np.int8)
    q = rng.integers(-128, 128, (3, 96)).astype(np.int8)
    ids, d, c = orc.sq8_search(codes, np.arange(400), q, 10)
    for i in range(3):
        s = -(codes.astype(np.int64) @ q[i].astype(np.int64))
        order = np.lexsort((np.arange(400), s))[:10]
        assert list(ids[i]) == list(order)
        assert np.array_equal(d[i], s[order].astype(np.float32))


def test_sq8_search_accept_ties_and_rescore():
    """Filter, tie-break by id on duplicate codes, and the rescore stage
    against an independent composition (numpy int64 matmul for the integer
    stage, orc.sq_asym -- pinned above -- for the f32 stage)."""
    rng = np.random.default_rng(9)
    n, dim = 300, 20
    x = rng.uniform(-1, 1, (n, dim)).astype(np.float32)
    x[50] = x[7]  # identical codes: the lower id wins the tie
    mn, sc, inv, _ = orc.sq_train(x)
    codes = orc.sq_encode(x, mn, inv, True, 1).view(np.int8)
    ids = (np.arange(n) * 3 + 1000).astype(np.uint64)
    accept = (np.arange(n) % 4 != 1).astype(np.uint8)
    qf = x[[7, 100, 201]] + np.float32(0.01)
    qc = orc.sq_encode(qf, mn, inv, True, 1).view(np.int8)
    got_i, got_d, got_c = orc.sq8_search(codes, ids, qc, 5, accept=accept, rescore=40, qf=qf, ranges=(mn, sc))
    int_i, int_d, _ = orc.sq8_search(codes, ids, qc, 5, accept=accept)
    for q in range(3):
        s = -(codes.astype(np.int64) @ qc[q].astype(np.int64))
        s = np.where(accept == 1, s, np.iinfo(np.int64).max)
        order = np.lexsort((ids, s))
        assert list(int_i[q]) == list(ids[order[:5]])
        assert np.array_equal(int_d[q], s[order[:5]].astype(np.float32))
        short = order[:40]
        rs = np.array([orc.sq_asym(True, qf[q], codes[j].view(np.uint8), mn, sc, True, 1) for j in short], np.float32)
        fin = np.lexsort((ids[short], rs))[:5]
        assert got_c[q] == 5
        assert list(got_i[q]) == list(ids[short][fin])
        assert np.array_equal(got_d[q].view(np.uint32), rs[fin].view(np.uint32))
    # the duplicated row: ids 1021 (slot 7) and 1150 (slot 50) tie; 1021 comes first
    first = list(int_i[0]).index(1021)
    assert 1150 in list(int_i[0]) and list(int_i[0]).index(1150) == first + 1


# --- product.rs tests ------------------------------------------------------------------
def _lcg_clustered(dim, count, seed):  # product.rs:635-654 fixture
    state = seed
    mask = (1 << 64) - 1

    def nxt():
        nonlocal state
        state = (state * 6_364_136_223_846_793_005 + 1) & mask
        return np.float32(np.float32(state >> 33) / np.float32(1 << 31)) - np.float32(0.5)

    centres = [[np.float32((c * 7 + d * 3) % 11) for d in range(dim)] for c in range(8)]
    out = np.zeros((count, dim), np.float32)
    for i in range(count):
        for d in range(dim):
            out[i, d] = centres[i % 8][d] + nxt() * np.float32(0.4)
    return out


def test_pq_uneven_split():  # product.rs:667-678
    w, o = orc.pq_layout(10, 4)
    assert w == [3, 3, 2, 2] and o == [0, 3, 6, 8, 10]
    w, o = orc.pq_layout(128, 16)
    assert w == [8] * 16


def test_pq_table_agrees_with_reconstruct_and_measure():  # product.rs:681-706
    t = _lcg_clustered(32, 512, 3)
    books, inertia, iters = orc.pq_train(t, 8)
    q = t[100]
    sq, dt = orc.pq_table(books, 32, 8, q)
    codes = orc.pq_encode(books, 32, 8, t[:64])
    for i in range(64):
        rec = orc.pq_decode(books, 32, 8, codes[i])
        direct = orc.squared_euclidean(q, rec)
        via = orc.pq_adc_l2(sq, codes[i])
        assert abs(via - direct) <= 1e-3 * max(direct, 1.0)
        via_ip = orc.pq_adc_ip(dt, codes[i])
        direct_ip = -orc.dot(q, rec)
        assert abs(via_ip - direct_ip) <= 1e-3 * max(abs(direct_ip), 1.0)


def test_pq_adc_sums_subspaces_in_order():
    # ADC is sum of table[s*256 + code[s]] for s ascending, starting at 0.0
    rng = np.random.default_rng(9)
    m = 16
    table = rng.standard_normal(m * 256).astype(np.float32)
    code = rng.integers(0, 256, m).astype(np.uint8)
    acc = np.float32(0.0)
    for s in range(m):
        acc = np.float32(acc + table[s * 256 + int(code[s])])
    assert orc.pq_adc_l2(table, code) == acc
    assert orc.pq_adc_ip(table, code) == -acc


def test_pq_m_equal_dim_is_exact_scalar_clustering():  # product.rs:747-762
    t = (np.arange(200, dtype=np.float32) * 0.25).reshape(200, 1)
    books, _, _ = orc.pq_train(t, 1)
    codes = orc.pq_encode(books, 1, 1, t)
    for i in range(200):
        assert abs(orc.pq_decode(books, 1, 1, codes[i])[0] - t[i, 0]) < 1e-3


def test_pq_tiny_training_set_pads_with_last_centroid():  # product.rs:765-772
    t = _lcg_clustered(8, 3, 6)
    books, _, _ = orc.pq_train(t, 2)
    b = books.reshape(-1)
    # subspace 0: 256 rows of width 4; rows 3..255 repeat row 2
    s0 = b[: 256 * 4].reshape(256, 4)
    assert all(np.array_equal(s0[r], s0[2]) for r in range(3, 256))


def test_pq_training_reproducible_and_seed_sensitive():  # product.rs:709-729
    t = _lcg_clustered(32, 512, 4)
    a = orc.pq_train(t, 8, seed=7)
    b = orc.pq_train(t, 8, seed=7)
    c = orc.pq_train(t, 8, seed=8)
    assert np.array_equal(a[0], b[0]) and a[1] == b[1] and a[2] == b[2]
    assert not np.array_equal(a[0], c[0])
    assert a[2] < 8 * 25


def test_pq_more_subspaces_less_error():  # product.rs:732-744
    t = _lcg_clustered(32, 1024, 5)
    _, coarse, _ = orc.pq_train(t, 2)
    _, fine, _ = orc.pq_train(t, 16)
    assert fine < coarse


# --- kmeans.rs tests ---------------------------------------------------------------------
def _blobs():  # kmeans.rs:259-268
    pts = []
    for cx, cy in [(0.0, 0.0), (100.0, 0.0), (0.0, 100.0)]:
        for i in range(30):
            j = np.float32(i) * np.float32(0.01)
            pts.append([np.float32(cx) + j, np.float32(cy) - j])
    return np.array(pts, np.float32)


def test_kmeans_recovers_blobs():  # kmeans.rs:271-285
    cents, inertia, iters = orc.kmeans(_blobs(), 3, 25, 0x00C0FFEE)
    found = sorted((int(round(c[0])), int(round(c[1]))) for c in cents)
    assert found == [(0, 0), (0, 100), (100, 0)]
    assert inertia < 1.4


def test_kmeans_deterministic_clamped_identical_empty():  # kmeans.rs:288-318
    a = orc.kmeans(_blobs(), 3, 25, 0x00C0FFEE)
    b = orc.kmeans(_blobs(), 3, 25, 0x00C0FFEE)
    assert np.array_equal(a[0], b[0]) and a[2] == b[2]
    c, _, _ = orc.kmeans(np.array([[1.0, 2.0], [3.0, 4.0]], np.float32), 16, 25, 1)
    assert c.shape == (2, 2)
    c, inertia, _ = orc.kmeans(np.full((16, 4), 7.0, np.float32), 8, 25, 1)
    assert inertia == 0.0 and np.all(c == 7.0)
    c, inertia, iters = orc.kmeans(np.zeros((0, 4), np.float32), 8, 25, 1)
    assert iters == 0


def test_kmeans_inertia_non_increasing():  # kmeans.rs:321-336
    prev = float("inf")
    for cap in range(1, 8):
        _, inertia, _ = orc.kmeans(_blobs(), 3, cap, 0x00C0FFEE)
        assert inertia <= prev + 1e-9
        prev = inertia


def test_lloyd_closed_form_on_1d():
    # points 0,1,2,10,11,12 with init centroids 0 and 12: one update gives the
    # means 1 and 11 exactly, then it converges (no change -> break at it=1).
    pts = np.array([[0.0], [1.0], [2.0], [10.0], [11.0], [12.0]], np.float32)
    cents, assign, inertia, iters = orc.kmeans_lloyd(pts, [[0.0], [12.0]], 25)
    assert list(cents[:, 0]) == [1.0, 11.0]
    assert list(assign) == [0, 0, 0, 1, 1, 1]
    assert iters == 2 and inertia == 4.0  # 1+0+1 + 1+0+1 from the last assignment pass


def test_lloyd_empty_cluster_takes_farthest_point():
    # centroid 2 at 1000 attracts nothing: it is re-seeded onto the point
    # farthest from its nearest centroid, using the partially updated array.
    pts = np.array([[0.0], [1.0], [9.0]], np.float32)
    cents, assign, inertia, iters = orc.kmeans_lloyd(pts, [[0.0], [1.0], [1000.0]], 1)
    # after the first pass: assign 0,1,1 ; c0 = 0, c1 = 5 (mean of 1 and 9),
    # c2 empty -> farthest from {0, 5, 1000} is 9 (distance 16)
    assert list(cents[:, 0]) == [0.0, 5.0, 9.0]


def test_lloyd_ties_go_to_lower_index():
    pts = np.array([[1.0]], np.float32)
    _, assign, _, _ = orc.kmeans_lloyd(pts, [[0.0], [2.0]], 1)
    assert assign[0] == 0


def test_kmeans_assign_matches_brute():
    rng = np.random.default_rng(10)
    p = rng.standard_normal((200, 8)).astype(np.float32)
    c = rng.standard_normal((17, 8)).astype(np.float32)
    a, d = orc.kmeans_assign(p, c)
    d64 = ((p[:, None, :].astype(np.float64) - c[None].astype(np.float64)) ** 2).sum(-1)
    assert np.array_equal(a, d64.argmin(1))
    assert np.allclose(d, d64.min(1), rtol=1e-5)


# --- RNG: ChaCha core pinned by RFC 7539 A.1 test vector #1 and #2 ------------------------
def test_chacha20_rfc_keystream():
    key = np.zeros(8, np.uint32)
    blk0 = orc.chacha_block(key, 0, 0, 20)
    assert [int(x) for x in blk0[:4]] == [0xADE0B876, 0x903DF1A0, 0xE56A5D40, 0x28BD8653]
    assert int(blk0[15]) == 0x8665EEB2
    blk1 = orc.chacha_block(key, 1, 0, 20)
    assert [int(x) for x in blk1[:2]] == [0xBEE7079F, 0x7A385155]


def test_rng_stream_is_the_block_sequence():
    r = orc.Rng(42, rounds=8)
    key = r.key()
    words = [r.next_u32() for _ in range(80)]
    expect = np.concatenate([orc.chacha_block(key, c, 0, 8) for c in range(5)])
    assert words == [int(x) for x in expect]
    r2 = orc.Rng(42, rounds=8)
    lo_hi = [r2.next_u64() for _ in range(3)]
    assert lo_hi[0] == (int(expect[1]) << 32) | int(expect[0])


def test_rng_samplers_ranges():
    r = orc.Rng(7)
    for n in (1, 2, 3, 1000, 2_000_000):
        for _ in range(50):
            assert 0 <= r.gen_range_usize(n) < n
    for _ in range(200):
        x = r.gen_range_f64(0.0, 3.5)
        assert 0.0 <= x < 3.5
        f = r.gen_f32()
        assert 0.0 <= f < 1.0 and float(np.float32(f) * 16777216.0).is_integer()


# --- fixture.rs tests ---------------------------------------------------------------------
def test_fixture_same_seed_same_bytes_shape_finite():  # fixture.rs:132-165
    a = orc.fixture_generate(200, 8, 4, 10, 7)
    b = orc.fixture_generate(200, 8, 4, 10, 7)
    c = orc.fixture_generate(200, 8, 4, 10, 8)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    assert not np.array_equal(a[0], c[0])
    v, q = orc.fixture_generate(2000, 32, 16, 50, 3)
    assert np.all(np.isfinite(v)) and np.all(np.isfinite(q))


def test_fixture_query_nearer_to_source():  # fixture.rs:168-180
    v, q = orc.fixture_generate(1000, 32, 20, 20, 5)
    for i in range(20):
        src = (i * 50) % 1000
        if src == 0:
            continue
        assert orc.squared_euclidean(q[i], v[src]) < orc.squared_euclidean(q[i], v[0])


def test_fixture_gaussian_moments():
    v, _ = orc.fixture_generate(4000, 16, 1, 0, 11)
    noise = v - v.mean(axis=0)
    assert abs(noise.std() - 1.0) < 0.05
