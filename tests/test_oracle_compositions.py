"""Composition pins of the oracle (oracle/oracle.cpp).

test_oracle_pins.py fixes the oracle's primitives (lane orders, sequential
sums, the NaN rule, the ChaCha8 stream and the rand 0.8 samplers). The tests
here fix how the oracle puts those primitives together, by composing the
expected result again in Python from the pinned primitives alone and comparing
it with the oracle's own composition:

- the k-means++ pick: the first index whose f64 cumulative sum reaches the
  target (kmeans.rs:161-181), and the whole seeding (kmeans.rs:146-194) from
  the raw generator;
- one generator advanced across PQ subspaces, padding by the last centroid,
  inertia and iteration totals (product.rs:244-283);
- IVF training: the div_ceil stride sample of live slots, coarse k-means and
  PQ each on a fresh generator from the same seed, residuals of the sample
  against the unrolled nearest centroid (ivfpq.rs:757-800);
- IVF search: coarse order (total_cmp, then list), the nprobe clamp
  (ivfpq.rs:993), the shortlist max(rerank, k), per-list residual tables (L2)
  or one shared table plus 1 - q.c (cosine), the ADC sum in subspace order,
  and exact rerank (ivfpq.rs:998-1110);
- the fixture generator's draw order and Box-Muller step (fixture.rs:71-123).

Each data set is chosen so that a plausible slip changes the answer, and each
test checks that power on its own data: the slip, composed in Python, gives a
different answer than the reference's rule. test_planted_mistakes_are_caught
(test_oracle_pins.py) plants those slips in copies of oracle.cpp and checks
that these tests fail on each.
"""
import numpy as np

from oracle import oracle as orc

F32 = np.float32
MIN_POSITIVE = F32(1.17549435e-38)
TAU = F32(6.2831855)  # std::f32::consts::TAU


def seq_sq(points, c):
    """kmeans.rs:234-241 `squared`, vectorised over points: a sequential f32
    sum of (p - c)^2 in dimension order (numpy float32 ufuncs round each
    operation; no fused multiply-add)."""
    acc = np.zeros(points.shape[0], F32)
    for j in range(points.shape[1]):
        d = points[:, j] - c[j]
        acc = acc + d * d
    return acc


def total_key(x):
    """f32::total_cmp as an unsigned key (topk.rs:63-67)."""
    b = int(F32(x).view(np.uint32))
    return (~b) & 0xFFFFFFFF if b >> 31 else b | 0x80000000


# --- k-means++ (kmeans.rs:146-194) --------------------------------------------------------
def test_pp_pick_first_index_reaching_target():
    # cumulative [1, 3, 6]: a target on a boundary picks that index (>=)
    ns = np.array([1, 2, 3], F32)
    assert orc.kmeans_pp_pick(ns, 3.0) == 1
    assert orc.kmeans_pp_pick(ns, 1.0) == 0
    assert orc.kmeans_pp_pick(ns, np.nextafter(3.0, 4.0)) == 2
    assert orc.kmeans_pp_pick(ns, 0.25) == 0
    # zeros (chosen centres) before the target are skipped; at a boundary the
    # first index to reach it wins, not a later zero-distance point
    assert orc.kmeans_pp_pick(np.array([0, 0, 2, 0, 0, 5], F32), 2.0) == 2
    assert orc.kmeans_pp_pick(np.array([0, 0, 2, 0, 0, 5], F32), 2.5) == 5


def test_pp_pick_accumulates_in_f64():
    # an f32 running sum stalls at 2^24 (2^24 + 1 rounds back to it) and would
    # fall through to the default n - 1; the f64 sum reaches 2^24 + 1.5 at 2
    ns = np.array([2.0 ** 24, 1, 1, 1, 0], F32)
    assert orc.kmeans_pp_pick(ns, 2.0 ** 24 + 1.5) == 2
    assert orc.kmeans_pp_pick(ns, 2.0 ** 24 + 2.5) == 3
    # a target past every cumulative sum falls back to n - 1
    assert orc.kmeans_pp_pick(np.array([1, 1, 0], F32), 5.0) == 2


def pp_py(points, k, rng, cum_dtype=np.float64):
    """kmeans_plus_plus restated from kmeans.rs:146-194 over the pinned
    generator: returns the picked point indices."""
    n = points.shape[0]
    first = rng.gen_range_usize(n)
    picks = [first]
    ns = seq_sq(points, points[first])
    for _ in range(1, k):
        total = np.cumsum(ns.astype(np.float64))[-1]  # sequential f64 sum
        if total <= 0.0:
            p = rng.gen_range_usize(n)
        else:
            target = rng.gen_range_f64(0.0, float(total))
            cum = np.cumsum(ns.astype(cum_dtype))
            hit = np.nonzero(cum >= target)[0]
            p = int(hit[0]) if hit.size else n - 1
        picks.append(p)
        d = seq_sq(points, points[p])
        ns = np.where(d < ns, d, ns)  # strict <
    return picks


def _rows_to_indices(points, rows):
    return [int(np.nonzero((points == r).all(axis=1))[0][0]) for r in rows]


def _pp_stall_data():
    # point 0 lies 2^11 away from 4096 points in the unit square: its nearest-
    # squared distance is ~2^22, whose f32 ulp (0.5) swallows the tail's
    # distances (all < 2), so an f32 cumulative sum drifts from the f64 one
    # across the tail
    rs = np.random.default_rng(11)
    pts = rs.random((4097, 2)).astype(F32)
    pts[0] = (2048.0, 0.0)
    return pts


# a seed whose first round lands in the tail (found by a search over seeds;
# test_kmeans_pp_composition checks that it still does)
PP_SEED = 299


def test_kmeans_pp_composition():
    pts = _pp_stall_data()
    k = 6
    want = pp_py(pts, k, orc.Rng(PP_SEED))
    got = _rows_to_indices(pts, orc.kmeans_pp(pts, k, PP_SEED))
    assert got == want
    # power: an f32 cumulative sum picks differently on this seed
    assert pp_py(pts, k, orc.Rng(PP_SEED), cum_dtype=np.float32) != want


def test_kmeans_pp_composition_random_and_duplicates():
    rs = np.random.default_rng(5)
    pts = (rs.standard_normal((700, 5)) * rs.uniform(0.1, 30.0, (700, 1))).astype(F32)
    for seed in (1, 77, 0x9E3779B9):
        assert _rows_to_indices(pts, orc.kmeans_pp(pts, 16, seed)) == pp_py(pts, 16, orc.Rng(seed))
    # three distinct points, k = 7: once all three are chosen the total is 0
    # and the remaining picks are uniform gen_range(0..n) draws
    dup = np.repeat(np.array([[0, 0], [3, 0], [0, 4]], F32), [5, 4, 6], axis=0)
    rs.shuffle(dup)
    want = pp_py(dup, 7, orc.Rng(42))
    got = orc.kmeans_pp(dup, 7, 42)
    assert np.array_equal(got, dup[want])


# --- PQ training: product.rs:244-283 --------------------------------------------------------
def _pq_compose(training, m, iters, seed):
    dim = training.shape[1]
    widths, offsets = orc.pq_layout(dim, m)
    rng = orc.Rng(seed)  # one generator for every subspace
    books, inertia, total_iters = [], 0.0, 0
    for s in range(m):
        proj = np.ascontiguousarray(training[:, offsets[s]:offsets[s] + widths[s]])
        cents, inn, it = orc.kmeans_with_rng(proj, 256, iters, rng)
        pad = np.repeat(cents[-1:], 256 - cents.shape[0], axis=0)
        books.append(np.concatenate([cents, pad]).reshape(-1))
        inertia += inn
        total_iters += it
    return np.concatenate(books), inertia, total_iters


def test_pq_train_one_generator_across_subspaces():
    rs = np.random.default_rng(3)
    for n, dim, m in ((300, 10, 4), (100, 8, 2)):  # widths [3,3,2,2]; n < 256 pads
        x = rs.standard_normal((n, dim)).astype(F32)
        x[:, 3:6] = x[:, 0:3] if m == 4 else x[:, 3:6]
        books, inertia, iters = orc.pq_train(x, m, max_iter=6, seed=0x5EED)
        wb, wi, wt = _pq_compose(x, m, 6, 0x5EED)
        assert np.array_equal(books.view(np.uint32), wb.view(np.uint32))
        assert inertia == wi and iters == wt


def test_pq_twin_subspaces_get_different_codebooks():
    # subspaces 0 and 1 see identical columns; the shared generator is further
    # along for subspace 1, so its k-means++ seeding (and codebook) differs.
    # Reseeding per subspace would make them equal.
    rs = np.random.default_rng(4)
    x = rs.standard_normal((400, 8)).astype(F32)
    x[:, 4:8] = x[:, 0:4]
    books, _, _ = orc.pq_train(x, 2, max_iter=4, seed=9)
    b0, b1 = books[: 256 * 4], books[256 * 4:]
    assert not np.array_equal(b0, b1)
    # ...and each equals k-means on its columns from the advanced generator
    rng = orc.Rng(9)
    c0, _, _ = orc.kmeans_with_rng(np.ascontiguousarray(x[:, :4]), 256, 4, rng)
    c1, _, _ = orc.kmeans_with_rng(np.ascontiguousarray(x[:, 4:]), 256, 4, rng)
    assert np.array_equal(b0, c0.reshape(-1)) and np.array_equal(b1, c1.reshape(-1))


def test_pq_padding_repeats_the_last_centroid():
    rs = np.random.default_rng(8)
    x = rs.standard_normal((40, 6)).astype(F32)
    books, _, _ = orc.pq_train(x, 3, max_iter=5, seed=2)
    for s in range(3):
        b = books[s * 512:(s + 1) * 512].reshape(256, 2)
        assert len({tuple(r) for r in b[:40]}) == 40  # 40 distinct centroids
        assert (b[40:] == b[39]).all()


# --- IVF training: ivfpq.rs:757-800 ------------------------------------------------------------
def _ivf_train_compose(vectors, live, nlist, m, iters, sample_size, seed):
    live_slots = np.nonzero(live)[0]
    stride = max(-(-len(live_slots) // sample_size), 1)  # div_ceil
    sample = np.ascontiguousarray(vectors[live_slots[::stride]])
    cents, cin, cit = orc.kmeans(sample, nlist, iters, seed)  # fresh generator
    resid = np.empty_like(sample)
    for i, v in enumerate(sample):
        d = np.array([orc.squared_euclidean(v, c) for c in cents], F32)  # unrolled kernel
        resid[i] = v - cents[int(np.argmin(d))]  # first minimum: strict <
    books, rin, _ = orc.pq_train(resid, m, max_iter=iters, seed=seed)  # fresh generator, same seed
    return sample, cents, books, cin, cit, rin


def test_ivf_train_composition():
    rs = np.random.default_rng(21)
    slots, dim = 700, 8
    x = (rs.standard_normal((12, dim))[rs.integers(0, 12, slots)] * 3 + rs.standard_normal((slots, dim))).astype(F32)
    live = np.ones(slots, np.uint8)
    live[[0, 5, 99, 100, 101, 350, 512, 600, 699]] = 0  # 691 live: not a multiple of 100
    cents, books, report = orc.ivf_train(x, 16, 4, max_iter=5, training_sample=100, seed=0xC0FFEE, live=live)
    sample, wc, wb, cin, cit, rin = _ivf_train_compose(x, live, 16, 4, 5, 100, 0xC0FFEE)
    assert int(report[3]) == sample.shape[0] == 99  # stride ceil(691/100) = 7
    assert np.array_equal(cents, wc) and np.array_equal(books, wb)
    assert report[0] == cin and report[1] == cit and report[2] == rin
    # power: the floored stride (6) samples 116 rows and fits other centroids
    floor_sample = np.ascontiguousarray(x[np.nonzero(live)[0][::6]])
    assert not np.array_equal(orc.kmeans(floor_sample, 16, 5, 0xC0FFEE)[0], wc)
    # power: PQ on a generator other than a fresh one from the seed differs
    resid_books = orc.pq_train(sample - wc[0], 4, max_iter=5, seed=0xC0FFEE + 1)[0]
    assert not np.array_equal(resid_books, wb)


# --- IVF search: ivfpq.rs:981-1110 -------------------------------------------------------------
def _adc(table, m, code):
    s = F32(0)
    for j in range(m):
        s = F32(s + table[j * 256 + int(code[j])])  # subspace order
    return s


def ivf_search_py(metric, cents, books, m, codes, list_of, ids, queries, k, nprobe, vectors=None, rerank=0,
                  live=None, accept=None, coarse_desc=False):
    """search_with_nprobe + search_prepared restated from ivfpq.rs:981-1110
    over the pinned primitives. coarse_desc breaks coarse ties by descending
    list instead (a slip the tests must tell apart)."""
    slots = codes.shape[0]
    live = np.ones(slots, bool) if live is None else live.astype(bool)
    dim = queries.shape[1]
    produced = cents.shape[0]
    npb = min(max(nprobe, 1), max(produced, 1))
    slot_of = {int(ids[s]): s for s in range(slots) if live[s]}
    out = []
    for q in queries:
        if k == 0 or not live.any():
            out.append([])
            continue
        cd = [orc.squared_euclidean(q, c) for c in cents]
        order = sorted(range(produced), key=lambda lst: (total_key(cd[lst]), -lst if coarse_desc else lst))[:npb]
        shortlist = max(rerank, k) if rerank > 0 else k
        if metric == orc.COSINE:
            _, dt = orc.pq_table(books, dim, m, q)
        cands = []
        for lst in order:
            if metric == orc.COSINE:
                qdc = orc.dot(q, cents[lst])
            else:
                sq, _ = orc.pq_table(books, dim, m, (q - cents[lst]).astype(F32))
            for s in range(slots):  # a list holds its slots in ascending order
                if not live[s] or list_of[s] != lst or (accept is not None and not accept[s]):
                    continue
                if metric == orc.COSINE:
                    score = F32(F32(F32(1) - F32(qdc)) + F32(-_adc(dt, m, codes[s])))
                else:
                    score = _adc(sq, m, codes[s])
                cands.append((total_key(score), int(ids[s]), float(score)))
        cands = sorted(cands)[:shortlist]
        if rerank == 0 or vectors is None:
            out.append([(i, d) for _, i, d in cands[:k]])
            continue
        ex = sorted((total_key(orc.space_distance(metric, q, vectors[slot_of[i]])), i,
                     float(orc.space_distance(metric, q, vectors[slot_of[i]]))) for _, i, _ in cands)
        out.append([(i, d) for _, i, d in ex[:k]])
    return out


def _oracle_lists(oi, od, oc):
    return [[(int(oi[r, j]), float(od[r, j])) for j in range(int(oc[r]))] for r in range(oi.shape[0])]


def _ivf_case(metric):
    rs = np.random.default_rng(31)
    dim, m, nl, slots = 8, 4, 6, 240
    cents = rs.standard_normal((nl, dim)).astype(F32)
    cents[4] = cents[2]  # twin lists: every query ties on them
    x = (cents[rs.integers(0, nl, slots)] + 0.4 * rs.standard_normal((slots, dim))).astype(F32)
    if metric == orc.COSINE:
        x = orc.prepare_rows(orc.COSINE, x)
        cents = orc.prepare_rows(orc.COSINE, cents)
    books = rs.standard_normal(256 * dim).astype(F32) * 0.3
    codes = rs.integers(0, 256, (slots, m)).astype(np.uint8)
    list_of = rs.integers(0, nl, slots).astype(np.uint32)  # lists 2 and 4 both hold entries
    ids = (rs.permutation(slots) * 7 + 3).astype(np.uint64)
    live = np.ones(slots, np.uint8)
    live[rs.integers(0, slots, 12)] = 0
    # the first two queries sit by the twins, so the twin cut decides their results
    q = (cents[[2, 2, 0, 1, 5]] + 0.3 * rs.standard_normal((5, dim))).astype(F32)
    if metric == orc.COSINE:
        q = orc.prepare_rows(orc.COSINE, q)
    return cents, books, codes, list_of, ids, live, x, q


def _twin_cut(cents, q):
    # nprobe that keeps exactly one of the twin lists 2 and 4 for query q
    cd = [orc.squared_euclidean(q, c) for c in cents]
    order = sorted(range(len(cents)), key=lambda lst: (total_key(cd[lst]), lst))
    return order.index(2) + 1


def test_ivf_search_composition_l2():
    cents, books, codes, list_of, ids, live, x, q = _ivf_case(orc.EUCLIDEAN)
    m = 4
    differs = 0
    for r in range(q.shape[0]):
        qq = q[r:r + 1]
        cut = _twin_cut(cents, qq[0])
        for k, nprobe, rerank in ((5, cut, 0), (5, cut, 2), (3, cut, 9), (4, 0, 0), (6, 99, 0), (6, 99, 20)):
            got = orc.ivf_search(orc.EUCLIDEAN, cents, books, codes, list_of, ids, qq, k, nprobe, m,
                                 vectors=x, rerank=rerank, live=live)
            want = ivf_search_py(orc.EUCLIDEAN, cents, books, m, codes, list_of, ids, qq, k, nprobe, vectors=x,
                                 rerank=rerank, live=live)
            assert _oracle_lists(*got) == want, (r, k, nprobe, rerank)
            if rerank == 2:
                assert len(want[0]) == k  # the shortlist keeps max(rerank, k)
        # power: descending ties probe the other twin and return other ids
        want = ivf_search_py(orc.EUCLIDEAN, cents, books, m, codes, list_of, ids, qq, 5, cut, live=live)
        desc = ivf_search_py(orc.EUCLIDEAN, cents, books, m, codes, list_of, ids, qq, 5, cut, live=live,
                             coarse_desc=True)
        differs += want != desc
    assert differs >= 2


def test_ivf_search_composition_cosine_filter_and_untrained_shape():
    cents, books, codes, list_of, ids, live, x, q = _ivf_case(orc.COSINE)
    m = 4
    accept = (np.arange(codes.shape[0]) % 3 != 1).astype(np.uint8)
    for k, nprobe, rerank in ((5, 2, 0), (5, 3, 2), (7, 6, 30)):
        got = orc.ivf_search(orc.COSINE, cents, books, codes, list_of, ids, q, k, nprobe, m, vectors=x,
                             rerank=rerank, live=live, accept=accept)
        want = ivf_search_py(orc.COSINE, cents, books, m, codes, list_of, ids, q, k, nprobe, vectors=x,
                             rerank=rerank, live=live, accept=accept)
        assert _oracle_lists(*got) == want, (k, nprobe, rerank)
    # k = 0 returns nothing
    got = orc.ivf_search(orc.COSINE, cents, books, codes, list_of, ids, q, 0, 2, m, vectors=x, live=live)
    assert not got[2].any()


# --- fixture::generate: fixture.rs:71-123 ----------------------------------------------------
def fixture_py(count, dim, clusters, queries, seed):
    """Draw order and Box-Muller restated over the pinned gen::<f32>() stream;
    ln and cos in float64 (the platform libm's f32 ln/cos are not
    Rust-defined: compared with a tolerance)."""
    rng = orc.Rng(seed)

    def gaussian():
        u1 = max(F32(rng.gen_f32()), MIN_POSITIVE)
        u2 = F32(rng.gen_f32())
        a = F32(np.sqrt(np.float64(F32(F32(-2.0) * F32(np.log(np.float64(u1)))))))
        return F32(a * F32(np.cos(np.float64(F32(TAU * u2)))))

    centres = np.array([F32(gaussian() * F32(4.0)) for _ in range(clusters * dim)], F32).reshape(clusters, dim)
    noise = np.array([gaussian() for _ in range(count * dim)], F32).reshape(count, dim)
    stride = max(count // max(queries, 1), 1)
    src = (np.arange(queries) * stride) % count
    qnoise = np.array([F32(gaussian() * F32(0.25)) for _ in range(queries * dim)], F32).reshape(queries, dim)
    base = centres[np.arange(count) % clusters]
    return base, noise, src, qnoise


def test_fixture_draw_order_and_box_muller():
    for count, dim, clusters, queries, seed in ((120, 8, 5, 7, 3), (64, 3, 64, 64, 0x9E3779B9)):
        v, q = orc.fixture_generate(count, dim, clusters, queries, seed)
        base, noise, src, qnoise = fixture_py(count, dim, clusters, queries, seed)
        # every value is a sum of two rounded terms; 2e-6 of their magnitudes
        # covers a few ulps of libm difference in each
        want_v = base + noise
        assert np.all(np.abs(v - want_v) <= 2e-6 * (np.abs(base) + np.abs(noise)) + 1e-30)
        want_q = v[src] + qnoise
        assert np.all(np.abs(q - want_q) <= 2e-6 * (np.abs(v[src]) + np.abs(qnoise)) + 1e-30)
        # power: Box-Muller with the two draws swapped gives other values
        rng = orc.Rng(seed)
        u1, u2 = F32(rng.gen_f32()), F32(rng.gen_f32())
        swapped = np.sqrt(-2.0 * np.log(max(u2, MIN_POSITIVE))) * np.cos(np.float64(TAU * u1)) * 4.0
        assert abs(swapped - base[0, 0]) > 1e-3 * (1 + abs(base[0, 0]))
