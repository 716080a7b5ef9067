"""GPU IVF-PQ against the oracle and the reference's ivfpq.rs tests.

Parity bar: with the same trained parts (centroids, codebooks, codes) the
GPU search returns the oracle's ids and ADC distances bit for bit (the coarse
stage, the distance tables and the ADC sums follow the reference's operation
order), with and without exact rerank, for L2 and cosine, with filters and
removals; and GPU training from the same seed reproduces the oracle's
centroids, codebooks, codes and list assignment."""
import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def corpus(count, dim, clusters):  # ivfpq.rs:1264-1276 (numpy f32 sin/cos)
    i = np.arange(count)[:, None].astype(np.float32)
    d = np.arange(dim)[None, :].astype(np.float32)
    cl = (np.arange(count) % clusters)[:, None].astype(np.float32)
    step = (np.arange(count) // clusters)[:, None].astype(np.float32)
    v = np.sin(cl * np.float32(1.7) + d * np.float32(0.11)) * np.float32(5.0) + \
        np.cos(step * np.float32(0.013) * (d + np.float32(1.0)))
    del i
    return v.astype(np.float32)


def build(px, data, config, metric=0):
    space = px.VectorSpace(data.shape[1], metric)
    idx = px.IvfPqIndex(space, config)
    idx.insert_batch(np.arange(data.shape[0], dtype=np.uint64), data)
    return idx


def assert_same(got, want):
    gi, gd, gc = got
    wi, wd, wc = want
    assert np.array_equal(gc, wc), (gc, wc)
    for q in range(gc.size):
        c = int(gc[q])
        assert np.array_equal(gi[q, :c], wi[q, :c]), (q, gi[q, :c], wi[q, :c], gd[q, :c], wd[q, :c])
        assert np.array_equal(gd[q, :c].view(np.uint32), wd[q, :c].view(np.uint32)), (q, gd[q, :c], wd[q, :c])


@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("rerank", [0, 50])
def test_search_parity_on_oracle_parts(gpu, metric, rerank):
    px = gpu
    n, dim, nlist, m = 3000, 32, 32, 16
    data = corpus(n, dim, 24) + np.random.default_rng(1).standard_normal((n, dim)).astype(np.float32) * 0.3
    prep = orc.prepare_rows(metric, data)
    cents, books, _ = orc.ivf_train(prep, nlist, m, max_iter=10, seed=5)
    codes, list_of = orc.ivf_encode(prep, cents, books, m)
    cfg = px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62).with_rerank(rerank).with_seed(5)
    idx = build(px, data, cfg, metric)
    idx.load_trained(cents, books, codes, list_of)
    q = data[::97] + 0.05
    qp = orc.prepare_rows(metric, q)
    for nprobe in (1, 4, 32):
        for k in (1, 10, 40):
            got = idx.search_batch(q, k, nprobe=nprobe)
            want = orc.ivf_search(metric, cents, books, codes, list_of, np.arange(n), qp, k, nprobe, m,
                                  vectors=prep if rerank else None, rerank=rerank, threads=8)
            assert_same(got, want)


def test_search_parity_with_removals_filter_and_reinsert(gpu):
    px = gpu
    n, dim, nlist, m = 2500, 16, 16, 8
    data = corpus(n, dim, 20)
    cents, books, _ = orc.ivf_train(data, nlist, m, max_iter=8, seed=3)
    codes, list_of = orc.ivf_encode(data, cents, books, m)
    idx = build(px, data, px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62))
    idx.load_trained(cents, books, codes, list_of)
    live = np.ones(n, np.uint8)
    for i in range(0, n, 7):
        idx.remove(i)
        live[i] = 0
    q = data[3::50] + 0.1
    want = orc.ivf_search(0, cents, books, codes, list_of, np.arange(n), q, 10, 6, m, live=live, threads=8)
    assert_same(idx.search_batch(q, 10, nprobe=6), want)
    acc = np.array([i % 3 == 0 for i in range(n)], np.uint8)
    want = orc.ivf_search(0, cents, books, codes, list_of, np.arange(n), q, 10, 6, m, live=live, accept=acc,
                          threads=8)
    assert_same(idx.search_batch(q, 10, lambda i, _m: i % 3 == 0, nprobe=6), want)
    # re-insert into the freed slots: encoded on the GPU exactly like encode_slot
    new = data[: n // 7 + 1] * 1.01
    new_ids = np.arange(10_000, 10_000 + new.shape[0], dtype=np.uint64)
    slots = idx.insert_batch(new_ids, new)
    data2, ids2 = data.copy(), np.arange(n, dtype=np.uint64)
    for s, i, v in zip(slots, new_ids, new):
        data2[s], ids2[s], live[s] = v, i, 1
    codes2, list_of2 = orc.ivf_encode(data2, cents, books, m, live=live)
    _, _, gc, glo = idx.parts()
    assert np.array_equal(glo[live.astype(bool)], list_of2[live.astype(bool)])
    assert np.array_equal(gc[live.astype(bool)], codes2[live.astype(bool)])
    want = orc.ivf_search(0, cents, books, codes2, list_of2, ids2, q, 10, 6, m, live=live, threads=8)
    assert_same(idx.search_batch(q, 10, nprobe=6), want)


@pytest.mark.parametrize("metric", [0, 1])
def test_gpu_training_matches_oracle(gpu, metric):
    px = gpu
    n, dim, nlist, m = 4000, 32, 24, 8
    data = corpus(n, dim, 24) + np.random.default_rng(2).standard_normal((n, dim)).astype(np.float32) * 0.2
    prep = orc.prepare_rows(metric, data)
    cfg = px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62).with_seed(11).with_max_iterations(12) \
        .with_training_sample(1500)
    idx = build(px, data, cfg, metric)
    rep = idx.train()
    cents, books, report = orc.ivf_train(prep, nlist, m, max_iter=12, training_sample=1500, seed=11)
    gcents, gbooks, gcodes, glist = idx.parts()
    assert np.array_equal(gcents.view(np.uint32), cents.view(np.uint32))
    assert np.array_equal(gbooks.view(np.uint32), books.view(np.uint32))
    codes, list_of = orc.ivf_encode(prep, cents, books, m)
    assert np.array_equal(gcodes, codes) and np.array_equal(glist, list_of)
    assert rep.sampled == int(report[3]) and rep.coarse_iterations == int(report[1])
    assert rep.coarse_inertia == report[0] and rep.residual_inertia == report[2]
    q = data[5::111]
    want = orc.ivf_search(metric, cents, books, codes, list_of, np.arange(n), orc.prepare_rows(metric, q), 10, 3, m,
                          threads=8)
    assert_same(idx.search_batch(q, 10, nprobe=3), want)


def test_gpu_training_on_matrix_cores_matches_oracle(gpu):
    """8000 sampled points into 96 lists: the Lloyd assignments and the
    encode pass go through the MFMA nearest-centroid pass and must still be
    the oracle's bit for bit."""
    px = gpu
    n, dim, nlist, m = 8000, 64, 96, 8
    data = corpus(n, dim, 90) + np.random.default_rng(12).standard_normal((n, dim)).astype(np.float32) * 0.3
    cfg = px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62).with_seed(3).with_max_iterations(8) \
        .with_training_sample(8000)
    idx = build(px, data, cfg)
    rep = idx.train()
    cents, books, report = orc.ivf_train(data, nlist, m, max_iter=8, training_sample=8000, seed=3)
    gcents, gbooks, gcodes, glist = idx.parts()
    assert np.array_equal(gcents.view(np.uint32), cents.view(np.uint32))
    assert np.array_equal(gbooks.view(np.uint32), books.view(np.uint32))
    codes, list_of = orc.ivf_encode(data, cents, books, m)
    assert np.array_equal(gcodes, codes) and np.array_equal(glist, list_of)
    assert rep.coarse_inertia == report[0] and rep.residual_inertia == report[2]


# --- ivfpq.rs:1282-1654 -------------------------------------------------------------
def test_rejects_metrics_it_cannot_serve(gpu):
    px = gpu
    for metric in (px.Metric.INNER_PRODUCT, px.Metric.MANHATTAN):
        with pytest.raises(px.Configuration) as e:
            px.IvfPqIndex(px.VectorSpace(8, metric), px.IvfPqConfig(4, 4))
        assert "metric" in str(e.value)


def test_untrained_index_is_exact(gpu):
    px = gpu
    data = corpus(200, 16, 24)
    idx = build(px, data, px.IvfPqConfig(8, 4).with_train_threshold(1 << 62))
    flat = px.FlatIndex(px.VectorSpace(16, 0))
    flat.insert_batch(np.arange(200, dtype=np.uint64), data)
    assert not idx.is_trained()
    for q in data[:10]:
        assert idx.search_all(q, 5) == flat.search_all(q, 5)


@pytest.mark.parametrize("metric", [0, 1])
def test_untrained_exact_scan_query_groups(gpu, metric):
    """An untrained index searches by the exact scan (ivfpq.rs:1008-1012), the
    flat index's kernel: 300-float rows over 131,149 rows (129 chunks of 1024,
    the last partial) take four queries per work item at 13 and 18 queries
    and one per item at 5. Ids and distances match the oracle's flat search
    bit for bit."""
    px = gpu
    rng = np.random.default_rng(1301 + metric)
    n, dim = 131_149, 300
    data = rng.standard_normal((n, dim)).astype(np.float32)
    idx = build(px, data, px.IvfPqConfig(64, 4).with_train_threshold(1 << 62), metric)
    assert not idx.is_trained()
    q = rng.standard_normal((18, dim)).astype(np.float32)
    ids = np.arange(n, dtype=np.uint64)
    pd = orc.prepare_rows(metric, data)
    for nq in (5, 13, 18):
        want = orc.flat_search(pd, ids, metric, orc.prepare_rows(metric, q[:nq]), 10, threads=16)
        assert_same(idx.search_batch(q[:nq], 10), want)


def test_training_populates_lists_and_auto_training(gpu):
    px = gpu
    idx = build(px, corpus(1000, 16, 24), px.IvfPqConfig(16, 8).with_seed(3).with_train_threshold(1 << 62))
    rep = idx.train()
    assert idx.is_trained() and rep.sampled == 1000 and rep.populated_lists > 1
    assert sum(idx.list_lengths()) == 1000 and idx.code_bytes_per_vector() == 8
    space = px.VectorSpace(8, 0)
    auto = px.IvfPqIndex(space, px.IvfPqConfig(4, 4).with_train_threshold(50))
    for i, v in enumerate(corpus(60, 8, 6)):
        auto.insert(i, v)
        assert auto.is_trained() == (i + 1 >= 50)
    assert sum(auto.list_lengths()) == 60
    batch = px.IvfPqIndex(space, px.IvfPqConfig(4, 4).with_train_threshold(50))
    batch.insert_batch(np.arange(60, dtype=np.uint64), corpus(60, 8, 6))  # splits at the threshold
    assert batch.is_trained() and sum(batch.list_lengths()) == 60
    for a, b in zip(auto.parts(), batch.parts()):
        assert np.array_equal(a, b)


def test_recall_monotone_in_nprobe_and_rerank_helps(gpu):
    px = gpu
    data = corpus(2000, 32, 24)
    idx = build(px, data, px.IvfPqConfig(32, 16).with_seed(11).with_train_threshold(1 << 62))
    idx.train()
    flat = px.FlatIndex(px.VectorSpace(32, 0))
    flat.insert_batch(np.arange(2000, dtype=np.uint64), data)
    qs = data[::40]
    truth = [set(h.id for h in flat.search_all(q, 10)) for q in qs]
    prev = 0.0
    for nprobe in (1, 4, 16, 32):
        hits = sum(len(t & set(h.id for h in idx.search_with_nprobe(q, 10, nprobe))) for q, t in zip(qs, truth))
        recall = hits / (10 * len(qs))
        assert recall + 0.02 >= prev
        prev = recall
    assert prev > 0.4
    base = px.IvfPqConfig(32, 8).with_seed(7).with_nprobe(8).with_train_threshold(1 << 62)
    plain = build(px, data, base.clone())
    plain.train()
    rr = build(px, data, base.clone().with_rerank(100))
    rr.train()

    def measure(ix):
        return sum(len(t & set(h.id for h in ix.search_all(q, 10))) for q, t in zip(qs, truth)) / (10 * len(qs))
    assert measure(rr) > measure(plain)


def test_dropping_vectors_and_retrain_refused(gpu):
    px = gpu
    idx = build(px, corpus(1000, 64, 24),
                px.IvfPqConfig(16, 8).with_seed(2).with_retain_vectors(False).with_train_threshold(1 << 62))
    idx.train()
    assert idx.vector_bytes() == 0 and idx.vector(0) is None
    assert idx.compressed_bytes() / len(idx) < 256
    assert len(idx.search_all(np.zeros(64, np.float32), 5)) == 5
    idx.insert(9999, np.ones(64, np.float32))
    assert idx.vector_bytes() == 0 and idx.contains(9999)
    with pytest.raises(px.Configuration) as e:
        idx.train()
    assert "retain_vectors" in str(e.value)


def test_remove_takes_slot_out_of_its_list(gpu):
    px = gpu
    idx = build(px, corpus(400, 16, 24), px.IvfPqConfig(8, 4).with_seed(1).with_train_threshold(1 << 62))
    idx.train()
    before = sum(idx.list_lengths())
    idx.remove(5)
    assert sum(idx.list_lengths()) == before - 1 and not idx.contains(5)
    assert all(h.id != 5 for h in idx.search_all(np.zeros(16, np.float32), 400))
    with pytest.raises(px.UnknownId):
        idx.remove(5)


def test_filters_cosine_seed_duplicates_stats(gpu):
    px = gpu
    data = corpus(800, 16, 24)
    idx = build(px, data, px.IvfPqConfig(16, 8).with_nprobe(16).with_seed(6).with_train_threshold(1 << 62))
    idx.train()
    for i in range(800):
        idx.set_metadata(i, {"even": i % 2 == 0})
    hits = idx.search(data[0], 10, lambda _i, m: m.get("even") is True)
    assert len(hits) == 10 and all(h.id % 2 == 0 for h in hits)
    # cosine within quantization error (ivfpq.rs:1574-1604)
    cdata = corpus(1000, 32, 20)
    space = px.VectorSpace(32, px.Metric.COSINE)
    cidx = px.IvfPqIndex(space, px.IvfPqConfig(8, 16).with_nprobe(8).with_seed(9).with_train_threshold(1 << 62))
    cidx.insert_batch(np.arange(1000, dtype=np.uint64), cdata)
    cidx.train()
    qp, _ = orc.prepare(orc.COSINE, cdata[3])
    for h in cidx.search_all(cdata[3], 20):
        exact = orc.space_distance(orc.COSINE, qp, cidx.vector(h.id))
        assert abs(h.distance - exact) < 0.25
    # same seed, same index
    cfg = px.IvfPqConfig(16, 8).with_seed(42).with_train_threshold(1 << 62)
    a, b = build(px, data, cfg.clone()), build(px, data, cfg.clone())
    a.train()
    b.train()
    assert a.list_lengths() == b.list_lengths()
    for q in data[::80]:
        assert a.search_all(q, 10) == b.search_all(q, 10)
    with pytest.raises(px.DuplicateId):
        a.insert(0, data[0])
    big = build(px, corpus(1000, 64, 24), px.IvfPqConfig(16, 8).with_seed(8).with_train_threshold(1 << 62))
    big.train()
    st = big.stats()
    assert st.len == 1000 and st.dim == 64 and st.deleted == 0
    assert st.graph_bytes >= 1000 * 8 and st.vector_bytes >= 1000 * 64 * 4


def test_insert_device_matches_host_insert(gpu):
    import torch
    px = gpu
    data = corpus(1500, 32, 24)
    for metric in (0, 1):
        cfg = px.IvfPqConfig(16, 8).with_seed(4).with_train_threshold(1 << 62)
        a = build(px, data, cfg.clone(), metric)
        b = px.IvfPqIndex(px.VectorSpace(32, metric), cfg.clone())
        b.insert_device(np.arange(1500, dtype=np.uint64), torch.from_numpy(data).cuda())
        a.train()
        b.train()
        for x, y in zip(a.parts(), b.parts()):
            assert np.array_equal(x, y)
        q = data[::150]
        for x, y in zip(a.search_batch(q, 10), b.search_batch(q, 10)):
            assert np.array_equal(x, y)
    bad = torch.from_numpy(data[:4].copy()).cuda()
    bad[2, 3] = float("nan")
    with pytest.raises(px.NonFinite):
        b.insert_device(np.arange(9000, 9004, dtype=np.uint64), bad)
    assert len(b) == 1500


@pytest.mark.parametrize("dim,m,k,rerank", [(20, 8, 10, 0), (32, 16, 100, 0), (32, 8, 10, 120), (24, 24, 70, 0),
                                            (32, 16, 200, 0), (64, 16, 10, 100), (128, 16, 128, 0), (64, 16, 65, 0)])
def test_search_parity_general_path(gpu, dim, m, k, rerank):
    """Shortlists above 64 (above 128 with 16 subspaces) and uneven subspace
    widths take the LDS-table scan; 16-subspace shortlists of 65 to 128 keep
    two keys per lane in the register-codebook scan."""
    px = gpu
    n, nlist = 2000, 16
    data = corpus(n, dim, 20) + np.random.default_rng(3).standard_normal((n, dim)).astype(np.float32) * 0.3
    cents, books, _ = orc.ivf_train(data, nlist, m, max_iter=6, seed=9)
    codes, list_of = orc.ivf_encode(data, cents, books, m)
    idx = build(px, data, px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62).with_rerank(rerank))
    idx.load_trained(cents, books, codes, list_of)
    q = data[::131] - 0.05
    want = orc.ivf_search(0, cents, books, codes, list_of, np.arange(n), q, k, 5, m,
                          vectors=data if rerank else None, rerank=rerank, threads=8)
    assert_same(idx.search_batch(q, k, nprobe=5), want)


@pytest.mark.parametrize("dim,nlist,nq", [(37, 700, 7), (64, 1100, 13), (8, 64, 4)])
def test_coarse_selection_many_lists(gpu, dim, nlist, nq):
    """Probe selection over many 64-list tiles split across waves, with a
    dimension tail, a partial last tile and a partial query group."""
    px = gpu
    n, m = 6000, 8 if dim != 37 else 1
    rng = np.random.default_rng(dim)
    data = corpus(n, dim, 40) + rng.standard_normal((n, dim)).astype(np.float32) * 0.5
    cents, books, _ = orc.ivf_train(data, nlist, m, max_iter=3, seed=2)
    codes, list_of = orc.ivf_encode(data, cents, books, m)
    idx = build(px, data, px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62))
    idx.load_trained(cents, books, codes, list_of)
    q = data[rng.integers(0, n, nq)] + 0.01
    for nprobe in (1, 33, 64):
        want = orc.ivf_search(0, cents, books, codes, list_of, np.arange(n), q, 10, nprobe, m, threads=8)
        assert_same(idx.search_batch(q, 10, nprobe=nprobe), want)


@pytest.mark.parametrize("dim", [16, 64, 128])
@pytest.mark.parametrize("metric", [0, 1])
def test_sixteen_subspace_scan_long_lists(gpu, dim, metric):
    """16 subspaces take the LDS-staged scan: lists of ~2500 entries (several
    64-entry chunks per wave and probe, chunks streamed across probe
    boundaries), query counts that give one probe group per query (results
    written by the scan) and several groups (merged afterwards), removals and
    a filter."""
    px = gpu
    n, nlist, m = 20000, 8, 16
    rng = np.random.default_rng(dim + metric)
    data = corpus(n, dim, 16) + rng.standard_normal((n, dim)).astype(np.float32) * 0.4
    prep = orc.prepare_rows(metric, data)
    cents, books, _ = orc.ivf_train(prep, nlist, m, max_iter=3, seed=4)
    codes, list_of = orc.ivf_encode(prep, cents, books, m)
    idx = build(px, data, px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62), metric)
    idx.load_trained(cents, books, codes, list_of)
    live = np.ones(n, np.uint8)
    for i in range(5, n, 11):
        idx.remove(i)
        live[i] = 0
    for nq in (5, 600):
        q = data[rng.integers(0, n, nq)] + np.float32(0.03)
        qp = orc.prepare_rows(metric, q)
        for nprobe, k in ((3, 10), (8, 64)):
            want = orc.ivf_search(metric, cents, books, codes, list_of, np.arange(n), qp, k, nprobe, m, live=live,
                                  threads=8)
            assert_same(idx.search_batch(q, k, nprobe=nprobe), want)
    q = data[:40] - np.float32(0.02)
    qp = orc.prepare_rows(metric, q)
    acc = np.array([i % 4 != 1 for i in range(n)], np.uint8)
    want = orc.ivf_search(metric, cents, books, codes, list_of, np.arange(n), qp, 10, 5, m, live=live, accept=acc,
                          threads=8)
    assert_same(idx.search_batch(q, 10, lambda i, _m: i % 4 != 1, nprobe=5), want)


def test_l2_one_dimension_subspaces_take_the_general_scan(gpu):
    """128 one-wide subspaces: two L2 tables would not fit in LDS, so the
    general scan serves them."""
    px = gpu
    n, dim, nlist, m = 1500, 128, 4, 128
    data = corpus(n, dim, 12) + np.random.default_rng(8).standard_normal((n, dim)).astype(np.float32) * 0.2
    cents, books, _ = orc.ivf_train(data, nlist, m, max_iter=2, seed=1)
    codes, list_of = orc.ivf_encode(data, cents, books, m)
    idx = build(px, data, px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62))
    idx.load_trained(cents, books, codes, list_of)
    q = data[::150] + np.float32(0.01)
    want = orc.ivf_search(0, cents, books, codes, list_of, np.arange(n), q, 10, 2, m, threads=8)
    assert_same(idx.search_batch(q, 10, nprobe=2), want)


@pytest.mark.parametrize("dim,metric,rerank", [(16, 0, 0), (32, 1, 0), (64, 0, 40), (128, 1, 40), (128, 0, 0),
                                               (64, 0, 100), (128, 1, 128)])
def test_large_batch_scan(gpu, dim, metric, rerank):
    """A 700-query batch over 12 lists (4200 and 8400 (query, probe) pairs,
    every list probed by hundreds of queries): ids and ADC distances match the
    oracle with rerank, a filter, removals, and a list that removals have
    emptied (probed when nprobe = nlist)."""
    px = gpu
    n, nlist, m = 20000, 12, 16
    rng = np.random.default_rng(100 + dim + metric)
    data = corpus(n, dim, 16) + rng.standard_normal((n, dim)).astype(np.float32) * 0.4
    prep = orc.prepare_rows(metric, data)
    cents, books, _ = orc.ivf_train(prep, nlist, m, max_iter=3, seed=4)
    codes, list_of = orc.ivf_encode(prep, cents, books, m)
    cfg = px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62).with_rerank(rerank)
    idx = build(px, data, cfg, metric)
    idx.load_trained(cents, books, codes, list_of)
    live = np.ones(n, np.uint8)
    emptied = int(np.argmin(np.bincount(list_of, minlength=nlist)))
    for i in list(np.flatnonzero(list_of == emptied)) + list(range(7, n, 13)):
        if live[i]:
            idx.remove(int(i))
            live[i] = 0
    q = data[rng.integers(0, n, 700)] + np.float32(0.03)
    qp = orc.prepare_rows(metric, q)
    vec = prep if rerank else None
    for nprobe, k in ((6, 10), (12, 33)):  # 4200 and 8400 pairs over 12 lists
        want = orc.ivf_search(metric, cents, books, codes, list_of, np.arange(n), qp, k, nprobe, m, live=live,
                              vectors=vec, rerank=rerank, threads=8)
        assert_same(idx.search_batch(q, k, nprobe=nprobe), want)
    acc = np.array([i % 5 != 2 for i in range(n)], np.uint8)
    want = orc.ivf_search(metric, cents, books, codes, list_of, np.arange(n), qp, 10, 7, m, live=live, accept=acc,
                          vectors=vec, rerank=rerank, threads=8)
    assert_same(idx.search_batch(q, 10, lambda i, _m: i % 5 != 2, nprobe=7), want)


@pytest.mark.parametrize("nlist,nprobe", [(2048, 64), (2048, 32), (100, 64), (40, 33)])
def test_coarse_selection_ties_and_group_bounds(gpu, nlist, nprobe):
    """Coarse centroids of entries +-1 all lie at squared distance exactly 16
    from the zero query, so its probes are the lowest list ids (the (distance,
    list) order). The selection's candidates (keys up to the nprobe-th
    smallest of 64 group minima) then number 2017 at nlist 2048, nprobe 64
    (over the 1024 the sort holds: the radix-select fallback) and 993 at
    nprobe 32; a query at 0.5 e0 splits the lists into two tied halves; with
    fewer than 64 lists per 64 groups some groups are empty."""
    px = gpu
    dim, m, n = 16, 16, 6000
    rng = np.random.default_rng(nlist + nprobe)
    signs = rng.choice(1 << dim, nlist, replace=False)
    cents = (((signs[:, None] >> np.arange(dim)) & 1) * 2 - 1).astype(np.float32)
    data = cents[rng.integers(0, nlist, n)] + rng.standard_normal((n, dim)).astype(np.float32) * np.float32(0.2)
    _, books, _ = orc.ivf_train(data, 16, m, max_iter=3, seed=2)
    codes, list_of = orc.ivf_encode(data, cents, books, m)
    idx = build(px, data, px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62))
    idx.load_trained(cents, books, codes, list_of)
    q = np.zeros((3, dim), np.float32)
    q[1, 0] = 0.5
    q[2] = data[5]
    want = orc.ivf_search(0, cents, books, codes, list_of, np.arange(n), orc.prepare_rows(0, q), 10, nprobe, m,
                          threads=8)
    assert_same(idx.search_batch(q, 10, nprobe=nprobe), want)


def test_scan_of_a_list_over_65536_entries(gpu):
    """One list of 70000 entries beside five short ones, all probed by 800
    queries: results match the oracle."""
    px = gpu
    dim, m, nlist = 16, 16, 6
    rng = np.random.default_rng(8)
    centres = rng.standard_normal((nlist, dim)).astype(np.float32) * np.float32(8)
    sizes = (70000, 800, 700, 600, 500, 400)
    data = np.concatenate([centres[i] + np.float32(0.3) * rng.standard_normal((s, dim)).astype(np.float32)
                           for i, s in enumerate(sizes)])
    n = data.shape[0]
    cents, books, _ = orc.ivf_train(data, nlist, m, max_iter=3, training_sample=8000, seed=1)
    codes, list_of = orc.ivf_encode(data, cents, books, m)
    assert np.bincount(list_of, minlength=nlist).max() > 65536
    idx = build(px, data, px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62))
    idx.load_trained(cents, books, codes, list_of)
    q = data[rng.integers(0, n, 800)] + np.float32(0.01)
    want = orc.ivf_search(0, cents, books, codes, list_of, np.arange(n), q, 10, nlist, m, threads=8)
    assert_same(idx.search_batch(q, 10, nprobe=nlist), want)


def test_training_rejects_non_finite_residuals(gpu):
    """ProductQuantizer::train validates every residual (product.rs:221-223):
    x - c overflows here although every vector is finite, and both the oracle
    and the GPU report NonFinite for the first such residual component."""
    px = gpu
    data = np.zeros((10, 4), np.float32)
    data[0, 0] = 3e38
    data[1:, 0] = -3e38
    data[1:, 1:] = np.arange(1, 4, dtype=np.float32)
    with pytest.raises(ValueError) as e:
        orc.ivf_train(data, 1, 2, max_iter=3, seed=1)
    comp, row = e.value.args[1], e.value.args[2]
    assert (comp, row) == (0, 0) and e.value.args[3] == float("inf")
    cfg = px.IvfPqConfig(1, 2).with_train_threshold(1 << 62).with_max_iterations(3).with_seed(1)
    idx = px.IvfPqIndex(px.VectorSpace(4, px.Metric.EUCLIDEAN), cfg)
    idx.insert_batch(np.arange(10, dtype=np.uint64), data)
    with pytest.raises(px.NonFinite) as g:
        idx.train()
    assert g.value.index == comp and g.value.value == float("inf")
    assert not idx.is_trained()


def test_corrupt_load_changes_nothing(gpu):
    """from_parts builds nothing when it fails (ivfpq.rs:624-717): a load with
    a list assignment beyond the centroids, or codes without assignments,
    leaves the index as it was, and it still searches the same."""
    px = gpu
    rng = np.random.default_rng(3)
    n, dim, nlist, m = 800, 16, 8, 4
    data = rng.standard_normal((n, dim)).astype(np.float32)
    cents, books, _ = orc.ivf_train(data, nlist, m, max_iter=4, seed=2)
    codes, list_of = orc.ivf_encode(data, cents, books, m)
    idx = build(px, data, px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62))
    idx.load_trained(cents, books, codes, list_of)
    q = data[::80] + 0.01
    before = idx.search_batch(q, 10, nprobe=4)
    bad = list_of.copy()
    bad[5] = nlist + 3
    with pytest.raises(px.Corruption):
        idx.load_trained(cents[:4] * 2, books * 2, codes, bad)
    with pytest.raises(px.Corruption):
        idx.load_trained(cents, books, codes, None)
    after = idx.search_batch(q, 10, nprobe=4)
    for a, b in zip(before, after):
        assert np.array_equal(a, b)
    assert np.array_equal(idx.parts()[0], cents)


def _oracle_state(idx, vectors_by_slot, cents, books, m):
    """The index's current slots (ids, live) and the oracle's own encoding of
    their vectors (ivfpq.rs:828-898)."""
    ids, live = idx.slots()
    codes, list_of = orc.ivf_encode(vectors_by_slot[: ids.size], cents, books, m, live=live)
    return ids, live, codes, list_of


@pytest.mark.parametrize("dim,m,rerank", [(32, 16, 0), (32, 16, 40), (16, 8, 0)])
def test_interleaved_mutations_and_searches(gpu, dim, m, rerank):
    """Removals and inserts between searches update the list view in place
    (appends, holes filled by each list's last entry, regions moved when
    full); every search equals the oracle's on the state at that moment
    (ivfpq.rs:1129-1180 then 998-1110)."""
    px = gpu
    rng = np.random.default_rng(dim + m + rerank)
    n, nlist = 6000, 24
    data = corpus(n, dim, 20) + rng.standard_normal((n, dim)).astype(np.float32) * 0.2
    cents, books, _ = orc.ivf_train(data, nlist, m, max_iter=8, seed=4)
    codes, list_of = orc.ivf_encode(data, cents, books, m)
    cfg = px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62).with_rerank(rerank)
    idx = build(px, data, cfg)
    idx.load_trained(cents, books, codes, list_of)
    vec = np.zeros((4 * n, dim), np.float32)  # vectors by slot
    vec[:n] = data
    q = data[5::211] + 0.07
    next_id = 10 ** 6
    idx.search_batch(q, 10, nprobe=4)  # lays the view out
    rebuilds0, _ = idx.view_stats()
    for cycle in range(6):
        ids, live = idx.slots()
        present = ids[live.astype(bool)]
        for i in rng.choice(present, size=150, replace=False):
            idx.remove(int(i))
        # new vectors: half near one centroid (its region fills and moves), half spread
        near = cents[cycle % nlist] + rng.standard_normal((200, dim)).astype(np.float32) * 0.05
        spread = data[rng.integers(0, n, 200)] * np.float32(1.02)
        new = np.concatenate([near, spread]).astype(np.float32)
        new_ids = np.arange(next_id, next_id + new.shape[0], dtype=np.uint64)
        next_id += new.shape[0]
        slots = idx.insert_batch(new_ids, new)
        vec[slots] = new
        ids, live, codes2, list_of2 = _oracle_state(idx, vec, cents, books, m)
        _, _, gc, glo = idx.parts()
        lv = live.astype(bool)
        assert np.array_equal(glo[lv], list_of2[lv]) and np.array_equal(gc[lv], codes2[lv])
        for nprobe, k in ((4, 10), (24, 7)):
            got = idx.search_batch(q, k, nprobe=nprobe)
            want = orc.ivf_search(0, cents, books, codes2, list_of2, ids, q, k, nprobe, m,
                                  vectors=vec[: ids.size] if rerank else None, rerank=rerank, live=live, threads=8)
            assert_same(got, want)
        acc = (ids % 3 != 0).astype(np.uint8)
        got = idx.search_batch(q, 10, lambda i, _m: i % 3 != 0, nprobe=6)
        want = orc.ivf_search(0, cents, books, codes2, list_of2, ids, q, 10, 6, m,
                              vectors=vec[: ids.size] if rerank else None, rerank=rerank, live=live, accept=acc,
                              threads=8)
        assert_same(got, want)
    rebuilds, moves = idx.view_stats()
    assert rebuilds == rebuilds0  # every mutation was applied in place
    assert moves > 0  # the filled regions moved


def test_list_view_growth_and_compaction(gpu):
    """A batch far beyond the slack of one list: its region moves and the pool
    grows in place; a compaction then lays the view out again. Results equal
    the oracle's throughout."""
    px = gpu
    rng = np.random.default_rng(3)
    n, dim, m, nlist = 3000, 16, 8, 8
    data = corpus(n, dim, 10)
    cents, books, _ = orc.ivf_train(data, nlist, m, max_iter=6, seed=2)
    codes, list_of = orc.ivf_encode(data, cents, books, m)
    idx = build(px, data, px.IvfPqConfig(nlist, m).with_train_threshold(1 << 62))
    idx.load_trained(cents, books, codes, list_of)
    q = data[::301] + 0.1
    idx.search_batch(q, 5, nprobe=2)
    r0, m0 = idx.view_stats()
    new = (cents[0] + rng.standard_normal((4 * n, dim)) * 0.01).astype(np.float32)
    slots = idx.insert_batch(np.arange(n, 5 * n, dtype=np.uint64), new)
    vec = np.zeros((5 * n, dim), np.float32)
    vec[:n] = data
    vec[slots] = new
    ids, live, codes2, list_of2 = _oracle_state(idx, vec, cents, books, m)
    assert_same(idx.search_batch(q, 5, nprobe=2),
                orc.ivf_search(0, cents, books, codes2, list_of2, ids, q, 5, 2, m, live=live, threads=8))
    r1, m1 = idx.view_stats()
    assert r1 == r0 and m1 > m0
    for i in range(0, n, 2):
        idx.remove(i)
    assert idx.compact() > 0
    ids, live = idx.slots()
    vec2 = np.zeros_like(vec)
    for s_, i in enumerate(ids):
        vec2[s_] = data[int(i)] if i < n else new[int(i) - n]
    ids, live, codes3, list_of3 = _oracle_state(idx, vec2, cents, books, m)
    assert_same(idx.search_batch(q, 5, nprobe=2),
                orc.ivf_search(0, cents, books, codes3, list_of3, ids, q, 5, 2, m, live=live, threads=8))
    assert idx.view_stats()[0] == r1 + 1
