"""Committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from the oracle): the oracle must still
reproduce them bit for bit (CPU), and the HIP library must return the same
ids, distances, codes, centroids and assignments (GPU)."""
import os

import numpy as np
import pytest

from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
L2, COS, IP = 0, 1, 2


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def same_results(got, ids, dist, count):
    gi, gd, gc = got
    assert np.array_equal(gc, count)
    for q in range(count.size):
        c = int(count[q])
        assert np.array_equal(gi[q, :c], ids[q, :c]), q
        assert np.array_equal(bits(gd[q, :c]), bits(dist[q, :c])), q


# --- the oracle against its own committed outputs (CPU) -----------------------------------
def test_oracle_flat_goldens():
    g = load("flat_l2_2000x64_k10")
    same_results(orc.flat_search(g["data"], g["ids"], L2, g["queries"], 10, threads=4), g["out_ids"], g["out_dist"],
                 g["out_count"])
    g = load("flat_cosine_2500x96_k100")
    same_results(orc.flat_search(orc.prepare_rows(COS, g["data"]), g["ids"], COS, orc.prepare_rows(COS, g["queries"]),
                                 100, threads=4), g["out_ids"], g["out_dist"], g["out_count"])


def test_oracle_sq8_golden():
    g = load("sq8_ip_3000x96_k10")
    mn, sc, inv, _ = orc.sq_train(g["data"][:1000], True)
    assert np.array_equal(bits(mn), bits(g["min"])) and np.array_equal(bits(inv), bits(g["inverse_scale"]))
    codes = orc.sq_encode(g["data"], mn, inv, True, 1).view(np.int8)
    assert np.array_equal(codes, g["codes"])
    qc = orc.sq_encode(g["queries"], mn, inv, True, 1).view(np.int8)
    ids = np.arange(codes.shape[0], dtype=np.uint64)
    same_results(orc.sq8_search(codes, ids, qc, 10, threads=4), g["out_ids"], g["out_dist"], g["out_count"])
    same_results(orc.sq8_search(codes, ids, qc, 10, threads=4, rescore=40, qf=g["queries"], ranges=(mn, sc)),
                 g["rescored_ids"], g["rescored_dist"], g["rescored_count"])


def test_oracle_ivfpq_golden():
    g = load("ivfpq_l2_3000x32_nlist32_m8")
    cents, books, report = orc.ivf_train(g["data"], 32, 8, max_iter=10, seed=17)
    assert np.array_equal(bits(cents), bits(g["cents"])) and np.array_equal(bits(books), bits(g["books"]))
    assert np.array_equal(report, g["report"])
    codes, list_of = orc.ivf_encode(g["data"], cents, books, 8)
    assert np.array_equal(codes, g["codes"]) and np.array_equal(list_of, g["list_of"])
    for nprobe in (1, 4, 32):
        got = orc.ivf_search(L2, cents, books, codes, list_of, np.arange(3000), g["queries"], 10, nprobe, 8,
                             threads=4)
        same_results(got, g[f"ids_np{nprobe}"], g[f"dist_np{nprobe}"], g[f"count_np{nprobe}"])


def test_oracle_kmeans_and_fixture_goldens():
    g = load("kmeans_2000x16_k24")
    assert np.array_equal(bits(orc.kmeans_pp(g["data"], 24, 23)), bits(g["seeds"]))
    cents, inertia, its = orc.kmeans(g["data"], 24, 10, 23)
    assert np.array_equal(bits(cents), bits(g["cents"])) and inertia == g["inertia"] and its == g["iterations"]
    a, d = orc.kmeans_assign(g["data"], cents)
    assert np.array_equal(a, g["assign"]) and np.array_equal(bits(d), bits(g["dist"]))
    f = load("fixture_200x8_c4_q10_s7")
    v, q = orc.fixture_generate(200, 8, 4, 10, 7)
    assert np.array_equal(bits(v), bits(f["vectors"])) and np.array_equal(bits(q), bits(f["queries"]))


# --- the HIP library against the goldens (GPU) ---------------------------------------------
@pytest.mark.gpu
def test_gpu_flat_goldens(gpu):
    px = gpu
    g = load("flat_l2_2000x64_k10")
    idx = px.FlatIndex(px.VectorSpace(64, px.Metric.EUCLIDEAN))
    idx.insert_batch(g["ids"], g["data"])
    same_results(idx.search_batch(g["queries"], 10), g["out_ids"], g["out_dist"], g["out_count"])
    g = load("flat_cosine_2500x96_k100")
    idx = px.FlatIndex(px.VectorSpace(96, px.Metric.COSINE))
    idx.insert_batch(g["ids"], g["data"])
    same_results(idx.search_batch(g["queries"], 100), g["out_ids"], g["out_dist"], g["out_count"])


@pytest.mark.gpu
def test_gpu_sq8_golden(gpu):
    px = gpu
    g = load("sq8_ip_3000x96_k10")
    idx = px.Sq8Index(px.VectorSpace(96, px.Metric.INNER_PRODUCT))
    idx.train(g["data"][:1000])
    qz = idx.quantizer()
    assert np.array_equal(bits(qz.min), bits(g["min"])) and np.array_equal(bits(qz.inverse_scale),
                                                                           bits(g["inverse_scale"]))
    idx.insert_batch(np.arange(3000, dtype=np.uint64), g["data"])
    for i in (0, 1234, 2999):
        assert np.array_equal(idx.code(i), g["codes"][i])
    for mode in (1, 2):  # integer MFMA, exact scan
        idx.set_search_mode(mode)
        same_results(idx.search_batch(g["queries"], 10), g["out_ids"], g["out_dist"], g["out_count"])
        same_results(idx.search_batch(g["queries"], 10, rescore=40), g["rescored_ids"], g["rescored_dist"],
                     g["rescored_count"])


@pytest.mark.gpu
def test_gpu_ivfpq_golden(gpu):
    px = gpu
    g = load("ivfpq_l2_3000x32_nlist32_m8")
    cfg = px.IvfPqConfig(32, 8).with_train_threshold(1 << 62).with_seed(17).with_max_iterations(10)
    idx = px.IvfPqIndex(px.VectorSpace(32, px.Metric.EUCLIDEAN), cfg)
    idx.insert_batch(np.arange(3000, dtype=np.uint64), g["data"])
    idx.train()
    cents, books, codes, list_of = idx.parts()
    assert np.array_equal(bits(cents), bits(g["cents"])) and np.array_equal(bits(books), bits(g["books"]))
    assert np.array_equal(codes, g["codes"]) and np.array_equal(list_of, g["list_of"])
    for nprobe in (1, 4, 32):
        same_results(idx.search_batch(g["queries"], 10, nprobe=nprobe), g[f"ids_np{nprobe}"], g[f"dist_np{nprobe}"],
                     g[f"count_np{nprobe}"])


@pytest.mark.gpu
def test_gpu_kmeans_and_fixture_goldens(gpu):
    px = gpu
    g = load("kmeans_2000x16_k24")
    assert np.array_equal(bits(px.kmeans_pp(g["data"], 24, 23)), bits(g["seeds"]))
    got = px.kmeans(g["data"], 16, 24, 10, 23)
    assert np.array_equal(bits(got.centroids), bits(g["cents"].reshape(-1)))
    assert got.inertia == g["inertia"] and got.iterations == g["iterations"]
    a, d = px.kmeans_assign(g["data"], g["cents"])
    assert np.array_equal(a, g["assign"]) and np.array_equal(bits(d), bits(g["dist"]))
    f = load("fixture_200x8_c4_q10_s7")
    v, q = px.fixture_generate(200, 8, 4, 10, 7)
    for got_, want in ((v, f["vectors"]), (q, f["queries"])):
        diff = np.abs(got_.astype(np.float64) - want.astype(np.float64))
        assert np.all(diff <= 4e-6 * np.maximum(1.0, np.abs(want)))
        assert np.mean(bits(got_) == bits(want)) > 0.8
