"""Writes the golden fixtures in this directory from the oracle (the C++
restatement of the reference under oracle/). Run from the repository root:

    python tests/golden/make_golden.py

Each .npz holds small synthetic inputs (seeded numpy draws, or the
reference's own ChaCha8 fixture stream) and the oracle's outputs for them:
ids, distances, codes, centroids, assignments. tests/test_golden.py checks
that the oracle still reproduces every file bit for bit (CPU) and that the
HIP library returns the same results (GPU). Re-running this script after a
deliberate oracle change regenerates them."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as orc  # noqa: E402

L2, COS, IP = 0, 1, 2


def mixture(rng, n, dim, clusters, sigma, centre_scale=1.0):
    c = rng.standard_normal((clusters, dim)).astype(np.float32) * np.float32(centre_scale)
    which = rng.integers(0, clusters, n)
    return (c[which] + np.float32(sigma) * rng.standard_normal((n, dim)).astype(np.float32)).astype(np.float32)


def flat_l2():
    """Config 1 (flat, Euclidean, k=10) at reduced size: 2000 x 64 from 20
    Gaussian clusters (centres N(0,1), sigma 0.15), 40 queries."""
    rng = np.random.default_rng(101)
    x = mixture(rng, 2040, 64, 20, 0.15)
    data, q = x[:2000], x[2000:]
    ids = np.arange(2000, dtype=np.uint64) * 3 + 1
    oi, od, oc = orc.flat_search(data, ids, L2, q, 10, threads=8)
    return dict(data=data, ids=ids, queries=q, k=np.int64(10), out_ids=oi, out_dist=od, out_count=oc)


def flat_cosine():
    """Config 2 (flat, cosine, k=100) as a subset: 2500 x 96, N(0,1) plus one
    of 16 cluster offsets, 16 queries; the index normalises."""
    rng = np.random.default_rng(102)
    off = rng.standard_normal((16, 96)).astype(np.float32)
    x = (rng.standard_normal((2516, 96)).astype(np.float32) + off[rng.integers(0, 16, 2516)]).astype(np.float32)
    data, q = x[:2500], x[2500:]
    ids = np.arange(2500, dtype=np.uint64)
    oi, od, oc = orc.flat_search(orc.prepare_rows(COS, data), ids, COS, orc.prepare_rows(COS, q), 100, threads=8)
    return dict(data=data, ids=ids, queries=q, k=np.int64(100), out_ids=oi, out_dist=od, out_count=oc)


def sq8_ip():
    """Config 3 (SQ8, inner product, k=10) at reduced size: 3000 x 96
    ~U(-1,1), per-dimension ranges from the first 1000, 30 queries; integer
    scores and rescore = 40."""
    rng = np.random.default_rng(103)
    x = rng.uniform(-1, 1, (3000, 96)).astype(np.float32)
    q = rng.uniform(-1, 1, (30, 96)).astype(np.float32)
    mn, sc, inv, _ = orc.sq_train(x[:1000], True)
    codes = orc.sq_encode(x, mn, inv, True, 1).view(np.int8)
    qc = orc.sq_encode(q, mn, inv, True, 1).view(np.int8)
    ids = np.arange(3000, dtype=np.uint64)
    oi, od, oc = orc.sq8_search(codes, ids, qc, 10, threads=8)
    ri, rd, rc = orc.sq8_search(codes, ids, qc, 10, threads=8, rescore=40, qf=q, ranges=(mn, sc))
    return dict(data=x, queries=q, min=mn, scale=sc, inverse_scale=inv, codes=codes, out_ids=oi, out_dist=od,
                out_count=oc, rescored_ids=ri, rescored_dist=rd, rescored_count=rc)


def ivfpq_tiny():
    """Config 4 (IVF-PQ, Euclidean, k=10) tiny: 3000 x 32 from 40 clusters,
    trained by the oracle (nlist 32, M 8, 10 iterations, seed 17), searched
    at nprobe 1, 4 and 32."""
    rng = np.random.default_rng(104)
    x = mixture(rng, 3000, 32, 40, 0.2)
    q = x[::150] + np.float32(0.05)
    cents, books, report = orc.ivf_train(x, 32, 8, max_iter=10, seed=17)
    codes, list_of = orc.ivf_encode(x, cents, books, 8)
    out = dict(data=x, queries=q, cents=cents, books=books, report=report, codes=codes, list_of=list_of)
    for nprobe in (1, 4, 32):
        oi, od, oc = orc.ivf_search(L2, cents, books, codes, list_of, np.arange(3000), q, 10, nprobe, 8, threads=8)
        out[f"ids_np{nprobe}"], out[f"dist_np{nprobe}"], out[f"count_np{nprobe}"] = oi, od, oc
    return out


def kmeans_tiny():
    """Config 5 (k-means) tiny: 2000 x 16 from 24 clusters (sigma 0.2) into
    24 centroids, 10 iterations, seed 23; k-means++ seeds, final centroids,
    inertia, iterations and the assignment against the final centroids."""
    rng = np.random.default_rng(105)
    x = mixture(rng, 2000, 16, 24, 0.2)
    seeds = orc.kmeans_pp(x, 24, 23)
    cents, inertia, its = orc.kmeans(x, 24, 10, 23)
    a, d = orc.kmeans_assign(x, cents)
    return dict(data=x, seeds=seeds, cents=cents, inertia=np.float64(inertia), iterations=np.int64(its), assign=a,
                dist=d)


def fixture_small():
    """fixture::generate(200, 8, 4, 10, 7) as the oracle computes it (host
    libm ln/cos)."""
    v, q = orc.fixture_generate(200, 8, 4, 10, 7)
    return dict(vectors=v, queries=q)


FILES = {"flat_l2_2000x64_k10": flat_l2, "flat_cosine_2500x96_k100": flat_cosine, "sq8_ip_3000x96_k10": sq8_ip,
         "ivfpq_l2_3000x32_nlist32_m8": ivfpq_tiny, "kmeans_2000x16_k24": kmeans_tiny,
         "fixture_200x8_c4_q10_s7": fixture_small}

if __name__ == "__main__":
    for name, make in FILES.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **make())
        print(path, os.path.getsize(path))
