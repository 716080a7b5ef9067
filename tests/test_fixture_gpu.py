"""GPU fixture generator (crates/proxima-cli/src/fixture.rs:71-123) against
the oracle and the reference's fixture.rs tests.

The ChaCha8 stream and the uniform draws are integer work and must be the
oracle's exactly. Only ln and cos of the Box-Muller step may differ: the
device computes them in f64 and rounds (correctly rounded f32), the oracle
calls the host libm's logf/cosf, which are faithfully rounded. A centre that
differs in its last bit shifts every point of its cluster, so a few percent
of the values differ (up to ~10% with one cluster of 8 dimensions), each by a
few ulps of its magnitude (tolerance below); the rest are bit-identical. A
wrong stream offset or sampler would miss the tolerance by orders of
magnitude, and a low-accuracy ln or cos would leave few values identical."""
import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def close(got, want):
    g, w = np.asarray(got, np.float32), np.asarray(want, np.float32)
    assert g.shape == w.shape
    same = np.mean(g.view(np.uint32) == w.view(np.uint32))
    diff = np.abs(g.astype(np.float64) - w.astype(np.float64))
    tol = 4e-6 * np.maximum(1.0, np.abs(w.astype(np.float64)))
    return same, bool(np.all(diff <= tol)), float(diff.max(initial=0.0))


@pytest.mark.parametrize("count,dim,clusters,queries,seed", [(3000, 16, 7, 50, 42), (1000, 37, 20, 20, 5),
                                                             (513, 8, 1, 0, 11), (64, 128, 64, 64, 0xDEADBEEF)])
def test_matches_oracle(gpu, count, dim, clusters, queries, seed):
    px = gpu
    v, q = px.fixture_generate(count, dim, clusters, queries, seed)
    wv, wq = orc.fixture_generate(count, dim, clusters, queries, seed)
    same, ok, worst = close(v, wv)
    assert ok and same > 0.8, (same, worst)
    if queries:
        same, ok, worst = close(q, wq.reshape(queries, dim))
        assert ok and same > 0.8, (same, worst)


def test_same_seed_same_bytes_and_shape(gpu):  # fixture.rs:132-150
    px = gpu
    a = px.fixture_generate(200, 8, 4, 10, 7)
    b = px.fixture_generate(200, 8, 4, 10, 7)
    c = px.fixture_generate(200, 8, 4, 10, 8)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    assert not np.array_equal(a[0], c[0])
    v, q = px.fixture_generate(500, 16, 10, 25, 1)
    assert v.shape == (500, 16) and q.shape == (25, 16) and v.nbytes == 500 * 16 * 4


def test_finite_and_queries_near_their_source(gpu):  # fixture.rs:153-180
    px = gpu
    v, q = px.fixture_generate(2000, 32, 16, 50, 3)
    assert np.all(np.isfinite(v)) and np.all(np.isfinite(q))
    v, q = px.fixture_generate(1000, 32, 20, 20, 5)
    for i in range(20):
        src = (i * 50) % 1000
        if src == 0:
            continue
        assert orc.squared_euclidean(q[i], v[src]) < orc.squared_euclidean(q[i], v[0])


def test_device_entry_point_matches_host(gpu):
    import torch
    px = gpu
    v, q = px.fixture_generate(4096, 24, 30, 100, 9)
    dv = torch.empty((4096, 24), dtype=torch.float32, device="cuda")
    dq = torch.empty((100, 24), dtype=torch.float32, device="cuda")
    px.fixture_generate_device(4096, 24, 30, 100, 9, dv, dq)
    assert np.array_equal(dv.cpu().numpy(), v) and np.array_equal(dq.cpu().numpy(), q)
    with pytest.raises(ValueError):
        px.fixture_generate_device(4096, 24, 30, 100, 9, dv[:10], dq)


# --- the benchmark configurations' inputs (no reference counterpart) ---------------
def _stream_words(seed, n):
    r = orc.Rng(seed)
    return np.array([r.next_u32() for _ in range(n)], np.uint64)


def _u01(w):
    return ((w >> 8).astype(np.float64) * 2.0 ** -24).astype(np.float32)


def _gaussians(words):
    u1 = np.maximum(_u01(words[0::2]), np.float32(1.17549435e-38))
    u2 = _u01(words[1::2])
    ln = np.log(u1.astype(np.float64)).astype(np.float32)
    a = (np.float32(6.2831855) * u2).astype(np.float32)
    c = np.cos(a.astype(np.float64)).astype(np.float32)
    return (np.sqrt((np.float32(-2.0) * ln).astype(np.float32)) * c).astype(np.float32)


@pytest.mark.parametrize("drawn", [False, True])
def test_mixture_matches_its_stated_stream(gpu, drawn):
    import torch
    px = gpu
    count, dim, clusters, queries, seed, scale, sigma = 301, 12, 7, 33, 0x9E3779B9, 1.0, 0.15
    cd, items = clusters * dim, count + queries
    gB = cd
    gC = gB + ((items + 1) // 2 if drawn else 0)
    gD = gC + count * dim
    words = _stream_words(seed, 2 * (gD + queries * dim))
    g = _gaussians(words)
    centres = (g[:cd] * np.float32(scale)).reshape(clusters, dim)
    if drawn:
        cw = words[2 * gB:2 * gB + items]
        cl = ((cw * np.uint64(clusters)) >> np.uint64(32)).astype(np.int64)
    else:
        cl = np.concatenate([np.arange(count) % clusters, np.arange(queries) % clusters])
    want_v = centres[cl[:count]] + np.float32(sigma) * g[gC:gD].reshape(count, dim)
    want_q = centres[cl[count:]] + np.float32(sigma) * g[gD:].reshape(queries, dim)
    v = torch.empty((count, dim), dtype=torch.float32, device="cuda")
    q = torch.empty((queries, dim), dtype=torch.float32, device="cuda")
    px.mixture_generate_device(count, dim, clusters, scale, sigma, queries, drawn, seed, v, q)
    for got, want in ((v.cpu().numpy(), want_v), (q.cpu().numpy(), want_q)):
        same, ok, worst = close(got, want)
        assert ok and same > 0.8, (same, worst)
    if drawn:
        assert len(set(cl.tolist())) == clusters  # drawn choices reach every cluster
    # the same seed gives the same bytes; another seed other bytes
    v2 = torch.empty_like(v)
    q2 = torch.empty_like(q)
    px.mixture_generate_device(count, dim, clusters, scale, sigma, queries, drawn, seed, v2, q2)
    assert torch.equal(v, v2) and torch.equal(q, q2)
    px.mixture_generate_device(count, dim, clusters, scale, sigma, queries, drawn, seed + 1, v2, q2)
    assert not torch.equal(v, v2)


def test_uniform_matches_its_stated_stream(gpu):
    import torch
    px = gpu
    count, dim, seed = 1000, 96, 0x9E3779B9 + 11
    w = _stream_words(seed, count * dim)
    want = (np.float32(-1.0) + np.float32(2.0) * _u01(w)).astype(np.float32).reshape(count, dim)
    out = torch.empty((count, dim), dtype=torch.float32, device="cuda")
    px.uniform_generate_device(count, dim, -1.0, 1.0, seed, out)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert got.min() >= -1.0 and got.max() < 1.0
    with pytest.raises(ValueError):
        px.uniform_generate_device(count, dim, -1.0, 1.0, seed, out[:10])
