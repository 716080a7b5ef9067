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
