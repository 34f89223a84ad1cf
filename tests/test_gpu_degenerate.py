"""GPU: degenerate shapes on every path that serves them - a single row, a single centre, fewer rows than one
64-row block, as many centres as rows (every row its own centre: distance 0), a few wide rows (768 to 1536 dims). Labels and best are
the oracle's rows loop (core.py:263-274) bit for bit, the totals agree with the oracle's, and a Lloyd step and a
fit with one centre end at the rows' mean (the reference's KMeans accepts n_clusters=1, estimator.py:7-230)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CENTRE_TOL = 1e-6


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def lib():
    from mlx_kmeans import _lib
    _lib.lib()
    return _lib


def served(path, d, k):
    if path == "mfma":    # the fused screen (d = 16, 32 with k <= 64; d = 64 with k <= 32) or the wide-row screen
        return d in (16, 32) and k <= 64 or d == 64 and k <= 32 or 16 < d <= 1536 and k <= 4096
    if path == "fused":   # the low-d single-read path: d <= 16, k (d + 2) <= 768
        return d <= 16 and k * (d + 2) <= 768
    return True


CASES = [(1, 3, 1), (5, 4, 1), (63, 16, 1), (65, 32, 2), (48, 32, 48), (64, 8, 64), (7, 48, 3), (40, 768, 2),
         (100, 32, 100), (3, 1536, 2), (33, 1000, 33)]


@pytest.mark.parametrize("n,d,k", CASES)
def test_degenerate_shapes_match_the_oracle(lib, n, d, k):
    import oracle
    rng = np.random.default_rng(n * 1000 + d * 10 + k)
    X = (rng.standard_normal((n, d)) * 3 + 1).astype(np.float32)
    C = X[:k].copy() if k == n else (rng.standard_normal((k, d)) * 3 + 1).astype(np.float32)
    ol, ob = oracle.assign(X, C)
    ot = oracle.totals(X, ol, ob, k)
    if k == n:
        assert np.array_equal(ol, np.arange(n, dtype=ol.dtype)) and not ob.any()
    ctx = lib.Context()
    ctx.set_parts([X])
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    ran = 0
    for path in ("auto", "rows", "mfma", "fused"):
        if not served(path, d, k):
            continue
        say(f"[gpu] degenerate n={n} d={d} k={k} path={path}")
        tot, labels, best = ctx.run_pass(C, path=lib.PATHS[path], labels=True, best=True)
        assert np.array_equal(labels, ol.astype(np.uint32)), (path, np.flatnonzero(labels != ol)[:10])
        assert np.array_equal(best.view(np.uint32), ob.view(np.uint32)), path
        assert np.array_equal(np.rint(tot[:, 0]).astype(np.int64), np.rint(ot[:, 0]).astype(np.int64)), path
        cnt = np.maximum(np.rint(ot[:, 0]), 1)[:, None]
        assert float(np.max(np.abs(tot[:, 2:] - ot[:, 2:]) / cnt)) / scale <= CENTRE_TOL, path
        np.testing.assert_allclose(tot[:, 1], ot[:, 1], rtol=1e-6, atol=1e-30)
        ran += 1
    assert ran >= 2
    if k == 1:
        C1, inertia, n_empty = ctx.lloyd_step(C)
        mean = X.astype(np.float64).mean(axis=0)
        assert n_empty == 0
        assert float(np.max(np.abs(C1[0].astype(np.float64) - mean))) <= 1e-6 * max(scale, 1.0)
        assert abs(inertia - float(ob.astype(np.float64).sum())) <= 1e-6 * float(ob.astype(np.float64).sum())
    ctx.close()


def test_single_cluster_fit_ends_at_the_mean(lib):
    from mlx_kmeans import KMeans
    rng = np.random.default_rng(11)
    X = (rng.standard_normal((3000, 32)) + 5).astype(np.float32)
    say("[gpu] KMeans(n_clusters=1)")
    km = KMeans(n_clusters=1, max_iter=10, random_state=0).fit(X)
    mean = X.astype(np.float64).mean(axis=0)
    assert km.cluster_centers_.shape == (1, 32)
    assert float(np.max(np.abs(km.cluster_centers_[0].astype(np.float64) - mean))) <= 1e-5
    assert not np.asarray(km.labels_).any()
    ref = float(((X.astype(np.float64) - km.cluster_centers_[0].astype(np.float64)) ** 2).sum())
    assert abs(km.inertia_ - ref) <= 1e-5 * ref
