"""Fit here, predict there (the reference's tests/reuse.py): a second array of the same shape, batches of one
shape with one rescaled, slices that share their first part, and a model saved in the reference's model.npz
format. This engine keeps no per-dataset state between calls, so every label must still be the oracle's."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def wrong(X, C, lab, tol=1e-5):
    """Rows whose label is farther than the float64 nearest centre by more than a float32 tie (the reference's
    criterion for the approximate mode, tests/reuse.py:20-35)."""
    X64, C64 = np.asarray(X, np.float64), np.asarray(C, np.float64)
    csq = (C64 * C64).sum(1)
    bad = 0
    for s in range(0, len(X64), 20_000):
        x = X64[s:s + 20_000]
        d2 = (x * x).sum(1)[:, None] + csq[None] - 2 * x @ C64.T
        excess = d2[np.arange(len(x)), lab[s:s + 20_000]] / np.maximum(d2.min(1), 1e-300) - 1
        bad += int(np.sum(excess > tol))
    return bad


@pytest.mark.parametrize("d,k,exact", [(8, 16, True), (32, 64, True), (48, 64, True), (128, 256, True),
                                       (64, 32, False), (256, 64, False)])
def test_fit_here_predict_there(d, k, exact):
    from mlx_kmeans import KMeans
    rng = np.random.default_rng(7 + d + k)
    n = 40_000
    A = rng.standard_normal((n, d)).astype(np.float32)
    say(f"[gpu] reuse d={d} k={k} exact={exact}")
    m = KMeans(n_clusters=k, max_iter=3, random_state=0, exact=exact).fit(A)
    B = (rng.standard_normal((n, d)) * 1.3 + 0.5).astype(np.float32)
    lab = m.predict(B)
    if exact:
        assert np.array_equal(m.labels_, oracle.assign(A, m.cluster_centers_)[0].astype(np.int64))
        assert np.array_equal(lab, oracle.assign(B, m.cluster_centers_)[0].astype(np.int64))
    else:
        assert wrong(B, m.cluster_centers_, lab) <= 0.1 * n
    # a second fit of the same shape is bit-identical to a fit of a copy
    m2 = KMeans(n_clusters=k, max_iter=3, random_state=0, exact=exact).fit(B)
    m3 = KMeans(n_clusters=k, max_iter=3, random_state=0, exact=exact).fit(B.copy())
    assert m2.inertia_ == m3.inertia_ and np.array_equal(m2.cluster_centers_, m3.cluster_centers_)


def test_batched_predict_one_batch_rescaled():
    from mlx_kmeans import KMeans
    rng = np.random.default_rng(11)
    T = rng.standard_normal((60_000, 128)).astype(np.float32)
    say("[gpu] batched predict d=128 k=256")
    m = KMeans(n_clusters=256, max_iter=5, random_state=0).fit(T)
    for i in range(4):
        b = (rng.standard_normal((15_000, 128)) * (0.1 if i == 2 else 1.0)).astype(np.float32)
        assert np.array_equal(m.predict(b), oracle.assign(b, m.cluster_centers_)[0].astype(np.int64)), i


def test_predict_on_slices_sharing_the_first_part():
    from mlx_kmeans import KMeans
    rng = np.random.default_rng(12)
    P, Q, R = (rng.standard_normal((20_000, 128)).astype(np.float32) for _ in range(3))
    say("[gpu] slices sharing the first part d=128 k=256")
    m = KMeans(n_clusters=256, max_iter=3, random_state=0).fit([P, Q])
    assert np.array_equal(m.labels_, oracle.assign(np.concatenate([P, Q]), m.cluster_centers_)[0].astype(np.int64))
    lab = m.predict([P, R])
    assert np.array_equal(lab, oracle.assign(np.concatenate([P, R]), m.cluster_centers_)[0].astype(np.int64))


def test_model_npz_round_trip_predicts_the_same(tmp_path):
    """A model saved in the reference's model.npz layout (files.py:178-179: centers, mean, scale, columns) and
    loaded without pickle predicts standardised rows exactly as the fitted model does."""
    from mlx_kmeans import KMeans
    rng = np.random.default_rng(13)
    raw = rng.standard_normal((30_000, 6)) * [1, 5, 10, 0.1, 2, 3] + [0, 1, -3, 5, 0, 2]
    mean, scale = raw.mean(0), raw.std(0)
    X = np.ascontiguousarray((raw - mean) / scale, dtype=np.float32)
    say("[gpu] model.npz round trip d=6 k=7")
    m = KMeans(n_clusters=7, n_init=2, random_state=0).fit(X)
    np.savez(tmp_path / "model.npz", centers=m.cluster_centers_, mean=mean, scale=scale,
             columns=np.array([f"f{i}" for i in range(6)]))
    z = np.load(tmp_path / "model.npz", allow_pickle=False)
    new = rng.standard_normal((5_000, 6)) * [1, 5, 10, 0.1, 2, 3] + [0, 1, -3, 5, 0, 2]
    Xn = np.ascontiguousarray((new - z["mean"]) / z["scale"], dtype=np.float32)
    loaded = KMeans.from_centers(z["centers"])
    assert np.array_equal(loaded.predict(Xn), m.predict(Xn))
    assert np.array_equal(loaded.predict(X), m.labels_)


@pytest.mark.parametrize("d,k", [(32, 48), (8, 12), (96, 64)])
def test_spherical_fit_matches_oracle_loop(d, k):
    """spherical=True (estimator.py:132-150): the starting centres and every step's centres renormalised. The
    engine's device loop from the k-means++ start against the oracle's restatement of the loop from the same
    start, on L2-normalised rows: same iteration count under the default tol, centres within 1e-5, labels_ the
    oracle's assignment to the returned centres, and every returned centre of unit length."""
    from mlx_kmeans import KMeans, core
    rng = np.random.default_rng(50 + d + k)
    n = 30_000
    cen = rng.standard_normal((k, d))
    X = cen[rng.integers(0, k, n)] + 0.25 * rng.standard_normal((n, d))
    X = (X / np.linalg.norm(X, axis=1, keepdims=True)).astype(np.float32)
    say(f"[gpu] spherical fit d={d} k={k}")
    m = KMeans(n_clusters=k, max_iter=40, random_state=3, spherical=True).fit(X)
    C0 = core.kmeans_pp_init([X], n, k, np.random.default_rng(3))
    C_ref, inertia_ref, it_ref, _ = oracle.fit_from(X, C0, 40, tol=1e-4, spherical=True)
    assert m.n_iter_ == it_ref
    assert float(np.max(np.abs(m.cluster_centers_.astype(np.float64) - C_ref))) <= 1e-5
    np.testing.assert_allclose(np.linalg.norm(m.cluster_centers_.astype(np.float64), axis=1), 1.0, atol=1e-6)
    ol, ob = oracle.assign(X, m.cluster_centers_)
    assert np.array_equal(m.labels_, ol.astype(np.int64))
    assert abs(m.inertia_ - float(ob.astype(np.float64).sum())) <= 1e-5 * m.inertia_
    assert abs(m.inertia_ - inertia_ref) <= 1e-4 * inertia_ref


def test_verbose_fit_prints_each_iteration_and_matches(capsys):
    """verbose=True runs the loop one lloyd_step at a time and prints "iter i: inertia ..." per iteration
    (estimator.py:143-144); the fit is the device loop's bit for bit, and with n_init > 1 each start's line
    (estimator.py:205-207) follows."""
    from mlx_kmeans import KMeans
    rng = np.random.default_rng(9)
    n, d, k = 20_000, 16, 24
    cen = rng.uniform(-5, 5, size=(k, d))
    X = (cen[rng.integers(0, k, n)] + rng.standard_normal((n, d))).astype(np.float32)
    say("[gpu] verbose fit")
    quiet = KMeans(n_clusters=k, max_iter=30, random_state=1, n_init=2).fit(X)
    capsys.readouterr()
    loud = KMeans(n_clusters=k, max_iter=30, random_state=1, n_init=2, verbose=True).fit(X)
    out = capsys.readouterr().out.splitlines()
    iters = [ln for ln in out if ln.startswith("iter ")]
    starts = [ln for ln in out if ln.startswith("start ")]
    assert len(starts) == 2 and starts[0].startswith("start 1/2: inertia ")
    assert iters and iters[0].startswith("iter 1: inertia ")
    assert np.array_equal(loud.cluster_centers_, quiet.cluster_centers_)
    assert loud.n_iter_ == quiet.n_iter_ and loud.inertia_ == quiet.inertia_
    assert np.array_equal(loud.labels_, quiet.labels_)
