"""GPU: which assignment a pass runs, against the reference's dispatch, and the wide-row screen's list overflow.

* exact=False (mode KM_APPROX) approximates only where the reference's _gpu_pass would (core.py:2036-2042): from 64
  dims when sqrt(max |x|^2 max |c|^2) < 65504 / 4 (core.py:1031, 1035, 1055-1058). Below 64 dims, and wherever
  that guard fails, the pass is exact - bit-identical to the oracle. (At 256 dims and more the reference's
  guard-failing case multiplies in float32, whose argmin differs from the exact labels only at rounding-level
  ties; the engine serves it exactly.)
* Approximate labels: best is the exact float32 distance to the chosen centre (the oracle's distances_to,
  core.py:851-856), so every best and the inertia are >= the exact ones; labels disagree with exact mode on at
  most 10 % of rows (the reference's bound, tests/reuse.py:61).
* A half-row whose candidate list overflows sends its row to the full scan even when the other half's list
  did not overflow (the row's code is written by the h = 0 lane).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def lib():
    from mlx_kmeans import _lib
    _lib.lib()
    return _lib


def _gauss(seed, n, d, k, centre_scale=1.0, noise=1.0):
    rng = np.random.default_rng(seed)
    cen = (centre_scale * rng.standard_normal((k, d))).astype(np.float32)
    X = (cen[rng.integers(0, k, n)] + noise * rng.standard_normal((n, d))).astype(np.float32)
    C = X[rng.choice(n, k, replace=False)].copy()
    return X, C


@pytest.mark.parametrize("d,k", [(48, 100), (32, 256), (17, 300), (63, 128)])
def test_approx_below_64_dims_is_exact(lib, d, k):
    """exact=False below 64 dims runs the exact kernels: labels and best bit-identical to the oracle, in a pass,
    a Lloyd step and a fit."""
    import oracle
    X, C = _gauss(100 + d + k, 40_000, d, k // 2, centre_scale=2.0, noise=0.8)
    ctx = lib.Context()
    ctx.set_parts([X])
    say(f"[gpu] approx below 64 dims d={d} k={k}")
    tot, labels, best = ctx.run_pass(C, mode=lib.KM_APPROX, labels=True, best=True)
    ol, ob = oracle.assign(X, C)
    assert np.array_equal(labels, ol), np.flatnonzero(labels != ol)[:10]
    assert np.array_equal(best.view(np.uint32), ob.view(np.uint32))
    C1, inertia, n_empty = ctx.lloyd_step(C, mode=lib.KM_APPROX)
    R1, r_in, r_empty, _, _, _ = oracle.lloyd_step(X, C)
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    assert n_empty == r_empty
    assert abs(inertia - r_in) <= 1e-6 * r_in
    assert float(np.max(np.abs(C1.astype(np.float64) - R1))) / scale <= 1e-6
    ctx.close()


@pytest.mark.parametrize("d,k", [(64, 128), (128, 256), (256, 96)])
def test_approx_guard_decides_per_scale(lib, d, k):
    """The same geometry at two scales. At scale 1 the half-precision guard holds, so exact=False takes the
    screen's argmin on trust: best is the exact distance to that label, labels disagree with exact mode on a few
    rows (near-ties are common in this data) and on at most 10 %. Scaled by 1024 (bf16 rounding of the scaled
    values is the same relative rounding) the guard fails, and the pass is exact: bit-identical to the oracle."""
    import oracle
    X, C = _gauss(7 + d + k, 30_000, d, k, centre_scale=0.35, noise=1.0)
    ctx = lib.Context()
    ctx.set_parts([X])
    say(f"[gpu] approx guard d={d} k={k} scale 1")
    te, le, be = ctx.run_pass(C, mode=lib.KM_EXACT, labels=True, best=True)
    ta, la, ba = ctx.run_pass(C, mode=lib.KM_APPROX, labels=True, best=True)
    ol, ob = oracle.assign(X, C)
    assert np.array_equal(le, ol) and np.array_equal(be.view(np.uint32), ob.view(np.uint32))
    assert np.array_equal(ba.view(np.uint32), oracle.distances_to(X, C, la).view(np.uint32))
    assert np.all(ba >= be)
    assert float(ta[:, 1].sum()) >= float(te[:, 1].sum())
    dis = float(np.mean(la != le))
    say(f"[gpu]   approx label disagreement {dis:.4%}")
    assert 0.0 < dis <= 0.10
    assert np.array_equal(np.rint(ta[:, 0]), np.bincount(la, minlength=k))
    ctx.close()

    Xs, Cs = X * np.float32(1024.0), C * np.float32(1024.0)
    ctx = lib.Context()
    ctx.set_parts([Xs])
    say(f"[gpu] approx guard d={d} k={k} scale 1024")
    ts, ls, bs = ctx.run_pass(Cs, mode=lib.KM_APPROX, labels=True, best=True)
    ol, ob = oracle.assign(Xs, Cs)
    assert np.array_equal(ls, ol), np.flatnonzero(ls != ol)[:10]
    assert np.array_equal(bs.view(np.uint32), ob.view(np.uint32))
    ctx.close()


def test_approx_embed_workload_full_size(lib):
    """exact=False on 1M x 768, k = 1024 unit-norm vMF-style rows (the guard holds: |x| = |c| = 1): best equals the
    oracle's distance to the chosen label bit for bit, every best and the inertia are >= the exact ones, labels
    disagree with exact mode on at most 10 % of rows, counts match the labels; and a 15-iteration fit lands within
    0.1 % of the exact fit's inertia (the reference reports 0.003 % on GIST1M, estimator.py:27-29)."""
    import oracle
    from mlx_kmeans import synthetic
    w = synthetic.embed_d768()
    X, C0, k = w["X"], w["C0"], w["k"]
    n = len(X)
    ctx = lib.Context()
    ctx.set_parts([X])
    say(f"[gpu] embed exact=False full size n={n}")
    te, le, be = ctx.run_pass(C0, mode=lib.KM_EXACT, labels=True, best=True)
    ta, la, ba = ctx.run_pass(C0, mode=lib.KM_APPROX, labels=True, best=True)
    assert ctx.last_path() == "mfma"
    assert np.array_equal(ba.view(np.uint32), oracle.distances_to(X, C0, la).view(np.uint32))
    assert np.all(ba >= be)
    assert float(ta[:, 1].sum()) >= float(te[:, 1].sum())
    dis = float(np.mean(la != le))
    say(f"[gpu]   approx label disagreement {dis:.4%}")
    assert 0.0 < dis <= 0.10
    counts = np.rint(ta[:, 0]).astype(np.int64)
    assert int(counts.sum()) == n and np.array_equal(counts, np.bincount(la, minlength=k))
    colsum = X.astype(np.float64).sum(0)
    assert np.max(np.abs(ta[:, 2:].sum(0) - colsum)) <= 1e-6 * np.abs(X).astype(np.float64).sum(0).max()
    say("[gpu]   embed fits exact / approx, 15 iterations")
    _, ie, ne, _ = ctx.fit(C0, 15, 0.0, mode=lib.KM_EXACT)
    _, ia, na, _ = ctx.fit(C0, 15, 0.0, mode=lib.KM_APPROX)
    say(f"[gpu]   fit inertia exact {ie:.8e} approx {ia:.8e}")
    assert ne == na == 15
    assert abs(ia - ie) <= 1e-3 * ie
    ctx.close()


def test_wide_screen_list_overflow_on_the_second_half(lib):
    """Rows near a point p; 32 centres at p + small offsets on the screen's second half-row (index % 8 in 4..7),
    all inside the error window, their exact distances ordered so that the nearest is the last (index 63, in the
    second chunk of 32); the first half-row's centres far away. The second half's list (16 entries) overflows
    while the first half's stays empty: the row must take the full scan, whose label and best are the oracle's.
    Exact passes with per-row outputs and Lloyd steps without them both go through the same screen."""
    import oracle
    rng = np.random.default_rng(2024)
    d, k, n = 48, 64, 4096
    p = rng.uniform(-2.0, 2.0, d).astype(np.float32)
    C = np.empty((k, d), np.float32)
    for c in range(k):
        if c % 8 >= 4:
            v = rng.standard_normal(d)
            v /= np.linalg.norm(v)
            C[c] = p + (1e-3 * (1.0 + (63 - c) / 64.0) * v).astype(np.float32)
        else:
            C[c] = p + 3.0 * rng.standard_normal(d).astype(np.float32)
    X = (p + 1e-6 * rng.standard_normal((n, d))).astype(np.float32)
    ctx = lib.Context()
    ctx.set_parts([X])
    say("[gpu] wide screen list overflow on the second half-row")
    tot, labels, best = ctx.run_pass(C, path=lib.KM_PATH_MFMA, labels=True, best=True)
    assert ctx.last_path() == "mfma"
    ol, ob = oracle.assign(X, C)
    assert np.all(ol // 32 == 1), "the nearest centres are in the second chunk"
    assert np.array_equal(labels, ol), np.flatnonzero(labels != ol)[:10]
    assert np.array_equal(best.view(np.uint32), ob.view(np.uint32))
    assert ctx.fallback_rows() >= n
    C1, inertia, n_empty = ctx.lloyd_step(C)
    R1, r_in, r_empty, _, _, _ = oracle.lloyd_step(X, C)
    assert n_empty == r_empty
    assert abs(inertia - r_in) <= 1e-6 * max(r_in, 1e-30)
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    assert float(np.max(np.abs(C1.astype(np.float64) - R1))) / scale <= 1e-6
    ctx.close()


def test_nonfinite_inertia_stops_the_fit_loop(lib):
    """A NaN in the data makes the first pass's inertia NaN: the device loop stops there (one iteration, not
    max_iter), as the reference raises at the first non-finite lloyd_step (estimator.py:140-141)."""
    X = np.random.default_rng(0).standard_normal((5000, 8)).astype(np.float32)
    X[10, 2] = np.nan
    ctx = lib.Context()
    ctx.set_parts([X])
    say("[gpu] non-finite inertia stops the loop")
    C, inertia, n_iter, _ = ctx.fit(X[:4].copy(), 300, 1e-4)
    assert not np.isfinite(inertia)
    assert n_iter == 1
    ctx.close()
