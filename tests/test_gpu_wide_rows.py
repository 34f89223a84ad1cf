"""GPU: rows of 769 to 1536 dims on the wide-row path (GIST-like 960-dim descriptors, 1024- and 1536-dim
embeddings), the reference's tiles design (core.py:616-651, 310-377) at the widths its tiles path takes.

From 49 K-steps of 16 dims the screen runs one block per CU (its 32 rows per wave held as matrix-core operands in
up to 384 registers) and the per-cluster sums take 14 to 24 dims per lane. Labels and best must be the rows loop's
(core.py:263-274) bit for bit against the oracle on every row, on every path that serves the shape; the totals
within the reference's accuracy bar (tests/accuracy.py:91-99); one Lloyd step against the oracle's; and a fit loop
whose passes take the change-only sums must reach the centres that single steps with full sums reach. Rows wider
than 1536 dims take the rows loop, in its tiled form from four centres on (as does the forced rows path from 65
dims), held to the same bar.
"""
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


def _blobs(seed, n, d, k, true_k, parts=1):
    rng = np.random.default_rng(seed)
    cen = rng.uniform(-1, 1, (true_k, d)).astype(np.float32)
    X = (cen[rng.integers(0, true_k, n)] + 0.35 * rng.standard_normal((n, d))).astype(np.float32)
    C = X[rng.choice(n, k, replace=False)].copy()
    cuts = np.linspace(0, n, parts + 1).astype(int)
    return X, C, [X[cuts[i]:cuts[i + 1]] for i in range(parts)]


@pytest.mark.parametrize("n,d,k,parts", [(20_000, 960, 304, 1), (10_007, 1000, 100, 2), (8_000, 1536, 64, 1),
                                         (6_001, 1100, 257, 3), (30_000, 1024, 1024, 1), (5_000, 770, 33, 1),
                                         (6_000, 1040, 4500, 1), (9_001, 769, 200, 1), (7_003, 784, 65, 2)])
def test_wide_rows_match_the_oracle(lib, n, d, k, parts):
    import oracle
    X, C, slices = _blobs(n + d + k, n, d, k, max(k // 4, 3), parts)
    ol, ob = oracle.assign(X, C)
    ot = oracle.totals(X, ol, ob, k)
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    ctx = lib.Context()
    ctx.set_parts(slices)
    for path in ("auto", "mfma", "rows"):
        say(f"[gpu] wide rows n={n} d={d} k={k} parts={parts} path={path}")
        tot, labels, best = ctx.run_pass(C, path=lib.PATHS[path], labels=True, best=True)
        assert ctx.last_path() == ("rows" if path == "rows" else "mfma")
        assert np.array_equal(labels, ol), (path, np.flatnonzero(labels != ol)[:10])
        assert np.array_equal(best.view(np.uint32), ob.view(np.uint32)), path
        counts = np.rint(tot[:, 0]).astype(np.int64)
        assert np.array_equal(counts, np.rint(ot[:, 0]).astype(np.int64)), path
        used = counts > 0
        err = float(np.max(np.abs(tot[used, 2:] - ot[used, 2:]) / counts[used, None])) / scale
        assert err <= CENTRE_TOL, (path, err)
        ri = float(ot[:, 1].sum())
        assert abs(float(tot[:, 1].sum()) - ri) <= 1e-6 * ri, path
    say(f"[gpu]   rows scored against every centre: {ctx.fallback_rows()}")
    C1, inertia, n_empty = ctx.lloyd_step(C)
    R1, r_in, r_empty, _, _, _ = oracle.lloyd_step(X, C)
    assert n_empty == r_empty
    assert abs(inertia - r_in) <= 1e-6 * r_in
    assert float(np.max(np.abs(C1.astype(np.float64) - R1))) / scale <= CENTRE_TOL
    ctx.close()


@pytest.mark.parametrize("d,ndup,overflow", [(1024, 40, False), (800, 40, False), (1536, 40, False),
                                             (1024, 80, True), (768, 40, True), (768, 24, False)])
def test_window_lists_at_their_capacity(lib, d, ndup, overflow):
    """Rows N(0, 1) scored against ndup near-identical centres at the origin (indices 64 .. 64 + ndup - 1, spread
    0.01 per dim) and 216 far ones (norm 100): every row's window holds all ndup near ones and no far one, ndup / 2
    per half-row. A half-row lists up to 32 centres above 768 dims and 16 up to 768; past that the row takes the
    full scan. Labels and best are the oracle's bit for bit either way (the rescoring's ascending order and strict
    '<' over nearly equal distances), and the rows sent to the full scan are all rows or none."""
    import oracle
    rng = np.random.default_rng(d + ndup)
    n, k = 4_000, 256
    X = rng.standard_normal((n, d)).astype(np.float32)
    far = rng.standard_normal((k, d))
    C = (100.0 * far / np.linalg.norm(far, axis=1, keepdims=True)).astype(np.float32)
    C[64:64 + ndup] = (0.01 * rng.standard_normal((ndup, d))).astype(np.float32)
    ol, ob = oracle.assign(X, C)
    ctx = lib.Context()
    ctx.set_parts([X])
    say(f"[gpu] window lists n={n} d={d} k={k} near centres={ndup}")
    _, labels, best = ctx.run_pass(C, labels=True, best=True)
    assert ctx.last_path() == "mfma"
    fb = ctx.fallback_rows()
    say(f"[gpu]   rows scored against every centre: {fb}")
    assert np.all((ol >= 64) & (ol < 64 + ndup))
    assert np.array_equal(labels, ol), np.flatnonzero(labels != ol)[:10]
    assert np.array_equal(best.view(np.uint32), ob.view(np.uint32))
    assert fb == (n if overflow else 0)
    ctx.close()


@pytest.mark.parametrize("d,k,parts", [(960, 48, 1), (1536, 24, 2)])
def test_wide_rows_fit_loop_matches_single_steps(lib, d, k, parts):
    """km_fit's passes after the first add only the rows that changed cluster when at most half of them did, and
    the full sums otherwise; twelve passes must reach the centres (within 1e-6 of the RMS) and inertia (1e-6) of
    twelve single Lloyd steps with full sums, and a rerun the same bits. The start is drawn from one corner of the
    data, so that both kinds of pass occur."""
    rng = np.random.default_rng(77 + d + k)
    n = 60_013
    cen = rng.uniform(-1, 1, size=(k, d)).astype(np.float32)
    X = (cen[rng.integers(0, k, n)] + 0.5 * rng.standard_normal((n, d))).astype(np.float32)
    order = np.argsort(X[:, 0])
    C0 = X[order[rng.choice(n // 20, k, replace=False)]].copy()
    cuts = np.linspace(0, n, parts + 1).astype(int)
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    ctx = lib.Context()
    ctx.set_parts([X[cuts[i]:cuts[i + 1]] for i in range(parts)])
    steps = 12
    say(f"[gpu] wide fit loop d={d} k={k} parts={parts}")
    C_fit, in_fit, it_fit, _ = ctx.fit(C0, steps, -1.0)
    assert it_fit == steps and ctx.last_path() == "mfma"
    C, moved, prev = C0, [], None
    for _ in range(steps):
        _, lab, _ = ctx.run_pass(C, labels=True)
        if prev is not None:
            moved.append(int((lab != prev).sum()))
        prev = lab
        C, inertia, _ = ctx.lloyd_step(C)
    say(f"[gpu]   rows changing cluster per pass: {moved}")
    assert any(0 < m <= n // 2 for m in moved), "some pass should take the change-only sums"
    assert float(np.max(np.abs(C_fit.astype(np.float64) - C.astype(np.float64)))) / scale <= CENTRE_TOL
    assert abs(in_fit - inertia) <= 1e-6 * inertia
    C2, in2, _, _ = ctx.fit(C0, steps, -1.0)
    assert np.array_equal(C2, C_fit) and in2 == in_fit
    ctx.close()


@pytest.mark.parametrize("n,d,k,parts", [(3_000, 2048, 100, 1), (2_001, 3000, 300, 2), (1_500, 4096, 1000, 1),
                                         (1_000, 1537, 4, 1), (700, 2500, 3, 1), (5_000, 100, 64, 2)])
def test_rows_wider_than_the_screen_match_the_oracle(lib, n, d, k, parts):
    import oracle
    X, C, slices = _blobs(n * 7 + d + k, n, d, k, max(k // 4, 3), parts)
    ol, ob = oracle.assign(X, C)
    ot = oracle.totals(X, ol, ob, k)
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    ctx = lib.Context()
    ctx.set_parts(slices)
    for path in ("auto", "rows"):
        say(f"[gpu] rows loop n={n} d={d} k={k} parts={parts} path={path}")
        tot, labels, best = ctx.run_pass(C, path=lib.PATHS[path], labels=True, best=True)
        if d > 1536:
            assert ctx.last_path() == "rows"
        assert np.array_equal(labels, ol), (path, np.flatnonzero(labels != ol)[:10])
        assert np.array_equal(best.view(np.uint32), ob.view(np.uint32)), path
        counts = np.rint(tot[:, 0]).astype(np.int64)
        assert np.array_equal(counts, np.rint(ot[:, 0]).astype(np.int64)), path
        used = counts > 0
        err = float(np.max(np.abs(tot[used, 2:] - ot[used, 2:]) / counts[used, None])) / scale
        assert err <= CENTRE_TOL, (path, err)
    C1, inertia, n_empty = ctx.lloyd_step(C)
    R1, r_in, r_empty, _, _, _ = oracle.lloyd_step(X, C)
    assert n_empty == r_empty
    assert abs(inertia - r_in) <= 1e-6 * r_in
    assert float(np.max(np.abs(C1.astype(np.float64) - R1))) / scale <= CENTRE_TOL
    ctx.close()


@pytest.mark.parametrize("d,k", [(3072, 32), (1536, 48)])
def test_estimator_on_wide_rows(lib, d, k):
    """KMeans end to end (k-means++ seeding on the device, the GPU-resident loop, final scoring, predict) at 3072
    dims (the tiled rows loop) and 1536 dims (the screen at 96 K-steps): labels_ are the oracle's assignment to the
    returned centres bit for bit, inertia_ the oracle's, predict(X) returns labels_."""
    import oracle
    from mlx_kmeans import KMeans
    rng = np.random.default_rng(d + k)
    n = 6_000
    cen = rng.standard_normal((k, d)).astype(np.float32)
    X = (cen[rng.integers(0, k, n)] + 0.5 * rng.standard_normal((n, d))).astype(np.float32)
    say(f"[gpu] KMeans on {n} x {d}, k = {k}")
    km = KMeans(n_clusters=k, max_iter=8, random_state=3).fit(X)
    ol, ob = oracle.assign(X, km.cluster_centers_)
    assert np.array_equal(km.labels_, ol.astype(np.int64))
    ref = float(ob.astype(np.float64).sum())
    assert abs(km.inertia_ - ref) <= 1e-5 * ref
    assert np.array_equal(km.predict(X), km.labels_)


@pytest.mark.parametrize("d,k", [(2048, 40), (1000, 70), (200, 16)])
def test_non_finite_rows_on_wide_paths(lib, d, k):
    """Rows holding NaN or +-inf, and one centre with an infinite coordinate: labels and best are still the rows
    loop's bit for bit (a NaN distance never compares below, a row whose distances are all NaN or +inf keeps label 0
    and best +inf) on the tiled rows loop and the wide-row screen."""
    import oracle
    X, C, _ = _blobs(d * 3 + k, 3_000, d, k, 8)
    X[5, 3] = np.nan
    X[17, :] = np.nan
    X[40, 0] = np.inf
    X[41, 1] = -np.inf
    C[k - 1, 2] = np.inf
    ol, ob = oracle.assign(X, C)
    ctx = lib.Context()
    ctx.set_parts([X])
    for path in ("auto", "mfma", "rows"):
        if path == "mfma" and d > 1536:
            continue
        say(f"[gpu] non-finite rows d={d} k={k} path={path}")
        _, labels, best = ctx.run_pass(C, path=lib.PATHS[path], labels=True, best=True)
        assert np.array_equal(labels, ol), (path, np.flatnonzero(labels != ol)[:10])
        assert np.array_equal(best.view(np.uint32), ob.view(np.uint32)), path
    ctx.close()


def test_approx_on_the_widest_screen(lib):
    """exact=False at 1536 dims (unit rows, so the half-precision guard holds): best is the oracle's distance to the
    chosen label bit for bit and never below the exact best, the inertia is at least the exact one, labels disagree
    with exact mode on at most 10 % of rows, and the counts match the labels."""
    import oracle
    from mlx_kmeans import synthetic
    w = synthetic.embed_d1536(n=100_000, k=256)
    X, C0, k = w["X"], w["C0"], w["k"]
    ctx = lib.Context()
    ctx.set_parts([X])
    say("[gpu] exact=False at 1536 dims")
    te, le, be = ctx.run_pass(C0, mode=lib.KM_EXACT, labels=True, best=True)
    ta, la, ba = ctx.run_pass(C0, mode=lib.KM_APPROX, labels=True, best=True)
    assert ctx.last_path() == "mfma"
    assert np.array_equal(ba.view(np.uint32), oracle.distances_to(X, C0, la).view(np.uint32))
    assert np.all(ba >= be)
    assert float(ta[:, 1].sum()) >= float(te[:, 1].sum())
    dis = float(np.mean(la != le))
    say(f"[gpu]   approx label disagreement {dis:.4%}")
    assert dis <= 0.10
    assert np.array_equal(np.rint(ta[:, 0]).astype(np.int64), np.bincount(la, minlength=k))
    ctx.close()
