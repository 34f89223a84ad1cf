"""GPU parity: the HIP engine against the CPU oracle, through the C ABI.

Labels and best distances must be bit-identical to the oracle's (the reference's exact mode, core.py:263-274)
on every kernel path; counts exact; sums within 1e-6 of the data's RMS per centre and inertia within 1e-6
relative (tests/accuracy.py:91-99); new centres within 1e-6 of the RMS (the same criterion) after each Lloyd
step. At full size, where the oracle cannot run every row, labels are checked on a random sample of rows and
the totals through identities that hold at any size.
"""
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
import make_golden as G  # noqa: E402

pytestmark = pytest.mark.gpu

CENTRE_TOL = 1e-6      # |centre - reference| / RMS(X)   (tests/accuracy.py:91-97)
INERTIA_TOL = 1e-6     # relative                      (tests/accuracy.py:98)


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def lib():
    from mlx_kmeans import _lib
    _lib.lib()
    return _lib


def mfma_served(d, k):
    """The fused screen serves d = 16, 24, 32 with k <= 128 and d = 40, 48, 56, 64 with k <= 64; the wide-row screen
    serves 16 < d <= 1536 with k <= 4096."""
    return (d in (16, 24, 32) and k <= 128 or d in (40, 48, 56, 64) and k <= 64
            or 16 < d <= 1536 and k <= 4096)


def fused_served(d, k):
    """The fused single-read path serves dims <= 16 with k * (dims + 2) <= 768 (its LDS tiles)."""
    return d <= 16 and k * (d + 2) <= 768


SERVED = {"rows": lambda d, k: True, "mfma": mfma_served, "fused": fused_served}


def check_totals(tot, X, labels, best, ref_tot, scale):
    k = tot.shape[0]
    counts = np.rint(tot[:, 0]).astype(np.int64)
    ref_counts = np.rint(ref_tot[:, 0]).astype(np.int64)
    assert np.array_equal(counts, ref_counts)
    used = ref_counts > 0
    err = np.max(np.abs(tot[used, 2:] - ref_tot[used, 2:]) / ref_counts[used, None]) / scale if used.any() else 0.0
    assert err <= CENTRE_TOL, err
    ri = float(ref_tot[:, 1].sum())
    assert abs(float(tot[:, 1].sum()) - ri) <= INERTIA_TOL * max(ri, 1e-30)
    assert k == ref_tot.shape[0]


@pytest.mark.parametrize("path", ["rows", "mfma", "fused"])
@pytest.mark.parametrize("name", G.CASES)
def test_pass_matches_oracle(lib, name, path):
    fx = np.load(G.fixture_path(name))
    parts, C0, steps = G.case_inputs(name)
    d, k = C0.shape[1], C0.shape[0]
    if not SERVED[path](d, k):
        pytest.skip(f"path {path} does not serve d={d} k={k}")
    X = np.concatenate(parts)
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean())) or 1.0
    ctx = lib.Context()
    ctx.set_parts(parts)
    C = fx["C0"]
    for s in range(steps):
        say(f"[gpu] pass {name} step {s} path={path} n={len(X)} d={d} k={k}")
        tot, labels, best = ctx.run_pass(C, path=lib.PATHS[path], labels=True, best=True)
        assert ctx.last_path() == path
        assert np.array_equal(labels, fx[f"labels_{s}"].astype(np.uint32)), f"labels differ at step {s}"
        assert np.array_equal(best.view(np.uint32), fx[f"best_{s}"].view(np.uint32)), f"best differs at step {s}"
        check_totals(tot, X, labels, best, fx[f"tot_{s}"], scale)
        # per-cluster best sums are exact on every path
        np.testing.assert_allclose(tot[:, 1], fx[f"tot_{s}"][:, 1], rtol=1e-6, atol=1e-30)
        C = fx[f"centres_{s + 1}"]
    ctx.close()


@pytest.mark.parametrize("name", G.CASES)
def test_lloyd_step_matches_oracle(lib, name):
    fx = np.load(G.fixture_path(name))
    parts, C0, steps = G.case_inputs(name)
    X = np.concatenate(parts)
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean())) or 1.0
    ctx = lib.Context()
    ctx.set_parts(parts)
    C = fx["C0"]
    for s in range(steps):
        say(f"[gpu] lloyd_step {name} step {s}")
        C_new, inertia, n_empty = ctx.lloyd_step(C)
        assert n_empty == int(fx[f"n_empty_{s}"])
        ri = float(fx[f"inertia_{s}"])
        assert abs(inertia - ri) <= INERTIA_TOL * max(ri, 1e-30)
        ref = fx[f"centres_{s + 1}"]
        err = float(np.max(np.abs(C_new.astype(np.float64) - ref.astype(np.float64)))) / scale
        assert err <= CENTRE_TOL, (s, err)
        C = ref            # continue from the oracle's centres so a float32 tie cannot compound
    ctx.close()


@pytest.mark.parametrize("name", ["blobs_d32", "outliers_d32", "lowd_d8", "relocation_d16_k32", "slices_d16_k100"])
def test_fit_loop_matches_oracle(lib, name):
    import oracle
    fx = np.load(G.fixture_path(name))
    parts, C0, steps = G.case_inputs(name)
    X = np.concatenate(parts)
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    ctx = lib.Context()
    ctx.set_parts(parts)
    say(f"[gpu] fit {name} iters={steps}")
    C, last_inertia, n_iter, n_rel = ctx.fit(fx["C0"], steps, 0.0)
    assert n_iter == steps
    assert n_rel == sum(int(fx[f"n_empty_{s}"]) for s in range(steps))
    ref = fx[f"centres_{steps}"]
    assert float(np.max(np.abs(C.astype(np.float64) - ref))) / scale <= 10 * CENTRE_TOL
    ri = float(fx[f"inertia_{steps - 1}"])
    assert abs(last_inertia - ri) <= 1e-5 * ri
    # the stopping rule: with a loose tol the loop stops early, and C is the centres after the stopping step
    ref_C, _, ref_iter, _ = oracle.fit_from(X, fx["C0"], max_iter=50, tol=1e-2)
    C2, _, it2, _ = ctx.fit(fx["C0"], 50, 1e-2)
    assert it2 == ref_iter
    assert float(np.max(np.abs(C2.astype(np.float64) - ref_C))) / scale <= 10 * CENTRE_TOL
    ctx.close()


@pytest.mark.parametrize("d,k", [(32, 64), (16, 64), (32, 32), (64, 32), (16, 32), (32, 40), (16, 8), (12, 20),
                                 (8, 8), (5, 33), (4, 12), (3, 7), (2, 64), (1, 5), (48, 100), (96, 33), (200, 64),
                                 (17, 5), (768, 40), (33, 300), (4, 32), (2, 48), (1, 70), (3, 40), (6, 27)])
def test_paths_are_bit_identical(lib, d, k):
    """Every path that serves a shape returns the rows path's labels and best bit for bit and the same counts;
    sums agree to the accumulation tolerance. 60,011 rows: a ragged tail for every block size."""
    rng = np.random.default_rng(5 + d * 1000 + k)
    n = 60_011
    X = (rng.uniform(-3, 3, size=(max(k // 4, 1), d))[rng.integers(0, max(k // 4, 1), n)]
         + rng.standard_normal((n, d))).astype(np.float32)
    C = X[rng.choice(len(X), k, replace=False)]
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    ctx = lib.Context()
    ctx.set_parts([X])
    say(f"[gpu] paths d={d} k={k}")
    t1, l1, b1 = ctx.run_pass(C, path=lib.KM_PATH_ROWS, labels=True, best=True)
    for name in ("mfma", "fused"):
        if not SERVED[name](d, k):
            continue
        t2, l2, b2 = ctx.run_pass(C, path=lib.PATHS[name], labels=True, best=True)
        assert ctx.last_path() == name
        assert np.array_equal(l1, l2) and np.array_equal(b1.view(np.uint32), b2.view(np.uint32)), name
        assert np.array_equal(np.rint(t1[:, 0]), np.rint(t2[:, 0])), name
        cnt = np.maximum(np.rint(t1[:, 0]), 1)[:, None]
        assert np.max(np.abs(t1[:, 2:] - t2[:, 2:]) / cnt) / scale <= CENTRE_TOL, name
        np.testing.assert_allclose(t2[:, 1], t1[:, 1], rtol=1e-6, atol=1e-30)
    ctx.close()


@pytest.mark.parametrize("d,k", [(48, 64), (48, 41), (48, 20), (64, 64), (64, 47), (32, 128), (32, 97),
                                 (16, 128), (16, 72), (24, 128), (24, 64), (24, 20), (40, 64), (40, 17), (56, 64),
                                 (56, 33)])
def test_fused_mfma_shapes_match_oracle(lib, d, k):
    """The fused matrix-core pass on the shapes of the reference's one-hot domain beyond 16-64 dims with 64
    centres (core.py:1639-1646: k a multiple of 8 up to 128, d up to 96): 24-, 40-, 48- and 56-dim rows (kept in
    order in LDS; 24, 40 and 56 padded to 32, 48 and 64 in the screen), 64 dims with up to 64 centres and 128
    centres at 16, 24 and 32 dims, over two uneven slices with duplicate centres and non-finite rows.
    Labels and best bit-identical to the oracle, counts exact, sums and inertia within tolerance, the fused
    kernel (not the wide-row screen) the one that ran, and a fit whose change-only passes match single steps."""
    import oracle
    rng = np.random.default_rng(900 + 7 * d + k)
    n = 70_001
    cen = rng.uniform(-3, 3, size=(max(k // 2, 2), d)).astype(np.float32)
    X = (cen[rng.integers(0, len(cen), n)] + 0.7 * rng.standard_normal((n, d))).astype(np.float32)
    C = X[rng.choice(n, k, replace=False)].copy()
    C[k - 1] = C[1]                               # duplicate centres: ties go to index 1
    X[100:110] = C[1]
    X[7] = np.nan
    X[8, d // 2] = np.inf
    parts = [X[:30_017], X[30_017:]]
    scale = float(np.sqrt((X[np.isfinite(X).all(1)].astype(np.float64) ** 2).mean()))
    ctx = lib.Context()
    ctx.set_parts(parts)
    say(f"[gpu] fused mfma shape d={d} k={k}")
    ctx.profile(True)
    tot, labels, best = ctx.run_pass(C, path=lib.KM_PATH_MFMA, labels=True, best=True)
    ran = ctx.profile_read()
    ctx.profile(False)
    assert "km_fused_mfma" in ran and "km_big_screen" not in ran, ran
    ol, ob = oracle.assign(X, C)
    assert np.array_equal(labels, ol), np.flatnonzero(labels != ol)[:10]
    assert np.array_equal(best.view(np.uint32), ob.view(np.uint32))
    assert np.array_equal(np.rint(tot[:, 0]).astype(np.int64), np.bincount(ol, minlength=k))
    ctx.close()
    fin = np.isfinite(X).all(1)
    # the fit loop on finite rows: change-only passes against one-at-a-time full steps
    Xf = X[fin]
    ctx = lib.Context()
    ctx.set_parts([Xf[:40_003], Xf[40_003:]] if d != 64 else [Xf])
    tot1, l1, b1 = ctx.run_pass(C, labels=True, best=True)
    check_totals(tot1, Xf, l1, b1, oracle.totals(Xf, *oracle.assign(Xf, C), k), scale)
    Cs = C.copy()
    for _ in range(6):
        Cs, _, _ = ctx.lloyd_step(Cs)
    Cf, inf, it, _ = ctx.fit(C, 6, -1.0)
    assert it == 6
    assert float(np.max(np.abs(Cf.astype(np.float64) - Cs))) / scale <= CENTRE_TOL
    # a second fit on the context: its change-only passes may take the kernel without candidate lists (chosen
    # from the open rows the first fit saw); the result is the first fit's, bit for bit
    Cg, ing, _, _ = ctx.fit(C, 6, -1.0)
    assert np.array_equal(Cg.view(np.uint32), Cf.view(np.uint32)) and ing == inf
    ctx.close()


@pytest.mark.parametrize("d,k", [(4, 32), (1, 70), (32, 64), (16, 32), (48, 100), (8, 76), (2, 150)])
def test_screen_edge_cases_match_the_rows_loop(lib, d, k):
    """The screened paths against the rows loop and the oracle on the cases a screen can get wrong: duplicate
    centres (exact ties, lowest index wins), rows equal to a centre (distance 0), NaN and infinite rows (label 0,
    best +inf or NaN as the rows loop leaves them), rows whose float32 distances overflow, and a zero row."""
    import oracle
    rng = np.random.default_rng(17 + d + k)
    n = 20_000
    cen = rng.uniform(-4, 4, size=(max(k // 3, 2), d)).astype(np.float32)
    X = (cen[rng.integers(0, len(cen), n)] + 0.5 * rng.standard_normal((n, d))).astype(np.float32)
    C = X[rng.choice(n, k, replace=False)].copy()
    C[5] = C[3]                                   # duplicate centres: ties go to index 3
    X[10:20] = C[3]                               # distance 0 to both duplicates
    X[20:30] = C[7]
    X[30] = np.nan
    X[31, 0] = np.inf
    X[32, -1] = -np.inf
    X[33] = 3.0e19                                # (x - c)^2 overflows for every centre
    X[34, 0] = 2.0e19
    X[35] = 0.0
    ctx = lib.Context()
    ctx.set_parts([X])
    say(f"[gpu] screen edge cases d={d} k={k}")
    t1, l1, b1 = ctx.run_pass(C, path=lib.KM_PATH_ROWS, labels=True, best=True)
    ol, ob = oracle.assign(X, C)
    assert np.array_equal(l1, ol) and np.array_equal(b1.view(np.uint32), ob.view(np.uint32))
    served = 0
    for name in ("mfma", "fused"):
        if not SERVED[name](d, k):
            continue
        served += 1
        t2, l2, b2 = ctx.run_pass(C, path=lib.PATHS[name], labels=True, best=True)
        assert ctx.last_path() == name
        assert np.array_equal(l1, l2), (name, np.flatnonzero(l1 != l2)[:10])
        assert np.array_equal(b1.view(np.uint32), b2.view(np.uint32)), name
    assert served
    ctx.close()


@pytest.mark.parametrize("d,k", [(3, 5), (2, 16), (4, 16), (16, 8), (2, 190), (8, 64), (12, 40), (16, 42)])
def test_fused_tile_layouts_match_oracle(lib, d, k):
    """The fused low-d path on both tile layouts (private columns at small k (d + 2), columns shared by four lanes
    where the private ones would cap occupancy) up to its largest k (d + 2) = 768, over two uneven slices:
    labels and best bit-identical to the oracle, counts exact, sums and inertia within tolerance, and a rerun
    bit-identical."""
    import oracle
    rng = np.random.default_rng(300 + 7 * d + k)
    n = 60_000
    cen = rng.uniform(-3, 3, size=(k, d)).astype(np.float32)
    X = (cen[rng.integers(0, k, n)] + 0.8 * rng.standard_normal((n, d))).astype(np.float32)
    C = X[rng.choice(n, k, replace=False)].copy()
    parts = [X[:20_011], X[20_011:]]
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    ctx = lib.Context()
    ctx.set_parts(parts)
    say(f"[gpu] fused tile layouts d={d} k={k}")
    tot, labels, best = ctx.run_pass(C, path=lib.KM_PATH_FUSED, labels=True, best=True)
    assert ctx.last_path() == "fused"
    ol, ob = oracle.assign(X, C)
    assert np.array_equal(labels, ol), np.flatnonzero(labels != ol)[:10]
    assert np.array_equal(best.view(np.uint32), ob.view(np.uint32))
    check_totals(tot, X, labels, best, oracle.totals(X, ol, ob, k), scale)
    t2, l2, b2 = ctx.run_pass(C, path=lib.KM_PATH_FUSED, labels=True, best=True)
    assert np.array_equal(t2.view(np.uint64), tot.view(np.uint64))
    ctx.close()


@pytest.mark.parametrize("d,k", [(48, 100), (96, 40)])
def test_wide_rows_over_slices(lib, d, k):
    """The wide-row path over three uneven slices: a pass with per-row outputs is the oracle's bit for bit; Lloyd
    steps without them (single-candidate rows unscored, multi-candidate rows listed per slice) match the oracle's
    centres, inertia and empty counts; three steps in a row keep matching."""
    import oracle
    rng = np.random.default_rng(41 + d + k)
    n = 50_000
    cen = rng.uniform(-2, 2, size=(k // 2, d)).astype(np.float32)
    X = (cen[rng.integers(0, len(cen), n)] + 0.7 * rng.standard_normal((n, d))).astype(np.float32)
    C = X[rng.choice(n, k, replace=False)].copy()
    parts = [X[:17_003], X[17_003:17_100], X[17_100:]]
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    ctx = lib.Context()
    ctx.set_parts(parts)
    say(f"[gpu] wide rows over slices d={d} k={k}")
    tot, labels, best = ctx.run_pass(C, labels=True, best=True)
    assert ctx.last_path() == "mfma"
    ol, ob = oracle.assign(X, C)
    assert np.array_equal(labels, ol) and np.array_equal(best.view(np.uint32), ob.view(np.uint32))
    for s in range(3):
        C_new, inertia, n_empty = ctx.lloyd_step(C)
        R_new, r_in, r_empty, _, _, _ = oracle.lloyd_step(X, C)
        assert n_empty == r_empty
        assert abs(inertia - r_in) <= INERTIA_TOL * r_in
        assert float(np.max(np.abs(C_new.astype(np.float64) - R_new.astype(np.float64)))) / scale <= CENTRE_TOL
        C = R_new
    ctx.close()


@pytest.mark.parametrize("name", ["outliers_d32", "lowd_d8", "pixels_d4"])
def test_reruns_are_bit_identical(lib, name):
    parts, C0, _ = G.case_inputs(name)
    ctx = lib.Context()
    ctx.set_parts(parts)
    say(f"[gpu] reruns {name}")
    a = ctx.run_pass(C0, labels=True, best=True)
    b = ctx.run_pass(C0, labels=True, best=True)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    f1 = ctx.fit(C0, 5, 0.0)
    f2 = ctx.fit(C0, 5, 0.0)
    assert np.array_equal(f1[0], f2[0]) and f1[1] == f2[1]
    ctx.close()


def test_estimator_known_answer_and_restarts():
    # tests/test_files.py:67-79
    from unittest.mock import patch
    from mlx_kmeans import KMeans
    X = np.array([[0., 0.], [1., 0.], [9., 0.], [10., 0.]], np.float32)
    say("[gpu] estimator known answer")
    fitted = KMeans(n_clusters=2, max_iter=1, random_state=3).fit(X)
    expected = np.min(((X[:, None] - fitted.cluster_centers_) ** 2).sum(2), axis=1).sum()
    assert abs(fitted.inertia_ - float(expected)) < 1e-5
    good = np.array([[.5, 0], [9.5, 0]], np.float32)
    bad = np.array([[0, 0], [1, 0]], np.float32)
    with patch.object(KMeans, '_one_run', side_effect=[(bad, 0., 1), (good, 999., 1)]):
        fitted = KMeans(n_clusters=2, n_init=2).fit(X)
    np.testing.assert_equal(fitted.cluster_centers_, good)
    assert abs(fitted.inertia_ - 1.0) < 1e-7
    assert fitted.labels_.dtype == np.int64 and fitted.labels_.tolist() == [0, 0, 1, 1]
    with pytest.raises(ValueError, match="features"):
        fitted.predict(np.zeros((3, 5), np.float32))


def test_estimator_exact_and_approx():
    """KMeans(exact=True) labels_ are the oracle's assignment to the returned centres, bit for bit, and inertia_ is
    the oracle's inertia of those labels; KMeans(exact=False) (estimator.py:18-30) fits the same data to nearly the
    same inertia (the reference quotes 0.003% more on GIST1M), and in both models predict(X) returns labels_."""
    import oracle
    from mlx_kmeans import KMeans
    rng = np.random.default_rng(5)
    n, d, k = 20_000, 256, 64
    cen = (3.0 * rng.standard_normal((k, d))).astype(np.float32)
    X = (cen[rng.integers(0, k, n)] + rng.standard_normal((n, d))).astype(np.float32)
    say("[gpu] estimator exact vs approx")
    ex = KMeans(n_clusters=k, max_iter=10, random_state=1).fit(X)
    ol, ob = oracle.assign(X, ex.cluster_centers_)
    assert np.array_equal(ex.labels_, ol.astype(np.int64))
    assert abs(ex.inertia_ - float(ob.astype(np.float64).sum())) <= 1e-5 * ex.inertia_
    ap = KMeans(n_clusters=k, max_iter=10, random_state=1, exact=False).fit(X)
    assert ap.inertia_ <= ex.inertia_ * (1 + 1e-3)
    for m in (ex, ap):
        assert np.array_equal(m.predict(X), m.labels_)


def test_estimator_nonfinite_is_explained():
    from mlx_kmeans import KMeans
    X = np.random.default_rng(0).standard_normal((1000, 4)).astype(np.float32)
    X[10, 2] = np.nan
    say("[gpu] estimator nan")
    with pytest.raises(ValueError, match="NaN or infinity"):
        KMeans(n_clusters=4, max_iter=3, random_state=0).fit(X)


def test_headline_workload_full_size(lib):
    """10M x 32, k=64 with 1% outliers: labels of a 200k-row sample bit-identical to the oracle's; counts sum to
    n; the per-cluster sums add up to the column sums of X; a rerun gives the same bits."""
    import oracle
    from mlx_kmeans import synthetic
    w = synthetic.outliers_d32()
    X, C0 = w["X"], w["C0"]
    n = len(X)
    ctx = lib.Context()
    ctx.set_parts([X])
    say(f"[gpu] headline full size n={n}")
    tot, labels, best = ctx.run_pass(C0, labels=True, best=True)
    assert ctx.last_path() == "mfma"
    rng = np.random.default_rng(1)
    idx = np.sort(rng.choice(n, 200_000, replace=False))
    ol, ob = oracle.assign(X[idx], C0)
    assert np.array_equal(labels[idx], ol)
    assert np.array_equal(best[idx].view(np.uint32), ob.view(np.uint32))
    assert int(np.rint(tot[:, 0]).sum()) == n
    colsum = X.astype(np.float64).sum(0)
    assert np.max(np.abs(tot[:, 2:].sum(0) - colsum)) <= 1e-6 * np.abs(X).sum(0).max()
    tot2, labels2, _ = ctx.run_pass(C0, labels=True)
    assert np.array_equal(tot, tot2) and np.array_equal(labels, labels2)
    # the fit loop's first iteration equals a pass + the oracle's update on the same labels
    C1, inertia, n_empty = ctx.lloyd_step(C0)
    C1_ref, inertia_ref, _ = oracle.update(oracle.totals(X, labels, best, 64), X, labels, best, C0)
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    assert float(np.max(np.abs(C1.astype(np.float64) - C1_ref))) / scale <= CENTRE_TOL
    assert abs(inertia - inertia_ref) <= INERTIA_TOL * inertia_ref
    ctx.close()


@pytest.mark.parametrize("name", ["lowd_d8", "pixels_d4"])
def test_lowd_workloads_full_size(lib, name):
    """10M x 8, k=8 and 96M x 4, k=12 at full size on the fused single-read path: labels and best of a
    200k-row sample bit-identical to the oracle's; counts sum to n; the per-cluster sums add up to the column
    sums of X and the best sums to the oracle's inertia of the sample scaled check; a rerun gives the same bits."""
    import oracle
    from mlx_kmeans import synthetic
    w = synthetic.WORKLOADS[name]()
    X, C0, k = w["X"], w["C0"], w["k"]
    n = len(X)
    ctx = lib.Context()
    ctx.set_parts([X])
    say(f"[gpu] {name} full size n={n}")
    tot, labels, best = ctx.run_pass(C0, labels=True, best=True)
    assert ctx.last_path() == "fused"
    rng = np.random.default_rng(2)
    idx = np.sort(rng.choice(n, 200_000, replace=False))
    ol, ob = oracle.assign(X[idx], C0)
    assert np.array_equal(labels[idx], ol)
    assert np.array_equal(best[idx].view(np.uint32), ob.view(np.uint32))
    counts = np.rint(tot[:, 0]).astype(np.int64)
    assert int(counts.sum()) == n
    assert np.array_equal(counts, np.bincount(labels, minlength=k))
    colsum = X.astype(np.float64).sum(0)
    assert np.max(np.abs(tot[:, 2:].sum(0) - colsum)) <= 1e-6 * np.abs(X).astype(np.float64).sum(0).max()
    bsum = np.bincount(labels, weights=best.astype(np.float64), minlength=k)
    np.testing.assert_allclose(tot[:, 1], bsum, rtol=1e-6)
    tot2, labels2, _ = ctx.run_pass(C0, labels=True)
    assert np.array_equal(tot, tot2) and np.array_equal(labels, labels2)
    ctx.close()


def test_approx_mode_properties(lib):
    """exact=False on wide rows (the reference's approximate path, core.py:1061-1088): labels come from the bf16
    screen's minimiser, best is the exact float32 direct-form distance to that label (bit-identical to the oracle's
    distance for the same label), so every row's best is >= its exact best and the inertia >= the exact inertia;
    labels agree with exact mode on nearly every row (the reference allows 10% disagreement, tests/reuse.py:61)."""
    import oracle
    rng = np.random.default_rng(11)
    n, d, k = 30_000, 256, 128
    cen = rng.standard_normal((k, d)).astype(np.float32)
    X = (cen[rng.integers(0, k, n)] + 0.3 * rng.standard_normal((n, d))).astype(np.float32)
    C = X[rng.choice(n, k, replace=False)]
    ctx = lib.Context()
    ctx.set_parts([X])
    say("[gpu] approx mode")
    te, le, be = ctx.run_pass(C, mode=lib.KM_EXACT, labels=True, best=True)
    ta, la, ba = ctx.run_pass(C, mode=lib.KM_APPROX, labels=True, best=True)
    assert ctx.last_path() == "mfma"
    ol, ob = oracle.assign(X, C)
    assert np.array_equal(le, ol) and np.array_equal(be.view(np.uint32), ob.view(np.uint32))
    db = oracle.distances_to(X, C, la)
    assert np.array_equal(ba.view(np.uint32), db.view(np.uint32))
    assert np.all(ba >= be)
    assert float(ta[:, 1].sum()) >= float(te[:, 1].sum())
    assert np.mean(la != le) <= 0.10
    assert int(np.rint(ta[:, 0]).sum()) == n
    ctx.close()


def test_embed_workload_full_size(lib):
    """1M x 768, k=1024 at full size on the wide-row screen: labels and best of a 3000-row sample bit-identical to
    the oracle's; counts sum to n and match the labels; per-cluster sums add up to the column sums of X; a rerun
    gives the same bits."""
    import oracle
    from mlx_kmeans import synthetic
    w = synthetic.embed_d768()
    X, C0, k = w["X"], w["C0"], w["k"]
    n = len(X)
    ctx = lib.Context()
    ctx.set_parts([X])
    say(f"[gpu] embed full size n={n}")
    tot, labels, best = ctx.run_pass(C0, labels=True, best=True)
    assert ctx.last_path() == "mfma"
    rng = np.random.default_rng(3)
    idx = np.sort(rng.choice(n, 3000, replace=False))
    ol, ob = oracle.assign(X[idx], C0)
    assert np.array_equal(labels[idx], ol)
    assert np.array_equal(best[idx].view(np.uint32), ob.view(np.uint32))
    counts = np.rint(tot[:, 0]).astype(np.int64)
    assert int(counts.sum()) == n
    assert np.array_equal(counts, np.bincount(labels, minlength=k))
    colsum = X.astype(np.float64).sum(0)
    assert np.max(np.abs(tot[:, 2:].sum(0) - colsum)) <= 1e-6 * np.abs(X).astype(np.float64).sum(0).max()
    bsum = np.bincount(labels, weights=best.astype(np.float64), minlength=k)
    np.testing.assert_allclose(tot[:, 1], bsum, rtol=1e-6)
    tot2, labels2, _ = ctx.run_pass(C0, labels=True)
    assert np.array_equal(tot, tot2) and np.array_equal(labels, labels2)
    ctx.close()


@pytest.mark.parametrize("n,d,k,path", [(200_003, 32, 64, "mfma"), (100_003, 128, 64, "wide")])
def test_fit_loop_totals_after_300_passes(lib, n, d, k, path):
    """KMeans' default max_iter is 300. On uniform data rows keep changing cluster for hundreds of passes (about
    150 of 200k per pass at pass 300), so the fit loop's change-only passes keep adding to the carried totals.
    The first 299 passes of a 300-pass fit are a 299-pass fit (reruns are bit-identical), so one full
    km_lloyd_step from the 299-pass fit's centres scores the same labels as the 300-pass fit's last pass: its
    centres must agree within 1e-6 of the RMS and its inertia within 1e-6 (the reference recomputes its sums
    every pass, core.py:2209-2242)."""
    rng = np.random.default_rng(300 + d)
    X = rng.random((n, d), dtype=np.float32)
    C0 = X[rng.choice(n, k, replace=False)].copy()
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    ctx = lib.Context()
    ctx.set_parts([X])
    say(f"[gpu] 300-pass fit n={n} d={d} k={k}")
    C300, in300, it300, _ = ctx.fit(C0, 300, -1.0)
    assert it300 == 300
    assert ctx.last_path() == "mfma"
    C299, _, it299, _ = ctx.fit(C0, 299, -1.0)
    assert it299 == 299
    _, lab_a, _ = ctx.run_pass(C299, labels=True)
    _, lab_b, _ = ctx.run_pass(ctx.lloyd_step(C299)[0], labels=True)
    say(f"[gpu]   rows changing cluster at pass 300: {int((lab_a != lab_b).sum())}")
    C_ref, in_ref, _ = ctx.lloyd_step(C299)
    err = float(np.max(np.abs(C300.astype(np.float64) - C_ref.astype(np.float64)))) / scale
    say(f"[gpu]   centre error {err:.2e}, inertia {in300:.9e} vs {in_ref:.9e}")
    assert err <= 1e-6
    assert abs(in300 - in_ref) <= 1e-6 * in_ref
    ctx.close()


@pytest.mark.parametrize("d,k,parts,path", [(32, 64, 1, "mfma"), (16, 40, 2, "mfma"), (64, 32, 1, "mfma"),
                                            (32, 20, 3, "mfma"), (16, 64, 1, "mfma"), (32, 128, 2, "mfma"),
                                            (24, 100, 1, "mfma"), (4, 12, 1, "fused"),
                                            (8, 8, 2, "fused"), (2, 40, 1, "fused"), (3, 30, 3, "fused"),
                                            (16, 8, 1, "fused"), (1, 200, 1, "fused"), (100, 100, 1, "wide"),
                                            (128, 300, 2, "wide"), (768, 64, 1, "wide"), (200, 40, 3, "wide")])
def test_fit_loop_change_accumulation_matches_full_steps(lib, d, k, parts, path):
    """The fit loop accumulates, after its first pass, only the rows whose label changed (into the new cluster, out of
    the old one) and adds that to the previous pass's totals. The same number of Lloyd steps run one at a time with
    a full accumulation each (km_lloyd_step) must reach the same centres (within 1e-6 of the RMS) and inertia
    (within 1e-6), with the same iteration count under a tolerance; reruns of the loop are bit-identical. The data
    keep rows moving between clusters for several passes (overlapping blobs, starting centres drawn from one
    corner). On the fused matrix-core path ("mfma") the loop accumulates only changed rows; on the fused low-d path
    ("fused", with and without the screen) it accumulates every row each pass, and must agree all the same. On the
    wide-row path ("wide", reported as "mfma") a pass takes the change-only sums when at most n/2 rows changed, and
    the full accumulation otherwise; its inertia then comes from the totals in centred form. The data make both
    happen within the passes. A change-only pass of the matrix-core path writes only the partials of the clusters
    its changed rows touched (a per-block mask of up to 128 clusters); 100 and 128 centres use every mask word."""
    rng = np.random.default_rng(900 + d + k + parts)
    n = 90_011
    cen = rng.uniform(-3, 3, size=(k, d)).astype(np.float32)
    X = (cen[rng.integers(0, k, n)] + 1.3 * rng.standard_normal((n, d))).astype(np.float32)
    order = np.argsort(X[:, 0])
    # wide shapes start from a tighter corner, so that early passes move more than half the rows (the full branch)
    C0 = X[order[rng.choice(n // 20 if path == "wide" else n // 3, k, replace=False)]].copy()
    cuts = np.linspace(0, n, parts + 1).astype(int)
    slices = [X[cuts[i]:cuts[i + 1]] for i in range(parts)]
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    ctx = lib.Context()
    ctx.set_parts(slices)
    steps = 12
    say(f"[gpu] change accumulation d={d} k={k} parts={parts}")
    C_fit, in_fit, it_fit, _ = ctx.fit(C0, steps, -1.0)
    assert it_fit == steps
    assert ctx.last_path() == ("mfma" if path == "wide" else path)
    C = C0
    moved = []
    prev_lab = None
    for s in range(steps):
        _, lab, _ = ctx.run_pass(C, labels=True)
        if prev_lab is not None:
            moved.append(int((lab != prev_lab).sum()))
        prev_lab = lab
        C, inertia, _ = ctx.lloyd_step(C)
    say(f"[gpu]   rows changing cluster per pass: {moved}")
    assert sum(moved[:3]) > 0, "the data should move rows between clusters"
    if path == "wide":
        limit = n // 2
        say(f"[gpu]   change-only limit {limit} rows")
        assert any(0 < m <= limit for m in moved), "some pass should take the change-only sums"
        assert any(m > limit for m in moved), "some pass should take the full accumulation"
    assert float(np.max(np.abs(C_fit.astype(np.float64) - C.astype(np.float64)))) / scale <= 1e-6
    assert abs(in_fit - inertia) <= 1e-6 * inertia
    C2, in2, _, _ = ctx.fit(C0, steps, -1.0)
    assert np.array_equal(C2, C_fit) and in2 == in_fit
    ref_C, _, ref_it, _ = __import__("oracle").fit_from(X, C0, max_iter=40, tol=1e-3)
    C3, _, it3, _ = ctx.fit(C0, 40, 1e-3)
    assert it3 == ref_it
    assert float(np.max(np.abs(C3.astype(np.float64) - ref_C))) / scale <= 1e-5
    ctx.close()
