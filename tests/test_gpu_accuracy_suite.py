"""GPU: the reference's accuracy suite (tests/accuracy.py:254-318) on its own inputs.

The suite draws every case from one default_rng(0) stream with its blob generator (accuracy.py:248-251); the
draws below are made in the same order with the same calls, so each case holds the rows and centres the
reference's run holds. Its bar (accuracy.py:86-99): no label worse than the float64 nearest centre by more than
float32 resolution, counts exact, centres within 1e-6 of the data's RMS, inertia within 1e-6. The bar here is
higher: labels and best equal the oracle's rows loop (core.py:263-274) bit for bit, on every path that serves the
shape. The relocation sequences (accuracy.py:294-303, 130-169) take eight Lloyd steps each, every step against
the float64 step (accuracy.py:108-129) on the step's own labels and, where one cluster empties, against
scikit-learn's lloyd. The bounds sequences (accuracy.py:305-318, 171-245) drive the per-centre bounds: the same
sequences of exact Lloyd steps (a restart at step 6, three slices, relocation, a column at 1e-6 scale), each step
held to the same bar, and, as the reference asserts (accuracy.py:209), at least a third of the steps run on the
bounds. The centres past float16 range (accuracy.py:218-245) are planted after five steps, with the gate at 0.5
as the reference sets it there, so that the pass runs on bounds a float16 cannot hold for that centre.
"""
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
from make_golden import _blobs as blobs  # noqa: E402  (the suite's generator, accuracy.py:248-251)

pytestmark = pytest.mark.gpu

CENTRE_TOL = 1e-6
INERTIA_TOL = 1e-6
SKLEARN_TOL = 1e-5


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def lib():
    from mlx_kmeans import _lib
    _lib.lib()
    return _lib


def _suite():
    """Every case of accuracy.py:main in its order: name -> dict(X, C, slice_rows, kind, ...)."""
    rng = np.random.default_rng(0)
    cases = {}

    def pick(X, m, pool=None):
        return X[rng.choice(len(X) if pool is None else pool, m, replace=False)]

    def put(name, X, C, kind="pass", **kw):
        cases[name] = dict(X=X, C=C, kind=kind, **kw)

    X = blobs(rng, 300_000, 8, 16, 10, 1)
    put("separated_d8_k16", X, pick(X, 16))
    X = blobs(rng, 300_000, 32, 32, 1, 1)
    put("overlapping_d32_k256", X, pick(X, 256))
    X = blobs(rng, 200_000, 16, 4, 10, 1)
    put("k_above_true_clusters_d16_k512", X, pick(X, 512))
    X = blobs(rng, 100_000, 8, 8, 10, 1)
    C = pick(X, 32)
    C[16:] = C[:16]
    put("duplicate_centres_d8_k32", X, C)
    X = np.repeat(blobs(rng, 5_000, 8, 8, 10, 1), 20, axis=0)
    put("duplicate_points_d8_k64", X, pick(X, 64))
    X = blobs(rng, 7, 3, 2, 10, 1)
    put("tiny_n7_d3_k5", X, X[:5].copy())
    X = (blobs(rng, 100_000, 8, 16, 10, 1) + 1000).astype(np.float32)
    put("offset_1000_d8_k64", X, pick(X, 64))
    X = rng.random((60_000, 128), dtype=np.float32) * 255
    put("uniform_255_d128_k1024", X, pick(X, 1024))
    X = blobs(rng, 120_000, 128, 64, 4, 1)
    X *= np.linspace(8.0, 0.05, 128).astype(np.float32)
    put("anisotropic_d128_k256", X, pick(X, 256))
    put("anisotropic_d128_k256_second_draw", X, pick(X, 256))
    X = blobs(rng, 20_000, 960, 50, 1, 1)
    put("high_dims_d960_k304", X, pick(X, 304))
    X = blobs(rng, 60_000, 64, 64, 1, 1)
    put("overlapping_d64_k256", X, pick(X, 256))
    X = np.concatenate([blobs(rng, 30_000, 64, 8, 10, 1), np.zeros((16, 64), np.float32)])
    put("zero_rows_tail_d64_k128", X[:30_009], pick(X, 128, pool=30_000))
    X = blobs(rng, 250_003, 16, 16, 5, 1)
    put("many_slices_d16_k100", X, pick(X, 100), slice_rows=60_001)
    X = (blobs(rng, 20_000_000, 2, 4, 10, 1) + 1000).astype(np.float32)
    put("accumulation_20m_offset_1000_d2_k4", X, pick(X, 4))
    X = blobs(rng, 200_000, 16, 8, 10, 1)
    put("relocation_8_empty_d16_k32", X,
        np.concatenate([pick(X, 24), rng.uniform(900, 1000, (8, 16)).astype(np.float32)]), kind="reloc")
    X = blobs(rng, 300_000, 50, 64, 10, 1)
    put("relocation_4_empty_d50_k64", X,
        np.concatenate([pick(X, 60), rng.uniform(900, 1000, (4, 50)).astype(np.float32)]), kind="reloc")
    X = blobs(rng, 200_000, 12, 16, 10, 1)
    put("relocation_1_empty_d12_k32", X,
        np.concatenate([pick(X, 31), rng.uniform(900, 1000, (1, 12)).astype(np.float32)]), kind="reloc",
        sklearn=True)
    X = blobs(rng, 60_000, 960, 50, 1, 1)
    C = pick(X, 1024)
    put("steps_d960_k1024_restart_at_6", X, C, kind="steps", steps=12, inject=(6, pick(X, 1024).copy()),
        sample=4_000, full_at=(0, 6, 11))
    X = blobs(rng, 50_000, 256, 40, 3, 1)
    put("steps_3_slices_d256_k64", X, pick(X, 64), kind="steps", steps=8, slice_rows=20_001)
    X = blobs(rng, 80_000, 256, 30, 10, 1)
    put("steps_relocation_d256_k64", X,
        np.concatenate([pick(X, 60), rng.uniform(900, 1000, (4, 256)).astype(np.float32)]), kind="steps", steps=8)
    X = blobs(rng, 60_000, 256, 40, 3, 1)
    X[:, 7] *= 1e-6
    put("steps_small_column_d256_k64", X, pick(X, 64), kind="steps", steps=8)
    X = blobs(rng, 40_000, 256, 30, 3, 1)
    put("centres_past_float16_d256_k64", X, pick(X, 64).copy(), kind="far")
    return cases


_CASES = None


def case(name):
    global _CASES
    if _CASES is None:
        _CASES = _suite()
    return _CASES[name]


PASS = ["separated_d8_k16", "overlapping_d32_k256", "k_above_true_clusters_d16_k512", "duplicate_centres_d8_k32",
        "duplicate_points_d8_k64", "tiny_n7_d3_k5", "offset_1000_d8_k64", "uniform_255_d128_k1024",
        "anisotropic_d128_k256", "anisotropic_d128_k256_second_draw", "high_dims_d960_k304", "overlapping_d64_k256",
        "zero_rows_tail_d64_k128", "many_slices_d16_k100", "accumulation_20m_offset_1000_d2_k4"]
RELOC = ["relocation_8_empty_d16_k32", "relocation_4_empty_d50_k64", "relocation_1_empty_d12_k32"]
STEPS = ["steps_d960_k1024_restart_at_6", "steps_3_slices_d256_k64", "steps_relocation_d256_k64",
         "steps_small_column_d256_k64"]


def served(path, d, k):
    if path == "mfma":    # the fused screen (d = 16, 32 with k <= 64; d = 64 with k <= 32) or the wide-row screen
        return d in (16, 32) and k <= 64 or d == 64 and k <= 32 or 16 < d <= 1536 and k <= 4096
    if path == "fused":   # the low-d single-read path: d <= 16, k (d + 2) <= 768
        return d <= 16 and k * (d + 2) <= 768
    return True


def _parts(X, slice_rows):
    if not slice_rows:
        return [X]
    return [X[s:s + slice_rows] for s in range(0, len(X), slice_rows)]


def _scale(X):
    return float(np.sqrt((X.astype(np.float64) ** 2).mean()))


def _check_labels(X, C, labels, best, rows=None):
    """Bit for bit the oracle's rows loop on the given rows (all rows when None)."""
    import oracle
    Xs = X if rows is None else X[rows]
    ol, ob = oracle.assign(Xs, C)
    lab = labels if rows is None else labels[rows]
    bst = best if rows is None else best[rows]
    assert np.array_equal(lab, ol), np.flatnonzero(lab != ol)[:10]
    assert np.array_equal(bst.view(np.uint32), ob.view(np.uint32))


def _check_suite_bar(X, C, labels, tot):
    """accuracy.py:86-99 on one pass: float64-optimal labels up to float32 resolution, counts exact, centres and
    inertia within 1e-6."""
    import oracle
    k = len(C)
    _, ref_d = oracle.reference_f64(X, C)
    assert oracle.label_tolerance(X, C, labels, ref_d) == 0
    X64, C64 = X.astype(np.float64), C.astype(np.float64)
    lab = labels.astype(np.int64)
    counts = np.bincount(lab, minlength=k)
    assert np.array_equal(np.rint(tot[:, 0]).astype(np.int64), counts)
    sums = np.zeros((k, X.shape[1]))
    order = np.argsort(lab, kind="stable")
    ls = lab[order]
    starts = np.flatnonzero(np.r_[True, ls[1:] != ls[:-1]])
    sums[ls[starts]] = np.add.reduceat(X64[order], starts, axis=0)
    used = counts > 0
    err = float(np.max(np.abs(tot[used, 2:] - sums[used]) / counts[used, None])) / _scale(X)
    assert err <= CENTRE_TOL, err
    ref_inertia = float(((X64 - C64[lab]) ** 2).sum())
    assert abs(float(tot[:, 1].sum()) - ref_inertia) <= INERTIA_TOL * max(ref_inertia, 1e-30)


@pytest.mark.parametrize("name", PASS)
def test_single_pass_cases(lib, name):
    c = case(name)
    X, C = c["X"], c["C"]
    n, d = X.shape
    k = len(C)
    ctx = lib.Context()
    ctx.set_parts(_parts(X, c.get("slice_rows")))
    ran = 0
    for path in ("auto", "rows", "mfma", "fused"):
        if not served(path, d, k):
            continue
        say(f"[gpu] accuracy suite {name}: {n} x {d}, k = {k}, path {path}")
        tot, labels, best = ctx.run_pass(C, path=lib.PATHS[path], labels=True, best=True)
        _check_labels(X, C, labels, best)
        if path == "auto":
            _check_suite_bar(X, C, labels, tot)
        else:   # every path's totals are the auto path's within the bar (its labels are the same bits)
            assert np.array_equal(np.rint(tot[:, 0]), np.rint(auto_tot[:, 0]))
            used = tot[:, 0] > 0
            err = np.max(np.abs(tot[used, 2:] - auto_tot[used, 2:]) / tot[used, :1]) / _scale(X)
            assert err <= 2 * CENTRE_TOL, (path, err)
        if path == "auto":
            auto_tot = tot
        ran += 1
    assert ran >= 2
    ctx.close()


def _steps(lib, X, C0, steps, slice_rows=None, inject=None, sample=None, full_at=None, sklearn=False):
    """Lloyd steps from C0; each step's labels bit for bit against the oracle (on `sample` seeded rows when given),
    its centres within 1e-6 of the float64 step on the same labels -> (empties relocated, steps whose Lloyd step ran
    on the per-centre bounds)."""
    import oracle
    ctx = lib.Context()
    ctx.set_parts(_parts(X, slice_rows))
    scale = _scale(X)
    rows = None
    if sample:
        rows = np.sort(np.random.default_rng(5).choice(len(X), sample, replace=False))
    C, empties, on_bounds = C0.copy(), 0, 0
    for step in range(steps):
        if inject is not None and step == inject[0]:
            C = inject[1]
        say(f"[gpu]   step {step}")
        tot, labels, best = ctx.run_pass(C, labels=True, best=True)
        _check_labels(X, C, labels, best, rows)
        if full_at is None or step in full_at:
            _check_suite_bar(X, C, labels, tot)
        before = ctx.bounds_info()["on_bounds"]
        ours, _, n_empty = ctx.lloyd_step(C)
        info = ctx.bounds_info()
        on_bounds += info["on_bounds"] > before
        say(f"[gpu]     bounds: {info}")
        ref, ref_empty = oracle.reference_lloyd_step(X, C, labels)
        assert n_empty == ref_empty
        err = float(np.max(np.abs(ours.astype(np.float64) - ref))) / scale
        assert err <= CENTRE_TOL, (step, err)
        if sklearn and n_empty:
            from sklearn.cluster import KMeans
            sk = KMeans(n_clusters=len(C), init=C, n_init=1, max_iter=1, tol=0.0, algorithm="lloyd").fit(X)
            e = float(np.max(np.abs(ours.astype(np.float64) - sk.cluster_centers_))) / scale
            if e > SKLEARN_TOL:   # a float32-level tie label: the inertias must agree (accuracy.py:159-164)
                a = float(ctx.run_pass(ours)[0][:, 1].sum())
                b = float(ctx.run_pass(sk.cluster_centers_.astype(np.float32))[0][:, 1].sum())
                assert abs(a - b) <= 1e-6 * b, (step, e)
        empties += n_empty
        C = ours
    ctx.close()
    return empties, on_bounds


@pytest.mark.parametrize("name", RELOC)
def test_relocation_sequences(lib, name):
    c = case(name)
    say(f"[gpu] accuracy suite {name}: {c['X'].shape}, k = {len(c['C'])}")
    empties, _ = _steps(lib, c["X"], c["C"], 8, sklearn=c.get("sklearn", False))
    assert empties > 0


@pytest.mark.parametrize("name", STEPS)
def test_step_sequences(lib, name):
    c = case(name)
    say(f"[gpu] accuracy suite {name}: {c['X'].shape}, k = {len(c['C'])}")
    _, on_bounds = _steps(lib, c["X"], c["C"], c["steps"], slice_rows=c.get("slice_rows"), inject=c.get("inject"),
                          sample=c.get("sample"), full_at=c.get("full_at"))
    say(f"[gpu]   Lloyd steps on the bounds: {on_bounds} of {c['steps']}")
    assert on_bounds >= c["steps"] // 3      # engaged, as accuracy.py:209 asks


def test_centres_past_float16(lib):
    """Two coordinates of one centre at 1e5 and 7e4 (past float16's 65504) after five Lloyd steps: every row's
    window must still hold its minimiser; labels and best bit for bit on every path, the suite's bar on auto."""
    c = case("centres_past_float16_d256_k64")
    X, C = c["X"], c["C"]
    ctx = lib.Context()
    ctx.set_parts([X])
    ctx.bounds(0.5)                      # the decision under test is the bounds', not the gate's (accuracy.py:230)
    for _ in range(5):
        C, _, _ = ctx.lloyd_step(C)
    C2 = C.copy()
    C2[0, 0] = 1e5
    C2[0, 1] = 7e4
    before = ctx.bounds_info()["on_bounds"]
    for path in ("auto", "mfma", "rows"):
        say(f"[gpu] accuracy suite centres past float16, path {path}")
        tot, labels, best = ctx.run_pass(C2, path=lib.PATHS[path], labels=True, best=True)
        _check_labels(X, C2, labels, best)
        if path == "auto":
            _check_suite_bar(X, C2, labels, tot)
            info = ctx.bounds_info()
            say(f"[gpu]   bounds: {info}")
            assert info["on_bounds"] > before, "the pass with the planted centre should run on the bounds"
    ctx.close()
