"""Pins the CPU oracle (oracle/kmeans_oracle.c) before anything is checked against it.

Each check comes from a direction independent of the oracle's own formula:
  * the known answer of the reference's tests/test_files.py:67-79;
  * integer-valued data, where every float32 operation of the direct form is exact, so the labels must be the
    float64 argmin with the lowest index on ties and best the exact integer distance;
  * the reference's float64 criterion (tests/accuracy.py:31-51, 86-99) on random, near-tie, duplicate-centre and
    offset data;
  * closed-form float64 sums and counts (np.add.at / bincount);
  * the reference's own float64 Lloyd step with relocation (tests/accuracy.py:108-129) and scikit-learn's lloyd
    (tests/accuracy.py:159-164) for the update and empty-cluster rules;
  * planted mutants in the oracle (a '<=' tie rule, a dropped dimension, a sign error) that must fail these checks.
"""
import numpy as np
import pytest


def blobs(rng, n, d, true_k, spread, noise):
    centres = rng.uniform(-spread, spread, size=(true_k, d))
    return (centres[rng.integers(0, true_k, n)] + rng.normal(0, noise, (n, d))).astype(np.float32)


def test_known_answer_final_inertia(oracle):
    # tests/test_files.py:67-79: centres [[.5,0],[9.5,0]] on X = [[0,0],[1,0],[9,0],[10,0]] give inertia 1.0
    X = np.array([[0., 0.], [1., 0.], [9., 0.], [10., 0.]], np.float32)
    C = np.array([[.5, 0], [9.5, 0]], np.float32)
    tot, labels, best = oracle.one_pass(X, C)
    assert float(tot[:, 1].sum()) == 1.0
    assert labels.tolist() == [0, 0, 1, 1]
    assert np.array_equal(np.rint(tot[:, 0]), [2, 2])
    C_new, inertia, n_empty = oracle.update(tot, X, labels, best, C)
    assert inertia == 1.0 and n_empty == 0
    assert np.array_equal(C_new, C)


def _integer_case(rng, n=4000, d=6, k=24):
    X = rng.integers(-20, 21, size=(n, d)).astype(np.float32)
    C = rng.integers(-20, 21, size=(k, d)).astype(np.float32)
    C[1] = C[0] + np.array([2] + [0] * (d - 1), np.float32)   # equidistant rows between centres 0 and 1
    C[k // 2:] = C[:k // 2]                     # exact duplicate centres: every row has an exact tie
    X[:50] = C[0] + np.array([1] + [0] * (d - 1), np.float32)
    return X, C


def _exact_argmin(X, C):
    D = ((X.astype(np.float64)[:, None, :] - C.astype(np.float64)[None]) ** 2).sum(2)
    return D.argmin(1), D.min(1)                # np.argmin: lowest index among equal minima


@pytest.mark.parametrize("variant", [0, 1])
def test_integer_data_is_exact(oracle, variant):
    rng = np.random.default_rng(11)
    X, C = _integer_case(rng)
    labels, best = oracle.assign(X, C, variant=variant)
    ref_l, ref_d = _exact_argmin(X, C)
    assert np.array_equal(labels, ref_l)
    assert np.array_equal(best.astype(np.float64), ref_d)
    assert labels.max() < len(C) // 2           # ties with the duplicate half go to the lower index
    assert np.all(labels[:50] == 0)             # equidistant between 0 and 1: the lower index


@pytest.mark.parametrize("mutant", [2, 3, 4])
def test_mutants_fail_integer_check(oracle, mutant):
    rng = np.random.default_rng(11)
    X, C = _integer_case(rng)
    labels, best = oracle.assign(X, C, variant=mutant)
    ref_l, ref_d = _exact_argmin(X, C)
    assert not (np.array_equal(labels, ref_l) and np.array_equal(best.astype(np.float64), ref_d))


CASES = [
    # (name, generator) - shapes of tests/accuracy.py:254-292 at sizes the oracle finishes in a second
    ("separated d8 k16", lambda r: (lambda X: (X, X[r.choice(len(X), 16, replace=False)]))(blobs(r, 30_000, 8, 16, 10, 1))),
    ("overlapping d32 k256", lambda r: (lambda X: (X, X[r.choice(len(X), 256, replace=False)]))(blobs(r, 8_000, 32, 32, 1, 1))),
    ("offset +1000 d8 k64", lambda r: (lambda X: (X, X[r.choice(len(X), 64, replace=False)]))(
        (blobs(r, 20_000, 8, 16, 10, 1) + 1000).astype(np.float32))),
    ("high dims d256 k64", lambda r: (lambda X: (X, X[r.choice(len(X), 64, replace=False)]))(blobs(r, 3_000, 256, 20, 1, 1))),
]


@pytest.mark.parametrize("name,gen", CASES, ids=[c[0] for c in CASES])
def test_float64_criterion(oracle, name, gen):
    rng = np.random.default_rng(0)
    X, C = gen(rng)
    ref_c, ref_d = oracle.reference_f64(X, C)
    for variant in (0, 1):
        labels, best = oracle.assign(X, C, variant=variant)
        assert oracle.label_tolerance(X, C, labels, ref_d) == 0, (name, variant)
        # best is the float32 direct form of the chosen centre: within its error bound of the float64 distance
        X64, C64 = X.astype(np.float64), C.astype(np.float64)
        d_lab = ((X64 - C64[labels.astype(np.int64)]) ** 2).sum(1)
        g = (X.shape[1] + 2) * 2.0 ** -24 * 1.01
        assert np.all(np.abs(best - d_lab) <= g * d_lab + 1e-30)


def test_mutants_fail_float64_criterion(oracle):
    rng = np.random.default_rng(3)
    X = blobs(rng, 20_000, 8, 16, 10, 1)
    C = X[rng.choice(len(X), 16, replace=False)]
    _, ref_d = oracle.reference_f64(X, C)
    for mutant in (3, 4):
        labels, _ = oracle.assign(X, C, variant=mutant)
        assert oracle.label_tolerance(X, C, labels, ref_d) > 0


def test_duplicate_centres_lower_index(oracle):
    rng = np.random.default_rng(5)
    X = blobs(rng, 20_000, 8, 8, 10, 1)
    C = X[rng.choice(len(X), 32, replace=False)].copy()
    C[16:] = C[:16]
    labels, _ = oracle.assign(X, C)
    assert labels.max() < 16
    labels_m, _ = oracle.assign(X, C, variant=2)
    assert labels_m.min() >= 16                 # the '<=' mutant takes the higher duplicate


def test_totals_closed_form(oracle):
    rng = np.random.default_rng(1)
    X = blobs(rng, 50_000, 12, 10, 10, 1)
    C = X[rng.choice(len(X), 40, replace=False)]
    tot, labels, best = oracle.one_pass(X, C)
    lab = labels.astype(np.int64)
    counts = np.bincount(lab, minlength=len(C))
    sums = np.zeros((len(C), X.shape[1]))
    np.add.at(sums, lab, X.astype(np.float64))
    ib = np.zeros(len(C))
    np.add.at(ib, lab, best.astype(np.float64))
    assert np.array_equal(np.rint(tot[:, 0]).astype(np.int64), counts)
    np.testing.assert_allclose(tot[:, 2:], sums, rtol=1e-12, atol=1e-9)
    np.testing.assert_allclose(tot[:, 1], ib, rtol=1e-12, atol=1e-12)


def test_update_against_reference_step_multi_empty(oracle):
    # tests/accuracy.py:294-297: 8 far centres empty at once; pairing order matters
    rng = np.random.default_rng(0)
    X = blobs(rng, 60_000, 16, 8, 10, 1)
    C = np.concatenate([X[rng.choice(len(X), 24, replace=False)],
                        rng.uniform(900, 1000, (8, 16)).astype(np.float32)])
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    empties = 0
    for _ in range(4):
        C_new, inertia, n_empty, labels, best, tot = oracle.lloyd_step(X, C)
        ref, ref_empty = oracle.reference_lloyd_step(X, C, labels)
        assert n_empty == ref_empty
        assert np.max(np.abs(C_new.astype(np.float64) - ref)) / scale <= 1e-6
        empties += n_empty
        C = C_new
    assert empties >= 8


def test_update_against_scikit_learn_single_empty(oracle):
    # tests/accuracy.py:298-303 and 159-164: one cluster empties; scikit-learn's lloyd from the same start
    sk = pytest.importorskip("sklearn.cluster")
    rng = np.random.default_rng(2)
    X = blobs(rng, 40_000, 12, 16, 10, 1)
    C = np.concatenate([X[rng.choice(len(X), 31, replace=False)],
                        rng.uniform(900, 1000, (1, 12)).astype(np.float32)])
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    C_new, inertia, n_empty, labels, best, tot = oracle.lloyd_step(X, C)
    assert n_empty == 1
    ref = sk.KMeans(n_clusters=len(C), init=C, n_init=1, max_iter=1, tol=0.0, algorithm="lloyd").fit(X)
    err = float(np.max(np.abs(C_new.astype(np.float64) - ref.cluster_centers_))) / scale
    if err > 1e-5:      # a float32-level tie label may differ: then the inertia must agree (accuracy.py:161-163)
        a = float(oracle.one_pass(X, C_new)[0][:, 1].sum())
        b = float(oracle.one_pass(X, ref.cluster_centers_.astype(np.float32))[0][:, 1].sum())
        assert abs(a - b) / b <= 1e-6
    # and scikit-learn's reported inertia of the starting centres matches ours
    sk_inertia = float(((X.astype(np.float64) - C.astype(np.float64)[labels.astype(np.int64)]) ** 2).sum())
    assert abs(inertia - sk_inertia) / sk_inertia <= 1e-6


def test_still_empty_takes_largest_cluster(oracle):
    # every row sits on a centre (best == 0), so no relocation happens: the empty centre takes the largest's
    X = np.array([[0, 0]] * 5 + [[5, 5]] * 3, np.float32)
    C = np.array([[0, 0], [5, 5], [100, 100]], np.float32)
    C_new, inertia, n_empty, *_ = oracle.lloyd_step(X, C)
    assert n_empty == 1 and inertia == 0.0
    assert np.array_equal(C_new[2], C_new[0])


def test_cpu_pass_agrees_with_oracle(oracle):
    rng = np.random.default_rng(4)
    X = blobs(rng, 100_000, 8, 16, 10, 1)
    C = X[rng.choice(len(X), 16, replace=False)]
    tot = oracle.cpu_pass(X, C, nthreads=4)
    ref, _, _ = oracle.one_pass(X, C)
    assert np.array_equal(np.rint(tot[:, 0]), np.rint(ref[:, 0]))
    np.testing.assert_allclose(tot[:, 2:], ref[:, 2:], rtol=1e-4, atol=1e-2)
    assert abs(tot[:, 1].sum() - ref[:, 1].sum()) / ref[:, 1].sum() < 1e-5


def test_a1_and_fma_variants_differ_only_at_ties(oracle):
    rng = np.random.default_rng(6)
    X = blobs(rng, 20_000, 32, 32, 1, 1)        # heavy overlap: many near-ties
    C = X[rng.choice(len(X), 256, replace=False)]
    la, _ = oracle.assign(X, C, variant=0)
    lf, _ = oracle.assign(X, C, variant=1)
    flips = int((la != lf).sum())
    _, ref_d = oracle.reference_f64(X, C)
    assert oracle.label_tolerance(X, C, lf, ref_d) == 0
    assert flips < len(X) * 0.01


def test_label_distances_pinned(oracle):
    """distances_to (core.py:851-856) on integer-valued data, where every float32 step is exact: equal to the
    integer squared distance to the given (arbitrary) labels; and equal bit for bit to assign's best for assign's
    own labels on float data."""
    rng = np.random.default_rng(4)
    X = rng.integers(-50, 50, size=(3000, 24)).astype(np.float32)
    C = rng.integers(-50, 50, size=(37, 24)).astype(np.float32)
    lab = rng.integers(0, 37, size=3000).astype(np.uint32)
    want = ((X.astype(np.int64) - C[lab].astype(np.int64)) ** 2).sum(1)
    assert np.array_equal(oracle.distances_to(X, C, lab), want.astype(np.float32))
    Xf = rng.standard_normal((4000, 40)).astype(np.float32)
    Cf = Xf[rng.choice(4000, 50, replace=False)]
    labels, best = oracle.assign(Xf, Cf)
    assert np.array_equal(oracle.distances_to(Xf, Cf, labels).view(np.uint32), best.view(np.uint32))
    with pytest.raises(ValueError):
        oracle.distances_to(Xf, Cf, np.full(4000, 50, np.uint32))


def test_kmeans_simple_pass_pinned(oracle):
    """kmeans_simple.py:45-78 restated: on integer-valued rows around well-separated integer centres every float32
    step is exact (products, sums below 2^24 per chunk), so its expanded-form argmin is the rows loop's label and
    its totals are the closed form: counts = bincount(labels), sums = np.add.at in float64, error = the sum of the
    exact distances. A sign slip in the expanded form (|c|^2 + 2 x.c) gives other labels, which the same check
    catches."""
    rng = np.random.default_rng(12)
    k, d, n = 9, 6, 50_000
    C = (rng.integers(-4, 5, size=(k, d)) * 40).astype(np.float32)
    lab = rng.integers(0, k, n)
    X = (C[lab] + rng.integers(-3, 4, size=(n, d))).astype(np.float32)
    sums, counts, err = oracle.kmeans_simple_pass(X, C, chunk=7_919)
    ol, ob = oracle.assign(X, C)
    assert np.array_equal(ol, lab.astype(np.uint32))
    assert np.array_equal(counts, np.bincount(ol, minlength=k).astype(np.float64))
    ref = np.zeros((k, d))
    np.add.at(ref, ol, X.astype(np.float64))
    assert np.array_equal(sums, ref)
    assert err == float(ob.astype(np.float64).sum())
    wrong = (C * C).sum(1)[None, :] + 2 * (X @ C.T)
    assert not np.array_equal(wrong.argmin(1), ol)


def test_normalise_pinned(oracle):
    """Spherical renormalisation (estimator.py:127-130): within one float32 rounding of the float64 unit vector,
    a zero centre left at zero, and a centre already of unit length (a power-of-two axis vector) unchanged."""
    rng = np.random.default_rng(13)
    C = (rng.standard_normal((50, 33)) * rng.uniform(0.01, 100, (50, 1))).astype(np.float32)
    C[7] = 0.0
    C[8] = 0.0
    C[8, 5] = 1.0
    N = oracle.normalise(C)
    C64 = C.astype(np.float64)
    nrm = np.linalg.norm(C64, axis=1, keepdims=True)
    want = np.where(nrm > 0, C64 / np.where(nrm > 0, nrm, 1), 0.0)
    assert np.all(np.abs(N.astype(np.float64) - want) <= 4 * 2.0**-24 * np.maximum(np.abs(want), 2.0**-30))
    assert np.all(N[7] == 0.0) and np.array_equal(N[8], C[8])


def test_fit_from_stop_rule_hand_computed(oracle):
    """KMeans._one_run's loop (estimator.py:137-150) on five 1-D points worked by hand. From C0 = [0, 1] the steps
    report the inertia of their input centres: 302 ([0, 1] -> [0, 8.5]), 21.75 (-> [0.5, 11]), 2.5 (-> [0.5, 11]),
    2.5. The loop stops after the first step whose inertia is within tol * prev of the previous one, never after the
    first step (no previous inertia), and the returned inertia scores the returned centres (estimator.py:201-204)."""
    X = np.array([[0.], [1.], [10.], [11.], [12.]], np.float32)
    C0 = np.array([[0.], [1.]], np.float32)
    cases = [  # (max_iter, tol) -> (n_iter, centres, final inertia)
        ((50, 0.0), (4, [0.5, 11.0], 2.5)),       # 2.5 == 2.5 at step 4
        ((50, 0.9), (3, [0.5, 11.0], 2.5)),       # |21.75 - 2.5| = 19.25 <= 0.9 * 21.75 = 19.575
        ((50, 0.885), (4, [0.5, 11.0], 2.5)),     # 19.25 > 0.885 * 21.75 = 19.249: one more step
        ((50, 1e9), (2, [0.5, 11.0], 2.5)),       # step 1 has no previous inertia; step 2 stops
        ((1, 0.0), (1, [0.0, 8.5], 21.75)),       # max_iter: the centres of step 1, scored
        ((2, 0.0), (2, [0.5, 11.0], 2.5)),
    ]
    for (max_iter, tol), (n_iter, C_want, inertia_want) in cases:
        C, inertia, it, labels = oracle.fit_from(X, C0, max_iter=max_iter, tol=tol)
        assert it == n_iter, (max_iter, tol, it)
        assert C[:, 0].tolist() == C_want, (max_iter, tol, C)
        assert inertia == inertia_want, (max_iter, tol, inertia)
        assert labels.tolist() == [0, 0, 1, 1, 1]   # both [0, 8.5] and [0.5, 11] send 1 to centre 0


def test_fit_from_spherical_order_hand_computed(oracle):
    """spherical=True (estimator.py:134-135, 143-144): the starting centres are normalised, and every step's
    centres are normalised before the stop test. On X = [(1,0), (0,1), (1,1)] from C0 = [(2,0), (0,3)]: step 1
    with [(1,0), (0,1)] sends (1,1) to centre 0 on a tie (inertia 1), the new centre 0 is (1, 0.5) / |.|
    = (2, 1) / sqrt(5); step 2 reports 5 - 2 sqrt(5) and step 3 the same, so the loop stops after three steps.
    Without the per-step normalisation step 2 would report 0.5 and centre 0 would stay (1, 0.5)."""
    X = np.array([[1., 0.], [0., 1.], [1., 1.]], np.float32)
    C0 = np.array([[2., 0.], [0., 3.]], np.float32)
    C, inertia, it, labels = oracle.fit_from(X, C0, max_iter=50, tol=0.0, spherical=True)
    assert it == 3
    assert labels.tolist() == [0, 1, 0]
    c0 = np.array([2.0, 1.0]) / np.sqrt(5.0)
    assert np.allclose(C.astype(np.float64), [c0, [0.0, 1.0]], rtol=0, atol=2e-7)
    assert abs(inertia - (5 - 2 * np.sqrt(5.0))) <= 1e-6
    C, inertia, it, _ = oracle.fit_from(X, C0, max_iter=1, tol=0.0, spherical=True)
    assert it == 1 and np.allclose(C.astype(np.float64), [c0, [0.0, 1.0]], rtol=0, atol=2e-7)
