"""GPU: empty-cluster relocation on the device (the reference's lloyd_step, core.py:2222-2242).

The empty clusters, ascending, take the rows with the largest best distance, lower row index first on ties; each
taken row leaves its old cluster; a cluster still empty takes the largest cluster's centre; with every row at
distance 0 nothing moves. Small cases are checked against the oracle's update (orc_update, pinned by
scikit-learn and tests/accuracy.py's restatement); the 96M-row case against the same rule applied in numpy to
the pass's own totals, labels and distances, bit for bit.
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


def _expected(tot, X, labels, best):
    """The relocation rule in numpy on a pass's float64 totals -> (centres float32, n_empty)."""
    k, w = tot.shape
    ws = tot.astype(np.float64).copy()
    counts = np.rint(ws[:, 0])
    empty = np.flatnonzero(counts == 0)
    if len(empty) and best.max() > 0:
        m = min(len(empty), len(X))
        key = np.where(best > 0, best, 0).astype(np.float64)
        cand = np.argpartition(-key, m - 1)[:m] if m < len(X) else np.arange(len(X))
        thr = key[cand].min()
        pool = np.flatnonzero(key >= thr)                       # every row that can be among the first m
        order = pool[np.lexsort((pool, -key[pool]))][:m]
        for nw, f in zip(empty, order):
            old = labels[f]
            ws[old, 2:] -= X[f].astype(np.float64)
            ws[old, 0] -= 1.0
            ws[nw, 2:] = X[f].astype(np.float64)
            ws[nw, 0] = 1.0
    cnt = np.rint(ws[:, 0])
    out = np.empty((k, w - 2), np.float32)
    has = cnt > 0
    out[has] = (ws[has, 2:] / cnt[has, None]).astype(np.float32)
    out[~has] = out[int(np.argmax(cnt))]
    return out, len(empty)


def _case(name):
    rng = np.random.default_rng(sum(map(ord, name)))
    if name == "ties_at_threshold":
        X = rng.uniform(0, 1, (50_000, 4)).astype(np.float32)
        far = [40_000, 3, 25_000, 7, 33_333, 11, 1_000, 2]        # identical rows: equal best distances
        X[far] = 5.0
        C = np.concatenate([X[rng.choice(988, 9, replace=False) + 12], np.full((3, 4), 100.0, np.float32)])
        return [X], C
    if name == "all_rows_at_distance_0":
        P = np.array([[0, 0, 0], [1, 2, 3], [-4, 5, 6]], np.float32)
        X = P[rng.integers(0, 3, 30_000)]
        return [X], np.concatenate([P, np.full((2, 3), 50.0, np.float32)])
    if name == "more_empties_than_far_rows":
        X = np.zeros((20_000, 6), np.float32)
        X[12_345] = 1.0
        return [X], np.concatenate([np.zeros((1, 6), np.float32), np.full((3, 6), 9.0, np.float32)])
    if name == "slices_d32":
        X = (rng.uniform(-3, 3, (16, 32))[rng.integers(0, 16, 60_001)]
             + rng.standard_normal((60_001, 32))).astype(np.float32)
        C = np.concatenate([X[rng.choice(len(X), 56, replace=False)], rng.uniform(500, 600, (8, 32)).astype(np.float32)])
        return [X[:20_000], X[20_000:41_000], X[41_000:]], C
    if name == "wide_d100":
        X = (rng.uniform(-2, 2, (8, 100))[rng.integers(0, 8, 30_011)]
             + rng.standard_normal((30_011, 100))).astype(np.float32)
        C = np.concatenate([X[rng.choice(len(X), 40, replace=False)], rng.uniform(90, 99, (5, 100)).astype(np.float32)])
        return [X], C
    raise KeyError(name)


@pytest.mark.parametrize("name", ["ties_at_threshold", "all_rows_at_distance_0", "more_empties_than_far_rows",
                                  "slices_d32", "wide_d100"])
def test_relocation_matches_the_oracle(lib, name):
    import oracle
    parts, C = _case(name)
    X = np.concatenate(parts)
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean())) or 1.0
    ctx = lib.Context()
    ctx.set_parts(parts)
    say(f"[gpu] relocation {name} n={len(X)} d={X.shape[1]} k={len(C)}")
    C1, inertia, n_empty = ctx.lloyd_step(C)
    R1, r_in, r_empty, ol, ob, _ = oracle.lloyd_step(X, C)
    assert n_empty == r_empty > 0
    assert abs(inertia - r_in) <= 1e-6 * max(r_in, 1e-30)
    assert float(np.max(np.abs(C1.astype(np.float64) - R1))) / scale <= 1e-6
    tot, labels, best = ctx.run_pass(C, labels=True, best=True)
    E1, e_empty = _expected(tot, X, labels, best)
    assert e_empty == n_empty
    assert np.array_equal(C1.view(np.uint32), E1.view(np.uint32))
    if name == "ties_at_threshold":   # the three lowest-indexed of the eight equal farthest rows, in row order
        assert np.array_equal(C1[9:], X[[2, 3, 7]])
    ctx.close()


def test_relocation_at_96m_rows(lib):
    """96M x 4 rows, k = 12 with three centres far from every row: each Lloyd step relocates three clusters onto
    the farthest rows - eight identical planted rows, spread over the array, of which the three lowest-indexed
    win. lloyd_step and the fit loop (two passes) against the rule applied to the pass's own outputs."""
    rng = np.random.default_rng(96)
    n = 96_000_000
    say(f"[gpu] relocation at scale: generating {n:,} x 4")
    X = rng.random((n, 4), dtype=np.float32)
    far = [95_000_000, 3, 50_000_000, 7, 77_000_000, 11, 1_000_000, 2]
    X[far] = 5.0
    C0 = np.concatenate([X[rng.choice(1_000_000, 9, replace=False) + 2_000_000], np.full((3, 4), 100.0, np.float32)])
    ctx = lib.Context()
    ctx.set_parts([X[: n // 2], X[n // 2:]])
    say("[gpu]   lloyd_step")
    C1, _, n_empty = ctx.lloyd_step(C0)
    assert n_empty == 3
    assert np.array_equal(C1[9:], X[[2, 3, 7]])
    tot, labels, best = ctx.run_pass(C0, labels=True, best=True)
    E1, _ = _expected(tot, X, labels, best)
    assert np.array_equal(C1.view(np.uint32), E1.view(np.uint32))
    say("[gpu]   fit, two passes")
    C2_step, _, _ = ctx.lloyd_step(C1)
    C2, _, n_iter, n_rel = ctx.fit(C0, 2, -1.0)
    assert n_iter == 2 and n_rel >= 3
    assert np.array_equal(C2.view(np.uint32), C2_step.view(np.uint32))
    ctx.close()
