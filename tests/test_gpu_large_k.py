"""GPU: more than 4096 centres on the wide-row path (the regime the reference's cascade pruning serves,
core.py:1091-1260, and its tests/large_k.py: k = 65,536 on 1.2M rows x 128).

Above 4096 centres the screen's keys carry no centre index (the index travels beside each listed key) and the
counting sort keeps its counters in global memory; rows of 16 dims or fewer take the rows loop, whose sums then
come from the same counting sort. Labels and best must still be the rows loop's bit for bit:
checked against the oracle on every row at moderate sizes, and at the reference's large-k size on a row sample,
with best bit-identical to the oracle's direct form for every row and the totals against float64 sums of the
pass's own labels.
"""
import time

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


def _data(seed, n, d, k, true_k, parts=1):
    rng = np.random.default_rng(seed)
    cen = rng.standard_normal((true_k, d)).astype(np.float32) * 4
    X = ((cen[rng.integers(0, true_k, n)] + rng.standard_normal((n, d)).astype(np.float32))
         * np.linspace(4, 0.25, d).astype(np.float32)).astype(np.float32)
    C = X[rng.choice(n, k, replace=False)].copy()
    cuts = np.linspace(0, n, parts + 1).astype(int)
    return X, C, [X[cuts[i]:cuts[i + 1]] for i in range(parts)]


def _check_totals(tot, X, labels, best, k):
    counts = np.bincount(labels, minlength=k)
    assert np.array_equal(np.rint(tot[:, 0]).astype(np.int64), counts)
    X64 = X.astype(np.float64)
    sums = np.zeros((k, X.shape[1]))
    order = np.argsort(labels, kind="stable")
    ls = labels[order]
    starts = np.flatnonzero(np.r_[True, ls[1:] != ls[:-1]])
    sums[ls[starts]] = np.add.reduceat(X64[order], starts, axis=0)
    scale = float(np.sqrt((X64 ** 2).mean()))
    used = counts > 0
    err = np.max(np.abs(tot[used, 2:] - sums[used]) / counts[used, None]) / scale
    assert err <= 1e-6, err
    ri = float(best.astype(np.float64).sum())
    assert abs(float(tot[:, 1].sum()) - ri) <= 1e-6 * ri


@pytest.mark.parametrize("n,d,k,parts", [(50_000, 32, 5000, 1), (30_011, 100, 8192, 2), (20_000, 17, 6000, 1),
                                         (6_000, 768, 4100, 1), (100_003, 8, 6000, 2), (60_000, 3, 20_000, 1)])
def test_large_k_matches_the_oracle(lib, n, d, k, parts):
    import oracle
    X, C, slices = _data(n + d + k, n, d, k, max(k // 16, 8), parts)
    ctx = lib.Context()
    ctx.set_parts(slices)
    say(f"[gpu] large k: n={n} d={d} k={k} parts={parts}")
    tot, labels, best = ctx.run_pass(C, labels=True, best=True)
    assert ctx.last_path() == ("mfma" if d > 16 else "rows")
    ol, ob = oracle.assign(X, C)
    assert np.array_equal(labels, ol), np.flatnonzero(labels != ol)[:10]
    assert np.array_equal(best.view(np.uint32), ob.view(np.uint32))
    say(f"[gpu]   rows scored against every centre: {ctx.fallback_rows()}")
    _check_totals(tot, X, labels, best, k)
    C1, inertia, n_empty = ctx.lloyd_step(C)
    R1, r_in, r_empty, _, _, _ = oracle.lloyd_step(X, C)
    scale = float(np.sqrt((X.astype(np.float64) ** 2).mean()))
    assert n_empty == r_empty
    assert abs(inertia - r_in) <= 1e-6 * r_in
    assert float(np.max(np.abs(C1.astype(np.float64) - R1))) / scale <= 1e-6
    ctx.close()


def test_large_k_at_the_references_size(lib):
    """tests/large_k.py's shape: 1.2M x 128, k = 65,536 centres drawn from the rows of a 4096-blob mixture with
    columns scaled from 4 down to 0.25, in two slices."""
    import oracle
    n, d, k = 1_200_000, 128, 65_536
    X, C, slices = _data(1, n, d, k, 4096, 2)
    ctx = lib.Context()
    ctx.set_parts(slices)
    say(f"[gpu] large k at size: n={n} d={d} k={k}")
    ctx.run_pass(C)                     # builds the bf16 row operands once
    t0 = time.perf_counter()
    tot, labels, best = ctx.run_pass(C, labels=True, best=True)
    say(f"[gpu]   pass with per-row outputs {time.perf_counter() - t0:.3f} s, "
        f"rows scored against every centre: {ctx.fallback_rows()}")
    assert ctx.last_path() == "mfma"
    rng = np.random.default_rng(2)
    sample = np.sort(rng.choice(n, 1500, replace=False))
    ol, ob = oracle.assign(X[sample], C)
    assert np.array_equal(labels[sample], ol), sample[np.flatnonzero(labels[sample] != ol)[:10]]
    assert np.array_equal(best[sample].view(np.uint32), ob.view(np.uint32))
    assert np.array_equal(best.view(np.uint32), oracle.distances_to(X, C, labels).view(np.uint32))
    _check_totals(tot, X, labels, best, k)
    ctx.profile(True)
    _, _, n_iter, _ = ctx.fit(C, 3, -1.0)
    t = ctx.profile_passes()
    ctx.profile(False)
    say(f"[gpu]   fit passes (ms): {' '.join(f'{v:.1f}' for v in t)}")
    assert n_iter == 3
    ctx.close()


@pytest.mark.parametrize("k,d", [(1000, 64), (5000, 40)])
def test_overflow_rows_scan_every_centre_range(lib, k, d):
    """Rows whose window holds more than 16 centres of a half-row take the full scan, which above 256 centres splits
    the centres into ranges over many blocks and keeps, per row, the smallest distance and the lowest index among
    equal ones. Here 40 identical centres sit on one blob's mean (indices 300-339), so every row of that blob
    overflows and must take label 300; two rows are NaN (the rows loop gives them label 0 and best +inf)."""
    import oracle
    rng = np.random.default_rng(k + d)
    n = 20_000
    blobs = rng.uniform(-20, 20, (5, d)).astype(np.float32)
    X = (blobs[rng.integers(0, 5, n)] + 0.3 * rng.standard_normal((n, d))).astype(np.float32)
    X[[7, 12_345]] = np.nan
    C = rng.uniform(60, 90, (k, d)).astype(np.float32)
    C[300:340] = blobs[0]
    C[10:14] = blobs[1:5]
    ctx = lib.Context()
    ctx.set_parts([X])
    say(f"[gpu] overflow rows: n={n} d={d} k={k}")
    tot, labels, best = ctx.run_pass(C, labels=True, best=True)
    over = ctx.fallback_rows()
    say(f"[gpu]   rows scored against every centre: {over}")
    assert over >= 3000                  # the blob on the 40 copies: about a fifth of the rows
    ol, ob = oracle.assign(X, C)
    assert np.array_equal(labels, ol), np.flatnonzero(labels != ol)[:10]
    assert np.array_equal(best.view(np.uint32), ob.view(np.uint32))
    assert labels[7] == 0 and best[7] == np.inf
    assert (labels == 300).sum() > 3000
    ctx.close()
