"""GPU: the per-centre bounds between passes (the reference's Elkan bounds, core.py:1690-2015).

A pass on the bounds scores exactly only the centres whose lower bound does not rule them out, then takes the rows
loop over them; its labels and best must be the rows loop's bit for bit, so a fit with the bounds must give the
same centres and inertia, bit for bit, as the same fit with them turned off (km_bounds(ctx, 0)), and must have run
passes on them where the reference's gate opens (at most 5 % of the (row, centre) pairs visited on a sample).
The shapes: well-separated blobs at 256 dims (k = 64, two slices) and 960 dims (k = 1024, GIST-like), rows that
are not finite (their bound is +inf: every centre, through the full scan), and the embedding workload's generator,
where the gate must stay shut.
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


def _blobs(seed, n, d, true_k, spread, noise, k):
    rng = np.random.default_rng(seed)
    cen = rng.uniform(-spread, spread, (true_k, d))
    X = (cen[rng.integers(0, true_k, n)] + rng.normal(0, noise, (n, d))).astype(np.float32)
    C = X[rng.choice(n, k, replace=False)].copy()
    return X, C


def _fit(lib, slices, C0, iters, max_visited):
    ctx = lib.Context()
    ctx.set_parts(slices)
    ctx.bounds(max_visited)
    C, inertia, it, _ = ctx.fit(C0, iters, -1.0)
    info = ctx.bounds_info()
    ctx.close()
    assert it == iters
    return C, inertia, info


@pytest.mark.parametrize("n,d,true_k,spread,k,parts,iters", [(100_003, 256, 40, 3.0, 64, 2, 15),
                                                             (60_000, 960, 50, 1.0, 1024, 1, 12),
                                                             (40_001, 512, 200, 2.0, 256, 3, 12)])
def test_fit_with_bounds_is_the_fit_without(lib, n, d, true_k, spread, k, parts, iters):
    X, C0 = _blobs(n + d + k, n, d, true_k, spread, 1.0, k)
    cuts = np.linspace(0, n, parts + 1).astype(int)
    slices = [X[cuts[i]:cuts[i + 1]] for i in range(parts)]
    say(f"[gpu] bounds fit n={n} d={d} k={k} parts={parts}: bounds off")
    C_off, in_off, info_off = _fit(lib, slices, C0, iters, 0.0)
    assert info_off["on_bounds"] == 0
    say(f"[gpu] bounds fit n={n} d={d} k={k} parts={parts}: bounds on")
    C_on, in_on, info = _fit(lib, slices, C0, iters, 0.05)
    say(f"[gpu]   {info}")
    assert info["on_bounds"] >= iters // 3, info
    assert np.array_equal(C_on.view(np.uint32), C_off.view(np.uint32))
    assert in_on == in_off


def test_lloyd_steps_on_bounds_match_the_oracle(lib):
    """Single steps through km_lloyd_step and km_pass keep the bounds between calls: every pass's labels and best
    against the oracle on a sample of rows (the whole pass against the bounds-off pass), with rows that are not
    finite among them."""
    import oracle
    X, C = _blobs(11, 30_011, 384, 60, 2.0, 1.0, 128)
    X[17] = np.nan
    X[29_999, 5] = np.inf
    rows = np.sort(np.random.default_rng(2).choice(len(X), 3000, replace=False))
    rows = np.union1d(rows, [17, 29_999])
    ctx, ref = lib.Context(), lib.Context()
    ctx.set_parts([X])
    ref.set_parts([X])
    ref.bounds(0.0)
    on = 0
    for step in range(10):
        say(f"[gpu] bounds steps: step {step}")
        before = ctx.bounds_info()["on_bounds"]
        tot, labels, best = ctx.run_pass(C, labels=True, best=True)
        tot0, labels0, best0 = ref.run_pass(C, labels=True, best=True)
        on += ctx.bounds_info()["on_bounds"] > before
        assert np.array_equal(labels, labels0), np.flatnonzero(labels != labels0)[:10]
        assert np.array_equal(best.view(np.uint32), best0.view(np.uint32))
        assert np.array_equal(tot.view(np.uint64), tot0.view(np.uint64))
        ol, ob = oracle.assign(X[rows], C)
        assert np.array_equal(labels[rows], ol)
        assert np.array_equal(best[rows].view(np.uint32), ob.view(np.uint32))
        C1, in1, _ = ctx.lloyd_step(C)
        C0, in0, _ = ref.lloyd_step(C)
        assert np.array_equal(C1.view(np.uint32), C0.view(np.uint32)) or not np.isfinite(in0)
        C = np.where(np.isfinite(C1), C1, C)      # the non-finite rows' cluster: keep its previous centre
    say(f"[gpu]   passes on the bounds: {on}, {ctx.bounds_info()}")
    assert on >= 3
    ctx.close()
    ref.close()


def test_gate_stays_shut_on_the_embedding_workload(lib):
    """200k rows of the 768-dim embedding workload (k = 1024, the k-means++ start): the sample says more than 5 %
    of the pairs would be visited at every pass, so no pass runs on the bounds and none builds them."""
    from mlx_kmeans import synthetic
    w = synthetic.embed_d768(n=200_000)
    ctx = lib.Context()
    ctx.set_parts([w["X"]])
    say("[gpu] embedding workload, 200k rows, 12 passes")
    ctx.fit(w["C0"], 12, -1.0)
    info = ctx.bounds_info()
    say(f"[gpu]   {info}")
    assert info["tracked"] == 12 and info["on_bounds"] == 0 and info["builds"] == 0, info
    ctx.close()
