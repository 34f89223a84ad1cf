"""Where the reference's per-centre (Elkan) bounds pay: the visited fraction per Lloyd pass, simulated on the CPU.

The reference keeps one lower bound per (row, centre) between Lloyd passes and uses them only while a pass would
visit at most BOUNDS_MAX_VISITED = 5 % of the n x k pairs (core.py:516, 2069-2084); a visited pair is one whose
lower bound, less its centre's drift since the bound was made, is below the row's exact distance to its own
centre (core.py:1690-1720). `simulate` runs the most favourable form of that scheme - exact bounds built from the
first pass, each pass's drifts subtracted, visited pairs refreshed exactly - and reports the visited fraction of
every pass. The reference's float16, round-down bounds and its float32 error slack only raise the fraction.

* On the reference's own bounds sequences (tests/accuracy.py:305-318: well-separated blobs, 60k x 960 with
  k = 1024, 50k x 256 and 80k x 256 with k = 64) the fraction falls to a few percent within a few passes: the gate
  opens there, and the engine's bounds path (tests/test_gpu_bounds.py, tests/test_gpu_accuracy_suite.py) runs
  those passes on the bounds.
* On the 1M x 768, k = 1024 embedding workload's generator (100,000 rows, the same cluster geometry and start) it
  stays above 5 % at every pass: near 100 % early, about 8.5 % at pass 20 (28 % on 200,000 rows). The gate stays
  shut and the pass screens every row, as the engine's gate decides on the device (tests/test_gpu_bounds.py).

The embedding passes also run the coarsest bound scheme, one lower bound per row (Hamerly's: the exact
second-smallest distance when the row was last scored in full, less the largest centre move of each pass since):
a row keeps its label without a screen when the exact distance to its own moved centre is below that bound. On
that data the second-best gap (median about 0.006) is an order of magnitude below the largest centre move (about
0.07), and at most about 1 % of the rows could skip the screen in any pass.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "mlx-kmeans_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

BOUNDS_MAX_VISITED = 0.05     # core.py:516


def _dist(X, xsq, C):
    """Squared distances in the expanded form (float32 GEMM), clamped at 0."""
    csq = (C.astype(np.float64) ** 2).sum(1).astype(np.float32)
    D = X @ C.T
    D *= -2.0
    D += xsq[:, None]
    D += csq[None, :]
    np.maximum(D, 0.0, out=D)
    return D


def _means(X, lab, C):
    order = np.argsort(lab, kind="stable")
    ls = lab[order]
    starts = np.flatnonzero(np.r_[True, ls[1:] != ls[:-1]])
    S = np.add.reduceat(X[order], starts, axis=0, dtype=np.float64)
    out = C.copy()
    ids = ls[starts]
    out[ids] = (S / np.diff(np.r_[starts, len(ls)])[:, None]).astype(np.float32)
    return out


def simulate(X, C, passes):
    """-> (per-pass fraction of (row, centre) pairs the per-centre bounds visit, per-pass fraction of rows the
    per-row bound lets skip the screen) over `passes` Lloyd passes from the centres C."""
    X, C = X.astype(np.float32), C.astype(np.float32)
    n = len(X)
    k = len(C)
    xsq = (X.astype(np.float64) ** 2).sum(1).astype(np.float32)
    rows = np.arange(n)
    D = _dist(X, xsq, C)
    lab = D.argmin(1)
    lb = np.sqrt(D)                      # bounds built from the first pass's exact distances
    hl = np.sqrt(np.partition(D, 1, axis=1)[:, 1])   # per-row bound: the second-smallest distance
    out, skips = [], []
    for _ in range(passes):
        Cn = _means(X, lab, C)
        drift = np.sqrt(((Cn.astype(np.float64) - C) ** 2).sum(1)).astype(np.float32)
        C = Cn
        lb -= drift[None, :]
        np.maximum(lb, 0.0, out=lb)
        D = _dist(X, xsq, C)
        ub = np.sqrt(D[rows, lab])
        hl -= drift.max()
        skip = ub < hl                   # no other centre can be nearer: the row keeps its label unscreened
        assert np.all(D[rows, lab][skip] <= D[skip].min(1))
        skips.append(float(skip.mean()))
        hl = np.where(skip, hl, np.sqrt(np.partition(D, 1, axis=1)[:, 1]))
        visit = lb < ub[:, None]
        visit[rows, lab] = False
        out.append(float(visit.sum()) / (n * k))
        np.sqrt(D, out=lb, where=visit)  # visited pairs are computed exactly: their bounds become exact
        lab = D.argmin(1)
    return out, skips


def _blobs(rng, n, d, true_k, spread, noise):
    """the accuracy suite's blob generator (tests/accuracy.py, its `blobs`)"""
    centres = rng.uniform(-spread, spread, size=(true_k, d))
    return (centres[rng.integers(0, true_k, n)] + rng.normal(0, noise, (n, d))).astype(np.float32)


def test_bounds_gate_opens_on_the_reference_bounds_sequences():
    """accuracy.py:305-318's three shapes, each from random rows as the start (the suite's relocation case plants
    four far centres among them, which empties them at the first pass; left out here, since the simulation has no
    relocation). The suite asks the bounds path to run at least a third of the steps (accuracy.py:209)."""
    rng = np.random.default_rng(0)
    for name, (n, d, true_k, spread, k, passes) in {"d960 k1024": (60_000, 960, 50, 1.0, 1024, 12),
                                                      "d256 k64 spread 3": (50_000, 256, 40, 3.0, 64, 8),
                                                      "d256 k64 spread 10": (80_000, 256, 30, 10.0, 64, 8)}.items():
        X = _blobs(rng, n, d, true_k, spread, 1.0)
        fr, _ = simulate(X, X[rng.choice(n, k, replace=False)], passes)
        print(f"{name}: visited fraction per pass:", " ".join(f"{f:.4f}" for f in fr))
        assert sum(f <= BOUNDS_MAX_VISITED for f in fr) >= passes // 3, (name, fr)


def test_bounds_gate_never_opens_on_the_embedding_workload():
    from mlx_kmeans import synthetic
    w = synthetic.embed_d768(n=100_000)
    fr, sk = simulate(w["X"], w["C0"], 20)
    print("visited fraction per pass:", " ".join(f"{f:.3f}" for f in fr))
    print("rows a per-row bound lets skip, per pass:", " ".join(f"{f:.4f}" for f in sk))
    assert len(fr) == 20
    assert min(fr) > BOUNDS_MAX_VISITED, fr
    assert fr[0] > 0.9                   # right after the first pass nearly every pair is visited
    assert max(sk) < 0.02, sk
