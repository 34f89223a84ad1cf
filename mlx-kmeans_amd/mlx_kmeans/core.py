"""Exact Lloyd k-means on MI355X: the reference's core API (kakollu/mlx-kmeans, mlx_kmeans/core.py) over the
HIP engine in libkmeans_hip.so.

Same names, arguments and results as the reference's functions, so callers switch by changing nothing but the
install:
    lloyd_step(parts, C)                      core.py:2209-2242  -> (C_new f32, inertia, n_empty)
    assign_mlx(parts, C, return_labels=...)   core.py:2200-2206  -> (sums f64, counts i64, inertia[, labels i64])
    _gpu_pass(parts, C)                       core.py:2018-2197  -> (tot f64 (k, d+2), [(labels u32, best f32)])
    kmeans_pp_init(parts, rows, k, rng)       core.py:153-192    greedy k-means++ on a subsample, on the GPU
    make_data_numpy, slice_rows, take_rows    core.py:19-40, 131-143
    kmeans(parts, rows, k, max_iter, tol, seed)   core.py:2247-2273

`parts` is a list of 2-D float32 slices (or one array): numpy arrays are copied to the device for the call,
torch CUDA tensors are read in place, and a DeviceData keeps a copy on the device across calls (the role of the
reference's MLX arrays). Every pass runs on the GPU; there is no CPU path.
"""
import os
import time

import numpy as np

from . import _lib

SLICE_ROWS = 100_000_000                # rows per slice that KMeans cuts its input into
PART_MAX_ELEMENTS = 2**32 - 1           # elements per slice: the reference's limit (its kernels' uint32 offsets),
                                        # refused above it as the reference does (core.py:2028-2032)

# Per-centre bounds between passes (core.py:1690-2015): exact wide-row passes from 256 dims and 64 centres keep a
# lower bound per (row, centre) and run on them while a sample of 2048 rows says at most this fraction of the
# pairs needs scoring (the reference's BOUNDS_MAX_VISITED, core.py:516). Read at every pass; 0 turns them off.
BOUNDS_MAX_VISITED = 0.05

# the reference's `method` names -> this engine's paths. "rows" is the direct-form scan; the matrix-core screen
# plays the part of the reference's "tiles"/"tiles1"; the others are reference-internal variants that map onto
# the automatic choice. Every path returns the same labels.
_METHODS = {"auto": "auto", "rows": "rows", "pairs": "rows", "tiles": "mfma", "tiles1": "mfma", "mfma": "mfma",
            "onehot": "auto", "cascade": "auto", "approx": "auto"}


def _device():
    return int(os.environ.get("MLX_KMEANS_DEVICE", "0"))


def slice_rows(dims):
    """Rows per slice: at most SLICE_ROWS, and few enough that rows * dims fits PART_MAX_ELEMENTS."""
    return min(SLICE_ROWS, PART_MAX_ELEMENTS // dims)


# ---------------------------------------------------------------- data

def make_data_numpy(rows, dims, k, seed):
    """Points scattered around k hidden centres (uniform in [-10, 10]^dims) with unit normal noise, generated in
    10M-row chunks with one seeded numpy Generator -> [X] (the distribution of core.py:30-40)."""
    rng = np.random.default_rng(seed)
    centres = rng.uniform(-10, 10, size=(k, dims)).astype(np.float32)
    X = np.empty((rows, dims), dtype=np.float32)
    step = 10_000_000
    for a in range(0, rows, step):
        b = min(a + step, rows)
        lab = rng.integers(0, k, size=b - a)
        X[a:b] = centres[lab] + rng.standard_normal((b - a, dims), dtype=np.float32)
    return [X]


class DeviceData:
    """Data slices resident on the GPU, for repeated passes over the same data without copying it again."""

    def __init__(self, parts, device=None):
        parts = _as_list(parts)
        _validate_parts(parts)
        self.parts = parts
        self.ctx = _lib.Context(_device() if device is None else device)
        self.ctx.set_parts(parts)
        self.rows = self.ctx.rows
        self.dims = self.ctx.dims
        self.shape = (self.rows, self.dims)

    def close(self):
        self.ctx.close()


def _as_list(parts):
    if isinstance(parts, DeviceData):
        return parts
    if isinstance(parts, (list, tuple)):
        return list(parts)
    return [parts]


def _validate_parts(parts):
    for p in parts:
        if len(p.shape) != 2:
            raise ValueError(f"each part must be 2-D (rows, dims), got {len(p.shape)}-D")
    d = parts[0].shape[1]
    bad = [p.shape[1] for p in parts if p.shape[1] != d]
    if bad:
        raise ValueError(f"slices have {bad[0]} and {d} columns; every slice needs the same features")
    # one slice holds at most PART_MAX_ELEMENTS values, as in the reference (core.py:2028-2032); KMeans cuts its
    # input into slices of slice_rows(dims) rows itself
    big = [tuple(p.shape) for p in parts if int(p.shape[0]) * int(p.shape[1]) > PART_MAX_ELEMENTS]
    if big:
        raise ValueError(f"a slice of shape {big[0]} has more than {PART_MAX_ELEMENTS:,} elements, the limit of one "
                         f"slice (the reference addresses a slice with 32-bit offsets); pass the data as a list of "
                         f"slices of at most slice_rows(dims) = {slice_rows(d):,} rows (KMeans does this itself)")


def _context(parts, C, method="auto"):
    """-> (DeviceData, owned, kernel path) for parts, checking the centres against them (core.py:2022-2035
    wording) and the method, all before any device work."""
    dd = parts if isinstance(parts, DeviceData) else None
    if dd is None:
        parts = _as_list(parts)
        _validate_parts(parts)
    d = dd.dims if dd is not None else parts[0].shape[1]
    C = np.asarray(C)
    if C.ndim != 2 or C.shape[0] < 1:
        raise ValueError(f"centers must be a nonempty 2-D (k, dims) array, got shape {C.shape}")
    if C.shape[1] != d:
        raise ValueError(f"data has {d} columns but the centers have {C.shape[1]}; "
                         f"fit and predict need the same features")
    path = _path(method, C.shape[0], d)
    if dd is None:
        dd, owned = DeviceData(parts), True
    else:
        owned = False
    dd.ctx.bounds(BOUNDS_MAX_VISITED)
    return dd, owned, path


def _path(method, k, d):
    if method not in _METHODS:
        raise ValueError(f"method must be one of {sorted(_METHODS)}, got {method!r}")
    if method == "tiles" and (k % 8 or d % 8):
        raise ValueError(f"method='tiles' needs k and dims to be multiples of 8 (got k={k}, dims={d}); 'auto' picks "
                         f"it only where it applies")
    return _lib.PATHS[_METHODS[method]]


def _mode(method):
    return _lib.KM_APPROX if method == "approx" else _lib.KM_EXACT


def take_rows(parts, idx):
    """Gather global row indices from a list of slices -> float32 numpy array (core.py:131-143)."""
    if isinstance(parts, DeviceData):
        parts = parts.parts
    parts = _as_list(parts)
    idx = np.asarray(idx, dtype=np.int64)
    out = np.empty((len(idx), parts[0].shape[1]), dtype=np.float32)
    offset = 0
    for p in parts:
        m = (idx >= offset) & (idx < offset + p.shape[0])
        if m.any():
            local = idx[m] - offset
            if type(p).__module__.startswith("torch"):
                import torch
                out[m] = p[torch.as_tensor(local, device=p.device)].float().cpu().numpy()
            else:
                out[m] = np.asarray(p)[local]
        offset += p.shape[0]
    return out


# ---------------------------------------------------------------- init

def kmeans_pp_init(parts, rows, k, rng, sample=None):
    """Greedy k-means++ on a random sample of the rows, every round on the GPU (core.py:153-192).

    The sample is min(200k, max(20k, 20 k)) rows unless given, drawn without replacement and sorted; then the
    first pick and k - 1 per-round seeds are drawn from rng, in the reference's order, so one rng state gives one
    seeding. Round r draws 2 + floor(ln k) candidates with probability proportional to each row's squared distance
    to the nearest pick so far (a counter-based hash of the round's seed, the row and the trial; the reference's
    Gumbel-max draw) and keeps the one that lowers the summed squared distance the most. -> (k, dims) float32.
    """
    if k > rows:
        raise ValueError(f"n_samples={rows} should be >= n_clusters={k}.")
    dd = parts if isinstance(parts, DeviceData) else DeviceData(_as_list(parts))
    try:
        if sample is None:
            sample = min(200_000, max(20_000, 20 * k))
        idx = np.sort(rng.choice(rows, size=min(sample, rows), replace=False))
        first = int(rng.integers(len(idx)))
        seeds = rng.integers(2**63 - 1, size=k - 1).astype(np.uint64)
        return dd.ctx.seed_pp(k, idx, first, seeds)
    finally:
        if dd is not parts:
            dd.close()


# ---------------------------------------------------------------- passes

def _gpu_pass(parts, C, method="auto", accumulate="auto", iterate=False):
    """One exact assignment pass -> (float64 totals (k, d+2) [count, inertia, sums...], [(labels u32, best f32)]
    per slice). core.py:2018-2197. `accumulate` is accepted for compatibility: every accumulation here is
    deterministic and compensated. `iterate` is accepted and has no effect: a DeviceData keeps its per-centre
    bounds across every kind of pass (each pass's labels and best are the rows loop's either way)."""
    del accumulate, iterate
    dd, owned, path = _context(parts, C, method)
    try:
        C = np.ascontiguousarray(C, dtype=np.float32)
        tot, labels, best = dd.ctx.run_pass(C, _mode(method), path, labels=True, best=True)
        out, a = [], 0
        rows_per = [p.shape[0] for p in (dd.parts if isinstance(dd.parts, list) else [dd.parts])]
        for r in rows_per:
            out.append((labels[a:a + r], best[a:a + r]))
            a += r
        return tot, out
    finally:
        if owned:
            dd.close()


def assign_mlx(parts, C, method="auto", return_labels=False, accumulate="auto"):
    """One Lloyd pass on the GPU -> (per-cluster sums f64 (k, d), counts i64 (k,), inertia[, labels i64 (n,)]).
    core.py:2200-2206."""
    del accumulate
    dd, owned, path = _context(parts, C, method)
    try:
        C = np.ascontiguousarray(C, dtype=np.float32)
        tot, labels, _ = dd.ctx.run_pass(C, _mode(method), path, labels=return_labels, best=False)
        result = (tot[:, 2:], np.rint(tot[:, 0]).astype(np.int64), float(tot[:, 1].sum()))
        if return_labels:
            result += (labels.astype(np.int64),)
        return result
    finally:
        if owned:
            dd.close()


def lloyd_step(parts, C, method="auto", accumulate="auto"):
    """One exact Lloyd iteration on the GPU -> (new centres float32, inertia of C, number of empty clusters).

    core.py:2209-2242: empty clusters take the rows farthest from their centres (farthest to the lowest-numbered
    empty cluster, ties to the lower row index), which leave their old clusters; a cluster still empty takes the
    largest cluster's centre."""
    del accumulate
    dd, owned, path = _context(parts, C, method)
    try:
        C = np.ascontiguousarray(C, dtype=np.float32)
        return dd.ctx.lloyd_step(C, _mode(method), path)
    finally:
        if owned:
            dd.close()


def lloyd_fit(parts, C0, max_iter, tol=0.0, method="auto", spherical=False):
    """Up to max_iter Lloyd iterations from C0 with the stopping rule |prev - inertia| <= tol * prev, run back to
    back on the GPU (the loop of estimator.py:136-150) -> (C, last inertia, iterations, empties relocated)."""
    dd, owned, _ = _context(parts, C0, method)
    try:
        return dd.ctx.fit(np.ascontiguousarray(C0, dtype=np.float32), max_iter, tol, _mode(method), spherical)
    finally:
        if owned:
            dd.close()


# ---------------------------------------------------------------- driver

def kmeans(parts, rows, k, max_iter, tol, seed, backend="mlx"):
    """k-means++ then Lloyd iterations with per-iteration prints, then the final scoring pass (core.py:2247-2273).
    Only the GPU backend exists here."""
    if backend not in ("mlx", "gpu"):
        raise ValueError(f"backend {backend!r} is not offered: this engine runs on the GPU only")
    dd = parts if isinstance(parts, DeviceData) else DeviceData(parts)
    rng = np.random.default_rng(seed)
    C = kmeans_pp_init(dd, rows, k, rng)
    prev = None
    for it in range(1, max_iter + 1):
        t = time.perf_counter()
        newC, inertia, n_empty = lloyd_step(dd, C)
        shift = float(np.sqrt(((newC - C) ** 2).sum(1)).max())
        C = newC
        note = f"  ({n_empty} empty clusters relocated)" if n_empty else ""
        print(f"iter {it:3d}  inertia {inertia:.6e}  max_center_shift {shift:.5f}  {time.perf_counter() - t:.3f}s{note}")
        if prev is not None and abs(prev - inertia) <= tol * prev:
            break
        prev = inertia
    inertia = assign_mlx(dd, C)[2]
    return C, inertia
