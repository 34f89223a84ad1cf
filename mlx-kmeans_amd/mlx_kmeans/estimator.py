"""scikit-learn-shaped estimator over the MI355X engine: the reference's KMeans (kakollu/mlx-kmeans,
mlx_kmeans/estimator.py:7-230) with the same parameters, attributes and error messages."""
import numpy as np

from . import core


class KMeans:
    """Exact k-means on an AMD Instinct MI355X GPU.

        KMeans(n_clusters=64).fit(X).cluster_centers_

    Parameters keep the reference's meaning (estimator.py:52-65): n_clusters, n_init, max_iter, tol (relative
    change of the inertia), random_state, verbose, spherical, exact. Every label is the centre with the smallest
    float32 distance sum((x - c)^2), lowest index on ties, whichever kernel path runs; empty clusters are relocated
    as scikit-learn does. The Lloyd iterations of one run go back to back on the GPU, with no host round trip per
    iteration.

    accumulate is accepted for compatibility; every accumulation here is deterministic and compensated, so
    "atomic" (the reference's non-reproducible option) is served by the deterministic path. exact=False allows the
    approximate assignment (estimator.py:18-30): where the wide-row path serves the shape, the label is the bf16
    matrix-core screen's argmin taken on trust; elsewhere the exact kernels are also the fastest and run unchanged.
    best and the sums are exact for the label chosen either way.
    algorithm="emeans" is not part of this engine.

    X may be anything array-like (numpy, pandas, lists of rows), a torch tensor (CUDA tensors are read in
    place), a list of such slices, or a core.DeviceData.
    """

    def __init__(self, n_clusters=8, n_init=1, max_iter=300, tol=1e-4, random_state=None, verbose=False,
                 spherical=False, accumulate="auto", exact=True, algorithm="lloyd", epochs=3, batch_size=None):
        self.n_clusters = n_clusters
        self.n_init = n_init
        self.max_iter = max_iter
        self.tol = tol
        self.random_state = random_state
        self.verbose = verbose
        self.spherical = spherical
        self.accumulate = accumulate
        self.exact = exact
        self.algorithm = algorithm
        self.epochs = epochs
        self.batch_size = batch_size

    @property
    def _method(self):
        return "auto" if self.exact else "approx"

    @property
    def _mode(self):
        return core._mode(self._method)

    @classmethod
    def from_centers(cls, centers, **kwargs):
        """A fitted model from saved centres: KMeans.from_centers(np.load("centers.npy")) (estimator.py:71-79)."""
        centers = np.ascontiguousarray(centers, dtype=np.float32)
        if not np.isfinite(centers).all():
            raise ValueError("centers contain NaN or infinity")
        model = cls(n_clusters=len(centers), **kwargs)
        model.cluster_centers_ = centers
        return model

    @staticmethod
    def _peak(parts):
        """max |x| over all slices (NaN if any value is NaN, inf if any is infinite)."""
        peak = 0.0
        for p in (parts.parts if isinstance(parts, core.DeviceData) else parts):
            if type(p).__module__.startswith("torch"):
                import torch
                v = float(torch.max(torch.abs(p)).item()) if p.numel() else 0.0
                if torch.isnan(p).any():
                    v = float("nan")
            else:
                a = np.asarray(p)
                v = float(np.max(np.abs(a))) if a.size else 0.0
            if not np.isfinite(v):
                return v
            peak = max(peak, v)
        return peak

    @classmethod
    def _explain_nonfinite(cls, parts):
        """Say why a pass came back non-finite, then raise (estimator.py:81-106): NaN/inf in the data, or values
        so large that sum((x - c)^2) overflows float32 (the limit is sqrt(float32_max / (4 dims)))."""
        peak = cls._peak(parts)
        d = parts.dims if isinstance(parts, core.DeviceData) else parts[0].shape[1]
        if not np.isfinite(peak):
            raise ValueError(
                "input contains NaN or infinity, which would produce nan centers rather than an error. "
                "Drop or impute those rows first (the file workflow's missing='drop' does this).")
        limit = float(np.sqrt(np.finfo(np.float32).max / (4.0 * d)))
        if peak > limit:
            raise ValueError(
                f"largest coordinate is {peak:.3e}, above the {limit:.3e} this many dimensions allow: "
                f"a squared distance would overflow float32 and return nan. Standardise the features "
                f"(see the README) or rescale before fitting.")
        raise ValueError("clustering produced a non-finite result, but the input values look usable; "
                         "please report this with the data shape and dtype.")

    @staticmethod
    def _parts(X):
        """-> list of 2-D float32 slices of at most slice_rows(dims) rows (estimator.py:108-125)."""
        if isinstance(X, core.DeviceData):
            return X
        if isinstance(X, list) and X and hasattr(X[0], "shape") and len(X[0].shape) == 2:
            return X                                       # already slices
        if type(X).__module__.startswith("torch"):
            if X.dim() != 2 or not all(X.shape):
                raise ValueError(f"expected a nonempty 2-D (rows, dims) array, got shape {tuple(X.shape)}")
            per = core.slice_rows(X.shape[1])
            return [X] if len(X) <= per else [X[s:s + per] for s in range(0, len(X), per)]
        if not isinstance(X, np.ndarray):
            X = np.asarray(X.to_numpy() if hasattr(X, "to_numpy") else X)
        X = np.ascontiguousarray(X, dtype=np.float32)
        if X.ndim != 2 or not all(X.shape):
            raise ValueError(f"expected a nonempty 2-D (rows, dims) array, got shape {X.shape}")
        per = core.slice_rows(X.shape[1])
        return [X[s:s + per] for s in range(0, len(X), per)]

    @staticmethod
    def _normalise(C):
        n = np.linalg.norm(C, axis=1, keepdims=True)
        return (C / np.where(n > 0, n, 1)).astype(np.float32)

    def _check_params(self):
        for name in ['n_clusters', 'n_init', 'max_iter']:
            value = getattr(self, name)
            if isinstance(value, bool) or not isinstance(value, (int, np.integer)) or value < 1:
                raise ValueError(f'{name} must be a positive integer')
        if not np.isfinite(self.tol) or self.tol < 0:
            raise ValueError('tol must be finite and nonnegative')
        algorithm = getattr(self, "algorithm", "lloyd")
        if algorithm not in ("lloyd", "emeans"):
            raise ValueError(f"algorithm must be 'lloyd' or 'emeans', got {algorithm!r}")
        if algorithm == "emeans":
            raise ValueError("algorithm='emeans' is not part of this engine (it serves the exact Lloyd algorithm)")

    def _one_run(self, data, rows, seed):
        """k-means++ then the Lloyd loop (estimator.py:132-150) -> (centres, last inertia, iterations)."""
        rng = np.random.default_rng(seed)
        C = core.kmeans_pp_init(data, rows, self.n_clusters, rng)
        if self.verbose:
            if self.spherical:
                C = self._normalise(C)
            prev = None
            for it in range(self.max_iter):
                C, inertia, n_empty = data.ctx.lloyd_step(C, mode=self._mode)
                if not np.isfinite(inertia):
                    self._explain_nonfinite(data)
                if self.spherical:
                    C = self._normalise(C)
                print(f"iter {it + 1}: inertia {inertia:.6e}" + (f", {n_empty} empty relocated" if n_empty else ""))
                if prev is not None and abs(prev - inertia) <= self.tol * prev:
                    break
                prev = inertia
            return C, inertia, it + 1
        C, inertia, iters, _ = data.ctx.fit(C, self.max_iter, self.tol, mode=self._mode,
                                            spherical=self.spherical)
        if not np.isfinite(inertia):
            self._explain_nonfinite(data)
        return C, inertia, iters

    def fit(self, X, y=None):
        self._check_params()
        parts = self._parts(X)
        data = parts if isinstance(parts, core.DeviceData) else core.DeviceData(parts)
        try:
            rows = data.rows
            if rows < self.n_clusters:
                raise ValueError('n_clusters cannot exceed the number of rows')
            best = None
            for run in range(self.n_init):                 # restarts reuse the data already on the GPU
                seed = None if self.random_state is None else self.random_state + run
                C, inertia, iters = self._one_run(data, rows, seed)
                # a Lloyd step reports the inertia before its update: score the final centres (estimator.py:199-204)
                tot, labels, _ = data.ctx.run_pass(C, mode=self._mode, labels=True)
                inertia = float(tot[:, 1].sum())
                if not np.isfinite(inertia):
                    self._explain_nonfinite(data)
                if self.verbose and self.n_init > 1:
                    print(f"start {run + 1}/{self.n_init}: inertia {inertia:.6e} after {iters} iterations")
                if best is None or inertia < best[1]:
                    best = (C, inertia, iters, labels.astype(np.int64))
            self.cluster_centers_, self.inertia_, self.n_iter_, self.labels_ = best
        finally:
            if data is not parts:
                data.close()
        return self

    def predict(self, X):
        """Cluster index (int64) for every row of X (estimator.py:217-227)."""
        parts = self._parts(X)
        d = parts.dims if isinstance(parts, core.DeviceData) else parts[0].shape[1]
        if d != self.cluster_centers_.shape[1]:
            raise ValueError(f"X has {d} features but this model was fitted with "
                             f"{self.cluster_centers_.shape[1]}")
        data = parts if isinstance(parts, core.DeviceData) else core.DeviceData(parts)
        try:
            tot, labels, _ = data.ctx.run_pass(self.cluster_centers_, mode=self._mode, labels=True)
            if not np.isfinite(tot[:, 1].sum()):
                self._explain_nonfinite(data)
            return labels.astype(np.int64)
        finally:
            if data is not parts:
                data.close()

    def fit_predict(self, X, y=None):
        return self.fit(X).labels_
