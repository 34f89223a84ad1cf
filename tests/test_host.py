"""Host-side logic that runs before any device call: argument checks with the reference's wording, the
benchmark's one-GPU contract and the synthetic workloads' shapes. No GPU and no HIP call needed."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


@pytest.mark.parametrize("kwargs,fragment", [
    (dict(n_clusters=0), "n_clusters must be a positive integer"),
    (dict(n_clusters=True), "n_clusters must be a positive integer"),
    (dict(n_init=0), "n_init must be a positive integer"),
    (dict(max_iter=-1), "max_iter must be a positive integer"),
    (dict(tol=-1e-3), "tol must be finite and nonnegative"),
    (dict(tol=float("nan")), "tol must be finite and nonnegative"),
    (dict(algorithm="emeans"), "emeans"),
    (dict(algorithm="elkan"), "algorithm must be"),
])
def test_estimator_parameter_errors(kwargs, fragment):
    from mlx_kmeans import KMeans
    with pytest.raises(ValueError, match=fragment):
        KMeans(**kwargs).fit(np.zeros((10, 2), np.float32))


def test_core_argument_errors():
    from mlx_kmeans import core
    X = np.zeros((20, 3), np.float32)
    with pytest.raises(ValueError, match="columns but the centers have"):
        core.lloyd_step([X], np.zeros((2, 4), np.float32))
    with pytest.raises(ValueError, match="nonempty 2-D"):
        core.lloyd_step([X], np.zeros((0, 3), np.float32))
    with pytest.raises(ValueError, match="must be 2-D"):
        core.lloyd_step([np.zeros(5, np.float32)], np.zeros((2, 1), np.float32))
    with pytest.raises(ValueError, match="every slice needs the same features"):
        core.lloyd_step([X, np.zeros((4, 2), np.float32)], np.zeros((2, 3), np.float32))
    with pytest.raises(ValueError, match="method must be one of"):
        core._path("bogus", 8, 8)
    with pytest.raises(ValueError, match="multiples of 8"):
        core._path("tiles", 12, 8)
    with pytest.raises(ValueError, match="should be >= n_clusters"):
        core.kmeans_pp_init([X], 20, 21, np.random.default_rng(0))
    with pytest.raises(ValueError, match="not offered"):
        core.kmeans([X], 20, 2, 5, 0.0, 0, backend="numpy")


def test_slice_element_limit(monkeypatch):
    """The reference's limit of one slice (tests/reuse.py:114-122): KMeans cuts an input over the limit into
    slices of slice_rows(dims) rows, and a single slice over it given to the core functions is refused with the
    reference's "32-bit" message before any device work."""
    from mlx_kmeans import KMeans, core
    monkeypatch.setattr(core, "PART_MAX_ELEMENTS", 1_000_000)
    parts = KMeans._parts(np.zeros((2500, 1000), np.float32))
    assert len(parts) == 3 and sum(len(p) for p in parts) == 2500
    big = [np.zeros((2500, 1000), np.float32)]
    C = np.zeros((8, 1000), np.float32)
    for call in (lambda: core.assign_mlx(big, C), lambda: core.lloyd_step(big, C), lambda: core._gpu_pass(big, C),
                 lambda: core.DeviceData(big)):
        with pytest.raises(ValueError, match="32-bit"):
            call()


def test_synthetic_workloads_small():
    from mlx_kmeans import synthetic
    w = synthetic.blobs_d32(n=3000)
    assert w["X"].shape == (3000, 32) and w["X"].dtype == np.float32 and w["C0"].shape == (64, 32)
    w2 = synthetic.blobs_d32(n=3000)
    assert np.array_equal(w["X"], w2["X"]) and np.array_equal(w["C0"], w2["C0"])   # seeded
    w = synthetic.lowd_d8(n=5000)
    assert w["X"].shape == (5000, 8) and w["k"] == 8
    # the start centres are rows of the data
    rows = {r.tobytes() for r in w["X"]}
    assert all(c.tobytes() in rows for c in w["C0"])


def test_input_checks_raise_before_the_device(monkeypatch):
    """The reference's reuse checks (tests/reuse.py:106-123) that need no GPU: a predict with another feature
    count and method='tiles' with k % 8 != 0 raise ValueError before any device work, and input over the
    per-slice element limit is cut into slices."""
    from mlx_kmeans import KMeans, core
    rng = np.random.default_rng(0)
    m = KMeans.from_centers(rng.standard_normal((8, 8)).astype(np.float32))
    with pytest.raises(ValueError, match="features"):
        m.predict(rng.standard_normal((300, 16)).astype(np.float32))
    X = rng.standard_normal((3000, 12)).astype(np.float32)
    with pytest.raises(ValueError, match="tiles"):
        core.assign_mlx([X], np.zeros((100, 12), np.float32), method="tiles")
    monkeypatch.setattr(core, "PART_MAX_ELEMENTS", 1_000_000)
    parts = KMeans._parts(np.zeros((2500, 1000), np.float32))
    assert len(parts) == 3 and sum(len(p) for p in parts) == 2500


def test_model_npz_format_loads_without_pickle(tmp_path):
    """The reference's file workflow saves model.npz as centers, mean, scale, columns (files.py:178-179); it loads
    with allow_pickle=False and its centres make a model through from_centers."""
    from mlx_kmeans import KMeans
    rng = np.random.default_rng(1)
    C = rng.standard_normal((5, 3)).astype(np.float32)
    np.savez(tmp_path / "model.npz", centers=C, mean=np.array([1.0, 2.0, 3.0]), scale=np.array([2.0, 1.0, 0.5]),
             columns=np.array(["spend", "visits", "age"]))
    z = np.load(tmp_path / "model.npz", allow_pickle=False)
    assert list(z["columns"]) == ["spend", "visits", "age"]
    m = KMeans.from_centers(z["centers"])
    assert m.n_clusters == 5 and np.array_equal(m.cluster_centers_, C)
    with pytest.raises(ValueError, match="NaN or infinity"):
        KMeans.from_centers(np.full((2, 3), np.nan, np.float32))
