"""Exact Lloyd k-means on AMD Instinct MI355X (gfx950): a drop-in for kakollu/mlx-kmeans's hot path.

    from mlx_kmeans import KMeans
    km = KMeans(n_clusters=64).fit(X)        # X: (rows, dims) float32
    km.cluster_centers_, km.labels_, km.inertia_

Every label is the centre with the smallest float32 distance sum((x - c)^2), lowest index on ties - the
reference's exact mode - computed by hand-written HIP kernels in libkmeans_hip.so (C ABI: include/kmeans_hip.h).
"""
from .core import (  # noqa: F401
    DeviceData, assign_mlx, kmeans, kmeans_pp_init, lloyd_fit, lloyd_step, make_data_numpy, slice_rows, take_rows,
)
from .core import _gpu_pass  # noqa: F401  (the reference exports it for tests and benchmarks)
from .estimator import KMeans  # noqa: F401

__version__ = "0.1.0"
__all__ = ["KMeans", "kmeans", "lloyd_step", "assign_mlx", "kmeans_pp_init", "lloyd_fit", "DeviceData"]
