"""python -m mlx_kmeans --rows N --dims D --k K: synthetic data, k-means++, Lloyd iterations (core.py:2247-2273)."""
import argparse

from . import core


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m mlx_kmeans")
    ap.add_argument("--rows", type=int, default=1_000_000)
    ap.add_argument("--dims", type=int, default=8)
    ap.add_argument("--k", type=int, default=16)
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--tol", type=float, default=1e-4)
    ap.add_argument("--seed", type=int, default=0)
    a = ap.parse_args(argv)
    parts = core.make_data_numpy(a.rows, a.dims, a.k, a.seed)
    C, inertia = core.kmeans(parts, a.rows, a.k, a.iters, a.tol, a.seed)
    print(f"final inertia {inertia:.6e}")


if __name__ == "__main__":
    main()
