"""Seeded synthetic workloads for the Lloyd pass, generated with numpy (default_rng, PCG64), float32 output.

    blobs_d32      100k x 32, k=64: 64-component isotropic Gaussian mixture, means ~U[-10,10]^32, sigma 1,
                   equal weights; start: greedy k-means++ on a 10k-row subsample; 20 iterations
    lowd_d8        10M x 8, k=8: 8-component mixture, means ~U[-5,5]^8, per-component diagonal sigma ~U[0.5,2];
                   start: 8 seeded distinct rows; 25 iterations
    outliers_d32   10M x 32, k=64: blobs_d32's mixture plus 1% of rows replaced by U[-20,20]^32 outliers;
                   start: k-means++ on a 10k-row subsample; 20 iterations   (the headline workload)
    pixels_d4      96M x 4, k=12: 12 classes, means ~U[0,1]^4, Dirichlet(0.5) class weights, correlated noise
                   Sigma_c = 0.02^2 (A A^T / 4 + I / 4), A ~ N(0,1)^{4x4}, clipped to [0,1]; start: 12 seeded
                   rows; 30 iterations
    embed_d768     1M x 768, k=1024: unit rows normalize(centre + N(0, 0.15^2 I)) around 1024 random unit
                   centres; start: 1024 seeded rows; 15 iterations
    embed_d1536    the same at 1536 dims (the widest rows the matrix-core screen takes)
    blobs_d48      10M x 48, k=64 \
    blobs_d32_k128 10M x 32, k=128 } blobs_d32's mixture (means ~U[-10,10]^d, sigma 1, one component per centre) at
    blobs_d96      10M x 96, k=64 /  the widths and centre counts of the reference's one-hot domain (core.py:1639-1646;
                   d = 96 with k = 64 lies past its k (d / 8 + 1) <= 640); start: k-means++ on a 10k-row subsample;
                   20 iterations
    blobs_d960     1M x 960, k=1024: GIST-like width, 1024-component isotropic mixture, means ~U[-1,1]^960, sigma 1
                   (the reference's bounds sequence, tests/accuracy.py:305-306, at 1M rows and one blob per
                   centre); start: greedy k-means++ on a 20,480-row subsample; 20 iterations. Well separated: the
                   per-centre bounds between passes take over once the fit settles.

Every generator takes n (rows) so tests can draw the same distribution at smaller sizes.
"""
import numpy as np

from .core import take_rows


def kmeans_pp_init(parts, rows, k, rng, sample=None):
    """Start centres of the synthetic workloads: greedy k-means++ on the host in float64 (the algorithm of
    core.py:153-192 with numpy's random stream), kept as it was so that each workload's start stays the same."""
    if sample is None:
        sample = min(200_000, max(20_000, 20 * k))
    idx = np.sort(rng.choice(rows, size=min(sample, rows), replace=False))
    S = take_rows(parts, idx).astype(np.float64)
    m = len(S)
    trials = 2 + int(np.log(k)) if k > 1 else 1
    ssq = (S * S).sum(1)
    first = int(rng.integers(m))
    picks = [first]
    d2 = np.maximum(ssq + ssq[first] - 2.0 * (S @ S[first]), 0.0)
    for _ in range(k - 1):
        total = d2.sum()
        if total > 0:
            cand = rng.choice(m, size=trials, p=d2 / total)
        else:
            cand = rng.integers(m, size=trials)
        dist = np.maximum(ssq[None, :] + ssq[cand][:, None] - 2.0 * (S[cand] @ S.T), 0.0)
        mins = np.minimum(d2[None, :], dist)
        b = int(np.argmin(mins.sum(1)))
        d2 = mins[b]
        picks.append(int(cand[b]))
    return S[picks].astype(np.float32)

CHUNK = 4_000_000


def _blobs(rng, n, d, k, spread, X=None):
    means = rng.uniform(-spread, spread, size=(k, d)).astype(np.float32)
    if X is None:
        X = np.empty((n, d), np.float32)
    for a in range(0, n, CHUNK):
        b = min(n, a + CHUNK)
        lab = rng.integers(0, k, size=b - a)
        X[a:b] = means[lab] + rng.standard_normal((b - a, d), dtype=np.float32)
    return X


def _distinct_rows(rng, X, k):
    """k seeded rows of X with distinct values (start centres that cannot tie)."""
    picks = []
    seen = set()
    while len(picks) < k:
        for i in rng.choice(len(X), size=4 * k, replace=False):
            key = X[i].tobytes()
            if key not in seen:
                seen.add(key)
                picks.append(i)
                if len(picks) == k:
                    break
    return X[np.array(picks)].copy()


def blobs_d32(n=100_000, seed=0):
    rng = np.random.default_rng(seed)
    X = _blobs(rng, n, 32, 64, 10.0)
    C0 = kmeans_pp_init([X], n, 64, rng, sample=10_000)
    return dict(name="blobs_d32", X=X, C0=C0, k=64, iters=20)


def lowd_d8(n=10_000_000, seed=0):
    rng = np.random.default_rng(seed)
    k, d = 8, 8
    means = rng.uniform(-5, 5, size=(k, d)).astype(np.float32)
    sig = rng.uniform(0.5, 2.0, size=(k, d)).astype(np.float32)
    X = np.empty((n, d), np.float32)
    for a in range(0, n, CHUNK):
        b = min(n, a + CHUNK)
        lab = rng.integers(0, k, size=b - a)
        X[a:b] = means[lab] + sig[lab] * rng.standard_normal((b - a, d), dtype=np.float32)
    C0 = _distinct_rows(rng, X, k)
    return dict(name="lowd_d8", X=X, C0=C0, k=k, iters=25)


def outliers_d32(n=10_000_000, seed=0):
    rng = np.random.default_rng(seed)
    X = _blobs(rng, n, 32, 64, 10.0)
    out = rng.choice(n, size=n // 100, replace=False)
    X[out] = rng.uniform(-20, 20, size=(len(out), 32)).astype(np.float32)
    C0 = kmeans_pp_init([X], n, 64, rng, sample=10_000)
    return dict(name="outliers_d32", X=X, C0=C0, k=64, iters=20)


def _onehot_blobs(name, n, d, k, seed):
    rng = np.random.default_rng(seed)
    X = _blobs(rng, n, d, k, 10.0)
    C0 = kmeans_pp_init([X], n, k, rng, sample=10_000)
    return dict(name=name, X=X, C0=C0, k=k, iters=20)


def blobs_d48(n=10_000_000, seed=0):
    return _onehot_blobs("blobs_d48", n, 48, 64, seed)


def blobs_d32_k128(n=10_000_000, seed=0):
    return _onehot_blobs("blobs_d32_k128", n, 32, 128, seed)


def blobs_d96(n=10_000_000, seed=0):
    return _onehot_blobs("blobs_d96", n, 96, 64, seed)


def pixels_d4(n=96_000_000, seed=0):
    rng = np.random.default_rng(seed)
    k, d = 12, 4
    means = rng.uniform(0, 1, size=(k, d))
    w = rng.dirichlet(0.5 * np.ones(k))
    L = np.empty((k, d, d))
    for c in range(k):
        A = rng.standard_normal((d, d))
        L[c] = np.linalg.cholesky(0.02 ** 2 * (A @ A.T / 4 + 0.25 * np.eye(d)))
    L32 = L.astype(np.float32)
    mu32 = means.astype(np.float32)
    X = np.empty((n, d), np.float32)
    for a in range(0, n, CHUNK):
        b = min(n, a + CHUNK)
        lab = rng.choice(k, size=b - a, p=w)
        z = rng.standard_normal((b - a, d), dtype=np.float32)
        X[a:b] = np.clip(mu32[lab] + np.einsum("nij,nj->ni", L32[lab], z), 0.0, 1.0)
    C0 = _distinct_rows(rng, X, k)
    return dict(name="pixels_d4", X=X, C0=C0, k=k, iters=30)


def _unit_rows(name, n, d, seed, k):
    rng = np.random.default_rng(seed)
    cen = rng.standard_normal((k, d), dtype=np.float32)
    cen /= np.linalg.norm(cen, axis=1, keepdims=True)
    X = np.empty((n, d), np.float32)
    step = 250_000
    for a in range(0, n, step):
        b = min(n, a + step)
        lab = rng.integers(0, k, size=b - a)
        r = cen[lab] + np.float32(0.15) * rng.standard_normal((b - a, d), dtype=np.float32)
        X[a:b] = r / np.linalg.norm(r, axis=1, keepdims=True)
    C0 = _distinct_rows(rng, X, k)
    return dict(name=name, X=X, C0=C0, k=k, iters=15)


def embed_d768(n=1_000_000, seed=0, k=1024):
    return _unit_rows("embed_d768", n, 768, seed, k)


def embed_d1536(n=1_000_000, seed=0, k=1024):
    return _unit_rows("embed_d1536", n, 1536, seed, k)


def blobs_d960(n=1_000_000, seed=0, k=1024):
    rng = np.random.default_rng(seed)
    means = rng.uniform(-1.0, 1.0, size=(k, 960)).astype(np.float32)
    X = np.empty((n, 960), np.float32)
    step = 250_000
    for a in range(0, n, step):
        b = min(n, a + step)
        lab = rng.integers(0, k, size=b - a)
        X[a:b] = means[lab] + rng.standard_normal((b - a, 960), dtype=np.float32)
    C0 = kmeans_pp_init([X], n, k, rng)
    return dict(name="blobs_d960", X=X, C0=C0, k=k, iters=20)


WORKLOADS = {
    "blobs_d32": blobs_d32,
    "lowd_d8": lowd_d8,
    "outliers_d32": outliers_d32,
    "pixels_d4": pixels_d4,
    "embed_d768": embed_d768,
    "embed_d1536": embed_d1536,
    "blobs_d960": blobs_d960,
    "blobs_d48": blobs_d48,
    "blobs_d32_k128": blobs_d32_k128,
    "blobs_d96": blobs_d96,
}
