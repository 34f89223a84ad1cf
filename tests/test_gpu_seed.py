"""GPU k-means++ seeding (km_seed_pp, the reference's kmeans_pp_init, mlx_kmeans/core.py:153-192) against the
oracle's restatement (oracle.seed_pp): the same picks, bit for bit, for the same sample, first pick and seeds."""
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


def blobs(rng, n, d, k, spread=8.0):
    means = rng.uniform(-spread, spread, size=(max(k // 2, 1), d))
    return (means[rng.integers(0, len(means), n)] + rng.standard_normal((n, d))).astype(np.float32)


@pytest.mark.parametrize("n,d,k,m", [(3000, 4, 12, 3000), (30000, 32, 64, 20000), (9000, 8, 8, 4500),
                                     (2500, 768, 40, 2500), (5000, 3, 1, 5000), (64, 5, 64, 64),
                                     (12000, 17, 300, 6000)])
def test_seeding_matches_oracle(lib, oracle, n, d, k, m):
    rng = np.random.default_rng(100 + n + d + k)
    X = blobs(rng, n, d, k)
    idx = np.sort(rng.choice(n, size=m, replace=False))
    first = int(rng.integers(m))
    seeds = rng.integers(2**63 - 1, size=k - 1).astype(np.uint64)
    say(f"[gpu] seed_pp n={n} d={d} k={k} m={m}")
    ctx = lib.Context()
    ctx.set_parts([X])
    C = ctx.seed_pp(k, idx, first, seeds)
    picks, C_ref = oracle.seed_pp(X[idx], k, first, seeds)
    assert np.array_equal(C, C_ref), np.nonzero(~(C == C_ref).all(1))[0][:5]
    ctx.close()


def test_seeding_over_slices_and_duplicate_rows(lib, oracle):
    """Sample rows taken from three slices; many identical rows (squared distances of 0) in the sample."""
    rng = np.random.default_rng(7)
    parts = [blobs(rng, 4000, 16, 20), blobs(rng, 1500, 16, 20), blobs(rng, 3000, 16, 20)]
    parts[1][:700] = parts[1][0]
    X = np.concatenate(parts)
    idx = np.sort(rng.choice(len(X), size=5000, replace=False))
    seeds = rng.integers(2**63 - 1, size=24).astype(np.uint64)
    say("[gpu] seed_pp over slices")
    ctx = lib.Context()
    ctx.set_parts(parts)
    C = ctx.seed_pp(25, idx, 3, seeds)
    _, C_ref = oracle.seed_pp(X[idx], 25, 3, seeds)
    assert np.array_equal(C, C_ref)
    ctx.close()


def test_kmeans_pp_init_draws_like_the_reference(lib, oracle):
    """core.kmeans_pp_init draws the sample, the first pick and the round seeds from rng in the reference's
    order (core.py:173-184) and seeds on the GPU: the oracle, fed the same draws, picks the same rows."""
    from mlx_kmeans import core
    rng = np.random.default_rng(21)
    X = blobs(rng, 50000, 24, 48)
    say("[gpu] kmeans_pp_init")
    C = core.kmeans_pp_init([X], len(X), 48, np.random.default_rng(5))
    r = np.random.default_rng(5)
    idx = np.sort(r.choice(len(X), size=min(200_000, max(20_000, 20 * 48)), replace=False))
    first = int(r.integers(len(idx)))
    seeds = r.integers(2**63 - 1, size=47).astype(np.uint64)
    _, C_ref = oracle.seed_pp(X[idx], 48, first, seeds)
    assert np.array_equal(C, C_ref)


def test_seeding_rejects_bad_arguments(lib):
    ctx = lib.Context()
    X = np.zeros((100, 4), np.float32)
    ctx.set_parts([X])
    with pytest.raises(ValueError):
        ctx.seed_pp(10, np.arange(5), 0, np.zeros(9, np.uint64))          # fewer sample rows than centres
    with pytest.raises(ValueError):
        ctx.seed_pp(3, np.array([5, 2, 9]), 0, np.zeros(2, np.uint64))    # not ascending
    with pytest.raises(ValueError):
        ctx.seed_pp(3, np.array([1, 2, 300]), 0, np.zeros(2, np.uint64))  # beyond the rows
    ctx.close()
