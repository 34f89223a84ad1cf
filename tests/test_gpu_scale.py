"""GPU: one 100M x 32 slice, k = 64, 90 % of the rows in one cluster, every value offset by +1000.

The fused pass adds each wave's rows into float32 matrix-core accumulators; on a slice this large one wave sees
about 50 000 rows, nearly all of one cluster. The per-cluster totals must still match float64 sums, as the
reference's one-hot pass keeps its float32 partials to 1024 rows (core.py:1562-1636).

The data are multiples of 1/16 within 1000 +- 21, so every value is exact in float32 and the exact per-cluster
sums are integers / 16, computed in int64 on the host. The rows repeat a 630-row pattern of clusters (nine rows of
cluster 0, then one of clusters 1..63 in turn), and the centres are the generating means, 4 or more apart against
noise under 0.71 in norm: every row's nearest centre is its own, so the labels are known without an oracle pass.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

PERIOD = 630
N = PERIOD * 158_730            # 99,999,900 rows
D, K = 32, 64


def say(*a):
    print(*a, flush=True)


def _pattern():
    p = np.zeros(PERIOD, np.int64)
    tens = np.arange(0, PERIOD, 10)
    p[tens] = 1 + np.arange(len(tens)) % 63
    return p


def test_skewed_offset_slice_100m_rows():
    from mlx_kmeans import _lib
    rng = np.random.default_rng(11)
    cen = (1000 + rng.integers(-20, 21, (K, D))).astype(np.float32)
    diff = cen[:, None, :].astype(np.float64) - cen[None, :, :]
    dist = np.sqrt((diff ** 2).sum(-1)) + np.eye(K) * 1e9
    assert dist.min() >= 4.0
    pat = _pattern()
    say(f"[gpu] skewed slice: generating {N:,} x {D}")
    noise = rng.integers(-2, 2, size=(N, D), dtype=np.int8)     # x = mean + noise / 16
    X = np.empty((N, D), np.float32)
    cp = cen[pat]                                                # (630, D) means of the pattern's rows
    sq = 0
    step = PERIOD * 4096
    for s in range(0, N, step):
        e = min(N, s + step)
        nz = noise[s:e].reshape(-1, PERIOD, D)
        xv = X[s:e].reshape(-1, PERIOD, D)
        np.multiply(nz, np.float32(1.0 / 16.0), out=xv, casting="unsafe")
        np.add(xv, cp[None], out=xv)
        sq += int(np.square(nz).sum(dtype=np.int64))
    S = noise.reshape(-1, PERIOD, D).sum(axis=0, dtype=np.int64)     # (630, D) noise sums per pattern row
    del noise
    reps = N // PERIOD
    counts = np.bincount(pat, minlength=K) * reps
    noise_sum = np.zeros((K, D), np.int64)
    np.add.at(noise_sum, pat, S)
    exact = counts[:, None] * cen.astype(np.float64) + noise_sum / 16.0   # exact in float64 (< 2^53 / 16)
    exact_inertia = sq / 256.0
    rms = float(np.sqrt((counts[:, None] * cen.astype(np.float64) ** 2).sum() / (N * D)))   # about 1000

    ctx = _lib.Context()
    ctx.set_parts([X])
    say("[gpu]   pass with labels")
    tot, labels, _ = ctx.run_pass(cen, labels=True)
    assert ctx.last_path() == "mfma"      # the fused matrix-core pass
    assert np.array_equal(labels.reshape(-1, PERIOD), np.broadcast_to(pat.astype(np.uint32), (reps, PERIOD)))
    assert np.array_equal(tot[:, 0], counts.astype(np.float64))
    err = np.abs(tot[:, 2:] - exact) / counts[:, None]
    say(f"[gpu]   max centre error {err.max():.3e} (RMS {rms:.1f}); inertia {tot[:, 1].sum():.6e} "
        f"exact {exact_inertia:.6e}")
    assert float(err.max()) <= 1e-6 * rms
    assert abs(float(tot[:, 1].sum()) - exact_inertia) <= 1e-6 * exact_inertia
    # the sums themselves: within 2^-24 of the cluster's total mass. One float32 run over a wave's ~45 000 rows
    # near 1000 would round every add to a multiple of 4 in the same direction (about 1e-3 relative); runs of
    # 1024 rows of multiples of 1/16 are exact, and only their few dozen partial sums per wave round.
    rel = np.abs(tot[:, 2:] - exact) / (counts[:, None] * np.abs(cen.astype(np.float64)))
    say(f"[gpu]   max relative sum error {rel.max():.3e}")
    assert float(rel.max()) <= 2.0 ** -24
    say("[gpu]   Lloyd step")
    C1, inertia, n_empty = ctx.lloyd_step(cen)
    assert n_empty == 0
    assert float(np.max(np.abs(C1.astype(np.float64) - exact / counts[:, None]))) <= 1e-6 * rms
    ctx.close()
