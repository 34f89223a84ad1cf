"""The k-means++ seeding oracle (oracle.seed_pp, the restatement of mlx_kmeans/core.py:153-192 and 70-106), pinned
without the GPU: splitmix64 against its published first output and an arbitrary-precision restatement, the
candidate draw against the distribution it must have (probability proportional to d2), and the greedy rounds
against properties fixed by the data."""
import math

import numpy as np
import pytest

M64 = (1 << 64) - 1


def splitmix64_int(z):
    """splitmix64's output function on Python ints, masked to 64 bits (Steele, Lea and Flood 2014)."""
    z = (z + 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def test_mix64_known_answer_and_wraparound(oracle):
    # the generator seeded with 0 starts 0xE220A8397B1DCDAF (its published first output)
    assert int(oracle.mix64(np.uint64(0))) == 0xE220A8397B1DCDAF
    rng = np.random.default_rng(3)
    z = rng.integers(0, 2**63, size=2000, dtype=np.uint64) * np.uint64(2) + np.uint64(1)
    got = oracle.mix64(z)
    assert all(int(g) == splitmix64_int(int(v)) for g, v in zip(got, z))


def test_candidate_draw_is_proportional_to_d2(oracle):
    d2 = np.array([0.0, 1.0, 2.0, 4.0, 8.0, 1.0], np.float32)
    p = d2 / d2.sum()
    counts = np.zeros(len(d2))
    n = 20000
    seeds = np.random.default_rng(11).integers(2**63 - 1, size=n).astype(np.uint64)
    for s in seeds:
        counts[int(np.argmax(oracle.pp_keys(d2, int(s), 3, 1)))] += 1
    assert counts[0] == 0                              # zero weight: never drawn
    expect = n * p
    nz = expect > 0
    chi2 = float((((counts - expect) ** 2)[nz] / expect[nz]).sum())
    assert chi2 < 25.0, (counts, expect)               # 4 degrees of freedom: p < 1e-4 of exceeding by chance
    # a key that ignores d2 (or inverts it) fails the same test
    wrong = np.zeros(len(d2))
    for s in seeds[:4000]:
        wrong[int(np.argmin(oracle.pp_keys(d2, int(s), 3, 1)))] += 1
    assert wrong[0] > 0.9 * 4000


def test_block_total_is_the_sum(oracle):
    v = np.random.default_rng(2).uniform(0, 3, size=1000).astype(np.float32)
    assert abs(oracle.pp_block_total(v) - math.fsum(v.astype(np.float64))) <= 1e-12 * math.fsum(v.astype(np.float64))


def test_one_pick_per_separated_blob(oracle):
    # eight blobs 100 apart with unit spread: every greedy round's best candidate opens a new blob
    rng = np.random.default_rng(4)
    means = rng.uniform(-1, 1, size=(8, 6)) * 100.0
    lab = rng.integers(0, 8, size=4000)
    S = (means[lab] + rng.standard_normal((4000, 6))).astype(np.float32)
    for trial in range(3):
        seeds = rng.integers(2**63 - 1, size=7).astype(np.uint64)
        first = int(rng.integers(4000))
        picks, C = oracle.seed_pp(S, 8, first, seeds)
        assert picks[0] == first
        assert sorted(lab[picks]) == list(range(8))
        assert np.array_equal(C, S[picks])


def test_single_centre_and_all_equal_rows(oracle):
    S = np.ones((50, 3), np.float32)
    picks, C = oracle.seed_pp(S, 1, 7, np.zeros(0, np.uint64))
    assert list(picks) == [7]
    # every d2 is 0: the draw falls back on the keys' randomness alone and still returns k distinct-index rows
    picks, C = oracle.seed_pp(S, 5, 0, np.arange(1, 5, dtype=np.uint64))
    assert len(picks) == 5 and np.all(C == 1.0)


def test_greedy_choice_lowers_the_potential_most(oracle):
    rng = np.random.default_rng(8)
    S = rng.standard_normal((600, 5)).astype(np.float32)
    seeds = rng.integers(2**63 - 1, size=5).astype(np.uint64)
    picks, _ = oracle.seed_pp(S, 6, 10, seeds)
    d2 = oracle.direct_sq(S, S[10])
    for r in range(5):
        trials = oracle.pp_trials(6)
        cand = [int(np.argmax(oracle.pp_keys(d2, int(seeds[r]), trials, t))) for t in range(trials)]
        assert picks[r + 1] in cand
        pots = [float(np.fmin(d2, oracle.direct_sq(S, S[c])).astype(np.float64).sum()) for c in cand]
        assert pots[cand.index(int(picks[r + 1]))] <= min(pots) * (1 + 1e-12)
        d2 = np.fmin(d2, oracle.direct_sq(S, S[picks[r + 1]]))
