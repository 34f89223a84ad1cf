"""ORACLE - test infrastructure only.

Python side of the CPU oracle for the exact Lloyd pass. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module, and only as the checker (or as the timed CPU baseline); the product
path (the mlx_kmeans package over libkmeans_hip.so) never does.

Two layers:
  * ctypes bindings to kmeans_oracle.c (built into oracle/build/liboracle.so by oracle/Makefile): the bit-level
    restatement of the reference's exact mode - see that file's header for the reference lines each function
    follows.
  * numpy restatements of the reference's own float64 test oracle (tests/accuracy.py), which pin the C
    restatement from an independent direction:
      reference_f64         tests/accuracy.py:31-51   float64 nearest centre, lowest index on exact ties
      label_tolerance       tests/accuracy.py:86-88   d64(x, label) <= d64(x, best) + 8*eps32*(|x|^2 + |c|^2)
      reference_lloyd_step  tests/accuracy.py:108-129 float64 Lloyd step with the relocation rules
  * kmeans_simple_pass: numpy restatement of kmeans_simple.py:45-78 (the reference's teaching CPU path:
    expanded-form distances, argmin, scatter-add, float64 totals). It is NOT exact; it is only timed.
  * seed_pp: numpy restatement of the reference's GPU k-means++ seeding (core.py:153-192 with its kernels
    _PP_PICK_SRC / _PP_EVAL_SRC, 70-106, and the hash of 43-48): counter-based candidate draws, direct-form
    float32 distances, float64 totals added in the device's order, so the device's picks must match bit for bit.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "liboracle.so")
EPS32 = float(np.finfo(np.float32).eps)

VARIANT_A1, VARIANT_FMA, MUTANT_LE_TIE, MUTANT_DROP_LAST_DIM, MUTANT_SIGN = 0, 1, 2, 3, 4

_lib = None


def build():
    """Compile liboracle.so from kmeans_oracle.c (gcc; seconds)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        f32p, f64p = ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_double)
        u32p, i32p = ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_int)
        i64 = ctypes.c_int64
        L.orc_assign.argtypes = [f32p, i64, ctypes.c_int, f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, u32p, f32p]
        L.orc_assign.restype = None
        L.orc_totals.argtypes = [f32p, i64, ctypes.c_int, u32p, f32p, ctypes.c_int, f64p]
        L.orc_totals.restype = None
        L.orc_update.argtypes = [f64p, ctypes.c_int, ctypes.c_int, f32p, i64, u32p, f32p, f32p, f32p, f64p, i32p]
        L.orc_update.restype = None
        L.orc_label_dist.argtypes = [f32p, i64, ctypes.c_int, f32p, u32p, f32p]
        L.orc_label_dist.restype = None
        L.orc_cpu_pass.argtypes = [f32p, i64, ctypes.c_int, f32p, ctypes.c_int, ctypes.c_int, f64p]
        L.orc_cpu_pass.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def default_threads():
    return max(1, min(16, os.cpu_count() or 1))


def assign(X, C, variant=VARIANT_A1, nthreads=None):
    """Exact labels (uint32) and best distances (float32) for every row: the rows-loop semantics."""
    X, C = _f32(X), _f32(C)
    n, d = X.shape
    k = C.shape[0]
    labels = np.empty(n, np.uint32)
    best = np.empty(n, np.float32)
    lib().orc_assign(_p(X, ctypes.c_float), n, d, _p(C, ctypes.c_float), k, variant,
                     nthreads or default_threads(), _p(labels, ctypes.c_uint32), _p(best, ctypes.c_float))
    return labels, best


def distances_to(X, C, labels):
    """The rows-loop float32 distance of every row to the centre its label names (core.py:851-856)."""
    X, C = _f32(X), _f32(C)
    n, d = X.shape
    labels = np.ascontiguousarray(labels, dtype=np.uint32)
    if len(labels) != n or (n and int(labels.max()) >= C.shape[0]):
        raise ValueError("one label per row, each naming a centre")
    out = np.empty(n, np.float32)
    lib().orc_label_dist(_p(X, ctypes.c_float), n, d, _p(C, ctypes.c_float), _p(labels, ctypes.c_uint32),
                         _p(out, ctypes.c_float))
    return out


def totals(X, labels, best, k):
    """(k, d+2) float64 [count, sum best, sum x...] over the given labels."""
    X = _f32(X)
    n, d = X.shape
    labels = np.ascontiguousarray(labels, dtype=np.uint32)
    best = _f32(best)
    tot = np.empty((k, d + 2), np.float64)
    lib().orc_totals(_p(X, ctypes.c_float), n, d, _p(labels, ctypes.c_uint32), _p(best, ctypes.c_float), k,
                     _p(tot, ctypes.c_double))
    return tot


def one_pass(X, C, variant=VARIANT_A1):
    """One assignment pass -> (tot (k, d+2) f64, labels u32, best f32); the shape of core.py's _gpu_pass."""
    labels, best = assign(X, C, variant)
    return totals(X, labels, best, C.shape[0]), labels, best


def update(tot, X, labels, best, C):
    """lloyd_step's host math on a pass's totals -> (C_new f32, inertia, n_empty)."""
    X, C = _f32(X), _f32(C)
    n, d = X.shape
    k = C.shape[0]
    tot = np.ascontiguousarray(tot, dtype=np.float64)
    labels = np.ascontiguousarray(labels, dtype=np.uint32)
    best = _f32(best)
    C_out = np.empty_like(C)
    inertia = ctypes.c_double()
    n_empty = ctypes.c_int()
    lib().orc_update(_p(tot, ctypes.c_double), k, d, _p(X, ctypes.c_float), n, _p(labels, ctypes.c_uint32),
                     _p(best, ctypes.c_float), _p(C, ctypes.c_float), _p(C_out, ctypes.c_float),
                     ctypes.byref(inertia), ctypes.byref(n_empty))
    return C_out, inertia.value, n_empty.value


def lloyd_step(X, C, variant=VARIANT_A1):
    """One exact Lloyd iteration -> (C_new, inertia, n_empty, labels, best, tot)."""
    tot, labels, best = one_pass(X, C, variant)
    C_new, inertia, n_empty = update(tot, X, labels, best, C)
    return C_new, inertia, n_empty, labels, best, tot


def normalise(C):
    """Spherical k-means' renormalisation (estimator.py:127-130): each centre over its float32 length, a zero
    centre left as is."""
    C = _f32(C)
    n = np.linalg.norm(C, axis=1, keepdims=True)
    return (C / np.where(n > 0, n, 1)).astype(np.float32)


def fit_from(X, C0, max_iter, tol=0.0, spherical=False):
    """KMeans._one_run's loop (estimator.py:132-150) from given starting centres - with spherical=True the
    starting centres and every step's centres renormalised - then the final scoring pass on the returned
    centres (estimator.py:201-204) -> (C, inertia_final, n_iter, labels)."""
    C = _f32(C0).copy()
    if spherical:
        C = normalise(C)
    prev = None
    it = 0
    for it in range(max_iter):
        C, inertia, _, _, _, _ = lloyd_step(X, C)
        if spherical:
            C = normalise(C)
        if prev is not None and abs(prev - inertia) <= tol * prev:
            break
        prev = inertia
    tot, labels, _ = one_pass(X, C)
    return C, float(tot[:, 1].sum()), it + 1, labels


def cpu_pass(X, C, nthreads=None):
    """kmeans.mm's CPU backend restated -> tot (k, d+2) float64."""
    X, C = _f32(X), _f32(C)
    n, d = X.shape
    k = C.shape[0]
    tot = np.empty((k, d + 2), np.float64)
    rc = lib().orc_cpu_pass(_p(X, ctypes.c_float), n, d, _p(C, ctypes.c_float), k, nthreads or default_threads(),
                            _p(tot, ctypes.c_double))
    if rc != 0:
        raise MemoryError("orc_cpu_pass could not allocate its job buffers")
    return tot


# ---------------------------------------------------------------- float64 restatements of tests/accuracy.py

def reference_f64(X, C, chunk_terms=20_000_000):
    """Exact float64 nearest centre (lowest index on exact ties) and its distance (tests/accuracy.py:31-51)."""
    X64, C64 = np.asarray(X, np.float64), np.asarray(C, np.float64)
    csq = (C64 ** 2).sum(1)
    n, k = len(X64), len(C64)
    best_d = np.empty(n)
    best_c = np.empty(n, np.int64)
    step = max(1, chunk_terms // (k * X64.shape[1]))
    for s in range(0, n, step):
        x = X64[s:s + step]
        approx = csq[None, :] - 2 * x @ C64.T
        lo = approx.min(1, keepdims=True)
        win = 1e-9 * ((x ** 2).sum(1, keepdims=True) + csq[None, :]) + 1e-300
        cand = approx <= lo + 2 * win
        dd = np.full(approx.shape, np.inf)
        rows, cols = np.nonzero(cand)
        dd[rows, cols] = ((x[rows] - C64[cols]) ** 2).sum(1)
        best_c[s:s + step] = dd.argmin(1)
        best_d[s:s + step] = dd[np.arange(len(x)), best_c[s:s + step]]
    return best_c, best_d


def label_tolerance(X, C, labels, ref_d):
    """-> number of labels that are not float64-optimal up to float32 resolution (tests/accuracy.py:86-88)."""
    X64, C64 = np.asarray(X, np.float64), np.asarray(C, np.float64)
    lab = np.asarray(labels, np.int64)
    d_lab = ((X64 - C64[lab]) ** 2).sum(1)
    tol = 8 * EPS32 * ((X64 ** 2).sum(1) + (C64[lab] ** 2).sum(1))
    return int((d_lab > ref_d + tol).sum())


def reference_lloyd_step(X, C, labels):
    """Independent float64 Lloyd step for given labels (tests/accuracy.py:108-129) -> (centres f64, n_empty)."""
    X64, C64 = np.asarray(X, np.float64), np.asarray(C, np.float64)
    labels = np.asarray(labels, np.int64)
    best = ((X64 - C64[labels]) ** 2).sum(1)
    k = len(C64)
    counts = np.bincount(labels, minlength=k)
    sums = np.zeros((k, X64.shape[1]))
    np.add.at(sums, labels, X64)
    empty = np.flatnonzero(counts == 0)
    if len(empty) and best.max() > 0:
        order = np.lexsort((np.arange(len(X64)), -best))[:len(empty)]
        for new, f in zip(empty, order):
            sums[labels[f]] -= X64[f]
            counts[labels[f]] -= 1
            sums[new] = X64[f]
            counts[new] = 1
    out = np.empty_like(C64)
    has = counts > 0
    out[has] = sums[has] / counts[has, None]
    out[~has] = out[np.argmax(counts)]
    return out, len(empty)


def kmeans_simple_pass(X, C, chunk=2_000_000):
    """One pass of kmeans_simple.py:45-78 in numpy: expanded distances, argmin, scatter-add, float64 totals.
    -> (sums (k, d) f64, counts (k,) f64, error f64). Approximate by design (the reference says so)."""
    X, C = _f32(X), _f32(C)
    k, d = C.shape
    sums = np.zeros((k, d))
    counts = np.zeros(k)
    err = 0.0
    csq = (C * C).sum(axis=1)
    for s in range(0, len(X), chunk):
        x = X[s:s + chunk]
        dist = csq[None, :] - 2 * (x @ C.T)
        nearest = dist.argmin(axis=1)
        cs = np.zeros((k, d), np.float32)
        np.add.at(cs, nearest, x)
        cc = np.bincount(nearest, minlength=k).astype(np.float32)
        ce = float(((x - C[nearest]) ** 2).sum())
        sums += cs
        counts += cc
        err += ce
    return sums, counts, err


# ---------------------------------------------------------------- k-means++ seeding

def mix64(z):
    """splitmix64's output function on uint64 arrays (the reference's mix64, mlx_kmeans/core.py:43-48)."""
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = z + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def pp_trials(k):
    """Candidates per round: 2 + floor(ln k) (core.py:181)."""
    return 2 + int(np.log(k)) if k > 1 else 1


def direct_sq(S, c):
    """Float32 |S_i - c|^2 in the direct form, dims ascending, product and add rounded separately."""
    s = np.zeros(len(S), np.float32)
    for j in range(S.shape[1]):
        q = S[:, j] - c[j]
        s = s + q * q
    return s


def pp_keys(d2, seed, trials, t):
    """Candidate keys of one trial: d2_i / (-ln u_i) in float64, u_i from the round's seed, the row and the trial
    (the ordering of the reference's Gumbel-max key ln d2 - ln(-ln u), core.py:70-76)."""
    i = np.arange(len(d2), dtype=np.uint64)
    with np.errstate(over="ignore"):
        h = mix64(np.uint64(seed) ^ mix64(i * np.uint64(trials) + np.uint64(t)))
    u = ((h >> np.uint64(40)).astype(np.float64) + 0.5) * 2.0**-24
    return np.maximum(d2.astype(np.float64), 1e-30) / -np.log(u)


def pp_block_total(v, block=32, lanes=64):
    """Float64 sum of float32 values the way the seeding kernels add them: per block of 32 rows a halving tree
    (element i += element i + h, h = 16 .. 1); then lane l of 64 adds the block sums b = l (mod 64) in ascending
    order, and the 64 lane sums go through a halving tree (lane l += lane l + h, h = 32 .. 1)."""
    v = v.astype(np.float64)
    nb = (len(v) + block - 1) // block
    x = np.zeros((nb, block))
    x.reshape(-1)[:len(v)] = v
    h = block // 2
    while h:
        x[:, :h] += x[:, h:2 * h]
        h //= 2
    bs = x[:, 0]
    ls = np.zeros(lanes)
    for b in range(nb):
        ls[b % lanes] = ls[b % lanes] + bs[b]
    h = lanes // 2
    while h:
        ls[:h] += ls[h:2 * h]
        h //= 2
    return float(ls[0])


def seed_pp(S, k, first, seeds):
    """Greedy k-means++ on the sample rows S (m, d) float32 -> (picked row indices, (k, d) float32 centres).

    Restates the reference's GPU seeding (core.py:153-192 with _PP_PICK_SRC / _PP_EVAL_SRC, 70-106): d2 starts
    as the direct-form distance to S[first]; round r draws, per trial t, the row with the largest key (lowest row
    on a tie), scores min(d2, distance to that row) per row, and keeps the first trial with the smallest total;
    its minima become d2."""
    S = np.ascontiguousarray(S, dtype=np.float32)
    trials = pp_trials(k)
    d2 = direct_sq(S, S[first])
    picks = [int(first)]
    for r in range(k - 1):
        cand = [int(np.argmax(pp_keys(d2, int(seeds[r]), trials, t))) for t in range(trials)]
        mins = [np.fmin(d2, direct_sq(S, S[c])) for c in cand]
        tot = [pp_block_total(m_) for m_ in mins]
        b = int(np.argmin(tot))
        d2 = mins[b]
        picks.append(cand[b])
    return np.array(picks), S[picks].copy()
