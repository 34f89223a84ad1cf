"""GPU: km_pass_noalloc, the allocation-free pass, through the C ABI against km_pass on the same input.

Two calls in a row on one context, the second with fewer rows (the scratch array keeps the first call's
contents); each must give km_pass's labels and best bit for bit, its counts exactly, and its sums and inertia
within 1e-6 relative (the same kernel family, summed over as many or fewer row blocks). Also two calls queued on
one stream with no synchronisation between them. Also: a shape whose
partials cannot fit the scratch is refused with a clear error before any launch.
"""
import ctypes

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


class _Hip:
    """The HIP runtime calls the test needs (device buffers, a stream), looked up through the engine library's
    own handle, so they are the runtime the library itself calls."""

    def __init__(self, L):
        self.L = L
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        for name, args in (("hipMalloc", [ctypes.POINTER(vp), sz]), ("hipFree", [vp]),
                           ("hipMemcpy", [vp, vp, sz, ctypes.c_int]), ("hipStreamCreate", [ctypes.POINTER(vp)]),
                           ("hipStreamSynchronize", [vp]), ("hipStreamDestroy", [vp])):
            f = getattr(L, name)
            f.restype = ctypes.c_int
            f.argtypes = args

    def check(self, rc, what):
        assert rc == 0, f"{what} failed: {rc}"

    def put(self, a):
        a = np.ascontiguousarray(a)
        p = ctypes.c_void_p()
        self.check(self.L.hipMalloc(ctypes.byref(p), max(a.nbytes, 1)), "hipMalloc")
        self.check(self.L.hipMemcpy(p, a.ctypes.data_as(ctypes.c_void_p), a.nbytes, 1), "hipMemcpy H2D")
        return p

    def get(self, p, like):
        out = np.empty_like(like)
        self.check(self.L.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), p, out.nbytes, 2), "hipMemcpy D2H")
        return out


def _noalloc_calls(lib, ctx, cases):
    """km_pass_noalloc once per (X, C) in `cases`, all queued on one stream of the test's own with no
    synchronisation between the calls -> [(totals f64, labels u32, best f32)] per call."""
    hip = _Hip(lib.lib())
    stream = ctypes.c_void_p()
    hip.check(hip.L.hipStreamCreate(ctypes.byref(stream)), "hipStreamCreate")
    calls, bufs = [], []
    try:
        for X, C in cases:
            n, d = X.shape
            k = C.shape[0]
            like = (np.full((k, d + 2), np.nan), np.full(n, 0xffffffff, np.uint32), np.full(n, np.nan, np.float32))
            b = [hip.put(X), hip.put(np.ascontiguousarray(C, np.float32))] + [hip.put(a) for a in like]
            bufs += b
            rc = lib.lib().km_pass_noalloc(ctx._h, b[0], n, d, b[1], k, b[2], b[3], b[4], stream)
            ctx._check(rc)
            calls.append((b, like))
        hip.check(hip.L.hipStreamSynchronize(stream), "hipStreamSynchronize")
        return [tuple(hip.get(p, a) for p, a in zip(b[2:], like)) for b, like in calls]
    finally:
        hip.check(hip.L.hipStreamSynchronize(stream), "hipStreamSynchronize")
        hip.L.hipStreamDestroy(stream)
        for p in bufs:
            hip.L.hipFree(p)


def _noalloc(lib, ctx, X, C):
    """One km_pass_noalloc call on a stream of the test's own -> (totals f64, labels u32, best f32)."""
    return _noalloc_calls(lib, ctx, [(X, C)])[0]


def _km_pass(lib, X, C):
    ref = lib.Context()
    ref.set_parts([X])
    out = ref.run_pass(C, labels=True, best=True)
    ref.close()
    return out


def _same(got, want):
    (t1, l1, b1), (t0, l0, b0) = got, want
    assert np.array_equal(l1, l0), np.flatnonzero(l1 != l0)[:10]
    assert np.array_equal(b1.view(np.uint32), b0.view(np.uint32))
    assert np.array_equal(np.rint(t1[:, 0]), np.rint(t0[:, 0]))
    fin = np.isfinite(t0)
    assert np.array_equal(fin, np.isfinite(t1))
    scale = np.maximum(np.abs(t0[fin]), 1.0)
    assert np.all(np.abs(t1[fin] - t0[fin]) <= 1e-6 * scale)


def _data(seed, n, d, k):
    rng = np.random.default_rng(seed)
    cen = rng.uniform(-4, 4, size=(max(k // 2, 1), d)).astype(np.float32)
    X = (cen[rng.integers(0, len(cen), n)] + rng.standard_normal((n, d))).astype(np.float32)
    X[5] = np.nan                                     # a non-finite row: label 0, best as the rows loop leaves it
    C = X[rng.choice(np.arange(10, n), k, replace=False)].copy()
    return X, C


# (dims, centres, rows of the two calls): the fused matrix-core, fused low-d and rows families, the rows loop's
# tiled form (d = 100, k = 64), and a shape km_pass sends to the wide-row screen while the allocation-free pass
# runs the tiled rows loop over as few row blocks as its scratch holds (d = 768, k = 256)
@pytest.mark.parametrize("d,k,ns", [(32, 64, (120_011, 33_007)), (48, 64, (90_011, 33_007)),
                                    (32, 128, (90_011, 33_007)), (4, 12, (120_011, 33_007)),
                                    (16, 40, (120_011, 33_007)), (48, 100, (120_011, 33_007)),
                                    (3, 300, (120_011, 33_007)), (100, 64, (50_011, 20_007)),
                                    (768, 256, (20_011, 9_007))])
def test_noalloc_pass_matches_km_pass(lib, d, k, ns):
    ctx = lib.Context()
    for call, n in enumerate(ns):
        X, C = _data(7 * d + k + call, n, d, k)
        say(f"[gpu] noalloc call {call} n={n} d={d} k={k}")
        _same(_noalloc(lib, ctx, X, C), _km_pass(lib, X, C))
    ctx.close()


def test_noalloc_back_to_back_on_one_stream(lib):
    """Two calls queued on one stream without a synchronisation between them (the second smaller, another
    family): the stream orders the second call's use of the scratch after the first's."""
    ctx = lib.Context()
    cases = [_data(101, 120_011, 32, 64), _data(102, 33_007, 4, 12)]
    say("[gpu] noalloc back to back: 120011 x 32 k=64, then 33007 x 4 k=12")
    got = _noalloc_calls(lib, ctx, cases)
    for g, (X, C) in zip(got, cases):
        _same(g, _km_pass(lib, X, C))
    ctx.close()


def test_noalloc_refuses_what_the_scratch_cannot_hold(lib):
    ctx = lib.Context()
    d, k = 700, 4096                                 # k * (d + 2) = 2.9M entries: 46 MB for one block
    n = 64
    X = np.zeros((n, d), np.float32)
    C = np.zeros((k, d), np.float32)
    say("[gpu] noalloc refusal")
    with pytest.raises(ValueError, match="scratch"):
        _noalloc(lib, ctx, X, C)
    ctx.close()
