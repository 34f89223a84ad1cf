"""ctypes binding to libkmeans_hip.so (the C ABI declared in include/kmeans_hip.h).

Nothing here computes: every pass runs in the HIP library. If the library is missing or no GPU is visible,
the calls raise - there is no CPU fallback.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libkmeans_hip.so")

KM_OK, KM_EINVAL, KM_EDEVICE, KM_ENOMEM, KM_ENODATA = 0, -1, -2, -3, -4
KM_HOST, KM_DEVICE = 0, 1
KM_EXACT, KM_APPROX = 0, 1
KM_PATH_AUTO, KM_PATH_ROWS, KM_PATH_MFMA, KM_PATH_FUSED = 0, 1, 2, 3
PATHS = {"auto": KM_PATH_AUTO, "rows": KM_PATH_ROWS, "mfma": KM_PATH_MFMA, "fused": KM_PATH_FUSED}

# every symbol include/kmeans_hip.h declares: (name, restype, argtypes)
_c = ctypes
_f32p, _f64p, _u32p, _i32p, _i64p = (_c.POINTER(_c.c_float), _c.POINTER(_c.c_double), _c.POINTER(_c.c_uint32),
                                     _c.POINTER(_c.c_int32), _c.POINTER(_c.c_int64))
SIGNATURES = [
    ("km_create", _c.c_void_p, [_c.c_int32]),
    ("km_destroy", None, [_c.c_void_p]),
    ("km_last_error", _c.c_char_p, [_c.c_void_p]),
    ("km_set_data", _c.c_int32, [_c.c_void_p, _c.c_void_p, _c.c_int64, _c.c_int32, _c.c_int32]),
    ("km_append_data", _c.c_int32, [_c.c_void_p, _c.c_void_p, _c.c_int64, _c.c_int32]),
    ("km_rows", _c.c_int64, [_c.c_void_p]),
    ("km_dims", _c.c_int32, [_c.c_void_p]),
    ("km_pass", _c.c_int32, [_c.c_void_p, _f32p, _c.c_int32, _c.c_int32, _c.c_int32, _f64p, _u32p, _f32p]),
    ("km_lloyd_step", _c.c_int32, [_c.c_void_p, _f32p, _c.c_int32, _c.c_int32, _c.c_int32, _f32p, _f64p, _i32p]),
    ("km_fit", _c.c_int32, [_c.c_void_p, _f32p, _c.c_int32, _c.c_int32, _c.c_double, _c.c_int32, _c.c_int32,
                            _f32p, _f64p, _i32p, _i32p]),
    ("km_seed_pp", _c.c_int32, [_c.c_void_p, _c.c_int32, _i64p, _c.c_int64, _c.c_int64,
                                _c.POINTER(_c.c_uint64), _f32p]),
    ("km_profile", _c.c_int32, [_c.c_void_p, _c.c_int32]),
    ("km_profile_read", _c.c_int32, [_c.c_void_p, _c.c_int32, _f64p, _i64p]),
    ("km_kernel_name", _c.c_char_p, [_c.c_int32]),
    ("km_last_path", _c.c_int32, [_c.c_void_p]),
    ("km_last_fallback_rows", _c.c_int64, [_c.c_void_p]),
    ("km_version", _c.c_int32, []),
    ("km_profile_passes", _c.c_int64, [_c.c_void_p, _f64p, _c.c_int64]),
    ("km_stream_probe", _c.c_int32, [_c.c_void_p, _c.c_int64, _c.c_int32, _f64p]),
    ("km_pass_noalloc", _c.c_int32, [_c.c_void_p, _c.c_void_p, _c.c_int64, _c.c_int32, _c.c_void_p, _c.c_int32,
                                     _c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_void_p]),
    ("km_bounds", _c.c_int32, [_c.c_void_p, _c.c_double]),
    ("km_bounds_info", _c.c_int32, [_c.c_void_p, _i64p, _i64p, _i64p, _f64p]),
]

_lib = None


def lib():
    """The loaded library, with argument types set. Raises RuntimeError if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() (or `make` in "
                               f"{os.path.dirname(_HERE)}) first. There is no CPU fallback.")
        L = ctypes.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _ptr(a, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


class Context:
    """One device context: a HIP stream, the data slices on the device, and the pass workspaces."""

    def __init__(self, device=0):
        L = lib()
        self._h = L.km_create(int(device))
        if not self._h:
            raise RuntimeError(f"km_create({device}) failed: no HIP device {device} is visible")
        self._keep = []          # host or torch objects whose memory a slice borrows
        self.rows = 0
        self.dims = 0

    def close(self):
        if getattr(self, "_h", None):
            lib().km_destroy(self._h)
            self._h = None
        self._keep = []

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc):
        if rc == KM_OK:
            return
        msg = (lib().km_last_error(self._h) or b"").decode(errors="replace")
        if rc == KM_EINVAL or rc == KM_ENODATA:
            raise ValueError(msg)
        if rc == KM_ENOMEM:
            raise MemoryError(msg)
        raise RuntimeError(msg)

    # ---- data
    def set_parts(self, parts):
        """parts: list of 2-D float32 slices - numpy arrays (copied to the device) or torch CUDA tensors
        (borrowed: they must stay alive and unchanged while this context uses them)."""
        L = lib()
        self._keep = []
        first = True
        for p in parts:
            ptr, rows, dims, where, keep = _slice_pointer(p)
            if first:
                self._check(L.km_set_data(self._h, ptr, rows, dims, where))
                first = False
            else:
                self._check(L.km_append_data(self._h, ptr, rows, where))
            if where == KM_DEVICE:
                self._keep.append(keep)
        self.rows = int(L.km_rows(self._h))
        self.dims = int(L.km_dims(self._h))

    # ---- passes
    def run_pass(self, C, mode=KM_EXACT, path=KM_PATH_AUTO, labels=False, best=False):
        """-> (tot (k, d+2) float64, labels uint32 or None, best float32 or None)."""
        C = np.ascontiguousarray(C, dtype=np.float32)
        k = C.shape[0]
        tot = np.empty((k, self.dims + 2), np.float64)
        lab = np.empty(self.rows, np.uint32) if labels else None
        bst = np.empty(self.rows, np.float32) if best else None
        self._check(lib().km_pass(self._h, _ptr(C, ctypes.c_float), k, mode, path, _ptr(tot, ctypes.c_double),
                                  _ptr(lab, ctypes.c_uint32) if lab is not None else None,
                                  _ptr(bst, ctypes.c_float) if bst is not None else None))
        return tot, lab, bst

    def lloyd_step(self, C, mode=KM_EXACT, path=KM_PATH_AUTO):
        C = np.ascontiguousarray(C, dtype=np.float32)
        out = np.empty_like(C)
        inertia = ctypes.c_double()
        n_empty = ctypes.c_int32()
        self._check(lib().km_lloyd_step(self._h, _ptr(C, ctypes.c_float), C.shape[0], mode, path,
                                        _ptr(out, ctypes.c_float), ctypes.byref(inertia), ctypes.byref(n_empty)))
        return out, inertia.value, n_empty.value

    def fit(self, C0, max_iter, tol, mode=KM_EXACT, spherical=False):
        """-> (C, last_inertia, n_iter, n_relocated): the GPU-resident Lloyd loop."""
        C0 = np.ascontiguousarray(C0, dtype=np.float32)
        out = np.empty_like(C0)
        inertia = ctypes.c_double()
        n_iter = ctypes.c_int32()
        n_rel = ctypes.c_int32()
        self._check(lib().km_fit(self._h, _ptr(C0, ctypes.c_float), C0.shape[0], int(max_iter), float(tol), mode,
                                 1 if spherical else 0, _ptr(out, ctypes.c_float), ctypes.byref(inertia),
                                 ctypes.byref(n_iter), ctypes.byref(n_rel)))
        return out, inertia.value, n_iter.value, n_rel.value

    def seed_pp(self, k, sample, first, seeds):
        """-> (k, dims) float32: greedy k-means++ on the device over the sample rows (ascending global row
        indices), starting from sample[first], with k - 1 per-round uint64 seeds."""
        sample = np.ascontiguousarray(sample, dtype=np.int64)
        seeds = np.ascontiguousarray(seeds, dtype=np.uint64)
        if seeds.size == 0:
            seeds = np.zeros(1, np.uint64)
        out = np.empty((int(k), self.dims), np.float32)
        self._check(lib().km_seed_pp(self._h, int(k), _ptr(sample, ctypes.c_int64), sample.shape[0], int(first),
                                     _ptr(seeds, ctypes.c_uint64), _ptr(out, ctypes.c_float)))
        return out

    # ---- per-centre bounds (the reference's Elkan bounds, core.py:1690-2015)
    def bounds(self, max_visited):
        """Sets the gate of the bounds path: a pass runs on the bounds while a sample says at most this fraction
        of (row, centre) pairs needs scoring (the reference's BOUNDS_MAX_VISITED); 0 turns them off."""
        self._check(lib().km_bounds(self._h, float(max_visited)))

    def bounds_info(self):
        """-> dict(tracked, on_bounds, builds, last_fraction) since the data was set."""
        t, b, u = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        f = ctypes.c_double()
        self._check(lib().km_bounds_info(self._h, ctypes.byref(t), ctypes.byref(b), ctypes.byref(u),
                                         ctypes.byref(f)))
        return {"tracked": t.value, "on_bounds": b.value, "builds": u.value, "last_fraction": f.value}

    # ---- timing and diagnostics
    def profile(self, enable=True):
        self._check(lib().km_profile(self._h, 1 if enable else 0))

    def profile_read(self):
        """-> {kernel name: (total ms, launches)} for kernels launched since profile(True)."""
        L = lib()
        out = {}
        i = 0
        while True:
            name = L.km_kernel_name(i).decode()
            if not name:
                break
            ms = ctypes.c_double()
            cnt = ctypes.c_int64()
            self._check(L.km_profile_read(self._h, i, ctypes.byref(ms), ctypes.byref(cnt)))
            if cnt.value:
                out[name] = (ms.value, cnt.value)
            i += 1
        return out

    def profile_passes(self):
        """-> float64 array of per-pass milliseconds of the fit loops run since profile(True)."""
        L = lib()
        n = int(L.km_profile_passes(self._h, None, 0))
        out = np.zeros(max(n, 1), np.float64)
        if n:
            L.km_profile_passes(self._h, _ptr(out, ctypes.c_double), n)
        return out[:n]

    def stream_probe(self, nbytes=1 << 30, reps=10):
        """-> GB/s of a plain streaming read of a fresh nbytes array (the best grid's median of reps)."""
        g = ctypes.c_double()
        self._check(lib().km_stream_probe(self._h, int(nbytes), int(reps), ctypes.byref(g)))
        return g.value

    def last_path(self):
        return {KM_PATH_ROWS: "rows", KM_PATH_MFMA: "mfma", KM_PATH_FUSED: "fused"}.get(
            int(lib().km_last_path(self._h)), "none")

    def fallback_rows(self):
        return int(lib().km_last_fallback_rows(self._h))


def _slice_pointer(p):
    """-> (pointer, rows, dims, where, object to keep alive) for one slice."""
    mod = type(p).__module__
    if mod.startswith("torch"):
        import torch
        if p.dim() != 2:
            raise ValueError(f"each part must be 2-D (rows, dims), got {p.dim()}-D")
        if p.dtype != torch.float32 or not p.is_contiguous():
            p = p.to(torch.float32).contiguous()
        if p.is_cuda:
            torch.cuda.synchronize(p.device)   # the library reads it on its own stream
            return ctypes.c_void_p(p.data_ptr()), p.shape[0], p.shape[1], KM_DEVICE, p
        p = p.numpy()
    a = np.ascontiguousarray(p, dtype=np.float32)
    if a.ndim != 2:
        raise ValueError(f"each part must be 2-D (rows, dims), got {a.ndim}-D")
    return a.ctypes.data_as(ctypes.c_void_p), a.shape[0], a.shape[1], KM_HOST, a
