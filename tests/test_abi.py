"""The C ABI: the library loads and exports every entry point include/kmeans_hip.h declares, and the ctypes
binding declares each of them. No compute calls: this runs without a GPU."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kmeans_hip.h")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(km_[a-z_]+)\s*\(", src)))


def test_header_declares_the_entry_points():
    names = declared()
    for must in ("km_create", "km_destroy", "km_set_data", "km_pass", "km_lloyd_step", "km_fit", "km_last_error"):
        assert must in names


def test_binding_covers_header():
    from mlx_kmeans import _lib
    bound = sorted(n for n, _, _ in _lib.SIGNATURES)
    assert bound == declared()


def test_library_exports_every_symbol():
    from mlx_kmeans import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} is not built: run __graft_entry__.build()")
    L = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared():
        assert hasattr(L, name), name
    L.km_version.restype = ctypes.c_int32
    assert L.km_version() == 1
    L.km_kernel_name.restype = ctypes.c_char_p
    L.km_kernel_name.argtypes = [ctypes.c_int32]
    assert L.km_kernel_name(0) and L.km_kernel_name(10**6) == b""


def test_create_without_a_gpu_returns_null():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    from mlx_kmeans import _lib
    L = _lib.lib()
    assert not L.km_create(0)
    assert L.km_last_error(None) == b"no context"
