"""Helpers for the GPU tests: load the package (its directory name has a hyphen), a library context, and device
buffers.

Device buffers come from the HIP runtime that lib/libom_hip.so itself links (/opt/rocm's libamdhip64), reached
through ctypes: no second GPU runtime is loaded into the test process (torch's wheel ships its own copies of the HIP
and HSA runtimes, and two runtimes in one process cannot both open the device). Every computation under test runs in
lib/libom_hip.so.
"""
import ctypes as C
import importlib.util
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# OM_TEST_PKG_DIR points the tests at another copy of the package (the sanitizer run of tests/test_sanitized_host.py
# loads a copy whose lib/libom_train.so is built with AddressSanitizer and UndefinedBehaviorSanitizer).
PKG_DIR = os.environ.get("OM_TEST_PKG_DIR") or os.path.join(ROOT, "onemodel-csharp_amd")


def load_pkg():
    if "onemodel_csharp_amd" in sys.modules:
        return sys.modules["onemodel_csharp_amd"]
    spec = importlib.util.spec_from_file_location("onemodel_csharp_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    m = importlib.util.module_from_spec(spec)
    sys.modules["onemodel_csharp_amd"] = m
    spec.loader.exec_module(m)
    return m


_HIP = None


def hip():
    """The HIP runtime libom_hip.so is linked against (already loaded with it, so the same instance)."""
    global _HIP
    if _HIP is None:
        load_pkg().load_hip()
        h = C.CDLL("libamdhip64.so.7")
        h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        h.hipFree.argtypes = [C.c_void_p]
        h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        h.hipDeviceSynchronize.argtypes = []
        _HIP = h
    return _HIP


H2D, D2H = 1, 2


class DevBuf:
    """A device allocation with a shape and dtype; `data_ptr()` is what the ABI calls take."""

    def __init__(self, shape, dtype):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self._p = C.c_void_p()
        st = hip().hipMalloc(C.byref(self._p), max(self.nbytes, 4))
        if st != 0:
            raise RuntimeError(f"hipMalloc({self.nbytes}) failed: {st}")

    def data_ptr(self):
        return self._p.value

    def __del__(self):
        try:
            if self._p:
                hip().hipDeviceSynchronize()
                hip().hipFree(self._p)
                self._p = C.c_void_p()
        except Exception:
            pass


class Dev:
    """Device buffers plus the library context."""

    def __init__(self):
        self.pkg = load_pkg()
        self.ctx = self.pkg.Context(0)
        self.hip = hip()

    def put(self, a):
        a = np.ascontiguousarray(a)
        b = DevBuf(a.shape, a.dtype)
        if b.nbytes:
            st = self.hip.hipMemcpy(b.data_ptr(), a.ctypes.data, b.nbytes, H2D)
            if st != 0:
                raise RuntimeError(f"hipMemcpy H2D failed: {st}")
        return b

    def empty(self, shape, dtype=np.float32, fill=None):
        if fill is not None:
            return self.put(np.full(tuple(shape), fill, dtype))
        return DevBuf(shape, dtype)

    def get(self, b):
        self.ctx.sync()
        out = np.empty(b.shape, b.dtype)
        if b.nbytes:
            st = self.hip.hipMemcpy(out.ctypes.data, b.data_ptr(), b.nbytes, D2H)
            if st != 0:
                raise RuntimeError(f"hipMemcpy D2H failed: {st}")
        return out

    def call(self, name, *args):
        conv = [a.data_ptr() if hasattr(a, "data_ptr") else a for a in args]
        self.ctx.call(name, *conv)

    def status(self, name, *args):
        conv = [a.data_ptr() if hasattr(a, "data_ptr") else a for a in args]
        return getattr(self.ctx.L, name)(self.ctx.h, *conv)


def ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None
