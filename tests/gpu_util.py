"""Helpers for the GPU tests: load the package (its directory name has a hyphen), a library context, and device
buffers. torch is used only to own device memory; every computation under test runs in lib/libom_hip.so."""
import ctypes as C
import importlib.util
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "onemodel-csharp_amd")


def load_pkg():
    if "onemodel_csharp_amd" in sys.modules:
        return sys.modules["onemodel_csharp_amd"]
    spec = importlib.util.spec_from_file_location("onemodel_csharp_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    m = importlib.util.module_from_spec(spec)
    sys.modules["onemodel_csharp_amd"] = m
    spec.loader.exec_module(m)
    return m


class Dev:
    """Device buffers from torch plus the library context; `sync()` orders torch's stream and the library's."""

    def __init__(self):
        import torch
        self.torch = torch
        self.pkg = load_pkg()
        self.ctx = self.pkg.Context(0)

    def put(self, a):
        t = self.torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
        self.torch.cuda.synchronize()
        return t

    def empty(self, shape, dtype=np.float32, fill=None):
        td = {np.float32: self.torch.float32, np.int32: self.torch.int32}[dtype]
        t = self.torch.empty(tuple(shape), dtype=td, device="cuda")
        if fill is not None:
            t.fill_(fill)
        self.torch.cuda.synchronize()
        return t

    def get(self, t):
        self.ctx.sync()
        self.torch.cuda.synchronize()
        return t.cpu().numpy()

    def call(self, name, *args):
        conv = [a.data_ptr() if hasattr(a, "data_ptr") else a for a in args]
        self.ctx.call(name, *conv)

    def status(self, name, *args):
        conv = [a.data_ptr() if hasattr(a, "data_ptr") else a for a in args]
        return getattr(self.ctx.L, name)(self.ctx.h, *conv)


def ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None
