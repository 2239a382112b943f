"""CPU checks of the boundary: both libraries load, export every symbol the headers declare, report errors without
a device, and the tape's host generator equals the oracle's (the reference's SplitMix64 and init formula)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from gpu_util import ROOT, load_pkg


def declared(header):
    src = open(os.path.join(ROOT, "include", header)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)  # declarations only, not prose
    return sorted(set(re.findall(r"\b(omt?_[a-z0-9_]+)\s*\(", src)) - {"om_status"})


def test_hip_library_exports_every_declared_symbol():
    pkg = load_pkg()
    L = pkg.load_hip()
    names = declared("om.h")
    assert len(names) >= 50
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(pkg.om_symbols())  # the ctypes binding covers the header exactly
    assert L.om_abi_version() == 105


def test_train_library_exports_every_declared_symbol():
    pkg = load_pkg()
    L = pkg.load_train()
    names = declared("om_train.h")
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(pkg.omt_symbols())


def test_errors_without_a_device_are_reported():
    pkg = load_pkg()
    L = pkg.load_hip()
    h = C.c_void_p()
    st = L.om_ctx_create(0, C.byref(h))
    if st == 0:
        L.om_ctx_destroy(h)
        pytest.skip("a device is present")
    assert st == 3 and b"device" in L.om_last_error(None)
    T = pkg.load_train()
    m = C.c_void_p()
    assert T.omt_config_create(0, 3, None, C.byref(m)) != 0 and T.omt_last_error(None)
    assert L.om_gemm(None, 0, 0, 1, 1, 1, None, 1, None, 1, None, 1, None, 0, None) == 1


def test_tape_generator_equals_oracle(oracle):
    pkg = load_pkg()
    T = pkg.load_train()
    for kind, lo, hi in ((0, -0.05, 0.05), (1, 0.0, 0.0), (2, 1, 37)):
        n = 4099
        out = np.empty(n, np.int32 if kind == 2 else np.float32)
        T.omt_generate(20261301, kind, lo, hi, out.ctypes.data, n)
        g = oracle.Generator(20261301)
        ref = g.uniform(lo, hi, (n,)) if kind == 0 else g.normal((n,)) if kind == 1 else g.ints(int(lo), int(hi), (n,))
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_adam_scalars_host_helper_matches_oracle(oracle):
    L = load_pkg().load_hip()
    for t in (1, 2, 10, 1000, 123456):
        a, b = C.c_float(), C.c_float()
        L.om_adam_scalars(1e-3, 0.9, 0.999, t, C.byref(a), C.byref(b))
        c, d = C.c_float(), C.c_float()
        oracle.lib().or_adam_scalars(C.c_float(1e-3), C.c_float(0.9), C.c_float(0.999), C.c_int64(t), C.byref(c),
                                     C.byref(d))
        assert (a.value, b.value) == (c.value, d.value)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus above 1 (or a WORLD_SIZE above 1 from a launcher) exits with status 2 and a
    message saying so, before it loads the library or touches a device."""
    import subprocess
    import sys
    for args, env in ((["--gpus", "2"], {}), (["--gpus", "1"], {"WORLD_SIZE": "8"})):
        r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                           env={**os.environ, **env}, timeout=120)
        assert r.returncode == 2, (args, env, r.stdout, r.stderr)
        assert "one GPU only" in r.stderr and r.stdout == ""
