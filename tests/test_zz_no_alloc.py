"""om_layernorm_bwd_noalloc: the allocation-free variant of om_layernorm_bwd, on the GPU through the C ABI.

Its results must equal om_layernorm_bwd's bit for bit (same kernels, same fixed-order sums, the partials only moved
into the library's fixed device array), on two calls in a row with the second smaller than the first (the array
keeps the first call's partials, which the second must not read); it must not allocate device memory (a fresh
context's first om_layernorm_bwd grows the context scratch, the allocation-free call does not); and a shape whose
partials exceed the fixed array is refused before anything runs.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

OM_E_ARG = 1
FIXED_BYTES = 8 << 20  # OM_NOALLOC_SCRATCH_BYTES


def _free_bytes():
    from gpu_util import hip
    h = hip()
    free, total = C.c_size_t(), C.c_size_t()
    h.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    assert h.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def _case(dev, rng, rows, cols):
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    g = rng.standard_normal((rows, cols)).astype(np.float32)
    gam = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    mu = x.mean(1).astype(np.float32)
    rs = (1 / np.sqrt(x.var(1) + 1e-5)).astype(np.float32)
    bufs = [dev.put(a) for a in (g, x, gam, mu, rs)]
    outs = [[dev.empty((rows, cols), fill=0.25), dev.empty((cols,), fill=0.5), dev.empty((cols,), fill=-0.5)]
            for _ in range(2)]
    return bufs, outs


def _run(dev, name, bufs, out, rows, cols, acc_dx, acc_p):
    st = dev.status(name, *bufs, *out, rows, cols, acc_dx, acc_p)
    assert st == 0, dev.ctx.L.om_last_error(dev.ctx.h)


def test_noalloc_equals_layernorm_bwd_and_allocates_nothing():
    from gpu_util import Dev
    dev = Dev()  # a fresh context: its scratch has never grown
    try:
        rng = np.random.default_rng(21)
        # C5's LayerNorm (4096 x 768: 3 MiB of partials), then a smaller, generic-width one on the same array
        shapes = [(4096, 768, 0, 0), (1000, 200, 1, 1)]
        cases = [_case(dev, rng, r, c) for r, c, _, _ in shapes]
        dev.ctx.sync()
        free0 = _free_bytes()
        for (rows, cols, acc_dx, acc_p), (bufs, outs) in zip(shapes, cases):
            _run(dev, "om_layernorm_bwd_noalloc", bufs, outs[1], rows, cols, acc_dx, acc_p)
        dev.ctx.sync()
        assert free0 - _free_bytes() < (16 << 20)  # no scratch growth (om_layernorm_bwd's first call takes 64 MiB)
        for (rows, cols, acc_dx, acc_p), (bufs, outs) in zip(shapes, cases):
            _run(dev, "om_layernorm_bwd", bufs, outs[0], rows, cols, acc_dx, acc_p)
            for ref, got in zip(outs[0], outs[1]):
                assert np.array_equal(dev.get(ref).view(np.uint32), dev.get(got).view(np.uint32)), (rows, cols)
        # and again, the smaller shape right after the larger one on the allocation-free path
        (bufs, outs) = cases[0]
        _run(dev, "om_layernorm_bwd_noalloc", bufs, outs[1], 4096, 768, 0, 0)
        rows, cols, acc_dx, acc_p = shapes[1]
        bufs, outs = cases[1]
        for o in outs:  # the same starting values for both paths (they accumulate)
            for b, v in zip(o, (0.25, 0.5, -0.5)):
                dev.call("om_fill", b, C.c_float(v), C.c_int64(b.nbytes // 4))
        _run(dev, "om_layernorm_bwd_noalloc", bufs, outs[1], rows, cols, acc_dx, acc_p)
        _run(dev, "om_layernorm_bwd", bufs, outs[0], rows, cols, acc_dx, acc_p)
        for ref, got in zip(outs[0], outs[1]):
            assert np.array_equal(dev.get(ref).view(np.uint32), dev.get(got).view(np.uint32))
    finally:
        dev.ctx.close()


def test_noalloc_refuses_partials_beyond_its_array():
    from gpu_util import Dev
    dev = Dev()
    try:
        cols = 768
        rows = (FIXED_BYTES // (16 * cols) + 1) * 16  # one 16-row chunk more than fits
        need = 16 * (rows // 16) * cols
        assert need > FIXED_BYTES
        small = [dev.empty((cols,)) for _ in range(5)]
        dg = dev.empty((cols,), fill=3.0)
        st = dev.status("om_layernorm_bwd_noalloc", *small, None, dg, None, rows, cols, 0, 0)
        assert st == OM_E_ARG and b"fixed scratch" in dev.ctx.L.om_last_error(dev.ctx.h)
        assert np.all(dev.get(dg) == 3.0)
    finally:
        dev.ctx.close()
