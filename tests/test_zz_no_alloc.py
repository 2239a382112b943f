"""om_layernorm_bwd_noalloc: the allocation-free variant of om_layernorm_bwd, on the GPU through the C ABI.

Its results must equal om_layernorm_bwd's bit for bit (same kernels, same fixed-order sums, the partials only moved
into the library's fixed device array), on two calls in a row with the second smaller than the first (the array
keeps the first call's partials, which the second must not read); it must not allocate device memory (a fresh
context's first om_layernorm_bwd grows the context scratch, the allocation-free call does not); a shape whose
partials exceed the fixed array is refused before anything runs; two contexts whose calls run at the same time on
one GPU (separate streams) each get om_layernorm_bwd's bits, since each holds a slot of its own; and a context that
finds every slot held by other live contexts is refused until one of them is destroyed.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

OM_E_ARG = 1
OM_E_STATE = 4
FIXED_BYTES = 8 << 20  # OM_NOALLOC_SCRATCH_BYTES: one context's slot
SLOTS = 4  # OM_NOALLOC_SLOTS


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


def test_noalloc_contexts_on_one_gpu_do_not_race():
    from gpu_util import Dev
    a, b = Dev(), Dev()  # two contexts, two streams, one GPU
    try:
        rng = np.random.default_rng(5)
        rows, cols = 4096, 768
        ca, cb = _case(a, rng, rows, cols), _case(b, rng, rows, cols)
        a.ctx.sync()
        b.ctx.sync()
        for _ in range(3):  # queued back to back on both streams, so the kernels of the two contexts overlap
            _run(a, "om_layernorm_bwd_noalloc", ca[0], ca[1][1], rows, cols, 0, 0)
            _run(b, "om_layernorm_bwd_noalloc", cb[0], cb[1][1], rows, cols, 0, 0)
        a.ctx.sync()
        b.ctx.sync()
        for dev, (bufs, outs) in ((a, ca), (b, cb)):
            _run(dev, "om_layernorm_bwd", bufs, outs[0], rows, cols, 0, 0)
            for ref, got in zip(outs[0], outs[1]):
                assert np.array_equal(dev.get(ref).view(np.uint32), dev.get(got).view(np.uint32))
    finally:
        a.ctx.close()
        b.ctx.close()


def test_noalloc_slots_are_per_live_context():
    from gpu_util import Dev
    devs = [Dev() for _ in range(SLOTS + 1)]
    try:
        rng = np.random.default_rng(9)
        rows, cols = 64, 384
        cases = [_case(d, rng, rows, cols) for d in devs]
        for d, (bufs, outs) in zip(devs[:SLOTS], cases):
            _run(d, "om_layernorm_bwd_noalloc", bufs, outs[1], rows, cols, 0, 0)
        last, (bufs, outs) = devs[SLOTS], cases[SLOTS]
        dg = outs[1][1]
        before = last.get(dg)
        st = last.status("om_layernorm_bwd_noalloc", *bufs, *outs[1], rows, cols, 0, 0)
        assert st == OM_E_STATE and b"slots" in last.ctx.L.om_last_error(last.ctx.h)
        assert np.array_equal(last.get(dg), before)  # nothing ran
        devs[0].ctx.close()  # its slot is released
        _run(last, "om_layernorm_bwd_noalloc", bufs, outs[1], rows, cols, 0, 0)
        _run(last, "om_layernorm_bwd", bufs, outs[0], rows, cols, 0, 0)
        for ref, got in zip(outs[0], outs[1]):
            assert np.array_equal(last.get(ref).view(np.uint32), last.get(got).view(np.uint32))
    finally:
        for d in devs[1:]:
            d.ctx.close()
