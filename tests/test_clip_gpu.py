"""Device gradient clipping (om_clip_grad_norm, om_clip_grad_value, om_adam_step_scaled) and the tape's clip and
schedule hooks, against the CPU oracle's restatement of GradClip (Schedules.cs:22-149), on the GPU.

Bars: the norm within 1e-6 relative of the oracle's serial double sum (the reference's own ClipNorm bar,
OptimizerTests.cs:93-104) — both round the same fp64 value to float, so it is normally equal; the coefficient within
one float ulp of the oracle's and every clipped gradient exactly g * coef; ClipValue bit-exact; the fused AdamW equal
to clip-then-step bit for bit. Full size (the C5 parameter arena, 28.36M gradients) is checked against an independent
float64 norm.
"""
import ctypes as C

import numpy as np
import pytest

from conftest import scaled

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    from gpu_util import Dev
    d = Dev()
    yield d
    d.ctx.close()


@pytest.fixture(scope="module")
def T():
    from oracle import tape
    return tape


def table(ptrs, lens):
    P = (C.c_void_p * max(len(ptrs), 1))(*ptrs)
    N = (C.c_int64 * max(len(lens), 1))(*lens)
    return P, N


def ulp(x):
    return float(np.spacing(np.float32(abs(x))))


def oracle_clip(T, arrays, max_norm, inf):
    ts = []
    for a in arrays:
        t = T.Tensor(np.zeros(1, np.float32), requires_grad=True)
        t.grad = None if a is None else a.copy()
        ts.append(t)
    total, coef = T.clip_grad_norm(ts, max_norm, inf)
    return float(total), float(coef), [t.grad for t in ts]


def device_clip(dev, arrays, max_norm, inf, offsets=None, in_place=1):
    """Uploads each array (at a float offset inside its buffer when asked, to test unaligned segments), clips on the
    device and returns (norm, coef, clipped arrays)."""
    bufs, ptrs, lens = [], [], []
    for i, a in enumerate(arrays):
        if a is None:
            ptrs.append(None)
            lens.append(0)
            continue
        off = offsets[i] if offsets else 0
        b = dev.put(np.concatenate([np.zeros(off, np.float32), a]))
        bufs.append((b, off, a.size))
        ptrs.append(b.data_ptr() + 4 * off)
        lens.append(a.size)
    out = dev.empty((2,), fill=-1.0)
    P, N = table(ptrs, lens)
    dev.call("om_clip_grad_norm", len(arrays), C.cast(P, C.c_void_p), C.cast(N, C.c_void_p), C.c_float(max_norm),
             int(inf), in_place, out.data_ptr(), out.data_ptr() + 4)
    total, coef = dev.get(out)
    res, k = [], 0
    for a in arrays:
        if a is None:
            res.append(None)
            continue
        b, off, n = bufs[k]
        k += 1
        res.append(dev.get(b)[off:off + n])
    return float(total), float(coef), res


SIZES = [[1000], [1, 3, 8191, 8192, 8193], [100_003, 0, 77, 65_536 * 3 + 5], [5] * 40 + [20_000] * 5]


@pytest.mark.parametrize("inf", [False, True])
@pytest.mark.parametrize("sizes", SIZES, ids=lambda s: f"{len(s)}seg-{sum(s)}")
@pytest.mark.parametrize("unaligned", [False, True])
def test_clip_norm_parity(dev, T, sizes, inf, unaligned):
    rng = np.random.default_rng(sum(sizes) + 7 * len(sizes) + inf)
    arrays = [(rng.standard_normal(n) * rng.uniform(0.1, 10)).astype(np.float32) if n else None for n in sizes]
    offsets = [(3 * i + 1) % 4 for i in range(len(sizes))] if unaligned else None
    for max_norm in (0.25, 1e9):
        t_or, c_or, g_or = oracle_clip(T, arrays, max_norm, inf)
        t_dev, c_dev, g_dev = device_clip(dev, arrays, max_norm, inf, offsets)
        assert abs(t_dev - t_or) <= 1e-6 * t_or, (t_dev, t_or)
        assert abs(c_dev - c_or) <= ulp(c_or), (c_dev, c_or)
        for a, gd, go in zip(arrays, g_dev, g_or):
            if a is None:
                continue
            want = a * np.float32(c_dev) if c_dev < 1.0 else a
            assert np.array_equal(gd.view(np.uint32), want.view(np.uint32))
            assert scaled(gd, go) <= 1e-6


@pytest.mark.parametrize("bad", [np.nan, np.inf])
@pytest.mark.parametrize("inf", [False, True])
def test_clip_norm_non_finite(dev, T, bad, inf):
    rng = np.random.default_rng(3)
    a = rng.standard_normal(50_000).astype(np.float32)
    a[31_337] = bad
    t_dev, c_dev, (g,) = device_clip(dev, [a], 1e-3, inf)
    assert (np.isnan(t_dev) if np.isnan(bad) else t_dev == np.inf) and c_dev == 1.0
    assert np.array_equal(g.view(np.uint32), a.view(np.uint32))


def test_clip_norm_empty_and_errors(dev):
    t_dev, c_dev, _ = device_clip(dev, [None, np.zeros(0, np.float32)], 1.0, False)
    assert t_dev == 0.0 and c_dev > 1.0
    P, N = table([None], [0])
    out = dev.empty((2,))
    assert dev.status("om_clip_grad_norm", 1, C.cast(P, C.c_void_p), C.cast(N, C.c_void_p), C.c_float(0.0), 0, 1,
                      out.data_ptr(), None) == 1
    assert dev.status("om_clip_grad_norm", 1, C.cast(P, C.c_void_p), C.cast(N, C.c_void_p), C.c_float(1.0), 0, 0,
                      out.data_ptr(), None) == 1
    P, N = table([out.data_ptr()], [-1])
    assert dev.status("om_clip_grad_norm", 1, C.cast(P, C.c_void_p), C.cast(N, C.c_void_p), C.c_float(1.0), 0, 1,
                      None, None) == 1
    assert dev.status("om_clip_grad_value", 1, C.cast(P, C.c_void_p), C.cast(N, C.c_void_p), C.c_float(-1.0)) == 1


def test_clip_norm_full_arena_size(dev, T):
    """The C5 arena's 28.36M gradients in one segment: against numpy's float64 2-norm and the oracle."""
    n = 28_358_409
    rng = np.random.default_rng(11)
    a = (rng.standard_normal(n, dtype=np.float32) * np.float32(1e-3))
    ref = float(np.linalg.norm(a.astype(np.float64)))
    t_or, c_or, _ = oracle_clip(T, [a], 1.0, False)
    t_dev, c_dev, (g,) = device_clip(dev, [a], 1.0, False)
    assert abs(t_dev - ref) <= 2 ** -24 * ref and abs(t_dev - t_or) <= 1e-6 * t_or
    assert abs(c_dev - c_or) <= ulp(c_or)
    want = a * np.float32(c_dev) if c_dev < 1.0 else a
    assert np.array_equal(g.view(np.uint32), want.view(np.uint32))


def test_clip_value_bit_exact(dev, T):
    rng = np.random.default_rng(4)
    arrays = [rng.standard_normal(n).astype(np.float32) for n in (10_001, 3, 8192)]
    arrays[0][:6] = [np.nan, np.inf, -np.inf, 0.6, -0.6, -0.0]
    ts = []
    for a in arrays:
        t = T.Tensor(np.zeros(1, np.float32), requires_grad=True)
        t.grad = a.copy()
        ts.append(t)
    T.clip_grad_value(ts, 0.6)
    bufs = [dev.put(np.concatenate([np.zeros(1, np.float32), a])) for a in arrays]  # unaligned segments
    P, N = table([b.data_ptr() + 4 for b in bufs], [a.size for a in arrays])
    dev.call("om_clip_grad_value", len(arrays), C.cast(P, C.c_void_p), C.cast(N, C.c_void_p), C.c_float(0.6))
    for b, t in zip(bufs, ts):
        assert np.array_equal(dev.get(b)[1:].view(np.uint32), t.grad.view(np.uint32))


def test_adam_step_scaled_equals_clip_then_step(dev, T):
    """Clip folded into AdamW's read of g == in-place clip + AdamW, on the device and in the oracle, bit for bit."""
    rng = np.random.default_rng(9)
    n = 1_000_004
    p0, g0 = rng.standard_normal(n).astype(np.float32), (rng.standard_normal(n) * 0.1).astype(np.float32)
    ss, sq = C.c_float(), C.c_float()
    dev.ctx.L.om_adam_scalars(1e-3, 0.9, 0.999, 1, C.byref(ss), C.byref(sq))
    hyper = (C.c_float(1e-3), C.c_float(0.9), C.c_float(0.999), C.c_float(1e-8), C.c_float(0.01), 1, ss, sq)
    results = []
    for fused in (False, True):
        P, G, M, V = dev.put(p0), dev.put(g0), dev.empty((n,), fill=0.0), dev.empty((n,), fill=0.0)
        out = dev.empty((2,))
        Pt, Nt = table([G.data_ptr()], [n])
        dev.call("om_clip_grad_norm", 1, C.cast(Pt, C.c_void_p), C.cast(Nt, C.c_void_p), C.c_float(2.0), 0,
                 0 if fused else 1, out.data_ptr(), out.data_ptr() + 4)
        if fused:
            dev.call("om_adam_step_scaled", P, G, M, V, None, n, *hyper, out.data_ptr() + 4)
            assert np.array_equal(dev.get(G).view(np.uint32), g0.view(np.uint32))  # gradients left unscaled
        else:
            dev.call("om_adam_step", P, G, M, V, None, n, *hyper)
        results.append((dev.get(P), dev.get(M), dev.get(V), dev.get(out)))
    for a, b in zip(results[0], results[1]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # the oracle: ClipNorm then Adam.UpdateRange on the host
    t_or, c_or, (g_or,) = oracle_clip(T, [g0], 2.0, False)
    assert float(results[0][3][1]) == c_or  # same coefficient (the norms agree to the float)
    p, m, v = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    T.lib().or_adam_update(T.fp(p), T.fp(g_or), T.fp(m), T.fp(v), None, C.c_int64(n), *hyper)
    assert np.array_equal(results[1][0].view(np.uint32), p.view(np.uint32))


# ------------------------------------------------------------------------------------------------ the tape
@pytest.fixture(scope="module")
def pkg():
    from gpu_util import load_pkg
    return load_pkg()


@pytest.mark.parametrize("cfg,sc", [(1, {}), (3, {"batch": 2})], ids=["C1", "C3-batch2"])
@pytest.mark.parametrize("inf", [False, True])
def test_tape_clip_norm(pkg, T, cfg, sc, inf):
    a = pkg.Model(cfg, **sc)
    b = pkg.Model(cfg, **sc)
    try:
        names = [nm for nm, _ in a.params()]
        a.forward_backward()
        g = [a.read_param(i, 1) for i in range(len(names))]
        max_norm = 0.3 * oracle_clip(T, g, 1e30, inf)[0]  # a bound the norm exceeds, so the scaling runs
        norm = a.clip_grad_norm(max_norm, inf)
        t_or, c_or, g_or = oracle_clip(T, g, max_norm, inf)
        assert abs(norm - t_or) <= 1e-6 * t_or and c_or < 1.0
        for i in range(len(names)):
            assert scaled(a.read_param(i, 1), g_or[i]) <= 1e-6, names[i]
        a.optimizer_step()
        # the same step with ClipNorm folded into AdamW: identical parameters and moments, gradients unscaled
        b.set_clip(max_norm, inf)
        b.step()
        assert b.last_grad_norm() == norm
        for i in range(len(names)):
            for which in (0, 2, 3):
                assert np.array_equal(a.read_param(i, which).view(np.uint32), b.read_param(i, which).view(np.uint32))
            assert np.array_equal(b.read_param(i, 1).view(np.uint32), g[i].view(np.uint32))
    finally:
        a.close()
        b.close()


def test_tape_clip_value(pkg):
    m = pkg.Model(1)
    try:
        m.forward_backward()
        g = [m.read_param(i, 1) for i in range(len(m.params()))]
        m.clip_grad_value(1e-3)
        for i, gi in enumerate(g):
            want = np.where(gi > np.float32(1e-3), np.float32(1e-3), np.where(gi < -np.float32(1e-3),
                                                                               -np.float32(1e-3), gi))
            assert np.array_equal(m.read_param(i, 1).view(np.uint32), want.astype(np.float32).view(np.uint32))
    finally:
        m.close()


def test_tape_schedule_applies_before_each_step(pkg):
    """LrSchedule.Apply before every step equals setting the rate by hand to LrAt(step count)."""
    from oracle import schedules as S
    sched = pkg.LrSchedule.warmup_cosine(1e-3, 2, 6, 0.1)
    ref = S.WarmupCosine(1e-3, 2, 6, 0.1)
    a = pkg.Model(1)
    b = pkg.Model(1)
    try:
        a.set_schedule(sched)
        for k in range(4):
            a.step()
            assert a.lr == float(ref.lr_at(k))
            b.lr = float(ref.lr_at(k))
            b.step()
        for i in range(len(a.params())):
            assert np.array_equal(a.read_param(i).view(np.uint32), b.read_param(i).view(np.uint32))
        with pytest.raises(pkg.OmError):
            b.lr = float("nan")
    finally:
        a.close()
        b.close()
