"""Gradient clipping and learning-rate schedules (Schedules.cs:9-422), CPU only.

The oracle is pinned against the reference's `optim` fixture with the reference's own bars (OptimizerTests.cs:93-150:
ClipNorm 1e-6 on gradients and norm, ClipValue exact, schedules 1e-6 relative over 100 steps) and against closed
forms and an independent norm routine; the product's schedules (C++ in libom_train.so, host only) must equal the
oracle's rates bit for bit.
"""
import math

import numpy as np
import pytest

from conftest import load_golden, scaled
from gpu_util import load_pkg
from oracle import schedules as S


def fixture_params(T, o):
    p = T.Tensor(o["in.p"].copy(), requires_grad=True)
    q = T.Tensor(o["in.q"].copy(), requires_grad=True)
    p.grad = o["in.grad.p.0"].copy()
    q.grad = o["in.grad.q.0"].copy()
    return p, q


def grads_of(T, *arrays):
    out = []
    for a in arrays:
        t = T.Tensor(np.zeros(np.shape(a), np.float32), requires_grad=True)
        t.grad = None if a is None else np.asarray(a, np.float32).copy()
        out.append(t)
    return out


# ---------------------------------------------------------------------------------------------- ClipNorm / ClipValue
@pytest.mark.parametrize("label,max_norm,inf", [("norm_small", 0.5, False), ("norm_large", 100.0, False),
                                                ("norm_inf", 0.7, True)])
def test_clip_norm_matches_reference_fixture(oracle, label, max_norm, inf):
    o = load_golden("training_optim")
    p, q = fixture_params(oracle, o)
    total, _ = oracle.clip_grad_norm([p, q], max_norm, inf)
    e = max(scaled(p.grad, o[f"out.clip.{label}.p"]), scaled(q.grad, o[f"out.clip.{label}.q"]))
    want = float(o[f"out.clip.{label}.total"][0])
    assert e <= 1e-6 and abs(float(total) - want) / want <= 1e-6, (label, e, total, want)


def test_clip_value_matches_reference_fixture_exactly(oracle):
    o = load_golden("training_optim")
    p, q = fixture_params(oracle, o)
    oracle.clip_grad_value([p, q], 0.6)
    assert np.array_equal(p.grad, o["out.clip.value.p"]) and np.array_equal(q.grad, o["out.clip.value.q"])


def test_clip_norm_closed_forms(oracle):
    T = oracle
    # 3-4-5 across two parameters: the norm spans every gradient, exactly 5; the scale is 1 below 5/(5+1e-6).
    a, b = grads_of(T, [3.0], [4.0])
    total, coef = T.clip_grad_norm([a, b], 10.0)
    assert total == 5.0 and coef >= 1.0 and a.grad[0] == 3.0 and b.grad[0] == 4.0
    a, b = grads_of(T, [3.0], [4.0])
    total, coef = T.clip_grad_norm([a, b], 1.0)
    assert total == 5.0 and 0.2 * (1 - 1e-6) < coef < 0.2
    assert a.grad[0] == np.float32(3.0) * coef and b.grad[0] == np.float32(4.0) * coef
    # Infinity norm: the largest magnitude wherever it is, sign ignored.
    a, b = grads_of(T, [-7.0, 2.0], [3.0])
    total, _ = T.clip_grad_norm([a, b], 1e3, infinity_norm=True)
    assert total == 7.0
    # A parameter without a gradient is skipped.
    a, b = grads_of(T, [3.0], None)
    total, _ = T.clip_grad_norm([a, b], 10.0)
    assert total == 3.0
    # Nothing at all: norm 0, nothing scaled.
    (a,) = grads_of(T, None)
    total, coef = T.clip_grad_norm([a], 1.0)
    assert total == 0.0 and coef > 1.0
    with pytest.raises(ValueError):
        T.clip_grad_norm([a], 0.0)


@pytest.mark.parametrize("inf", [False, True])
@pytest.mark.parametrize("bad", [np.nan, np.inf])
def test_clip_norm_non_finite_scales_nothing(oracle, inf, bad):
    T = oracle
    g = np.random.default_rng(1).standard_normal(1000).astype(np.float32)
    g[417] = bad
    (a,) = grads_of(T, g)
    total, coef = T.clip_grad_norm([a], 1e-3, infinity_norm=inf)
    assert (np.isnan(total) if np.isnan(bad) else total == np.inf) and coef == 1.0
    assert np.array_equal(a.grad.view(np.uint32), g.view(np.uint32))


def test_clip_norm_against_independent_norm(oracle):
    """The serial double sum against numpy's own 2-norm and max-abs in float64 (a different summation)."""
    T = oracle
    rng = np.random.default_rng(7)
    arrays = [rng.standard_normal(n).astype(np.float32) * s for n, s in ((5000, 1.0), (33, 1e3), (70001, 1e-3))]
    flat = np.concatenate([x.astype(np.float64) for x in arrays])
    for inf, ref in ((False, float(np.linalg.norm(flat))), (True, float(np.max(np.abs(flat))))):
        ps = grads_of(T, *arrays)
        total, coef = T.clip_grad_norm(ps, 1e6, infinity_norm=inf)
        assert abs(float(total) - ref) <= 2 ** -24 * ref, (inf, total, ref)
        for p, x in zip(ps, arrays):
            assert np.array_equal(p.grad, x)  # far below the maximum: untouched


def test_clip_value_rules(oracle):
    T = oracle
    g = np.array([0.5, -0.5, 0.7, -0.7, np.nan, np.inf, -np.inf, 0.0], np.float32)
    (a,) = grads_of(T, g)
    T.clip_grad_value([a], 0.6)
    want = np.array([0.5, -0.5, 0.6, -0.6, np.nan, 0.6, -0.6, 0.0], np.float32)
    assert np.array_equal(a.grad, want, equal_nan=True)
    with pytest.raises(ValueError):
        T.clip_grad_value([a], -1.0)


# ---------------------------------------------------------------------------------------------- schedules
FIXTURE_SCHEDULES = {
    "step": lambda: S.Step(0.1, 10, 0.5),
    "cosine": lambda: S.Cosine(0.1, 100, 1e-3),
    "warmup_cosine": lambda: S.Warmup(S.Cosine(0.1, 90, 1e-3), 10, 0.01),
    "onecycle": lambda: S.OneCycle(0.1, 100),
}


@pytest.mark.parametrize("name", sorted(FIXTURE_SCHEDULES))
def test_schedules_match_reference_fixture(name):
    want = load_golden("training_optim")["out.lr." + name]
    s = FIXTURE_SCHEDULES[name]()
    worst = max(abs(float(s.lr_at(i)) - float(w)) / float(w) for i, w in enumerate(want))
    assert worst <= 1e-6, (name, worst)


def test_cos_series_accuracy_and_symmetry():
    worst = max(abs(S.cos_pi(i / 10000.0) - math.cos(math.pi * i / 10000.0)) for i in range(10001))
    assert worst < 1e-15
    assert S.cos_pi(0.0) == 1.0 and S.cos_pi(1.0) == -1.0 and abs(S.cos_pi(0.5)) < 1e-15
    assert S.cos_pi(-3.0) == 1.0 and S.cos_pi(7.0) == -1.0 and S.cos_pi(float("nan")) == 1.0
    for t in (0.125, 0.25, 0.375, 0.4375):  # dyadic, so 1 - (1 - t) == t and the reduction is exact
        assert S.cos_pi(1.0 - t) == -S.cos_pi(t)


def test_schedule_closed_forms():
    base = S.f32(0.1)
    s = S.WarmupCosine(0.1, 10, 110)
    assert [float(s.lr_at(i)) for i in range(3)] == [float(np.float32(base * k / 10)) for k in (1, 2, 3)]
    assert s.lr_at(9) == np.float32(0.1) and s.lr_at(10) == np.float32(0.1)  # peak at the end of the warm-up
    assert abs(float(s.lr_at(60)) - base / 2) <= 1e-7 * base  # half-way down the half cosine
    assert s.lr_at(110) == 0.0 and s.lr_at(10 ** 9) == 0.0
    f = S.WarmupCosine(0.1, 10, 110, 0.25)
    assert abs(float(f.lr_at(110)) - 0.25 * base) <= 1e-7 * base
    st = S.Step(0.1, 3, 0.5)
    assert [float(st.lr_at(i)) for i in (0, 2, 3, 6, 9)] == [float(np.float32(base * 0.5 ** k)) for k in (0, 0, 1, 2, 3)]
    c = S.Cosine(0.1, 100)
    assert c.lr_at(0) == np.float32(0.1) and c.lr_at(100) == 0.0 and c.lr_at(-4) == c.lr_at(0)
    oc = S.OneCycle(0.1, 100)
    assert abs(float(oc.lr_at(0)) - base / 25) <= 1e-7 * base
    assert oc.lr_at(29) == np.float32(0.1)  # the peak sits at pct_start * total - 1
    assert abs(float(oc.lr_at(99)) - base / 25 / 1e4) <= 1e-6 * base / 25 / 1e4
    w = S.Warmup(S.Constant(0.2), 4, 0.5)
    assert [float(w.lr_at(i)) for i in range(6)] == [float(np.float32(S.f32(0.2) * (0.5 + 0.5 * k / 4)))
                                                     for k in range(4)] + [float(np.float32(0.2))] * 2


def product_schedules(pkg):
    P = pkg.LrSchedule
    return [
        (P.constant(0.03), S.Constant(0.03)),
        (P.step(0.1, 10, 0.5), S.Step(0.1, 10, 0.5)),
        (P.step(0.3, 1, 0.97), S.Step(0.3, 1, 0.97)),
        (P.cosine(0.1, 100, 1e-3), S.Cosine(0.1, 100, 1e-3)),
        (P.cosine(0.7, 1), S.Cosine(0.7, 1)),
        (P.warmup(P.cosine(0.1, 90, 1e-3), 10, 0.01), S.Warmup(S.Cosine(0.1, 90, 1e-3), 10, 0.01)),
        (P.warmup(P.step(0.05, 7, 0.3), 3), S.Warmup(S.Step(0.05, 7, 0.3), 3)),
        (P.warmup_cosine(0.1, 10, 100, 0.1), S.WarmupCosine(0.1, 10, 100, 0.1)),
        (P.warmup_cosine(3e-4, 1, 2), S.WarmupCosine(3e-4, 1, 2)),
        (P.onecycle(0.1, 100), S.OneCycle(0.1, 100)),
        (P.onecycle(0.01, 37, 0.2, 10.0, 100.0), S.OneCycle(0.01, 37, 0.2, 10.0, 100.0)),
        (P.onecycle(0.01, 2, 0.1), S.OneCycle(0.01, 2, 0.1)),
    ]


def test_product_schedules_equal_oracle_bit_for_bit():
    pkg = load_pkg()
    steps = list(range(-3, 400)) + [10 ** 6, 2 ** 40]
    for prod, ref in product_schedules(pkg):
        got = np.array([prod.lr_at(i) for i in steps], np.float32)
        want = np.array([ref.lr_at(i) for i in steps], np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), type(ref).__name__
    L = pkg.load_train()
    ts = [i / 997.0 for i in range(998)] + [-1.0, 2.0, float("nan")]
    assert all(L.omt_lr_cos(t) == S.cos_pi(t) for t in ts)


@pytest.mark.parametrize("make", [
    lambda P: P.step(0.1, 0), lambda P: P.cosine(0.1, 0), lambda P: P.warmup(P.constant(0.1), 0),
    lambda P: P.warmup_cosine(0.1, 0, 10), lambda P: P.warmup_cosine(0.1, 10, 10),
    lambda P: P.warmup_cosine(0.1, 1, 10, -0.5), lambda P: P.warmup_cosine(0.1, 1, 10, 1.5),
    lambda P: P.onecycle(0.1, 1), lambda P: P.onecycle(0.1, 10, 0.0), lambda P: P.onecycle(0.1, 10, 1.0),
])
def test_product_schedules_reject_what_the_reference_rejects(make):
    pkg = load_pkg()
    with pytest.raises(pkg.OmError):
        make(pkg.LrSchedule)
