"""Pins the CPU oracle (oracle/) against the reference's own golden vectors and known answers (CPU only).

Fixtures are the reference's testdata files copied as data (tests/golden/PROVENANCE.md). Tolerances are the
reference's own: optimizer steps 1e-6 scaled (OptimizerTests.cs:55-75), model gradients 1e-4 scaled with the
zero-in-theory rule (AutogradModelTests.cs:32-81), CTC losses 1e-5 relative (RnnOracleTests.cs:86-127), training
curves 1e-3 (TrainingCurveTests.cs:75-106).
"""
import math

import numpy as np
import pytest

from conftest import load_golden, scaled


# ------------------------------------------------------------------------------------------------- optimizers
OPT_CONFIGS = {
    "sgd_plain": dict(kind="sgd", lr=0.1),
    "sgd_momentum": dict(kind="sgd", lr=0.1, momentum=0.9),
    "sgd_nesterov_wd": dict(kind="sgd", lr=0.1, momentum=0.9, wd=1e-2, nesterov=True),
    "sgd_dampening_wd": dict(kind="sgd", lr=0.05, momentum=0.8, dampening=0.5, wd=1e-3),
    "adam": dict(kind="adam", lr=1e-2),
    "adam_l2": dict(kind="adam", lr=1e-2, wd=0.1),
    "adam_amsgrad": dict(kind="adam", lr=1e-2, amsgrad=True),
    "adam_betas": dict(kind="adam", lr=3e-3, beta1=0.8, beta2=0.95, eps=1e-6),
    "adamw": dict(kind="adamw", lr=1e-2, wd=0.05),
    "adamw_amsgrad": dict(kind="adamw", lr=1e-2, wd=0.05, amsgrad=True),
}


def make_opt(T, params, c):
    c = dict(c)
    kind = c.pop("kind")
    if kind == "sgd":
        return T.Sgd(params, c["lr"], momentum=c.get("momentum", 0.0), dampening=c.get("dampening", 0.0),
                     wd=c.get("wd", 0.0), nesterov=c.get("nesterov", False))
    return T.AdamW(params, lr=c["lr"], beta1=c.get("beta1", 0.9), beta2=c.get("beta2", 0.999),
                   eps=c.get("eps", 1e-8), wd=c.get("wd", 0.01 if kind == "adamw" else 0.0),
                   decoupled=(kind == "adamw"), amsgrad=c.get("amsgrad", False))


@pytest.mark.parametrize("name", sorted(OPT_CONFIGS))
def test_optimizer_steps_match_reference_fixture(oracle, name):
    T = oracle
    o = load_golden("training_optim")
    p = T.Tensor(o["in.p"].copy(), requires_grad=True)
    q = T.Tensor(o["in.q"].copy(), requires_grad=True)
    opt = make_opt(T, [p, q], OPT_CONFIGS[name])
    for k in range(5):
        p.grad = o[f"in.grad.p.{k}"].copy()
        q.grad = o[f"in.grad.q.{k}"].copy()
        opt.step()
        if k in (0, 4):
            e = max(scaled(p.data, o[f"out.{name}.p.{k + 1}"]), scaled(q.data, o[f"out.{name}.q.{k + 1}"]))
            assert e <= 1e-6, (name, k, e)
    assert opt.step_count == 5


def test_adam_skips_parameters_without_gradient(oracle):
    T = oracle
    o = load_golden("training_optim")
    p = T.Tensor(o["in.p"].copy(), requires_grad=True)
    q = T.Tensor(o["in.q"].copy(), requires_grad=True)
    opt = T.AdamW([p, q], lr=1e-2, wd=0.0, decoupled=False)
    p.grad = o["in.grad.p.0"].copy()
    opt.step()
    assert np.array_equal(q.data, o["in.q"])
    assert not np.array_equal(p.data, o["in.p"])


def test_adam_scalars_closed_form(oracle):
    """BeginStep (Optimizers.cs:501-508) against the closed form: step 1 gives lr/(1-b1) and sqrt(1-b2)."""
    T = oracle
    opt = T.AdamW([T.Tensor(np.zeros(1, np.float32), True)], lr=1e-3)
    lr, b1, b2 = (float(np.float32(v)) for v in (1e-3, 0.9, 0.999))  # the float hyper-parameters, widened
    ss, sq = opt.scalars()
    assert ss == np.float32(lr / (1 - b1))
    assert sq == np.float32(math.sqrt(1 - b2))
    opt.step_count = 9
    ss, sq = opt.scalars()
    assert ss == np.float32(lr / (1 - b1 ** 10))
    assert abs(sq - math.sqrt(1 - b2 ** 10)) <= 1e-7


# ------------------------------------------------------------------------------------------------- model gradients
def compare_grads(o, grads, tol):
    largest = max(float(np.max(np.abs(o["grad." + k]))) for k in grads)
    worst = 0.0
    for k, g in grads.items():
        exp = o["grad." + k]
        assert g.shape == exp.shape, k
        if float(np.max(np.abs(exp))) < 1e-5 * largest:
            noise = float(np.max(np.abs(g))) / largest
            assert noise < 1e-5, (k, noise)
            continue
        e = scaled(g, exp)
        worst = max(worst, e)
        assert e <= tol, (k, e)
    return worst


def test_encoder_fixture(oracle):
    from oracle import models
    o = load_golden("autograd_encoder")
    loss, grads, y = models.encoder_fixture(o)
    ref = float(o["out.loss"][0])
    assert abs(loss - ref) <= abs(ref) * 1e-4
    assert scaled(y, o["out.y"]) < 1e-4
    assert compare_grads(o, grads, 1e-4) < 1e-4


def test_cnn_fixture(oracle):
    from oracle import models
    o = load_golden("autograd_cnn")
    loss, grads, stats = models.cnn_fixture(o)
    assert abs(loss - float(o["out.loss"][0])) <= 1e-5
    compare_grads(o, grads, 1e-4)
    assert scaled(stats["rm1"], o["out.rm1"]) < 1e-5
    assert scaled(stats["rv2"], o["out.rv2"]) < 1e-5


def test_mse_mean_sub_permute_closed_forms(oracle):
    """The C3 loss path and the view backward, pinned by closed forms: Mse = Mean((p - t)^2) with the double sum of
    the squares, dL/dp = 2 (p - t) / n and dL/dt = -dL/dp (one float rounding of each factor apart); Permute backward
    applies the inverse permutation exactly."""
    T = oracle
    rng = np.random.default_rng(11)
    p = rng.standard_normal((3, 5, 4)).astype(np.float32)
    t = rng.standard_normal((3, 5, 4)).astype(np.float32)
    P, Tt = T.Tensor(p.copy(), True), T.Tensor(t.copy(), True)
    loss = T.mse(P, Tt)
    d = (p - t).astype(np.float32)
    assert float(loss.data) == np.float32(np.sum((d * d).astype(np.float64)) / d.size)
    T.backward(loss)
    exact = 2.0 * d.astype(np.float64) / d.size
    assert np.all(np.abs(P.grad - exact) <= 2.0 ** -22 * np.abs(exact))
    assert np.array_equal(Tt.grad, -P.grad)
    # a mean over all elements spreads g / n
    X = T.Tensor(p.copy(), True)
    T.backward(T.mean_all(X))
    assert np.all(X.grad == np.float32(1.0) / np.float32(p.size))
    # permute backward is the inverse permutation, bit for bit
    X = T.Tensor(p.copy(), True)
    W = rng.standard_normal((4, 3, 5)).astype(np.float32)
    T.backward(T.sum_all(T.mul(T.permute(X, (2, 0, 1)), T.Tensor(W))))
    assert np.array_equal(X.grad, W.transpose(1, 2, 0))


def test_mlp_training_curve(oracle):
    from oracle import models
    o = load_golden("training_mlp")
    losses, final = models.mlp_curve(o)
    want = o["out.loss"]
    rel = np.max(np.abs(losses.astype(np.float64) - want) / np.abs(want))
    assert rel <= 1e-3, rel
    for k in ("w1", "b1", "w2", "b2"):
        assert scaled(final[k], o["out." + k]) <= 1e-3, k
    assert losses[-1] < losses[0]


# ------------------------------------------------------------------------------------------------- CTC
def ctc_case():
    o = load_golden("autograd_crnn")
    ints = lambda k: o[k].astype(np.int32)
    return o, ints("in.targets"), ints("in.input_lengths"), ints("in.target_lengths")


def test_ctc_reductions_match_reference_fixture(oracle):
    T = oracle
    o, tg, il, tl = ctc_case()
    lp = T.Tensor(o["out.lp"].copy())
    for key, red in (("none", T.CTC_NONE), ("sum", T.CTC_SUM), ("mean", T.CTC_MEAN)):
        got = np.atleast_1d(T.ctc_loss(lp, tg, il, tl, 0, red).data)
        exp = np.atleast_1d(o["out.ctc_" + key])
        assert np.all(np.abs(got - exp) / np.abs(exp) < 1e-5), key
    short = np.array([il[0], 2], np.int32)
    inf = T.ctc_loss(lp, tg, short, tl, 0, T.CTC_NONE).data
    assert np.isposinf(o["out.ctc_inf_none"][1]) and np.isposinf(inf[1])
    zero = T.ctc_loss(lp, tg, short, tl, 0, T.CTC_NONE, zero_inf=True).data
    assert zero[1] == o["out.ctc_zeroinf_none"][1]
    assert abs(zero[0] - o["out.ctc_zeroinf_none"][0]) < 1e-4


def test_ctc_gradient_differs_from_torch_by_softmax_term(oracle):
    """RnnOracleTests.cs:131-160: torch's d/dlp carries an extra exp(lp)*w on used frames."""
    T = oracle
    o, tg, il, tl = ctc_case()
    lp = T.Tensor(o["out.lp"].copy(), requires_grad=True)
    T.backward(T.ctc_loss(lp, tg, il, tl))
    ours, torch_g, lpv = lp.grad, o["grad.lp"], o["out.lp"]
    Tn, B, C = lpv.shape
    exp = ours.astype(np.float64).copy()
    for t in range(Tn):
        for b in range(B):
            w = 1.0 / max(1, tl[b]) / B
            if t < il[b]:
                exp[t, b] += np.exp(lpv[t, b].astype(np.float64)) * w
    assert np.max(np.abs(exp - torch_g)) < 1e-5


def test_ctc_closed_forms(oracle):
    """CtcLossTests.cs:11-39: one frame gives -log p; two frames sum three alignments; impossible gives +inf or 0."""
    T = oracle
    lp = T.Tensor(np.log(np.array([0.25, 0.75], np.float32)).reshape(1, 1, 2))
    v = float(T.ctc_loss(lp, [1], [1], [1], reduction=T.CTC_SUM).data)
    assert abs(v - (-math.log(np.float32(0.75)))) < 1e-6
    p0, p1 = [0.4, 0.7], [0.6, 0.3]
    lpv = np.log(np.array([p0[0], p1[0], p0[1], p1[1]], np.float32)).reshape(2, 1, 2)
    v = float(T.ctc_loss(T.Tensor(lpv), [1], [2], [1], reduction=T.CTC_NONE).data[0])
    p = 0.6 * 0.3 + 0.4 * 0.3 + 0.6 * 0.7
    assert abs(v - (-math.log(p))) < 1e-5
    lp3 = T.log_softmax(T.Tensor(np.zeros((2, 1, 3), np.float32)))
    assert np.isposinf(T.ctc_loss(lp3, [1, 1], [2], [2], reduction=T.CTC_NONE).data[0])
    assert T.ctc_loss(lp3, [1, 1], [2], [2], reduction=T.CTC_NONE, zero_inf=True).data[0] == 0.0


def test_ctc_double_math_against_libm(oracle):
    """CtcMath (Ctc.cs:515-616) is documented at below 1e-15 relative error on the ranges used (docs/ctc.md:59)."""
    L = oracle.lib()
    for x in np.linspace(-60, 5, 301):
        assert abs(L.or_ctc_exp(float(x)) - math.exp(x)) <= 2e-15 * math.exp(x)
    for x in np.exp(np.linspace(-40, 40, 301)):
        assert abs(L.or_ctc_log(float(x)) - math.log(x)) <= 2e-15 * max(1.0, abs(math.log(x)))
    assert L.or_ctc_exp(-701.0) == 0.0 and L.or_ctc_log(0.0) == -math.inf
    assert abs(L.or_ctc_logadd(math.log(0.25), math.log(0.5)) - math.log(0.75)) < 1e-15


# ------------------------------------------------------------------------------------------------- generator, polynomials
def test_splitmix64_known_answers(oracle):
    """SplitMix64 seeded with 0 (Steele, Lea, Flood 2014; Vigna's reference splitmix64.c)."""
    g = oracle.Generator(0)
    assert [g.next_u64() for _ in range(3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_uniform_init_formula(oracle):
    """Generator.NextSingle/Uniform (Generator.cs:33-38): low + (high-low)*((u64>>40)*2^-24), in float32."""
    g1, g2 = oracle.Generator(7), oracle.Generator(7)
    vals = g1.uniform(-0.5, 0.5, (1000,))
    exp = np.array([np.float32(-0.5) + np.float32(1.0) * (np.float32(g2.next_u64() >> 40) * np.float32(2.0 ** -24))
                    for _ in range(1000)], np.float32)
    assert np.array_equal(vals, exp)
    assert vals.min() >= -0.5 and vals.max() < 0.5


def test_polynomials_accuracy(oracle):
    """The reference's polynomials (docs/exact-transcendentals.md) against libm in double: a wrong coefficient or a
    dropped term shows as an error far above their few-ulp accuracy."""
    L = oracle.lib()
    xs = np.linspace(-20, 20, 4001, dtype=np.float32)
    for x in xs:
        e = L.or_exp(float(x))
        assert abs(e - math.exp(float(x))) <= 4e-7 * math.exp(float(x)) + 1e-38
        assert abs(L.or_erf(float(x)) - math.erf(float(x))) <= 4e-7
        gl = 0.5 * float(x) * (1 + math.erf(float(x) / math.sqrt(2)))
        assert abs(L.or_gelu(float(x)) - gl) <= 1e-6 * max(1.0, abs(gl)) or abs(gl) < 1e-30
    for x in np.linspace(-80, 0, 2001, dtype=np.float32):
        assert abs(L.or_exp_nonpos(float(x)) - math.exp(float(x))) <= 4e-7 * math.exp(float(x))


# ------------------------------------------------------------------------------------------------- brute force and FD
def test_gemm_against_double_bound(oracle):
    """Higham's bound for sequential fp32 accumulation (docs/kernels-gemm.md "Accuracy"), for all transposes."""
    T = oracle
    rng = np.random.default_rng(1)
    import ctypes
    for ta in (0, 1):
        for tb in (0, 1):
            m, n, k = 37, 29, 301
            A = rng.standard_normal((k, m) if ta else (m, k)).astype(np.float32)
            B = rng.standard_normal((n, k) if tb else (k, n)).astype(np.float32)
            C = np.empty((m, n), np.float32)
            T.lib().or_gemm(ta, tb, m, n, k, T.fp(A), A.shape[1], T.fp(B), B.shape[1], T.fp(C), n, 0)
            A64 = (A.T if ta else A).astype(np.float64)
            B64 = (B.T if tb else B).astype(np.float64)
            ref = A64 @ B64
            bound = k * 2.0 ** -24 * (np.abs(A64) @ np.abs(B64)) + 1e-30
            assert np.all(np.abs(C - ref) <= bound)


def test_maxpool_index_rules(oracle):
    """TensorKernels.cs:259-283: first of equal maxima wins; a NaN wins and the first NaN is reported."""
    T = oracle
    x = np.array([[[[1, 3, 3, 0], [3, 2, 1, np.nan], [0, 0, -1, -1], [0, np.nan, -1, -2]]]], np.float32)
    y, idx = T.max_pool2d(T.Tensor(x), 2, 2)
    assert idx.reshape(-1).tolist() == [1, 7, 13, 10]
    assert y.data.reshape(-1)[0] == 3.0 and np.isnan(y.data.reshape(-1)[1])
    rng = np.random.default_rng(3)
    xr = rng.integers(-2, 3, (2, 3, 6, 8)).astype(np.float32)  # many ties
    y, idx = T.max_pool2d(T.Tensor(xr), 2, 2)
    for n in range(2):
        for c in range(3):
            for oy in range(3):
                for ox in range(4):
                    win = [(oy * 2 + ky, ox * 2 + kx) for ky in range(2) for kx in range(2)]
                    vals = [xr[n, c, a, b] for a, b in win]
                    best = win[int(np.argmax(vals))]  # argmax returns the first maximum
                    assert idx[n, c, oy, ox] == ((n * 3 + c) * 6 + best[0]) * 8 + best[1]


def gradcheck(T, build, inputs, h=1e-2, tol=5e-3, seed=0):
    """GradCheck.Run (tests/OneModel.Tests/Tensors/GradCheck.cs:11-34): L = sum(W*f(x)) with seeded W, central
    differences in double over float64 copies of the inputs, scaled error."""
    rng = np.random.default_rng(seed)
    ts = [T.Tensor(a.copy(), requires_grad=True) for a in inputs]
    out = build(ts)
    W = rng.uniform(-1, 1, out.data.shape).astype(np.float32)
    T.backward(T.sum_all(T.mul(out, T.Tensor(W))))
    for i, a in enumerate(inputs):
        num = np.zeros(a.size)
        flat = a.reshape(-1)
        for j in range(a.size):
            vals = []
            for sgn in (1, -1):
                b = flat.copy()
                b[j] = np.float32(b[j] + sgn * h)
                xs = [T.Tensor(x.copy()) for x in inputs]
                xs[i] = T.Tensor(b.reshape(a.shape))
                vals.append(float(np.sum(build(xs).data.astype(np.float64) * W)))
            num[j] = (vals[0] - vals[1]) / (2 * h)
        assert scaled(ts[i].grad.reshape(-1), num) <= tol, (i, scaled(ts[i].grad.reshape(-1), num))


def test_fd_layernorm_gelu_linear(oracle):
    T = oracle
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 8)).astype(np.float32)
    w = (rng.standard_normal((6, 8)) * 0.3).astype(np.float32)
    b = (rng.standard_normal(6) * 0.1).astype(np.float32)
    gm = (1 + 0.1 * rng.standard_normal(8)).astype(np.float32)
    bt = (0.1 * rng.standard_normal(8)).astype(np.float32)
    gradcheck(T, lambda t: T.gelu(T.linear(T.layer_norm(t[0], t[3], t[4]), t[1], t[2])), [x, w, b, gm, bt])


def test_fd_softmax(oracle):
    """The standalone softmax backward (or_softmax_bwd, BackwardNn.cs:26-52) against central differences, on rows
    of moderate and of wide-ranging logits."""
    T = oracle
    rng = np.random.default_rng(12)
    gradcheck(T, lambda t: T.softmax(t[0]), [rng.standard_normal((4, 7)).astype(np.float32)])
    gradcheck(T, lambda t: T.softmax(t[0]), [(3 * rng.standard_normal((2, 3, 5))).astype(np.float32)], seed=3)


def test_softmax_backward_closed_forms(oracle):
    """What the mathematics fixes for dx = J^T g with J = diag(y) - y y^T, each failing a plausible slip:
    - a one-hot row (y = e_k exactly) has J = 0, so dx = 0 whatever g is (a dropped factor y, or g*(y - dot) with
      the operands swapped, leaves g_k or g_k (1 - g_k) there);
    - a uniform row (y = 1/n) gives dx = (g - mean(g)) / n (a wrong sign or a missing 1/n fails);
    - every row of dx sums to zero, since sum_j y_j (g_j - y.g) = y.g (1 - sum_j y_j) (a wrong index in the dot
      product, e.g. summing g alone, breaks it), within the rounding of y.g and of the n products."""
    T = oracle
    rng = np.random.default_rng(13)
    n = 9
    # one-hot rows: a gap of 200 makes every other exp underflow to exactly 0 in float32
    x = np.full((4, n), -200.0, np.float32)
    for r in range(4):
        x[r, (2 * r + 1) % n] = 0.0
    t = T.Tensor(x.copy(), requires_grad=True)
    g = rng.standard_normal((4, n)).astype(np.float32)
    T.backward(T.sum_all(T.mul(T.softmax(t), T.Tensor(g))))
    assert np.array_equal(T.softmax(T.Tensor(x)).data, (x == 0).astype(np.float32))
    assert np.all(t.grad == 0.0)
    # uniform rows
    x = np.tile(rng.standard_normal((5, 1)).astype(np.float32), (1, n))
    t = T.Tensor(x.copy(), requires_grad=True)
    g = rng.standard_normal((5, n)).astype(np.float32)
    T.backward(T.sum_all(T.mul(T.softmax(t), T.Tensor(g))))
    expect = (g.astype(np.float64) - g.astype(np.float64).mean(1, keepdims=True)) / n
    assert np.max(np.abs(t.grad - expect)) <= 4 * np.finfo(np.float32).eps * np.max(np.abs(g)) / n
    # rows of dx sum to zero
    x = (2 * rng.standard_normal((16, 33))).astype(np.float32)
    t = T.Tensor(x.copy(), requires_grad=True)
    g = rng.standard_normal((16, 33)).astype(np.float32)
    T.backward(T.sum_all(T.mul(T.softmax(t), T.Tensor(g))))
    y = T.softmax(T.Tensor(x)).data.astype(np.float64)
    bound = 4 * 33 * np.finfo(np.float32).eps * np.max(np.abs(g), axis=1) * np.max(y, axis=1)
    assert np.all(np.abs(t.grad.astype(np.float64).sum(1)) <= bound)


def test_fd_attention_masked(oracle):
    T = oracle
    rng = np.random.default_rng(6)
    q, k, v = (rng.standard_normal((2, 2, 5, 4)).astype(np.float32) for _ in range(3))
    mask = np.where(rng.random((2, 5, 5)) < 0.3, -np.inf, 0.0).astype(np.float32)
    mask[:, :, 0] = 0.0
    gradcheck(T, lambda t: T.attention(t[0], t[1], t[2], mask), [q, k, v])


def test_fd_conv_pool_ce(oracle):
    T = oracle
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 2, 6, 4)).astype(np.float32)
    w = (0.4 * rng.standard_normal((3, 2, 3, 3))).astype(np.float32)
    b = (0.1 * rng.standard_normal(3)).astype(np.float32)
    lw = (0.4 * rng.standard_normal((4, 12))).astype(np.float32)

    def f(t):
        h, _ = T.max_pool2d(T.relu(T.conv2d(t[0], t[1], t[2], 1, 1)), 2, 1)
        h = T.mean_axis(h, 2)
        return T.log_softmax(T.linear(T.reshape(h, (2, 12)), t[3], None))
    gradcheck(T, f, [x, w, b, lw], h=2e-3)  # a smaller step keeps the differences off the ReLU/max kinks


def test_fd_ctc(oracle):
    """CtcLossTests.cs:41-55 case: three sequences incl. repeated labels; gradient through LogSoftmax."""
    T = oracle
    rng = np.random.default_rng(8)
    z = rng.uniform(-1.5, 1.5, (7, 3, 4)).astype(np.float32)
    for red in (T.CTC_NONE, T.CTC_MEAN, T.CTC_SUM):
        def f(t, red=red):
            out = T.ctc_loss(T.log_softmax(t[0]), [1, 2, 2, 3, 1, 1], [7, 6, 4], [2, 3, 1], 0, red)
            return out if out.data.ndim else T.reshape(out, (1,))
        gradcheck(T, f, [z])


def test_cnn_training_curve(oracle):
    """TrainingCurveTests.ConvNetAdamWCosineClipMatchesTorch (TrainingCurveTests.cs:100-124): losses and final
    parameters 1e-3, gradient norms 1e-3 relative with clipping engaged, running variance 1e-3; the zero-gradient
    conv biases in front of batch norm (0.bias, 4.bias) are noise, as the reference reports them."""
    from oracle import models
    o = load_golden("training_cnn")
    losses, norms, final, stats = models.cnn_curve(o)
    want = o["out.loss"]
    assert np.max(np.abs(losses.astype(np.float64) - want) / np.abs(want)) <= 1e-3
    for p, k in models.CNN_MAP:
        if p in ("0.bias", "4.bias"):
            continue
        assert scaled(final[p], o["out." + k]) <= 1e-3, p
    wn = o["out.gradnorm"]
    assert np.max(np.abs(norms.astype(np.float64) - wn) / wn) < 1e-3
    assert int(np.sum(wn > 0.5)) > 5
    assert scaled(stats["rv2"], o["out.rv2"]) < 1e-3
    assert losses[-1] < losses[0]


def test_encoder_training_curve(oracle):
    """TrainingCurveTests.TransformerAdamWarmupMatchesTorch (TrainingCurveTests.cs:126-128): losses and final
    parameters 1e-3 (the attention key biases, zero-gradient in theory, reported apart)."""
    from oracle import models
    o = load_golden("training_encoder")
    losses, final = models.encoder_curve(o)
    want = o["out.loss"]
    assert np.max(np.abs(losses.astype(np.float64) - want) / np.abs(want)) <= 1e-3
    for p, k in models.encoder_map():
        if p.endswith("attn.k.bias"):
            continue
        assert scaled(final[p], o["out." + k]) <= 1e-3, p
    assert losses[-1] < losses[0]


def test_dropout_mask_is_the_generator_stream(oracle):
    """Dropout's mask (Layers.cs:341-368) is the pinned SplitMix64 Generator read from state Mix(seed + draw*G):
    element i keeps iff that generator's (i+1)-th NextSingle is >= p; plus the reference's own properties
    (ModuleAndLossTests.cs:62-100): about p dropped, kept values scaled by exactly 1/(1-p), draws give new masks."""
    T = oracle
    G = 0x9E3779B97F4A7C15
    M = (1 << 64) - 1
    n, p = 1000, 0.3
    x = np.ones(n, np.float32)
    masks = []
    for draw in (0, 1, 5):
        y = T.dropout(T.Tensor(x), p, 42, draw).data
        stream = T.Generator((42 + draw * G - G) & M).next_u64()  # = Mix(seed + draw*G)
        u = T.Generator(stream).uniform(0.0, 1.0, (n,))
        keep = u >= np.float32(p)
        assert np.array_equal(y != 0, keep)
        assert np.all(y[keep] == np.float32(1.0) / np.float32(1.0 - np.float32(p)))
        masks.append(keep)
        if draw == 0:
            assert 240 <= int(np.sum(~keep)) <= 360
    assert not np.array_equal(masks[0], masks[1])
    # backward: g * mask with the same mask (DropoutBackwardUsesTheMask)
    X = T.Tensor(np.full(64, 2.0, np.float32), requires_grad=True)
    Y = T.dropout(X, 0.5, 7, 0)
    T.backward(T.sum_all(Y))
    assert np.array_equal(X.grad, np.where(Y.data == 0, 0.0, 2.0).astype(np.float32))
    assert T.dropout(X, 0.0, 7, 0) is X
