"""Kernel-level parity of lib/libom_hip.so against the CPU oracle (oracle/om_oracle.c), on the GPU.

Bars (the benchmark's stated parity bar): floating-point results within 1e-5 scaled error (max|a-b|/max|ref|, the
reference's metric, AutogradModelTests.cs:20-30); integer work (pool indices) and the optimizer update bit-exact;
kernels that restate the reference's fixed-order arithmetic (LayerNorm forward, softmax rows, GELU, CTC) are checked
bit-for-bit as well.
"""
import ctypes as C
import math

import numpy as np
import pytest

from conftest import scaled

pytestmark = pytest.mark.gpu

TOL = 1e-5


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


def rnd(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


# ------------------------------------------------------------------------------------------------ GEMM
def oracle_gemm(T, ta, tb, A, B, m, n, k):
    Cm = np.empty((m, n), np.float32)
    T.lib().or_gemm(ta, tb, m, n, k, T.fp(A), A.shape[1], T.fp(B), B.shape[1], T.fp(Cm), n, 0)
    return Cm


def test_mfma_fragment_layout(dev):
    """One 16x16x4 product with distinct small integers: exact in fp32, so any lane-layout mistake shows."""
    A = np.arange(64, dtype=np.float32).reshape(16, 4) - 20
    B = (np.arange(64, dtype=np.float32).reshape(4, 16) % 7) - 3
    a, b, c = dev.put(A), dev.put(B), dev.empty((16, 16))
    dev.call("om_gemm", 0, 0, 16, 16, 4, a, 4, b, 16, c, 16, None, 0, None)
    assert np.array_equal(dev.get(c), A @ B)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,n,k", [(64, 64, 64), (37, 53, 29), (256, 384, 384), (5, 300, 1000), (384, 384, 4096),
                                   (130, 10, 257),
                                   # inner dimensions shorter than one MFMA step or chunk (masked k loads)
                                   (70, 50, 1), (33, 129, 3), (600, 2, 7),
                                   # C5's products: the FFN pair and the 768-wide projections over 4096 tokens, and
                                   # the weight-gradient shapes with K = 4096 (the tuned table's C5 rows)
                                   (4096, 3072, 768), (4096, 768, 3072), (4096, 768, 768), (3072, 768, 4096)])
def test_gemm_parity(dev, T, ta, tb, m, n, k):
    rng = np.random.default_rng(m * 1000 + n + k)
    A = rnd(rng, *((k, m) if ta else (m, k)))
    B = rnd(rng, *((n, k) if tb else (k, n)))
    ref = oracle_gemm(T, ta, tb, A, B, m, n, k)
    a, b, c = dev.put(A), dev.put(B), dev.empty((m, n))
    dev.call("om_gemm", ta, tb, m, n, k, a, A.shape[1], b, B.shape[1], c, n, None, 0, None)
    got = dev.get(c)
    assert scaled(got, ref) <= TOL
    # and the GPU product obeys the same sequential-accumulation bound as the CPU one
    A64 = (A.T if ta else A).astype(np.float64)
    B64 = (B.T if tb else B).astype(np.float64)
    bound = k * 2.0 ** -24 * (np.abs(A64) @ np.abs(B64)) + 1e-30
    assert np.all(np.abs(got - A64 @ B64) <= bound)


def test_gemm_accumulate_bias_and_batch(dev, T):
    rng = np.random.default_rng(7)
    m, n, k, H, L = 24, 16, 32, 3, 24
    # A in [B, L, H, D] head-interleaved layout, batch item z = b*H + h
    Bsz = 2
    Q = rnd(rng, Bsz, L, H, k)
    Kt = rnd(rng, Bsz, L, H, n * 0 + k)
    base = rnd(rng, Bsz * H, L, L)
    q, kk, c = dev.put(Q), dev.put(Kt), dev.put(base)
    pkg = dev.pkg
    bt = pkg.om_batch(Bsz * H, H, L * H * k, k, L * H * k, k, H * L * L, L * L)
    dev.call("om_gemm", 0, 1, L, L, k, q, H * k, kk, H * k, c, L, None, 1, C.byref(bt))
    got = dev.get(c)
    for b in range(Bsz):
        for h in range(H):
            ref = oracle_gemm(T, 0, 1, np.ascontiguousarray(Q[b, :, h]), np.ascontiguousarray(Kt[b, :, h]), L, L, k)
            assert scaled(got[b * H + h], base[b * H + h] + ref) <= TOL
    bias = rnd(rng, n)
    A, Bm = rnd(rng, m, k), rnd(rng, k, n)
    a, b2, c2, bb = dev.put(A), dev.put(Bm), dev.empty((m, n)), dev.put(bias)
    dev.call("om_gemm", 0, 0, m, n, k, a, k, b2, n, c2, n, bb, 0, None)
    assert scaled(dev.get(c2), oracle_gemm(T, 0, 0, A, Bm, m, n, k) + bias) <= TOL


def test_gemm_rejects_bad_shapes(dev):
    a = dev.empty((4, 4))
    assert dev.status("om_gemm", 0, 0, 4, 4, 4, a, 2, a, 4, a, 4, None, 0, None) == 1
    assert b"leading dimensions" in dev.ctx.L.om_last_error(dev.ctx.h)


# ------------------------------------------------------------------------------------------------ Linear
@pytest.mark.parametrize("rows,inf,outf", [(64, 784, 256), (64, 256, 10), (4096, 384, 1536), (300, 37, 9),
                                           # one-launch small layers (C2's head, bounds of the small path)
                                           (32, 64, 10), (256, 37, 32), (1, 5, 1), (256, 300, 27),
                                           (512, 256, 128), (4096, 1536, 384), (4096, 384, 1152),
                                           # C5 at full size: FFN pair, attention output, packed q|k|v, token head
                                           (4096, 768, 3072), (4096, 3072, 768), (4096, 768, 768), (4096, 768, 2304),
                                           (4096, 768, 9),
                                           # narrow layers (out <= 64 past the one-launch bounds): C4's head, an
                                           # output count at the top of a rounded-up instance, unaligned rows,
                                           # several input chunks, one output, the row-chunk cap
                                           (1024, 256, 37), (2048, 100, 64), (1000, 33, 33), (300, 2000, 5),
                                           (257, 17, 1), (20000, 8, 3),
                                           # one input feature on the small, narrow and dense paths
                                           (64, 1, 10), (100, 1, 40), (2048, 1, 384),
                                           # one-launch MFMA layers over a small batch (C1's first layer above):
                                           # one block, K blocks that leave some wavefronts a short last round,
                                           # the block-count bound, a long K
                                           (16, 16, 16), (64, 208, 80), (256, 256, 256), (16, 4096, 128)])
def test_linear_fwd_bwd(dev, T, rows, inf, outf):
    rng = np.random.default_rng(rows + inf + outf)
    x, w, b, g = rnd(rng, rows, inf), rnd(rng, outf, inf, scale=0.1), rnd(rng, outf), rnd(rng, rows, outf)
    y_ref = np.empty((rows, outf), np.float32)
    T.lib().or_linear_fwd(T.fp(x), T.fp(w), T.fp(b), T.fp(y_ref), rows, inf, outf)
    dx_r, dw_r, db_r = np.empty_like(x), np.empty_like(w), np.empty_like(b)
    T.lib().or_linear_bwd(T.fp(g), T.fp(x), T.fp(w), T.fp(dx_r), T.fp(dw_r), T.fp(db_r), rows, inf, outf)
    X, W, Bb, G = dev.put(x), dev.put(w), dev.put(b), dev.put(g)
    Y, DX, DW, DB = dev.empty((rows, outf)), dev.empty(x.shape), dev.empty(w.shape), dev.empty(b.shape)
    dev.call("om_linear_fwd", X, W, Bb, Y, rows, inf, outf)
    dev.call("om_linear_bwd", G, X, W, DX, DW, DB, rows, inf, outf, 0, 0, 0)
    assert scaled(dev.get(Y), y_ref) <= TOL
    # Linear then ReLU in one call: om_linear_fwd then om_relu_fwd, bit for bit, on every path
    YR, RR = dev.empty((rows, outf)), dev.empty((rows, outf))
    dev.call("om_linear_relu_fwd", X, W, Bb, YR, rows, inf, outf)
    dev.call("om_relu_fwd", Y, RR, rows * outf)
    assert np.array_equal(dev.get(YR).view(np.uint32), dev.get(RR).view(np.uint32))
    # the input gradient with a residual's gradient added in the epilogue: om_linear_bwd's dx then om_axpy, bit for bit
    RG = dev.put(rnd(rng, rows, inf))
    DXR, DX1 = dev.empty(x.shape), dev.empty(x.shape)
    dev.call("om_linear_bwd_dx_resid", G, W, RG, DXR, rows, inf, outf)
    dev.call("om_linear_bwd", G, X, W, DX1, None, None, rows, inf, outf, 0, 0, 0)
    dev.call("om_axpy", C.c_float(1.0), RG, DX1, rows * inf)
    assert np.array_equal(dev.get(DXR).view(np.uint32), dev.get(DX1).view(np.uint32))
    # and its backward: the ReLU's rule then om_linear_bwd, bit for bit, with and without dx
    GP = dev.empty((rows, outf))
    dev.call("om_relu_bwd", G, YR, GP, rows * outf, 0)
    for with_dx in (False, True):
        outs1 = [dev.empty(x.shape) if with_dx else None, dev.empty(w.shape), dev.empty(b.shape)]
        outs2 = [dev.empty(x.shape) if with_dx else None, dev.empty(w.shape), dev.empty(b.shape)]
        dev.call("om_linear_bwd", GP, X, W, *outs1, rows, inf, outf, 0, 0, 0)
        dev.call("om_linear_relu_bwd", G, YR, X, W, *outs2, rows, inf, outf, 0, 0, 0)
        for o1, o2 in zip(outs1, outs2):
            if o1 is not None:
                assert np.array_equal(dev.get(o1).view(np.uint32), dev.get(o2).view(np.uint32)), with_dx
    assert scaled(dev.get(DX), dx_r) <= TOL
    assert scaled(dev.get(DW), dw_r) <= TOL
    assert scaled(dev.get(DB), db_r) <= 1e-7  # fp64 column sums: equal after rounding
    if dev.ctx.L.om_linear_small(rows, inf, outf):
        # the one-launch path accumulates in the reference's order (one fmaf chain in increasing k, then the bias;
        # db in double by increasing row): the oracle's bits exactly
        for got, ref in ((Y, y_ref), (DX, dx_r), (DW, dw_r), (DB, db_r)):
            assert np.array_equal(dev.get(got).view(np.uint32), ref.view(np.uint32))
    elif outf <= 64 and inf <= 8192:
        # narrow layers: y and dx are the same chains (bit for bit); dW and db add row chunks, within tolerance
        for got, ref in ((Y, y_ref), (DX, dx_r)):
            assert np.array_equal(dev.get(got).view(np.uint32), ref.view(np.uint32))
    # accumulate into existing leaves
    dev.call("om_linear_bwd", G, X, W, DX, DW, DB, rows, inf, outf, 1, 1, 1)
    assert scaled(dev.get(DW), dw_r + dw_r) <= TOL
    assert scaled(dev.get(DB), db_r + db_r) <= 1e-7


@pytest.mark.parametrize("rows,shapes", [
    (4096, [(384, 1536), (1536, 384)]),                # the FFN pair (in, out): one grouped launch, 64 x 96 tiles
    (4096, [(384, 384), (384, 1152), (384, 384)]),     # attention-shaped: three products, 64 x 96 tiles
    (512, [(64, 192), (128, 64)]),                     # 64 x 64 tiles, few splits
    (100, [(20, 36), (36, 20)]),                       # ragged: item by item through om_linear_bwd
    (4096, [(768, 3072), (3072, 768), (768, 768), (768, 2304)]),  # C5's four weight gradients of one layer
    (4096, [(768, 768)]),                              # C5's attention output alone
    (4096, [(768, 9), (768, 768), (20, 36), (768, 2304)]),  # mixed: the two that fit grouped, the others alone
], ids=["ffn-pair", "attention-triple", "small-64", "ragged", "c5-layer", "c5-single", "mixed"])
def test_linear_dw_group(dev, T, rows, shapes):
    """om_linear_bwd_dw_group: every item's dW and db to the GEMM tolerance against the oracle (the last item of
    each group without a bias gradient), then a second call accumulating into the same leaves."""
    rng = np.random.default_rng(rows + len(shapes))
    Item = dev.pkg.om_linear_dw
    refs, bufs, items = [], [], (Item * len(shapes))()
    for i, (inf, outf) in enumerate(shapes):
        x, g = rnd(rng, rows, inf), rnd(rng, rows, outf)
        w = rnd(rng, outf, inf, scale=0.1)
        dx_r, dw_r, db_r = np.empty_like(x), np.empty_like(w), np.empty(outf, np.float32)
        T.lib().or_linear_bwd(T.fp(g), T.fp(x), T.fp(w), T.fp(dx_r), T.fp(dw_r), T.fp(db_r), rows, inf, outf)
        X, G, DW = dev.put(x), dev.put(g), dev.empty((outf, inf), fill=7.0)
        DB = dev.empty((outf,), fill=7.0) if i + 1 < len(shapes) else None
        bufs.append((X, G, DW, DB))
        refs.append((dw_r, db_r))
        items[i] = Item(G.data_ptr(), X.data_ptr(), DW.data_ptr(), DB.data_ptr() if DB is not None else None, inf,
                        outf, 0, 0)
    dev.call("om_linear_bwd_dw_group", len(shapes), C.cast(items, C.c_void_p), rows)
    for (X, G, DW, DB), (dw_r, db_r) in zip(bufs, refs):
        assert scaled(dev.get(DW), dw_r) <= TOL
        if DB is not None:
            assert scaled(dev.get(DB), db_r) <= 1e-7
    for i in range(len(shapes)):
        items[i].acc_dw = items[i].acc_db = 1
    # the second call through om_param_grads_group, with a column sum riding in the same launches
    part = rng.standard_normal((9, 70))
    P, OUT = dev.put(part), dev.empty((70,))
    cs = (dev.pkg.om_column_sum * 1)(dev.pkg.om_column_sum(P.data_ptr(), OUT.data_ptr(), 9, 70, 0))
    dev.call("om_param_grads_group", len(shapes), C.cast(items, C.c_void_p), rows, 1, C.cast(cs, C.c_void_p))
    assert scaled(dev.get(OUT), part.sum(axis=0).astype(np.float32)) <= 1e-7
    for (X, G, DW, DB), (dw_r, db_r) in zip(bufs, refs):
        assert scaled(dev.get(DW), dw_r + dw_r) <= TOL
        if DB is not None:
            assert scaled(dev.get(DB), db_r + db_r) <= 1e-7


OM_GELU_FAST, OM_GELU_REFERENCE = 0, 1


def _gelu64(x):
    """GELU and its slope in double precision (scipy's erfc)."""
    from scipy.special import erfc
    x = x.astype(np.float64)
    cdf = 0.5 * erfc(-x / np.sqrt(2.0))
    return x * cdf, cdf + x * np.exp(-0.5 * x * x) / np.sqrt(2.0 * np.pi)


# The fast pair's stated error (om_ctx_set_gelu): GELU within 1.2e-7 max(1, |x|) and its slope within 2.2e-7 of the
# exact values for correctly rounded reciprocal and exponential; the hardware's are within 1 ulp, which the bounds
# below allow for (about 1e-7 more each).
FAST_GELU_TOL, FAST_SLOPE_TOL = 2.5e-7, 4e-7


@pytest.mark.parametrize("rows,inf,outf", [(4096, 384, 1536), (4096, 1536, 384), (256, 64, 192), (100, 36, 20),
                                           (4096, 768, 3072), (4096, 3072, 768), (4096, 768, 768)])
@pytest.mark.parametrize("mode", [OM_GELU_REFERENCE, OM_GELU_FAST], ids=["reference", "fast"])
def test_linear_fused_epilogues(dev, T, rows, inf, outf, mode):
    """om_linear_fwd_resid (Linear then the residual Add), om_linear_gelu_fwd (Linear then GELU, keeping the
    pre-activation) and om_linear_bwd_dx_gelu (GELU's backward of g w): the GEMM part to the GEMM tolerance; with
    the reference's polynomials (OM_GELU_REFERENCE) the fused element-wise steps bit for bit on the device's own
    GEMM results, with the fast pair (OM_GELU_FAST, the default) within its stated error of the exact GELU and
    slope of those results."""
    dev.call("om_ctx_set_gelu", mode)
    try:
        _fused_epilogues(dev, T, rows, inf, outf, mode)
    finally:
        dev.call("om_ctx_set_gelu", OM_GELU_FAST)


def _fused_epilogues(dev, T, rows, inf, outf, mode):
    exact = mode == OM_GELU_REFERENCE
    rng = np.random.default_rng(rows + 3 * inf + outf)
    x, w, b = rnd(rng, rows, inf), rnd(rng, outf, inf, scale=0.1), rnd(rng, outf)
    resid, g = rnd(rng, rows, outf), rnd(rng, rows, outf)
    lin = np.empty((rows, outf), np.float32)
    T.lib().or_linear_fwd(T.fp(x), T.fp(w), T.fp(b), T.fp(lin), rows, inf, outf)
    X, W, Bb, R = dev.put(x), dev.put(w), dev.put(b), dev.put(resid)
    Y, H, A = dev.empty((rows, outf)), dev.empty((rows, outf)), dev.empty((rows, outf))
    dev.call("om_linear_fwd_resid", X, W, Bb, R, Y, rows, inf, outf)
    assert scaled(dev.get(Y), resid + lin) <= TOL
    dev.call("om_linear_fwd", X, W, Bb, H, rows, inf, outf)
    plain = dev.get(H)
    assert np.array_equal(dev.get(Y), (resid + plain).astype(np.float32))  # Linear, then one rounded Add
    dev.call("om_linear_gelu_fwd", X, W, Bb, H, A, rows, inf, outf)
    h = dev.get(H)
    assert scaled(h, lin) <= TOL
    if exact:
        a_ref = np.empty_like(h)
        T.lib().or_gelu_fwd(T.fp(h), T.fp(a_ref), C.c_int64(h.size))
        assert np.array_equal(dev.get(A).view(np.uint32), a_ref.view(np.uint32))
    else:
        a64, _ = _gelu64(h)
        assert np.all(np.abs(dev.get(A) - a64) <= FAST_GELU_TOL * np.maximum(1.0, np.abs(h)))
    # dh = GELU'(h) * (g w): g [rows, outf] against w [outf, inf] is the backward of a Linear(inf -> outf) whose
    # input went through GELU; here h plays that input, so use a pre-activation of shape [rows, inf].
    hin = rnd(rng, rows, inf, scale=2.0)
    da = np.empty((rows, inf), np.float32)
    T.lib().or_gemm(0, 0, rows, inf, outf, T.fp(g), outf, T.fp(w), inf, T.fp(da), inf, 0)
    dh_ref = np.empty_like(da)
    T.lib().or_gelu_bwd(T.fp(da), T.fp(hin), T.fp(dh_ref), C.c_int64(da.size))
    G, HI, DH, DA = dev.put(g), dev.put(hin), dev.empty((rows, inf)), dev.empty((rows, inf))
    dev.call("om_linear_bwd_dx_gelu", G, W, HI, DH, rows, inf, outf)
    assert scaled(dev.get(DH), dh_ref) <= TOL
    # GeluGradBin applied to the epilogue kernel's own product: om_linear_bwd_dx_slope with a unit slope yields that
    # product exactly (x * 1 = x) from the tile every epilogue launch of this shape takes. A plain om_linear_bwd may
    # take a tile that carries no epilogue (the eight-wavefront 128 x 128 one at 4096 x 3072 x 768), whose partial
    # sums combine in another order, so it is held to the GEMM tolerance only.
    ONES = dev.put(np.ones((rows, inf), np.float32))
    dev.call("om_linear_bwd_dx_slope", G, W, ONES, DA, rows, inf, outf)
    da_dev = dev.get(DA)
    assert scaled(da_dev, da) <= TOL
    if exact:
        dh_exact = np.empty_like(da_dev)
        T.lib().or_gelu_bwd(T.fp(da_dev), T.fp(hin), T.fp(dh_exact), C.c_int64(da_dev.size))
        assert np.array_equal(dev.get(DH).view(np.uint32), dh_exact.view(np.uint32))
    else:
        # the fast GELU backward of the same product (its tile may differ from the slope product's, so the product
        # is held to the GEMM tolerance and the slope to its stated error)
        _, s64 = _gelu64(hin)
        assert scaled(dev.get(DH), da_dev.astype(np.float64) * s64) <= TOL
    dev.call("om_linear_bwd", G, X, W, DA, None, None, rows, inf, outf, 0, 0, 0)
    assert scaled(dev.get(DA), da) <= TOL
    # The slope pair: the forward's a equals om_linear_gelu_fwd's, its s is GELU's slope at h (GeluGradBin with a unit
    # gradient), and the backward from a saved slope equals om_linear_bwd_dx_gelu bit for bit.
    A2, S = dev.empty((rows, outf)), dev.empty((rows, outf))
    dev.call("om_linear_gelu_fwd_slope", X, W, Bb, A2, S, rows, inf, outf)
    assert np.array_equal(dev.get(A2).view(np.uint32), dev.get(A).view(np.uint32))
    if exact:
        s_ref = np.empty_like(h)
        T.lib().or_gelu_bwd(T.fp(np.ones_like(h)), T.fp(h), T.fp(s_ref), C.c_int64(h.size))
        assert np.array_equal(dev.get(S).view(np.uint32), s_ref.view(np.uint32))
        s_in = np.empty_like(hin)
        T.lib().or_gelu_bwd(T.fp(np.ones_like(hin)), T.fp(hin), T.fp(s_in), C.c_int64(hin.size))
        SI, DH2 = dev.put(s_in), dev.empty((rows, inf))
        dev.call("om_linear_bwd_dx_slope", G, W, SI, DH2, rows, inf, outf)
        assert np.array_equal(dev.get(DH2).view(np.uint32), dev.get(DH).view(np.uint32))
    else:
        _, s64 = _gelu64(h)
        assert np.all(np.abs(dev.get(S) - s64) <= FAST_SLOPE_TOL)


def test_fast_gelu_pair_accuracy(dev):
    """The fast pair itself over [-12, 12] (inputs passed through an identity product, which reproduces them
    exactly): GELU and its slope within the stated error of double-precision values, signs and the tails right."""
    rows, n = 4096, 64
    x = np.linspace(-12.0, 12.0, rows * n).astype(np.float32).reshape(rows, n)
    X, I = dev.put(x), dev.put(np.eye(n, dtype=np.float32))
    A, S = dev.empty((rows, n)), dev.empty((rows, n))
    dev.call("om_ctx_set_gelu", OM_GELU_FAST)
    dev.call("om_linear_gelu_fwd_slope", X, I, None, A, S, rows, n, n)
    a, s = dev.get(A), dev.get(S)
    a64, s64 = _gelu64(x)
    assert np.all(np.abs(a - a64) <= FAST_GELU_TOL * np.maximum(1.0, np.abs(x)))
    assert np.all(np.abs(s - s64) <= FAST_SLOPE_TOL)
    assert np.all(a[x > 0] > 0) and np.all(a[x < -1e-3] <= 0)
    assert np.array_equal(a[x >= 6], x[x >= 6])  # cdf rounds to 1 there
    assert np.all(np.abs(a[x <= -9]) <= 1e-17)


# ------------------------------------------------------------------------------------------------ element-wise
def test_relu_gelu_bit_exact(dev, T):
    rng = np.random.default_rng(3)
    x = np.concatenate([rnd(rng, 100003, scale=3.0), np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -7.0, 6.0],
                                                               np.float32)])
    g = rnd(rng, x.size)
    n = x.size
    X, G, Y, D = dev.put(x), dev.put(g), dev.empty(x.shape), dev.empty(x.shape)
    ry, rd = np.empty_like(x), np.empty_like(x)
    T.lib().or_relu_fwd(T.fp(x), T.fp(ry), C.c_int64(n))
    dev.call("om_relu_fwd", X, Y, n)
    assert np.array_equal(dev.get(Y).view(np.uint32), ry.view(np.uint32))
    T.lib().or_relu_bwd(T.fp(g), T.fp(ry), T.fp(rd), C.c_int64(n))
    dev.call("om_relu_bwd", G, Y, D, n, 0)
    assert np.array_equal(dev.get(D).view(np.uint32), rd.view(np.uint32))
    dev.call("om_ctx_set_gelu", OM_GELU_REFERENCE)
    try:  # the reference's polynomials, bit for bit
        T.lib().or_gelu_fwd(T.fp(x), T.fp(ry), C.c_int64(n))
        dev.call("om_gelu_fwd", X, Y, n)
        assert np.array_equal(dev.get(Y).view(np.uint32), ry.view(np.uint32))
        T.lib().or_gelu_bwd(T.fp(g), T.fp(x), T.fp(rd), C.c_int64(n))
        dev.call("om_gelu_bwd", G, X, D, n, 0)
        assert np.array_equal(dev.get(D).view(np.uint32), rd.view(np.uint32))
    finally:
        dev.call("om_ctx_set_gelu", OM_GELU_FAST)
    # the default fast pair: within its stated error, and the reference's special values
    dev.call("om_gelu_fwd", X, Y, n)
    dev.call("om_gelu_bwd", G, X, D, n, 0)
    y, d = dev.get(Y), dev.get(D)
    fin = np.isfinite(x)
    a64, s64 = _gelu64(x[fin])
    assert np.all(np.abs(y[fin] - a64) <= FAST_GELU_TOL * np.maximum(1.0, np.abs(x[fin])))
    bound = (FAST_SLOPE_TOL + 1e-7) * np.abs(g[fin]) + 1e-30  # the slope's error plus the product's rounding
    assert np.all(np.abs(d[fin] - g[fin].astype(np.float64) * s64) <= bound)
    assert y[x == np.inf][0] == np.inf and y[x == -np.inf][0] == 0.0 and np.isnan(y[np.isnan(x)][0])


def test_add_sub_mul_axpy_mean(dev, T):
    rng = np.random.default_rng(4)
    a, b = rnd(rng, 1001), rnd(rng, 1001)
    A, B, Y = dev.put(a), dev.put(b), dev.empty((1001,))
    for name, f in (("om_add", np.add), ("om_sub", np.subtract), ("om_mul", np.multiply)):
        dev.call(name, A, B, Y, 1001)
        assert np.array_equal(dev.get(Y), f(a, b))
    dev.call("om_axpy", C.c_float(-1.0), A, Y, 1001)
    assert np.array_equal(dev.get(Y), a * b - a)
    x = rnd(rng, 3, 7, 5)
    X, M = dev.put(x), dev.empty((3, 5))
    dev.call("om_mean_axis", X, M, 3, 7, 5)
    ref = np.empty((3, 5), np.float32)
    T.lib().or_mean_axis(T.fp(x), T.fp(ref), 3, 7, 5)
    assert np.array_equal(dev.get(M), ref)
    x2 = rnd(rng, 40, 3136)
    X2, M2 = dev.put(x2), dev.empty((40,))
    dev.call("om_mean_axis", X2, M2, 40, 3136, 1)
    ref2 = np.empty(40, np.float32)
    T.lib().or_mean_axis(T.fp(x2), T.fp(ref2), 40, 3136, 1)
    assert scaled(dev.get(M2), ref2) <= 1e-7
    S = dev.empty((1,))
    dev.call("om_sum_all", X2, S, x2.size, 1)
    assert abs(dev.get(S)[0] - T.lib().or_sum_all(T.fp(x2), C.c_int64(x2.size), 1)) <= 1e-7 * max(1, abs(x2.mean()))
    g = dev.put(np.array([0.75], np.float32))
    D = dev.empty(x2.shape)
    dev.call("om_mean_all_bwd", g, D, x2.size, 0)
    assert np.all(dev.get(D) == np.float32(0.75) / np.float32(x2.size))


def test_mse_and_its_unit_gradient(dev, T):
    """om_mse_fwd / om_mse_bwd against the oracle's Losses.Mse chain, and om_mse_fwd_unit's gradient for a unit
    upstream gradient equal to om_mse_bwd with g = 1 bit for bit."""
    from oracle import tape as OT
    rng = np.random.default_rng(21)
    pred, tgt = rnd(rng, 4096, 384), rnd(rng, 4096, 384)
    n = pred.size
    P, TG = dev.put(pred), dev.put(tgt)
    D, LOSS, D2, LOSS2, UNIT = (dev.empty(pred.shape), dev.empty((1,)), dev.empty(pred.shape), dev.empty((1,)),
                                dev.empty(pred.shape))
    dev.call("om_mse_fwd", P, TG, D, LOSS, C.c_int64(n))
    dev.call("om_mse_fwd_unit", P, TG, D2, LOSS2, UNIT, C.c_int64(n))
    assert np.array_equal(dev.get(LOSS), dev.get(LOSS2)) and np.array_equal(dev.get(D), dev.get(D2))
    ONE, DP = dev.put(np.ones(1, np.float32)), dev.empty(pred.shape)
    dev.call("om_mse_bwd", ONE, D, DP, C.c_int64(n), 0)
    assert np.array_equal(dev.get(UNIT).view(np.uint32), dev.get(DP).view(np.uint32))
    # without diff (NULL: not written), the same loss and unit gradient; om_sub restates the skipped diff
    LOSS3, UNIT3, D3 = dev.empty((1,)), dev.empty(pred.shape), dev.empty(pred.shape)
    dev.call("om_mse_fwd_unit", P, TG, None, LOSS3, UNIT3, C.c_int64(n))
    assert np.array_equal(dev.get(LOSS3), dev.get(LOSS)) and np.array_equal(dev.get(UNIT3), dev.get(UNIT))
    dev.call("om_sub", P, TG, D3, C.c_int64(n))
    assert np.array_equal(dev.get(D3).view(np.uint32), dev.get(D).view(np.uint32))
    tp = OT.Tensor(pred.copy(), True)
    loss = OT.mse(tp, OT.Tensor(tgt.copy()))
    OT.backward(loss)
    ref = float(loss.data.reshape(-1)[0])
    assert abs(float(dev.get(LOSS)[0]) - ref) <= 1e-6 * abs(ref)
    assert scaled(dev.get(UNIT), tp.grad) <= 1e-6


# ------------------------------------------------------------------------------------------------ norms and softmax
@pytest.mark.parametrize("rows,cols", [(4096, 384), (512, 768), (7, 1536), (33, 2000), (17, 12), (9, 10), (40, 960),
                                       (37, 384), (21, 768)])
def test_layernorm(dev, T, rows, cols):
    rng = np.random.default_rng(rows + cols)
    x, g = rnd(rng, rows, cols, scale=2.0) + 0.5, rnd(rng, rows, cols)
    # rows of zero variance (rstd = 1/sqrt(eps)), and a row whose mean is far above its spread (the variance's
    # differences cancel): still the reference's bits
    x[2], x[5] = np.float32(1.5), np.float32(0.0)
    x[6] = np.float32(1000.0) + np.float32(0.01) * x[6]
    gam, bet = (1 + 0.1 * rnd(rng, cols)), 0.1 * rnd(rng, cols)
    y, mu, iv = np.empty_like(x), np.empty(rows, np.float32), np.empty(rows, np.float32)
    T.lib().or_layernorm_fwd(T.fp(x), T.fp(gam), T.fp(bet), T.fp(y), T.fp(mu), T.fp(iv), rows, cols, C.c_float(1e-5))
    X, G, GA, BE = dev.put(x), dev.put(g), dev.put(gam), dev.put(bet)
    Y, MU, IV = dev.empty(x.shape), dev.empty((rows,)), dev.empty((rows,))
    dev.call("om_layernorm_fwd", X, GA, BE, Y, MU, IV, rows, cols, C.c_float(1e-5))
    assert np.array_equal(dev.get(Y), y)  # the reference's Sum16 order, bit for bit
    assert np.array_equal(dev.get(MU), mu) and np.array_equal(dev.get(IV), iv)
    dx, dg, db = np.empty_like(x), np.empty(cols, np.float32), np.empty(cols, np.float32)
    T.lib().or_layernorm_bwd(T.fp(g), T.fp(x), T.fp(gam), T.fp(mu), T.fp(iv), T.fp(dx), T.fp(dg), T.fp(db), rows, cols)
    DX, DG, DB = dev.empty(x.shape), dev.empty((cols,)), dev.empty((cols,))
    dev.call("om_layernorm_bwd", G, X, GA, MU, IV, DX, DG, DB, rows, cols, 0, 0)
    assert scaled(dev.get(DX), dx) <= 1e-6
    assert scaled(dev.get(DG), dg) <= 1e-7 and scaled(dev.get(DB), db) <= 1e-7
    # dx accumulated into an existing gradient equals dx written beside it from that gradient as an addend
    prev = rnd(rng, rows, cols)
    ACC, ADD, OUT = dev.put(prev), dev.put(prev), dev.empty(x.shape, fill=np.nan)
    dev.call("om_layernorm_bwd", G, X, GA, MU, IV, ACC, None, None, rows, cols, 1, 0)
    dev.call("om_layernorm_bwd_add", G, X, GA, MU, IV, ADD, OUT, None, None, rows, cols, 0)
    assert np.array_equal(dev.get(OUT).view(np.uint32), dev.get(ACC).view(np.uint32))
    assert np.array_equal(dev.get(ADD), prev)  # the addend is only read
    assert scaled(dev.get(OUT), prev + dx) <= 1e-6
    # partials now, column sums later through om_param_grads_group: the same bits as om_layernorm_bwd
    L = dev.ctx.L
    chunks = L.om_layernorm_bwd_chunks(rows, cols)
    PG, PB = dev.empty((chunks, cols), np.float64), dev.empty((chunks, cols), np.float64)
    DX2, DG2, DB2 = dev.empty(x.shape), dev.empty((cols,), fill=3.0), dev.empty((cols,), fill=3.0)
    dev.call("om_layernorm_bwd_partials", G, X, GA, MU, IV, None, DX2, 0, PG, PB, rows, cols)
    items = (dev.pkg.om_column_sum * 2)(dev.pkg.om_column_sum(PG.data_ptr(), DG2.data_ptr(), chunks, cols, 0),
                                        dev.pkg.om_column_sum(PB.data_ptr(), DB2.data_ptr(), chunks, cols, 1))
    dev.call("om_param_grads_group", 0, None, 0, 2, C.cast(items, C.c_void_p))
    assert np.array_equal(dev.get(DX2).view(np.uint32), dev.get(DX).view(np.uint32))
    assert np.array_equal(dev.get(DG2).view(np.uint32), dev.get(DG).view(np.uint32))
    assert np.array_equal(dev.get(DB2), (dev.get(DB) + np.float32(3.0)).astype(np.float32))  # accumulated


@pytest.mark.parametrize("rows,cols", [(1000, 128), (300, 512), (17, 37)])
def test_softmax_rows(dev, T, rows, cols):
    rng = np.random.default_rng(rows)
    x = rnd(rng, rows, cols, scale=3.0)
    x[0, 5:] = -np.inf
    x[1, :] = -np.inf  # all masked: NaN row, as the reference
    ref = np.empty_like(x)
    T.lib().or_softmax_rows(T.fp(x), T.fp(ref), rows, cols)
    X, Y = dev.put(x), dev.empty(x.shape)
    dev.call("om_softmax_fwd", X, Y, rows, cols)
    got = dev.get(Y)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    g = rnd(rng, rows, cols)
    g[1] = 0
    dref = np.empty_like(x)
    T.lib().or_softmax_bwd(T.fp(g), T.fp(ref), T.fp(dref), rows, cols)
    G, D = dev.put(g), dev.empty(x.shape)
    dev.call("om_softmax_bwd", G, Y, D, rows, cols, 0)
    dgot = dev.get(D)
    ok = np.isfinite(dref)
    assert np.array_equal(np.isfinite(dgot), ok) and scaled(dgot[ok], dref[ok]) <= 1e-6


@pytest.mark.parametrize("mean,ignore,all_ignored", [(0, 0, False), (1, 0, False), (0, -100, False), (1, 0, True),
                                                    (0, 0, True)], ids=["sum-ignore0", "mean-ignore0", "sum",
                                                                        "mean-all-ignored", "sum-all-ignored"])
def test_nll_reductions_and_ignore_index(dev, T, mean, ignore, all_ignored):
    """NllLoss with sum reduction and a real class as ignore_index (GradCheckTests.cs:144: "NllLoss sum ignore=0"),
    and batches whose every row is ignored (the count in the mean is then taken as 1, so the loss is 0 and the
    gradient 0): om_nll_fwd, om_nll_bwd and the fused om_xent_bwd against the oracle."""
    rows, cols = 300, 7
    rng = np.random.default_rng(rows + mean + 3 * all_ignored)
    z = rnd(rng, rows, cols, scale=2.0)
    tg = np.full(rows, ignore, np.int32) if all_ignored else rng.integers(0, cols, rows).astype(np.int32)
    lp = np.empty_like(z)
    T.lib().or_logsoftmax_fwd(T.fp(z), T.fp(lp), rows, cols)
    bad = C.c_int(0)
    loss = T.lib().or_nll_fwd(T.fp(lp), T.ip(tg), rows, cols, mean, ignore, C.byref(bad))
    gval = np.float32(0.75)
    dn, dz = np.empty_like(z), np.empty_like(z)
    T.lib().or_nll_bwd(C.c_float(gval), T.ip(tg), T.fp(dn), rows, cols, mean, ignore)
    T.lib().or_logsoftmax_bwd(T.fp(dn), T.fp(lp), T.fp(dz), rows, cols)
    if all_ignored:
        assert loss == 0.0 and not dn.any()
    LP, TG, L, BAD = dev.put(lp), dev.put(tg), dev.empty((1,)), dev.empty((1,), np.int32)
    GS, DN, DZ = dev.put(np.array([gval], np.float32)), dev.empty(z.shape, fill=9.0), dev.empty(z.shape)
    dev.call("om_nll_fwd", LP, TG, L, BAD, rows, cols, mean, ignore)
    dev.call("om_nll_bwd", GS, TG, DN, rows, cols, mean, ignore, 0)
    dev.call("om_xent_bwd", GS, LP, TG, DZ, rows, cols, mean, ignore, 0)
    assert abs(dev.get(L)[0] - loss) <= 1e-6 * max(1.0, abs(loss)) and dev.get(BAD)[0] == -1
    assert np.array_equal(dev.get(DN).view(np.uint32), dn.view(np.uint32))
    assert scaled(dev.get(DZ), dz) <= 1e-6


@pytest.mark.parametrize("rows,cols", [(64, 10), (4096, 9), (1024, 37), (7, 3), (1000, 100), (1025, 5)])
def test_cross_entropy(dev, T, rows, cols):
    rng = np.random.default_rng(cols)
    z = rnd(rng, rows, cols, scale=2.0)
    z[1] *= np.float32(500.0)  # logits far beyond exp's range: the row maximum is subtracted first
    z[2] = np.float32(-3.0e4)  # a constant, very negative row: log(cols) below its value
    tg = rng.integers(0, cols, rows).astype(np.int32)
    tg[3] = -100  # ignored row
    lp = np.empty_like(z)
    T.lib().or_logsoftmax_fwd(T.fp(z), T.fp(lp), rows, cols)
    bad = C.c_int(0)
    loss = T.lib().or_nll_fwd(T.fp(lp), T.ip(tg), rows, cols, 1, -100, C.byref(bad))
    dn, dz = np.empty_like(z), np.empty_like(z)
    T.lib().or_nll_bwd(C.c_float(1.0), T.ip(tg), T.fp(dn), rows, cols, 1, -100)
    T.lib().or_logsoftmax_bwd(T.fp(dn), T.fp(lp), T.fp(dz), rows, cols)
    Z, TG, LP, L, BAD, DZ = dev.put(z), dev.put(tg), dev.empty(z.shape), dev.empty((1,)), dev.empty((1,), np.int32), \
        dev.empty(z.shape)
    one = dev.put(np.ones(1, np.float32))
    dev.call("om_logsoftmax_fwd", Z, LP, rows, cols)
    dev.call("om_nll_fwd", LP, TG, L, BAD, rows, cols, 1, -100)
    dev.call("om_xent_bwd", one, LP, TG, DZ, rows, cols, 1, -100, 0)
    assert scaled(dev.get(LP), lp) <= 1e-6
    assert abs(dev.get(L)[0] - loss) <= 1e-6 * abs(loss) and dev.get(BAD)[0] == -1
    assert scaled(dev.get(DZ), dz) <= 1e-6
    # the fused forward with the unit gradient gives the same bits as the three separate launches (g = 1)
    LP2, L2, BAD2, DZ2 = dev.empty(z.shape), dev.empty((1,)), dev.empty((1,), np.int32), dev.empty(z.shape)
    dev.call("om_xent_fwd_unit", Z, TG, LP2, L2, BAD2, DZ2, rows, cols, -100, None)
    for a, b in ((LP2, LP), (L2, L), (DZ2, DZ)):
        assert np.array_equal(dev.get(a).view(np.uint32), dev.get(b).view(np.uint32))
    assert dev.get(BAD2)[0] == -1
    tg[5] = cols  # out of range: reported, as the reference's ArgumentOutOfRangeException
    dev.call("om_nll_fwd", LP, dev.put(tg), L, BAD, rows, cols, 1, -100)
    assert dev.get(BAD)[0] == 5
    dev.call("om_xent_fwd_unit", Z, dev.put(tg), LP2, L2, BAD2, DZ2, rows, cols, -100, None)
    assert dev.get(BAD2)[0] == 5 and np.isnan(dev.get(L2)[0])


# ------------------------------------------------------------------------------------------------ attention
@pytest.mark.parametrize("B,H,L,D,masked", [(2, 3, 40, 32, True), (2, 12, 128, 32, True), (1, 4, 512, 64, False)])
def test_attention(dev, T, B, H, L, D, masked):
    rng = np.random.default_rng(L + D)
    q, k, v, g = (rnd(rng, B, L, H, D) for _ in range(4))  # [B, L, H, D] interleaved, as the Linear outputs
    mask = None
    if masked:
        lens = rng.integers(L // 2, L + 1, B)
        mask = np.zeros((B, L, L), np.float32)
        for b in range(B):
            mask[b, :, lens[b]:] = -np.inf
    tq, tk, tv, tg = (np.ascontiguousarray(a.transpose(0, 2, 1, 3)) for a in (q, k, v, g))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    o_ref = np.empty_like(tq)
    T.lib().or_attention_fwd(T.fp(tq), T.fp(tk), T.fp(tv), T.fp(mask) if masked else None, 1, T.fp(o_ref), B, H, L, L,
                             D, C.c_float(scale))
    dq, dk, dv = np.empty_like(tq), np.empty_like(tk), np.empty_like(tv)
    T.lib().or_attention_bwd(T.fp(tq), T.fp(tk), T.fp(tv), T.fp(mask) if masked else None, 1, T.fp(tg), T.fp(dq),
                             T.fp(dk), T.fp(dv), B, H, L, L, D, C.c_float(scale))
    Q, K, V, G = dev.put(q), dev.put(k), dev.put(v), dev.put(g)
    M = dev.put(mask) if masked else None
    O, P, DS = dev.empty(q.shape), dev.empty((B, H, L, L)), dev.empty((B, H, L, L))
    DQ, DK, DV = dev.empty(q.shape), dev.empty(q.shape), dev.empty(q.shape)
    dev.call("om_attention_fwd", Q, K, V, M, 1, O, P, B, H, L, L, D, C.c_float(scale))
    dev.call("om_attention_bwd", Q, K, V, P, G, DQ, DK, DV, DS, B, H, L, L, D, C.c_float(scale), 0)
    back = lambda t: dev.get(t).transpose(0, 2, 1, 3)
    assert scaled(back(O), o_ref) <= TOL
    for got, ref in ((DQ, dq), (DK, dk), (DV, dv)):
        assert scaled(back(got), ref) <= TOL


@pytest.mark.parametrize("B,H,L,D", [(2, 3, 40, 32), (4, 12, 128, 32)])
def test_attention_packed_qkv_strides(dev, T, B, H, L, D):
    """om_attention_*_ld on q|k|v packed as one [B, L, 3*H*D] projection output, with o and dq|dk|dv in the same
    packed layouts: the same results as the oracle on the unpacked tensors."""
    rng = np.random.default_rng(B * L + D)
    W = H * D
    qkv = rnd(rng, B, L, 3 * W)
    g = rnd(rng, B, L, W)
    lens = rng.integers(L // 2, L + 1, B)
    mask = np.zeros((B, L, L), np.float32)
    for b in range(B):
        mask[b, :, lens[b]:] = -np.inf
    heads = lambda a: np.ascontiguousarray(a.reshape(B, L, H, D).transpose(0, 2, 1, 3))
    tq, tk, tv = (heads(qkv[:, :, i * W:(i + 1) * W]) for i in range(3))
    tg = heads(g)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    o_ref = np.empty_like(tq)
    T.lib().or_attention_fwd(T.fp(tq), T.fp(tk), T.fp(tv), T.fp(mask), 1, T.fp(o_ref), B, H, L, L, D, C.c_float(scale))
    dq, dk, dv = np.empty_like(tq), np.empty_like(tk), np.empty_like(tv)
    T.lib().or_attention_bwd(T.fp(tq), T.fp(tk), T.fp(tv), T.fp(mask), 1, T.fp(tg), T.fp(dq), T.fp(dk), T.fp(dv), B, H,
                             L, L, D, C.c_float(scale))
    QKV, G, M = dev.put(qkv), dev.put(g), dev.put(mask)
    O, P, DS, DQKV = dev.empty((B, L, W)), dev.empty((B, H, L, L)), dev.empty((B, H, L, L)), dev.empty((B, L, 3 * W))
    off = lambda buf, i: buf.data_ptr() + 4 * i * W
    dev.call("om_attention_fwd_ld", QKV, off(QKV, 1), off(QKV, 2), 3 * W, M, 1, O, W, P, B, H, L, L, D,
             C.c_float(scale))
    dev.call("om_attention_bwd_ld", QKV, off(QKV, 1), off(QKV, 2), 3 * W, P, G, W, DQKV, off(DQKV, 1), off(DQKV, 2),
             3 * W, DS, B, H, L, L, D, C.c_float(scale), 0)
    assert scaled(heads(dev.get(O)), o_ref) <= TOL
    d = dev.get(DQKV)
    for i, ref in enumerate((dq, dk, dv)):
        assert scaled(heads(d[:, :, i * W:(i + 1) * W]), ref) <= TOL


@pytest.mark.parametrize("B,H,L,D,masked,packed", [(4, 12, 128, 32, True, True), (3, 2, 64, 32, True, False),
                                                     (2, 3, 128, 32, False, False), (2, 3, 40, 32, True, False),
                                                     (1, 2, 128, 64, True, True), (24, 12, 128, 32, True, True),
                                                     (24, 12, 64, 32, False, False)])
def test_attention_fused_recompute(dev, T, B, H, L, D, masked, packed):
    """om_attention_{fwd,bwd}_fused (no saved weights; the backward recomputes P): the fused kernels for D = 32 and
    L in {64, 128}, the GEMM fallback otherwise; against the oracle, and accumulating into existing gradients."""
    rng = np.random.default_rng(B * L + D + H)
    W = H * D
    ld = 3 * W if packed else W
    qkv = rnd(rng, B, L, 3 * W)
    g = rnd(rng, B, L, W)
    mask = None
    if masked:
        lens = rng.integers(L // 2, L + 1, B)
        mask = np.zeros((B, L, L), np.float32)
        for b in range(B):
            mask[b, :, lens[b]:] = -np.inf
    heads = lambda a: np.ascontiguousarray(a.reshape(B, L, H, D).transpose(0, 2, 1, 3))
    parts = [qkv[:, :, i * W:(i + 1) * W] for i in range(3)]
    tq, tk, tv = (heads(a) for a in parts)
    tg = heads(g)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    o_ref = np.empty_like(tq)
    mp = T.fp(mask) if masked else None
    T.lib().or_attention_fwd(T.fp(tq), T.fp(tk), T.fp(tv), mp, 1, T.fp(o_ref), B, H, L, L, D, C.c_float(scale))
    dq, dk, dv = np.empty_like(tq), np.empty_like(tk), np.empty_like(tv)
    T.lib().or_attention_bwd(T.fp(tq), T.fp(tk), T.fp(tv), mp, 1, T.fp(tg), T.fp(dq), T.fp(dk), T.fp(dv), B, H, L, L,
                             D, C.c_float(scale))
    if packed:
        QKV = dev.put(qkv)
        qp = [QKV.data_ptr() + 4 * i * W for i in range(3)]
        DQKV = dev.empty((B, L, 3 * W), fill=0.5)
        dp = [DQKV.data_ptr() + 4 * i * W for i in range(3)]
        got = lambda: [dev.get(DQKV)[:, :, i * W:(i + 1) * W] for i in range(3)]
    else:
        QS = [dev.put(np.ascontiguousarray(a)) for a in parts]
        qp = [t.data_ptr() for t in QS]
        DS = [dev.empty((B, L, W), fill=0.5) for _ in range(3)]
        dp = [t.data_ptr() for t in DS]
        got = lambda: [dev.get(t) for t in DS]
    G, M = dev.put(g), (dev.put(mask) if masked else None)
    O = dev.empty((B, L, W))
    dev.call("om_attention_fwd_fused", qp[0], qp[1], qp[2], ld, M, 1, O, W, B, H, L, D, C.c_float(scale))
    assert scaled(heads(dev.get(O)), o_ref) <= TOL
    dev.call("om_attention_bwd_fused", qp[0], qp[1], qp[2], ld, M, 1, G, W, dp[0], dp[1], dp[2], ld, B, H, L, D,
             C.c_float(scale), 1)
    for gd, ref in zip(got(), (dq, dk, dv)):
        assert scaled(heads(gd) - np.float32(0.5), ref) <= TOL


@pytest.mark.parametrize("B,H,L,D,masked,packed,acc", [
    (8, 12, 512, 64, False, True, 0),   # C5 at full size: the packed q|k|v projection, no mask
    (2, 3, 128, 64, True, False, 1),
    (2, 4, 256, 32, True, True, 1),     # D = 32 beyond the whole-row kernels' 128
    (1, 2, 64, 64, True, True, 0),      # one chunk
    (3, 2, 192, 64, True, False, 1),    # three chunks, padding masks of different lengths
    (32, 12, 128, 32, True, True, 0),   # C3 at full size: the whole-row kernels, two key blocks per (batch, head)
    (3, 2, 128, 32, False, False, 1),   # whole rows, no mask, accumulating
    (2, 3, 64, 32, True, True, 1),      # whole rows of 64: one key block, dQ written without a reduce
], ids=["c5", "L128-d64", "L256-d32", "L64-d64", "L192-d64", "c3", "L128-d32", "L64-d32"])
def test_attention_flash(dev, T, B, H, L, D, masked, packed, acc):
    """om_attention_{fwd,bwd}_flash (keys, then queries streamed through the workgroup, or whole rows of 64 or 128 at
    D = 32; the forward's row statistics feed the backward; dQ summed over key blocks in a fixed order) against the
    oracle's reference attention: O and
    dQ, dK, dV within 1e-5 scaled, accumulating into existing gradients when asked; the forward's statistics are each
    row's maximum logit (log2 units) and inverse sum; and two runs give the same bits."""
    rng = np.random.default_rng(B * L + D + H + 7)
    W = H * D
    ld = 3 * W if packed else W
    qkv = rnd(rng, B, L, 3 * W)
    g = rnd(rng, B, L, W)
    mask = None
    if masked:
        lens = rng.integers(L // 2, L + 1, B)
        mask = np.zeros((B, L, L), np.float32)
        for b in range(B):
            mask[b, :, lens[b]:] = -np.inf
    heads = lambda a: np.ascontiguousarray(a.reshape(B, L, H, D).transpose(0, 2, 1, 3))
    parts = [qkv[:, :, i * W:(i + 1) * W] for i in range(3)]
    tq, tk, tv = (heads(a) for a in parts)
    tg = heads(g)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    o_ref = np.empty_like(tq)
    mp = T.fp(mask) if masked else None
    T.lib().or_attention_fwd(T.fp(tq), T.fp(tk), T.fp(tv), mp, 1, T.fp(o_ref), B, H, L, L, D, C.c_float(scale))
    dq, dk, dv = np.empty_like(tq), np.empty_like(tk), np.empty_like(tv)
    T.lib().or_attention_bwd(T.fp(tq), T.fp(tk), T.fp(tv), mp, 1, T.fp(tg), T.fp(dq), T.fp(dk), T.fp(dv), B, H, L, L,
                             D, C.c_float(scale))
    base = 0.5 if acc else 0.0
    if packed:
        QKV = dev.put(qkv)
        qp = [QKV.data_ptr() + 4 * i * W for i in range(3)]
        DQKV = dev.empty((B, L, 3 * W), fill=base)
        dp = [DQKV.data_ptr() + 4 * i * W for i in range(3)]
        got = lambda: [dev.get(DQKV)[:, :, i * W:(i + 1) * W] for i in range(3)]
    else:
        QS = [dev.put(np.ascontiguousarray(a)) for a in parts]
        qp = [t.data_ptr() for t in QS]
        DS = [dev.empty((B, L, W), fill=base) for _ in range(3)]
        dp = [t.data_ptr() for t in DS]
        got = lambda: [dev.get(t) for t in DS]
    G, M = dev.put(g), (dev.put(mask) if masked else None)
    O, ST = dev.empty((B, L, W)), dev.empty((2, B, H, L))
    dev.call("om_attention_fwd_flash", qp[0], qp[1], qp[2], ld, M, 1, O, W, ST, B, H, L, D, C.c_float(scale))
    o_dev = dev.get(O)
    assert scaled(heads(o_dev), o_ref) <= TOL
    # the statistics: row maximum of x = S scale log2(e) + mask log2(e), and 1 / sum of 2^(x - max)
    st = dev.get(ST)
    x = (np.matmul(tq.astype(np.float64), tk.astype(np.float64).transpose(0, 1, 3, 2)) * scale
         + (mask[:, None].astype(np.float64) if masked else 0.0)) * np.log2(np.e)
    mx = x.max(-1)
    assert np.max(np.abs(st[0] - mx)) <= 1e-5 * max(1.0, float(np.max(np.abs(mx))))
    assert np.max(np.abs(st[1] * np.exp2(x - mx[..., None]).sum(-1) - 1.0)) <= 1e-5
    runs = []
    for rep in range(2):
        if rep:
            for t_ in ([DQKV] if packed else DS):
                dev.call("om_fill", t_, C.c_float(base), C.c_int64(t_.nbytes // 4))
        dev.call("om_attention_bwd_flash", qp[0], qp[1], qp[2], ld, M, 1, O, W, ST, G, W, dp[0], dp[1], dp[2], ld, B,
                 H, L, D, C.c_float(scale), acc)
        runs.append([a.copy() for a in got()])
    for gd, ref in zip(runs[0], (dq, dk, dv)):
        assert scaled(heads(gd) - np.float32(base), ref) <= TOL
    for a, b in zip(runs[0], runs[1]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _attention_oracle(T, tq, tk, tv, tg, mask, B, H, Lq, Lk, D, scale):
    """The oracle's attention forward and backward on [B, H, L, D] tensors (mask [B, Lq, Lk] or None)."""
    o = np.empty_like(tq)
    mp = T.fp(mask) if mask is not None else None
    T.lib().or_attention_fwd(T.fp(tq), T.fp(tk), T.fp(tv), mp, 1, T.fp(o), B, H, Lq, Lk, D, C.c_float(scale))
    dq, dk, dv = np.empty_like(tq), np.empty_like(tk), np.empty_like(tv)
    T.lib().or_attention_bwd(T.fp(tq), T.fp(tk), T.fp(tv), mp, 1, T.fp(tg), T.fp(dq), T.fp(dk), T.fp(dv), B, H, Lq,
                             Lk, D, C.c_float(scale))
    return o, dq, dk, dv


def _same_nans_then_close(got, ref, what):
    """NaN exactly where the oracle has NaN; every other entry within the 1e-5 scaled bar."""
    assert np.array_equal(np.isnan(got), np.isnan(ref)), what
    fin = ~np.isnan(ref)
    assert scaled(got[fin], ref[fin]) <= TOL, what


@pytest.mark.parametrize("B,H,Lq,Lk,D,mask_kind,scale", [
    (2, 2, 5, 7, 4, None, 0.0),      # GradCheckTests.cs:151: Lq 5, Lk 7, D 4, the default scale 1/sqrt(D)
    (2, 2, 5, 7, 4, "finite", 0.0),  # :152-160: a [B, Lq, Lk] mask with a quarter of its entries -3
    (1, 2, 4, 4, 6, None, 0.3),      # :161: an explicit scale
    (2, 2, 8, 8, 4, "row", 0.0),     # a query row with every key masked
], ids=["lq5-lk7", "lq5-lk7-mask-3", "scale0.3", "masked-row"])
def test_attention_reference_gradcheck_shapes(dev, T, B, H, Lq, Lk, D, mask_kind, scale):
    """The reference's own attention gradient-check shapes (cross-attention lengths, a small even D, a finite
    additive mask, an explicit scale) through om_attention_fwd / om_attention_bwd against the oracle, and a fully
    masked query row, which gives NaN in that row's outputs (docs/kernels-attention.md:33-35) and, through the
    backward, in that row's dQ and in dK and dV of its (batch, head): the same NaN positions as the oracle, every
    other value within 1e-5 scaled."""
    rng = np.random.default_rng(Lq * 100 + Lk * 10 + D)
    q, g = rnd(rng, B, Lq, H, D), rnd(rng, B, Lq, H, D)
    k, v = rnd(rng, B, Lk, H, D), rnd(rng, B, Lk, H, D)
    mask = None
    if mask_kind == "finite":
        mask = np.where(rng.integers(0, 4, (B, Lq, Lk)) == 0, -3.0, 0.0).astype(np.float32)
    elif mask_kind == "row":
        mask = np.where(rng.integers(0, 4, (B, Lq, Lk)) == 0, -np.inf, 0.0).astype(np.float32)
        mask[:, :, 0] = 0.0  # every other row keeps a key
        mask[1, 3, :] = -np.inf
    sc = float(np.float32(1.0) / np.sqrt(np.float32(D))) if scale == 0.0 else scale
    tq, tk, tv, tg = (np.ascontiguousarray(a.transpose(0, 2, 1, 3)) for a in (q, k, v, g))
    o_ref, dq, dk, dv = _attention_oracle(T, tq, tk, tv, tg, mask, B, H, Lq, Lk, D, sc)
    if mask_kind == "row":
        assert np.isnan(o_ref[1, :, 3]).all() and np.isnan(dk[1]).all() and np.isnan(dv[1]).all()
        assert not any(np.isnan(t[0]).any() for t in (o_ref, dq, dk, dv))
    Q, K, V, G = dev.put(q), dev.put(k), dev.put(v), dev.put(g)
    M = dev.put(mask) if mask is not None else None
    O, P, DS = dev.empty(q.shape), dev.empty((B, H, Lq, Lk)), dev.empty((B, H, Lq, Lk))
    DQ, DK, DV = dev.empty(q.shape), dev.empty(k.shape), dev.empty(v.shape)
    dev.call("om_attention_fwd", Q, K, V, M, 1, O, P, B, H, Lq, Lk, D, C.c_float(sc))
    dev.call("om_attention_bwd", Q, K, V, P, G, DQ, DK, DV, DS, B, H, Lq, Lk, D, C.c_float(sc), 0)
    back = lambda t: dev.get(t).transpose(0, 2, 1, 3)
    _same_nans_then_close(back(O), o_ref, "o")
    for name, got, ref in (("dq", DQ, dq), ("dk", DK, dk), ("dv", DV, dv)):
        _same_nans_then_close(back(got), ref, name)


@pytest.mark.parametrize("L", [1, 3, 65, 100])
def test_attention_flash_entry_at_other_lengths(dev, T, L):
    """The entry points the tape calls (om_attention_{fwd,bwd}_flash) at sequence lengths none of the fast kernels
    takes (one key, a few, just past a block of 64, and not a multiple of 64): they fall back to the recomputing
    path and still match the oracle within 1e-5 scaled, with a padding mask."""
    B, H, D = 3, 2, 32
    W = H * D
    rng = np.random.default_rng(L + 1000)
    qkv, g = rnd(rng, B, L, 3 * W), rnd(rng, B, L, W)
    lens = rng.integers((L + 1) // 2, L + 1, B)
    mask = np.zeros((B, L, L), np.float32)
    for b in range(B):
        mask[b, :, lens[b]:] = -np.inf
    heads = lambda a: np.ascontiguousarray(a.reshape(B, L, H, D).transpose(0, 2, 1, 3))
    tq, tk, tv = (heads(qkv[:, :, i * W:(i + 1) * W]) for i in range(3))
    sc = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    o_ref, dq, dk, dv = _attention_oracle(T, tq, tk, tv, heads(g), mask, B, H, L, L, D, sc)
    QKV, G, M = dev.put(qkv), dev.put(g), dev.put(mask)
    qp = [QKV.data_ptr() + 4 * i * W for i in range(3)]
    DQKV = dev.empty((B, L, 3 * W), fill=0.0)
    dp = [DQKV.data_ptr() + 4 * i * W for i in range(3)]
    O, ST = dev.empty((B, L, W)), dev.empty((2, B, H, L))
    dev.call("om_attention_fwd_flash", qp[0], qp[1], qp[2], 3 * W, M, 1, O, W, ST, B, H, L, D, C.c_float(sc))
    dev.call("om_attention_bwd_flash", qp[0], qp[1], qp[2], 3 * W, M, 1, O, W, ST, G, W, dp[0], dp[1], dp[2], 3 * W,
             B, H, L, D, C.c_float(sc), 0)
    assert scaled(heads(dev.get(O)), o_ref) <= TOL
    d = dev.get(DQKV)
    for i, ref in enumerate((dq, dk, dv)):
        assert scaled(heads(d[:, :, i * W:(i + 1) * W]), ref) <= TOL


@pytest.mark.parametrize("L,D,path", [(64, 32, "flash"), (128, 32, "flash"), (128, 64, "flash"), (64, 32, "fused")],
                         ids=["rows-L64", "rows-L128", "stream-d64", "fused-L64"])
def test_attention_fully_masked_row(dev, T, L, D, path):
    """A query row whose keys are all masked through the entry points the tape calls (the whole-row kernels with
    statistics at D = 32, the streaming kernels at D = 64, the exact fused kernels): NaN in the row's output and, in
    the backward, NaN in that row's dQ and in dK and dV of its (batch, head), as the oracle; everything else within
    1e-5 scaled."""
    B, H = 2, 3
    W = H * D
    rng = np.random.default_rng(L + D + (path == "fused"))
    qkv, g = rnd(rng, B, L, 3 * W), rnd(rng, B, L, W)
    lens = rng.integers(L // 2, L + 1, B)
    mask = np.zeros((B, L, L), np.float32)
    for b in range(B):
        mask[b, :, lens[b]:] = -np.inf
    mask[1, 5, :] = -np.inf
    heads = lambda a: np.ascontiguousarray(a.reshape(B, L, H, D).transpose(0, 2, 1, 3))
    tq, tk, tv = (heads(qkv[:, :, i * W:(i + 1) * W]) for i in range(3))
    sc = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    o_ref, dq, dk, dv = _attention_oracle(T, tq, tk, tv, heads(g), mask, B, H, L, L, D, sc)
    # the case the test is for: NaN in row 5 of batch 1 and its dQ, in all of batch 1's dK and dV, nowhere in batch 0
    assert np.isnan(o_ref[1, :, 5]).all() and np.isnan(dq[1, :, 5]).all() and np.isnan(dk[1]).all()
    assert np.isnan(dv[1]).all() and not any(np.isnan(t[0]).any() for t in (o_ref, dq, dk, dv))
    QKV, G, M = dev.put(qkv), dev.put(g), dev.put(mask)
    qp = [QKV.data_ptr() + 4 * i * W for i in range(3)]
    DQKV = dev.empty((B, L, 3 * W), fill=0.0)
    dp = [DQKV.data_ptr() + 4 * i * W for i in range(3)]
    O = dev.empty((B, L, W))
    if path == "flash":
        ST = dev.empty((2, B, H, L))
        dev.call("om_attention_fwd_flash", qp[0], qp[1], qp[2], 3 * W, M, 1, O, W, ST, B, H, L, D, C.c_float(sc))
        dev.call("om_attention_bwd_flash", qp[0], qp[1], qp[2], 3 * W, M, 1, O, W, ST, G, W, dp[0], dp[1], dp[2],
                 3 * W, B, H, L, D, C.c_float(sc), 0)
    else:
        dev.call("om_attention_fwd_fused", qp[0], qp[1], qp[2], 3 * W, M, 1, O, W, B, H, L, D, C.c_float(sc))
        dev.call("om_attention_bwd_fused", qp[0], qp[1], qp[2], 3 * W, M, 1, G, W, dp[0], dp[1], dp[2], 3 * W, B, H,
                 L, D, C.c_float(sc), 0)
    _same_nans_then_close(heads(dev.get(O)), o_ref, "o")
    d = dev.get(DQKV)
    for i, (name, ref) in enumerate((("dq", dq), ("dk", dk), ("dv", dv))):
        _same_nans_then_close(heads(d[:, :, i * W:(i + 1) * W]), ref, name)


@pytest.mark.parametrize("L,masked", [(128, True), (128, False), (64, True)])
def test_attention_bwd_kernels_agree(dev, L, masked):
    """The backward's two fused kernels give the same bits: 24 x 12 (head, batch) pairs run the quarter-staged
    kernel (more pairs than CUs), each half of the batch alone the one-pass kernel; same inputs, accumulating into
    the same initial gradients."""
    B, H, D = 24, 12, 32
    W = H * D
    rng = np.random.default_rng(L + masked)
    qkv, g = rnd(rng, B, L, 3 * W), rnd(rng, B, L, W)
    mask = np.where(rng.random((B, L, L)) < 0.15, -1e9, 0.0).astype(np.float32) if masked else None
    init = rnd(rng, B, L, 3 * W)
    QKV, G, M = dev.put(qkv), dev.put(g), (dev.put(mask) if masked else None)
    outs = []
    for halves in (1, 2):
        D3 = dev.put(init)
        bh = B // halves
        for i in range(halves):
            off = i * bh * L
            q = QKV.data_ptr() + 4 * off * 3 * W
            m = (M.data_ptr() + 4 * i * bh * L * L) if masked else None
            dq = D3.data_ptr() + 4 * off * 3 * W
            dev.call("om_attention_bwd_fused", q, q + 4 * W, q + 8 * W, 3 * W, m, 1, G.data_ptr() + 4 * off * W, W,
                     dq, dq + 4 * W, dq + 8 * W, 3 * W, bh, H, L, D, C.c_float(0.0), 1)
        outs.append(dev.get(D3))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


# ------------------------------------------------------------------------------------------------ conv and pool
@pytest.mark.parametrize("N,Cin,H,W,Cout,K,S,P", [(2, 64, 14, 14, 64, 3, 1, 1), (2, 1, 32, 128, 32, 3, 1, 1),
                                                  (3, 32, 16, 64, 64, 3, 1, 1), (2, 5, 9, 11, 7, 3, 2, 1),
                                                  (1, 128, 4, 32, 256, 3, 1, 1),
                                                  # C2 at full size: dW reduces over 32 images x 3136 pixels
                                                  (32, 64, 56, 56, 64, 3, 1, 1),
                                                  # C4's four stages at full batch
                                                  (32, 1, 32, 128, 32, 3, 1, 1), (32, 32, 16, 64, 64, 3, 1, 1),
                                                  (32, 64, 8, 32, 128, 3, 1, 1), (32, 128, 4, 32, 256, 3, 1, 1),
                                                  # the staged 3x3 kernels at widths that are not multiples of 16,
                                                  # images smaller than a tile, and both channel blocks
                                                  (3, 16, 7, 12, 32, 3, 1, 1), (2, 32, 9, 20, 64, 3, 1, 1),
                                                  (2, 48, 5, 36, 96, 3, 1, 1),
                                                  # one input channel at odd sizes and a ragged last band
                                                  (3, 1, 7, 9, 5, 3, 1, 1), (2, 1, 33, 20, 16, 3, 1, 1),
                                                  (2, 1, 6, 130, 9, 3, 1, 1)])
def test_conv2d(dev, T, N, Cin, H, W, Cout, K, S, P):
    rng = np.random.default_rng(N * Cin + Cout)
    x, w, b = rnd(rng, N, Cin, H, W), rnd(rng, Cout, Cin, K, K, scale=0.2), rnd(rng, Cout)
    OH, OW = (H + 2 * P - K) // S + 1, (W + 2 * P - K) // S + 1
    g = rnd(rng, N, Cout, OH, OW)
    y = np.empty((N, Cout, OH, OW), np.float32)
    T.lib().or_conv2d_fwd(T.fp(x), T.fp(w), T.fp(b), T.fp(y), N, Cin, H, W, Cout, K, K, S, P)
    dx, dw, db = np.empty_like(x), np.empty_like(w), np.empty_like(b)
    T.lib().or_conv2d_bwd(T.fp(g), T.fp(x), T.fp(w), T.fp(dx), T.fp(dw), T.fp(db), N, Cin, H, W, Cout, K, K, S, P)
    X, Wd, Bd, G = dev.put(x), dev.put(w), dev.put(b), dev.put(g)
    Y, DX, DW, DB = dev.empty(y.shape), dev.empty(x.shape), dev.empty(w.shape), dev.empty(b.shape)
    dev.call("om_conv2d_fwd", X, Wd, Bd, Y, N, Cin, H, W, Cout, K, K, S, P)
    dev.call("om_conv2d_bwd", G, X, Wd, DX, DW, DB, N, Cin, H, W, Cout, K, K, S, P, 0, 0)
    assert scaled(dev.get(Y), y) <= TOL
    assert scaled(dev.get(DX), dx) <= TOL
    assert scaled(dev.get(DW), dw) <= TOL
    assert scaled(dev.get(DB), db) <= 1e-7
    # the ReLU in the convolution's epilogue: the same bits as the convolution followed by om_relu_fwd
    YR, YR2 = dev.empty(y.shape), dev.empty(y.shape)
    dev.call("om_conv2d_relu_fwd", X, Wd, Bd, YR, N, Cin, H, W, Cout, K, K, S, P)
    dev.call("om_relu_fwd", Y, YR2, y.size)
    assert np.array_equal(dev.get(YR).view(np.uint32), dev.get(YR2).view(np.uint32))
    # a conv stage in one call (the ReLU's zeros make ties in most windows): a, the pooled values and their indices
    # equal om_conv2d_relu_fwd then om_maxpool_fwd, for windows that tile the output and ones that do not
    for (kh, kw), (sh, sw) in (((2, 2), (2, 2)), ((2, 1), (2, 1)), ((3, 3), (2, 2))):
        if kh > OH or kw > OW:
            continue
        PH, PW = (OH - kh) // sh + 1, (OW - kw) // sw + 1
        A1, P1, I1 = dev.empty(y.shape), dev.empty((N, Cout, PH, PW)), dev.empty((N, Cout, PH, PW), np.int32)
        P2, I2 = dev.empty((N, Cout, PH, PW)), dev.empty((N, Cout, PH, PW), np.int32)
        dev.call("om_conv2d_relu_pool_fwd", X, Wd, Bd, A1, P1, I1, N, Cin, H, W, Cout, K, K, S, P, kh, kw, sh, sw)
        dev.call("om_maxpool_fwd", YR, P2, I2, N, Cout, OH, OW, kh, kw, sh, sw, 0, 0)
        assert np.array_equal(dev.get(A1).view(np.uint32), dev.get(YR).view(np.uint32)), (kh, kw)
        assert np.array_equal(dev.get(P1).view(np.uint32), dev.get(P2).view(np.uint32)), (kh, kw)
        assert np.array_equal(dev.get(I1), dev.get(I2)), (kh, kw)
    # accumulating into the existing gradients, and the same bits on a second run
    first = [dev.get(t).copy() for t in (DX, DW, DB)]
    dev.call("om_conv2d_bwd", G, X, Wd, DX, DW, DB, N, Cin, H, W, Cout, K, K, S, P, 1, 1)
    assert scaled(dev.get(DX), dx + dx) <= TOL
    assert scaled(dev.get(DW), dw + dw) <= TOL
    dev.call("om_conv2d_bwd", G, X, Wd, DX, DW, DB, N, Cin, H, W, Cout, K, K, S, P, 0, 0)
    for a, t in zip(first, (DX, DW, DB)):
        assert np.array_equal(a.view(np.uint32), dev.get(t).view(np.uint32))


@pytest.mark.parametrize("B,Cc,H,W", [(32, 256, 2, 32), (3, 5, 7, 11), (1, 1, 1, 1)])
def test_mean_permute_bit_exact(dev, B, Cc, H, W):
    """The CRNN's sequence head in one call each way: om_mean_permute_fwd equals om_mean_axis (axis 2) then
    om_permute(2, 0, 1), and om_mean_permute_bwd equals the permute's backward then om_mean_axis_bwd, bit for bit,
    also accumulating."""
    rng = np.random.default_rng(B * Cc + H * W)
    x, g = rnd(rng, B, Cc, H, W), rnd(rng, W, B, Cc)
    X, G = dev.put(x), dev.put(g)
    Y, M, YP = dev.empty((W, B, Cc)), dev.empty((B, Cc, W)), dev.empty((W, B, Cc))
    dev.call("om_mean_permute_fwd", X, Y, B, Cc, H, W)
    dev.call("om_mean_axis", X, M, B * Cc, H, W)
    shape, perm = (C.c_int32 * 3)(B, Cc, W), (C.c_int32 * 3)(2, 0, 1)
    dev.call("om_permute", M, YP, 3, shape, perm, 0)
    assert np.array_equal(dev.get(Y).view(np.uint32), dev.get(YP).view(np.uint32))
    GB, DX1, DX2 = dev.empty((B, Cc, W)), dev.empty(x.shape), dev.empty(x.shape)
    gshape, gperm = (C.c_int32 * 3)(W, B, Cc), (C.c_int32 * 3)(1, 2, 0)
    dev.call("om_permute", G, GB, 3, gshape, gperm, 0)
    for acc in (0, 1):
        dev.call("om_mean_permute_bwd", G, DX1, B, Cc, H, W, acc)
        dev.call("om_mean_axis_bwd", GB, DX2, B * Cc, H, W, acc)
        assert np.array_equal(dev.get(DX1).view(np.uint32), dev.get(DX2).view(np.uint32)), acc


@pytest.mark.parametrize("shape,k,s,p", [((2, 3, 8, 12), (2, 2), (2, 2), (0, 0)), ((2, 4, 8, 6), (2, 1), (2, 1), (0, 0)),
                                         ((1, 2, 9, 9), (3, 3), (2, 2), (0, 0)),
                                         # GradCheckTests.cs:86: 3x3, stride 2, padding 1 (overlapping windows, and
                                         # windows at the border whose padded taps never win)
                                         ((2, 3, 9, 10), (3, 3), (2, 2), (1, 1))])
def test_maxpool_bit_exact(dev, T, shape, k, s, p):
    rng = np.random.default_rng(sum(shape))
    x = rng.integers(-2, 3, shape).astype(np.float32)  # many ties
    x.reshape(-1)[7] = np.nan
    N, Cc, H, W = shape
    OH, OW = (H + 2 * p[0] - k[0]) // s[0] + 1, (W + 2 * p[1] - k[1]) // s[1] + 1
    y, idx = np.empty((N, Cc, OH, OW), np.float32), np.empty((N, Cc, OH, OW), np.int32)
    T.lib().or_maxpool_fwd(T.fp(x), T.fp(y), T.ip(idx), N, Cc, H, W, k[0], k[1], s[0], s[1], p[0], p[1])
    g = rnd(rng, *y.shape)
    dx = np.empty_like(x)
    T.lib().or_maxpool_bwd(T.fp(g), T.ip(idx), T.fp(dx), C.c_int64(idx.size), C.c_int64(x.size))
    X, Y, I, G, DX = dev.put(x), dev.empty(y.shape), dev.empty(y.shape, np.int32), dev.put(g), dev.empty(x.shape)
    dev.call("om_maxpool_fwd", X, Y, I, N, Cc, H, W, k[0], k[1], s[0], s[1], p[0], p[1])
    dev.call("om_maxpool_bwd", G, I, DX, N, Cc, H, W, OH, OW, k[0], k[1], s[0], s[1], p[0], p[1], 0)
    assert np.array_equal(dev.get(I), idx)
    assert np.array_equal(dev.get(Y).view(np.uint32), y.view(np.uint32))
    assert np.array_equal(dev.get(DX), dx)
    # with the backward of the ReLU that produced the pool's input (x read as that ReLU's output): the pooled
    # gradient where x > 0, the same bits as om_maxpool_bwd then om_relu_bwd, accumulating as asked
    DX2 = dev.empty(x.shape, fill=0.5)
    dev.call("om_maxpool_relu_bwd", G, I, X, DX2, N, Cc, H, W, OH, OW, k[0], k[1], s[0], s[1], p[0], p[1], 1)
    ref = np.where(x > 0, dx, np.float32(0.0)).astype(np.float32) + np.float32(0.5)
    assert np.array_equal(dev.get(DX2).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("N,Cc,H,W", [(32, 64, 56, 56), (2, 3, 5, 7), (4, 16, 1, 300)])
def test_relu_mean_plane(dev, T, N, Cc, H, W):
    """ReLU + mean over each plane (forward and backward) in one launch each: the same bits as om_relu_fwd +
    om_mean_axis and om_mean_axis_bwd + om_relu_bwd, which the oracle pins (mean within 1e-7, ReLU bit-exact)."""
    rng = np.random.default_rng(N + H)
    x = rnd(rng, N, Cc, H, W)
    x.reshape(-1)[3] = 0.0
    x.reshape(-1)[5] = -0.0
    g = rnd(rng, N, Cc)
    P = H * W
    X, G = dev.put(x), dev.put(g)
    Y, R, Y2 = dev.empty((N, Cc)), dev.empty(x.shape), dev.empty((N, Cc))
    dev.call("om_relu_mean_rows", X, Y, N * Cc, P)
    dev.call("om_relu_fwd", X, R, x.size)
    dev.call("om_mean_axis", R, Y2, N * Cc, P, 1)
    assert np.array_equal(dev.get(Y).view(np.uint32), dev.get(Y2).view(np.uint32))
    r = np.maximum(x, np.float32(0.0))
    assert scaled(dev.get(Y), r.reshape(N * Cc, P).astype(np.float64).mean(axis=1).reshape(N, Cc)) <= 1e-7
    DX, T1, DX2 = dev.empty(x.shape, fill=0.25), dev.empty(x.shape), dev.empty(x.shape, fill=0.25)
    dev.call("om_relu_mean_rows_bwd", G, X, DX, N * Cc, P, 1)
    dev.call("om_mean_axis_bwd", G, T1, N * Cc, P, 1, 0)
    dev.call("om_relu_bwd", T1, R, DX2, x.size, 1)
    assert np.array_equal(dev.get(DX).view(np.uint32), dev.get(DX2).view(np.uint32))
    ref = np.where(x > 0, (g / np.float32(P)).astype(np.float32)[:, :, None, None], np.float32(0)) + np.float32(0.25)
    assert np.array_equal(dev.get(DX).view(np.uint32), ref.astype(np.float32).view(np.uint32))


# ------------------------------------------------------------------------------------------------ CTC
def ctc_cases():
    from conftest import load_golden
    o = load_golden("autograd_crnn")
    yield "fixture", o["out.lp"], o["in.targets"].astype(np.int32), o["in.input_lengths"].astype(np.int32), \
        o["in.target_lengths"].astype(np.int32), 0, 0
    rng = np.random.default_rng(11)
    Tn, B, Cc = 32, 32, 37
    z = rng.standard_normal((Tn, B, Cc)).astype(np.float32)
    lp = (z - np.log(np.exp(z.astype(np.float64)).sum(-1, keepdims=True))).astype(np.float32)
    tl = rng.integers(1, 11, B).astype(np.int32)
    tl[0] = 0
    il = np.full(B, Tn, np.int32)
    il[1] = 3  # too short for its target: +inf / zero gradient
    tl[1] = 5
    labels = rng.integers(1, Cc, int(tl.sum())).astype(np.int32)
    yield "c4", lp, labels, il, tl, 0, 0
    # the same shape with the last class as the blank and zero_infinity (sequence 1's +inf loss becomes 0)
    yield "c4-blank-last", lp, (labels - 1).astype(np.int32), il, tl, Cc - 1, 1
    # long sequences: T x (2 L + 1) doubles beyond what the kernels keep in LDS (4096), so alpha and beta live in
    # device scratch
    Tn, B, Cc = 160, 3, 12
    z = rng.standard_normal((Tn, B, Cc)).astype(np.float32)
    lp = (z - np.log(np.exp(z.astype(np.float64)).sum(-1, keepdims=True))).astype(np.float32)
    tl = np.array([30, 12, 40], np.int32)
    il = np.array([Tn, 100, Tn], np.int32)
    labels = rng.integers(1, Cc, int(tl.sum())).astype(np.int32)
    yield "long", lp, labels, il, tl, 0, 0
    # CtcLossTests.cs:58-64: LogSoftmax of uniform(-1.5, 1.5) [5, 4, 4], targets [0, 1, 2, 2], input lengths
    # [5, 5, 2, 1], target lengths [0, 2, 2, 0], blank 3, zero_infinity: two empty targets, and [2, 2] needs three
    # frames where its input has two (loss +inf, zeroed)
    z = rng.uniform(-1.5, 1.5, (5, 4, 4)).astype(np.float32)
    lp = (z - np.log(np.exp(z.astype(np.float64)).sum(-1, keepdims=True))).astype(np.float32)
    yield "empty-impossible-blank3", lp, np.array([0, 1, 2, 2], np.int32), np.array([5, 5, 2, 1], np.int32), \
        np.array([0, 2, 2, 0], np.int32), 3, 1


@pytest.mark.parametrize("red", [0, 1, 2])
def test_ctc_bit_exact(dev, T, red):
    for name, lp, tg, il, tl, blank, zi in ctc_cases():
        Tn, B, Cc = lp.shape
        n_out = B if red == 0 else 1
        ref = np.empty(n_out, np.float32)
        T.lib().or_ctc_loss(T.fp(lp), T.ip(tg), T.ip(il), T.ip(tl), Tn, B, Cc, blank, red, zi, T.fp(ref))
        assert np.isfinite(ref).all() or not zi, name
        gin = np.linspace(0.5, 1.5, n_out).astype(np.float32)
        dref = np.empty_like(lp)
        T.lib().or_ctc_grad(T.fp(lp), T.ip(tg), T.ip(il), T.ip(tl), T.fp(gin), Tn, B, Cc, blank, red, T.fp(dref))
        LP, TG, IL, TL, L, GIN, D = dev.put(lp), dev.put(tg), dev.put(il), dev.put(tl), dev.empty((n_out,)), \
            dev.put(gin), dev.empty(lp.shape, fill=123.0)
        hil, htl, htg = (a.ctypes.data_as(C.c_void_p) for a in (il, tl, tg))
        dev.call("om_ctc_fwd", LP, TG, IL, TL, hil, htl, htg, tg.size, Tn, B, Cc, blank, red, zi, L)
        dev.call("om_ctc_bwd", LP, TG, IL, TL, hil, htl, htg, tg.size, GIN, D, Tn, B, Cc, blank, red, 0)
        got = dev.get(L)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), name
        assert np.array_equal(dev.get(D).view(np.uint32), dref.view(np.uint32)), name
        # the pair that runs each recursion once (beta beside alpha in the forward, tables kept): the same bits
        tb = dev.ctx.L.om_ctc_tables_bytes(Tn, B, int(tl.max()) if tl.size else 0)
        TB, L2, D2 = dev.empty((tb // 4 + 1,)), dev.empty((n_out,)), dev.empty(lp.shape, fill=123.0)
        dev.call("om_ctc_fwd_tables", LP, TG, IL, TL, hil, htl, htg, tg.size, Tn, B, Cc, blank, red, zi, L2, TB, tb)
        dev.call("om_ctc_bwd_tables", LP, TG, IL, TL, hil, htl, htg, tg.size, GIN, D2, Tn, B, Cc, blank, red, 0, TB,
                 tb)
        assert np.array_equal(dev.get(L2).view(np.uint32), ref.view(np.uint32)), name
        assert np.array_equal(dev.get(D2).view(np.uint32), dref.view(np.uint32)), name
        # a tables buffer smaller than om_ctc_tables_bytes is refused before any launch
        assert dev.status("om_ctc_fwd_tables", LP, TG, IL, TL, hil, htl, htg, tg.size, Tn, B, Cc, blank, red, zi, L2,
                          TB, tb - 8) == 1
        assert b"om_ctc_tables_bytes" in dev.ctx.L.om_last_error(dev.ctx.h)


def test_ctc_rejects_bad_targets(dev):
    lp = dev.empty((3, 1, 4), fill=0.0)
    tg = np.array([0], np.int32)  # the blank as a label
    il, tl = np.array([3], np.int32), np.array([1], np.int32)
    st = dev.status("om_ctc_fwd", lp, dev.put(tg), dev.put(il), dev.put(tl), il.ctypes.data_as(C.c_void_p),
                    tl.ctypes.data_as(C.c_void_p), tg.ctypes.data_as(C.c_void_p), 1, 3, 1, 4, 0, 1, 0, lp)
    assert st == 1 and b"differ from the blank" in dev.ctx.L.om_last_error(dev.ctx.h)


def test_ctc_bwd_rejects_what_it_would_index_with(dev):
    """om_ctc_bwd checks the host copies of the lengths and labels before it launches anything: an input length past
    T, target lengths that do not sum to the labels given, a label outside [0, C) or equal to the blank, and a blank
    outside [0, C) are refused with OM_E_ARG (each would make the kernel read lp or write dlp and its scratch out of
    bounds), and dlp is left untouched."""
    Tn, B, Cc = 4, 2, 5
    lp = dev.empty((Tn, B, Cc), fill=-1.0)
    g = dev.put(np.ones(1, np.float32))
    dlp = dev.empty((Tn, B, Cc), fill=7.0)

    def call(il, tl, tg, blank=0):
        il, tl, tg = (np.asarray(a, np.int32) for a in (il, tl, tg))
        st = dev.status("om_ctc_bwd", lp, dev.put(tg if tg.size else np.zeros(1, np.int32)), dev.put(il),
                        dev.put(tl), il.ctypes.data_as(C.c_void_p), tl.ctypes.data_as(C.c_void_p),
                        tg.ctypes.data_as(C.c_void_p), int(tg.size), g, dlp, Tn, B, Cc, blank, 1, 0)
        return st, dev.ctx.L.om_last_error(dev.ctx.h)

    cases = [
        (([5, 4], [1, 1], [1, 2]), b"Input length 5"),             # past T
        (([4, 4], [2, 1], [1, 2]), b"sum to 3 but 2 labels"),      # more labels claimed than given
        (([4, 4], [1, 1], [1, 5]), b"Target label 5"),             # label == C
        (([4, 4], [1, 1], [0, 2]), b"differ from the blank"),      # the blank as a label
        (([4, -1], [1, 1], [1, 2]), b"Input length -1"),           # negative input length
        (([4, 4], [1, -1], [1]), b"Target length -1"),             # negative target length
    ]
    for args, msg in cases:
        st, err = call(*args)
        assert st == 1 and msg in err, (args, st, err)
    st, err = call([4, 4], [1, 1], [1, 2], blank=5)
    assert st == 1 and b"blank index 5" in err
    assert np.all(dev.get(dlp) == 7.0)
    st, _ = call([4, 4], [1, 1], [1, 2])  # the same call with valid arguments runs
    assert st == 0


# ------------------------------------------------------------------------------------------------ optimizers
@pytest.mark.parametrize("cfg", [dict(wd=0.01, dec=1, ams=0), dict(wd=0.1, dec=0, ams=0), dict(wd=0.05, dec=1, ams=1),
                                 dict(wd=0.0, dec=0, ams=0)])
def test_adam_bit_exact(dev, T, cfg):
    rng = np.random.default_rng(5)
    n = 1_000_003
    p0, m0, v0 = rnd(rng, n), rnd(rng, n, scale=0.01), np.abs(rnd(rng, n, scale=1e-4))
    vm0 = v0 * 1.5
    P, M, V, VM = dev.put(p0), dev.put(m0), dev.put(v0), dev.put(vm0)
    p, m, v, vm = p0.copy(), m0.copy(), v0.copy(), vm0.copy()
    for t in range(1, 4):
        g = rnd(rng, n, scale=0.1)
        ss, sq = C.c_float(), C.c_float()
        T.lib().or_adam_scalars(C.c_float(1e-3), C.c_float(0.9), C.c_float(0.999), C.c_int64(t), C.byref(ss),
                                C.byref(sq))
        T.lib().or_adam_update(T.fp(p), T.fp(g), T.fp(m), T.fp(v), T.fp(vm) if cfg["ams"] else None, C.c_int64(n),
                               C.c_float(1e-3), C.c_float(0.9), C.c_float(0.999), C.c_float(1e-8),
                               C.c_float(cfg["wd"]), cfg["dec"], ss, sq)
        ss2, sq2 = C.c_float(), C.c_float()
        dev.ctx.L.om_adam_scalars(1e-3, 0.9, 0.999, t, C.byref(ss2), C.byref(sq2))
        assert ss2.value == ss.value and sq2.value == sq.value
        dev.call("om_adam_step", P, dev.put(g), M, V, VM if cfg["ams"] else None, n, C.c_float(1e-3), C.c_float(0.9),
                 C.c_float(0.999), C.c_float(1e-8), C.c_float(cfg["wd"]), cfg["dec"], ss2, sq2)
    for got, ref in ((P, p), (M, m), (V, v)):
        assert np.array_equal(dev.get(got).view(np.uint32), ref.view(np.uint32))


def test_sgd_bit_exact(dev, T):
    rng = np.random.default_rng(6)
    n = 10007
    p0 = rnd(rng, n)
    P, BUF = dev.put(p0), dev.empty((n,), fill=0.0)
    p, buf = p0.copy(), np.zeros(n, np.float32)
    for t in range(3):
        g = rnd(rng, n)
        T.lib().or_sgd_update(T.fp(p), T.fp(g), T.fp(buf), C.c_int64(n), C.c_float(0.1), C.c_float(0.9),
                              C.c_float(0.0), C.c_float(1e-2), 1, int(t == 0))
        dev.call("om_sgd_step", P, dev.put(g), BUF, n, C.c_float(0.1), C.c_float(0.9), C.c_float(0.0),
                 C.c_float(1e-2), 1, int(t == 0))
    assert np.array_equal(dev.get(P), p) and np.array_equal(dev.get(BUF), buf)
