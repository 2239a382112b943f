"""BatchNorm2d, AvgPool2d, Embedding and Dropout kernels of lib/libom_hip.so against the CPU oracle, on the GPU.

Bars: AvgPool2d, Embedding and Dropout restate the reference's order of operations and are compared bit for bit;
BatchNorm2d sums in fp64 in a different order than the reference's serial loops, so its outputs and gradients are
held to 1e-5 scaled error (in practice they agree to the float) and its running statistics likewise.
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


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("n,c,h,w", [(8, 4, 12, 12), (3, 5, 7, 9), (2, 64, 56, 56), (1, 3, 1, 1)])
@pytest.mark.parametrize("training", [1, 0])
def test_batchnorm2d(dev, T, n, c, h, w, training):
    rng = np.random.default_rng(n * 100 + c + training)
    plane = h * w
    x = (rng.standard_normal((n, c, h, w)) * 2 + 0.5).astype(np.float32)
    gam = rng.standard_normal(c).astype(np.float32)
    bet = rng.standard_normal(c).astype(np.float32)
    rm0 = (rng.standard_normal(c) * 0.1).astype(np.float32)
    rv0 = (1 + rng.random(c)).astype(np.float32)
    g = rng.standard_normal((n, c, h, w)).astype(np.float32)
    # oracle
    rm, rv = rm0.copy(), rv0.copy()
    y = np.empty_like(x)
    mean, inv = np.empty(c, np.float32), np.empty(c, np.float32)
    if training:
        T.lib().or_batchnorm_fwd(T.fp(x), T.fp(gam), T.fp(bet), T.fp(rm), T.fp(rv), T.fp(y), T.fp(mean), T.fp(inv), n,
                                 c, plane, C.c_float(0.1), C.c_float(1e-5))
        dx, dg, db = np.empty_like(x), np.empty(c, np.float32), np.empty(c, np.float32)
        T.lib().or_batchnorm_bwd(T.fp(g), T.fp(x), T.fp(gam), T.fp(mean), T.fp(inv), T.fp(dx), T.fp(dg), T.fp(db), n,
                                 c, plane)
    else:  # evaluation: statistics are the running ones (Ops.Layers.cs:215-223), dx = gamma * inv * g
        mean, inv = rm0.copy(), (np.float32(1) / np.sqrt(rv0 + np.float32(1e-5))).astype(np.float32)
        y = ((((x - mean[None, :, None, None]) * inv[None, :, None, None]) * gam[None, :, None, None])
             + bet[None, :, None, None]).astype(np.float32)
        dx = ((gam * inv)[None, :, None, None] * g).astype(np.float32)
        xhat = ((x - mean[None, :, None, None]) * inv[None, :, None, None]).astype(np.float32)
        dg = np.sum((g * xhat).astype(np.float64), axis=(0, 2, 3)).astype(np.float32)
        db = np.sum(g.astype(np.float64), axis=(0, 2, 3)).astype(np.float32)
    # device
    X, G, GA, BE = dev.put(x), dev.put(g), dev.put(gam), dev.put(bet)
    RM, RV = dev.put(rm0), dev.put(rv0)
    Y, MU, IV = dev.empty(x.shape), dev.empty((c,)), dev.empty((c,))
    dev.call("om_batchnorm2d_fwd", X, GA, BE, RM, RV, Y, MU, IV, n, c, plane, training, C.c_float(0.1),
             C.c_float(1e-5))
    DX, DG, DB = dev.empty(x.shape), dev.empty((c,), fill=0.5), dev.empty((c,), fill=0.5)
    dev.call("om_batchnorm2d_bwd", G, X, GA, MU, IV, DX, DG, DB, n, c, plane, training, 0, 1)
    assert scaled(dev.get(MU), mean) <= 1e-6 and scaled(dev.get(IV), inv) <= 1e-6
    assert scaled(dev.get(Y), y) <= 1e-5
    assert scaled(dev.get(DX), dx) <= 1e-5
    assert scaled(dev.get(DG), dg + np.float32(0.5)) <= 1e-5 and scaled(dev.get(DB), db + np.float32(0.5)) <= 1e-5
    if training:
        assert scaled(dev.get(RM), rm) <= 1e-6 and scaled(dev.get(RV), rv) <= 1e-6
    else:
        assert np.array_equal(bits(dev.get(RM)), bits(rm0)) and np.array_equal(bits(dev.get(RV)), bits(rv0))


@pytest.mark.parametrize("geo", [
    # (N*C, H, W, K, S, P, count_include_pad)
    (32, 6, 6, 2, 2, 0, 1), (12, 7, 9, 3, 2, 1, 1), (12, 7, 9, 3, 2, 1, 0), (5, 11, 10, 3, 1, 1, 0),
    (4, 8, 8, 4, 3, 2, 1), (1000, 14, 14, 2, 2, 0, 1),
], ids=str)
def test_avgpool2d_bit_exact(dev, T, geo):
    planes, h, w, k, s, p, cip = geo
    rng = np.random.default_rng(planes + h)
    x = rng.standard_normal((planes, h, w)).astype(np.float32)
    oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    g = rng.standard_normal((planes, oh, ow)).astype(np.float32)
    y, dx = np.empty((planes, oh, ow), np.float32), np.empty_like(x)
    T.lib().or_avgpool_fwd(T.fp(x), T.fp(y), planes, h, w, k, k, s, s, p, p, cip)
    T.lib().or_avgpool_bwd(T.fp(g), T.fp(dx), planes, h, w, k, k, s, s, p, p, cip)
    Y, DX = dev.empty(y.shape), dev.empty(x.shape, fill=0.25)
    dev.call("om_avgpool2d_fwd", dev.put(x), Y, planes, h, w, k, k, s, s, p, p, cip)
    dev.call("om_avgpool2d_bwd", dev.put(g), DX, planes, h, w, k, k, s, s, p, p, cip, 1)
    assert np.array_equal(bits(dev.get(Y)), bits(y))
    assert np.array_equal(bits(dev.get(DX)), bits(dx + np.float32(0.25)))


# The last three take the sorted path (rows x ids above 2^22): ids drawn from 40 values (long runs per id) or from the
# whole vocabulary, and a padding id that appears.
@pytest.mark.parametrize("rows,dim,n_ids,pad,spread", [(11, 16, 96, -1, 40), (50, 8, 1000, 3, 40),
                                                       (300, 130, 257, 0, 40), (1024, 64, 4096, 5, 40),
                                                       (30522, 64, 4096, 0, 40), (30522, 768, 4096, 7, 30522),
                                                       (4000, 33, 20000, 2, 4000)])
def test_embedding_bit_exact(dev, T, rows, dim, n_ids, pad, spread):
    rng = np.random.default_rng(rows + n_ids)
    table = rng.standard_normal((rows, dim)).astype(np.float32)
    ids = rng.integers(0, min(rows, spread), n_ids).astype(np.int32)  # repeated ids: order of the sums matters
    ids[::97] = pad if pad >= 0 else ids[::97]
    g = rng.standard_normal((n_ids, dim)).astype(np.float32)
    y, dt = np.empty((n_ids, dim), np.float32), np.empty_like(table)
    T.lib().or_embedding_fwd(T.fp(table), T.ip(ids), T.fp(y), n_ids, dim)
    T.lib().or_embedding_bwd(T.fp(g), T.ip(ids), T.fp(dt), n_ids, dim, rows, pad)
    I = dev.put(ids)
    Y, DT = dev.empty(y.shape), dev.empty(table.shape, fill=1.0)
    dev.call("om_embedding_fwd", dev.put(table), I, Y, n_ids, dim, rows)
    dev.call("om_embedding_bwd", dev.put(g), I, DT, n_ids, dim, rows, pad, 1)
    assert np.array_equal(bits(dev.get(Y)), bits(y))
    assert np.array_equal(bits(dev.get(DT)), bits(dt + np.float32(1.0)))


def test_embedding_out_of_range_reads_nothing(dev):
    table = np.ones((4, 8), np.float32)
    ids = np.array([0, 7, -2, 3], np.int32)
    Y = dev.empty((4, 8))
    dev.call("om_embedding_fwd", dev.put(table), dev.put(ids), Y, 4, 8, 4)
    y = dev.get(Y)
    assert np.all(y[[0, 3]] == 1.0) and np.all(np.isnan(y[[1, 2]]))


@pytest.mark.parametrize("n,p,seed,draw", [(1000, 0.3, 42, 0), (1000, 0.3, 42, 1), (1_000_003, 0.1, 3, 17),
                                           (64, 0.5, 7, 0), (77, 0.0, 1, 0)])
def test_dropout_bit_exact(dev, T, n, p, seed, draw):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    g = rng.standard_normal(n).astype(np.float32)
    y, dx = np.empty_like(x), np.empty_like(x)
    T.lib().or_dropout(T.fp(x), T.fp(y), C.c_int64(n), C.c_float(p), C.c_uint64(seed), C.c_int64(draw))
    T.lib().or_dropout(T.fp(g), T.fp(dx), C.c_int64(n), C.c_float(p), C.c_uint64(seed), C.c_int64(draw))
    Y, DX = dev.empty((n,)), dev.empty((n,), fill=-1.0)
    dev.call("om_dropout_fwd", dev.put(x), Y, n, C.c_float(p), C.c_uint64(seed), draw)
    dev.call("om_dropout_bwd", dev.put(g), DX, n, C.c_float(p), C.c_uint64(seed), draw, 1)
    assert np.array_equal(bits(dev.get(Y)), bits(y))
    assert np.array_equal(bits(dev.get(DX)), bits(dx + np.float32(-1.0)))
    if p > 0:
        assert dev.status("om_dropout_fwd", dev.put(x), Y, n, C.c_float(1.0), C.c_uint64(seed), draw) == 1
