"""TEST INFRASTRUCTURE ONLY: the CPU oracle's reverse-mode tape and models.

A small Python restatement of the reference's autograd engine (src/OneModel/Tensors/Autograd/Engine.cs:124-344) over the
C restatement of its kernels (oracle/om_oracle.c). It exists so that parity tests can run the reference's training
path on the CPU, on the same inputs as the HIP library, and compare. Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg import it; the product never does.

Every op below cites the reference op it restates. Tensors are numpy arrays (float32, C-contiguous; int32 for ids,
labels and pool indices).
"""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

F32P = ctypes.POINTER(ctypes.c_float)
I32P = ctypes.POINTER(ctypes.c_int32)


def lib():
    """Loads oracle/_build/liboracle.so (built by `make -C oracle`)."""
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "_build", "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run `make -C oracle`)")
        L = ctypes.CDLL(path)
        L.or_splitmix_next.restype = ctypes.c_uint64
        L.or_splitmix_next.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.or_next_single.restype = ctypes.c_float
        L.or_next_single.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        for name in ("or_exp", "or_exp_nonpos", "or_erf", "or_gelu"):
            getattr(L, name).restype = ctypes.c_float
            getattr(L, name).argtypes = [ctypes.c_float]
        for name in ("or_ctc_exp", "or_ctc_log"):
            getattr(L, name).restype = ctypes.c_double
            getattr(L, name).argtypes = [ctypes.c_double]
        L.or_ctc_logadd.restype = ctypes.c_double
        L.or_ctc_logadd.argtypes = [ctypes.c_double, ctypes.c_double]
        L.or_sum_all.restype = ctypes.c_float
        L.or_nll_fwd.restype = ctypes.c_float
        L.or_clip_norm.restype = ctypes.c_float
        L.or_clip_norm.argtypes = [ctypes.POINTER(F32P), ctypes.POINTER(ctypes.c_int64), ctypes.c_int,
                                   ctypes.c_float, ctypes.c_int, F32P]
        L.or_clip_value.restype = None
        L.or_clip_value.argtypes = [ctypes.POINTER(F32P), ctypes.POINTER(ctypes.c_int64), ctypes.c_int,
                                    ctypes.c_float]
        _LIB = L
    return _LIB


def fp(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous, (a.dtype, a.flags)
    return a.ctypes.data_as(F32P)


def ip(a):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(I32P)


def c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ----------------------------------------------------------------------------------------------------------- generator
class Generator:
    """SplitMix64 generator of Generator.cs:10-48 (the reference's init source)."""

    def __init__(self, seed: int):
        self.state = ctypes.c_uint64(seed & 0xFFFFFFFFFFFFFFFF)

    def next_u64(self) -> int:
        return lib().or_splitmix_next(ctypes.byref(self.state))

    def uniform(self, low: float, high: float, shape) -> np.ndarray:
        out = np.empty(shape, np.float32)
        lib().or_fill_uniform(ctypes.byref(self.state), ctypes.c_float(low), ctypes.c_float(high), fp(out),
                              ctypes.c_int64(out.size))
        return out

    def normal(self, shape) -> np.ndarray:
        out = np.empty(shape, np.float32)
        lib().or_fill_normal(ctypes.byref(self.state), fp(out), ctypes.c_int64(out.size))
        return out

    def ints(self, lo: int, hi: int, shape) -> np.ndarray:
        out = np.empty(shape, np.int32)
        lib().or_fill_int(ctypes.byref(self.state), ctypes.c_int32(lo), ctypes.c_int32(hi), ip(out),
                          ctypes.c_int64(out.size))
        return out


def fan_in_bound(fan_in: int) -> float:
    """1/sqrt(fanIn) in float32, as `1f / MathF.Sqrt(inFeatures)` (Layers.cs:59)."""
    return float(np.float32(1.0) / np.sqrt(np.float32(fan_in)))


# ----------------------------------------------------------------------------------------------------------- tape
class Tensor:
    __slots__ = ("data", "requires_grad", "grad_fn", "grad", "name")

    def __init__(self, data, requires_grad=False, name=None):
        self.data = data
        self.requires_grad = requires_grad
        self.grad_fn = None
        self.grad = None
        self.name = name

    @property
    def shape(self):
        return self.data.shape


class Record:
    """A BackwardRecord (BackwardRecord.cs:17-150): inputs in order, a backward rule, the pending gradient."""

    __slots__ = ("inputs", "rule", "pending", "mark")

    def __init__(self, inputs, rule):
        self.inputs = inputs
        self.rule = rule
        self.pending = None
        self.mark = 0


def _tracked(*xs):
    return any(isinstance(x, Tensor) and x.requires_grad for x in xs)


def _attach(out_data, inputs, rule):
    t = Tensor(out_data)
    if _tracked(*inputs):
        t.requires_grad = True
        t.grad_fn = Record(list(inputs), rule)
    return t


def needs(x):
    return isinstance(x, Tensor) and x.requires_grad


_PASS = [0]


def backward(root: Tensor):
    """Backprop.Run + Engine.Execute (Engine.cs:28-74, 124-207): DFS post-order over input edges in input order,
    reversed; one pending gradient per record; Emit accumulates into the producer or the leaf (Engine.cs:210-344)."""
    assert root.requires_grad and root.data.size == 1
    g = np.ones(root.data.shape, np.float32)
    if root.grad_fn is None:
        _accumulate_leaf(root, g)
        return
    _PASS[0] += 1
    mark = _PASS[0]
    order, stack = [], [(root.grad_fn, 0)]
    root.grad_fn.mark = mark
    while stack:
        rec, nxt = stack[-1]
        if nxt < len(rec.inputs):
            stack[-1] = (rec, nxt + 1)
            x = rec.inputs[nxt]
            prod = x.grad_fn if isinstance(x, Tensor) else None
            if prod is not None and prod.mark != mark:
                prod.mark = mark
                stack.append((prod, 0))
        else:
            order.append(rec)
            stack.pop()
    root.grad_fn.pending = g
    for rec in reversed(order):
        gi = rec.pending
        rec.pending = None
        if gi is None:
            continue
        grads = rec.rule(gi)
        for x, gx in zip(rec.inputs, grads):
            if gx is None or not needs(x):
                continue
            _emit(x, gx)


def _emit(x: Tensor, g: np.ndarray):
    if x.grad_fn is None:
        _accumulate_leaf(x, g)
    elif x.grad_fn.pending is None:
        x.grad_fn.pending = np.array(g, np.float32, copy=True)
    else:
        x.grad_fn.pending += g  # Engine.AddInto: dst += src in element order


def _accumulate_leaf(x: Tensor, g: np.ndarray):
    if x.grad is None:
        x.grad = np.array(g, np.float32, copy=True)
    else:
        x.grad += g


def zero_grad(params):
    """Backprop.ZeroGrad (Engine.cs:77-91)."""
    for p in params:
        if p.grad is not None:
            p.grad[...] = 0.0


# ----------------------------------------------------------------------------------------------------------- ops
def sum_to(g: np.ndarray, shape) -> np.ndarray:
    """BackwardOps.SumTo (BackwardOps.cs:201-269): fp64 sum over broadcast axes in increasing element order, rounded
    once. Covers the leading-axes broadcast the configs use (a bias [n] against [rows, n]); numpy's axis-0 reduction
    of a C-contiguous array adds whole rows in row order, which is the reference's order."""
    shape = tuple(shape)
    if tuple(g.shape) == shape:
        return g
    n = int(np.prod(shape)) if shape else 1
    if tuple(g.shape[g.ndim - len(shape):]) != shape:
        raise NotImplementedError(f"sum_to {g.shape} -> {shape}")
    return g.reshape(-1, n).astype(np.float64).sum(axis=0).reshape(shape).astype(np.float32)


def add(a: Tensor, b: Tensor) -> Tensor:
    """Ops.Add (Ops.cs:15-21) with backward EmitSummed (BackwardOps.cs:155-194)."""
    y = (a.data + b.data).astype(np.float32)
    sa, sb = a.data.shape, b.data.shape
    return _attach(y, [a, b], lambda g: [sum_to(g, sa), sum_to(g, sb)])


def sub(a: Tensor, b: Tensor) -> Tensor:
    """Ops.Sub (Ops.cs:24-30): the second gradient is negated (Ops.Neg = multiply by -1)."""
    y = (a.data - b.data).astype(np.float32)
    sa, sb = a.data.shape, b.data.shape
    return _attach(y, [a, b], lambda g: [sum_to(g, sa), (sum_to(g, sb) * np.float32(-1.0)).astype(np.float32)])


def mul(a: Tensor, b: Tensor) -> Tensor:
    """Ops.Mul (Ops.cs:36-56) with backward (BackwardOps.cs:23-38): g*b summed to a, g*a summed to b."""
    av, bv = a.data, b.data
    y = (av * bv).astype(np.float32)
    return _attach(y, [a, b], lambda g: [sum_to((g * bv).astype(np.float32), av.shape) if needs(a) else None,
                                         sum_to((g * av).astype(np.float32), bv.shape) if needs(b) else None])


def relu(x: Tensor) -> Tensor:
    """Ops.Relu (Ops.cs:94-107), backward ReluGradBin (TrainElementwise.cs:41-45)."""
    y = np.empty_like(x.data)
    lib().or_relu_fwd(fp(x.data), fp(y), ctypes.c_int64(y.size))

    def rule(g):
        dx = np.empty_like(g)
        lib().or_relu_bwd(fp(c32(g)), fp(y), fp(dx), ctypes.c_int64(dx.size))
        return [dx]
    return _attach(y, [x], rule)


def gelu(x: Tensor) -> Tensor:
    """Ops.Gelu erf form (Ops.Nn.cs:86-112), backward GeluGradBin (TrainElementwise.cs:59-85)."""
    xv = c32(x.data)
    y = np.empty_like(xv)
    lib().or_gelu_fwd(fp(xv), fp(y), ctypes.c_int64(y.size))

    def rule(g):
        dx = np.empty_like(xv)
        lib().or_gelu_bwd(fp(c32(g)), fp(xv), fp(dx), ctypes.c_int64(dx.size))
        return [dx]
    return _attach(y, [x], rule)


def linear(x: Tensor, w: Tensor, b: Tensor | None) -> Tensor:
    """Ops.Linear (Ops.Layers.cs:715-733) = MatMul(x, W^T) + bias; backward via MatMul/Permute/SumTo
    (BackwardOps.cs:69-82, 107-118, 201-269)."""
    xv = c32(x.data)
    inf, outf = w.data.shape[1], w.data.shape[0]
    if xv.shape[-1] != inf or (b is not None and b.data.shape != (outf,)):
        raise ValueError(f"Linear: input {xv.shape} does not fit weights {w.data.shape}")
    rows = xv.size // inf
    y = np.empty(xv.shape[:-1] + (outf,), np.float32)
    lib().or_linear_fwd(fp(xv), fp(w.data), fp(b.data) if b is not None else None, fp(y), rows, inf, outf)

    def rule(g):
        g = c32(g)
        dx = np.empty_like(xv) if needs(x) else None
        dw = np.empty_like(w.data) if needs(w) else None
        db = np.empty_like(b.data) if (b is not None and needs(b)) else None
        lib().or_linear_bwd(fp(g), fp(xv), fp(w.data), fp(dx) if dx is not None else None,
                            fp(dw) if dw is not None else None, fp(db) if db is not None else None, rows, inf, outf)
        return [dx, dw, db] if b is not None else [dx, dw]
    return _attach(y, [x, w, b] if b is not None else [x, w], rule)


def reshape(x: Tensor, shape) -> Tensor:
    """Reshape view; backward emits g reshaped to the input shape (BackwardOps.cs:120-122)."""
    s0 = x.data.shape
    return _attach(np.ascontiguousarray(x.data.reshape(shape)), [x], lambda g: [g.reshape(s0)])


def permute(x: Tensor, perm) -> Tensor:
    """Permute view; backward is the inverse permutation, cloned (BackwardOps.cs:107-118)."""
    inv = [0] * len(perm)
    for i, p in enumerate(perm):
        inv[p] = i
    return _attach(np.ascontiguousarray(x.data.transpose(perm)), [x],
                   lambda g: [np.ascontiguousarray(g.transpose(inv))])


def sum_all(x: Tensor) -> Tensor:
    """Ops.Sum of all elements (Ops.Nn.cs:162, 218-227): fp64 in element order. Backward broadcasts g."""
    xv = c32(x.data)
    y = np.array([lib().or_sum_all(fp(xv), ctypes.c_int64(xv.size), 0)], np.float32).reshape(())
    return _attach(y, [x], lambda g: [np.full(xv.shape, g.reshape(-1)[0], np.float32)])


def mean_all(x: Tensor) -> Tensor:
    """Ops.Mean of all elements; backward g broadcast then divided by n in float (BackwardNn.cs:145-168)."""
    xv = c32(x.data)
    y = np.array([lib().or_sum_all(fp(xv), ctypes.c_int64(xv.size), 1)], np.float32).reshape(())
    n = np.float32(xv.size)
    return _attach(y, [x], lambda g: [(np.full(xv.shape, g.reshape(-1)[0], np.float32) / n).astype(np.float32)])


def mean_axis(x: Tensor, axis: int) -> Tensor:
    """Ops.Mean over one axis (Ops.Nn.cs:186-231), keepDim false."""
    xv = c32(x.data)
    ax = axis % xv.ndim
    outer = int(np.prod(xv.shape[:ax])) if ax > 0 else 1
    n = xv.shape[ax]
    inner = int(np.prod(xv.shape[ax + 1:])) if ax + 1 < xv.ndim else 1
    oshape = xv.shape[:ax] + xv.shape[ax + 1:]
    y = np.empty(oshape, np.float32)
    lib().or_mean_axis(fp(xv), fp(y), outer, n, inner)

    def rule(g):
        dx = np.empty_like(xv)
        lib().or_mean_axis_bwd(fp(c32(g)), fp(dx), outer, n, inner)
        return [dx]
    return _attach(y, [x], rule)


def softmax(x: Tensor) -> Tensor:
    """Ops.Softmax over the last axis (Ops.Layers.cs:17-39; Softmax.Rows, Softmax.cs:27-133), backward
    BackwardNn.cs:26-52 (dx = y * (g - (float) fp64 sum of g*y), the record saving the output)."""
    xv = c32(x.data)
    cols = xv.shape[-1]
    rows = xv.size // cols
    y = np.empty_like(xv)
    lib().or_softmax_rows(fp(xv), fp(y), rows, cols)

    def rule(g):
        dx = np.empty_like(xv)
        lib().or_softmax_bwd(fp(c32(g)), fp(y), fp(dx), rows, cols)
        return [dx]
    return _attach(y, [x], rule)


def log_softmax(x: Tensor) -> Tensor:
    """Ops.LogSoftmax over the last axis (Ops.Layers.cs:47-96), backward BackwardNn.cs:54-80."""
    xv = c32(x.data)
    cols = xv.shape[-1]
    rows = xv.size // cols
    y = np.empty_like(xv)
    lib().or_logsoftmax_fwd(fp(xv), fp(y), rows, cols)

    def rule(g):
        dx = np.empty_like(xv)
        lib().or_logsoftmax_bwd(fp(c32(g)), fp(y), fp(dx), rows, cols)
        return [dx]
    return _attach(y, [x], rule)


def nll_loss(logp: Tensor, target: np.ndarray, mean=True, ignore=-100) -> Tensor:
    """Ops.NllLoss (Ops.Layers.cs:644-699), backward NllBackward (BackwardNn.cs:602-632)."""
    lv = c32(logp.data)
    rows, cols = lv.shape
    tg = np.ascontiguousarray(target, np.int32)
    bad = ctypes.c_int(0)
    val = lib().or_nll_fwd(fp(lv), ip(tg), rows, cols, int(mean), ignore, ctypes.byref(bad))
    if bad.value >= 0:
        raise IndexError(f"Target {tg[bad.value]} at row {bad.value} is outside {cols} classes.")
    y = np.array(val, np.float32)

    def rule(g):
        dx = np.empty_like(lv)
        lib().or_nll_bwd(ctypes.c_float(float(g.reshape(-1)[0])), ip(tg), fp(dx), rows, cols, int(mean), ignore)
        return [dx]
    return _attach(y, [logp], rule)


def cross_entropy(logits: Tensor, target: np.ndarray) -> Tensor:
    """Losses.CrossEntropy without smoothing (Losses.cs:21-57) = NllLoss(LogSoftmax(logits))."""
    return nll_loss(log_softmax(logits), target)


def mse(pred: Tensor, target: Tensor) -> Tensor:
    """Losses.Mse (Losses.cs:86-91): d = pred - target; Mean(d*d)."""
    d = sub(pred, target)
    return mean_all(mul(d, d))


def layer_norm(x: Tensor, gamma: Tensor, beta: Tensor, eps=1e-5) -> Tensor:
    """Ops.LayerNorm (Ops.Layers.cs:109-141), backward LayerNormBackward (BackwardNn.cs:170-223)."""
    xv = c32(x.data)
    cols = xv.shape[-1]
    rows = xv.size // cols
    y = np.empty_like(xv)
    mean = np.empty(rows, np.float32)
    inv = np.empty(rows, np.float32)
    lib().or_layernorm_fwd(fp(xv), fp(gamma.data), fp(beta.data), fp(y), fp(mean), fp(inv), rows, cols,
                           ctypes.c_float(eps))

    def rule(g):
        dx = np.empty_like(xv)
        dg = np.empty(cols, np.float32)
        db = np.empty(cols, np.float32)
        lib().or_layernorm_bwd(fp(c32(g)), fp(xv), fp(gamma.data), fp(mean), fp(inv), fp(dx), fp(dg), fp(db), rows,
                               cols)
        return [dx, dg, db]
    return _attach(y, [x, gamma, beta], rule)


def attention(q: Tensor, k: Tensor, v: Tensor, mask: np.ndarray | None, scale: float = 0.0) -> Tensor:
    """Ops.Attention (Ops.Layers.cs:746-807), backward AttentionBackward (BackwardNn.cs:636-701). q,k,v [B,H,L,D];
    mask [Lq,Lk] or [B,Lq,Lk] additive, no gradient."""
    qv, kv, vv = c32(q.data), c32(k.data), c32(v.data)
    B, H, lq, d = qv.shape
    lk = kv.shape[2]
    if scale == 0.0 or math.isnan(scale):
        scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    mv = c32(mask) if mask is not None else None
    mb = 1 if (mv is not None and mv.ndim == 3) else 0
    out = np.empty_like(qv)
    lib().or_attention_fwd(fp(qv), fp(kv), fp(vv), fp(mv) if mv is not None else None, mb, fp(out), B, H, lq, lk, d,
                           ctypes.c_float(scale))

    def rule(g):
        dq, dk, dv = np.empty_like(qv), np.empty_like(kv), np.empty_like(vv)
        lib().or_attention_bwd(fp(qv), fp(kv), fp(vv), fp(mv) if mv is not None else None, mb, fp(c32(g)), fp(dq),
                               fp(dk), fp(dv), B, H, lq, lk, d, ctypes.c_float(scale))
        return [dq, dk, dv]
    return _attach(out, [q, k, v], rule)


def conv2d(x: Tensor, w: Tensor, b: Tensor | None, stride=1, pad=0) -> Tensor:
    """Ops.Conv2d, groups 1 (Ops.Layers.cs:279-336), backward ConvBackward (BackwardNn.cs:317-402)."""
    xv = c32(x.data)
    N, Cin, H, W = xv.shape
    Cout, _, KH, KW = w.data.shape
    OH, OW = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    y = np.empty((N, Cout, OH, OW), np.float32)
    lib().or_conv2d_fwd(fp(xv), fp(w.data), fp(b.data) if b is not None else None, fp(y), N, Cin, H, W, Cout, KH, KW,
                        stride, pad)

    def rule(g):
        g = c32(g)
        dx = np.empty_like(xv) if needs(x) else None
        dw = np.empty_like(w.data) if needs(w) else None
        db = np.empty(Cout, np.float32) if (b is not None and needs(b)) else None
        lib().or_conv2d_bwd(fp(g), fp(xv), fp(w.data), fp(dx) if dx is not None else None,
                            fp(dw) if dw is not None else None, fp(db) if db is not None else None, N, Cin, H, W, Cout,
                            KH, KW, stride, pad)
        return [dx, dw, db] if b is not None else [dx, dw]
    return _attach(y, [x, w, b] if b is not None else [x, w], rule)


def max_pool2d(x: Tensor, kh, kw, sh=None, sw=None, ph=0, pw=0):
    """Ops.MaxPool2d (Ops.cs:151-178; TensorKernels.cs:242-296); backward scatters to the saved Int32 index
    (BackwardOps.cs:285-298). Returns (tensor, indices)."""
    sh = kh if sh is None else sh
    sw = kw if sw is None else sw
    xv = c32(x.data)
    N, C, H, W = xv.shape
    OH, OW = (H + 2 * ph - kh) // sh + 1, (W + 2 * pw - kw) // sw + 1
    y = np.empty((N, C, OH, OW), np.float32)
    idx = np.empty((N, C, OH, OW), np.int32)
    lib().or_maxpool_fwd(fp(xv), fp(y), ip(idx), N, C, H, W, kh, kw, sh, sw, ph, pw)

    def rule(g):
        dx = np.empty_like(xv)
        lib().or_maxpool_bwd(fp(c32(g)), ip(idx), fp(dx), ctypes.c_int64(idx.size), ctypes.c_int64(xv.size))
        return [dx]
    return _attach(y, [x], rule), idx


def avg_pool2d(x: Tensor, k, s=None, p=0, count_include_pad=True) -> Tensor:
    """Ops.AvgPool2d (Ops.Layers.cs:412-455), backward AvgPoolBackward (BackwardNn.cs:464-492)."""
    s = k if s is None else s
    xv = c32(x.data)
    N, C, H, W = xv.shape
    OH, OW = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    y = np.empty((N, C, OH, OW), np.float32)
    lib().or_avgpool_fwd(fp(xv), fp(y), N * C, H, W, k, k, s, s, p, p, int(count_include_pad))

    def rule(g):
        dx = np.empty_like(xv)
        lib().or_avgpool_bwd(fp(c32(g)), fp(dx), N * C, H, W, k, k, s, s, p, p, int(count_include_pad))
        return [dx]
    return _attach(y, [x], rule)


def batch_norm2d(x: Tensor, gamma: Tensor, beta: Tensor, rm: np.ndarray, rv: np.ndarray, momentum=0.1, eps=1e-5):
    """Ops.BatchNorm2d training mode (Ops.Layers.cs:158-264), backward BatchNormBackward (BackwardNn.cs:244-307).
    rm/rv are updated in place."""
    xv = c32(x.data)
    N, C, H, W = xv.shape
    y = np.empty_like(xv)
    mean = np.empty(C, np.float32)
    inv = np.empty(C, np.float32)
    lib().or_batchnorm_fwd(fp(xv), fp(gamma.data), fp(beta.data), fp(rm), fp(rv), fp(y), fp(mean), fp(inv), N, C,
                           H * W, ctypes.c_float(momentum), ctypes.c_float(eps))

    def rule(g):
        dx = np.empty_like(xv)
        dg = np.empty(C, np.float32)
        db = np.empty(C, np.float32)
        lib().or_batchnorm_bwd(fp(c32(g)), fp(xv), fp(gamma.data), fp(mean), fp(inv), fp(dx), fp(dg), fp(db), N, C,
                               H * W)
        return [dx, dg, db]
    return _attach(y, [x, gamma, beta], rule)


def embedding(table: Tensor, ids: np.ndarray, pad=-1) -> Tensor:
    """Ops.Embedding dense (Ops.Layers.cs:549), backward EmbeddingBackward dense branch (BackwardNn.cs:521-540)."""
    iv = np.ascontiguousarray(ids, np.int32)
    rows, dim = table.data.shape
    y = np.empty(iv.shape + (dim,), np.float32)
    lib().or_embedding_fwd(fp(table.data), ip(iv), fp(y), iv.size, dim)

    def rule(g):
        dt = np.empty_like(table.data)
        lib().or_embedding_bwd(fp(c32(g)), ip(iv), fp(dt), iv.size, dim, rows, pad)
        return [dt]
    return _attach(y, [table], rule)


def dropout(x: Tensor, p: float, seed: int, draw: int) -> Tensor:
    """Dropout.Forward in training mode (Layers.cs:341-368) as Ops.Mul(x, mask), backward g * mask; the caller keeps
    the module's draw counter. p == 0 returns x itself, as the reference does."""
    if p == 0.0:
        return x
    xv = c32(x.data)
    y = np.empty_like(xv)
    lib().or_dropout(fp(xv), fp(y), ctypes.c_int64(xv.size), ctypes.c_float(p), ctypes.c_uint64(seed),
                     ctypes.c_int64(draw))

    def rule(g):
        dx = np.empty_like(xv)
        lib().or_dropout(fp(c32(g)), fp(dx), ctypes.c_int64(xv.size), ctypes.c_float(p), ctypes.c_uint64(seed),
                         ctypes.c_int64(draw))
        return [dx]
    return _attach(y, [x], rule)


CTC_NONE, CTC_MEAN, CTC_SUM = 0, 1, 2


def ctc_loss(lp: Tensor, targets, in_len, tgt_len, blank=0, reduction=CTC_MEAN, zero_inf=False) -> Tensor:
    """Ops.CtcLoss (CtcLoss.cs:40-153), backward CtcBackward (BackwardRecurrent.cs:253-296)."""
    lv = c32(lp.data)
    T, B, C = lv.shape
    tg = np.ascontiguousarray(targets, np.int32)
    il = np.ascontiguousarray(in_len, np.int32)
    tl = np.ascontiguousarray(tgt_len, np.int32)
    out = np.empty(B if reduction == CTC_NONE else 1, np.float32)
    lib().or_ctc_loss(fp(lv), ip(tg), ip(il), ip(tl), T, B, C, blank, reduction, int(zero_inf), fp(out))
    y = out if reduction == CTC_NONE else out.reshape(())

    def rule(g):
        d = np.empty_like(lv)
        gg = c32(np.asarray(g).reshape(-1))
        lib().or_ctc_grad(fp(lv), ip(tg), ip(il), ip(tl), fp(gg), T, B, C, blank, reduction, fp(d))
        return [d]
    return _attach(y, [lp], rule)


# ----------------------------------------------------------------------------------------------------------- optimizers
class AdamW:
    """Adam/AdamW (Optimizers.cs:374-608): BeginStep computes step size and sqrt(bc2) in double (IntPow), then the
    IEEE per-element update (UpdateRange, Optimizers.cs:554-589) over parameters in list order."""

    def __init__(self, params, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, wd=0.01, decoupled=True, amsgrad=False):
        self.params = list(params)
        self.lr, self.b1, self.b2, self.eps, self.wd = lr, beta1, beta2, eps, wd
        self.decoupled, self.amsgrad = decoupled, amsgrad
        self.m = [np.zeros_like(p.data) for p in self.params]
        self.v = [np.zeros_like(p.data) for p in self.params]
        self.vmax = [np.zeros_like(p.data) for p in self.params] if amsgrad else None
        self.step_count = 0

    def scalars(self):
        ss, sq = ctypes.c_float(), ctypes.c_float()
        lib().or_adam_scalars(ctypes.c_float(self.lr), ctypes.c_float(self.b1), ctypes.c_float(self.b2),
                              ctypes.c_int64(self.step_count + 1), ctypes.byref(ss), ctypes.byref(sq))
        return ss.value, sq.value

    def step(self):
        ss, sq = self.scalars()
        for i, p in enumerate(self.params):
            if not p.requires_grad or p.grad is None:
                continue
            lib().or_adam_update(fp(p.data), fp(c32(p.grad)), fp(self.m[i]), fp(self.v[i]),
                                 fp(self.vmax[i]) if self.vmax is not None else None, ctypes.c_int64(p.data.size),
                                 ctypes.c_float(self.lr), ctypes.c_float(self.b1), ctypes.c_float(self.b2),
                                 ctypes.c_float(self.eps), ctypes.c_float(self.wd), int(self.decoupled),
                                 ctypes.c_float(ss), ctypes.c_float(sq))
        self.step_count += 1

    def zero_grad(self):
        zero_grad(self.params)


class Sgd:
    """Sgd (Optimizers.cs, class Sgd): momentum buffers start from the first gradient."""

    def __init__(self, params, lr, momentum=0.0, dampening=0.0, wd=0.0, nesterov=False):
        self.params = list(params)
        self.lr, self.mu, self.damp, self.wd, self.nesterov = lr, momentum, dampening, wd, nesterov
        self.buf = [np.zeros_like(p.data) for p in self.params] if momentum != 0.0 else None
        self.init = [False] * len(self.params)
        self.step_count = 0

    def step(self):
        for i, p in enumerate(self.params):
            if not p.requires_grad or p.grad is None:
                continue
            first = not self.init[i]
            self.init[i] = True
            lib().or_sgd_update(fp(p.data), fp(c32(p.grad)), fp(self.buf[i]) if self.buf is not None else None,
                                ctypes.c_int64(p.data.size), ctypes.c_float(self.lr), ctypes.c_float(self.mu),
                                ctypes.c_float(self.damp), ctypes.c_float(self.wd), int(self.nesterov), int(first))
        self.step_count += 1

    def zero_grad(self):
        zero_grad(self.params)


# ----------------------------------------------------------------------------------------------------- gradient clipping
def _grad_table(params):
    """Pointer and length tables over the gradients of `params` (a parameter without one gets a NULL entry, which
    the clip functions skip, as GradClip does). Gradients are made float32 C-contiguous in place first."""
    ptrs, lens = (F32P * len(params))(), (ctypes.c_int64 * len(params))()
    for i, p in enumerate(params):
        if p.grad is None:
            lens[i] = 0
            continue
        p.grad = c32(p.grad)
        ptrs[i] = fp(p.grad)
        lens[i] = p.grad.size
    return ptrs, lens


def clip_grad_norm(params, max_norm, infinity_norm=False):
    """GradClip.ClipNorm (Schedules.cs:22-100) in place over the parameters' gradients; returns (norm as float32,
    coefficient: the scale applied when below 1, or 1 for a non-finite norm)."""
    if not max_norm > 0:
        raise ValueError("the maximum norm must be positive")
    params = list(params)
    ptrs, lens = _grad_table(params)
    coef = ctypes.c_float()
    total = lib().or_clip_norm(ptrs, lens, len(params), ctypes.c_float(max_norm), int(infinity_norm),
                               ctypes.byref(coef))
    return np.float32(total), np.float32(coef.value)


def clip_grad_value(params, clip_value):
    """GradClip.ClipValue (Schedules.cs:119-149) in place."""
    if not clip_value >= 0:
        raise ValueError("the bound must not be negative")
    params = list(params)
    ptrs, lens = _grad_table(params)
    lib().or_clip_value(ptrs, lens, len(params), ctypes.c_float(clip_value))
