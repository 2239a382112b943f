"""TEST INFRASTRUCTURE ONLY: the reference's modules and the benchmark configurations, on the CPU oracle tape.

Modules restate src/OneModel.Training/Layers.cs (registration order = parameter order, NnModule.cs:139-165, 289-311;
initial values from the SplitMix64 Generator, Layers.cs:11-21, 41-116). The configurations C1..C5 are the workloads of
the benchmark (one fwd+bwd+AdamW training step each); their synthetic inputs come from the same generator with
seed 20261201 + 100*config + tensor index. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline import
this file.
"""
from __future__ import annotations

import numpy as np

from . import tape as T

SEED = 20261201


def cfg_seed(cfg: int, index: int) -> int:
    return SEED + 100 * cfg + index


# ----------------------------------------------------------------------------------------------------------- modules
class Module:
    def __init__(self):
        self._params: list[tuple[str, T.Tensor]] = []
        self._children: list[tuple[str, Module]] = []

    def param(self, name, data):
        t = T.Tensor(np.ascontiguousarray(data, np.float32), requires_grad=True, name=name)
        self._params.append((name, t))
        return t

    def child(self, name, m):
        self._children.append((name, m))
        return m

    def named_parameters(self, prefix=""):
        """NnModule.NamedParameters (NnModule.cs:139-165): own parameters in registration order, then children."""
        out = [(prefix + n, t) for n, t in self._params]
        for cn, c in self._children:
            out += c.named_parameters(prefix + cn + ".")
        return out

    def parameters(self):
        return [t for _, t in self.named_parameters()]


class Linear(Module):
    """Linear (Layers.cs:41-70): weight [out,in] then bias [out], both U(-1/sqrt(in), 1/sqrt(in))."""

    def __init__(self, inf, outf, g: T.Generator, bias=True):
        super().__init__()
        b = T.fan_in_bound(inf)
        self.weight = self.param("weight", g.uniform(-b, b, (outf, inf)))
        self.bias = self.param("bias", g.uniform(-b, b, (outf,))) if bias else None

    def __call__(self, x):
        return T.linear(x, self.weight, self.bias)


class Conv2d(Module):
    """Conv2d (Layers.cs:73-116), groups 1: bound 1/sqrt(in*k*k), weight then bias."""

    def __init__(self, cin, cout, k, g: T.Generator, padding=0, stride=1):
        super().__init__()
        b = T.fan_in_bound(cin * k * k)
        self.pad, self.stride = padding, stride
        self.weight = self.param("weight", g.uniform(-b, b, (cout, cin, k, k)))
        self.bias = self.param("bias", g.uniform(-b, b, (cout,)))

    def __call__(self, x):
        return T.conv2d(x, self.weight, self.bias, self.stride, self.pad)


class LayerNorm(Module):
    """LayerNorm (Layers.cs:241-265): gamma = 1, beta = 0, eps 1e-5."""

    def __init__(self, n, eps=1e-5):
        super().__init__()
        self.eps = eps
        self.weight = self.param("weight", np.ones(n, np.float32))
        self.bias = self.param("bias", np.zeros(n, np.float32))

    def __call__(self, x):
        return T.layer_norm(x, self.weight, self.bias, self.eps)


class MultiHeadAttention(Module):
    """MultiHeadAttention (Layers.cs:459-517): q, k, v, o Linear(width, width); heads split by reshape/permute."""

    def __init__(self, width, heads, g):
        super().__init__()
        self.heads = heads
        self.q = self.child("q", Linear(width, width, g))
        self.k = self.child("k", Linear(width, width, g))
        self.v = self.child("v", Linear(width, width, g))
        self.o = self.child("o", Linear(width, width, g))

    def __call__(self, x, mask=None):
        b, n, d = x.shape
        dh = d // self.heads

        def split(z):
            return T.permute(T.reshape(z, (b, n, self.heads, dh)), (0, 2, 1, 3))
        a = T.attention(split(self.q(x)), split(self.k(x)), split(self.v(x)), mask)
        return self.o(T.reshape(T.permute(a, (0, 2, 1, 3)), (b, n, d)))


class TransformerEncoderLayer(Module):
    """Post-norm TransformerEncoderLayer (Layers.cs:523-578): x1 = LN(x + Attn(x)); y = LN(x1 + FF2(GELU(FF1 x1)))."""

    def __init__(self, width, heads, ff, g):
        super().__init__()
        self.attn = self.child("attn", MultiHeadAttention(width, heads, g))
        self.norm1 = self.child("norm1", LayerNorm(width))
        self.ff1 = self.child("ff1", Linear(width, ff, g))
        self.ff2 = self.child("ff2", Linear(ff, width, g))
        self.norm2 = self.child("norm2", LayerNorm(width))

    def __call__(self, x, mask=None):
        x1 = self.norm1(T.add(x, self.attn(x, mask)))
        return self.norm2(T.add(x1, self.ff2(T.gelu(self.ff1(x1)))))


class PreNormEncoderBlock(Module):
    """The C3 block, composed from the reference's pieces (it has no pre-norm module): children ln1, attn, ln2, ff1,
    ff2; h = x + Attn(LN1 x); y = h + FF2(GELU(FF1(LN2 h)))."""

    def __init__(self, width, heads, ff, g):
        super().__init__()
        self.ln1 = self.child("ln1", LayerNorm(width))
        self.attn = self.child("attn", MultiHeadAttention(width, heads, g))
        self.ln2 = self.child("ln2", LayerNorm(width))
        self.ff1 = self.child("ff1", Linear(width, ff, g))
        self.ff2 = self.child("ff2", Linear(ff, width, g))

    def __call__(self, x, mask=None):
        h = T.add(x, self.attn(self.ln1(x), mask))
        return T.add(h, self.ff2(T.gelu(self.ff1(self.ln2(h)))))


# ----------------------------------------------------------------------------------------------------------- configs
class Config:
    """One benchmark configuration: model, inputs, loss, AdamW(lr 1e-3, wd 0.01)."""

    def __init__(self, cfg, model, loss_fn, inputs):
        self.cfg, self.model, self.loss_fn, self.inputs = cfg, model, loss_fn, inputs
        self.params = model.parameters()
        self.leaves = list(self.params) + [t for t in inputs.values() if isinstance(t, T.Tensor) and t.requires_grad]
        self.opt = T.AdamW(self.params, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, wd=0.01)

    def step(self) -> float:
        """ZeroGrad, forward, backward, AdamW step (TrainCase.cs step shape); returns the loss."""
        T.zero_grad(self.leaves)
        loss = self.loss_fn(self)
        T.backward(loss)
        self.opt.step()
        return float(loss.data.reshape(-1)[0])


def padding_mask(lengths, L):
    """Additive mask [B, L, L]: 0 for keys < len_b, -inf for the rest."""
    B = len(lengths)
    m = np.zeros((B, L, L), np.float32)
    for b, n in enumerate(lengths):
        m[b, :, n:] = -np.inf
    return m


def make_config(cfg: int, scale: dict | None = None) -> Config:
    """Builds config `cfg` (1..5, or 10: a Linear applied twice). `scale` shrinks sizes for fast parity tests (keys: batch, seq, layers, hw)."""
    s = scale or {}
    g = T.Generator(cfg_seed(cfg, 0))
    if cfg == 1:
        B = s.get("batch", 64)
        model = Module()
        l1 = model.child("0", Linear(784, 256, g))
        l2 = model.child("2", Linear(256, 10, g))
        x = T.Tensor(T.Generator(cfg_seed(1, 1)).normal((B, 784)))
        y = T.Generator(cfg_seed(1, 2)).ints(0, 10, (B,))

        def loss(c):
            return T.cross_entropy(l2(T.relu(l1(x))), y)
        return Config(1, model, loss, {"x": x, "labels": y})
    if cfg == 2:
        B, HW = s.get("batch", 32), s.get("hw", 56)
        model = Module()
        conv = model.child("0", Conv2d(64, 64, 3, g, padding=1))
        fc = model.child("4", Linear(64, 10, g))
        x = T.Tensor(T.Generator(cfg_seed(2, 1)).normal((B, 64, HW, HW)), requires_grad=True)
        y = T.Generator(cfg_seed(2, 2)).ints(0, 10, (B,))

        def loss(c):
            h = T.relu(conv(x))
            n, ch = h.shape[0], h.shape[1]
            gap = T.reshape(T.mean_axis(T.reshape(h, (n, ch, -1)), 2), (n, ch, 1, 1))
            return T.cross_entropy(fc(T.reshape(gap, (n, ch))), y)
        return Config(2, model, loss, {"x": x, "labels": y})
    if cfg == 3:
        B, L = s.get("batch", 32), s.get("seq", 128)
        D, H, F = 384, 12, 1536
        model = PreNormEncoderBlock(D, H, F, g)
        x = T.Tensor(T.Generator(cfg_seed(3, 1)).normal((B, L, D)))
        tgt = T.Tensor(T.Generator(cfg_seed(3, 2)).normal((B, L, D)))
        lo = min(64, L)
        lengths = T.Generator(cfg_seed(3, 3)).ints(lo, L + 1, (B,))
        mask = padding_mask(lengths, L)

        def loss(c):
            return T.mse(model(x, mask), tgt)
        return Config(3, model, loss, {"x": x, "target": tgt, "lengths": lengths, "mask": mask})
    if cfg == 4:
        B = s.get("batch", 32)
        model = Module()
        chans = [1, 32, 64, 128, 256]
        convs = [model.child(str(3 * i), Conv2d(chans[i], chans[i + 1], 3, g, padding=1)) for i in range(4)]
        head = model.child("out", Linear(256, 37, g))
        x = T.Tensor(T.Generator(cfg_seed(4, 1)).uniform(0.0, 1.0, (B, 1, 32, 128)))
        tl = T.Generator(cfg_seed(4, 2)).ints(1, 11, (B,))
        labels = T.Generator(cfg_seed(4, 3)).ints(1, 37, (int(tl.sum()),))
        il = np.full(B, 32, np.int32)
        pools = [(2, 2), (2, 2), (2, 1), (2, 1)]

        def loss(c):
            h = x
            for conv, (ph, pw) in zip(convs, pools):
                h, _ = T.max_pool2d(T.relu(conv(h)), ph, pw)
            f = T.mean_axis(h, 2)                      # [B, 256, T]
            seq = T.permute(f, (2, 0, 1))               # [T, B, 256]
            lp = T.log_softmax(head(seq))               # [T, B, 37]
            return T.ctc_loss(lp, labels, il, tl, 0, T.CTC_MEAN)
        return Config(4, model, loss, {"x": x, "labels": labels, "in_len": il, "tgt_len": tl})
    if cfg == 5:
        B, L, NL = s.get("batch", 8), s.get("seq", 512), s.get("layers", 4)
        D, H, F = 768, 12, 3072
        model = Module()
        layers = [model.child(f"layer{i}", TransformerEncoderLayer(D, H, F, g)) for i in range(NL)]
        head = model.child("head", Linear(D, 9, g))
        x = T.Tensor(T.Generator(cfg_seed(5, 1)).normal((B, L, D)))
        y = T.Generator(cfg_seed(5, 2)).ints(0, 9, (B * L,))

        def loss(c):
            h = x
            for layer in layers:
                h = layer(h)
            return T.cross_entropy(T.reshape(head(h), (B * L, 9)), y)
        return Config(5, model, loss, {"x": x, "labels": y})
    if cfg == 10:  # one Linear applied twice: its gradient sums both uses (BackwardEngineTests.cs:13-25)
        B = s.get("batch", 256)
        model = Module()
        l1 = model.child("0", Linear(64, 128, g))
        t = model.child("1", Linear(128, 128, g))
        l2 = model.child("2", Linear(128, 64, g))
        x = T.Tensor(T.Generator(cfg_seed(10, 1)).normal((B, 64)))
        y = T.Generator(cfg_seed(10, 2)).ints(0, 64, (B,))

        def loss(c):
            h = T.relu(l1(x))
            return T.cross_entropy(l2(T.relu(t(T.relu(t(h))))), y)
        return Config(10, model, loss, {"x": x, "labels": y})
    raise ValueError(cfg)


# ----------------------------------------------------------------------------------------------------------- fixtures
def encoder_fixture(o):
    """EncoderModel of tests/OneModel.Tests/Tensors/AutogradModels.cs:133-199 over a loaded fixture `o` (dict name ->
    array). Returns (loss, grads by parameter name)."""
    D, Hh, NL, B, N = 16, 2, 2, 2, 5
    params = {k[3:]: T.Tensor(o[k].copy(), requires_grad=True) for k in o
              if k.startswith("in.") and k not in ("in.ids", "in.mask", "in.proj")}
    ids = o["in.ids"].astype(np.int32)
    mask, proj = o["in.mask"], T.Tensor(o["in.proj"])

    def split(z):
        return T.permute(T.reshape(z, (B, N, Hh, D // Hh)), (0, 2, 1, 3))
    x = T.embedding(params["emb"], ids)
    for i in range(NL):
        p = f"l{i}."
        P = params
        q = split(T.linear(x, P[p + "wq"], P[p + "bq"]))
        k = split(T.linear(x, P[p + "wk"], P[p + "bk"]))
        v = split(T.linear(x, P[p + "wv"], P[p + "bv"]))
        a = T.reshape(T.permute(T.attention(q, k, v, mask), (0, 2, 1, 3)), (B, N, D))
        x1 = T.layer_norm(T.add(x, T.linear(a, P[p + "wo"], P[p + "bo"])), P[p + "ln1g"], P[p + "ln1b"])
        f = T.linear(T.gelu(T.linear(x1, P[p + "w1"], P[p + "b1"])), P[p + "w2"], P[p + "b2"])
        x = T.layer_norm(T.add(x1, f), P[p + "ln2g"], P[p + "ln2b"])
    loss = T.sum_all(T.mul(x, proj))
    T.backward(loss)
    return float(loss.data), {k: v.grad for k, v in params.items()}, x.data


def cnn_fixture(o):
    """CnnModel of AutogradModels.cs:88-131. Returns (loss, grads, running stats)."""
    names = ["c1w", "c1b", "bn1g", "bn1b", "c2w", "c2b", "bn2g", "bn2b", "fcw", "fcb"]
    P = {n: T.Tensor(o["in." + n].copy(), requires_grad=True) for n in names}
    X = T.Tensor(o["in.x"].copy(), requires_grad=True)
    P["x"] = X
    tg = o["in.targets"].astype(np.int32)
    rm1, rv1 = np.zeros(4, np.float32), np.ones(4, np.float32)
    rm2, rv2 = np.zeros(8, np.float32), np.ones(8, np.float32)
    h = T.conv2d(X, P["c1w"], P["c1b"], 1, 1)
    h = T.batch_norm2d(h, P["bn1g"], P["bn1b"], rm1, rv1)
    h, _ = T.max_pool2d(T.relu(h), 2, 2)
    h = T.conv2d(h, P["c2w"], P["c2b"], 1, 1)
    h = T.batch_norm2d(h, P["bn2g"], P["bn2b"], rm2, rv2)
    h = T.avg_pool2d(T.relu(h), 2)
    logits = T.linear(T.reshape(h, (4, 72)), P["fcw"], P["fcb"])
    loss = T.nll_loss(T.log_softmax(logits), tg)
    T.backward(loss)
    return float(loss.data), {k: v.grad for k, v in P.items()}, {"rm1": rm1, "rv1": rv1, "rm2": rm2, "rv2": rv2}


def mlp_curve(o, steps=None):
    """TrainCase.Mlp (tests/OneModel.Tests/Training/TrainCase.cs:114-143): Linear(20,32)-ReLU-Linear(32,4), CE,
    SGD(lr 0.05, momentum 0.9, wd 1e-4), batches by the fixture's order rows. Returns (losses, final params)."""
    P = {k: T.Tensor(o["in." + k].copy(), requires_grad=True) for k in ("w1", "b1", "w2", "b2")}
    opt = T.Sgd([P["w1"], P["b1"], P["w2"], P["b2"]], 0.05, momentum=0.9, wd=1e-4)
    x, y, order = o["in.x"], o["in.y"], o["in.order"].astype(np.int64)
    n = order.shape[0] if steps is None else steps
    losses = []
    for i in range(n):
        idx = order[i]
        xb = T.Tensor(np.ascontiguousarray(x[idx]))
        yb = y[idx].astype(np.int32)
        loss = T.cross_entropy(T.linear(T.relu(T.linear(xb, P["w1"], P["b1"])), P["w2"], P["b2"]), yb)
        losses.append(float(loss.data))
        opt.zero_grad()
        T.backward(loss)
        opt.step()
    return np.array(losses, np.float32), {k: v.data for k, v in P.items()}


# ----------------------------------------------------------------------------------------------------------- curves
class BatchNorm2d(Module):
    """BatchNorm2d (Layers.cs:202-238): weight 1, bias 0, running mean 0 / variance 1 (buffers), momentum 0.1,
    eps 1e-5, training mode."""

    def __init__(self, c):
        super().__init__()
        self.weight = self.param("weight", np.ones(c, np.float32))
        self.bias = self.param("bias", np.zeros(c, np.float32))
        self.running_mean = np.zeros(c, np.float32)
        self.running_var = np.ones(c, np.float32)

    def __call__(self, x):
        return T.batch_norm2d(x, self.weight, self.bias, self.running_mean, self.running_var)


class Seq(Module):
    """Sequential (Layers.cs:581-640): children named by position; entries without parameters are plain callables."""

    def __init__(self, *layers):
        super().__init__()
        self.layers = layers
        for i, l in enumerate(layers):
            if isinstance(l, Module):
                self.child(str(i), l)

    def __call__(self, x):
        for l in self.layers:
            x = l(x)
        return x


class EncoderClassifier(Module):
    """The encoder classifier of the reference's training-curve test (TrainCase.cs:9-38): Embedding, post-norm
    encoder layers, mean over the sequence, Linear head."""

    def __init__(self, vocab, width, heads, ff, layers, classes, g):
        super().__init__()
        b = 1.7320508
        self.emb = self.param("emb.weight", g.uniform(-b, b, (vocab, width)))
        self.layers = [self.child(f"layer{i}", TransformerEncoderLayer(width, heads, ff, g)) for i in range(layers)]
        self.cls = self.child("cls", Linear(width, classes, g))

    def __call__(self, ids):
        x = T.embedding(self.emb, ids)
        for l in self.layers:
            x = l(x)
        return self.cls(T.mean_axis(x, 1))


def _load(model, o, mapping):
    named = dict(model.named_parameters())
    for p, k in mapping:
        named[p].data[...] = o["in." + k].reshape(named[p].data.shape)


CNN_MAP = [("0.weight", "c1w"), ("0.bias", "c1b"), ("1.weight", "bn1g"), ("1.bias", "bn1b"), ("4.weight", "c2w"),
           ("4.bias", "c2b"), ("5.weight", "bn2g"), ("5.bias", "bn2b"), ("9.weight", "fcw"), ("9.bias", "fcb")]


def encoder_map(layers=2):
    m = [("emb.weight", "emb")]
    for i in range(layers):
        for q in "qkvo":
            m += [(f"layer{i}.attn.{q}.weight", f"l{i}.w{q}"), (f"layer{i}.attn.{q}.bias", f"l{i}.b{q}")]
        m += [(f"layer{i}.norm1.weight", f"l{i}.ln1g"), (f"layer{i}.norm1.bias", f"l{i}.ln1b"),
              (f"layer{i}.ff1.weight", f"l{i}.w1"), (f"layer{i}.ff1.bias", f"l{i}.b1"),
              (f"layer{i}.ff2.weight", f"l{i}.w2"), (f"layer{i}.ff2.bias", f"l{i}.b2"),
              (f"layer{i}.norm2.weight", f"l{i}.ln2g"), (f"layer{i}.norm2.bias", f"l{i}.ln2b")]
    return m + [("cls.weight", "clsw"), ("cls.bias", "clsb")]


def cnn_curve(o, steps=None):
    """TrainCase.Cnn (TrainCase.cs:145-183): conv-BN-ReLU-maxpool-conv-BN-ReLU-avgpool-flatten-linear, CE,
    AdamW(3e-3, wd 0.01) with CosineLr(3e-3, steps) applied before each step and ClipNorm(0.5) after each backward.
    Returns (losses, gradient norms, final parameters by name, running statistics)."""
    from . import schedules as S
    g = T.Generator(2)
    bn1, bn2 = BatchNorm2d(4), BatchNorm2d(8)
    model = Seq(Conv2d(1, 4, 3, g, padding=1), bn1, T.relu, lambda x: T.max_pool2d(x, 2, 2)[0],
                Conv2d(4, 8, 3, g, padding=1), bn2, T.relu, lambda x: T.avg_pool2d(x, 2),
                lambda x: T.reshape(x, (x.shape[0], -1)), Linear(72, 5, g))
    _load(model, o, CNN_MAP)
    n = o["in.order"].shape[0] if steps is None else steps
    params = model.parameters()
    opt = T.AdamW(params, lr=3e-3, wd=0.01)
    sched = S.Cosine(3e-3, o["in.order"].shape[0])
    x, y, order = o["in.x"], o["in.y"], o["in.order"].astype(np.int64)
    losses, norms = [], []
    for i in range(n):
        idx = order[i]
        loss = T.cross_entropy(model(T.Tensor(np.ascontiguousarray(x[idx]))), y[idx].astype(np.int32))
        losses.append(float(loss.data))
        T.zero_grad(params)
        T.backward(loss)
        norms.append(float(T.clip_grad_norm(params, 0.5)[0]))
        opt.lr = float(sched.lr_at(opt.step_count))
        opt.step()
    stats = {"rm1": bn1.running_mean, "rv1": bn1.running_var, "rm2": bn2.running_mean, "rv2": bn2.running_var}
    return (np.array(losses, np.float32), np.array(norms, np.float32),
            {k: t.data for k, t in model.named_parameters()}, stats)


def encoder_curve(o, steps=None):
    """TrainCase.Encoder (TrainCase.cs:185-237): EncoderClassifier(vocab 11, width 16, heads 2, ff 32, 2 layers,
    2 classes), CE, Adam(2e-3) with WarmupLr(ConstantLr(2e-3), 10, 0.1) applied before each step. Returns (losses,
    final parameters by name)."""
    from . import schedules as S
    model = EncoderClassifier(11, 16, 2, 32, 2, 2, T.Generator(3))
    _load(model, o, encoder_map())
    params = model.parameters()
    opt = T.AdamW(params, lr=2e-3, wd=0.0, decoupled=False)
    sched = S.Warmup(S.Constant(2e-3), 10, 0.1)
    ids, y, order = o["in.ids"].astype(np.int32), o["in.y"], o["in.order"].astype(np.int64)
    n = order.shape[0] if steps is None else steps
    losses = []
    for i in range(n):
        idx = order[i]
        loss = T.cross_entropy(model(np.ascontiguousarray(ids[idx])), y[idx].astype(np.int32))
        losses.append(float(loss.data))
        T.zero_grad(params)
        T.backward(loss)
        opt.lr = float(sched.lr_at(opt.step_count))
        opt.step()
    return np.array(losses, np.float32), {k: t.data for k, t in model.named_parameters()}
