"""Benchmark: training steps per second of one fwd+bwd+AdamW step of the MiniLM-shaped pre-LN encoder block (C3:
hidden 384, 12 heads of 32, FFN 1536 GELU, seq 128, batch 32, padding mask, MSE, AdamW) on one MI355X, through the
C++ tape (lib/libom_train.so) and the gfx950 kernels (lib/libom_hip.so).

A step is ZeroGrad + forward + loss.Backward() + optimizer.Step() + loss readback, on inputs already resident in HBM.
Prints one JSON line with the throughput, the roofline of the dominant kernel (timed live inside 50 training steps
with a HIP event pair around the launch on the library's stream; also alone on cold operands) and the CPU baseline
(the oracle's C restatement of the reference CPU path, timed on this host's cores on a bounded sample of the same
workload).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--config 3] [--cpu-seconds S] [--no-cpu] [--no-kernels]
    python bench.py --pmc-probe     # the launches the FETCH_SIZE / WRITE_SIZE counter runs read
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "train steps/sec (fwd+bwd+AdamW) at 1 GPU; bwd MFMA util % and HBM GB/s"
FP32_MFMA_PEAK = 157.3  # TFLOP/s, MI355X dense fp32 matrix
HBM_PEAK = 8000.0       # GB/s

WORKLOADS = {
    1: ("C1: MLP 784-256-10, batch 64, CE, AdamW", 64, 0),
    2: ("C2: Conv2d 3x3 64->64 on 32x64x56x56, ReLU, GAP, Linear 64->10, CE, AdamW", 32, 0),
    3: ("C3: MiniLM-shaped pre-LN encoder block, hidden 384, 12 heads (d=32), FFN 1536 GELU, seq 128, batch 32, "
        "padding mask, MSE, AdamW", 32, 128),
    4: ("C4: CRNN 4 conv3x3+ReLU+maxpool stages (32/64/128/256) on 32x1x32x128, Linear 256->37, CTC, AdamW", 32, 32),
    5: ("C5: BERT-base-shaped 4 post-LN encoder layers, hidden 768, 12 heads, FFN 3072, seq 512, batch 8, "
        "token head 768->9, CE, AdamW", 8, 512),
}


def load_pkg():
    import importlib.util
    pkg_dir = os.path.join(ROOT, "onemodel-csharp_amd")
    spec = importlib.util.spec_from_file_location("onemodel_csharp_amd", os.path.join(pkg_dir, "__init__.py"),
                                                  submodule_search_locations=[pkg_dir])
    m = importlib.util.module_from_spec(spec)
    sys.modules["onemodel_csharp_amd"] = m
    spec.loader.exec_module(m)
    return m


class HipEvents:
    """hipEvent timing on a given stream through the HIP runtime the library already loaded."""

    def __init__(self):
        self.hip = C.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [C.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.hip.hipEventDestroy.argtypes = [C.c_void_p]

    def per_step(self, stream, fn, reps: int) -> list:
        """Milliseconds of each of reps calls of fn(), between events recorded on `stream` after each call: the
        device time from the end of one call's queued work to the end of the next one's."""
        evs = []
        for _ in range(reps + 1):
            e = C.c_void_p()
            assert self.hip.hipEventCreate(C.byref(e)) == 0
            evs.append(e)
        self.hip.hipEventRecord(evs[0], stream)
        for i in range(reps):
            fn()
            self.hip.hipEventRecord(evs[i + 1], stream)
        self.hip.hipEventSynchronize(evs[-1])
        out = []
        for i in range(reps):
            ms = C.c_float()
            self.hip.hipEventElapsedTime(C.byref(ms), evs[i], evs[i + 1])
            out.append(ms.value)
        for e in evs:
            self.hip.hipEventDestroy(e)
        return out

    def time(self, stream, fn, reps: int) -> float:
        """Average milliseconds of fn() over reps launches, measured between two events on `stream`. fn may be a
        list of launches over distinct buffer sets, called in turn (see MALL_BYTES)."""
        fns = fn if isinstance(fn, (list, tuple)) else [fn]
        e0, e1 = C.c_void_p(), C.c_void_p()
        assert self.hip.hipEventCreate(C.byref(e0)) == 0 and self.hip.hipEventCreate(C.byref(e1)) == 0
        self.hip.hipEventRecord(e0, stream)
        for i in range(reps):
            fns[i % len(fns)]()
        self.hip.hipEventRecord(e1, stream)
        self.hip.hipEventSynchronize(e1)
        ms = C.c_float()
        self.hip.hipEventElapsedTime(C.byref(ms), e0, e1)
        self.hip.hipEventDestroy(e0)
        self.hip.hipEventDestroy(e1)
        return ms.value / reps


# MI355X keeps a 256 MB Infinity Cache (MALL) in front of HBM. A kernel timed over and over on one working set
# smaller than that reads it from the cache, not from HBM, and can show more than the HBM peak. The HBM-priced
# timings below therefore cycle through enough distinct buffer sets that every launch finds its operands evicted:
# sets = ceil(2 * MALL_BYTES / bytes per set).
MALL_BYTES = 256 << 20


def _sets(bytes_per_set: int) -> int:
    return max(1, -(-2 * MALL_BYTES // bytes_per_set))


def _dev_buf(L, ctx, n, value):
    p = C.c_void_p()
    assert L.om_alloc(ctx, 0, 4 * n, C.byref(p)) == 0, L.om_last_error(ctx)
    assert L.om_fill(ctx, p, value, n) == 0
    return p


def _dev_rand(L, ctx, n, scale, seed):
    """A device buffer of n floats drawn from N(0, scale^2): MFMA power, and so the clock the GPU holds, depends on
    the operand bits, so timing on constant data would flatter the kernel."""
    import numpy as np
    h = (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)
    p = C.c_void_p()
    assert L.om_alloc(ctx, 0, 4 * n, C.byref(p)) == 0, L.om_last_error(ctx)
    assert L.om_upload(ctx, p, h.ctypes.data_as(C.c_void_p), 4 * n) == 0, L.om_last_error(ctx)
    return p


# The four Linear layers of the C3 block as (in, out): FFN 1536 -> 384 and 384 -> 1536, attention output 384 -> 384,
# packed q|k|v 384 -> 1152; their weight gradients share K = 4096 tokens.
DOMINANT_ROWS = 4096
DOMINANT_SHAPES = [(1536, 384), (384, 1536), (384, 384), (384, 1152)]


def time_dominant_in_step(pkg, model, graphed: bool, steps: int = 50):
    """The dominant launch as the training step runs it: the C3 step's one om_param_grads_group call (the grouped
    weight gradients of the block's four Linear layers with their fused bias gradients, the MFMA kernel plus its
    split-K reduce), bracketed by HIP events on the model's stream by the library's launch probe (om_ctx_probe) over
    `steps` eager training steps. Step graphs are switched off for these steps (a replayed graph makes no library
    calls to bracket, and a step that records one brackets nothing) whatever their state, and switched back on after
    when `graphed` (the bench's mode). Returns (calls recorded, mean ms per call)."""
    L = pkg.load_hip()
    ctx = model.ctx
    model.set_step_graph(False)
    assert L.om_ctx_probe(ctx, 1) == 0, L.om_last_error(ctx)
    for _ in range(steps):
        model.step()
    calls, mean = C.c_int(), C.c_double()
    assert L.om_ctx_probe(ctx, 0) == 0, L.om_last_error(ctx)
    assert L.om_ctx_probe_read(ctx, C.byref(calls), C.byref(mean)) == 0, L.om_last_error(ctx)
    if graphed:
        model.set_step_graph(True)
    return calls.value, mean.value


def time_dominant_kernel(pkg, model, ev, reps: int = 50):
    """The largest launch of the C3 step: the grouped weight and bias gradients of the block's four Linear layers (one
    om_linear_bwd_dw_group call = the MFMA kernel plus its split-K reduce), on random operands rotated through buffer
    sets larger than the MALL together, timed with HIP events on the model's stream."""
    import numpy as np
    L = pkg.load_hip()
    ctx = model.ctx
    rows, shapes = DOMINANT_ROWS, DOMINANT_SHAPES
    Item = pkg.om_linear_dw
    per_set = 4 * sum(rows * (i + o) + i * o + o for i, o in shapes)
    rng = np.random.default_rng(7)
    xs = {i: rng.standard_normal(rows * i).astype(np.float32) for i in sorted({i for i, _ in shapes})}
    gs = {o: (rng.standard_normal(rows * o) * 1e-3).astype(np.float32) for o in sorted({o for _, o in shapes})}

    def up(a):
        p = C.c_void_p()
        assert L.om_alloc(ctx, 0, 4 * a.size, C.byref(p)) == 0, L.om_last_error(ctx)
        assert L.om_upload(ctx, p, a.ctypes.data_as(C.c_void_p), 4 * a.size) == 0, L.om_last_error(ctx)
        return p

    keep, launches = [], []
    for _ in range(_sets(per_set)):
        items = (Item * len(shapes))()
        for j, (i, o) in enumerate(shapes):
            g, x = up(gs[o]), up(xs[i])
            dw, db = _dev_buf(L, ctx, o * i, 0.0), _dev_buf(L, ctx, o, 0.0)
            items[j] = Item(g.value, x.value, dw.value, db.value, i, o, 0, 0)
        keep.append(items)

        def launch(items=items):
            if L.om_linear_bwd_dw_group(ctx, len(shapes), C.cast(items, C.c_void_p), rows) != 0:
                raise RuntimeError(L.om_last_error(ctx).decode())
        launches.append(launch)
    for f in launches:
        f()
    ms = ev.time(L.om_ctx_stream(ctx), launches, reps)
    flops = sum(2.0 * rows * i * o for i, o in shapes)
    achieved = flops / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "kernel": "om_linear_bwd_dw_group: the C3 block's four weight gradients (1536x384, "
            "384x1536, 384x384, 384x1152; K = 4096) with fused bias gradients, incl. split-K reduce",
            "achieved": round(achieved, 2), "peak": FP32_MFMA_PEAK, "unit": "TFLOP/s",
            "frac": round(achieved / FP32_MFMA_PEAK, 4), "traffic": measured_traffic(), "ms_per_launch": round(ms, 5),
            "flops_per_launch": flops}


def time_adamw(pkg, model, ev, reps: int = 50):
    """The fused AdamW over C5's parameter count (28.36M) — 28 algorithmic bytes per parameter — on the same stream."""
    L = pkg.load_hip()
    ctx = model.ctx
    n = 28_358_409
    ss, sq = C.c_float(), C.c_float()
    L.om_adam_scalars(1e-3, 0.9, 0.999, 1, C.byref(ss), C.byref(sq))
    launches = []
    for k in range(_sets(16 * n)):
        p, g = _dev_rand(L, ctx, n + 3, 0.05, 3 + 100 * k), _dev_rand(L, ctx, n + 3, 1e-3, 4 + 100 * k)
        m, v = _dev_buf(L, ctx, n + 3, 0.0), _dev_buf(L, ctx, n + 3, 0.0)
        launches.append(lambda p=p, g=g, m=m, v=v: L.om_adam_step(ctx, p, g, m, v, None, n, 1e-3, 0.9, 0.999, 1e-8,
                                                                  0.01, 1, ss, sq))
    for f in launches:
        f()
    ms = ev.time(L.om_ctx_stream(ctx), launches, reps)
    gbs = 28.0 * n / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "kernel": "om_adam_step (C5 arena, 28.36M params)", "achieved": round(gbs, 1),
            "peak": HBM_PEAK, "unit": "GB/s", "frac": round(gbs / HBM_PEAK, 4), "ms_per_launch": round(ms, 5)}


def time_staged(pkg, model, steps: int):
    """Steps/s when every step's inputs (C3: x, target, lengths, mask = 14.7 MB) cross PCIe: each batch goes through
    a pinned staging slot and is uploaded on the copy stream while the previous step computes (omt_batch_*). The three
    pinned slots are filled once; each step re-commits one, so the timed work is the upload plus the step, not the
    host-side copy into the slot (a producer writes batches into the slot in place)."""
    L = pkg.load_train()
    ins = model.inputs()
    for _ in range(3):
        model.stage_batch(ins)
    host = C.c_void_p()

    def one():
        model.step()
        if L.omt_batch_begin(model.h, C.byref(host)) != 0 or L.omt_batch_commit(model.h) != 0:
            raise RuntimeError(L.omt_last_error(model.h).decode())

    for _ in range(10):
        one()
    pkg.load_hip().om_ctx_sync(model.ctx)
    t0 = time.perf_counter()
    for _ in range(steps):
        one()
    pkg.load_hip().om_ctx_sync(model.ctx)
    el = time.perf_counter() - t0
    for _ in range(L.omt_batch_queued(model.h)):  # drain
        model.step()
    nbytes = int(L.omt_batch_bytes(model.h))
    return {"value": round(steps / el, 3), "unit": "steps/s", "bytes_per_step": nbytes,
            "h2d_GBps": round(nbytes * steps / el / 1e9, 2),
            "note": "inputs uploaded from pinned staging slots every step, overlapped with the previous step"}


def time_clip(pkg, model, ev, reps: int = 50):
    """GradClip.ClipNorm on the device over C5's parameter count (28.36M gradients, one segment): the norm alone
    (partials + final: g read once, 4 algorithmic bytes per gradient) and norm + in-place scaling (g read and written
    once, 8 bytes per gradient; the scaling pass's second read of g comes from the Infinity Cache when the gradients
    fit in it, as C5's 113 MB do)."""
    L = pkg.load_hip()
    ctx = model.ctx
    n = 28_358_409
    slot = _dev_buf(L, ctx, 2, 0.0)
    coef = C.c_void_p(slot.value + 4)
    tables = []
    for k in range(_sets(4 * n)):
        g = _dev_rand(L, ctx, n, 1e-3, 12 + k)
        tables.append(((C.c_void_p * 1)(g.value), (C.c_int64 * 1)(n)))
    out = {}
    for name, in_place, per in (("clip_grad_norm", 0, 4.0), ("clip_grad_norm_scale", 1, 8.0)):
        def launch(ptrs, lens, in_place=in_place):
            # max_norm below every set's norm, so the in-place variant always runs its scaling pass
            st = L.om_clip_grad_norm(ctx, 1, C.cast(ptrs, C.c_void_p), C.cast(lens, C.c_void_p), C.c_float(1e-3),
                                     0, in_place, slot, coef)
            if st != 0:
                raise RuntimeError(L.om_last_error(ctx).decode())
        launches = [lambda t=t: launch(*t) for t in tables]
        for f in launches:
            f()
        ms = ev.time(L.om_ctx_stream(ctx), launches, reps)
        gbs = per * n / (ms * 1e-3) / 1e9
        out[name] = {"bound": "hbm", "kernel": f"om_clip_grad_norm (C5 arena, 28.36M grads, "
                     f"{'norm and in-place scale' if in_place else 'norm only'})", "achieved": round(gbs, 1),
                     "peak": HBM_PEAK, "unit": "GB/s", "frac": round(gbs / HBM_PEAK, 4), "ms_per_launch": round(ms, 5)}
    return out


def time_row_kernels(pkg, model, ev, reps: int = 50):
    """The C3 step's LayerNorm forward/backward (4096 x 384, om_layernorm_bwd including its fp64 column-sum final;
    cycling through buffer sets larger than the Infinity Cache) and fused attention forward/backward (B 32, H 12,
    L 128, D 32, padding mask), on random data, HIP events on the model's stream. LayerNorm is priced in algorithmic HBM bytes (forward 8 B/elem + 8 B/row + 8 B/col, backward
    12 B/elem + 8 B/row + 12 B/col), attention in MFMA flops (forward 2 products, backward 5, of 2 B H L^2 D)."""
    import numpy as np
    L = pkg.load_hip()
    ctx = model.ctx
    st = L.om_ctx_stream(ctx)
    out = {}
    R, Cc = 4096, 384
    gam, bet = _dev_rand(L, ctx, Cc, 0.1, 7), _dev_rand(L, ctx, Cc, 0.1, 8)
    dg, db = _dev_buf(L, ctx, Cc, 0.0), _dev_buf(L, ctx, Cc, 0.0)
    fwds, bwds = [], []
    for k in range(_sets(16 * R * Cc)):
        x, g = _dev_rand(L, ctx, R * Cc, 1.0, 5 + 100 * k), _dev_rand(L, ctx, R * Cc, 1.0, 6 + 100 * k)
        y, dx = _dev_buf(L, ctx, R * Cc, 0.0), _dev_buf(L, ctx, R * Cc, 0.0)
        mu, rs = _dev_buf(L, ctx, R, 0.0), _dev_buf(L, ctx, R, 0.0)
        fwds.append(lambda x=x, y=y, mu=mu, rs=rs: L.om_layernorm_fwd(ctx, x, gam, bet, y, mu, rs, R, Cc,
                                                                      C.c_float(1e-5)))
        bwds.append(lambda x=x, g=g, dx=dx, mu=mu, rs=rs: L.om_layernorm_bwd(ctx, g, x, gam, mu, rs, dx, dg, db, R,
                                                                             Cc, 0, 0))
    # The same bytes as the forward through the plainest kernel there is (y = max(x, 0)): what one launch moving
    # 6.3 MB in and 6.3 MB out reaches at all, the ceiling the LayerNorm launches are read against.
    streams = []
    for k in range(_sets(8 * R * Cc)):
        x, y = _dev_rand(L, ctx, R * Cc, 1.0, 500 + k), _dev_buf(L, ctx, R * Cc, 0.0)
        streams.append(lambda x=x, y=y: L.om_relu_fwd(ctx, x, y, R * Cc))
    for f in fwds:
        assert f() == 0  # statistics for the backward
    for name, fs, nbytes in (("stream_reference", streams, 8 * R * Cc),
                             ("layernorm_fwd", fwds, 8 * R * Cc + 8 * R + 8 * Cc),
                             ("layernorm_bwd", bwds, 12 * R * Cc + 8 * R + 12 * Cc)):
        for f in fs:
            assert f() == 0
        ms = ev.time(st, fs, reps)
        gbs = nbytes / (ms * 1e-3) / 1e9
        kern = "om_relu_fwd over 4096x384 (6.3 MB in, 6.3 MB out)" if name == "stream_reference" else \
            f"om_{name} 4096x384"
        out[name] = {"bound": "hbm", "kernel": kern, "achieved": round(gbs, 1), "peak": HBM_PEAK,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK, 4), "ms_per_launch": round(ms, 5)}
    B, H, Ls, D = 32, 12, 128, 32
    W = H * D
    qkv = _dev_rand(L, ctx, B * Ls * 3 * W, 1.0, 9)
    go = _dev_rand(L, ctx, B * Ls * W, 1.0, 10)
    rng = np.random.default_rng(11)
    mask = np.zeros((B, Ls, Ls), np.float32)
    for b in range(B):
        mask[b, :, rng.integers(64, 129):] = -np.inf
    M = C.c_void_p()
    assert L.om_alloc(ctx, 0, mask.nbytes, C.byref(M)) == 0
    assert L.om_upload(ctx, M, mask.ctypes.data_as(C.c_void_p), mask.nbytes) == 0
    o, dqkv = _dev_buf(L, ctx, B * Ls * W, 0.0), _dev_buf(L, ctx, B * Ls * 3 * W, 0.0)
    stats = _dev_buf(L, ctx, 2 * B * H * Ls, 0.0)
    off = lambda p, i: C.c_void_p(p.value + 4 * i * W)
    sc = C.c_float(0.0)
    # the entry points the tape calls (at this shape they run the whole-row kernels)
    afwd = lambda: L.om_attention_fwd_flash(ctx, qkv, off(qkv, 1), off(qkv, 2), 3 * W, M, 1, o, W, stats, B, H, Ls,
                                            D, sc)
    abwd = lambda: L.om_attention_bwd_flash(ctx, qkv, off(qkv, 1), off(qkv, 2), 3 * W, M, 1, o, W, stats, go, W,
                                            dqkv, off(dqkv, 1), off(dqkv, 2), 3 * W, B, H, Ls, D, sc, 0)
    unit = 2.0 * B * H * Ls * Ls * D
    for name, f, flops in (("attention_fwd", afwd, 2 * unit), ("attention_bwd", abwd, 5 * unit)):
        for _ in range(3):
            assert f() == 0
        ms = ev.time(st, f, reps)
        tf = flops / (ms * 1e-3) / 1e12
        out[name] = {"bound": "mfma", "kernel": f"om_{name}_flash B32 H12 L128 D32 masked (whole-row kernels)",
                     "achieved": round(tf, 2),
                     "peak": FP32_MFMA_PEAK, "unit": "TFLOP/s", "frac": round(tf / FP32_MFMA_PEAK, 4),
                     "ms_per_launch": round(ms, 5)}
    return out


def time_conv(pkg, model, ev, reps: int = 20):
    """C2's convolution (Conv2d 3x3, stride 1, padding 1, 64 -> 64 channels on 32 x 64 x 56 x 56) as the step runs it:
    the forward (om_conv2d_fwd with bias), the input gradient alone and the weight + bias gradients alone
    (om_conv2d_bwd with the other outputs NULL), each 2 N Cout Hout Wout Cin k^2 = 7.40 GFLOP, on random data,
    HIP events on the model's stream."""
    L = pkg.load_hip()
    ctx = model.ctx
    N, Ci, H, W, Co, K = 32, 64, 56, 56, 64, 3
    x, g = _dev_rand(L, ctx, N * Ci * H * W, 1.0, 31), _dev_rand(L, ctx, N * Co * H * W, 1e-2, 32)
    w, b = _dev_rand(L, ctx, Co * Ci * K * K, 0.05, 33), _dev_rand(L, ctx, Co, 0.1, 34)
    y, dx = _dev_buf(L, ctx, N * Co * H * W, 0.0), _dev_buf(L, ctx, N * Ci * H * W, 0.0)
    dw, db = _dev_buf(L, ctx, Co * Ci * K * K, 0.0), _dev_buf(L, ctx, Co, 0.0)
    geo = (N, Ci, H, W, Co, K, K, 1, 1)
    runs = (("conv_fwd", lambda: L.om_conv2d_fwd(ctx, x, w, b, y, *geo)),
            ("conv_dx", lambda: L.om_conv2d_bwd(ctx, g, x, w, dx, None, None, *geo, 0, 0)),
            ("conv_dw", lambda: L.om_conv2d_bwd(ctx, g, x, w, None, dw, db, *geo, 0, 0)))
    flops = 2.0 * N * Co * H * W * Ci * K * K
    out = {}
    for name, f in runs:
        for _ in range(3):
            assert f() == 0, L.om_last_error(ctx)
        ms = ev.time(L.om_ctx_stream(ctx), f, reps)
        tf = flops / (ms * 1e-3) / 1e12
        out[name] = {"bound": "mfma", "kernel": f"om_conv2d ({name[5:]}) C2: 32x64x56x56, 64->64, 3x3 p1",
                     "achieved": round(tf, 2), "peak": FP32_MFMA_PEAK, "unit": "TFLOP/s",
                     "frac": round(tf / FP32_MFMA_PEAK, 4), "ms_per_launch": round(ms, 5)}
    return out


def time_c5_rows(pkg, model, ev, reps: int = 20):
    """C5's LayerNorm forward / backward (4096 x 768, buffer sets cycled past the Infinity Cache) and attention forward
    / backward through the fused entry points (B 8, H 12, L 512, D 64, no mask), priced as time_row_kernels prices
    the C3 shapes."""
    L = pkg.load_hip()
    ctx = model.ctx
    st = L.om_ctx_stream(ctx)
    out = {}
    R, Cc = 4096, 768
    gam, bet = _dev_rand(L, ctx, Cc, 0.1, 41), _dev_rand(L, ctx, Cc, 0.1, 42)
    dg, db = _dev_buf(L, ctx, Cc, 0.0), _dev_buf(L, ctx, Cc, 0.0)
    fwds, bwds = [], []
    for k in range(_sets(16 * R * Cc)):
        x, g = _dev_rand(L, ctx, R * Cc, 1.0, 43 + 100 * k), _dev_rand(L, ctx, R * Cc, 1.0, 44 + 100 * k)
        y, dx = _dev_buf(L, ctx, R * Cc, 0.0), _dev_buf(L, ctx, R * Cc, 0.0)
        mu, rs = _dev_buf(L, ctx, R, 0.0), _dev_buf(L, ctx, R, 0.0)
        fwds.append(lambda x=x, y=y, mu=mu, rs=rs: L.om_layernorm_fwd(ctx, x, gam, bet, y, mu, rs, R, Cc,
                                                                      C.c_float(1e-5)))
        bwds.append(lambda x=x, g=g, dx=dx, mu=mu, rs=rs: L.om_layernorm_bwd(ctx, g, x, gam, mu, rs, dx, dg, db, R,
                                                                             Cc, 0, 0))
    for f in fwds:
        assert f() == 0
    for name, fs, nbytes in (("c5_layernorm_fwd", fwds, 8 * R * Cc + 8 * R + 8 * Cc),
                             ("c5_layernorm_bwd", bwds, 12 * R * Cc + 8 * R + 12 * Cc)):
        for f in fs:
            assert f() == 0
        ms = ev.time(st, fs, reps)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"bound": "hbm", "kernel": f"om_{name[3:]} 4096x768", "achieved": round(gbs, 1),
                     "peak": HBM_PEAK, "unit": "GB/s", "frac": round(gbs / HBM_PEAK, 4), "ms_per_launch": round(ms, 5)}
    B, H, Ls, D = 8, 12, 512, 64
    W = H * D
    qkv = _dev_rand(L, ctx, B * Ls * 3 * W, 1.0, 45)
    go = _dev_rand(L, ctx, B * Ls * W, 1.0, 46)
    o, dqkv = _dev_buf(L, ctx, B * Ls * W, 0.0), _dev_buf(L, ctx, B * Ls * 3 * W, 0.0)
    stats = _dev_buf(L, ctx, 2 * B * H * Ls, 0.0)
    off = lambda p, i: C.c_void_p(p.value + 4 * i * W)
    sc = C.c_float(0.0)
    afwd = lambda: L.om_attention_fwd_flash(ctx, qkv, off(qkv, 1), off(qkv, 2), 3 * W, None, 0, o, W, stats, B, H,
                                            Ls, D, sc)
    abwd = lambda: L.om_attention_bwd_flash(ctx, qkv, off(qkv, 1), off(qkv, 2), 3 * W, None, 0, o, W, stats, go, W,
                                            dqkv, off(dqkv, 1), off(dqkv, 2), 3 * W, B, H, Ls, D, sc, 0)
    unit = 2.0 * B * H * Ls * Ls * D
    for name, f, flops in (("c5_attention_fwd", afwd, 2 * unit), ("c5_attention_bwd", abwd, 5 * unit)):
        for _ in range(3):
            assert f() == 0, L.om_last_error(ctx)
        ms = ev.time(st, f, reps)
        tf = flops / (ms * 1e-3) / 1e12
        out[name] = {"bound": "mfma", "kernel": f"om_{name[3:]}_flash B8 H12 L512 D64 (streaming kernels; the "
                     f"backward's 5 products priced, its delta pre-pass and dQ reduce included)", "achieved": round(tf, 2),
                     "peak": FP32_MFMA_PEAK, "unit": "TFLOP/s", "frac": round(tf / FP32_MFMA_PEAK, 4),
                     "ms_per_launch": round(ms, 5)}
    return out


COPY_PROBE_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "dominant_kernel_traffic.json")


def pmc_probe(pkg, model):
    """Launches, in order, three plain device copies of COPY_PROBE_BYTES, three dominant launches (grouped weight
    gradients) and three AdamW steps, and nothing else, so that a `rocprofv3 --pmc FETCH_SIZE` (then WRITE_SIZE) run over this mode reads the
    counters of a copy of known size beside those of the kernels it scales."""
    L = pkg.load_hip()
    ctx = model.ctx
    n = COPY_PROBE_BYTES // 4
    src, dst = _dev_buf(L, ctx, n, 1.0), _dev_buf(L, ctx, n, 0.0)
    L.om_ctx_sync(ctx)
    for _ in range(3):
        assert L.om_copy(ctx, dst, src, COPY_PROBE_BYTES) == 0
    L.om_ctx_sync(ctx)
    time_dominant_kernel(pkg, model, HipEvents(), reps=3)
    time_adamw(pkg, model, HipEvents(), reps=3)
    L.om_ctx_sync(ctx)


# The dense products of one C3 step, as (name, m, n, k, ta, tb): C[m,n] = op(A) op(B) with A [m,k] (or [k,m] when ta)
# and B [k,n] (or [n,k] when tb).
C3_PRODUCTS = [("q, k, v projection", 4096, 1152, 384, 0, 1), ("attention output", 4096, 384, 384, 0, 1),
               ("FFN 384->1536", 4096, 1536, 384, 0, 1), ("FFN 1536->384", 4096, 384, 1536, 0, 1),
               ("dX FFN 1536->384", 4096, 1536, 384, 0, 0), ("dX FFN 384->1536", 4096, 384, 1536, 0, 0),
               ("dX attention output", 4096, 384, 384, 0, 0), ("dX q, k, v", 4096, 384, 1152, 0, 0)]


def vendor_gemm(reps: int = 30):
    """This library's products at the C3 shapes beside torch.mm in fp32 (hipBLASLt / rocBLAS), same random operands,
    warm, HIP events on each side's stream: a calibration of the GEMM engine against the vendor library. The weight
    gradients are compared as the C3 step runs them: the library's one grouped launch (with its reduce and bias
    sums) against four torch.mm calls (without bias sums). Prints a markdown table."""
    import numpy as np
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False
    pkg = load_pkg()
    L = pkg.load_hip()
    ctx = C.c_void_p()
    assert L.om_ctx_create(0, C.byref(ctx)) == 0
    ev = HipEvents()
    dev = torch.device("cuda")
    tev = lambda: torch.cuda.Event(enable_timing=True)

    def torch_time(f):
        for _ in range(3):
            f()
        e0, e1 = tev(), tev()
        e0.record()
        for _ in range(reps):
            f()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    rows = ["| product | m x n x k | this library us | TFLOP/s | torch.mm us | TFLOP/s |", "|---|---|---:|---:|---:|---:|"]
    big = 4096 * 1536
    a, b, c = _dev_rand(L, ctx, big, 0.1, 1), _dev_rand(L, ctx, big, 0.1, 2), _dev_buf(L, ctx, big, 0.0)
    for name, m, n, k, ta, tb in C3_PRODUCTS:
        lda, ldb = (m if ta else k), (k if tb else n)
        f = lambda: L.om_gemm(ctx, ta, tb, m, n, k, a, lda, b, ldb, c, n, None, 0, None)
        for _ in range(3):
            assert f() == 0, L.om_last_error(ctx)
        ms = ev.time(L.om_ctx_stream(ctx), f, reps)
        A = torch.randn(k, m, device=dev).t() if ta else torch.randn(m, k, device=dev)
        B = torch.randn(n, k, device=dev).t() if tb else torch.randn(k, n, device=dev)
        tm = torch_time(lambda: torch.mm(A, B))
        fl = 2.0 * m * n * k
        rows.append(f"| {name} | {m} x {n} x {k} | {ms * 1e3:.1f} | {fl / ms / 1e9:.1f} | {tm * 1e3:.1f} | "
                    f"{fl / tm / 1e9:.1f} |")
    items = (pkg.om_linear_dw * 4)()
    for i, (inf, outf) in enumerate(DOMINANT_SHAPES):
        g, x = _dev_rand(L, ctx, DOMINANT_ROWS * outf, 0.1, 10 + i), _dev_rand(L, ctx, DOMINANT_ROWS * inf, 0.1, 20 + i)
        dw, db = _dev_buf(L, ctx, outf * inf, 0.0), _dev_buf(L, ctx, outf, 0.0)
        items[i] = pkg.om_linear_dw(g.value, x.value, dw.value, db.value, inf, outf, 0, 0)
    f = lambda: L.om_linear_bwd_dw_group(ctx, 4, C.cast(items, C.c_void_p), DOMINANT_ROWS)
    for _ in range(3):
        assert f() == 0, L.om_last_error(ctx)
    ms = ev.time(L.om_ctx_stream(ctx), f, reps)
    ts = [(torch.randn(DOMINANT_ROWS, outf, device=dev), torch.randn(DOMINANT_ROWS, inf, device=dev))
          for inf, outf in DOMINANT_SHAPES]
    tm = torch_time(lambda: [torch.mm(g.t(), x) for g, x in ts])
    fl = sum(2.0 * DOMINANT_ROWS * i * o for i, o in DOMINANT_SHAPES)
    rows.append(f"| the four weight gradients (dW = g^T x, K = 4096) | 1536x384, 384x1536, 384x384, 1152x384 | "
                f"{ms * 1e3:.1f} | {fl / ms / 1e9:.1f} | {tm * 1e3:.1f} | {fl / tm / 1e9:.1f} |")
    A, B = torch.randn(8192, 8192, device=dev), torch.randn(8192, 8192, device=dev)
    tm = torch_time(lambda: torch.mm(A, B))
    rows.append(f"| (large square, torch only) | 8192 x 8192 x 8192 | | | {tm * 1e3:.1f} | {2.0 * 8192 ** 3 / tm / 1e9:.1f} |")
    L.om_ctx_destroy(ctx)
    print("\n".join(rows))


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from the committed counter summary (two rocprofv3 --pmc runs of
    `bench.py --pmc-probe`, each counter scaled by its reading for the known-size copy), or None without one."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return int(t["fetch_bytes"] + t["write_bytes"])
    except (OSError, ValueError, KeyError):
        return None


def cpu_model() -> str:
    """The host CPU's model name as `lscpu` reports it (from /proc/cpuinfo when lscpu is absent)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], stdout=subprocess.PIPE, stderr=subprocess.DEVNULL, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _omp_threads(n: int):
    """Sets the OpenMP thread count of the oracle library's runtime (libgomp, already loaded with it)."""
    try:
        C.CDLL("libgomp.so.1").omp_set_num_threads(C.c_int(n))
    except OSError:
        pass


def _cpu_run(oc, seconds: float, min_steps: int, warm: bool = True):
    if warm:
        oc.step()  # warm-up (page-in, thread pool)
    times = []
    t0 = time.perf_counter()
    while True:
        t = time.perf_counter()
        oc.step()
        times.append(time.perf_counter() - t)
        if len(times) >= min_steps and time.perf_counter() - t0 >= seconds:
            break
    times.sort()
    return len(times), sum(times), times[len(times) // 2]


def cpu_baseline(cfg: int, seconds: float):
    """The oracle's step (C restatement of the reference CPU path) on this host's cores, at the benchmark's full
    size: with all the threads OpenMP is given (OMP_NUM_THREADS, else the core count) for about `seconds`, and on one
    thread for about half as long; each reports the median step time of its sample (at least two steps). Where one
    full step on one thread would not fit that budget (C5), the one-thread sample runs the same model at a smaller
    batch and scales its step time by the batch ratio (the step's work is linear in the batch)."""
    from oracle import models
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    oc = models.make_config(cfg)
    _omp_threads(threads)
    n, tot, med = _cpu_run(oc, seconds, 2)
    _omp_threads(1)
    full = WORKLOADS[cfg][1]
    b = full
    while b > 1 and med * threads * b / full > seconds / 4:  # a generous guess of one thread's step time
        b //= 2
    if b == full:
        n1, tot1, med1 = _cpu_run(oc, seconds / 2, 2, warm=False)
        one_sample = f"{n1} full-size steps, {tot1:.1f} s"
    else:
        n1, tot1, med1 = _cpu_run(models.make_config(cfg, {"batch": b}), seconds / 2, 1, warm=False)
        one_sample = (f"{n1} steps at batch {b} of {full}, {tot1:.1f} s; the median step time scaled by {full // b} "
                      f"to the full batch")
        med1 *= full / b
    _omp_threads(threads)
    return {"value": round(1.0 / med, 4), "unit": "steps/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "nproc": os.cpu_count(),
            "one_core": {"value": round(1.0 / med1, 4), "unit": "steps/s", "cores": 1, "sample": one_sample},
            "sample": f"median of {n} full-size C{cfg} steps (ZeroGrad+fwd+bwd+AdamW) of oracle/om_oracle.c via "
                      f"oracle/tape.py, {tot:.1f} s, OpenMP {threads} threads"}


def time_per_op(pkg, cfg, steps, warmup, graph=True):
    """The same configuration built with the reference's own record structure (omt_config_create_records,
    OMT_RECORDS_PER_OP: every rule one C-ABI call when the engine reaches it, no composite records, no colocated q|k|v,
    no grouped weight gradients), timed like the headline: eager launches, then (unless graph is False) from a step
    graph."""
    m = pkg.Model(cfg, per_op=True)
    try:
        out = {"step_graph": None}
        for mode in ("eager", "step_graph") if graph else ("eager",):
            if mode == "step_graph":
                m.set_step_graph(True)
            for _ in range(warmup):
                m.step()
            pkg.load_hip().om_ctx_sync(m.ctx)
            t0 = time.perf_counter()
            for _ in range(steps):
                m.step()
            pkg.load_hip().om_ctx_sync(m.ctx)
            out[mode] = round(steps / (time.perf_counter() - t0), 3)
        per = sorted(HipEvents().per_step(pkg.load_hip().om_ctx_stream(m.ctx), m.step, max(50, steps)))
        out["median_ms"] = round(per[len(per) // 2], 4)
        return out
    finally:
        m.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-kernels", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="time the step without step graphs only")
    ap.add_argument("--no-per-op", action="store_true",
                    help="skip the per-op record structure's rate (profiling runs of the fused step alone)")
    ap.add_argument("--pmc-probe", action="store_true", help="only the launches a counter run needs (no timing line)")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="only the C3 products beside torch.mm (hipBLASLt / rocBLAS), as a markdown table")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    if a.vendor_gemm:
        vendor_gemm()
        return
    pkg = load_pkg()
    model = pkg.Model(a.config)
    if a.pmc_probe:
        pmc_probe(pkg, model)
        model.close()
        return
    def timed_window():
        for _ in range(a.warmup):
            model.step()
        pkg.load_hip().om_ctx_sync(model.ctx)
        t0 = time.perf_counter()
        last = None
        for _ in range(a.steps):
            last = model.step()  # each step returns once its loss has landed on the host
        pkg.load_hip().om_ctx_sync(model.ctx)
        return time.perf_counter() - t0, last

    # The step as the tape runs it launch by launch, then (unless --no-graph) the same step recorded once into a
    # HIP graph and replayed (omt_set_step_graph; bit-identical results): the headline is the faster of the two.
    el_eager, loss = timed_window()
    el, el_graph = el_eager, None
    if not a.no_graph:
        model.set_step_graph(True)
        el_graph, loss_g = timed_window()
        if not model.step_graph_ready:
            raise SystemExit(f"bench.py: C{a.config} did not run from a step graph")
        if el_graph < el_eager:
            el, loss = el_graph, loss_g
        else:
            model.set_step_graph(False)
    graphed = el_graph is not None and el == el_graph
    sps = a.steps / el
    # per-step device times: HIP events on the model's stream after each step, over at least 50 further steps
    # (a separate pass, so the events do not touch the timed window above)
    per = sorted(HipEvents().per_step(pkg.load_hip().om_ctx_stream(model.ctx), model.step, max(50, a.steps)))
    q = lambda f: per[min(len(per) - 1, int(f * len(per)))]
    desc, batch, seq = WORKLOADS[a.config]
    out = {
        "metric": METRIC, "value": round(sps, 3), "unit": "steps/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(1000.0 * el / a.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": desc, "global_batch": batch, "seq_len": seq, "parallelism": "none (1 GPU)"},
        "step_ms": {"median": round(q(0.5), 4), "p10": round(q(0.1), 4), "p90": round(q(0.9), 4), "n": len(per),
                    "median_steps_per_s": round(1000.0 / q(0.5), 3), "timing": "hipEvent per step"},
        "final_loss": loss,
        "mode": "step graph" if graphed else "eager",
        "modes": {"eager": round(a.steps / el_eager, 3),
                  "step_graph": round(a.steps / el_graph, 3) if el_graph else None,
                  "note": "steps/s of the same step launched kernel by kernel from the host tape (eager) and "
                          "replayed from a recorded HIP graph (omt_set_step_graph); the results are bit-identical, "
                          "value is the faster of the two"},
    }
    po = None if a.no_per_op else time_per_op(pkg, a.config, a.steps, a.warmup, graph=not a.no_graph)
    if po:
        out["modes"]["per_op"] = po["eager"]
        out["modes"]["per_op_step_graph"] = po["step_graph"]
        out["modes"]["per_op_median_ms"] = po["median_ms"]
    out["modes"]["per_op_note"] = ("the reference's own records (omt_config_create_records, OMT_RECORDS_PER_OP): "
                                   "Linear as Reshape/MatMul/Add/Reshape, three q/k/v Linears over weights of their "
                                   "own, Conv2d/Relu/MaxPool2d apart, Mean then Permute, Mse as Sub/Mul/Mean, "
                                   "CrossEntropy as LogSoftmax/NllLoss, every rule one C-ABI call made when the engine "
                                   "reaches it (no grouped weight gradients); eager launches and from a step graph")
    if a.config == 3:
        out["pcie_inclusive"] = time_staged(pkg, model, a.steps)
    if a.config == 3:
        # the roofline of the dominant launch as it runs inside training steps (events around the launch itself)
        calls, ms = time_dominant_in_step(pkg, model, graphed)
        flops = sum(2.0 * DOMINANT_ROWS * i * o for i, o in DOMINANT_SHAPES)
        if calls != 50 or ms <= 0.0:
            raise SystemExit(f"bench.py: the launch probe recorded {calls} grouped weight-gradient calls in 50 steps")
        achieved = flops / (ms * 1e-3) / 1e12
        out["roofline"] = {
            "bound": "mfma", "kernel": "om_param_grads_group inside the C3 step: the block's four weight gradients "
            "(1536x384, 384x1536, 384x384, 384x1152; K = 4096) with fused bias gradients, the MFMA kernel plus its "
            "split-K reduce", "achieved": round(achieved, 2), "peak": FP32_MFMA_PEAK, "unit": "TFLOP/s",
            "frac": round(achieved / FP32_MFMA_PEAK, 4), "traffic": measured_traffic(),
            "ms_per_launch": round(ms, 5), "flops_per_launch": flops, "launches_timed": calls,
            "timing": "hipEvent pair around the launch on the model's stream (om_ctx_probe), 50 eager training steps"}
    if not a.no_kernels:
        ev = HipEvents()
        cold = time_dominant_kernel(pkg, model, ev)
        if "roofline" in out:
            out["roofline"]["cold"] = {k: cold[k] for k in ("achieved", "frac", "ms_per_launch")}
            out["roofline"]["cold"]["note"] = ("the same launch alone on random operands rotated through buffer sets "
                                               "larger than the MALL")
        else:
            out["roofline"] = cold  # other configurations: C3's dominant launch alone, cold
        out["kernels"] = {"adamw": time_adamw(pkg, model, ev), **time_row_kernels(pkg, model, ev),
                          **time_clip(pkg, model, ev), **time_conv(pkg, model, ev), **time_c5_rows(pkg, model, ev)}
    if not a.no_cpu:
        cb = cpu_baseline(a.config, a.cpu_seconds)
        cb["gpu_over_cpu"] = round(sps / cb["value"], 1)
        out["cpu_baseline"] = cb
    model.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
