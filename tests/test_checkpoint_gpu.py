"""Checkpoints of device models (omt_checkpoint_save / omt_checkpoint_load), on the GPU.

Pins: the writer's bytes equal the file assembled here from the documented layout (docs/training.md section 6 of
the reference: header, compact manifest in field order, 64-aligned raw tensors) for a model-only and a full
checkpoint; saving is deterministic and a load restores every bit (CheckpointTests.cs:20-43); a run saved at step k
and resumed in a fresh model equals the uninterrupted run bit for bit, for the SGD-momentum MLP, the conv net with
BatchNorm, clipping and a cosine schedule, and the encoder classifier with dropout (CheckpointTests.cs:45-86);
model-only files, optimizer kind mismatches and foreign models fail as the reference's do and change nothing
(CheckpointTests.cs:88-127).
"""
import json
import struct

import numpy as np
import pytest

from conftest import load_golden

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pkg():
    from gpu_util import load_pkg
    return load_pkg()


def feeder(cfg):
    if cfg == 6:
        o = load_golden("training_mlp")
        return lambda m, i: (m.write_input("x", o["in.x"][o["in.order"][i].astype(int)]),
                             m.write_input("labels", o["in.y"][o["in.order"][i].astype(int)].astype(np.int32)))
    if cfg == 7:
        o = load_golden("training_cnn")
        return lambda m, i: (m.write_input("x", o["in.x"][o["in.order"][i].astype(int)]),
                             m.write_input("labels", o["in.y"][o["in.order"][i].astype(int)].astype(np.int32)))
    o = load_golden("training_encoder")
    ids = o["in.ids"].astype(np.int32)
    return lambda m, i: (m.write_input("ids", ids[o["in.order"][i].astype(int)]),
                         m.write_input("labels", o["in.y"][o["in.order"][i].astype(int)].astype(np.int32)))


def full_state(m):
    """Every bit of the training state: parameters, gradients aside, both moment blocks, buffers, step, rate."""
    out = {}
    for i, (n, _) in enumerate(m.params()):
        for which in (0, 2, 3):
            out[(n, which)] = m.read_param(i, which).view(np.uint32).copy()
    for n, b in m.buffers().items():
        out[(n, "buf")] = b.view(np.uint32).copy()
    out["step"] = m.step_count
    out["lr"] = np.float32(m.lr).view(np.uint32)
    return out


def same(a, b):
    assert a.keys() == b.keys()
    for k in a:
        assert np.array_equal(a[k], b[k]), k


def test_writer_bytes_follow_the_documented_layout(pkg, tmp_path):
    m = pkg.Model(6)
    try:
        f = feeder(6)
        for i in range(3):
            f(m, i)
            m.step()
        names = [(n, s) for n, s in m.params()]
        vals = [m.read_param(i) for i in range(len(names))]
        bufs = [m.read_param(i, 2) for i in range(len(names))]

        def layout(tensors):
            offs, cur = [], 0
            for t in tensors:
                offs.append(cur)
                cur = (cur + t.nbytes + 63) // 64 * 64
            data = bytearray(cur)
            for t, o in zip(tensors, offs):
                data[o:o + t.nbytes] = np.ascontiguousarray(t).tobytes()
            return offs, bytes(data)

        def entries(ns, ts, offs, dtype="f32"):
            return ",".join('{"name":"%s","dtype":"%s","shape":[%s],"offset":%d,"length":%d}'
                            % (n, dtype, ",".join(map(str, t.shape)), o, t.nbytes) for n, t, o in zip(ns, ts, offs))

        def frame(manifest, data):
            mb = manifest.encode()
            doff = (64 + len(mb) + 63) // 64 * 64
            head = b"ONEMCKPT" + struct.pack("<IIQQQQQQ", 1, 0, 64, len(mb), doff, len(data), doff + len(data), 0)
            return head + mb + bytes(doff - 64 - len(mb)) + data

        # model only
        offs, data = layout(vals)
        want = frame('{"format":"onemodel-checkpoint","version":1,"model":[%s],"extra":[]}'
                     % entries([n for n, _ in names], vals, offs), data)
        p = tmp_path / "m.ckpt"
        m.save_checkpoint(str(p), optimizer=False)
        assert p.read_bytes() == want
        # with the SGD optimizer: hyper-parameters as float bits, "initialized" flags, momentum buffers
        flags = np.ones(len(names), np.int32)
        offs, data = layout(vals + [flags] + bufs)
        bits = lambda v: struct.unpack("<I", struct.pack("<f", v))[0]
        hyper = ",".join('{"name":"%s","bits":%d}' % (k, bits(v)) for k, v in
                         (("lr", 0.05), ("momentum", 0.9), ("dampening", 0.0), ("weight_decay", 1e-4),
                          ("nesterov", 0.0)))
        state = (entries(["initialized"], [flags], offs[len(vals):len(vals) + 1], "i32") + "," +
                 entries([f"momentum_buffer.{i}" for i in range(len(names))], bufs, offs[len(vals) + 1:]))
        want = frame('{"format":"onemodel-checkpoint","version":1,"model":[%s],"optimizer":{"kind":"sgd","step":3,'
                     '"hyper":[%s],"state":[%s]},"extra":[{"key":"epoch","value":0},{"key":"step","value":3}]}'
                     % (entries([n for n, _ in names], vals, offs), hyper, state), data)
        m.save_checkpoint(str(p), extra={"step": 3, "epoch": 0})
        assert p.read_bytes() == want
        json.loads(want[64:64 + struct.unpack("<Q", want[24:32])[0]])  # and it is JSON
    finally:
        m.close()


def test_round_trip_is_bit_exact_and_saving_is_deterministic(pkg, tmp_path):
    a, b = pkg.Model(9), pkg.Model(9)
    try:
        f = feeder(9)
        for i in range(6):
            f(a, i)
            a.step()
        p1, p2, p3 = (str(tmp_path / n) for n in ("1.ckpt", "2.ckpt", "3.ckpt"))
        a.save_checkpoint(p1, extra={"step": 6, "epoch": 0})
        a.save_checkpoint(p2, extra={"epoch": 0, "step": 6})
        assert open(p1, "rb").read() == open(p2, "rb").read()  # extras are written in key order
        for i, (_, s) in enumerate(b.params()):
            b.write_param(i, np.full(s, 0.25, np.float32))
        had, extra = b.load_checkpoint(p1)
        assert had and extra == {"epoch": 0, "step": 6}
        same(full_state(a), full_state(b))
        b.save_checkpoint(p3, extra={"step": 6, "epoch": 0})
        assert open(p1, "rb").read() == open(p3, "rb").read()
        assert b.step_count == 6
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("cfg,total,cut", [(9, 20, 9), (7, 24, 11), (6, 30, 13)],
                         ids=["encoder-dropout", "cnn-bn-clip-cosine", "mlp-sgd-momentum"])
def test_resume_equals_uninterrupted_run(pkg, tmp_path, cfg, total, cut):
    f = feeder(cfg)
    whole = pkg.Model(cfg)
    first = pkg.Model(cfg)
    second = pkg.Model(cfg)
    try:
        lw = []
        for i in range(total):
            f(whole, i)
            lw.append(whole.step())
        ls = []
        for i in range(cut):
            f(first, i)
            ls.append(first.step())
        p = str(tmp_path / "r.ckpt")
        first.save_checkpoint(p, extra={"step": cut})
        _, extra = second.load_checkpoint(p)
        for i in range(extra["step"], total):
            f(second, i)
            ls.append(second.step())
        assert np.array_equal(np.array(lw, np.float32).view(np.uint32), np.array(ls, np.float32).view(np.uint32))
        same(full_state(whole), full_state(second))
    finally:
        whole.close()
        first.close()
        second.close()


def test_model_only_and_optimizer_requirements(pkg, tmp_path):
    a, b = pkg.Model(6), pkg.Model(6)
    try:
        f = feeder(6)
        f(a, 0)
        a.step()
        p = str(tmp_path / "m.ckpt")
        a.save_checkpoint(p, optimizer=False)
        had, _ = b.load_checkpoint(p, optimizer=False)
        assert not had
        for i in range(len(a.params())):
            assert np.array_equal(a.read_param(i).view(np.uint32), b.read_param(i).view(np.uint32))
        with pytest.raises(pkg.CheckpointError) as e:
            b.load_checkpoint(p)
        assert e.value.kind == "Mismatch"
        q = str(tmp_path / "full.ckpt")
        a.save_checkpoint(q)
        had, _ = b.load_checkpoint(q, optimizer=False)  # a full file loads into a model alone
        assert had
    finally:
        a.close()
        b.close()


def test_mismatches_change_nothing(pkg, tmp_path):
    a = pkg.Model(6)
    c = pkg.Model(7)
    d = pkg.Model(6)
    try:
        f = feeder(6)
        f(a, 0)
        a.step()
        p = str(tmp_path / "m.ckpt")
        a.save_checkpoint(p)
        before = full_state(c)
        with pytest.raises(pkg.CheckpointError) as e:
            c.load_checkpoint(p, optimizer=False)
        assert e.value.kind == "Mismatch"
        same(before, full_state(c))
        d.set_optimizer("adam", 1e-3)  # an optimizer of another kind
        before = full_state(d)
        with pytest.raises(pkg.CheckpointError) as e:
            d.load_checkpoint(p)
        assert e.value.kind == "Mismatch"
        same(before, full_state(d))
        d.set_optimizer("sgd", 0.05, momentum=0.5, weight_decay=1e-4)  # same kind, other fixed setting
        with pytest.raises(pkg.CheckpointError) as e:
            d.load_checkpoint(p)
        assert e.value.kind == "Mismatch"
    finally:
        a.close()
        c.close()
        d.close()
