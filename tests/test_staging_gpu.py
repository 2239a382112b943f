"""Host data staging (om_stager_*, omt_batch_*), on the GPU.

A run fed through pinned staging slots, each batch committed one step ahead so its upload overlaps the previous
step, must equal the same run fed with omt_input_write bit for bit; the slot protocol refuses a fourth waiting
batch, a slot not yet released, and out-of-range labels, and never changes the data it carries.
"""
import ctypes as C

import numpy as np
import pytest

from conftest import load_golden

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pkg():
    from gpu_util import load_pkg
    return load_pkg()


def cnn_batches(n):
    o = load_golden("training_cnn")
    out = []
    for i in range(n):
        idx = o["in.order"][i].astype(int)
        out.append({"x": o["in.x"][idx], "labels": o["in.y"][idx].astype(np.int32)})
    return out


def state(m):
    return [m.read_param(i, w).view(np.uint32).copy() for i in range(len(m.params())) for w in (0, 2, 3)]


def test_staged_run_equals_written_run(pkg):
    batches = cnn_batches(10)
    a, b = pkg.Model(7), pkg.Model(7)
    try:
        la = []
        for bt in batches:
            for k, v in bt.items():
                a.write_input(k, v)
            la.append(a.step())
        lb = []
        b.stage_batch(batches[0])
        for i in range(len(batches)):
            if i + 1 < len(batches):
                b.stage_batch(batches[i + 1])  # committed before step i runs: its upload overlaps step i
            lb.append(b.step())
        assert pkg.load_train().omt_batch_queued(b.h) == 0
        assert np.array_equal(np.array(la, np.float32).view(np.uint32), np.array(lb, np.float32).view(np.uint32))
        for x, y in zip(state(a), state(b)):
            assert np.array_equal(x, y)
        bufs_a, bufs_b = a.buffers(), b.buffers()
        for k in bufs_a:
            assert np.array_equal(bufs_a[k].view(np.uint32), bufs_b[k].view(np.uint32)), k
    finally:
        a.close()
        b.close()


def test_staged_c3_batch_equals_resident_inputs(pkg):
    """The benchmark block with its own inputs staged each step: the same losses as the resident inputs."""
    a, b = pkg.Model(3, batch=4), pkg.Model(3, batch=4)
    try:
        ins = b.inputs()
        la = [a.step() for _ in range(3)]
        lb = []
        b.stage_batch(ins)
        for i in range(3):
            if i < 2:
                b.stage_batch(ins)
            lb.append(b.step())
        assert np.array_equal(np.array(la, np.float32).view(np.uint32), np.array(lb, np.float32).view(np.uint32))
    finally:
        a.close()
        b.close()


def test_queue_limit_and_range_checks(pkg):
    m = pkg.Model(7)
    try:
        bt = cnn_batches(4)
        for i in range(3):
            m.stage_batch(bt[i])
        L = pkg.load_train()
        host = C.c_void_p()
        assert L.omt_batch_begin(m.h, C.byref(host)) == 4  # OM_E_STATE: three batches already wait
        m.step()
        bad = dict(bt[3])
        bad["labels"] = np.full(8, 5, np.int32)  # five classes: 5 is out of range
        with pytest.raises(pkg.OmError):
            m.stage_batch(bad)
        assert L.omt_batch_queued(m.h) == 2
        m.step()
        m.step()
        assert L.omt_batch_queued(m.h) == 0
    finally:
        m.close()


def test_stager_protocol_carries_data_unchanged(pkg):
    from gpu_util import Dev
    d = Dev()
    L = d.ctx.L
    s = C.c_void_p()
    n = 1 << 20
    d.call("om_stager_create", C.c_uint64(4 * n), 2, C.byref(s))
    try:
        assert L.om_stager_slot_bytes(s) == 4 * n
        out = d.empty((n,))
        rng = np.random.default_rng(0)
        for it in range(5):
            host, slot = C.c_void_p(), C.c_int()
            assert L.om_stager_begin(s, C.byref(host), C.byref(slot)) == 0
            assert slot.value == it % 2
            a = rng.standard_normal(n).astype(np.float32)
            C.memmove(host.value, a.ctypes.data, a.nbytes)
            dev = C.c_void_p()
            assert L.om_stager_commit(s, slot, C.c_uint64(a.nbytes), C.byref(dev)) == 0
            assert L.om_stager_acquire(s, slot) == 0
            d.call("om_copy", out, dev, C.c_uint64(a.nbytes))
            assert L.om_stager_release(s, slot) == 0
            assert np.array_equal(d.get(out).view(np.uint32), a.view(np.uint32))
        # a slot whose batch is not released cannot be begun again
        host, slot = C.c_void_p(), C.c_int()
        for _ in range(2):
            assert L.om_stager_begin(s, C.byref(host), C.byref(slot)) == 0
            assert L.om_stager_commit(s, slot, C.c_uint64(16), None) == 0
        assert L.om_stager_begin(s, C.byref(host), C.byref(slot)) == 4
        assert L.om_stager_commit(s, 0, C.c_uint64(8 * n), None) != 0  # more than a slot holds
    finally:
        L.om_stager_destroy(s)
        d.ctx.close()


def test_readback_takes_the_value_at_its_place_in_the_stream(pkg):
    """om_readback_post copies the value as the stream has it at the post; work queued after it (here a fill of the
    same buffer) does not change what om_readback_wait returns, and the next post sees the fill."""
    from gpu_util import Dev
    d = Dev()
    L = d.ctx.L
    r = C.c_void_p()
    d.call("om_readback_create", C.c_uint64(64), C.byref(r))
    try:
        for k in range(3):  # successive posts of one buffer (the sequence number moves on each time)
            src = d.put(np.full(16, float(k), np.float32))
            assert L.om_readback_post(r, src.data_ptr(), C.c_uint64(64)) == 0
            got = np.zeros(16, np.float32)
            assert L.om_readback_wait(r, got.ctypes.data, C.c_uint64(64)) == 0
            assert np.array_equal(got, np.full(16, float(k), np.float32))
        a = np.arange(16, dtype=np.float32) * 0.5 - 3.0
        src = d.put(a)
        assert L.om_readback_post(r, src.data_ptr(), C.c_uint64(64)) == 0
        d.call("om_fill", src, C.c_float(7.0), C.c_int64(16))
        out = np.zeros(16, np.float32)
        assert L.om_readback_wait(r, out.ctypes.data, C.c_uint64(64)) == 0
        assert np.array_equal(out.view(np.uint32), a.view(np.uint32))
        assert L.om_readback_post(r, src.data_ptr(), C.c_uint64(8)) == 0
        two = np.zeros(2, np.float32)
        assert L.om_readback_wait(r, two.ctypes.data, C.c_uint64(8)) == 0
        assert np.array_equal(two, np.full(2, 7.0, np.float32))
        assert L.om_readback_wait(r, out.ctypes.data, C.c_uint64(16)) != 0  # more than the last post carried
        assert L.om_readback_post(r, src.data_ptr(), C.c_uint64(128)) != 0  # more than the buffer holds
    finally:
        L.om_readback_destroy(r)
        d.ctx.close()


def test_readback_wait_before_any_post_is_refused(pkg):
    from gpu_util import Dev
    d = Dev()
    L = d.ctx.L
    r = C.c_void_p()
    d.call("om_readback_create", C.c_uint64(4), C.byref(r))
    try:
        v = np.zeros(1, np.float32)
        assert L.om_readback_wait(r, v.ctypes.data, C.c_uint64(4)) == 4  # OM_E_STATE
        big = C.c_void_p()
        assert L.om_readback_create(d.ctx.h, C.c_uint64((64 << 10) + 1), C.byref(big)) == 1  # beyond 64 KiB
        assert not big.value
    finally:
        L.om_readback_destroy(r)
        d.ctx.close()


def test_mse_posts_its_loss_from_its_own_launch(pkg):
    """om_mse_fwd_post: the loss, diff and unit gradient of om_mse_fwd_unit bit for bit, and the same loss landed in
    the readback buffer with no readback launch of its own; over sizes from one workgroup to the grid-stride range,
    posts in a row, and a readback of another context refused."""
    from gpu_util import Dev
    d = Dev()
    L = d.ctx.L
    r = C.c_void_p()
    d.call("om_readback_create", C.c_uint64(4), C.byref(r))
    rng = np.random.default_rng(5)
    try:
        for n in (1, 255, 256, 1000, 65536, 1572864, 262144 * 4 + 17):
            pred = rng.standard_normal(n).astype(np.float32)
            tgt = rng.standard_normal(n).astype(np.float32)
            P, TG = d.put(pred), d.put(tgt)
            D1, L1, U1 = d.empty((n,)), d.empty((1,)), d.empty((n,))
            D2, L2, U2 = d.empty((n,)), d.empty((1,)), d.empty((n,))
            d.call("om_mse_fwd_unit", P, TG, D1, L1, U1, C.c_int64(n))
            d.call("om_mse_fwd_post", P, TG, D2, L2, U2, C.c_int64(n), r)
            got = np.zeros(1, np.float32)
            assert L.om_readback_wait(r, got.ctypes.data, C.c_uint64(4)) == 0
            loss = d.get(L1)
            assert np.array_equal(d.get(L2).view(np.uint32), loss.view(np.uint32)), n
            assert np.array_equal(got.view(np.uint32), loss.view(np.uint32)), n
            assert np.array_equal(d.get(D2), d.get(D1)) and np.array_equal(d.get(U2), d.get(U1))
            ref = np.mean((pred.astype(np.float64) - tgt) ** 2)
            assert abs(float(loss[0]) - ref) <= 1e-6 * ref, n
        # without a unit gradient, and two posts back to back: the second waits for the first's copy
        pred = rng.standard_normal(4096).astype(np.float32)
        P, TG, DD, LA, LB = d.put(pred), d.put(np.zeros(4096, np.float32)), d.empty((4096,)), d.empty((1,)), d.empty((1,))
        d.call("om_mse_fwd_post", P, TG, DD, LA, None, C.c_int64(4096), r)
        d.call("om_mse_fwd_post", TG, TG, DD, LB, None, C.c_int64(4096), r)
        got = np.zeros(1, np.float32)
        assert L.om_readback_wait(r, got.ctypes.data, C.c_uint64(4)) == 0
        assert got[0] == 0.0 and d.get(LB)[0] == 0.0
        assert abs(float(d.get(LA)[0]) - np.mean(pred.astype(np.float64) ** 2)) <= 1e-6
        other = Dev()
        try:
            assert other.status("om_mse_fwd_post", P, TG, DD, LA, None, C.c_int64(4096), r) != 0
        finally:
            other.ctx.close()
        # refused: no readback, neither diff nor a unit gradient, an empty input; om_mse_fwd_unit without its unit
        assert d.status("om_mse_fwd_post", P, TG, DD, LA, None, C.c_int64(4096), None) != 0
        assert d.status("om_mse_fwd_post", P, TG, None, LA, None, C.c_int64(4096), r) != 0
        assert d.status("om_mse_fwd_post", P, TG, DD, LA, None, C.c_int64(0), r) != 0
        assert d.status("om_mse_fwd_unit", P, TG, DD, LA, None, C.c_int64(4096)) != 0
        # the readback still works after the refusals
        d.call("om_mse_fwd_post", P, TG, None, LA, DD, C.c_int64(4096), r)
        assert L.om_readback_wait(r, got.ctypes.data, C.c_uint64(4)) == 0
        assert got.view(np.uint32)[0] == d.get(LA).view(np.uint32)[0]
    finally:
        L.om_readback_destroy(r)
        d.ctx.close()


@pytest.mark.parametrize("rows,inf,outf", [(4096, 1536, 384), (4096, 3072, 768), (256, 64, 192), (100, 36, 20),
                                           (300, 96, 40)])
def test_linear_resid_mse_in_one_product(pkg, rows, inf, outf):
    """om_linear_fwd_resid_mse: y and the unit gradient bit for bit those of om_linear_fwd_resid followed by
    om_mse_fwd_unit, the loss within fp64 reordering of theirs (and of the float64 mean), and with a readback the same
    loss posted; shapes that take the epilogue (tile-exact products) and shapes that take the two calls."""
    from gpu_util import Dev
    d = Dev()
    L = d.ctx.L
    r = C.c_void_p()
    d.call("om_readback_create", C.c_uint64(4), C.byref(r))
    rng = np.random.default_rng(rows + inf + outf)
    try:
        x = rng.standard_normal((rows, inf)).astype(np.float32)
        w = (0.05 * rng.standard_normal((outf, inf))).astype(np.float32)
        b = rng.standard_normal(outf).astype(np.float32)
        res = rng.standard_normal((rows, outf)).astype(np.float32)
        tgt = rng.standard_normal((rows, outf)).astype(np.float32)
        X, W, B, R, TG = d.put(x), d.put(w), d.put(b), d.put(res), d.put(tgt)
        n = rows * outf
        Y1, L1, U1 = d.empty((rows, outf)), d.empty((1,)), d.empty((n,))
        d.call("om_linear_fwd_resid", X, W, B, R, Y1, rows, inf, outf)
        d.call("om_mse_fwd_unit", Y1, TG, None, L1, U1, C.c_int64(n))
        for post in (None, r):
            Y2, L2, U2 = d.empty((rows, outf)), d.empty((1,)), d.empty((n,))
            d.call("om_linear_fwd_resid_mse", X, W, B, R, TG, Y2, U2, L2, rows, inf, outf, post)
            assert np.array_equal(d.get(Y2).view(np.uint32), d.get(Y1).view(np.uint32))
            assert np.array_equal(d.get(U2).view(np.uint32), d.get(U1).view(np.uint32))
            l1, l2 = float(d.get(L1)[0]), float(d.get(L2)[0])
            assert abs(l2 - l1) <= 2.5e-7 * abs(l1), (l1, l2)
            ref = np.mean((d.get(Y1).astype(np.float64) - tgt) ** 2)
            assert abs(l2 - ref) <= 1e-6 * ref
            if post is not None:
                got = np.zeros(1, np.float32)
                assert L.om_readback_wait(r, got.ctypes.data, C.c_uint64(4)) == 0
                assert got[0] == np.float32(l2)
    finally:
        L.om_readback_destroy(r)
        d.ctx.close()
