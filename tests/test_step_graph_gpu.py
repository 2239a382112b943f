"""Step graphs (omt_set_step_graph over om_graph_*): a training step recorded once into a HIP graph and replayed.

The bar is bit-identity with the same model stepped without graphs: the replayed launches are the recorded ones, and
the values that change per step (the rate, Adam's bias corrections, the loss readback's sequence number) are read by
the kernels from the graph's device block, formed on the host exactly as the eager step forms them. Every replay is
compared with the eager model, with eager work and host synchronisation (parameter reads) between replays, and the
graph is re-recorded where a recorded launch would go stale (a new optimizer, a new clip setting, new CTC lengths).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pkg():
    from gpu_util import load_pkg
    return load_pkg()


def _state(m, which=(0, 1, 2, 3)):
    n = len(m.params())
    return [m.read_param(i, w).view(np.uint32).copy() for w in which for i in range(n)]


def _same(a, b):
    sa, sb = _state(a), _state(b)
    assert len(sa) == len(sb)
    for k, (x, y) in enumerate(zip(sa, sb)):
        assert np.array_equal(x, y), f"tensor {k} differs"


def _bits(v):
    return np.float32(v).view(np.uint32)


CASES = [
    (1, {}),
    (2, {"batch": 4}),
    (3, {"batch": 4}),
    (4, {"batch": 4}),
    (5, {"batch": 1, "layers": 1, "seq": 128}),
    (7, {}),   # AdamW + CosineLr + ClipNorm inside the step, BatchNorm running statistics
    (8, {}),   # Adam + WarmupLr, Embedding
    (10, {}),  # a weight used twice
]


@pytest.mark.parametrize("cfg,sc", CASES, ids=[f"c{c}" for c, _ in CASES])
def test_replays_equal_eager_steps(pkg, cfg, sc):
    a, b = pkg.Model(cfg, **sc), pkg.Model(cfg, **sc)
    try:
        b.set_step_graph(True)
        ready = []
        for k in range(6):
            ready.append(b.step_graph_ready)
            la, lb = a.step(), b.step()
            assert _bits(la) == _bits(lb), f"step {k}: loss {la} vs {lb}"
            if k in (2, 5):
                _same(a, b)
        # step 0 runs outside a graph, step 1 is recorded, steps 2.. replay
        assert ready == [False, False, True, True, True, True]
        assert a.step_count == b.step_count == 6
        if cfg == 7:
            assert _bits(a.last_grad_norm()) == _bits(b.last_grad_norm())
            ba, bb = a.buffers(), b.buffers()
            assert list(ba) == list(bb) and ba
            for n in ba:
                assert np.array_equal(ba[n].view(np.uint32), bb[n].view(np.uint32)), n
    finally:
        a.close()
        b.close()


def test_eager_work_between_replays(pkg):
    """forward_backward / optimizer_step / a new rate between replays land in the replayed steps as in eager ones."""
    a, b = pkg.Model(3, batch=2), pkg.Model(3, batch=2)
    try:
        b.set_step_graph(True)
        for m in (a, b):
            for _ in range(3):
                m.step()
        assert b.step_graph_ready
        for m in (a, b):
            m.forward_backward()
            m.optimizer_step()
            m.lr = 5e-4
        _same(a, b)
        for k in range(3):
            assert _bits(a.step()) == _bits(b.step()), k
            _same(a, b)
        assert b.step_graph_ready
        assert a.lr == b.lr == np.float32(5e-4)
    finally:
        a.close()
        b.close()


def test_recorded_again_after_changes(pkg):
    """A new optimizer, a new clip setting and new CTC target lengths each drop the graph; the steps after them are
    recorded again and still equal the eager model's."""
    a, b = pkg.Model(4, batch=4), pkg.Model(4, batch=4)
    try:
        b.set_step_graph(True)
        for _ in range(3):
            assert _bits(a.step()) == _bits(b.step())
        assert b.step_graph_ready
        tl = b.inputs()["tgt_len"].copy()
        tl2 = np.roll(tl, 1).astype(np.int32)  # the same total, so the labels array keeps its size
        assert not np.array_equal(tl, tl2)
        for m in (a, b):
            m.write_input("tgt_len", tl2)
        assert not b.step_graph_ready
        for _ in range(3):
            assert _bits(a.step()) == _bits(b.step())
        _same(a, b)
        assert b.step_graph_ready
        for m in (a, b):
            m.set_optimizer("adam", 2e-3, weight_decay=0.001)  # Adam with L2 decay, fresh state
        assert not b.step_graph_ready
        for m in (a, b):
            m.set_clip(0.25)
        for _ in range(4):
            assert _bits(a.step()) == _bits(b.step())
        _same(a, b)
        assert b.step_graph_ready
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("cfg", [6, 9])
def test_models_that_run_without_graphs(pkg, cfg):
    """SGD (host-valued rate and first-step flags) and dropout (a new mask seed each step) never record a graph and
    step exactly as without the setting."""
    a, b = pkg.Model(cfg), pkg.Model(cfg)
    try:
        b.set_step_graph(True)
        for _ in range(4):
            assert _bits(a.step()) == _bits(b.step())
            assert not b.step_graph_ready
        _same(a, b)
    finally:
        a.close()
        b.close()


def test_switching_off(pkg):
    a, b = pkg.Model(1), pkg.Model(1)
    try:
        b.set_step_graph(True)
        for _ in range(3):
            a.step()
            b.step()
        b.set_step_graph(False)
        assert not b.step_graph_ready
        for _ in range(2):
            assert _bits(a.step()) == _bits(b.step())
        _same(a, b)
    finally:
        a.close()
        b.close()


def test_capture_refuses_host_waits(pkg):
    """Inside a capture, a call that would wait for the device fails with OM_E_STATE and the capture can be
    aborted; the context then runs launches again."""
    from gpu_util import Dev
    d = Dev()
    L = d.ctx.L
    x = d.put(np.arange(8, dtype=np.float32))
    assert L.om_graph_capture_begin(d.ctx.h) == 0
    host = np.zeros(8, np.float32)
    assert L.om_download(d.ctx.h, host.ctypes.data, x.data_ptr(), 32) == 4
    assert L.om_ctx_sync(d.ctx.h) == 4
    assert L.om_graph_capture_abort(d.ctx.h) == 0
    d.call("om_fill", x, 3.0, 8)
    assert np.array_equal(d.get(x), np.full(8, 3.0, np.float32))


def test_launch_probe(pkg):
    """om_ctx_probe brackets om_param_grads_group calls with events: one call per C3 step is recorded, none while
    the probe is off or inside a step graph's replays, and a new series starts from zero."""
    import ctypes as C
    m = pkg.Model(3, batch=2)
    try:
        L = pkg.load_hip()
        calls, ms = C.c_int(), C.c_double()
        assert L.om_ctx_probe(m.ctx, 1) == 0
        for _ in range(3):
            m.step()
        assert L.om_ctx_probe(m.ctx, 0) == 0
        m.step()  # not recorded
        assert L.om_ctx_probe_read(m.ctx, C.byref(calls), C.byref(ms)) == 0
        assert calls.value == 3 and 0.0 < ms.value < 100.0
        m.set_step_graph(True)
        assert L.om_ctx_probe(m.ctx, 1) == 0
        for _ in range(4):
            m.step()  # eager, recorded, then replays with no library calls
        assert L.om_ctx_probe_read(m.ctx, C.byref(calls), C.byref(ms)) == 0
        assert calls.value == 1  # only the first (eager) step; the capture records nothing
    finally:
        m.close()
