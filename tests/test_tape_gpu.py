"""The tape's safety checks and the device arena (ActivationScope / BufferPool / SavedTensor), on the GPU.

- A tensor saved for the backward pass and written in place before the backward fails that backward with the code of
  TensorVersionException (SavedTensor.Unpack, Autograd.cs:222-237; BackwardEngineTests.cs:67-75); a write to a
  tensor no record saved (a bias, which only Add reads) does not.
- A second backward through a released graph fails (Engine.cs:136-141).
- forward() + backward() is the same computation as forward_backward(), bit for bit.
- The arena: a steady run allocates nothing new (AutogradModelTests.cs:179-212's "no growth" check, in bytes of the
  arena's regions), om_step_reset rewinds the step region, and a step that outgrows its slab chains another whose
  addresses stay valid until the reset (the ActivationScope.Dispose equivalent).
- A staged batch is returned when the step that took it fails, so the staging ring never runs dry.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

OM_E_STATE = 4
OMT_E_TENSOR_VERSION = 21


@pytest.fixture(scope="module")
def pkg():
    from gpu_util import load_pkg
    return load_pkg()


def _grads(m):
    return [m.read_param(i, 1).view(np.uint32).copy() for i in range(len(m.params()))]


def test_forward_then_backward_equals_forward_backward(pkg):
    a, b = pkg.Model(3, batch=2), pkg.Model(3, batch=2)
    try:
        la = a.forward_backward()
        lb = b.forward()
        b.backward()
        assert np.float32(la).view(np.uint32) == np.float32(lb).view(np.uint32)
        for x, y in zip(_grads(a), _grads(b)):
            assert np.array_equal(x, y)
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("how", ["param_write", "optimizer_step", "input_write"])
def test_saved_tensor_written_in_place_fails_the_backward(pkg, how):
    m = pkg.Model(1)
    try:
        names = [n for n, _ in m.params()]
        w = names.index("0.weight")  # saved by the first Linear's MatMul
        m.forward_backward()  # gradients exist, so the optimizer has something to update
        m.forward()
        if how == "param_write":
            m.write_param(w, m.read_param(w))  # the same values: a write is a modification (MutableData)
        elif how == "optimizer_step":
            m.optimizer_step()
        else:
            m.write_input("x", m.inputs()["x"])
        with pytest.raises(pkg.OmError) as e:
            m.backward()
        assert e.value.code == OMT_E_TENSOR_VERSION
        assert "modified in place (saved at version" in str(e.value)
        # a fresh forward saves the current versions: the next backward runs
        m.forward()
        m.backward()
    finally:
        m.close()


def test_ctc_labels_written_between_forward_and_backward(pkg):
    """The CTC loss reads the model's label and length inputs from their device copies, and saves them for the
    backward like the log-probabilities: rewriting the labels between forward and backward fails that backward."""
    m = pkg.Model(4, batch=4)
    try:
        ins = m.inputs()
        m.forward()
        m.write_input("labels", ins["labels"])
        with pytest.raises(pkg.OmError) as e:
            m.backward()
        assert e.value.code == OMT_E_TENSOR_VERSION
        a = m.forward_backward()
        b = m.forward_backward()
        assert a == b
    finally:
        m.close()


def test_write_to_an_unsaved_tensor_is_not_a_version_error(pkg):
    """The first layer's bias enters through Add, which saves nothing (BackwardOps.cs Add rule), so rewriting it
    between forward and backward is allowed, as in the reference."""
    m = pkg.Model(1)
    try:
        names = [n for n, _ in m.params()]
        bias = names.index("0.bias")
        ref = m.forward_backward()
        g_ref = _grads(m)
        m.forward()
        m.write_param(bias, m.read_param(bias))
        m.backward()
        assert ref == m.forward_backward()
        for x, y in zip(g_ref, _grads(m)):
            assert np.array_equal(x, y)
    finally:
        m.close()


def test_second_backward_through_a_released_graph_fails(pkg):
    m = pkg.Model(1)
    try:
        with pytest.raises(pkg.OmError) as e:
            m.backward()  # nothing to run backward through yet
        assert e.value.code == OM_E_STATE
        m.forward()
        m.backward()
        g1 = _grads(m)
        with pytest.raises(pkg.OmError) as e:
            m.backward()
        assert e.value.code == OM_E_STATE and "already freed" in str(e.value)
        for x, y in zip(g1, _grads(m)):  # the failed call wrote nothing
            assert np.array_equal(x, y)
        m.forward()  # a new forward records a new graph
        m.backward()
    finally:
        m.close()


def _arena(pkg, m):
    L = pkg.load_hip()
    out = {}
    for region in (0, 1):
        used, res = C.c_uint64(), C.c_uint64()
        assert L.om_arena_stats(m.ctx, region, C.byref(used), C.byref(res)) == 0
        out[region] = (used.value, res.value)
    return out


@pytest.mark.parametrize("cfg", [3, 4])
def test_steady_steps_allocate_nothing_new(pkg, cfg):
    m = pkg.Model(cfg)
    try:
        for _ in range(3):
            m.step()
        first = _arena(pkg, m)
        for _ in range(5):
            m.step()
            assert _arena(pkg, m) == first  # same bytes in use, nothing new reserved, in both regions
        assert first[1][0] > 0 and first[1][0] <= first[1][1]
    finally:
        m.close()


def test_step_reset_rewinds_and_chained_slabs_stay_valid(pkg):
    from gpu_util import DevBuf  # noqa: F401  (loads the HIP runtime the library uses)
    ctx = pkg.Context()
    L = ctx.L
    try:
        ctx.call("om_arena_reserve", C.c_uint64(0), C.c_uint64(1 << 20))

        def alloc(nbytes):
            p = C.c_void_p()
            ctx.call("om_alloc", 1, C.c_uint64(nbytes), C.byref(p))
            return p.value

        def stats():
            used, res = C.c_uint64(), C.c_uint64()
            ctx.call("om_arena_stats", 1, C.byref(used), C.byref(res))
            return used.value, res.value

        a = alloc(768 << 10)
        b = alloc(512 << 10)  # does not fit the 1 MiB slab: a second slab is chained
        used, res = stats()
        assert used == (768 + 512) << 10 and res > (1 << 20)
        assert a % 256 == 0 and b % 256 == 0
        na, nb = (768 << 10) // 4, (512 << 10) // 4
        ctx.call("om_fill", C.c_void_p(a), C.c_float(1.5), C.c_int64(na))
        ctx.call("om_fill", C.c_void_p(b), C.c_float(-2.0), C.c_int64(nb))
        ha, hb = np.empty(na, np.float32), np.empty(nb, np.float32)
        ctx.call("om_download", ha.ctypes.data_as(C.c_void_p), C.c_void_p(a), C.c_uint64(ha.nbytes))
        ctx.call("om_download", hb.ctypes.data_as(C.c_void_p), C.c_void_p(b), C.c_uint64(hb.nbytes))
        assert np.all(ha == 1.5) and np.all(hb == -2.0)  # both slabs' memory is live at once
        ctx.call("om_step_reset")
        assert stats() == (0, res)
        assert alloc(768 << 10) == a  # rewound to the start
        assert alloc(512 << 10) == b  # the chained slab is reused, not allocated again
        assert stats() == ((768 + 512) << 10, res)
        st = L.om_alloc(ctx.h, 2, C.c_uint64(16), C.byref(C.c_void_p()))
        assert st == 1  # no such region
    finally:
        ctx.close()


def test_failed_step_returns_its_staged_batch(pkg):
    """A backward that fails (here: a saved weight written in place) still returns the staged batch it took, so the
    three-slot ring keeps working and the inputs point at the model's own buffers again."""
    m = pkg.Model(1)
    try:
        names = [n for n, _ in m.params()]
        w = names.index("0.weight")
        ins = m.inputs()
        x, labels = ins["x"], ins["labels"]
        home = m.forward_backward()  # the model's own inputs
        L = pkg.load_train()
        for k in range(4):  # more failures than there are slots
            m.stage_batch({"x": x * (1.0 + k), "labels": labels})
            m.forward()
            m.write_param(w, m.read_param(w))
            with pytest.raises(pkg.OmError):
                m.backward()
            assert L.omt_batch_queued(m.h) == 0
        assert m.forward_backward() == home  # inputs point home again
        for k in range(3):  # the ring still takes a full set of batches
            m.stage_batch({"x": x, "labels": labels})
        for k in range(3):
            assert m.forward_backward() == home
    finally:
        m.close()


OM_E_OOM = 2
OM_REGION_STEP = 1


@pytest.mark.parametrize("cfg,sc,frac", [(3, {"batch": 4}, 0.3), (3, {"batch": 4}, 0.97), (4, {"batch": 4}, 0.6),
                                         (1, {}, 0.5), (5, {"batch": 1, "layers": 1}, 0.9)],
                         ids=["C3-forward", "C3-backward", "C4", "C1", "C5"])
def test_out_of_memory_mid_step_leaves_the_training_state_intact(pkg, cfg, sc, frac):
    """A device allocation that fails in the middle of a step (om_arena_set_limit caps the step region below what the
    step takes, so om_alloc returns OM_E_OOM there, as on a full device): the step fails with OM_E_OOM; parameters,
    Adam's moments and the step count are unchanged (the optimizer never ran); with the limit lifted the next step
    succeeds, and the run equals an undisturbed one bit for bit (the failed step left nothing behind that a later
    step reads)."""
    import ctypes as C
    a, b = pkg.Model(cfg, **sc), pkg.Model(cfg, **sc)
    try:
        L = pkg.load_hip()
        n = len(a.params())
        assert a.step() == b.step()
        used = C.c_uint64()
        assert L.om_arena_stats(b.ctx, OM_REGION_STEP, C.byref(used), None) == 0 and used.value > 0
        state = [[b.read_param(i, w) for w in (0, 2, 3)] for i in range(n)]
        assert L.om_arena_set_limit(b.ctx, OM_REGION_STEP, int(used.value * frac)) == 0
        with pytest.raises(pkg.OmError) as e:
            b.step()
        assert e.value.code == OM_E_OOM and "om_arena_set_limit" in str(e.value)
        assert b.step_count == 1
        for i in range(n):
            for w, before in zip((0, 2, 3), state[i]):
                assert np.array_equal(b.read_param(i, w).view(np.uint32), before.view(np.uint32)), (i, w)
        assert L.om_arena_set_limit(b.ctx, OM_REGION_STEP, 0) == 0
        for _ in range(2):
            assert a.step() == b.step()
        assert a.step_count == b.step_count == 3
        for i in range(n):
            for w in (0, 1, 2, 3):
                assert np.array_equal(a.read_param(i, w).view(np.uint32), b.read_param(i, w).view(np.uint32)), (i, w)
    finally:
        a.close()
        b.close()


def test_checked_build_hands_out_poisoned_memory(pkg):
    """In a checked build (om_build_checked) a fresh allocation reads as 0xFF bytes (a NaN for floats), so a kernel
    that computes from memory nothing wrote produces NaN; the product build leaves it as it is."""
    import ctypes as C
    L = pkg.load_hip()
    if not L.om_build_checked():
        pytest.skip("product build: allocations are not filled")
    ctx = pkg.Context(0)
    try:
        p = C.c_void_p()
        assert L.om_alloc(ctx.h, OM_REGION_STEP, 4096, C.byref(p)) == 0
        out = np.zeros(1024, np.uint32)
        assert L.om_download(ctx.h, out.ctypes.data, p, 4096) == 0
        assert np.all(out == 0xFFFFFFFF)
    finally:
        ctx.close()
