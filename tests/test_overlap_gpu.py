"""Overlap mode of the backward (om_ctx_set_overlap), on the GPU.

Overlap mode moves weight-gradient products to a second stream beside the input-gradient chain. It may not change
a bit: training runs with the mode on equal the serial run in losses, parameters, gradients and moments.
"""
import os

import numpy as np
import pytest

from conftest import load_golden

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pkg():
    from gpu_util import load_pkg
    return load_pkg()


def make(pkg, cfg, mode, **kw):
    """A model whose context is made with OMT_OVERLAP set for `mode` (read once, at creation)."""
    saved = {k: os.environ.get(k) for k in ("OMT_OVERLAP",)}
    os.environ["OMT_OVERLAP"] = "1" if mode == "overlap" else "0"
    try:
        return pkg.Model(cfg, **kw)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def state(m):
    return [m.read_param(i, w).view(np.uint32).copy() for i in range(len(m.params())) for w in (0, 1, 2, 3)]


def run(m, cfg, steps):
    if cfg == 9:
        o = load_golden("training_encoder")
        ids = o["in.ids"].astype(np.int32)
        out = []
        for i in range(steps):
            idx = o["in.order"][i].astype(int)
            m.write_input("ids", ids[idx])
            m.write_input("labels", o["in.y"][idx].astype(np.int32))
            out.append(m.step())
        return out
    return [m.step() for _ in range(steps)]


@pytest.mark.parametrize("cfg,kw,steps", [(3, {"batch": 4}, 4), (9, {}, 6)], ids=["c3-block", "encoder-dropout"])
def test_modes_equal_the_serial_run(pkg, cfg, kw, steps):
    models = {mode: make(pkg, cfg, mode, **kw) for mode in ("serial", "overlap")}
    try:
        losses = {mode: np.array(run(m, cfg, steps), np.float32) for mode, m in models.items()}
        ref = state(models["serial"])
        for mode in ("overlap",):
            assert np.array_equal(losses[mode].view(np.uint32), losses["serial"].view(np.uint32)), mode
            for a, b in zip(state(models[mode]), ref):
                assert np.array_equal(a, b), mode
    finally:
        for m in models.values():
            m.close()

