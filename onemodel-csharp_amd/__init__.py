"""onemodel-csharp_amd: MI355X (gfx950) kernels and training tape for OneModel's training path.

The product is native: lib/libom_hip.so (HIP kernels behind the C ABI of include/om.h) and lib/libom_train.so (the
C++ tape of include/om_train.h: modules, losses, Tensor.Backward, SGD/Adam/AdamW). This module is the ctypes
binding a Python caller (tests, bench.py) uses; it loads the in-tree libraries and raises if they are missing —
there is no fallback implementation.
"""
from __future__ import annotations

import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG, "lib")

vp = C.c_void_p
i32, i64, u64, f32 = C.c_int32, C.c_int64, C.c_uint64, C.c_float
ci = C.c_int


class om_batch(C.Structure):
    _fields_ = [("batch", i32), ("batch_div", i32), ("sa_outer", i64), ("sa_inner", i64), ("sb_outer", i64),
                ("sb_inner", i64), ("sc_outer", i64), ("sc_inner", i64)]


# name -> argument types (all return om_status unless listed in _RESTYPE)
_OM_SIGS = {
    "om_ctx_create": [ci, C.POINTER(vp)],
    "om_ctx_destroy": [vp],
    "om_ctx_sync": [vp],
    "om_last_error": [vp],
    "om_ctx_stream": [vp],
    "om_ctx_probe": [vp, ci],
    "om_ctx_set_gelu": [vp, ci],
    "om_ctx_probe_read": [vp, C.POINTER(ci), C.POINTER(C.c_double)],
    "om_abi_version": [],
    "om_build_checked": [],
    "om_arena_reserve": [vp, u64, u64],
    "om_alloc": [vp, ci, u64, C.POINTER(vp)],
    "om_step_reset": [vp],
    "om_arena_stats": [vp, ci, C.POINTER(u64), C.POINTER(u64)],
    "om_arena_set_limit": [vp, ci, u64],
    "om_upload": [vp, vp, vp, u64],
    "om_download": [vp, vp, vp, u64],
    "om_copy": [vp, vp, vp, u64],
    "om_zero": [vp, vp, u64],
    "om_fill": [vp, vp, f32, i64],
    "om_gemm": [vp, ci, ci, ci, ci, ci, vp, ci, vp, ci, vp, ci, vp, ci, C.POINTER(om_batch)],
    "om_linear_fwd": [vp, vp, vp, vp, vp, ci, ci, ci],
    "om_linear_small": [ci, ci, ci],
    "om_linear_bwd": [vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci],
    "om_linear_fwd_resid": [vp, vp, vp, vp, vp, vp, ci, ci, ci],
    "om_linear_fwd_resid_mse": [vp, vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, vp],
    "om_linear_relu_fwd": [vp, vp, vp, vp, vp, ci, ci, ci],
    "om_linear_bwd_dx_resid": [vp, vp, vp, vp, vp, ci, ci, ci],
    "om_mean_permute_fwd": [vp, vp, vp, ci, ci, ci, ci],
    "om_mean_permute_bwd": [vp, vp, vp, ci, ci, ci, ci, ci],
    "om_conv2d_relu_pool_fwd": [vp, vp, vp, vp, vp, vp, vp] + [ci] * 13,
    "om_linear_relu_bwd": [vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci],
    "om_linear_gelu_fwd": [vp, vp, vp, vp, vp, vp, ci, ci, ci],
    "om_linear_bwd_dx_gelu": [vp, vp, vp, vp, vp, ci, ci, ci],
    "om_linear_gelu_fwd_slope": [vp, vp, vp, vp, vp, vp, ci, ci, ci],
    "om_linear_bwd_dx_slope": [vp, vp, vp, vp, vp, ci, ci, ci],
    "om_linear_bwd_dw_group": [vp, ci, vp, ci],
    "om_param_grads_group": [vp, ci, vp, ci, ci, vp],
    "om_colsum": [vp, vp, vp, ci, ci, ci],
    "om_relu_fwd": [vp, vp, vp, i64],
    "om_relu_bwd": [vp, vp, vp, vp, i64, ci],
    "om_gelu_fwd": [vp, vp, vp, i64],
    "om_gelu_bwd": [vp, vp, vp, vp, i64, ci],
    "om_add": [vp, vp, vp, vp, i64],
    "om_add_rows": [vp, vp, vp, vp, ci, ci],
    "om_sub": [vp, vp, vp, vp, i64],
    "om_mul": [vp, vp, vp, vp, i64],
    "om_axpy": [vp, f32, vp, vp, i64],
    "om_scale": [vp, f32, vp, vp, i64],
    "om_permute": [vp, vp, vp, ci, vp, vp, ci],
    "om_mse_fwd": [vp, vp, vp, vp, vp, i64],
    "om_mse_fwd_unit": [vp, vp, vp, vp, vp, vp, i64],
    "om_mse_fwd_post": [vp, vp, vp, vp, vp, vp, i64, vp],
    "om_xent_fwd_unit": [vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, vp],
    "om_mse_bwd": [vp, vp, vp, vp, i64, ci],
    "om_sum_all": [vp, vp, vp, i64, ci],
    "om_sum_all_post": [vp, vp, vp, i64, ci, vp],
    "om_mean_axis": [vp, vp, vp, ci, ci, ci],
    "om_mean_axis_bwd": [vp, vp, vp, ci, ci, ci, ci],
    "om_mean_all_bwd": [vp, vp, vp, i64, ci],
    "om_relu_mean_rows": [vp, vp, vp, ci, ci],
    "om_relu_mean_rows_bwd": [vp, vp, vp, vp, ci, ci, ci],
    "om_layernorm_fwd": [vp, vp, vp, vp, vp, vp, vp, ci, ci, f32],
    "om_layernorm_bwd": [vp, vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci],
    "om_layernorm_bwd_add": [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci],
    "om_layernorm_bwd_chunks": [ci, ci],
    "om_layernorm_bwd_partials": [vp, vp, vp, vp, vp, vp, vp, vp, ci, vp, vp, ci, ci],
    "om_softmax_fwd": [vp, vp, vp, ci, ci],
    "om_softmax_bwd": [vp, vp, vp, vp, ci, ci, ci],
    "om_logsoftmax_fwd": [vp, vp, vp, ci, ci],
    "om_logsoftmax_bwd": [vp, vp, vp, vp, ci, ci, ci],
    "om_nll_fwd": [vp, vp, vp, vp, vp, ci, ci, ci, ci],
    "om_xent_bwd": [vp, vp, vp, vp, vp, ci, ci, ci, ci, ci],
    "om_nll_bwd": [vp, vp, vp, vp, ci, ci, ci, ci, ci],
    "om_attention_fwd": [vp, vp, vp, vp, vp, ci, vp, vp, ci, ci, ci, ci, ci, f32],
    "om_attention_bwd": [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, f32, ci],
    "om_attention_fwd_ld": [vp, vp, vp, vp, ci, vp, ci, vp, ci, vp, ci, ci, ci, ci, ci, f32],
    "om_attention_bwd_ld": [vp, vp, vp, vp, ci, vp, vp, ci, vp, vp, vp, ci, vp, ci, ci, ci, ci, ci, f32, ci],
    "om_attention_fwd_fused": [vp, vp, vp, vp, ci, vp, ci, vp, ci, ci, ci, ci, ci, f32],
    "om_attention_bwd_fused": [vp, vp, vp, vp, ci, vp, ci, vp, ci, vp, vp, vp, ci, ci, ci, ci, ci, f32, ci],
    "om_conv2d_fwd": [vp, vp, vp, vp, vp] + [ci] * 9,
    "om_conv2d_relu_fwd": [vp, vp, vp, vp, vp] + [ci] * 9,
    "om_conv2d_bwd": [vp, vp, vp, vp, vp, vp, vp] + [ci] * 9 + [ci, ci],
    "om_maxpool_fwd": [vp, vp, vp, vp] + [ci] * 10,
    "om_maxpool_bwd": [vp, vp, vp, vp] + [ci] * 12 + [ci],
    "om_maxpool_relu_bwd": [vp, vp, vp, vp, vp] + [ci] * 12 + [ci],
    "om_ctc_fwd": [vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci, ci, vp],
    "om_ctc_bwd": [vp, vp, vp, vp, vp, vp, vp, vp, ci, vp, vp, ci, ci, ci, ci, ci, ci],
    "om_ctc_tables_bytes": [ci, ci, ci],
    "om_ctc_fwd_tables": [vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci, ci, vp, vp, u64],
    "om_ctc_bwd_tables": [vp, vp, vp, vp, vp, vp, vp, vp, ci, vp, vp, ci, ci, ci, ci, ci, ci, vp, u64],
    "om_adam_step": [vp, vp, vp, vp, vp, vp, i64, f32, f32, f32, f32, f32, ci, f32, f32],
    "om_adam_scalars": [f32, f32, f32, i64, C.POINTER(f32), C.POINTER(f32)],
    "om_adam_step_scaled": [vp, vp, vp, vp, vp, vp, i64, f32, f32, f32, f32, f32, ci, f32, f32, vp],
    "om_sgd_step": [vp, vp, vp, vp, i64, f32, f32, f32, f32, ci, ci],
    "om_clip_grad_norm": [vp, ci, vp, vp, f32, ci, ci, vp, vp],
    "om_stager_create": [vp, u64, ci, C.POINTER(vp)],
    "om_readback_create": [vp, u64, C.POINTER(vp)],
    "om_readback_destroy": [vp],
    "om_readback_post": [vp, vp, u64],
    "om_readback_wait": [vp, vp, u64],
    "om_graph_capture_begin": [vp],
    "om_graph_capture_end": [vp, C.POINTER(vp)],
    "om_graph_capture_abort": [vp],
    "om_graph_launch": [vp, vp],
    "om_graph_destroy": [vp],
    "om_stager_destroy": [vp],
    "om_stager_slot_bytes": [vp],
    "om_stager_begin": [vp, C.POINTER(vp), C.POINTER(ci)],
    "om_stager_commit": [vp, ci, u64, C.POINTER(vp)],
    "om_stager_acquire": [vp, ci],
    "om_stager_release": [vp, ci],
    "om_avgpool2d_fwd": [vp, vp, vp, ci, ci, ci, ci, ci, ci, ci, ci, ci, ci],
    "om_avgpool2d_bwd": [vp, vp, vp, ci, ci, ci, ci, ci, ci, ci, ci, ci, ci, ci],
    "om_batchnorm2d_fwd": [vp, vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, f32, f32],
    "om_batchnorm2d_bwd": [vp, vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci],
    "om_embedding_fwd": [vp, vp, vp, vp, i64, ci, ci],
    "om_embedding_bwd": [vp, vp, vp, vp, i64, ci, ci, ci, ci],
    "om_dropout_fwd": [vp, vp, vp, i64, f32, u64, i64],
    "om_dropout_bwd": [vp, vp, vp, i64, f32, u64, i64, ci],
    "om_clip_grad_value": [vp, ci, vp, vp, f32],
    "om_layernorm_bwd_noalloc": [vp, vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci],
    "om_attention_fwd_flash": [vp, vp, vp, vp, ci, vp, ci, vp, ci, vp, ci, ci, ci, ci, f32],
    "om_attention_bwd_flash": [vp, vp, vp, vp, ci, vp, ci, vp, ci, vp, vp, ci, vp, vp, vp, ci, ci, ci, ci, ci, f32, ci],
}
_RESTYPE = {"om_last_error": C.c_char_p, "om_ctx_stream": vp, "om_abi_version": ci, "om_build_checked": ci,
            "om_adam_scalars": None,
            "om_ctc_tables_bytes": u64,
            "om_linear_small": ci,
            "om_layernorm_bwd_chunks": ci,
            "om_stager_slot_bytes": u64}

_HIP = None


class OmError(RuntimeError):
    """A failed library call; `code` is its status (OM_E_* / OMT_E_*) when there was one."""

    def __init__(self, message, code=None):
        super().__init__(message)
        self.code = code


def lib_path(name: str = "libom_hip.so") -> str:
    return os.path.join(LIB_DIR, name)


def load_hip():
    """Loads lib/libom_hip.so and declares every entry point of include/om.h. Raises if the library is missing."""
    global _HIP
    if _HIP is not None:
        return _HIP
    path = lib_path()
    if not os.path.exists(path):
        raise OmError(f"{path} is missing: build it with `python onemodel-csharp_amd/build.py`")
    L = C.CDLL(path)
    for name, args in _OM_SIGS.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, i32)
    _HIP = L
    return L


def om_symbols():
    return list(_OM_SIGS)


class om_linear_dw(C.Structure):
    _fields_ = [("g", vp), ("x", vp), ("dw", vp), ("db", vp), ("in_", i32), ("out", i32), ("acc_dw", i32),
                ("acc_db", i32)]


class om_column_sum(C.Structure):
    _fields_ = [("part", vp), ("out", vp), ("chunks", i32), ("cols", i32), ("acc", i32)]


class omt_scale(C.Structure):
    _fields_ = [("batch", i32), ("seq", i32), ("layers", i32), ("hw", i32)]


_OMT_SIGS = {
    "omt_config_create": ([ci, ci, C.POINTER(omt_scale), C.POINTER(vp)], i32),
    "omt_config_create_records": ([ci, ci, C.POINTER(omt_scale), ci, C.POINTER(vp)], i32),
    "omt_set_gelu": ([vp, ci], i32),
    "omt_destroy": ([vp], None),
    "omt_last_error": ([vp], C.c_char_p),
    "omt_step": ([vp, C.POINTER(f32)], i32),
    "omt_set_step_graph": ([vp, ci], i32),
    "omt_step_graph_ready": ([vp], ci),
    "omt_forward_backward": ([vp, C.POINTER(f32)], i32),
    "omt_forward": ([vp, C.POINTER(f32)], i32),
    "omt_backward": ([vp], i32),
    "omt_optimizer_step": ([vp], i32),
    "omt_ctx": ([vp], vp),
    "omt_param_count": ([vp], ci),
    "omt_param_info": ([vp, ci, C.c_char_p, ci, C.POINTER(ci), C.POINTER(i32)], i32),
    "omt_param_read": ([vp, ci, ci, vp, i64], i32),
    "omt_param_write": ([vp, ci, ci, vp, i64], i32),
    "omt_step_count": ([vp], i64),
    "omt_input_count": ([vp], ci),
    "omt_input_info": ([vp, ci, C.c_char_p, ci, C.POINTER(ci), C.POINTER(ci), C.POINTER(i32)], i32),
    "omt_input_read": ([vp, ci, vp, i64], i32),
    "omt_input_grad": ([vp, ci, vp, i64], i32),
    "omt_generate": ([u64, ci, f32, f32, vp, i64], None),
    "omt_input_write": ([vp, ci, vp, i64], i32),
    "omt_batch_bytes": ([vp], u64),
    "omt_batch_layout": ([vp, ci, C.POINTER(u64), C.POINTER(u64)], i32),
    "omt_batch_begin": ([vp, C.POINTER(vp)], i32),
    "omt_batch_commit": ([vp], i32),
    "omt_batch_queued": ([vp], ci),
    "omt_buffer_count": ([vp], ci),
    "omt_buffer_info": ([vp, ci, C.c_char_p, ci, C.POINTER(i64)], i32),
    "omt_buffer_read": ([vp, ci, vp, i64], i32),
    "omt_buffer_write": ([vp, ci, vp, i64], i32),
    "omt_set_optimizer": ([vp, ci, f32, f32, f32, f32, f32, f32, f32, ci, ci], i32),
    "omt_checkpoint_save": ([vp, C.c_char_p, ci, ci, C.POINTER(C.c_char_p), C.POINTER(i64)], i32),
    "omt_checkpoint_load": ([vp, C.c_char_p, ci, C.POINTER(ci)], i32),
    "omt_checkpoint_extra_count": ([vp], ci),
    "omt_checkpoint_extra": ([vp, ci, C.c_char_p, ci, C.POINTER(i64)], i32),
    "omt_checkpoint_check": ([C.c_char_p, vp, ci], i32),
    "omt_lr": ([vp], f32),
    "omt_set_lr": ([vp, f32], i32),
    "omt_lr_constant": ([f32, C.POINTER(vp)], i32),
    "omt_lr_step": ([f32, i64, f32, C.POINTER(vp)], i32),
    "omt_lr_cosine": ([f32, i64, f32, C.POINTER(vp)], i32),
    "omt_lr_warmup": ([vp, i64, f32, C.POINTER(vp)], i32),
    "omt_lr_warmup_cosine": ([f32, i64, i64, f32, C.POINTER(vp)], i32),
    "omt_lr_onecycle": ([f32, i64, f32, f32, f32, C.POINTER(vp)], i32),
    "omt_lr_free": ([vp], None),
    "omt_lr_at": ([vp, i64], f32),
    "omt_lr_cos": ([C.c_double], C.c_double),
    "omt_set_lr_schedule": ([vp, vp], i32),
    "omt_clip_grad_norm": ([vp, f32, ci, C.POINTER(f32)], i32),
    "omt_clip_grad_value": ([vp, f32], i32),
    "omt_set_clip": ([vp, f32, ci], i32),
    "omt_last_grad_norm": ([vp, C.POINTER(f32)], i32),
}
_TRAIN = None


def load_train():
    """Loads lib/libom_train.so (the C++ tape, linked against libom_hip.so). Raises if it is missing."""
    global _TRAIN
    if _TRAIN is not None:
        return _TRAIN
    load_hip()
    path = lib_path("libom_train.so")
    if not os.path.exists(path):
        raise OmError(f"{path} is missing: build it with `python onemodel-csharp_amd/build.py`")
    L = C.CDLL(path)
    for name, (args, res) in _OMT_SIGS.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _TRAIN = L
    return L


def omt_symbols():
    return list(_OMT_SIGS)


class Model:
    """One benchmark configuration on the device (include/om_train.h): `step()` is ZeroGrad + forward +
    loss.Backward() + AdamW.Step() and returns the loss."""

    def __init__(self, cfg: int, device: int = 0, batch=0, seq=0, layers=0, hw=0, per_op: bool = False):
        """per_op: build the reference's own record structure (omt_config_create_records, OMT_RECORDS_PER_OP)
        instead of the composite records."""
        import numpy as np
        self.np = np
        self.L = load_train()
        h = vp()
        sc = omt_scale(batch, seq, layers, hw)
        st = self.L.omt_config_create_records(device, cfg, C.byref(sc), 1 if per_op else 0, C.byref(h))
        if st != 0:
            raise OmError(f"omt_config_create({cfg}) failed ({st}): {self.L.omt_last_error(None).decode()}")
        self.h = h
        self.cfg = cfg

    def _check(self, st, what):
        if st != 0:
            raise OmError(f"{what} failed ({st}): {self.L.omt_last_error(self.h).decode()}", st)

    def step(self) -> float:
        v = f32()
        self._check(self.L.omt_step(self.h, C.byref(v)), "omt_step")
        return v.value

    def set_gelu(self, mode: int):
        """GELU epilogues of the feed-forward products: 0 fast (default), 1 the reference's polynomials bit for bit
        (omt_set_gelu)."""
        self._check(self.L.omt_set_gelu(self.h, int(mode)), "omt_set_gelu")

    def set_step_graph(self, on: bool = True):
        """Runs later step() calls from a recorded HIP graph of the step (omt_set_step_graph)."""
        self._check(self.L.omt_set_step_graph(self.h, int(bool(on))), "omt_set_step_graph")

    @property
    def step_graph_ready(self) -> bool:
        """True when the next step() replays a recorded graph."""
        return bool(self.L.omt_step_graph_ready(self.h))

    def forward_backward(self) -> float:
        v = f32()
        self._check(self.L.omt_forward_backward(self.h, C.byref(v)), "omt_forward_backward")
        return v.value

    def forward(self) -> float:
        """ZeroGrad + forward; the graph is kept for backward()."""
        v = f32()
        self._check(self.L.omt_forward(self.h, C.byref(v)), "omt_forward")
        return v.value

    def backward(self):
        """loss.Backward() over the last forward()'s graph (released afterwards)."""
        self._check(self.L.omt_backward(self.h), "omt_backward")

    def optimizer_step(self):
        self._check(self.L.omt_optimizer_step(self.h), "omt_optimizer_step")

    @property
    def ctx(self):
        return self.L.omt_ctx(self.h)

    def params(self):
        """[(name, shape)] in Parameters() order."""
        out = []
        for i in range(self.L.omt_param_count(self.h)):
            name = C.create_string_buffer(256)
            nd = ci()
            dims = (i32 * 8)()
            self._check(self.L.omt_param_info(self.h, i, name, 256, C.byref(nd), dims), "omt_param_info")
            out.append((name.value.decode(), tuple(dims[:nd.value])))
        return out

    def read_param(self, i, which=0):
        np = self.np
        shape = self.params()[i][1]
        a = np.empty(shape, np.float32)
        self._check(self.L.omt_param_read(self.h, i, which, a.ctypes.data, a.size), "omt_param_read")
        return a

    def write_param(self, i, values, which=0):
        np = self.np
        a = np.ascontiguousarray(values, np.float32)
        self._check(self.L.omt_param_write(self.h, i, which, a.ctypes.data, a.size), "omt_param_write")

    def inputs(self):
        """{name: numpy array} host copies of the synthetic inputs."""
        np = self.np
        out = {}
        for i in range(self.L.omt_input_count(self.h)):
            name = C.create_string_buffer(64)
            is_int, nd = ci(), ci()
            dims = (i32 * 8)()
            self._check(self.L.omt_input_info(self.h, i, name, 64, C.byref(is_int), C.byref(nd), dims), "input_info")
            a = np.empty(tuple(dims[:nd.value]), np.int32 if is_int.value else np.float32)
            self._check(self.L.omt_input_read(self.h, i, a.ctypes.data, a.size), "omt_input_read")
            out[name.value.decode()] = a
        return out

    def write_input(self, name, values):
        """Uploads a new value for a named input (the next step's batch)."""
        np = self.np
        names = [self._input_name(i) for i in range(self.L.omt_input_count(self.h))]
        i = names.index(name)
        a = np.ascontiguousarray(values)
        a = a.astype(np.int32 if a.dtype.kind in "iu" else np.float32, copy=False)
        self._check(self.L.omt_input_write(self.h, i, a.ctypes.data, a.size), "omt_input_write")

    def stage_batch(self, values):
        """Writes a batch {input name: array} into the next pinned staging slot and commits its upload (the next
        step consumes it); inputs not named keep the slot's previous contents."""
        np = self.np
        host = vp()
        self._check(self.L.omt_batch_begin(self.h, C.byref(host)), "omt_batch_begin")
        try:
            names = [self._input_name(i) for i in range(self.L.omt_input_count(self.h))]
            for name, v in values.items():
                i = names.index(name)
                off, nb = u64(), u64()
                self._check(self.L.omt_batch_layout(self.h, i, C.byref(off), C.byref(nb)), "omt_batch_layout")
                a = np.ascontiguousarray(v)
                a = a.astype(np.int32 if a.dtype.kind in "iu" else np.float32, copy=False)
                if a.nbytes != nb.value:
                    raise OmError(f"stage_batch: {name} has {a.nbytes} bytes, the model expects {nb.value}")
                C.memmove(host.value + off.value, a.ctypes.data, a.nbytes)
        finally:
            self._check(self.L.omt_batch_commit(self.h), "omt_batch_commit")

    def _input_name(self, i):
        name = C.create_string_buffer(64)
        self._check(self.L.omt_input_info(self.h, i, name, 64, None, None, None), "omt_input_info")
        return name.value.decode()

    def buffers(self):
        """{name: numpy array} of the model's state buffers (BatchNorm running statistics)."""
        np = self.np
        out = {}
        for i in range(self.L.omt_buffer_count(self.h)):
            name = C.create_string_buffer(256)
            n = i64()
            self._check(self.L.omt_buffer_info(self.h, i, name, 256, C.byref(n)), "omt_buffer_info")
            a = np.empty(n.value, np.float32)
            self._check(self.L.omt_buffer_read(self.h, i, a.ctypes.data, a.size), "omt_buffer_read")
            out[name.value.decode()] = a
        return out

    def set_optimizer(self, kind, lr, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0, momentum=0.0,
                      dampening=0.0, nesterov=False, amsgrad=False):
        """kind: "sgd", "adam" or "adamw" (a fresh optimizer over Parameters())."""
        k = {"sgd": 0, "adam": 1, "adamw": 2}[kind]
        self._check(self.L.omt_set_optimizer(self.h, k, lr, beta1, beta2, eps, weight_decay, momentum, dampening,
                                             int(nesterov), int(amsgrad)), "omt_set_optimizer")

    def input_grad(self, name):
        np = self.np
        ins = self.inputs()
        i = list(ins).index(name)
        a = np.empty(ins[name].shape, np.float32)
        self._check(self.L.omt_input_grad(self.h, i, a.ctypes.data, a.size), "omt_input_grad")
        return a

    @property
    def step_count(self):
        return self.L.omt_step_count(self.h)

    def save_checkpoint(self, path, optimizer=True, extra=None):
        """Checkpoint.Save of the model (and its optimizer); extra: {key: int}."""
        extra = extra or {}
        keys = (C.c_char_p * max(len(extra), 1))(*[k.encode() for k in extra])
        vals = (i64 * max(len(extra), 1))(*extra.values())
        self._check(self.L.omt_checkpoint_save(self.h, os.fsencode(path), int(optimizer), len(extra), keys, vals),
                    "omt_checkpoint_save")

    def load_checkpoint(self, path, optimizer=True):
        """Checkpoint.Load; returns (had_optimizer, extra). Raises CheckpointError with the failed check's kind."""
        had = ci()
        st = self.L.omt_checkpoint_load(self.h, os.fsencode(path), int(optimizer), C.byref(had))
        if st in CKPT_KINDS:
            raise CheckpointError(CKPT_KINDS[st], self.L.omt_last_error(self.h).decode())
        self._check(st, "omt_checkpoint_load")
        extra = {}
        for i in range(self.L.omt_checkpoint_extra_count(self.h)):
            k = C.create_string_buffer(256)
            v = i64()
            self._check(self.L.omt_checkpoint_extra(self.h, i, k, 256, C.byref(v)), "omt_checkpoint_extra")
            extra[k.value.decode()] = v.value
        return bool(had.value), extra

    @property
    def lr(self) -> float:
        return self.L.omt_lr(self.h)

    @lr.setter
    def lr(self, value: float):
        self._check(self.L.omt_set_lr(self.h, value), "omt_set_lr")

    def set_schedule(self, schedule):
        """LrSchedule.Apply before every optimizer step (None detaches)."""
        self._check(self.L.omt_set_lr_schedule(self.h, schedule.h if schedule is not None else None),
                    "omt_set_lr_schedule")

    def clip_grad_norm(self, max_norm: float, infinity_norm: bool = False) -> float:
        """GradClip.ClipNorm over Parameters() on the device, in place; returns the norm."""
        v = f32()
        self._check(self.L.omt_clip_grad_norm(self.h, max_norm, int(infinity_norm), C.byref(v)),
                    "omt_clip_grad_norm")
        return v.value

    def clip_grad_value(self, clip_value: float):
        self._check(self.L.omt_clip_grad_value(self.h, clip_value), "omt_clip_grad_value")

    def set_clip(self, max_norm: float, infinity_norm: bool = False):
        """ClipNorm inside step() (folded into AdamW); 0 switches it off."""
        self._check(self.L.omt_set_clip(self.h, max_norm, int(infinity_norm)), "omt_set_clip")

    def last_grad_norm(self) -> float:
        v = f32()
        self._check(self.L.omt_last_grad_norm(self.h, C.byref(v)), "omt_last_grad_norm")
        return v.value

    def close(self):
        if getattr(self, "h", None):
            self.L.omt_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


CKPT_KINDS = {16: "BadHeader", 17: "BadManifest", 18: "BadTensor", 19: "Mismatch", 20: "UnsupportedStream"}


class CheckpointError(OmError):
    """A checkpoint that is malformed or does not fit (CheckpointException); `kind` names the failed check."""

    def __init__(self, kind, message):
        super().__init__(f"{kind}: {message}")
        self.kind = kind


class omt_tensor_spec(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dtype", i32), ("ndim", i32), ("dims", C.POINTER(i32))]


def checkpoint_check(path, target):
    """Checks a checkpoint file against a model-state target [(name, "f32"|"i32"|"i64", shape)] on the host (no
    device), as a model-only load would; raises CheckpointError with the failed check's kind."""
    L = load_train()
    dt = {"f32": 0, "i32": 1, "i64": 2}
    keep = []
    specs = (omt_tensor_spec * max(len(target), 1))()
    for i, (name, dtype, shape) in enumerate(target):
        dims = (i32 * max(len(shape), 1))(*shape)
        keep.append(dims)
        specs[i] = omt_tensor_spec(name.encode(), dt[dtype], len(shape), dims)
    st = L.omt_checkpoint_check(os.fsencode(path), C.cast(specs, vp), len(target))
    if st in CKPT_KINDS:
        raise CheckpointError(CKPT_KINDS[st], L.omt_last_error(None).decode())
    if st != 0:
        raise OmError(f"omt_checkpoint_check failed ({st}): {L.omt_last_error(None).decode()}")


class LrSchedule:
    """A learning-rate schedule of libom_train.so (include/om_train.h): `LrSchedule.constant(...)`, `.step(...)`,
    `.cosine(...)`, `.warmup(inner, ...)`, `.warmup_cosine(...)`, `.onecycle(...)`; `lr_at(step)` is LrAt."""

    def __init__(self, make, *args):
        self.L = load_train()
        h = vp()
        st = getattr(self.L, make)(*args, C.byref(h))
        if st != 0:
            raise OmError(f"{make} failed ({st}): {self.L.omt_last_error(None).decode()}")
        self.h = h

    @classmethod
    def constant(cls, lr):
        return cls("omt_lr_constant", lr)

    @classmethod
    def step(cls, base_lr, step_size, gamma=0.1):
        return cls("omt_lr_step", base_lr, step_size, gamma)

    @classmethod
    def cosine(cls, base_lr, total_steps, min_lr=0.0):
        return cls("omt_lr_cosine", base_lr, total_steps, min_lr)

    @classmethod
    def warmup(cls, after, warmup_steps, start_factor=0.0):
        return cls("omt_lr_warmup", after.h, warmup_steps, start_factor)

    @classmethod
    def warmup_cosine(cls, base_lr, warmup_steps, total_steps, floor_fraction=0.0):
        return cls("omt_lr_warmup_cosine", base_lr, warmup_steps, total_steps, floor_fraction)

    @classmethod
    def onecycle(cls, max_lr, total_steps, pct_start=0.3, div_factor=25.0, final_div_factor=1e4):
        return cls("omt_lr_onecycle", max_lr, total_steps, pct_start, div_factor, final_div_factor)

    def lr_at(self, step: int) -> float:
        return self.L.omt_lr_at(self.h, step)

    def __del__(self):
        try:
            if self.h:
                self.L.omt_lr_free(self.h)
                self.h = None
        except Exception:
            pass


class Context:
    """An om_ctx on one device: calls go through `call(name, *args)`, which raises OmError with om_last_error."""

    def __init__(self, device: int = 0):
        self.L = load_hip()
        h = vp()
        st = self.L.om_ctx_create(device, C.byref(h))
        if st != 0:
            raise OmError(f"om_ctx_create failed ({st}): {self.L.om_last_error(None).decode()}")
        self.h = h

    def call(self, name, *args):
        st = getattr(self.L, name)(self.h, *args)
        if st != 0:
            raise OmError(f"{name} failed ({st}): {self.L.om_last_error(self.h).decode()}", st)

    @property
    def stream(self) -> int:
        return self.L.om_ctx_stream(self.h) or 0

    def sync(self):
        self.call("om_ctx_sync")

    def close(self):
        if self.h:
            self.L.om_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
