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
    "om_abi_version": [],
    "om_arena_reserve": [vp, u64, u64],
    "om_alloc": [vp, ci, u64, C.POINTER(vp)],
    "om_step_reset": [vp],
    "om_arena_stats": [vp, ci, C.POINTER(u64), C.POINTER(u64)],
    "om_upload": [vp, vp, vp, u64],
    "om_download": [vp, vp, vp, u64],
    "om_copy": [vp, vp, vp, u64],
    "om_zero": [vp, vp, u64],
    "om_fill": [vp, vp, f32, i64],
    "om_gemm": [vp, ci, ci, ci, ci, ci, vp, ci, vp, ci, vp, ci, vp, ci, C.POINTER(om_batch)],
    "om_linear_fwd": [vp, vp, vp, vp, vp, ci, ci, ci],
    "om_linear_bwd": [vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci],
    "om_colsum": [vp, vp, vp, ci, ci, ci],
    "om_relu_fwd": [vp, vp, vp, i64],
    "om_relu_bwd": [vp, vp, vp, vp, i64, ci],
    "om_gelu_fwd": [vp, vp, vp, i64],
    "om_gelu_bwd": [vp, vp, vp, vp, i64, ci],
    "om_add": [vp, vp, vp, vp, i64],
    "om_sub": [vp, vp, vp, vp, i64],
    "om_mul": [vp, vp, vp, vp, i64],
    "om_axpy": [vp, f32, vp, vp, i64],
    "om_scale": [vp, f32, vp, vp, i64],
    "om_sum_all": [vp, vp, vp, i64, ci],
    "om_mean_axis": [vp, vp, vp, ci, ci, ci],
    "om_mean_axis_bwd": [vp, vp, vp, ci, ci, ci, ci],
    "om_mean_all_bwd": [vp, vp, vp, i64, ci],
    "om_layernorm_fwd": [vp, vp, vp, vp, vp, vp, vp, ci, ci, f32],
    "om_layernorm_bwd": [vp, vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci],
    "om_softmax_fwd": [vp, vp, vp, ci, ci],
    "om_softmax_bwd": [vp, vp, vp, vp, ci, ci, ci],
    "om_logsoftmax_fwd": [vp, vp, vp, ci, ci],
    "om_logsoftmax_bwd": [vp, vp, vp, vp, ci, ci, ci],
    "om_nll_fwd": [vp, vp, vp, vp, vp, ci, ci, ci, ci],
    "om_xent_bwd": [vp, vp, vp, vp, vp, ci, ci, ci, ci, ci],
    "om_attention_fwd": [vp, vp, vp, vp, vp, ci, vp, vp, ci, ci, ci, ci, ci, f32],
    "om_attention_bwd": [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, f32, ci],
    "om_conv2d_fwd": [vp, vp, vp, vp, vp] + [ci] * 9,
    "om_conv2d_bwd": [vp, vp, vp, vp, vp, vp, vp] + [ci] * 9 + [ci, ci],
    "om_maxpool_fwd": [vp, vp, vp, vp] + [ci] * 10,
    "om_maxpool_bwd": [vp, vp, vp, vp] + [ci] * 12 + [ci],
    "om_ctc_fwd": [vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci, ci, vp],
    "om_ctc_bwd": [vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci, ci],
    "om_adam_step": [vp, vp, vp, vp, vp, vp, i64, f32, f32, f32, f32, f32, ci, f32, f32],
    "om_adam_scalars": [f32, f32, f32, i64, C.POINTER(f32), C.POINTER(f32)],
    "om_sgd_step": [vp, vp, vp, vp, i64, f32, f32, f32, f32, ci, ci],
}
_RESTYPE = {"om_last_error": C.c_char_p, "om_ctx_stream": vp, "om_abi_version": ci, "om_adam_scalars": None}

_HIP = None


class OmError(RuntimeError):
    pass


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
            raise OmError(f"{name} failed ({st}): {self.L.om_last_error(self.h).decode()}")

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
