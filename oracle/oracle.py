"""ctypes bindings for the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP library.  Only
tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg import
this module.  Each wrapper takes numpy arrays (float32 / int64, C-contiguous)
and mirrors the argument order of the reference kernel it restates.
"""
from __future__ import annotations

import ctypes as ct
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

F = ct.POINTER(ct.c_float)
I = ct.POINTER(ct.c_int64)
i64 = ct.c_int64
f32 = ct.c_float
f64 = ct.c_double
u64 = ct.c_uint64


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []), check=True)
    return _LIB_PATH


class OrcConfig(ct.Structure):
    _fields_ = [(n, ct.c_int64) for n in (
        "sequence_len", "vocab_size", "n_layer", "n_head", "n_kv_head", "n_embd", "head_dim", "kv_dim")]


_SIGS = {
    "orc_embedding_fwd": [F, F, I, i64, i64],
    "orc_rmsnorm_fwd": [F, F, F, i64, i64],
    "orc_linear_fwd": [F, F, F, i64, i64, i64],
    "orc_rope_fwd": [F, F, F, F, i64, i64, i64],
    "orc_flash_attn_fwd": [F, F, F, F, F, i64, i64, i64, i64, i64],
    "orc_flash_attn_bwd_precompute_d": [F, F, F, i64, i64, i64, i64],
    "orc_flash_attn_bwd_dq": [F, F, F, F, F, F, F, i64, i64, i64, i64, i64],
    "orc_flash_attn_bwd_dkv": [F, F, F, F, F, F, F, F, i64, i64, i64, i64, i64],
    "orc_relu_squared_fwd": [F, F, i64],
    "orc_softcap_fwd": [F, F, f32, i64],
    "orc_ve_gate_fwd": [F, F, F, i64, i64, i64, i64],
    "orc_ve_apply_fwd": [F, F, F, i64, i64, i64],
    "orc_add_residual_fwd": [F, F, F, i64],
    "orc_scaled_add_fwd": [F, F, F, F, F, i64, i64],
    "orc_cross_entropy_fwd": [F, F, I, i64, i64],
    "orc_mean_reduce": [F, F, i64],
    "orc_cross_entropy_softcap_bwd": [F, F, I, f32, i64, i64, f32],
    "orc_linear_bwd_dx": [F, F, F, i64, i64, i64],
    "orc_linear_bwd_dw": [F, F, F, i64, i64, i64],
    "orc_rmsnorm_bwd": [F, F, F, F, i64, i64],
    "orc_rope_bwd": [F, F, F, F, i64, i64, i64],
    "orc_relu_squared_bwd": [F, F, F, i64],
    "orc_embedding_bwd": [F, F, I, i64, i64],
    "orc_scaled_add_bwd": [F, F, F, F, F, i64, i64],
    "orc_ve_apply_bwd": [F, F, F, F, F, i64, i64, i64],
    "orc_ve_gate_bwd": [F, F, F, F, F, F, i64, i64, i64, i64],
    "orc_scalar_grad_reduce": [F, F, F, i64, i64],
    "orc_zero_buffer": [F, i64],
    "orc_adamw": [F, F, F, F, f32, f32, f32, f32, f32, f32, f32, i64],
    "orc_nesterov_momentum": [F, F, F, f32, i64],
    "orc_normalize_frobenius": [F, i64],
    "orc_scale_add": [F, F, F, f32, f32, i64],
    "orc_muon_update": [F, F, f32, f32, i64],
    "orc_muon_step": [F, F, F, i64, i64, f64, f64, f64, f64],
    "orc_fill_normal": [F, u64, f32, i64],
    "orc_fill_uniform": [F, u64, f32, f32, i64],
    "orc_fill_zeros": [F, i64],
    "orc_fill_value": [F, f32, i64],
    "orc_precompute_rope": [F, F, i64, i64, f64],
}


def lib():
    global _lib
    if _lib is None:
        build()
        L = ct.CDLL(_LIB_PATH)
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = None
        L.orc_model_create.argtypes = [ct.POINTER(OrcConfig), i64, i64, i64]
        L.orc_model_create.restype = ct.c_void_p
        L.orc_model_destroy.argtypes = [ct.c_void_p]
        L.orc_model_init_weights.argtypes = [ct.c_void_p, u64]
        L.orc_model_num_tensors.argtypes = [ct.c_void_p]
        L.orc_model_num_tensors.restype = i64
        L.orc_model_tensor_info.argtypes = [ct.c_void_p, i64, I, ct.POINTER(ct.c_char_p)]
        L.orc_model_tensor_info.restype = i64
        L.orc_model_num_params.argtypes = [ct.c_void_p]
        L.orc_model_num_params.restype = i64
        L.orc_model_params.argtypes = [ct.c_void_p]
        L.orc_model_params.restype = F
        L.orc_model_grads.argtypes = [ct.c_void_p]
        L.orc_model_grads.restype = F
        L.orc_model_zero_grads.argtypes = [ct.c_void_p]
        L.orc_model_forward.argtypes = [ct.c_void_p, I, I]
        L.orc_model_forward.restype = f32
        L.orc_model_backward.argtypes = [ct.c_void_p, I, I, f32]
        L.orc_model_optimizer_step.argtypes = [ct.c_void_p, f64]
        L.orc_model_train_step.argtypes = [ct.c_void_p, I, I, f64]
        L.orc_model_train_step.restype = f32
        L.orc_model_token_loss.argtypes = [ct.c_void_p]
        L.orc_model_token_loss.restype = F
        L.orc_num_threads.restype = ct.c_int
        L.orc_model_scalar_grad_l1.argtypes = [ct.c_void_p, ct.POINTER(ct.c_double), ct.POINTER(ct.c_double)]
        _lib = L
    return _lib


def _p(a):
    """Pointer to a C-contiguous numpy array (float32 or int64)."""
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    if a.dtype == np.float32:
        return a.ctypes.data_as(F)
    if a.dtype == np.int64:
        return a.ctypes.data_as(I)
    raise TypeError(f"unsupported dtype {a.dtype}")


def call(name, *args):
    """Call orc_<name> converting numpy arrays to pointers."""
    conv = [(_p(a) if isinstance(a, np.ndarray) else a) for a in args]
    getattr(lib(), "orc_" + name)(*conv)


class Model:
    """Whole-model oracle: model.mojo + optimizer.mojo + train.mojo step."""

    def __init__(self, cfg: dict, B: int, T: int, rope_period: int = 0):
        L = lib()
        self.cfg = OrcConfig(**cfg)
        self.B, self.T = B, T
        self.h = L.orc_model_create(ct.byref(self.cfg), B, T, rope_period)
        self.n = L.orc_model_num_params(self.h)
        # held by the instance: at interpreter exit the module globals (lib,
        # _lib) may already be gone when __del__ runs
        self._destroy = L.orc_model_destroy

    def close(self):
        if getattr(self, "h", None):
            self._destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def init_weights(self, seed0: int = 42):
        lib().orc_model_init_weights(self.h, seed0)

    def tensors(self):
        L = lib()
        out = []
        for i in range(L.orc_model_num_tensors(self.h)):
            off = ct.c_int64()
            nm = ct.c_char_p()
            size = L.orc_model_tensor_info(self.h, i, ct.byref(off), ct.byref(nm))
            out.append((nm.value.decode(), off.value, size))
        return out

    def params(self) -> np.ndarray:
        return np.ctypeslib.as_array(lib().orc_model_params(self.h), shape=(self.n,))

    def grads(self) -> np.ndarray:
        return np.ctypeslib.as_array(lib().orc_model_grads(self.h), shape=(self.n,))

    def token_loss(self) -> np.ndarray:
        return np.ctypeslib.as_array(lib().orc_model_token_loss(self.h), shape=(self.B * self.T,))

    def zero_grads(self):
        lib().orc_model_zero_grads(self.h)

    def scalar_grad_l1(self):
        """(resid, x0) arrays of sum |g x| per layer from the last backward."""
        n = self.cfg.n_layer
        a, b = np.zeros(n), np.zeros(n)
        lib().orc_model_scalar_grad_l1(self.h, a.ctypes.data_as(ct.POINTER(ct.c_double)),
                                       b.ctypes.data_as(ct.POINTER(ct.c_double)))
        return a, b

    def forward(self, inputs: np.ndarray, targets: np.ndarray) -> float:
        return float(lib().orc_model_forward(self.h, _p(inputs), _p(targets)))

    def backward(self, inputs, targets, loss_scale: float = 1.0):
        lib().orc_model_backward(self.h, _p(inputs), _p(targets), loss_scale)

    def optimizer_step(self, progress: float = 0.0):
        lib().orc_model_optimizer_step(self.h, progress)

    def train_step(self, inputs, targets, progress: float = 0.0) -> float:
        return float(lib().orc_model_train_step(self.h, _p(inputs), _p(targets), progress))
