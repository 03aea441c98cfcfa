"""GPT training step over the C ABI (mirrors model.mojo / optimizer.mojo /
train.mojo: ModelWeights + ForwardBuffers + AdamWState + MuonState).

All state lives in device memory owned by the native ``ar_gpt`` object; this
class only forwards calls and exposes the flat parameter / gradient arenas as
torch tensor views for tests and benchmarks.
"""
from __future__ import annotations

import ctypes as ct
from dataclasses import dataclass

import torch

from ._lib import check, load

FP32, BF16 = 0, 1


@dataclass
class GPTConfig:
    """config.mojo:9-43 (GPTConfig); ``default`` follows its depth rule."""
    sequence_len: int
    vocab_size: int
    n_layer: int
    n_head: int
    n_kv_head: int
    n_embd: int
    head_dim: int
    kv_dim: int

    @staticmethod
    def default(vocab_size: int, depth: int) -> "GPTConfig":
        head_dim = 128
        model_dim = ((depth * 64 + head_dim - 1) // head_dim) * head_dim
        nh = model_dim // head_dim
        return GPTConfig(2048, vocab_size, depth, nh, nh, model_dim, model_dim // nh, nh * (model_dim // nh))

    def has_ve(self, i: int) -> bool:
        return i % 2 == (self.n_layer - 1) % 2

    def window_size(self, i: int) -> int:
        if i == self.n_layer - 1:
            return self.sequence_len
        return self.sequence_len // 2 if i % 4 < 3 else self.sequence_len

    def as_dict(self) -> dict:
        return dict(sequence_len=self.sequence_len, vocab_size=self.vocab_size, n_layer=self.n_layer,
                    n_head=self.n_head, n_kv_head=self.n_kv_head, n_embd=self.n_embd, head_dim=self.head_dim,
                    kv_dim=self.kv_dim)


class _CConfig(ct.Structure):
    _fields_ = [(n, ct.c_int64) for n in (
        "sequence_len", "vocab_size", "n_layer", "n_head", "n_kv_head", "n_embd", "head_dim", "kv_dim")]


class GPT:
    """One model + optimizer state on the current GPU.

    precision: FP32 (reference semantics) or BF16 (bf16 matrix-core compute,
    fp32 master weights).  rope_period: 0 = the reference's flat-token RoPE
    table rows (needs B*T <= 2048), T = per-sequence positions.
    """

    def __init__(self, cfg: GPTConfig, B: int, T: int, precision: int = FP32, rope_period: int = 0):
        self.lib = load()
        self.cfg, self.B, self.T = cfg, B, T
        self._c = _CConfig(**cfg.as_dict())
        h = ct.c_void_p()
        stream = torch.cuda.current_stream().cuda_stream
        check(self.lib.ar_gpt_create(ct.byref(h), ct.byref(self._c), B, T, precision, rope_period, stream),
              "gpt_create")
        self.h = h
        self.n = self.lib.ar_gpt_num_params(self.h)

    def close(self):
        if getattr(self, "h", None):
            self.lib.ar_gpt_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- arenas ----
    def _view(self, ptr: int) -> torch.Tensor:
        # Wrap device memory owned by the library as a torch tensor (no copy).
        return _DeviceArray(ptr, self.n).tensor()

    def params(self) -> torch.Tensor:
        return self._view(self.lib.ar_gpt_params(self.h))

    def grads(self) -> torch.Tensor:
        return self._view(self.lib.ar_gpt_grads(self.h))

    def tensors(self):
        out = []
        for i in range(self.lib.ar_gpt_num_tensors(self.h)):
            off = ct.c_int64()
            nm = ct.c_void_p()
            size = self.lib.ar_gpt_tensor_info(self.h, i, ct.byref(off), ct.byref(nm))
            out.append((ct.cast(nm, ct.c_char_p).value.decode(), off.value, size))
        return out

    def token_loss(self) -> torch.Tensor:
        return _DeviceArray(self.lib.ar_gpt_token_loss(self.h), self.B * self.T).tensor()

    # ---- step pieces ----
    def init_weights(self, seed0: int = 42):
        check(self.lib.ar_gpt_init_weights(self.h, seed0), "gpt_init_weights")

    def zero_grads(self):
        check(self.lib.ar_gpt_zero_grads(self.h), "gpt_zero_grads")

    def forward(self, inputs: torch.Tensor, targets: torch.Tensor) -> float:
        loss = ct.c_float()
        check(self.lib.ar_gpt_forward(self.h, _ptr(inputs), _ptr(targets), ct.byref(loss)), "gpt_forward")
        return loss.value

    def backward(self, inputs, targets, loss_scale: float = 1.0):
        check(self.lib.ar_gpt_backward(self.h, _ptr(inputs), _ptr(targets), loss_scale), "gpt_backward")

    def optimizer_step(self, progress: float = 0.0):
        check(self.lib.ar_gpt_optimizer_step(self.h, progress), "gpt_optimizer_step")

    def train_step(self, inputs, targets, progress: float = 0.0, sync_loss: bool = True):
        if sync_loss:
            loss = ct.c_float()
            check(self.lib.ar_gpt_train_step(self.h, _ptr(inputs), _ptr(targets), progress, ct.byref(loss)),
                  "gpt_train_step")
            return loss.value
        check(self.lib.ar_gpt_train_step(self.h, _ptr(inputs), _ptr(targets), progress, None), "gpt_train_step")
        return None

    def train_step_graph(self, inputs, targets, progress: float = 0.0, sync_loss: bool = True):
        """train_step replayed from a HIP graph (same buffers every call; the
        model must have been created on a non-default stream)."""
        loss = ct.c_float()
        check(self.lib.ar_gpt_train_step_graph(self.h, _ptr(inputs), _ptr(targets), progress,
                                               ct.byref(loss) if sync_loss else None), "gpt_train_step_graph")
        return loss.value if sync_loss else None


def _ptr(t: torch.Tensor) -> int:
    if not (t.is_cuda and t.dtype == torch.int64 and t.is_contiguous()):
        raise ValueError("token ids must be a contiguous int64 device tensor")
    return t.data_ptr()


class _DeviceArray:
    """Exposes library-owned float32 device memory as a torch tensor view."""

    def __init__(self, ptr: int, n: int):
        self.ptr, self.n = ptr, n

    @property
    def __cuda_array_interface__(self):
        return {"shape": (self.n,), "typestr": "<f4", "data": (self.ptr, False), "version": 2, "strides": None}

    def tensor(self) -> torch.Tensor:
        return torch.as_tensor(self, device="cuda")
