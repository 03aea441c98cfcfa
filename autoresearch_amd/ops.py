"""Reference-named operator surface over the C ABI (kernels/ops.mojo,
optimizer.mojo, model.mojo kernels).

Each function takes device tensors (torch, on the GPU) in the reference
kernel's argument order and meaning, launches on torch's current stream and
raises ``ArError`` where the reference would raise.  Tensors must be
contiguous float32 (int64 for indices).  Nothing here computes on the host.
"""
from __future__ import annotations

import torch

from ._lib import check, load

__all__ = [
    "Workspace", "embedding_fwd", "rmsnorm_fwd", "linear_fwd", "rope_fwd", "flash_attn_fwd",
    "flash_attn_bwd_precompute_d", "flash_attn_bwd_dq", "flash_attn_bwd_dkv", "relu_squared_fwd",
    "softcap_fwd", "ve_gate_fwd", "ve_apply_fwd", "add_residual_fwd", "scaled_add_fwd", "softmax_fwd",
    "cross_entropy_fwd", "mean_reduce", "cross_entropy_softcap_bwd", "linear_bwd_dx", "linear_bwd_dw",
    "rmsnorm_bwd", "rope_bwd", "relu_squared_bwd", "embedding_bwd", "scaled_add_bwd", "ve_apply_bwd",
    "ve_gate_bwd", "scalar_grad_reduce", "zero_buffer", "adamw_kernel", "adamw_step_group",
    "nesterov_momentum_kernel", "normalize_frobenius_kernel", "scale_add_kernel", "muon_update_kernel",
    "muon_step", "fill_normal_kernel", "fill_uniform_kernel", "fill_zeros_kernel", "fill_value_kernel",
    "precompute_rope",
]


def _stream():
    return torch.cuda.current_stream().cuda_stream


class Workspace:
    """Device scratch for the entry points that need some (ar_workspace_*).

    Created once by the host (it is the one allocation), then bound to the
    streams whose per-op calls should use it.  Calls on a stream with no
    workspace bound, or one too small, raise ``ArError`` naming the bytes
    they need; no call allocates behind the caller's back."""

    def __init__(self, nbytes: int):
        import ctypes as ct
        self._lib = load()
        h = ct.c_void_p()
        check(self._lib.ar_workspace_create(ct.byref(h), int(nbytes)), "workspace_create")
        self.h = h

    @property
    def nbytes(self) -> int:
        return int(self._lib.ar_workspace_bytes(self.h))

    def bind(self, stream=None):
        """Bind to `stream` (a torch stream, a raw handle, or None = torch's current stream)."""
        s = _stream() if stream is None else getattr(stream, "cuda_stream", stream)
        check(self._lib.ar_workspace_bind(s, self.h), "workspace_bind")
        return self

    def close(self):
        if getattr(self, "h", None):
            check(self._lib.ar_workspace_destroy(self.h), "workspace_destroy")
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _p(t: torch.Tensor | None):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("device tensor required (no CPU path)")
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    if t.dtype not in (torch.float32, torch.int64):
        raise TypeError(f"unsupported dtype {t.dtype}")
    return t.data_ptr()


def _call(name: str, *args):
    fn = getattr(load(), "ar_" + name)
    conv = [(_p(a) if isinstance(a, torch.Tensor) else a) for a in args]
    check(fn(_stream(), *conv), name)


def _sfx(bf16: bool) -> str:
    return "_bf16" if bf16 else ""


# ---- kernels/ops.mojo ----
def embedding_fwd(output, weight, indices, num_tokens, embd_dim):
    _call("embedding_fwd", output, weight, indices, num_tokens, embd_dim)


def rmsnorm_fwd(output, rms_out, input, num_rows, dim):
    _call("rmsnorm_fwd", output, rms_out, input, num_rows, dim)


def linear_fwd(output, input, weight, M, N, K, bf16=False):
    _call("linear_fwd" + _sfx(bf16), output, input, weight, M, N, K)


def rope_fwd(output, input, cos_buf, sin_buf, num_tokens, num_heads, head_dim):
    _call("rope_fwd", output, input, cos_buf, sin_buf, num_tokens, num_heads, head_dim)


def flash_attn_fwd(output, lse_out, q, k, v, B, T, num_heads, head_dim, window_size, bf16=False):
    _call("flash_attn_fwd" + _sfx(bf16), output, lse_out, q, k, v, B, T, num_heads, head_dim, window_size)


def flash_attn_bwd_precompute_d(d_out, output, grad_output, B, T, num_heads, head_dim, bf16=False):
    _call("flash_attn_bwd_precompute_d" + _sfx(bf16), d_out, output, grad_output, B, T, num_heads, head_dim)


def flash_attn_bwd_dq(grad_q, q, k, v, grad_output, lse, d_buf, B, T, num_heads, head_dim, window_size, bf16=False):
    _call("flash_attn_bwd_dq" + _sfx(bf16), grad_q, q, k, v, grad_output, lse, d_buf, B, T, num_heads, head_dim,
          window_size)


def flash_attn_bwd_dkv(grad_k, grad_v, q, k, v, grad_output, lse, d_buf, B, T, num_heads, head_dim, window_size,
                       bf16=False):
    _call("flash_attn_bwd_dkv" + _sfx(bf16), grad_k, grad_v, q, k, v, grad_output, lse, d_buf, B, T, num_heads,
          head_dim, window_size)


def relu_squared_fwd(output, input, size):
    _call("relu_squared_fwd", output, input, size)


def softcap_fwd(output, input, cap, size):
    _call("softcap_fwd", output, input, cap, size)


def ve_gate_fwd(gate_out, x_norm, gate_weight, num_tokens, n_kv_head, gate_channels, embd_dim):
    _call("ve_gate_fwd", gate_out, x_norm, gate_weight, num_tokens, n_kv_head, gate_channels, embd_dim)


def ve_apply_fwd(v, gate, ve, num_tokens, n_kv_head, head_dim):
    _call("ve_apply_fwd", v, gate, ve, num_tokens, n_kv_head, head_dim)


def add_residual_fwd(output, residual, input, size):
    _call("add_residual_fwd", output, residual, input, size)


def scaled_add_fwd(output, a, b, scale_a, scale_b, idx, size):
    _call("scaled_add_fwd", output, a, b, scale_a, scale_b, idx, size)


def softmax_fwd(output, input, num_rows, cols):
    _call("softmax_fwd", output, input, num_rows, cols)


def cross_entropy_fwd(loss_out, logits, targets, num_tokens, vocab_size):
    _call("cross_entropy_fwd", loss_out, logits, targets, num_tokens, vocab_size)


def mean_reduce(output, input, size):
    _call("mean_reduce", output, input, size)


def cross_entropy_softcap_bwd(grad_logits, logits, targets, cap, num_tokens, vocab_size, loss_scale):
    _call("cross_entropy_softcap_bwd", grad_logits, logits, targets, cap, num_tokens, vocab_size, loss_scale)


def linear_bwd_dx(grad_input, grad_output, weight, M, N, K, bf16=False):
    _call("linear_bwd_dx" + _sfx(bf16), grad_input, grad_output, weight, M, N, K)


def linear_bwd_dw(grad_weight, grad_output, input, M, N, K, bf16=False):
    _call("linear_bwd_dw" + _sfx(bf16), grad_weight, grad_output, input, M, N, K)


def rmsnorm_bwd(grad_input, grad_output, input, rms_saved, num_rows, dim):
    _call("rmsnorm_bwd", grad_input, grad_output, input, rms_saved, num_rows, dim)


def rope_bwd(grad_input, grad_output, cos_buf, sin_buf, num_tokens, num_heads, head_dim):
    _call("rope_bwd", grad_input, grad_output, cos_buf, sin_buf, num_tokens, num_heads, head_dim)


def relu_squared_bwd(grad_input, grad_output, input, size):
    _call("relu_squared_bwd", grad_input, grad_output, input, size)


def embedding_bwd(grad_weight, grad_output, indices, num_tokens, embd_dim):
    _call("embedding_bwd", grad_weight, grad_output, indices, num_tokens, embd_dim)


def scaled_add_bwd(grad_a, grad_b, grad_output, scale_a, scale_b, idx, size):
    _call("scaled_add_bwd", grad_a, grad_b, grad_output, scale_a, scale_b, idx, size)


def ve_apply_bwd(grad_ve, grad_gate, grad_v, gate, ve, num_tokens, n_kv_head, head_dim):
    _call("ve_apply_bwd", grad_ve, grad_gate, grad_v, gate, ve, num_tokens, n_kv_head, head_dim)


def ve_gate_bwd(grad_x_norm_out, grad_gate_weight, grad_gate, gate, x_norm, gate_weight, num_tokens, n_kv_head,
                gate_channels, embd_dim):
    _call("ve_gate_bwd", grad_x_norm_out, grad_gate_weight, grad_gate, gate, x_norm, gate_weight, num_tokens,
          n_kv_head, gate_channels, embd_dim)


def scalar_grad_reduce(grad_scalar, grad_output, input, idx, size):
    _call("scalar_grad_reduce", grad_scalar, grad_output, input, idx, size)


def zero_buffer(buf, size):
    _call("zero_buffer", buf, size)


# ---- optimizer.mojo ----
def adamw_kernel(params, grads, exp_avg, exp_avg_sq, lr, beta1, beta2, eps, weight_decay, bias_corr1, bias_corr2,
                 size):
    _call("adamw", params, grads, exp_avg, exp_avg_sq, lr, beta1, beta2, eps, weight_decay, bias_corr1, bias_corr2,
          size)


def adamw_step_group(params, grads, exp_avg, exp_avg_sq, size, lr, beta1, beta2, eps, weight_decay, lr_multiplier,
                     step):
    _call("adamw_step_group", params, grads, exp_avg, exp_avg_sq, size, lr, beta1, beta2, eps, weight_decay,
          lr_multiplier, step)


def nesterov_momentum_kernel(output, grads, momentum_buf, momentum, size):
    _call("nesterov_momentum", output, grads, momentum_buf, momentum, size)


def normalize_frobenius_kernel(data, size):
    _call("normalize_frobenius", data, size)


def scale_add_kernel(output, a, b, sa, sb, size):
    _call("scale_add", output, a, b, sa, sb, size)


def muon_update_kernel(params, grads, lr, wd, size):
    _call("muon_update", params, grads, lr, wd, size)


def muon_step(params, grads, momentum_buf, rows, cols, initial_lr, lr_multiplier, momentum, weight_decay,
              bf16=False):
    _call("muon_step", params, grads, momentum_buf, rows, cols, initial_lr, lr_multiplier, momentum, weight_decay,
          1 if bf16 else 0)


# ---- model.mojo init ----
def fill_normal_kernel(output, seed_base, std, size):
    _call("fill_normal", output, seed_base, std, size)


def fill_uniform_kernel(output, seed_base, low, high, size):
    _call("fill_uniform", output, seed_base, low, high, size)


def fill_zeros_kernel(output, size):
    _call("fill_zeros", output, size)


def fill_value_kernel(output, value, size):
    _call("fill_value", output, value, size)


def precompute_rope(cos_buf, sin_buf, seq_len, head_dim, base=10000.0):
    _call("precompute_rope", cos_buf, sin_buf, seq_len, head_dim, base)
