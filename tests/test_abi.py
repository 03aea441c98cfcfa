"""CPU checks of the boundary: the built C-ABI library loads and exports every
function include/ar_ops.h declares (no compute calls: no GPU here)."""
import ctypes as ct
import os

import pytest

from autoresearch_amd import _lib

# Reference kernels (kernels/ops.mojo, optimizer.mojo, model.mojo) -> ABI names.
REFERENCE_KERNELS = {
    "embedding_fwd": "ar_embedding_fwd", "rmsnorm_fwd": "ar_rmsnorm_fwd", "linear_fwd": "ar_linear_fwd",
    "rope_fwd": "ar_rope_fwd", "flash_attn_fwd": "ar_flash_attn_fwd",
    "flash_attn_bwd_precompute_d": "ar_flash_attn_bwd_precompute_d", "flash_attn_bwd_dq": "ar_flash_attn_bwd_dq",
    "flash_attn_bwd_dkv": "ar_flash_attn_bwd_dkv", "relu_squared_fwd": "ar_relu_squared_fwd",
    "softcap_fwd": "ar_softcap_fwd", "ve_gate_fwd": "ar_ve_gate_fwd", "ve_apply_fwd": "ar_ve_apply_fwd",
    "add_residual_fwd": "ar_add_residual_fwd", "scaled_add_fwd": "ar_scaled_add_fwd",
    "softmax_fwd": "ar_softmax_fwd", "cross_entropy_fwd": "ar_cross_entropy_fwd", "mean_reduce": "ar_mean_reduce",
    "cross_entropy_softcap_bwd": "ar_cross_entropy_softcap_bwd", "linear_bwd_dx": "ar_linear_bwd_dx",
    "linear_bwd_dw": "ar_linear_bwd_dw", "rmsnorm_bwd": "ar_rmsnorm_bwd", "rope_bwd": "ar_rope_bwd",
    "relu_squared_bwd": "ar_relu_squared_bwd", "embedding_bwd": "ar_embedding_bwd",
    "scaled_add_bwd": "ar_scaled_add_bwd", "ve_apply_bwd": "ar_ve_apply_bwd", "ve_gate_bwd": "ar_ve_gate_bwd",
    "scalar_grad_reduce": "ar_scalar_grad_reduce", "zero_buffer": "ar_zero_buffer", "adamw_kernel": "ar_adamw",
    "nesterov_momentum_kernel": "ar_nesterov_momentum", "normalize_frobenius_kernel": "ar_normalize_frobenius",
    "scale_add_kernel": "ar_scale_add", "muon_update_kernel": "ar_muon_update",
    "fill_normal_kernel": "ar_fill_normal", "fill_uniform_kernel": "ar_fill_uniform",
    "fill_zeros_kernel": "ar_fill_zeros", "fill_value_kernel": "ar_fill_value",
    "precompute_rope": "ar_precompute_rope", "AdamWState.step_group": "ar_adamw_step_group",
    "MuonState.step": "ar_muon_step", "forward": "ar_gpt_forward", "backward": "ar_gpt_backward",
    "zero_grads": "ar_gpt_zero_grads", "init_weights": "ar_gpt_init_weights",
}


def test_library_built():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"


def test_header_symbols_exported():
    decls = _lib.parse_header()
    assert len(decls) >= 60
    lib = ct.CDLL(_lib.LIB_PATH)
    missing = [n for n in decls if not hasattr(lib, n)]
    assert not missing, missing


def test_every_reference_kernel_has_an_entry_point():
    decls = _lib.parse_header()
    missing = {k: v for k, v in REFERENCE_KERNELS.items() if v not in decls}
    assert not missing, missing


def test_load_sets_signatures():
    lib = _lib.load()
    assert lib.ar_version() == 2  # 2: caller-created workspaces (ar_workspace_*)
    assert lib.ar_gpt_create.restype is ct.c_int32
    assert lib.ar_gpt_params.restype is ct.c_void_p


def test_error_path_without_gpu():
    """Argument validation happens before any device work, so it runs here."""
    lib = _lib.load()
    st = lib.ar_linear_fwd(None, None, None, None, 8, 8, 8)
    assert st == -1
    assert b"null" in lib.ar_last_error()
    st = lib.ar_flash_attn_fwd(None, 16, 16, 16, 16, 16, 1, 8, 1, 256, 0)
    assert st in (-1, -2)
    st = lib.ar_workspace_create(None, 1 << 20)
    assert st == -1 and b"null" in lib.ar_last_error()
    assert lib.ar_workspace_bytes(None) == 0
    assert lib.ar_workspace_destroy(None) == 0


_NULL_PROBE = r"""
import ctypes as ct, json, sys
sys.path.insert(0, sys.argv[1])
from autoresearch_amd import _lib
lib = _lib.load()
out = {}
for h in _lib.HEADERS:
    for name, (res, args) in _lib.parse_header(h).items():
        vals = [None if a in (ct.c_void_p, ct.c_char_p) else 1.0 if a in (ct.c_float, ct.c_double)
                else 0 if a is ct.c_int32 else 8 for a in args]
        if name == "ar_last_error":
            continue
        r = getattr(lib, name)(*vals)
        out[name] = r
        print(name, r, flush=True)  # names the entry if the next call crashes
print("RESULT " + json.dumps(out))
"""


def test_every_entry_point_rejects_null_arguments():
    """Every function of the headers, called with null pointers (and small
    sizes): the status-returning entry points answer AR_EINVAL (-1) before
    any device work, the accessors 0 / -1 / NULL, and nothing dereferences a
    null handle.  Exceptions, each the documented behaviour: ar_version,
    unbinding (a null workspace) in ar_workspace_bind, which asks HIP for the
    current device (AR_EHIP without a GPU), and the destroy functions (no-op)."""
    import json
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _NULL_PROBE, root], capture_output=True, text=True, timeout=300)
    last = r.stdout.strip().splitlines()[-1:] or [""]
    assert r.returncode == 0, f"crashed after: {last[0]!r}\n{r.stderr[-2000:]}"
    res = json.loads(last[0][len("RESULT "):])
    special = {"ar_version", "ar_workspace_bind", "ar_workspace_destroy", "ar_gpt_destroy", "ar_loader_destroy",
               "ar_workspace_bytes", "ar_gpt_num_tensors", "ar_gpt_tensor_info", "ar_gpt_num_params",
               "ar_gpt_params", "ar_gpt_grads", "ar_gpt_token_loss", "ar_gpt_mean_loss"}
    bad = {n: v for n, v in res.items() if n not in special and v != -1}
    assert not bad, bad
    assert res["ar_version"] >= 1
    assert res["ar_workspace_bind"] in (0, -3)
    assert res["ar_workspace_destroy"] == res["ar_gpt_destroy"] == res["ar_loader_destroy"] == 0
    assert res["ar_workspace_bytes"] == res["ar_gpt_num_tensors"] == res["ar_gpt_num_params"] == 0
    assert res["ar_gpt_tensor_info"] == -1
    assert all(res[n] is None for n in ("ar_gpt_params", "ar_gpt_grads", "ar_gpt_token_loss", "ar_gpt_mean_loss"))
    assert len(res) > 70


_NEG_PROBE = r"""
import ctypes as ct, json, sys
sys.path.insert(0, sys.argv[1])
from autoresearch_amd import _lib
lib = _lib.load()
# opaque handles (model, loader, workspace) cannot be faked with a buffer
HANDLE = ("ar_gpt_", "ar_loader_", "ar_workspace_")
out = {}
bufs = []
for h in _lib.HEADERS:
    for name, (res, args) in _lib.parse_header(h).items():
        if res is not ct.c_int32 or name.startswith(HANDLE) and name != "ar_gpt_create":
            continue
        if not any(a is ct.c_int64 for a in args):
            continue
        vals = []
        for a in args:
            if a is ct.c_void_p:
                b = (ct.c_char * (1 << 16))()
                bufs.append(b)
                vals.append(ct.addressof(b))
            elif a is ct.c_char_p:
                vals.append(b"/nonexistent")
            elif a in (ct.c_float, ct.c_double):
                vals.append(1.0)
            elif a is ct.c_int32:
                vals.append(0)
            else:
                vals.append(-1)
        print(name, flush=True)
        out[name] = getattr(lib, name)(*vals)
print("RESULT " + json.dumps(out))
"""


def test_negative_sizes_are_rejected():
    """Every status-returning entry point that takes int64 sizes, called with
    host buffers for its pointers and -1 for every size: AR_EINVAL before
    any device work (a negative extent must never reach a launch)."""
    import json
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _NEG_PROBE, root], capture_output=True, text=True, timeout=300)
    last = r.stdout.strip().splitlines()[-1:] or [""]
    assert r.returncode == 0, f"crashed in: {last[0]!r}\n{r.stderr[-2000:]}"
    res = json.loads(last[0][len("RESULT "):])
    bad = {n: v for n, v in res.items() if v != -1}
    assert not bad, bad
    assert len(res) > 50


def test_gpt_config_default():
    from autoresearch_amd.model import GPTConfig
    c = GPTConfig.default(8192, 8)  # config.mojo:27-43
    assert (c.n_embd, c.n_head, c.head_dim, c.kv_dim, c.sequence_len) == (512, 4, 128, 512, 2048)
    assert [c.window_size(i) for i in range(8)] == [1024, 1024, 1024, 2048, 1024, 1024, 1024, 2048]
    assert [c.has_ve(i) for i in range(8)] == [False, True] * 4
    c12 = GPTConfig.default(8192, 12)
    assert (c12.n_embd, c12.n_head) == (768, 6)
