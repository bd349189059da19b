"""ctypes binding of libviktor_hip.so (the C ABI declared in include/viktor_hip.h).

torch is imported first so that the library's HIP runtime dependency (soname libamdhip64.so.7)
resolves to the runtime torch already loaded: kernels launched through this binding run on torch's
streams and are recorded by torch.cuda graphs. There is no fallback: if the library is missing or the
device is not a ROCm GPU, every op raises.
"""

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libviktor_hip.so")

VK_OK = 0
VK_DTYPE_BF16 = 0
VK_DTYPE_F32 = 1

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F = ctypes.c_float

# name -> argument types (mirrors include/viktor_hip.h)
SIGNATURES = {
    "vk_version": [],
    "vk_last_error": [],
    "vk_device_cus": [],
    "vk_add_rmsnorm": [_P, _P, _P, _P, _I64, _I32, _F, _P],
    "vk_embed_rmsnorm": [_P, _P, _I64, _P, _P, _P, _I64, _I32, _F, _P],
    "vk_qkv_rope_cache": [_P, _P, _P, _I32, _P, _P, _I32, _I64, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P,
                          _I64, _F, _I32, _I32, _I32, _P],
    "vk_linear": [_P, _P, _P, _I64, _I32, _I32, _I32, _I32, _P, _P],
    "vk_swiglu": [_P, _P, _I64, _I32, _P],
    "vk_decode_attention": [_P, _P, _P, _P, _P, _I64, _P, _I64, _I32, _I32, _I32, _I64, _I64, _I64, _P, _I64, _P],
    "vk_decode_attention_workspace": [_I64, _I32, _I64, ctypes.POINTER(_I64)],
    "vk_decode_attention_noalloc": [_P, _P, _P, _P, _P, _I64, _P, _I64, _I32, _I32, _I32, _I64, _I64, _I64, _P],
    "vk_varlen_attention": [_P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I64, _P, _I32, _I32, _I32, _I32, _P, _P],
    "vk_varlen_attention_prefixed": [_P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I64, _P, _P, _P, _P, _I64, _P, _I32,
                                     _I32, _I32, _I32, _P, _P],
    "vk_select_update": [_P, _P, _P, _F, _P, _I32, _I32, _P, _P, _P, _I32, _F, _P, _I64, _I64, _I32, _P, _P, _P, _P, _P, _P,
                         _P, _I64, _I64, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _P],
    "vk_decode_attention_grouped": [_P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _I32,
                                    _I32, _I32, _I32, _P, _I64, _P],
    "vk_decode_attention_grouped_workspace": [_I64, _I32, _I64, _I64, ctypes.POINTER(_I64)],
    "vk_decode_attention_grouped_layout": [_I64, _I32, _I64, _I64, ctypes.POINTER(_I32), ctypes.POINTER(_I32)],
    "vk_norm_qkv_rope_cache": [_P, _P, _I64, _P, _P, _F, _P, _P, _P, _P, _P, _I32, _I64, _P, _P, _P, _P, _P, _P, _I64,
                               _I64, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _P, _P],
    "vk_linear_residual": [_P, _P, _P, _I64, _I32, _I32, _P, _P],
    "vk_norm_linear": [_P, _P, _F, _P, _P, _I64, _I32, _I32, _I32, _I32, _P, _P],
    "vk_gspo_score": [_P, _I32, _P, _P, _P, _P, _P, _F, _F, _F, _P, _P, _P, _P, _P, _I64, _I64, _I32, _P],
    "vk_group_advantage": [_P, _I64, _I32, _I32, _F, _P, _P, _P],
    "vk_attention_backward": [_P, _P, _P, _P, _P, _P, _P, _I32, _P, _I32, _P, _I32, _I64, _I64, _P, _P, _P, _P, _I32,
                              _I32, _I32, _P],
    "vk_attention_backward_prefixed": [_P, _P, _P, _P, _P, _P, _P, _I32, _P, _I32, _P, _I32, _I64, _I64, _P, _P, _P,
                                       _P, _I64, _I32, _P, _P, _P, _P, _I32, _I32, _I32, _P],
    "vk_wgrad": [_P, _I64, _P, _I64, _I64, _I32, _I32, _P, _I32, _P, _I64, _P],
    "vk_wgrad_workspace": [_I64, _I32, _I32, ctypes.POINTER(_I64)],
    "vk_bias_act": [_P, _P, _P, _P, _I64, _I32, _I32, _P],
    "vk_act_backward_blocks": [_I64, _I32, ctypes.POINTER(_I32)],
    "vk_act_backward": [_P, _P, _P, _P, _I32, _I64, _I32, _I32, _P],
    "vk_embed_grad_workspace": [_I64, _I32, _I32, ctypes.POINTER(_I64)],
    "vk_embed_grad": [_P, _I32, _I64, _P, _I64, _I32, _I32, _P, _P, _I64, _P],
    "vk_rmsnorm_backward_blocks": [_I64, ctypes.POINTER(_I32)],
    "vk_rmsnorm_backward": [_P, _I32, _P, _I32, _P, _I32, _P, _P, _P, _P, _I64, _I32, _F, _P],
    "vk_colsum": [_P, _P, _I32, _I32, _I32, _P],
    "vk_qknorm_rope_backward": [_P, _P, _P, _I32, _P, _P, _I32, _I64, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _F,
                                _P],
    "vk_swiglu_backward": [_P, _P, _P, _I64, _I32, _P],
    "vk_grad_norm_clip": [_P, _I64, _F, _P, _I32, _P, _P],
    "vk_adamw": [_P, _P, _P, _P, _I64, _P, _F, _F, _F, _F, _F, _I64, _P],
    "vk_strict_identity": [_P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _F, _P, _P, _P, _P],
    "vk_encoder_conv_first": [_P, _P, _P, _P, _P, _I32, _I64, _P, _P, _I32, _I32, _I32, _I32, _P, _P],
    "vk_encoder_conv": [_P, _I64, _P, _I32, _I32, _P, _P, _P, _P, _P, _I32, _I64, _I32, _P, _I64, _P],
    "vk_window_attention": [_P, _I64, _P, _P, _I32, _I32, _I32, _I32, _I32, _P, _P, _I32, _I32, _I32, _P, _I64, _P],
    "vk_deepnorm_rmsnorm": [_P, _P, _P, _F, _P, _F, _I64, _I32, _P],
    "vk_gemm_rows": [_P, _P, _P, _I64, _I32, _I32, _I32, _P],
    "vk_group_rows_equal": [_P, _I64, _I32, _I64, _P, _P],
    "vk_linear_residual_big": [_P, _P, _P, _I32, _I64, _I32, _I32, _P, _F, _P, _P, _P],
    "vk_rmsnorm_apply_ss": [_P, _I32, _P, _I32, _P, _I32, _P, _I64, _I32, _F, _P],
    "vk_rmsnorm_f32": [_P, _P, _P, _I64, _I32, _F, _P],
    "vk_timestamp": [_P, _I64, _P],
    "vk_timestamp_rate_khz": [ctypes.POINTER(_I64)],
    "vk_linear_qkv_rope": [_P, _P, _I64, _I32, _P, _P, _I32, _F, _P, _P, _I32, _I64, _P, _P, _P, _P, _I64, _P, _P, _I64, _I64,
                           _I64, _I64, _P, _P, _I64, _P, _I32, _I32, _I32, _P],
}

_lock = threading.Lock()
_lib = None


class HipLibraryError(RuntimeError):
    """The HIP kernel library is missing, failed to load, or a kernel call returned an error."""


def load(path=LIB_PATH):
    """Load (once) and return the ctypes handle of libviktor_hip.so. Raises HipLibraryError if absent."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise HipLibraryError(f"{path} is not built: run `python -m viktor_amd.build` (needs hipcc)")
        try:
            lib = ctypes.CDLL(path)
        except OSError as e:
            raise HipLibraryError(f"cannot load {path}: {e}") from e
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_char_p if name == "vk_last_error" else ctypes.c_int
        _lib = lib
        return lib


def exported_symbols():
    return list(SIGNATURES)


def check(rc, what):
    if rc != VK_OK:
        msg = load().vk_last_error().decode(errors="replace")
        raise HipLibraryError(f"{what} failed (status {rc}): {msg}")


def call(name, *args):
    """Call one C entry point and raise on a non-zero status."""
    rc = getattr(load(), name)(*args)
    check(rc, name)


def require_device(t: torch.Tensor, what: str):
    """The HIP path runs on ROCm devices only."""
    if not (t.is_cuda and torch.version.hip is not None):
        raise HipLibraryError(f"{what}: the HIP kernels need a tensor on a ROCm GPU (got {t.device})")


def stream_handle():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    """Device pointer of a tensor, or NULL for None."""
    return ctypes.c_void_p(0 if t is None else t.data_ptr())
