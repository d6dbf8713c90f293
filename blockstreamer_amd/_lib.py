"""ctypes binding of ``libbsamd.so`` (the C ABI declared in include/bsamd.h).

The library is built in-tree by ``blockstreamer_amd.build``.  There is no
fallback: if the library is missing or a device tensor is not on a ROCm GPU,
the calls raise.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libbsamd.so"

BSA_OK, BSA_EINVAL, BSA_EHIP = 0, 1, 2
ABI_MAJOR = 3  # BSA_VERSION_MAJOR of include/bsamd.h: the signatures declared below
DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p
_f32 = ctypes.c_float

# name -> argtypes; every symbol returns int unless listed in _RESTYPE.
_SIGNATURES = {
    "bsa_last_error": [],
    "bsa_version": [],
    "bsa_dequant_mxfp4": [_ptr, _ptr, _ptr, _int, _i64, _i64, _i64, _ptr],
    "bsa_dequant_mxfp4_mode": [_ptr, _ptr, _ptr, _int, _i64, _i64, _i64, _int, _ptr],
    "bsa_dequant_mxfp4_layout": [_ptr, _ptr, _ptr, _int, _i64, _i64, _i64, _int, _int, _ptr],
    "bsa_mxfp4_to_kpair": [_ptr, _ptr, _i64, _i64, _i64, _ptr],
    "bsa_mxfp4_from_kpair": [_ptr, _ptr, _i64, _i64, _i64, _ptr],
    "bsa_moe_workspace_bytes": [_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_i64)],
    "bsa_moe_experts_fwd": [
        _ptr, _i64, _i64, _i64, _i64, _i64,      # hidden, T, H, I, E, k
        _ptr, _ptr, _int,                        # indices, weights, weight dtype
        _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _int,  # gate_up b/s/bias, down b/s/bias, bias dtype
        _f32, _f32,                              # alpha, limit
        _ptr, _int, _ptr, _i64, _ptr, _int,       # out, out dtype, ws, ws bytes, save, path
        _int, _ptr,                               # blocks layout, stream
    ],
    "bsa_moe_experts_fwd_noalloc": [
        _ptr, _i64, _i64, _i64, _i64, _i64,      # hidden, T, H, I, E, k
        _ptr, _ptr, _int,                        # indices, weights, weight dtype
        _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _int,  # gate_up b/s/bias, down b/s/bias, bias dtype
        _f32, _f32,                              # alpha, limit
        _ptr, _int, _ptr, _int,                  # out, out dtype, save, path
        _int, _ptr,                               # blocks layout, stream
    ],
    "bsa_moe_dispatch": [_ptr, _i64, _i64, _i64, _i64, _i64, _ptr, _i64, _ptr],
    "bsa_moe_gate_up": [_ptr, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr, _ptr, _int, _f32, _f32,
                        _ptr, _i64, _ptr, _int, _int, _ptr],
    "bsa_moe_down": [_i64, _i64, _i64, _i64, _i64, _ptr, _ptr, _ptr, _int, _ptr, _i64, _int, _int,
                     _ptr],
    "bsa_moe_combine": [_ptr, _ptr, _int, _i64, _i64, _i64, _i64, _i64, _ptr, _i64, _ptr, _int,
                        _ptr],
    "bsa_router_fwd": [_ptr, _int, _i64, _i64, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr],
    "bsa_router_topk": [_ptr, _int, _i64, _i64, _i64, _ptr, _ptr, _ptr],
    "bsa_quant_mxfp8": [_ptr, _int, _i64, _i64, _ptr, _ptr, _i64, _ptr],
    "bsa_quant_mxfp8_split": [_ptr, _int, _i64, _i64, _ptr, _ptr, _i64, _ptr],
    "bsa_mxfp4_matmul_workspace_bytes": [_i64, _i64, _i64, _int, _int, ctypes.POINTER(_i64)],
    "bsa_mxfp4_matmul": [_ptr, _int, _i64, _i64, _i64, _ptr, _ptr, _int, _int, _ptr, _int, _ptr, _i64, _ptr],
    "bsa_moe_bwd_workspace_bytes": [_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_i64)],
    "bsa_moe_experts_bwd": [
        _ptr, _int, _i64, _i64, _i64, _i64, _i64,  # grad_out, dtype, T, H, I, E, k
        _ptr, _ptr, _int,                          # indices, weights, weight dtype
        _ptr, _ptr, _ptr, _ptr,                    # gate_up b/s, down b/s
        _f32, _f32,                                # alpha, limit
        _ptr, _i64, _ptr, _ptr, _i64,              # ws, ws bytes, save, bwd ws, bwd bytes
        _ptr, _int, _ptr, _int, _ptr,              # grad_hidden, dtype, grad_weights, layout, stream
    ],
    "bsa_rmsnorm_fwd": [_ptr, _int, _i64, _i64, _ptr, _int, _f32, _ptr, _ptr],
    "bsa_rmsnorm_bwd": [_ptr, _ptr, _int, _i64, _i64, _ptr, _int, _f32, _ptr, _ptr],
    "bsa_attention_fwd": [
        _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,  # q, q strides, k, k strides, v, v strides, sinks
        _i64, _i64, _i64, _i64, _i64, _i64,        # B, Tq, Tk, Hq, Hkv, head_dim
        _int, _i64, _f32,                          # causal, window, scaling
        _ptr, _ptr, _ptr, _ptr,                    # out, out strides, lse, stream
    ],
    "bsa_attention_split_workspace_bytes": [_i64, _i64, _i64, _i64, _i64, _int, _i64],
    "bsa_attention_fwd_split": [
        _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,  # q, q strides, k, k strides, v, v strides, sinks
        _i64, _i64, _i64, _i64, _i64, _i64,        # B, Tq, Tk, Hq, Hkv, head_dim
        _int, _i64, _f32,                          # causal, window, scaling
        _ptr, _ptr, _ptr, _ptr, _i64, _ptr,        # out, out strides, lse, workspace, bytes, stream
    ],
    "bsa_attention_bwd": [
        _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,  # grad_out, q, k, v (each with strides)
        _ptr, _ptr, _ptr,                          # out, out strides, lse
        _i64, _i64, _i64, _i64, _i64, _i64,        # B, Tq, Tk, Hq, Hkv, head_dim
        _int, _i64, _f32,                          # causal, window, scaling
        _ptr, _ptr, _ptr, _ptr, _ptr,              # grad_q, grad_k, grad_v, row_dot, stream
    ],
}
_RESTYPE = {"bsa_last_error": ctypes.c_char_p, "bsa_attention_split_workspace_bytes": ctypes.c_int64}

_lib = None


def lib() -> ctypes.CDLL:
    """Load ``libbsamd.so`` once and declare its signatures."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m blockstreamer_amd.build`"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, args in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, ctypes.c_int)
        version = handle.bsa_version()
        if version // 100 != ABI_MAJOR:
            raise RuntimeError(f"{LIB_PATH} has ABI version {version}; this binding needs major version "
                               f"{ABI_MAJOR} (rebuild with `python -m blockstreamer_amd.build`)")
        _lib = handle
    return _lib


def symbols() -> list[str]:
    """Names of the C entry points this binding declares."""
    return list(_SIGNATURES)


def check(rc: int, what: str) -> None:
    """Raise for a non-zero status: ValueError for bad arguments, else RuntimeError."""
    if rc == BSA_OK:
        return
    msg = lib().bsa_last_error().decode(errors="replace")
    if rc == BSA_EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (status {rc})")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def stream_handle(device: torch.device) -> int:
    """The current torch stream of ``device`` as a raw hipStream_t."""
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one ROCm device; returns it.  No CPU path exists."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(
                "blockstreamer_amd runs on the GPU only: got a tensor on "
                f"{t.device}; move inputs to a ROCm device"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no device tensor given")
    return dev


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected bfloat16, float16 or float32")
