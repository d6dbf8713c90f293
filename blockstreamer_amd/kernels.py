"""Tensor-level wrappers over the C ABI (one function per kernel family).

Each wrapper validates shapes and dtypes on the host, allocates outputs and
workspace from the torch caching allocator (so ``record_stream`` protection
of the caller applies), and launches on ``torch.cuda.current_stream()`` of
the tensors' device.  Nothing here synchronises the host.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib


def _as_u8(t: Tensor) -> Tensor:
    if t.dtype != torch.uint8:
        t = t.to(torch.uint8)
    return t if t.is_contiguous() else t.contiguous()


def dequantize_mxfp4(blocks: Tensor, scales: Tensor, dtype: torch.dtype = torch.bfloat16,
                     out: Tensor | None = None, mode: int = 0) -> Tensor:
    """Dense ``[E, G*32, R]`` weights from packed ``[E, R, G, 16]`` MXFP4.

    The transformers ``convert_moe_packed_tensors`` contract for a 4-D input
    (TF/integrations/mxfp4.py:257-313): bit-exact in bf16/f16/f32.
    """
    if blocks.dim() != 4 or blocks.shape[-1] != 16:
        raise ValueError(f"packed blocks must be [E, rows, groups, 16], got {tuple(blocks.shape)}")
    if tuple(scales.shape) != tuple(blocks.shape[:-1]):
        raise ValueError(
            f"scales shape {tuple(scales.shape)} does not match blocks {tuple(blocks.shape[:-1])}"
        )
    code = _lib.dtype_code(dtype)
    dev = _lib.require_gpu(blocks, scales)
    blocks = _as_u8(blocks)
    scales = _as_u8(scales)
    E, R, G, _ = blocks.shape
    if out is None:
        out = torch.empty((E, G * 32, R), dtype=dtype, device=dev)
    elif out.shape != (E, G * 32, R) or out.dtype != dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous [E, G*32, R] tensor of the requested dtype")
    with torch.cuda.device(dev):
        _lib.call("bsa_dequant_mxfp4_mode", blocks.data_ptr(), scales.data_ptr(), out.data_ptr(),
                  code, E, R, G, mode, _lib.stream_handle(dev))
    return out
