"""gpt-oss MXFP4 experts on MI355X: the drop-in for ``block_streamer.gptoss``.

Same public names, signatures, parameter names and error behaviour as
block_streamer/gptoss.py:1-189, so ``StreamedModel``'s ``functional_call``
binding (streamer.py:151-180), the LoRA recompute backward
(_autograd.py:125-175) and ``install_mxfp4_experts`` callers work unchanged.
The arithmetic runs in hand-written gfx950 HIP kernels (``libbsamd.so``).
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import kernels


def dequantize_expert(
    blocks: Tensor, scales: Tensor, dtype: torch.dtype = torch.bfloat16
) -> Tensor:
    """Dequantize one expert's packed MXFP4 weight to a dense matrix.

    block_streamer/gptoss.py:24-42: ``blocks`` is ``[1, rows, groups, 16]``
    uint8 and ``scales`` ``[1, rows, groups]``; returns ``[groups * 32, rows]``
    in ``dtype``.  A missing expert dimension raises ``ValueError`` whose
    message contains "packed blocks" (tests/test_offload.py:405-414).
    """
    if blocks.dim() != 4:
        raise ValueError(
            f"Expected [1, rows, groups, 16] packed blocks, got {tuple(blocks.shape)}"
        )
    dense = kernels.dequantize_mxfp4(blocks, scales, dtype)
    return dense.squeeze(0)
