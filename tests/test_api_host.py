"""Host-side behaviour of the drop-in module that needs no GPU."""

from __future__ import annotations

import pytest
import torch

from blockstreamer_amd import gptoss


def test_dequantize_expert_requires_expert_dimension():
    """tests/test_offload.py:405-414: 3-D input raises ValueError("packed blocks")."""
    blocks = torch.randint(0, 255, (64, 4, 16), dtype=torch.uint8)
    scales = torch.randint(120, 134, (64, 4), dtype=torch.uint8)
    with pytest.raises(ValueError, match="packed blocks"):
        gptoss.dequantize_expert(blocks, scales)


def test_cpu_tensors_are_refused_loudly():
    blocks = torch.randint(0, 255, (1, 64, 4, 16), dtype=torch.uint8)
    scales = torch.randint(120, 134, (1, 64, 4), dtype=torch.uint8)
    with pytest.raises(ValueError, match="GPU only"):
        gptoss.dequantize_expert(blocks, scales)


def test_scale_shape_mismatch():
    blocks = torch.zeros(1, 8, 4, 16, dtype=torch.uint8)
    scales = torch.zeros(1, 8, 3, dtype=torch.uint8)
    with pytest.raises(ValueError, match="does not match"):
        gptoss.dequantize_expert(blocks, scales)
