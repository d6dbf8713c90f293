"""Synthetic gpt-oss MoE layer inputs (for tests and benchmarks).

No checkpoint is needed: packed MXFP4 codes are uniform bytes (two independent
uniform nibbles), E8M0 scale bytes are uniform in ``[scale_lo, scale_hi]``,
activations are N(0, 1) in bfloat16, router weights N(0, 0.02) and biases as
the workload asks.  Everything is drawn from one seeded ``torch.Generator`` on
the requested device, so the same seed gives the same bytes on every run.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor


@dataclass(frozen=True)
class MoEShape:
    experts: int
    top_k: int
    hidden: int
    intermediate: int
    tokens: int


# The layer shapes the parity tests and the benchmark use.
TINY = MoEShape(8, 2, 256, 256, 64)              # gpt-oss-style tiny layer
GPTOSS_20B = MoEShape(32, 4, 2880, 2880, 2048)    # gpt-oss-20b layer, 2048 tokens
GPTOSS_120B_DECODE = MoEShape(128, 4, 2880, 2880, 64)
GPTOSS_120B_PREFILL = MoEShape(128, 4, 2880, 2880, 8192)


def _gen(device: torch.device | str, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def packed_weights(experts: int, rows: int, groups: int, *, seed: int, scale_lo: int,
                   scale_hi: int, device="cpu") -> tuple[Tensor, Tensor]:
    """Uniform packed bytes ``[E, rows, groups, 16]`` and scales ``[E, rows, groups]``."""
    g = _gen(device, seed)
    blocks = torch.randint(0, 256, (experts, rows, groups, 16), generator=g, dtype=torch.uint8,
                           device=device)
    scales = torch.randint(scale_lo, scale_hi + 1, (experts, rows, groups), generator=g,
                           dtype=torch.uint8, device=device)
    return blocks, scales


def moe_layer(shape: MoEShape, *, seed: int, scale_lo: int, scale_hi: int,
              router_bias_std: float = 0.0, dtype: torch.dtype = torch.bfloat16,
              device="cpu") -> dict[str, Tensor]:
    """All tensors of one MoE layer: activations, router and packed experts.

    Keys follow the checkpoint names of ``MXFP4Experts`` (gate_up_proj_*,
    down_proj_*) plus ``hidden``, ``router_weight`` and ``router_bias``.
    """
    E, H, I, T = shape.experts, shape.hidden, shape.intermediate, shape.tokens
    g = _gen(device, seed)
    out: dict[str, Tensor] = {}
    out["hidden"] = torch.randn(T, H, generator=g, device=device).to(dtype)
    out["router_weight"] = (torch.randn(E, H, generator=g, device=device) * 0.02).to(dtype)
    out["router_bias"] = (torch.randn(E, generator=g, device=device) * router_bias_std).to(dtype)
    out["gate_up_proj_blocks"] = torch.randint(0, 256, (E, 2 * I, H // 32, 16), generator=g,
                                               dtype=torch.uint8, device=device)
    out["gate_up_proj_scales"] = torch.randint(scale_lo, scale_hi + 1, (E, 2 * I, H // 32),
                                               generator=g, dtype=torch.uint8, device=device)
    out["gate_up_proj_bias"] = (torch.randn(E, 2 * I, generator=g, device=device) * 0.01).to(dtype)
    out["down_proj_blocks"] = torch.randint(0, 256, (E, H, I // 32, 16), generator=g,
                                            dtype=torch.uint8, device=device)
    out["down_proj_scales"] = torch.randint(scale_lo, scale_hi + 1, (E, H, I // 32), generator=g,
                                            dtype=torch.uint8, device=device)
    out["down_proj_bias"] = (torch.randn(E, H, generator=g, device=device) * 0.01).to(dtype)
    return out


def random_routing(tokens: int, experts: int, top_k: int, *, seed: int,
                   dtype: torch.dtype = torch.bfloat16, device="cpu") -> tuple[Tensor, Tensor]:
    """Distinct top-k expert indices per token and softmax routing weights."""
    g = _gen("cpu", seed)
    scores = torch.rand(tokens, experts, generator=g)
    idx = scores.argsort(dim=-1, descending=True)[:, :top_k].contiguous()
    w = torch.softmax(torch.randn(tokens, top_k, generator=g), dim=-1)
    return idx.to(device), w.to(dtype).to(device)
