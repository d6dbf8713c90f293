"""The no-allocation forward (bsa_moe_experts_fwd_noalloc) against the
workspace forward (bsa_moe_experts_fwd), through the C ABI.

The entry point takes its workspace from the library's static per-GPU
scratch instead of the caller.  It runs the same kernels, so its output must
equal the workspace entry point's bit for bit.  Two calls run back to back,
the second on a smaller batch, so the second reads a scratch that still holds
the first call's larger contents.  Shapes: the gpt-oss-120b decode layer
(128 experts, top-4, hidden = intermediate = 2880) at 64 then 8 tokens (the
weight-streaming kernels); a gpt-oss-20b-shaped layer (32 experts, top-4) at
200 then 150 tokens, whose 25 and 19 rows per expert take the MX prefill
kernels; and the tiny layer (8 experts, top-2, 256 wide) at 300 then 100
tokens on the bf16 tiled kernels.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from blockstreamer_amd import kernels, synthetic
from tests.conftest import announce
from tests.moe_util import assert_layer_close, expert_args, oracle_tokens

pytestmark = pytest.mark.gpu


def _layer(shape, seed, device):
    t = synthetic.moe_layer(shape, seed=seed, scale_lo=115, scale_hi=131, router_bias_std=0.5,
                            device=device)
    _, scores, idx = oracle.router_ref(t["hidden"].cpu().float(), t["router_weight"].cpu().float(),
                                       t["router_bias"].cpu().float(), shape.top_k)
    return t, idx.to(device), scores.to(device)


def _same_bits(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("path", ["auto", "tiled"])
def test_noalloc_equals_workspace_forward_twice(device, path):
    big = synthetic.GPTOSS_120B_DECODE                       # 64 tokens
    small = synthetic.MoEShape(big.experts, big.top_k, big.hidden, big.intermediate, 8)
    t1, i1, s1 = _layer(big, 71, device)
    t2, i2, s2 = _layer(small, 72, device)
    announce(f"no-alloc forward, path={path}: 64 tokens then 8 tokens")
    got1 = kernels.moe_experts_forward(t1["hidden"], i1, s1, *expert_args(t1), path=path, noalloc=True)
    got2 = kernels.moe_experts_forward(t2["hidden"], i2, s2, *expert_args(t2), path=path, noalloc=True)
    torch.cuda.synchronize()
    want1 = kernels.moe_experts_forward(t1["hidden"], i1, s1, *expert_args(t1), path=path)
    want2 = kernels.moe_experts_forward(t2["hidden"], i2, s2, *expert_args(t2), path=path)
    torch.cuda.synchronize()
    assert _same_bits(got1, want1), "64 tokens: no-alloc differs from the workspace forward"
    assert _same_bits(got2, want2), "8 tokens after 64: no-alloc differs from the workspace forward"
    # and the result is the layer: the oracle on a few tokens of each call
    tok = torch.arange(4)
    assert_layer_close(got1.cpu()[tok], oracle_tokens(t1, i1, s1, tok), "no-alloc 64 tokens vs oracle")
    assert_layer_close(got2.cpu()[tok], oracle_tokens(t2, i2, s2, tok), "no-alloc 8 tokens vs oracle")


def test_noalloc_refuses_a_batch_beyond_the_scratch(device):
    big = synthetic.GPTOSS_120B_PREFILL                      # 8192 tokens: far beyond 16 MiB
    shape = synthetic.MoEShape(big.experts, big.top_k, big.hidden, big.intermediate, 1024)
    t, idx, scores = _layer(shape, 73, device)
    with pytest.raises(ValueError, match="static scratch"):
        kernels.moe_experts_forward(t["hidden"], idx, scores, *expert_args(t), noalloc=True)


@pytest.mark.parametrize("shape,path", [
    ((32, 4, 2880, 2880, 200, 150), "auto"),     # 25 / 19 rows per expert: the MX kernels
    ((8, 2, 256, 256, 300, 100), "tiled"),       # the bf16 tiled kernels
], ids=["20b-width-mx", "tiny-tiled"])
def test_noalloc_prefill_kernels_twice(device, shape, path):
    E, k, H, I, T1, T2 = shape
    t1, i1, s1 = _layer(synthetic.MoEShape(E, k, H, I, T1), 74, device)
    t2, i2, s2 = _layer(synthetic.MoEShape(E, k, H, I, T2), 75, device)
    assert kernels.moe_workspace_bytes(T1, H, I, E, k) <= 16 << 20
    announce(f"no-alloc forward {shape} path={path}")
    got1 = kernels.moe_experts_forward(t1["hidden"], i1, s1, *expert_args(t1), path=path, noalloc=True)
    got2 = kernels.moe_experts_forward(t2["hidden"], i2, s2, *expert_args(t2), path=path, noalloc=True)
    torch.cuda.synchronize()
    want1 = kernels.moe_experts_forward(t1["hidden"], i1, s1, *expert_args(t1), path=path)
    want2 = kernels.moe_experts_forward(t2["hidden"], i2, s2, *expert_args(t2), path=path)
    torch.cuda.synchronize()
    assert _same_bits(got1, want1), f"{T1} tokens: no-alloc differs from the workspace forward"
    assert _same_bits(got2, want2), f"{T2} tokens after {T1}: no-alloc differs from the workspace forward"
    tok = torch.arange(4)
    assert_layer_close(got2.cpu()[tok], oracle_tokens(t2, i2, s2, tok), f"no-alloc {T2} tokens vs oracle")
