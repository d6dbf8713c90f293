"""Decode weight-streaming kernels on the gpt-oss shape (K = 2880).

The persistent kernel (persistent workgroups walking (expert, pass, slice)
items through LDS DMA rings) multiplies the packed MXFP4 weights on the
block-scaled MFMA with the activations split into two MXFP8 terms (hi + lo,
exact for every element above 2^-14 of its 32-element block's maximum).  The part kernel decodes
the weights to bf16 and multiplies on the bf16 MFMA.  Both approximate the
same float32 product; they are compared with each other (relative L2 <= 2e-3,
the difference being the bf16 roundings of the two) and with the oracle at
the layer bar.  A bias view that is only 2-byte aligned sends the same call to
the part kernel (the persistent kernel DMAs the bias and needs 16-byte
alignment).
"""

from __future__ import annotations

import pytest
import torch

import oracle
from blockstreamer_amd import kernels, synthetic
from tests.conftest import announce
from tests.moe_util import assert_layer_close, errors, expert_args, oracle_tokens

KERNEL_AGREEMENT = 2e-3


def _agree(persist, parts, what):
    rel_l2, max_abs, scale = errors(persist, parts)
    msg = f"{what}: persistent vs part kernel rel_l2={rel_l2:.3e} max_abs={max_abs:.3e} (|max| {scale:.3e})"
    print(msg)
    assert rel_l2 <= KERNEL_AGREEMENT, msg

pytestmark = pytest.mark.gpu


def _shifted(x: torch.Tensor) -> torch.Tensor:
    """Same values, storage starting one element (2 bytes) later."""
    buf = torch.empty(x.numel() + 1, dtype=x.dtype, device=x.device)
    buf[1:] = x.reshape(-1)
    v = buf[1:].view(x.shape)
    assert v.data_ptr() % 16 == 2
    return v


def _both_kernels(t, idx, w):
    args = list(expert_args(t))
    persist = kernels.moe_experts_forward(t["hidden"], idx, w, *args, path="stream")
    args[2] = _shifted(args[2])
    args[5] = _shifted(args[5])
    parts = kernels.moe_experts_forward(t["hidden"], idx, w, *args, path="stream")
    torch.cuda.synchronize()
    return persist, parts


@pytest.mark.parametrize("T", [1, 64])
def test_persistent_equals_part_kernel(device, T):
    shape = synthetic.MoEShape(128, 4, 2880, 2880, T)
    t = synthetic.moe_layer(shape, seed=4, scale_lo=115, scale_hi=131, router_bias_std=0.5,
                            device=device)
    _, w, idx = kernels.router_forward(t["hidden"], t["router_weight"], t["router_bias"], 4)
    announce(f"persistent vs part kernel T={T}")
    persist, parts = _both_kernels(t, idx, w)
    _agree(persist, parts, f"T={T}")
    tokens = torch.arange(min(T, 6))
    want = oracle_tokens(t, idx.cpu(), w.cpu(), tokens)
    assert_layer_close(persist.cpu()[tokens], want, f"persistent T={T}")


def test_persistent_multi_pass_expert(device):
    """An expert with 40 rows (three 16-row passes) next to experts with one."""
    T = 48
    shape = synthetic.MoEShape(128, 4, 2880, 2880, T)
    t = synthetic.moe_layer(shape, seed=21, scale_lo=116, scale_hi=120, device=device)
    idx, w = synthetic.random_routing(T, 128, 4, seed=22, device=device)
    idx = idx.clone()
    hot = 77
    idx[idx == hot] = (hot + 1) % 128       # keep each token's experts distinct
    idx[:40, 0] = hot
    idx = idx.contiguous()
    assert int((idx == hot).sum()) == 40
    announce("persistent kernel, 40-row expert")
    persist, parts = _both_kernels(t, idx, w)
    _agree(persist, parts, "40-row expert")
    tokens = torch.tensor([0, 17, 39, 40, 47])
    want = oracle_tokens(t, idx.cpu(), w.cpu(), tokens)
    assert_layer_close(persist.cpu()[tokens], want, "40-row expert", absolute=True)


def test_persistent_float32_bias_vs_oracle(device):
    T = 16
    shape = synthetic.MoEShape(128, 4, 2880, 2880, T)
    t = synthetic.moe_layer(shape, seed=31, scale_lo=116, scale_hi=120, device=device)
    t["gate_up_proj_bias"] = t["gate_up_proj_bias"].float()
    t["down_proj_bias"] = t["down_proj_bias"].float()
    idx, w = synthetic.random_routing(T, 128, 4, seed=32, device=device)
    announce("persistent kernel, float32 biases")
    got = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(t), path="stream")
    args = [a.cpu() for a in expert_args(t)]
    want = oracle.experts_ref(t["hidden"].cpu(), idx.cpu(), w.cpu().float(), *args)
    assert_layer_close(got, want, "float32 biases", absolute=True)


def test_persistent_single_expert_most_workgroups_idle(device):
    """T=1, k=1: 180 down items and 360 gate_up items over one workgroup per CU."""
    shape = synthetic.MoEShape(128, 1, 2880, 2880, 1)
    t = synthetic.moe_layer(shape, seed=41, scale_lo=116, scale_hi=120, device=device)
    idx = torch.tensor([[127]], device=device)
    w = torch.ones(1, 1, dtype=torch.bfloat16, device=device)
    announce("persistent kernel, one token one expert")
    persist, parts = _both_kernels(t, idx, w)
    _agree(persist, parts, "one token one expert")
    want = oracle.experts_ref(t["hidden"].cpu(), idx.cpu(), w.cpu().float(),
                              *[a.cpu() for a in expert_args(t)])
    assert_layer_close(persist, want, "one token one expert", absolute=True)


@pytest.mark.parametrize("bias", ["f16", "none"])
def test_persistent_f16_or_no_bias_vs_oracle(device, bias):
    T = 24
    shape = synthetic.MoEShape(128, 4, 2880, 2880, T)
    t = synthetic.moe_layer(shape, seed=51, scale_lo=116, scale_hi=120, device=device)
    idx, w = synthetic.random_routing(T, 128, 4, seed=52, device=device)
    args = list(expert_args(t))
    if bias == "f16":
        args[2] = args[2].half()
        args[5] = args[5].half()
        ref_args = [a.cpu() for a in args]
    else:
        ref_args = [a.cpu() for a in args]
        ref_args[2] = torch.zeros_like(ref_args[2])
        ref_args[5] = torch.zeros_like(ref_args[5])
        args[2] = None
        args[5] = None
    announce(f"persistent kernel, bias {bias}")
    got = kernels.moe_experts_forward(t["hidden"], idx, w, *args, path="stream")
    want = oracle.experts_ref(t["hidden"].cpu(), idx.cpu(), w.cpu().float(), *ref_args)
    assert_layer_close(got, want, f"bias {bias}", absolute=True)
