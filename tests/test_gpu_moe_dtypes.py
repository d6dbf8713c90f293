"""MXFP4Experts on float32 and float16 hidden states (no narrowing to bf16).

The reference dequantises to the hidden states' dtype and multiplies in it
(block_streamer/gptoss.py:58-62, 158-176), and StreamedModel's own parity
runs float32 and float16 blocks (tests/test_parity.py:49-70).  Here those
dtypes run the reference's per-expert loop in their own dtype with every
product on the exact multi-term packed kernels of ``mxfp4_matmul``, so:

* float32: the output and the gradients of the hidden states and routing
  weights equal the float32 oracle (its torch autograd for the gradients)
  to float32 summation accuracy -- relative L2 <= 2e-5 and max-abs <=
  1e-4 of the largest value, far below the bf16 layer bar;
* float16: the reference's rounding points (products, bias add, SwiGLU and
  combine rounded to float16): against the oracle evaluated in float16 on
  the CPU, relative L2 <= 1e-3; against float32, the float16 layer bar.

No warning is emitted (the bf16 narrowing it announced is gone).
"""

from __future__ import annotations

import warnings
from types import SimpleNamespace

import pytest
import torch

import oracle
from blockstreamer_amd import gptoss, synthetic
from tests.conftest import announce
from tests.moe_util import errors

pytestmark = pytest.mark.gpu

NAMES = ("gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
         "down_proj_blocks", "down_proj_scales", "down_proj_bias")
SHAPES = [(8, 2, 256, 256, 64), (16, 4, 2880, 2880, 24)]


def _module_and_state(E, k, H, I, T, seed, device):
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=seed, scale_lo=116, scale_hi=120)
    cfg = SimpleNamespace(num_local_experts=E, hidden_size=H, intermediate_size=I, num_experts_per_tok=k)
    mod = gptoss.MXFP4Experts(cfg, torch.bfloat16)
    state = {n: t[n].to(device) for n in NAMES}
    idx, w = synthetic.random_routing(T, E, k, seed=seed + 1, dtype=torch.float32)
    return t, mod, state, idx, w


def _run(mod, state, h, idx, w):
    with warnings.catch_warnings():
        warnings.simplefilter("error")            # any warning fails the test
        return torch.func.functional_call(mod, state, (h, idx, w), strict=True)


@pytest.mark.parametrize("shape", SHAPES, ids=[f"E{s[0]}H{s[2]}T{s[4]}" for s in SHAPES])
def test_float32_forward_and_backward_to_float32_accuracy(device, shape):
    E, k, H, I, T = shape
    t, mod, state, idx, w = _module_and_state(E, k, H, I, T, 91, device)
    x = t["hidden"].float()
    g = torch.randn(T, H, generator=torch.Generator().manual_seed(92))
    xd = x.to(device).requires_grad_(True)
    wd = w.to(device).requires_grad_(True)
    announce(f"float32 experts {shape}")
    out = _run(mod, state, xd, idx.to(device), wd)
    assert out.dtype == torch.float32
    (out * g.to(device)).sum().backward()
    torch.cuda.synchronize()

    xr = x.clone().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    ref = oracle.experts_ref(xr, idx, wr, *[t[n] for n in NAMES])
    (ref * g).sum().backward()
    for what, got, want, rel_bar in (("output", out, ref, 2e-5), ("d hidden", xd.grad, xr.grad, 2e-5),
                                     ("d routing weights", wd.grad, wr.grad, 2e-5)):
        rel, mx, scale = errors(got, want)
        print(f"float32 {shape} {what}: rel_l2={rel:.3e} max_abs={mx:.3e} (|ref|max {scale:.3e})")
        assert rel <= rel_bar and mx <= 1e-4 * scale, what


def test_float16_keeps_the_reference_rounding_points(device):
    E, k, H, I, T = SHAPES[0]
    t, mod, state, idx, w = _module_and_state(E, k, H, I, T, 93, device)
    for n in ("gate_up_proj_bias", "down_proj_bias"):   # a float16 model: float16 biases
        t[n] = t[n].to(torch.float16)
        state[n] = t[n].to(device)
    x16 = t["hidden"].to(torch.float16)
    w16 = w.to(torch.float16)
    announce("float16 experts")
    out = _run(mod, state, x16.to(device), idx.to(device), w16.to(device))
    torch.cuda.synchronize()
    assert out.dtype == torch.float16
    ref16 = oracle.experts_ref(x16, idx, w16, *[t[n] for n in NAMES], dtype=torch.float16)
    ref32 = oracle.experts_ref(x16.float(), idx, w16.float(), *[t[n] for n in NAMES])
    rel16, _, _ = errors(out, ref16)
    rel32, mx32, scale = errors(out, ref32)
    print(f"float16: vs the float16 oracle rel_l2={rel16:.3e}; vs float32 rel_l2={rel32:.3e} "
          f"max_abs={mx32:.3e} (|ref|max {scale:.3e})")
    assert rel16 <= 1e-3
    assert rel32 <= 5e-3 and mx32 <= 2e-2 * max(scale, 1.0)


def test_float32_drops_out_of_range_indices_like_the_fused_path(device):
    E, k, H, I, T = SHAPES[0]
    t, mod, state, idx, w = _module_and_state(E, k, H, I, T, 95, device)
    idx = idx.clone()
    idx[::3, 0] = E          # the masking index
    idx[1::5, 1] = -1
    keep = (idx >= 0) & (idx < E)
    announce("float32 experts, dropped pairs")
    out = _run(mod, state, t["hidden"].float().to(device), idx.to(device), w.to(device))
    torch.cuda.synchronize()
    # dropped pairs contribute nothing: the oracle on the kept pairs (weight 0, any valid expert)
    ref = oracle.experts_ref(t["hidden"].float(), torch.where(keep, idx, 0), torch.where(keep, w, 0.0),
                             *[t[n] for n in NAMES])
    rel, mx, scale = errors(out, ref)
    assert rel <= 2e-5 and mx <= 1e-4 * scale
