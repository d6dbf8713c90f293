"""Two MoE layers running at once on two HIP streams (as a serving process
overlapping a decode batch with a prefill chunk).  The library keeps no state
between calls beyond the per-call workspace (the no-allocation entry point's
static scratch aside, which is documented as shared), so every overlapped
result must equal the serial one bit for bit."""

from __future__ import annotations

import pytest
import torch

from blockstreamer_amd import kernels, synthetic
from tests.conftest import announce
from tests.moe_util import expert_args

pytestmark = pytest.mark.gpu


def _layer_fn(E, k, T, seed, device):
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, 2880, 2880, T), seed=seed, scale_lo=116,
                            scale_hi=122, router_bias_std=0.5, device=device)
    args = expert_args(t)

    def run():
        _, scores, idx = kernels.router_forward(t["hidden"], t["router_weight"], t["router_bias"], k)
        return kernels.moe_experts_forward(t["hidden"], idx, scores, *args)

    return run


def test_two_layers_on_two_streams_equal_serial(device):
    decode = _layer_fn(32, 4, 64, 51, device)     # the decode kernels
    prefill = _layer_fn(32, 4, 512, 52, device)   # the MX prefill kernels
    announce("two streams: decode T=64 beside prefill T=512")
    want_d, want_p = decode().clone(), prefill().clone()
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    got_d, got_p = [], []
    for _ in range(4):
        with torch.cuda.stream(s1):
            got_d.append(decode())
        with torch.cuda.stream(s2):
            got_p.append(prefill())
    torch.cuda.current_stream().wait_stream(s1)
    torch.cuda.current_stream().wait_stream(s2)
    torch.cuda.synchronize()
    for i, (d, p) in enumerate(zip(got_d, got_p)):
        assert torch.equal(d.view(torch.int16), want_d.view(torch.int16)), f"decode {i}"
        assert torch.equal(p.view(torch.int16), want_p.view(torch.int16)), f"prefill {i}"
