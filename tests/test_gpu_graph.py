"""The MoE layer (router, dispatch, expert GEMMs, combine) captured in a HIP
graph and replayed, as a serving loop does for decode.  The library makes no
allocation, copy, memset or synchronisation, so the whole layer captures.
Every replay, with eager work and synchronisations in between and a new
input each time, must equal the eager call on the same input bit for bit.
The cases cover the decode kernels at 1, 8 and 64 tokens, the bf16 tiled
kernels and the MX prefill kernels (the automatic path at 512 tokens)."""

from __future__ import annotations

import pytest
import torch

from blockstreamer_amd import kernels, synthetic
from tests.conftest import announce
from tests.moe_util import expert_args

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("E,k,T,path", [(32, 4, 1, "auto"), (32, 4, 8, "auto"), (128, 4, 64, "auto"),
                                        (32, 4, 256, "tiled"), (32, 4, 512, "auto")])
def test_layer_graph_replays_equal_eager(device, E, k, T, path):
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, 2880, 2880, T), seed=E + T, scale_lo=116,
                            scale_hi=122, router_bias_std=0.5, device=device)
    args = expert_args(t)
    x = t["hidden"].clone()

    def layer(h):
        _, scores, idx = kernels.router_forward(h, t["router_weight"], t["router_bias"], k)
        return kernels.moe_experts_forward(h, idx, scores, *args, path=path)

    announce(f"graph replay E={E} k={k} T={T} {path}")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            layer(x)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = layer(x)
    gen = torch.Generator().manual_seed(T)
    for i in range(3):
        new = torch.randn(T, 2880, generator=gen).to(torch.bfloat16).to(device)
        x.copy_(new)
        want = layer(new)            # eager, on its own copy of the input
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {i}"
