"""The MoE layer (router + dispatch + expert GEMMs + combine) captured in a HIP
graph: every replay equals the eager layer bit for bit.

Decode serving replays captured graphs.  The library records no memset and
synchronises nothing, and every workspace comes from torch's allocator (the
graph's private pool under capture), so the whole layer captures as it is.
Replays are interleaved with eager calls of the same layer and with
synchronisations, and each replay is checked, not only the last."""

from __future__ import annotations

import pytest
import torch

from blockstreamer_amd import kernels, synthetic
from tests.conftest import announce
from tests.moe_util import expert_args

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T", [1, 64, 512], ids=["decode_t1", "decode_t64", "prefill_t512"])
def test_layer_graph_replays_match_eager(device, T):
    E, k, H, I = 32, 4, 2880, 2880
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=21 + T, scale_lo=116, scale_hi=120,
                            router_bias_std=0.5, device=device)
    x, args = t["hidden"], expert_args(t)

    def step():
        _, scores, idx = kernels.router_forward(x, t["router_weight"], t["router_bias"], k)
        return kernels.moe_experts_forward(x, idx, scores, *args)

    announce(f"layer graph replay T={T}")
    want = step().clone()
    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = step()
    for rep in range(3):
        eager = step()
        torch.cuda.synchronize()
        assert torch.equal(eager, want), f"eager call {rep} (T={T})"
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {rep} (T={T})"
