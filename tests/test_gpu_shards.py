"""The expert layer run from a staged k-pair shard (GPU).

A block is written with ``blockstreamer_amd.shards`` (k-pair expert blocks,
16-byte aligned tensors, the layout field), its bytes staged into one flat
uint8 device buffer as the reference's disk pool stages them
(block_streamer/diskpool.py:163-195), the tensors taken as views of that
buffer (shards.py:57-60) and bound to ``MXFP4Experts`` by name through
``functional_call`` (streamer.py:161-167).  The layer must equal the same
call on the checkpoint-layout tensors bit for bit (every kernel reads the
k-pair layout to the same LDS contents), on the decode kernels and on the MX
prefill kernels, and the staged bytes must be left untouched.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from blockstreamer_amd import gptoss, kernels, shards, synthetic
from tests.conftest import announce

pytestmark = pytest.mark.gpu

EXPERTS = ("gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
           "down_proj_blocks", "down_proj_scales", "down_proj_bias")


@pytest.mark.parametrize("T,kernel", [(64, "stream"), (256, "mx")])
def test_layer_from_a_staged_kpair_shard(device, tmp_path, T, kernel):
    E, k, H, I = 16, 4, 2880, 2880
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=81, scale_lo=116, scale_hi=120)
    state = {f"mlp.experts.{n}": t[n] for n in EXPERTS}
    state["post_attention_layernorm.weight"] = torch.ones(H)
    manifest = shards.convert_modules(iter([(3, state)]), tmp_path)
    m = shards.load_manifest(tmp_path)
    block = m["blocks"][0]
    assert shards.block_layouts(m, 3) == {"mlp.experts.gate_up_proj_blocks": "kpair",
                                          "mlp.experts.down_proj_blocks": "kpair"}
    host = torch.empty(block["nbytes"], dtype=torch.uint8)
    shards.read_block(tmp_path, block, host)
    blob = host.to(device)                              # the staged block: one flat device buffer
    views = shards.materialize(block, blob)
    staged = {n: views[f"mlp.experts.{n}"] for n in EXPERTS}
    assert kernels.blocks_layout(staged["gate_up_proj_blocks"]) == kernels.LAYOUT_KPAIR
    assert all(v.data_ptr() % 16 == 0 for v in staged.values())
    before = blob.clone()

    cfg = SimpleNamespace(num_local_experts=E, hidden_size=H, intermediate_size=I, num_experts_per_tok=k)
    mod = gptoss.MXFP4Experts(cfg, torch.bfloat16)
    x = t["hidden"].to(device)
    idx, w = synthetic.random_routing(T, E, k, seed=82, device=device)
    announce(f"experts from a staged k-pair shard, T={T} ({kernel} kernels)")
    with torch.no_grad():
        got = torch.func.functional_call(mod, staged, (x, idx, w), strict=True)
    dev = {n: t[n].to(device) for n in EXPERTS}
    want = kernels.moe_experts_forward(x, idx, w, *(dev[n] for n in EXPERTS))
    resolved = kernels._whole_forward_path("auto", T, k, E, H, I, staged["gate_up_proj_blocks"],
                                           staged["gate_up_proj_scales"], staged["down_proj_blocks"],
                                           staged["down_proj_scales"])
    torch.cuda.synchronize()
    assert resolved == kernels.PATHS["mx" if kernel == "mx" else "auto"]
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(blob, before)
    assert manifest["blockstreamer_amd"]["alignment"] == 16
