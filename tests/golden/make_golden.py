"""Write the golden fixtures under tests/golden/ (run once, on a CPU).

The reference path's arithmetic lives in the third-party ``transformers``
package (version 5.15.0 is the one installed and pinned here), which
block_streamer/gptoss.py calls: ``convert_moe_packed_tensors``
(TF/integrations/mxfp4.py:316-338), ``GptOssTopKRouter``
(TF/models/gpt_oss/modeling_gpt_oss.py:117-131) and the dense experts twin
``GptOssExperts`` (modeling_gpt_oss.py:68-114, which
block_streamer/gptoss.py:137-177 mirrors with per-expert dequantisation).
This script runs those library routines in float32 on the CPU on seeded
synthetic inputs and stores their outputs:

* ``dequant_table.npz``: every (scale byte, packed byte) pair through
  ``convert_moe_packed_tensors`` for bf16, f16 and f32 outputs.
* ``tiny_layer.npz``: the tiny layer (8 experts, top-2, hidden 256,
  intermediate 256, 64 tokens, scales in [119, 129], seed 1): router logits,
  scores and indices, and the experts output, plus SHA-256 digests of the
  regenerated inputs so a test can prove it rebuilt the same bytes.

Usage: ``python tests/golden/make_golden.py``
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from blockstreamer_amd import synthetic  # noqa: E402

TINY_SEED = 1
TINY_SCALES = (119, 129)


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def exhaustive_inputs() -> tuple[torch.Tensor, torch.Tensor]:
    """[1, 256, 16, 16]: row r has scale r, byte (g, j) = 16 g + j."""
    blocks = torch.arange(256, dtype=torch.int32).reshape(16, 16).to(torch.uint8)
    blocks = blocks.expand(256, 16, 16).unsqueeze(0).contiguous()
    scales = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(256, 1)
    scales = scales.expand(256, 16).unsqueeze(0).contiguous()
    return blocks, scales


def tiny_layer() -> dict[str, torch.Tensor]:
    return synthetic.moe_layer(synthetic.TINY, seed=TINY_SEED, scale_lo=TINY_SCALES[0],
                               scale_hi=TINY_SCALES[1], router_bias_std=0.0)


def main() -> None:
    from transformers.integrations.mxfp4 import convert_moe_packed_tensors
    from transformers.models.gpt_oss import modeling_gpt_oss as gpt_oss
    from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig

    # --- exhaustive dequant table -------------------------------------------------
    blocks, scales = exhaustive_inputs()
    table = {}
    for name, dt in (("bf16", torch.bfloat16), ("f16", torch.float16), ("f32", torch.float32)):
        dense = convert_moe_packed_tensors(blocks, scales, dtype=dt)  # [1, 512, 256]
        bits = dense.view(torch.int16 if dt != torch.float32 else torch.int32).numpy()
        table[name] = bits[0].copy()  # [K=512, R=256]
    np.savez_compressed(HERE / "dequant_table.npz", **table)

    # --- tiny layer -----------------------------------------------------------------
    shape = synthetic.TINY
    t = tiny_layer()
    cfg = GptOssConfig(num_local_experts=shape.experts, hidden_size=shape.hidden,
                       intermediate_size=shape.intermediate,
                       num_experts_per_tok=shape.top_k, num_hidden_layers=1)
    router = gpt_oss.GptOssTopKRouter(cfg)
    with torch.no_grad():
        router.weight.copy_(t["router_weight"].float())
        router.bias.copy_(t["router_bias"].float())
    experts = gpt_oss.GptOssExperts(cfg)
    with torch.no_grad():
        experts.gate_up_proj.copy_(convert_moe_packed_tensors(
            t["gate_up_proj_blocks"], t["gate_up_proj_scales"], dtype=torch.float32))
        experts.gate_up_proj_bias.copy_(t["gate_up_proj_bias"].float())
        experts.down_proj.copy_(convert_moe_packed_tensors(
            t["down_proj_blocks"], t["down_proj_scales"], dtype=torch.float32))
        experts.down_proj_bias.copy_(t["down_proj_bias"].float())
        h = t["hidden"].float()
        logits, scores, idx = router(h)
        out = experts(h, idx, scores)
    np.savez_compressed(
        HERE / "tiny_layer.npz",
        router_logits=logits.numpy(),
        router_scores=scores.numpy(),
        router_indices=idx.numpy(),
        experts_out=out.numpy(),
        **{f"sha256_{k}": np.array(digest(v)) for k, v in t.items()},
    )
    print("wrote", HERE / "dequant_table.npz", HERE / "tiny_layer.npz")


if __name__ == "__main__":
    main()
