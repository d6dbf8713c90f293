"""Helpers for the MoE parity tests: tolerances and reference computations.

Tolerance (written here once, used by every layer-output test): against the
float32 reference, relative L2 error <= 5e-3 and max-abs error <= 2e-2.
With the workload's weight distribution (E8M0 scales uniform in [115, 131]
or [119, 129]) the layer outputs reach 1e3..1e5, where one bfloat16 ulp is
far above 2e-2, so for those the max-abs bound is applied to the error
divided by max|reference|; tests on weights scaled like a trained model
(scales in [116, 120], outputs of order 1) apply 2e-2 absolutely.
"""

from __future__ import annotations

import torch

import oracle

REL_L2 = 5e-3
MAX_ABS = 2e-2


def errors(got: torch.Tensor, want: torch.Tensor) -> tuple[float, float, float]:
    got = got.detach().float().cpu()
    want = want.detach().float().cpu()
    d = got - want
    rel_l2 = (d.norm() / want.norm().clamp_min(1e-30)).item()
    max_abs = d.abs().max().item() if d.numel() else 0.0
    scale = want.abs().max().item() if want.numel() else 0.0
    return rel_l2, max_abs, scale


def assert_layer_close(got, want, what: str, absolute: bool = False) -> None:
    rel_l2, max_abs, scale = errors(got, want)
    bound = MAX_ABS if absolute else MAX_ABS * max(scale, 1.0)
    msg = f"{what}: rel_l2={rel_l2:.3e} max_abs={max_abs:.3e} (|ref|max={scale:.3e}, bound {bound:.3e})"
    print(msg)
    assert rel_l2 <= REL_L2, msg
    assert max_abs <= bound, msg


EXPERT_KEYS = ("gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
               "down_proj_blocks", "down_proj_scales", "down_proj_bias")


def expert_args(t: dict) -> tuple:
    return tuple(t[k] for k in EXPERT_KEYS)


def oracle_tokens(t: dict, idx: torch.Tensor, w: torch.Tensor, tokens: torch.Tensor) -> torch.Tensor:
    """Oracle output for a subset of tokens, moving only their experts to the CPU.

    The layer is token-wise, so out[tokens] depends only on those tokens'
    rows and experts.
    """
    tokens = tokens.cpu()
    idx_s = idx.cpu()[tokens]
    w_s = w.cpu()[tokens].float()
    used = torch.unique(idx_s)
    remap = torch.full((t["gate_up_proj_blocks"].shape[0],), -1, dtype=torch.int64)
    remap[used] = torch.arange(len(used))
    args = [t[k].index_select(0, used.to(t[k].device)).cpu() for k in EXPERT_KEYS]
    return oracle.experts_ref(t["hidden"].cpu()[tokens], remap[idx_s], w_s, *args)


def gpu_reference(t: dict, idx: torch.Tensor, w: torch.Tensor, alpha=1.702, limit=7.0):
    """float32 torch reference on the GPU (gptoss.py:137-177 semantics).

    Dense weights come from the dequant kernel, which the exhaustive table
    pins bit-exactly; GEMMs and SwiGLU run in float32 torch.
    """
    from blockstreamer_amd import kernels

    h = t["hidden"].float()
    out = torch.zeros_like(h)
    E = t["gate_up_proj_blocks"].shape[0]
    idx_cpu = idx.cpu()
    for e in torch.unique(idx_cpu).tolist():
        if e < 0 or e >= E:
            continue
        tok, pos = torch.where(idx == e)
        wgu = kernels.dequantize_mxfp4(t["gate_up_proj_blocks"][e:e + 1],
                                       t["gate_up_proj_scales"][e:e + 1], torch.float32)[0]
        wdn = kernels.dequantize_mxfp4(t["down_proj_blocks"][e:e + 1],
                                       t["down_proj_scales"][e:e + 1], torch.float32)[0]
        gu = h[tok] @ wgu + t["gate_up_proj_bias"][e].float()
        act = oracle.apply_gate_ref(gu, alpha, limit)
        o = act @ wdn + t["down_proj_bias"][e].float()
        out.index_add_(0, tok, o * w[tok, pos, None].float())
    return out
