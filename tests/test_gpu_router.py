"""Router (logits, top-k, softmax over the top-k) parity on the GPU."""

from __future__ import annotations

import pytest
import torch

import oracle
from blockstreamer_amd import gptoss, kernels, synthetic
from tests.conftest import announce
from tests.moe_util import assert_layer_close, expert_args

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("E,k", [(8, 2), (32, 4), (128, 4), (256, 16), (5, 5)])
def test_topk_bit_exact_given_fp32_logits(device, E, k):
    g = torch.Generator().manual_seed(E * 10 + k)
    logits = torch.randn(300, E, generator=g)
    # engineered ties and signed zeros: lower index must win
    logits[0, :] = 1.0
    logits[1, : min(E, 6)] = torch.tensor([0.0, -0.0, 0.0, -0.0, 2.0, 2.0])[: min(E, 6)]
    logits[2, :] = torch.arange(E, dtype=torch.float32).flip(0)
    announce(f"router topk E={E} k={k}")
    scores, idx = kernels.router_topk(logits.to(device), k)
    _, ref_scores, ref_idx = oracle.topk_softmax_ref(logits, k)
    assert torch.equal(idx.cpu(), ref_idx)
    torch.testing.assert_close(scores.cpu(), ref_scores, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_topk_half_logits(device, dt):
    logits = (torch.randn(64, 128, generator=torch.Generator().manual_seed(3))).to(dt)
    scores, idx = kernels.router_topk(logits.to(device), 4)
    _, ref_scores, ref_idx = oracle.topk_softmax_ref(logits, 4)
    assert torch.equal(idx.cpu(), ref_idx)
    torch.testing.assert_close(scores.cpu().float(), ref_scores.float(), rtol=1e-2, atol=1e-3)


def _near_tie_rows(logits: torch.Tensor, k: int, gap: float) -> torch.Tensor:
    """Rows whose k-th and (k+1)-th largest logits are closer than gap."""
    top = torch.topk(logits.float(), k + 1, dim=-1).values
    return (top[:, k - 1] - top[:, k]).abs() < gap


def test_router_fp32_module(device):
    T, H, E, k = 200, 2880, 128, 4
    g = torch.Generator().manual_seed(4)
    h = torch.randn(T, H, generator=g)
    w = torch.randn(E, H, generator=g) * 0.02
    b = torch.randn(E, generator=g) * 0.5
    announce("router fp32 module")
    logits, scores, idx = kernels.router_forward(h.to(device), w.to(device), b.to(device), k)
    rl, rs, ri = oracle.router_ref(h, w, b, k)
    torch.testing.assert_close(logits.cpu(), rl, rtol=1e-5, atol=1e-5)
    ok = ~_near_tie_rows(rl, k, 1e-4)
    assert ok.sum() > T * 0.95
    assert torch.equal(idx.cpu()[ok], ri[ok])
    torch.testing.assert_close(scores.cpu()[ok], rs[ok], rtol=1e-4, atol=1e-5)
    # given its own logits, the selection is the oracle's exactly
    _, _, self_idx = oracle.topk_softmax_ref(logits.cpu(), k)
    assert torch.equal(idx.cpu(), self_idx)


@pytest.mark.parametrize("T,E,k", [(64, 8, 2), (2048, 32, 4), (64, 128, 4), (8192, 128, 4)])
def test_router_bf16_module(device, T, E, k):
    """The real case: bf16 hidden and router weights (logits rounded to bf16)."""
    H = 256 if E == 8 else 2880
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, H, T), seed=E + T, scale_lo=119,
                            scale_hi=125, router_bias_std=0.5 if E == 128 else 0.01, device=device)
    announce(f"router bf16 T={T} E={E}")
    logits, scores, idx = kernels.router_forward(t["hidden"], t["router_weight"], t["router_bias"], k)
    # float32 oracle logits rounded to bf16: within one bf16 rounding
    rl32 = oracle.router_ref(t["hidden"].cpu(), t["router_weight"].cpu(), t["router_bias"].cpu(), k)[0]
    diff = (logits.cpu().float() - rl32).abs()
    assert (diff <= rl32.abs() * 2 ** -8 + 1e-6).all(), diff.max()
    # selection and softmax are exact functions of the bf16 logits
    _, ref_scores, ref_idx = oracle.topk_softmax_ref(logits.cpu(), k)
    assert torch.equal(idx.cpu(), ref_idx)
    torch.testing.assert_close(scores.cpu().float(), ref_scores.float(), rtol=8e-3, atol=1e-3)
    # and agree with the float32 oracle wherever no near-tie could flip them:
    # the selected set where the k-th / (k+1)-th gap is clear, the order too
    # where every adjacent gap among the top k+1 is clear
    ri = oracle.topk_softmax_ref(rl32, k)[2]
    ok = ~_near_tie_rows(rl32, k, 0.05)
    assert ok.float().mean() > 0.5
    assert torch.equal(idx.cpu()[ok].sort(-1).values, ri[ok].sort(-1).values)
    top = torch.topk(rl32, k + 1, dim=-1).values
    clear = ((top[:, :-1] - top[:, 1:]).abs() >= 0.05).all(-1)
    assert torch.equal(idx.cpu()[clear], ri[clear])


def test_router_backward_vs_transformers(device):
    gpt_oss = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")
    from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig

    T, H, E, k = 96, 256, 32, 4
    cfg = GptOssConfig(num_local_experts=E, hidden_size=H, intermediate_size=H,
                       num_experts_per_tok=k, num_hidden_layers=1)
    ref = gpt_oss.GptOssTopKRouter(cfg)
    mine = gptoss.MXFP4TopKRouter(cfg, torch.float32).to(device)
    g = torch.Generator().manual_seed(7)
    with torch.no_grad():
        ref.weight.copy_(torch.randn(E, H, generator=g) * 0.1)
        ref.bias.copy_(torch.randn(E, generator=g) * 0.1)
        mine.weight.copy_(ref.weight)
        mine.bias.copy_(ref.bias)
    x = torch.randn(T, H, generator=g)
    gs = torch.randn(T, k, generator=g)
    gl = torch.randn(T, E, generator=g)
    xr = x.clone().requires_grad_(True)
    rl, rs, ri = ref(xr)
    ((rs * gs).sum() + (rl * gl).sum()).backward()
    xm = x.to(device).requires_grad_(True)
    announce("router backward")
    ml, ms, mi = mine(xm)
    assert torch.equal(mi.cpu(), ri)
    ((ms * gs.to(device)).sum() + (ml * gl.to(device)).sum()).backward()
    torch.testing.assert_close(xm.grad.cpu(), xr.grad, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(mine.weight.grad.cpu(), ref.weight.grad, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(mine.bias.grad.cpu(), ref.bias.grad, rtol=1e-4, atol=1e-5)


def test_fused_mlp_end_to_end(device):
    """MXFP4MLP (GptOssMLP drop-in): router + experts, [B, S, H] in and out."""
    from torch.func import functional_call
    from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig

    shape = synthetic.MoEShape(32, 4, 2880, 2880, 256)
    cfg = GptOssConfig(num_local_experts=32, hidden_size=2880, intermediate_size=2880,
                       num_experts_per_tok=4, num_hidden_layers=1)
    mlp = gptoss.MXFP4MLP(cfg, torch.bfloat16)
    t = synthetic.moe_layer(shape, seed=31, scale_lo=116, scale_hi=120, router_bias_std=0.01,
                            device=device)
    state = {"router.weight": t["router_weight"], "router.bias": t["router_bias"]}
    state.update({f"experts.{n}": t[n] for n in ("gate_up_proj_blocks", "gate_up_proj_scales",
                                                 "gate_up_proj_bias", "down_proj_blocks",
                                                 "down_proj_scales", "down_proj_bias")})
    h = t["hidden"].reshape(4, 64, 2880)
    announce("fused MLP end to end")
    with torch.no_grad():
        out, scores = functional_call(mlp, state, (h,), strict=True)
    assert out.shape == (4, 64, 2880) and scores.shape == (256, 4)
    logits, s2, idx = kernels.router_forward(t["hidden"], t["router_weight"], t["router_bias"], 4)
    torch.testing.assert_close(scores, s2, rtol=0, atol=0)
    want = oracle.experts_ref(t["hidden"].cpu(), idx.cpu(), scores.cpu().float(),
                              *[a.cpu() for a in expert_args(t)])
    assert_layer_close(out.reshape(256, 2880), want, "fused MLP", absolute=True)
