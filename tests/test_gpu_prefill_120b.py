"""gpt-oss-120b-shaped prefill on the GPU: 128 experts, top-4, hidden =
intermediate = 2880, 8192 tokens (32,768 routed pairs), forward on every
prefill kernel path and both blocks layouts, and the input-gradient backward
used by LoRA training (block_streamer/gptoss.py:137-177 and :64-71).

Every token is compared with a float32 torch reference on the GPU (dense
weights from the dequant kernel, which the exhaustive table pins bit-exactly),
and 64 seeded random tokens with the CPU oracle.  Bars: the layer bar of
tests/moe_util.py (relative L2 <= 5e-3; max-abs <= 2e-2 * max|ref| at these
synthetic scales, whose outputs reach 1e4) for the forward, the gradient bar
of tests/test_gpu_moe_backward.py (relative L2 <= 1e-2, max-abs <= 5e-2 *
max|ref|) for the backward.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from blockstreamer_amd import kernels, synthetic
from tests.conftest import announce
from tests.moe_util import assert_layer_close, errors, expert_args, gpu_reference, oracle_tokens
from tests.test_gpu_moe_backward import GRAD_REL_L2, assert_grad_close

pytestmark = pytest.mark.gpu

SHAPE = synthetic.GPTOSS_120B_PREFILL  # E128 k4 H=I=2880 T8192


@pytest.fixture(scope="module")
def layer(device):
    """The layer, its float32 router's routing, the float32 GPU reference of
    every token and the CPU oracle of 64 sampled tokens."""
    announce("120b prefill: inputs and references")
    t = synthetic.moe_layer(SHAPE, seed=5, scale_lo=115, scale_hi=131, router_bias_std=0.0,
                            device=device)
    _, scores, idx = oracle.router_ref(t["hidden"].cpu(), t["router_weight"].cpu(),
                                       t["router_bias"].cpu(), SHAPE.top_k)
    idx, scores = idx.to(device), scores.to(device)
    ref = gpu_reference(t, idx, scores)
    tokens = torch.randperm(SHAPE.tokens, generator=torch.Generator().manual_seed(55))[:64]
    want = oracle_tokens(t, idx, scores, tokens)
    kp = dict(t)
    kp["gate_up_proj_blocks"] = kernels.to_kpair(t["gate_up_proj_blocks"])
    kp["down_proj_blocks"] = kernels.to_kpair(t["down_proj_blocks"])
    torch.cuda.synchronize()
    return dict(t=t, kp=kp, idx=idx, scores=scores, ref=ref, tokens=tokens, want=want)


@pytest.mark.parametrize("layout", ["checkpoint", "kpair"])
@pytest.mark.parametrize("path", ["auto", "tiled", "mx"])
def test_prefill_forward_every_token(layer, path, layout):
    t = layer["t"] if layout == "checkpoint" else layer["kp"]
    announce(f"120b prefill forward path={path} layout={layout}")
    got = kernels.moe_experts_forward(t["hidden"], layer["idx"], layer["scores"], *expert_args(t),
                                      path=path)
    torch.cuda.synchronize()
    assert got.shape == (SHAPE.tokens, SHAPE.hidden) and got.dtype == torch.bfloat16
    assert torch.isfinite(got).all()
    assert_layer_close(got, layer["ref"], f"120b prefill {path} {layout}: all tokens vs fp32 GPU")
    tok = layer["tokens"]
    assert_layer_close(got.cpu()[tok], layer["want"], f"120b prefill {path} {layout}: 64 tokens vs oracle")


@pytest.fixture(scope="module")
def trained_layer(device):
    """The same layer shape with E8M0 scales in [116, 120], the range of a
    trained checkpoint: outputs of order one, where the layer bar's max-abs
    2e-2 applies as an absolute bound."""
    announce("120b prefill at trained scales: inputs and references")
    t = synthetic.moe_layer(SHAPE, seed=15, scale_lo=116, scale_hi=120, router_bias_std=0.0,
                            device=device)
    _, scores, idx = oracle.router_ref(t["hidden"].cpu(), t["router_weight"].cpu(),
                                       t["router_bias"].cpu(), SHAPE.top_k)
    idx, scores = idx.to(device), scores.to(device)
    ref = gpu_reference(t, idx, scores)
    torch.cuda.synchronize()
    return dict(t=t, idx=idx, scores=scores, ref=ref)


@pytest.mark.parametrize("path", ["auto", "tiled", "mx"])
def test_prefill_forward_absolute_bar_at_trained_scales(trained_layer, path):
    t = trained_layer["t"]
    announce(f"120b prefill forward at trained scales path={path}")
    got = kernels.moe_experts_forward(t["hidden"], trained_layer["idx"], trained_layer["scores"],
                                      *expert_args(t), path=path)
    torch.cuda.synchronize()
    assert_layer_close(got, trained_layer["ref"], f"120b prefill {path}, trained scales: all tokens vs fp32 GPU",
                       absolute=True)


def test_prefill_layouts_bit_identical(layer):
    """Both blocks layouts give the same bits on the tiled path."""
    announce("120b prefill layouts bit for bit")
    outs = [kernels.moe_experts_forward(t["hidden"], layer["idx"], layer["scores"], *expert_args(t),
                                        path="tiled") for t in (layer["t"], layer["kp"])]
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def _save_by_pair(fac: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """The forward's saved SwiGLU derivative factors ``[T*k, 2I]``
    (expert-sorted rows, stable in the pair index t*k + slot) as
    ``[T, k, 2I]``."""
    T, k = idx.shape
    order = torch.argsort(idx.flatten(), stable=True)
    out = torch.empty_like(fac)
    out[order] = fac
    return out.view(T, k, -1)


# pre-activations farther than this from a clamp bound take the same
# decision in any float32 summation order
NEAR = 0.05


def _fp32_grads(t, idx, w, g, fac_pairs=None, alpha=1.702, limit=7.0):
    """float32 autograd on the GPU of block_streamer/gptoss.py:137-177, dense
    weights from the dequant kernel.  With ``fac_pairs`` (the kernel's saved
    derivative factors) the clamps of the SwiGLU (gptoss.py:131-133) take the
    kernel's pass/clamp decision instead of the float32 one (the values stay
    float32), so a pre-activation that the kernel's summation order puts on
    the other side of +-7 does not count as an arithmetic error.  A factor is
    zero where the kernel clamped; within NEAR of a bound that is the
    decision, farther away (or where the factor is zero for another reason)
    the float32 one.  Returns the gradients and the
    number of clamp decisions that differ."""
    h = t["hidden"].detach().float().clone().requires_grad_(True)
    wr = w.detach().float().clone().requires_grad_(True)
    out = torch.zeros_like(h)
    flips = 0
    for e in torch.unique(idx).tolist():
        tok, pos = torch.where(idx == e)
        wgu = kernels.dequantize_mxfp4(t["gate_up_proj_blocks"][e:e + 1],
                                       t["gate_up_proj_scales"][e:e + 1], torch.float32)[0]
        wdn = kernels.dequantize_mxfp4(t["down_proj_blocks"][e:e + 1],
                                       t["down_proj_scales"][e:e + 1], torch.float32)[0]
        gu = h[tok] @ wgu + t["gate_up_proj_bias"][e].float()
        gate, up = gu[:, 0::2], gu[:, 1::2]
        if fac_pairs is None:
            gate, up = gate.clamp(max=limit), up.clamp(min=-limit, max=limit)
        else:
            fg, fu = fac_pairs[tok, pos, 0::2], fac_pairs[tok, pos, 1::2]
            with torch.no_grad():
                g_pass = (fg != 0) | (gate < limit - NEAR)
                # where gate * sigmoid(alpha gate) underflows the up factor is
                # zero whatever up's clamp decided (and the decision changes
                # neither the value nor the gradient): the float32 decision
                glu0 = (gate * torch.sigmoid(gate * alpha)).abs() < 1e-30
                u_in = torch.where(glu0, up.abs() <= limit, (fu != 0) | (up.abs() < limit - NEAR))
                flips += int((g_pass != (gate <= limit)).sum()) + int((u_in != (up.abs() <= limit)).sum())
            gate = torch.where(g_pass, gate, torch.full_like(gate, limit))
            up = torch.where(u_in, up, torch.sign(up.detach()) * limit)
        act = (up + 1) * (gate * torch.sigmoid(gate * alpha))
        o = act @ wdn + t["down_proj_bias"][e].float()
        out = out.index_add(0, tok, o * wr[tok, pos, None])
    out.backward(g.float())
    return h.grad, wr.grad, flips


def test_prefill_backward_full_size(layer):
    """Forward with the save for the backward, then d(hidden) and d(routing
    weights) at full size, against float32 autograd on the GPU; the k-pair
    layout gives the same gradients bit for bit.

    At these synthetic weight scales (2^-12 .. 2^4 per block) gate_up
    pre-activations reach the thousands and a few of the 189 million land
    within float32 summation-order distance of a clamp at +-7, where the
    SwiGLU's derivative jumps; each such decision moves one token's gradient
    by up to the size of its largest entries.  So: relative L2 against the
    plain float32 autograd, and max-abs against the float32 autograd whose
    clamp decisions follow the kernel's (read from its saved derivative
    factors; the count of differing decisions is printed and must stay a
    tiny fraction)."""
    t = layer["t"]
    idx = layer["idx"]
    g = (torch.randn(SHAPE.tokens, SHAPE.hidden, generator=torch.Generator(device=t["hidden"].device)
                     .manual_seed(57), device=t["hidden"].device) * 1e-3).to(torch.bfloat16)
    w = layer["scores"].float()
    announce("120b prefill backward, checkpoint layout")
    _, ws, fac = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(t), save=True)
    gh, gw = kernels.moe_experts_backward(g, t["hidden"], idx, w, t["gate_up_proj_blocks"],
                                          t["gate_up_proj_scales"], t["down_proj_blocks"],
                                          t["down_proj_scales"], ws, fac)
    announce("120b prefill backward, k-pair layout")
    kp = layer["kp"]
    _, ws2, fac2 = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(kp), save=True)
    gh_kp, gw_kp = kernels.moe_experts_backward(g, t["hidden"], idx, w, kp["gate_up_proj_blocks"],
                                                kp["gate_up_proj_scales"], kp["down_proj_blocks"],
                                                kp["down_proj_scales"], ws2, fac2)
    torch.cuda.synchronize()
    assert torch.equal(fac.view(torch.int16), fac2.view(torch.int16))
    assert torch.equal(gh.view(torch.int16), gh_kp.view(torch.int16))
    assert torch.equal(gw, gw_kp)
    announce("120b prefill backward: float32 autograd references")
    fac_pairs = _save_by_pair(fac, idx)
    rh, rw, _ = _fp32_grads(t, idx, w, g)
    mh, mw, flips = _fp32_grads(t, idx, w, g, fac_pairs)
    n = SHAPE.tokens * SHAPE.top_k * 2 * SHAPE.intermediate
    print(f"clamp decisions differing from float32: {flips} of {n}")
    assert flips <= n * 1e-5
    rel_h, max_h, scale_h = errors(gh, rh)
    rel_w, _, _ = errors(gw, rw)
    print(f"120b prefill vs float32 autograd: d hidden rel_l2={rel_h:.3e} max_abs={max_h:.3e} "
          f"(|ref|max {scale_h:.3e}); d weights rel_l2={rel_w:.3e}")
    assert rel_h <= GRAD_REL_L2 and rel_w <= GRAD_REL_L2
    assert_grad_close(gh, mh, "120b prefill d hidden (kernel's clamp decisions)")
    assert_grad_close(gw, mw, "120b prefill d routing weights (kernel's clamp decisions)")


def _bf16_arithmetic_flips(t, idx, limit=7.0):
    """Clamp decisions that the reference's own bf16 arithmetic takes
    differently from float32: it rounds the gate_up product to bf16 and adds
    the bf16 bias in bf16 (block_streamer/gptoss.py:158-166 on bf16 hidden
    states) before clamping (:131-133)."""
    h = t["hidden"].float()
    flips = 0
    for e in torch.unique(idx).tolist():
        tok, _ = torch.where(idx == e)
        wgu = kernels.dequantize_mxfp4(t["gate_up_proj_blocks"][e:e + 1], t["gate_up_proj_scales"][e:e + 1],
                                       torch.float32)[0]
        prod = h[tok] @ wgu
        bias = t["gate_up_proj_bias"][e]
        gu32 = prod + bias.float()
        gu16 = (prod.to(torch.bfloat16) + bias.to(torch.bfloat16)).float()
        flips += int(((gu16[:, 0::2] <= limit) != (gu32[:, 0::2] <= limit)).sum())
        flips += int(((gu16[:, 1::2].abs() <= limit) != (gu32[:, 1::2].abs() <= limit)).sum())
    return flips


def test_prefill_backward_mx_training(layer):
    """The training forward on the MX kernels (``path="mx"`` with the save;
    ``MXFP4Experts.mx_training``) at full size, followed by the backward.
    The block-scaled MFMA's accumulation moves more gate_up pre-activations
    across +-7 than the bf16 kernels do: the bars are the count of differing
    clamp decisions (at most 1e-5 of them, and no more than the reference's own
    bf16 arithmetic moves) and the gradients against float32 autograd whose
    clamp decisions follow the kernel's."""
    t = layer["t"]
    idx = layer["idx"]
    g = (torch.randn(SHAPE.tokens, SHAPE.hidden, generator=torch.Generator(device=t["hidden"].device)
                     .manual_seed(57), device=t["hidden"].device) * 1e-3).to(torch.bfloat16)
    w = layer["scores"].float()
    announce("120b prefill backward after the MX training forward")
    _, ws, fac = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(t), save=True, path="mx")
    gh, gw = kernels.moe_experts_backward(g, t["hidden"], idx, w, t["gate_up_proj_blocks"],
                                          t["gate_up_proj_scales"], t["down_proj_blocks"],
                                          t["down_proj_scales"], ws, fac)
    torch.cuda.synchronize()
    announce("120b prefill MX training: float32 references")
    mh, mw, flips = _fp32_grads(t, idx, w, g, _save_by_pair(fac, idx))
    ref_flips = _bf16_arithmetic_flips(t, idx)
    n = SHAPE.tokens * SHAPE.top_k * 2 * SHAPE.intermediate
    print(f"MX training: clamp decisions differing from float32: {flips} of {n}; the reference's bf16 "
          f"arithmetic: {ref_flips}")
    assert flips <= n * 1e-5 and flips <= ref_flips
    assert_grad_close(gh, mh, "120b MX training d hidden (kernel's clamp decisions)")
    assert_grad_close(gw, mw, "120b MX training d routing weights (kernel's clamp decisions)")
