"""The drop-in inside transformers' own GptOssDecoderLayer, called the way a
layer-streaming runner calls it: packed experts and the fused post-attention
norm installed (the fused router as well in the whole-model test).

Per layer: the layer's parameters arrive through
``torch.func.functional_call(layer, state, args, kwargs, strict=True)`` with
the packed expert tensors staged under their checkpoint names, the layer's
inputs and keyword arguments are exactly the ones the model's own forward
passes (captured with pre-hooks), and no staged tensor may be modified
(block_streamer/streamer.py:151-180).  The backward is the recompute form:
the layer is called again under ``enable_grad`` and ``autograd.grad`` taken
with respect to the hidden states (block_streamer/_autograd.py:125-175).

Reference: the same transformers layer in float32 with dense float32 expert
weights dequantised (bit-exactly) from the packed tensors, fed the routing
our layer chose, so that near-tied router logits cannot pick different
experts.  Bars: the layer bar for the experts output (relative L2 <= 5e-3,
max-abs <= 2e-2 of the largest value) and the gradient bar for the
hidden-state gradient through the whole layer (relative L2 <= 1e-2).
"""

from __future__ import annotations

import copy

import pytest
import torch

from blockstreamer_amd import gptoss, kernels, synthetic
from tests.conftest import announce
from tests.moe_util import errors

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")
from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig  # noqa: E402
from transformers.models.gpt_oss.modeling_gpt_oss import GptOssForCausalLM  # noqa: E402

E, K, H, I, L, S = 8, 2, 256, 256, 2, 48
PACKED = ("gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
          "down_proj_blocks", "down_proj_scales", "down_proj_bias")


def _config() -> GptOssConfig:
    cfg = GptOssConfig(vocab_size=64, hidden_size=H, intermediate_size=I, num_hidden_layers=L,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                       num_local_experts=E, num_experts_per_tok=K, sliding_window=16,
                       max_position_embeddings=128, use_cache=False)
    cfg._attn_implementation = "eager"
    return cfg


def _build(device):
    """Reference model (bf16, dense experts from the packed tensors), its
    float32 copy, our model (packed experts installed) and per-layer packs."""
    torch.manual_seed(0)
    cfg = _config()
    ref = GptOssForCausalLM(cfg).to(device=device, dtype=torch.bfloat16).eval()
    packs = [synthetic.moe_layer(synthetic.MoEShape(E, K, H, I, S), seed=100 + i, scale_lo=116,
                                 scale_hi=122, device=device) for i in range(L)]
    for layer, p in zip(ref.model.layers, packs):
        ex = layer.mlp.experts
        with torch.no_grad():
            ex.gate_up_proj.copy_(kernels.dequantize_mxfp4(p["gate_up_proj_blocks"], p["gate_up_proj_scales"]))
            ex.down_proj.copy_(kernels.dequantize_mxfp4(p["down_proj_blocks"], p["down_proj_scales"]))
            ex.gate_up_proj_bias.copy_(p["gate_up_proj_bias"])
            ex.down_proj_bias.copy_(p["down_proj_bias"])
    ref32 = copy.deepcopy(ref).float()
    for layer, p in zip(ref32.model.layers, packs):
        ex = layer.mlp.experts
        with torch.no_grad():  # exact: every MXFP4 value is a float32
            ex.gate_up_proj.copy_(kernels.dequantize_mxfp4(p["gate_up_proj_blocks"], p["gate_up_proj_scales"],
                                                           torch.float32))
            ex.down_proj.copy_(kernels.dequantize_mxfp4(p["down_proj_blocks"], p["down_proj_scales"],
                                                        torch.float32))
    ours = copy.deepcopy(ref)
    assert gptoss.install_mxfp4_experts(ours, cfg, torch.bfloat16) == L
    assert gptoss.install_fused_post_attention_norm(ours) == L
    return cfg, ref, ref32, ours, packs


def _layer_state(ref_layer, pack) -> dict:
    """What a streaming runner stages for one layer: every parameter by name,
    the experts as their packed checkpoint tensors."""
    state = {n: p.detach() for n, p in ref_layer.named_parameters() if not n.startswith("mlp.experts.")}
    for n in PACKED:
        state[f"mlp.experts.{n}"] = pack[n]
    return state


def _capture_layer_inputs(model, x):
    calls = []
    hooks = [lyr.register_forward_pre_hook(lambda m, a, kw: calls.append((a, kw)), with_kwargs=True)
             for lyr in model.model.layers]
    with torch.no_grad():
        model.model(inputs_embeds=x, use_cache=False)
    for h in hooks:
        h.remove()
    return calls


def _run_layer(layer, state, args, kwargs, grad=False):
    """functional_call as the runner does; returns the output, the MLP's input,
    the router's (scores, indices), the experts' output and the post-attention
    norm's input."""
    seen = {}
    hooks = [
        layer.post_attention_layernorm.register_forward_hook(lambda m, a, o: seen.__setitem__("norm_in", a[0])),
        layer.mlp.register_forward_hook(lambda m, a, o: seen.__setitem__("mlp_in", a[0])),
        layer.mlp.router.register_forward_hook(lambda m, a, o: seen.__setitem__("route", (o[1], o[2]))),
        layer.mlp.experts.register_forward_hook(lambda m, a, o: seen.__setitem__("experts", o)),
    ]
    versions = {n: t._version for n, t in state.items()}
    try:
        with torch.set_grad_enabled(grad):
            out = torch.func.functional_call(layer, state, args, kwargs, strict=True)
    finally:
        for h in hooks:
            h.remove()
    assert all(t._version == versions[n] for n, t in state.items()), "a staged tensor was modified"
    return out, seen


def test_decoder_layers_forward_vs_float32_transformers(device):
    cfg, ref, ref32, ours, packs = _build(device)
    x = (torch.randn(1, S, H, generator=torch.Generator().manual_seed(1)) * 0.5).to(torch.bfloat16).to(device)
    calls = _capture_layer_inputs(ref, x)
    announce("decoder layers forward, functional_call")
    for i, (args, kwargs) in enumerate(calls):
        state = _layer_state(ref.model.layers[i], packs[i])
        out, seen = _run_layer(ours.model.layers[i], state, args, kwargs)
        assert out.shape == args[0].shape and out.dtype == torch.bfloat16 and torch.isfinite(out).all()
        # the fused post-attention norm against the transformers module it
        # replaced, on the same input: at most one bf16 ulp apart
        want_norm = ref.model.layers[i].post_attention_layernorm(seen["norm_in"])
        a, b = seen["mlp_in"].float(), want_norm.float()
        assert ((a - b).abs() <= 2.0 ** -7 * b.abs() * (1 + 1e-5) + 1e-30).all()
        print(f"layer {i}: norm differs from transformers on {(a != b).float().mean().item():.3%}")
        scores, idx = seen["route"]
        tokens = seen["mlp_in"].reshape(-1, H)
        want = ref32.model.layers[i].mlp.experts(tokens.float(), idx, scores.float())
        got = seen["experts"].reshape(-1, H)
        rel_l2, max_abs, scale = errors(got, want)
        print(f"layer {i}: experts rel_l2={rel_l2:.3e} max_abs={max_abs:.3e} (|ref|max={scale:.3e})")
        assert rel_l2 <= 5e-3 and max_abs <= 2e-2 * scale


class _FixedRouting(torch.nn.Module):
    """float32 router logits, top-k taken at given indices (differentiable)."""

    def __init__(self, router, idx):
        super().__init__()
        self.router, self.idx = router, idx

    def forward(self, h):
        logits = torch.nn.functional.linear(h, self.router.weight, self.router.bias)
        vals = logits.gather(-1, self.idx)
        return logits, torch.softmax(vals, dim=-1), self.idx


def test_decoder_layer_recompute_backward(device):
    cfg, ref, ref32, ours, packs = _build(device)
    x = (torch.randn(1, S, H, generator=torch.Generator().manual_seed(2)) * 0.5).to(torch.bfloat16).to(device)
    calls = _capture_layer_inputs(ref, x)
    g = (torch.randn(1, S, H, generator=torch.Generator().manual_seed(3)) * 0.1).to(torch.bfloat16).to(device)
    announce("decoder layer recompute backward")
    for i, (args, kwargs) in enumerate(calls):
        state = _layer_state(ref.model.layers[i], packs[i])
        h = args[0].detach().clone().requires_grad_(True)
        out, seen = _run_layer(ours.model.layers[i], state, (h,), kwargs, grad=True)
        (gh,) = torch.autograd.grad(out, [h], g)
        # float32 reference through the same layer, with our routing
        lyr32 = copy.deepcopy(ref32.model.layers[i])
        lyr32.mlp.router = _FixedRouting(lyr32.mlp.router, seen["route"][1])
        kw32 = {k: (tuple(t.float() for t in v) if k == "position_embeddings" else
                    v.float() if torch.is_tensor(v) and v.is_floating_point() else v)
                for k, v in kwargs.items()}
        h32 = args[0].detach().float().requires_grad_(True)
        (gh32,) = torch.autograd.grad(lyr32(h32, **kw32), [h32], g.float())
        rel_l2, max_abs, scale = errors(gh, gh32)
        print(f"layer {i}: d hidden rel_l2={rel_l2:.3e} max_abs={max_abs:.3e} (|ref|max={scale:.3e})")
        assert gh.dtype == torch.bfloat16 and torch.isfinite(gh).all()
        assert rel_l2 <= 1e-2


@pytest.mark.parametrize("mask", ["runner", "model"])
def test_decoder_layer_native_attention(device, mask):
    """The layer on the HIP attention as well, called as the streaming runner
    calls it (attention_mask=None: every key visible, runners.py:327-335) or
    with the model's own causal / sliding-window masks; forward and the
    recompute backward against the float32 layer (eager attention) with our
    routing."""
    cfg, ref, ref32, ours, packs = _build(device)
    assert gptoss.install_native_attention(ours) == L
    x = (torch.randn(1, S, H, generator=torch.Generator().manual_seed(5)) * 0.5).to(torch.bfloat16).to(device)
    calls = _capture_layer_inputs(ref, x)
    g = (torch.randn(1, S, H, generator=torch.Generator().manual_seed(6)) * 0.1).to(torch.bfloat16).to(device)
    announce(f"decoder layer on the native attention, mask {mask}")
    for i, (args, kwargs) in enumerate(calls):
        kw = dict(kwargs)
        if mask == "runner":
            kw["attention_mask"] = None
        state = _layer_state(ref.model.layers[i], packs[i])
        h = args[0].detach().clone().requires_grad_(True)
        out, seen = _run_layer(ours.model.layers[i], state, (h,), kw, grad=True)
        (gh,) = torch.autograd.grad(out, [h], g)
        lyr32 = copy.deepcopy(ref32.model.layers[i])
        lyr32.mlp.router = _FixedRouting(lyr32.mlp.router, seen["route"][1])
        kw32 = {k: (tuple(t.float() for t in v) if k == "position_embeddings" else
                    v.float() if torch.is_tensor(v) and v.is_floating_point() else v)
                for k, v in kw.items()}
        h32 = args[0].detach().float().requires_grad_(True)
        out32 = lyr32(h32, **kw32)
        (gh32,) = torch.autograd.grad(out32, [h32], g.float())
        rel_o, _, _ = errors(out, out32)
        rel_g, _, _ = errors(gh, gh32)
        print(f"layer {i} ({mask}): out rel_l2={rel_o:.3e}  d hidden rel_l2={rel_g:.3e}")
        assert torch.isfinite(out).all() and torch.isfinite(gh).all()
        assert rel_o <= 1e-2 and rel_g <= 1e-2


def test_whole_model_with_fused_router_through_functional_call(device):
    """Both drop-ins (experts and fused router) in the model, every parameter
    bound by one functional_call: runs, leaves the staged tensors alone, and
    tracks the bf16 transformers model (routing may differ on near ties)."""
    cfg, ref, ref32, ours, packs = _build(device)
    assert gptoss.install_mxfp4_router(ours, cfg, torch.bfloat16) == L
    state = {n: p.detach() for n, p in ref.model.named_parameters() if ".mlp.experts." not in n}
    state.update({n: b for n, b in ref.model.named_buffers()})
    for i, p in enumerate(packs):
        for n in PACKED:
            state[f"layers.{i}.mlp.experts.{n}"] = p[n]
    x = (torch.randn(1, S, H, generator=torch.Generator().manual_seed(4)) * 0.5).to(torch.bfloat16).to(device)
    versions = {n: t._version for n, t in state.items()}
    announce("whole model, fused router and experts")
    with torch.no_grad():
        got = torch.func.functional_call(ours.model, state, (), {"inputs_embeds": x, "use_cache": False},
                                         strict=True).last_hidden_state
        want = ref.model(inputs_embeds=x, use_cache=False).last_hidden_state
    assert all(t._version == versions[n] for n, t in state.items())
    rel_l2, _, _ = errors(got, want)
    print(f"whole model vs bf16 transformers: rel_l2={rel_l2:.3e}")
    # a sanity bound only: the two bf16 routers round their logits differently,
    # so a near-tied token may take another expert and move its output a lot
    # (measured 4.8e-2 here); the per-layer tests above carry the numerics bar
    assert torch.isfinite(got).all() and rel_l2 <= 0.15
