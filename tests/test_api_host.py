"""Host-side behaviour of the drop-in module that needs no GPU."""

from __future__ import annotations

import pytest
import torch

from blockstreamer_amd import gptoss


def test_dequantize_expert_requires_expert_dimension():
    """tests/test_offload.py:405-414: 3-D input raises ValueError("packed blocks")."""
    blocks = torch.randint(0, 255, (64, 4, 16), dtype=torch.uint8)
    scales = torch.randint(120, 134, (64, 4), dtype=torch.uint8)
    with pytest.raises(ValueError, match="packed blocks"):
        gptoss.dequantize_expert(blocks, scales)


def test_cpu_tensors_are_refused_loudly():
    blocks = torch.randint(0, 255, (1, 64, 4, 16), dtype=torch.uint8)
    scales = torch.randint(120, 134, (1, 64, 4), dtype=torch.uint8)
    with pytest.raises(ValueError, match="GPU only"):
        gptoss.dequantize_expert(blocks, scales)


def test_scale_shape_mismatch():
    blocks = torch.zeros(1, 8, 4, 16, dtype=torch.uint8)
    scales = torch.zeros(1, 8, 3, dtype=torch.uint8)
    with pytest.raises(ValueError, match="does not match"):
        gptoss.dequantize_expert(blocks, scales)


def test_blocks_layout_and_shape_from_rank():
    from blockstreamer_amd import kernels
    ck = torch.zeros(3, 32, 6, 16, dtype=torch.uint8)
    kp = torch.zeros(3, 2, 3, 16, 2, 16, dtype=torch.uint8)
    assert kernels.blocks_layout(ck) == kernels.LAYOUT_CHECKPOINT
    assert kernels.blocks_layout(kp) == kernels.LAYOUT_KPAIR
    assert kernels.packed_shape(ck) == kernels.packed_shape(kp) == (3, 32, 6)
    for bad in (torch.zeros(3, 32, 6, 8, dtype=torch.uint8), torch.zeros(3, 2, 3, 16, 4, 16, dtype=torch.uint8),
                torch.zeros(32, 6, 16, dtype=torch.uint8)):
        with pytest.raises(ValueError, match="k-pair layout"):
            kernels.blocks_layout(bad)


def test_experts_refuse_mixed_layouts_before_the_gpu():
    """gate_up in one layout and down in the other is a shape error, raised
    before any device check."""
    from blockstreamer_amd import kernels
    E, k, H, I, T = 2, 1, 64, 64, 4
    h = torch.zeros(T, H, dtype=torch.bfloat16)
    idx = torch.zeros(T, k, dtype=torch.int64)
    w = torch.ones(T, k)
    gub = torch.zeros(E, 2 * I // 16, H // 64, 16, 2, 16, dtype=torch.uint8)   # k-pair
    gus = torch.zeros(E, 2 * I, H // 32, dtype=torch.uint8)
    dnb = torch.zeros(E, H, I // 32, 16, dtype=torch.uint8)                     # checkpoint
    dns = torch.zeros(E, H, I // 32, dtype=torch.uint8)
    with pytest.raises(ValueError, match="same layout"):
        kernels.moe_experts_forward(h, idx, w, gub, gus, None, dnb, dns, None)
    wrong_k = torch.zeros(E, 2 * I, H // 32 + 1, 16, dtype=torch.uint8)
    with pytest.raises(ValueError, match="gate_up_proj_blocks must be"):
        kernels.moe_experts_forward(h, idx, w, wrong_k, gus, None, dnb, dns, None)


def _small_experts(E=2, H=64, I=64, layout="checkpoint"):
    if layout == "kpair":
        gub = torch.zeros(E, 2 * I // 16, H // 64, 16, 2, 16, dtype=torch.uint8)
        dnb = torch.zeros(E, H // 16, I // 64, 16, 2, 16, dtype=torch.uint8)
    else:
        gub = torch.zeros(E, 2 * I, H // 32, 16, dtype=torch.uint8)
        dnb = torch.zeros(E, H, I // 32, 16, dtype=torch.uint8)
    return (gub, torch.zeros(E, 2 * I, H // 32, dtype=torch.uint8), torch.zeros(E, 2 * I, dtype=torch.bfloat16),
            dnb, torch.zeros(E, H, I // 32, dtype=torch.uint8), torch.zeros(E, H, dtype=torch.bfloat16))


@pytest.mark.parametrize("which,shape", [("gate_up_proj", (128,)), ("gate_up_proj", (2, 64)),
                                         ("down_proj", (2, 32)), ("down_proj", (3, 64))])
def test_experts_refuse_wrong_bias_shapes_before_the_gpu(which, shape):
    """The kernels read the biases as [E, 2I] and [E, H]; any other shape is a
    ValueError on the host (it would read past the tensor on the device)."""
    from blockstreamer_amd import kernels
    E, k, H, I, T = 2, 1, 64, 64, 4
    h = torch.zeros(T, H, dtype=torch.bfloat16)
    idx = torch.zeros(T, k, dtype=torch.int64)
    w = torch.ones(T, k)
    gub, gus, gubias, dnb, dns, dnbias = _small_experts(E, H, I)
    bad = torch.zeros(shape, dtype=torch.bfloat16)
    if which == "gate_up_proj":
        gubias = bad
    else:
        dnbias = bad
    with pytest.raises(ValueError, match=f"{which}_bias must be"):
        kernels.moe_experts_forward(h, idx, w, gub, gus, gubias, dnb, dns, dnbias)
    with pytest.raises(ValueError, match=f"{which}_bias must be"):
        kernels.MoEStages(h, idx, w, gub, gus, gubias, dnb, dns, dnbias)


def test_backward_refuses_bad_arguments_before_the_gpu():
    """Shapes and dtypes of every backward input are checked on the host."""
    from blockstreamer_amd import kernels
    E, k, H, I, T = 2, 2, 64, 64, 4
    h = torch.zeros(T, H, dtype=torch.bfloat16)
    idx = torch.zeros(T, k, dtype=torch.int64)
    w = torch.ones(T, k)
    gub, gus, _, dnb, dns, _ = _small_experts(E, H, I)
    ws = torch.zeros(1 << 20, dtype=torch.uint8)
    fac = torch.zeros(T * k, 2 * I, dtype=torch.bfloat16)
    g = torch.zeros(T, H, dtype=torch.bfloat16)

    def call(**over):
        args = dict(grad_out=g, hidden=h, router_indices=idx, routing_weights=w, gate_up_blocks=gub,
                    gate_up_scales=gus, down_blocks=dnb, down_scales=dns, workspace=ws, swiglu_grad=fac)
        args.update(over)
        return kernels.moe_experts_backward(**args)

    with pytest.raises(ValueError, match="grad_out must be"):
        call(grad_out=torch.zeros(T, H + 32, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="swiglu_grad must be"):
        call(swiglu_grad=fac.float())
    with pytest.raises(ValueError, match="swiglu_grad must be"):
        call(swiglu_grad=fac[:-1])
    with pytest.raises(ValueError, match="down_proj_blocks must be"):
        call(down_blocks=torch.zeros(E, H, I // 32 + 1, 16, dtype=torch.uint8))
    with pytest.raises(ValueError, match="gate_up_proj_scales must be"):
        call(gate_up_scales=gus[:, :-1])
    with pytest.raises(ValueError, match="routing_weights must match"):
        call(routing_weights=w[:, :1])
    with pytest.raises(ValueError, match="workspace"):
        call(workspace=ws[:16])
    with pytest.raises(ValueError, match="same layout"):
        kp = _small_experts(E, H, I, "kpair")
        call(gate_up_blocks=kp[0])
    # well-formed arguments get as far as the device check
    with pytest.raises(ValueError, match="GPU only"):
        call()


def _causal_additive(T: int) -> torch.Tensor:
    vis = torch.ones(T, T, dtype=torch.bool).tril()
    return torch.where(vis, 0.0, torch.finfo(torch.float32).min).reshape(1, 1, T, T)


def test_mask_kind_does_not_reuse_a_verdict_at_a_reused_address():
    """A causal mask is checked, then dropped; a padded mask of the same shape
    is then built in the same storage without a version bump (written
    through ``.data``), so it has the freed mask's address, shape and
    version.  It must still be refused: the verdict belongs to the checked
    tensor object, not to its address."""
    from blockstreamer_amd import attention

    buf = torch.empty(1, 1, 8, 8)
    buf.data.copy_(_causal_additive(8))
    first = buf.view(1, 1, 8, 8)
    assert attention.mask_kind(first, 8, 8, None) == (True, 0)
    ptr, version = first.data_ptr(), first._version
    del first
    padded = _causal_additive(8)
    padded[..., 0] = torch.finfo(torch.float32).min  # the first key is padding
    buf.data.copy_(padded)
    second = buf.view(1, 1, 8, 8)
    assert (second.data_ptr(), second._version) == (ptr, version)
    with pytest.raises(ValueError, match="no padding"):
        attention.mask_kind(second, 8, 8, None)


def test_mask_kind_verdict_is_reused_for_the_same_mask_and_dropped_on_change():
    from blockstreamer_amd import attention

    m = _causal_additive(8)
    assert attention.mask_kind(m, 8, 8, None) == (True, 0)
    assert attention.mask_kind(m, 8, 8, None) == (True, 0)  # the cached verdict
    m[..., 0] = torch.finfo(torch.float32).min              # an in-place edit bumps the version
    with pytest.raises(ValueError):
        attention.mask_kind(m, 8, 8, None)


def _tiny_gptoss(dtype):
    transformers = pytest.importorskip("transformers")
    from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssForCausalLM

    cfg = GptOssConfig(vocab_size=64, hidden_size=64, intermediate_size=64, num_hidden_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=16, num_local_experts=4,
                       num_experts_per_tok=2, sliding_window=16, max_position_embeddings=64, use_cache=False)
    torch.manual_seed(0)
    return cfg, GptOssForCausalLM(cfg).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_install_router_keeps_device_dtype_and_values(dtype):
    """The fused router replaces transformers' in place: on the old router's
    device, in its dtype (no silent recast of a float32 router), with its
    weight and bias values and their requires_grad."""
    cfg, model = _tiny_gptoss(dtype)
    model.model.layers[0].mlp.router.weight.requires_grad_(False)
    olds = [(layer.mlp.router.weight.detach().clone(), layer.mlp.router.bias.detach().clone(),
             layer.mlp.router.weight.requires_grad) for layer in model.model.layers]
    assert gptoss.install_mxfp4_router(model, cfg) == 2
    for layer, (w, b, rg) in zip(model.model.layers, olds):
        r = layer.mlp.router
        assert isinstance(r, gptoss.MXFP4TopKRouter)
        assert r.weight.device == w.device and r.weight.dtype == dtype and r.bias.dtype == dtype
        assert torch.equal(r.weight, w) and torch.equal(r.bias, b)
        assert r.weight.requires_grad == rg
    # an explicit dtype still wins
    cfg, model = _tiny_gptoss(torch.float32)
    assert gptoss.install_mxfp4_router(model, cfg, torch.bfloat16) == 2
    assert model.model.layers[1].mlp.router.weight.dtype == torch.bfloat16


def test_install_router_on_a_meta_model_stays_on_meta():
    transformers = pytest.importorskip("transformers")
    from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssForCausalLM

    cfg = GptOssConfig(vocab_size=64, hidden_size=64, intermediate_size=64, num_hidden_layers=1,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=16, num_local_experts=4,
                       num_experts_per_tok=2, max_position_embeddings=64)
    with torch.device("meta"):
        model = GptOssForCausalLM(cfg)
    assert gptoss.install_mxfp4_router(model, cfg) == 1
    assert model.model.layers[0].mlp.router.weight.device.type == "meta"
