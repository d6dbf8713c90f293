"""Input-gradient backward parity on the GPU (the LoRA training path).

Reference gradients come from torch autograd of the float32 oracle (CPU) or,
at the gpt-oss-20b shape, of a float32 torch reference on the GPU.
Tolerance for gradients: relative L2 <= 1e-2 and max-abs <= 5e-2 * max|ref|
-- the backward rounds twice more to bfloat16 than the forward (the weighted
output gradient and the gate_up gradient feed bf16 MFMAs).
"""

from __future__ import annotations

import pytest
import torch

import oracle
from blockstreamer_amd import gptoss, kernels, synthetic
from tests.conftest import announce
from tests.moe_util import errors, expert_args

pytestmark = pytest.mark.gpu

GRAD_REL_L2 = 1e-2
GRAD_MAX_ABS = 5e-2


def assert_grad_close(got, want, what):
    rel_l2, max_abs, scale = errors(got, want)
    msg = f"{what}: rel_l2={rel_l2:.3e} max_abs={max_abs:.3e} (|ref|max={scale:.3e})"
    print(msg)
    assert rel_l2 <= GRAD_REL_L2, msg
    assert max_abs <= GRAD_MAX_ABS * max(scale, 1e-30), msg


def _oracle_grads(t, idx, w, g):
    h = t["hidden"].cpu().float().requires_grad_(True)
    wr = w.cpu().float().requires_grad_(True)
    out = oracle.experts_ref(h, idx.cpu(), wr, *[a.cpu() for a in expert_args(t)])
    out.backward(g.cpu().float())
    return out.detach(), h.grad, wr.grad


def _gpu_grads(t, idx, w, g):
    h = t["hidden"].detach().clone().requires_grad_(True)
    wr = w.detach().clone().requires_grad_(True)
    args = expert_args(t)
    out = gptoss._MoEExperts.apply(h, idx, wr, *args, 1.702, 7.0)
    out.backward(g)
    return out.detach(), h.grad, wr.grad


CASES = [
    # (E, k, H, I, T, scale_lo, scale_hi)
    (8, 2, 256, 256, 64, 119, 129),
    (8, 2, 256, 256, 64, 116, 120),
    (16, 4, 512, 256, 129, 116, 120),
    (4, 1, 128, 192, 77, 117, 121),
    (4, 2, 64, 32, 5, 117, 121),   # one k-tile in both products, one column block
]


@pytest.mark.parametrize("case", CASES, ids=[f"E{c[0]}k{c[1]}H{c[2]}I{c[3]}T{c[4]}s{c[5]}" for c in CASES])
def test_backward_vs_oracle_autograd(device, case):
    E, k, H, I, T, lo, hi = case
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=T + E, scale_lo=lo,
                            scale_hi=hi, device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=T + 3, dtype=torch.float32, device=device)
    g = torch.randn(T, H, generator=torch.Generator().manual_seed(T), dtype=torch.float32)
    g = g.to(torch.bfloat16).to(device)
    announce(f"moe backward {case}")
    out, gh, gw = _gpu_grads(t, idx, w, g)
    _, rh, rw = _oracle_grads(t, idx, w, g)
    assert gh.dtype == torch.bfloat16 and gw.dtype == torch.float32
    assert_grad_close(gh, rh, f"d hidden {case}")
    assert_grad_close(gw, rw, f"d routing weights {case}")


def test_backward_through_module_like_recompute(device):
    """functional_call + autograd.grad on [hidden, weights], as _autograd.py:127-175 does."""
    from torch.func import functional_call
    from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig

    E, k, H, I, T = 8, 2, 256, 256, 48
    cfg = GptOssConfig(num_local_experts=E, hidden_size=H, intermediate_size=I,
                       num_experts_per_tok=k, num_hidden_layers=1)
    mod = gptoss.MXFP4Experts(cfg, torch.bfloat16)
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=41, scale_lo=116,
                            scale_hi=120, device=device)
    state = {n: t[n] for n in ("gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
                               "down_proj_blocks", "down_proj_scales", "down_proj_bias")}
    idx, w = synthetic.random_routing(T, E, k, seed=42, dtype=torch.bfloat16, device=device)
    h = t["hidden"].detach().clone().requires_grad_(True)
    wr = w.detach().clone().requires_grad_(True)
    announce("moe backward via functional_call")
    with torch.enable_grad():
        out = functional_call(mod, state, (h, idx, wr), strict=True)
        g = torch.ones_like(out)
        gh, gw = torch.autograd.grad(out, [h, wr], g)
    _, rh, rw = _oracle_grads(t, idx, w.float(), g.float())
    assert gw.dtype == torch.bfloat16
    assert_grad_close(gh, rh, "module d hidden")
    assert_grad_close(gw.float(), rw, "module d routing weights")


def test_no_grad_forward_saves_nothing(device):
    E, k, H, I, T = 8, 2, 256, 256, 16
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=5, scale_lo=119, scale_hi=125,
                            device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=6, device=device)
    with torch.no_grad():
        out = gptoss._MoEExperts.apply(t["hidden"], idx, w, *expert_args(t), 1.702, 7.0)
    assert out.grad_fn is None


def _gpu_fp32_reference_grads(t, idx, w, g):
    """float32 torch autograd on the GPU, dense weights from the dequant kernel."""
    h = t["hidden"].float().requires_grad_(True)
    wr = w.detach().float().clone().requires_grad_(True)
    out = torch.zeros_like(h)
    for e in torch.unique(idx).tolist():
        tok, pos = torch.where(idx == e)
        wgu = kernels.dequantize_mxfp4(t["gate_up_proj_blocks"][e:e + 1],
                                       t["gate_up_proj_scales"][e:e + 1], torch.float32)[0]
        wdn = kernels.dequantize_mxfp4(t["down_proj_blocks"][e:e + 1],
                                       t["down_proj_scales"][e:e + 1], torch.float32)[0]
        gu = h[tok] @ wgu + t["gate_up_proj_bias"][e].float()
        o = oracle.apply_gate_ref(gu) @ wdn + t["down_proj_bias"][e].float()
        out = out.index_add(0, tok, o * wr[tok, pos, None])
    out.backward(g.float())
    return h.grad, wr.grad


def test_backward_gptoss_20b_shape(device):
    E, k, H, I, T = 32, 4, 2880, 2880, 512
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=23, scale_lo=116, scale_hi=120,
                            device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=24, dtype=torch.float32, device=device)
    g = (torch.randn(T, H, device=device) * 0.1).to(torch.bfloat16)
    announce("moe backward 20b shape")
    _, gh, gw = _gpu_grads(t, idx, w, g)
    rh, rw = _gpu_fp32_reference_grads(t, idx, w, g)
    assert_grad_close(gh, rh, "20b d hidden")
    assert_grad_close(gw, rw, "20b d routing weights")


def test_mx_training_module_20b_shape(device):
    """``MXFP4Experts.mx_training``: the forward that saves for the backward
    runs the native MX kernels (its output equals the MX inference forward bit
    for bit), and the gradients meet the same bars against float32 autograd as
    the bf16 kernels' do (at these trained weight scales no clamp decision of
    the 11.8 million differs from float32's, for either kernel)."""
    from types import SimpleNamespace

    E, k, H, I, T = 32, 4, 2880, 2880, 512
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=23, scale_lo=116, scale_hi=120,
                            device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=24, dtype=torch.float32, device=device)
    g = (torch.randn(T, H, device=device) * 0.1).to(torch.bfloat16)
    cfg = SimpleNamespace(num_local_experts=E, hidden_size=H, intermediate_size=I, num_experts_per_tok=k)
    mod = gptoss.MXFP4Experts(cfg, torch.bfloat16)
    mod.mx_training = True
    state = {n: t[n] for n in ("gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
                               "down_proj_blocks", "down_proj_scales", "down_proj_bias")}
    h = t["hidden"].detach().clone().requires_grad_(True)
    wr = w.detach().clone().requires_grad_(True)
    announce("MX training forward + backward, 20b shape")
    out = torch.func.functional_call(mod, state, (h, idx, wr), strict=True)
    out.backward(g)
    mx_inference = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(t), path="mx")
    torch.cuda.synchronize()
    assert torch.equal(out.detach().view(torch.int16), mx_inference.view(torch.int16))
    rh, rw = _gpu_fp32_reference_grads(t, idx, w, g)
    assert_grad_close(h.grad, rh, "20b MX training d hidden")
    assert_grad_close(wr.grad, rw, "20b MX training d routing weights")


def _fp32_sum_bound(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Bound on the float32 summation error of x @ w: 4 * K * 2^-24 * (|x| @ |w|)."""
    return 4 * x.shape[-1] * 2.0 ** -24 * (x.double().abs() @ w.double().abs())


def test_mxfp4_matmul_gradient_and_memory(device):
    """tests/test_offload.py:369-402 on this build: float32 mxfp4_matmul is
    x @ dequantize_expert(...) to float32 accuracy (the packed kernels sum in
    another order than the library GEMM, so not bit for bit: within
    4 K 2^-24 |x||W| of the float64 product), the input gradient likewise, and
    no dense weight is retained across calls."""
    torch.manual_seed(0)
    blocks = torch.randint(0, 255, (1, 64, 4, 16), dtype=torch.uint8, device=device)
    scales = torch.randint(120, 134, (1, 64, 4), dtype=torch.uint8, device=device)
    weight = gptoss.dequantize_expert(blocks, scales, torch.float32)
    x = torch.randn(8, 128, device=device, requires_grad=True)
    announce("mxfp4_matmul gradient and memory")
    actual = gptoss.mxfp4_matmul(x, blocks, scales)
    assert actual.dtype == torch.float32 and actual.shape == (8, 64)
    exact = x.detach().double() @ weight.double()
    assert ((actual.double() - exact).abs() <= _fp32_sum_bound(x.detach(), weight)).all()
    assert torch.allclose(actual, x.detach() @ weight, rtol=1e-5, atol=1e-5)
    grad = torch.randn_like(actual)
    actual.backward(grad)
    gx = grad.double() @ weight.double().T
    assert ((x.grad.double() - gx).abs() <= _fp32_sum_bound(grad, weight.T)).all()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    chained = [gptoss.mxfp4_matmul(x, blocks, scales) for _ in range(64)]
    peak = torch.cuda.max_memory_allocated() - base
    sum(y.sum() for y in chained).backward()
    dense_bytes = weight.numel() * weight.element_size()
    assert peak < dense_bytes * 16


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows", [5, 200])
def test_mxfp4_matmul_gptoss_shape(device, dtype, rows):
    """gpt-oss gate_up weight (N = 5760 rows of K = 2880): the forward and the
    input gradient against float64 products of the exact weight, to the
    output dtype's rounding plus the float32 summation bound; the k-pair
    layout gives the same bits.  5 rows run the weight-streaming kernels, 200
    the tiled ones."""
    b, s = synthetic.packed_weights(1, 5760, 90, seed=rows, scale_lo=116, scale_hi=121, device=device)
    w = gptoss.dequantize_expert(b, s, torch.float32).double()
    g = torch.Generator().manual_seed(rows + 1)
    x = torch.randn(rows, 2880, generator=g).to(dtype).to(device)
    dy = torch.randn(rows, 5760, generator=g).to(dtype).to(device)
    announce(f"mxfp4_matmul gpt-oss shape {dtype} rows={rows}")
    y = kernels.mxfp4_matmul(x, b, s)
    gx = kernels.mxfp4_matmul(dy, b, s, transpose=True)
    y_kp = kernels.mxfp4_matmul(x, kernels.to_kpair(b), s)
    gx_kp = kernels.mxfp4_matmul(dy, kernels.to_kpair(b), s, transpose=True)
    torch.cuda.synchronize()
    assert y.dtype == dtype and gx.dtype == dtype
    eps = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -24}[dtype]
    for what, got, a, m in (("forward", y, x, w), ("input gradient", gx, dy, w.T)):
        exact = a.double() @ m
        bound = exact.abs() * eps + _fp32_sum_bound(a, m)
        err = (got.double() - exact).abs()
        print(f"{dtype} rows={rows} {what}: max err / bound {(err / bound).max().item():.3f}")
        assert (err <= bound).all(), what
    assert torch.equal(y, y_kp) and torch.equal(gx, gx_kp)


def test_mxfp4_matmul_under_autocast(device):
    """Inside torch.autocast(bfloat16) the product runs in bfloat16 and
    returns it, as x @ W does there; the input gradient comes back in the
    input's dtype (block_streamer/_autograd.py:144-151 recomputes under the
    caller's autocast)."""
    b, s = synthetic.packed_weights(1, 256, 8, seed=3, scale_lo=118, scale_hi=122, device=device)
    w = gptoss.dequantize_expert(b, s, torch.float32)
    x = torch.randn(32, 256, device=device, requires_grad=True)
    announce("mxfp4_matmul under autocast")
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = gptoss.mxfp4_matmul(x, b, s)
        ref = x @ w
    assert y.dtype == ref.dtype == torch.bfloat16
    exact = x.detach().to(torch.bfloat16).double() @ w.double()
    assert ((y.double() - exact).abs() <= exact.abs() * 2.0 ** -8 + _fp32_sum_bound(x.detach(), w)).all()
    y.float().sum().backward()
    assert x.grad.dtype == torch.float32 and torch.isfinite(x.grad).all()
    gx = torch.ones(32, 256, device=device, dtype=torch.float64) @ w.double().T
    assert torch.allclose(x.grad.double(), gx, rtol=2e-2, atol=1e-3)


def test_mlp_under_autocast_vs_oracle(device):
    """MXFP4MLP (router + experts) under torch.autocast(bfloat16) on float32
    activations: the layer bar against the float32 oracle, the output in the
    input dtype."""
    shape = synthetic.MoEShape(8, 2, 256, 256, 64)
    t = synthetic.moe_layer(shape, seed=81, scale_lo=116, scale_hi=120, router_bias_std=0.01)
    from types import SimpleNamespace
    cfg = SimpleNamespace(num_local_experts=8, hidden_size=256, intermediate_size=256, num_experts_per_tok=2)
    mlp = gptoss.MXFP4MLP(cfg, torch.bfloat16)
    state = {"router.weight": t["router_weight"].float(), "router.bias": t["router_bias"].float()}
    for n in expert_args_names():
        state["experts." + n] = t[n]
    state = {n: v.to(device) for n, v in state.items()}
    h = t["hidden"].float().to(device).reshape(1, 64, 256)
    announce("MXFP4MLP under autocast")
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out, scores = torch.func.functional_call(mlp, state, (h,), strict=True)
    # the routing the module took (its router kernel, run again on the same inputs)
    _, _, idx = kernels.router_forward(h.reshape(64, 256), state["router.weight"], state["router.bias"], 2)
    want = oracle.experts_ref(t["hidden"].float(), idx.cpu(), scores.detach().cpu().float(),
                              *[t[n] for n in expert_args_names()])
    from tests.moe_util import assert_layer_close
    assert out.dtype == torch.float32
    assert_layer_close(out.reshape(64, 256), want, "MXFP4MLP under autocast", absolute=True)


def expert_args_names():
    return ("gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
            "down_proj_blocks", "down_proj_scales", "down_proj_bias")


def _shift(x: torch.Tensor, by: int) -> torch.Tensor:
    """Same bytes (uint8), storage starting `by` bytes past a 16-byte boundary."""
    buf = torch.empty(x.numel() + 16, dtype=x.dtype, device=x.device)
    off = (by - buf.data_ptr()) % 16
    v = buf[off:off + x.numel()].view(x.shape)
    v.copy_(x)
    assert v.data_ptr() % 16 == by
    return v


def _backward_call(t, idx, w, g, blocks_scales):
    _, ws, pre = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(t), save=True)
    gub, gus, dnb, dns = blocks_scales
    return kernels.moe_experts_backward(g, t["hidden"], idx, w, gub, gus, dnb, dns, ws, pre)


@pytest.mark.parametrize("by", [8, 4, 1])
def test_backward_unaligned_weight_views(device, by):
    """Weights viewed `by` bytes past a 16-byte boundary (staging-blob views are
    8-byte aligned): 8 and 4 take the 4-byte DMA kernel, 1 a copy made by the
    wrapper.  Every result is the aligned call's, bit for bit."""
    E, k, H, I, T = 8, 2, 256, 256, 40
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=61, scale_lo=116,
                            scale_hi=122, device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=62, dtype=torch.float32, device=device)
    g = torch.randn(T, H, device=device).to(torch.bfloat16)
    keys = ("gate_up_proj_blocks", "gate_up_proj_scales", "down_proj_blocks", "down_proj_scales")
    announce(f"moe backward, weight views {by} bytes off alignment")
    gh0, gw0 = _backward_call(t, idx, w, g, [t[n] for n in keys])
    gh1, gw1 = _backward_call(t, idx, w, g, [_shift(t[n], by) for n in keys])
    torch.cuda.synchronize()
    assert torch.equal(gh0, gh1) and torch.equal(gw0, gw1)


def test_backward_c_abi_rejects_unaligned_weights(device, monkeypatch):
    """The C entry point refuses weights that are not 4-byte aligned."""
    E, k, H, I, T = 8, 2, 256, 256, 8
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=63, scale_lo=116, scale_hi=122,
                            device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=64, dtype=torch.float32, device=device)
    g = torch.randn(T, H, device=device).to(torch.bfloat16)
    monkeypatch.setattr(kernels, "_aligned", lambda x, n: x)
    keys = ("gate_up_proj_blocks", "gate_up_proj_scales", "down_proj_blocks", "down_proj_scales")
    bs = [t[n] for n in keys]
    bs[3] = _shift(bs[3], 2)
    announce("moe backward C-ABI, unaligned down scales")
    with pytest.raises(ValueError, match="4-byte aligned"):
        _backward_call(t, idx, w, g, bs)


def _shift2(x: torch.Tensor) -> torch.Tensor:
    """Same values, storage starting 2 bytes past a 16-byte boundary."""
    buf = torch.empty(x.numel() + 16, dtype=x.dtype, device=x.device)
    off = (2 // x.element_size() - buf.data_ptr() // x.element_size()) % (16 // x.element_size())
    v = buf[off:off + x.numel()].view(x.shape)
    v.copy_(x)
    assert v.data_ptr() % 16 == 2
    return v


def test_backward_grad_out_dtypes_and_layouts(device):
    """bf16, float32 and float16 output gradients (vectorised prep) and a bf16
    view 2 bytes off alignment (element-wise prep) give the same gradients."""
    E, k, H, I, T = 8, 2, 256, 256, 24
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=71, scale_lo=116,
                            scale_hi=122, device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=72, dtype=torch.float32, device=device)
    # multiples of 1/64 in [-1, 1): exact in every dtype
    g = (torch.randint(-64, 64, (T, H), device=device) / 64).to(torch.bfloat16)
    keys = ("gate_up_proj_blocks", "gate_up_proj_scales", "down_proj_blocks", "down_proj_scales")
    bs = [t[n] for n in keys]
    announce("moe backward, grad_out dtypes and layouts")
    gh0, gw0 = _backward_call(t, idx, w, g, bs)
    for what, gg in (("float32", g.float()), ("float16", g.half()), ("unaligned", _shift2(g))):
        gh1, gw1 = _backward_call(t, idx, w, gg, bs)
        torch.cuda.synchronize()
        assert torch.equal(gh0, gh1), what
        assert torch.allclose(gw0, gw1, rtol=1e-5, atol=1e-6), what
