"""Attention with sinks on the HIP kernels against the oracle.

The oracle (``oracle.attention_ref``, pinned against transformers'
``eager_attention_forward`` on the CPU) runs in float64 on the same
bf16-rounded inputs.  Forward bar: the layer bar for bf16 activations
(relative L2 <= 5e-3, max-abs <= 2e-2 of the output scale).  Backward bar:
relative L2 <= 1e-2 per gradient (the probabilities and dS enter the
bf16 MFMAs rounded; the gradients are rounded to bf16 once).
"""

from __future__ import annotations

import copy

import pytest
import torch

import oracle
from blockstreamer_amd import attention as A
from tests.conftest import announce

pytestmark = pytest.mark.gpu

FWD_REL_L2 = 5e-3
FWD_MAX_ABS = 2e-2
BWD_REL_L2 = 1e-2


def _rel_l2(got: torch.Tensor, want: torch.Tensor) -> float:
    g, w = got.double().cpu(), want.double().cpu()
    return float((g - w).norm() / w.norm().clamp_min(1e-30))


def _inputs(B, Hq, Hkv, Tq, Tk, device, seed=0, layout="bthd", sinks=True):
    g = torch.Generator().manual_seed(seed)

    def make(H, T):
        x = torch.randn(B, T, H, 64, generator=g).to(torch.bfloat16)
        if layout == "bthd":  # the projection output viewed [B, H, T, D] (q_proj(..).view().transpose())
            return x.to(device).transpose(1, 2)
        return x.transpose(1, 2).contiguous().to(device)  # [B, H, T, D] contiguous (after RoPE)

    q, k, v = make(Hq, Tq), make(Hkv, Tk), make(Hkv, Tk)
    s = (torch.randn(Hq, generator=g) * 2).to(device) if sinks else None
    return q, k, v, s


def _check_fwd(got, q, k, v, s, scaling, causal, window, what):
    want = oracle.attention_ref(q.cpu(), k.cpu(), v.cpu(), None if s is None else s.cpu(), scaling,
                                causal=causal, window=window)
    rel = _rel_l2(got, want)
    mx = float((got.double().cpu() - want).abs().max())
    scale = float(want.abs().max())
    print(f"{what}: rel_l2={rel:.3e} max_abs={mx:.3e} (|max| {scale:.3e})")
    assert rel <= FWD_REL_L2, what
    assert mx <= FWD_MAX_ABS * max(1.0, scale), what


CASES = [
    # B, Hq, Hkv, Tq, Tk, causal, window
    (2, 8, 2, 100, 100, True, 0),
    (1, 8, 2, 70, 70, False, 0),
    (2, 8, 2, 200, 200, True, 16),
    (1, 64, 8, 1, 300, True, 0),
    (1, 64, 8, 1, 300, True, 128),
    (2, 8, 8, 5, 77, True, 0),
    (1, 4, 1, 33, 129, False, 0),
    (1, 64, 8, 257, 257, True, 128),
]


@pytest.mark.parametrize("B,Hq,Hkv,Tq,Tk,causal,window", CASES)
def test_forward_vs_oracle(device, B, Hq, Hkv, Tq, Tk, causal, window):
    announce(f"attention fwd B={B} Hq={Hq} Hkv={Hkv} Tq={Tq} Tk={Tk} causal={causal} window={window}")
    q, k, v, s = _inputs(B, Hq, Hkv, Tq, Tk, device, seed=Tq + 7 * Tk)
    got = A.attention_forward(q, k, v, s, 0.125, causal, window)
    torch.cuda.synchronize()
    assert got.shape == (B, Tq, Hq, 64)
    _check_fwd(got, q, k, v, s, 0.125, causal, window, f"fwd {B},{Hq},{Hkv},{Tq},{Tk},{causal},{window}")


@pytest.mark.parametrize("layout", ["bthd", "bhtd"])
def test_forward_layouts_and_no_sink(device, layout):
    announce(f"attention fwd layout {layout}")
    for sinks in (True, False):
        q, k, v, s = _inputs(1, 16, 4, 130, 130, device, seed=3, layout=layout, sinks=sinks)
        got = A.attention_forward(q, k, v, s, 0.125, True, 0)
        _check_fwd(got, q, k, v, s, 0.125, True, 0, f"layout {layout} sinks {sinks}")


def test_forward_deterministic_and_lse(device):
    announce("attention fwd determinism, lse")
    q, k, v, s = _inputs(1, 64, 8, 96, 96, device, seed=5)
    a, lse = A.attention_forward(q, k, v, s, 0.125, True, 0, return_lse=True)
    b = A.attention_forward(q, k, v, s, 0.125, True, 0)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    # lse: log2 of sum_j 2^(s_j) + 2^(sink) in units of scaling * log2(e)
    qd, kd = q.double().cpu(), k.double().cpu().repeat_interleave(8, dim=1)
    z = (qd @ kd.transpose(2, 3)) * 0.125
    z = z.masked_fill(torch.ones(96, 96, dtype=torch.bool).triu(1), float("-inf"))
    z = torch.cat([z, s.double().cpu().reshape(1, 64, 1, 1).expand(1, 64, 96, 1)], -1)
    want = torch.logsumexp(z, -1) / torch.log(torch.tensor(2.0, dtype=torch.float64))
    torch.testing.assert_close(lse.double().cpu(), want, rtol=1e-4, atol=1e-3)


SPLIT_CASES = [
    # B, Hq, Hkv, Tq, Tk, causal, window, sinks: short query grids, keys split over workgroups
    (1, 64, 8, 1, 4096, True, 0, True),
    (1, 64, 8, 1, 4096, True, 1000, True),
    (2, 64, 8, 1, 1000, False, 0, True),
    (1, 64, 8, 4, 2049, True, 0, False),
    (3, 8, 2, 1, 600, True, 0, True),
    (1, 64, 8, 1, 2563, True, 0, True),
    (4, 64, 8, 2, 700, True, 600, True),
]


def _single_launch(q, k, v, s, scaling, causal, window):
    """bsa_attention_fwd (one launch, no split) on the same inputs: output and lse."""
    from blockstreamer_amd import _lib
    B, Hq, Tq, D = q.shape
    Hkv, Tk = k.shape[1], k.shape[2]
    out = torch.empty(B, Tq, Hq, D, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(B, Hq, Tq, dtype=torch.float32, device=q.device)
    sf = s.float().contiguous() if s is not None else None
    _lib.call("bsa_attention_fwd", q.data_ptr(), A._strides(q, 2, 1), k.data_ptr(), A._strides(k, 2, 1),
              v.data_ptr(), A._strides(v, 2, 1), sf.data_ptr() if sf is not None else None,
              B, Tq, Tk, Hq, Hkv, D, 1 if causal else 0, window, scaling, out.data_ptr(), A._strides(out, 1, 2),
              lse.data_ptr(), _lib.stream_handle(q.device))
    return out, lse


def _lse_ref(q, k, s, scaling, causal, window):
    """float64 log2 of sum_j 2^(visible scaled logits) + 2^(sink), in units of scaling * log2(e)."""
    G = q.shape[1] // k.shape[1]
    qd, kd = q.double().cpu(), k.double().cpu().repeat_interleave(G, dim=1)
    z = (qd @ kd.transpose(2, 3)) * scaling
    Tq, Tk = q.shape[2], k.shape[2]
    if causal:
        z = z.masked_fill(~A._pattern(Tq, Tk, window, "cpu"), float("-inf"))
    if s is not None:
        B, Hq = q.shape[0], q.shape[1]
        z = torch.cat([z, s.double().cpu().reshape(1, Hq, 1, 1).expand(B, Hq, Tq, 1)], -1)
    return torch.logsumexp(z, -1) / torch.log(torch.tensor(2.0, dtype=torch.float64))


@pytest.mark.parametrize("B,Hq,Hkv,Tq,Tk,causal,window,sinks", SPLIT_CASES)
def test_split_forward_vs_oracle_and_single_launch(device, B, Hq, Hkv, Tq, Tk, causal, window, sinks):
    from blockstreamer_amd import _lib
    announce(f"attention split fwd B={B} Hq={Hq} Hkv={Hkv} Tq={Tq} Tk={Tk} causal={causal} window={window}")
    assert _lib.lib().bsa_attention_split_workspace_bytes(B, Tq, Tk, Hq, Hkv, int(causal), window) > 0
    q, k, v, s = _inputs(B, Hq, Hkv, Tq, Tk, device, seed=Tk + 13 * Tq, sinks=sinks)
    got, lse = A.attention_forward(q, k, v, s, 0.125, causal, window, return_lse=True)
    again = A.attention_forward(q, k, v, s, 0.125, causal, window)
    one, lse1 = _single_launch(q, k, v, s, 0.125, causal, window)
    torch.cuda.synchronize()
    assert torch.equal(got, again)  # the merge adds the splits in a fixed order
    _check_fwd(got, q, k, v, s, 0.125, causal, window, f"split {B},{Hq},{Hkv},{Tq},{Tk},{causal},{window}")
    rel = _rel_l2(got, one)
    print(f"split vs single launch: rel_l2={rel:.3e}")
    assert rel <= 4e-3  # the probabilities round to bf16 against each split's own running maximum
    torch.testing.assert_close(lse, lse1, rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(lse.double().cpu(), _lse_ref(q, k, s, 0.125, causal, window), rtol=1e-4, atol=1e-3)


BWD_CASES = [
    (1, 64, 8, 1, 1000, True, 0),  # a decode step: the forward splits the keys, its lse feeds the backward
    (1, 8, 2, 100, 100, True, 0),
    (2, 8, 2, 70, 70, False, 0),
    (1, 8, 2, 200, 200, True, 16),
    (1, 64, 8, 3, 150, True, 0),
    (1, 64, 8, 192, 192, True, 128),
    (1, 4, 4, 50, 130, True, 0),
]


@pytest.mark.parametrize("B,Hq,Hkv,Tq,Tk,causal,window", BWD_CASES)
def test_backward_vs_oracle_autograd(device, B, Hq, Hkv, Tq, Tk, causal, window):
    announce(f"attention bwd B={B} Hq={Hq} Hkv={Hkv} Tq={Tq} Tk={Tk} causal={causal} window={window}")
    q, k, v, s = _inputs(B, Hq, Hkv, Tq, Tk, device, seed=11 + Tq)
    g = torch.Generator().manual_seed(99)
    dout = torch.randn(B, Tq, Hq, 64, generator=g).to(torch.bfloat16)
    qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    sg = s.detach().clone().requires_grad_(True)
    out = A.attention(qg, kg, vg, sg, 0.125, causal, window)
    out.backward(dout.to(device))
    torch.cuda.synchronize()
    qr, kr, vr = (t.detach().cpu().double().requires_grad_(True) for t in (q, k, v))
    sr = s.detach().cpu().double().requires_grad_(True)
    ref = oracle.attention_ref(qr, kr, vr, sr, 0.125, causal=causal, window=window)
    ref.backward(dout.double())
    for name, got, want in (("dq", qg.grad, qr.grad), ("dk", kg.grad, kr.grad), ("dv", vg.grad, vr.grad),
                            ("dsinks", sg.grad, sr.grad)):
        assert got.shape == want.shape, name
        rel = _rel_l2(got, want)
        print(f"{name}: rel_l2={rel:.3e}")
        assert rel <= BWD_REL_L2, name


def test_backward_deterministic(device):
    announce("attention bwd determinism")
    q, k, v, s = _inputs(1, 64, 8, 128, 128, device, seed=21)
    dout = torch.randn(1, 128, 64, 64, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(device)
    out, lse = A.attention_forward(q, k, v, s, 0.125, True, 0, return_lse=True)
    r1 = A.attention_backward(dout, q, k, v, s, out, lse, 0.125, True, 0)
    r2 = A.attention_backward(dout, q, k, v, s, out, lse, 0.125, True, 0)
    torch.cuda.synchronize()
    for a, b in zip(r1[:3], r2[:3]):
        assert torch.equal(a, b)


def test_gpt_oss_attention_module(device):
    """GptOssAttention from transformers on the registered implementation
    against the same module on eager attention (float32, CPU), with the masks
    transformers builds: none, causal, sliding window."""
    tf = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")
    from transformers import GptOssConfig
    from transformers.masking_utils import causal_mask_function, eager_mask, sliding_window_causal_mask_function

    announce("GptOssAttention on the registered implementation")
    A.register()
    T = 96
    cfg = GptOssConfig(hidden_size=256, num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                       sliding_window=24, num_hidden_layers=2, layer_types=["sliding_attention", "full_attention"],
                       intermediate_size=256, num_local_experts=4, num_experts_per_tok=2)
    torch.manual_seed(0)
    rope = tf.GptOssRotaryEmbedding(cfg)
    pos = torch.arange(T)[None]
    h = torch.randn(1, T, 256)
    cos, sin = rope(h, pos)
    for layer_idx in (0, 1):
        ref_mod = tf.GptOssAttention(cfg, layer_idx)
        with torch.no_grad():
            for p in ref_mod.parameters():
                p.normal_(0, 0.05)
            ref_mod.sinks.normal_(0, 1)
        gpu_mod = tf.GptOssAttention(cfg, layer_idx)
        gpu_mod.load_state_dict(ref_mod.state_dict())
        gpu_mod = gpu_mod.to(device=device, dtype=torch.bfloat16)
        ref_mod.config._attn_implementation = "eager"
        gpu_mod.config = copy.deepcopy(cfg)
        gpu_mod.config._attn_implementation = A.NAME
        window = cfg.sliding_window if layer_idx == 0 else 0
        fn = sliding_window_causal_mask_function(window) if window else causal_mask_function
        for kind in ("none", "mask"):
            m32 = None if kind == "none" else eager_mask(1, T, T, mask_function=fn, dtype=torch.float32)
            mbf = None if kind == "none" else eager_mask(1, T, T, mask_function=fn, dtype=torch.bfloat16).to(device)
            hb = h.to(torch.bfloat16)
            want, _ = ref_mod(hb.float(), (cos, sin), m32)
            got, _ = gpu_mod(hb.to(device), (cos.to(torch.bfloat16).to(device), sin.to(torch.bfloat16).to(device)),
                             mbf)
            torch.cuda.synchronize()
            rel = _rel_l2(got, want)
            print(f"layer {layer_idx} mask {kind}: rel_l2={rel:.3e}")
            # the bf16 projections and rotary dominate this difference
            assert rel <= 2e-2, (layer_idx, kind)


def test_mask_kind_rejects_padding(device):
    from transformers.masking_utils import causal_mask_function, eager_mask

    m = eager_mask(1, 8, 8, mask_function=causal_mask_function, dtype=torch.float32).to(device)
    assert A.mask_kind(m, 8, 8, None) == (True, 0)
    m[..., 0] = torch.finfo(torch.float32).min  # a padded first key
    with pytest.raises(ValueError):
        A.mask_kind(m, 8, 8, None)


@pytest.mark.parametrize("window", [0, 128])
def test_forward_gptoss_prefill_8192_sampled_rows(device, window):
    """The full 8192-token gpt-oss prefill (64 query heads, 8 key heads), causal
    or windowed: sampled query rows of every head against float64."""
    announce(f"attention fwd T=8192 window={window}")
    B, Hq, Hkv, T = 1, 64, 8, 8192
    q, k, v, s = _inputs(B, Hq, Hkv, T, T, device, seed=77 + window)
    got = A.attention_forward(q, k, v, s, 0.125, True, window)
    torch.cuda.synchronize()
    rows = torch.tensor([0, 1, 63, 64, 127, 128, 129, 4095, 4096, 8000, 8190, 8191])
    kd = k.double().cpu().repeat_interleave(Hq // Hkv, dim=1)
    vd = v.double().cpu().repeat_interleave(Hq // Hkv, dim=1)
    qd = q.double().cpu()[:, :, rows]
    z = (qd @ kd.transpose(2, 3)) * 0.125                      # [1, Hq, rows, T]
    j = torch.arange(T)[None, :]
    vis = j <= rows[:, None]
    if window:
        vis &= j > rows[:, None] - window
    z = z.masked_fill(~vis, float("-inf"))
    z = torch.cat([z, s.double().cpu().reshape(1, Hq, 1, 1).expand(1, Hq, len(rows), 1)], -1)
    p = torch.softmax(z - z.max(-1, keepdim=True).values, -1)[..., :T]
    want = (p @ vd).transpose(1, 2)                             # [1, rows, Hq, 64]
    rel = _rel_l2(got[:, rows], want)
    mx = float((got[:, rows].double().cpu() - want).abs().max())
    print(f"T=8192 window={window}: sampled rows rel_l2={rel:.3e} max_abs={mx:.3e}")
    assert rel <= FWD_REL_L2 and mx <= FWD_MAX_ABS * max(1.0, float(want.abs().max()))


@pytest.mark.parametrize("window", [0, 128])
def test_forward_backward_2048_vs_float32(device, window):
    """2048 tokens at the gpt-oss head shape, forward and gradients against a
    float32 torch reference on the GPU (the oracle's arithmetic in float32)."""
    announce(f"attention fwd+bwd T=2048 window={window} vs float32")
    B, Hq, Hkv, T = 1, 64, 8, 2048
    q, k, v, s = _inputs(B, Hq, Hkv, T, T, device, seed=55 + window)
    dout = torch.randn(B, T, Hq, 64, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).to(device)
    qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    sg = s.detach().clone().requires_grad_(True)
    out = A.attention(qg, kg, vg, sg, 0.125, True, window)
    out.backward(dout)
    qr, kr, vr = (t.detach().float().requires_grad_(True) for t in (q, k, v))
    sr = s.detach().float().requires_grad_(True)
    ref = oracle.attention_ref(qr, kr, vr, sr, 0.125, causal=True, window=window, dtype=torch.float32)
    ref.backward(dout.float())
    torch.cuda.synchronize()
    rel = _rel_l2(out, ref)
    print(f"T=2048 window={window}: out rel_l2={rel:.3e}")
    assert rel <= FWD_REL_L2
    for name, got, want in (("dq", qg.grad, qr.grad), ("dk", kg.grad, kr.grad), ("dv", vg.grad, vr.grad),
                            ("dsinks", sg.grad, sr.grad)):
        r = _rel_l2(got, want)
        print(f"  {name}: rel_l2={r:.3e}")
        assert r <= BWD_REL_L2, name
    # the same call again gives the same bits
    q2, k2, v2 = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    out2 = A.attention(q2, k2, v2, s, 0.125, True, window)
    out2.backward(dout)
    torch.cuda.synchronize()
    assert torch.equal(out, out2) and torch.equal(qg.grad, q2.grad) and torch.equal(kg.grad, k2.grad)
