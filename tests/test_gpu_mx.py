"""Native block-scaled MX path on the GPU: the activations as two MXFP8 terms
(hi + lo) against the packed MXFP4 weights as they are, two
v_mfma_scale_f32_32x32x64_f8f6f4 per 64-element k-step.

Parity bars:
* MXFP8 quantisation and the two-term split: bit-exact with the oracle
  (codes and scale bytes).
* MX layer output against the float32 reference (unquantised activations,
  block_streamer/gptoss.py:137-177): the layer bar of tests/moe_util.py,
  relative L2 <= 5e-3 and max-abs <= 2e-2 (scaled by max|ref| on the
  synthetic-scale cases, absolute on the trained-scale ones), as for the
  bf16 path.  The two terms reproduce the bf16 activations exactly unless an
  element is below 2^-14 of its 32-element block's maximum.
* Against the oracle of the same arithmetic (``experts_mx_ref``: the split
  dequantised, float64 GEMMs): the same bar.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from blockstreamer_amd import kernels, synthetic
from tests.conftest import announce
from tests.moe_util import assert_layer_close, errors, expert_args

pytestmark = pytest.mark.gpu



@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_quant_mxfp8_bit_exact(device, dtype):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(130, 640, generator=g)
    x[0] *= 1e-30 if dtype != torch.float16 else 1e-6         # tiny blocks
    x[1] *= 1e4                                               # large blocks
    x[2, :32] = 0.0                                           # zero block
    x[2, 32:64] = -0.0
    x[3, 70] = float("inf")                                   # non-finite blocks
    x[4, 100] = float("nan")
    x[5, :32] = torch.tensor([448.0, 1.0625, 1.1875, 2.0 ** -9, 2.0 ** -10] + [0.0] * 27)
    x = x.to(dtype)
    announce(f"mxfp8 quantisation {dtype}")
    q, s = kernels.quantize_mxfp8(x.to(device))
    rq, rs = oracle.mxfp8_quant_ref(x)
    q, s = q.cpu().numpy(), s.cpu().numpy()
    assert np.array_equal(s, rs)
    assert np.array_equal(q, rq)


def _layer(E, k, H, I, T, seed, lo=116, hi=120, bias_std=0.01, device=None):
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=seed, scale_lo=lo, scale_hi=hi,
                            router_bias_std=bias_std, device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=seed + 1, device=device)
    return t, idx, w


MX_CASES = [
    # (E, k, H, I, T)
    (8, 2, 256, 256, 64),
    (16, 4, 512, 256, 300),
    (4, 1, 128, 192, 77),
    (32, 4, 2880, 2880, 96),
    # one and three 64-wide k-steps: the k loop's prologue and tail alone
    (4, 2, 64, 64, 40),
    (8, 2, 192, 64, 130),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_quant_mxfp8_split_bit_exact(device, dtype):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(130, 640, generator=g)
    x *= torch.exp2(torch.randint(-12, 12, (130, 640), generator=g).float())   # wide blocks
    x[0] *= 1e-30 if dtype != torch.float16 else 1e-3         # tiny blocks
    x[1] *= 1e4 if dtype != torch.float16 else 1.0
    x[2, :32] = 0.0                                           # zero blocks
    x[2, 32:64] = -0.0
    x[3, 70] = float("inf")                                   # non-finite blocks
    x[4, 100] = float("nan")
    x[5, :32] = 1.0 + 2.0 ** -7
    x = x.to(dtype)
    announce(f"mxfp8 split {dtype}")
    hi, lo, s = kernels.quantize_mxfp8_split(x.to(device))
    rhi, rlo, rs = oracle.mxfp8_split_ref(x)
    hi, lo, s = hi.cpu().numpy(), lo.cpu().numpy(), s.cpu().numpy()
    assert np.array_equal(s, rs)
    assert np.array_equal(hi, rhi)
    assert np.array_equal(lo, rlo)


@pytest.mark.parametrize("case", MX_CASES, ids=[f"E{c[0]}k{c[1]}H{c[2]}I{c[3]}T{c[4]}" for c in MX_CASES])
@pytest.mark.parametrize("scales", [(116, 120), (115, 131)], ids=["trained", "synthetic"])
def test_mx_layer_vs_float32_and_mx_oracle(device, case, scales):
    E, k, H, I, T = case
    lo, hi = scales
    t, idx, w = _layer(E, k, H, I, T, seed=E + T, lo=lo, hi=hi, device=device)
    announce(f"MX layer {case} scales {scales}")
    got = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(t), path="mx")
    args = [a.cpu() for a in expert_args(t)]
    exact = oracle.experts_ref(t["hidden"].cpu(), idx.cpu(), w.cpu().float(), *args)
    trained = scales == (116, 120)
    assert_layer_close(got, exact, f"MX vs float32 {case} {scales}", absolute=trained)
    want = oracle.experts_mx_ref(t["hidden"].cpu(), idx.cpu(), w.cpu().float(), *args)
    assert_layer_close(got, want, f"MX vs MX oracle {case} {scales}", absolute=trained)
    bf16 = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(t), path="tiled"
                                       if H % 64 == 0 and I % 64 == 0 else "auto")
    print(f"bf16 path vs float32 {case} {scales}: rel_l2={errors(bf16, exact)[0]:.3e}")


def test_mx_stages_match_fused_call(device):
    """MoEStages with path "mx" equals the single fused C call bit for bit."""
    t, idx, w = _layer(16, 4, 512, 512, 257, seed=9, device=device)
    announce("MX stages vs fused")
    fused = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(t), path="mx")
    st = kernels.MoEStages(t["hidden"], idx, w, *expert_args(t), path="mx")
    staged = st.run()
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), staged.view(torch.int16))


def test_mx_rejects_unsupported_shapes(device):
    t, idx, w = _layer(4, 2, 96, 64, 16, seed=2, device=device)   # H % 64 != 0
    with pytest.raises(ValueError, match="64"):
        kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(t), path="mx")


def test_mx_dropped_pairs(device):
    """Router indices outside [0, E) are dropped on the MX path too: the
    hidden rows are split per token into the sorted rows of its kept pairs
    only, and the layer matches the float32 oracle with those pairs' weights
    set to zero."""
    E, k, H, I, T = 16, 4, 512, 256, 200
    t, idx, w = _layer(E, k, H, I, T, seed=23, device=device)
    idx = idx.clone()
    idx[::7, 0] = -1
    idx[3::11, 2] = E
    announce("MX layer with dropped pairs")
    got = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(t), path="mx")
    keep = (idx >= 0) & (idx < E)
    args = [a.cpu() for a in expert_args(t)]
    want = oracle.experts_ref(t["hidden"].cpu(), idx.clamp(0, E - 1).cpu(), (w * keep).cpu().float(), *args)
    assert_layer_close(got, want, "MX dropped pairs", absolute=True)


def test_mx_scales_aligned_to_4_and_8_bytes_bit_identical(device):
    """Scale tensors that start 4 or 8 bytes past a 16-byte boundary (the
    reference's shard planner aligns tensors to 8 bytes) take the MX kernels'
    4-byte B-scale preload instead of the 16-byte one; the products are the
    same bit for bit."""
    E, k, H, I, T = 8, 2, 256, 192, 300   # 600 pairs > 16 per expert: MX
    t, idx, w = _layer(E, k, H, I, T, seed=31, device=device)
    args = list(expert_args(t))
    announce("MX with 4- and 8-byte aligned scales")
    want = kernels.moe_experts_forward(t["hidden"], idx, w, *args, path="mx")

    def at_offset(x, off):
        buf = torch.empty(x.numel() + 32, dtype=torch.uint8, device=device)
        base = (-buf.data_ptr()) % 16
        v = buf[base + off:base + off + x.numel()].view(x.shape)
        v.copy_(x)
        assert v.data_ptr() % 16 == off
        return v

    args[1] = at_offset(args[1], 4)
    args[4] = at_offset(args[4], 8)
    got = kernels.moe_experts_forward(t["hidden"], idx, w, *args, path="mx")
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_mx_concentrated_and_duplicate_routing(device):
    """The MX kernels when routing piles up: every token on the same two
    experts (three row tiles each, the last one partial), and every token
    sent twice to one expert (both pairs count), against the float32 oracle."""
    E, k, H, I, T = 8, 2, 256, 256, 300
    t, idx, w = _layer(E, k, H, I, T, seed=41, device=device)
    args = expert_args(t)
    cpu_args = [a.cpu() for a in args]
    idx_two = torch.zeros_like(idx)
    idx_two[:, 1] = 3
    idx_dup = idx.clone()
    idx_dup[:, 1] = idx_dup[:, 0]
    for what, ix in (("two experts", idx_two), ("duplicate slot", idx_dup)):
        announce(f"MX {what}")
        got = kernels.moe_experts_forward(t["hidden"], ix, w, *args, path="mx")
        want = oracle.experts_ref(t["hidden"].cpu(), ix.cpu(), w.cpu().float(), *cpu_args)
        assert_layer_close(got, want, f"MX {what}", absolute=True)
