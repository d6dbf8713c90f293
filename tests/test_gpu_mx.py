"""Native block-scaled MX path (MXFP8 activations x MXFP4 weights) on the GPU.

Parity bars:
* MXFP8 quantisation: bit-exact with the oracle (codes and scale bytes).
* MX layer output against the oracle of the same arithmetic
  (``experts_mx_ref``: activations quantised to MXFP8, float64 GEMMs):
  relative L2 <= 5e-3 and max-abs <= 2e-2 * max|ref| (the kernel accumulates
  in the MFMA's own precision, and its bf16 gated activations can sit one
  bf16 ulp from the oracle's, moving an E4M3 rounding now and then).
* Against the float32 reference path (unquantised activations) the MX path
  carries the activation quantisation error; it is measured and printed,
  and bounded at relative L2 <= 6e-2.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from blockstreamer_amd import kernels, synthetic
from tests.conftest import announce
from tests.moe_util import errors, expert_args

pytestmark = pytest.mark.gpu

MX_REL_L2 = 5e-3
MX_MAX_ABS = 2e-2
MX_VS_FP32_REL_L2 = 6e-2


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
]


@pytest.mark.parametrize("case", MX_CASES, ids=[f"E{c[0]}k{c[1]}H{c[2]}I{c[3]}T{c[4]}" for c in MX_CASES])
def test_mx_layer_vs_mx_oracle(device, case):
    E, k, H, I, T = case
    t, idx, w = _layer(E, k, H, I, T, seed=E + T, device=device)
    announce(f"MX layer {case}")
    got = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(t), path="mx")
    args = [a.cpu() for a in expert_args(t)]
    want = oracle.experts_mx_ref(t["hidden"].cpu(), idx.cpu(), w.cpu().float(), *args)
    rel_l2, max_abs, scale = errors(got, want)
    msg = f"MX vs MX oracle {case}: rel_l2={rel_l2:.3e} max_abs={max_abs:.3e} (|ref|max {scale:.3e})"
    print(msg)
    assert rel_l2 <= MX_REL_L2, msg
    assert max_abs <= MX_MAX_ABS * max(scale, 1.0), msg
    exact = oracle.experts_ref(t["hidden"].cpu(), idx.cpu(), w.cpu().float(), *args)
    err = errors(got, exact)[0]
    print(f"MX path vs float32 reference {case}: rel_l2={err:.3e}")
    assert err <= MX_VS_FP32_REL_L2


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
