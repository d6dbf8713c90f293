"""The post-attention RMSNorm (one launch, forward and input gradient) against
the float64 oracle and transformers' own GptOssRMSNorm.

Bars, per element:
* float32 rows: |got - ref| <= 4e-6 |ref| (float32 rounding of the sum of
  squares and two products; a mean over H - 1 instead of H, or a dropped eps
  on small rows, is 1e-4 or more);
* bf16 / f16 rows: within half an ulp of the float64 value plus the float32
  error above (|got - ref| <= 2^-8 |ref| (1 + 1e-5) for bf16, 2^-11 for f16),
  and no more than 0.1% of elements rounded differently from the correctly
  rounded float64 value (only values within float32 error of a rounding
  boundary may; measured <= 0.004%);
* input gradients: the same half-ulp bound plus 1e-5 of the row's largest
  gradient (the two terms of the gradient cancel), at most 0.2% of elements
  rounded differently.
Against transformers' module on the GPU (bf16 input, float32 weight, the
checkpoint layout): at most one ulp apart (plus 1e-5 of the row's largest
value for the gradient), on at most 0.1% of the outputs and 0.2% of the
gradients.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from blockstreamer_amd import _lib, gptoss, kernels
from tests.conftest import announce

pytestmark = pytest.mark.gpu

ULP_REL = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}

# (T, H, dtype, weight dtype, element offset of the rows): vector path
# (bf16/f16, H % 8 == 0, H <= 3072, 16-byte aligned) and element path
CASES = [
    (64, 2880, torch.bfloat16, torch.float32, 0),
    (8192, 2880, torch.bfloat16, torch.bfloat16, 0),
    (7, 64, torch.float16, torch.float16, 0),
    (33, 3072, torch.bfloat16, torch.float32, 0),
    (5, 2880, torch.float32, torch.float32, 0),
    (3, 100, torch.bfloat16, torch.float32, 0),
    (33, 4096, torch.bfloat16, torch.float32, 0),
    (17, 2880, torch.bfloat16, torch.float32, 1),
    (1, 8, torch.bfloat16, torch.bfloat16, 0),
]


def _ids(c):
    T, H, dt, wdt, off = c
    return f"T{T}H{H}{str(dt)[6:]}w{str(wdt)[6:]}o{off}"


def _inputs(T, H, dt, wdt, off, device, scale=1.0, seed=0):
    """(host, device) pairs; the device rows start ``off`` elements into
    their allocation, so off = 1 gives 2-byte aligned rows on the GPU."""
    g = torch.Generator().manual_seed(seed + T * 7 + H)
    xb = (torch.randn(T * H + off, generator=g) * scale).to(dt)
    w = (torch.randn(H, generator=g) * 0.3 + 1.0).to(wdt)
    gb = (torch.randn(T * H + off, generator=g) * 0.1).to(dt)
    rows = lambda b: b[off:].view(T, H)  # noqa: E731
    return ((rows(xb), rows(xb.to(device))), (w, w.to(device)), (rows(gb), rows(gb.to(device))))


def _check(got, ref, dt, what, row_scale=None, max_frac=1e-3):
    got = got.detach().float().cpu().double()
    err = (got - ref).abs()
    slack = 0 if row_scale is None else 1e-5 * row_scale
    if dt == torch.float32:
        bound = 4e-6 * ref.abs() + slack
        assert (err <= bound + 1e-30).all(), f"{what}: max err {err.max():.3e}"
        return
    bound = ULP_REL[dt] * ref.abs() * (1 + 1e-5) + slack
    bad = (err > bound + 1e-30).sum().item()
    rounded = ref.to(dt).double()
    diff = (got != rounded).float().mean().item() if got.numel() else 0.0
    print(f"{what}: max err {err.max().item() if err.numel() else 0:.3e}, "
          f"{diff * 100:.3f}% not correctly rounded")
    assert bad == 0, f"{what}: {bad} elements beyond half an ulp"
    assert diff <= max_frac, f"{what}: {diff:.3%} differ from the correctly rounded value"


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_rmsnorm_forward_vs_oracle(device, case):
    T, H, dt, wdt, off = case
    eps = 1e-5
    for scale in (1.0, 1e-3):  # eps negligible, then eps comparable to the mean square
        (x, xd), (w, wd), _ = _inputs(T, H, dt, wdt, off, device, scale)
        announce(f"rmsnorm forward {_ids(case)} scale {scale}")
        got = kernels.rmsnorm_forward(xd, wd, eps)
        assert got.dtype == dt and got.shape == (T, H)
        _check(got, oracle.rmsnorm_ref(x, w, eps), dt, f"{_ids(case)} scale {scale}")


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_rmsnorm_backward_vs_oracle(device, case):
    T, H, dt, wdt, off = case
    eps = 1e-5
    (x, xd), (w, wd), (dy, dyd) = _inputs(T, H, dt, wdt, off, device, seed=1)
    announce(f"rmsnorm backward {_ids(case)}")
    got = kernels.rmsnorm_backward(dyd, xd, wd, eps)
    assert got.dtype == dt and got.shape == (T, H)
    ref = oracle.rmsnorm_bwd_ref(dy, x, w, eps)
    row = ref.abs().amax(-1, keepdim=True) if ref.numel() else None
    # near-zero gradients carry the cancellation error: a few more of them may
    # round the other way than in the forward
    _check(got, ref, dt, f"d x {_ids(case)}", row_scale=row, max_frac=2e-3)


def test_rmsnorm_empty_and_errors(device):
    w = torch.ones(64, device=device)
    out = kernels.rmsnorm_forward(torch.empty(0, 64, device=device, dtype=torch.bfloat16), w, 1e-5)
    assert out.shape == (0, 64)
    with pytest.raises(ValueError):
        kernels.rmsnorm_forward(torch.ones(4, 64, device=device), torch.ones(32, device=device), 1e-5)
    with pytest.raises(ValueError):
        kernels.rmsnorm_forward(torch.ones(4, 64), torch.ones(64), 1e-5)  # CPU tensors: no CPU path
    lib = _lib.lib()
    rc = lib.bsa_rmsnorm_fwd(None, 0, 4, 0, None, 0, 1e-5, None, None)
    assert rc != 0 and b"bad shape" in lib.bsa_last_error()


def test_rmsnorm_matches_transformers_module(device):
    """bf16 activations, float32 weight (transformers keeps the norm in
    float32 when loading a checkpoint): our module and GptOssRMSNorm on the
    same GPU inputs, forward and autograd input gradient."""
    gpt_oss = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")
    H, eps = 2880, 1e-5
    ref = gpt_oss.GptOssRMSNorm(H, eps=eps).to(device)
    with torch.no_grad():
        ref.weight.copy_(torch.randn(H, generator=torch.Generator().manual_seed(3)) * 0.3 + 1.0)
    ours = gptoss.FusedRMSNorm(H, eps, torch.float32, device)
    ours.load_state_dict(ref.state_dict())
    x = (torch.randn(2, 40, H, generator=torch.Generator().manual_seed(4))).to(torch.bfloat16).to(device)
    dy = (torch.randn(2, 40, H, generator=torch.Generator().manual_seed(5)) * 0.1).to(torch.bfloat16).to(device)
    announce("rmsnorm vs transformers module")
    xa = x.clone().requires_grad_(True)
    xb = x.clone().requires_grad_(True)
    ya, yb = ours(xa), ref(xb)
    assert ya.dtype == yb.dtype == torch.bfloat16 and ya.shape == yb.shape
    ga, gw = torch.autograd.grad(ya, [xa, ours.weight], dy)
    gb, gwb = torch.autograd.grad(yb, [xb, ref.weight], dy)
    for what, a, b, slack, max_frac in (("y", ya, yb, 0.0, 1e-3), ("d x", ga, gb, 1e-5, 2e-3)):
        a, b = a.detach().float(), b.detach().float()
        bound = 2.0 ** -7 * b.abs() * (1 + 1e-5) + slack * b.abs().amax(-1, keepdim=True)
        far = ((a - b).abs() > bound + 1e-30).sum().item()
        frac = (a != b).float().mean().item()
        print(f"{what}: {frac * 100:.3f}% differ from transformers")
        assert far == 0 and frac <= max_frac, f"{what}: {far} beyond one ulp, {frac:.3%} differ"
    # weight gradient (torch ops, float32): same math, summation order aside
    assert torch.allclose(gw, gwb, rtol=1e-4, atol=1e-4 * gwb.abs().max().item())


def test_rmsnorm_in_cuda_graph(device):
    H, eps = 2880, 1e-5
    w = (torch.randn(H, generator=torch.Generator().manual_seed(6)) * 0.3 + 1.0).to(device)
    x = torch.empty(64, H, dtype=torch.bfloat16, device=device)
    announce("rmsnorm graph capture")
    x.copy_(torch.randn(64, H).to(torch.bfloat16))
    kernels.rmsnorm_forward(x, w, eps)  # warm up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = kernels.rmsnorm_forward(x, w, eps)
    for i in range(3):
        x.copy_(torch.randn(64, H, generator=torch.Generator().manual_seed(10 + i)).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        want = kernels.rmsnorm_forward(x, w, eps)
        assert torch.equal(y, want), f"replay {i} differs from eager"


def test_rmsnorm_special_rows_match_transformers(device):
    """Rows of zeros (the result is 0: r = eps^-1/2 times 0), values whose
    squares overflow float32 (r = 0, so 0 out), and rows holding inf or NaN
    (NaN out): the same as transformers' module, NaN for NaN."""
    gpt_oss = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")
    H, eps = 2880, 1e-5
    ref = gpt_oss.GptOssRMSNorm(H, eps=eps).to(device)
    ours = gptoss.FusedRMSNorm(H, eps, torch.float32, device)
    rows = torch.randn(6, H, generator=torch.Generator().manual_seed(8))
    rows[0] = 0.0
    rows[1] = 3e38
    rows[2, 5] = float("inf")
    rows[3, 7] = float("nan")
    rows[4] *= 1e-30
    for dt in (torch.float32, torch.bfloat16):
        x = rows.to(dt).to(device)
        announce(f"rmsnorm special rows {dt}")
        with torch.no_grad():
            got, want = ours(x), ref(x)
        assert torch.equal(torch.isnan(got), torch.isnan(want)), f"{dt}: NaN positions differ"
        fin = ~torch.isnan(want)
        g, w = got[fin].float(), want[fin].float()
        assert torch.equal(torch.isinf(g), torch.isinf(w))
        ok = torch.isfinite(w)
        assert ((g[ok] - w[ok]).abs() <= 2.0 ** -7 * w[ok].abs() + 1e-30).all(), f"{dt}: finite values differ"
