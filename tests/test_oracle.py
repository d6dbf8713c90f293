"""Pin the oracle (CPU only).

Each oracle function is checked against something independent of its own
formula: the exhaustive closed form of E2M1 x E8M0, the other dequant
restatement, the committed golden vectors produced by the transformers
routines the reference calls, the installed transformers modules themselves,
and invariants of the MoE layer.  A planted mistake in the oracle (wrong
nibble order, dropped bias, wrong clamp side, transposed weight) fails at
least one of these.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from blockstreamer_amd import synthetic

GOLDEN = Path(__file__).resolve().parent / "golden"
DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
FLT_MAX = float(np.finfo(np.float32).max)


def _decode(bits: int, name: str) -> float:
    if name == "f32":
        return float(np.array([bits], dtype=np.uint32).view(np.float32)[0])
    if name == "bf16":
        return float(np.array([bits << 16], dtype=np.uint32).view(np.float32)[0])
    return float(np.array([bits], dtype=np.uint16).view(np.float16)[0])


@pytest.mark.parametrize("name", list(DTYPES))
def test_dequant_table_closed_form(name):
    """Every (code, scale) of the C oracle against value * 2^(s-127)."""
    tab = oracle.dequant_table_c(DTYPES[name])
    for s in range(256):
        for c in range(16):
            got = _decode(int(tab[s, c]), name)
            mag = oracle.FP4_VALUES[c]
            if s == 255:
                # float32 pow(2, 128) = inf: +-0 * inf = NaN, else +-inf
                if c in (0, 8):
                    assert math.isnan(got), (s, c, got)
                else:
                    assert math.isinf(got) and math.copysign(1, got) == math.copysign(1, mag)
                continue
            exact = math.ldexp(mag, s - 127)  # exact in double
            if name == "f16":
                # torch.ldexp on float16 rounds pow(2, s-127) to float16 first
                p2 = float(np.float16(math.ldexp(1.0, s - 127))) if s - 127 < 16 else math.inf
                if math.isinf(p2):
                    want = math.nan if mag == 0 else math.copysign(math.inf, mag)
                else:
                    want = float(np.float16(mag * p2))
                if math.isnan(want):
                    assert math.isnan(got), (s, c, got)
                    continue
            else:
                want = exact if abs(exact) <= FLT_MAX else math.copysign(math.inf, exact)
            assert got == want and math.copysign(1, got) == math.copysign(1, want), (name, s, c, got, want)


@pytest.mark.parametrize("name", list(DTYPES))
def test_dequant_c_matches_torch_restatement(name):
    dt = DTYPES[name]
    g = torch.Generator().manual_seed(11)
    blocks = torch.randint(0, 256, (3, 40, 5, 16), generator=g, dtype=torch.uint8)
    scales = torch.randint(0, 256, (3, 40, 5), generator=g, dtype=torch.uint8)
    a = oracle.dequant_c(blocks, scales, dt)
    b = oracle.dequant_torch(blocks, scales, dt)
    assert a.shape == (3, 160, 40)
    view = torch.int32 if dt == torch.float32 else torch.int16
    ok = oracle.bits_equal_or_both_nan(a.view(view).numpy(), b.view(view).numpy(), dt)
    assert ok.all()


def _exhaustive():
    from tests.golden.make_golden import exhaustive_inputs
    return exhaustive_inputs()


@pytest.mark.parametrize("name", list(DTYPES))
def test_dequant_oracle_matches_golden_table(name):
    """Golden vectors written by transformers' convert_moe_packed_tensors."""
    dt = DTYPES[name]
    want = np.load(GOLDEN / "dequant_table.npz")[name]
    blocks, scales = _exhaustive()
    got = oracle.dequant_c(blocks, scales, dt)[0]
    view = torch.int32 if dt == torch.float32 else torch.int16
    ok = oracle.bits_equal_or_both_nan(got.view(view).numpy(), want, dt)
    assert ok.all(), np.argwhere(~ok)[:5]
    # nibble order: low nibble -> even column (mxfp4.py:296-304)
    assert _decode(int(np.uint16(want[0, 127 * 0 + 127]) if name != "f32" else want[0, 127]), name) == 0.0


def test_dequantize_expert_ref_contract():
    """tests/test_offload.py:405-414 restated on the oracle."""
    g = torch.Generator().manual_seed(0)
    blocks = torch.randint(0, 255, (64, 4, 16), generator=g, dtype=torch.uint8)
    scales = torch.randint(120, 134, (64, 4), generator=g, dtype=torch.uint8)
    with pytest.raises(ValueError, match="packed blocks"):
        oracle.dequantize_expert_ref(blocks, scales)
    out = oracle.dequantize_expert_ref(blocks.unsqueeze(0), scales.unsqueeze(0), torch.float32)
    assert out.shape == (128, 64)
    # element check against the definition for one byte
    b = int(blocks[5, 2, 7])
    s = int(scales[5, 2])
    assert out[32 * 2 + 14, 5].item() == math.ldexp(oracle.FP4_VALUES[b & 15], s - 127)
    assert out[32 * 2 + 15, 5].item() == math.ldexp(oracle.FP4_VALUES[b >> 4], s - 127)


def test_dequant_matches_transformers_random():
    tf = pytest.importorskip("transformers.integrations.mxfp4")
    g = torch.Generator().manual_seed(5)
    blocks = torch.randint(0, 256, (2, 24, 3, 16), generator=g, dtype=torch.uint8)
    scales = torch.randint(100, 160, (2, 24, 3), generator=g, dtype=torch.uint8)
    for dt in DTYPES.values():
        want = tf.convert_moe_packed_tensors(blocks, scales, dtype=dt)
        got = oracle.dequant_c(blocks, scales, dt)
        view = torch.int32 if dt == torch.float32 else torch.int16
        assert oracle.bits_equal_or_both_nan(got.view(view).numpy(), want.view(view).numpy(), dt).all()


# ----------------------------------------------------------------------------- router

def test_topk_softmax_invariants():
    """Selected set dominates the rest, descending order, softmax ratios."""
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(50, 16, generator=g)
    vals, scores, idx = oracle.topk_softmax_ref(logits, 4)
    for t in range(50):
        sel = set(idx[t].tolist())
        assert len(sel) == 4
        rest = [logits[t, e].item() for e in range(16) if e not in sel]
        assert min(logits[t, list(sel)]).item() > max(rest)
        assert all(vals[t, i] >= vals[t, i + 1] for i in range(3))
        assert torch.allclose(vals[t], logits[t, idx[t]])
    assert torch.allclose(scores.sum(-1), torch.ones(50), atol=1e-6)
    r = scores[:, 0] / scores[:, 1]
    assert torch.allclose(r, torch.exp(vals[:, 0] - vals[:, 1]), rtol=1e-5)


def test_topk_ties_lower_index_first():
    logits = torch.tensor([[1.0, 3.0, 3.0, 0.5, 3.0]])
    _, _, idx = oracle.topk_softmax_ref(logits, 2)
    assert idx.tolist() == [[1, 2]]


def test_router_matches_transformers():
    gpt_oss = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")
    from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig
    cfg = GptOssConfig(num_local_experts=32, hidden_size=128, intermediate_size=128,
                       num_experts_per_tok=4, num_hidden_layers=1)
    r = gpt_oss.GptOssTopKRouter(cfg)
    g = torch.Generator().manual_seed(9)
    with torch.no_grad():
        r.weight.copy_(torch.randn(32, 128, generator=g) * 0.1)
        r.bias.copy_(torch.randn(32, generator=g) * 0.1)
        h = torch.randn(40, 128, generator=g)
        want = r(h)
    got = oracle.router_ref(h, r.weight.detach(), r.bias.detach(), 4)
    assert torch.equal(got[0], want[0])
    assert torch.equal(got[2], want[2])
    assert torch.equal(got[1], want[1])


# ----------------------------------------------------------------------------- rmsnorm

def _tf_norm(H, eps, weight):
    gpt_oss = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")
    m = gpt_oss.GptOssRMSNorm(H, eps=eps)
    with torch.no_grad():
        m.weight.copy_(weight)
    return m


@pytest.mark.parametrize("H,eps,scale", [(2880, 1e-5, 1.0), (100, 1e-5, 1e-3), (64, 1e-6, 30.0)])
def test_rmsnorm_ref_matches_transformers_forward_and_autograd(H, eps, scale):
    """The module upcasts its input to float32 itself, so it is pinned in
    float32 (bit-exact, same operations) and the float64 reference within
    float32 rounding; the closed-form gradient against float64 autograd of
    the restated forward and against the module's own float32 autograd."""
    g = torch.Generator().manual_seed(H)
    x = torch.randn(9, H, generator=g) * scale
    w = torch.randn(H, generator=g) * 0.5 + 1.0
    dy = torch.randn(9, H, generator=g)
    m = _tf_norm(H, eps, w)
    xr = x.clone().requires_grad_(True)
    want = m(xr)
    (want_dx,) = torch.autograd.grad(want, [xr], dy)
    assert torch.equal(oracle.rmsnorm_ref(x, w, eps, dtype=torch.float32), want.detach())
    got = oracle.rmsnorm_ref(x, w, eps)
    assert torch.allclose(got, want.detach().double(), rtol=2e-6, atol=0)
    x64 = x.double().requires_grad_(True)
    (auto_dx,) = torch.autograd.grad(oracle.rmsnorm_ref(x64, w, eps), [x64], dy.double())
    got_dx = oracle.rmsnorm_bwd_ref(dy, x, w, eps)
    assert (got_dx - auto_dx).abs().max() <= 1e-12 * auto_dx.abs().max()
    assert (got_dx - want_dx.double()).abs().max() <= 1e-5 * auto_dx.abs().max()


def test_rmsnorm_ref_invariants():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(4, 256, generator=g, dtype=torch.float64)
    w = torch.ones(256, dtype=torch.float64)
    # scale invariance without eps; unit RMS output with unit weight
    a = oracle.rmsnorm_ref(x, w, 0.0)
    b = oracle.rmsnorm_ref(x * 37.5, w, 0.0)
    assert torch.allclose(a, b, rtol=1e-14, atol=0)
    assert torch.allclose(a.pow(2).mean(-1), torch.ones(4, dtype=torch.float64), rtol=1e-14)
    # eps-dominated rows: x * rsqrt(eps)
    tiny = x * 1e-9
    assert torch.allclose(oracle.rmsnorm_ref(tiny, w, 1e-2), tiny * 10.0, rtol=1e-9)
    # the gradient is orthogonal to x when eps = 0 (scale invariance)
    dy = torch.randn(4, 256, generator=g, dtype=torch.float64)
    dx = oracle.rmsnorm_bwd_ref(dy, x, w, 0.0)
    assert (dx * x).sum(-1).abs().max() <= 1e-12 * dx.abs().max() * x.abs().max() * 256


# ----------------------------------------------------------------------------- k-pair layout

def test_to_kpair_ref_index_map():
    g = torch.Generator().manual_seed(3)
    E, R, G = 2, 32, 6
    blocks = torch.randint(0, 256, (E, R, G, 16), generator=g, dtype=torch.uint8)
    kp = oracle.to_kpair_ref(blocks)
    assert kp.shape == (E, R // 16, G // 2, 16, 2, 16)
    for e in range(E):
        for r in range(R):
            for gg in range(G):
                assert torch.equal(kp[e, r // 16, gg // 2, r % 16, gg % 2], blocks[e, r, gg])
    # a band occupies the same bytes in both layouts
    flat_b = blocks.reshape(E, R // 16, -1)
    flat_k = kp.reshape(E, R // 16, -1)
    assert torch.equal(flat_b.sort(dim=-1).values, flat_k.sort(dim=-1).values)


# ----------------------------------------------------------------------------- experts

def _tiny():
    from tests.golden.make_golden import tiny_layer
    return tiny_layer()


def _expert_args(t):
    return (t["gate_up_proj_blocks"], t["gate_up_proj_scales"], t["gate_up_proj_bias"],
            t["down_proj_blocks"], t["down_proj_scales"], t["down_proj_bias"])


def test_tiny_inputs_regenerate_bit_identically():
    gold = np.load(GOLDEN / "tiny_layer.npz")
    from tests.golden.make_golden import digest
    for k, v in _tiny().items():
        assert str(gold[f"sha256_{k}"]) == digest(v), k


def test_experts_oracle_matches_golden():
    gold = np.load(GOLDEN / "tiny_layer.npz")
    t = _tiny()
    logits, scores, idx = oracle.router_ref(t["hidden"], t["router_weight"], t["router_bias"], 2)
    assert np.array_equal(idx.numpy(), gold["router_indices"])
    assert np.array_equal(logits.numpy(), gold["router_logits"])
    assert np.allclose(scores.numpy(), gold["router_scores"], rtol=0, atol=1e-7)
    out = oracle.experts_ref(t["hidden"], torch.from_numpy(gold["router_indices"]),
                             torch.from_numpy(gold["router_scores"]), *_expert_args(t))
    want = torch.from_numpy(gold["experts_out"])
    assert torch.equal(out, want)


def test_experts_oracle_matches_transformers_dense_twin():
    gpt_oss = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")
    from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig
    from transformers.integrations.mxfp4 import convert_moe_packed_tensors
    shape = synthetic.MoEShape(6, 3, 96, 64, 20)
    t = synthetic.moe_layer(shape, seed=21, scale_lo=118, scale_hi=126)
    idx, w = synthetic.random_routing(20, 6, 3, seed=22, dtype=torch.float32)
    cfg = GptOssConfig(num_local_experts=6, hidden_size=96, intermediate_size=64,
                       num_experts_per_tok=3, num_hidden_layers=1)
    ex = gpt_oss.GptOssExperts(cfg)
    with torch.no_grad():
        ex.gate_up_proj.copy_(convert_moe_packed_tensors(t["gate_up_proj_blocks"], t["gate_up_proj_scales"], dtype=torch.float32))
        ex.gate_up_proj_bias.copy_(t["gate_up_proj_bias"].float())
        ex.down_proj.copy_(convert_moe_packed_tensors(t["down_proj_blocks"], t["down_proj_scales"], dtype=torch.float32))
        ex.down_proj_bias.copy_(t["down_proj_bias"].float())
        want = ex(t["hidden"].float(), idx, w)
    got = oracle.experts_ref(t["hidden"], idx, w, *_expert_args(t))
    assert torch.equal(got, want)


def test_experts_invariants():
    shape = synthetic.MoEShape(5, 2, 64, 64, 12)
    t = synthetic.moe_layer(shape, seed=31, scale_lo=119, scale_hi=125)
    idx, w = synthetic.random_routing(12, 5, 2, seed=32, dtype=torch.float32)
    args = _expert_args(t)
    h = t["hidden"]
    full = oracle.experts_ref(h, idx, w, *args)
    # a zero routing weight removes that slot's contribution
    w0 = w.clone()
    w0[:, 1] = 0
    only0 = oracle.experts_ref(h, idx[:, :1], w[:, :1], *args)
    assert torch.allclose(oracle.experts_ref(h, idx, w0, *args), only0, rtol=1e-6, atol=1e-3)
    # permuting tokens permutes the output
    perm = torch.randperm(12, generator=torch.Generator().manual_seed(1))
    permuted = oracle.experts_ref(h[perm], idx[perm], w[perm], *args)
    assert torch.allclose(permuted, full[perm], rtol=1e-5, atol=1e-2)
    # linearity in the routing weights
    twice = oracle.experts_ref(h, idx, 2 * w, *args)
    assert torch.allclose(twice, 2 * full, rtol=1e-6, atol=1e-2)
    # a different bias changes the output by exactly w * bias for that expert's tokens
    args2 = list(args)
    args2[5] = args[5] + 1.0
    shifted = oracle.experts_ref(h, idx, w, *args2)
    assert torch.allclose(shifted - full, w.sum(-1, keepdim=True).expand_as(full), atol=5e-2)


def test_apply_gate_ref_clamps():
    gu = torch.tensor([[10.0, 10.0, -3.0, -9.0, 0.5, 0.25]])
    got = oracle.apply_gate_ref(gu)
    # gate clamps only from above, up on both sides
    assert torch.allclose(got[0, 0], torch.tensor(7.0 * torch.sigmoid(torch.tensor(7 * 1.702)) * 8.0))
    g = torch.tensor(-3.0)
    assert torch.allclose(got[0, 1], g * torch.sigmoid(g * 1.702) * (-6.0))
    g = torch.tensor(0.5)
    assert torch.allclose(got[0, 2], g * torch.sigmoid(g * 1.702) * 1.25)


# ----------------------------------------------------------------------------- MXFP8 oracle
def _f8(x):
    return torch.tensor(x, dtype=torch.float64).to(torch.float32).to(torch.float8_e4m3fn)


def test_e4m3_decode_matches_torch_float8():
    """The E4M3 table against torch.float8_e4m3fn (OCP E4M3FN) for all 256 codes."""
    codes = np.arange(256, dtype=np.uint8)
    ours = oracle.e4m3_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan) and nan.sum() == 2   # 0x7F, 0xFF
    assert np.array_equal(ours[~nan], ref[~nan])
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9 and ours[0x08] == 2.0 ** -6
    assert ours[0x38] == 1.0 and ours[0x80] == 0.0 and np.signbit(ours[0x80])


@pytest.mark.parametrize("mag", [1e-3, 1.0, 3.0, 1e4])
def test_mxfp8_quant_matches_torch_cast_and_scale_rule(mag):
    """Elements: torch's RNE float8_e4m3fn cast of x / 2^X.  Scales: the rule's
    closed form 224 < amax / 2^X <= 448 for every nonzero block."""
    g = torch.Generator().manual_seed(int(mag * 1000) % 9973)
    x = (torch.randn(96, 320, generator=g) * mag).to(torch.bfloat16).float()
    x[3, :32] = 0.0                                         # all-zero block
    q, s = oracle.mxfp8_quant_ref(x)
    X = s.astype(np.int64) - 127
    blk = x.double().numpy().reshape(96, 10, 32)
    amax = np.abs(blk).max(-1)
    nz = amax > 0
    ratio = amax[nz] / np.exp2(X[nz])
    assert (ratio > 224).all() and (ratio <= 448).all()
    assert s[3, 0] == 0
    y = (blk / np.exp2(X)[..., None]).reshape(96, 320)
    cast = torch.from_numpy(y).float().to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(cast, q)


def test_mxfp8_quant_known_answers():
    """Hand-worked block: amax 448 gives X = 0; ties round to even."""
    row = np.zeros(32)
    vals = [448.0, 1.0625, 1.1875, 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -10, -0.0, -6.5, 224.5]
    row[:len(vals)] = vals
    q, s = oracle.mxfp8_quant_ref(torch.from_numpy(row[None]).double())
    assert s[0, 0] == 127
    # 448 -> 0x7E; 1.0625 tie -> 1.0 (0x38); 1.1875 tie -> 1.25 (0x3A); 2^-9 -> 0x01;
    # 2^-10 tie -> 0; 3*2^-10 tie -> 2^-8 (0x02); -0 -> 0x80; -6.5 -> 0xCD (-6.5 exact);
    # 224.5 -> 224 (0x76)
    assert list(q[0, :len(vals)]) == [0x7E, 0x38, 0x3A, 0x01, 0x00, 0x02, 0x80, 0xCD, 0x76]
    # amax 1.0 -> X = ceil(log2(1/448)) = -8, element 1.0 -> 256 (0x78)
    q, s = oracle.mxfp8_quant_ref(torch.ones(1, 32))
    assert s[0, 0] == 119 and (q == 0x78).all()
    # amax 449 -> X = 1 (449/2 = 224.5 -> 224)
    q, s = oracle.mxfp8_quant_ref(torch.full((1, 32), 449.0))
    assert s[0, 0] == 128 and (q == 0x76).all()
    # a non-finite element makes the block NaN (scale 255)
    bad = torch.ones(1, 64)
    bad[0, 40] = float("inf")
    q, s = oracle.mxfp8_quant_ref(bad)
    assert list(s[0]) == [119, 255] and (q[0, 32:] & 0x7F == 0x7F).all()


def test_mxfp8_roundtrip_of_representable_blocks():
    """Blocks built from E4M3 codes whose largest magnitude is in (224, 448]
    quantise back to the same codes and scale."""
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 0x7E, size=(50, 32), dtype=np.int64)
    codes[:, 0] = rng.integers(0x77, 0x7F, size=50)           # 240 .. 448
    codes |= rng.integers(0, 2, size=(50, 32)) << 7
    X = rng.integers(-20, 20, size=50)
    v = oracle.e4m3_decode(codes) * np.exp2(X)[:, None]
    q, s = oracle.mxfp8_quant_ref(torch.from_numpy(v))
    want = codes.astype(np.uint8)
    zero = (want & 0x7F) == 0                                 # +-0 keep their sign
    assert np.array_equal(q[~zero], want[~zero])
    assert np.array_equal(s[:, 0], (X + 127).astype(np.uint8))


@pytest.mark.parametrize("mag", [1e-3, 1.0, 1e4])
def test_mxfp8_split_lo_matches_torch_cast_of_the_residual(mag):
    """hi and the scales are the single-term quantisation's; lo is torch's
    RNE float8_e4m3fn cast of (x - hi * 2^X) / 2^(X-4), with the residual
    formed from torch's own cast of x / 2^X."""
    g = torch.Generator().manual_seed(int(mag * 100) % 997 + 1)
    x = (torch.randn(64, 256, generator=g) * mag).to(torch.bfloat16).float()
    x[1, :32] = 0.0
    hi, lo, s = oracle.mxfp8_split_ref(x)
    q1, s1 = oracle.mxfp8_quant_ref(x)
    assert np.array_equal(hi, q1) and np.array_equal(s, s1)
    X = torch.from_numpy(s.astype(np.float64) - 127.0).repeat_interleave(32, dim=1)
    xd = x.double()
    hv = (xd / torch.exp2(X)).float().to(torch.float8_e4m3fn).double() * torch.exp2(X)
    y = (xd - hv) / torch.exp2(torch.clamp(X - 4, min=-127))
    cast = y.float().to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(cast, lo)


def test_mxfp8_split_reconstructs_bf16_exactly():
    """hi * 2^X + lo * 2^(X-4) is every bfloat16 element above 2^-13 of its
    block maximum exactly, and misses smaller ones by less than 2^-21 of it."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(128, 512, generator=g)
    x = x * torch.exp2(torch.randint(-20, 20, (128, 512), generator=g).float())   # wide blocks
    x = x.to(torch.bfloat16).float()
    rec = oracle.mxfp8_split_dequant_ref(*oracle.mxfp8_split_ref(x)).double()
    xd = x.double()
    amax = xd.view(128, 16, 32).abs().amax(-1, keepdim=True).expand(128, 16, 32).reshape(128, 512)
    big = xd.abs() >= amax * 2.0 ** -13
    assert torch.equal(rec[big], xd[big])
    assert ((rec - xd).abs() <= amax * 2.0 ** -21).all()
    # a single MXFP8 term is far from exact on the same data
    one = oracle.mxfp8_dequant_ref(*oracle.mxfp8_quant_ref(x)).double()
    assert not torch.equal(one[big], xd[big])


def test_mxfp8_split_known_answers():
    """1 + 2^-7 in a block whose maximum it is: X = -8, x / 2^X = 258 rounds to
    256 (hi 0x78), the residual 2^-7 is 32 * 2^-12 (lo 0x60); zero blocks
    split to zeros; a non-finite element makes hi NaN, lo zero, scale 255."""
    x = torch.zeros(1, 128, dtype=torch.float64)
    x[0, :32] = 1.0 + 2.0 ** -7
    x[0, 96:] = 1.0
    x[0, 100] = float("nan")
    hi, lo, s = oracle.mxfp8_split_ref(x)
    assert list(s[0]) == [119, 0, 0, 255]
    assert (hi[0, :32] == 0x78).all() and (lo[0, :32] == 0x60).all()
    assert (hi[0, 32:96] == 0).all() and (lo[0, 32:96] == 0).all()
    assert (hi[0, 96:] & 0x7F == 0x7F).all() and (lo[0, 96:] == 0).all()
