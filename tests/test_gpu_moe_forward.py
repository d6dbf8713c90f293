"""MoE expert forward parity on the GPU (fused dispatch, grouped GEMMs, combine)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from blockstreamer_amd import gptoss, kernels, synthetic
from tests.conftest import announce
from tests.golden.make_golden import tiny_layer
from tests.moe_util import assert_layer_close, expert_args, gpu_reference, oracle_tokens

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
PATHS = ["stream", "tiled"]


def _to(t: dict, device) -> dict:
    return {k: v.to(device) for k, v in t.items()}


@pytest.mark.parametrize("path", PATHS)
def test_tiny_layer_matches_golden(device, path):
    """8 experts, top-2, hidden 256, intermediate 256, 64 tokens vs transformers fp32."""
    gold = np.load(GOLDEN / "tiny_layer.npz")
    t = _to(tiny_layer(), device)
    idx = torch.from_numpy(gold["router_indices"]).to(device)
    w = torch.from_numpy(gold["router_scores"]).to(device)
    announce(f"moe tiny golden path={path}")
    out = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(t), path=path)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    assert_layer_close(out, torch.from_numpy(gold["experts_out"]), f"tiny {path}")


def test_module_drop_in_tiny(device):
    """MXFP4Experts bound through functional_call, like StreamedModel does."""
    from torch.func import functional_call
    from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig

    gold = np.load(GOLDEN / "tiny_layer.npz")
    shape = synthetic.TINY
    cfg = GptOssConfig(num_local_experts=shape.experts, hidden_size=shape.hidden,
                       intermediate_size=shape.intermediate, num_experts_per_tok=shape.top_k,
                       num_hidden_layers=1)
    mod = gptoss.MXFP4Experts(cfg, torch.bfloat16)
    t = _to(tiny_layer(), device)
    state = {k: t[k] for k in ("gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
                               "down_proj_blocks", "down_proj_scales", "down_proj_bias")}
    versions = {k: v._version for k, v in state.items()}
    idx = torch.from_numpy(gold["router_indices"]).to(device)
    w = torch.from_numpy(gold["router_scores"]).to(torch.bfloat16).to(device)
    announce("moe module functional_call")
    with torch.no_grad():
        out = functional_call(mod, state, (t["hidden"], idx, w), strict=True)
    assert all(v._version == versions[k] for k, v in state.items())
    assert_layer_close(out, torch.from_numpy(gold["experts_out"]), "module tiny")


CASES = [
    # (E, k, H, I, T, scale_lo, scale_hi)
    (6, 3, 96, 64, 20, 118, 126),
    (8, 2, 256, 256, 1, 119, 129),
    (32, 4, 256, 128, 300, 119, 129),
    (16, 4, 512, 256, 129, 116, 120),
    (4, 1, 128, 192, 77, 119, 127),
]


@pytest.mark.parametrize("case", CASES, ids=[f"E{c[0]}k{c[1]}H{c[2]}I{c[3]}T{c[4]}" for c in CASES])
@pytest.mark.parametrize("path", PATHS)
def test_random_shapes_vs_oracle(device, case, path):
    E, k, H, I, T, lo, hi = case
    shape = synthetic.MoEShape(E, k, H, I, T)
    t = synthetic.moe_layer(shape, seed=E * 7 + T, scale_lo=lo, scale_hi=hi)
    idx, w = synthetic.random_routing(T, E, k, seed=T + 1)
    want = oracle.experts_ref(t["hidden"], idx, w.float(), *expert_args(t))
    g = _to(t, device)
    announce(f"moe random {case} path={path}")
    got = kernels.moe_experts_forward(g["hidden"], idx.to(device), w.to(device), *expert_args(g),
                                      path=path)
    assert_layer_close(got, want, f"{case} {path}", absolute=(hi <= 120))


def _realistic(device, shape, seed, bias_std=0.0):
    return synthetic.moe_layer(shape, seed=seed, scale_lo=116, scale_hi=120,
                               router_bias_std=bias_std, device=device)


@pytest.mark.parametrize("T", [1, 8, 64])
def test_gptoss_120b_decode_vs_oracle(device, T):
    """128 experts, top-4, hidden = intermediate = 2880, skewed router bias N(0, 0.5)."""
    shape = synthetic.MoEShape(128, 4, 2880, 2880, T)
    t = synthetic.moe_layer(shape, seed=4, scale_lo=115, scale_hi=131, router_bias_std=0.5,
                            device=device)
    _, scores, idx = oracle.router_ref(t["hidden"].cpu(), t["router_weight"].cpu(),
                                       t["router_bias"].cpu(), 4)
    announce(f"moe 120b decode T={T}")
    got = kernels.moe_experts_forward(t["hidden"], idx.to(device), scores.to(device),
                                      *expert_args(t))
    tokens = torch.arange(T)  # every token of the batch
    want = oracle_tokens(t, idx, scores, tokens)
    assert_layer_close(got.cpu()[tokens], want, f"120b decode T={T}")


def test_gptoss_120b_decode_realistic_scales_absolute(device):
    shape = synthetic.MoEShape(128, 4, 2880, 2880, 64)
    t = _realistic(device, shape, seed=14, bias_std=0.5)
    _, scores, idx = oracle.router_ref(t["hidden"].cpu(), t["router_weight"].cpu(),
                                       t["router_bias"].cpu(), 4)
    announce("moe 120b decode realistic scales")
    got = kernels.moe_experts_forward(t["hidden"], idx.to(device), scores.to(device),
                                      *expert_args(t))
    tokens = torch.arange(64)
    want = oracle_tokens(t, idx, scores, tokens)
    assert_layer_close(got.cpu()[tokens], want, "120b decode realistic", absolute=True)


@pytest.mark.parametrize("path", PATHS + ["auto", "mx"])
def test_gptoss_20b_full_layer(device, path):
    """32 experts, top-4, 2048 tokens: every token vs a float32 GPU reference,
    a subset vs the CPU oracle.  "auto" is the path the benchmark reports for
    this workload (it resolves to the MX kernels at 256 rows per expert)."""
    shape = synthetic.MoEShape(32, 4, 2880, 2880, 2048)
    t = synthetic.moe_layer(shape, seed=3, scale_lo=115, scale_hi=131, router_bias_std=0.01,
                            device=device)
    _, scores, idx = oracle.router_ref(t["hidden"].cpu(), t["router_weight"].cpu(),
                                       t["router_bias"].cpu(), 4)
    idx, scores = idx.to(device), scores.to(device)
    announce(f"moe 20b full layer path={path}")
    got = kernels.moe_experts_forward(t["hidden"], idx, scores, *expert_args(t), path=path)
    ref = gpu_reference(t, idx, scores)
    assert_layer_close(got, ref, f"20b all tokens {path}")
    tokens = torch.randperm(2048, generator=torch.Generator().manual_seed(20))[:64]
    assert_layer_close(got.cpu()[tokens], oracle_tokens(t, idx, scores, tokens), f"20b oracle {path}")


def test_deterministic_and_permutation_equivariant(device):
    """Bitwise: two runs agree, and permuting tokens permutes the output."""
    shape = synthetic.MoEShape(32, 4, 2880, 2880, 512)
    t = synthetic.moe_layer(shape, seed=8, scale_lo=115, scale_hi=131, device=device)
    idx, w = synthetic.random_routing(512, 32, 4, seed=9, device=device)
    announce("moe determinism / permutation")
    a = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(t))
    b = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(t))
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    perm = torch.randperm(512, generator=torch.Generator().manual_seed(3)).to(device)
    c = kernels.moe_experts_forward(t["hidden"][perm], idx[perm], w[perm], *expert_args(t))
    assert torch.equal(c.view(torch.int16), a[perm].view(torch.int16))


def test_edge_cases(device):
    shape = synthetic.MoEShape(8, 2, 256, 256, 37)
    t = synthetic.moe_layer(shape, seed=5, scale_lo=119, scale_hi=125, device=device)
    idx, w = synthetic.random_routing(37, 8, 2, seed=6, device=device)
    args = expert_args(t)
    announce("moe edge cases")
    # the masking index E (and anything outside [0, E)) contributes nothing
    idx_m = idx.clone()
    idx_m[:, 1] = 8
    only_first = kernels.moe_experts_forward(t["hidden"], idx[:, :1].contiguous(), w[:, :1].contiguous(), *args)
    masked = kernels.moe_experts_forward(t["hidden"], idx_m, w, *args)
    assert torch.equal(masked.view(torch.int16), only_first.view(torch.int16))
    # zero routing weight contributes nothing (up to the float32 sum order)
    w0 = w.clone()
    w0[:, 1] = 0
    assert_layer_close(kernels.moe_experts_forward(t["hidden"], idx, w0, *args), only_first, "zero weight")
    # every token on one expert: many row tiles of one expert
    idx_one = torch.zeros_like(idx)
    idx_one[:, 1] = 3
    for path in PATHS:
        got = kernels.moe_experts_forward(t["hidden"], idx_one, w, *args, path=path)
        want = oracle.experts_ref(t["hidden"].cpu(), idx_one.cpu(), w.cpu().float(),
                                  *[a.cpu() for a in args])
        assert_layer_close(got, want, f"one expert {path}")
    # a token routed twice to the same expert gets both contributions
    idx_dup = idx.clone()
    idx_dup[:, 1] = idx_dup[:, 0]
    got = kernels.moe_experts_forward(t["hidden"], idx_dup, w, *args)
    want = oracle.experts_ref(t["hidden"].cpu(), idx_dup.cpu(), w.cpu().float(), *[a.cpu() for a in args])
    assert_layer_close(got, want, "duplicate slot")
    # no tokens
    empty = kernels.moe_experts_forward(t["hidden"][:0], idx[:0], w[:0], *args)
    assert empty.shape == (0, 256)


@pytest.mark.parametrize("path", PATHS)
def test_shard_blob_views_8_byte_aligned(device, path):
    """Packed weights as 8-byte-aligned views into one byte blob (the NVMe
    staging layout) take the register-copy kernels; results match the oracle."""
    shape = synthetic.MoEShape(8, 2, 256, 256, 150)
    t = synthetic.moe_layer(shape, seed=12, scale_lo=119, scale_hi=127, device=device)
    idx, w = synthetic.random_routing(150, 8, 2, seed=13, device=device)
    views = dict(t)
    for name in ("gate_up_proj_blocks", "gate_up_proj_scales", "down_proj_blocks", "down_proj_scales"):
        src = t[name]
        blob = torch.zeros(src.numel() + 64, dtype=torch.uint8, device=device)
        blob[8:8 + src.numel()] = src.reshape(-1)
        views[name] = blob[8:8 + src.numel()].view(src.shape)
        assert views[name].data_ptr() % 16 == 8
    announce(f"moe 8-byte aligned views path={path}")
    got = kernels.moe_experts_forward(t["hidden"], idx, w, *expert_args(views), path=path)
    want = oracle.experts_ref(t["hidden"].cpu(), idx.cpu(), w.cpu().float(),
                              *[a.cpu() for a in expert_args(t)])
    assert_layer_close(got, want, f"8-byte views {path}")


@pytest.mark.parametrize("k", [2, 3, 4])
def test_combine_batched_equals_split(device, k):
    """1100 tokens take the batched combine (all loads of a token in flight),
    550 the per-slice one: same slot order and sums, so the outputs agree bit
    for bit, with masked (index E) and repeated slots."""
    E, H, I, T = 8, 256, 256, 1100
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=80 + k, scale_lo=118,
                            scale_hi=124, device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=90 + k, device=device)
    idx = idx.clone()
    idx[::7, k - 1] = E                 # masked slot
    idx[3::11, 0] = idx[3::11, k - 1]   # repeated expert (masked where that slot is)
    idx = idx.contiguous()
    args = expert_args(t)
    announce(f"combine batched vs split, k={k}")
    full = kernels.moe_experts_forward(t["hidden"], idx, w, *args, path="tiled")
    parts = [kernels.moe_experts_forward(t["hidden"][s].contiguous(), idx[s].contiguous(),
                                         w[s].contiguous(), *args, path="tiled")
             for s in (slice(0, 550), slice(550, T))]
    assert torch.equal(full.view(torch.int16), torch.cat(parts).view(torch.int16))


@pytest.mark.parametrize("path", PATHS + ["auto", "mx"])
def test_gptoss_20b_full_layer_trained_scales_absolute(device, path):
    """The 20b-shaped layer (2048 tokens) with E8M0 scales in [116, 120]:
    outputs of order one, every token against the float32 GPU reference with
    the layer bar's max-abs 2e-2 as an absolute bound."""
    shape = synthetic.MoEShape(32, 4, 2880, 2880, 2048)
    t = _realistic(device, shape, seed=13, bias_std=0.01)
    _, scores, idx = oracle.router_ref(t["hidden"].cpu(), t["router_weight"].cpu(),
                                       t["router_bias"].cpu(), 4)
    idx, scores = idx.to(device), scores.to(device)
    announce(f"moe 20b full layer, trained scales, path={path}")
    got = kernels.moe_experts_forward(t["hidden"], idx, scores, *expert_args(t), path=path)
    assert_layer_close(got, gpu_reference(t, idx, scores), f"20b trained scales {path}", absolute=True)
