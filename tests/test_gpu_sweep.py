"""Seeded sweep of layer shapes: forward on every applicable GEMM kernel and
the input-gradient backward, against the float32 oracle.

Shapes are drawn once from a fixed seed within the library's constraints
(hidden % 64 == 0, intermediate % 32 == 0, top-k <= experts): few to many
experts, top-1 to top-8, single tokens to a few hundred, so that tiles are
partial, experts go unhit, and rows, columns and k-tiles end at every kind of
boundary.  Bars: the layer bar for the forward (tests/moe_util.py), the
gradient bar for the backward (relative L2 <= 1e-2).  The MX path is checked
against the oracle's emulation of its own arithmetic (MXFP8 activations).
Where both projections have an even group count, the forward is also run on
the blocks in the k-pair shard layout and must give the same bits.
"""

from __future__ import annotations

import random

import pytest
import torch

import oracle
from blockstreamer_amd import kernels, synthetic
from tests.conftest import announce
from tests.moe_util import assert_layer_close, errors, expert_args

pytestmark = pytest.mark.gpu


def _shapes(n: int = 12, seed: int = 2024):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        E = rng.choice([2, 3, 5, 8, 16, 32, 64])
        k = rng.randint(1, min(8, E))
        H = 64 * rng.randint(1, 6)
        I = 32 * rng.randint(1, 8)
        T = rng.choice([1, 2, 7, 33, 64, 100, 257])
        out.append((E, k, H, I, T))
    return out


SHAPES = _shapes()


def _inputs(shape, device):
    E, k, H, I, T = shape
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=E * 31 + H + I + T, scale_lo=116,
                            scale_hi=122)
    idx, w = synthetic.random_routing(T, E, k, seed=T * 3 + E, dtype=torch.float32)
    return t, idx, w


@pytest.mark.parametrize("shape", SHAPES, ids=[f"E{s[0]}k{s[1]}H{s[2]}I{s[3]}T{s[4]}" for s in SHAPES])
def test_sweep_forward(device, shape):
    E, k, H, I, T = shape
    t, idx, w = _inputs(shape, device)
    want = oracle.experts_ref(t["hidden"], idx, w, *expert_args(t))
    g = {n: (v.to(device) if torch.is_tensor(v) else v) for n, v in t.items()}
    # the k-pair shard layout where the shape allows it (both projections with an
    # even group count): the same bits as the checkpoint layout
    kp = (I // 32) % 2 == 0
    kp_args = list(expert_args(g))
    if kp:
        kp_args[0], kp_args[3] = kernels.to_kpair(kp_args[0]), kernels.to_kpair(kp_args[3])
    for path in ("auto", "stream", "tiled"):
        announce(f"sweep forward {shape} {path}")
        got = kernels.moe_experts_forward(g["hidden"], idx.to(device), w.to(device), *expert_args(g), path=path)
        assert_layer_close(got, want, f"{shape} {path}", absolute=True)
        if kp:
            got_kp = kernels.moe_experts_forward(g["hidden"], idx.to(device), w.to(device), *kp_args, path=path)
            assert torch.equal(got_kp.view(torch.int16), got.view(torch.int16)), f"{shape} {path} k-pair"
    if H % 64 == 0 and I % 64 == 0:
        announce(f"sweep forward {shape} mx")
        want_mx = oracle.experts_mx_ref(t["hidden"], idx, w, *expert_args(t))
        got = kernels.moe_experts_forward(g["hidden"], idx.to(device), w.to(device), *expert_args(g), path="mx")
        assert_layer_close(got, want_mx, f"{shape} mx vs MX oracle", absolute=True)
        assert_layer_close(got, want, f"{shape} mx vs float32", absolute=True)


@pytest.mark.parametrize("shape", SHAPES, ids=[f"E{s[0]}k{s[1]}H{s[2]}I{s[3]}T{s[4]}" for s in SHAPES])
def test_sweep_backward(device, shape):
    from blockstreamer_amd import gptoss

    E, k, H, I, T = shape
    t, idx, w = _inputs(shape, device)
    gout = (torch.randn(T, H, generator=torch.Generator().manual_seed(T + H)) * 0.1).to(torch.bfloat16)
    h = t["hidden"].float().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    out = oracle.experts_ref(h, idx, wr, *expert_args(t))
    out.backward(gout.float())
    g = {n: (v.to(device) if torch.is_tensor(v) else v) for n, v in t.items()}
    hd = g["hidden"].detach().clone().requires_grad_(True)
    wd = w.to(device).requires_grad_(True)
    announce(f"sweep backward {shape}")
    o = gptoss._MoEExperts.apply(hd, idx.to(device), wd, *expert_args(g), 1.702, 7.0)
    o.backward(gout.to(device))
    for what, got, want in (("d hidden", hd.grad, h.grad), ("d weights", wd.grad, wr.grad)):
        rel_l2, max_abs, scale = errors(got, want)
        print(f"{shape} {what}: rel_l2={rel_l2:.3e} max_abs={max_abs:.3e} (|ref|max={scale:.3e})")
        assert rel_l2 <= 1e-2 and max_abs <= 5e-2 * max(scale, 1e-30)
