"""The k-pair shard layout of the packed blocks.

Repacking is checked against the layout's definition (``oracle.to_kpair_ref``).
Every kernel that reads packed blocks -- dequant, the decode kernels (the
persistent one, its part-pipelined fallback, the generic streaming one), the
prefill tile kernel, the MX kernel and the backward -- only changes where it
reads each 16-byte group from, so the bar is bit-for-bit equality with the
same call on the checkpoint layout.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from blockstreamer_amd import gptoss, kernels, synthetic
from tests.conftest import announce

pytestmark = pytest.mark.gpu

NAMES = ("gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
         "down_proj_blocks", "down_proj_scales", "down_proj_bias")


def _kp_args(g):
    a = [g[n] for n in NAMES]
    a[0] = kernels.to_kpair(a[0])
    a[3] = kernels.to_kpair(a[3])
    return a


def _same(a, b):
    return torch.equal(a.contiguous().view(torch.int16 if a.element_size() == 2 else torch.int32),
                       b.contiguous().view(torch.int16 if b.element_size() == 2 else torch.int32))


@pytest.mark.parametrize("shape", [(1, 16, 2), (3, 32, 4), (8, 512, 8), (2, 5760, 90)])
def test_repack_matches_definition_and_round_trips(device, shape):
    E, R, G = shape
    blocks = torch.randint(0, 256, (E, R, G, 16), generator=torch.Generator().manual_seed(R + G),
                           dtype=torch.uint8)
    announce(f"k-pair repack {shape}")
    kp = kernels.to_kpair(blocks.to(device))
    assert kernels.blocks_layout(kp) == kernels.LAYOUT_KPAIR
    assert torch.equal(kp.cpu(), oracle.to_kpair_ref(blocks))
    back = kernels.from_kpair(kp)
    assert torch.equal(back.cpu(), blocks)


def test_repack_refuses_bad_shapes(device):
    with pytest.raises(ValueError, match="rows % 16"):
        kernels.to_kpair(torch.zeros(1, 24, 4, 16, dtype=torch.uint8, device=device))
    with pytest.raises(ValueError, match="checkpoint"):
        kernels.to_kpair(torch.zeros(1, 1, 2, 16, 2, 16, dtype=torch.uint8, device=device))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_dequant_same_in_both_layouts(device, dtype):
    t = synthetic.moe_layer(synthetic.MoEShape(4, 2, 256, 256, 8), seed=3, scale_lo=110, scale_hi=140)
    b, s = t["gate_up_proj_blocks"].to(device), t["gate_up_proj_scales"].to(device)
    announce(f"k-pair dequant {dtype}")
    want = kernels.dequantize_mxfp4(b, s, dtype)
    got = kernels.dequantize_mxfp4(kernels.to_kpair(b), s, dtype)
    assert _same(got, want)


# (E, k, H, I, T, path): the generic streaming kernel (K = 256), the
# persistent decode kernel and the prefill tile kernel at the gpt-oss
# hidden size, and the MX kernel
FWD_CASES = [
    (8, 2, 256, 256, 64, "stream"),
    (8, 2, 256, 256, 64, "tiled"),
    (8, 2, 256, 256, 64, "mx"),
    (16, 4, 2880, 2880, 8, "stream"),
    (16, 4, 2880, 2880, 64, "auto"),
    (32, 4, 2880, 2880, 512, "tiled"),
    (32, 4, 2880, 2880, 512, "mx"),
]


@pytest.mark.parametrize("case", FWD_CASES, ids=[f"E{c[0]}k{c[1]}H{c[2]}T{c[4]}-{c[5]}" for c in FWD_CASES])
def test_forward_same_in_both_layouts(device, case):
    E, k, H, I, T, path = case
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=E + T, scale_lo=116, scale_hi=122,
                            device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=T, dtype=torch.float32)
    idx, w = idx.to(device), w.to(device)
    args = [t[n] for n in NAMES]
    announce(f"k-pair forward {case}")
    want = kernels.moe_experts_forward(t["hidden"], idx, w, *args, path=path)
    got = kernels.moe_experts_forward(t["hidden"], idx, w, *_kp_args(t), path=path)
    assert _same(got, want)


def test_decode_fallback_kernel_same_in_both_layouts(device):
    """A bias view that is not 16-byte aligned sends the decode to the
    part-pipelined kernel."""
    E, k, H, I, T = 16, 4, 2880, 2880, 8
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=5, scale_lo=116, scale_hi=122,
                            device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=2, dtype=torch.float32)
    idx, w = idx.to(device), w.to(device)
    args = [t[n] for n in NAMES]
    for j in (2, 5):  # biases as 4-byte aligned views
        buf = torch.empty(args[j].numel() + 2, dtype=args[j].dtype, device=device)
        view = buf[2:].view(args[j].shape)
        view.copy_(args[j])
        args[j] = view
    kp = list(args)
    kp[0], kp[3] = kernels.to_kpair(args[0]), kernels.to_kpair(args[3])
    announce("k-pair decode fallback kernel")
    want = kernels.moe_experts_forward(t["hidden"], idx, w, *args, path="stream")
    got = kernels.moe_experts_forward(t["hidden"], idx, w, *kp, path="stream")
    assert _same(got, want)


@pytest.mark.parametrize("shape", [(8, 2, 256, 256, 64), (32, 4, 2880, 2880, 256)])
def test_backward_same_in_both_layouts(device, shape):
    E, k, H, I, T = shape
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=7, scale_lo=116, scale_hi=122,
                            device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=3, dtype=torch.float32)
    idx, w = idx.to(device), w.to(device)
    gout = (torch.randn(T, H, generator=torch.Generator().manual_seed(9)) * 0.1).to(torch.bfloat16).to(device)
    res = []
    for args in ([t[n] for n in NAMES], _kp_args(t)):
        h = t["hidden"].detach().clone().requires_grad_(True)
        wr = w.clone().requires_grad_(True)
        announce(f"k-pair backward {shape} layout {kernels.blocks_layout(args[0])}")
        out = gptoss._MoEExperts.apply(h, idx, wr, *args, 1.702, 7.0)
        out.backward(gout)
        res.append((out.detach(), h.grad, wr.grad))
    for a, b in zip(*res):
        assert _same(a, b)


def test_module_binds_k_pair_tensors(device):
    """MXFP4Experts takes k-pair blocks through functional_call under the
    checkpoint names and returns what the checkpoint layout gives."""
    from types import SimpleNamespace
    E, k, H, I, T = 8, 2, 256, 256, 32
    cfg = SimpleNamespace(num_local_experts=E, hidden_size=H, intermediate_size=I, num_experts_per_tok=k)
    mod = gptoss.MXFP4Experts(cfg, torch.bfloat16)
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=11, scale_lo=116, scale_hi=122,
                            device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=4, dtype=torch.bfloat16)
    idx, w = idx.to(device), w.to(device)
    ck = {n: t[n] for n in NAMES}
    kp = dict(ck, gate_up_proj_blocks=kernels.to_kpair(ck["gate_up_proj_blocks"]),
              down_proj_blocks=kernels.to_kpair(ck["down_proj_blocks"]))
    announce("k-pair module binding")
    want = torch.func.functional_call(mod, ck, (t["hidden"], idx, w), strict=True)
    got = torch.func.functional_call(mod, kp, (t["hidden"], idx, w), strict=True)
    assert _same(got, want)


def _at_offset(x: torch.Tensor, by: int) -> torch.Tensor:
    """Same bytes, storage starting ``by`` bytes past a 16-byte boundary."""
    buf = torch.empty(x.numel() + 32, dtype=torch.uint8, device=x.device)
    off = (by - buf.data_ptr()) % 16
    v = buf[off:off + x.numel()].view(x.shape)
    v.copy_(x)
    assert v.data_ptr() % 16 == by
    return v


def test_misaligned_k_pair_blocks_are_refused(device):
    """k-pair blocks at an 8-byte offset (a blob written with the checkpoint's
    8-byte alignment) are a ValueError, not a copy on every call."""
    E, k, H, I, T = 8, 2, 256, 256, 16
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=12, scale_lo=116, scale_hi=122,
                            device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=6, dtype=torch.float32, device=device)
    kp = _kp_args(t)
    kp[0] = _at_offset(kp[0], 8)
    announce("k-pair misaligned blocks refused")
    with pytest.raises(ValueError, match="16-byte aligned"):
        kernels.moe_experts_forward(t["hidden"], idx, w, *kp)
    with pytest.raises(ValueError, match="16-byte aligned"):
        kernels.dequantize_mxfp4(kp[0], kp[1])
    ws = torch.zeros(kernels.moe_workspace_bytes(T, H, I, E, k), dtype=torch.uint8, device=device)
    fac = torch.zeros(T * k, 2 * I, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="16-byte aligned"):
        kernels.moe_experts_backward(t["hidden"], t["hidden"], idx, w, kp[0], kp[1], kp[3], kp[4], ws, fac)


@pytest.mark.parametrize("dims", [(8, 2, 256, 256, 16), (8, 2, 256, 256, 300), (4, 4, 2880, 2880, 8)],
                         ids=["small-decode", "small-prefill", "gptoss-decode"])
@pytest.mark.parametrize("by", [8, 4])
def test_k_pair_blocks_with_unaligned_scales(device, dims, by):
    """k-pair blocks on a 16-byte boundary with scales only 8- or 4-byte
    aligned (the checkpoint's shard alignment): every forward path and the
    backward give the checkpoint layout's bits.  The checkpoint call gets the
    same scale alignment, since alignment picks the kernel (at K = 2880 the
    persistent decode kernel needs 16-byte aligned scales, and the streaming
    kernel that replaces it rounds differently)."""
    E, k, H, I, T = dims
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=13 + T, scale_lo=116, scale_hi=122,
                            device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=7, dtype=torch.float32, device=device)
    kp = _kp_args(t)
    kp[1] = _at_offset(kp[1], by)
    kp[4] = _at_offset(kp[4], by)
    ck = [t[n] for n in NAMES]
    ck[1] = _at_offset(ck[1], by)
    ck[4] = _at_offset(ck[4], by)
    for path in ("auto", "stream", "tiled", "mx"):
        announce(f"k-pair blocks, scales {by} bytes off, path={path}, {dims}")
        want = kernels.moe_experts_forward(t["hidden"], idx, w, *ck, path=path)
        got = kernels.moe_experts_forward(t["hidden"], idx, w, *kp, path=path)
        assert _same(got, want), path
    announce(f"k-pair blocks, scales {by} bytes off, backward, {dims}")
    g = torch.randn(T, H, device=device).to(torch.bfloat16)
    outs = []
    for a in (ck, kp):
        _, ws, pre = kernels.moe_experts_forward(t["hidden"], idx, w, *a, save=True)
        outs.append(kernels.moe_experts_backward(g, t["hidden"], idx, w, a[0], a[1], a[3], a[4], ws, pre))
    torch.cuda.synchronize()
    assert _same(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
