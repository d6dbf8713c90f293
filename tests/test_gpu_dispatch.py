"""Device dispatch (block_streamer/gptoss.py:143-154) against a torch
restatement: per-expert counts and offsets, the expert-sorted pair order
(stable: token, then slot), its inverse, and the 128-row tile list.  Covers
the one-workgroup kernel (up to 4096 pairs) and the chunked two-launch one,
with dropped pairs (indices outside [0, E))."""

from __future__ import annotations

import pytest
import torch

from blockstreamer_amd import _lib, kernels
from tests.conftest import announce

pytestmark = pytest.mark.gpu

BM = 128


def _align(x: int) -> int:
    return (x + 255) // 256 * 256


def _read_workspace(ws: torch.Tensor, T: int, E: int, k: int):
    """The dispatch fields at the head of the forward workspace, in order:
    counts [E], offsets [E+1], row_pair [P], pair_pos [P], tiles [P/128+E]
    int2, num_tiles, each starting on a 256-byte boundary."""
    P = T * k
    max_tiles = (P + BM - 1) // BM + E
    sizes = [E * 4, (E + 1) * 4, P * 4, P * 4, max_tiles * 8, 4]
    off, views = 0, []
    for n in sizes:
        views.append(ws[off:off + n].view(torch.int32).cpu())
        off = _align(off + n)
    counts, offsets, row_pair, pair_pos, tiles, num_tiles = views
    return counts, offsets, row_pair, pair_pos, tiles.view(-1, 2), int(num_tiles[0])


def _reference(idx: torch.Tensor, E: int):
    e = idx.flatten().to(torch.int64)
    valid = (e >= 0) & (e < E)
    counts = torch.bincount(e[valid], minlength=E).to(torch.int32)
    offsets = torch.zeros(E + 1, dtype=torch.int32)
    offsets[1:] = torch.cumsum(counts, 0)
    key = torch.where(valid, e, torch.full_like(e, E))
    order = torch.argsort(key, stable=True)[: int(valid.sum())].to(torch.int32)
    pair_pos = torch.full((e.numel(),), -1, dtype=torch.int32)
    pair_pos[order.long()] = torch.arange(order.numel(), dtype=torch.int32)
    tiles = [(x, int(offsets[x]) + BM * j) for x in range(E) for j in range((int(counts[x]) + BM - 1) // BM)]
    return counts, offsets, order, pair_pos, torch.tensor(tiles, dtype=torch.int32).view(-1, 2)


@pytest.mark.parametrize("T,E,k", [(64, 128, 4), (1100, 8, 4), (3000, 32, 3), (8192, 128, 4), (5000, 256, 1)])
def test_dispatch_matches_restatement(device, T, E, k):
    g = torch.Generator().manual_seed(T + E + k)
    idx = torch.randint(0, E, (T, k), generator=g)
    idx[::13, 0] = E        # the masking index
    idx[5::17, k - 1] = -1  # any index outside [0, E)
    H = I = 64
    nb = kernels.moe_workspace_bytes(T, H, I, E, k)
    ws = kernels._aligned_bytes(nb, device)
    idx_d = idx.to(device)
    announce(f"dispatch T={T} E={E} k={k}")
    _lib.call("bsa_moe_dispatch", idx_d.data_ptr(), T, H, I, E, k, ws.data_ptr(), nb,
              _lib.stream_handle(device))
    torch.cuda.synchronize()
    counts, offsets, row_pair, pair_pos, tiles, ntiles = _read_workspace(ws, T, E, k)
    rc, ro, rr, rp, rt = _reference(idx, E)
    assert torch.equal(counts, rc)
    assert torch.equal(offsets, ro)
    assert torch.equal(row_pair[: rr.numel()], rr)
    assert torch.equal(pair_pos, rp)
    assert ntiles == rt.shape[0]
    assert torch.equal(tiles[:ntiles], rt)


@pytest.mark.parametrize("T", [1, 8, 64, 256, 257, 400])
def test_dispatch_folded_into_the_decode_gemm(device, T):
    """At decode batches the forward folds the dispatch into the persistent
    gate_up launch (every workgroup builds it and writes the same arrays).
    The workspace then holds exactly the dispatch of the restatement, dropped
    pairs included, and the layer equals the staged call (dispatch kernel,
    then the GEMMs) bit for bit.  Above 1024 pairs (T = 257, 400 at top-4)
    the decode kernels keep running with the dispatch as its own launch; the
    workspace and the output are the same."""
    from blockstreamer_amd import synthetic
    from tests.moe_util import expert_args

    E, k, H, I = 128, 4, 2880, 2880
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=31, scale_lo=116, scale_hi=120,
                            device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=32, device=device)
    idx = idx.clone()
    idx[::5, 1] = -1           # dropped pairs
    idx = idx.contiguous()
    announce(f"folded dispatch T={T}")
    gu_b, gu_s, gu_bias, dn_b, dn_s, dn_bias = expert_args(t)
    x = t["hidden"].contiguous()
    out = torch.empty(T, H, dtype=x.dtype, device=device)
    nb = kernels.moe_workspace_bytes(T, H, I, E, k)
    ws = kernels._aligned_bytes(nb, device)
    ws.fill_(0xFF)             # nothing left over from an earlier call
    bias_code = _lib.dtype_code(gu_bias.dtype)
    _lib.call("bsa_moe_experts_fwd", x.data_ptr(), T, H, I, E, k, idx.data_ptr(), w.data_ptr(),
              _lib.dtype_code(w.dtype), gu_b.data_ptr(), gu_s.data_ptr(), gu_bias.data_ptr(), dn_b.data_ptr(),
              dn_s.data_ptr(), dn_bias.data_ptr(), bias_code, 1.702, 7.0, out.data_ptr(), _lib.dtype_code(x.dtype),
              ws.data_ptr(), nb, None, 1, 0, _lib.stream_handle(device))  # path 1: the decode kernels
    staged = kernels.MoEStages(x, idx, w, gu_b, gu_s, gu_bias, dn_b, dn_s, dn_bias, path="stream").run()
    torch.cuda.synchronize()
    counts, offsets, row_pair, pair_pos, tiles, ntiles = _read_workspace(ws, T, E, k)
    rc, ro, rr, rp, rt = _reference(idx.cpu(), E)
    assert torch.equal(counts, rc)
    assert torch.equal(offsets, ro)
    assert torch.equal(row_pair[: rr.numel()], rr)
    assert torch.equal(pair_pos, rp)
    assert ntiles == rt.shape[0]
    assert torch.equal(tiles[:ntiles], rt)
    assert torch.equal(out.view(torch.int16), staged.view(torch.int16))


@pytest.mark.parametrize("T", [1, 64])
def test_decode_with_every_pair_dropped(device, T):
    """Every router index outside [0, E) (the masking index E and -1): the
    folded dispatch leaves every expert empty, every persistent workgroup
    returns right after writing it, and the layer is zero, as the reference
    adds nothing to its zeros (gptoss.py:143-176); the staged call agrees."""
    from blockstreamer_amd import synthetic
    from tests.moe_util import expert_args

    E, k, H, I = 128, 4, 2880, 2880
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=41, scale_lo=116, scale_hi=120,
                            device=device)
    idx = torch.full((T, k), -1, dtype=torch.int64, device=device)
    idx[:, 1::2] = E
    w = torch.full((T, k), 0.25, dtype=torch.float32, device=device)
    announce(f"every pair dropped T={T}")
    gu_b, gu_s, gu_bias, dn_b, dn_s, dn_bias = expert_args(t)
    x = t["hidden"].contiguous()
    out = torch.full((T, H), 7.0, dtype=x.dtype, device=device)
    nb = kernels.moe_workspace_bytes(T, H, I, E, k)
    ws = kernels._aligned_bytes(nb, device)
    ws.fill_(0xFF)
    _lib.call("bsa_moe_experts_fwd", x.data_ptr(), T, H, I, E, k, idx.data_ptr(), w.data_ptr(),
              _lib.dtype_code(w.dtype), gu_b.data_ptr(), gu_s.data_ptr(), gu_bias.data_ptr(), dn_b.data_ptr(),
              dn_s.data_ptr(), dn_bias.data_ptr(), _lib.dtype_code(gu_bias.dtype), 1.702, 7.0, out.data_ptr(),
              _lib.dtype_code(x.dtype), ws.data_ptr(), nb, None, 1, 0, _lib.stream_handle(device))
    staged = kernels.MoEStages(x, idx, w, gu_b, gu_s, gu_bias, dn_b, dn_s, dn_bias, path="stream").run()
    torch.cuda.synchronize()
    counts, offsets, _, pair_pos, _, ntiles = _read_workspace(ws, T, E, k)
    assert int(counts.abs().sum()) == 0 and int(offsets.abs().sum()) == 0
    assert torch.equal(pair_pos, torch.full_like(pair_pos, -1))
    assert ntiles == 0
    assert int(torch.count_nonzero(out)) == 0
    assert torch.equal(out.view(torch.int16), staged.view(torch.int16))


@pytest.mark.parametrize("T", [1, 64])
def test_decode_part_kernel_runs_on_a_dispatched_workspace(device, T):
    """A decode batch whose biases are only 2-byte aligned cannot take the
    persistent kernel (it DMAs the bias), so its gate_up runs the part
    kernel, which does not build the dispatch: the forward must then launch
    the dispatch itself.  The workspace starts zeroed (an undispatched
    workspace would give every expert zero rows and a bias-only layer, not
    out-of-range indices), and must end up holding the restatement's
    dispatch, with the layer equal to the staged call bit for bit."""
    from blockstreamer_amd import synthetic
    from tests.moe_util import expert_args

    E, k, H, I = 128, 4, 2880, 2880
    t = synthetic.moe_layer(synthetic.MoEShape(E, k, H, I, T), seed=61, scale_lo=116, scale_hi=120,
                            device=device)
    idx, w = synthetic.random_routing(T, E, k, seed=62, device=device)
    gu_b, gu_s, gu_bias, dn_b, dn_s, dn_bias = expert_args(t)

    def shifted(b):  # same values, storage 2 bytes past a 16-byte boundary
        buf = torch.empty(b.numel() + 1, dtype=b.dtype, device=device)
        buf[1:] = b.reshape(-1)
        return buf[1:].view(b.shape)

    gu_bias, dn_bias = shifted(gu_bias), shifted(dn_bias)
    assert gu_bias.data_ptr() % 16 == 2
    x = t["hidden"].contiguous()
    out = torch.empty(T, H, dtype=x.dtype, device=device)
    nb = kernels.moe_workspace_bytes(T, H, I, E, k)
    ws = kernels._aligned_bytes(nb, device)
    ws.zero_()
    announce(f"decode part kernel on a zeroed workspace T={T}")
    _lib.call("bsa_moe_experts_fwd", x.data_ptr(), T, H, I, E, k, idx.data_ptr(), w.data_ptr(),
              _lib.dtype_code(w.dtype), gu_b.data_ptr(), gu_s.data_ptr(), gu_bias.data_ptr(), dn_b.data_ptr(),
              dn_s.data_ptr(), dn_bias.data_ptr(), _lib.dtype_code(gu_bias.dtype), 1.702, 7.0, out.data_ptr(),
              _lib.dtype_code(x.dtype), ws.data_ptr(), nb, None, 1, 0, _lib.stream_handle(device))
    staged = kernels.MoEStages(x, idx, w, gu_b, gu_s, gu_bias, dn_b, dn_s, dn_bias, path="stream").run()
    torch.cuda.synchronize()
    counts, offsets, row_pair, pair_pos, tiles, ntiles = _read_workspace(ws, T, E, k)
    rc, ro, rr, rp, rt = _reference(idx.cpu(), E)
    assert torch.equal(counts, rc) and torch.equal(offsets, ro)
    assert torch.equal(row_pair[: rr.numel()], rr) and torch.equal(pair_pos, rp)
    assert torch.equal(out.view(torch.int16), staged.view(torch.int16))
