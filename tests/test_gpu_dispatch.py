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
