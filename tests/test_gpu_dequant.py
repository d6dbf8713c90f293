"""MXFP4 dequant kernel parity on the GPU (bit-exact against the oracle)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from blockstreamer_amd import gptoss, kernels, synthetic
from tests.conftest import announce
from tests.golden.make_golden import exhaustive_inputs

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
NAN_BITS = {"bf16": 0x7FC0, "f16": 0x7E00, "f32": 0x7FC00000}


def _bits(t: torch.Tensor) -> np.ndarray:
    view = torch.int32 if t.dtype == torch.float32 else torch.int16
    return t.detach().cpu().contiguous().view(view).numpy()


def _assert_bitexact(got: torch.Tensor, want: torch.Tensor, what: str):
    ok = oracle.bits_equal_or_both_nan(_bits(got), _bits(want), want.dtype)
    if not ok.all():
        bad = np.argwhere(~ok)
        raise AssertionError(f"{what}: {len(bad)} mismatches, first {bad[:5].tolist()}")


@pytest.mark.parametrize("name", list(DTYPES))
@pytest.mark.parametrize("mode", [0, 1])
def test_exhaustive_byte_scale_table(device, name, mode):
    """All 256 packed bytes under all 256 scale bytes vs oracle and golden table."""
    dt = DTYPES[name]
    blocks, scales = exhaustive_inputs()
    announce(f"dequant exhaustive dtype={name} mode={mode}")
    got = kernels.dequantize_mxfp4(blocks.to(device), scales.to(device), dt, mode=mode)
    torch.cuda.synchronize()
    want = oracle.dequant_c(blocks, scales, dt)
    _assert_bitexact(got, want, f"exhaustive {name} mode {mode}")
    gold = np.load(GOLDEN / "dequant_table.npz")[name]
    assert oracle.bits_equal_or_both_nan(_bits(got)[0], gold, dt).all()
    # NaN comes out as the canonical quiet NaN
    bits = _bits(got).astype(np.int64) & (0xFFFFFFFF if name == "f32" else 0xFFFF)
    nan_mask = torch.isnan(got.cpu()).numpy()
    assert (bits[nan_mask] == NAN_BITS[name]).all()


def test_hardware_converter_range(device):
    """The gfx950 converter (mode 2) is exact on the scale range mode 0 uses it for."""
    blocks, scales = exhaustive_inputs()
    announce("dequant hw converter validation")
    got = kernels.dequantize_mxfp4(blocks.to(device), scales.to(device), torch.bfloat16, mode=2)
    want = oracle.dequant_c(blocks, scales, torch.bfloat16)
    ok = oracle.bits_equal_or_both_nan(_bits(got), _bits(want), torch.bfloat16)[0]  # [K, R=scale]
    exact_scales = [s for s in range(256) if ok[:, s].all()]
    bad = sorted(set(range(256)) - set(exact_scales))
    print(f"hw converter inexact for scale bytes: {bad}")
    # scale byte 255 (E8M0 NaN) is the one the automatic mode keeps off the converter
    assert bad == [255], bad


@pytest.mark.parametrize("name", list(DTYPES))
@pytest.mark.parametrize("E,R,G", [(3, 64, 8), (2, 40, 5), (2, 24, 90), (1, 13, 3), (2, 8, 1), (4, 136, 9)])
def test_random_shapes(device, name, E, R, G):
    dt = DTYPES[name]
    blocks, scales = synthetic.packed_weights(E, R, G, seed=E * 1000 + R * 10 + G, scale_lo=0,
                                              scale_hi=255)
    announce(f"dequant random E={E} R={R} G={G} dtype={name}")
    got = kernels.dequantize_mxfp4(blocks.to(device), scales.to(device), dt)
    _assert_bitexact(got, oracle.dequant_c(blocks, scales, dt), f"E{E} R{R} G{G} {name}")


@pytest.mark.parametrize("offset", [8, 1])
def test_unaligned_views(device, offset):
    """Staged tensors are views into one byte blob with 8-byte offsets."""
    E, R, G = 2, 64, 6
    blocks, scales = synthetic.packed_weights(E, R, G, seed=77, scale_lo=110, scale_hi=140)
    n = blocks.numel()
    blob = torch.zeros(n + 64, dtype=torch.uint8, device=device)
    blob[offset:offset + n] = blocks.reshape(-1).to(device)
    view = blob[offset:offset + n].view(E, R, G, 16)
    assert view.data_ptr() % 16 == offset % 16
    announce(f"dequant unaligned offset={offset}")
    got = kernels.dequantize_mxfp4(view, scales.to(device), torch.bfloat16)
    _assert_bitexact(got, oracle.dequant_c(blocks, scales, torch.bfloat16), f"offset {offset}")


def test_dequantize_expert_contract(device):
    """tests/test_offload.py:405-414 on the GPU: orientation [G*32, rows]."""
    g = torch.Generator().manual_seed(0)
    blocks = torch.randint(0, 255, (1, 64, 4, 16), generator=g, dtype=torch.uint8)
    scales = torch.randint(120, 134, (1, 64, 4), generator=g, dtype=torch.uint8)
    announce("dequantize_expert contract")
    out = gptoss.dequantize_expert(blocks.to(device), scales.to(device), torch.float32)
    assert out.shape == (128, 64)
    assert torch.equal(out.cpu(), oracle.dequantize_expert_ref(blocks, scales, torch.float32))


def test_gptoss_120b_layer_full_size(device):
    """One gpt-oss-120b layer of experts: all 128 experts, both projections.

    Sampled experts are compared bit for bit with the oracle; the whole
    output is compared with the integer decoder (mode 1), which the
    exhaustive table pins, so every element of the fast path is checked.
    """
    for name, rows, seed in (("gate_up", 5760, 2), ("down", 2880, 3)):
        blocks, scales = synthetic.packed_weights(128, rows, 90, seed=seed, scale_lo=115,
                                                  scale_hi=131, device=device)
        announce(f"dequant gpt-oss-120b {name} [128,{rows},90,16]")
        fast = kernels.dequantize_mxfp4(blocks, scales, torch.bfloat16)
        exact = kernels.dequantize_mxfp4(blocks, scales, torch.bfloat16, mode=1)
        assert torch.equal(fast.view(torch.int16), exact.view(torch.int16)), name
        del exact
        for e in (0, 77, 127):
            want = oracle.dequant_c(blocks[e:e + 1].cpu(), scales[e:e + 1].cpu(), torch.bfloat16)
            assert torch.equal(fast[e:e + 1].cpu().view(torch.int16), want.view(torch.int16)), (name, e)
        del fast, blocks, scales
        torch.cuda.empty_cache()
