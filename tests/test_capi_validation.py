"""Argument checking of every C-ABI entry point (CPU).

Each case breaks one rule that the entry point checks on the host before any
HIP call, so it returns BSA_EINVAL with a message naming the rule; empty
problems (T = 0 or R = 0) return BSA_OK without touching memory.  The
pointers passed are never dereferenced: every case fails (or returns) in the
host-side checks, which this file also asserts on a machine without a GPU,
where a call that got past them would fail with BSA_EHIP instead.
"""

from __future__ import annotations

import ctypes

import pytest

from blockstreamer_amd import _lib

FAKE = 1 << 20          # a 1 MiB-aligned address, never dereferenced
BF16, F16, F32 = 0, 1, 2
GPTOSS = dict(T=4, H=2880, I=2880, E=128, k=4)
_OUT = ctypes.c_int64(0)
OUT = ctypes.byref(_OUT)  # the size functions' output


def _ws_bytes(T, H, I, E, k, fn="bsa_moe_workspace_bytes"):
    n = ctypes.c_int64(0)
    assert getattr(_lib.lib(), fn)(T, H, I, E, k, ctypes.byref(n)) == _lib.BSA_OK
    return n.value


def _fwd_args(T=4, H=2880, I=2880, E=128, k=4, hidden=FAKE, wdt=BF16, bdt=BF16, odt=BF16, path=0,
              ptr=FAKE, ws=FAKE, ws_bytes=None, layout=0, scales=None):
    if ws_bytes is None:
        ws_bytes = _ws_bytes(max(T, 0), H, I, E, k) if min(H, I, E, k) > 0 and T >= 0 else 0
    sc = ptr if scales is None else scales
    return (hidden, T, H, I, E, k, ptr, ptr, wdt, ptr, sc, ptr, ptr, sc, ptr, bdt, 1.702, 7.0, ptr, odt,
            ws, ws_bytes, None, path, layout, None)


def _noalloc_args(T=4, H=2880, I=2880, E=128, k=4, hidden=FAKE, ptr=FAKE, path=0, save=None):
    """bsa_moe_experts_fwd_noalloc: the forward's arguments without the workspace pair."""
    a = _fwd_args(T=T, H=H, I=I, E=E, k=k, hidden=hidden, ptr=ptr, path=path, ws_bytes=0)
    return a[:20] + (save,) + a[23:]


def _bwd_args(T=4, H=2880, I=2880, E=128, k=4, gdt=BF16, blocks=FAKE, save=FAKE, bwd_ws=FAKE,
              bwd_bytes=None, ghdt=BF16, layout=0):
    ws_bytes = _ws_bytes(T, H, I, E, k) if min(H, I, E, k) > 0 and T >= 0 else 0
    if bwd_bytes is None:
        bwd_bytes = _ws_bytes(T, H, I, E, k, "bsa_moe_bwd_workspace_bytes") if ws_bytes else 0
    return (FAKE, gdt, T, H, I, E, k, FAKE, FAKE, BF16, blocks, FAKE, FAKE, FAKE, 1.702, 7.0, FAKE, ws_bytes,
            save, bwd_ws, bwd_bytes, FAKE, ghdt, FAKE, layout, None)


_ST = (ctypes.c_int64 * 3)(64 * 64 * 8, 64 * 64, 64)      # [B, T, H, 64] strides of a 64-head tensor
_ST_BAD = (ctypes.c_int64 * 3)(64 * 64 * 8, 64 * 64, 60)  # a head stride that is not a multiple of 8


def _attn_args(B=1, Tq=8, Tk=8, Hq=64, Hkv=8, D=64, causal=1, window=0, q=FAKE, st=_ST):
    return (q, st, FAKE, _ST, FAKE, _ST, None, B, Tq, Tk, Hq, Hkv, D, causal, window, 0.125, FAKE, _ST, None, None)


def _attn_bwd_args(B=1, Tq=8, Tk=8, Hq=64, Hkv=8, D=64, causal=1, window=0, gq=FAKE, stats=FAKE):
    return (FAKE, _ST, FAKE, _ST, FAKE, _ST, FAKE, _ST, FAKE, _ST, FAKE, B, Tq, Tk, Hq, Hkv, D, causal, window,
            0.125, gq, FAKE, FAKE, stats, None)


def _attn_split_args(B=1, Tq=1, Tk=4096, D=64, q=FAKE, ws=FAKE, ws_bytes=1 << 20):
    """A decode shape (one query over 4096 keys of 8 key heads): split over 32 workgroups per head."""
    return (q, _ST, FAKE, _ST, FAKE, _ST, None, B, Tq, Tk, 64, 8, D, 1, 0, 0.125, FAKE, _ST, None, ws, ws_bytes,
            None)


CASES = [
    ("attn head_dim", "bsa_attention_fwd", _attn_args(D=128), _lib.BSA_EINVAL, b"head_dim"),
    ("attn groups", "bsa_attention_fwd", _attn_args(Hkv=6), _lib.BSA_EINVAL, b"multiple of Hkv"),
    ("attn window without causal", "bsa_attention_fwd", _attn_args(causal=0, window=16), _lib.BSA_EINVAL,
     b"window needs the causal"),
    ("attn causal Tq > Tk", "bsa_attention_fwd", _attn_args(Tq=9, Tk=8), _lib.BSA_EINVAL, b"more queries"),
    ("attn null", "bsa_attention_fwd", _attn_args(q=None), _lib.BSA_EINVAL, b"null"),
    ("attn alignment", "bsa_attention_fwd", _attn_args(q=FAKE + 8), _lib.BSA_EINVAL, b"16-byte aligned"),
    ("attn strides", "bsa_attention_fwd", _attn_args(st=_ST_BAD), _lib.BSA_EINVAL, b"multiples of 8"),
    ("attn no keys", "bsa_attention_fwd", _attn_args(Tk=0, causal=0), _lib.BSA_EINVAL, b"without keys"),
    ("attn B = 0", "bsa_attention_fwd", _attn_args(B=0, q=None), _lib.BSA_OK, None),
    ("attn split no workspace", "bsa_attention_fwd_split", _attn_split_args(ws=None, ws_bytes=0), _lib.BSA_EINVAL,
     b"workspace"),
    ("attn split small workspace", "bsa_attention_fwd_split", _attn_split_args(ws_bytes=4096), _lib.BSA_EINVAL,
     b"workspace"),
    ("attn split misaligned workspace", "bsa_attention_fwd_split", _attn_split_args(ws=FAKE + 128),
     _lib.BSA_EINVAL, b"256-byte"),
    ("attn split head_dim", "bsa_attention_fwd_split", _attn_split_args(D=128), _lib.BSA_EINVAL, b"head_dim"),
    ("attn split B = 0", "bsa_attention_fwd_split", _attn_split_args(B=0, q=None, ws=None, ws_bytes=0),
     _lib.BSA_OK, None),
    ("attn bwd head_dim", "bsa_attention_bwd", _attn_bwd_args(D=32), _lib.BSA_EINVAL, b"head_dim"),
    ("attn bwd null", "bsa_attention_bwd", _attn_bwd_args(stats=None), _lib.BSA_EINVAL, b"null"),
    ("attn bwd alignment", "bsa_attention_bwd", _attn_bwd_args(gq=FAKE + 4), _lib.BSA_EINVAL, b"16-byte"),
    ("attn bwd Tq = 0", "bsa_attention_bwd", _attn_bwd_args(Tq=0), _lib.BSA_OK, None),
    # name, entry point, arguments, expected status, message fragment
    ("ws size null", "bsa_moe_workspace_bytes", (4, 64, 64, 8, 2, None), _lib.BSA_EINVAL, b"null"),
    ("ws size shape", "bsa_moe_workspace_bytes", (4, 0, 64, 8, 2, OUT), _lib.BSA_EINVAL, b"bad shape"),
    ("bwd ws size shape", "bsa_moe_bwd_workspace_bytes", (-1, 64, 64, 8, 2, OUT), _lib.BSA_EINVAL,
     b"bad shape"),
    ("fwd k = 0", "bsa_moe_experts_fwd", _fwd_args(k=0), _lib.BSA_EINVAL, b"bad shape"),
    ("fwd H % 32", "bsa_moe_experts_fwd", _fwd_args(H=48), _lib.BSA_EINVAL, b"multiples of 32"),
    ("fwd E > 1024", "bsa_moe_experts_fwd", _fwd_args(E=2000), _lib.BSA_EINVAL, b"1024 experts"),
    ("fwd k > 16", "bsa_moe_experts_fwd", _fwd_args(k=17), _lib.BSA_EINVAL, b"top-k"),
    ("fwd T = 0", "bsa_moe_experts_fwd", _fwd_args(T=0, ptr=None, hidden=None), _lib.BSA_OK, None),
    ("fwd dtype", "bsa_moe_experts_fwd", _fwd_args(odt=7), _lib.BSA_EINVAL, b"dtype"),
    ("fwd path", "bsa_moe_experts_fwd", _fwd_args(path=9), _lib.BSA_EINVAL, b"path"),
    ("fwd null", "bsa_moe_experts_fwd", _fwd_args(ptr=None), _lib.BSA_EINVAL, b"null"),
    ("fwd hidden alignment", "bsa_moe_experts_fwd", _fwd_args(hidden=FAKE + 2), _lib.BSA_EINVAL,
     b"16-byte aligned"),
    ("fwd workspace too small", "bsa_moe_experts_fwd", _fwd_args(ws_bytes=1024), _lib.BSA_EINVAL, b"workspace"),
    ("fwd workspace alignment", "bsa_moe_experts_fwd", _fwd_args(ws=FAKE + 16), _lib.BSA_EINVAL, b"aligned"),
    ("fwd unknown layout", "bsa_moe_experts_fwd", _fwd_args(layout=5), _lib.BSA_EINVAL, b"layout"),
    ("fwd k-pair odd groups", "bsa_moe_experts_fwd", _fwd_args(H=96, layout=1), _lib.BSA_EINVAL,
     b"even group count"),
    ("fwd k-pair blocks alignment", "bsa_moe_experts_fwd", _fwd_args(layout=1, ptr=FAKE + 8), _lib.BSA_EINVAL,
     b"16-byte aligned blocks"),
    ("no-alloc k = 0", "bsa_moe_experts_fwd_noalloc", _noalloc_args(k=0), _lib.BSA_EINVAL, b"bad shape"),
    ("no-alloc T = 0", "bsa_moe_experts_fwd_noalloc", _noalloc_args(T=0, ptr=None, hidden=None), _lib.BSA_OK,
     None),
    ("no-alloc null", "bsa_moe_experts_fwd_noalloc", _noalloc_args(ptr=None), _lib.BSA_EINVAL, b"null"),
    ("no-alloc path", "bsa_moe_experts_fwd_noalloc", _noalloc_args(path=9), _lib.BSA_EINVAL, b"path"),
    ("no-alloc beyond the scratch", "bsa_moe_experts_fwd_noalloc", _noalloc_args(T=1024), _lib.BSA_EINVAL,
     b"static scratch"),
    ("no-alloc save for backward", "bsa_moe_experts_fwd_noalloc", _noalloc_args(save=FAKE), _lib.BSA_EINVAL,
     b"save_swiglu_grad must be null"),
    ("gate_up unknown layout", "bsa_moe_gate_up",
     (FAKE, 4, 64, 64, 8, 2, FAKE, FAKE, None, BF16, 1.702, 7.0, FAKE, 1 << 20, None, 0, 3, None),
     _lib.BSA_EINVAL, b"layout"),
    ("down k-pair alignment", "bsa_moe_down",
     (4, 64, 64, 8, 2, FAKE + 8, FAKE, None, BF16, FAKE, 1 << 20, 0, 1, None), _lib.BSA_EINVAL,
     b"16-byte aligned"),
    ("bwd k-pair alignment", "bsa_moe_experts_bwd", _bwd_args(blocks=FAKE + 4, layout=1), _lib.BSA_EINVAL,
     b"16-byte aligned blocks"),
    ("bwd H % 64", "bsa_moe_experts_bwd", _bwd_args(H=96), _lib.BSA_EINVAL, b"hidden % 64"),
    ("bwd T = 0", "bsa_moe_experts_bwd", _bwd_args(T=0), _lib.BSA_OK, None),
    ("bwd dtype", "bsa_moe_experts_bwd", _bwd_args(ghdt=5), _lib.BSA_EINVAL, b"dtype"),
    ("bwd blocks alignment", "bsa_moe_experts_bwd", _bwd_args(blocks=FAKE + 2), _lib.BSA_EINVAL,
     b"4-byte aligned"),
    ("bwd save alignment", "bsa_moe_experts_bwd", _bwd_args(save=FAKE + 4), _lib.BSA_EINVAL, b"16-byte"),
    ("bwd workspace too small", "bsa_moe_experts_bwd", _bwd_args(bwd_bytes=256), _lib.BSA_EINVAL,
     b"backward workspace"),
    ("bwd workspace alignment", "bsa_moe_experts_bwd", _bwd_args(bwd_ws=FAKE + 64), _lib.BSA_EINVAL,
     b"256-byte"),
    ("router E > 256", "bsa_router_fwd", (FAKE, BF16, 4, 64, 300, 4, FAKE, None, FAKE, FAKE, FAKE, None),
     _lib.BSA_EINVAL, b"E <= 256"),
    ("router k > E", "bsa_router_fwd", (FAKE, BF16, 4, 64, 4, 8, FAKE, None, FAKE, FAKE, FAKE, None),
     _lib.BSA_EINVAL, b"k <= min(E"),
    ("router dtype", "bsa_router_fwd", (FAKE, 3, 4, 64, 8, 2, FAKE, None, FAKE, FAKE, FAKE, None),
     _lib.BSA_EINVAL, b"dtype"),
    ("router T = 0", "bsa_router_fwd", (None, BF16, 0, 64, 8, 2, None, None, None, None, None, None),
     _lib.BSA_OK, None),
    ("router null", "bsa_router_fwd", (FAKE, BF16, 4, 64, 8, 2, None, None, FAKE, FAKE, FAKE, None),
     _lib.BSA_EINVAL, b"null"),
    ("topk k > 16", "bsa_router_topk", (FAKE, F32, 4, 64, 17, FAKE, FAKE, None), _lib.BSA_EINVAL, b"k <= min"),
    ("topk T = 0", "bsa_router_topk", (None, F32, 0, 64, 4, None, None, None), _lib.BSA_OK, None),
    ("mxfp8 K % 32", "bsa_quant_mxfp8", (FAKE, BF16, 4, 48, FAKE, FAKE, 2, None), _lib.BSA_EINVAL, b"K % 32"),
    ("mxfp8 scale stride", "bsa_quant_mxfp8", (FAKE, BF16, 4, 128, FAKE, FAKE, 2, None), _lib.BSA_EINVAL,
     b"stride"),
    ("mxfp8 alignment", "bsa_quant_mxfp8", (FAKE + 8, BF16, 4, 128, FAKE, FAKE, 4, None), _lib.BSA_EINVAL,
     b"aligned"),
    ("mxfp8 R = 0", "bsa_quant_mxfp8", (None, BF16, 0, 128, None, None, 4, None), _lib.BSA_OK, None),
    ("split K % 64", "bsa_quant_mxfp8_split", (FAKE, BF16, 4, 96, FAKE, FAKE, 3, None), _lib.BSA_EINVAL,
     b"K % 64"),
    ("split alignment", "bsa_quant_mxfp8_split", (FAKE + 8, BF16, 4, 128, FAKE, FAKE, 4, None), _lib.BSA_EINVAL,
     b"aligned"),
    ("split R = 0", "bsa_quant_mxfp8_split", (None, BF16, 0, 128, None, None, 4, None), _lib.BSA_OK, None),
    ("matmul ws size K % 32", "bsa_mxfp4_matmul_workspace_bytes", (8, 48, 64, F32, 0, OUT), _lib.BSA_EINVAL,
     b"K % 32"),
    ("matmul ws size null", "bsa_mxfp4_matmul_workspace_bytes", (8, 128, 64, F32, 0, None), _lib.BSA_EINVAL,
     b"null"),
    ("matmul transpose N % 64", "bsa_mxfp4_matmul",
     (FAKE, F32, 8, 128, 96, FAKE, FAKE, 0, 1, FAKE, F32, FAKE, 1 << 20, None), _lib.BSA_EINVAL, b"N % 64"),
    ("matmul bad transpose", "bsa_mxfp4_matmul",
     (FAKE, F32, 8, 128, 64, FAKE, FAKE, 0, 2, FAKE, F32, FAKE, 1 << 20, None), _lib.BSA_EINVAL, b"transpose"),
    ("matmul dtype", "bsa_mxfp4_matmul",
     (FAKE, 7, 8, 128, 64, FAKE, FAKE, 0, 0, FAKE, F32, FAKE, 1 << 20, None), _lib.BSA_EINVAL, b"dtype"),
    ("matmul null", "bsa_mxfp4_matmul",
     (FAKE, F32, 8, 128, 64, None, FAKE, 0, 0, FAKE, F32, FAKE, 1 << 20, None), _lib.BSA_EINVAL, b"null"),
    ("matmul blocks alignment", "bsa_mxfp4_matmul",
     (FAKE, F32, 8, 128, 64, FAKE + 4, FAKE, 0, 0, FAKE, F32, FAKE, 1 << 20, None), _lib.BSA_EINVAL,
     b"8-byte"),
    ("matmul workspace too small", "bsa_mxfp4_matmul",
     (FAKE, F32, 8, 128, 64, FAKE, FAKE, 0, 0, FAKE, F32, FAKE, 256, None), _lib.BSA_EINVAL, b"workspace"),
    ("matmul M = 0", "bsa_mxfp4_matmul",
     (None, F32, 0, 128, 64, None, None, 0, 0, None, F32, None, 0, None), _lib.BSA_OK, None),
    ("dequant unknown layout", "bsa_dequant_mxfp4_layout", (FAKE, FAKE, FAKE, BF16, 1, 32, 4, 0, 2, None),
     _lib.BSA_EINVAL, b"layout"),
    ("dequant k-pair rows", "bsa_dequant_mxfp4_layout", (FAKE, FAKE, FAKE, BF16, 1, 24, 4, 0, 1, None),
     _lib.BSA_EINVAL, b"rows % 16"),
    ("dequant k-pair unaligned", "bsa_dequant_mxfp4_layout", (FAKE + 8, FAKE, FAKE, BF16, 1, 32, 4, 0, 1, None),
     _lib.BSA_EINVAL, b"16-byte aligned"),
    ("to k-pair odd groups", "bsa_mxfp4_to_kpair", (FAKE, FAKE * 2, 1, 32, 3, None), _lib.BSA_EINVAL,
     b"even group count"),
    ("to k-pair in place", "bsa_mxfp4_to_kpair", (FAKE, FAKE, 1, 32, 4, None), _lib.BSA_EINVAL, b"distinct"),
    ("from k-pair unaligned", "bsa_mxfp4_from_kpair", (FAKE + 4, FAKE * 2, 1, 32, 4, None), _lib.BSA_EINVAL,
     b"16-byte aligned"),
    ("to k-pair empty", "bsa_mxfp4_to_kpair", (None, None, 0, 32, 4, None), _lib.BSA_OK, None),
    ("norm H = 0", "bsa_rmsnorm_fwd", (FAKE, BF16, 4, 0, FAKE, F32, 1e-5, FAKE, None), _lib.BSA_EINVAL,
     b"bad shape"),
    ("norm dtype", "bsa_rmsnorm_fwd", (FAKE, 4, 4, 64, FAKE, F32, 1e-5, FAKE, None), _lib.BSA_EINVAL,
     b"dtype"),
    ("norm T = 0", "bsa_rmsnorm_fwd", (None, BF16, 0, 64, None, F32, 1e-5, None, None), _lib.BSA_OK, None),
    ("norm null", "bsa_rmsnorm_fwd", (FAKE, BF16, 4, 64, None, F32, 1e-5, FAKE, None), _lib.BSA_EINVAL,
     b"null"),
    ("norm bwd weight dtype", "bsa_rmsnorm_bwd", (FAKE, FAKE, BF16, 4, 64, FAKE, 9, 1e-5, FAKE, None),
     _lib.BSA_EINVAL, b"dtype"),
    ("norm bwd null", "bsa_rmsnorm_bwd", (None, FAKE, BF16, 4, 64, FAKE, F32, 1e-5, FAKE, None),
     _lib.BSA_EINVAL, b"null"),
]


@pytest.mark.parametrize("name,fn,args,rc,msg", CASES, ids=[c[0] for c in CASES])
def test_entry_point_rejects_before_any_gpu_call(name, fn, args, rc, msg):
    lib = _lib.lib()
    got = getattr(lib, fn)(*args)
    err = lib.bsa_last_error()
    assert got == rc, f"{name}: status {got}, message {err!r}"
    if msg is not None:
        assert msg in err, f"{name}: message {err!r} lacks {msg!r}"
    else:
        assert err in (b"", None), f"{name}: unexpected message {err!r}"


def test_workspace_sizes_grow_with_tokens():
    a = _ws_bytes(64, **{k: v for k, v in GPTOSS.items() if k != "T"})
    b = _ws_bytes(8192, **{k: v for k, v in GPTOSS.items() if k != "T"})
    assert 0 < a < b and a % 256 == 0 and b % 256 == 0
    c = _ws_bytes(64, **{k: v for k, v in GPTOSS.items() if k != "T"}, fn="bsa_moe_bwd_workspace_bytes")
    assert c > 0


def test_noalloc_scratch_covers_decode_batches():
    """The static scratch holds the 120b layer's workspace up to 226 tokens
    (the decode batches), not 227."""
    dims = {k: v for k, v in GPTOSS.items() if k != "T"}
    assert _ws_bytes(226, **dims) <= 16 << 20 < _ws_bytes(227, **dims)


def test_python_call_raises_value_error_with_the_message():
    with pytest.raises(ValueError, match="top-k"):
        _lib.call("bsa_moe_experts_fwd", *_fwd_args(k=17))


def test_attention_split_workspace_follows_the_shape():
    """Decode grids split (32 shares of 4096 keys x 64 heads x 66 floats, two 256-byte aligned parts);
    prefill grids and short key ranges do not (no workspace)."""
    f = _lib.lib().bsa_attention_split_workspace_bytes
    assert f(1, 1, 4096, 64, 8, 1, 0) == 32 * 64 * 64 * 4 + 32 * 64 * 2 * 4
    assert f(64, 1, 4096, 64, 8, 1, 0) == 0          # 512 workgroups already
    assert f(1, 8192, 8192, 64, 8, 1, 0) == 0        # prefill
    assert f(1, 1, 100, 64, 8, 1, 0) == 0            # two key tiles: nothing to split
    # a window bounds the keys a row block sees: 128 + 1 keys -> 4 tiles, too few to split; 1000 -> 17 tiles
    assert f(1, 1, 4096, 64, 8, 1, 128) == 0
    assert f(1, 1, 4096, 64, 8, 1, 1000) == 8 * 64 * 64 * 4 + 8 * 64 * 2 * 4
    assert f(1, 1, 448, 64, 8, 1, 0) == 0             # 7 key tiles: too few
    assert f(1, 1, 449, 64, 8, 1, 0) == 4 * 64 * 64 * 4 + 4 * 64 * 2 * 4  # 8 tiles: 4 shares
    assert f(2, 4, 1000, 64, 8, 1, 0) > 0
