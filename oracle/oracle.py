"""CPU restatement of BlockStreamer's gpt-oss MoE expert path (the oracle).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, never by the product package.

Every function cites the reference line it restates.  The reference is
hareramray/BlockStreamer ``block_streamer/gptoss.py``; its arithmetic lives in
the third-party ``transformers`` package (installed version 5.15.0, the
version this restatement follows), cited below as ``TF/<path>:<line>``.

Pinning (how each function is checked, see ``tests/test_oracle.py``):

* dequant (C and torch restatements): the closed form of OCP MX E2M1 x E8M0
  over the exhaustive 16-code x 256-scale table, agreement between the two
  independent restatements, and the installed transformers
  ``convert_moe_packed_tensors`` on random inputs and on every (byte, scale)
  pair.  NaN payloads for scale byte 255 are platform dependent (0 * inf), so
  NaN is compared as NaN, not by bit pattern.
* router: brute force over all k-subsets on tiny tie-free inputs, and the
  installed transformers ``GptOssTopKRouter``.
* MXFP8 quantisation (the native MX path only): against torch's
  float8_e4m3fn cast for in-range values (a library routine, RNE), closed
  forms at the format's boundaries (max 448, min normal 2^-6, min subnormal
  2^-9, ties), and exact round trips of representable inputs.
* RMSNorm (the post-attention norm in front of the path): the installed
  transformers ``GptOssRMSNorm`` in float64, forward and its autograd
  backward (against the closed-form gradient), plus scale invariance and the
  eps-dominated regime.
* k-pair layout (this build's shard format, no reference counterpart): its
  defining index map checked element by element on small inputs.
* experts: the installed transformers dense twin ``GptOssExperts``
  (TF/models/gpt_oss/modeling_gpt_oss.py:68-114) fed the dequantised
  weights, plus invariants (zero routing weight contributes nothing, token
  permutation commutes, a single expert with k=1 and weight 1 equals the dense
  chain of library GEMMs).
* attention with sinks (the other half of the decoder layer): the installed
  transformers ``eager_attention_forward`` in float64 with the masks its
  ``masking_utils.eager_mask`` builds (none, causal, sliding window, queries
  offset into a longer key sequence), plus closed forms: a sink of -inf gives
  the library's ``scaled_dot_product_attention``, one visible key gives
  ``sigmoid(s - sink) * v``, and grouped heads equal their repeated keys.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle_mxfp4.so"
_lib = None

# TF/integrations/mxfp4.py:29-46 -- E2M1 code -> value, bit 3 is the sign.
FP4_VALUES = [
    +0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0,
    -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0,
]

_DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        subprocess.run(["make", "-C", str(_HERE)], check=True,
                       stdout=subprocess.DEVNULL)
    lib = ctypes.CDLL(str(_LIB_PATH))
    lib.oracle_dequant_mxfp4.argtypes = [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_int64, ctypes.c_int, ctypes.c_void_p,
    ]
    lib.oracle_dequant_mxfp4.restype = None
    lib.oracle_dequant_one.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.oracle_dequant_one.restype = ctypes.c_uint32
    lib.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
    lib.oracle_f32_to_bf16.restype = ctypes.c_uint16
    lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
    lib.oracle_f32_to_f16.restype = ctypes.c_uint16
    _lib = lib
    return lib


def dequant_c(blocks: torch.Tensor, scales: torch.Tensor,
              dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """C restatement of TF/integrations/mxfp4.py:257-313 for [E,R,G,16] input.

    Returns the dense ``[E, G*32, R]`` tensor in ``dtype`` (bf16/f16/f32).
    """
    lib = _load()
    blocks = blocks.detach().to("cpu", torch.uint8).contiguous()
    scales = scales.detach().to("cpu", torch.uint8).contiguous()
    if blocks.dim() != 4 or blocks.shape[-1] != 16 or tuple(scales.shape) != tuple(blocks.shape[:-1]):
        raise ValueError(f"bad packed shapes {tuple(blocks.shape)} / {tuple(scales.shape)}")
    E, R, G, _ = blocks.shape
    out = torch.empty((E, G * 32, R), dtype=dtype)
    lib.oracle_dequant_mxfp4(blocks.data_ptr(), scales.data_ptr(), E, R, G,
                             _DTYPE_CODE[dtype], out.data_ptr())
    return out


def dequant_table_c(dtype: torch.dtype = torch.bfloat16) -> np.ndarray:
    """Exhaustive [256 scale, 16 code] table of output bit patterns."""
    lib = _load()
    code = _DTYPE_CODE[dtype]
    tab = np.empty((256, 16), dtype=np.uint32)
    for s in range(256):
        for c in range(16):
            tab[s, c] = lib.oracle_dequant_one(c, s, code)
    return tab


def dequant_torch(blocks: torch.Tensor, scales: torch.Tensor,
                  dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """torch restatement of TF/integrations/mxfp4.py:257-313, op for op.

    LUT gather on the low and high nibbles into even and odd columns
    (mxfp4.py:294-304), ``ldexp`` by ``scale - 127`` (mxfp4.py:271, 307),
    reshape to ``[..., R, G*32]`` and ``transpose(1, 2)`` (mxfp4.py:311-313).
    """
    blocks = blocks.to(torch.uint8)
    exp = scales.to(torch.int32) - 127
    lut = torch.tensor(FP4_VALUES, dtype=dtype, device=blocks.device)
    *prefix, G, B = blocks.shape
    rows = int(np.prod(prefix)) * G
    blk = blocks.reshape(rows, B)
    exp = exp.reshape(rows, 1)
    out = torch.empty(rows, B * 2, dtype=dtype, device=blocks.device)
    out[:, 0::2] = lut[(blk & 0x0F).to(torch.int)]
    out[:, 1::2] = lut[(blk >> 4).to(torch.int)]
    torch.ldexp(out, exp, out=out)
    out = out.reshape(*prefix, G, B * 2).view(*prefix, G * B * 2)
    return out.transpose(1, 2).contiguous()


def dequantize_expert_ref(blocks: torch.Tensor, scales: torch.Tensor,
                          dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """block_streamer/gptoss.py:24-42: [1,R,G,16] -> [G*32, R]."""
    if blocks.dim() != 4:
        raise ValueError(
            f"Expected [1, rows, groups, 16] packed blocks, got {tuple(blocks.shape)}"
        )
    return dequant_torch(blocks, scales, dtype).squeeze(0)


def topk_softmax_ref(logits: torch.Tensor, k: int):
    """TF/models/gpt_oss/modeling_gpt_oss.py:128-129 on given logits.

    ``topk`` sorted descending; equal logits are ordered lower index first (a
    stable sort), which is the rule the HIP kernel implements.  Softmax over
    the k selected values in their own dtype (``softmax(dtype=vals.dtype)``
    computes in float32 internally for half types and rounds once).
    """
    order = torch.sort(logits.float(), dim=-1, descending=True, stable=True).indices
    idx = order[..., :k].contiguous()
    vals = torch.gather(logits, -1, idx)
    scores = torch.softmax(vals.float(), dim=-1).to(logits.dtype)
    return vals, scores, idx


def router_ref(h: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, k: int,
               dtype: torch.dtype = torch.float32):
    """TF/models/gpt_oss/modeling_gpt_oss.py:126-131 (GptOssTopKRouter.forward).

    Computed in ``dtype`` (float32 for the parity reference).  Returns
    ``(logits [T,E], scores [T,k], indices [T,k] int64)``.
    """
    logits = F.linear(h.to(dtype), weight.to(dtype), bias.to(dtype))
    _, scores, idx = topk_softmax_ref(logits, k)
    return logits, scores, idx


def rmsnorm_ref(x: torch.Tensor, weight: torch.Tensor, eps: float,
                dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """TF/models/gpt_oss/modeling_gpt_oss.py:57-62 (GptOssRMSNorm.forward)
    over the last dimension, computed in ``dtype`` and not rounded back to the
    input dtype (float64 for the parity reference)."""
    x = x.to(dtype)
    r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return weight.to(dtype) * (x * r)


def rmsnorm_bwd_ref(grad: torch.Tensor, x: torch.Tensor, weight: torch.Tensor, eps: float,
                    dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """Input gradient of ``rmsnorm_ref`` in closed form: with g = weight * grad
    and r = rsqrt(mean(x^2) + eps), dx = r g - x r^3 sum(g x) / H (the
    derivative of modeling_gpt_oss.py:60-62 with respect to hidden_states)."""
    x = x.to(dtype)
    g = weight.to(dtype) * grad.to(dtype)
    H = x.shape[-1]
    r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return r * g - x * (r ** 3 * (g * x).sum(-1, keepdim=True) / H)


def attention_ref(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, sinks: torch.Tensor | None,
                  scaling: float, causal: bool = False, window: int = 0,
                  dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """TF/models/gpt_oss/modeling_gpt_oss.py:235-264 (eager_attention_forward,
    with repeat_kv :203-212) in ``dtype``, not rounded back.

    q ``[B, Hq, Tq, D]``, k and v ``[B, Hkv, Tk, D]`` (the layout
    GptOssAttention.forward :311-320 hands over), sinks ``[Hq]`` or None.
    Key j is visible to query t (absolute position p = Tk - Tq + t) always
    when ``causal`` is False (the eager path with attention_mask=None), else
    when j <= p and, with ``window`` > 0, p - j < window (masking_utils
    causal_mask_function and sliding_window_overlay).  Returns
    ``[B, Tq, Hq, D]`` (:262, attn_output.transpose(1, 2))."""
    B, Hq, Tq, D = q.shape
    Hkv, Tk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    k = k[:, :, None].expand(B, Hkv, G, Tk, D).reshape(B, Hq, Tk, D)
    v = v[:, :, None].expand(B, Hkv, G, Tk, D).reshape(B, Hq, Tk, D)
    s = torch.matmul(q, k.transpose(2, 3)) * scaling
    if causal:
        pos = torch.arange(Tq, device=q.device)[:, None] + (Tk - Tq)
        j = torch.arange(Tk, device=q.device)[None, :]
        vis = j <= pos
        if window > 0:
            vis = vis & (j > pos - window)
        s = s.masked_fill(~vis, float("-inf"))
    if sinks is not None:
        s = torch.cat([s, sinks.to(dtype).reshape(1, Hq, 1, 1).expand(B, Hq, Tq, 1)], dim=-1)
    s = s - s.max(dim=-1, keepdim=True).values
    p = torch.softmax(s, dim=-1)[..., :Tk]
    return torch.matmul(p, v).transpose(1, 2)


def to_kpair_ref(blocks: torch.Tensor) -> torch.Tensor:
    """The k-pair shard layout of checkpoint blocks ``[E, R, G, 16]``: group g
    of row r at ``[e][r // 16][g // 2][r % 16][g % 2]`` (no reference
    counterpart; the definition the HIP repacking and every kernel reading
    that layout are checked against)."""
    E, R, G, _ = blocks.shape
    return blocks.reshape(E, R // 16, 16, G // 2, 2, 16).permute(0, 1, 3, 2, 4, 5).contiguous()


def apply_gate_ref(gate_up: torch.Tensor, alpha: float = 1.702,
                   limit: float = 7.0) -> torch.Tensor:
    """block_streamer/gptoss.py:130-135: interleaved clamped SwiGLU."""
    gate, up = gate_up[..., ::2], gate_up[..., 1::2]
    gate = gate.clamp(max=limit)
    up = up.clamp(min=-limit, max=limit)
    glu = gate * torch.sigmoid(gate * alpha)
    return (up + 1) * glu


def experts_ref(h: torch.Tensor, router_indices: torch.Tensor,
                routing_weights: torch.Tensor,
                gate_up_blocks: torch.Tensor, gate_up_scales: torch.Tensor,
                gate_up_bias: torch.Tensor, down_blocks: torch.Tensor,
                down_scales: torch.Tensor, down_bias: torch.Tensor,
                alpha: float = 1.702, limit: float = 7.0,
                dtype: torch.dtype = torch.float32,
                dense_cache: dict | None = None) -> torch.Tensor:
    """block_streamer/gptoss.py:137-177 (MXFP4Experts.forward), op for op.

    Runs on the CPU in ``dtype`` (float32 for the parity reference).  ``h``
    and ``routing_weights`` may require grad; the result is then
    differentiable by torch autograd, which is the reference for the
    input-gradient backward (gptoss.py:64-71 plus autograd of 130-176).
    ``dense_cache`` (optional dict) memoises per-expert dense weights.
    """
    h = h.to(dtype)
    routing_weights = routing_weights.to(dtype)
    E = gate_up_blocks.shape[0]
    next_states = torch.zeros_like(h)                                   # :143
    with torch.no_grad():
        mask = F.one_hot(router_indices.to(torch.int64), num_classes=E).permute(2, 1, 0)  # :145-147
        hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero()       # :148
    for entry in hit:                                                  # :149
        expert = int(entry[0])
        top_k_pos, token_idx = torch.where(mask[expert])               # :153
        current = h[token_idx]                                         # :154
        key = ("gu", expert)
        if dense_cache is not None and key in dense_cache:
            w_gu = dense_cache[key]
        else:
            w_gu = dequant_torch(gate_up_blocks[expert:expert + 1],
                                 gate_up_scales[expert:expert + 1], dtype).squeeze(0)
            if dense_cache is not None:
                dense_cache[key] = w_gu
        gate_up = current @ w_gu + gate_up_bias[expert].to(dtype)       # :158-165
        gated = apply_gate_ref(gate_up, alpha, limit)                  # :166
        key = ("dn", expert)
        if dense_cache is not None and key in dense_cache:
            w_dn = dense_cache[key]
        else:
            w_dn = dequant_torch(down_blocks[expert:expert + 1],
                                 down_scales[expert:expert + 1], dtype).squeeze(0)
            if dense_cache is not None:
                dense_cache[key] = w_dn
        out = gated @ w_dn + down_bias[expert].to(dtype)               # :167-174
        out = out * routing_weights[token_idx, top_k_pos, None]        # :175
        next_states = next_states.index_add(0, token_idx, out.to(h.dtype))  # :176
    return next_states


def mlp_ref(h: torch.Tensor, router_weight: torch.Tensor, router_bias: torch.Tensor,
            k: int, *expert_params, alpha: float = 1.702, limit: float = 7.0,
            dtype: torch.dtype = torch.float32):
    """TF/models/gpt_oss/modeling_gpt_oss.py:140-146 (GptOssMLP.forward).

    ``h`` is ``[B, S, H]``; returns ``(out [B,S,H], scores [T,k])``.
    """
    B, S, H = h.shape
    flat = h.reshape(-1, H)
    _, scores, idx = router_ref(flat, router_weight, router_bias, k, dtype)
    out = experts_ref(flat, idx, scores, *expert_params, alpha=alpha, limit=limit,
                      dtype=dtype)
    return out.reshape(B, S, H), scores


# ----------------------------------------------------------------------------- MXFP8
# The native block-scaled MFMA path quantises activations to OCP MXFP8.  The
# reference has no such step (it multiplies unquantised activations,
# block_streamer/gptoss.py:45-75); this restates the published OCP
# Microscaling Formats v1.0 conversion (section 6.3: shared exponent from
# floor(log2(amax)) - emax_elem, emax_elem = 8 for E4M3), with the exponent
# taken one higher where the block maximum would otherwise exceed 448 (so
# X = ceil(log2(amax / 448)) and nothing saturates), and round-to-nearest-
# even elements; in float64 with frexp -- a different method from the
# kernel's bit arithmetic.

E4M3_MAX = 448.0


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """OCP E4M3 (bias 7, no infinities, 0x7F/0xFF = NaN) -> float64."""
    c = np.asarray(codes).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 15
    m = c & 7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    mag = np.where((c & 0x7F) == 0x7F, np.nan, mag)
    return sign * mag


def _mx_shared_exp(blk: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Blocks ``[..., 32]`` (float64) -> (X int64 [...], bad bool [...])."""
    amax = np.abs(blk).max(-1)
    bad = ~np.isfinite(blk).all(-1)
    f, e = np.frexp(np.where(np.isfinite(amax), amax, 1.0))   # amax = f * 2^e, f in [0.5, 1)
    X = np.clip(e - 1 - 8 + (2 * f > 1.75), -127, 127)
    X = np.where(amax == 0, -127, X)
    return X.astype(np.int64), bad


def _e4m3_codes(y: np.ndarray) -> np.ndarray:
    """E4M3 codes (int64) of float64 values, round to nearest even,
    saturating at 448; the sign bit follows the sign of y (-0 included)."""
    mag = np.minimum(np.abs(y), E4M3_MAX)
    _, ee = np.frexp(mag)
    ee = np.maximum(ee - 1, -6)                       # subnormals: fixed step 2^-9
    step = np.exp2(ee - 3.0)
    q = np.minimum(np.rint(mag / step) * step, E4M3_MAX)
    _, e2 = np.frexp(q)
    e2 = e2 - 1
    normal = q >= 2.0 ** -6
    mant = np.where(normal, q / np.exp2(e2.astype(np.float64)) * 8 - 8, q / 2.0 ** -9)
    with np.errstate(invalid="ignore"):   # NaN inputs: their blocks are overwritten by the callers
        m = np.rint(mant).astype(np.int64)
    code = np.where(normal, ((e2 + 7) << 3) + m, m)
    return code | (np.signbit(y).astype(np.int64) << 7)


def mxfp8_quant_ref(x: torch.Tensor) -> tuple[np.ndarray, np.ndarray]:
    """[R, K] floats -> (E4M3 codes uint8 [R, K], E8M0 scale bytes uint8 [R, K/32])."""
    a = x.detach().double().cpu().numpy()
    R, K = a.shape
    blk = a.reshape(R, K // 32, 32)
    X, bad = _mx_shared_exp(blk)
    scales = np.where(bad, 255, X + 127).astype(np.uint8)
    y = blk / np.exp2(X.astype(np.float64))[..., None]
    code = _e4m3_codes(y)
    code = np.where(bad[..., None], (np.signbit(blk).astype(np.int64) << 7) | 0x7F, code)
    return code.reshape(R, K).astype(np.uint8), scales


def mxfp8_split_ref(x: torch.Tensor) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Two-term MXFP8 split of [R, K] floats (the MX GEMM path's activations):
    (hi codes uint8 [R, K], lo codes uint8 [R, K], scale bytes uint8 [R, K/32]).

    hi and the scales are ``mxfp8_quant_ref``'s; lo = E4M3 of the residual
    x - hi * 2^X over 2^Xl, Xl = max(X - 4, -127), rounded to nearest even.
    The residual is formed in float64, where it is exact (as it is in the
    kernel's float32: x minus x rounded to 4 significant bits).  Blocks with
    inf or NaN: hi = 0x7F with the sign, lo = 0, scale 255."""
    hi, scales = mxfp8_quant_ref(x)
    a = x.detach().double().cpu().numpy()
    R, K = a.shape
    blk = a.reshape(R, K // 32, 32)
    X, bad = _mx_shared_exp(blk)
    hv = e4m3_decode(hi.reshape(R, K // 32, 32)) * np.exp2(X.astype(np.float64))[..., None]
    res = np.where(bad[..., None], 0.0, blk - np.where(bad[..., None], 0.0, hv))
    Xl = np.maximum(X - 4, -127)
    lo = _e4m3_codes(res / np.exp2(Xl.astype(np.float64))[..., None])
    lo = np.where(bad[..., None], 0, lo)
    return hi, lo.reshape(R, K).astype(np.uint8), scales


def mxfp8_split_dequant_ref(hi: np.ndarray, lo: np.ndarray, scales: np.ndarray) -> torch.Tensor:
    """hi * 2^X + lo * 2^max(X - 4, -127) per 32-element block -> float32."""
    v_hi, v_lo = e4m3_decode(hi), e4m3_decode(lo)
    R, K = v_hi.shape
    X = np.asarray(scales).astype(np.float64) - 127.0
    out = (v_hi.reshape(R, K // 32, 32) * np.exp2(X)[..., None]
           + v_lo.reshape(R, K // 32, 32) * np.exp2(np.maximum(X - 4, -127))[..., None])
    return torch.from_numpy(out.reshape(R, K).astype(np.float32))


def mxfp8_dequant_ref(codes: np.ndarray, scales: np.ndarray) -> torch.Tensor:
    """E4M3 codes [R, K] x 2^(scale - 127) per 32 -> float32 tensor."""
    v = e4m3_decode(codes)
    R, K = v.shape
    s = np.exp2(np.asarray(scales).astype(np.float64) - 127.0)
    out = v.reshape(R, K // 32, 32) * s[..., None]
    return torch.from_numpy(out.reshape(R, K).astype(np.float32))


def experts_mx_ref(h: torch.Tensor, router_indices: torch.Tensor, routing_weights: torch.Tensor,
                   gate_up_blocks, gate_up_scales, gate_up_bias, down_blocks, down_scales,
                   down_bias, alpha: float = 1.702, limit: float = 7.0) -> torch.Tensor:
    """The MX path's arithmetic: ``experts_ref`` with both GEMMs' activations
    replaced by their two-term MXFP8 split (hidden per token; the gated
    activations after their rounding to bfloat16), float64 GEMMs."""
    E = gate_up_blocks.shape[0]
    hq = mxfp8_split_dequant_ref(*mxfp8_split_ref(h.float()))
    out = torch.zeros(h.shape, dtype=torch.float32)
    mask = F.one_hot(router_indices.to(torch.int64), num_classes=E).permute(2, 1, 0)
    for e in range(E):
        top_k_pos, token_idx = torch.where(mask[e])
        if token_idx.numel() == 0:
            continue
        w_gu = dequant_torch(gate_up_blocks[e:e + 1], gate_up_scales[e:e + 1], torch.float32)[0]
        w_dn = dequant_torch(down_blocks[e:e + 1], down_scales[e:e + 1], torch.float32)[0]
        gu = hq[token_idx].double() @ w_gu.double() + gate_up_bias[e].double()
        act = apply_gate_ref(gu.float(), alpha, limit).to(torch.bfloat16)
        aq = mxfp8_split_dequant_ref(*mxfp8_split_ref(act))
        o = (aq.double() @ w_dn.double() + down_bias[e].double()).float()
        o = o * routing_weights[token_idx, top_k_pos, None].float()
        out = out.index_add(0, token_idx, o)
    return out


# OCP MX E2M3 (FP6): sign bit 5, two exponent bits (bias 1), three mantissa
# bits, no infinities or NaN; largest magnitude 7.5, subnormal step 1/8.
E2M3_MAX = 7.5


def e2m3_decode(codes: np.ndarray) -> np.ndarray:
    """OCP E2M3 codes (6 bits; sign = bit 5) -> float64."""
    c = np.asarray(codes).astype(np.int64)
    sign = np.where(c & 0x20, -1.0, 1.0)
    e = (c >> 3) & 3
    m = c & 7
    mag = np.where(e == 0, m / 8.0, (1.0 + m / 8.0) * np.exp2(e - 1.0))
    return sign * mag


def _e2m3_codes(y: np.ndarray) -> np.ndarray:
    """E2M3 codes (int64) of float64 values, round to nearest even,
    saturating at 7.5; the sign bit follows the sign of y (-0 included).
    The grid steps are 1/8 below 2 (subnormals and the first binade alike),
    1/4 in [2, 4) and 1/2 in [4, 7.5], and a code is its value's position
    on that grid, so ties to even codes are ties to even mantissas."""
    mag = np.minimum(np.abs(y), E2M3_MAX)
    code = np.where(mag < 2.0, np.rint(mag * 8.0),
                    np.where(mag < 4.0, 16.0 + np.rint((mag - 2.0) * 4.0), 24.0 + np.rint((mag - 4.0) * 2.0)))
    code = np.minimum(code, 31.0).astype(np.int64)
    return code | (np.signbit(y).astype(np.int64) << 5)


def _mx6_shared_exp(blk: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Blocks ``[..., 32]`` (float64) -> (X int64 [...], bad bool [...]).

    X = ceil(log2(amax / 7.5)): floor(log2(amax)) - 2, plus 1 when amax's
    significand exceeds 1.875 (7.5 = 1.875 * 2^2), so that no element of
    the block saturates; clamped to [-127, 127]; -127 for an all-zero block."""
    amax = np.abs(blk).max(-1)
    bad = ~np.isfinite(blk).all(-1)
    f, e = np.frexp(np.where(np.isfinite(amax), amax, 1.0))   # amax = f * 2^e, f in [0.5, 1)
    X = np.clip(e - 1 - 2 + (2 * f > 1.875), -127, 127)
    X = np.where(amax == 0, -127, X)
    return X.astype(np.int64), bad


def mxfp6_split_ref(x: torch.Tensor, terms: int = 2) -> tuple[np.ndarray, np.ndarray]:
    """Multi-term MXFP6 (E2M3) split of ``[R, K]`` floats: ``(codes uint8
    [terms, R, K], scale bytes uint8 [R, K/32])``.

    No reference counterpart: the activation format of this build's FP6 MX
    path.  Per 32-element block with shared exponent X (``_mx6_shared_exp``),
    term t holds E2M3((x - sum of the earlier terms) / 2^Xt), Xt =
    max(X - 4t, -127), rounded to nearest even; the residuals are exact in
    float64.  The scale byte is that of X (term t's is max(byte - 4t, 0)).
    Blocks holding inf or NaN: scale byte 255 (the E8M0 NaN), every code 0."""
    a = x.detach().double().cpu().numpy()
    R, K = a.shape
    blk = a.reshape(R, K // 32, 32)
    X, bad = _mx6_shared_exp(blk)
    res = np.where(bad[..., None], 0.0, blk)
    codes = []
    for t in range(terms):
        sc = np.exp2(np.maximum(X - 4 * t, -127).astype(np.float64))[..., None]
        c = _e2m3_codes(res / sc)
        res = res - e2m3_decode(c) * sc
        codes.append(np.where(bad[..., None], 0, c).reshape(R, K))
    scales = np.where(bad, 255, X + 127).astype(np.uint8)
    return np.stack(codes).astype(np.uint8), scales


def mxfp6_split_dequant_ref(codes: np.ndarray, scales: np.ndarray) -> torch.Tensor:
    """sum over terms t of E2M3(codes[t]) * 2^max(X - 4t, -127) per 32-element
    block (X = scale byte - 127) -> float32; NaN for blocks of scale 255."""
    terms, R, K = codes.shape
    s = np.asarray(scales).astype(np.int64)
    X = s - 127
    out = np.zeros((R, K // 32, 32))
    for t in range(terms):
        out += e2m3_decode(codes[t]).reshape(R, K // 32, 32) * np.exp2(np.maximum(X - 4 * t, -127))[..., None]
    out = np.where((s == 255)[..., None], np.nan, out)
    return torch.from_numpy(out.reshape(R, K).astype(np.float32))


def experts_mx6_ref(h: torch.Tensor, router_indices: torch.Tensor, routing_weights: torch.Tensor,
                    gate_up_blocks, gate_up_scales, gate_up_bias, down_blocks, down_scales,
                    down_bias, alpha: float = 1.702, limit: float = 7.0, terms: int = 2) -> torch.Tensor:
    """The FP6 MX path's arithmetic: ``experts_ref`` with both GEMMs'
    activations replaced by their ``terms``-term MXFP6 split (hidden per
    token; the gated activations after their rounding to bfloat16), float64
    GEMMs."""
    E = gate_up_blocks.shape[0]
    hq = mxfp6_split_dequant_ref(*mxfp6_split_ref(h.float(), terms))
    out = torch.zeros(h.shape, dtype=torch.float32)
    mask = F.one_hot(router_indices.to(torch.int64), num_classes=E).permute(2, 1, 0)
    for e in range(E):
        top_k_pos, token_idx = torch.where(mask[e])
        if token_idx.numel() == 0:
            continue
        w_gu = dequant_torch(gate_up_blocks[e:e + 1], gate_up_scales[e:e + 1], torch.float32)[0]
        w_dn = dequant_torch(down_blocks[e:e + 1], down_scales[e:e + 1], torch.float32)[0]
        gu = hq[token_idx].double() @ w_gu.double() + gate_up_bias[e].double()
        act = apply_gate_ref(gu.float(), alpha, limit).to(torch.bfloat16)
        aq = mxfp6_split_dequant_ref(*mxfp6_split_ref(act, terms))
        o = (aq.double() @ w_dn.double() + down_bias[e].double()).float()
        o = o * routing_weights[token_idx, top_k_pos, None].float()
        out = out.index_add(0, token_idx, o)
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even, NaN -> 0x7FC0."""
    lib = _load()
    flat = np.asarray(x, dtype=np.float32).ravel()
    return np.array([lib.oracle_f32_to_bf16(float(v)) for v in flat],
                    dtype=np.uint16).reshape(np.shape(x))


def bits_equal_or_both_nan(a_bits: np.ndarray, b_bits: np.ndarray,
                           dtype: torch.dtype) -> np.ndarray:
    """Element-wise: identical bit patterns, or both NaN in ``dtype``."""
    a_bits = np.asarray(a_bits).astype(np.uint32)
    b_bits = np.asarray(b_bits).astype(np.uint32)
    if dtype == torch.float32:
        exp_mask, man_mask = 0x7F800000, 0x007FFFFF
    elif dtype == torch.bfloat16:
        exp_mask, man_mask = 0x7F80, 0x007F
    else:
        exp_mask, man_mask = 0x7C00, 0x03FF

    def isnan(v):
        return ((v & exp_mask) == exp_mask) & ((v & man_mask) != 0)

    return (a_bits == b_bits) | (isnan(a_bits) & isnan(b_bits))

