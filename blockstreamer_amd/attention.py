"""Attention core of the gpt-oss decoder layer on the HIP kernels.

The drop-in point is transformers' attention-function interface: GptOssAttention
(TF/models/gpt_oss/modeling_gpt_oss.py:295-336) calls
``ALL_ATTENTION_FUNCTIONS[config._attn_implementation]`` with the projected,
rotated query/key/value; gpt-oss declares no SDPA support, so the default is
``eager_attention_forward`` (:235-264).  ``gpt_oss_attention`` takes its place
with the same signature and the same meaning of ``attention_mask``:

* ``None``: every key visible (the eager path adds no mask; the streaming
  runner calls its decoder layers this way, block_streamer/runners.py:327-335);
* a 4-D mask from ``masking_utils`` (``[B, 1, Tq, Tk]``, 0 or the dtype's
  minimum, or boolean): it must be the causal mask or the sliding-window
  causal mask of ``module.sliding_window`` over the last Tq of Tk positions
  (what ``create_causal_mask`` / ``create_sliding_window_causal_mask`` build
  without padding); any other mask raises.

``register()`` adds it under the name ``"blockstreamer_amd"`` (with eager-style
masks), so ``model.config._attn_implementation = "blockstreamer_amd"`` switches
a model over.  There is no fallback: without the HIP library or a ROCm device
the calls raise.
"""

from __future__ import annotations

import ctypes
import functools
import weakref

import torch
from torch import Tensor

from . import _lib

HEAD_DIM = 64
NAME = "blockstreamer_amd"


def _strides(t: Tensor, seq_dim: int, head_dim_idx: int) -> "ctypes.Array":
    """Element strides (batch, sequence, head) of a 4-D tensor."""
    return (ctypes.c_int64 * 3)(t.stride(0), t.stride(seq_dim), t.stride(head_dim_idx))


def _usable(t: Tensor) -> bool:
    return (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
            and all(s % 8 == 0 and s >= 0 for s in t.stride()[:-1]))


@functools.lru_cache(maxsize=256)
def _split_bytes(B: int, Tq: int, Tk: int, Hq: int, Hkv: int, causal: int, window: int) -> int:
    """Workspace of the key-split forward for a shape (0: not split), a function of the shape."""
    return int(_lib.lib().bsa_attention_split_workspace_bytes(B, Tq, Tk, Hq, Hkv, causal, window))


def attention_forward(query: Tensor, key: Tensor, value: Tensor, sinks: Tensor | None, scaling: float,
                      causal: bool = False, window: int = 0, return_lse: bool = False):
    """``softmax([q k^T * scaling | sink]) v`` per head, the sink column dropped.

    query ``[B, Hq, Tq, 64]``, key/value ``[B, Hkv, Tk, 64]`` bf16 (any strides
    with a contiguous head dimension: the layout GptOssAttention hands over),
    sinks ``[Hq]`` (any float dtype) or None.  Returns the output
    ``[B, Tq, Hq, 64]`` bf16 and, with ``return_lse``, the float32 ``[B, Hq, Tq]``
    log2 softmax denominators the backward uses."""
    dev = _lib.require_gpu(query, key, value, sinks)
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        raise ValueError("attention: query, key and value must be 4-D [B, heads, seq, head_dim]")
    B, Hq, Tq, D = query.shape
    Bk, Hkv, Tk, Dk = key.shape
    if value.shape != key.shape or Bk != B or Dk != D:
        raise ValueError(f"attention: shapes q {tuple(query.shape)} k {tuple(key.shape)} v {tuple(value.shape)}")
    if D != HEAD_DIM:
        raise ValueError(f"attention: head_dim must be {HEAD_DIM} (got {D})")
    for name, t in (("query", query), ("key", key), ("value", value)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"attention: {name} must be bfloat16 (got {t.dtype})")
    q, k, v = (t if _usable(t) else t.contiguous() for t in (query, key, value))
    s = None
    if sinks is not None:
        if sinks.shape != (Hq,):
            raise ValueError(f"attention: sinks must be [{Hq}] (got {tuple(sinks.shape)})")
        s = sinks.detach().to(torch.float32).contiguous()
    out = torch.empty(B, Tq, Hq, D, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, Hq, Tq, dtype=torch.float32, device=dev) if return_lse else None
    # short query grids (decoding) split each row block's keys over several
    # workgroups; the library says from the shape whether, and how much
    # workspace that takes
    ws_bytes = _split_bytes(B, Tq, Tk, Hq, Hkv, 1 if causal else 0, int(window))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
    with torch.cuda.device(dev):
        _lib.call("bsa_attention_fwd_split",
                  q.data_ptr(), _strides(q, 2, 1), k.data_ptr(), _strides(k, 2, 1),
                  v.data_ptr(), _strides(v, 2, 1), s.data_ptr() if s is not None else None,
                  B, Tq, Tk, Hq, Hkv, D, 1 if causal else 0, int(window), float(scaling),
                  out.data_ptr(), _strides(out, 1, 2), lse.data_ptr() if lse is not None else None,
                  ws.data_ptr() if ws is not None else None, ws_bytes, _lib.stream_handle(dev))
    return (out, lse) if return_lse else out


def attention_backward(grad_out: Tensor, query: Tensor, key: Tensor, value: Tensor, sinks: Tensor | None,
                       out: Tensor, lse: Tensor, scaling: float, causal: bool = False, window: int = 0,
                       sinks_grad: bool = False):
    """Gradients of ``attention_forward`` (autograd's through eager_attention_forward,
    TF/models/gpt_oss/modeling_gpt_oss.py:235-264): ``(dq, dk, dv, dsinks)`` shaped
    like query ``[B, Hq, Tq, 64]``, key and value ``[B, Hkv, Tk, 64]`` (bf16 views of
    contiguous ``[B, T, H, 64]`` buffers) and sinks (None unless ``sinks_grad``).
    ``out`` and ``lse`` are the forward's output and log2 denominators."""
    dev = _lib.require_gpu(grad_out, query, key, value, out, lse)
    B, Hq, Tq, D = query.shape
    Hkv, Tk = key.shape[1], key.shape[2]
    if grad_out.shape != (B, Tq, Hq, D) or out.shape != (B, Tq, Hq, D) or lse.shape != (B, Hq, Tq):
        raise ValueError("attention backward: grad_out/out must be [B, Tq, Hq, 64] and lse [B, Hq, Tq]")
    g = grad_out.to(torch.bfloat16)
    q, k, v, g, o = (t if _usable(t) else t.contiguous() for t in (query, key, value, g, out))
    lse = lse.contiguous()
    dq = torch.empty(B, Tq, Hq, D, dtype=torch.bfloat16, device=dev)
    dk = torch.empty(B, Tk, Hkv, D, dtype=torch.bfloat16, device=dev)
    dv = torch.empty_like(dk)
    # per row R = t * (Hq / Hkv) + i of key head hk: (L, D), D = grad_out . out
    row_stats = torch.empty(B, Hkv, Tq * (Hq // Hkv), 2, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("bsa_attention_bwd",
                  g.data_ptr(), _strides(g, 1, 2), q.data_ptr(), _strides(q, 2, 1),
                  k.data_ptr(), _strides(k, 2, 1), v.data_ptr(), _strides(v, 2, 1),
                  o.data_ptr(), _strides(o, 1, 2), lse.data_ptr(),
                  B, Tq, Tk, Hq, Hkv, D, 1 if causal else 0, int(window), float(scaling),
                  dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), row_stats.data_ptr(), _lib.stream_handle(dev))
    dsinks = None
    if sinks_grad:
        # d sink[h] = -sum_t p_sink[t] D[t], p_sink = 2^(sink log2(e) - lse)
        G = Hq // Hkv
        row_dot = row_stats[..., 1].reshape(B, Hkv, Tq, G).permute(0, 1, 3, 2).reshape(B, Hq, Tq)
        p_sink = torch.exp2(sinks.detach().float().reshape(1, Hq, 1) * 1.4426950408889634 - lse)
        dsinks = (-(p_sink * row_dot).sum(dim=(0, 2))).to(sinks.dtype)
    return dq.transpose(1, 2), dk.transpose(1, 2), dv.transpose(1, 2), dsinks


# ---------------------------------------------------------------------------
# transformers attention-function interface
# ---------------------------------------------------------------------------
# Verdicts of mask_kind, keyed by (id(mask), sliding_window) and holding a
# weak reference to the mask itself: a hit needs the very same tensor object
# (alive, so its address cannot have been handed to another tensor) at the
# same version.  transformers builds one mask per forward and passes it to
# every layer, so one check serves the whole model.  A mask written through
# ``.data`` (which bypasses the version counter) between two calls with the
# same tensor object is not seen.
_mask_cache: dict = {}


def _visible(mask: Tensor) -> Tensor:
    """Boolean visibility ``[B, Tq, Tk]`` of an eager (additive) or boolean mask."""
    m = mask[:, 0] if mask.dim() == 4 else mask
    return m if m.dtype == torch.bool else m == 0


def _pattern(Tq: int, Tk: int, window: int, device) -> Tensor:
    pos = torch.arange(Tq, device=device)[:, None] + (Tk - Tq)
    j = torch.arange(Tk, device=device)[None, :]
    vis = j <= pos
    if window > 0:
        vis = vis & (j > pos - window)
    return vis


def mask_kind(attention_mask: Tensor | None, Tq: int, Tk: int, sliding_window: int | None) -> tuple[bool, int]:
    """(causal, window) for the kernel from an eager-interface mask; raises
    for masks the kernel does not express (padding, arbitrary patterns)."""
    if attention_mask is None:
        return False, 0
    if attention_mask.dim() != 4 or attention_mask.shape[1] != 1 or tuple(attention_mask.shape[2:]) != (Tq, Tk):
        raise ValueError(f"attention: mask of shape {tuple(attention_mask.shape)}; expected [B, 1, {Tq}, {Tk}]")
    key = (id(attention_mask), sliding_window)
    hit = _mask_cache.get(key)
    if hit is not None and hit[0]() is attention_mask and hit[1] == attention_mask._version:
        return hit[2]
    vis = _visible(attention_mask)
    result = None
    for window in ([sliding_window] if sliding_window else []) + [0]:
        if bool(torch.all(vis == _pattern(Tq, Tk, window, vis.device))):
            result = (True, int(window))
            break
    if result is None:
        raise ValueError("attention: only the causal and sliding-window causal masks (no padding) are supported")
    if len(_mask_cache) > 64:
        _mask_cache.clear()
    _mask_cache[key] = (weakref.ref(attention_mask), attention_mask._version, result)
    return result


def gpt_oss_attention(module, query: Tensor, key: Tensor, value: Tensor, attention_mask: Tensor | None,
                      scaling: float, dropout: float = 0.0, **kwargs):
    """Drop-in for eager_attention_forward (TF/models/gpt_oss/modeling_gpt_oss.py:235-264)
    through the attention-function interface: returns ``(attn_output [B, Tq, Hq, D], None)``
    (no attention probabilities are materialised)."""
    if dropout and module.training:
        raise ValueError("attention: dropout is not supported (gpt-oss trains with attention_dropout 0)")
    Tq, Tk = query.shape[2], key.shape[2]
    causal, window = mask_kind(attention_mask, Tq, Tk, getattr(module, "sliding_window", None))
    sinks = getattr(module, "sinks", None)
    out = attention(query, key, value, sinks, scaling, causal, window)
    return out, None


def attention(query: Tensor, key: Tensor, value: Tensor, sinks: Tensor | None, scaling: float,
              causal: bool = False, window: int = 0) -> Tensor:
    """``attention_forward`` with autograd (gradients of query, key and value;
    the sinks' gradient when they require one)."""
    return _Attention.apply(query, key, value, sinks, float(scaling), bool(causal), int(window))


class _Attention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, query, key, value, sinks, scaling, causal, window):
        need = any(ctx.needs_input_grad[:4])
        out, lse = attention_forward(query, key, value, sinks, scaling, causal, window, return_lse=True)
        if need:
            ctx.save_for_backward(query, key, value, sinks, out, lse)
        ctx.args = (scaling, causal, window)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        query, key, value, sinks, out, lse = ctx.saved_tensors
        scaling, causal, window = ctx.args
        dq, dk, dv, dsinks = attention_backward(
            grad_out, query, key, value, sinks, out, lse, scaling, causal, window,
            sinks_grad=sinks is not None and ctx.needs_input_grad[3])
        return dq, dk, dv, dsinks, None, None, None


def register() -> None:
    """Make ``"blockstreamer_amd"`` a transformers attention implementation
    (``config._attn_implementation = "blockstreamer_amd"``), with eager masks."""
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, eager_mask

    AttentionInterface.register(NAME, gpt_oss_attention)
    AttentionMaskInterface.register(NAME, eager_mask)
