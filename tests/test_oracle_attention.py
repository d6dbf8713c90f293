"""Pins the oracle's attention restatement (CPU only).

``oracle.attention_ref`` is checked against the installed transformers
``eager_attention_forward`` (TF/models/gpt_oss/modeling_gpt_oss.py:235-264) in
float64, with the masks transformers' own ``masking_utils.eager_mask`` builds,
and against closed forms that a dropped term, a wrong sign, a transposed
operand or an off-by-one mask would break.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

import oracle

tf_gptoss = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")
masking = pytest.importorskip("transformers.masking_utils")


class _Module(torch.nn.Module):
    """The attributes eager_attention_forward reads from GptOssAttention."""

    def __init__(self, sinks: torch.Tensor, groups: int):
        super().__init__()
        self.sinks = torch.nn.Parameter(sinks, requires_grad=False)
        self.num_key_value_groups = groups
        self.training = False


def _inputs(B, Hq, Hkv, Tq, Tk, D=64, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, Tq, D, generator=g, dtype=torch.float64) * scale
    k = torch.randn(B, Hkv, Tk, D, generator=g, dtype=torch.float64) * scale
    v = torch.randn(B, Hkv, Tk, D, generator=g, dtype=torch.float64)
    sinks = torch.randn(Hq, generator=g, dtype=torch.float64) * 2
    return q, k, v, sinks


def _tf(q, k, v, sinks, scaling, mask):
    mod = _Module(sinks, q.shape[1] // k.shape[1])
    out, _ = tf_gptoss.eager_attention_forward(mod, q, k, v, mask, scaling=scaling, dropout=0.0)
    return out


def _mask(kind, B, Tq, Tk, window=0):
    if kind == "none":
        return None
    fn = (masking.causal_mask_function if kind == "causal"
          else masking.sliding_window_causal_mask_function(window))
    return masking.eager_mask(batch_size=B, q_length=Tq, kv_length=Tk, q_offset=Tk - Tq,
                              mask_function=fn, dtype=torch.float64)


@pytest.mark.parametrize("kind,Tq,Tk,window", [
    ("none", 7, 7, 0), ("none", 3, 11, 0),
    ("causal", 9, 9, 0), ("causal", 4, 13, 0), ("causal", 1, 10, 0),
    ("sliding", 12, 12, 4), ("sliding", 5, 17, 3), ("sliding", 1, 9, 4), ("sliding", 8, 8, 1),
])
def test_attention_ref_matches_transformers_eager(kind, Tq, Tk, window):
    B, Hq, Hkv = 2, 8, 2
    q, k, v, sinks = _inputs(B, Hq, Hkv, Tq, Tk, seed=Tq * 31 + Tk)
    scaling = 64 ** -0.5
    want = _tf(q, k, v, sinks, scaling, _mask(kind, B, Tq, Tk, window))
    got = oracle.attention_ref(q, k, v, sinks, scaling, causal=kind != "none", window=window)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)


def test_attention_ref_without_sink_is_sdpa():
    """A sink of -inf contributes exp(-inf) = 0: plain softmax attention."""
    B, Hq, Hkv, T = 1, 4, 4, 10
    q, k, v, _ = _inputs(B, Hq, Hkv, T, T, seed=3)
    scaling = 0.125
    for causal in (False, True):
        want = F.scaled_dot_product_attention(q, k, v, is_causal=causal, scale=scaling).transpose(1, 2)
        got = oracle.attention_ref(q, k, v, torch.full((Hq,), float("-inf"), dtype=torch.float64), scaling,
                                   causal=causal)
        torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
        got = oracle.attention_ref(q, k, v, None, scaling, causal=causal)
        torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)


def test_attention_ref_one_visible_key_is_sigmoid():
    """Query 0 under the causal mask sees key 0 only: p = e^s / (e^s + e^sink)."""
    B, Hq, Hkv, T = 1, 2, 1, 5
    q, k, v, sinks = _inputs(B, Hq, Hkv, T, T, seed=5)
    scaling = 0.3
    got = oracle.attention_ref(q, k, v, sinks, scaling, causal=True)
    for h in range(Hq):
        s = float((q[0, h, 0] * k[0, 0, 0]).sum()) * scaling
        p = 1.0 / (1.0 + math.exp(float(sinks[h]) - s))
        torch.testing.assert_close(got[0, 0, h], p * v[0, 0, 0], rtol=1e-12, atol=1e-12)
    # a window of 1 leaves every query only its own key
    got = oracle.attention_ref(q, k, v, sinks, scaling, causal=True, window=1)
    for t in range(T):
        s = float((q[0, 1, t] * k[0, 0, t]).sum()) * scaling
        p = 1.0 / (1.0 + math.exp(float(sinks[1]) - s))
        torch.testing.assert_close(got[0, t, 1], p * v[0, 0, t], rtol=1e-12, atol=1e-12)


def test_attention_ref_grouped_heads_equal_repeated_keys():
    B, Hq, Hkv, Tq, Tk = 2, 8, 2, 6, 9
    q, k, v, sinks = _inputs(B, Hq, Hkv, Tq, Tk, seed=9)
    G = Hq // Hkv
    got = oracle.attention_ref(q, k, v, sinks, 0.2, causal=True, window=5)
    want = oracle.attention_ref(q, k.repeat_interleave(G, dim=1), v.repeat_interleave(G, dim=1), sinks, 0.2,
                                causal=True, window=5)
    torch.testing.assert_close(got, want, rtol=0, atol=0)


def test_attention_ref_rows_sum_below_one():
    """With V = 1 every output is the visible probability mass: 1 - p_sink."""
    B, Hq, Hkv, T = 1, 4, 2, 8
    q, k, _, sinks = _inputs(B, Hq, Hkv, T, T, seed=11)
    v = torch.ones(B, Hkv, T, 64, dtype=torch.float64)
    got = oracle.attention_ref(q, k, v, sinks, 0.125, causal=True)
    assert torch.all(got < 1) and torch.all(got > 0)
    no_sink = oracle.attention_ref(q, k, v, None, 0.125, causal=True)
    torch.testing.assert_close(no_sink, torch.ones_like(no_sink), rtol=1e-12, atol=1e-12)
