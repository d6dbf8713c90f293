"""gpt-oss MXFP4 experts on MI355X: the drop-in for ``block_streamer.gptoss``.

Same public names, signatures, parameter names and error behaviour as
block_streamer/gptoss.py:1-189, so ``StreamedModel``'s ``functional_call``
binding (streamer.py:151-180), the LoRA recompute backward
(_autograd.py:125-175) and ``install_mxfp4_experts`` callers work unchanged.
The arithmetic runs in hand-written gfx950 HIP kernels (``libbsamd.so``):

* ``MXFP4Experts.forward`` on bf16 hidden states (and under autocast) is
  one device-side dispatch, two grouped GEMMs that decode MXFP4 on the fly
  (bias and clamped SwiGLU fused), and a combine -- no host synchronisation
  and no dense weight in memory; float32 and float16 hidden states keep
  their precision: the reference's per-expert loop in their dtype, each
  product on ``mxfp4_matmul``'s exact multi-term kernels;
* ``mxfp4_matmul`` runs one expert's product and its input gradient on the
  packed GEMM kernels (float32 inputs to float32 accuracy);
* ``dequantize_expert`` is the dequant kernel, bit-exact with the reference.

The module reads its parameters at every call and never caches device
pointers or mutates them (the StreamedModel contract, streamer.py:159-174).
"""

from __future__ import annotations

import torch
from torch import Tensor, nn

from . import kernels


def dequantize_expert(
    blocks: Tensor, scales: Tensor, dtype: torch.dtype = torch.bfloat16
) -> Tensor:
    """One expert's MXFP4 weight as a dense ``[K, N]`` matrix, in ``dtype``.

    block_streamer/gptoss.py:24-42.  Input: packed codes ``[1, N, K/32, 16]``
    (uint8) and E8M0 exponents ``[1, N, K/32]``, with the expert axis present;
    output ``[K, N]`` (the GEMM's right operand).  Input without the expert
    axis is refused with a ``ValueError`` naming the expected "packed blocks"
    shape (tests/test_offload.py:405-414).  Bit-exact with the transformers
    converter the reference calls.
    """
    if blocks.dim() != 4:
        raise ValueError(
            f"Expected [1, rows, groups, 16] packed blocks, got {tuple(blocks.shape)}"
        )
    dense = kernels.dequantize_mxfp4(blocks, scales, dtype)
    return dense.squeeze(0)


def _autocast_dtype(x: Tensor) -> torch.dtype:
    """The dtype a matmul on ``x`` runs in: the autocast dtype while GPU
    autocast is on (as ``x @ W`` would be cast inside an autocast region),
    else ``x``'s own."""
    if x.is_cuda and torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return x.dtype


class _MXFP4Matmul(torch.autograd.Function):
    """Packed-weight product for one expert (block_streamer/gptoss.py:45-71).

    Both directions run the hand-written packed GEMMs (``kernels.mxfp4_matmul``):
    the forward reads the MXFP4 blocks as the B operand, the input gradient
    reads the same blocks along their rows.  No dense weight is formed, and
    the context keeps only the packed tensors (already resident as staged
    state), so nothing of size K x N outlives the call.  The weights are
    frozen: only the input gets a gradient.
    """

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, x: Tensor, blocks: Tensor, scales: Tensor) -> Tensor:
        dtype = _autocast_dtype(x)
        ctx.save_for_backward(blocks, scales)
        ctx.x_dtype = x.dtype
        return kernels.mxfp4_matmul(x.to(dtype), blocks, scales)

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, grad: Tensor) -> tuple[Tensor | None, None, None]:
        if not ctx.needs_input_grad[0]:
            return None, None, None
        blocks, scales = ctx.saved_tensors
        return kernels.mxfp4_matmul(grad, blocks, scales, transpose=True, out_dtype=ctx.x_dtype), None, None


def mxfp4_matmul(x: Tensor, blocks: Tensor, scales: Tensor) -> Tensor:
    """``x @ dequantize_expert(blocks, scales, x.dtype)``, differentiable in
    ``x`` (block_streamer/gptoss.py:74-75), without the dense weight."""
    return _MXFP4Matmul.apply(x, blocks, scales)


class _MoEExperts(torch.autograd.Function):
    """Fused expert forward; backward gives d(hidden) and d(routing weights).

    Saves the packed weights (already resident as the block's staged state),
    the inputs, the device-side dispatch and the SwiGLU's bf16 derivative
    factors (the size of the bf16 gate_up the reference's autograd keeps) --
    never a dense weight (the rationale of block_streamer/gptoss.py:46-56).
    """

    @staticmethod
    def forward(ctx, hidden, router_indices, routing_weights, gu_blocks, gu_scales, gu_bias,
                dn_blocks, dn_scales, dn_bias, alpha, limit, train_path="auto"):
        needs = ctx.needs_input_grad[0] or ctx.needs_input_grad[2]
        if needs:
            out, ws, fac = kernels.moe_experts_forward(
                hidden, router_indices, routing_weights, gu_blocks, gu_scales, gu_bias,
                dn_blocks, dn_scales, dn_bias, alpha, limit, save=True, path=train_path)
            ctx.save_for_backward(hidden, router_indices, routing_weights, gu_blocks, gu_scales,
                                  gu_bias, dn_blocks, dn_scales, dn_bias, ws, fac)
            ctx.alpha, ctx.limit = alpha, limit
        else:
            out = kernels.moe_experts_forward(
                hidden, router_indices, routing_weights, gu_blocks, gu_scales, gu_bias,
                dn_blocks, dn_scales, dn_bias, alpha, limit)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        (hidden, idx, w, gu_b, gu_s, gu_bias, dn_b, dn_s, dn_bias, ws,
         fac) = ctx.saved_tensors
        grad_h, grad_w = kernels.moe_experts_backward(
            grad_out, hidden, idx, w, gu_b, gu_s, dn_b, dn_s, ws, fac, ctx.alpha, ctx.limit,
            need_hidden=ctx.needs_input_grad[0], need_weights=ctx.needs_input_grad[2])
        return grad_h, None, grad_w, None, None, None, None, None, None, None, None, None


class MXFP4Experts(nn.Module):
    """gpt-oss expert block over packed MXFP4 weights (block_streamer/gptoss.py:78-177).

    Replaces transformers' dense ``GptOssExperts``.  Its six parameters carry
    the gpt-oss checkpoint's own tensor names, which is what lets a
    ``functional_call`` bind staged shard tensors to the module by name.
    The placeholders live on the meta device and use ``hidden_size // 32``
    groups for both projections, as gptoss.py:92 does; the kernels read every
    shape from the tensors actually bound at call time.

    ``mx_training`` (default False): a forward that saves for the backward
    (training) runs the bf16 kernels, whose clamp decisions at +-7 are the
    closest to float32's; set it to run the native MX kernels there as well
    for prefill-sized batches (faster).  Their products carry the block-scaled
    MFMA's accumulation error, which moves a few more pre-activations across
    the clamp than the bf16 kernels do -- far fewer than the reference's own
    bf16 arithmetic, which rounds the pre-activations to bf16 first.
    """

    def __init__(self, config, dtype: torch.dtype = torch.bfloat16) -> None:
        super().__init__()
        self.num_experts = config.num_local_experts
        self.hidden_size = config.hidden_size
        self.expert_dim = config.intermediate_size
        self.alpha = 1.702
        self.limit = getattr(config, "swiglu_limit", 7.0)
        self.mx_training = False
        groups = self.hidden_size // 32

        def packed(rows: int) -> nn.Parameter:
            return nn.Parameter(
                torch.empty(self.num_experts, rows, groups, 16, dtype=torch.uint8, device="meta"),
                requires_grad=False,
            )

        def scale(rows: int) -> nn.Parameter:
            return nn.Parameter(
                torch.empty(self.num_experts, rows, groups, dtype=torch.uint8, device="meta"),
                requires_grad=False,
            )

        self.gate_up_proj_blocks = packed(2 * self.expert_dim)
        self.gate_up_proj_scales = scale(2 * self.expert_dim)
        self.gate_up_proj_bias = nn.Parameter(
            torch.empty(self.num_experts, 2 * self.expert_dim, dtype=dtype, device="meta"),
            requires_grad=False,
        )
        self.down_proj_blocks = packed(self.hidden_size)
        self.down_proj_scales = scale(self.hidden_size)
        self.down_proj_bias = nn.Parameter(
            torch.empty(self.num_experts, self.hidden_size, dtype=dtype, device="meta"),
            requires_grad=False,
        )

    def _apply_gate(self, gate_up: Tensor) -> Tensor:
        """block_streamer/gptoss.py:130-135 (the fused kernels apply it in-register)."""
        gate, up = gate_up[..., ::2], gate_up[..., 1::2]
        gate = gate.clamp(max=self.limit)
        up = up.clamp(min=-self.limit, max=self.limit)
        glu = gate * torch.sigmoid(gate * self.alpha)
        return (up + 1) * glu

    def forward(
        self,
        hidden_states: Tensor,
        router_indices: Tensor | None = None,
        routing_weights: Tensor | None = None,
    ) -> Tensor:
        if router_indices is None or routing_weights is None:
            raise ValueError("MXFP4Experts.forward needs router_indices and routing_weights")
        shape = hidden_states.shape
        flat = hidden_states.reshape(-1, shape[-1])
        if flat.dtype in (torch.float32, torch.float16) and not (flat.is_cuda and torch.is_autocast_enabled("cuda")):
            return self._forward_in_dtype(flat, router_indices, routing_weights).reshape(shape)
        train_path = "auto"
        if self.mx_training:
            # where an inference forward would take the MX kernels: prefill-sized
            # batches, widths multiples of 64, aligned blocks and scales
            E, I = kernels._experts_dims(self.gate_up_proj_blocks)
            if kernels._whole_forward_path("auto", flat.shape[0], router_indices.shape[-1], E, flat.shape[1], I,
                                           self.gate_up_proj_blocks, self.gate_up_proj_scales,
                                           self.down_proj_blocks, self.down_proj_scales) == kernels.PATHS["mx"]:
                train_path = "mx"
        out = _MoEExperts.apply(
            flat, router_indices, routing_weights,
            self.gate_up_proj_blocks, self.gate_up_proj_scales, self.gate_up_proj_bias,
            self.down_proj_blocks, self.down_proj_scales, self.down_proj_bias,
            float(self.alpha), float(self.limit), train_path,
        )
        return out.reshape(shape)


    def _forward_in_dtype(self, hidden: Tensor, router_indices: Tensor, routing_weights: Tensor) -> Tensor:
        """float32 / float16 hidden states: block_streamer/gptoss.py:143-176 op
        for op in the hidden states' own dtype, one expert at a time, each
        product on the packed kernels of ``mxfp4_matmul`` (the input split into
        bf16 terms whose sum is it exactly -- three for float32, two for
        float16 -- times the exactly decoded weights, summed in float32 and
        rounded once to the input dtype).  So the rounding points are the
        reference's: its ``x @ dequantize(..., x.dtype)``, the bias add, the
        SwiGLU and the combine all happen in the input dtype.  Differentiable
        through ``mxfp4_matmul``'s own backward.  Router indices outside
        [0, E) are dropped, as in the fused path."""
        E = self.gate_up_proj_blocks.shape[0]
        out = torch.zeros_like(hidden)
        idx = router_indices.reshape(hidden.shape[0], -1).to(torch.int64)
        w = routing_weights.reshape(idx.shape)
        with torch.no_grad():
            valid = (idx >= 0) & (idx < E)
            hit = torch.unique(idx[valid]).tolist()                      # ascending, as gptoss.py:148
        for e in hit:
            top_k_pos, token_idx = torch.where(idx.t() == e)             # (slot, token) order, gptoss.py:153
            current = hidden[token_idx]
            gate_up = (mxfp4_matmul(current, self.gate_up_proj_blocks[e:e + 1], self.gate_up_proj_scales[e:e + 1])
                       + self.gate_up_proj_bias[e])
            gated = self._apply_gate(gate_up)
            o = (mxfp4_matmul(gated, self.down_proj_blocks[e:e + 1], self.down_proj_scales[e:e + 1])
                 + self.down_proj_bias[e])
            o = o * w[token_idx, top_k_pos, None]
            out = out.index_add(0, token_idx, o.to(hidden.dtype))
        return out


class _Router(torch.autograd.Function):
    """Fused router forward; backward through the softmax over the top-k
    values and the linear layer, as torch autograd differentiates
    TF/models/gpt_oss/modeling_gpt_oss.py:127-129 (gradients flow only into the
    k selected logits)."""

    @staticmethod
    def forward(ctx, hidden, weight, bias, top_k):
        logits, scores, idx = kernels.router_forward(hidden, weight, bias, top_k)
        ctx.save_for_backward(hidden, weight, scores, idx)
        ctx.has_bias = bias is not None
        ctx.mark_non_differentiable(idx)
        return logits, scores, idx

    @staticmethod
    def backward(ctx, d_logits, d_scores, _d_idx):
        hidden, weight, scores, idx = ctx.saved_tensors
        T, E = hidden.shape[0], weight.shape[0]
        dl = torch.zeros((T, E), dtype=torch.float32, device=hidden.device)
        if d_logits is not None:
            dl += d_logits.float()
        if d_scores is not None:
            s = scores.float()
            ds = d_scores.float()
            dvals = s * (ds - (s * ds).sum(dim=-1, keepdim=True))  # softmax backward
            dl.scatter_add_(1, idx, dvals)
        dl = dl.to(hidden.dtype)
        dh = dl @ weight.to(hidden.dtype) if ctx.needs_input_grad[0] else None
        dw = dl.t() @ hidden if ctx.needs_input_grad[1] else None
        db = dl.sum(0) if (ctx.has_bias and ctx.needs_input_grad[2]) else None
        return dh, dw, db, None


class MXFP4TopKRouter(nn.Module):
    """Drop-in for ``GptOssTopKRouter`` (TF/models/gpt_oss/modeling_gpt_oss.py:117-131)
    with the logits, top-k and softmax in one HIP kernel.  Same parameter
    names (``weight [E, H]``, ``bias [E]``) and return value
    ``(logits, scores, indices)``."""

    def __init__(self, config, dtype: torch.dtype = torch.bfloat16, device=None) -> None:
        super().__init__()
        self.top_k = config.num_experts_per_tok
        self.num_experts = config.num_local_experts
        self.hidden_dim = config.hidden_size
        self.weight = nn.Parameter(torch.zeros(self.num_experts, self.hidden_dim, dtype=dtype, device=device))
        self.bias = nn.Parameter(torch.zeros(self.num_experts, dtype=dtype, device=device))

    def forward(self, hidden_states: Tensor):
        flat = hidden_states.reshape(-1, self.hidden_dim)
        return _Router.apply(flat, self.weight, self.bias, self.top_k)


class MXFP4MLP(nn.Module):
    """Drop-in for ``GptOssMLP`` (TF/models/gpt_oss/modeling_gpt_oss.py:133-146):
    fused router plus packed experts; ``forward(h [B, S, H])`` returns
    ``(out [B, S, H], router_scores [T, k])``."""

    def __init__(self, config, dtype: torch.dtype = torch.bfloat16) -> None:
        super().__init__()
        self.router = MXFP4TopKRouter(config, dtype)
        self.experts = MXFP4Experts(config, dtype)

    def forward(self, hidden_states: Tensor):
        batch_size, sequence_length, hidden_dim = hidden_states.shape
        flat = hidden_states.reshape(-1, hidden_dim)
        _, router_scores, router_indices = self.router(flat)
        out = self.experts(flat, router_indices, router_scores)
        return out.reshape(batch_size, sequence_length, hidden_dim), router_scores


class _RMSNorm(torch.autograd.Function):
    """One-launch RMSNorm; the input gradient in one launch as well.  The
    weight gradient (frozen in LoRA training) is formed with torch ops only
    when it is asked for."""

    @staticmethod
    def forward(ctx, hidden, weight, eps):
        out = kernels.rmsnorm_forward(hidden, weight, eps)
        ctx.save_for_backward(hidden, weight)
        ctx.eps = eps
        return out

    @staticmethod
    def backward(ctx, grad):
        hidden, weight = ctx.saved_tensors
        dh = kernels.rmsnorm_backward(grad, hidden, weight, ctx.eps) if ctx.needs_input_grad[0] else None
        dw = None
        if ctx.needs_input_grad[1]:
            h32 = hidden.float()
            normed = h32 * torch.rsqrt(h32.pow(2).mean(-1, keepdim=True) + ctx.eps)
            dw = (grad.float() * normed).reshape(-1, hidden.shape[-1]).sum(0).to(weight.dtype)
        return dh, dw, None


class FusedRMSNorm(nn.Module):
    """Drop-in for ``GptOssRMSNorm`` (TF/models/gpt_oss/modeling_gpt_oss.py:47-62):
    same parameter (``weight [H]``), attribute (``variance_epsilon``) and
    result dtype (that of the input), computed in one HIP launch instead of
    the eager module's chain of elementwise kernels."""

    def __init__(self, hidden_size: int, eps: float = 1e-6, dtype: torch.dtype = torch.float32,
                 device=None) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size, dtype=dtype, device=device))
        self.variance_epsilon = eps

    def forward(self, hidden_states: Tensor) -> Tensor:
        return _RMSNorm.apply(hidden_states, self.weight, self.variance_epsilon)

    def extra_repr(self) -> str:
        return f"{tuple(self.weight.shape)}, eps={self.variance_epsilon}"


def install_fused_post_attention_norm(model: nn.Module) -> int:
    """Swap every layer's ``post_attention_layernorm`` (the norm in front of
    the router and experts, modeling_gpt_oss.py:373) for ``FusedRMSNorm``.

    No counterpart in the reference, which keeps the transformers module; the
    parameter name, dtype and device are kept, so checkpoints and shards bind
    as before.  Returns the number of layers changed.
    """
    from transformers.models.gpt_oss import modeling_gpt_oss as gpt_oss

    replaced = 0
    for layer in model.model.layers:
        old = layer.post_attention_layernorm
        if isinstance(old, gpt_oss.GptOssRMSNorm):
            new = FusedRMSNorm(old.weight.shape[0], old.variance_epsilon, old.weight.dtype,
                               None if old.weight.device.type == "meta" else old.weight.device)
            if old.weight.device.type != "meta":
                with torch.no_grad():
                    new.weight.copy_(old.weight)
            new.weight.requires_grad_(old.weight.requires_grad)
            layer.post_attention_layernorm = new
            replaced += 1
    return replaced


def install_native_attention(model: nn.Module) -> int:
    """Run every GptOssAttention of ``model`` on the HIP attention kernels:
    registers ``blockstreamer_amd.attention.gpt_oss_attention`` with
    transformers' attention-function interface (eager-style masks) and selects
    it in ``model.config``, the switch GptOssAttention.forward reads
    (modeling_gpt_oss.py:322-324).

    No counterpart in the reference, which runs transformers' eager attention.
    No parameter changes.  Returns the number of attention modules switched.
    """
    from transformers.models.gpt_oss import modeling_gpt_oss as gpt_oss

    from . import attention

    attention.register()
    model.config._attn_implementation = attention.NAME
    count = 0
    for mod in model.modules():
        if isinstance(mod, gpt_oss.GptOssAttention):
            mod.config._attn_implementation = attention.NAME
            count += 1
    return count


def install_mxfp4_router(model: nn.Module, config, dtype: torch.dtype | None = None) -> int:
    """Swap every ``GptOssTopKRouter`` for the fused ``MXFP4TopKRouter``.

    No counterpart in the reference, which keeps the transformers router;
    parameter names are unchanged, so checkpoints and shards bind as before.
    Each new router lives on the old one's device (meta stays meta) and, unless
    ``dtype`` is given, keeps its dtype; its weight and bias are copied over,
    as is their ``requires_grad``.  Returns the number of layers changed.
    """
    from transformers.models.gpt_oss import modeling_gpt_oss as gpt_oss

    replaced = 0
    for layer in model.model.layers:
        if isinstance(layer.mlp.router, gpt_oss.GptOssTopKRouter):
            old = layer.mlp.router
            new = MXFP4TopKRouter(config, dtype or old.weight.dtype, device=old.weight.device)
            if old.weight.device.type != "meta":
                with torch.no_grad():
                    new.weight.copy_(old.weight)
                    new.bias.copy_(old.bias)
            new.weight.requires_grad_(old.weight.requires_grad)
            new.bias.requires_grad_(old.bias.requires_grad)
            layer.mlp.router = new
            replaced += 1
    return replaced


def install_mxfp4_experts(model: nn.Module, config, dtype=torch.bfloat16) -> int:
    """Put an ``MXFP4Experts`` (packed weights, fused HIP kernels) in place of
    each layer's dense ``GptOssExperts``.

    block_streamer/gptoss.py:180-189; returns how many layers changed.
    """
    from transformers.models.gpt_oss import modeling_gpt_oss as gpt_oss

    replaced = 0
    for layer in model.model.layers:
        if isinstance(layer.mlp.experts, gpt_oss.GptOssExperts):
            layer.mlp.experts = MXFP4Experts(config, dtype)
            replaced += 1
    return replaced
