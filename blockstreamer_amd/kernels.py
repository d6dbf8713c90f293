"""Tensor-level wrappers over the C ABI (one function per kernel family).

Each wrapper validates shapes and dtypes on the host, allocates outputs and
workspace from the torch caching allocator (so ``record_stream`` protection
of the caller applies), and launches on ``torch.cuda.current_stream()`` of
the tensors' device.  Nothing here synchronises the host.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib


def _as_u8(t: Tensor) -> Tensor:
    if t.dtype != torch.uint8:
        t = t.to(torch.uint8)
    return t if t.is_contiguous() else t.contiguous()


# Layouts of packed MXFP4 blocks (scales are always [E, rows, groups]):
# checkpoint [E, rows, groups, 16], and the k-pair shard layout
# [E, rows/16, groups/2, 16, 2, 16] (group g of row r at [e][r/16][g/2][r%16][g%2]).
LAYOUT_CHECKPOINT, LAYOUT_KPAIR = 0, 1


def blocks_layout(blocks: Tensor) -> int:
    """The layout of a packed blocks tensor, from its shape."""
    if blocks.dim() == 4 and blocks.shape[-1] == 16:
        return LAYOUT_CHECKPOINT
    if blocks.dim() == 6 and tuple(blocks.shape[3:]) == (16, 2, 16):
        return LAYOUT_KPAIR
    raise ValueError(
        f"packed blocks must be [E, rows, groups, 16] or the k-pair layout "
        f"[E, rows/16, groups/2, 16, 2, 16], got {tuple(blocks.shape)}"
    )


def packed_shape(blocks: Tensor) -> tuple[int, int, int]:
    """``(E, rows, groups)`` of a packed blocks tensor in either layout."""
    if blocks_layout(blocks) == LAYOUT_CHECKPOINT:
        E, R, G, _ = blocks.shape
        return E, R, G
    E, bands, pairs = blocks.shape[:3]
    return E, bands * 16, pairs * 2


def to_kpair(blocks: Tensor) -> Tensor:
    """Checkpoint-layout blocks ``[E, R, G, 16]`` in the k-pair layout
    ``[E, R/16, G/2, 16, 2, 16]`` (R % 16 == 0, G even), bit for bit."""
    return _repack(blocks, to_kp=True)


def from_kpair(blocks: Tensor) -> Tensor:
    """The inverse of ``to_kpair``."""
    return _repack(blocks, to_kp=False)


def _repack(blocks: Tensor, to_kp: bool) -> Tensor:
    want = LAYOUT_CHECKPOINT if to_kp else LAYOUT_KPAIR
    if blocks_layout(blocks) != want:
        raise ValueError(f"expected {'checkpoint' if to_kp else 'k-pair'} layout blocks, got {tuple(blocks.shape)}")
    E, R, G = packed_shape(blocks)
    if R % 16 or G % 2:
        raise ValueError(f"the k-pair layout needs rows % 16 == 0 and an even group count (rows={R}, groups={G})")
    dev = _lib.require_gpu(blocks)
    src = _aligned(_as_u8(blocks), 16)
    shape = (E, R // 16, G // 2, 16, 2, 16) if to_kp else (E, R, G, 16)
    out = torch.empty(shape, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _lib.call("bsa_mxfp4_to_kpair" if to_kp else "bsa_mxfp4_from_kpair", src.data_ptr(), out.data_ptr(),
                  E, R, G, _lib.stream_handle(dev))
    return out


def dequantize_mxfp4(blocks: Tensor, scales: Tensor, dtype: torch.dtype = torch.bfloat16,
                     out: Tensor | None = None, mode: int = 0) -> Tensor:
    """Dense ``[E, G*32, R]`` weights from packed ``[E, R, G, 16]`` MXFP4
    (or the same blocks in the k-pair layout).

    The transformers ``convert_moe_packed_tensors`` contract for a 4-D input
    (TF/integrations/mxfp4.py:257-313): bit-exact in bf16/f16/f32.
    """
    layout = blocks_layout(blocks)
    E, R, G = packed_shape(blocks)
    if tuple(scales.shape) != (E, R, G):
        raise ValueError(f"scales shape {tuple(scales.shape)} does not match blocks {(E, R, G)}")
    code = _lib.dtype_code(dtype)
    dev = _lib.require_gpu(blocks, scales)
    blocks = _as_u8(blocks)
    scales = _as_u8(scales)
    if layout == LAYOUT_KPAIR:
        _require_kpair_aligned(blocks, "blocks")
    if out is None:
        out = torch.empty((E, G * 32, R), dtype=dtype, device=dev)
    elif out.shape != (E, G * 32, R) or out.dtype != dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous [E, G*32, R] tensor of the requested dtype")
    with torch.cuda.device(dev):
        _lib.call("bsa_dequant_mxfp4_layout", blocks.data_ptr(), scales.data_ptr(), out.data_ptr(),
                  code, E, R, G, mode, layout, _lib.stream_handle(dev))
    return out


def mxfp4_matmul(x: Tensor, blocks: Tensor, scales: Tensor, transpose: bool = False,
                 out_dtype: torch.dtype | None = None) -> Tensor:
    """One expert's packed matmul with no dense weight (block_streamer/
    gptoss.py:45-75): ``x [..., K] @ W`` (``W`` the ``[K, N]`` matrix
    ``dequantize_expert`` returns), or with ``transpose=True``
    ``x [..., N] @ W.T``, from ``blocks [1, N, K/32, 16]`` and
    ``scales [1, N, K/32]`` (the expert axis as the reference passes it; the
    k-pair layout is accepted too).  bf16, f16 and f32 ``x``; the result is in
    ``out_dtype`` (default ``x.dtype``).  f32 ``x`` keeps float32 accuracy
    (three exact bf16 terms, one GEMM pass each)."""
    layout = blocks_layout(blocks)
    E, N, G = packed_shape(blocks)
    if E != 1 or tuple(scales.shape) != (1, N, G):
        raise ValueError(f"expected one expert's blocks [1, N, K/32, 16] and scales [1, N, K/32], got "
                         f"{tuple(blocks.shape)} and {tuple(scales.shape)}")
    K = G * 32
    kin, nout = (N, K) if transpose else (K, N)
    if x.shape[-1] != kin:
        raise ValueError(f"x has {x.shape[-1]} columns; this product needs {kin}")
    dev = _lib.require_gpu(x, blocks, scales)
    code = _lib.dtype_code(x.dtype)
    out_dtype = out_dtype or x.dtype
    blocks, scales = _as_u8(blocks), _as_u8(scales)
    if layout == LAYOUT_KPAIR:
        _require_kpair_aligned(blocks, "blocks")
    blocks = _aligned(blocks, 8)
    scales = _aligned(scales, 4)
    lead = x.shape[:-1]
    x2 = x.reshape(-1, kin).contiguous()
    M = x2.shape[0]
    out = torch.empty((M, nout), dtype=out_dtype, device=dev)
    import ctypes
    n = ctypes.c_int64(0)
    _lib.call("bsa_mxfp4_matmul_workspace_bytes", M, K, N, code, int(transpose), ctypes.byref(n))
    ws = _aligned_bytes(n.value, dev)
    with torch.cuda.device(dev):
        _lib.call("bsa_mxfp4_matmul", x2.data_ptr(), code, M, K, N, blocks.data_ptr(), scales.data_ptr(),
                  layout, int(transpose), out.data_ptr(), _lib.dtype_code(out_dtype), ws.data_ptr(), n.value,
                  _lib.stream_handle(dev))
    return out.reshape(*lead, nout)


# Expert GEMM kernels: "stream" (weight streaming, decode), "tiled" (bf16
# MFMA over LDS tiles, prefill), "auto" (by rows per expert) -- all bf16
# activations x exactly dequantised MXFP4 weights; "mx" (the activations as
# two MXFP8 terms x the packed MXFP4 weights on the block-scaled f8f6f4 MFMA,
# prefill: the bf16 activations exactly, elements below 2^-14 of their
# 32-element block's maximum aside).
PATHS = {"auto": 0, "stream": 1, "tiled": 2, "mx": 3}


def quantize_mxfp8(x: Tensor) -> tuple[Tensor, Tensor]:
    """OCP MXFP8 (E4M3 + one E8M0 scale per 32) of a ``[R, K]`` tensor.

    Returns ``(codes uint8 [R, K], scales uint8 [R, K/32])``.  The A operand
    format of the ``"mx"`` GEMM path; no reference counterpart.
    """
    if x.dim() != 2 or x.shape[1] % 32 != 0:
        raise ValueError(f"x must be [rows, K] with K % 32 == 0, got {tuple(x.shape)}")
    dev = _lib.require_gpu(x)
    code = _lib.dtype_code(x.dtype)
    x = x.contiguous()
    R, K = x.shape
    q = torch.empty((R, K), dtype=torch.uint8, device=dev)
    s = torch.empty((R, K // 32), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _lib.call("bsa_quant_mxfp8", x.data_ptr(), code, R, K, q.data_ptr(), s.data_ptr(), K // 32,
                  _lib.stream_handle(dev))
    return q, s


def quantize_mxfp8_split(x: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """Two-term MXFP8 split of a ``[R, K]`` tensor (K % 64 == 0): the
    activation format of the ``"mx"`` GEMM path; no reference counterpart.

    Returns ``(hi uint8 [R, K], lo uint8 [R, K], scales uint8 [R, K/32])``:
    x ~ hi * 2^X + lo * 2^max(X - 4, -127) per 32-element block, X = scale - 127.
    The kernel interleaves hi and lo per 64-element k-tile; they are returned
    here as two views of that buffer.
    """
    if x.dim() != 2 or x.shape[1] % 64 != 0:
        raise ValueError(f"x must be [rows, K] with K % 64 == 0, got {tuple(x.shape)}")
    dev = _lib.require_gpu(x)
    code = _lib.dtype_code(x.dtype)
    x = x.contiguous()
    R, K = x.shape
    q = torch.empty((R, 2 * K), dtype=torch.uint8, device=dev)
    s = torch.empty((R, K // 32), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _lib.call("bsa_quant_mxfp8_split", x.data_ptr(), code, R, K, q.data_ptr(), s.data_ptr(), K // 32,
                  _lib.stream_handle(dev))
    tiles = q.view(R, K // 64, 2, 64)
    return tiles[:, :, 0].reshape(R, K), tiles[:, :, 1].reshape(R, K), s


def moe_workspace_bytes(T: int, H: int, I: int, E: int, k: int) -> int:
    import ctypes
    out = ctypes.c_int64(0)
    _lib.call("bsa_moe_workspace_bytes", T, H, I, E, k, ctypes.byref(out))
    return out.value


def _aligned(t: Tensor, n: int) -> Tensor:
    """``t`` itself when its storage starts on an n-byte boundary, else a copy."""
    return t if t.data_ptr() % n == 0 else t.clone()


def _require_kpair_aligned(blocks: Tensor, what: str) -> Tensor:
    """k-pair layout blocks move in 16-byte pieces only, so they must start
    on a 16-byte boundary.  The reference's shard planner aligns tensors to
    8 bytes (block_streamer/shards.py:148-165); a writer that stores the
    k-pair layout aligns them to 16.  Copying on every call would move the
    whole tensor each time, so a misaligned tensor is refused instead."""
    if blocks.data_ptr() % 16:
        raise ValueError(f"{what} in the k-pair layout must be 16-byte aligned (address % 16 = "
                         f"{blocks.data_ptr() % 16}); write k-pair shards with 16-byte tensor alignment, "
                         f"or repack with from_kpair()")
    return blocks


def _aligned_bytes(nbytes: int, device, align: int = 256) -> Tensor:
    buf = torch.empty(nbytes + align, dtype=torch.uint8, device=device)
    off = (-buf.data_ptr()) % align
    return buf[off:off + nbytes]


def _check_packed(blocks: Tensor, scales: Tensor, E: int, rows: int, K: int, what: str) -> int:
    """Checks the shapes; returns the blocks' layout."""
    want = (E, rows, K // 32)
    try:
        layout = blocks_layout(blocks)
        got = packed_shape(blocks)
    except ValueError:
        layout, got = -1, None
    if got != want:
        raise ValueError(f"{what}_blocks must be {list(want) + [16]} (or that in the k-pair layout), "
                         f"got {list(blocks.shape)}")
    if tuple(scales.shape) != want:
        raise ValueError(f"{what}_scales must be {list(want)}, got {list(scales.shape)}")
    return layout


def _check_bias(bias: Tensor | None, E: int, n: int, what: str) -> None:
    """The kernels read a bias as ``[E][n]``; anything else would read past it."""
    if bias is not None and tuple(bias.shape) != (E, n):
        raise ValueError(f"{what}_bias must be [{E}, {n}], got {list(bias.shape)}")


def _experts_dims(gate_up_blocks: Tensor) -> tuple[int, int]:
    """``(E, I)`` from the gate_up blocks in either layout."""
    E, rows, _ = packed_shape(gate_up_blocks)
    return E, rows // 2


def moe_experts_forward(hidden: Tensor, router_indices: Tensor, routing_weights: Tensor,
                        gate_up_blocks: Tensor, gate_up_scales: Tensor, gate_up_bias: Tensor | None,
                        down_blocks: Tensor, down_scales: Tensor, down_bias: Tensor | None,
                        alpha: float = 1.702, limit: float = 7.0, *, save: bool = False,
                        path: str = "auto", noalloc: bool = False, out_dtype: torch.dtype | None = None):
    """Fused MoE experts forward (block_streamer/gptoss.py:137-177).

    ``hidden [T, H]``, ``router_indices [T, k]``, ``routing_weights [T, k]``;
    packed experts in the checkpoint layout.  Returns ``out [T, H]`` in the
    dtype of ``hidden``; with ``save=True`` also ``(workspace, swiglu_grad)``
    for the input-gradient backward: ``swiglu_grad`` is bf16 ``[T*k, 2I]`` in
    expert-sorted row order, per activation column j the clamped SwiGLU's
    derivatives w.r.t. gate (column 2j) and up (2j+1) at the float32
    pre-activations, the clamp masks applied.  Activations enter the MFMA as bfloat16,
    except on ``path="mx"`` (two MXFP8 terms, see ``PATHS``).

    ``out_dtype`` (default: that of ``hidden``) is the dtype the combine
    writes, e.g. float32 to see the layer before its final rounding.

    ``noalloc=True`` runs the same kernels through
    ``bsa_moe_experts_fwd_noalloc``, whose workspace is the library's static
    per-GPU scratch (16 MiB: decode batches); only the output is allocated
    here.  Calls of it that overlap on one GPU race, and it cannot save for
    the backward (the next call overwrites the scratch).
    """
    if noalloc and save:
        raise ValueError("noalloc=True cannot save for the backward: the scratch is shared by every call")
    if hidden.dim() != 2:
        raise ValueError(f"hidden_states must be [tokens, hidden], got {tuple(hidden.shape)}")
    if router_indices.dim() != 2 or router_indices.shape[0] != hidden.shape[0]:
        raise ValueError("router_indices must be [tokens, top_k]")
    if tuple(routing_weights.shape) != tuple(router_indices.shape):
        raise ValueError("routing_weights must match router_indices in shape")
    T, H = hidden.shape
    k = router_indices.shape[1]
    E, I = _experts_dims(gate_up_blocks)
    layout = _check_packed(gate_up_blocks, gate_up_scales, E, 2 * I, H, "gate_up_proj")
    if _check_packed(down_blocks, down_scales, E, H, I, "down_proj") != layout:
        raise ValueError("gate_up and down blocks must be in the same layout")
    _check_bias(gate_up_bias, E, 2 * I, "gate_up_proj")
    _check_bias(down_bias, E, H, "down_proj")
    dev = _lib.require_gpu(hidden, router_indices, routing_weights, gate_up_blocks,
                           gate_up_scales, down_blocks, down_scales, gate_up_bias, down_bias)
    out_dtype = out_dtype or hidden.dtype
    out_code = _lib.dtype_code(out_dtype)
    x = hidden if hidden.dtype == torch.bfloat16 else hidden.to(torch.bfloat16)
    x = x.contiguous()
    idx = router_indices.to(torch.int64).contiguous()
    w = routing_weights.contiguous()
    w_code = _lib.dtype_code(w.dtype)
    bias_dtype = (gate_up_bias if gate_up_bias is not None else down_bias)
    bias_code = _lib.dtype_code(bias_dtype.dtype) if bias_dtype is not None else 0
    gub = gate_up_bias.to(bias_dtype.dtype).contiguous() if gate_up_bias is not None else None
    dnb = down_bias.to(bias_dtype.dtype).contiguous() if down_bias is not None else None
    gu_b, gu_s, dn_b, dn_s = (_as_u8(x) for x in (gate_up_blocks, gate_up_scales, down_blocks, down_scales))
    if layout == LAYOUT_KPAIR:  # the k-pair layout moves in 16-byte pieces only
        _require_kpair_aligned(gu_b, "gate_up_proj_blocks")
        _require_kpair_aligned(dn_b, "down_proj_blocks")
    out = torch.empty((T, H), dtype=out_dtype, device=dev)

    def ptr(t):
        return t.data_ptr() if t is not None else None

    common = (x.data_ptr(), T, H, I, E, k, idx.data_ptr(), w.data_ptr(), w_code, gu_b.data_ptr(),
              gu_s.data_ptr(), ptr(gub), dn_b.data_ptr(), dn_s.data_ptr(), ptr(dnb), bias_code,
              float(alpha), float(limit), out.data_ptr(), out_code)
    if noalloc:
        with torch.cuda.device(dev):
            _lib.call("bsa_moe_experts_fwd_noalloc", *common, None, PATHS[path], layout,
                      _lib.stream_handle(dev))
        return out
    ws_bytes = moe_workspace_bytes(T, H, I, E, k)
    ws = _aligned_bytes(ws_bytes, dev)
    save_grad = torch.empty((T * k, 2 * I), dtype=torch.bfloat16, device=dev) if save else None
    with torch.cuda.device(dev):
        _lib.call("bsa_moe_experts_fwd", *common, ws.data_ptr(), ws_bytes, ptr(save_grad), PATHS[path],
                  layout, _lib.stream_handle(dev))
    if save:
        return out, ws, save_grad
    return out


def _whole_forward_path(path: str, T: int, k: int, E: int, H: int, I: int, gu_b: Tensor, gu_s: Tensor,
                        dn_b: Tensor, dn_s: Tensor) -> int:
    """The path code the fused forward runs for ``path`` (the C library's
    rule for a whole forward): "auto" takes the MX kernels for prefill-sized
    batches (more than 16 rows per expert on average) when both projections
    can run them -- H and I multiples of 64, 16-byte aligned blocks, 4-byte
    aligned scales -- because its gate_up stage leaves split activations for
    its down stage.  (A forward saving for the backward keeps the bf16
    products; the stage runner never saves.)"""
    if path != "auto":
        return PATHS[path]
    ok = (T * k > 16 * E and H % 64 == 0 and I % 64 == 0 and gu_b.data_ptr() % 16 == 0
          and dn_b.data_ptr() % 16 == 0 and gu_s.data_ptr() % 4 == 0 and dn_s.data_ptr() % 4 == 0)
    return PATHS["mx"] if ok else PATHS["auto"]


class MoEStages:
    """The four forward stages of one MoE layer call, launched one by one.

    Used where the stages must be timed or reused separately (the benchmark
    brackets each with HIP events); ``moe_experts_forward`` runs the same
    four launches through one C call.
    """

    def __init__(self, hidden: Tensor, router_indices: Tensor, routing_weights: Tensor,
                 gate_up_blocks, gate_up_scales, gate_up_bias, down_blocks, down_scales,
                 down_bias, alpha: float = 1.702, limit: float = 7.0, path: str = "auto"):
        self.T, self.H = hidden.shape
        self.k = router_indices.shape[1]
        self.E, self.I = _experts_dims(gate_up_blocks)
        self.layout = _check_packed(gate_up_blocks, gate_up_scales, self.E, 2 * self.I, self.H, "gate_up_proj")
        if _check_packed(down_blocks, down_scales, self.E, self.H, self.I, "down_proj") != self.layout:
            raise ValueError("gate_up and down blocks must be in the same layout")
        _check_bias(gate_up_bias, self.E, 2 * self.I, "gate_up_proj")
        _check_bias(down_bias, self.E, self.H, "down_proj")
        if down_bias is not None and gate_up_bias is not None and down_bias.dtype != gate_up_bias.dtype:
            raise ValueError("MoEStages takes gate_up and down biases of one dtype")
        self.dev = _lib.require_gpu(hidden, router_indices, routing_weights, gate_up_blocks)
        if hidden.dtype != torch.bfloat16 or not hidden.is_contiguous():
            raise ValueError("MoEStages takes contiguous bfloat16 hidden states")
        self.hidden = hidden
        self.idx = router_indices.to(torch.int64).contiguous()
        self.w = routing_weights.contiguous()
        self.gu = (_as_u8(gate_up_blocks), _as_u8(gate_up_scales), gate_up_bias)
        self.dn = (_as_u8(down_blocks), _as_u8(down_scales), down_bias)
        self.bias_code = _lib.dtype_code(gate_up_bias.dtype) if gate_up_bias is not None else 0
        # the stage entry points see one projection each: the path of the
        # whole forward is resolved here, as the fused call resolves it
        self.alpha, self.limit = float(alpha), float(limit)
        self.path = _whole_forward_path(path, self.T, self.k, self.E, self.H, self.I, self.gu[0], self.gu[1],
                                        self.dn[0], self.dn[1])
        self.ws_bytes = moe_workspace_bytes(self.T, self.H, self.I, self.E, self.k)
        self.ws = _aligned_bytes(self.ws_bytes, self.dev)
        self.out = torch.empty((self.T, self.H), dtype=torch.bfloat16, device=self.dev)
        self.shape = (self.T, self.H, self.I, self.E, self.k)

    def _stream(self):
        return _lib.stream_handle(self.dev)

    def dispatch(self):
        _lib.call("bsa_moe_dispatch", self.idx.data_ptr(), *self.shape, self.ws.data_ptr(),
                  self.ws_bytes, self._stream())

    def gate_up(self):
        b, s, bias = self.gu
        _lib.call("bsa_moe_gate_up", self.hidden.data_ptr(), *self.shape, b.data_ptr(),
                  s.data_ptr(), bias.data_ptr() if bias is not None else None, self.bias_code,
                  self.alpha, self.limit, self.ws.data_ptr(), self.ws_bytes, None, self.path,
                  self.layout, self._stream())

    def down(self):
        b, s, bias = self.dn
        _lib.call("bsa_moe_down", *self.shape, b.data_ptr(), s.data_ptr(),
                  bias.data_ptr() if bias is not None else None, self.bias_code,
                  self.ws.data_ptr(), self.ws_bytes, self.path, self.layout, self._stream())

    def combine(self):
        _lib.call("bsa_moe_combine", self.idx.data_ptr(), self.w.data_ptr(),
                  _lib.dtype_code(self.w.dtype), *self.shape, self.ws.data_ptr(), self.ws_bytes,
                  self.out.data_ptr(), 0, self._stream())

    def run(self) -> Tensor:
        self.dispatch()
        self.gate_up()
        self.down()
        self.combine()
        return self.out


def moe_bwd_workspace_bytes(T: int, H: int, I: int, E: int, k: int) -> int:
    import ctypes
    out = ctypes.c_int64(0)
    _lib.call("bsa_moe_bwd_workspace_bytes", T, H, I, E, k, ctypes.byref(out))
    return out.value


def moe_experts_backward(grad_out: Tensor, hidden: Tensor, router_indices: Tensor,
                         routing_weights: Tensor, gate_up_blocks: Tensor, gate_up_scales: Tensor,
                         down_blocks: Tensor, down_scales: Tensor, workspace: Tensor,
                         swiglu_grad: Tensor, alpha: float = 1.702, limit: float = 7.0, *,
                         need_hidden: bool = True, need_weights: bool = True):
    """Input-gradient backward of ``moe_experts_forward(..., save=True)``.

    Returns ``(grad_hidden or None, grad_routing_weights or None)`` in the
    dtypes of ``hidden`` and ``routing_weights``.  Expert weights and biases
    get no gradient (frozen under LoRA, block_streamer/lora.py:138-148).
    """
    if hidden.dim() != 2:
        raise ValueError(f"hidden_states must be [tokens, hidden], got {tuple(hidden.shape)}")
    T, H = hidden.shape
    if tuple(grad_out.shape) != (T, H):
        raise ValueError(f"grad_out must be [{T}, {H}] like the hidden states, got {list(grad_out.shape)}")
    if router_indices.dim() != 2 or router_indices.shape[0] != T:
        raise ValueError("router_indices must be [tokens, top_k]")
    if tuple(routing_weights.shape) != tuple(router_indices.shape):
        raise ValueError("routing_weights must match router_indices in shape")
    k = router_indices.shape[1]
    E, I = _experts_dims(gate_up_blocks)
    layout = _check_packed(gate_up_blocks, gate_up_scales, E, 2 * I, H, "gate_up_proj")
    if _check_packed(down_blocks, down_scales, E, H, I, "down_proj") != layout:
        raise ValueError("gate_up and down blocks must be in the same layout")
    if swiglu_grad.dtype != torch.bfloat16 or tuple(swiglu_grad.shape) != (T * k, 2 * I):
        raise ValueError(f"swiglu_grad must be the forward's bfloat16 [{T * k}, {2 * I}] save, "
                         f"got {swiglu_grad.dtype} {list(swiglu_grad.shape)}")
    ws_need = moe_workspace_bytes(T, H, I, E, k)
    if workspace.dtype != torch.uint8 or workspace.numel() < ws_need:
        raise ValueError(f"workspace must be the forward's uint8 workspace of >= {ws_need} bytes")
    dev = _lib.require_gpu(grad_out, hidden, router_indices, routing_weights, workspace, swiglu_grad,
                           gate_up_blocks, gate_up_scales, down_blocks, down_scales)
    if T == 0:
        return (torch.zeros_like(hidden) if need_hidden else None,
                torch.zeros_like(routing_weights) if need_weights else None)
    g = grad_out.contiguous()
    g_code = _lib.dtype_code(g.dtype)
    idx = router_indices.to(torch.int64).contiguous()
    w = routing_weights.contiguous()
    # the backward kernels DMA the packed weights in 16- or 4-byte pieces
    # (staging-blob views are 8-byte aligned; the k-pair layout moves in
    # 16-byte pieces only) and the saved derivative factors in 16
    gub, gus, dnb, dns = (_as_u8(x) for x in (gate_up_blocks, gate_up_scales, down_blocks, down_scales))
    if layout == LAYOUT_KPAIR:
        _require_kpair_aligned(gub, "gate_up_proj_blocks")
        _require_kpair_aligned(dnb, "down_proj_blocks")
    else:
        gub, dnb = _aligned(gub, 4), _aligned(dnb, 4)
    gus, dns = _aligned(gus, 4), _aligned(dns, 4)
    fac = _aligned(swiglu_grad.contiguous(), 16)
    bwd_bytes = moe_bwd_workspace_bytes(T, H, I, E, k)
    bws = _aligned_bytes(bwd_bytes, dev)
    grad_h = torch.empty((T, H), dtype=hidden.dtype, device=dev) if need_hidden else None
    grad_w = torch.empty((T, k), dtype=torch.float32, device=dev) if need_weights else None
    with torch.cuda.device(dev):
        _lib.call("bsa_moe_experts_bwd", g.data_ptr(), g_code, T, H, I, E, k, idx.data_ptr(),
                  w.data_ptr(), _lib.dtype_code(w.dtype), gub.data_ptr(), gus.data_ptr(),
                  dnb.data_ptr(), dns.data_ptr(), float(alpha), float(limit),
                  workspace.data_ptr(), workspace.numel(), fac.data_ptr(), bws.data_ptr(),
                  bwd_bytes, grad_h.data_ptr() if grad_h is not None else None,
                  _lib.dtype_code(hidden.dtype),
                  grad_w.data_ptr() if grad_w is not None else None, layout, _lib.stream_handle(dev))
    if grad_w is not None:
        grad_w = grad_w.to(routing_weights.dtype)
    return grad_h, grad_w


def router_forward(hidden: Tensor, weight: Tensor, bias: Tensor | None, top_k: int):
    """GptOssTopKRouter.forward (TF/models/gpt_oss/modeling_gpt_oss.py:126-131).

    Returns ``(logits [T, E], scores [T, k], indices [T, k] int64)`` in the
    dtype of ``hidden`` (the module dtype).
    """
    if hidden.dim() != 2:
        raise ValueError(f"router input must be [tokens, hidden], got {tuple(hidden.shape)}")
    T, H = hidden.shape
    E = weight.shape[0]
    if tuple(weight.shape) != (E, H):
        raise ValueError(f"router weight must be [{E}, {H}], got {tuple(weight.shape)}")
    dev = _lib.require_gpu(hidden, weight, bias)
    dt = hidden.dtype
    code = _lib.dtype_code(dt)
    h = hidden.contiguous()
    w = weight.to(dt).contiguous()
    b = bias.to(dt).contiguous() if bias is not None else None
    logits = torch.empty((T, E), dtype=dt, device=dev)
    scores = torch.empty((T, top_k), dtype=dt, device=dev)
    idx = torch.empty((T, top_k), dtype=torch.int64, device=dev)
    with torch.cuda.device(dev):
        _lib.call("bsa_router_fwd", h.data_ptr(), code, T, H, E, top_k, w.data_ptr(),
                  b.data_ptr() if b is not None else None, logits.data_ptr(), scores.data_ptr(),
                  idx.data_ptr(), _lib.stream_handle(dev))
    return logits, scores, idx


def router_topk(logits: Tensor, top_k: int):
    """Top-k (descending, lower index first on ties) and softmax of given logits."""
    if logits.dim() != 2:
        raise ValueError("logits must be [tokens, experts]")
    T, E = logits.shape
    dev = _lib.require_gpu(logits)
    lg = logits.contiguous()
    scores = torch.empty((T, top_k), dtype=lg.dtype, device=dev)
    idx = torch.empty((T, top_k), dtype=torch.int64, device=dev)
    with torch.cuda.device(dev):
        _lib.call("bsa_router_topk", lg.data_ptr(), _lib.dtype_code(lg.dtype), T, E, top_k,
                  scores.data_ptr(), idx.data_ptr(), _lib.stream_handle(dev))
    return scores, idx


def _norm_args(x: Tensor, weight: Tensor):
    H = x.shape[-1]
    if weight.dim() != 1 or weight.shape[0] != H:
        raise ValueError(f"norm weight must be [{H}], got {tuple(weight.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"norm input dtype {x.dtype} is not bf16, f16 or f32")
    w = weight if weight.dtype in (torch.bfloat16, torch.float16, torch.float32) else weight.float()
    return H, x.numel() // H if H else 0, w.contiguous()


def rmsnorm_forward(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """GptOssRMSNorm.forward (TF/models/gpt_oss/modeling_gpt_oss.py:57-62) in
    one launch: ``dtype(float32(weight) * x32 * rsqrt(mean(x32^2) + eps))``
    over the last dimension, in the dtype of ``x``."""
    dev = _lib.require_gpu(x, weight)
    H, T, w = _norm_args(x, weight)
    xc = x.contiguous()
    out = torch.empty_like(xc)
    with torch.cuda.device(dev):
        _lib.call("bsa_rmsnorm_fwd", xc.data_ptr(), _lib.dtype_code(xc.dtype), T, H, w.data_ptr(),
                  _lib.dtype_code(w.dtype), float(eps), out.data_ptr(), _lib.stream_handle(dev))
    return out


def rmsnorm_backward(grad_out: Tensor, x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """Input gradient of ``rmsnorm_forward`` in the dtype of ``x``."""
    dev = _lib.require_gpu(grad_out, x, weight)
    H, T, w = _norm_args(x, weight)
    if grad_out.shape != x.shape:
        raise ValueError(f"grad_out shape {tuple(grad_out.shape)} != input shape {tuple(x.shape)}")
    xc = x.contiguous()
    g = grad_out.to(xc.dtype).contiguous()
    dx = torch.empty_like(xc)
    with torch.cuda.device(dev):
        _lib.call("bsa_rmsnorm_bwd", g.data_ptr(), xc.data_ptr(), _lib.dtype_code(xc.dtype), T, H,
                  w.data_ptr(), _lib.dtype_code(w.dtype), float(eps), dx.data_ptr(), _lib.stream_handle(dev))
    return dx
