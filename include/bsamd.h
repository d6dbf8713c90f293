/*
 * blockstreamer_amd -- C ABI of the MI355X (gfx950) gpt-oss MoE expert path.
 *
 * Every entry point takes plain device pointers, element counts and a HIP
 * stream (hipStream_t passed as void*; NULL = the legacy default stream), is
 * asynchronous on that stream, never synchronises and never allocates: the
 * caller owns every buffer, workspace included (bsa_moe_experts_fwd_noalloc
 * alone takes its workspace from a static array of the library instead).
 * The return value is a
 * status code; on failure bsa_last_error() returns a thread-local message.
 *
 * Tensors are dense row-major.  Packed MXFP4 weights keep the gpt-oss
 * checkpoint layout: blocks uint8 [E, R, G, 16] (byte j of group g of row r
 * holds codes for columns 32g+2j (low nibble) and 32g+2j+1 (high nibble)),
 * scales uint8 [E, R, G] (E8M0, value 2^(s-127)).
 */
#ifndef BSAMD_H_
#define BSAMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define BSA_OK 0
#define BSA_EINVAL 1 /* bad shape, dtype, alignment or argument */
#define BSA_EHIP 2   /* HIP runtime / launch error */

/* element types */
#define BSA_DTYPE_BF16 0
#define BSA_DTYPE_F16 1
#define BSA_DTYPE_F32 2

/*
 * Layouts of the packed MXFP4 blocks (scales always keep the checkpoint
 * layout [E, R, G]).
 *
 * BSA_LAYOUT_CHECKPOINT  uint8 [E, R, G, 16]: the checkpoint's own layout
 *                        (gate_up_proj_blocks / down_proj_blocks).
 * BSA_LAYOUT_KPAIR       uint8 [E, R/16, G/2, 16, 2, 16]: group g of row r at
 *                        [e][r / 16][g / 2][r % 16][g % 2] -- 16-row bands,
 *                        inside a band the groups two by two, each pair
 *                        holding the band's 16 rows (512 contiguous bytes).
 *                        A band occupies the same bytes in both layouts.  An
 *                        on-disk shard format for the prefill kernels, whose
 *                        weight tiles become 512-byte runs instead of 32-byte
 *                        ones; no counterpart in the reference (its shards
 *                        store the checkpoint layout, shards.py:148-165).
 *                        Needs R % 16 == 0, G even, and 16-byte aligned
 *                        blocks and scales.
 */
#define BSA_LAYOUT_CHECKPOINT 0
#define BSA_LAYOUT_KPAIR 1

/* Thread-local message describing the last failure of this thread. */
const char *bsa_last_error(void);

/* ABI version of this library (major * 100 + minor).  The major number
 * changes whenever an existing signature or the meaning of an argument
 * changes: 2 inserted the blocks_layout argument before the stream in
 * bsa_moe_experts_fwd, bsa_moe_gate_up, bsa_moe_down and
 * bsa_moe_experts_bwd; 3 made the forward's save for the backward the
 * SwiGLU's bf16 derivative factors (save_swiglu_grad) instead of float32
 * pre-activations.  The minor number counts added entry points (the
 * no-allocation forward, the MXFP8 split and the packed matmul came with
 * major 2; minor 1 of major 3 added the attention entry points, minor 2 the
 * key-split forward and its workspace query).  A binding
 * checks the major number before its first call. */
#define BSA_VERSION_MAJOR 3
int bsa_version(void);

/*
 * MXFP4 -> dense dequantisation.
 *
 * Replaces transformers integrations/mxfp4.py:316-338
 * (convert_moe_packed_tensors -> _convert_moe_packed_tensors :257-313) as
 * called by block_streamer/gptoss.py:41 (dequantize_expert, :24-42).
 *
 *   blocks  uint8 [E, R, G, 16]     scales uint8 [E, R, G]
 *   out     out_dtype [E, G*32, R]  (the transposed [K, N] orientation)
 *
 * out[e][32g + 2j + h][r] = FP4[nibble h of blocks[e][r][g][j]] * 2^(s - 127)
 * with s = scales[e][r][g], evaluated as torch.ldexp does: the power of two
 * rounded to out_dtype (bf16, f16 or f32; 2^128 = inf, and for f16 also
 * 2^(>=16) = inf and 2^(<=-25) = 0), times the code in float32, rounded once
 * to out_dtype.  Bit-exact with the reference; NaN (0 * inf) is returned as
 * the canonical quiet NaN.  Any pointer alignment is accepted; 8-byte
 * aligned blocks with a 16-byte aligned out and R % 8 == 0 take the
 * vectorised path.
 */
int bsa_dequant_mxfp4(const void *blocks, const void *scales, void *out,
                      int out_dtype, int64_t E, int64_t R, int64_t G,
                      void *stream);

/*
 * As bsa_dequant_mxfp4, with the element decoder chosen explicitly:
 * mode 0 = automatic (what bsa_dequant_mxfp4 does), 1 = integer decoder
 * only, 2 = gfx950 hardware converter wherever the layout allows it (used
 * by the tests that validate the hardware converter over every (byte,
 * scale) pair).  No reference counterpart; a test and tuning hook.
 */
int bsa_dequant_mxfp4_mode(const void *blocks, const void *scales, void *out,
                           int out_dtype, int64_t E, int64_t R, int64_t G,
                           int mode, void *stream);

/*
 * As bsa_dequant_mxfp4_mode, for blocks in either layout (blocks_layout
 * BSA_LAYOUT_CHECKPOINT or BSA_LAYOUT_KPAIR); the output is the same.  The
 * k-pair layout also needs a 16-byte aligned out.
 */
int bsa_dequant_mxfp4_layout(const void *blocks, const void *scales,
                             void *out, int out_dtype, int64_t E, int64_t R,
                             int64_t G, int mode, int blocks_layout,
                             void *stream);

/*
 * Repack checkpoint-layout blocks uint8 [E, R, G, 16] into the k-pair layout
 * (bsa_mxfp4_to_kpair) and back (bsa_mxfp4_from_kpair): a permutation of
 * 16-byte groups, bit for bit.  R % 16 == 0, G even, both buffers 16-byte
 * aligned and distinct.  The conversion a shard writer runs once, before
 * writing (block_streamer/shards.py:167-176 writes tensors as they are).
 */
int bsa_mxfp4_to_kpair(const void *blocks, void *out, int64_t E, int64_t R,
                       int64_t G, void *stream);
int bsa_mxfp4_from_kpair(const void *blocks, void *out, int64_t E, int64_t R,
                         int64_t G, void *stream);

/*
 * Bytes of workspace bsa_moe_experts_fwd needs for T tokens, hidden H,
 * intermediate I, E experts and top-k k (written to *bytes).  No reference
 * counterpart: the reference allocates per expert inside its loop.
 */
int bsa_moe_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E,
                            int64_t k, int64_t *bytes);

/*
 * Fused MoE expert forward.
 *
 * Replaces block_streamer/gptoss.py:137-177 (MXFP4Experts.forward: dispatch
 * :143-154, per-expert mxfp4_matmul + bias :158-165 and :167-174, clamped
 * SwiGLU :130-135 / :166, routing-weight scale and index_add_ :175-176).
 *
 *   hidden          bf16 [T, H] (16-byte aligned)
 *   router_indices  int64 [T, k]; entries outside [0, E) are dropped
 *   routing_weights weight_dtype [T, k]
 *   gate_up_blocks  uint8 [E, 2I, H/32, 16], gate_up_scales uint8 [E, 2I, H/32]
 *   gate_up_bias    bias_dtype [E, 2I] (may be NULL)
 *   down_blocks     uint8 [E, H, I/32, 16],  down_scales uint8 [E, H, I/32]
 *   down_bias       bias_dtype [E, H] (may be NULL)
 *   out             out_dtype [T, H]
 *   workspace       >= bsa_moe_workspace_bytes(...) bytes, 256-byte aligned;
 *                   holds the expert-sorted dispatch and intermediates, and is
 *                   what a later backward reads
 *   save_swiglu_grad optional bf16 [T*k, 2I] (16-byte aligned), written for
 *                   the backward in expert-sorted row order: per activation
 *                   column j, d act/d gate at 2j and d act/d up at 2j+1 of
 *                   the clamped SwiGLU at the float32 pre-activations, the
 *                   clamp masks applied (torch autograd's derivative of
 *                   gptoss.py:130-135; the reference's autograd keeps the
 *                   bf16 gate_up, the same size)
 *   path            0 = automatic (path 3 when more than 16 rows per expert
 *                   on average, both projections can take it and
 *                   save_swiglu_grad is NULL, else 1 up to 16 rows per expert and
 *                   2 beyond), 1 = weight-streaming kernel, 2 = tiled kernel,
 *                   3 = native block-scaled MX kernel (activations split into
 *                   two MXFP8 terms by bsa_quant_mxfp8_split's rule, then two
 *                   v_mfma_scale_f32_32x32x64_f8f6f4 per 64-element k-step on
 *                   the packed MXFP4 weights as they are; needs H and I
 *                   multiples of 64, 16-byte aligned blocks, 4-byte aligned
 *                   scales; not bit-compatible with paths 0-2, whose products
 *                   it equals up to the matrix cores' accumulation order: the
 *                   two terms hold every bf16 activation exactly unless it is
 *                   below 2^-14 of its 32-element block's maximum)
 *   blocks_layout   layout of gate_up_blocks and down_blocks:
 *                   BSA_LAYOUT_CHECKPOINT or BSA_LAYOUT_KPAIR (the results
 *                   are the same bit for bit)
 *
 * Gate and up columns are interleaved (gate = even, up = odd), alpha and
 * limit parameterise the clamped SwiGLU.  Each token's k contributions are
 * summed in ascending expert order in float32 and rounded once.
 */
int bsa_moe_experts_fwd(
    const void *hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
    const int64_t *router_indices, const void *routing_weights,
    int weight_dtype, const void *gate_up_blocks, const void *gate_up_scales,
    const void *gate_up_bias, const void *down_blocks, const void *down_scales,
    const void *down_bias, int bias_dtype, float alpha, float limit, void *out,
    int out_dtype, void *workspace, int64_t workspace_bytes,
    void *save_swiglu_grad, int path, int blocks_layout, void *stream);

/*
 * bsa_moe_experts_fwd without the workspace arguments: the same kernels and
 * the same results bit for bit, with the workspace taken from a static
 * device array of the library (BSA_NOALLOC_SCRATCH_BYTES, one copy per GPU,
 * held until the process ends).  Nothing is allocated: no hipMalloc, no
 * hipFree, no allocating library call.
 *
 * No counterpart in the reference.  It is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, and
 * harnesses that forbid allocation.
 *
 * Limit: the shape's bsa_moe_workspace_bytes must be at most
 * BSA_NOALLOC_SCRATCH_BYTES (16 MiB: up to 226 tokens at top-4 with
 * H = I = 2880, i.e. decode batches); larger shapes return BSA_EINVAL.
 * Every call on one GPU shares that GPU's array, so calls that overlap on a
 * GPU (concurrent streams, threads) race; order them.  The array's contents
 * after a call are those of the last call; no call relies on them.
 * save_swiglu_grad must be null (BSA_EINVAL otherwise): the backward also
 * reads the forward's workspace, which here the next call overwrites, so
 * this entry point serves inference only.
 */
#define BSA_NOALLOC_SCRATCH_BYTES (16ll << 20)
int bsa_moe_experts_fwd_noalloc(
    const void *hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
    const int64_t *router_indices, const void *routing_weights,
    int weight_dtype, const void *gate_up_blocks, const void *gate_up_scales,
    const void *gate_up_bias, const void *down_blocks, const void *down_scales,
    const void *down_bias, int bias_dtype, float alpha, float limit, void *out,
    int out_dtype, void *save_swiglu_grad, int path, int blocks_layout,
    void *stream);

/*
 * The four stages bsa_moe_experts_fwd runs, callable one by one (same
 * arguments and workspace; run in this order on one stream).
 *
 * bsa_moe_dispatch   replaces gptoss.py:143-154 (one_hot / nonzero / where):
 *                    expert-sorted rows, per-expert offsets and the tile list,
 *                    built on the device.
 * bsa_moe_gate_up    replaces gptoss.py:158-166: gate_up GEMM + bias + clamped
 *                    SwiGLU into the workspace's [T*k, I] activations.
 * bsa_moe_down       replaces gptoss.py:167-174: down GEMM + bias into the
 *                    workspace's float32 [T*k, H] rows.
 * bsa_moe_combine    replaces gptoss.py:175-176: routing-weight scale and the
 *                    per-token sum (ascending expert order) into out.
 * blocks_layout is that of the blocks argument, as for bsa_moe_experts_fwd.
 * path is as for bsa_moe_experts_fwd, except that 0 never selects path 3
 * here (a stage sees one projection only); a caller that wants path 3 for a
 * layer passes 3 to both bsa_moe_gate_up and bsa_moe_down (the gate_up stage
 * of path 3 leaves split activations that only path 3's down stage reads).
 */
int bsa_moe_dispatch(const int64_t *router_indices, int64_t T, int64_t H,
                     int64_t I, int64_t E, int64_t k, void *workspace,
                     int64_t workspace_bytes, void *stream);
int bsa_moe_gate_up(const void *hidden, int64_t T, int64_t H, int64_t I,
                    int64_t E, int64_t k, const void *blocks,
                    const void *scales, const void *bias, int bias_dtype,
                    float alpha, float limit, void *workspace,
                    int64_t workspace_bytes, void *save_swiglu_grad, int path,
                    int blocks_layout, void *stream);
int bsa_moe_down(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                 const void *blocks, const void *scales, const void *bias,
                 int bias_dtype, void *workspace, int64_t workspace_bytes,
                 int path, int blocks_layout, void *stream);
int bsa_moe_combine(const int64_t *router_indices, const void *routing_weights,
                    int weight_dtype, int64_t T, int64_t H, int64_t I,
                    int64_t E, int64_t k, void *workspace,
                    int64_t workspace_bytes, void *out, int out_dtype,
                    void *stream);

/*
 * Router forward.
 *
 * Replaces transformers models/gpt_oss/modeling_gpt_oss.py:126-131
 * (GptOssTopKRouter.forward, called at :143):
 *   logits  dtype [T, E] = hidden [T, H] @ weight[E, H]^T + bias[E]
 *   indices int64 [T, k] = top-k of logits, descending (equal logits: lower
 *           index first; -0 == +0)
 *   scores  dtype [T, k] = softmax of the k selected logits (float32, rounded)
 * dtype is the module dtype of hidden, weight, bias (bias may be NULL).
 * E <= 256, k <= 16.
 */
int bsa_router_fwd(const void *hidden, int dtype, int64_t T, int64_t H,
                   int64_t E, int64_t k, const void *weight, const void *bias,
                   void *logits, void *scores, int64_t *indices, void *stream);

/*
 * Top-k and softmax of given logits [T, E] (modeling_gpt_oss.py:128-129):
 * the same selection and softmax as bsa_router_fwd.
 */
int bsa_router_topk(const void *logits, int dtype, int64_t T, int64_t E,
                    int64_t k, void *scores, int64_t *indices, void *stream);

/*
 * OCP MXFP8 quantisation (E4M3 elements, one E8M0 scale per 32 consecutive
 * elements of a row): the activation format of path 3 above.  No reference
 * counterpart (the reference multiplies unquantised activations,
 * block_streamer/gptoss.py:45-75).
 *
 *   x       dtype [R, K] (K % 32 == 0, 16-byte aligned)
 *   q       uint8 [R, K] E4M3 codes
 *   scales  uint8 [R, scale_ld] (scale_ld >= K/32)
 *
 * Per block: X = ceil(log2(max |x| / 448)) clamped to [-127, 127] (-127 for
 * an all-zero block; 448 is the largest E4M3 value, so nothing saturates),
 * scale byte X + 127 (255 when the block holds inf or NaN), q = E4M3(x / 2^X)
 * rounded to nearest even.
 */
int bsa_quant_mxfp8(const void *x, int dtype, int64_t R, int64_t K, void *q,
                    void *scales, int64_t scale_ld, void *stream);

/*
 * Two-term MXFP8 split: the activation format of path 3 above.  No
 * reference counterpart (the reference multiplies unquantised activations,
 * block_streamer/gptoss.py:45-75; two terms reproduce a bfloat16 element
 * exactly unless it is below about 2^-14 of its block's maximum).
 *
 *   x       dtype [R, K] (K % 64 == 0, 16-byte aligned)
 *   q       uint8 [R, 2K]: per 64-element k-tile t, bytes 128t .. 128t+63
 *           hold the hi codes of elements 64t .. 64t+63 and the next 64
 *           bytes their lo codes
 *   scales  uint8 [R, scale_ld] (scale_ld >= K/32): hi's scale bytes, as
 *           bsa_quant_mxfp8 writes them
 *
 * hi = the codes bsa_quant_mxfp8 writes (X, its scale); lo = E4M3 of the
 * residual x - hi * 2^X divided by 2^Xl, Xl = max(X - 4, -127), rounded to
 * nearest even (lo's scale byte is max(byte - 4, 0)).  Blocks holding inf or
 * NaN: scale byte 255, hi codes 0x7F with the element's sign, lo codes 0.
 */
int bsa_quant_mxfp8_split(const void *x, int dtype, int64_t R, int64_t K,
                          void *q, void *scales, int64_t scale_ld,
                          void *stream);

/*
 * One expert's packed matmul.  Replaces block_streamer/gptoss.py:45-75
 * (_MXFP4Matmul / mxfp4_matmul: x @ dequantize_expert(blocks, scales) and
 * its input gradient g @ W^T), with no dense weight: W = the [K, N] matrix
 * of gptoss.py:41 from blocks uint8 [N, K/32, 16] (or the k-pair layout) and
 * scales uint8 [N, K/32].
 *
 *   transpose 0: out [M, N] = x [M, K] @ W
 *   transpose 1: out [M, K] = x [M, N] @ W^T   (needs N % 64 == 0)
 *
 * x is bf16, f16 or f32 (x_dtype); out is out_dtype.  The activation operand
 * enters the matrix cores as bf16: f16 x is split into 2 bf16 terms and f32
 * x into 3 (their sum is x exactly), one pass per term; the float32 partial
 * products are summed in term order and rounded once to out_dtype, so an f32
 * x gets float32 accuracy (a different summation order from a library
 * GEMM's).  K % 32 == 0; blocks 8-byte and scales 4-byte aligned; workspace
 * >= bsa_mxfp4_matmul_workspace_bytes(...), 256-byte aligned.
 */
int bsa_mxfp4_matmul_workspace_bytes(int64_t M, int64_t K, int64_t N,
                                     int x_dtype, int transpose,
                                     int64_t *bytes);
int bsa_mxfp4_matmul(const void *x, int x_dtype, int64_t M, int64_t K,
                     int64_t N, const void *blocks, const void *scales,
                     int blocks_layout, int transpose, void *out,
                     int out_dtype, void *workspace, int64_t workspace_bytes,
                     void *stream);

/*
 * Bytes of the extra workspace bsa_moe_experts_bwd needs (the per-row
 * gradients: weighted output gradient, gate_up gradient, input gradient).
 * The weights are read packed; no dense copy is made.
 */
int bsa_moe_bwd_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E,
                                int64_t k, int64_t *bytes);

/*
 * Input-gradient backward of bsa_moe_experts_fwd (the LoRA training path,
 * where expert weights and biases are frozen).
 *
 * Replaces the autograd of block_streamer/gptoss.py:137-177:
 * _MXFP4Matmul.backward (:64-71, grad @ W^T re-dequantising from the packed
 * tensors) for both projections, the backward of the clamped SwiGLU
 * (:130-135) and of the routing-weight product and index_add_ (:175-176).
 *
 *   grad_out        grad_dtype [T, H]
 *   workspace       the forward's workspace, unchanged since that call
 *   save_swiglu_grad the forward's bf16 [T*k, 2I] derivative factors
 *   bwd_workspace   >= bsa_moe_bwd_workspace_bytes(...) bytes, 256-aligned
 *   grad_hidden     grad_hidden_dtype [T, H], or NULL to skip
 *   grad_weights    float32 [T, k] gradient of routing_weights, or NULL
 *
 * H must be a multiple of 64.  The packed blocks and scales must be 4-byte
 * aligned (16-byte aligned ones move in 16-byte DMA pieces, others in 4-byte
 * pieces) and save_swiglu_grad 16-byte aligned; otherwise BSA_EINVAL.  Dropped (token, slot) pairs get a zero
 * routing-weight gradient.  blocks_layout is that of both blocks tensors.
 */
int bsa_moe_experts_bwd(
    const void *grad_out, int grad_dtype, int64_t T, int64_t H, int64_t I,
    int64_t E, int64_t k, const int64_t *router_indices,
    const void *routing_weights, int weight_dtype, const void *gate_up_blocks,
    const void *gate_up_scales, const void *down_blocks,
    const void *down_scales, float alpha, float limit, void *workspace,
    int64_t workspace_bytes, const void *save_swiglu_grad, void *bwd_workspace,
    int64_t bwd_workspace_bytes, void *grad_hidden, int grad_hidden_dtype,
    float *grad_weights, int blocks_layout, void *stream);

/*
 * RMSNorm of a decoder layer, in one launch: the post-attention norm that
 * feeds the router and the experts (and any other GptOssRMSNorm).
 *
 * Replaces transformers models/gpt_oss/modeling_gpt_oss.py:57-62
 * (GptOssRMSNorm.forward; the post-attention call is at :373), in its
 * operation order:
 *   x32 = float32(x); r = 1 / sqrt(sum(x32^2) / H + eps)
 *   out dtype [T, H] = dtype(float32(weight) * (x32 * r))
 *   x       dtype [T, H]
 *   weight  weight_dtype [H] (transformers keeps this module in float32 when
 *           loading a checkpoint, modeling_gpt_oss.py:398)
 * The sum runs in a fixed order, so the result is reproducible; it differs
 * from torch's by float32 rounding of the sum only.  Any T >= 0, H >= 1.
 */
int bsa_rmsnorm_fwd(const void *x, int dtype, int64_t T, int64_t H,
                    const void *weight, int weight_dtype, float eps,
                    void *out, void *stream);

/*
 * Input gradient of bsa_rmsnorm_fwd (what autograd computes for
 * modeling_gpt_oss.py:57-62 with respect to hidden_states), rounded once:
 *   g = float32(weight) * float32(grad_out)
 *   grad_x dtype [T, H] = dtype(r * g - x32 * (r^3 * sum(g * x32) / H))
 * The weight gradient is not computed (the LoRA path keeps it frozen).
 */
int bsa_rmsnorm_bwd(const void *grad_out, const void *x, int dtype, int64_t T,
                    int64_t H, const void *weight, int weight_dtype,
                    float eps, void *grad_x, void *stream);

/*
 * Attention core of the gpt-oss decoder layer (grouped-query attention with a
 * per-head sink logit).  Replaces eager_attention_forward of transformers
 * 5.15.0 models/gpt_oss/modeling_gpt_oss.py:235-264 as GptOssAttention.forward
 * (:295-336) calls it; the streaming runner reaches it through the decoder
 * layer (block_streamer/runners.py:327-335).
 *   out[b, t, h] = sum_j p[t, j] v[b, j, h / G]   (G = Hq / Hkv)
 *   p[t, :]      = softmax([q[b,t,h] . k[b,j,h/G] * scaling (visible j), sinks[h]])[:Tk]
 * q [B, Tq, Hq, 64], k and v [B, Tk, Hkv, 64], out [B, Tq, Hq, 64]: bf16,
 * addressed through element strides (batch, sequence, head), each a multiple
 * of 8, the head dimension contiguous, base pointers 16-byte aligned.
 * sinks: float32 [Hq], or null for no sink.  Masks: causal = 0 shows every
 * key (what the eager path does with attention_mask = None); causal = 1 shows
 * key j to query t when j <= Tk - Tq + t, and window > 0 also requires
 * Tk - Tq + t - j < window.  lse (optional, float32 [B, Hq, Tq]) receives
 * log2 of each row's softmax denominator (sink included) in units of
 * scaling * log2(e) times the dot products: what bsa_attention_bwd needs.
 * Float32 accumulation; probabilities rounded to bf16 for the value product.
 */
int bsa_attention_fwd(const void *q, const int64_t *q_strides, const void *k,
                      const int64_t *k_strides, const void *v,
                      const int64_t *v_strides, const float *sinks, int64_t B,
                      int64_t Tq, int64_t Tk, int64_t Hq, int64_t Hkv,
                      int64_t head_dim, int causal, int64_t window,
                      float scaling, void *out, const int64_t *out_strides,
                      float *lse, void *stream);

/*
 * Workspace bytes bsa_attention_fwd_split needs for a shape (0: the shape is
 * not split and the workspace may be null).  Splitting is chosen from the
 * shape alone: when the (128-row block, key head, batch) grid has fewer than
 * about 512 workgroups -- decoding, or short prompts over a long cache -- and
 * a row block sees at least 512 keys, the keys of each row block are split
 * over up to 64 workgroups of at least two 64-key tiles each.  Replaces no reference interface: the eager path
 * (modeling_gpt_oss.py:235-264) has no such knob.
 */
int64_t bsa_attention_split_workspace_bytes(int64_t B, int64_t Tq, int64_t Tk,
                                            int64_t Hq, int64_t Hkv, int causal,
                                            int64_t window);

/*
 * bsa_attention_fwd for short query grids (the same arguments and meaning,
 * modeling_gpt_oss.py:235-264): each workgroup takes a contiguous share of a
 * row block's keys and writes its rows' unnormalised float32 sums and
 * (running maximum, sum) to the workspace (>= the query above, 256-byte
 * aligned), and a second launch merges the shares in a fixed order
 * (deterministic).  Shapes that are not split run bsa_attention_fwd's single
 * launch.  The sum order differs from the single launch, so the results agree
 * with it to float rounding, not bit for bit.
 */
int bsa_attention_fwd_split(const void *q, const int64_t *q_strides,
                            const void *k, const int64_t *k_strides,
                            const void *v, const int64_t *v_strides,
                            const float *sinks, int64_t B, int64_t Tq,
                            int64_t Tk, int64_t Hq, int64_t Hkv,
                            int64_t head_dim, int causal, int64_t window,
                            float scaling, void *out,
                            const int64_t *out_strides, float *lse,
                            void *workspace, int64_t workspace_bytes,
                            void *stream);

/*
 * Gradients of bsa_attention_fwd (what autograd computes through
 * eager_attention_forward, modeling_gpt_oss.py:235-264), from its output and
 * lse:  p = 2^(scaling log2(e) q.k - lse),  D[t] = grad_out[t] . out[t],
 *   grad_q = scaling sum_j p (dP - D) k,  grad_k = scaling sum_t p (dP - D) q,
 *   grad_v = sum_t p grad_out,  with dP[t, j] = grad_out[t] . v[j].
 * grad_out and out [B, Tq, Hq, 64] and q, k, v as for the forward (strides
 * per tensor); grad_q [B, Tq, Hq, 64], grad_k and grad_v [B, Tk, Hkv, 64]
 * contiguous bf16; row_stats float32 [B, Hkv, Tq * G, 2] (G = Hq / Hkv)
 * receives (lse, D) of row R = t * G + i, query t of head G * hk + i, from
 * which the sinks' gradient is -sum_t 2^(sink log2(e) - lse) D.  Two
 * launches, no atomics (results are deterministic).
 */
int bsa_attention_bwd(const void *grad_out, const int64_t *grad_strides,
                      const void *q, const int64_t *q_strides, const void *k,
                      const int64_t *k_strides, const void *v,
                      const int64_t *v_strides, const void *out,
                      const int64_t *out_strides, const float *lse, int64_t B,
                      int64_t Tq, int64_t Tk, int64_t Hq, int64_t Hkv,
                      int64_t head_dim, int causal, int64_t window,
                      float scaling, void *grad_q, void *grad_k, void *grad_v,
                      float *row_stats, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* BSAMD_H_ */
