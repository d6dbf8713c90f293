/*
 * blockstreamer_amd -- C ABI of the MI355X (gfx950) gpt-oss MoE expert path.
 *
 * Every entry point takes plain device pointers, element counts and a HIP
 * stream (hipStream_t passed as void*; NULL = the legacy default stream), is
 * asynchronous on that stream, never synchronises and never allocates: the
 * caller owns every buffer, workspace included.  The return value is a
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

/* Thread-local message describing the last failure of this thread. */
const char *bsa_last_error(void);

/* ABI version of this library (major * 100 + minor). */
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

#ifdef __cplusplus
}
#endif

#endif /* BSAMD_H_ */
