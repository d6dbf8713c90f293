/*
 * TEST INFRASTRUCTURE ONLY -- the oracle.  Nothing in the product links this
 * file; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * load it, and only to check results against.
 *
 * CPU restatement of the MXFP4 expert-weight dequantisation that BlockStreamer
 * reaches through block_streamer/gptoss.py:24-42 (dequantize_expert), which
 * calls transformers 5.15.0 integrations/mxfp4.py:257-313
 * (_convert_moe_packed_tensors).  That function, for packed bytes
 * b = blocks[..., r, g, j] and exponent byte s = scales[..., r, g]:
 *
 *   lut        = FP4_VALUES in the output dtype            (mxfp4.py:29-46, :275)
 *   sub[2j]    = lut[b & 0x0F]                             (mxfp4.py:296-299)
 *   sub[2j+1]  = lut[b >> 4]                               (mxfp4.py:301-304)
 *   sub        = ldexp(sub, s - 127)                       (mxfp4.py:271, :307)
 *   out        = reshape(..., G*32).transpose(1, 2)        (mxfp4.py:311-313)
 *
 * torch.ldexp(x, e) on a tensor x of a floating dtype D evaluates the power
 * of two in D as well (observed with torch 2.10: ldexp(float16(0.5), 16) is
 * inf and ldexp(float16(6), -25) is 0), then multiplies in float32 and rounds
 * once to D.  So the scale is pow(2, s-127) rounded to D: for bf16 and f32 it
 * is exact with 2^128 = inf; for f16 it is inf for s >= 143 and 0 for
 * s <= 102.  This file follows exactly that arithmetic with IEEE float32
 * operations (no integer bit tricks), so it is an independent restatement of
 * the GPU kernel, which builds the bits.
 *
 * Output layout: out[e][32*g + 2*j + h][r], i.e. [E, G*32, R] row-major, the
 * dense [K, N] orientation returned by dequantize_expert.
 *
 * out_dtype: 0 = bfloat16 (uint16 bits), 1 = float16 (uint16 bits),
 *            2 = float32.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* transformers integrations/mxfp4.py:29-46 */
static const float FP4_VALUES[16] = {
    +0.0f, +0.5f, +1.0f, +1.5f, +2.0f, +3.0f, +4.0f, +6.0f,
    -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f,
};

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* float32 -> bfloat16, round to nearest even; NaN -> 0x7FC0 (the c10
 * scalar conversion, c10/util/BFloat16.h round_to_nearest_even). */
static uint16_t f32_to_bf16_rne(float f) {
    if (isnan(f)) return 0x7FC0u;
    uint32_t u = f32_bits(f);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}

/* float32 -> IEEE binary16, round to nearest even, with subnormals,
 * overflow to inf and NaN -> 0x7E00. */
static uint16_t f32_to_f16_rne(float f) {
    uint32_t u = f32_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    if (isnan(f)) return 0x7E00u;
    float a = fabsf(f);
    if (isinf(a)) return sign | 0x7C00u;
    if (a >= 65520.0f) return sign | 0x7C00u; /* rounds to inf */
    if (a < 6.103515625e-05f) {
        /* subnormal range: value / 2^-24, rounded to nearest even */
        float q = a * 16777216.0f; /* exact: power-of-two scaling */
        float r = nearbyintf(q);   /* default rounding mode: ties to even */
        return sign | (uint16_t)r;
    }
    int e;
    float m = frexpf(a, &e); /* a = m * 2^e, m in [0.5, 1) */
    /* 11 significant bits: scale mantissa to [1024, 2048) */
    float q = nearbyintf(m * 2048.0f);
    if (q >= 2048.0f) {
        q = 1024.0f;
        e += 1;
    }
    int be = e - 1 + 15;
    if (be >= 31) return sign | 0x7C00u;
    return sign | (uint16_t)(be << 10) | (uint16_t)((uint32_t)q - 1024u);
}

static float f16_bits_to_f32(uint16_t h) {
    const int sign = (h >> 15) & 1;
    const int ex = (h >> 10) & 31;
    const int man = h & 1023;
    float v;
    if (ex == 0) v = ldexpf((float)man, -24);
    else if (ex == 31) v = man ? NAN : INFINITY;
    else v = ldexpf((float)(man + 1024), ex - 25);
    return sign ? -v : v;
}

/* x rounded to the output dtype and widened back to float32 */
static float round_to_dtype(float x, int out_dtype) {
    if (out_dtype == 0) return bits_f32((uint32_t)f32_to_bf16_rne(x) << 16);
    if (out_dtype == 1) return f16_bits_to_f32(f32_to_f16_rne(x));
    return x;
}

static float pow2_f32(int e) {
    /* pow(2.0, e) evaluated in float32: exact powers of two, float32
     * subnormals below 2^-126, inf at and above 2^128. */
    return (float)ldexp(1.0, e) /* double is exact here; the cast rounds */;
}

void oracle_dequant_mxfp4(const uint8_t *blocks, const uint8_t *scales,
                          int64_t E, int64_t R, int64_t G, int out_dtype,
                          void *out) {
    const int64_t K = G * 32;
    for (int64_t e = 0; e < E; ++e) {
        for (int64_t r = 0; r < R; ++r) {
            for (int64_t g = 0; g < G; ++g) {
                const int64_t rg = (e * R + r) * G + g;
                const float scale =
                    round_to_dtype(pow2_f32((int)scales[rg] - 127), out_dtype);
                const uint8_t *b = blocks + rg * 16;
                for (int j = 0; j < 16; ++j) {
                    for (int h = 0; h < 2; ++h) {
                        const int code = h ? (b[j] >> 4) : (b[j] & 0x0F);
                        const float v = FP4_VALUES[code] * scale;
                        const int64_t k = 32 * g + 2 * j + h;
                        const int64_t idx = (e * K + k) * R + r;
                        if (out_dtype == 0)
                            ((uint16_t *)out)[idx] = f32_to_bf16_rne(v);
                        else if (out_dtype == 1)
                            ((uint16_t *)out)[idx] = f32_to_f16_rne(v);
                        else
                            ((float *)out)[idx] = v;
                    }
                }
            }
        }
    }
}

/* One element of the map, for the exhaustive (byte, scale) table tests. */
uint32_t oracle_dequant_one(int code, int scale, int out_dtype) {
    const float v = FP4_VALUES[code & 15] *
                    round_to_dtype(pow2_f32(scale - 127), out_dtype);
    if (out_dtype == 0) return f32_to_bf16_rne(v);
    if (out_dtype == 1) return f32_to_f16_rne(v);
    return f32_bits(v);
}

/* Exposed for the oracle's own unit tests of its conversions. */
uint16_t oracle_f32_to_bf16(float f) { return f32_to_bf16_rne(f); }
uint16_t oracle_f32_to_f16(float f) { return f32_to_f16_rne(f); }
float oracle_bits_to_f32(uint32_t u) { return bits_f32(u); }
