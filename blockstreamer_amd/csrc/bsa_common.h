// Shared definitions for the blockstreamer_amd HIP library (gfx950 / CDNA4).
//
// Error model: every extern "C" entry point returns an int status
// (BSA_OK, BSA_EINVAL for bad shapes/dtypes/alignment, BSA_EHIP for a HIP
// launch or runtime error) and leaves a thread-local message readable through
// bsa_last_error().  Entry points never synchronise the stream and never
// allocate: the caller passes every buffer, workspace included.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/bsamd.h"

namespace bsa {

void set_error(const char* fmt, ...);
void clear_error();

#define BSA_REQUIRE(cond, ...)                 \
  do {                                         \
    if (!(cond)) {                             \
      ::bsa::set_error(__VA_ARGS__);           \
      return BSA_EINVAL;                       \
    }                                          \
  } while (0)

#define BSA_LAUNCH_CHECK(what)                                               \
  do {                                                                       \
    hipError_t _e = hipGetLastError();                                       \
    if (_e != hipSuccess) {                                                  \
      ::bsa::set_error("%s: %s", (what), hipGetErrorString(_e));             \
      return BSA_EHIP;                                                       \
    }                                                                        \
  } while (0)

typedef uint16_t bf16_bits;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
// Pointer type of the LDS operand of __builtin_amdgcn_global_load_lds.
typedef __attribute__((address_space(3))) void lds_void;

// ---------------------------------------------------------------------------
// MXFP4 element decode.
//
// An element is an OCP MX E2M1 code (bit 3 sign, 2 exponent bits, 1 mantissa
// bit: magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6) times 2^(s-127) for the block's
// E8M0 byte s, evaluated the way the reference does it: a float32 product of
// the value and float32 pow(2, s-127) (2^128 = inf, so s = 255 gives +-inf for
// nonzero codes and NaN for +-0 codes), rounded once to the output type.  All
// finite products below are exact in bfloat16 and float32.
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32, round to nearest even
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// Exact float32 bit pattern of code * 2^(s-127), built with integer
// arithmetic so that it does not depend on the float denormal mode.
__device__ __forceinline__ uint32_t mx_fp32_bits(uint32_t code, uint32_t s) {
  const uint32_t sign = (code & 8u) << 28;
  const uint32_t m = code & 7u;
  if (s == 255u) return m ? (sign | 0x7F800000u) : 0x7FC00000u;
  if (m == 0u) return sign;
  // m == 1 is the E2M1 subnormal 0.5 = 1.0 * 2^-1; m >= 2 is
  // (1 + (m & 1) / 2) * 2^((m >> 1) - 1).
  const int eoff = (m == 1u) ? -1 : (int)(m >> 1) - 1;
  const uint32_t mant = (m == 1u) ? 0u : (m & 1u);
  const int be = (int)s + eoff;  // biased exponent of the product
  if (be >= 255) return sign | 0x7F800000u;
  if (be >= 1) return sign | ((uint32_t)be << 23) | (mant << 22);
  // be in {0, -1}: a float32 subnormal, (1 + mant/2) * 2^(be-127)
  return sign | ((2u + mant) << (21 + be));
}

// Two codes of one packed byte -> bfloat16x2 (low nibble in the low half),
// exact path.
__device__ __forceinline__ uint32_t mx_byte_to_bf16x2_exact(uint32_t byte, uint32_t s) {
  const uint32_t lo = mx_fp32_bits(byte & 15u, s) >> 16;
  const uint32_t hi = mx_fp32_bits((byte >> 4) & 15u, s) >> 16;
  return lo | (hi << 16);
}

// float16 element: torch.ldexp on a float16 tensor rounds pow(2, s-127) to
// float16 first, so the scale is inf for s >= 143 (2^16) and 0 for s <= 102
// (2^-25 rounds to 0); in between the float32 product is rounded once.
__device__ __forceinline__ uint32_t mx_f16_bits(uint32_t code, uint32_t s) {
  const uint32_t sign = (code & 8u) << 12;
  if (s >= 143u) return (code & 7u) ? (sign | 0x7C00u) : 0x7E00u;
  if (s <= 102u) return sign;
  return f32_to_f16_bits(__uint_as_float(mx_fp32_bits(code, s)));
}

__device__ __forceinline__ uint32_t mx_byte_to_f16x2(uint32_t byte, uint32_t s) {
  return mx_f16_bits(byte & 15u, s) | (mx_f16_bits((byte >> 4) & 15u, s) << 16);
}

// Scale bytes for which the gfx950 hardware converter is used.  Measured
// over every (byte, scale) pair on an MI355X, v_cvt_scalef32_pk_bf16_fp4
// reproduces the reference bit for bit for scale bytes 0..254 (subnormal and
// overflowing products included); 255, the E8M0 NaN code, gives NaN for
// every code where the reference gives +-inf, so it takes the integer path.
__device__ __forceinline__ bool mx_scale_hw_ok(uint32_t s) { return s != 255u; }

// The converter reads the E8M0 scale from the exponent field of a float32.
__device__ __forceinline__ float mx_scale_f32(uint32_t s) { return __uint_as_float(s << 23); }

// Byte `sel` of `dword` -> bfloat16x2 with the gfx950 converter
// (v_cvt_scalef32_pk_bf16_fp4).  Only valid for mx_scale_hw_ok(s).
template <int SEL>
__device__ __forceinline__ uint32_t mx_byte_to_bf16x2_hw(uint32_t dword, float scale) {
  bf16x2_t v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(dword, scale, SEL);
  return __builtin_bit_cast(uint32_t, v);
}

// Four packed bytes (8 codes) -> 4 dwords of bfloat16x2, in code order.
__device__ __forceinline__ void mx_dword_to_bf16x8(uint32_t dword, uint32_t s, bool hw,
                                                   uint32_t out[4]) {
  if (hw) {
    const float sf = mx_scale_f32(s);
    out[0] = mx_byte_to_bf16x2_hw<0>(dword, sf);
    out[1] = mx_byte_to_bf16x2_hw<1>(dword, sf);
    out[2] = mx_byte_to_bf16x2_hw<2>(dword, sf);
    out[3] = mx_byte_to_bf16x2_hw<3>(dword, sf);
  } else {
    out[0] = mx_byte_to_bf16x2_exact(dword & 0xFFu, s);
    out[1] = mx_byte_to_bf16x2_exact((dword >> 8) & 0xFFu, s);
    out[2] = mx_byte_to_bf16x2_exact((dword >> 16) & 0xFFu, s);
    out[3] = mx_byte_to_bf16x2_exact(dword >> 24, s);
  }
}

__device__ __forceinline__ uint32_t pack_lo16(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);  // a.lo | b.lo << 16
}
__device__ __forceinline__ uint32_t pack_hi16(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);  // a.hi | b.hi << 16
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}

// float32 -> bfloat16 bits, round to nearest even, NaN -> 0x7FC0.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// bf16 bits of f by gfx950's v_cvt_pk_bf16_f32 (round to nearest even, one
// instruction; a NaN stays a quiet NaN of the same sign where
// f32_to_bf16_bits returns the positive canonical one).
__device__ __forceinline__ uint32_t bf16_bits_hw(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// The value of lane ^ 1 / lane ^ 2 of the same quad: a DPP quad_perm operand
// of one VALU move, not a round trip through the LDS crossbar (ds_bpermute)
// as __shfl_xor compiles to.  Every lane of the quad must be active.
__device__ __forceinline__ int quad_xor1(int x) { return __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ int quad_xor2(int x) { return __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false); }
__device__ __forceinline__ float quad_xor1(float x) { return __int_as_float(quad_xor1(__float_as_int(x))); }
__device__ __forceinline__ float quad_xor2(float x) { return __int_as_float(quad_xor2(__float_as_int(x))); }

// Two floats -> packed bf16 by one v_cvt_pk_bf16_f32 (the same bits as
// pack_bf16x2 for every non-NaN input).
__device__ __forceinline__ uint32_t pack_bf16x2_hw(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}


// Byte offset of 16-byte group g of packed row n from the start of row n0 of
// the tensor (n0 a multiple of 16, rows counted across experts), G groups per
// row.  Checkpoint layout [rows][G][16]; k-pair layout [rows/16][G/2][16][2]
// [16]: 16-row bands, inside a band the groups two by two, each pair holding
// the band's 16 rows.  A band occupies the same bytes in both layouts.
__device__ __forceinline__ int64_t bq_off(int kp, int64_t n, int g, int G) {
  return kp ? ((((n >> 4) * (G >> 1) + (g >> 1)) * 32 + (n & 15) * 2 + (g & 1)) * 16) : ((n * G + g) * 16);
}

// ---------------------------------------------------------------------------
// OCP MXFP8 (E4M3 elements, one E8M0 scale per 32) arithmetic shared by the
// activation quantisers.
// ---------------------------------------------------------------------------
// E4M3 code of v (RNE, saturating); |v| < 2^9 by construction of the scale.
__device__ __forceinline__ uint32_t e4m3_rne_sat(float v) {
  const uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
  const float a = fabsf(v);
  uint32_t c;
  if (a >= 448.f) {
    c = 0x7Eu;
  } else if (a < 0.015625f) {  // below 2^-6: subnormal steps of 2^-9
    c = (uint32_t)rintf(a * 512.f);
  } else {
    // round the float32 mantissa to 3 bits (ties to even), carrying into the
    // exponent; then rebias the exponent from 127 to 7
    const uint32_t b = __float_as_uint(a);
    c = ((b + 0x7FFFFu + ((b >> 20) & 1u)) >> 20) - (120u << 3);
    c = c > 0x7Eu ? 0x7Eu : c;
  }
  return sign | c;
}

// 2^-X as a float for X in [-127, 127] (2^-127 is a float32 subnormal).
__device__ __forceinline__ float pow2_neg(int X) {
  return X == 127 ? __uint_as_float(0x00400000u) : __uint_as_float((uint32_t)(127 - X) << 23);
}

// Shared exponent X of a block with largest magnitude amax (finite, >= 0):
// ceil(log2(amax / 448)), i.e. floor(log2(amax)) - 8, plus 1 when amax's
// significand exceeds 1.75; clamped to [-127, 127]; -127 for amax = 0.
__device__ __forceinline__ int mx_shared_exp(float amax) {
  if (!(amax > 0.f)) return -127;
  const uint32_t ab = __float_as_uint(amax);
  const int e = (ab >> 23) ? (int)(ab >> 23) - 127 : (31 - (int)__clz(ab & 0x7FFFFFu)) - 149;
  // a float32 subnormal amax clamps to -127 either way
  return min(max(e - 8 + ((ab & 0x7FFFFFu) > 0x600000u ? 1 : 0), -127), 127);
}

// Value of a finite E4M3 code (bias 7; subnormals m * 2^-9).
__device__ __forceinline__ float e4m3_value(uint32_t c) {
  const uint32_t e = (c >> 3) & 15u, m = c & 7u;
  const float mag = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : (float)m * 0.001953125f;
  return (c & 0x80u) ? -mag : mag;
}

// Two-term MXFP8 split of the 8 elements v of one lane, four consecutive
// lanes holding a 32-element block: hi = E4M3(v / 2^X), lo =
// E4M3((v - hi * 2^X) / 2^max(X-4, -127)) (round to nearest even); X the
// block's shared exponent.  Every lane of the four must call it (the block
// maximum goes through two lane shuffles).  Returns the scale byte (255 for
// a block holding inf or NaN: then hi = 0x7F with the sign, lo = 0); hi and
// lo get the 8 codes of the lane, element i in byte i % 4 of word i / 4.
__device__ __forceinline__ uint32_t mx_split8(const float (&v)[8], uint32_t (&hi)[2], uint32_t (&lo)[2]) {
  float amax = 0.f;
  int bad = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float a = fabsf(v[i]);
    bad |= !(a <= 3.402823466e38f);  // inf or NaN
    amax = fmaxf(amax, a);
  }
  amax = fmaxf(amax, quad_xor1(amax));
  amax = fmaxf(amax, quad_xor2(amax));
  bad |= quad_xor1(bad);
  bad |= quad_xor2(bad);
  const int X = mx_shared_exp(amax);
  hi[0] = hi[1] = lo[0] = lo[1] = 0;
  if (!bad && X >= -122) {
    // both scales 2^X and 2^(X-4) are normal floats: gfx950's scaled
    // converters divide by the scale and round to nearest even
    typedef short v2s __attribute__((ext_vector_type(2)));
    typedef float v2f __attribute__((ext_vector_type(2)));
    const float s = __uint_as_float((uint32_t)(X + 127) << 23);
    const float sl = __uint_as_float((uint32_t)(X + 123) << 23);
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      v2s q = {0, 0};
      q = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(q, v[4 * d], v[4 * d + 1], s, false);
      q = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(q, v[4 * d + 2], v[4 * d + 3], s, true);
      const uint32_t w = __builtin_bit_cast(uint32_t, q);
      hi[d] = w;
      const v2f b0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)w, s, false);
      const v2f b1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)w, s, true);
      v2s r = {0, 0};
      r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, v[4 * d] - b0[0], v[4 * d + 1] - b0[1], sl, false);
      r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, v[4 * d + 2] - b1[0], v[4 * d + 3] - b1[1], sl, true);
      lo[d] = __builtin_bit_cast(uint32_t, r);
    }
  } else {
    // tiny blocks (a scale below 2^-122 would be a float subnormal) and
    // blocks holding inf or NaN: the same rounding in integer arithmetic
    const int Xl = max(X - 4, -127);
    const float inv = pow2_neg(X);
    const float inv_l = pow2_neg(Xl);
    const float sc = __uint_as_float(X > -127 ? (uint32_t)(X + 127) << 23 : 0x00400000u);  // 2^X
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t ch = e4m3_rne_sat(v[i] * inv);
      const float res = v[i] - e4m3_value(ch) * sc;
      const uint32_t cl = e4m3_rne_sat(res * inv_l);
      hi[i >> 2] |= (bad ? ((__float_as_uint(v[i]) >> 24 & 0x80u) | 0x7Fu) : ch) << (8 * (i & 3));
      lo[i >> 2] |= (bad ? 0u : cl) << (8 * (i & 3));
    }
  }
  return bad ? 255u : (uint32_t)(X + 127);
}

// Where the two-term MXFP8 split of an activation matrix goes: the 128 code
// bytes (64 hi, 64 lo) of 64-element k-tile t of row r at
// r * q_row + t * q_kt, block g's scale byte at r * s_row + (g / 2) * s_kt +
// g % 2.  Row-major: q_row = 2K, q_kt = 128, s_row = scale row stride, s_kt
// = 2.  K-tile-major (the MX GEMM's operand): q_row = 128, q_kt = 128 *
// rows, s_row = 4, s_kt = 4 * rows (two scale bytes and two spare per row).
struct SplitLayout {
  int64_t q_row, q_kt, s_row, s_kt;
};

// Activation / weight element types accepted by the kernels.
enum DType : int { DT_BF16 = BSA_DTYPE_BF16, DT_F16 = BSA_DTYPE_F16, DT_F32 = BSA_DTYPE_F32 };

}  // namespace bsa
