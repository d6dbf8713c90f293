// MXFP8 (OCP MX, E4M3 elements with one E8M0 scale per 32) quantisation of
// activations, the A operand of the native block-scaled MFMA path
// (v_mfma_scale_f32_32x32x64_f8f6f4: MXFP8 activations x MXFP4 weights).
//
// No reference counterpart: BlockStreamer multiplies bf16/fp32 activations
// by dequantised weights (block_streamer/gptoss.py:45-75).  This path trades
// that for the gfx950 MXFP4 matrix cores.  Two kernels: mx_quant_kernel, one
// MXFP8 term per element (the conversion below; 2.7 % relative L2 error on
// N(0,1) rows, too coarse for float32 parity), and mx_split_kernel, the two
// terms hi + lo the MX prefill kernels multiply (exact for bf16 elements
// above ~2^-14 of their block's maximum; described at the kernel).
//
// Conversion, per 32-element block of a row (OCP Microscaling Formats v1.0,
// section 6.3, with the shared exponent taken one higher where the
// specification's floor(log2(amax)) - 8 would make the block's largest
// elements saturate):
//   amax  = max |x|;  shared exponent X = ceil(log2(amax / 448)), i.e.
//           floor(log2(amax)) - 8, plus 1 when amax's significand exceeds
//           1.75 (448 = 1.75 * 2^8 is the largest E4M3 value); clamped to
//           [-127, 127]; X = -127 for an all-zero block; the scale byte is
//           X + 127, or 255 (NaN) when the block holds an inf or NaN
//   q_i   = E4M3(x_i / 2^X), round to nearest even (|x_i / 2^X| <= 448, so
//           nothing saturates; the kernel still clamps to 448 defensively);
//           NaN blocks store 0x7F codes.
// On N(0,1) activations this gives 2.7 % relative L2 error instead of 2.9 %
// with the saturating exponent.
#include "bsa_common.h"

namespace bsa {

// Four lanes per 32-element block, eight elements per lane.
template <int IN>
__global__ __launch_bounds__(256) void mx_quant_kernel(const void* __restrict__ x, int64_t ldx,
                                                       int64_t nblk, int G, uint8_t* __restrict__ q,
                                                       int64_t ldq, uint8_t* __restrict__ s,
                                                       int64_t lds) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const bool ok = (gid >> 2) < nblk;
  const int64_t blk = ok ? (gid >> 2) : nblk - 1;
  const int part = threadIdx.x & 3;
  const int64_t r = blk / G;
  const int g = (int)(blk - r * G);
  const int64_t off = r * ldx + g * 32 + part * 8;
  float v[8];
  if constexpr (IN == DT_BF16) {
    const u32x4_t w = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(x) + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  } else if constexpr (IN == DT_F32) {
    const float* p = static_cast<const float*>(x) + off;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = p[i];
  } else {
    const uint16_t* p = static_cast<const uint16_t*>(x) + off;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)__builtin_bit_cast(_Float16, p[i]);
  }
  float amax = 0.f;
  int bad = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float a = fabsf(v[i]);
    bad |= !(a <= 3.402823466e38f);  // inf or NaN
    amax = fmaxf(amax, a);
  }
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  amax = fmaxf(amax, __shfl_xor(amax, 2));
  bad |= __shfl_xor(bad, 1);
  bad |= __shfl_xor(bad, 2);
  const int X = mx_shared_exp(amax);
  const float inv = pow2_neg(X);
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t c = e4m3_rne_sat(v[i] * inv);
    if (bad) c = (__float_as_uint(v[i]) >> 24 & 0x80u) | 0x7Fu;
    if (i < 4)
      lo |= c << (8 * i);
    else
      hi |= c << (8 * (i - 4));
  }
  if (ok) {
    *reinterpret_cast<uint2*>(q + r * ldq + g * 32 + part * 8) = make_uint2(lo, hi);
    if (part == 0) s[r * lds + g] = (uint8_t)(bad ? 255 : X + 127);
  }
}

// Two-term MXFP8 split (the A operand of the MX prefill kernel).  Each
// 32-element block x gets the MXFP8 scale X of mx_quant_kernel and
//   hi = E4M3(x / 2^X)                      (the codes mx_quant_kernel writes)
//   lo = E4M3((x - hi * 2^X) / 2^Xl),       Xl = max(X - 4, -127),
// both round to nearest even.  x / 2^X is at most 448, where E4M3 steps are
// at most 32, so the residual is at most 16 * 2^X and lo at most 256.  A
// bfloat16 element keeps 8 significant bits, its residual at most 4, so
// hi * 2^X + lo * 2^Xl equals x exactly for every element above about 2^-14
// of the block maximum (E4M3 keeps 4 bits down to 2^-6).  The residual is
// exact in float32 (x minus x rounded to 4 bits).  Blocks with an inf or NaN
// get scale byte 255, hi codes 0x7F (NaN, sign kept) and lo codes 0.
// Output: the codes of 64-element k-tile t of row r at q + r * L.q_row +
// t * L.q_kt, 64 hi bytes then 64 lo bytes; block g's scale byte (that of X;
// lo's is max(byte - 4, 0)) at s + r * L.s_row + (g / 2) * L.s_kt + g % 2.
// With dest (the dispatch's pair_pos), input row t is split once and written
// to output rows dest[t * topk + j] for its topk slots j (-1: dropped), so
// each token's row is read and split once whatever its top-k.
template <int IN>
__global__ __launch_bounds__(256) void mx_split_kernel(const void* __restrict__ x, int64_t ldx,
                                                       const int* __restrict__ dest, int topk, int64_t nblk,
                                                       int G, uint8_t* __restrict__ q, uint8_t* __restrict__ s,
                                                       SplitLayout L) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const bool ok = (gid >> 2) < nblk;
  const int64_t blk = ok ? (gid >> 2) : nblk - 1;
  const int part = threadIdx.x & 3;
  const int64_t r = blk / G;
  const int g = (int)(blk - r * G);
  const int64_t off = r * ldx + g * 32 + part * 8;
  float v[8];
  if constexpr (IN == DT_BF16) {
    const u32x4_t w = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(x) + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  } else if constexpr (IN == DT_F32) {
    const float* p = static_cast<const float*>(x) + off;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = p[i];
  } else {
    const uint16_t* p = static_cast<const uint16_t*>(x) + off;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)__builtin_bit_cast(_Float16, p[i]);
  }
  uint32_t h[2], l[2];
  const uint32_t sbyte = mx_split8(v, h, l);
  if (!ok) return;
  for (int j = 0; j < (dest ? topk : 1); ++j) {
    const int64_t o = dest ? (int64_t)dest[r * topk + j] : r;
    if (o < 0) continue;
    uint8_t* row = q + o * L.q_row + (g >> 1) * L.q_kt + (g & 1) * 32 + part * 8;
    *reinterpret_cast<uint2*>(row) = make_uint2(h[0], h[1]);
    *reinterpret_cast<uint2*>(row + 64) = make_uint2(l[0], l[1]);
    if (part == 0) s[o * L.s_row + (g >> 1) * L.s_kt + (g & 1)] = (uint8_t)sbyte;
  }
}

// Quantise R rows of K (K % 32 == 0) elements, row stride ldx elements, into
// q [R][ldq] E4M3 codes and s [R][lds] scale bytes.
int launch_quant_mxfp8(const void* x, int in_dtype, int64_t R, int64_t K, int64_t ldx, uint8_t* q,
                       int64_t ldq, uint8_t* s, int64_t lds, hipStream_t st) {
  if (R == 0) return BSA_OK;
  const int G = (int)(K / 32);
  const int64_t nblk = R * G;
  const int64_t grid = (nblk * 4 + 255) / 256;
  if (grid > INT32_MAX) {
    set_error("mxfp8 quantisation: too many blocks");
    return BSA_EINVAL;
  }
  if (in_dtype == DT_BF16)
    hipLaunchKernelGGL(mx_quant_kernel<DT_BF16>, dim3((unsigned)grid), dim3(256), 0, st, x, ldx, nblk,
                       G, q, ldq, s, lds);
  else if (in_dtype == DT_F32)
    hipLaunchKernelGGL(mx_quant_kernel<DT_F32>, dim3((unsigned)grid), dim3(256), 0, st, x, ldx, nblk,
                       G, q, ldq, s, lds);
  else
    hipLaunchKernelGGL(mx_quant_kernel<DT_F16>, dim3((unsigned)grid), dim3(256), 0, st, x, ldx, nblk,
                       G, q, ldq, s, lds);
  BSA_LAUNCH_CHECK("mxfp8 quantisation launch");
  return BSA_OK;
}

// Two-term split of R rows of K (K % 64 == 0) elements (input row stride
// ldx; row r reads row_map[r] / topk when row_map is given) into the layout L.
int launch_quant_mxfp8_split(const void* x, int in_dtype, int64_t R, int64_t K, int64_t ldx, const int* dest,
                             int topk, uint8_t* q, uint8_t* s, SplitLayout L, hipStream_t st) {
  if (R == 0) return BSA_OK;
  const int G = (int)(K / 32);
  const int64_t nblk = R * G;
  const int64_t grid = (nblk * 4 + 255) / 256;
  if (grid > INT32_MAX) {
    set_error("mxfp8 split: too many blocks");
    return BSA_EINVAL;
  }
  if (in_dtype == DT_BF16)
    hipLaunchKernelGGL(mx_split_kernel<DT_BF16>, dim3((unsigned)grid), dim3(256), 0, st, x, ldx, dest, topk,
                       nblk, G, q, s, L);
  else if (in_dtype == DT_F32)
    hipLaunchKernelGGL(mx_split_kernel<DT_F32>, dim3((unsigned)grid), dim3(256), 0, st, x, ldx, dest, topk,
                       nblk, G, q, s, L);
  else
    hipLaunchKernelGGL(mx_split_kernel<DT_F16>, dim3((unsigned)grid), dim3(256), 0, st, x, ldx, dest, topk,
                       nblk, G, q, s, L);
  BSA_LAUNCH_CHECK("mxfp8 split launch");
  return BSA_OK;
}

}  // namespace bsa

using namespace bsa;

extern "C" int bsa_quant_mxfp8_split(const void* x, int dtype, int64_t R, int64_t K, void* q, void* scales,
                                     int64_t scale_ld, void* stream) {
  clear_error();
  BSA_REQUIRE(R >= 0 && K > 0 && K % 64 == 0, "mxfp8 split: needs K %% 64 == 0 (K=%lld)", (long long)K);
  BSA_REQUIRE(scale_ld >= K / 32, "mxfp8 split: scale row stride %lld < K/32", (long long)scale_ld);
  BSA_REQUIRE(dtype == DT_BF16 || dtype == DT_F16 || dtype == DT_F32, "mxfp8 split: bad dtype %d", dtype);
  if (R == 0) return BSA_OK;
  BSA_REQUIRE(x && q && scales, "mxfp8 split: null pointer");
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 8 == 0,
              "mxfp8 split: x must be 16-byte and q 8-byte aligned");
  // row-major: row r's k-tiles one after another, its scale bytes in order
  const SplitLayout L{2 * K, 128, scale_ld, 2};
  return launch_quant_mxfp8_split(x, dtype, R, K, K, nullptr, 1, static_cast<uint8_t*>(q),
                                  static_cast<uint8_t*>(scales), L, static_cast<hipStream_t>(stream));
}

extern "C" int bsa_quant_mxfp8(const void* x, int dtype, int64_t R, int64_t K, void* q, void* scales,
                               int64_t scale_ld, void* stream) {
  clear_error();
  BSA_REQUIRE(R >= 0 && K > 0 && K % 32 == 0, "mxfp8 quantisation: needs K %% 32 == 0 (K=%lld)",
              (long long)K);
  BSA_REQUIRE(scale_ld >= K / 32, "mxfp8 quantisation: scale row stride %lld < K/32",
              (long long)scale_ld);
  BSA_REQUIRE(dtype == DT_BF16 || dtype == DT_F16 || dtype == DT_F32,
              "mxfp8 quantisation: bad dtype %d", dtype);
  if (R == 0) return BSA_OK;
  BSA_REQUIRE(x && q && scales, "mxfp8 quantisation: null pointer");
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 8 == 0,
              "mxfp8 quantisation: x must be 16-byte and q 8-byte aligned");
  return launch_quant_mxfp8(x, dtype, R, K, K, static_cast<uint8_t*>(q), K,
                            static_cast<uint8_t*>(scales), scale_ld, static_cast<hipStream_t>(stream));
}
