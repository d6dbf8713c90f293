// MXFP4 -> dense dequantisation.
//
// Replaces transformers integrations/mxfp4.py:257-313
// (_convert_moe_packed_tensors), reached from block_streamer/gptoss.py:41.
// The reference builds int32 index temporaries, gathers a LUT twice, scales
// in place with ldexp and then transposes with a full copy; here one pass
// reads each packed byte once and writes each output element once.
//
// Vectorised path: a workgroup owns 64 consecutive packed rows r of one
// expert and 32 of their groups, one 8-group tile per wave, and exits (short
// workgroups measured faster than ones walking all G groups).  Each lane
// decodes 8 consecutive rows of one group (8 x 16-byte loads; for a fixed row
// the 8 lanes of a row-group read 128 contiguous bytes), then transposes in
// registers so that for each of the group's 32 output rows k it stores the 8
// adjacent columns r..r+7 as one 16-byte store (for a fixed k, 8 lanes write
// 128 contiguous bytes).  Everything is HBM-bound: 2.53 bytes of traffic per
// bf16 output element.  Each scale byte is read by the one lane that decodes
// its 32 elements, straight from memory: a lane owns whole groups, so an LDS
// broadcast would have no second reader.
#include <algorithm>

#include "bsa_common.h"

namespace bsa {

constexpr int DQ_ROWG = 8;             // row-groups of 8 rows per wave
constexpr int DQ_GPW = 64 / DQ_ROWG;   // groups per wave
constexpr int DQ_ROWS = 8 * DQ_ROWG;   // rows per workgroup (64)
constexpr int DQ_GPB = 4 * DQ_GPW;     // groups per workgroup (32): one group tile per wave

template <int OUT>
__device__ __forceinline__ void dq_store8(void* out, size_t elem_off, const uint32_t v2[4]) {
  // v2 holds 8 16-bit values (columns r..r+7 of one output row): bfloat16
  // for bf16 and f32 outputs (every f32 result is exact in bf16), float16
  // for f16 outputs.
  if constexpr (OUT == DT_F32) {
    u32x4_t a = {v2[0] << 16, v2[0] & 0xFFFF0000u, v2[1] << 16, v2[1] & 0xFFFF0000u};
    u32x4_t b = {v2[2] << 16, v2[2] & 0xFFFF0000u, v2[3] << 16, v2[3] & 0xFFFF0000u};
    u32x4_t* p = reinterpret_cast<u32x4_t*>(static_cast<float*>(out) + elem_off);
    __builtin_nontemporal_store(a, p);
    __builtin_nontemporal_store(b, p + 1);
  } else {
    u32x4_t v = {v2[0], v2[1], v2[2], v2[3]};
    // streaming output, written once and not read back here: non-temporal
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(out) + elem_off));
  }
}

template <int OUT, bool HW>
__device__ __forceinline__ uint32_t dq_decode_byte(uint32_t d, int b, uint32_t s) {
  const uint32_t byte = (d >> (8 * b)) & 0xFFu;
  if constexpr (OUT == DT_F16) {
    return mx_byte_to_f16x2(byte, s);
  } else if constexpr (HW) {
    return mx_byte_to_bf16x2_hw<0>(byte, mx_scale_f32(s));
  } else {
    return mx_byte_to_bf16x2_exact(byte, s);
  }
}

template <int OUT, bool HW>
__device__ __forceinline__ void dq_decode_store(const u32x4_t (&pk)[8], const uint32_t (&s)[8],
                                                void* out, size_t out_base, int R) {
  // out_base = element offset of (k = 32g, r) for this lane's first row.
  // One packed byte column (codes 2j, 2j+1 of the 8 rows) at a time, so that
  // only 8 decoded words are live next to the packed bytes.
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      uint32_t c[8];  // c[row] = bf16x2 of codes (2j, 2j+1), j = 4q + b
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = dq_decode_byte<OUT, HW>(pk[i][q], b, s[i]);
      const int k = 2 * (4 * q + b);
      uint32_t ev[4], od[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        ev[p] = pack_lo16(c[2 * p], c[2 * p + 1]);
        od[p] = pack_hi16(c[2 * p], c[2 * p + 1]);
      }
      dq_store8<OUT>(out, out_base + (size_t)k * R, ev);
      dq_store8<OUT>(out, out_base + (size_t)(k + 1) * R, od);
    }
  }
}

// The packed bytes and scales of group g for this lane's 8 rows.
template <bool ALIGN16>
__device__ __forceinline__ void dq_load(const uint8_t* __restrict__ blocks, const uint8_t* __restrict__ scales,
                                        size_t row0, int g, int G, int kp, u32x4_t (&pk)[8], uint32_t (&s)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint8_t* p = blocks + bq_off(kp, (int64_t)(row0 + i), g, G);
    if constexpr (ALIGN16) {
      pk[i] = *reinterpret_cast<const u32x4_t*>(p);
    } else {
      const uint2 a = *reinterpret_cast<const uint2*>(p);
      const uint2 b = *reinterpret_cast<const uint2*>(p + 8);
      pk[i] = u32x4_t{a.x, a.y, b.x, b.y};
    }
    s[i] = scales[(row0 + i) * G + g];
  }
}

template <int OUT, bool ALIGN16>
__global__ __launch_bounds__(256) void dequant_vec_kernel(const uint8_t* __restrict__ blocks,
                                                          const uint8_t* __restrict__ scales,
                                                          void* __restrict__ out, int R, int G,
                                                          int row_tiles, int mode, int kp) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int gchunks = (G + DQ_GPB - 1) / DQ_GPB;
  const int ert = blockIdx.x / gchunks;
  const int gc = blockIdx.x - ert * gchunks;
  const int e = ert / row_tiles;
  const int rt = ert - e * row_tiles;
  const int r = rt * DQ_ROWS + 8 * (lane % DQ_ROWG);
  const int g = gc * DQ_GPB + wave * DQ_GPW + lane / DQ_ROWG;
  if (r >= R || g >= G) return;  // R % 8 == 0, so a lane owns either 8 valid rows or none
  const size_t row0 = (size_t)e * R + r;
  u32x4_t pk[8];
  uint32_t s[8];
  dq_load<ALIGN16>(blocks, scales, row0, g, G, kp, pk, s);
  bool in_range = true;
#pragma unroll
  for (int i = 0; i < 8; ++i) in_range = in_range && mx_scale_hw_ok(s[i]);
  // one decoder per wave: lanes that returned above count as in range
  const bool hw = (mode == 2) || (mode == 0 && __all(in_range));
  const size_t out_base = ((size_t)e * G * 32 + (size_t)32 * g) * R + r;
  if (hw && OUT != DT_F16)
    dq_decode_store<OUT, true>(pk, s, out, out_base, R);
  else
    dq_decode_store<OUT, false>(pk, s, out, out_base, R);
}

// Fallback for any shape or alignment: one thread per packed byte.
template <int OUT>
__global__ __launch_bounds__(256) void dequant_generic_kernel(const uint8_t* __restrict__ blocks,
                                                              const uint8_t* __restrict__ scales,
                                                              void* __restrict__ out, int64_t E,
                                                              int64_t R, int64_t G) {
  const int64_t n = E * R * G * 16;
  const int64_t K = G * 32;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t rg = i >> 4;
    const int j = (int)(i & 15);
    const int64_t g = rg % G;
    const int64_t er = rg / G;
    const int64_t r = er % R;
    const int64_t e = er / R;
    const uint32_t byte = blocks[i];
    const uint32_t s = scales[rg];
    const int64_t k = 32 * g + 2 * j;
    const int64_t o0 = (e * K + k) * R + r;
    const int64_t o1 = o0 + R;
    const uint32_t v0 = mx_fp32_bits(byte & 15u, s);
    const uint32_t v1 = mx_fp32_bits(byte >> 4, s);
    if constexpr (OUT == DT_BF16) {
      static_cast<uint16_t*>(out)[o0] = (uint16_t)(v0 >> 16);
      static_cast<uint16_t*>(out)[o1] = (uint16_t)(v1 >> 16);
    } else if constexpr (OUT == DT_F32) {
      static_cast<uint32_t*>(out)[o0] = v0;
      static_cast<uint32_t*>(out)[o1] = v1;
    } else {
      static_cast<uint16_t*>(out)[o0] = (uint16_t)mx_f16_bits(byte & 15u, s);
      static_cast<uint16_t*>(out)[o1] = (uint16_t)mx_f16_bits(byte >> 4, s);
    }
  }
}

template <int OUT>
static int launch_dequant(const uint8_t* blocks, const uint8_t* scales, void* out, int64_t E,
                          int64_t R, int64_t G, int mode, int kp, hipStream_t stream) {
  const uintptr_t bp = reinterpret_cast<uintptr_t>(blocks);
  const uintptr_t op = reinterpret_cast<uintptr_t>(out);
  // The vectorised kernel decodes in whichever way `mode` asks (mode 1 makes
  // it take the integer decoder for every wave).
  const bool vec = (R % 8 == 0) && (op % 16 == 0) && (bp % 8 == 0) && R <= INT32_MAX / 2 &&
                   G <= INT32_MAX / 64;
  // the k-pair layout is read by the vectorised kernel only
  if (kp && !(vec && bp % 16 == 0)) {
    set_error("dequant: the k-pair layout needs 16-byte aligned blocks and output");
    return BSA_EINVAL;
  }
  if (vec) {
    const int row_tiles = (int)((R + DQ_ROWS - 1) / DQ_ROWS);
    const int64_t nblk = E * row_tiles * ((G + DQ_GPB - 1) / DQ_GPB);
    if (nblk > INT32_MAX) {
      set_error("dequant: grid too large (E=%lld R=%lld)", (long long)E, (long long)R);
      return BSA_EINVAL;
    }
    if (bp % 16 == 0)
      hipLaunchKernelGGL((dequant_vec_kernel<OUT, true>), dim3((unsigned)nblk), dim3(256), 0,
                         stream, blocks, scales, out, (int)R, (int)G, row_tiles, mode, kp);
    else
      hipLaunchKernelGGL((dequant_vec_kernel<OUT, false>), dim3((unsigned)nblk), dim3(256), 0,
                         stream, blocks, scales, out, (int)R, (int)G, row_tiles, mode, 0);
  } else {
    const int64_t n = E * R * G * 16;
    int64_t nb = (n + 255) / 256;
    if (nb > 65536) nb = 65536;
    hipLaunchKernelGGL((dequant_generic_kernel<OUT>), dim3((unsigned)nb), dim3(256), 0, stream,
                       blocks, scales, out, E, R, G);
  }
  BSA_LAUNCH_CHECK("dequant launch");
  return BSA_OK;
}

// Checkpoint <-> k-pair layout of packed blocks: one 16-byte group per
// thread, i = row * G + g in checkpoint order (rows counted across experts;
// R % 16 == 0 makes every band lie inside one expert).  Reads of the
// checkpoint side are coalesced; the k-pair side is written (read) in
// 32-byte pairs.
template <bool TO_KP>
__global__ __launch_bounds__(256) void kpair_repack_kernel(const u32x4_t* __restrict__ in,
                                                           u32x4_t* __restrict__ out, int64_t rows, int G) {
  const int64_t n = rows * G;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / G;
    const int g = (int)(i - r * G);
    const int64_t k = bq_off(1, r, g, G) >> 4;
    if constexpr (TO_KP)
      out[k] = in[i];
    else
      out[i] = in[k];
  }
}

static int kpair_repack(const void* blocks, void* out, int64_t E, int64_t R, int64_t G, void* stream,
                        bool to_kp, const char* what) {
  clear_error();
  BSA_REQUIRE(E >= 0 && R >= 0 && G >= 0, "%s: negative shape E=%lld R=%lld G=%lld", what, (long long)E,
              (long long)R, (long long)G);
  BSA_REQUIRE(R % 16 == 0 && G % 2 == 0 && G <= INT32_MAX,
              "%s: needs rows %% 16 == 0 and an even group count (R=%lld G=%lld)", what, (long long)R,
              (long long)G);
  if (E == 0 || R == 0 || G == 0) return BSA_OK;
  BSA_REQUIRE(blocks && out, "%s: null pointer", what);
  BSA_REQUIRE(blocks != out, "%s: input and output must be distinct buffers", what);
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(blocks) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0,
              "%s: blocks and out must be 16-byte aligned", what);
  BSA_REQUIRE(E <= INT64_MAX / 16 / (R * G), "%s: size overflow", what);
  const int64_t n = E * R * G;
  const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, 65536);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const u32x4_t* in = static_cast<const u32x4_t*>(blocks);
  u32x4_t* o = static_cast<u32x4_t*>(out);
  if (to_kp)
    hipLaunchKernelGGL(kpair_repack_kernel<true>, dim3(grid), dim3(256), 0, st, in, o, E * R, (int)G);
  else
    hipLaunchKernelGGL(kpair_repack_kernel<false>, dim3(grid), dim3(256), 0, st, in, o, E * R, (int)G);
  BSA_LAUNCH_CHECK("k-pair repack launch");
  return BSA_OK;
}

}  // namespace bsa

extern "C" int bsa_dequant_mxfp4_layout(const void* blocks, const void* scales, void* out,
                                        int out_dtype, int64_t E, int64_t R, int64_t G, int mode,
                                        int blocks_layout, void* stream) {
  using namespace bsa;
  clear_error();
  BSA_REQUIRE(E >= 0 && R >= 0 && G >= 0, "dequant: negative shape E=%lld R=%lld G=%lld",
              (long long)E, (long long)R, (long long)G);
  BSA_REQUIRE(mode >= 0 && mode <= 2, "dequant: mode must be 0, 1 or 2 (got %d)", mode);
  BSA_REQUIRE(out_dtype == DT_BF16 || out_dtype == DT_F16 || out_dtype == DT_F32,
              "dequant: unsupported output dtype %d", out_dtype);
  BSA_REQUIRE(blocks_layout == BSA_LAYOUT_CHECKPOINT || blocks_layout == BSA_LAYOUT_KPAIR,
              "dequant: unknown blocks layout %d", blocks_layout);
  BSA_REQUIRE(blocks_layout == BSA_LAYOUT_CHECKPOINT || (R % 16 == 0 && G % 2 == 0),
              "dequant: the k-pair layout needs rows %% 16 == 0 and an even group count (R=%lld G=%lld)",
              (long long)R, (long long)G);
  if (E == 0 || R == 0 || G == 0) return BSA_OK;
  BSA_REQUIRE(blocks && scales && out, "dequant: null pointer");
  BSA_REQUIRE(E <= INT64_MAX / 16 / (R * G) , "dequant: size overflow");
  const uint8_t* b = static_cast<const uint8_t*>(blocks);
  const uint8_t* s = static_cast<const uint8_t*>(scales);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int kp = blocks_layout == BSA_LAYOUT_KPAIR;
  switch (out_dtype) {
    case DT_BF16: return launch_dequant<DT_BF16>(b, s, out, E, R, G, mode, kp, st);
    case DT_F16: return launch_dequant<DT_F16>(b, s, out, E, R, G, mode, kp, st);
    default: return launch_dequant<DT_F32>(b, s, out, E, R, G, mode, kp, st);
  }
}

extern "C" int bsa_dequant_mxfp4_mode(const void* blocks, const void* scales, void* out,
                                      int out_dtype, int64_t E, int64_t R, int64_t G, int mode,
                                      void* stream) {
  return bsa_dequant_mxfp4_layout(blocks, scales, out, out_dtype, E, R, G, mode, BSA_LAYOUT_CHECKPOINT, stream);
}

extern "C" int bsa_dequant_mxfp4(const void* blocks, const void* scales, void* out,
                                 int out_dtype, int64_t E, int64_t R, int64_t G, void* stream) {
  return bsa_dequant_mxfp4_mode(blocks, scales, out, out_dtype, E, R, G, 0, stream);
}

extern "C" int bsa_mxfp4_to_kpair(const void* blocks, void* out, int64_t E, int64_t R, int64_t G, void* stream) {
  return bsa::kpair_repack(blocks, out, E, R, G, stream, true, "to k-pair layout");
}

extern "C" int bsa_mxfp4_from_kpair(const void* blocks, void* out, int64_t E, int64_t R, int64_t G, void* stream) {
  return bsa::kpair_repack(blocks, out, E, R, G, stream, false, "from k-pair layout");
}
