// The post-attention RMSNorm in front of the MoE path, one launch instead of
// the half-dozen elementwise kernels of the eager module.
//
// Replaces GptOssRMSNorm.forward (transformers models/gpt_oss/
// modeling_gpt_oss.py:57-62) with its operation order kept:
//   x32 = float32(x); r = rsqrt(mean(x32^2) + eps);
//   y = dtype(float32(weight) * (x32 * r))
// and its input-gradient backward, the derivative of that expression:
//   g = float32(weight) * float32(dy);
//   dx = r * g - x32 * (r^3 * sum(g * x32) / H)
// One wave per token.  bf16/f16 rows with H % 8 == 0 and H <= 3072 take the
// vector path (16-byte accesses, the row held in registers so HBM sees it
// once); other shapes and float32 take an element loop.  Sums run in a
// fixed order (each lane over its elements in increasing index, then a
// butterfly over the 64 lanes), so results are reproducible.
#include <initializer_list>

#include "bsa_common.h"

namespace bsa {

__device__ __forceinline__ float nload(const void* p, int64_t i, int dt) {
  if (dt == DT_F32) return static_cast<const float*>(p)[i];
  const uint32_t b = static_cast<const uint16_t*>(p)[i];
  if (dt == DT_BF16) return __uint_as_float(b << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

__device__ __forceinline__ void nstore(void* p, int64_t i, float v, int dt) {
  if (dt == DT_F32)
    static_cast<float*>(p)[i] = v;
  else if (dt == DT_BF16)
    static_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_bf16_bits(v);
  else
    static_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_f16_bits(v);
}

// RMSNorm arithmetic of the vector path.  A row is reduced in 16-byte chunks
// of 8 elements (bf16 or f16): lane l of a wave sums the squares of chunks
// l, l + 64, ... in increasing index, then rms_wave_sum adds the 64 lane sums
// by a butterfly.
__device__ __forceinline__ void rms_unpack8(const u32x4_t q, int dt, float (&v)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (dt == DT_BF16) {
      v[2 * j] = __uint_as_float(q[j] << 16);
      v[2 * j + 1] = __uint_as_float(q[j] & 0xFFFF0000u);
    } else {
      v[2 * j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(q[j] & 0xFFFFu));
      v[2 * j + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(q[j] >> 16));
    }
  }
}

__device__ __forceinline__ float rms_sumsq8(const u32x4_t q, int dt, float ss) {
  float v[8];
  rms_unpack8(q, dt, v);
#pragma unroll
  for (int j = 0; j < 8; ++j) ss += v[j] * v[j];
  return ss;
}

__device__ __forceinline__ float rms_wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ float rms_inv(float sumsq, int H, float eps) {
  return 1.0f / sqrtf(sumsq / (float)H + eps);
}

// y = dtype(g * (x * r)) for one chunk (g: the weight as float32).
__device__ __forceinline__ u32x4_t rms_apply8(const u32x4_t q, int dt, const float (&g)[8], float r) {
  float v[8];
  rms_unpack8(q, dt, v);
  u32x4_t o;
  if (dt == DT_BF16) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = f32_to_bf16_bits(g[2 * j] * (v[2 * j] * r)) | (f32_to_bf16_bits(g[2 * j + 1] * (v[2 * j + 1] * r)) << 16);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = f32_to_f16_bits(g[2 * j] * (v[2 * j] * r)) | (f32_to_f16_bits(g[2 * j + 1] * (v[2 * j + 1] * r)) << 16);
  }
  return o;
}

// weight[i .. i+8) -> float32 (i % 8 == 0; the weight 16-byte aligned).
__device__ __forceinline__ void rms_weight8(const void* w, int64_t i, int wdt, float (&g)[8]) {
  if (wdt == DT_F32) {
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(static_cast<const float*>(w) + i);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(static_cast<const float*>(w) + i + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      g[j] = a[j];
      g[4 + j] = b[j];
    }
  } else {
    rms_unpack8(*reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(w) + i), wdt, g);
  }
}

__device__ __forceinline__ u32x4_t load16(const void* p, int64_t elem) {
  return *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p) + elem);
}

__device__ __forceinline__ uint32_t pack2(float a, float b, int dt) {
  if (dt == DT_BF16) return f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16);
  return f32_to_f16_bits(a) | (f32_to_f16_bits(b) << 16);
}

// 16-byte chunks of a row that one lane keeps in registers on the vector
// path: rows up to 64 * 6 * 8 = 3072 elements are read from HBM once.
constexpr int NORM_RC = 6;

// Vector path: x, y (dy, dx) are bf16 or f16 with 16-byte aligned rows,
// H % 8 == 0, H / 8 <= 64 * NORM_RC, weight 16-byte aligned.  Lane l holds
// chunks l, l + 64, ... of its wave's row.
template <int DT>
__global__ __launch_bounds__(256, 4) void rmsnorm_fwd_vec_kernel(const void* __restrict__ x, int T, int H,
                                                              const void* __restrict__ w, int wdt, float eps,
                                                              void* __restrict__ y) {
  constexpr int dt = DT;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int64_t row = (int64_t)t * H;
  const int nc = H / 8;
  u32x4_t xr[NORM_RC];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NORM_RC; ++i) {
    const int c = lane + 64 * i;
    if (c < nc) xr[i] = load16(x, row + 8 * c);
  }
#pragma unroll
  for (int i = 0; i < NORM_RC; ++i)
    if (lane + 64 * i < nc) ss = rms_sumsq8(xr[i], dt, ss);
  const float r = rms_inv(rms_wave_sum(ss), H, eps);
#pragma unroll
  for (int i = 0; i < NORM_RC; ++i) {
    const int c = lane + 64 * i;
    if (c < nc) {
      float g[8];
      rms_weight8(w, 8 * c, wdt, g);
      *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(y) + row + 8 * c) = rms_apply8(xr[i], dt, g, r);
    }
  }
}

// Element path: any dtype, alignment and H.
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const void* __restrict__ x, int dt, int T, int H,
                                                          const void* __restrict__ w, int wdt, float eps,
                                                          void* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int64_t row = (int64_t)t * H;
  float ss = 0.f;
  for (int h = lane; h < H; h += 64) {
    const float v = nload(x, row + h, dt);
    ss += v * v;
  }
  const float r = rms_inv(rms_wave_sum(ss), H, eps);
  for (int h = lane; h < H; h += 64) nstore(y, row + h, nload(w, h, wdt) * (nload(x, row + h, dt) * r), dt);
}

__global__ __launch_bounds__(256, 4) void rmsnorm_bwd_vec_kernel(const void* __restrict__ dy,
                                                              const void* __restrict__ x, int dt, int T, int H,
                                                              const void* __restrict__ w, int wdt, float eps,
                                                              void* __restrict__ dx) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int64_t row = (int64_t)t * H;
  const int nc = H / 8;
  u32x4_t xr[NORM_RC], gr[NORM_RC];
#pragma unroll
  for (int i = 0; i < NORM_RC; ++i) {
    const int c = lane + 64 * i;
    if (c < nc) {
      xr[i] = load16(x, row + 8 * c);
      gr[i] = load16(dy, row + 8 * c);
    }
  }
  float ss = 0.f, dot = 0.f;
#pragma unroll
  for (int i = 0; i < NORM_RC; ++i) {
    const int c = lane + 64 * i;
    if (c < nc) {
      float v[8], d[8], g[8];
      rms_unpack8(xr[i], dt, v);
      rms_unpack8(gr[i], dt, d);
      rms_weight8(w, 8 * c, wdt, g);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        ss += v[j] * v[j];
        dot += (g[j] * d[j]) * v[j];
      }
    }
  }
  const float r = rms_inv(rms_wave_sum(ss), H, eps);
  const float c3 = r * r * r * rms_wave_sum(dot) / (float)H;
#pragma unroll
  for (int i = 0; i < NORM_RC; ++i) {
    const int c = lane + 64 * i;
    if (c < nc) {
      float v[8], d[8], g[8];
      rms_unpack8(xr[i], dt, v);
      rms_unpack8(gr[i], dt, d);
      rms_weight8(w, 8 * c, wdt, g);
      u32x4_t o;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack2(r * (g[2 * j] * d[2 * j]) - v[2 * j] * c3, r * (g[2 * j + 1] * d[2 * j + 1]) - v[2 * j + 1] * c3,
                     dt);
      *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(dx) + row + 8 * c) = o;
    }
  }
}

__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const void* __restrict__ dy, const void* __restrict__ x,
                                                          int dt, int T, int H, const void* __restrict__ w, int wdt,
                                                          float eps, void* __restrict__ dx) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int64_t row = (int64_t)t * H;
  float ss = 0.f, dot = 0.f;
  for (int h = lane; h < H; h += 64) {
    const float v = nload(x, row + h, dt);
    ss += v * v;
    dot += (nload(w, h, wdt) * nload(dy, row + h, dt)) * v;
  }
  const float r = rms_inv(rms_wave_sum(ss), H, eps);
  const float c3 = r * r * r * rms_wave_sum(dot) / (float)H;
  for (int h = lane; h < H; h += 64)
    nstore(dx, row + h, r * (nload(w, h, wdt) * nload(dy, row + h, dt)) - nload(x, row + h, dt) * c3, dt);
}

static bool norm_dtype_ok(int d) { return d == DT_BF16 || d == DT_F16 || d == DT_F32; }

static bool norm_vec_ok(int dt, int64_t H, std::initializer_list<const void*> ptrs) {
  if (dt == DT_F32 || H % 8 != 0 || H / 8 > 64 * NORM_RC) return false;
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
  return true;
}

}  // namespace bsa

using namespace bsa;

extern "C" int bsa_rmsnorm_fwd(const void* x, int dtype, int64_t T, int64_t H, const void* weight, int weight_dtype,
                               float eps, void* out, void* stream) {
  clear_error();
  BSA_REQUIRE(T >= 0 && H > 0 && T < INT32_MAX / 4 && H < INT32_MAX, "rmsnorm: bad shape T=%lld H=%lld",
              (long long)T, (long long)H);
  BSA_REQUIRE(norm_dtype_ok(dtype) && norm_dtype_ok(weight_dtype), "rmsnorm: bad dtype code");
  if (T == 0) return BSA_OK;
  BSA_REQUIRE(x && weight && out, "rmsnorm: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((T + 3) / 4));
  if (norm_vec_ok(dtype, H, {x, out, weight}))
    hipLaunchKernelGGL(dtype == DT_BF16 ? rmsnorm_fwd_vec_kernel<DT_BF16> : rmsnorm_fwd_vec_kernel<DT_F16>, grid,
                       dim3(256), 0, st, x, (int)T, (int)H, weight, weight_dtype, eps, out);
  else
    hipLaunchKernelGGL(rmsnorm_fwd_kernel, grid, dim3(256), 0, st, x, dtype, (int)T, (int)H, weight,
                       weight_dtype, eps, out);
  BSA_LAUNCH_CHECK("rmsnorm launch");
  return BSA_OK;
}

extern "C" int bsa_rmsnorm_bwd(const void* grad_out, const void* x, int dtype, int64_t T, int64_t H,
                               const void* weight, int weight_dtype, float eps, void* grad_x, void* stream) {
  clear_error();
  BSA_REQUIRE(T >= 0 && H > 0 && T < INT32_MAX / 4 && H < INT32_MAX, "rmsnorm bwd: bad shape T=%lld H=%lld",
              (long long)T, (long long)H);
  BSA_REQUIRE(norm_dtype_ok(dtype) && norm_dtype_ok(weight_dtype), "rmsnorm bwd: bad dtype code");
  if (T == 0) return BSA_OK;
  BSA_REQUIRE(grad_out && x && weight && grad_x, "rmsnorm bwd: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((T + 3) / 4));
  if (norm_vec_ok(dtype, H, {grad_out, x, grad_x, weight}))
    hipLaunchKernelGGL(rmsnorm_bwd_vec_kernel, grid, dim3(256), 0, st, grad_out, x, dtype, (int)T, (int)H,
                       weight, weight_dtype, eps, grad_x);
  else
    hipLaunchKernelGGL(rmsnorm_bwd_kernel, grid, dim3(256), 0, st, grad_out, x, dtype, (int)T, (int)H,
                       weight, weight_dtype, eps, grad_x);
  BSA_LAUNCH_CHECK("rmsnorm bwd launch");
  return BSA_OK;
}
