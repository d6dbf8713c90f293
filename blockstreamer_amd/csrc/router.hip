// Fused router: logits, top-k, softmax over the top-k.
//
// Replaces transformers models/gpt_oss/modeling_gpt_oss.py:126-131
// (GptOssTopKRouter.forward):
//   logits = F.linear(h, W, b)                 [T, E] in the module dtype
//   vals, idx = topk(logits, k)                sorted descending
//   scores = softmax(vals, dim=1, dtype=vals.dtype)
//
// bf16 modules (the gpt-oss case): a tiled logits kernel on
// v_mfma_f32_16x16x32_bf16 (16x16 token x expert tiles, 32x32 once T >= 4096;
// float32 accumulation, bias added in float32, one rounding to bf16, as a
// bf16 GEMM with a bias epilogue does), then a top-k kernel over the bf16
// logits.  float32 and float16 modules: one fused kernel of float32 VALU dot
// products per 16 tokens.  Top-k: each wave selects one token's k largest by
// k rounds of a wave-wide arg-max on a 64-bit key (orderable value, then
// lower expert index first; -0 and +0 compare equal), and takes the softmax
// of the k values in float32 rounded once to the module dtype.
#include "bsa_common.h"

namespace bsa {

constexpr int RT_MAX_E = 256;   // experts
constexpr int RT_MAX_K = 16;

typedef __attribute__((ext_vector_type(8))) short rs16x8_t;

__device__ __forceinline__ float ld_any(const void* p, int64_t i, int dtype) {
  if (dtype == DT_F32) return static_cast<const float*>(p)[i];
  const uint32_t b = static_cast<const uint16_t*>(p)[i];
  if (dtype == DT_BF16) return __uint_as_float(b << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

// float -> value rounded to dtype and back (the module-dtype logit)
__device__ __forceinline__ float round_to(float v, int dtype) {
  if (dtype == DT_BF16) return __uint_as_float(f32_to_bf16_bits(v) << 16);
  if (dtype == DT_F16) return (float)(_Float16)v;
  return v;
}

__device__ __forceinline__ void st_any(void* p, int64_t i, float v, int dtype) {
  if (dtype == DT_F32) {
    static_cast<float*>(p)[i] = v;
  } else if (dtype == DT_BF16) {
    static_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_bf16_bits(v);
  } else {
    static_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_f16_bits(v);
  }
}

// Larger key = larger value; equal values: lower index wins.
__device__ __forceinline__ uint64_t topk_key(float v, int e) {
  v = v + 0.0f;  // -0 -> +0
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e);
}

// Top-k and softmax of one token's E logits held in LDS row `row`.
__device__ void topk_softmax_wave(const float* row, int E, int k, int lane, int out_dtype,
                                  void* scores, int64_t* indices, int64_t t) {
  constexpr int PER = RT_MAX_E / 64;
  uint64_t key[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = lane + 64 * j;
    key[j] = e < E ? topk_key(row[e], e) : 0ull;
  }
  float vals[RT_MAX_K];
  int ids[RT_MAX_K];
  for (int r = 0; r < k; ++r) {
    uint64_t best = 0ull;
#pragma unroll
    for (int j = 0; j < PER; ++j) best = key[j] > best ? key[j] : best;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const uint64_t o = __shfl_xor(best, off);
      best = o > best ? o : best;
    }
    const int e = (int)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (key[j] == best) key[j] = 0ull;
    ids[r] = e;
    vals[r] = row[e];
  }
  if (lane == 0) {
    float mx = vals[0];
    for (int r = 1; r < k; ++r) mx = fmaxf(mx, vals[r]);
    float sum = 0.f;
    for (int r = 0; r < k; ++r) sum += __expf(vals[r] - mx);
    const float inv = 1.0f / sum;
    // each exponential again rather than kept in a dynamically indexed array
    // (such an array can go to scratch memory); the same expression, the same value
    for (int r = 0; r < k; ++r) {
      st_any(scores, t * k + r, __expf(vals[r] - mx) * inv, out_dtype);
      indices[t * k + r] = ids[r];
    }
  }
}

// bf16 logits tile: RT*16 tokens x RE*16 experts per workgroup.  The W
// waves split the hidden dimension (wave w takes k-steps w, w+W, ...); their
// float32 partial sums are added in wave order (deterministic), the bias is
// added in float32 and the result rounded once to bf16.  Small batches use
// W = 16, so that each wave's loads of the whole hidden dimension are in
// flight at once (few tiles, one round trip).  Tiles are ordered
// so that all expert tiles of one token tile run on one XCD (the token rows
// are then fetched from HBM once into that XCD's L2).
template <int RT, int RE, int W>
__global__ __launch_bounds__(64 * W) void logits_bf16_kernel(const uint16_t* __restrict__ hidden,
                                                          const uint16_t* __restrict__ weight,
                                                          const uint16_t* __restrict__ bias,
                                                          int T, int H, int E,
                                                          uint16_t* __restrict__ logits) {
  __shared__ float s_part[W - 1][RT][RE][4][64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lr = lane & 15;
  const int lk = lane >> 4;
  const int n_te = (E + 16 * RE - 1) / (16 * RE);
  const int nblk = gridDim.x;
  const int bid = blockIdx.x;
  const int L = (nblk & 7) == 0 ? (bid & 7) * (nblk >> 3) + (bid >> 3) : bid;
  const int t0 = (L / n_te) * 16 * RT;
  const int e0 = (L % n_te) * 16 * RE;
  const int nks = H / 32;

  const uint16_t* arow[RT];
  const uint16_t* brow[RE];
  bool bok[RE];
#pragma unroll
  for (int r = 0; r < RT; ++r)
    arow[r] = hidden + (int64_t)min(t0 + r * 16 + lr, T - 1) * H + lk * 8;
#pragma unroll
  for (int j = 0; j < RE; ++j) {
    const int e = e0 + j * 16 + lr;
    bok[j] = e < E;
    brow[j] = weight + (int64_t)(bok[j] ? e : 0) * H + lk * 8;
  }
  f32x4_t acc[RT][RE];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int j = 0; j < RE; ++j) acc[r][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // D k-steps per round: all loads of a round are issued before its MFMAs
  constexpr int D = RT * RE == 1 ? 8 : 4;
  for (int base = wave; base < nks; base += W * D) {
    rs16x8_t av[D][RT], bv[D][RE];
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int ks = min(base + W * u, nks - 1);
#pragma unroll
      for (int r = 0; r < RT; ++r) av[u][r] = *reinterpret_cast<const rs16x8_t*>(arow[r] + ks * 32);
#pragma unroll
      for (int j = 0; j < RE; ++j) {
        bv[u][j] = *reinterpret_cast<const rs16x8_t*>(brow[j] + ks * 32);
        if (!bok[j]) bv[u][j] = rs16x8_t{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int u = 0; u < D; ++u) {
      if (base + W * u >= nks) break;
#pragma unroll
      for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int j = 0; j < RE; ++j)
          acc[r][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av[u][r]),
                                                              __builtin_bit_cast(bf16x8_t, bv[u][j]),
                                                              acc[r][j], 0, 0, 0);
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int j = 0; j < RE; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) s_part[wave - 1][r][j][i][lane] = acc[r][j][i];
  }
  __syncthreads();
  if (wave != 0) return;
  // C layout: lane (lr, lk) holds expert e0 + 16j + lr, tokens 16r + 4lk + i
#pragma unroll
  for (int j = 0; j < RE; ++j) {
    const int e = e0 + j * 16 + lr;
    if (e >= E) continue;
    const float bv = bias ? __uint_as_float((uint32_t)bias[e] << 16) : 0.f;
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + r * 16 + 4 * lk + i;
        float v = acc[r][j][i];
#pragma unroll
        for (int w = 0; w < W - 1; ++w) v += s_part[w][r][j][i][lane];
        if (t < T) logits[(int64_t)t * E + e] = (uint16_t)f32_to_bf16_bits(v + bv);
      }
  }
}

// float32 / float16 modules: float32 VALU dot products, 16 tokens per workgroup.
__global__ __launch_bounds__(256) void router_valu_kernel(const void* __restrict__ hidden, int dtype,
                                                         int T, int H, int E, int k,
                                                         const void* __restrict__ weight,
                                                         const void* __restrict__ bias,
                                                         void* __restrict__ logits,
                                                         void* __restrict__ scores,
                                                         int64_t* __restrict__ indices) {
  __shared__ float s_log[16][RT_MAX_E + 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int t0 = blockIdx.x * 16;
  for (int idx = tid; idx < 16 * E; idx += 256) {
    const int tt = idx / E;
    const int e = idx - tt * E;
    const int t = min(t0 + tt, T - 1);
    float acc = 0.f;
    for (int h = 0; h < H; ++h)
      acc += ld_any(hidden, (int64_t)t * H + h, dtype) * ld_any(weight, (int64_t)e * H + h, dtype);
    const float bv = bias ? ld_any(bias, e, dtype) : 0.f;
    s_log[tt][e] = round_to(acc + bv, dtype);
  }
  __syncthreads();
  for (int idx = tid; idx < 16 * E; idx += 256) {
    const int tt = idx / E;
    const int e = idx - tt * E;
    if (t0 + tt < T) st_any(logits, (int64_t)(t0 + tt) * E + e, s_log[tt][e], dtype);
  }
  for (int tt = wave; tt < 16; tt += 4)
    if (t0 + tt < T) topk_softmax_wave(s_log[tt], E, k, lane, dtype, scores, indices, t0 + tt);
}

// Top-k + softmax of given logits [T, E] (one wave per token).
__global__ __launch_bounds__(256) void topk_kernel(const void* __restrict__ logits, int dtype,
                                                   int T, int E, int k, void* __restrict__ scores,
                                                   int64_t* __restrict__ indices) {
  __shared__ float s_row[4][RT_MAX_E];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  for (int e = lane; e < E; e += 64) s_row[wave][e] = ld_any(logits, (int64_t)t * E + e, dtype);
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  topk_softmax_wave(s_row[wave], E, k, lane, dtype, scores, indices, t);
}

}  // namespace bsa

using namespace bsa;

extern "C" int bsa_router_fwd(const void* hidden, int dtype, int64_t T, int64_t H, int64_t E,
                              int64_t k, const void* weight, const void* bias, void* logits,
                              void* scores, int64_t* indices, void* stream) {
  clear_error();
  BSA_REQUIRE(T >= 0 && H > 0 && E > 0 && k > 0, "router: bad shape T=%lld H=%lld E=%lld k=%lld",
              (long long)T, (long long)H, (long long)E, (long long)k);
  BSA_REQUIRE(E <= RT_MAX_E && k <= RT_MAX_K && k <= E, "router: needs E <= %d and k <= min(E, %d)",
              RT_MAX_E, RT_MAX_K);
  BSA_REQUIRE(dtype == DT_BF16 || dtype == DT_F16 || dtype == DT_F32, "router: bad dtype %d", dtype);
  BSA_REQUIRE(T < INT32_MAX && H < INT32_MAX, "router: too large");
  if (T == 0) return BSA_OK;
  BSA_REQUIRE(hidden && weight && logits && scores && indices, "router: null pointer");
  const bool mfma = dtype == DT_BF16 && H % 32 == 0 && reinterpret_cast<uintptr_t>(hidden) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(weight) % 16 == 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (mfma) {
    // logits tiles, then top-k + softmax from the (L2-resident) logits
    if (T >= 4096) {
      // 32 tokens x 64 experts per workgroup (measured at 8192 tokens: 48.6 us
      // for the router against 56-57 us with 32 x 32 and 65-67 us with 16 x 64
      // or 16 x 128; the sums, and so the logits, do not depend on the tile)
      const int64_t nblk = ((T + 31) / 32) * ((E + 63) / 64);
      hipLaunchKernelGGL((logits_bf16_kernel<2, 4, 4>), dim3((unsigned)nblk), dim3(256), 0, st,
                         static_cast<const uint16_t*>(hidden), static_cast<const uint16_t*>(weight),
                         static_cast<const uint16_t*>(bias), (int)T, (int)H, (int)E,
                         static_cast<uint16_t*>(logits));
    } else {
      const int64_t nblk = ((T + 15) / 16) * ((E + 15) / 16);
      hipLaunchKernelGGL((logits_bf16_kernel<1, 1, 16>), dim3((unsigned)nblk), dim3(1024), 0, st,
                         static_cast<const uint16_t*>(hidden), static_cast<const uint16_t*>(weight),
                         static_cast<const uint16_t*>(bias), (int)T, (int)H, (int)E,
                         static_cast<uint16_t*>(logits));
    }
    BSA_LAUNCH_CHECK("router logits launch");
    hipLaunchKernelGGL(topk_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, st, logits, dtype,
                       (int)T, (int)E, (int)k, scores, indices);
  } else {
    hipLaunchKernelGGL(router_valu_kernel, dim3((unsigned)((T + 15) / 16)), dim3(256), 0, st,
                       hidden, dtype, (int)T, (int)H, (int)E, (int)k, weight, bias, logits, scores,
                       indices);
  }
  BSA_LAUNCH_CHECK("router launch");
  return BSA_OK;
}

extern "C" int bsa_router_topk(const void* logits, int dtype, int64_t T, int64_t E, int64_t k,
                               void* scores, int64_t* indices, void* stream) {
  clear_error();
  BSA_REQUIRE(T >= 0 && E > 0 && k > 0, "router topk: bad shape");
  BSA_REQUIRE(E <= RT_MAX_E && k <= RT_MAX_K && k <= E, "router topk: needs E <= %d and k <= min(E, %d)",
              RT_MAX_E, RT_MAX_K);
  BSA_REQUIRE(dtype == DT_BF16 || dtype == DT_F16 || dtype == DT_F32, "router topk: bad dtype %d", dtype);
  if (T == 0) return BSA_OK;
  BSA_REQUIRE(logits && scores && indices, "router topk: null pointer");
  hipLaunchKernelGGL(topk_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), logits, dtype, (int)T, (int)E, (int)k,
                     scores, indices);
  BSA_LAUNCH_CHECK("router topk launch");
  return BSA_OK;
}
