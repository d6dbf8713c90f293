// Token -> expert dispatch and the weighted combine.
//
// Dispatch replaces block_streamer/gptoss.py:143-154 (one_hot, permute, sum,
// nonzero, where, and the gather of hidden rows), which costs three host
// synchronisations per call.  Here the device builds (one workgroup, or two
// launches over chunks for large batches) the expert-sorted order of the
// T*k (token, slot) pairs:
//   counts[e], offsets[e] (exclusive scan), row_pair[pos] = t*k + p for the
//   pos-th sorted row, pair_pos[t*k + p] = pos (or -1 for a dropped pair), and
//   the grouped-GEMM tile list (expert, first row) for tiles of BM rows.
// Rows of one expert are ordered by pair index (token, then slot), so the
// layout is deterministic.  Indices outside [0, E) are dropped, like the
// masking index skipped at gptoss.py:151.
//
// Combine replaces gptoss.py:175-176 (scale by the routing weight, then
// index_add_ into the output): each token gathers its k rows and adds them in
// ascending expert order (the reference's loop order) in float32, rounding
// once to the output type.  No atomics, so the result is reproducible.
#include "bsa_common.h"
#include "dispatch.h"

namespace bsa {

constexpr int DISPATCH_THREADS = 1024;
constexpr int DISPATCH_WAVES = DISPATCH_THREADS / 64;
constexpr int DISPATCH_MAX_E = 1024;

// Small batches: one workgroup does everything.
__global__ __launch_bounds__(DISPATCH_THREADS) void moe_dispatch_kernel(
    const int64_t* __restrict__ idx, int P, int E, int BM, int* __restrict__ counts,
    int* __restrict__ offsets, int* __restrict__ row_pair, int* __restrict__ pair_pos,
    int2* __restrict__ tiles, int* __restrict__ num_tiles) {
  __shared__ int s_cnt[DISPATCH_MAX_E];
  __shared__ int s_off[DISPATCH_MAX_E];
  __shared__ int s_run[DISPATCH_MAX_E];
  __shared__ int s_scan[2 * DISPATCH_WAVES];
  __shared__ uint8_t s_wc[DISPATCH_WAVES][DISPATCH_MAX_E];
  dispatch_block<DISPATCH_THREADS, DISPATCH_MAX_E>(idx, P, E, BM, counts, offsets, row_pair, pair_pos, tiles,
                                                   num_tiles, s_cnt, s_off, s_run, s_scan, s_wc);
}

// Large batches, in two launches over chunks of DISPATCH_CHUNK pairs: the
// per-chunk expert histograms, then each chunk's workgroup derives every
// expert's first row (all chunks' histograms) and its own chunk's base within
// each expert (the earlier chunks'), and places its pairs.  The result is the
// single-workgroup kernel's, entry for entry.
constexpr int DISPATCH_CHUNK = 2048;

__global__ __launch_bounds__(DISPATCH_THREADS) void moe_dispatch_hist_kernel(const int64_t* __restrict__ idx,
                                                                              int P, int E,
                                                                              int* __restrict__ hist) {
  __shared__ int s_cnt[DISPATCH_MAX_E];
  const int tid = threadIdx.x;
  const int begin = blockIdx.x * DISPATCH_CHUNK;
  const int end = min(P, begin + DISPATCH_CHUNK);
  for (int e = tid; e < E; e += DISPATCH_THREADS) s_cnt[e] = 0;
  __syncthreads();
  for (int i = begin + tid; i < end; i += DISPATCH_THREADS) {
    const int64_t e = idx[i];
    if (e >= 0 && e < E) atomicAdd(&s_cnt[(int)e], 1);
  }
  __syncthreads();
  for (int e = tid; e < E; e += DISPATCH_THREADS) hist[(int64_t)blockIdx.x * E + e] = s_cnt[e];
}

__global__ __launch_bounds__(DISPATCH_THREADS) void moe_dispatch_place_kernel(
    const int64_t* __restrict__ idx, int P, int E, int BM, const int* __restrict__ hist,
    int* __restrict__ counts, int* __restrict__ offsets, int* __restrict__ row_pair,
    int* __restrict__ pair_pos, int2* __restrict__ tiles, int* __restrict__ num_tiles) {
  __shared__ int s_off[DISPATCH_MAX_E];
  __shared__ int s_run[DISPATCH_MAX_E];
  __shared__ int s_scan[2 * DISPATCH_WAVES];
  __shared__ uint8_t s_wc[DISPATCH_WAVES][DISPATCH_MAX_E];
  const int tid = threadIdx.x;
  const int chunk = blockIdx.x;
  int total = 0, before = 0;
  if (tid < E) {
    for (int c = 0; c < (int)gridDim.x; ++c) {
      const int h = hist[(int64_t)c * E + tid];
      total += h;
      if (c < chunk) before += h;
    }
    s_run[tid] = 0;
  }
  const int start =
      dispatch_scan<DISPATCH_THREADS>(total, E, BM, s_scan, chunk == 0, counts, offsets, tiles, num_tiles);
  if (tid < E) s_off[tid] = start + before;
  __syncthreads();
  const int begin = chunk * DISPATCH_CHUNK;
  dispatch_place<DISPATCH_THREADS, DISPATCH_MAX_E>(idx, begin, min(P, begin + DISPATCH_CHUNK), E, s_off, s_run,
                                                   s_wc, row_pair, pair_pos);
}

__device__ __forceinline__ float load_f32(const void* p, int64_t i, int dtype) {
  if (dtype == DT_F32) return static_cast<const float*>(p)[i];
  const uint32_t b = static_cast<const uint16_t*>(p)[i];
  if (dtype == DT_BF16) return __uint_as_float(b << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

__device__ __forceinline__ void store_f32_as(void* p, int64_t i, float v, int dtype) {
  if (dtype == DT_F32) {
    static_cast<float*>(p)[i] = v;
  } else if (dtype == DT_BF16) {
    static_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_bf16_bits(v);
  } else {
    static_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_f16_bits(v);
  }
}

constexpr int COMBINE_MAX_K = 16;

// out[t][h] = sum over valid slots p of w[t,p] * Y[pair_pos[t*k+p]][h], slots
// taken in ascending expert order.  Y is float32 [P, H].  One workgroup per
// token; each thread handles 4 adjacent columns.
__global__ __launch_bounds__(256) void moe_combine_kernel(
    const float* __restrict__ Y, const int64_t* __restrict__ idx, const void* __restrict__ w,
    int w_dtype, const int* __restrict__ pair_pos, int T, int k, int H, void* __restrict__ out,
    int out_dtype) {
  const int t = blockIdx.x;
  int pos[COMBINE_MAX_K];
  float wt[COMBINE_MAX_K];
  int64_t ex[COMBINE_MAX_K];
  int n = 0;
  for (int p = 0; p < k; ++p) {
    const int ps = pair_pos[(int64_t)t * k + p];
    if (ps < 0) continue;
    const int64_t e = idx[(int64_t)t * k + p];
    const float wv = w ? load_f32(w, (int64_t)t * k + p, w_dtype) : 1.0f;
    // insertion by expert id (ties keep slot order)
    int j = n;
    while (j > 0 && ex[j - 1] > e) {
      ex[j] = ex[j - 1];
      pos[j] = pos[j - 1];
      wt[j] = wt[j - 1];
      --j;
    }
    ex[j] = e;
    pos[j] = ps;
    wt[j] = wv;
    ++n;
  }
  const int64_t obase = (int64_t)t * H;
  if ((H & 3) == 0) {
    // blockIdx.y selects a slice of 4 * blockDim.x columns
    for (int h = (blockIdx.y * blockDim.x + threadIdx.x) * 4; h < H; h += gridDim.y * blockDim.x * 4) {
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      if (n <= 4) {
        // the common top-k: all rows' loads in flight together
        float4 y[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (j < n) y[j] = *reinterpret_cast<const float4*>(Y + (int64_t)pos[j] * H + h);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (j < n) {
            acc.x += wt[j] * y[j].x;
            acc.y += wt[j] * y[j].y;
            acc.z += wt[j] * y[j].z;
            acc.w += wt[j] * y[j].w;
          }
      } else {
        for (int j = 0; j < n; ++j) {
          const float4 y = *reinterpret_cast<const float4*>(Y + (int64_t)pos[j] * H + h);
          acc.x += wt[j] * y.x;
          acc.y += wt[j] * y.y;
          acc.z += wt[j] * y.z;
          acc.w += wt[j] * y.w;
        }
      }
      if (out_dtype == DT_BF16) {
        uint2 v = make_uint2(pack_bf16x2(acc.x, acc.y), pack_bf16x2(acc.z, acc.w));
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + obase + h) = v;
      } else {
        store_f32_as(out, obase + h, acc.x, out_dtype);
        store_f32_as(out, obase + h + 1, acc.y, out_dtype);
        store_f32_as(out, obase + h + 2, acc.z, out_dtype);
        store_f32_as(out, obase + h + 3, acc.w, out_dtype);
      }
    }
  } else {
    for (int h = blockIdx.y * blockDim.x + threadIdx.x; h < H; h += gridDim.y * blockDim.x) {
      float acc = 0.f;
      for (int j = 0; j < n; ++j) acc += wt[j] * Y[(int64_t)pos[j] * H + h];
      store_f32_as(out, obase + h, acc, out_dtype);
    }
  }
}

// moe_combine_kernel for top-k <= 4 and H <= 4096 (H % 4 == 0, 16-byte
// aligned rows): the slot entries are loaded together, and all of a token's
// row loads (IT passes of 1024 columns x k rows, 16 bytes each) are in flight
// before the first sum.  Same slot order, same sums.
template <int IT>
__global__ __launch_bounds__(256) void moe_combine4_kernel(
    const float* __restrict__ Y, const int64_t* __restrict__ idx, const void* __restrict__ w,
    int w_dtype, const int* __restrict__ pair_pos, int k, int H, void* __restrict__ out,
    int out_dtype) {
  const int64_t t = blockIdx.x;
  int ps[4];
  int64_t ex[4];
  float wv[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    ps[p] = p < k ? pair_pos[t * k + p] : -1;
    ex[p] = p < k ? idx[t * k + p] : 0;
    wv[p] = p < k ? (w ? load_f32(w, t * k + p, w_dtype) : 1.0f) : 0.f;
  }
  // valid slots in ascending expert order (ties keep slot order)
  int pos[4];
  float wt[4];
  int64_t es[4];
  int n = 0;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    if (ps[p] < 0) continue;
    int j = n;
#pragma unroll
    for (int q = 3; q > 0; --q)
      if (q == j && es[q - 1] > ex[p]) {
        es[q] = es[q - 1];
        pos[q] = pos[q - 1];
        wt[q] = wt[q - 1];
        --j;
      }
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (q == j) {
        es[q] = ex[p];
        pos[q] = ps[p];
        wt[q] = wv[p];
      }
    ++n;
  }
  float4 y[IT][4];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int h = (it * 256 + (int)threadIdx.x) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (h < H && j < n) y[it][j] = *reinterpret_cast<const float4*>(Y + (int64_t)pos[j] * H + h);
  }
  const int64_t obase = t * H;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int h = (it * 256 + (int)threadIdx.x) * 4;
    if (h >= H) continue;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < n) {
        acc.x += wt[j] * y[it][j].x;
        acc.y += wt[j] * y[it][j].y;
        acc.z += wt[j] * y[it][j].z;
        acc.w += wt[j] * y[it][j].w;
      }
    if (out_dtype == DT_BF16) {
      uint2 v = make_uint2(pack_bf16x2(acc.x, acc.y), pack_bf16x2(acc.z, acc.w));
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + obase + h) = v;
    } else {
      store_f32_as(out, obase + h, acc.x, out_dtype);
      store_f32_as(out, obase + h + 1, acc.y, out_dtype);
      store_f32_as(out, obase + h + 2, acc.z, out_dtype);
      store_f32_as(out, obase + h + 3, acc.w, out_dtype);
    }
  }
}

// Backward prep, one wave per (token, slot) pair (block_streamer/gptoss.py:175
// differentiated): grad_w[t,p] = <dOut[t], y[pos]> (y = down output + bias,
// before the routing weight) and dY[pos] = bf16(dOut[t] * w[t,p]).
__global__ __launch_bounds__(256) void moe_bwd_prep_kernel(
    const void* __restrict__ dout, int dout_dtype, const float* __restrict__ y,
    const void* __restrict__ w, int w_dtype, const int* __restrict__ pair_pos, int P, int k,
    int H, uint16_t* __restrict__ dy, float* __restrict__ grad_w) {
  const int lane = threadIdx.x & 63;
  const int pair = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pair >= P) return;
  const int pos = pair_pos[pair];
  if (pos < 0) {
    if (lane == 0) grad_w[pair] = 0.f;
    return;
  }
  const int64_t t = pair / k;
  const float wv = load_f32(w, pair, w_dtype);
  float dot = 0.f;
  for (int h = lane; h < H; h += 64) {
    const float g = load_f32(dout, t * H + h, dout_dtype);
    dot += g * y[(int64_t)pos * H + h];
    dy[(int64_t)pos * H + h] = (uint16_t)f32_to_bf16_bits(g * wv);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) dot += __shfl_xor(dot, off);
  if (lane == 0) grad_w[pair] = dot;
}

// The same with 8 consecutive elements per lane and 16-byte accesses
// (H % 8 == 0, 16-byte aligned rows); DT is dout's dtype.
template <int DT>
__global__ __launch_bounds__(256) void moe_bwd_prep_vec_kernel(
    const void* __restrict__ dout, const float* __restrict__ y, const void* __restrict__ w, int w_dtype,
    const int* __restrict__ pair_pos, int P, int k, int H, uint16_t* __restrict__ dy,
    float* __restrict__ grad_w) {
  const int lane = threadIdx.x & 63;
  const int pair = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pair >= P) return;
  const int pos = pair_pos[pair];
  if (pos < 0) {
    if (lane == 0) grad_w[pair] = 0.f;
    return;
  }
  const int64_t t = pair / k;
  const float wv = load_f32(w, pair, w_dtype);
  const f32x4_t* yr = reinterpret_cast<const f32x4_t*>(y + (int64_t)pos * H);
  u32x4_t* dyr = reinterpret_cast<u32x4_t*>(dy + (int64_t)pos * H);
  float dot = 0.f;
  for (int c = lane; c < H / 8; c += 64) {
    float g[8];
    if constexpr (DT == DT_F32) {
      const f32x4_t* gr = reinterpret_cast<const f32x4_t*>(static_cast<const float*>(dout) + t * H);
      const f32x4_t a = gr[2 * c], b = gr[2 * c + 1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        g[i] = a[i];
        g[4 + i] = b[i];
      }
    } else {
      const u32x4_t q = reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(dout) + t * H)[c];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (DT == DT_BF16) {
          g[2 * i] = __uint_as_float(q[i] << 16);
          g[2 * i + 1] = __uint_as_float(q[i] & 0xFFFF0000u);
        } else {
          g[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(q[i] & 0xFFFFu));
          g[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(q[i] >> 16));
        }
      }
    }
    const f32x4_t y0 = yr[2 * c], y1 = yr[2 * c + 1];
#pragma unroll
    for (int i = 0; i < 4; ++i) dot += g[i] * y0[i] + g[4 + i] * y1[i];
    u32x4_t o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(g[2 * i] * wv, g[2 * i + 1] * wv);
    dyr[c] = o;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) dot += __shfl_xor(dot, off);
  if (lane == 0) grad_w[pair] = dot;
}

int launch_bwd_prep(const void* dout, int dout_dtype, const float* y, const void* w, int w_dtype,
                    const int* pair_pos, int P, int k, int H, uint16_t* dy, float* grad_w,
                    hipStream_t st) {
  if (P == 0) return BSA_OK;
  auto al16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
  if (H % 8 == 0 && al16(dout) && al16(y) && al16(dy)) {
    const dim3 grid((P + 3) / 4);
    if (dout_dtype == DT_F32)
      hipLaunchKernelGGL(moe_bwd_prep_vec_kernel<DT_F32>, grid, dim3(256), 0, st, dout, y, w, w_dtype,
                         pair_pos, P, k, H, dy, grad_w);
    else if (dout_dtype == DT_F16)
      hipLaunchKernelGGL(moe_bwd_prep_vec_kernel<DT_F16>, grid, dim3(256), 0, st, dout, y, w, w_dtype,
                         pair_pos, P, k, H, dy, grad_w);
    else
      hipLaunchKernelGGL(moe_bwd_prep_vec_kernel<DT_BF16>, grid, dim3(256), 0, st, dout, y, w, w_dtype,
                         pair_pos, P, k, H, dy, grad_w);
    BSA_LAUNCH_CHECK("backward prep launch");
    return BSA_OK;
  }
  hipLaunchKernelGGL(moe_bwd_prep_kernel, dim3((P + 3) / 4), dim3(256), 0, st, dout, dout_dtype, y,
                     w, w_dtype, pair_pos, P, k, H, dy, grad_w);
  BSA_LAUNCH_CHECK("backward prep launch");
  return BSA_OK;
}

int launch_dispatch(const int64_t* idx, int P, int E, int BM, int* counts, int* offsets,
                    int* row_pair, int* pair_pos, int2* tiles, int* num_tiles, int* hist,
                    hipStream_t st) {
  if (hist && P > 2 * DISPATCH_CHUNK) {
    const int nc = (P + DISPATCH_CHUNK - 1) / DISPATCH_CHUNK;
    hipLaunchKernelGGL(moe_dispatch_hist_kernel, dim3(nc), dim3(DISPATCH_THREADS), 0, st, idx, P, E, hist);
    BSA_LAUNCH_CHECK("dispatch launch");
    hipLaunchKernelGGL(moe_dispatch_place_kernel, dim3(nc), dim3(DISPATCH_THREADS), 0, st, idx, P, E, BM,
                       hist, counts, offsets, row_pair, pair_pos, tiles, num_tiles);
    BSA_LAUNCH_CHECK("dispatch launch");
    return BSA_OK;
  }
  hipLaunchKernelGGL(moe_dispatch_kernel, dim3(1), dim3(DISPATCH_THREADS), 0, st, idx, P, E, BM,
                     counts, offsets, row_pair, pair_pos, tiles, num_tiles);
  BSA_LAUNCH_CHECK("dispatch launch");
  return BSA_OK;
}

int launch_combine(const float* Y, const int64_t* idx, const void* w, int w_dtype,
                   const int* pair_pos, int T, int k, int H, void* out, int out_dtype,
                   hipStream_t st) {
  if (T == 0) return BSA_OK;
  if (T >= 1024 && k <= 4 && H % 4 == 0 && H <= 4096 && reinterpret_cast<uintptr_t>(Y) % 16 == 0 &&
      (out_dtype != DT_BF16 || reinterpret_cast<uintptr_t>(out) % 8 == 0)) {
    const int it = (H + 1023) / 1024;
    auto fn = it == 1 ? moe_combine4_kernel<1>
              : it == 2 ? moe_combine4_kernel<2>
              : it == 3 ? moe_combine4_kernel<3>
                        : moe_combine4_kernel<4>;
    hipLaunchKernelGGL(fn, dim3((unsigned)T), dim3(256), 0, st, Y, idx, w, w_dtype, pair_pos, k, H, out,
                       out_dtype);
    BSA_LAUNCH_CHECK("combine launch");
    return BSA_OK;
  }
  // small batches: several workgroups per token (more loads in flight)
  int slices = (H + 1023) / 1024;
  if (slices > 4) slices = 4;
  if (T >= 1024) slices = 1;
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)T, (unsigned)slices), dim3(256), 0, st, Y, idx, w,
                     w_dtype, pair_pos, T, k, H, out, out_dtype);
  BSA_LAUNCH_CHECK("combine launch");
  return BSA_OK;
}

}  // namespace bsa
