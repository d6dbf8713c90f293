// Grouped expert GEMMs on gfx950 MFMA with MXFP4 weights dequantised on the
// fly, and the fused MoE expert forward built from them.
//
// Replaces the per-expert loop of block_streamer/gptoss.py:149-176:
//   gate_up = mxfp4_matmul(x_e, gate_up_blocks[e], ...) + gate_up_bias[e]   (:158-165)
//   gated   = _apply_gate(gate_up)                                           (:166, :130-135)
//   out     = mxfp4_matmul(gated, down_blocks[e], ...) + down_bias[e]        (:167-174)
// where mxfp4_matmul (gptoss.py:45-75) materialises a dense 47 MiB weight per
// expert.  Here the packed weight is read once and decoded in registers.
//
// GEMM view: C[m, n] = sum_k A[row(m), k] * B[n, k] where B is the packed
// weight [E][N][K/32][16] (+ E8M0 scales [E][N][K/32]): row n of the packed
// tensor holds output column n with K contiguous, which is exactly the
// per-lane layout of an MFMA B operand, so no transpose is ever needed.
//
// Two kernels:
//  * moe_stream_kernel (decode, few rows per expert): one workgroup per
//    (expert, 32-column slice).  The slice's packed bytes are one contiguous
//    32*K/2-byte span; it is copied to LDS with 16-byte loads, then four
//    waves split K and run v_mfma_f32_16x16x32_bf16 on 16-row blocks, with A
//    rows prefetched 8 steps ahead.  Partial sums are reduced through LDS.
//    Bound: HBM (each hit expert's weights are read exactly once).
//  * moe_tiled_kernel (prefill): 128x128 output tiles of one expert, BK=64,
//    LDS double buffering, 2x2 waves of 64x64 using
//    v_mfma_f32_32x32x16_bf16.  The B tile is decoded into LDS as bf16.
//    Bound: MFMA.
//
// For the gate_up projection the weight rows interleave gate (even) and up
// (odd) columns (gptoss.py:131).  Both kernels place gate column j and up
// column j in the same lane, so the clamped SwiGLU runs in registers.
#include "bsa_common.h"

namespace bsa {

int launch_dispatch(const int64_t* idx, int P, int E, int BM, int* counts, int* offsets,
                    int* row_pair, int* pair_pos, int2* tiles, int* num_tiles, hipStream_t st);
int launch_combine(const float* Y, const int64_t* idx, const void* w, int w_dtype,
                   const int* pair_pos, int T, int k, int H, void* out, int out_dtype,
                   hipStream_t st);

enum Epi : int {
  EPI_SWIGLU = 0,    // out bf16 [P][N/2] = swiglu(acc + bias), optional f32 pre-activation save
  EPI_BIAS_F32 = 1,  // out f32 [P][N] = acc + bias
  EPI_STORE = 2,     // out (out_dtype) [P][N] = acc (+ bias if given)
};

struct GemmArgs {
  const uint16_t* A;     // bf16 activations, row stride lda
  int64_t lda;
  const int* row_pair;   // non-null: A row of sorted row pos is row_pair[pos] / topk
  int topk;
  const uint8_t* Bq;     // packed [E][N][K/32][16]
  const uint8_t* Bs;     // scales [E][N][K/32]
  const void* bias;      // [E][N] or null
  int bias_dtype;
  const int* counts;     // rows per expert
  const int* offsets;    // first sorted row per expert
  int E, N, K;
  void* out;
  int64_t ldo;
  int out_dtype;
  float* save_pre;       // EPI_SWIGLU: optional f32 [P][N] pre-activation (incl. bias)
  float alpha, limit;
  const int2* tiles;     // tiled kernel: (expert, first sorted row) per row tile
  const int* num_tiles;
  int n_tiles_n;         // column tiles per row tile
};

typedef __attribute__((ext_vector_type(8))) short s16x8_t;

__device__ __forceinline__ f32x4_t mfma16(s16x8_t a, s16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma32(s16x8_t a, s16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// 8 MXFP4 codes (4 packed bytes) -> 8 bf16 in code order.
__device__ __forceinline__ s16x8_t decode8(uint32_t q, uint32_t s) {
  uint32_t d[4];
  mx_dword_to_bf16x8(q, s, mx_scale_hw_ok(s), d);
  u32x4_t v = {d[0], d[1], d[2], d[3]};
  return __builtin_bit_cast(s16x8_t, v);
}

__device__ __forceinline__ float bias_at(const void* bias, int dtype, int64_t i) {
  if (!bias) return 0.f;
  if (dtype == DT_F32) return static_cast<const float*>(bias)[i];
  const uint32_t b = static_cast<const uint16_t*>(bias)[i];
  if (dtype == DT_BF16) return __uint_as_float(b << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

// block_streamer/gptoss.py:130-135 in float32.
__device__ __forceinline__ float swiglu(float g, float u, float alpha, float limit) {
  g = fminf(g, limit);
  u = fminf(fmaxf(u, -limit), limit);
  const float sig = 1.0f / (1.0f + __expf(-alpha * g));
  return (u + 1.0f) * (g * sig);
}

__device__ __forceinline__ void store_out(void* out, int dtype, int64_t i, float v) {
  if (dtype == DT_F32) {
    static_cast<float*>(out)[i] = v;
  } else if (dtype == DT_BF16) {
    static_cast<uint16_t*>(out)[i] = (uint16_t)f32_to_bf16_bits(v);
  } else {
    static_cast<uint16_t*>(out)[i] = (uint16_t)f32_to_f16_bits(v);
  }
}

template <bool ALIGN16>
__device__ __forceinline__ u32x4_t load16(const uint8_t* p) {
  if constexpr (ALIGN16) {
    return *reinterpret_cast<const u32x4_t*>(p);
  } else {
    const uint2 a = *reinterpret_cast<const uint2*>(p);
    const uint2 b = *reinterpret_cast<const uint2*>(p + 8);
    return u32x4_t{a.x, a.y, b.x, b.y};
  }
}

// ---------------------------------------------------------------------------
// Epilogue shared by both kernels: one output element pair (SwiGLU) or one
// element, for sorted row pos and weight-row index n.
// ---------------------------------------------------------------------------
template <int EPI>
__device__ __forceinline__ void epilogue_swiglu(const GemmArgs& a, int e, int64_t pos, int n_gate,
                                                float accg, float accu) {
  const float g = accg + bias_at(a.bias, a.bias_dtype, (int64_t)e * a.N + n_gate);
  const float u = accu + bias_at(a.bias, a.bias_dtype, (int64_t)e * a.N + n_gate + 1);
  if (a.save_pre) {
    float2* sp = reinterpret_cast<float2*>(a.save_pre + pos * a.N + n_gate);
    *sp = make_float2(g, u);
  }
  static_cast<uint16_t*>(a.out)[pos * a.ldo + (n_gate >> 1)] =
      (uint16_t)f32_to_bf16_bits(swiglu(g, u, a.alpha, a.limit));
}

template <int EPI>
__device__ __forceinline__ void epilogue_one(const GemmArgs& a, int e, int64_t pos, int n, float acc) {
  const float v = acc + bias_at(a.bias, a.bias_dtype, (int64_t)e * a.N + n);
  if constexpr (EPI == EPI_BIAS_F32)
    static_cast<float*>(a.out)[pos * a.ldo + n] = v;
  else
    store_out(a.out, a.out_dtype, pos * a.ldo + n, v);
}

// ---------------------------------------------------------------------------
// Weight-streaming kernel (decode).
// ---------------------------------------------------------------------------
constexpr int ST_BN = 32;     // weight rows (output columns) per workgroup
constexpr int ST_MAXRB = 2;   // 16-row blocks per pass
constexpr int ST_PF = 8;      // A prefetch distance (k-steps)

__host__ __device__ inline int st_lds_row(int K) { return K / 2 + 16; }
inline size_t st_smem_bytes(int K) {
  const size_t b = (size_t)ST_BN * st_lds_row(K) + (size_t)ST_BN * (K / 32);
  const size_t red = (size_t)4 * ST_MAXRB * 2 * 64 * sizeof(f32x4_t);
  return (b > red ? b : red) + 16;
}

template <int EPI, bool ALIGN16>
__global__ __launch_bounds__(256) void moe_stream_kernel(GemmArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int slices = (a.N + ST_BN - 1) / ST_BN;
  const int e = blockIdx.x / slices;
  const int slice = blockIdx.x - e * slices;
  const int cnt = a.counts[e];
  if (cnt == 0) return;
  const int row0 = a.offsets[e];
  const int n0 = slice * ST_BN;
  const int nvalid = min(ST_BN, a.N - n0);
  const int G = a.K / 32;
  const int rowbytes = a.K / 2;
  const int ldsrow = st_lds_row(a.K);
  uint8_t* sB = smem;
  uint8_t* sS = smem + ST_BN * ldsrow;
  f32x4_t* sRed = reinterpret_cast<f32x4_t*>(smem);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lr = lane & 15;
  const int lk = lane >> 4;

  const uint8_t* gB = a.Bq + ((int64_t)e * a.N + n0) * rowbytes;
  const uint8_t* gS = a.Bs + ((int64_t)e * a.N + n0) * G;

  // weight rows of this lane's two 16-column blocks
  const int bc0 = (EPI == EPI_SWIGLU) ? 2 * lr : lr;
  const int bc1 = (EPI == EPI_SWIGLU) ? 2 * lr + 1 : 16 + lr;

  for (int pass0 = 0; pass0 < cnt; pass0 += 16 * ST_MAXRB) {
    // (re)load the packed slice; the LDS also serves the cross-wave reduction
    const int units = nvalid * rowbytes / 16;
    for (int u = tid; u < units; u += 256) {
      const int byte = u * 16;
      const int r = byte / rowbytes;
      const int c = byte - r * rowbytes;
      *reinterpret_cast<u32x4_t*>(sB + r * ldsrow + c) = load16<ALIGN16>(gB + byte);
    }
    for (int u = tid; u < (ST_BN - nvalid) * ldsrow / 16; u += 256)
      reinterpret_cast<u32x4_t*>(sB + nvalid * ldsrow)[u] = u32x4_t{0u, 0u, 0u, 0u};
    for (int u = tid; u < ST_BN * G; u += 256) sS[u] = u < nvalid * G ? gS[u] : 0;
    __syncthreads();

    const int nrb = min(ST_MAXRB, (cnt - pass0 + 15) / 16);
    const uint16_t* arow[ST_MAXRB];
    bool aval[ST_MAXRB];
#pragma unroll
    for (int rb = 0; rb < ST_MAXRB; ++rb) {
      const int r = pass0 + rb * 16 + lr;
      aval[rb] = rb < nrb && r < cnt;
      const int64_t pos = row0 + (aval[rb] ? r : 0);
      const int64_t src = a.row_pair ? (int64_t)(a.row_pair[pos] / a.topk) : pos;
      arow[rb] = a.A + src * a.lda + lk * 8;
    }
    f32x4_t acc[ST_MAXRB][2];
#pragma unroll
    for (int rb = 0; rb < ST_MAXRB; ++rb) {
      acc[rb][0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      acc[rb][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    const uint8_t* b0p = sB + bc0 * ldsrow + lk * 4;
    const uint8_t* b1p = sB + bc1 * ldsrow + lk * 4;
    const uint8_t* s0p = sS + bc0 * G;
    const uint8_t* s1p = sS + bc1 * G;
    // this wave's k-steps: ks = wave + 4 * it
    const int nit = (G - wave + 3) / 4;
    s16x8_t abuf[ST_PF][ST_MAXRB];
#pragma unroll
    for (int p = 0; p < ST_PF; ++p) {
#pragma unroll
      for (int rb = 0; rb < ST_MAXRB; ++rb) {
        const int ks = wave + 4 * p;
        abuf[p][rb] = (p < nit && aval[rb])
                          ? *reinterpret_cast<const s16x8_t*>(arow[rb] + ks * 32)
                          : s16x8_t{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
    for (int it0 = 0; it0 < nit; it0 += ST_PF) {
#pragma unroll
      for (int p = 0; p < ST_PF; ++p) {
        const int it = it0 + p;
        if (it < nit) {
          const int ks = wave + 4 * it;
          s16x8_t acur[ST_MAXRB];
#pragma unroll
          for (int rb = 0; rb < ST_MAXRB; ++rb) {
            acur[rb] = abuf[p][rb];
            const int itn = it + ST_PF;
            if (itn < nit && aval[rb])
              abuf[p][rb] = *reinterpret_cast<const s16x8_t*>(arow[rb] + (wave + 4 * itn) * 32);
          }
          const uint32_t q0 = *reinterpret_cast<const uint32_t*>(b0p + ks * 16);
          const uint32_t q1 = *reinterpret_cast<const uint32_t*>(b1p + ks * 16);
          const s16x8_t bf0 = decode8(q0, s0p[ks]);
          const s16x8_t bf1 = decode8(q1, s1p[ks]);
#pragma unroll
          for (int rb = 0; rb < ST_MAXRB; ++rb) {
            if (rb < nrb) {
              acc[rb][0] = mfma16(acur[rb], bf0, acc[rb][0]);
              acc[rb][1] = mfma16(acur[rb], bf1, acc[rb][1]);
            }
          }
        }
      }
    }
    __syncthreads();  // all waves done with sB: reuse it for the reduction
#pragma unroll
    for (int rb = 0; rb < ST_MAXRB; ++rb) {
      sRed[((wave * ST_MAXRB + rb) * 2 + 0) * 64 + lane] = acc[rb][0];
      sRed[((wave * ST_MAXRB + rb) * 2 + 1) * 64 + lane] = acc[rb][1];
    }
    __syncthreads();
    if (wave < nrb) {
      const int rb = wave;
      f32x4_t c0 = f32x4_t{0.f, 0.f, 0.f, 0.f}, c1 = c0;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        c0 += sRed[((w * ST_MAXRB + rb) * 2 + 0) * 64 + lane];
        c1 += sRed[((w * ST_MAXRB + rb) * 2 + 1) * 64 + lane];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = pass0 + rb * 16 + lk * 4 + j;
        if (r >= cnt) continue;
        const int64_t pos = row0 + r;
        if constexpr (EPI == EPI_SWIGLU) {
          const int ng = n0 + 2 * lr;
          if (2 * lr + 1 < nvalid) epilogue_swiglu<EPI>(a, e, pos, ng, c0[j], c1[j]);
        } else {
          if (lr < nvalid) epilogue_one<EPI>(a, e, pos, n0 + lr, c0[j]);
          if (16 + lr < nvalid) epilogue_one<EPI>(a, e, pos, n0 + 16 + lr, c1[j]);
        }
      }
    }
    __syncthreads();  // reduction buffer is the next pass's weight slice
  }
}

// ---------------------------------------------------------------------------
// LDS-tiled kernel (prefill).
// ---------------------------------------------------------------------------
constexpr int TL_BM = 128;
constexpr int TL_BN = 128;
constexpr int TL_BK = 64;
constexpr int TL_LDK = TL_BK + 8;  // padded row, bf16 elements (144 bytes)

template <int EPI, bool ALIGN16>
__global__ __launch_bounds__(256, 2) void moe_tiled_kernel(GemmArgs a) {
  __shared__ __align__(16) uint16_t sA[2][TL_BM * TL_LDK];
  __shared__ __align__(16) uint16_t sB[2][TL_BN * TL_LDK];

  // XCD-aware order: workgroups dispatched round-robin over the 8 XCDs get
  // consecutive logical indices per XCD, so the column tiles of one row tile
  // (and the row tiles of one expert) share an L2.
  const int nblk = gridDim.x;  // multiple of 8
  const int L = (blockIdx.x & 7) * (nblk >> 3) + (blockIdx.x >> 3);
  const int tile = L / a.n_tiles_n;
  const int nt = L - tile * a.n_tiles_n;
  if (tile >= *a.num_tiles) return;
  const int2 te = a.tiles[tile];
  const int e = te.x;
  const int m0 = te.y;
  const int rows = min(TL_BM, a.offsets[e] + a.counts[e] - m0);
  const int n0 = nt * TL_BN;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int G = a.K / 32;
  const int KT = a.K / TL_BK;

  // A: 4 units of 16 bytes per thread per k-tile, fixed rows
  const uint16_t* aptr[4];
  bool aok[4];
  const int akc = tid & 7;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (tid >> 3) + 32 * i;
    aok[i] = r < rows;
    const int64_t pos = m0 + (aok[i] ? r : 0);
    const int64_t src = a.row_pair ? (int64_t)(a.row_pair[pos] / a.topk) : pos;
    aptr[i] = a.A + src * a.lda + akc * 8;
  }
  // B: one 16-byte packed unit (32 codes of one group) per thread per k-tile
  const int brr = tid >> 1;
  const int bgs = tid & 1;
  const bool bok = n0 + brr < a.N;
  const uint8_t* bq = a.Bq + ((int64_t)e * a.N + (bok ? n0 + brr : 0)) * G * 16 + bgs * 16;
  const uint8_t* bs = a.Bs + ((int64_t)e * a.N + (bok ? n0 + brr : 0)) * G + bgs;
  const int bcol = (EPI == EPI_SWIGLU) ? ((brr & 1) ? 64 + (brr >> 1) : (brr >> 1)) : brr;

  u32x4_t ra[4];
  u32x4_t rb;
  uint32_t rs;
  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ra[i] = aok[i] ? *reinterpret_cast<const u32x4_t*>(aptr[i] + kt * TL_BK)
                     : u32x4_t{0u, 0u, 0u, 0u};
    rb = bok ? load16<ALIGN16>(bq + kt * 32) : u32x4_t{0u, 0u, 0u, 0u};
    rs = bok ? (uint32_t)bs[kt * 2] : 127u;
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (tid >> 3) + 32 * i;
      *reinterpret_cast<u32x4_t*>(&sA[buf][r * TL_LDK + akc * 8]) = ra[i];
    }
    uint16_t* dst = &sB[buf][bcol * TL_LDK + bgs * 32];
    const bool hw = mx_scale_hw_ok(rs);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t d[4];
      mx_dword_to_bf16x8(rb[q], rs, hw, d);
      *reinterpret_cast<u32x4_t*>(dst + q * 8) = u32x4_t{d[0], d[1], d[2], d[3]};
    }
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int cb0 = (EPI == EPI_SWIGLU) ? 32 * wn : 64 * wn;
  const int cb1 = (EPI == EPI_SWIGLU) ? 64 + 32 * wn : 64 * wn + 32;
  const int l32 = lane & 31;
  const int lh = lane >> 5;

  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
    for (int kk = 0; kk < TL_BK / 16; ++kk) {
      s16x8_t af[2], bf[2];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
        af[mb] = *reinterpret_cast<const s16x8_t*>(
            &sA[buf][(wm * 64 + mb * 32 + l32) * TL_LDK + kk * 16 + lh * 8]);
      bf[0] = *reinterpret_cast<const s16x8_t*>(&sB[buf][(cb0 + l32) * TL_LDK + kk * 16 + lh * 8]);
      bf[1] = *reinterpret_cast<const s16x8_t*>(&sB[buf][(cb1 + l32) * TL_LDK + kk * 16 + lh * 8]);
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = mfma32(af[mb], bf[nb], acc[mb][nb]);
    }
    if (kt + 1 < KT) lstore(buf ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds column l32 of each 32x32 block, rows 8*(v/4) + 4*lh + v%4
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int r = wm * 64 + mb * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
      if (r >= rows) continue;
      const int64_t pos = m0 + r;
      if constexpr (EPI == EPI_SWIGLU) {
        const int ng = n0 + 2 * (32 * wn + l32);
        if (ng < a.N) epilogue_swiglu<EPI>(a, e, pos, ng, acc[mb][0][v], acc[mb][1][v]);
      } else {
        const int n_a = n0 + cb0 + l32;
        const int n_b = n0 + cb1 + l32;
        if (n_a < a.N) epilogue_one<EPI>(a, e, pos, n_a, acc[mb][0][v]);
        if (n_b < a.N) epilogue_one<EPI>(a, e, pos, n_b, acc[mb][1][v]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
enum Path : int { PATH_AUTO = 0, PATH_STREAM = 1, PATH_TILED = 2 };

static inline int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

struct Workspace {
  int* counts;
  int* offsets;
  int* row_pair;
  int* pair_pos;
  int2* tiles;
  int* num_tiles;
  uint16_t* act;  // [P][I] bf16 gated activations
  float* y;       // [P][H] f32 down-projection output (before the routing weight)
  int64_t bytes;
};

static Workspace carve(void* base, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k) {
  const int64_t P = T * k;
  const int64_t max_tiles = (P + TL_BM - 1) / TL_BM + E;
  char* p = static_cast<char*>(base);
  int64_t off = 0;
  Workspace w{};
  auto take = [&](int64_t bytes) {
    char* r = p ? p + off : nullptr;
    off = align_up(off + bytes, 256);
    return r;
  };
  w.counts = reinterpret_cast<int*>(take(E * 4));
  w.offsets = reinterpret_cast<int*>(take((E + 1) * 4));
  w.row_pair = reinterpret_cast<int*>(take(P * 4));
  w.pair_pos = reinterpret_cast<int*>(take(P * 4));
  w.tiles = reinterpret_cast<int2*>(take(max_tiles * 8));
  w.num_tiles = reinterpret_cast<int*>(take(4));
  w.act = reinterpret_cast<uint16_t*>(take(P * I * 2));
  w.y = reinterpret_cast<float*>(take(P * H * 4));
  w.bytes = off;
  return w;
}

template <int EPI>
static int launch_gemm(const GemmArgs& a, int path, int64_t P, hipStream_t st) {
  const bool align16 = (reinterpret_cast<uintptr_t>(a.Bq) % 16) == 0;
  if (path == PATH_STREAM) {
    const int slices = (a.N + ST_BN - 1) / ST_BN;
    const int64_t grid = (int64_t)a.E * slices;
    const size_t smem = st_smem_bytes(a.K);
    if (smem > 160 * 1024) {
      set_error("stream GEMM: K=%d needs %zu bytes of LDS", a.K, smem);
      return BSA_EINVAL;
    }
    if (align16)
      hipLaunchKernelGGL((moe_stream_kernel<EPI, true>), dim3((unsigned)grid), dim3(256), smem, st, a);
    else
      hipLaunchKernelGGL((moe_stream_kernel<EPI, false>), dim3((unsigned)grid), dim3(256), smem, st, a);
  } else {
    const int64_t max_tiles = (P + TL_BM - 1) / TL_BM + a.E;
    int64_t grid = max_tiles * a.n_tiles_n;
    grid = align_up(grid, 8);
    if (grid > INT32_MAX) {
      set_error("tiled GEMM: grid too large");
      return BSA_EINVAL;
    }
    if (align16)
      hipLaunchKernelGGL((moe_tiled_kernel<EPI, true>), dim3((unsigned)grid), dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((moe_tiled_kernel<EPI, false>), dim3((unsigned)grid), dim3(256), 0, st, a);
  }
  BSA_LAUNCH_CHECK("grouped GEMM launch");
  return BSA_OK;
}

static int pick_path(int path, int64_t P, int64_t E, int64_t K) {
  if (K % TL_BK != 0) return PATH_STREAM;  // the tiled kernel steps K by 64
  if (path != PATH_AUTO) return path;
  // rows per expert on average: weight streaming while they fit one or two
  // 16-row MFMA blocks, LDS tiles beyond
  return (P <= 16 * E) ? PATH_STREAM : PATH_TILED;
}

}  // namespace bsa

using namespace bsa;

extern "C" int bsa_moe_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                                       int64_t* bytes) {
  clear_error();
  BSA_REQUIRE(bytes, "workspace size: null output pointer");
  BSA_REQUIRE(T >= 0 && H > 0 && I > 0 && E > 0 && k > 0, "workspace size: bad shape");
  *bytes = carve(nullptr, T, H, I, E, k).bytes;
  return BSA_OK;
}

extern "C" int bsa_moe_experts_fwd(
    const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
    const int64_t* router_indices, const void* routing_weights, int weight_dtype,
    const void* gate_up_blocks, const void* gate_up_scales, const void* gate_up_bias,
    const void* down_blocks, const void* down_scales, const void* down_bias, int bias_dtype,
    float alpha, float limit, void* out, int out_dtype, void* workspace, int64_t workspace_bytes,
    void* save_gate_up, int path, void* stream) {
  clear_error();
  BSA_REQUIRE(T >= 0 && H > 0 && I > 0 && E > 0 && k > 0, "experts fwd: bad shape T=%lld H=%lld I=%lld E=%lld k=%lld",
              (long long)T, (long long)H, (long long)I, (long long)E, (long long)k);
  BSA_REQUIRE(H % 32 == 0 && I % 32 == 0, "experts fwd: hidden and intermediate must be multiples of 32");
  BSA_REQUIRE(E <= 1024, "experts fwd: at most 1024 experts (got %lld)", (long long)E);
  BSA_REQUIRE(k <= 16, "experts fwd: top-k at most 16 (got %lld)", (long long)k);
  BSA_REQUIRE(T * k < INT32_MAX / 2 && (T * k) * (2 * I) < INT64_MAX / 4, "experts fwd: too many tokens");
  BSA_REQUIRE(weight_dtype >= 0 && weight_dtype <= 2 && bias_dtype >= 0 && bias_dtype <= 2 &&
                  out_dtype >= 0 && out_dtype <= 2, "experts fwd: bad dtype code");
  BSA_REQUIRE(path >= 0 && path <= 2, "experts fwd: path must be 0, 1 or 2");
  if (T == 0) return BSA_OK;
  BSA_REQUIRE(hidden && router_indices && routing_weights && gate_up_blocks && gate_up_scales &&
                  down_blocks && down_scales && out && workspace,
              "experts fwd: null pointer");
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(hidden) % 16 == 0, "experts fwd: hidden must be 16-byte aligned");
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(gate_up_blocks) % 8 == 0 && reinterpret_cast<uintptr_t>(down_blocks) % 8 == 0,
              "experts fwd: packed blocks must be 8-byte aligned");
  const Workspace w = carve(workspace, T, H, I, E, k);
  BSA_REQUIRE(workspace_bytes >= w.bytes, "experts fwd: workspace of %lld bytes, need %lld",
              (long long)workspace_bytes, (long long)w.bytes);
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "experts fwd: workspace must be 256-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t P = T * k;

  int rc = launch_dispatch(router_indices, (int)P, (int)E, TL_BM, w.counts, w.offsets, w.row_pair,
                           w.pair_pos, w.tiles, w.num_tiles, st);
  if (rc) return rc;

  // gate_up: [P, H] x [2I, H]^T -> SwiGLU -> act [P, I] bf16
  GemmArgs g1{};
  g1.A = static_cast<const uint16_t*>(hidden);
  g1.lda = H;
  g1.row_pair = w.row_pair;
  g1.topk = (int)k;
  g1.Bq = static_cast<const uint8_t*>(gate_up_blocks);
  g1.Bs = static_cast<const uint8_t*>(gate_up_scales);
  g1.bias = gate_up_bias;
  g1.bias_dtype = bias_dtype;
  g1.counts = w.counts;
  g1.offsets = w.offsets;
  g1.E = (int)E;
  g1.N = (int)(2 * I);
  g1.K = (int)H;
  g1.out = w.act;
  g1.ldo = I;
  g1.out_dtype = DT_BF16;
  g1.save_pre = static_cast<float*>(save_gate_up);
  g1.alpha = alpha;
  g1.limit = limit;
  g1.tiles = w.tiles;
  g1.num_tiles = w.num_tiles;
  g1.n_tiles_n = (int)((2 * I + TL_BN - 1) / TL_BN);
  rc = launch_gemm<EPI_SWIGLU>(g1, pick_path(path, P, E, H), P, st);
  if (rc) return rc;

  // down: [P, I] x [H, I]^T + bias -> y [P, H] f32
  GemmArgs g2 = g1;
  g2.A = w.act;
  g2.lda = I;
  g2.row_pair = nullptr;
  g2.Bq = static_cast<const uint8_t*>(down_blocks);
  g2.Bs = static_cast<const uint8_t*>(down_scales);
  g2.bias = down_bias;
  g2.N = (int)H;
  g2.K = (int)I;
  g2.out = w.y;
  g2.ldo = H;
  g2.out_dtype = DT_F32;
  g2.save_pre = nullptr;
  g2.n_tiles_n = (int)((H + TL_BN - 1) / TL_BN);
  rc = launch_gemm<EPI_BIAS_F32>(g2, pick_path(path, P, E, I), P, st);
  if (rc) return rc;

  return launch_combine(w.y, router_indices, routing_weights, weight_dtype, w.pair_pos, (int)T,
                        (int)k, (int)H, out, out_dtype, st);
}
