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
// The same blocks may come in the k-pair shard layout (GemmArgs::kp,
// bq_off): every kernel only changes where it reads each 16-byte group from,
// the LDS contents and the results are the same bit for bit.
//
// Kernels:
//  * moe_stream_persist_kernel (decode, K = 2880): persistent workgroups,
//    two per CU, walking (expert, 16-row pass, 16-weight-row slice) items
//    through LDS DMA rings; the packed weights go to the block-scaled MFMA
//    as they are, against the activations split into two MXFP8 terms.
//    Bound: HBM (each hit expert's weights are read exactly once).
//  * moe_stream_parts_kernel (decode, K = 2880 with operands the persistent
//    kernel cannot DMA) and moe_stream_kernel (decode, any other K): one
//    workgroup per (expert, column slice), weights decoded to bf16 for
//    v_mfma_f32_16x16x32_bf16.
//  * moe_tiled2_kernel (prefill, 16-byte aligned operands): 128x256 output
//    tiles of one expert, BK=64, two LDS stages filled by global_load_lds
//    DMA, packed B decoded from LDS into MFMA operands by the one wave that
//    uses them, v_mfma_f32_32x32x16_bf16.  Bound: MFMA, in practice L1->L2
//    requests.
//  * moe_mx_kernel (prefill: chosen automatically above 16 routed rows per
//    expert on average):
//    128x256 tiles of one expert on the block-scaled
//    v_mfma_scale_f32_32x32x64_f8f6f4, the packed weights as they are
//    against activations split into two MXFP8 terms (hi, lo), two stages
//    of global_load_lds DMA and LDS reads issued half a step ahead of the
//    MFMAs (mx_split_step).  Bound: MFMA issue and the L2->LDS stream.
//  * moe_tiled_kernel (prefill for operands aligned to less than 16 bytes):
//    128x128 tiles, BK=64, register-staged LDS double buffering.
//  * moe_bwd_packed_kernel (the input-gradient backward): the packed weights
//    read along their rows (the reduction index) and decoded in registers.
// Weights are decoded with the gfx950 converter (v_cvt_scalef32_pk_bf16_fp4),
// which follows OCP MX: a block whose E8M0 scale byte is 255 (the NaN code)
// decodes to NaN, so the outputs it touches are NaN.  The reference's
// float32 ldexp gives +-inf there instead (and NaN for zero codes), which
// mixed-sign products also turn into NaN; the standalone dequant kernel
// reproduces the reference bit for bit, this case included.
//
// For the gate_up projection the weight rows interleave gate (even) and up
// (odd) columns (gptoss.py:131).  Every forward kernel places gate column j
// and up column j in the same lane (or adjacent lanes), so the clamped SwiGLU
// runs in registers.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "bsa_common.h"
#include "dispatch.h"

namespace bsa {

int launch_dispatch(const int64_t* idx, int P, int E, int BM, int* counts, int* offsets,
                    int* row_pair, int* pair_pos, int2* tiles, int* num_tiles, int* hist,
                    hipStream_t st);
int launch_combine(const float* Y, const int64_t* idx, const void* w, int w_dtype,
                   const int* pair_pos, int T, int k, int H, void* out, int out_dtype,
                   hipStream_t st);
int launch_bwd_prep(const void* dout, int dout_dtype, const float* y, const void* w, int w_dtype,
                    const int* pair_pos, int P, int k, int H, uint16_t* dy, float* grad_w,
                    hipStream_t st);
int launch_quant_mxfp8_split(const void* x, int in_dtype, int64_t R, int64_t K, int64_t ldx, const int* dest,
                             int topk, uint8_t* q, uint8_t* s, SplitLayout L, hipStream_t st);

enum Epi : int {
  EPI_SWIGLU = 0,    // out bf16 [P][N/2] = swiglu(acc + bias), optional f32 pre-activation save
  EPI_BIAS_F32 = 1,  // out f32 [P][N] = acc + bias
  EPI_STORE = 2,     // out (out_dtype) [P][N] = acc (+ bias if given)
  EPI_SWIGLU_BWD = 3,  // out bf16 [P][2N] = d(gate_up) from acc = d(act) and the forward's
                       // saved derivative factors save_grad [P][N] (bf16 pairs)
  EPI_SWIGLU_MX = 4,   // as EPI_SWIGLU, the bf16 activations then split into two MXFP8
                       // terms, stored in the SplitLayout {ldo, out_kt, ldos, out_s_kt}
                       // (codes at out, scale bytes at out_s)
};

struct GemmArgs {
  const uint16_t* A;     // bf16 activations, row stride lda
  int64_t lda;
  const int* row_pair;   // non-null: A row of sorted row pos is row_pair[pos] / topk
  int topk;
  const uint8_t* Bq;     // packed [E][N][K/32][16], or the k-pair layout when kp (below)
  const uint8_t* Bs;     // scales [E][N][K/32]
  const void* bias;      // [E][N] or null
  int bias_dtype;
  const int* counts;     // rows per expert
  const int* offsets;    // first sorted row per expert
  int E, N, K;
  void* out;
  int64_t ldo;
  int out_dtype;
  uint32_t* save_grad;   // EPI_SWIGLU: optional [P][N/2] bf16 pairs, the SwiGLU's derivative
                         // factors (swiglu_fwd_grad); EPI_SWIGLU_BWD reads them [P][N]
  float alpha, limit;
  const int2* tiles;     // tiled kernel: (expert, first sorted row) per row tile
  const int* num_tiles;
  int n_tiles_n;         // column tiles per row tile
  const uint8_t* Aq;     // MX path: split activations, k-tile-major: k-tile kt of sorted row
                         // pos at Aq + kt * ldq + pos * 128
  const uint8_t* As;     // MX path: their scale bytes, at As + kt * ldas + pos * 4 (+ 0, 1)
  int64_t ldq, ldas;
  int kp;                // Bq in the k-pair layout [E][N/16][K/64][16][2][16]
  uint8_t* out_s;        // EPI_SWIGLU_MX: scale bytes of the split activations
  int64_t ldos;
  int64_t out_kt, out_s_kt;  // EPI_SWIGLU_MX: k-tile strides of the codes and scales
  // decode gate_up with the dispatch folded in (moe_stream_persist_kernel):
  // non-null fuse_idx makes every workgroup first build the dispatch of its
  // fuse_P router indices (row tiles of fuse_bm) and write it -- every
  // workgroup the same values -- to the arrays counts / offsets / row_pair
  // above point to, and to pair_pos and the tile list, for the later launches
  const int64_t* fuse_idx;
  int fuse_P, fuse_bm;
  int* fuse_counts;
  int* fuse_offsets;
  int* fuse_row_pair;
  int* fuse_pair_pos;
  int2* fuse_tiles;
  int* fuse_num_tiles;
};


typedef __attribute__((ext_vector_type(8))) short s16x8_t;
typedef __attribute__((ext_vector_type(8))) int i32x8_t;

__device__ __forceinline__ f32x4_t mfma16(s16x8_t a, s16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma32(s16x8_t a, s16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// 8 MXFP4 codes (4 packed bytes) -> 8 bf16 in code order.  HW: the gfx950
// converter, valid when no scale byte in play is 255 (callers make that
// decision uniform across the wave); otherwise the integer decoder.
template <bool HW>
__device__ __forceinline__ s16x8_t decode8(uint32_t q, uint32_t s) {
  uint32_t d[4];
  if constexpr (HW) {
    const float sf = mx_scale_f32(s);
    d[0] = mx_byte_to_bf16x2_hw<0>(q, sf);
    d[1] = mx_byte_to_bf16x2_hw<1>(q, sf);
    d[2] = mx_byte_to_bf16x2_hw<2>(q, sf);
    d[3] = mx_byte_to_bf16x2_hw<3>(q, sf);
  } else {
    mx_dword_to_bf16x8(q, s, false, d);
  }
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

// block_streamer/gptoss.py:130-135 in float32 (the sigmoid's reciprocal by
// v_rcp_f32, within 1 ulp: an IEEE division is ten instructions, and the
// result is rounded to bf16 next).
__device__ __forceinline__ float swiglu(float g, float u, float alpha, float limit) {
  g = fminf(g, limit);
  u = fminf(fmaxf(u, -limit), limit);
  const float sig = __builtin_amdgcn_rcpf(1.0f + __expf(-alpha * g));
  return (u + 1.0f) * (g * sig);
}

// swiglu() and, for the backward, its partial derivatives w.r.t. the raw
// gate and up pre-activations as torch autograd differentiates
// gptoss.py:130-135: clamp(max=limit) passes the gradient where g <= limit,
// clamp(-limit, limit) where -limit <= u <= limit, and
// d(x * sigmoid(a x))/dx = s + a x s (1 - s).  The factors are returned as
// one bf16 pair (d act/d gate low, d act/d up high): the backward's
// d(gate, up) = d(act) * factors, with the clamp decisions taken here on
// the float32 pre-activations.
__device__ __forceinline__ float swiglu_fwd_grad(float g, float u, float alpha, float limit,
                                                 uint32_t* factors) {
  const float gc = fminf(g, limit);
  const float uc = fminf(fmaxf(u, -limit), limit);
  const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-alpha * gc));
  const float glu = gc * sg;
  const float fu = (u >= -limit && u <= limit) ? glu : 0.0f;
  const float fg = (g <= limit) ? (uc + 1.0f) * (sg + alpha * gc * sg * (1.0f - sg)) : 0.0f;
  *factors = pack_bf16x2_hw(fg, fu);
  return (uc + 1.0f) * glu;
}

// d(gate, up) as one bf16 pair from d(act) and the saved factors.
__device__ __forceinline__ uint32_t swiglu_bwd(uint32_t factors, float dout) {
  return pack_bf16x2_hw(dout * __uint_as_float(factors << 16), dout * __uint_as_float(factors & 0xFFFF0000u));
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
// Bias values are loaded once per lane before the K loop (each lane owns
// fixed columns) and passed in, so the epilogue issues no dependent loads.
template <int EPI>
__device__ __forceinline__ void epilogue_swiglu(const GemmArgs& a, int64_t pos, int n_gate,
                                                float accg, float accu, float bg, float bu) {
  const float g = accg + bg;
  const float u = accu + bu;
  float act;
  if (a.save_grad) {
    uint32_t f;
    act = swiglu_fwd_grad(g, u, a.alpha, a.limit, &f);
    a.save_grad[pos * (a.N >> 1) + (n_gate >> 1)] = f;
  } else {
    act = swiglu(g, u, a.alpha, a.limit);
  }
  static_cast<uint16_t*>(a.out)[pos * a.ldo + (n_gate >> 1)] = (uint16_t)f32_to_bf16_bits(act);
}

template <int EPI>
__device__ __forceinline__ void epilogue_one(const GemmArgs& a, int64_t pos, int n, float acc,
                                             float b) {
  const float v = acc + b;
  if constexpr (EPI == EPI_BIAS_F32) {
    static_cast<float*>(a.out)[pos * a.ldo + n] = v;
  } else if constexpr (EPI == EPI_SWIGLU_BWD) {
    *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.out) + pos * a.ldo + 2 * n) =
        swiglu_bwd(a.save_grad[pos * a.N + n], v);
  } else {
    store_out(a.out, a.out_dtype, pos * a.ldo + n, v);
  }
}


// Epilogue of one wave's (32*MB) x (32*NBW) block of a tiled kernel (MB x
// NBW blocks of 32 x 32 MFMA results: lane holds weight row n0w + 32*nb +
// (lane & 31), block rows 8*(v/4) + 4*(lane >> 5) + v%4), starting at row
// r0w of the tile, staged through the wave's own LDS (epi_lds_bytes) so that
// every global store is 16 contiguous bytes.
//  * EPI_SWIGLU: lanes 2j (gate) and 2j+1 (up) hold the same rows; the even
//    lane finishes rows v < 8 and the odd lane rows v >= 8, trading halves
//    with one shuffle; the bf16 activations of 32*MB rows x 16*NBW columns
//    go to LDS, then out to act[m0 + r][n0w/2 ..] (the optional saved
//    derivative factors, one bf16 pair per activation, are stored directly);
//  * EPI_BIAS_F32: 32 rows x 32*CB float32 at a time (CB = min(NBW, 2)).
// Needs 16-byte aligned output rows (ldo * element size % 16 == 0).
__host__ __device__ constexpr int epi_lds_bytes(int MB, int NBW) {
  return (1024 * MB * NBW > 4096 * (NBW < 2 ? NBW : 2)) ? 1024 * MB * NBW : 4096 * (NBW < 2 ? NBW : 2);
}

// The SwiGLU half of epilogue_staged: the wave's bf16 activations into its
// LDS staging t ([32*MB][16*NBW]), and with SAVE the derivative factors
// straight to a.save_grad (a separate instantiation, so the per-element
// loop carries no run-time branch).
template <bool SAVE, int MB, int NBW>
__device__ __forceinline__ void swiglu_to_lds(const GemmArgs& a, const f32x16_t (&acc)[MB][NBW],
                                              const float (&bias)[NBW], int m0, int r0w, int rows, int n0w,
                                              uint16_t* t, int lane) {
  constexpr int AC = 16 * NBW;  // activation columns of the wave
  const int l32 = lane & 31;
  const int lh = lane >> 5;
  const bool odd = l32 & 1;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
      const int ng = n0w + nb * 32 + (l32 & ~1);
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const float lo = acc[mb][nb][v] + bias[nb];
        const float hi = acc[mb][nb][v + 8] + bias[nb];
        const float recv = quad_xor1(odd ? lo : hi);
        const float g = odd ? recv : lo;
        const float u = odd ? hi : recv;
        const int vv = odd ? v + 8 : v;
        const int r = mb * 32 + 8 * (vv >> 2) + 4 * lh + (vv & 3);
        float act;
        if constexpr (SAVE) {
          uint32_t f;
          act = swiglu_fwd_grad(g, u, a.alpha, a.limit, &f);
          if (r0w + r < rows && ng + 1 < a.N) a.save_grad[(int64_t)(m0 + r0w + r) * (a.N >> 1) + (ng >> 1)] = f;
        } else {
          act = swiglu(g, u, a.alpha, a.limit);
        }
        t[r * AC + nb * 16 + (l32 >> 1)] = (uint16_t)bf16_bits_hw(act);
      }
    }
  }
}

template <int EPI, int MB, int NBW>
__device__ __forceinline__ void epilogue_staged(const GemmArgs& a, const f32x16_t (&acc)[MB][NBW],
                                                const float (&bias)[NBW], int m0, int r0w, int rows,
                                                int n0w, uint8_t* wl, int lane) {
  static_assert(EPI == EPI_SWIGLU || EPI == EPI_SWIGLU_MX || EPI == EPI_BIAS_F32, "staged epilogue");
  const int l32 = lane & 31;
  const int lh = lane >> 5;
  if constexpr (EPI == EPI_SWIGLU || EPI == EPI_SWIGLU_MX) {
    constexpr int AC = 16 * NBW;                   // activation columns of the wave
    uint16_t* t = reinterpret_cast<uint16_t*>(wl);  // [32*MB][AC] bf16
    if (a.save_grad)
      swiglu_to_lds<true>(a, acc, bias, m0, r0w, rows, n0w, t, lane);
    else
      swiglu_to_lds<false>(a, acc, bias, m0, r0w, rows, n0w, t, lane);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    constexpr int LPR = 2 * NBW;                   // lanes (16-byte pieces) per row
    const int half_n = a.N >> 1;
#pragma unroll
    for (int i = 0; i < MB * NBW; ++i) {
      const int r = i * (64 / LPR) + lane / LPR;
      const int ch = lane % LPR;
      const int c0 = (n0w >> 1) + ch * 8;
      const u32x4_t piece = *reinterpret_cast<const u32x4_t*>(wl + r * (2 * AC) + ch * 16);
      const bool ok = r0w + r < rows && c0 + 8 <= half_n;
      if constexpr (EPI == EPI_SWIGLU) {
        if (ok)
          *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(a.out) + (int64_t)(m0 + r0w + r) * a.ldo + c0) =
              piece;
      } else {
        // the four lanes ch & ~3 .. ch | 3 hold one 32-element block (c0 is
        // a multiple of 32 there: n0w / 2 is a multiple of 16 * NBW >= 32)
        float v[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[2 * j] = __uint_as_float(piece[j] << 16);
          v[2 * j + 1] = __uint_as_float(piece[j] & 0xFFFF0000u);
        }
        uint32_t hq[2], lq[2];
        const uint32_t sbyte = mx_split8(v, hq, lq);
        if (ok) {
          const int b = c0 >> 5;  // block of the row
          const int64_t row = m0 + r0w + r;
          uint8_t* q = static_cast<uint8_t*>(a.out) + row * a.ldo + (b >> 1) * a.out_kt + (b & 1) * 32 +
                       (ch & 3) * 8;
          *reinterpret_cast<uint2*>(q) = make_uint2(hq[0], hq[1]);
          *reinterpret_cast<uint2*>(q + 64) = make_uint2(lq[0], lq[1]);
          if ((ch & 3) == 0) a.out_s[row * a.ldos + (b >> 1) * a.out_s_kt + (b & 1)] = (uint8_t)sbyte;
        }
      }
    }
  } else {
    constexpr int CB = NBW < 2 ? NBW : 2;          // column blocks per staging round
    constexpr int WC = 32 * CB;                    // staged columns
    constexpr int LPR = 8 * CB;                    // lanes (16-byte pieces) per row
    float* t = reinterpret_cast<float*>(wl);       // [32][WC] float32
    float* out = static_cast<float*>(a.out);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int nc = 0; nc < NBW; nc += CB) {
#pragma unroll
        for (int nb = 0; nb < CB; ++nb)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            t[(8 * (v >> 2) + 4 * lh + (v & 3)) * WC + nb * 32 + l32] = acc[mb][nc + nb][v] + bias[nc + nb];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int i = 0; i < 4 * CB; ++i) {
          const int r = i * (64 / LPR) + lane / LPR;
          const int ch = lane % LPR;
          const int c0 = n0w + nc * 32 + ch * 4;
          if (r0w + mb * 32 + r < rows && c0 + 4 <= a.N)
            *reinterpret_cast<u32x4_t*>(out + (int64_t)(m0 + r0w + mb * 32 + r) * a.ldo + c0) =
                *reinterpret_cast<const u32x4_t*>(t + r * WC + ch * 4);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Weight-streaming kernel (decode).
//
// One workgroup per (expert, 32 consecutive weight rows).  The slice is one
// contiguous 32*K/2-byte span, copied to LDS at once.  K is walked in steps
// of 4 scale groups (128 k); in a step, the lane with column col = lane%16
// and quarter c = lane/16 decodes all 32 codes of group 4*step + c of its
// weight row (one 16-byte LDS read, one scale byte) and feeds them to four
// v_mfma_f32_16x16x32_bf16, whose k slots it fills with that group's codes
// [8m, 8m+8) for m = 0..3; the A lanes of quarter c read the same k.  The
// four waves take alternate steps and are summed through LDS.  Gate/up
// columns of the gate_up projection are adjacent lanes; the SwiGLU pairs
// them with one lane exchange.
// ---------------------------------------------------------------------------
constexpr int ST_BN = 32;  // weight rows (output columns) per workgroup

inline size_t st_smem_bytes(int K) {
  const size_t b = (size_t)ST_BN * (K / 2) + (size_t)ST_BN * (K / 32);
  const size_t red = (size_t)4 * 2 * 64 * sizeof(f32x4_t);
  return (b > red ? b : red) + 16;
}

// Cache-policy operand of global_load_lds for data that is read exactly once
// (the decode weight stream): the non-temporal bit (nt).  A read-bandwidth
// probe over 4 GiB measured 7.07 TB/s for 16-byte DMA with it against 6.27
// without, and 6.03 against 5.64 at two workgroups per CU; the decode layer
// at 64 tokens went from 0.262 to 0.236 ms.  It is set on the persistent
// decode kernel's stream.  The prefill and backward weight tiles keep the
// default policy: several row tiles re-read them from L2 (nt there made the
// prefill 45 % slower).
constexpr int CPOL_STREAM = 2;

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt not waited on)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Wait until at most min(ahead, MAXAHEAD) tiles of PER loads each are in
// flight.
template <int PER, int MAXAHEAD>
__device__ __forceinline__ void wait_tiles_ahead(int ahead) {
  if constexpr (MAXAHEAD <= 0) {
    wait_vmcnt<0>();
  } else {
    if (ahead >= MAXAHEAD) {
      wait_vmcnt<MAXAHEAD * PER>();
      return;
    }
    wait_tiles_ahead<PER, MAXAHEAD - 1>(ahead);
  }
}


// Copy `bytes` (a multiple of 16) from global to LDS.  DMA: gfx950
// global_load_lds_dwordx4, each wave moving 1 KiB per instruction with every
// load of the workgroup in flight at once (16-byte aligned source).
// Otherwise a register copy with 8-byte loads, 8 in flight per thread.
template <bool DMA>
__device__ __forceinline__ void copy_to_lds(uint8_t* dst, const uint8_t* src, int bytes, int tid) {
  if constexpr (DMA) {
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int chunks = (bytes + 1023) >> 10;
    for (int c = wave; c < chunks; c += 4) {
      const int off = (c << 10) + lane * 16;
      if (off < bytes)
        __builtin_amdgcn_global_load_lds(src + off, (lds_void*)(dst + (c << 10)), 16, 0, 0);
    }
  } else {
    const int units = bytes >> 4;
    for (int u0 = 0; u0 < units; u0 += 8 * 256) {
      u32x4_t r[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int u = u0 + tid + 256 * i;
        if (u < units) r[i] = load16<false>(src + u * 16);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int u = u0 + tid + 256 * i;
        if (u < units) *reinterpret_cast<u32x4_t*>(dst + u * 16) = r[i];
      }
    }
  }
}

// All 32 codes of one packed group (16 bytes) -> four 8-element bf16 operands.
template <bool HW>
__device__ __forceinline__ void decode32(const u32x4_t& q, uint32_t s, s16x8_t (&op)[4]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) op[m] = decode8<HW>(q[m], s);
}

template <int EPI, bool HW>
__device__ __forceinline__ void st_kloop(const GemmArgs& a, const uint8_t* sB, const uint8_t* sS,
                                         const uint16_t* arow, int wave, int col, int c,
                                         f32x4_t (&acc)[2]) {
  const int G = a.K / 32;
  const int nsteps = (G + 3) >> 2;
  const bool full_last = (G & 3) == 0;
  // A for this lane: the 64 contiguous bytes of group 4*step + c.  Rows past
  // the expert's count and groups past K read a clamped valid address: the
  // former are never stored, the latter meet zero B codes.
  u32x4_t an[4];
  auto loadA = [&](int step, u32x4_t (&dst)[4]) {
    const int g = min(4 * step + c, G - 1);
    const u32x4_t* p = reinterpret_cast<const u32x4_t*>(arow + g * 32);
#pragma unroll
    for (int m = 0; m < 4; ++m) dst[m] = p[m];
  };
  // LDS byte offsets of this lane's two weight rows, group c (the slice is
  // the tensor's bytes as they are), and the advance per 4-group step
  const uint32_t boff0 = (uint32_t)bq_off(a.kp, col, c, G);
  const uint32_t boff1 = (uint32_t)bq_off(a.kp, 16 + col, c, G);
  const uint32_t bstep = a.kp ? 1024u : 64u;
  const uint32_t soff0 = (uint32_t)(col * G + c);
  const uint32_t soff1 = (uint32_t)((16 + col) * G + c);
  if (wave < nsteps) loadA(wave, an);
  for (int step = wave; step < nsteps; step += 4) {
    u32x4_t ac[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) ac[m] = an[m];
    if (step + 4 < nsteps) loadA(step + 4, an);
    const uint32_t gofs = (uint32_t)(step * 4);
    u32x4_t q0 = *reinterpret_cast<const u32x4_t*>(sB + boff0 + step * bstep);
    u32x4_t q1 = *reinterpret_cast<const u32x4_t*>(sB + boff1 + step * bstep);
    uint32_t s0 = sS[soff0 + gofs];
    uint32_t s1 = sS[soff1 + gofs];
    if (!full_last && step == nsteps - 1 && 4 * step + c >= G) {
      // past the last group: zero codes (their LDS bytes may be another row's)
      q0 = u32x4_t{0u, 0u, 0u, 0u};
      q1 = q0;
      s0 = s1 = 127u;
    }
    s16x8_t bop[2][4];
    decode32<HW>(q0, s0, bop[0]);
    decode32<HW>(q1, s1, bop[1]);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const s16x8_t av = __builtin_bit_cast(s16x8_t, ac[m]);
      acc[0] = mfma16(av, bop[0][m], acc[0]);
      acc[1] = mfma16(av, bop[1][m], acc[1]);
    }
  }
}

template <int EPI, bool DMA>
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
  uint8_t* sB = smem;
  uint8_t* sS = smem + ST_BN * rowbytes;
  f32x4_t* sRed = reinterpret_cast<f32x4_t*>(smem);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;  // MFMA column (B) / row (A) within the block
  const int c = lane >> 4;    // quarter: group 4*step + c / C rows 4c..4c+3

  const uint8_t* gB = a.Bq + ((int64_t)e * a.N + n0) * rowbytes;
  const uint8_t* gS = a.Bs + ((int64_t)e * a.N + n0) * G;
  const float bias0 = col < nvalid ? bias_at(a.bias, a.bias_dtype, (int64_t)e * a.N + n0 + col) : 0.f;
  const float bias1 =
      16 + col < nvalid ? bias_at(a.bias, a.bias_dtype, (int64_t)e * a.N + n0 + 16 + col) : 0.f;

  for (int pass0 = 0; pass0 < cnt; pass0 += 16) {
    // (re)load the slice: its LDS also holds the cross-wave reduction
    copy_to_lds<DMA>(sB, gB, nvalid * rowbytes, tid);
    if (DMA && nvalid == ST_BN) {
      copy_to_lds<true>(sS, gS, ST_BN * G, tid);
    } else {
      for (int u = tid; u < ST_BN * G; u += 256) sS[u] = u < nvalid * G ? gS[u] : 0;
    }
    for (int u = tid; u < (ST_BN - nvalid) * rowbytes / 16; u += 256)
      reinterpret_cast<u32x4_t*>(sB + nvalid * rowbytes)[u] = u32x4_t{0u, 0u, 0u, 0u};
    if constexpr (DMA) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    const int r = pass0 + col;
    const int64_t pos = row0 + (r < cnt ? r : 0);
    const int64_t src = a.row_pair ? (int64_t)(a.row_pair[pos] / a.topk) : pos;
    const uint16_t* arow = a.A + src * a.lda;
    f32x4_t acc[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
    st_kloop<EPI, true>(a, sB, sS, arow, wave, col, c, acc);

    __syncthreads();  // all waves done with sB: reuse it for the reduction
    sRed[(wave * 2 + 0) * 64 + lane] = acc[0];
    sRed[(wave * 2 + 1) * 64 + lane] = acc[1];
    __syncthreads();
    if (wave < 2) {
      // wave b finishes column block b
      const int b = wave;
      f32x4_t v = sRed[(0 * 2 + b) * 64 + lane];
#pragma unroll
      for (int w = 1; w < 4; ++w) v += sRed[(w * 2 + b) * 64 + lane];
      const int n = n0 + 16 * b + col;
      const float bias = b ? bias1 : bias0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int rr = pass0 + 4 * c + j;
        const float val = v[j] + bias;
        if constexpr (EPI == EPI_SWIGLU) {
          // even column = gate, odd column = up of the same output index
          const float up = __shfl_xor(val, 1);
          if (rr < cnt && (col & 1) == 0 && 16 * b + col + 1 < nvalid)
            epilogue_swiglu<EPI>(a, row0 + rr, n, val, up, 0.f, 0.f);
        } else {
          if (rr < cnt && 16 * b + col < nvalid) epilogue_one<EPI>(a, row0 + rr, n, val, 0.f);
        }
      }
    }
    __syncthreads();  // the reduction buffer is the next pass's weight slice
  }
}

// ---------------------------------------------------------------------------
// Part-pipelined weight-streaming kernel (decode) for a K = 32*G known at
// compile time.  Same work split as moe_stream_kernel (one workgroup per
// expert x 32 weight rows; in 4-group k-step `step` the lane (col, c) of
// wave step % 4 handles group 4*step + c of weight rows col and 16 + col),
// but the slice streams in as parts of four k-steps (16 groups, 8 KiB) and
// each wave computes its step of part p as soon as part p has landed, while
// the later parts are still in flight.  vmcnt completes in order, so the A
// operands of every step of the wave are loaded into registers before the
// first DMA is issued; all DMA counts are compile-time constants, which
// keeps both the explicit part waits and the compiler's own waits exact.
// LDS part layout [32 rows][16 slots][16 bytes], group g of row r in slot
// (g % 16) ^ (r % 16), so the 16 rows read by one lane quarter hit 16
// different bank groups.  The cross-wave reduction reuses part 0, which a
// further pass over more than 16 rows reloads.
// ---------------------------------------------------------------------------
template <int EPI, int G>
__global__ __launch_bounds__(256, 3) void moe_stream_parts_kernel(GemmArgs a) {
  constexpr int NSTEPS = (G + 3) / 4;
  constexpr int NPART = (NSTEPS + 3) / 4;   // = k-steps per wave
  constexpr int PART = ST_BN * 16 * 16;     // 8 KiB
  constexpr int SCALE_BYTES = ST_BN * G;
  constexpr int SC_PIECES = (SCALE_BYTES + 1023) / 1024;
  constexpr int SC_PER_WAVE = (SC_PIECES + 3) / 4;
  static_assert(2 * NPART + SC_PER_WAVE < 64, "vmcnt range");
  __shared__ __align__(1024) uint8_t sB[NPART * PART];
  __shared__ __align__(1024) uint8_t sS[SC_PIECES * 1024];
  f32x4_t* sRed = reinterpret_cast<f32x4_t*>(sB);  // part 0, once every wave is done with it

  const int slices = a.N / ST_BN;
  const int e = blockIdx.x / slices;
  const int slice = blockIdx.x - e * slices;
  const int cnt = a.counts[e];
  if (cnt == 0) return;
  const int row0 = a.offsets[e];
  const int n0 = slice * ST_BN;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;
  const int c = lane >> 4;
  const uint8_t* gB = a.Bq + ((int64_t)e * a.N + n0) * G * 16;
  const uint8_t* gS = a.Bs + ((int64_t)e * a.N + n0) * G;

  // --- A operands of this wave's steps for rows 0..15, and the bias --------
  u32x4_t an[NPART][4];
  // (only lanes of existing rows load: at decode an expert has a few rows,
  // and the address unit would otherwise spend most of its time on copies of
  // row 0; the other lanes' operands are zero and their rows never stored)
  auto load_a = [](const GemmArgs& ga, int r0, int cn, int pass0, int cl, int cq, int wv,
                   u32x4_t (&dst)[NPART][4]) {
    const int r = pass0 + cl;
    if (r < cn) {
      const int64_t pos = r0 + r;
      const int64_t src = ga.row_pair ? (int64_t)(ga.row_pair[pos] / ga.topk) : pos;
      const uint16_t* arow = ga.A + src * ga.lda;
#pragma unroll
      for (int i = 0; i < NPART; ++i) {
        const int g = min(4 * (wv + 4 * i) + cq, G - 1);
        const u32x4_t* pp = reinterpret_cast<const u32x4_t*>(arow + g * 32);
#pragma unroll
        for (int m = 0; m < 4; ++m) dst[i][m] = pp[m];
      }
    } else {
#pragma unroll
      for (int i = 0; i < NPART; ++i)
#pragma unroll
        for (int m = 0; m < 4; ++m) dst[i][m] = u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  load_a(a, row0, cnt, 0, col, c, wave, an);
  const float bias0 = bias_at(a.bias, a.bias_dtype, (int64_t)e * a.N + n0 + col);
  const float bias1 = bias_at(a.bias, a.bias_dtype, (int64_t)e * a.N + n0 + 16 + col);

  // --- DMA: scales, then the parts in order --------------------------------
#pragma unroll
  for (int j = 0; j < SC_PER_WAVE; ++j) {
    const int q = min(wave + 4 * j, SC_PIECES - 1);
    const int off = q * 1024 + lane * 16;
    __builtin_amdgcn_global_load_lds(gS + (off + 16 <= SCALE_BYTES ? off : 0), (lds_void*)(sS + q * 1024),
                                     16, 0, 0);
  }
  // part p, piece i (2 per wave): rows 4i .. 4i+3, lane -> row 4i + lane/16,
  // slot lane%16 holding group 16p + ((lane%16) ^ (row%16)); groups past G
  // read group 0 (never used)
  auto issue_part = [](const uint8_t* gb, uint8_t* sb, int p, int wv, int ln, int kp) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = 2 * wv + j;
      const int row = 4 * i + (ln >> 4);
      const int g = 16 * p + ((ln & 15) ^ (row & 15));
      __builtin_amdgcn_global_load_lds(gb + bq_off(kp, row, g < G ? g : 0, G),
                                       (lds_void*)(sb + p * PART + i * 1024), 16, 0, 0);
    }
  };
#pragma unroll
  for (int p = 0; p < NPART; ++p) issue_part(gB, sB, p, wave, lane, a.kp);

  // LDS offsets of this lane's two rows (col, 16 + col) for its step of any
  // part: slot (4*wave + c) ^ col
  const uint32_t boff0 = (uint32_t)(col * 256 + (((4 * wave + c) ^ col) * 16));
  const uint32_t boff1 = (uint32_t)((16 + col) * 256 + (((4 * wave + c) ^ col) * 16));

  for (int pass0 = 0; pass0 < cnt; pass0 += 16) {
    if (pass0 > 0) {
      // part 0 held the reduction: reload it, and the A rows of this pass
      load_a(a, row0, cnt, pass0, col, c, wave, an);
      issue_part(gB, sB, 0, wave, lane, a.kp);
      wait_vmcnt<0>();
      asm volatile("s_barrier" ::: "memory");
    }
    f32x4_t acc[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int p = 0; p < NPART; ++p) {
      if (pass0 == 0) {
        // part p has landed once the later parts' pieces are all that is left
        wait_tiles_ahead<2, NPART - 1>(NPART - 1 - p);
        asm volatile("s_barrier" ::: "memory");
      }
      const int step = 4 * p + wave;
      if (step < NSTEPS) {
        const int g = 4 * step + c;
        u32x4_t q0 = *reinterpret_cast<const u32x4_t*>(sB + p * PART + boff0);
        u32x4_t q1 = *reinterpret_cast<const u32x4_t*>(sB + p * PART + boff1);
        uint32_t s0 = sS[col * G + (g < G ? g : 0)];
        uint32_t s1 = sS[(16 + col) * G + (g < G ? g : 0)];
        if (g >= G) {
          q0 = u32x4_t{0u, 0u, 0u, 0u};
          q1 = q0;
          s0 = s1 = 127u;
        }
        // decode one 8-code quarter of each row per MFMA pair (few live registers)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const s16x8_t av = __builtin_bit_cast(s16x8_t, an[p][m]);
          acc[0] = mfma16(av, decode8<true>(q0[m], s0), acc[0]);
          acc[1] = mfma16(av, decode8<true>(q1[m], s1), acc[1]);
        }
      }
    }

    // LDS-only synchronisation (a bare barrier after the LDS counter): a
    // __syncthreads() fence would also wait for outstanding global stores
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");  // every wave is done with part 0: it becomes sRed
    sRed[(wave * 2 + 0) * 64 + lane] = acc[0];
    sRed[(wave * 2 + 1) * 64 + lane] = acc[1];
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("s_barrier" ::: "memory");
    if (wave < 2) {
      const int b = wave;
      f32x4_t v = sRed[(0 * 2 + b) * 64 + lane];
#pragma unroll
      for (int w = 1; w < 4; ++w) v += sRed[(w * 2 + b) * 64 + lane];
      const int n = n0 + 16 * b + col;
      const float bias = b ? bias1 : bias0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int rr = pass0 + 4 * c + j;
        const float val = v[j] + bias;
        if constexpr (EPI == EPI_SWIGLU) {
          const float up = __shfl_xor(val, 1);  // even column = gate, odd = up
          if (rr < cnt && (col & 1) == 0) epilogue_swiglu<EPI>(a, row0 + rr, n, val, up, 0.f, 0.f);
        } else {
          if (rr < cnt) epilogue_one<EPI>(a, row0 + rr, n, val, 0.f);
        }
      }
    }
    if (pass0 + 16 < cnt) {
      // sRed (part 0) is reloaded by the next pass
      __builtin_amdgcn_s_waitcnt(0xC07F);
      asm volatile("s_barrier" ::: "memory");
    }
  }
}

// ---------------------------------------------------------------------------
// Persistent weight-streaming kernel (decode) for a K = 32*G known at compile
// time.  Persistent workgroups (WPC per CU) each walk a contiguous run of
// work items; an item is 16 weight rows (one 16x16x32 MFMA column block) of
// one expert against one 16-row pass of that expert's sorted rows, items
// ordered by (hit expert, pass, weight-row slice).  Consecutive items of a
// workgroup share the expert, so the A operands stay in registers and are
// reloaded only when the (expert, pass) changes.
//
// The items' packed bytes stream through a ring of NB LDS slots by
// global_load_lds DMA, NB - 1 items ahead of the computation.  A slot holds
// the item's blocks as G/16 parts [16 rows][16 slots][16 B], group g of row r
// in slot (g % 16) ^ r, so the 16 rows one lane quarter reads sit in 16
// different bank groups.  The last part has 16 - G % 16 unused slots per row
// (groups past G); they carry the item's 16*G scale bytes and its 16 bias
// values, chunk j (16 bytes) in row j / UN, slot (G % 16 + j % UN) ^ (j / UN).
// So every wave issues exactly G/16 DMA instructions per item and "item i
// has landed" is vmcnt <= (G/16) * (items issued after i).  The epilogue's
// stores also count in vmcnt; leaving them out of that bound only makes the
// wait stricter.  A reload of the A operands waits for everything.
//
// Waves split K as the part kernel does (wave w takes groups 16p + 4w + c).
// All four partial sums go through LDS; wave w finishes rows 4c + w, adding
// the partials in wave order, so results equal the part kernel's bit for bit.
// LDS reads of the ring are inline assembly: the compiler cannot tell which
// slot a computed address falls in, and for an ordinary LDS load it would
// wait for every global_load_lds in flight (vmcnt(0)), draining the ring.
// ---------------------------------------------------------------------------
constexpr int PS_TEAM_NB = 3;   // ring slots per team
constexpr int PS_TEAMS = 1;     // teams per workgroup (1: two workgroups per CU)

template <int G>
struct PsCfg {
  static constexpr int NP = (G + 15) / 16;                 // 4 KiB parts per item
  static constexpr int PART = 16 * 16 * 16;
  static constexpr int SLOT = NP * PART;
  static constexpr int UN = 16 * NP - G;                   // unused slots per row of the last part
  static constexpr int LAST = (NP - 1) * PART;
  static_assert(UN > 0 && 16 * UN >= G + 4, "scales and bias fit the last part's spare slots");
};

// LDS byte offset, within a slot, of byte b of spare chunk j.
template <int G>
__host__ __device__ constexpr uint32_t ps_chunk_off(int j, int b) {
  using C = PsCfg<G>;
  return (uint32_t)(C::LAST + (j / C::UN) * 256 + (((G % 16) + j % C::UN) ^ (j / C::UN)) * 16 + b);
}

// Position in a workgroup's item sequence: hit-list entry h (expert e with
// cnt rows), pass (16-row block of those rows), slice s (16 weight rows).
struct PsIt {
  int h, pass, s, e, cnt;
};

__device__ __forceinline__ void ps_entry(PsIt& it, const int* sHit) {
  const int v = __builtin_amdgcn_readfirstlane(sHit[it.h]);
  it.e = v & 0x3FF;
  it.cnt = v >> 10;
}

__device__ __forceinline__ void ps_next(PsIt& it, const int* sHit, int S, int nhit) {
  if (++it.s == S) {
    it.s = 0;
    if (++it.pass * 16 >= it.cnt) {
      it.pass = 0;
      if (++it.h < nhit) ps_entry(it, sHit);
    }
  }
}

// DMA of one item (expert e, weight rows n0 .. n0+15) into slot sb: G/16
// instructions per wave, wave w filling rows 4w .. 4w+3 of every part.
template <int G>
__device__ __forceinline__ void ps_issue(const GemmArgs& a, uint8_t* sb, int e, int n0, int wave,
                                         int lane, int eb) {
  using C = PsCfg<G>;
  const int64_t r0 = (int64_t)e * a.N + n0;
  const uint8_t* gB = a.Bq + r0 * (G * 16);
  const uint8_t* gS = a.Bs + r0 * G;
  const int row = 4 * wave + (lane >> 4);
  const int sl = (lane & 15) ^ row;
#pragma unroll
  for (int p = 0; p < C::NP; ++p) {
    const uint8_t* src = gB + bq_off(a.kp, row, 16 * p + sl, G);
    if (p == C::NP - 1 && 16 * p + sl >= G) {
      // a spare slot: scale chunk j, then the bias chunks, else anything valid
      const int j = row * C::UN + (16 * p + sl - G);
      if (j < G)
        src = gS + j * 16;
      else if (a.bias && (j - G) * 16 < 16 * eb)
        src = static_cast<const uint8_t*>(a.bias) + r0 * eb + (j - G) * 16;
      else
        src = gS;
    }
    __builtin_amdgcn_global_load_lds(src, (lds_void*)(sb + p * C::PART + wave * 1024), 16, 0, CPOL_STREAM);
  }
}

// Activations as two MXFP8 terms.  A bf16 block x (32 values sharing one
// E8M0 scale) is written hi + lo with
//   hi = E4M3(x / 2^X),              X = ceil(log2(amax|x| / 448)),
//   lo = E4M3((x - hi*2^X) / 2^(X-4)),
// both rounded to nearest even (v_cvt_scalef32_pk_fp8_f32 divides by the
// scale).  Every x/2^X is at most 448, where E4M3 steps are at most 32, so
// the residual is at most 16 * 2^X and lo at most 256: nothing saturates.  A
// bf16 value has 8 significant bits and E4M3 4, and E4M3 keeps 4 bits down to
// 2^-6: hi*2^X + lo*2^(X-4) equals x for every element above 2^-14 of the
// block maximum, and misses smaller ones by less than 2^-22 of it.  The
// packed MXFP4 weights then go to the block-scaled MFMA as they are, two
// instructions (hi, lo) per 128 k.
//
// 16 values of one lane (two u32x4 of bf16) -> 16 hi and 16 lo codes; the
// block is completed by the partner lane 16 lanes away (lane group c ^ 1).
// The hi scale byte (E8M0, X + 127) is returned; lo's is 4 less.
__device__ __forceinline__ int mx_block_exp(float amax) {
  const uint32_t ab = __float_as_uint(amax);
  const int e = (int)(ab >> 23) - 127;
  // significand above 1.75 needs the next exponent (448 = 1.75 * 2^8)
  const int X = e - 8 + ((ab & 0x7FFFFFu) > 0x600000u ? 1 : 0);
  return min(max(X, -126), 127);
}

__device__ __forceinline__ void mx_split16(const u32x4_t& v0, const u32x4_t& v1, bool valid, u32x4_t& hi,
                                           u32x4_t& lo, uint32_t& sh) {
  float f[16];
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    const uint32_t w = d < 4 ? v0[d] : v1[d - 4];
    f[2 * d] = valid ? __uint_as_float(w << 16) : 0.f;
    f[2 * d + 1] = valid ? __uint_as_float(w & 0xFFFF0000u) : 0.f;
  }
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) amax = fmaxf(amax, fabsf(f[j]));
  amax = fmaxf(amax, __shfl_xor(amax, 16));
  const int X = mx_block_exp(amax);
  const float s = __uint_as_float((uint32_t)(X + 127) << 23);
  float r[16];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    typedef short v2s __attribute__((ext_vector_type(2)));
    typedef float v2f __attribute__((ext_vector_type(2)));
    v2s q = {0, 0};
    q = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(q, f[4 * d], f[4 * d + 1], s, false);
    q = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(q, f[4 * d + 2], f[4 * d + 3], s, true);
    const uint32_t w = __builtin_bit_cast(uint32_t, q);
    hi[d] = w;
    const v2f d0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)w, s, false);
    const v2f d1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)w, s, true);
    r[4 * d] = f[4 * d] - d0[0];
    r[4 * d + 1] = f[4 * d + 1] - d0[1];
    r[4 * d + 2] = f[4 * d + 2] - d1[0];
    r[4 * d + 3] = f[4 * d + 3] - d1[1];
  }
  // 2^(X-4); X >= -126, so for X < -122 the float is subnormal-free only
  // down to 2^-126: clamp (such blocks hold values below 2^-118)
  const float sr = __uint_as_float((uint32_t)max(X + 123, 1) << 23);
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    typedef short v2s __attribute__((ext_vector_type(2)));
    v2s q = {0, 0};
    q = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(q, r[4 * d], r[4 * d + 1], sr, false);
    q = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(q, r[4 * d + 2], r[4 * d + 3], sr, true);
    lo[d] = __builtin_bit_cast(uint32_t, q);
  }
  sh = (uint32_t)(X + 127);
}

// v_mfma_scale_f32_16x16x128_f8f6f4 with E4M3 A, E2M1 B; the A scale is byte
// `sel` of sa (sel folds to a constant once the caller's loop is unrolled).
__device__ __forceinline__ f32x4_t mfma_mx16(const i32x8_t& a, const i32x8_t& b, f32x4_t c, uint32_t sa,
                                             int sel, uint32_t sb) {
  switch (sel) {
    case 0: return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 4, 0, (int)sa, 0, (int)sb);
    case 1: return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 4, 1, (int)sa, 0, (int)sb);
    case 2: return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 4, 2, (int)sa, 0, (int)sb);
    default: return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 4, 3, (int)sa, 0, (int)sb);
  }
}

// FP8 A operands (hi and lo) of this lane for pass `pass` of an expert whose
// sorted rows start at row0, for the 16x16x128 block-scaled MFMA over the
// 4-group window 16p + 4*wave of part p: lane group c holds k 16c .. 16c+15
// (bytes 0-15) and 64+16c .. 64+16c+15 (bytes 16-31) of the window and
// supplies the scale of window block c.  Rows past cnt repeat the last valid
// row (their outputs are never stored).  Scale bytes of parts 0-3 / 4-5 are
// packed into sh[0] / sh[1] (byte p % 4), likewise sl.
template <int G>
__device__ __forceinline__ void ps_load_a_raw(const GemmArgs& a, int row0, int cnt, int pass, int col, int c,
                                              int wave, u32x4_t (&raw)[PsCfg<G>::NP][4]) {
  constexpr int NP = PsCfg<G>::NP;
  const int r = min(pass * 16 + col, cnt - 1);
  const int64_t pos = row0 + r;
  const int64_t src = a.row_pair ? (int64_t)(a.row_pair[pos] / a.topk) : pos;
  const uint16_t* arow = a.A + src * a.lda;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int gw = 16 * p + 4 * wave;
    const int k0 = gw + (c >> 1) < G ? 32 * gw + 16 * c : 0;
    const int k1 = gw + 2 + (c >> 1) < G ? 32 * gw + 64 + 16 * c : 0;
    const u32x4_t* p0 = reinterpret_cast<const u32x4_t*>(arow + k0);
    const u32x4_t* p1 = reinterpret_cast<const u32x4_t*>(arow + k1);
    raw[p][0] = p0[0];
    raw[p][1] = p0[1];
    raw[p][2] = p1[0];
    raw[p][3] = p1[1];
  }
}

template <int G>
__device__ __forceinline__ void ps_quant_a(const u32x4_t (&raw)[PsCfg<G>::NP][4], int c, int wave,
                                           i32x8_t (&ah)[PsCfg<G>::NP], i32x8_t (&al)[PsCfg<G>::NP],
                                           uint32_t (&sh)[2], uint32_t (&sl)[2]) {
  constexpr int NP = PsCfg<G>::NP;
  sh[0] = sh[1] = sl[0] = sl[1] = 0u;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int gw = 16 * p + 4 * wave;
    u32x4_t h0, l0, h1, l1;
    uint32_t xh0, xh1;
    mx_split16(raw[p][0], raw[p][1], gw + (c >> 1) < G, h0, l0, xh0);
    mx_split16(raw[p][2], raw[p][3], gw + 2 + (c >> 1) < G, h1, l1, xh1);
    ah[p] = i32x8_t{(int)h0[0], (int)h0[1], (int)h0[2], (int)h0[3], (int)h1[0], (int)h1[1], (int)h1[2], (int)h1[3]};
    al[p] = i32x8_t{(int)l0[0], (int)l0[1], (int)l0[2], (int)l0[3], (int)l1[0], (int)l1[1], (int)l1[2], (int)l1[3]};
    // lane group c must supply the scale of window block c: groups 0 and 3
    // hold it (blocks 0 and 3 are their first / second halves), groups 1 and
    // 2 trade (block 1 is group 2's first half, block 2 group 1's second)
    const uint32_t offer_h = c == 1 ? xh1 : xh0;
    const uint32_t got_h = __shfl_xor(offer_h, 48);
    const uint32_t bh = c == 0 ? xh0 : (c == 3 ? xh1 : got_h);
    const uint32_t bl = bh > 4u ? bh - 4u : 1u;   // lo scale 2^(X-4), as in mx_split16
    sh[p >> 2] |= bh << (8 * (p & 3));
    sl[p >> 2] |= bl << (8 * (p & 3));
  }
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p);
}
__device__ __forceinline__ u32x4_t lds_read_b128(uint32_t addr) {
  u32x4_t r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}
__device__ __forceinline__ uint32_t lds_read_u8(uint32_t addr) {
  uint32_t r;
  asm volatile("ds_read_u8 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}
__device__ __forceinline__ uint32_t lds_read_b32(uint32_t addr) {
  uint32_t r;
  asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}

// Epilogue of one item: row rr of the pass (rows 4c + wave), column n; the
// four waves' partial sums are added in wave order.  The bias value (raw
// bits read from the item's slot) is bias_raw's half selected by col.
template <int EPI>
__device__ __forceinline__ void ps_epilogue(const GemmArgs& a, const f32x4_t* sRed, int lane, int wave,
                                            int col, uint32_t braw, int n, int rr, int cnt, int64_t row0) {
  const float* red = reinterpret_cast<const float*>(sRed) + lane * 4 + wave;
  float v = red[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) v += red[w * 256];
  float bias = 0.f;
  if (a.bias) {
    const int eb = a.bias_dtype == DT_F32 ? 4 : 2;
    const uint32_t bh = (col * eb) & 2 ? braw >> 16 : braw & 0xFFFFu;
    if (a.bias_dtype == DT_F32)
      bias = __uint_as_float(braw);
    else if (a.bias_dtype == DT_BF16)
      bias = __uint_as_float(bh << 16);
    else
      bias = (float)__builtin_bit_cast(_Float16, (uint16_t)bh);
  }
  const float val = v + bias;
  if constexpr (EPI == EPI_SWIGLU) {
    const float up = __shfl_xor(val, 1);  // even column = gate, odd = up
    if (rr < cnt && (col & 1) == 0) epilogue_swiglu<EPI>(a, row0 + rr, n, val, up, 0.f, 0.f);
  } else {
    if (rr < cnt) epilogue_one<EPI>(a, row0 + rr, n, val, 0.f);
  }
}

// TEAMS teams of four waves per workgroup, each team with its own
// PS_TEAM_NB-slot ring and its own share of the workgroup's contiguous run of
// items.  TEAMS = 2: one 512-thread workgroup per CU whose teams meet at every
// barrier, so both halves of a CU finish together.  TEAMS = 1: two
// independent 256-thread workgroups per CU (more overlap between them, but
// the CU serves them unevenly).
template <int EPI, int G, int TEAMS>
__global__ __launch_bounds__(256 * TEAMS, 3 - TEAMS) void moe_stream_persist_kernel(GemmArgs a) {
  using C = PsCfg<G>;
  constexpr int NP = C::NP;
  constexpr int NB = PS_TEAM_NB;
  constexpr int NT = 256 * TEAMS;                            // threads
  constexpr int MAXE = NT;                                   // experts the hit-list tables hold
  static_assert(NP == 6, "the ring reads below are written out for six parts");
  extern __shared__ __align__(1024) uint8_t ring[];          // TEAMS x NB slots
  __shared__ f32x4_t sRed[TEAMS * 4 * 64];                   // partial sums, [team][wave][lane]
  __shared__ int sHit[MAXE];                                 // e | cnt << 10, in expert order
  __shared__ int sRow0[MAXE];                                // first sorted row of entry h
  __shared__ int sSeg[2];                                    // each team's steps to its next reload
  int* sScan = reinterpret_cast<int*>(sRed);                 // prologue scratch: NT + 2 ints
  int* sHPre = sScan + NT + 2;                               // prologue: passes before entry h

  const int tid = threadIdx.x;
  if (a.fuse_idx) {
    // the dispatch, in the ring's LDS before any DMA lands there (E <= NT)
    int* s_cnt = reinterpret_cast<int*>(ring);
    int* s_off = s_cnt + NT;
    int* s_run = s_off + NT;
    int* s_dsc = s_run + NT;
    uint8_t(*s_wc)[NT] = reinterpret_cast<uint8_t(*)[NT]>(s_dsc + 2 * (NT / 64));
    dispatch_block<NT, NT>(a.fuse_idx, a.fuse_P, a.E, a.fuse_bm, a.fuse_counts, a.fuse_offsets, a.fuse_row_pair,
                           a.fuse_pair_pos, a.fuse_tiles, a.fuse_num_tiles, s_cnt, s_off, s_run, s_dsc, s_wc);
    __syncthreads();  // this workgroup's writes are visible to its reads below
  }
  const int lane = tid & 63;
  const int team = TEAMS == 2 ? __builtin_amdgcn_readfirstlane(tid >> 8) : 0;
  const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);   // wave within the team
  const int col = lane & 15;
  const int c = lane >> 4;
  const int S = a.N / 16;
  const int eb = a.bias_dtype == DT_F32 ? 4 : 2;

  // --- hit list: experts with rows, their pass prefix, in expert order -----
  const int cnt_t = tid < a.E ? a.counts[tid] : 0;
  const int off_t = tid < a.E ? a.offsets[tid] : 0;
  const int mine = (cnt_t > 0 ? 1 : 0) | (((cnt_t + 15) >> 4) << 16);
  // inclusive scan: shuffles within each wave, then the wave totals
  int incl = mine;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(incl, off);
    if (lane >= off) incl += v;
  }
  if (lane == 63) sScan[tid >> 6] = incl;
  __syncthreads();
  int last = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    const int v = sScan[w];
    if (w < (tid >> 6)) incl += v;
    last += v;
  }
  const int excl = incl - mine;
  if (cnt_t > 0) {
    sHit[excl & 0xFFFF] = tid | (cnt_t << 10);
    sHPre[excl & 0xFFFF] = excl >> 16;
    sRow0[excl & 0xFFFF] = off_t;
  }
  const int nhit = last & 0xFFFF;
  const int total = (last >> 16) * S;
  const int chunk = (total + (int)gridDim.x - 1) / (int)gridDim.x;
  const int start = (int)blockIdx.x * chunk;
  const int n_items = min(total - start, chunk);
  __syncthreads();
  if (n_items <= 0) return;
  // the workgroup's run: team 0 takes the first half, team 1 the rest
  const int half = TEAMS == 2 ? (n_items + 1) >> 1 : n_items;
  const int tstart = start + (team ? half : 0);
  const int tn = team ? n_items - half : half;   // team 1 may have one item less (or none)
  // entries holding each team's first pass
  if (tid < 2) sScan[NT + tid] = 0;
  __syncthreads();
  if (tid < nhit) {
    const int np = ((sHit[tid] >> 10) + 15) >> 4;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int q = min(start + (t ? half : 0), total - 1) / S;
      if (sHPre[tid] <= q && q < sHPre[tid] + np) sScan[NT + t] = tid;
    }
  }
  __syncthreads();
  PsIt ci;
  const int tq0 = min(tstart, total - 1) / S;
  ci.h = __builtin_amdgcn_readfirstlane(sScan[NT + team]);
  ps_entry(ci, sHit);
  ci.pass = tq0 - __builtin_amdgcn_readfirstlane(sHPre[ci.h]);
  ci.s = min(tstart, total - 1) - tq0 * S;
  PsIt ii = ci;
  __syncthreads();  // the prologue scratch becomes the partial-sum buffer

  uint8_t* tring = ring + team * (NB * C::SLOT);
  f32x4_t* tred = sRed + team * 256;

  // --- A operands of the first group (loaded before any DMA is in flight),
  // then the team's first NB items' DMA, then the quantisation -------------
  i32x8_t ah[NP], al[NP];   // FP8 hi / lo activation operands
  uint32_t sah[2], sal[2];   // their scale bytes, byte p % 4 of word p / 4
  int row0 = 0;
  if (tn > 0) {
    row0 = __builtin_amdgcn_readfirstlane(sRow0[ci.h]);
    u32x4_t raw[NP][4];
    ps_load_a_raw<G>(a, row0, ci.cnt, ci.pass, col, c, wave, raw);
    wait_vmcnt<0>();
    const int npre = min(NB, tn);
    for (int j = 0; j < npre; ++j) {
      ps_issue<G>(a, tring + j * C::SLOT, ii.e, ii.s * 16, wave, lane, eb);
      ps_next(ii, sHit, S, nhit);
    }
    ps_quant_a<G>(raw, c, wave, ah, al, sah, sal);
  }
  const uint32_t boff = (uint32_t)(col * 256 + (((4 * wave + c) ^ col) * 16));
  uint32_t soff[NP];  // this lane's scale byte of group 16p + 4*wave + c, row col
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int o = col * G + min(16 * p + 4 * wave + c, G - 1);
    soff[p] = ps_chunk_off<G>(o >> 4, o & 15);
  }
  const uint32_t bofs = ps_chunk_off<G>(G + (col * eb) / 16, ((col * eb) & 15) & ~3);
  const uint32_t ring0 = lds_addr(tring);

  // Per step k (one item per team, team item k): wait for its DMA, barrier,
  // finish the epilogue of item k-1 (its partial sums were written before
  // this barrier), read item k's slot into registers, barrier (the slot is
  // free), refill the slot with item k+NB, and only then multiply.  Segments
  // end where either team's (expert, pass) changes; that team then reloads
  // its A operands (waiting for everything it has in flight).
  const int nsteps = half;
  int k = 0;
  bool pend = false;                    // an item waits for its epilogue
  int p_n = 0, p_rr = 0, p_cnt = 0;     // that item's column, row, rows, first row
  int64_t p_row0 = 0;
  uint32_t p_braw = 0;
  while (true) {
    // steps until the next group change of either team
    const int mine_left = k < tn ? min(tn - k, S - ci.s) : nsteps - k;
    int seg_end = k + mine_left;
    if constexpr (TEAMS == 2) {
      // (LDS-only barriers: __syncthreads() would also wait for every DMA in flight)
      if (lane == 0 && wave == 0) sSeg[team] = mine_left;
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      asm volatile("s_barrier" ::: "memory");
      seg_end = k + min(sSeg[0], sSeg[1]);
      __builtin_amdgcn_s_waitcnt(0xC07F);
      asm volatile("s_barrier" ::: "memory");
    }
    for (; k < seg_end; ++k) {
      const bool act = k < tn;
      const int slot = k % NB;
      const uint32_t sb = ring0 + (uint32_t)(slot * C::SLOT);
      if (act) wait_tiles_ahead<NP, NB - 1>(min(NB - 1, tn - 1 - k));
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's partial sums are written
      asm volatile("s_barrier" ::: "memory");
      if (pend) ps_epilogue<EPI>(a, tred, lane, wave, col, p_braw, p_n, p_rr, p_cnt, p_row0);
      pend = false;

      u32x4_t q[NP];
      uint32_t sc[NP];
      uint32_t braw = 0;
      if (act) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          q[p] = lds_read_b128(sb + p * C::PART + boff);
          sc[p] = lds_read_u8(sb + soff[p]);
        }
        if (a.bias) braw = lds_read_b32(sb + bofs);
      }
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(q[4]), "+v"(q[5]),
                     "+v"(sc[0]), "+v"(sc[1]), "+v"(sc[2]), "+v"(sc[3]), "+v"(sc[4]), "+v"(sc[5]),
                     "+v"(braw));
      // every wave has its operands (and is done with the partial sums of
      // the previous item): the slot and the partial-sum buffer are free
      asm volatile("s_barrier" ::: "memory");
      if (act) {
        if (k + NB < tn) {
          ps_issue<G>(a, tring + slot * C::SLOT, ii.e, ii.s * 16, wave, lane, eb);
          ps_next(ii, sHit, S, nhit);
        }
        // groups past G meet zero activations (their slots hold scales)
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          if (16 * p + 4 * wave < G) {
            const i32x8_t bq = i32x8_t{(int)q[p][0], (int)q[p][1], (int)q[p][2], (int)q[p][3], 0, 0, 0, 0};
            acc = mfma_mx16(ah[p], bq, acc, sah[p >> 2], p & 3, sc[p]);
            acc = mfma_mx16(al[p], bq, acc, sal[p >> 2], p & 3, sc[p]);
          }
        }
        tred[wave * 64 + lane] = acc;
        pend = true;
        p_braw = braw;
        p_n = ci.s * 16 + col;
        p_rr = ci.pass * 16 + 4 * c + wave;
        p_cnt = ci.cnt;
        p_row0 = row0;
        ++ci.s;
      }
    }
    if (k >= nsteps) break;
    // this team's group changed: reload its A operands
    if (k < tn && ci.s == S) {
      ci.s = S - 1;
      ps_next(ci, sHit, S, nhit);
      row0 = __builtin_amdgcn_readfirstlane(sRow0[ci.h]);
      u32x4_t raw[NP][4];
      ps_load_a_raw<G>(a, row0, ci.cnt, ci.pass, col, c, wave, raw);
      wait_vmcnt<0>();
      ps_quant_a<G>(raw, c, wave, ah, al, sah, sal);
    }
  }
  // the last items' epilogues
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
  if (pend) ps_epilogue<EPI>(a, tred, lane, wave, col, p_braw, p_n, p_rr, p_cnt, p_row0);
}

// Logical tile index of this workgroup for the tiled kernels.  The live
// tiles (num_tiles row tiles x n_tiles_n column tiles; the row-tile count is
// only known on the device, the grid is sized for the maximum) are split
// into 8 equal contiguous chunks, one per XCD (workgroups are dispatched
// round-robin over the 8 XCDs): every XCD gets the same share of the work,
// and the tiles of one expert (tile_of orders them) stay on one XCD's L2.  -1: no tile for this workgroup.  Needs a grid that
// is a multiple of 8 and at least the live tile count.
__device__ __forceinline__ int xcd_tile_index(int live) {
  const int chunk = (live + 7) >> 3;
  const int slot = (int)(blockIdx.x >> 3);
  if (slot >= chunk) return -1;
  const int L = (int)(blockIdx.x & 7) * chunk + slot;
  return L < live ? L : -1;
}

#ifndef BSA_TILE_ORDER
#define BSA_TILE_ORDER 1
#endif

// Row tile and column tile of logical tile L.  The dispatch lists expert e's
// row tiles consecutively (tiles[t0 + j] = (e, offsets[e] + BM*j), j < c =
// ceil(counts[e] / BM)), so positions [t0*NT, (t0+c)*NT) belong to e; inside
// that run the c row tiles of one column tile come next to each other.  The
// workgroups that read one weight column tile then run together on one XCD
// and the later ones find it in that XCD's L2 (column tiles fastest would put
// NT - 1 other tiles between them).
template <int BM>
__device__ __forceinline__ void tile_of(const GemmArgs& a, int L, int& tile, int& nt) {
  const int NT = a.n_tiles_n;
#if BSA_TILE_ORDER
  const int tq = L / NT;
  const int2 q = a.tiles[tq];
  const int t0 = tq - (q.y - a.offsets[q.x]) / BM;
  const int c = (a.counts[q.x] + BM - 1) / BM;
  const int r = L - t0 * NT;
  nt = r / c;
  tile = t0 + (r - nt * c);
#else
  tile = L / NT;
  nt = L - tile * NT;
#endif
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

  const int L = xcd_tile_index(*a.num_tiles * a.n_tiles_n);
  if (L < 0) return;
  int tile, nt;
  tile_of<TL_BM>(a, L, tile, nt);
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
  const uint8_t* bq = a.Bq + (int64_t)e * a.N * G * 16 + bq_off(a.kp, bok ? n0 + brr : 0, bgs, G);
  const int bkt = a.kp ? 512 : 32;  // bytes per k-tile (two groups) along a row
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
    rb = bok ? load16<ALIGN16>(bq + kt * bkt) : u32x4_t{0u, 0u, 0u, 0u};
    rs = bok ? (uint32_t)bs[kt * 2] : 127u;
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (tid >> 3) + 32 * i;
      *reinterpret_cast<u32x4_t*>(&sA[buf][r * TL_LDK + akc * 8]) = ra[i];
    }
    uint16_t* dst = &sB[buf][bcol * TL_LDK + bgs * 32];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t d[4];
      mx_dword_to_bf16x8(rb[q], rs, true, d);
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
  // this lane's output columns and their biases
  const int ng_sw = n0 + 2 * (32 * wn + l32);
  const int n_a = n0 + cb0 + l32;
  const int n_b = n0 + cb1 + l32;
  const int64_t eb = (int64_t)e * a.N;
  float bias0 = 0.f, bias1 = 0.f;
  if constexpr (EPI == EPI_SWIGLU_BWD) {
  } else if constexpr (EPI == EPI_SWIGLU) {
    bias0 = ng_sw < a.N ? bias_at(a.bias, a.bias_dtype, eb + ng_sw) : 0.f;
    bias1 = ng_sw < a.N ? bias_at(a.bias, a.bias_dtype, eb + ng_sw + 1) : 0.f;
  } else {
    bias0 = n_a < a.N ? bias_at(a.bias, a.bias_dtype, eb + n_a) : 0.f;
    bias1 = n_b < a.N ? bias_at(a.bias, a.bias_dtype, eb + n_b) : 0.f;
  }

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
        if (ng_sw < a.N) epilogue_swiglu<EPI>(a, pos, ng_sw, acc[mb][0][v], acc[mb][1][v], bias0, bias1);
      } else {
        if (n_a < a.N) epilogue_one<EPI>(a, pos, n_a, acc[mb][0][v], bias0);
        if (n_b < a.N) epilogue_one<EPI>(a, pos, n_b, acc[mb][1][v], bias1);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Pipelined LDS-tiled kernel (prefill), 16-byte aligned operands.
//
// Tile 128 rows x 256 weight rows, BK = 64 (two scale groups), NS LDS stages
// filled only by global_load_lds DMA (no register staging).  The L1 -> L2
// path is limited by the number of requests, so every DMA covers contiguous
// runs:
//  * A stage [128][64] bf16, 8 lanes per row (128 contiguous bytes); row r's
//    16-byte chunk c is stored at chunk c ^ ((r >> 1) & 7), so fragment reads
//    are bank-conflict free (a ds_read_b128 pass serves 16 lanes from 64
//    banks, 256 bytes: two rows);
//  * B stage kept packed, [256 rows][2 groups][16 bytes], 2 lanes per row
//    (32 contiguous bytes), the two halves of row q swapped when bit 3 of q
//    is set (conflict-free 16-lane reads);
//  * the B scales of the tile's 256 weight rows, one contiguous 256*G-byte
//    span of the checkpoint tensor, are loaded once per tile.
// The four waves split N: each computes 128 x 64 (4 x 2 blocks of
// v_mfma_f32_32x32x16_bf16), so every B fragment is decoded by one wave
// only.  k order inside a group: MFMA m (0, 1) takes, in lane half lh,
// k = 16*lh + 8*m .. +8, for both A and B; a lane reads its row's whole
// 16-byte group once (rows consecutive: conflict free) and decodes its half.
// Bound: MFMA.
// ---------------------------------------------------------------------------
constexpr int T2_BM = 128;
constexpr int T2_BN = 256;
constexpr int T2_BK = 64;
constexpr int T2_A_BYTES = T2_BM * T2_BK * 2;          // 16 KiB
constexpr int T2_B_BYTES = T2_BN * 32;                 // 8 KiB
constexpr int T2_STAGE = T2_A_BYTES + T2_B_BYTES;
constexpr int T2_DMA_PER_TILE = 4 + 2;                 // per wave: A, B

// The E8M0 scales of weight rows n0 .. n0+BN-1 of expert e: bytes
// [(e*N + n0)*G, +BN*G) of the [E][N][G] tensor, one contiguous span, into
// LDS sbs [BN][G] with coalesced DMA (16-byte pieces when the tensor is
// 16-byte aligned -- the span start then is too, as N % 32 == 0 -- else
// 4-byte pieces).  Pieces past the expert's last row read the span's first
// piece instead (those rows are never used).  Issued by all WAVES waves.
template <bool SB16, int BN, int WAVES>
__device__ __forceinline__ void preload_b_scales(const uint8_t* Bs, int e, int N, int n0, int G,
                                                 uint8_t* sbs, int wave, int lane) {
  const uint8_t* span = Bs + ((int64_t)e * N + n0) * G;
  const int valid = min(BN, N - n0) * G;
  constexpr int PIECE = SB16 ? 16 : 4;
  const int npiece = BN * G / PIECE;
  for (int j = wave; j * 64 < npiece; j += WAVES) {
    const int c = j * 64 + lane;
    if (c < npiece) {
      const uint8_t* src = span + ((c + 1) * PIECE <= valid ? c * PIECE : 0);
      if constexpr (SB16)
        __builtin_amdgcn_global_load_lds(src, (lds_void*)(sbs + j * 64 * PIECE), 16, 0, 0);
      else
        __builtin_amdgcn_global_load_lds(src, (lds_void*)(sbs + j * 64 * PIECE), 4, 0, 0);
    }
  }
}

// One BK = 64 step of a wave's 128 x 64 block from LDS stage st, software
// pipelined by hand: the LDS reads for step s+1 are issued before the eight
// MFMAs of step s, and sched_barrier fences keep the compiler from sinking
// them back next to their uses, so each wait covers reads issued a full step
// (8 x 32 MFMA cycles) earlier.  Branch free.  Only the first NMB 32-row
// blocks are read and multiplied (the tile's rows; an expert's last row tile
// often holds fewer than 128).
template <int SCHED, int NMB>
__device__ __forceinline__ void t2_ktile(f32x16_t (&acc)[4][2], const uint8_t* st,
                                         const uint32_t (&sc)[2], const uint32_t (&aoff)[4],
                                         const uint32_t (&boff)[2], uint32_t bsw, int lh) {
  s16x8_t afr[2][4];
  u32x4_t bq[2][2];  // [h][nb] packed group of each B row
  auto loadA = [&](int step, s16x8_t (&dst)[4]) {
    const uint8_t* p = st + aoff[step];
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) dst[mb] = *reinterpret_cast<const s16x8_t*>(p + mb * 4096);
  };
  auto loadB = [&](int h) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
      bq[h][nb] = *reinterpret_cast<const u32x4_t*>(st + T2_A_BYTES + boff[nb] + ((h ^ bsw) * 16));
  };
  loadB(0);
  loadA(0, afr[0]);
  loadB(1);
  s16x8_t bop[2][2];
#pragma unroll
  for (int step = 0; step < 4; ++step) {
    const int h = step >> 1;
    const int m = step & 1;
    if (step + 1 < 4) loadA(step + 1, afr[(step + 1) & 1]);
    if constexpr (SCHED) __builtin_amdgcn_sched_barrier(0);
    if (m == 0) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const uint32_t sv = (sc[nb] >> (8 * h)) & 0xFFu;
        const uint32_t q0 = lh ? bq[h][nb][2] : bq[h][nb][0];
        const uint32_t q1 = lh ? bq[h][nb][3] : bq[h][nb][1];
        bop[nb][0] = decode8<true>(q0, sv);
        bop[nb][1] = decode8<true>(q1, sv);
      }
    }
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
      acc[mb][0] = mfma32(afr[step & 1][mb], bop[0][m], acc[mb][0]);
      acc[mb][1] = mfma32(afr[step & 1][mb], bop[1][m], acc[mb][1]);
    }
    if constexpr (SCHED) __builtin_amdgcn_sched_barrier(0);
  }
}

template <int EPI, int T2_NS, int SCHED, bool SB16>
__global__ __launch_bounds__(256, 2) void moe_tiled2_kernel(GemmArgs a) {
  extern __shared__ __align__(1024) uint8_t smem[];  // T2_NS stages, then [256][G] B scales
  const int L = xcd_tile_index(*a.num_tiles * a.n_tiles_n);
  if (L < 0) return;
  int tile, nt;
  tile_of<TL_BM>(a, L, tile, nt);
  const int2 te = a.tiles[tile];
  const int e = te.x;
  const int m0 = te.y;
  const int rows = min(T2_BM, a.offsets[e] + a.counts[e] - m0);
  const int n0 = nt * T2_BN;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // column quarter: weight rows 64*wave .. +64
  const int G = a.K / 32;
  const int KT = a.K / T2_BK;
  const int l32 = lane & 31;
  const int lh = lane >> 5;

  // --- per-lane DMA sources (every lane always issues all of them, so the
  //     per-wave vmcnt arithmetic below is exact; rows/columns past the tile
  //     read a clamped valid address and are never stored) ----------------
  const uint16_t* asrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 8 * (4 * wave + i) + (lane >> 3);
    const int ch = (lane & 7) ^ ((r >> 1) & 7);
    const int64_t pos = m0 + (r < rows ? r : 0);
    const int64_t src = a.row_pair ? (int64_t)(a.row_pair[pos] / a.topk) : pos;
    asrc[i] = a.A + src * a.lda + ch * 8;
  }
  // B: instruction i = 2*wave + h2 covers rows 32i .. 32i+31, 2 lanes per row;
  // row q's group h sits in half h ^ ((q >> 3) & 1) of its 32 bytes, so the
  // 16 rows of one LDS read pass hit 16 different 4-bank groups
  const uint8_t* bsrc[2];
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2) {
    const int q = 32 * (2 * wave + h2) + (lane >> 1);
    const bool ok = n0 + q < a.N;
    const int grp = (lane & 1) ^ ((q >> 3) & 1);
    bsrc[h2] = a.Bq + (int64_t)e * a.N * G * 16 + bq_off(a.kp, ok ? n0 + q : n0, grp, G);
  }
  const int bkt = a.kp ? 512 : 32;  // bytes per k-tile (two groups) along a row
  uint8_t* sbs = smem + T2_NS * T2_STAGE;
  preload_b_scales<SB16, T2_BN, 4>(a.Bs, e, a.N, n0, G, sbs, wave, lane);

  auto issue = [&](int kt) {
    uint8_t* st = smem + (kt % T2_NS) * T2_STAGE;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds(asrc[i] + kt * T2_BK,
                                       (lds_void*)(st + (4 * wave + i) * 1024), 16, 0, 0);
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2)
      __builtin_amdgcn_global_load_lds(bsrc[h2] + kt * bkt,
                                       (lds_void*)(st + T2_A_BYTES + (2 * wave + h2) * 1024), 16, 0, 0);
  };

  // this lane's two B rows (weight rows n0 + bq[nb]) and their bias
  int bq[2];
  float bias[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    bq[nb] = wave * 64 + nb * 32 + l32;
    const bool ok = n0 + bq[nb] < a.N;
    bias[nb] = ok ? bias_at(a.bias, a.bias_dtype, (int64_t)e * a.N + n0 + bq[nb]) : 0.f;
  }
  // LDS byte offsets (within a stage) of this lane's A fragments for step
  // (h, m): chunk 4h + 2lh + m of row l32 sits at chunk ^ ((row >> 1) & 7)
  // (16 lanes of one ds_read_b128 pass then cover all 64 banks: two
  // 128-byte rows share them); rows mb*32 + l32 add mb * 4096.  And of its
  // two B rows.
  const int rsw = (l32 >> 1) & 7;
  uint32_t aoff[4];
#pragma unroll
  for (int step = 0; step < 4; ++step) {
    const int h = step >> 1, m = step & 1;
    aoff[step] = (uint32_t)(l32 * 128 + (((4 * h + 2 * lh + m) ^ rsw) * 16));
  }
  // (half h of row q is at q*32 + ((h ^ bsw) * 16); bsw is the same for both rows)
  const uint32_t bsw = (uint32_t)((bq[0] >> 3) & 1);
  uint32_t boff[2] = {(uint32_t)(bq[0] * 32), (uint32_t)(bq[1] * 32)};

  f32x16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // a wave whose 64 weight rows all lie past N (in the last column tile)
  // multiplies nothing; it still issues its DMA share and meets every barrier.
  // nmb: the tile's 32-row blocks holding rows (the same for every wave).
  const bool live = n0 + wave * 64 < a.N;
  const int nmb = (rows + 31) >> 5;
  for (int i = 0; i < T2_NS - 1; ++i)
    if (i < KT) issue(i);
  // the k loop, one instantiation per live row-block count (a run-time
  // choice inside the loop body spilled the accumulators)
  auto kloop = [&](auto nmb_c) {
  constexpr int NMB = decltype(nmb_c)::value;
  for (int kt = 0; kt < KT; ++kt) {
    // this wave's DMA for tile kt has landed once at most one tile's worth
    // (the next tile's) is outstanding; the barrier then covers every wave.
    // A bare s_barrier: __syncthreads' release fence would wait for the
    // next tiles' loads too and serialise the pipeline.  The previous use of
    // the stage refilled below ended before this barrier (its LDS reads fed
    // MFMAs that have issued).
    // tiles issued after kt and still allowed in flight (the scale preload
    // is older than every tile, so the first wait covers it too)
    wait_tiles_ahead<T2_DMA_PER_TILE, T2_NS - 2>(min(T2_NS - 2, KT - 1 - kt));
    asm volatile("s_barrier" ::: "memory");
    if (kt + T2_NS - 1 < KT) issue(kt + T2_NS - 1);
    const uint8_t* st = smem + (kt % T2_NS) * T2_STAGE;
    // scale bytes of groups 2kt, 2kt+1 (G is even: a 2-byte aligned pair)
    uint32_t sc[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) sc[nb] = *reinterpret_cast<const uint16_t*>(sbs + bq[nb] * G + 2 * kt);
    if (live) t2_ktile<SCHED, NMB>(acc, st, sc, aoff, boff, bsw, lh);
  }
  };
  if (nmb == 4)
    kloop(std::integral_constant<int, 4>{});
  else if (nmb == 3)
    kloop(std::integral_constant<int, 3>{});
  else if (nmb == 2)
    kloop(std::integral_constant<int, 2>{});
  else
    kloop(std::integral_constant<int, 1>{});

  // epilogue through LDS: the stage buffers are free once every wave is done
  __syncthreads();
  epilogue_staged<EPI, 4, 2>(a, acc, bias, m0, 0, rows, n0 + wave * 64, smem + wave * 8192, lane);
}


// ---------------------------------------------------------------------------
// Native block-scaled MX kernel (prefill): the activations as two MXFP8
// terms (hi + lo, launch_quant_mxfp8_split) x MXFP4 weights on
// v_mfma_scale_f32_32x32x64_f8f6f4, two instructions per 64-element k-step,
// no weight decode at all.  The two terms hold every bf16 activation exactly
// unless it is below 2^-14 of its block's maximum, so the products are the
// bf16 path's up to the accumulation order.
//
// Operand layout of that instruction (measured on gfx950): for 32 x 32 x 64,
// lane l = 32*g + i supplies row/column i; its E2M1 operand is the 32
// consecutive K values 32g .. 32g+31 (nibble j = K offset j, low nibble
// first) -- exactly one packed 16-byte group of the checkpoint layout -- and
// its scale byte is that block's E8M0 scale; its E4M3 operand is K values
// 16g .. 16g+15 (bytes 0-15) and 32+16g .. 32+16g+15 (bytes 16-31), while
// its scale byte is still the scale of K block g.
//
// Tile 128 rows x BN weight rows, BK = 64 (two MX blocks), NS LDS stages
// filled only by global_load_lds DMA, every DMA covering whole contiguous
// runs:
//  * A stage [128][128 B]: per row the k-tile's 64 hi codes then 64 lo codes
//    (the split's row layout), 8 lanes per row; row r's 16-byte chunk c sits
//    at chunk c ^ ((r >> 1) & 7), so the fragment reads are bank-conflict
//    free (ds_read_b128 serves 16 lanes a cycle from 64 banks, i.e. 256
//    bytes: two 128-byte rows share the banks, so the swizzle pairs them);
//  * B stage [BN rows][2 groups][16 bytes], 2 lanes per row (32 contiguous
//    bytes, 512 in the k-pair layout), the two halves of row q swapped when
//    bit 3 of q is set;
//  * A scales, 4 B per row, per stage: the split writes the activations
//    k-tile-major (k-tile kt of sorted row p at kt*ldq + 128p, its two scale
//    bytes at kt*ldas + 4p), so a stage's codes and scales are each one
//    contiguous run; lo's scale byte is hi's minus 4;
//  * the B scales of the tile's BN weight rows, one contiguous BN*G-byte
//    span of the checkpoint tensor, are loaded once per tile.
// A 2 x WN grid of waves (default 2 x 2: each wave 64 rows x 128 weight rows,
// 2 x 4 blocks of 32 x 32, two workgroups per CU) splits the tile; 64 x 128
// per wave reads 12 LDS fragments per 16 MFMAs where 128 x 64 reads 18.
// Bound: the L2-to-LDS DMA rate and MFMA issue at the FP8 rate (two
// instructions per step: the bf16 rate), each alone close to the whole.
// ---------------------------------------------------------------------------

constexpr int MX_BM = 128;
constexpr int MX_BK = 64;
constexpr int MX_A_BYTES = MX_BM * MX_BK * 2;   // 16 KiB: hi and lo codes

// Activation row read for sorted row r of a tile that starts at sorted row
// m0 and holds `rows` rows (rows past the tile read the tile's first row).
// A device function, not a lambda: HIP-Clang does not emit the host-side
// handle of this kernel template when its body calls a capturing lambda.
__device__ __forceinline__ int64_t tile_src_row(const GemmArgs& a, int m0, int rows, int r) {
  const int64_t pos = m0 + (r < rows ? r : 0);
  return a.row_pair ? (int64_t)(a.row_pair[pos] / a.topk) : pos;
}

// Per-configuration sizes: a 2 x WN wave grid, wave (wm, wn) owning the two
// row blocks 2wm, 2wm+1 and NB column blocks of 32 x 32 (rows 64*wm ..,
// weight rows 32*NB*wn .. of the tile); BN = 32 * NB * WN weight rows per
// tile.  A stage holds the A codes (16 KiB), the A scale dwords and the B
// codes.  The scale dwords sit in one 256-byte slot per wave: its AS_ROWS
// rows, then padding that the wave's other lanes fill with copies, so the
// scale DMA is a whole-wave instruction (no divergent branch in the k loop).
// The B scales of the tile's weight rows are loaded once per tile (per-stage
// loads of their two bytes per row measured slower: one request per row).
template <int WN, int NB>
struct MxCfg {
  static constexpr int W = 2 * WN;                    // waves
  static constexpr int NBLK = NB;
  static constexpr int WCOLS = 32 * NB;
  static constexpr int BN = WCOLS * WN;
  static constexpr int B_BYTES = BN * 32;
  static constexpr int AS_ROWS = MX_BM / W;           // A scale rows per wave (one dword each)
  static constexpr int AS_BYTES = W * 256;
  static constexpr int AS_BLOCK = 32 / AS_ROWS * 256; // slot bytes per 32-row block
  static constexpr int B_OFF = MX_A_BYTES + AS_BYTES;
  static constexpr int STAGE = B_OFF + B_BYTES;
  static constexpr int A_DMA = 16 / W;                // A instructions per wave per stage
  static constexpr int B_DMA = BN / 32 / W;           // B instructions per wave per stage
  static constexpr int DMA_PER_TILE = A_DMA + 1 + B_DMA;
  static constexpr int EPI_LDS = epi_lds_bytes(2, NB);  // per-wave epilogue staging bytes
};

// Dynamic LDS bytes of moe_mx_kernel with ns stages: the stages and the B
// scales.
template <class C>
inline size_t mx_smem_bytes(int ns, int K) {
  return (size_t)ns * C::STAGE + (size_t)C::BN * (K / 32);
}

// Workgroups per CU (the launch bound); two hide each other's barrier and
// DMA waits, and the 2 x 2 wave grid's stages and B scales fit both in LDS.
#ifndef BSA_MX_WG_PER_CU
#define BSA_MX_WG_PER_CU 2
#endif

// Per-lane DMA sources (workgroup-uniform bases plus 32-bit per-lane
// offsets) and LDS read offsets of one tile, set up once.
template <class C>
struct MxLane {
  const uint8_t* abase;  // the tile's A codes, k-tile 0
  const uint8_t* sbase;  // the tile's A scale dwords, k-tile 0
  const uint8_t* bbase;  // the expert's packed weights
  uint32_t aoff_src[C::A_DMA];
  uint32_t soff_src;
  uint32_t boff_src[C::B_DMA];
  int64_t lda_kt, lds_kt;
  int bkt, wave, lane, G;
  uint32_t aoff0, aoff1, aoff2, aoff3, asoff, boff;
  const uint8_t* sb_row;
};

// A workgroup-uniform pointer as scalar registers: the DMA addresses then
// take the scalar-base form (base + 32-bit lane offset) instead of the
// compiler strength-reducing them into 64-bit per-lane induction variables.
__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo);
}

// Step kt's DMA into stage kt % MX_NS: the A codes, the A scale slot and
// the B codes.  A device function rather than a lambda: HIP-Clang does not
// emit the host-side handle of these kernel templates when their bodies call
// a capturing lambda.
template <class C, int MX_NS>
__device__ __forceinline__ void mx_issue(uint8_t* smem, int kt, const MxLane<C>& l) {
  uint8_t* st = smem + (kt % MX_NS) * C::STAGE;
  const int wave = l.wave;
  const uint8_t* a = uniform_ptr(l.abase + kt * l.lda_kt);
#pragma unroll
  for (int j = 0; j < C::A_DMA; ++j) {
    const uint8_t* src = a + l.aoff_src[j];
    __builtin_amdgcn_global_load_lds(src, (lds_void*)(st + (C::A_DMA * wave + j) * 1024), 16, 0, 0);
  }
  const uint8_t* ssrc = uniform_ptr(l.sbase + kt * l.lds_kt) + l.soff_src;
  __builtin_amdgcn_global_load_lds(ssrc, (lds_void*)(st + MX_A_BYTES + 256 * wave), 4, 0, 0);
  const uint8_t* b = uniform_ptr(l.bbase + (int64_t)kt * l.bkt);
#pragma unroll
  for (int h = 0; h < C::B_DMA; ++h) {
    const uint8_t* src = b + l.boff_src[h];
    __builtin_amdgcn_global_load_lds(src, (lds_void*)(st + C::B_OFF + (C::B_DMA * wave + h) * 1024), 16, 0, 0);
  }
}

// --- split-step pipeline ---------------------------------------------------
// Step kt's MFMAs run in two halves, row block 0 then row block 1, and every
// LDS read is issued one half ahead of the MFMAs that use it:
//   read A1(kt) | MFMAs row 0 (B(kt), A0(kt)) | wait for stage kt+1, barrier,
//   DMA step kt+NS into stage kt, read B(kt+1), A0(kt+1) | MFMAs row 1
//   (B(kt), A1(kt)).
// So a wave does not wait on its own LDS reads; B alternates between two
// register sets (row 1 still multiplies B(kt) while B(kt+1) lands), A0 and
// A1 are overwritten in place once their MFMAs have issued.  The one barrier
// per step certifies both that step kt+1 has landed and that every wave is
// done reading stage kt (its A1 reads are waited for before the barrier).

// Operands of one 32-row block of a 64-k step: hi and lo codes and hi's
// scale byte (lo's is max(sa - 4, 0)).
struct MxA {
  i32x8_t hi, lo;
  int sa;
};
// The NB column blocks' packed weights and scale bytes of a step.
template <int NB>
struct MxB {
  u32x4_t b[NB];
  int sb[NB];
};

template <int NB>
__device__ __forceinline__ void mx_read_b(MxB<NB>& f, const uint8_t* st, uint32_t boff, const uint8_t* sb_row, int G,
                                          int kt) {
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    f.sb[nb] = sb_row[nb * 32 * G + 2 * kt];
    f.b[nb] = *reinterpret_cast<const u32x4_t*>(st + boff + nb * 1024);
  }
}

// A row block's operands: ar = the stage's A codes + the block's first row,
// as = its scale byte.
__device__ __forceinline__ void mx_read_a(MxA& f, const uint8_t* ar, const uint8_t* as, uint32_t aoff0,
                                          uint32_t aoff1, uint32_t aoff2, uint32_t aoff3) {
  const u32x4_t w0 = *reinterpret_cast<const u32x4_t*>(ar + aoff0);
  const u32x4_t w1 = *reinterpret_cast<const u32x4_t*>(ar + aoff1);
  const u32x4_t w2 = *reinterpret_cast<const u32x4_t*>(ar + aoff2);
  const u32x4_t w3 = *reinterpret_cast<const u32x4_t*>(ar + aoff3);
  f.hi = i32x8_t{(int)w0[0], (int)w0[1], (int)w0[2], (int)w0[3], (int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3]};
  f.lo = i32x8_t{(int)w2[0], (int)w2[1], (int)w2[2], (int)w2[3], (int)w3[0], (int)w3[1], (int)w3[2], (int)w3[3]};
  f.sa = *as;
}

// One row block's MFMAs of a step, from the j0-th on: every column block's
// hi term, then every lo term (so the two products into one accumulator are
// NB MFMAs apart).  j0/j1 split the sequence, [j0, j1) of 2 * NB.
template <int NB, int J0 = 0, int J1 = 2 * NB>
__device__ __forceinline__ void mx_mfma_row(f32x16_t (&acc)[NB], const MxA& a, const MxB<NB>& b) {
#pragma unroll
  for (int j = J0; j < J1; ++j) {
    const int nb = j % NB;
    const i32x8_t bb = {(int)b.b[nb][0], (int)b.b[nb][1], (int)b.b[nb][2], (int)b.b[nb][3], 0, 0, 0, 0};
    if (j < NB)
      acc[nb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a.hi, bb, acc[nb], 0, 4, 0, a.sa, 0, b.sb[nb]);
    else
      acc[nb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a.lo, bb, acc[nb], 0, 4, 0, a.sa > 4 ? a.sa - 4 : 0,
                                                                0, b.sb[nb]);
  }
}

// s_waitcnt lgkmcnt(0) (vmcnt and expcnt not waited on)
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Step kt of the split-step pipeline for a wave holding NMB (0..2) row
// blocks of the tile; bc holds B(kt) and a0 A0(kt) (reads issued), bn
// receives B(kt+1).  ISSUE: whether this step issues step kt + MX_NS's DMA
// (decided per call site, so the steady-state steps are one basic block and
// the first half's MFMAs stay above the barrier).  On the last step the
// reads of "step kt+1" fetch a stale stage (in bounds, never used) and the
// wait and barrier are no-ops, so every wave passes KT + 1 barriers whatever
// NMB is.
template <class C, int MX_NS, int NMB, int ISSUE>
__device__ __forceinline__ void mx_split_step(f32x16_t (&acc)[2][C::NBLK], MxB<C::NBLK>& bc, MxB<C::NBLK>& bn,
                                              MxA& a0, MxA& a1, int kt, int KT, uint8_t* smem, const MxLane<C>& l) {
  constexpr int NB = C::NBLK;
  const uint8_t* st = smem + (kt % MX_NS) * C::STAGE;
  // the first MFMA before the A1 reads: its operands were read a half step
  // ago, and the wait the compiler puts before it then covers only them
  if constexpr (NMB > 0) mx_mfma_row<NB, 0, 1>(acc[0], a0, bc);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (NMB > 1)
    mx_read_a(a1, st + 32 * 128, st + l.asoff + C::AS_BLOCK, l.aoff0, l.aoff1, l.aoff2, l.aoff3);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (NMB > 0) mx_mfma_row<NB, 1, 2 * NB>(acc[0], a0, bc);
  __builtin_amdgcn_sched_barrier(0);
  // step kt+1 has landed for every wave, and every wave is done reading
  // stage kt (its A1 reads waited for here)
  if constexpr (ISSUE == 1)
    wait_vmcnt<(MX_NS - 2) * C::DMA_PER_TILE>();
  else
    wait_tiles_ahead<C::DMA_PER_TILE, MX_NS - 2>(min(MX_NS - 2, KT - 2 - kt));
  wait_lgkm0();
  asm volatile("s_barrier" ::: "memory");
  if constexpr (ISSUE == 1)
    mx_issue<C, MX_NS>(smem, kt + MX_NS, l);
  else if (kt + MX_NS < KT)
    mx_issue<C, MX_NS>(smem, kt + MX_NS, l);
  if constexpr (NMB > 0) {
    const uint8_t* sn = smem + ((kt + 1) % MX_NS) * C::STAGE;
    mx_read_b(bn, sn, l.boff, l.sb_row, l.G, min(kt + 1, KT - 1));
    mx_read_a(a0, sn, sn + l.asoff, l.aoff0, l.aoff1, l.aoff2, l.aoff3);
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (NMB > 1) mx_mfma_row(acc[1], a1, bc);
  __builtin_amdgcn_sched_barrier(0);
}

// The whole k loop: all MX_NS stages issued up front (after the B scales),
// then the steps two at a time (B's register sets swap roles): the steps
// that issue a later stage's DMA first (ISSUE = 1, no branch), then the
// last few with a run-time test (ISSUE = 0).  Ends with every DMA and LDS
// read complete.
template <class C, int MX_NS, int NMB>
__device__ __forceinline__ void mx_kloop(f32x16_t (&acc)[2][C::NBLK], int KT, uint8_t* smem, const MxLane<C>& l) {
  for (int i = 0; i < MX_NS; ++i)
    if (i < KT) mx_issue<C, MX_NS>(smem, i, l);
  wait_tiles_ahead<C::DMA_PER_TILE, MX_NS - 1>(min(MX_NS - 1, KT - 1));
  asm volatile("s_barrier" ::: "memory");
  MxB<C::NBLK> b0, b1;
  MxA a0, a1;
  if constexpr (NMB > 0) {
    mx_read_b(b0, smem, l.boff, l.sb_row, l.G, 0);
    mx_read_a(a0, smem, smem + l.asoff, l.aoff0, l.aoff1, l.aoff2, l.aoff3);
  }
  int kt = 0;
  for (; kt + 1 < KT - MX_NS; kt += 2) {
    mx_split_step<C, MX_NS, NMB, 1>(acc, b0, b1, a0, a1, kt, KT, smem, l);
    mx_split_step<C, MX_NS, NMB, 1>(acc, b1, b0, a0, a1, kt + 1, KT, smem, l);
  }
  for (; kt < KT; kt += 2) {
    mx_split_step<C, MX_NS, NMB, 0>(acc, b0, b1, a0, a1, kt, KT, smem, l);
    if (kt + 1 < KT) mx_split_step<C, MX_NS, NMB, 0>(acc, b1, b0, a0, a1, kt + 1, KT, smem, l);
  }
  wait_vmcnt<0>();
  wait_lgkm0();
}

template <int EPI, int MX_NS, bool SB16, int WM, int WN, int NB>
__global__ __launch_bounds__(64 * WM * WN, BSA_MX_WG_PER_CU) void moe_mx_kernel(GemmArgs a) {
  static_assert(WM == 2, "two row blocks per wave (the split-step pipeline)");
  using C = MxCfg<WN, NB>;
  constexpr int W = C::W;
  static_assert(MX_NS >= 2 && MX_NS <= 6, "pipeline depth");
  static_assert(W == 4 || W == 8, "wave grid");
  static_assert(C::B_DMA * W * 32 == C::BN, "B stage split over the waves");
  static_assert(32 % C::AS_ROWS == 0, "whole scale slots per row block");
  constexpr int BN = C::BN;
  extern __shared__ __align__(1024) uint8_t smem[];
  const int L = xcd_tile_index(*a.num_tiles * a.n_tiles_n);
  if (L < 0) return;
  int tile, nt;
  tile_of<TL_BM>(a, L, tile, nt);
  const int2 te = a.tiles[tile];
  const int e = te.x;
  const int m0 = te.y;
  const int rows = min(MX_BM, a.offsets[e] + a.counts[e] - m0);
  const int n0 = nt * BN;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN;   // rows 64*wm .. of the tile
  const int wn = wave % WN;   // weight rows WCOLS*wn .. of the tile
  const int G = a.K / 32;
  const int KT = a.K / MX_BK;
  const int l32 = lane & 31;
  const int lh = lane >> 5;
  uint8_t* sbs = smem + MX_NS * C::STAGE;  // [BN][G] B scales
  preload_b_scales<SB16, BN, W>(a.Bs, e, a.N, n0, G, sbs, wave, lane);

  // --- per-lane stage DMA sources (every lane always issues all of them, so
  //     the per-wave vmcnt arithmetic is exact; rows or columns past the tile
  //     are loaded from valid addresses and never stored) ------------------
  MxLane<C> l;
  // A: the tile's 128 sorted rows of k-tile kt are one contiguous 16 KiB run
  // (rows past the valid ones belong to the next expert, or to the 128 spare
  // rows at the end).  Instruction i = A_DMA*wave + j covers rows 8i .. 8i+7,
  // 8 lanes per row; row r's chunk c lands in slot c ^ ((r >> 1) & 7).
  l.abase = a.Aq + (int64_t)m0 * 128;
#pragma unroll
  for (int j = 0; j < C::A_DMA; ++j) {
    const int r = 8 * (C::A_DMA * wave + j) + (lane >> 3);
    l.aoff_src[j] = (uint32_t)(r * 128 + (((lane & 7) ^ ((r >> 1) & 7)) * 16));
  }
  // A scales: one dword (two scale bytes, two spare) per row; wave w's slot
  // holds rows AS_ROWS*w .. +AS_ROWS (lanes past AS_ROWS repeat them)
  l.sbase = a.As + (int64_t)m0 * 4;
  l.soff_src = (uint32_t)((C::AS_ROWS * wave + lane % C::AS_ROWS) * 4);
  // B: instruction i = B_DMA*wave + h covers rows 32i .. 32i+31, 2 lanes per
  // row; row q's group g sits in half g ^ ((q >> 3) & 1) of its 32 bytes
  l.bbase = a.Bq + (int64_t)e * a.N * G * 16;
#pragma unroll
  for (int h = 0; h < C::B_DMA; ++h) {
    const int q = 32 * (C::B_DMA * wave + h) + (lane >> 1);
    const int grp = (lane & 1) ^ ((q >> 3) & 1);
    l.boff_src[h] = (uint32_t)bq_off(a.kp, n0 + q < a.N ? n0 + q : n0, grp, G);
  }
  l.lda_kt = a.ldq;
  l.lds_kt = a.ldas;
  l.bkt = a.kp ? 512 : 32;  // bytes per k-tile (two groups) along a row
  l.wave = wave;
  l.lane = lane;
  l.G = G;

  // this lane's B rows (one per 32-column block) and their bias
  int bq[NB];
  float bias[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    bq[nb] = wn * C::WCOLS + nb * 32 + l32;
    const bool ok = n0 + bq[nb] < a.N;
    bias[nb] = ok ? bias_at(a.bias, a.bias_dtype, (int64_t)e * a.N + n0 + bq[nb]) : 0.f;
  }
  // LDS byte offsets of this lane's A chunks in row 64*wm + l32 (row block
  // 1: 32 rows on): hi codes in chunks lh and 2 + lh, lo codes in 4 + lh and
  // 6 + lh (the row's swizzle (r >> 1) & 7 does not depend on the row block)
  const int rsw = (l32 >> 1) & 7;
  const uint32_t abase = (uint32_t)(64 * wm * 128 + l32 * 128);
  l.aoff0 = abase + (uint32_t)((lh ^ rsw) * 16);
  l.aoff1 = abase + (uint32_t)(((2 + lh) ^ rsw) * 16);
  l.aoff2 = abase + (uint32_t)(((4 + lh) ^ rsw) * 16);
  l.aoff3 = abase + (uint32_t)(((6 + lh) ^ rsw) * 16);
  // the row's scale byte lh in its wave slot (row block 1: + AS_BLOCK)
  const int srow = 64 * wm + l32;
  l.asoff = (uint32_t)(MX_A_BYTES + (srow / C::AS_ROWS) * 256 + (srow % C::AS_ROWS) * 4 + lh);
  // B: half lh ^ bsw of row bq (bsw = bit 3 of the row, the same for every nb)
  l.boff = (uint32_t)(C::B_OFF + bq[0] * 32 + ((lh ^ ((bq[0] >> 3) & 1)) * 16));
  l.sb_row = sbs + bq[0] * G + lh;  // + nb*32*G + 2kt

  f32x16_t acc[2][NB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // Row blocks past the tile's rows are neither read nor multiplied (nmb: the
  // wave's row blocks holding rows of the tile, uniform across the wave; the
  // loop's barrier count does not depend on it).  Nor is anything of a wave
  // whose weight rows all lie past N (in the last column tile: half of it at
  // gate_up's N = 5760, and at down's N = 2880).
  const int nmb = n0 + wn * C::WCOLS < a.N ? min(2, max(0, (rows - 64 * wm + 31) / 32)) : 0;
  if (nmb == 2)
    mx_kloop<C, MX_NS, 2>(acc, KT, smem, l);
  else if (nmb == 1)
    mx_kloop<C, MX_NS, 1>(acc, KT, smem, l);
  else
    mx_kloop<C, MX_NS, 0>(acc, KT, smem, l);

  // epilogue through LDS: the stage buffers are free once every wave is done
  __syncthreads();
  epilogue_staged<EPI, 2, NB>(a, acc, bias, m0, 64 * wm, rows, n0 + wn * C::WCOLS, smem + wave * C::EPI_LDS, lane);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
enum Path : int { PATH_AUTO = 0, PATH_STREAM = 1, PATH_TILED = 2, PATH_MX = 3 };

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
  uint8_t* hq;    // MX path: split hidden rows per pair (in y's bytes) and scale bytes
  uint8_t* hs;
  uint8_t* aq;    // MX path: split activations (in act's bytes) and scale bytes
  uint8_t* as;
  int64_t rows_mx;  // rows of the MX split buffers: P plus MX_BM spare
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
  // MX path: the split hidden rows (one per pair, in sorted order, with
  // MX_BM spare rows after the last) are dead once gate_up is done, before
  // down writes y over them; the split activations take the place of the
  // bf16 ones.  Both are k-tile-major (SplitLayout); the scale bytes sit in
  // their own 4-byte-per-row arrays.
  const int64_t Pp = P + MX_BM;
  w.act = reinterpret_cast<uint16_t*>(take(Pp * I * 2));
  w.y = reinterpret_cast<float*>(take(std::max(P * H * 4, Pp * H * 2)));
  w.hq = reinterpret_cast<uint8_t*>(w.y);
  w.hs = reinterpret_cast<uint8_t*>(take(Pp * (H / 64) * 4));
  w.aq = reinterpret_cast<uint8_t*>(w.act);
  w.as = reinterpret_cast<uint8_t*>(take(Pp * (I / 64) * 4));
  w.rows_mx = Pp;
  w.bytes = off;
  return w;
}

// ---------------------------------------------------------------------------
// Backward products straight from the packed weights (no dense copy).
// out[pos][n] = sum_k A[pos][k] * W[e][k][n] where W is the MXFP4 checkpoint
// tensor read along its rows: Bq [E][K][N/32][16] (row k of expert e holds
// output columns n, 32 per block) and Bs [E][K][N/32].  For the input
// gradient, K is the forward GEMM's output index (2I for gate_up, H for
// down) and N its reduction index.  The scales vary along K within an MFMA's
// reduction, so the weights are decoded to bf16 (not the block-scaled MFMA).
//
// Tile 128 rows x 512 columns, BK = 64 weight rows, four waves, one
// workgroup per CU.  Wave w owns every row and columns 128w .. 128w+127; lane
// (c = lane & 31, g = lane >> 5) of MFMA column block j (0..3) is column
// 128w + 4c + j, so the lane's four columns are one packed 16-bit word per
// weight row.  Per 16-k step the lane reads, for its 8 rows k = 8g .. 8g+7,
// that word and the row's scale byte, converts each byte with
// v_cvt_scalef32_pk_bf16_fp4 (two columns of one row) and pairs rows with
// v_perm: 16 conversions + 16 permutes feed 16 MFMAs (4 x 4 blocks of
// v_mfma_f32_32x32x16_bf16), and the epilogue stores 4 contiguous columns.
// Stage (NS of them, global_load_lds DMA only):
//  * A [128][64] bf16, 16-byte chunk c of row r at chunk c ^ ((r >> 1) & 7)
//    (a ds_read_b128 pass serves 16 lanes from 64 banks: 256 bytes, two
//    rows, so the swizzle pairs rows);
//  * Q [64][256 B] packed weights, chunk c of row r at chunk c ^ (r & 15);
//  * S: the 16 scale bytes of each weight row (blocks 16 nt .. 16 nt + 15,
//    an unaligned run) as the two aligned 16-byte chunks that cover it;
//    rows 16 v .. 16 v + 15 at [v][row & 15][32 B] (1 KiB per wave's DMA,
//    lanes 32..63 repeating lanes 0..31).
// The byte offset of a row's run within its first chunk repeats every 64
// rows (64 * N/32 is a multiple of 16), so it is computed once per tile.
// ---------------------------------------------------------------------------
constexpr int BT_BM = 128;
static_assert(T2_BM == TL_BM && MX_BM == TL_BM && BT_BM == TL_BM,
              "tile_of and the dispatch's tile list use TL_BM rows per tile");
constexpr int BT_BN = 512;
constexpr int BT_BK = 64;
constexpr int BT_A_BYTES = BT_BM * BT_BK * 2;  // 16 KiB
constexpr int BT_Q_BYTES = BT_BK * BT_BN / 2;  // 16 KiB
constexpr int BT_S_BYTES = 4 * 1024;
constexpr int BT_STAGE = BT_A_BYTES + BT_Q_BYTES + BT_S_BYTES;
constexpr int BT_NS = 4;

// DMA sources of one workgroup tile.  The activations (this library's own
// buffers) always move in 16-byte pieces.  The packed weights move in 16-byte
// pieces when they are 16-byte aligned (QW4 = false: 4 instructions per wave
// per stage) and in 4-byte pieces otherwise (QW4 = true: 16; views into a
// staging blob are only 8-byte aligned); the scales likewise (SW4 = false: 1
// instruction, true: 2).  Either way the stage layout is the one described
// above.  The k-pair blocks layout takes the 16-byte weight pieces only.
template <bool QW4, bool SW4>
struct BtSrc {
  static constexpr int DMA_PER_TILE = 4 + (QW4 ? 16 : 4) + (SW4 ? 2 : 1);  // per wave: A, Q, S
  const uint16_t* asrc[4];
  const uint8_t* bq;
  const uint8_t* bs;
  int64_t q[QW4 ? 1 : 4];   // byte offsets into bq (QW4: of this lane's word in instruction 0)
  int64_t sc[SW4 ? 2 : 1];  // byte offsets into bs of this lane's chunk
  int qsw, qvalid;          // QW4: the lane's chunk position; valid chunks of the tile
  int64_t qrow, qstep, sstep, slast;

  __device__ __forceinline__ void init(const GemmArgs& a, int m0, int rows, int nt, int64_t wrow0, int NB,
                                       int wave, int lane) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 8 * (4 * wave + j) + (lane >> 3);
      const int ch = (lane & 7) ^ ((r >> 1) & 7);
      asrc[j] = a.A + tile_src_row(a, m0, rows, r) * a.lda + ch * 8;
    }
    bq = a.Bq;
    bs = a.Bs;
    qvalid = NB - nt * 16;  // chunks of the tile's columns that exist (>= 16: all)
    qrow = (int64_t)NB * 16;
    qstep = (int64_t)BT_BK * NB * 16;
    sstep = (int64_t)BT_BK * NB;
    slast = (int64_t)a.E * a.K * NB - 16;  // last whole chunk (the size is a multiple of 16)
    if constexpr (QW4) {
      // instruction j: weight row 16 wave + j, lane = 4-byte word of the row's
      // 256 bytes (checkpoint layout only)
      qsw = lane >> 2;
      q[0] = ((wrow0 + 16 * wave) * NB + nt * 16) * 16 + (lane & 3) * 4;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * (4 * wave + j) + (lane >> 4);
        const int c = (lane & 15) ^ (r & 15);
        q[j] = bq_off(a.kp, wrow0 + r, nt * 16 + (c < qvalid ? c : 0), NB);  // past N: any chunk
      }
    }
    if constexpr (SW4) {
      // instruction i: rows 16 wave + 8 i + lane / 8, word lane % 8 of the two chunks
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = 16 * wave + 8 * i + (lane >> 3);
        const int64_t o = (wrow0 + r) * NB + nt * 16;
        sc[i] = (o & ~(int64_t)15) + 16 * ((lane & 7) >> 2);
      }
    } else {
      // rows 16 wave .. +15, two chunks each; lanes 32..63 repeat 0..31
      const int r = 16 * wave + ((lane & 31) >> 1);
      const int64_t o = (wrow0 + r) * NB + nt * 16;
      sc[0] = (o & ~(int64_t)15) + 16 * (lane & 1);
    }
  }

  __device__ __forceinline__ void issue(uint8_t* smem, int kt, int wave, int lane) const {
    uint8_t* st = smem + (kt % BT_NS) * BT_STAGE;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_global_load_lds(asrc[j] + kt * BT_BK, (lds_void*)(st + (4 * wave + j) * 1024), 16, 0, 0);
    uint8_t* sq = st + BT_A_BYTES;
    uint8_t* ss = st + BT_A_BYTES + BT_Q_BYTES + wave * 1024;
    // the second chunk of the tensor's last rows may start past its end: read
    // the last whole chunk instead (those bytes are not used)
    if constexpr (QW4) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int c = qsw ^ j;  // row 16 wave + j keeps source chunk c at position qsw
        const int64_t off = q[0] + kt * qstep + j * qrow + (c < qvalid ? c : 0) * 16;
        __builtin_amdgcn_global_load_lds(bq + off, (lds_void*)(sq + (16 * wave + j) * 256), 4, 0, 0);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        __builtin_amdgcn_global_load_lds(bq + q[j] + kt * qstep, (lds_void*)(sq + (4 * wave + j) * 1024), 16, 0,
                                         0);
    }
    if constexpr (SW4) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
        __builtin_amdgcn_global_load_lds(bs + min(sc[i] + kt * sstep, slast) + (lane & 3) * 4,
                                         (lds_void*)(ss + i * 256), 4, 0, 0);
    } else {
      __builtin_amdgcn_global_load_lds(bs + min(sc[0] + kt * sstep, slast), (lds_void*)ss, 16, 0, 0);
    }
  }
};

// Step s's weight words (one 16-bit word per row: the lane's 4 columns) and
// scale bytes of the lane's 8 rows.
__device__ __forceinline__ void bt_read_q(const uint8_t* st, int s, const uint32_t (&qa)[8],
                                          const uint32_t (&sa)[8], uint32_t (&raw)[8], uint32_t (&sb)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    raw[i] = *reinterpret_cast<const uint16_t*>(st + qa[i] + 4096 * s);
    sb[i] = st[sa[i] + 1024 * s];
  }
}

// The NMB 32-row A fragments of one 16-k step (aoff: the step's offset).
template <int NMB>
__device__ __forceinline__ void bt_read_a(const uint8_t* st, uint32_t aoff, s16x8_t (&af)[NMB]) {
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb) af[mb] = *reinterpret_cast<const s16x8_t*>(st + aoff + mb * 4096);
}

// 8 rows x 4 columns of E2M1 codes -> the 4 columns' B fragments (8 k values
// each, rows in order, two per dword).
__device__ __forceinline__ void bt_decode(const uint32_t (&raw)[8], const uint32_t (&sb)[8], u32x4_t (&bq)[4]) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const float s0 = mx_scale_f32(sb[2 * d]), s1 = mx_scale_f32(sb[2 * d + 1]);
    const uint32_t lo0 = mx_byte_to_bf16x2_hw<0>(raw[2 * d], s0);
    const uint32_t lo1 = mx_byte_to_bf16x2_hw<0>(raw[2 * d + 1], s1);
    const uint32_t hi0 = mx_byte_to_bf16x2_hw<1>(raw[2 * d], s0);
    const uint32_t hi1 = mx_byte_to_bf16x2_hw<1>(raw[2 * d + 1], s1);
    bq[0][d] = pack_lo16(lo0, lo1);
    bq[1][d] = pack_hi16(lo0, lo1);
    bq[2][d] = pack_lo16(hi0, hi1);
    bq[3][d] = pack_hi16(hi0, hi1);
  }
}

// Four adjacent output columns n .. n+3 of row pos; fac holds the row's saved
// derivative factors of those columns (EPI_SWIGLU_BWD).
template <int EPI>
__device__ __forceinline__ void bt_store4(const GemmArgs& a, int64_t pos, int n, const float (&v)[4],
                                          const u32x4_t& fac) {
  if constexpr (EPI == EPI_SWIGLU_BWD) {
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = swiglu_bwd(fac[j], v[j]);
    *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(a.out) + pos * a.ldo + 2 * n) = o;
  } else {
    static_assert(EPI == EPI_STORE, "packed-weight backward epilogue");
    f32x4_t o = {v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4_t*>(static_cast<float*>(a.out) + pos * a.ldo + n) = o;
  }
}

// One tile with NMB live 32-row blocks (rows <= 32 NMB): the A reads, MFMAs,
// accumulators and epilogue of the blocks past them are left out (an
// expert's last row tile often holds a few rows only).
template <int EPI, bool QW4, bool SW4, int NMB>
__device__ __forceinline__ void bt_tile(const GemmArgs& a, uint8_t* smem, int e, int m0, int rows, int nt) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31;
  const int g = lane >> 5;
  const int KT = a.K / BT_BK;
  const int NB = a.N >> 5;               // scale bytes (and 16-byte chunks) per weight row
  const int64_t wrow0 = (int64_t)e * a.K;  // first weight row of the expert

  BtSrc<QW4, SW4> src;
  src.init(a, m0, rows, nt, wrow0, NB, wave, lane);
  constexpr int DPT = BtSrc<QW4, SW4>::DMA_PER_TILE;

  // --- fragment addresses (step s adds 4096 s to Q, 1024 s to S) -------------
  uint32_t aoff[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) aoff[s] = (uint32_t)(c * 128 + (((2 * s + g) ^ ((c >> 1) & 7)) * 16));
  uint32_t qa[8], sa[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int rr = 8 * g + i;  // row within the 16-row step
    qa[i] = (uint32_t)(BT_A_BYTES + rr * 256 + (((4 * wave + (c >> 3)) ^ rr) * 16) + 2 * (c & 7));
    const int run = (int)(((wrow0 + rr) * NB) & 15);
    sa[i] = (uint32_t)(BT_A_BYTES + BT_Q_BYTES + rr * 32 + run + 4 * wave + (c >> 3));
  }

  f32x16_t acc[NMB][4];
#pragma unroll
  for (int i = 0; i < NMB; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // Software pipeline: during step s of tile kt the wave runs step s's 16
  // MFMAs, decodes step s+1's B fragments (words read one step earlier) and
  // reads step s+1's A fragments and step s+2's weight words -- across the
  // tile boundary, from tile kt+1's stage.  So the barrier at the top of
  // iteration kt certifies tile kt+1 (tile kt was certified one iteration
  // earlier), and the stage refilled there (kt+3's, last read for tile kt-1)
  // is free.  Words of step t sit in buffer t % 2.
  for (int i = 0; i < BT_NS - 1; ++i)
    if (i < KT) src.issue(smem, i, wave, lane);
  wait_tiles_ahead<DPT, BT_NS - 2>(min(BT_NS - 2, KT - 1));
  asm volatile("s_barrier" ::: "memory");
  uint32_t raw0[8], sb0[8], raw1[8], sb1[8];
  s16x8_t af[NMB];
  u32x4_t bq[4];
  bt_read_q(smem, 0, qa, sa, raw0, sb0);
  bt_read_q(smem, 1, qa, sa, raw1, sb1);
  bt_read_a<NMB>(smem, aoff[0], af);
  bt_decode(raw0, sb0, bq);
  for (int kt = 0; kt < KT; ++kt) {
    // tile kt+1 has landed once at most the tiles issued after it are in
    // flight; a bare s_barrier (a __syncthreads() fence would wait for them too)
    wait_tiles_ahead<DPT, BT_NS - 3>(KT - 2 - kt);
    asm volatile("s_barrier" ::: "memory");
    if (kt + BT_NS - 1 < KT) src.issue(smem, kt + BT_NS - 1, wave, lane);
    const uint8_t* st = smem + (kt % BT_NS) * BT_STAGE;
    // past the last tile this stage holds stale data: read, never used
    const uint8_t* sn = smem + ((kt + 1) % BT_NS) * BT_STAGE;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      s16x8_t afn[NMB];
      bt_read_a<NMB>(s < 3 ? st : sn, aoff[(s + 1) & 3], afn);
      if (s % 2 == 0)
        bt_read_q(s < 2 ? st : sn, (s + 2) & 3, qa, sa, raw0, sb0);
      else
        bt_read_q(s < 2 ? st : sn, (s + 2) & 3, qa, sa, raw1, sb1);
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[mb][j] = mfma32(af[mb], __builtin_bit_cast(s16x8_t, bq[j]), acc[mb][j]);
      u32x4_t bqn[4];
      if (s % 2 == 0)
        bt_decode(raw1, sb1, bqn);
      else
        bt_decode(raw0, sb0, bqn);
      // interleave: each MFMA followed by 2-3 decode VALU ops and 1-2 LDS reads
      // (the full tile; partial tiles take the compiler's schedule)
      if constexpr (NMB == 4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      }
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) af[mb] = afn[mb];
#pragma unroll
      for (int j = 0; j < 4; ++j) bq[j] = bqn[j];
    }
  }

  // epilogue: block (mb, j), register v is row 32 mb + 8 (v / 4) + 4 g + v % 4,
  // column 128 wave + 4 c + j
  const int n = nt * BT_BN + 128 * wave + 4 * c;
  if (n >= a.N) return;
  if constexpr (EPI == EPI_SWIGLU_BWD) {
    // The saved derivative factors, 8 rows (one half of a 32-row block's 16
    // registers) per load batch, two batches in flight: the half after next
    // is loaded while a half is stored, so one memory round trip per tile is
    // exposed instead of one per row block.
    u32x4_t fh[2][8];
    auto load_half = [&](int hb, u32x4_t (&f)[8]) {
      const int mb = hb >> 1;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int v = 8 * (hb & 1) + i;
        const int r = 32 * mb + 8 * (v >> 2) + 4 * g + (v & 3);
        f[i] = *reinterpret_cast<const u32x4_t*>(a.save_grad + (int64_t)(m0 + min(r, rows - 1)) * a.N + n);
      }
    };
    load_half(0, fh[0]);
    load_half(1, fh[1]);
#pragma clang loop unroll(full)
    for (int hb = 0; hb < 2 * NMB; ++hb) {
      const int mb = hb >> 1;
      u32x4_t f[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = fh[hb & 1][i];
      if (hb + 2 < 2 * NMB) load_half(hb + 2, fh[hb & 1]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int v = 8 * (hb & 1) + i;
        const int r = 32 * mb + 8 * (v >> 2) + 4 * g + (v & 3);
        if (r < rows) {
          const float o[4] = {acc[mb][0][v], acc[mb][1][v], acc[mb][2][v], acc[mb][3][v]};
          bt_store4<EPI>(a, m0 + r, n, o, f[i]);
        }
      }
    }
  } else {
    const u32x4_t none{0u, 0u, 0u, 0u};
#pragma clang loop unroll(full)
    for (int mb = 0; mb < NMB; ++mb)
#pragma clang loop unroll(full)
      for (int v = 0; v < 16; ++v) {
        const int r = 32 * mb + 8 * (v >> 2) + 4 * g + (v & 3);
        if (r < rows) {
          const float o[4] = {acc[mb][0][v], acc[mb][1][v], acc[mb][2][v], acc[mb][3][v]};
          bt_store4<EPI>(a, m0 + r, n, o, none);
        }
      }
  }
}

template <int EPI, bool QW4, bool SW4>
__global__ __launch_bounds__(256, 1) void moe_bwd_packed_kernel(GemmArgs a) {
  extern __shared__ __align__(1024) uint8_t smem[];  // BT_NS stages
  const int L = xcd_tile_index(*a.num_tiles * a.n_tiles_n);
  if (L < 0) return;
  int tile, nt;
  tile_of<TL_BM>(a, L, tile, nt);
  const int2 te = a.tiles[tile];
  const int e = te.x;
  const int m0 = te.y;
  const int rows = min(BT_BM, a.offsets[e] + a.counts[e] - m0);
  switch ((rows + 31) >> 5) {
    case 1: bt_tile<EPI, QW4, SW4, 1>(a, smem, e, m0, rows, nt); break;
    case 2: bt_tile<EPI, QW4, SW4, 2>(a, smem, e, m0, rows, nt); break;
    case 3: bt_tile<EPI, QW4, SW4, 3>(a, smem, e, m0, rows, nt); break;
    default: bt_tile<EPI, QW4, SW4, 4>(a, smem, e, m0, rows, nt); break;
  }
}

static int allow_big_lds(const void* fn, int kind, int epi, int bytes);

// Explicit instantiations: the host compiler otherwise drops the handle of
// the first of these named in the launcher below.
template __global__ void moe_bwd_packed_kernel<EPI_STORE, false, false>(GemmArgs);
template __global__ void moe_bwd_packed_kernel<EPI_STORE, false, true>(GemmArgs);
template __global__ void moe_bwd_packed_kernel<EPI_STORE, true, true>(GemmArgs);
template __global__ void moe_bwd_packed_kernel<EPI_SWIGLU_BWD, false, false>(GemmArgs);
template __global__ void moe_bwd_packed_kernel<EPI_SWIGLU_BWD, false, true>(GemmArgs);
template __global__ void moe_bwd_packed_kernel<EPI_SWIGLU_BWD, true, true>(GemmArgs);

// Grouped GEMM on the packed weights read along their rows (the backward
// products): a.Bq [E][K][N/32][16], a.Bs [E][K][N/32].
static bool bwd_packed_ok(const GemmArgs& a) {
  auto al = [](const void* p, int n) { return reinterpret_cast<uintptr_t>(p) % n == 0; };
  return a.N % 32 == 0 && a.K % BT_BK == 0 && al(a.A, 16) && a.lda % 8 == 0 && al(a.Bq, 4) && al(a.Bs, 4) &&
         al(a.out, 16) && !a.row_pair && ((int64_t)a.E * a.K * (a.N / 32)) % 16 == 0;
}

template <int EPI>
static int launch_gemm_packed_rows(const GemmArgs& a, int64_t P, hipStream_t st) {
  GemmArgs b = a;
  b.n_tiles_n = (a.N + BT_BN - 1) / BT_BN;
  const int64_t max_tiles = (P + BT_BM - 1) / BT_BM + a.E;
  const int64_t grid = align_up(max_tiles * b.n_tiles_n, 8);
  if (grid > INT32_MAX) {
    set_error("packed-weight grouped GEMM: grid too large");
    return BSA_EINVAL;
  }
  const size_t smem = (size_t)BT_NS * BT_STAGE;
  // the k-pair layout is read in 16-byte weight pieces only (its blocks are
  // 16-byte aligned by contract); scales take 4-byte pieces below 16
  const bool q16 = reinterpret_cast<uintptr_t>(a.Bq) % 16 == 0;
  const bool s16 = q16 && reinterpret_cast<uintptr_t>(a.Bs) % 16 == 0;
  if (a.kp && !q16) {
    set_error("packed-weight grouped GEMM: k-pair blocks must be 16-byte aligned");
    return BSA_EINVAL;
  }
  void (*fn)(GemmArgs) = s16 ? moe_bwd_packed_kernel<EPI, false, false>
                         : q16 ? moe_bwd_packed_kernel<EPI, false, true>
                               : moe_bwd_packed_kernel<EPI, true, true>;
  int rc = allow_big_lds(reinterpret_cast<const void*>(fn), s16 ? 3 : (q16 ? 1 : 2), EPI, (int)smem);
  if (rc) return rc;
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(256), smem, st, b);
  BSA_LAUNCH_CHECK("packed-weight grouped GEMM launch");
  return BSA_OK;
}

constexpr int T2_LAUNCH_NS = 2;  // and of the launched bf16 tiled kernel

// Kernels using more than 64 KiB of dynamic LDS must be allowed to, once per
// kernel and device.  `kind` (0..7) x `epi` (0..3) names the kernel.
static int allow_big_lds(const void* fn, int kind, int epi, int bytes = 160 * 1024) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    set_error("no current HIP device");
    return BSA_EHIP;
  }
  // kinds: 1-3 packed-weight backward kernel, 4-5 tiled kernel, 6 persistent
  // decode kernel, 8-15 MX kernel configurations
  static bool allowed[64][16][8];
  if (!allowed[dev][kind][epi]) {
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) {
      set_error("cannot allow %d bytes of dynamic LDS for a GEMM kernel", bytes);
      return BSA_EHIP;
    }
    allowed[dev][kind][epi] = true;
  }
  return BSA_OK;
}

template <int EPI, int NS, int WM, int WN, int NB>
static int launch_mx_cfg(const GemmArgs& a, int64_t P, size_t smem, hipStream_t st) {
  using C = MxCfg<WN, NB>;
  const int64_t max_tiles = (P + MX_BM - 1) / MX_BM + a.E;
  GemmArgs b = a;
  b.n_tiles_n = (a.N + C::BN - 1) / C::BN;
  const int64_t grid = align_up(max_tiles * b.n_tiles_n, 8);
  if (grid > INT32_MAX) {
    set_error("MX GEMM: grid too large");
    return BSA_EINVAL;
  }
  const bool sb16 = reinterpret_cast<uintptr_t>(a.Bs) % 16 == 0;
  const void* fn = sb16 ? reinterpret_cast<const void*>(moe_mx_kernel<EPI, NS, true, WM, WN, NB>)
                        : reinterpret_cast<const void*>(moe_mx_kernel<EPI, NS, false, WM, WN, NB>);
  int rc = allow_big_lds(fn, 8 + (sb16 ? 1 : 0), EPI);
  if (rc) return rc;
  if (sb16)
    hipLaunchKernelGGL((moe_mx_kernel<EPI, NS, true, WM, WN, NB>), dim3((unsigned)grid), dim3(64 * C::W), smem,
                       st, b);
  else
    hipLaunchKernelGGL((moe_mx_kernel<EPI, NS, false, WM, WN, NB>), dim3((unsigned)grid), dim3(64 * C::W),
                       smem, st, b);
  BSA_LAUNCH_CHECK("MX grouped GEMM launch");
  return BSA_OK;
}

// Block-scaled MX grouped GEMM (K % 64 == 0; 16-byte aligned blocks, 4-byte
// aligned weight scales; a.Aq / a.As the k-tile-major split of the sorted
// activation rows, with 128 spare rows after the last).
// Pipeline depth BSA_MX_NS, a 2 x BSA_MX_WN wave grid with BSA_MX_NB
// 32-column blocks per wave (a build-time choice; the defaults measured
// fastest at the gpt-oss-120b prefill shapes: a third stage does not fit two
// workgroups per CU, and 8-wave grids at one workgroup per CU ran 7-10%
// slower).  BSA_MX_WM stays 2: the split-step pipeline multiplies two row
// blocks per wave.
#ifndef BSA_MX_NS
#define BSA_MX_NS 2
#endif
#ifndef BSA_MX_WM
#define BSA_MX_WM 2
#endif
#ifndef BSA_MX_WN
#define BSA_MX_WN 2
#endif
#ifndef BSA_MX_NB
#define BSA_MX_NB 4
#endif
template <int EPI>
static int launch_gemm_mx(const GemmArgs& a, int64_t P, hipStream_t st) {
  if (a.K % MX_BK != 0 || reinterpret_cast<uintptr_t>(a.Bq) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(a.Bs) % 4 != 0 || a.ldas % 4 != 0 || a.ldq % 16 != 0 ||
      reinterpret_cast<uintptr_t>(a.Aq) % 16 != 0 || reinterpret_cast<uintptr_t>(a.As) % 4 != 0) {
    set_error("MX GEMM: needs K %% 64 == 0 (K=%d), 16-byte aligned blocks and 4-byte aligned scales",
              a.K);
    return BSA_EINVAL;
  }
  using C = MxCfg<BSA_MX_WN, BSA_MX_NB>;
  // the epilogue stages each wave's results in the (then idle) stages and
  // B-scale buffer
  const size_t smem = std::max(mx_smem_bytes<C>(BSA_MX_NS, a.K), (size_t)C::W * C::EPI_LDS);
  if (smem > 160 * 1024) {
    set_error("MX GEMM: K=%d needs %zu bytes of LDS", a.K, smem);
    return BSA_EINVAL;
  }
  return launch_mx_cfg<EPI, BSA_MX_NS, BSA_MX_WM, BSA_MX_WN, BSA_MX_NB>(a, P, smem, st);
}

// Compute units of the current device (cached per device).
static int cu_count() {
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

// Whether the decode path's GEMM with these arguments runs the persistent
// kernel (else the one-workgroup-per-slice stream kernel).
static bool persist_ok(const GemmArgs& a, int64_t P) {
  auto al16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
  return a.K == 2880 && a.N % 16 == 0 && a.E <= 256 * PS_TEAMS && al16(a.Bq) && al16(a.Bs) && al16(a.bias) &&
         al16(a.A) && a.lda % 8 == 0 && P <= (1 << 19) && cu_count() > 0;
}

// Pairs up to which the decode gate_up folds the dispatch into its prologue
// (each persistent workgroup then places PS_FUSE_MAX_P / 256 rounds of pairs).
#ifndef BSA_FUSE_DISPATCH
#define BSA_FUSE_DISPATCH 1
#endif
constexpr int64_t PS_FUSE_MAX_P = BSA_FUSE_DISPATCH ? 1024 : 0;

// A dispatch that has not run yet: the router indices and the workspace
// arrays it fills (launch_gemm runs it, folded or as its own launch).
struct PendingDispatch {
  const int64_t* idx;
  const Workspace* w;
};

static int run_dispatch(const int64_t* idx, int64_t P, int E, const Workspace& w, hipStream_t st) {
  // the chunked dispatch's per-chunk histograms ([P/2048][E] int32) live in
  // the activation buffer, which gate_up overwrites afterwards
  return launch_dispatch(idx, (int)P, E, TL_BM, w.counts, w.offsets, w.row_pair, w.pair_pos, w.tiles,
                         w.num_tiles, reinterpret_cast<int*>(w.act), st);
}

// `pending` (non-null for the first GEMM of a forward whose dispatch has not
// run): the dispatch runs here, in the branch that picks the kernel, so that
// it is folded into the prologue of the persistent kernel only, the one
// kernel that builds it, and runs as its own launch before any other kernel.
// No kernel can then read a workspace that nothing has dispatched into.
template <int EPI>
static int launch_gemm(const GemmArgs& a, int path, int64_t P, hipStream_t st,
                       const PendingDispatch* pending = nullptr) {
  const bool align16 = (reinterpret_cast<uintptr_t>(a.Bq) % 16) == 0;
  const int cus = cu_count();
  if (path == PATH_STREAM && persist_ok(a, P)) {
    // the gpt-oss hidden / intermediate size: persistent workgroups, 512
    // threads per CU
    GemmArgs b = a;
    if (pending && P <= PS_FUSE_MAX_P) {
      const Workspace& w = *pending->w;
      b.fuse_idx = pending->idx;
      b.fuse_P = (int)P;
      b.fuse_bm = TL_BM;
      b.fuse_counts = w.counts;
      b.fuse_offsets = w.offsets;
      b.fuse_row_pair = w.row_pair;
      b.fuse_pair_pos = w.pair_pos;
      b.fuse_tiles = w.tiles;
      b.fuse_num_tiles = w.num_tiles;
    } else if (pending) {
      int rc = run_dispatch(pending->idx, P, a.E, *pending->w, st);
      if (rc) return rc;
    }
    constexpr int ring = PS_TEAMS * PS_TEAM_NB * PsCfg<90>::SLOT;
    const void* fn = reinterpret_cast<const void*>(moe_stream_persist_kernel<EPI, 90, PS_TEAMS>);
    int rc = allow_big_lds(fn, 6, EPI, ring);
    if (rc) return rc;
    hipLaunchKernelGGL((moe_stream_persist_kernel<EPI, 90, PS_TEAMS>), dim3((unsigned)(cus * (3 - PS_TEAMS))),
                       dim3(256 * PS_TEAMS), ring, st, b);
    BSA_LAUNCH_CHECK("grouped GEMM launch");
    return BSA_OK;
  }
  if (pending) {
    int rc = run_dispatch(pending->idx, P, a.E, *pending->w, st);
    if (rc) return rc;
  }
  if (path == PATH_STREAM && a.K == 2880 && a.N % ST_BN == 0 && align16 &&
             reinterpret_cast<uintptr_t>(a.Bs) % 16 == 0) {
    // the gpt-oss hidden / intermediate size: the part-pipelined kernel
    const int64_t grid = (int64_t)a.E * (a.N / ST_BN);
    hipLaunchKernelGGL((moe_stream_parts_kernel<EPI, 90>), dim3((unsigned)grid), dim3(256), 0, st, a);
  } else if (path == PATH_STREAM) {
    const int slices = (a.N + ST_BN - 1) / ST_BN;
    const int64_t grid = (int64_t)a.E * slices;
    const size_t smem = st_smem_bytes(a.K);
    if (smem > 160 * 1024) {
      set_error("stream GEMM: K=%d needs %zu bytes of LDS", a.K, smem);
      return BSA_EINVAL;
    }
    const bool dma = align16 && (reinterpret_cast<uintptr_t>(a.Bs) % 16) == 0;
    if (dma)
      hipLaunchKernelGGL((moe_stream_kernel<EPI, true>), dim3((unsigned)grid), dim3(256), smem, st, a);
    else
      hipLaunchKernelGGL((moe_stream_kernel<EPI, false>), dim3((unsigned)grid), dim3(256), smem, st, a);
  } else if (align16 && (reinterpret_cast<uintptr_t>(a.Bs) % 4) == 0 &&
             (reinterpret_cast<uintptr_t>(a.A) % 16) == 0 && (a.lda % 8) == 0) {
    const int64_t max_tiles = (P + T2_BM - 1) / T2_BM + a.E;
    GemmArgs b = a;
    b.n_tiles_n = (a.N + T2_BN - 1) / T2_BN;
    int64_t grid = align_up(max_tiles * b.n_tiles_n, 8);
    if (grid > INT32_MAX) {
      set_error("tiled GEMM: grid too large");
      return BSA_EINVAL;
    }
    const size_t smem = (size_t)T2_LAUNCH_NS * T2_STAGE + (size_t)T2_BN * (a.K / 32);
    if (smem > 160 * 1024) {
      set_error("tiled GEMM: K=%d needs %zu bytes of LDS", a.K, smem);
      return BSA_EINVAL;
    }
    const bool sb16 = reinterpret_cast<uintptr_t>(a.Bs) % 16 == 0;
    const void* fn = sb16 ? reinterpret_cast<const void*>(moe_tiled2_kernel<EPI, T2_LAUNCH_NS, 0, true>)
                          : reinterpret_cast<const void*>(moe_tiled2_kernel<EPI, T2_LAUNCH_NS, 0, false>);
    int rc = allow_big_lds(fn, 4 + (sb16 ? 1 : 0), EPI);
    if (rc) return rc;
    if (sb16)
      hipLaunchKernelGGL((moe_tiled2_kernel<EPI, T2_LAUNCH_NS, 0, true>), dim3((unsigned)grid), dim3(256),
                         smem, st, b);
    else
      hipLaunchKernelGGL((moe_tiled2_kernel<EPI, T2_LAUNCH_NS, 0, false>), dim3((unsigned)grid), dim3(256),
                         smem, st, b);
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
  if (path == PATH_MX) return PATH_MX;     // checks its own shape
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

namespace bsa {

struct MoeShape {
  int64_t T, H, I, E, k;
};

// The path of a whole forward (both projections).  Automatic selection takes
// the MX kernels for prefill-sized batches when both projections can run
// them: their gate_up stage leaves the split activations, not bf16 ones, for
// the down stage, so the choice is made once, from both weights' alignment.
// (The single-stage entry points see one projection only; for them automatic
// selection stays on paths 1-2.)  A forward that saves its gate_up
// pre-activations for the backward keeps the bf16 products: the block-scaled
// instruction's accumulation puts ten times as many pre-activations on the
// other side of the SwiGLU clamps from float32 (measured at the gpt-oss-120b
// prefill shape: 246 against 26 of 189M), and each such flip moves a token's
// input gradient by the size of its largest entries.
static int resolve_path(int path, const MoeShape& m, const void* gu_b, const void* gu_s, const void* dn_b,
                        const void* dn_s, bool saving) {
  if (path != PATH_AUTO || saving) return path;
  const bool a16 = reinterpret_cast<uintptr_t>(gu_b) % 16 == 0 && reinterpret_cast<uintptr_t>(dn_b) % 16 == 0;
  const bool s4 = reinterpret_cast<uintptr_t>(gu_s) % 4 == 0 && reinterpret_cast<uintptr_t>(dn_s) % 4 == 0;
  const int64_t P = m.T * m.k;
  if (P > 16 * m.E && m.H % MX_BK == 0 && m.I % MX_BK == 0 && a16 && s4) return PATH_MX;
  return PATH_AUTO;
}

static int check_shape(const MoeShape& m, const char* what) {
  BSA_REQUIRE(m.T >= 0 && m.H > 0 && m.I > 0 && m.E > 0 && m.k > 0,
              "%s: bad shape T=%lld H=%lld I=%lld E=%lld k=%lld", what, (long long)m.T,
              (long long)m.H, (long long)m.I, (long long)m.E, (long long)m.k);
  BSA_REQUIRE(m.H % 32 == 0 && m.I % 32 == 0, "%s: hidden and intermediate must be multiples of 32", what);
  BSA_REQUIRE(m.E <= 1024, "%s: at most 1024 experts (got %lld)", what, (long long)m.E);
  BSA_REQUIRE(m.k <= 16, "%s: top-k at most 16 (got %lld)", what, (long long)m.k);
  BSA_REQUIRE(m.T * m.k < INT32_MAX / 2 && (m.T * m.k) * (2 * m.I) < INT64_MAX / 4,
              "%s: too many tokens", what);
  return BSA_OK;
}

static int check_ws(const MoeShape& m, void* workspace, int64_t bytes, Workspace* w, const char* what) {
  BSA_REQUIRE(workspace, "%s: null workspace", what);
  *w = carve(workspace, m.T, m.H, m.I, m.E, m.k);
  BSA_REQUIRE(bytes >= w->bytes, "%s: workspace of %lld bytes, need %lld", what, (long long)bytes,
              (long long)w->bytes);
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "%s: workspace must be 256-byte aligned", what);
  return BSA_OK;
}

static int stage_dispatch(const MoeShape& m, const int64_t* idx, const Workspace& w, hipStream_t st) {
  return run_dispatch(idx, m.T * m.k, (int)m.E, w, st);
}

// blocks_layout of one packed weight with `rows` rows of K/32 groups.
static int check_layout(int layout, const void* blocks, int64_t rows, int64_t K, const char* what) {
  BSA_REQUIRE(layout == BSA_LAYOUT_CHECKPOINT || layout == BSA_LAYOUT_KPAIR, "%s: unknown blocks layout %d", what,
              layout);
  if (layout == BSA_LAYOUT_KPAIR) {
    BSA_REQUIRE(rows % 16 == 0 && (K / 32) % 2 == 0,
                "%s: the k-pair layout needs rows %% 16 == 0 and an even group count (rows=%lld K=%lld)", what,
                (long long)rows, (long long)K);
    BSA_REQUIRE(reinterpret_cast<uintptr_t>(blocks) % 16 == 0, "%s: the k-pair layout needs 16-byte aligned blocks",
                what);
  }
  return BSA_OK;
}

// dispatch_idx: the router indices when the dispatch has not run yet (it then
// runs here: folded into the decode GEMM's prologue when launch_gemm picks the
// persistent kernel and the batch is small, else as its own launch first);
// null when the caller ran it.
static int stage_gate_up(const MoeShape& m, const void* hidden, const void* blocks, const void* scales,
                         const void* bias, int bias_dtype, float alpha, float limit, const Workspace& w,
                         void* save_swiglu_grad, int path, int layout, hipStream_t st,
                         const int64_t* dispatch_idx = nullptr) {
  // the backward reads each row's factors in 16-byte pieces
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(save_swiglu_grad) % 16 == 0,
              "gate_up: save_swiglu_grad must be 16-byte aligned");
  GemmArgs g{};
  g.kp = layout == BSA_LAYOUT_KPAIR;
  g.A = static_cast<const uint16_t*>(hidden);
  g.lda = m.H;
  g.row_pair = w.row_pair;
  g.topk = (int)m.k;
  g.Bq = static_cast<const uint8_t*>(blocks);
  g.Bs = static_cast<const uint8_t*>(scales);
  g.bias = bias;
  g.bias_dtype = bias_dtype;
  g.counts = w.counts;
  g.offsets = w.offsets;
  g.E = (int)m.E;
  g.N = (int)(2 * m.I);
  g.K = (int)m.H;
  g.out = w.act;
  g.ldo = m.I;
  g.out_dtype = DT_BF16;
  g.save_grad = static_cast<uint32_t*>(save_swiglu_grad);
  g.alpha = alpha;
  g.limit = limit;
  g.tiles = w.tiles;
  g.num_tiles = w.num_tiles;
  g.n_tiles_n = (int)((2 * m.I + TL_BN - 1) / TL_BN);
  const int64_t P = m.T * m.k;
  const int chosen = pick_path(path, P, m.E, m.H);
  const PendingDispatch pending{dispatch_idx, &w};
  if (chosen == PATH_MX) {
    // each token's hidden row is split once and written to each of its pairs
    if (m.H % MX_BK != 0 || m.I % MX_BK != 0) {
      set_error("gate_up (MX path): hidden %lld and intermediate %lld must be multiples of 64",
                (long long)m.H, (long long)m.I);
      return BSA_EINVAL;
    }
    if (dispatch_idx) {  // the split below writes through the dispatch's pair_pos
      int rc = stage_dispatch(m, dispatch_idx, w, st);
      if (rc) return rc;
    }
    // every token's hidden row split once and written to its pairs' sorted
    // rows, k-tile-major, so a tile's rows of one k-tile are one contiguous run
    const SplitLayout hl{128, w.rows_mx * 128, 4, w.rows_mx * 4};
    int rc = launch_quant_mxfp8_split(hidden, DT_BF16, m.T, m.H, m.H, w.pair_pos, (int)m.k, w.hq, w.hs, hl, st);
    if (rc) return rc;
    g.Aq = w.hq;
    g.ldq = hl.q_kt;
    g.As = w.hs;
    g.ldas = hl.s_kt;
    // the epilogue splits the activations for the down GEMM itself
    g.out = w.aq;
    g.ldo = 128;
    g.out_kt = w.rows_mx * 128;
    g.out_s = w.as;
    g.ldos = 4;
    g.out_s_kt = w.rows_mx * 4;
    return launch_gemm_mx<EPI_SWIGLU_MX>(g, P, st);
  }
  return launch_gemm<EPI_SWIGLU>(g, chosen, P, st, dispatch_idx ? &pending : nullptr);
}

static int stage_down(const MoeShape& m, const void* blocks, const void* scales, const void* bias,
                      int bias_dtype, const Workspace& w, int path, int layout, hipStream_t st) {
  GemmArgs g{};
  g.kp = layout == BSA_LAYOUT_KPAIR;
  g.A = w.act;
  g.lda = m.I;
  g.row_pair = nullptr;
  g.topk = (int)m.k;
  g.Bq = static_cast<const uint8_t*>(blocks);
  g.Bs = static_cast<const uint8_t*>(scales);
  g.bias = bias;
  g.bias_dtype = bias_dtype;
  g.counts = w.counts;
  g.offsets = w.offsets;
  g.E = (int)m.E;
  g.N = (int)m.H;
  g.K = (int)m.I;
  g.out = w.y;
  g.ldo = m.H;
  g.out_dtype = DT_F32;
  g.tiles = w.tiles;
  g.num_tiles = w.num_tiles;
  g.n_tiles_n = (int)((m.H + TL_BN - 1) / TL_BN);
  const int64_t P = m.T * m.k;
  const int chosen = pick_path(path, P, m.E, m.I);
  if (chosen == PATH_MX) {
    if (m.I % MX_BK != 0) {
      set_error("down (MX path): intermediate %lld is not a multiple of 64", (long long)m.I);
      return BSA_EINVAL;
    }
    g.Aq = w.aq;  // written by the gate_up epilogue
    g.ldq = w.rows_mx * 128;
    g.As = w.as;
    g.ldas = w.rows_mx * 4;
    return launch_gemm_mx<EPI_BIAS_F32>(g, P, st);
  }
  return launch_gemm<EPI_BIAS_F32>(g, chosen, P, st);
}

static bool dtype_ok(int d) { return d >= 0 && d <= 2; }

}  // namespace bsa

extern "C" int bsa_moe_dispatch(const int64_t* router_indices, int64_t T, int64_t H, int64_t I,
                                int64_t E, int64_t k, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  clear_error();
  const MoeShape m{T, H, I, E, k};
  int rc = check_shape(m, "dispatch");
  if (rc || T == 0) return rc;
  BSA_REQUIRE(router_indices, "dispatch: null router_indices");
  Workspace w;
  if ((rc = check_ws(m, workspace, workspace_bytes, &w, "dispatch"))) return rc;
  return stage_dispatch(m, router_indices, w, static_cast<hipStream_t>(stream));
}

extern "C" int bsa_moe_gate_up(const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E,
                               int64_t k, const void* blocks, const void* scales, const void* bias,
                               int bias_dtype, float alpha, float limit, void* workspace,
                               int64_t workspace_bytes, void* save_swiglu_grad, int path, int blocks_layout,
                               void* stream) {
  clear_error();
  const MoeShape m{T, H, I, E, k};
  int rc = check_shape(m, "gate_up");
  if (rc || T == 0) return rc;
  BSA_REQUIRE(hidden && blocks && scales, "gate_up: null pointer");
  BSA_REQUIRE(dtype_ok(bias_dtype) && path >= 0 && path <= 3, "gate_up: bad dtype or path");
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(hidden) % 16 == 0 && reinterpret_cast<uintptr_t>(blocks) % 8 == 0,
              "gate_up: hidden must be 16-byte and blocks 8-byte aligned");
  if ((rc = check_layout(blocks_layout, blocks, 2 * I, H, "gate_up"))) return rc;
  Workspace w;
  if ((rc = check_ws(m, workspace, workspace_bytes, &w, "gate_up"))) return rc;
  return stage_gate_up(m, hidden, blocks, scales, bias, bias_dtype, alpha, limit, w, save_swiglu_grad,
                       path, blocks_layout, static_cast<hipStream_t>(stream));
}

extern "C" int bsa_moe_down(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                            const void* blocks, const void* scales, const void* bias,
                            int bias_dtype, void* workspace, int64_t workspace_bytes, int path,
                            int blocks_layout, void* stream) {
  clear_error();
  const MoeShape m{T, H, I, E, k};
  int rc = check_shape(m, "down");
  if (rc || T == 0) return rc;
  BSA_REQUIRE(blocks && scales, "down: null pointer");
  BSA_REQUIRE(dtype_ok(bias_dtype) && path >= 0 && path <= 3, "down: bad dtype or path");
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(blocks) % 8 == 0, "down: blocks must be 8-byte aligned");
  if ((rc = check_layout(blocks_layout, blocks, H, I, "down"))) return rc;
  Workspace w;
  if ((rc = check_ws(m, workspace, workspace_bytes, &w, "down"))) return rc;
  return stage_down(m, blocks, scales, bias, bias_dtype, w, path, blocks_layout, static_cast<hipStream_t>(stream));
}

extern "C" int bsa_moe_combine(const int64_t* router_indices, const void* routing_weights,
                               int weight_dtype, int64_t T, int64_t H, int64_t I, int64_t E,
                               int64_t k, void* workspace, int64_t workspace_bytes, void* out,
                               int out_dtype, void* stream) {
  clear_error();
  const MoeShape m{T, H, I, E, k};
  int rc = check_shape(m, "combine");
  if (rc || T == 0) return rc;
  BSA_REQUIRE(router_indices && routing_weights && out, "combine: null pointer");
  BSA_REQUIRE(dtype_ok(weight_dtype) && dtype_ok(out_dtype), "combine: bad dtype");
  Workspace w;
  if ((rc = check_ws(m, workspace, workspace_bytes, &w, "combine"))) return rc;
  return launch_combine(w.y, router_indices, routing_weights, weight_dtype, w.pair_pos, (int)T,
                        (int)k, (int)H, out, out_dtype, static_cast<hipStream_t>(stream));
}

namespace bsa {

// ---------------------------------------------------------------------------
// Workspace of the no-allocation forward: a file-scope device array, one copy
// per GPU, alive until the process ends.  Host code never passes the array's
// name to a kernel (on the host it is only a stand-in symbol); it passes the
// device address hipGetSymbolAddress returns, looked up once per device with
// that device current.  Every no-allocation call on a GPU uses that GPU's
// copy, so such calls must not overlap on one GPU (one stream at a time, or
// ordered by events).  The forward writes every workspace word it later
// reads, so nothing needs clearing between calls.
// ---------------------------------------------------------------------------
constexpr int64_t NOALLOC_SCRATCH_BYTES = BSA_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[NOALLOC_MAX_DEVICES];

// Device address of `scratch` on the device that owns stream `st` (the
// current device for the null stream).
static int scratch_of_stream(hipStream_t st, void** out) {
  int dev = -1;
  hipError_t e = st ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("no-alloc scratch: cannot find the stream's device: %s", hipGetErrorString(e));
    return BSA_EHIP;
  }
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) {
    set_error("no-alloc scratch: device %d beyond the %d supported", dev, NOALLOC_MAX_DEVICES);
    return BSA_EINVAL;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if ((e = hipGetDevice(&cur)) == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur >= 0 && cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p) {
      set_error("no-alloc scratch: hipGetSymbolAddress on device %d: %s", dev,
                e != hipSuccess ? hipGetErrorString(e) : "null address");
      return BSA_EHIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return BSA_OK;
}

// The whole forward (dispatch, gate_up, down, combine) on one workspace;
// `what` names the entry point in error messages.  With `noalloc` the
// workspace is the static scratch of the stream's device.
static int experts_fwd(
    const char* what, bool noalloc, const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
    const int64_t* router_indices, const void* routing_weights, int weight_dtype,
    const void* gate_up_blocks, const void* gate_up_scales, const void* gate_up_bias,
    const void* down_blocks, const void* down_scales, const void* down_bias, int bias_dtype,
    float alpha, float limit, void* out, int out_dtype, void* workspace, int64_t workspace_bytes,
    void* save_swiglu_grad, int path, int blocks_layout, void* stream) {
  const MoeShape m{T, H, I, E, k};
  int rc = check_shape(m, what);
  if (rc || T == 0) return rc;
  BSA_REQUIRE(dtype_ok(weight_dtype) && dtype_ok(bias_dtype) && dtype_ok(out_dtype),
              "%s: bad dtype code", what);
  BSA_REQUIRE(path >= 0 && path <= 3, "%s: path must be 0, 1, 2 or 3", what);
  BSA_REQUIRE(hidden && router_indices && routing_weights && gate_up_blocks && gate_up_scales &&
                  down_blocks && down_scales && out,
              "%s: null pointer", what);
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(hidden) % 16 == 0, "%s: hidden must be 16-byte aligned", what);
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(gate_up_blocks) % 8 == 0 &&
                  reinterpret_cast<uintptr_t>(down_blocks) % 8 == 0,
              "%s: packed blocks must be 8-byte aligned", what);
  if ((rc = check_layout(blocks_layout, gate_up_blocks, 2 * I, H, "experts fwd (gate_up)")) ||
      (rc = check_layout(blocks_layout, down_blocks, H, I, "experts fwd (down)")))
    return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  path = resolve_path(path, m, gate_up_blocks, gate_up_scales, down_blocks, down_scales, save_swiglu_grad != nullptr);
  if (noalloc) {
    workspace_bytes = carve(nullptr, T, H, I, E, k).bytes;
    BSA_REQUIRE(workspace_bytes <= NOALLOC_SCRATCH_BYTES,
                "%s: this shape needs %lld bytes of workspace and the static scratch holds %lld; "
                "call bsa_moe_experts_fwd with a workspace instead",
                what, (long long)workspace_bytes, (long long)NOALLOC_SCRATCH_BYTES);
    if ((rc = scratch_of_stream(st, &workspace))) return rc;
  }
  Workspace w;
  if ((rc = check_ws(m, workspace, workspace_bytes, &w, what))) return rc;
  if ((rc = stage_gate_up(m, hidden, gate_up_blocks, gate_up_scales, gate_up_bias, bias_dtype, alpha,
                          limit, w, save_swiglu_grad, path, blocks_layout, st, router_indices)))
    return rc;
  if ((rc = stage_down(m, down_blocks, down_scales, down_bias, bias_dtype, w, path, blocks_layout, st)))
    return rc;
  return launch_combine(w.y, router_indices, routing_weights, weight_dtype, w.pair_pos, (int)T,
                        (int)k, (int)H, out, out_dtype, st);
}

}  // namespace bsa

extern "C" int bsa_moe_experts_fwd(
    const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
    const int64_t* router_indices, const void* routing_weights, int weight_dtype,
    const void* gate_up_blocks, const void* gate_up_scales, const void* gate_up_bias,
    const void* down_blocks, const void* down_scales, const void* down_bias, int bias_dtype,
    float alpha, float limit, void* out, int out_dtype, void* workspace, int64_t workspace_bytes,
    void* save_swiglu_grad, int path, int blocks_layout, void* stream) {
  clear_error();
  return experts_fwd("experts fwd", false, hidden, T, H, I, E, k, router_indices, routing_weights, weight_dtype,
                     gate_up_blocks, gate_up_scales, gate_up_bias, down_blocks, down_scales, down_bias,
                     bias_dtype, alpha, limit, out, out_dtype, workspace, workspace_bytes, save_swiglu_grad,
                     path, blocks_layout, stream);
}

extern "C" int bsa_moe_experts_fwd_noalloc(
    const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
    const int64_t* router_indices, const void* routing_weights, int weight_dtype,
    const void* gate_up_blocks, const void* gate_up_scales, const void* gate_up_bias,
    const void* down_blocks, const void* down_scales, const void* down_bias, int bias_dtype,
    float alpha, float limit, void* out, int out_dtype, void* save_swiglu_grad, int path,
    int blocks_layout, void* stream) {
  clear_error();
  // the backward reads the forward's workspace (the dispatch arrays), which
  // here is the shared scratch that the next call overwrites: nothing saved
  // by this entry point could be consumed safely
  BSA_REQUIRE(save_swiglu_grad == nullptr,
              "experts fwd (no-alloc): save_swiglu_grad must be null (the backward needs the forward's "
              "workspace, and this entry point's is the shared static scratch)");
  return experts_fwd("experts fwd (no-alloc)", true, hidden, T, H, I, E, k, router_indices, routing_weights,
                     weight_dtype, gate_up_blocks, gate_up_scales, gate_up_bias, down_blocks, down_scales,
                     down_bias, bias_dtype, alpha, limit, out, out_dtype, nullptr, 0, save_swiglu_grad, path,
                     blocks_layout, stream);
}

namespace bsa {

struct BwdWorkspace {
  uint16_t* dy;         // [P][H] bf16: dOut rows scaled by the routing weight
  uint16_t* dgu;        // [P][2I] bf16: gradient of the gate_up pre-activations
  float* dx;            // [P][H] f32: per-row input gradients
  float* dw;            // [P] f32: routing-weight gradients
  int64_t bytes;
};

static BwdWorkspace carve_bwd(void* base, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k) {
  const int64_t P = T * k;
  char* p = static_cast<char*>(base);
  int64_t off = 0;
  BwdWorkspace w{};
  auto take = [&](int64_t bytes) {
    char* r = p ? p + off : nullptr;
    off = align_up(off + bytes, 256);
    return r;
  };
  w.dy = reinterpret_cast<uint16_t*>(take(P * H * 2));
  w.dgu = reinterpret_cast<uint16_t*>(take(P * 2 * I * 2));
  w.dx = reinterpret_cast<float*>(take(P * H * 4));
  w.dw = reinterpret_cast<float*>(take(P * 4));
  w.bytes = off;
  return w;
}

}  // namespace bsa

extern "C" int bsa_moe_bwd_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                                           int64_t* bytes) {
  clear_error();
  BSA_REQUIRE(bytes, "backward workspace size: null output pointer");
  BSA_REQUIRE(T >= 0 && H > 0 && I > 0 && E > 0 && k > 0, "backward workspace size: bad shape");
  *bytes = carve_bwd(nullptr, T, H, I, E, k).bytes;
  return BSA_OK;
}

extern "C" int bsa_moe_experts_bwd(
    const void* grad_out, int grad_dtype, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
    const int64_t* router_indices, const void* routing_weights, int weight_dtype,
    const void* gate_up_blocks, const void* gate_up_scales, const void* down_blocks,
    const void* down_scales, float alpha, float limit, void* workspace, int64_t workspace_bytes,
    const void* save_swiglu_grad, void* bwd_workspace, int64_t bwd_workspace_bytes, void* grad_hidden,
    int grad_hidden_dtype, float* grad_weights, int blocks_layout, void* stream) {
  clear_error();
  const MoeShape m{T, H, I, E, k};
  int rc = check_shape(m, "experts bwd");
  if (rc || T == 0) return rc;
  BSA_REQUIRE(dtype_ok(grad_dtype) && dtype_ok(weight_dtype) && dtype_ok(grad_hidden_dtype),
              "experts bwd: bad dtype code");
  BSA_REQUIRE(H % 64 == 0 && I % 32 == 0, "experts bwd: needs hidden % 64 == 0 and intermediate % 32 == 0");
  BSA_REQUIRE(grad_out && router_indices && routing_weights && gate_up_blocks && gate_up_scales &&
                  down_blocks && down_scales && save_swiglu_grad && bwd_workspace,
              "experts bwd: null pointer");
  Workspace w;
  if ((rc = check_ws(m, workspace, workspace_bytes, &w, "experts bwd"))) return rc;
  const BwdWorkspace b = carve_bwd(bwd_workspace, T, H, I, E, k);
  BSA_REQUIRE(bwd_workspace_bytes >= b.bytes, "experts bwd: backward workspace of %lld bytes, need %lld",
              (long long)bwd_workspace_bytes, (long long)b.bytes);
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(bwd_workspace) % 256 == 0,
              "experts bwd: backward workspace must be 256-byte aligned");
  auto al = [](const void* q, int n) { return reinterpret_cast<uintptr_t>(q) % n == 0; };
  BSA_REQUIRE(al(gate_up_blocks, 4) && al(gate_up_scales, 4) && al(down_blocks, 4) && al(down_scales, 4),
              "experts bwd: gate_up/down blocks and scales must be 4-byte aligned");
  BSA_REQUIRE(al(save_swiglu_grad, 16), "experts bwd: save_swiglu_grad must be 16-byte aligned");
  if ((rc = check_layout(blocks_layout, gate_up_blocks, 2 * I, H, "experts bwd (gate_up)")) ||
      (rc = check_layout(blocks_layout, down_blocks, H, I, "experts bwd (down)")))
    return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t P = T * k;

  // 1. routing-weight gradients and the weighted output gradient rows
  if ((rc = launch_bwd_prep(grad_out, grad_dtype, w.y, routing_weights, weight_dtype, w.pair_pos,
                            (int)P, (int)k, (int)H, b.dy, grad_weights ? grad_weights : b.dw, st)))
    return rc;
  if (!grad_hidden) return BSA_OK;

  // 2. d(act) = dY @ W_down^T with the SwiGLU backward in the epilogue -> d(gate_up)
  GemmArgs g{};
  g.A = b.dy;
  g.lda = H;
  g.counts = w.counts;
  g.offsets = w.offsets;
  g.E = (int)E;
  g.N = (int)I;
  g.K = (int)H;
  g.out = b.dgu;
  g.ldo = 2 * I;
  g.save_grad = const_cast<uint32_t*>(static_cast<const uint32_t*>(save_swiglu_grad));
  g.alpha = alpha;
  g.limit = limit;
  g.tiles = w.tiles;
  g.num_tiles = w.num_tiles;
  // 3. dX rows = d(gate_up) @ W_gate_up^T
  GemmArgs g2{};
  g2.A = b.dgu;
  g2.lda = 2 * I;
  g2.counts = w.counts;
  g2.offsets = w.offsets;
  g2.E = (int)E;
  g2.N = (int)H;
  g2.K = (int)(2 * I);
  g2.out = b.dx;
  g2.ldo = H;
  g2.out_dtype = DT_F32;
  g2.tiles = w.tiles;
  g2.num_tiles = w.num_tiles;

  // The checkpoint tensors read along their rows are exactly the transposed
  // weights: W_down [E][H][I/32] blocks give rows = hidden (reduction),
  // columns = intermediate.
  g.Bq = static_cast<const uint8_t*>(down_blocks);
  g.Bs = static_cast<const uint8_t*>(down_scales);
  g2.Bq = static_cast<const uint8_t*>(gate_up_blocks);
  g2.Bs = static_cast<const uint8_t*>(gate_up_scales);
  g.kp = g2.kp = blocks_layout == BSA_LAYOUT_KPAIR;
  BSA_REQUIRE(bwd_packed_ok(g) && bwd_packed_ok(g2), "experts bwd: unsupported operand layout");
  if ((rc = launch_gemm_packed_rows<EPI_SWIGLU_BWD>(g, P, st))) return rc;
  if ((rc = launch_gemm_packed_rows<EPI_STORE>(g2, P, st))) return rc;

  // 4. per-token sum of its k rows (ascending expert order)
  return launch_combine(b.dx, router_indices, nullptr, DT_F32, w.pair_pos, (int)T, (int)k, (int)H,
                        grad_hidden, grad_hidden_dtype, st);
}

// ---------------------------------------------------------------------------
// One expert's packed matmul: block_streamer/gptoss.py:45-75 (mxfp4_matmul),
// forward x @ W and its input gradient g @ W^T, with W = dequant(blocks,
// scales) in the [K, N] orientation of gptoss.py:41.  No dense W exists: the
// forward runs the grouped GEMMs above on a one-expert dispatch, the
// transposed product the packed-row kernel of the backward.  The activation
// operand enters the MFMA as bf16; a float16 x is split into 2 bf16 terms and
// a float32 x into 3 (their sum is x exactly), one pass per term, and the
// float32 partial products are summed in term order and rounded once.  The
// products of the terms with the weights are exact, so a float32 x gets
// float32 accuracy (the sum order differs from a library GEMM's).
// ---------------------------------------------------------------------------
namespace bsa {

__global__ void mm_setup_kernel(int M, int* counts, int* offsets, int2* tiles, int* num_tiles) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int nt = (M + TL_BM - 1) / TL_BM;
  if (i < nt) tiles[i] = make_int2(0, i * TL_BM);
  if (i == 0) {
    counts[0] = M;
    offsets[0] = 0;
    offsets[1] = M;
    *num_tiles = nt;
  }
}

// x (n elements, dtype) -> `terms` bf16 arrays [terms][n] whose sum is x.
__global__ void mm_split_kernel(const void* __restrict__ x, int dtype, int64_t n, int terms,
                                uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float v;
  if (dtype == DT_F32)
    v = static_cast<const float*>(x)[i];
  else if (dtype == DT_BF16)
    v = __uint_as_float((uint32_t) static_cast<const uint16_t*>(x)[i] << 16);
  else
    v = (float)__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(x)[i]);
  for (int t = 0; t < terms; ++t) {
    const uint32_t b = f32_to_bf16_bits(v);
    out[t * n + i] = (uint16_t)b;
    v -= __uint_as_float(b << 16);  // exact: v minus v rounded to 8 bits
  }
}

// out[i] = sum over t of parts[t][i], rounded once to out_dtype.
__global__ void mm_sum_kernel(const float* __restrict__ parts, int terms, int64_t n, void* __restrict__ out,
                              int out_dtype) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float v = parts[i];
  for (int t = 1; t < terms; ++t) v += parts[t * n + i];
  if (out_dtype == DT_F32)
    static_cast<float*>(out)[i] = v;
  else if (out_dtype == DT_BF16)
    static_cast<uint16_t*>(out)[i] = (uint16_t)f32_to_bf16_bits(v);
  else
    static_cast<uint16_t*>(out)[i] = (uint16_t)f32_to_f16_bits(v);
}

struct MmWorkspace {
  int* counts;
  int* offsets;
  int2* tiles;
  int* num_tiles;
  uint16_t* terms;  // [terms][M][kin] bf16
  float* parts;     // [terms][M][nout] f32
  int64_t bytes;
};

static int mm_terms(int dtype) { return dtype == DT_F32 ? 3 : (dtype == DT_F16 ? 2 : 1); }

// kin / nout: the activation's and the output's columns (K, N forward; N, K
// transposed).
static MmWorkspace carve_mm(void* base, int64_t M, int64_t kin, int64_t nout, int terms) {
  char* p = static_cast<char*>(base);
  int64_t off = 0;
  MmWorkspace w{};
  auto take = [&](int64_t bytes) {
    char* r = p ? p + off : nullptr;
    off = align_up(off + bytes, 256);
    return r;
  };
  w.counts = reinterpret_cast<int*>(take(4));
  w.offsets = reinterpret_cast<int*>(take(8));
  w.tiles = reinterpret_cast<int2*>(take(((M + TL_BM - 1) / TL_BM + 1) * 8));
  w.num_tiles = reinterpret_cast<int*>(take(4));
  w.terms = reinterpret_cast<uint16_t*>(take(terms * M * kin * 2));
  w.parts = reinterpret_cast<float*>(take(terms * M * nout * 4));
  w.bytes = off;
  return w;
}

static int mm_check(int64_t M, int64_t K, int64_t N, int x_dtype, int transpose, const char* what) {
  BSA_REQUIRE(M >= 0 && K > 0 && N > 0 && K % 32 == 0, "%s: bad shape M=%lld K=%lld N=%lld (K %% 32 == 0)",
              what, (long long)M, (long long)K, (long long)N);
  BSA_REQUIRE(dtype_ok(x_dtype), "%s: bad dtype %d", what, x_dtype);
  BSA_REQUIRE(transpose == 0 || transpose == 1, "%s: transpose must be 0 or 1", what);
  BSA_REQUIRE(M * (K > N ? K : N) * 3 < ((int64_t)1 << 40) && M < INT32_MAX / 2, "%s: too large", what);
  if (transpose)
    BSA_REQUIRE(N % 64 == 0 && N % 8 == 0 && (N * (K / 32)) % 16 == 0,
                "%s: the transposed product needs N %% 64 == 0 (N=%lld)", what, (long long)N);
  return BSA_OK;
}

}  // namespace bsa

extern "C" int bsa_mxfp4_matmul_workspace_bytes(int64_t M, int64_t K, int64_t N, int x_dtype, int transpose,
                                                int64_t* bytes) {
  clear_error();
  BSA_REQUIRE(bytes, "mxfp4 matmul workspace size: null output pointer");
  int rc = mm_check(M, K, N, x_dtype, transpose, "mxfp4 matmul workspace size");
  if (rc) return rc;
  *bytes = carve_mm(nullptr, M, transpose ? N : K, transpose ? K : N, mm_terms(x_dtype)).bytes;
  return BSA_OK;
}

extern "C" int bsa_mxfp4_matmul(const void* x, int x_dtype, int64_t M, int64_t K, int64_t N, const void* blocks,
                                const void* scales, int blocks_layout, int transpose, void* out, int out_dtype,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  int rc = mm_check(M, K, N, x_dtype, transpose, "mxfp4 matmul");
  if (rc || M == 0) return rc;
  BSA_REQUIRE(dtype_ok(out_dtype), "mxfp4 matmul: bad output dtype %d", out_dtype);
  BSA_REQUIRE(x && blocks && scales && out && workspace, "mxfp4 matmul: null pointer");
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(blocks) % 8 == 0 && reinterpret_cast<uintptr_t>(scales) % 4 == 0,
              "mxfp4 matmul: blocks must be 8-byte and scales 4-byte aligned");
  BSA_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "mxfp4 matmul: workspace must be 256-byte aligned");
  BSA_REQUIRE(x_dtype == DT_F32 ? reinterpret_cast<uintptr_t>(x) % 4 == 0 : reinterpret_cast<uintptr_t>(x) % 2 == 0,
              "mxfp4 matmul: x not aligned to its element size");
  if ((rc = check_layout(blocks_layout, blocks, N, K, "mxfp4 matmul"))) return rc;
  const int terms = mm_terms(x_dtype);
  const int64_t kin = transpose ? N : K, nout = transpose ? K : N;
  const MmWorkspace w = carve_mm(workspace, M, kin, nout, terms);
  BSA_REQUIRE(workspace_bytes >= w.bytes, "mxfp4 matmul: workspace of %lld bytes, need %lld",
              (long long)workspace_bytes, (long long)w.bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nt = (M + TL_BM - 1) / TL_BM;
  hipLaunchKernelGGL(mm_setup_kernel, dim3((unsigned)((nt + 255) / 256)), dim3(256), 0, st, (int)M, w.counts,
                     w.offsets, w.tiles, w.num_tiles);
  const int64_t nin = M * kin, nres = M * nout;
  hipLaunchKernelGGL(mm_split_kernel, dim3((unsigned)((nin + 255) / 256)), dim3(256), 0, st, x, x_dtype, nin,
                     terms, w.terms);
  BSA_LAUNCH_CHECK("mxfp4 matmul set-up launch");
  for (int t = 0; t < terms; ++t) {
    GemmArgs g{};
    g.kp = blocks_layout == BSA_LAYOUT_KPAIR;
    g.A = w.terms + t * nin;
    g.lda = kin;
    g.row_pair = nullptr;
    g.topk = 1;
    g.Bq = static_cast<const uint8_t*>(blocks);
    g.Bs = static_cast<const uint8_t*>(scales);
    g.counts = w.counts;
    g.offsets = w.offsets;
    g.E = 1;
    g.out = w.parts + t * nres;
    g.ldo = nout;
    g.out_dtype = DT_F32;
    g.tiles = w.tiles;
    g.num_tiles = w.num_tiles;
    if (!transpose) {
      g.N = (int)N;
      g.K = (int)K;
      g.n_tiles_n = (int)((N + TL_BN - 1) / TL_BN);
      rc = launch_gemm<EPI_BIAS_F32>(g, pick_path(PATH_AUTO, M, 1, K), M, st);
    } else {
      // the packed rows (N of them) are the reduction; outputs run along K
      g.N = (int)K;
      g.K = (int)N;
      BSA_REQUIRE(bwd_packed_ok(g), "mxfp4 matmul: unsupported operand layout for the transposed product");
      rc = launch_gemm_packed_rows<EPI_STORE>(g, M, st);
    }
    if (rc) return rc;
  }
  hipLaunchKernelGGL(mm_sum_kernel, dim3((unsigned)((nres + 255) / 256)), dim3(256), 0, st, w.parts, terms, nres,
                     out, out_dtype);
  BSA_LAUNCH_CHECK("mxfp4 matmul sum launch");
  return BSA_OK;
}
