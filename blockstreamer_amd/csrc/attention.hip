// Attention core of the gpt-oss decoder layer: grouped-query attention with a
// learned per-head sink logit, causal and sliding-window masks.
//
// Semantics (transformers 5.15.0 models/gpt_oss/modeling_gpt_oss.py:235-264,
// eager_attention_forward, called from GptOssAttention.forward :295-336):
//   S[t, j]  = (q[t] . k[j]) * scaling  (+ mask: -inf where key j is hidden)
//   probs    = softmax over [S[t, 0..Tk-1], sink[h]]  (the sink column is
//              the head's logit, unscaled), then the sink column is dropped
//   out[t]   = sum_j probs[t, j] v[j]
// with key head h / (Hq / Hkv) serving query head h (repeat_kv, :203-212).
// Masks: none (every key visible: what the eager path does with
// attention_mask=None, the way the streaming runner calls the decoder,
// block_streamer/runners.py:327-335), causal (key j visible to query t at
// absolute position p = Tk - Tq + t when j <= p), or causal with a window w
// (also p - j < w: masking_utils' sliding-window overlay).
//
// The sink enters the online softmax as its starting state: running maximum
// = sink, running sum = exp(sink - sink) = 1, accumulator = 0.  Products run
// on bf16 MFMA (v_mfma_f32_32x32x16_bf16) with float32 accumulation; the
// probabilities are rounded to bf16 for the P.V product (as the eager path's
// cast to the value dtype).
//
// Rows: a workgroup of the forward and of the dq backward takes 128 rows of
// one (batch, key head); row R = t * G + i is query t of head G * hk + i
// (G = Hq / Hkv), so the G heads sharing a key head read each K/V tile once.
// Four waves, 32 rows each (lane c = row c of the wave), key tiles of 64.
// Short query grids (decoding: one row block per sequence and key head) split
// each row block's key tiles over several workgroups that write unnormalised
// partial sums; attn_split_combine_kernel merges them (bsa_attention_fwd_split).
//
// Orientation: S^T = K Q^T puts a query in each lane, so its row maximum and
// sum are one exchange between the two lane halves.  The K rows enter that
// MFMA permuted (pi below): lane half g then holds keys 8g .. 8g+7 and
// 16 + 8g .. 16 + 8g + 7 of each 32-key block, which is exactly the B
// operand of O^T += V^T P^T, so the probabilities never leave registers and
// the online-softmax rescale of query c stays in lane c.
//
// LDS: every tile is the natural row-major copy a DMA (global_load_lds)
// brings in: 64 rows x 128 bytes, 16-byte chunk c of row R at position
// c ^ sw(R), sw(R) = 4 * ((R >> 1) & 1) | ((R >> 2) & 3).  Two kinds of read
// use it: ds_read_b128 of 16 rows at one chunk (the operands K, V, Q, dO
// with rows permuted), whose 16 (R & 1, sw) pairs are distinct, and the
// transposing ds_read_b64_tr_b16 (V^T, K^T, Q^T, dO^T: in each 16-lane
// group, lane s addresses 4 elements of row k0 + s/4 at column m0 + 4(s%4)
// and lane i receives element i%4 of lanes i/4, 4 + i/4, 8 + i/4, 12 + i/4:
// column m0 + i at rows k0 .. k0+3), whose four rows land in four different
// 64-byte quarters of the 256-byte bank period.  Tiles stream through a ring
// of AT_NS stages, AT_NS - 1 ahead of the computation.
// ---------------------------------------------------------------------------
#include "bsa_common.h"

namespace bsa {

constexpr int AT_D = 64;                    // head dimension
constexpr int AT_BR = 128;                  // rows per workgroup (forward, dq)
constexpr int AT_BC = 64;                   // keys per tile
constexpr int AT_TILE = AT_BC * AT_D * 2;   // 8 KiB
#ifndef BSA_AT_NS
#define BSA_AT_NS 2
#endif
constexpr int AT_NS = BSA_AT_NS;            // ring stages (forward, dq)
#ifndef BSA_AT_NS_DKV
#define BSA_AT_NS_DKV 2
#endif
constexpr int AT_NS_DKV = BSA_AT_NS_DKV;    // ring stages of dk/dv (2, 3, 4 and 6 measured; 2 fastest)

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const float* sinks;   // [Hq] or null (no sink)
  uint16_t* out;
  float* lse;           // [B][Hq][Tq] log2 of the softmax denominator in
                        // scaled-logit units (with the sink), or null
  int64_t sqb, sqt, sqh, skb, skt, skh, svb, svt, svh, sob, sot, soh;
  int Tq, Tk, Hq, G;
  int causal, window;
  float scale2;         // scaling * log2(e)
  // key-split forward (nsplit > 1): workgroup x = row block * nsplit + split
  // takes a contiguous share of the row block's key tiles and writes its rows'
  // unnormalised accumulators and (running max, sum) to part_o / part_ml at
  // row ((split * B + b) * Hkv + hk) * (Tq * G) + R; attn_split_combine_kernel
  // merges them
  int nsplit;
  float* part_o;        // [nsplit][B][Hkv][Tq * G][64]
  float* part_ml;       // [nsplit][B][Hkv][Tq * G][2]
};

typedef short s16x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int at_sw(int row) { return (((row >> 1) & 1) << 2) | ((row >> 2) & 3); }

// Byte offset of 16-byte chunk `ch` of row `row` of a tile.
__device__ __forceinline__ uint32_t at_off(int row, int ch) {
  return (uint32_t)(row * 128 + ((ch ^ at_sw(row)) << 4));
}

// Transposing read: the address this lane supplies so that, for the rows
// k0 .. k0+3 (k0 = 16 s + 8 g + 4 h, g = lane / 32) and columns m0 + 0..15
// of its 16-lane group (m0 = 32 mb + 16 ((lane >> 4) & 1)), lane receives
// column m0 + lane % 16 at those four rows.
__device__ __forceinline__ uint32_t at_tr_off(int lane, int s, int h, int mb) {
  const int sl = lane & 15;
  const int row = 16 * s + 8 * (lane >> 5) + 4 * h + (sl >> 2);
  const int col = 32 * mb + 16 * ((lane >> 4) & 1) + 4 * (sl & 3);
  return (uint32_t)(row * 128 + ((((col >> 3) ^ at_sw(row)) << 4) | ((col & 7) << 1)));
}

__device__ __forceinline__ u32x4_t at_tr8(const uint8_t* tile, uint32_t o0, uint32_t o1) {
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
  const s16x4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + o0));
  const s16x4_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + o1));
  const uint2 ua = __builtin_bit_cast(uint2, a), ub = __builtin_bit_cast(uint2, b);
  return u32x4_t{ua.x, ua.y, ub.x, ub.y};
}

// MFMA row r of S^T (or S) takes key (row) pi(r): with r = 8a + 4g + b
// (a 0..3, g 0..1, b 0..3), pi(r) = 16 (a >> 1) + 8g + 4 (a & 1) + b, so that
// output register v of lane half g is 8g + v (v < 8) or 16 + 8g + v - 8.
__device__ __forceinline__ int at_pi(int r) {
  const int a = r >> 3, g = (r >> 2) & 1, b = r & 3;
  return 16 * (a >> 1) + 8 * g + 4 * (a & 1) + b;
}

__device__ __forceinline__ f32x16_t at_mfma(const u32x4_t& a, const u32x4_t& b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                 c, 0, 0, 0);
}

// Two floats -> packed bf16 (v_cvt_pk_bf16_f32: round to nearest even).
__device__ __forceinline__ uint32_t at_pack2(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// max / sum of a value and its copy in lane ^ 32 (v_permlane32_swap: the
// pair holds both halves' values; combining them symmetrically gives every
// lane the same result, operands in the same order)
__device__ __forceinline__ float at_max32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float at_add32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt not waited on)
template <int N>
__device__ __forceinline__ void at_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Wait until at most min(ahead, MAXAHEAD) tiles of PER loads each are in flight.
template <int PER, int MAXAHEAD>
__device__ __forceinline__ void wait_vmcnt_tiles(int ahead) {
  if constexpr (MAXAHEAD <= 0) {
    at_wait_vmcnt<0>();
  } else {
    if (ahead >= MAXAHEAD) {
      at_wait_vmcnt<MAXAHEAD * PER>();
      return;
    }
    wait_vmcnt_tiles<PER, MAXAHEAD - 1>(ahead);
  }
}

// DMA of one 64-row x 128-byte tile by four waves: instruction m of wave w
// fills LDS bytes (256 m + 64 w + lane) * 16, i.e. row 32 m + 8 w + lane / 8,
// position lane & 7, from source chunk position ^ sw(row) of row row0 + row
// (clamped to rmax).
__device__ __forceinline__ void at_dma_tile(const uint16_t* src, int64_t stride, int row0, int rmax, uint8_t* tile,
                                            int wave, int lane) {
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int row = 32 * m + 8 * wave + (lane >> 3);
    const int ch = (lane & 7) ^ at_sw(row);
    const int r = min(row0 + row, rmax);
    __builtin_amdgcn_global_load_lds(src + (int64_t)r * stride + ch * 8, (lds_void*)(tile + (256 * m + 64 * wave) * 16),
                                     16, 0, 0);
  }
}

// Per-workgroup row geometry of the forward and the dq backward.
struct AtRows {
  int R, t, h, qpos, rows, R0, kt0, kt1, pos_first, pos_last;
  bool live_wave;
};

__device__ __forceinline__ AtRows at_rows(int Tq, int Tk, int G, int causal, int window, int rb, int hk, int wave,
                                          int c) {
  AtRows r;
  r.rows = Tq * G;
  r.R0 = rb * AT_BR;
  r.R = min(r.R0 + 32 * wave + c, r.rows - 1);  // rows past the end repeat the last (never stored)
  r.t = r.R / G;
  r.h = hk * G + (r.R - r.t * G);
  r.qpos = Tk - Tq + r.t;
  const int Rl = min(r.R0 + AT_BR, r.rows) - 1;
  r.pos_first = Tk - Tq + r.R0 / G;
  r.pos_last = Tk - Tq + Rl / G;
  const int j_end = causal ? min(Tk, r.pos_last + 1) : Tk;
  const int j_begin = window > 0 ? max(0, r.pos_first - window + 1) : 0;
  r.kt0 = j_begin / AT_BC;
  r.kt1 = (j_end + AT_BC - 1) / AT_BC;
  r.live_wave = r.R0 + 32 * wave < r.rows;
  return r;
}

__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(AttnArgs a) {
  extern __shared__ __align__(1024) uint8_t at_smem[];  // AT_NS stages of [K tile][V tile]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 31;
  const int g = lane >> 5;
  // the last row blocks have the most keys under a causal mask: start them first
  const int nsplit = a.nsplit > 1 ? a.nsplit : 1;
  const int sp = (int)blockIdx.x % nsplit;
  const int rb = (int)gridDim.x / nsplit - 1 - (int)blockIdx.x / nsplit;
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  const AtRows rw = at_rows(a.Tq, a.Tk, a.G, a.causal, a.window, rb, hk, wave, c);
  // this workgroup's key tiles: all of the row block's, or split sp's share
  int kt_lo = rw.kt0, kt_hi = rw.kt1;
  if (nsplit > 1) {
    const int per = (rw.kt1 - rw.kt0 + nsplit - 1) / nsplit;
    kt_lo = min(rw.kt1, rw.kt0 + sp * per);
    kt_hi = min(rw.kt1, kt_lo + per);
  }

  // Q fragments (B operand of S^T): d 16s + 8g .. +7 of row c
  const uint16_t* qrow = a.q + b * a.sqb + (int64_t)rw.t * a.sqt + (int64_t)rw.h * a.sqh;
  u32x4_t qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) qf[s] = *reinterpret_cast<const u32x4_t*>(qrow + 16 * s + 8 * g);

  const uint16_t* kbase = a.k + b * a.skb + (int64_t)hk * a.skh;
  const uint16_t* vbase = a.v + b * a.svb + (int64_t)hk * a.svh;
  auto issue = [&](int kt) {
    uint8_t* st = at_smem + (kt % AT_NS) * (2 * AT_TILE);
    at_dma_tile(kbase, a.skt, kt * AT_BC, a.Tk - 1, st, wave, lane);
    at_dma_tile(vbase, a.svt, kt * AT_BC, a.Tk - 1, st + AT_TILE, wave, lane);
  };
  constexpr int DPT = 4;  // DMA instructions per wave per tile

  // read offsets: K rows 32 kb + pi(c) at d chunk 2s + g (kb adds 4096);
  // V^T via transposing reads (d block db, 16-key step s adds 2048, halves h)
  uint32_t koff[4], voff[2][2];
#pragma unroll
  for (int s = 0; s < 4; ++s) koff[s] = at_off(at_pi(c), 2 * s + g);
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int h = 0; h < 2; ++h) voff[db][h] = at_tr_off(lane, 0, h, db);

  constexpr float LOG2E = 1.4426950408889634f;
  // the sink is the starting state of split 0 only
  float m = a.sinks && sp == 0 ? a.sinks[rw.h] * LOG2E : -INFINITY;
  float l = a.sinks && sp == 0 ? 1.f : 0.f;
  f32x16_t o[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[db][v] = 0.f;

  // the Q loads above are waited for here with the first tile
  for (int i = 0; i < AT_NS - 1; ++i)
    if (kt_lo + i < kt_hi) issue(kt_lo + i);
  for (int kt = kt_lo; kt < kt_hi; ++kt) {
    // tile kt has landed once at most the tiles issued after it are in
    // flight; the barrier also certifies every wave is done with tile kt-1,
    // whose stage takes tile kt + AT_NS - 1 (bare s_barrier: a
    // __syncthreads() fence would wait for that DMA too)
    wait_vmcnt_tiles<DPT, AT_NS - 2>(kt_hi - 1 - kt);
    asm volatile("s_barrier" ::: "memory");
    if (kt + AT_NS - 1 < kt_hi) issue(kt + AT_NS - 1);
    if (!rw.live_wave) continue;
    const uint8_t* K = at_smem + (kt % AT_NS) * (2 * AT_TILE);
    const uint8_t* V = K + AT_TILE;

    f32x16_t sc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) sc[kb][v] = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        sc[kb] = at_mfma(*reinterpret_cast<const u32x4_t*>(K + koff[s] + 4096 * kb), qf[s], sc[kb]);
    }
    const int j0 = kt * AT_BC;
    const bool full = j0 + AT_BC <= a.Tk && (!a.causal || j0 + AT_BC - 1 <= rw.pos_first) &&
                      (a.window <= 0 || j0 > rw.pos_last - a.window);
    // the maximum of the raw products (scale2 > 0), hidden keys at -inf
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        if (!full) {
          const int j = j0 + 32 * kb + (v < 8 ? 8 * g + v : 16 + 8 * g + v - 8);
          const bool vis = j < a.Tk && (!a.causal || j <= rw.qpos) && (a.window <= 0 || j > rw.qpos - a.window);
          sc[kb][v] = vis ? sc[kb][v] : -INFINITY;
        }
        mt = fmaxf(mt, sc[kb][v]);
      }
    // the accumulator is rescaled only when some row's maximum moved (every
    // other row has alpha = 1 exactly, or an accumulator still 0)
    const float mt2 = at_max32(mt) * a.scale2;
    const bool grow = mt2 > m;
    const float mn = grow ? mt2 : m;
    // a row that has seen nothing yet (no sink, every key so far hidden) keeps 0
    const float ms = mn == -INFINITY ? 0.f : mn;
    const float alpha = __builtin_amdgcn_exp2f(m - ms);
    float rs = 0.f;
    u32x4_t pf[4];  // P^T operands of the four 16-key steps
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        float p[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kb][8 * half + i], a.scale2, -ms));
          rs += p[i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) pf[2 * kb + half][i] = at_pack2(p[2 * i], p[2 * i + 1]);
      }
    rs = at_add32(rs);
    l = l * alpha + rs;
    m = mn;
    if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[db][v] *= alpha;
    }
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        o[db] = at_mfma(at_tr8(V + 2048 * s, voff[db][0], voff[db][1]), pf[s], o[db]);
  }

  if (rw.R0 + 32 * wave + c >= rw.rows) return;
  if (nsplit > 1) {
    const int64_t pidx = (((int64_t)sp * gridDim.z + b) * gridDim.y + hk) * rw.rows + rw.R;
    float* po = a.part_o + pidx * AT_D;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = 32 * db + 8 * q4 + 4 * g;
        *reinterpret_cast<f32x4_t*>(po + d) =
            f32x4_t{o[db][4 * q4], o[db][4 * q4 + 1], o[db][4 * q4 + 2], o[db][4 * q4 + 3]};
      }
    if (g == 0) *reinterpret_cast<float2*>(a.part_ml + pidx * 2) = make_float2(m, l);
    return;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t* orow = a.out + b * a.sob + (int64_t)rw.t * a.sot + (int64_t)rw.h * a.soh;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = 32 * db + 8 * q4 + 4 * g;
      uint2 w;
      w.x = at_pack2(o[db][4 * q4] * inv, o[db][4 * q4 + 1] * inv);
      w.y = at_pack2(o[db][4 * q4 + 2] * inv, o[db][4 * q4 + 3] * inv);
      *reinterpret_cast<uint2*>(orow + d) = w;
    }
  // __builtin_amdgcn_logf is log2
  if (a.lse && g == 0) a.lse[((int64_t)b * a.Hq + rw.h) * a.Tq + rw.t] = m + __builtin_amdgcn_logf(l);
}

// Merge of the key splits, one wave per row (lane = d): with M = max_s m_s,
// w_s = 2^(m_s - M), out = sum_s w_s o_s / sum_s w_s l_s and lse = M +
// log2(sum_s w_s l_s), the splits added in split order (deterministic).
__global__ __launch_bounds__(256) void attn_split_combine_kernel(AttnArgs a, int B, int Hkv) {
  const int lane = threadIdx.x & 63;
  const int rows = a.Tq * a.G;
  const int64_t q = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (b, hk, R)
  if (q >= (int64_t)B * Hkv * rows) return;
  const int R = (int)(q % rows);
  const int64_t bh = q / rows;
  const int hk = (int)(bh % Hkv);
  const int b = (int)(bh / Hkv);
  const int ns = a.nsplit;  // <= 64
  const int64_t stride = (int64_t)B * Hkv * rows;  // rows per split
  float ms = -INFINITY, ls = 0.f;
  if (lane < ns) {
    const float2 v = *reinterpret_cast<const float2*>(a.part_ml + (lane * stride + q) * 2);
    ms = v.x;
    ls = v.y;
  }
  float mt = ms;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mt = fmaxf(mt, __shfl_xor(mt, off));
  const float w = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - mt);
  float lt = w * ls;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) lt += __shfl_xor(lt, off);
  // eight splits' loads in flight at a time (added in split order); a split
  // with weight 0 holds zeros
  float acc = 0.f;
  const float* po = a.part_o + q * AT_D + lane;
  const int wi = __builtin_bit_cast(int, w);
  int sp = 0;
  for (; sp + 8 <= ns; sp += 8) {
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = po[(sp + j) * stride * AT_D];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += __builtin_bit_cast(float, __builtin_amdgcn_readlane(wi, sp + j)) * x[j];
  }
  for (; sp < ns; ++sp) acc += __builtin_bit_cast(float, __builtin_amdgcn_readlane(wi, sp)) * po[sp * stride * AT_D];
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  const int t = R / a.G;
  const int h = hk * a.G + (R - t * a.G);
  const __bf16 y = (__bf16)(acc * inv);
  a.out[b * a.sob + (int64_t)t * a.sot + (int64_t)h * a.soh + lane] = __builtin_bit_cast(uint16_t, y);
  if (a.lse && lane == 0) a.lse[((int64_t)b * a.Hq + h) * a.Tq + t] = mt + __builtin_amdgcn_logf(lt);
}

// ---------------------------------------------------------------------------
// Backward (the gradients autograd takes through eager_attention_forward,
// modeling_gpt_oss.py:235-264), from the forward's log2 denominators L:
//   p[t, j]  = 2^(S[t, j] * scaling * log2(e) - L[t])      (visible j, else 0)
//   D[t]     = dO[t] . O[t]       (= sum_j p dP: the sink has no value row)
//   dP[t, j] = dO[t] . v[j],   dS[t, j] = p (dP - D[t])
//   dq[t] = scaling * sum_j dS k[j],  dk[j] = scaling * sum_t dS q[t],
//   dv[j] = sum_t p[t, j] dO[t]
//   d sink[h] = -sum_t p_sink[t] D[t],  p_sink = 2^(sink log2(e) - L[t])
// Two kernels, no atomics: attn_bwd_dq (the forward's row blocks; it also
// writes each row's (L, D) in row order) and attn_bwd_dkv (key blocks, every
// row that sees them).
// ---------------------------------------------------------------------------
struct AttnBwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;    // forward output (strides so)
  const uint16_t* dout; // (strides sd)
  const float* lse;     // [B][Hq][Tq]
  float* stats;         // [B][Hkv][Tq * G][2]: (L, D) of row R, written by attn_bwd_dq
  uint16_t* dq;         // [B, Tq, Hq, 64] contiguous
  uint16_t* dk;         // [B, Tk, Hkv, 64] contiguous
  uint16_t* dv;
  int64_t sqb, sqt, sqh, skb, skt, skh, svb, svt, svh, sob, sot, soh, sdb, sdt, sdh;
  int Tq, Tk, Hq, Hkv, G;
  int causal, window;
  int kpairs;           // dk/dv workgroups take key blocks x and nblocks - 1 - x
  float scale2, scaling;
};

// 16 bf16 of a u32x4 pair -> float dot with another pair
__device__ __forceinline__ float at_dot8(const u32x4_t& x, const u32x4_t& y) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    s += __uint_as_float(x[i] << 16) * __uint_as_float(y[i] << 16) +
         __uint_as_float(x[i] & 0xFFFF0000u) * __uint_as_float(y[i] & 0xFFFF0000u);
  return s;
}

// dq: the forward's row blocks and K/V tile ring.  Per tile: S^T = K Q^T and
// dP^T = V dO^T (K and V rows permuted), dS^T in registers, dq^T += K^T dS^T
// (K^T by transposing reads of the K tile).
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_kernel(AttnBwdArgs a) {
  extern __shared__ __align__(1024) uint8_t at_smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 31;
  const int g = lane >> 5;
  const int rb = (int)gridDim.x - 1 - (int)blockIdx.x;
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  const AtRows rw = at_rows(a.Tq, a.Tk, a.G, a.causal, a.window, rb, hk, wave, c);

  const uint16_t* qrow = a.q + b * a.sqb + (int64_t)rw.t * a.sqt + (int64_t)rw.h * a.sqh;
  const uint16_t* drow = a.dout + b * a.sdb + (int64_t)rw.t * a.sdt + (int64_t)rw.h * a.sdh;
  const uint16_t* orow = a.o + b * a.sob + (int64_t)rw.t * a.sot + (int64_t)rw.h * a.soh;
  u32x4_t qf[4], df[4];
  float D = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    qf[s] = *reinterpret_cast<const u32x4_t*>(qrow + 16 * s + 8 * g);
    df[s] = *reinterpret_cast<const u32x4_t*>(drow + 16 * s + 8 * g);
    D += at_dot8(df[s], *reinterpret_cast<const u32x4_t*>(orow + 16 * s + 8 * g));
  }
  D = at_add32(D);
  const float L = a.lse[((int64_t)b * a.Hq + rw.h) * a.Tq + rw.t];
  if (g == 0 && rw.R0 + 32 * wave + c < rw.rows) {
    const float2 st2 = {L, D};
    *reinterpret_cast<float2*>(a.stats + (((int64_t)b * a.Hkv + hk) * rw.rows + rw.R) * 2) = st2;
  }

  const uint16_t* kbase = a.k + b * a.skb + (int64_t)hk * a.skh;
  const uint16_t* vbase = a.v + b * a.svb + (int64_t)hk * a.svh;
  auto issue = [&](int kt) {
    uint8_t* st = at_smem + (kt % AT_NS) * (2 * AT_TILE);
    at_dma_tile(kbase, a.skt, kt * AT_BC, a.Tk - 1, st, wave, lane);
    at_dma_tile(vbase, a.svt, kt * AT_BC, a.Tk - 1, st + AT_TILE, wave, lane);
  };
  constexpr int DPT = 4;
  uint32_t koff[4], toff[2][2];
#pragma unroll
  for (int s = 0; s < 4; ++s) koff[s] = at_off(at_pi(c), 2 * s + g);
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int h = 0; h < 2; ++h) toff[db][h] = at_tr_off(lane, 0, h, db);

  f32x16_t dq[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) dq[db][v] = 0.f;

  for (int i = 0; i < AT_NS - 1; ++i)
    if (rw.kt0 + i < rw.kt1) issue(rw.kt0 + i);
  for (int kt = rw.kt0; kt < rw.kt1; ++kt) {
    wait_vmcnt_tiles<DPT, AT_NS - 2>(rw.kt1 - 1 - kt);
    asm volatile("s_barrier" ::: "memory");
    if (kt + AT_NS - 1 < rw.kt1) issue(kt + AT_NS - 1);
    if (!rw.live_wave) continue;
    const uint8_t* K = at_smem + (kt % AT_NS) * (2 * AT_TILE);
    const uint8_t* V = K + AT_TILE;
    f32x16_t sc[2], dp[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) sc[kb][v] = dp[kb][v] = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        sc[kb] = at_mfma(*reinterpret_cast<const u32x4_t*>(K + koff[s] + 4096 * kb), qf[s], sc[kb]);
        dp[kb] = at_mfma(*reinterpret_cast<const u32x4_t*>(V + koff[s] + 4096 * kb), df[s], dp[kb]);
      }
    }
    const int j0 = kt * AT_BC;
    const bool full = j0 + AT_BC <= a.Tk && (!a.causal || j0 + AT_BC - 1 <= rw.pos_first) &&
                      (a.window <= 0 || j0 > rw.pos_last - a.window);
    u32x4_t sf[4];  // dS^T operands of the four 16-key steps
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        float ds[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int v = 8 * half + i;
          float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kb][v], a.scale2, -L));
          if (!full) {
            const int j = j0 + 32 * kb + (v < 8 ? 8 * g + v : 16 + 8 * g + v - 8);
            const bool vis = j < a.Tk && (!a.causal || j <= rw.qpos) && (a.window <= 0 || j > rw.qpos - a.window);
            p = vis ? p : 0.f;
          }
          ds[i] = p * (dp[kb][v] - D);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) sf[2 * kb + half][i] = at_pack2(ds[2 * i], ds[2 * i + 1]);
      }
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int s = 0; s < 4; ++s) dq[db] = at_mfma(at_tr8(K + 2048 * s, toff[db][0], toff[db][1]), sf[s], dq[db]);
  }

  if (rw.R0 + 32 * wave + c >= rw.rows) return;
  uint16_t* out = a.dq + (((int64_t)b * a.Tq + rw.t) * a.Hq + rw.h) * AT_D;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = 32 * db + 8 * q4 + 4 * g;
      uint2 w;
      w.x = at_pack2(dq[db][4 * q4] * a.scaling, dq[db][4 * q4 + 1] * a.scaling);
      w.y = at_pack2(dq[db][4 * q4 + 2] * a.scaling, dq[db][4 * q4 + 3] * a.scaling);
      *reinterpret_cast<uint2*>(out + d) = w;
    }
}

constexpr int AT_KB = 128;  // keys per dk/dv block (32 per key-wave)
constexpr int AT_RT = 64;   // rows per step of the dk/dv loop (a tile)
constexpr int AT_DKV_STAGE = 2 * AT_TILE + 8 * 256;  // q tile, dO tile, each wave's (L, D) of its 32 rows
constexpr int AT_DKV_RED = 4 * 64 * 32 * 4;          // row-wave 1's dk or dv partials (4 waves x 64 lanes x 32 floats)

// dk, dv: key blocks of 128 keys of one (batch, key head); eight waves,
// key-wave kw = w % 4 keeping keys 32 kw .. 32 kw + 31 (their k and v rows as
// the B operands of S = Q K^T and dP = dO V^T, lane c = key c) and row-wave
// rw = w / 4 taking rows 32 rw .. 32 rw + 31 of each 64-row tile.  The
// workgroup walks the tiles (rows R = t * G + i as in the forward) of every
// row that sees one of its keys, through a DMA ring: the q and dO tiles (rows
// permuted as A operands; q^T and dO^T by transposing reads for
// dv^T += dO^T P and dk^T += q^T dS) and (L, D) of each wave's rows.  At
// the end the two row-waves of a key-wave add their dk^T and dv^T through
// LDS.  Under a causal mask without a window, workgroup x takes key block x
// and then block nblocks - 1 - x, so every workgroup walks about the same
// number of rows.
__global__ __launch_bounds__(512, 1) void attn_bwd_dkv_kernel(AttnBwdArgs a) {
  extern __shared__ __align__(1024) uint8_t at_smem[];  // AT_NS_DKV stages, reused for the reduction
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int kw = wave & 3;
  const int rw = wave >> 2;
  const int c = lane & 31;
  const int g = lane >> 5;
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  const int rows = a.Tq * a.G;
  const int off = a.Tk - a.Tq;  // position of query 0
  const int nkb = (a.Tk + AT_KB - 1) / AT_KB;
  const uint16_t* qbase = a.q + b * a.sqb;
  const uint16_t* dbase = a.dout + b * a.sdb;
  const float* sbase = a.stats + ((int64_t)b * a.Hkv + hk) * rows * 2;

  // A operands: rows 32 rw + pi(c) at d chunk 2s + g; transposing reads of
  // rows 32 rw + 16 s + ... (s the 16-row step)
  uint32_t aoff[4], toff[2][2][2];
#pragma unroll
  for (int s = 0; s < 4; ++s) aoff[s] = at_off(32 * rw + at_pi(c), 2 * s + g);
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int h = 0; h < 2; ++h) toff[s][db][h] = at_tr_off(lane, 2 * rw + s, h, db);

  for (int pass = 0; pass < (a.kpairs ? 2 : 1); ++pass) {
    const int kbk = pass == 0 ? (int)blockIdx.x : nkb - 1 - (int)blockIdx.x;
    if (pass == 1 && kbk <= (int)blockIdx.x) break;  // the middle block of an odd count
    const int j0 = kbk * AT_KB;
    // rows that see a key of [j0, j0 + 128)
    int t_begin = 0, t_end = a.Tq;
    if (a.causal) {
      t_begin = max(0, j0 - off);
      if (a.window > 0) t_end = min(a.Tq, j0 + AT_KB - 1 + a.window - off);
    }
    const int r_begin = t_begin * a.G;
    const int r_end = max(r_begin, t_end * a.G);
    const int nt = (r_end - r_begin + AT_RT - 1) / AT_RT;

    const int jk = j0 + 32 * kw + c;
    const int jc = min(jk, a.Tk - 1);
    const uint16_t* krow = a.k + b * a.skb + (int64_t)jc * a.skt + (int64_t)hk * a.skh;
    const uint16_t* vrow = a.v + b * a.svb + (int64_t)jc * a.svt + (int64_t)hk * a.svh;
    u32x4_t kf[4], vf[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      kf[s] = *reinterpret_cast<const u32x4_t*>(krow + 16 * s + 8 * g);
      vf[s] = *reinterpret_cast<const u32x4_t*>(vrow + 16 * s + 8 * g);
    }
    // tile i: wave w fills rows 8w + lane / 8 of the q and dO tiles (source
    // row of t = R / G, head hk G + R % G, clamped to the last row) and its
    // own copy of (L, D) of rows 32 rw .. 32 rw + 31
    auto issue = [&](int i) {
      uint8_t* st = at_smem + (i % AT_NS_DKV) * AT_DKV_STAGE;
      const int row = 8 * wave + (lane >> 3);
      const int ch = (lane & 7) ^ at_sw(row);
      const int R = min(r_begin + i * AT_RT + row, rows - 1);
      const int t = R / a.G;
      const int h = hk * a.G + (R - t * a.G);
      __builtin_amdgcn_global_load_lds(qbase + (int64_t)t * a.sqt + (int64_t)h * a.sqh + ch * 8,
                                       (lds_void*)(st + 64 * wave * 16), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(dbase + (int64_t)t * a.sdt + (int64_t)h * a.sdh + ch * 8,
                                       (lds_void*)(st + AT_TILE + 64 * wave * 16), 16, 0, 0);
      const int Rs = min(r_begin + i * AT_RT + 32 * rw + (lane >> 1), rows - 1);
      __builtin_amdgcn_global_load_lds(sbase + (int64_t)Rs * 2 + (lane & 1),
                                       (lds_void*)(st + 2 * AT_TILE + wave * 256), 4, 0, 0);
    };
    constexpr int DPT = 3;

    f32x16_t dk[2], dv[2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int v = 0; v < 16; ++v) dk[db][v] = dv[db][v] = 0.f;

    // every wave is done with the previous pass's stages and reduction
    // buffer (and its k, v loads have landed) before they are refilled
    __syncthreads();
    for (int i = 0; i < AT_NS_DKV - 1; ++i)
      if (i < nt) issue(i);
    for (int it = 0; it < nt; ++it) {
      wait_vmcnt_tiles<DPT, AT_NS_DKV - 2>(nt - 1 - it);
      asm volatile("s_barrier" ::: "memory");
      if (it + AT_NS_DKV - 1 < nt) issue(it + AT_NS_DKV - 1);
      const uint8_t* Q = at_smem + (it % AT_NS_DKV) * AT_DKV_STAGE;
      const uint8_t* DO = Q + AT_TILE;
      const float* ST = reinterpret_cast<const float*>(Q + 2 * AT_TILE + wave * 256);
      const int rbase = r_begin + it * AT_RT + 32 * rw;  // this wave's first row
      // every row of the wave's half sees every key of the block
      const bool full = rbase + 32 <= r_end && j0 + AT_KB <= a.Tk &&
                        (!a.causal || off + rbase / a.G >= j0 + AT_KB - 1) &&
                        (a.window <= 0 || off + (rbase + 31) / a.G - a.window < j0);
      f32x16_t sc, dp;
#pragma unroll
      for (int v = 0; v < 16; ++v) sc[v] = dp[v] = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        sc = at_mfma(*reinterpret_cast<const u32x4_t*>(Q + aoff[s]), kf[s], sc);
        dp = at_mfma(*reinterpret_cast<const u32x4_t*>(DO + aoff[s]), vf[s], dp);
      }
      // register v: row 8g + v (v < 8) or 16 + 8g + v - 8 of the half, key c
      u32x4_t pf[2], sf[2];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        float p[8], ds[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = 16 * half + 8 * g + i;
          const float2 sd = *reinterpret_cast<const float2*>(ST + 2 * r);
          float x = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[8 * half + i], a.scale2, -sd.x));
          if (!full) {
            const int R = rbase + r;
            const int qp = off + R / a.G;
            const bool vis =
                R < r_end && jk < a.Tk && (!a.causal || jk <= qp) && (a.window <= 0 || jk > qp - a.window);
            x = vis ? x : 0.f;
          }
          p[i] = x;
          ds[i] = x * (dp[8 * half + i] - sd.y);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pf[half][i] = at_pack2(p[2 * i], p[2 * i + 1]);
          sf[half][i] = at_pack2(ds[2 * i], ds[2 * i + 1]);
        }
      }
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          dv[db] = at_mfma(at_tr8(DO, toff[s][db][0], toff[s][db][1]), pf[s], dv[db]);
          dk[db] = at_mfma(at_tr8(Q, toff[s][db][0], toff[s][db][1]), sf[s], dk[db]);
        }
    }

    // row-wave 1 hands its partial sums to row-wave 0 (dk, then dv)
    float* red = reinterpret_cast<float*>(at_smem) + (kw * 64 + lane) * 32;
#pragma unroll
    for (int which = 0; which < 2; ++which) {
      f32x16_t* acc = which == 0 ? dk : dv;
      __syncthreads();  // the ring (or the previous round) is no longer read
      if (rw == 1) {
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int v4 = 0; v4 < 4; ++v4)
            *reinterpret_cast<f32x4_t*>(red + 16 * db + 4 * v4) =
                f32x4_t{acc[db][4 * v4], acc[db][4 * v4 + 1], acc[db][4 * v4 + 2], acc[db][4 * v4 + 3]};
      }
      __syncthreads();
      if (rw == 0) {
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int v4 = 0; v4 < 4; ++v4) {
            const f32x4_t x = *reinterpret_cast<const f32x4_t*>(red + 16 * db + 4 * v4);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[db][4 * v4 + e] += x[e];
          }
      }
    }

    if (rw == 0 && jk < a.Tk) {
      uint16_t* okr = a.dk + (((int64_t)b * a.Tk + jk) * a.Hkv + hk) * AT_D;
      uint16_t* ovr = a.dv + (((int64_t)b * a.Tk + jk) * a.Hkv + hk) * AT_D;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int d = 32 * db + 8 * q4 + 4 * g;
          uint2 wk, wv;
          wk.x = at_pack2(dk[db][4 * q4] * a.scaling, dk[db][4 * q4 + 1] * a.scaling);
          wk.y = at_pack2(dk[db][4 * q4 + 2] * a.scaling, dk[db][4 * q4 + 3] * a.scaling);
          wv.x = at_pack2(dv[db][4 * q4], dv[db][4 * q4 + 1]);
          wv.y = at_pack2(dv[db][4 * q4 + 2], dv[db][4 * q4 + 3]);
          *reinterpret_cast<uint2*>(okr + d) = wk;
          *reinterpret_cast<uint2*>(ovr + d) = wv;
        }
    }
  }
}

constexpr int AT_FWD_LDS = AT_NS * 2 * AT_TILE;
constexpr int AT_DKV_LDS = AT_NS_DKV * AT_DKV_STAGE > AT_DKV_RED ? AT_NS_DKV * AT_DKV_STAGE : AT_DKV_RED;

static int at_allow_lds(const void* fn, int idx, int bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    set_error("no current HIP device");
    return BSA_EHIP;
  }
  static bool done[64][3];
  if (!done[dev][idx]) {
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) {
      set_error("attention: cannot allow %d bytes of LDS", bytes);
      return BSA_EHIP;
    }
    done[dev][idx] = true;
  }
  return BSA_OK;
}

static int at_check_common(const char* what, int64_t B, int64_t Tq, int64_t Tk, int64_t Hq, int64_t Hkv,
                           int64_t head_dim, int causal, int64_t window) {
  BSA_REQUIRE(head_dim == AT_D, "%s: head_dim must be %d (got %lld)", what, AT_D, (long long)head_dim);
  BSA_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= 64, "%s: Hq (%lld) must be a multiple of Hkv (%lld), at most 64x", what,
              (long long)Hq, (long long)Hkv);
  BSA_REQUIRE(window >= 0 && (window == 0 || causal), "%s: a window needs the causal mask", what);
  BSA_REQUIRE(!causal || Tq <= Tk, "%s: causal with more queries (%lld) than keys (%lld)", what, (long long)Tq,
              (long long)Tk);
  BSA_REQUIRE(B < 65536 && Hkv < 65536 && Tq * (Hq / Hkv) < INT32_MAX / 2 && Tk < INT32_MAX / 2 && window < INT32_MAX,
              "%s: too large", what);
  return BSA_OK;
}

static int at_check_strides(const char* what, const int64_t* const* st, int n) {
  for (int j = 0; j < n; ++j)
    for (int i = 0; i < 3; ++i)
      BSA_REQUIRE(st[j][i] % 8 == 0 && st[j][i] >= 0,
                  "%s: strides (batch, sequence, head) must be non-negative multiples of 8 elements", what);
  return BSA_OK;
}

static inline bool at_al16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Key splits of the forward for a shape: enough workgroups for the chip
// (about AT_SPLIT_TARGET in all) when the (row block, key head, batch) grid
// alone is short of it and a row block sees at least AT_SPLIT_MIN_TILES key
// tiles; at least two tiles per split, at most 64 splits.  A function of the
// shape only, so results do not depend on the device.
#ifndef BSA_AT_SPLIT_TARGET
#define BSA_AT_SPLIT_TARGET 512
#endif
constexpr int64_t AT_SPLIT_TARGET = BSA_AT_SPLIT_TARGET;
constexpr int64_t AT_SPLIT_MIN_TILES = 8;
static int at_split_count(int64_t B, int64_t Tq, int64_t Tk, int64_t Hq, int64_t Hkv, int causal, int64_t window) {
  if (B <= 0 || Tq <= 0 || Tk <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv) return 1;
  const int64_t G = Hq / Hkv;
  const int64_t base = (Tq * G + AT_BR - 1) / AT_BR * Hkv * B;
  if (base >= AT_SPLIT_TARGET) return 1;
  // key tiles of the row block that sees the most keys
  const int64_t keys = causal && window > 0 ? std::min<int64_t>(Tk, window + std::min<int64_t>(Tq, AT_BR)) : Tk;
  const int64_t tiles = (keys + AT_BC - 1) / AT_BC + (causal && window > 0 ? 1 : 0);
  if (tiles < AT_SPLIT_MIN_TILES) return 1;  // the merge launch costs more than a short range saves
  int64_t n = std::min<int64_t>((AT_SPLIT_TARGET + base - 1) / base, tiles / 2);
  n = std::min<int64_t>(n, 64);
  return n >= 2 ? (int)n : 1;
}

// Workspace layout of the key-split forward: part_o, then part_ml at a
// 256-byte boundary.
static int64_t at_split_bytes(int64_t nsplit, int64_t B, int64_t Tq, int64_t Hq) {
  if (nsplit <= 1) return 0;
  const int64_t rows = nsplit * B * Hq * Tq;  // = nsplit * B * Hkv * (Tq * G)
  const int64_t o = (rows * AT_D * 4 + 255) / 256 * 256;
  return o + (rows * 2 * 4 + 255) / 256 * 256;
}

// Shared checks and arguments of the two forward entry points.
static int at_fwd_args(AttnArgs& a, const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                       const void* v, const int64_t* v_strides, const float* sinks, int64_t B, int64_t Tq,
                       int64_t Tk, int64_t Hq, int64_t Hkv, int64_t head_dim, int causal, int64_t window,
                       float scaling, void* out, const int64_t* out_strides, float* lse) {
  BSA_REQUIRE(Tk > 0, "attention: queries without keys");
  BSA_REQUIRE(q && k && v && out && q_strides && k_strides && v_strides && out_strides, "attention: null pointer");
  int rc = at_check_common("attention", B, Tq, Tk, Hq, Hkv, head_dim, causal, window);
  if (rc) return rc;
  BSA_REQUIRE(at_al16(q) && at_al16(k) && at_al16(v) && at_al16(out), "attention: q, k, v and out must be 16-byte aligned");
  const int64_t* st[4] = {q_strides, k_strides, v_strides, out_strides};
  if ((rc = at_check_strides("attention", st, 4))) return rc;
  a = AttnArgs{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.sinks = sinks;
  a.out = static_cast<uint16_t*>(out);
  a.lse = lse;
  a.sqb = q_strides[0], a.sqt = q_strides[1], a.sqh = q_strides[2];
  a.skb = k_strides[0], a.skt = k_strides[1], a.skh = k_strides[2];
  a.svb = v_strides[0], a.svt = v_strides[1], a.svh = v_strides[2];
  a.sob = out_strides[0], a.sot = out_strides[1], a.soh = out_strides[2];
  a.Tq = (int)Tq;
  a.Tk = (int)Tk;
  a.Hq = (int)Hq;
  a.G = (int)(Hq / Hkv);
  a.causal = causal ? 1 : 0;
  a.window = (int)window;
  a.scale2 = scaling * 1.4426950408889634f;
  a.nsplit = 1;
  return BSA_OK;
}

static int at_fwd_launch(const AttnArgs& a, int64_t B, int64_t Hkv, hipStream_t st) {
  const int64_t rblocks = ((int64_t)a.Tq * a.G + AT_BR - 1) / AT_BR;
  int rc = at_allow_lds(reinterpret_cast<const void*>(attn_fwd_kernel), 0, AT_FWD_LDS);
  if (rc) return rc;
  hipLaunchKernelGGL(attn_fwd_kernel, dim3((unsigned)(rblocks * a.nsplit), (unsigned)Hkv, (unsigned)B), dim3(256),
                     AT_FWD_LDS, st, a);
  BSA_LAUNCH_CHECK("attention launch");
  if (a.nsplit > 1) {
    const int64_t nrow = B * Hkv * (int64_t)a.Tq * a.G;
    hipLaunchKernelGGL(attn_split_combine_kernel, dim3((unsigned)((nrow + 3) / 4)), dim3(256), 0, st, a, (int)B,
                       (int)Hkv);
    BSA_LAUNCH_CHECK("attention split combine launch");
  }
  return BSA_OK;
}

}  // namespace bsa

using namespace bsa;

extern "C" int bsa_attention_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                                 const void* v, const int64_t* v_strides, const float* sinks, int64_t B,
                                 int64_t Tq, int64_t Tk, int64_t Hq, int64_t Hkv, int64_t head_dim, int causal,
                                 int64_t window, float scaling, void* out, const int64_t* out_strides, float* lse,
                                 void* stream) {
  clear_error();
  BSA_REQUIRE(B >= 0 && Tq >= 0 && Tk >= 0 && Hq > 0 && Hkv > 0, "attention: bad shape");
  if (B == 0 || Tq == 0) return BSA_OK;
  AttnArgs a;
  int rc = at_fwd_args(a, q, q_strides, k, k_strides, v, v_strides, sinks, B, Tq, Tk, Hq, Hkv, head_dim, causal,
                       window, scaling, out, out_strides, lse);
  if (rc) return rc;
  return at_fwd_launch(a, B, Hkv, static_cast<hipStream_t>(stream));
}

extern "C" int64_t bsa_attention_split_workspace_bytes(int64_t B, int64_t Tq, int64_t Tk, int64_t Hq, int64_t Hkv,
                                                       int causal, int64_t window) {
  return at_split_bytes(at_split_count(B, Tq, Tk, Hq, Hkv, causal, window), B, Tq, Hq);
}

extern "C" int bsa_attention_fwd_split(const void* q, const int64_t* q_strides, const void* k,
                                       const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                       const float* sinks, int64_t B, int64_t Tq, int64_t Tk, int64_t Hq,
                                       int64_t Hkv, int64_t head_dim, int causal, int64_t window, float scaling,
                                       void* out, const int64_t* out_strides, float* lse, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  clear_error();
  BSA_REQUIRE(B >= 0 && Tq >= 0 && Tk >= 0 && Hq > 0 && Hkv > 0, "attention: bad shape");
  if (B == 0 || Tq == 0) return BSA_OK;
  AttnArgs a;
  int rc = at_fwd_args(a, q, q_strides, k, k_strides, v, v_strides, sinks, B, Tq, Tk, Hq, Hkv, head_dim, causal,
                       window, scaling, out, out_strides, lse);
  if (rc) return rc;
  const int ns = at_split_count(B, Tq, Tk, Hq, Hkv, causal, window);
  if (ns > 1) {
    const int64_t need = at_split_bytes(ns, B, Tq, Hq);
    BSA_REQUIRE(workspace && reinterpret_cast<uintptr_t>(workspace) % 256 == 0 && workspace_bytes >= need,
                "attention: the key-split forward needs a 256-byte aligned workspace of %lld bytes (got %lld)",
                (long long)need, (long long)workspace_bytes);
    const int64_t rows = (int64_t)ns * B * Hq * Tq;
    a.nsplit = ns;
    a.part_o = static_cast<float*>(workspace);
    a.part_ml = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + (rows * AT_D * 4 + 255) / 256 * 256);
  }
  return at_fwd_launch(a, B, Hkv, static_cast<hipStream_t>(stream));
}

extern "C" int bsa_attention_bwd(const void* grad_out, const int64_t* grad_strides, const void* q,
                                 const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
                                 const int64_t* v_strides, const void* out, const int64_t* out_strides,
                                 const float* lse, int64_t B, int64_t Tq, int64_t Tk, int64_t Hq, int64_t Hkv,
                                 int64_t head_dim, int causal, int64_t window, float scaling, void* grad_q,
                                 void* grad_k, void* grad_v, float* row_stats, void* stream) {
  clear_error();
  BSA_REQUIRE(B >= 0 && Tq >= 0 && Tk >= 0 && Hq > 0 && Hkv > 0, "attention bwd: bad shape");
  if (B == 0 || Tq == 0 || Tk == 0) return BSA_OK;
  BSA_REQUIRE(grad_out && q && k && v && out && lse && grad_q && grad_k && grad_v && row_stats && grad_strides &&
                  q_strides && k_strides && v_strides && out_strides,
              "attention bwd: null pointer");
  int rc = at_check_common("attention bwd", B, Tq, Tk, Hq, Hkv, head_dim, causal, window);
  if (rc) return rc;
  BSA_REQUIRE(at_al16(grad_out) && at_al16(q) && at_al16(k) && at_al16(v) && at_al16(out) && at_al16(grad_q) &&
                  at_al16(grad_k) && at_al16(grad_v) && at_al16(row_stats),
              "attention bwd: tensors must be 16-byte aligned");
  const int64_t* st[5] = {grad_strides, q_strides, k_strides, v_strides, out_strides};
  if ((rc = at_check_strides("attention bwd", st, 5))) return rc;
  AttnBwdArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o = static_cast<const uint16_t*>(out);
  a.dout = static_cast<const uint16_t*>(grad_out);
  a.lse = lse;
  a.stats = row_stats;
  a.dq = static_cast<uint16_t*>(grad_q);
  a.dk = static_cast<uint16_t*>(grad_k);
  a.dv = static_cast<uint16_t*>(grad_v);
  a.sdb = grad_strides[0], a.sdt = grad_strides[1], a.sdh = grad_strides[2];
  a.sqb = q_strides[0], a.sqt = q_strides[1], a.sqh = q_strides[2];
  a.skb = k_strides[0], a.skt = k_strides[1], a.skh = k_strides[2];
  a.svb = v_strides[0], a.svt = v_strides[1], a.svh = v_strides[2];
  a.sob = out_strides[0], a.sot = out_strides[1], a.soh = out_strides[2];
  a.Tq = (int)Tq;
  a.Tk = (int)Tk;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.G = (int)(Hq / Hkv);
  a.causal = causal ? 1 : 0;
  a.window = (int)window;
  a.scale2 = scaling * 1.4426950408889634f;
  a.scaling = scaling;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t rblocks = (Tq * a.G + AT_BR - 1) / AT_BR;
  if ((rc = at_allow_lds(reinterpret_cast<const void*>(attn_bwd_dq_kernel), 1, AT_FWD_LDS))) return rc;
  hipLaunchKernelGGL(attn_bwd_dq_kernel, dim3((unsigned)rblocks, (unsigned)Hkv, (unsigned)B), dim3(256), AT_FWD_LDS, s,
                     a);
  BSA_LAUNCH_CHECK("attention bwd (dq) launch");
  const int nkb = (int)((Tk + AT_KB - 1) / AT_KB);
  // causal without a window: a key block's row count falls linearly with its
  // index, so blocks x and nkb - 1 - x share a workgroup
  a.kpairs = (causal && window == 0 && nkb > 1) ? 1 : 0;
  const int kgrid = a.kpairs ? (nkb + 1) / 2 : nkb;
  if ((rc = at_allow_lds(reinterpret_cast<const void*>(attn_bwd_dkv_kernel), 2, AT_DKV_LDS))) return rc;
  hipLaunchKernelGGL(attn_bwd_dkv_kernel, dim3((unsigned)kgrid, (unsigned)Hkv, (unsigned)B), dim3(512), AT_DKV_LDS, s,
                     a);
  BSA_LAUNCH_CHECK("attention bwd (dk, dv) launch");
  return BSA_OK;
}
