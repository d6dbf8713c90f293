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
// on bf16 MFMA with float32 accumulation; the probabilities are rounded to
// bf16 for the P.V product (as the eager path's cast to the value dtype).
//
// Kernel (gfx950): a workgroup takes 128 rows of one (batch, key head): row
// R = t * G + i is query t of head G * hk + i (G = Hq / Hkv), so the G heads
// sharing a key head read each K/V tile once.  Four waves, 32 rows each;
// key tiles of 64 in LDS, double buffered.  Per tile a wave computes
//   S^T = K Q^T  (v_mfma_f32_32x32x16_bf16, lane c = query c): the row max
//                and sum of a query are one exchange between the two lane
//                halves.  The K rows enter the MFMA permuted (pi below), so
//                lane half g holds keys 8g .. 8g+7 and 16+8g .. 16+8g+7 of
//                each 32-key block: exactly the B operand of
//   O^T += V^T P^T  with V^T staged transposed in LDS.  The accumulator
//                rows are head dimensions and its columns queries, so the
//                online-softmax rescale of query c stays in lane c.
// LDS tiles: K [64 keys][64 d] and V^T [64 d][64 keys], bf16, 128-byte rows
// whose 16-byte chunk c sits at chunk c ^ ((row >> 1) & 7) (a ds_read_b128
// pass serves 16 lanes from 64 banks, 256 bytes: two rows, so the swizzle
// pairs rows).
// ---------------------------------------------------------------------------
#include "bsa_common.h"

namespace bsa {

constexpr int AT_D = 64;                    // head dimension
constexpr int AT_BR = 128;                  // rows per workgroup
constexpr int AT_BC = 64;                   // keys per tile
constexpr int AT_TILE = AT_BC * AT_D * 2;   // 8 KiB

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
};

// Byte offset of 16-byte chunk `ch` of row `row` in a 128-byte-row LDS tile.
__device__ __forceinline__ uint32_t at_off(int row, int ch) {
  return (uint32_t)(row * 128 + ((ch ^ ((row >> 1) & 7)) << 4));
}

// MFMA row r of the S^T product takes key pi(r): with r = 8a + 4g + b
// (a 0..3, g 0..1, b 0..3), pi(r) = 16 (a >> 1) + 8g + 4 (a & 1) + b, so that
// output register v of lane half g is key 8g + v (v < 8) or 16 + 8g + v - 8.
__device__ __forceinline__ int at_pi(int r) {
  const int a = r >> 3, g = (r >> 2) & 1, b = r & 3;
  return 16 * (a >> 1) + 8 * g + 4 * (a & 1) + b;
}

__device__ __forceinline__ f32x16_t at_mfma(const u32x4_t& a, const u32x4_t& b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                 c, 0, 0, 0);
}

__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(AttnArgs a) {
  __shared__ __align__(16) uint8_t sK[2][AT_TILE];
  __shared__ __align__(16) uint8_t sV[2][AT_TILE];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 31;
  const int g = lane >> 5;
  // the last row blocks have the most keys under a causal mask: start them first
  const int rb = (int)gridDim.x - 1 - (int)blockIdx.x;
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  const int rows = a.Tq * a.G;
  const int R0 = rb * AT_BR;

  // --- this lane's query row ------------------------------------------------
  const int R = min(R0 + 32 * wave + c, rows - 1);  // rows past the end repeat the last (never stored)
  const int t = R / a.G;
  const int h = hk * a.G + (R - t * a.G);
  const int qpos = a.Tk - a.Tq + t;

  // --- the workgroup's key tiles ------------------------------------------
  const int Rl = min(R0 + AT_BR, rows) - 1;
  const int pos_first = a.Tk - a.Tq + R0 / a.G;
  const int pos_last = a.Tk - a.Tq + Rl / a.G;
  const int j_end = a.causal ? min(a.Tk, pos_last + 1) : a.Tk;
  const int j_begin = a.window > 0 ? max(0, pos_first - a.window + 1) : 0;
  const int kt0 = j_begin / AT_BC;
  const int kt1 = (j_end + AT_BC - 1) / AT_BC;

  // --- Q fragments (B operand of S^T): d 16s + 8g .. +7 of row c -----------
  const uint16_t* qrow = a.q + b * a.sqb + (int64_t)t * a.sqt + (int64_t)h * a.sqh;
  u32x4_t qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) qf[s] = *reinterpret_cast<const u32x4_t*>(qrow + 16 * s + 8 * g);

  // --- tile loaders --------------------------------------------------------
  const uint16_t* kbase = a.k + b * a.skb + (int64_t)hk * a.skh;
  const uint16_t* vbase = a.v + b * a.svb + (int64_t)hk * a.svh;
  // K by DMA: instruction m of wave w fills LDS bytes (256m + 64w + lane) * 16:
  // row 32m + 8w + lane / 8, position lane & 7 (source chunk position ^ swizzle)
  auto issue_k = [&](int kt, int buf) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int row = 32 * m + 8 * wave + (lane >> 3);
      const int ch = (lane & 7) ^ ((row >> 1) & 7);
      const int j = min(kt * AT_BC + row, a.Tk - 1);
      __builtin_amdgcn_global_load_lds(kbase + (int64_t)j * a.skt + ch * 8,
                                       (lds_void*)(&sK[buf][0] + (256 * m + 64 * wave) * 16), 16, 0, 0);
    }
  };
  // V through registers: lane = key, wave w = head dimensions 16w .. 16w+15,
  // written transposed
  u32x4_t vr[2];
  auto load_v = [&](int kt) {
    const int j = min(kt * AT_BC + lane, a.Tk - 1);
    const u32x4_t* p = reinterpret_cast<const u32x4_t*>(vbase + (int64_t)j * a.svt + 16 * wave);
    vr[0] = p[0];
    vr[1] = p[1];
  };
  auto store_vt = [&](int buf) {
    uint8_t* base = &sV[buf][0];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = 16 * wave + i;
      const uint32_t w = vr[i >> 3][(i & 7) >> 1];
      const uint16_t val = (uint16_t)((i & 1) ? (w >> 16) : (w & 0xFFFFu));
      *reinterpret_cast<uint16_t*>(base + at_off(row, lane >> 3) + (lane & 7) * 2) = val;
    }
  };

  // --- per-lane LDS read offsets ---------------------------------------------
  // S^T A operand: K row 32 kb + pi(c), d chunk 2s + g
  uint32_t koff[2][4];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int s = 0; s < 4; ++s) koff[kb][s] = at_off(32 * kb + at_pi(c), 2 * s + g);
  // O^T A operand: V^T row 32 db + c, key chunk 2s + g
  uint32_t voff[2][4];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int s = 0; s < 4; ++s) voff[db][s] = at_off(32 * db + c, 2 * s + g);

  // --- state -------------------------------------------------------------
  constexpr float LOG2E = 1.4426950408889634f;
  float m = a.sinks ? a.sinks[h] * LOG2E : -INFINITY;
  float l = a.sinks ? 1.f : 0.f;
  f32x16_t o[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[db][v] = 0.f;

  if (kt0 < kt1) {
    load_v(kt0);
    issue_k(kt0, 0);
  }
  for (int kt = kt0; kt < kt1; ++kt) {
    const int buf = (kt - kt0) & 1;
    // V^T of this tile into its buffer (last read two tiles ago, before the
    // previous barrier), then wait for this tile's K and meet every wave
    store_vt(buf);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (kt + 1 < kt1) {
      load_v(kt + 1);
      issue_k(kt + 1, buf ^ 1);
    }
    const uint8_t* K = &sK[buf][0];
    const uint8_t* V = &sV[buf][0];

    // S^T: two 32-key blocks
    f32x16_t sc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) sc[kb][v] = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        sc[kb] = at_mfma(*reinterpret_cast<const u32x4_t*>(K + koff[kb][s]), qf[s], sc[kb]);
    }
    // scale, mask, running maximum
    const int j0 = kt * AT_BC;
    const bool full = j0 + AT_BC <= a.Tk && (!a.causal || j0 + AT_BC - 1 <= pos_first) &&
                      (a.window <= 0 || j0 > pos_last - a.window);
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        float x = sc[kb][v] * a.scale2;
        if (!full) {
          const int j = j0 + 32 * kb + (v < 8 ? 8 * g + v : 16 + 8 * g + v - 8);
          const bool vis = j < a.Tk && (!a.causal || j <= qpos) && (a.window <= 0 || j > qpos - a.window);
          x = vis ? x : -INFINITY;
        }
        sc[kb][v] = x;
        mt = fmaxf(mt, x);
      }
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float mn = fmaxf(m, mt);
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
          p[i] = __builtin_amdgcn_exp2f(sc[kb][8 * half + i] - ms);
          rs += p[i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) pf[2 * kb + half][i] = pack_bf16x2(p[2 * i], p[2 * i + 1]);
      }
    rs += __shfl_xor(rs, 32);
    l = l * alpha + rs;
    m = mn;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
#pragma unroll
      for (int v = 0; v < 16; ++v) o[db][v] *= alpha;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        o[db] = at_mfma(*reinterpret_cast<const u32x4_t*>(V + voff[db][s]), pf[s], o[db]);
    }
  }

  // --- output --------------------------------------------------------------
  if (R0 + 32 * wave + c >= rows) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t* orow = a.out + b * a.sob + (int64_t)t * a.sot + (int64_t)h * a.soh;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = 32 * db + 8 * q4 + 4 * g;
      uint2 w;
      w.x = pack_bf16x2(o[db][4 * q4] * inv, o[db][4 * q4 + 1] * inv);
      w.y = pack_bf16x2(o[db][4 * q4 + 2] * inv, o[db][4 * q4 + 3] * inv);
      *reinterpret_cast<uint2*>(orow + d) = w;
    }
  // __builtin_amdgcn_logf is log2
  if (a.lse && g == 0) a.lse[((int64_t)b * a.Hq + h) * a.Tq + t] = m + __builtin_amdgcn_logf(l);
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
  BSA_REQUIRE(Tk > 0, "attention: queries without keys");
  BSA_REQUIRE(head_dim == AT_D, "attention: head_dim must be %d (got %lld)", AT_D, (long long)head_dim);
  BSA_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= 64, "attention: Hq (%lld) must be a multiple of Hkv (%lld), at most 64x",
              (long long)Hq, (long long)Hkv);
  BSA_REQUIRE(q && k && v && out && q_strides && k_strides && v_strides && out_strides, "attention: null pointer");
  BSA_REQUIRE(window >= 0 && (window == 0 || causal), "attention: a window needs the causal mask");
  BSA_REQUIRE(!causal || Tq <= Tk, "attention: causal with more queries (%lld) than keys (%lld)", (long long)Tq,
              (long long)Tk);
  BSA_REQUIRE(B < 65536 && Hkv < 65536 && Tq * (Hq / Hkv) < INT32_MAX / 2 && Tk < INT32_MAX / 2 &&
                  window < INT32_MAX,
              "attention: too large");
  auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  BSA_REQUIRE(al16(q) && al16(k) && al16(v) && al16(out), "attention: q, k, v and out must be 16-byte aligned");
  for (int i = 0; i < 3; ++i)
    BSA_REQUIRE(q_strides[i] % 8 == 0 && k_strides[i] % 8 == 0 && v_strides[i] % 8 == 0 && out_strides[i] % 8 == 0 &&
                    q_strides[i] >= 0 && k_strides[i] >= 0 && v_strides[i] >= 0 && out_strides[i] >= 0,
                "attention: strides (batch, sequence, head) must be non-negative multiples of 8 elements");
  AttnArgs a{};
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
  const int64_t rblocks = (Tq * a.G + AT_BR - 1) / AT_BR;
  BSA_REQUIRE(rblocks < INT32_MAX, "attention: too many rows");
  hipLaunchKernelGGL(attn_fwd_kernel, dim3((unsigned)rblocks, (unsigned)Hkv, (unsigned)B), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  BSA_LAUNCH_CHECK("attention launch");
  return BSA_OK;
}

namespace bsa {

// ---------------------------------------------------------------------------
// Backward (the gradients autograd takes through eager_attention_forward,
// modeling_gpt_oss.py:235-264), from the forward's log2 denominators L:
//   p[t, j]  = 2^(S[t, j] * scaling * log2(e) - L[t])      (visible j, else 0)
//   D[t]     = dO[t] . O[t]       (= sum_j p dP: the sink has no value row)
//   dP[t, j] = dO[t] . v[j],   dS[t, j] = p (dP - D[t])
//   dq[t] = scaling * sum_j dS k[j],  dk[j] = scaling * sum_t dS q[t],
//   dv[j] = sum_t p[t, j] dO[t]
//   d sink[h] = -sum_t p_sink[t] D[t],  p_sink = 2^(sink log2(e) - L[t])
// Two kernels, no atomics: attn_bwd_dq (the forward's row blocks, writing D)
// and attn_bwd_dkv (blocks of 128 keys, every row that sees them).
// ---------------------------------------------------------------------------
struct AttnBwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;    // forward output [B, Tq, Hq, 64] (strides so, like out)
  const uint16_t* dout; // [B, Tq, Hq, 64] (strides sd)
  const float* lse;     // [B][Hq][Tq]
  float* drow;          // [B][Hq][Tq]: D, written by attn_bwd_dq, read by attn_bwd_dkv
  uint16_t* dq;         // [B, Tq, Hq, 64] contiguous
  uint16_t* dk;         // [B, Tk, Hkv, 64] contiguous
  uint16_t* dv;
  int64_t sqb, sqt, sqh, skb, skt, skh, svb, svt, svh, sob, sot, soh, sdb, sdt, sdh;
  int Tq, Tk, Hq, Hkv, G;
  int causal, window;
  float scale2, scaling;
};

__device__ __forceinline__ bool at_visible(const AttnBwdArgs& a, int j, int qpos) {
  return j < a.Tk && (!a.causal || j <= qpos) && (a.window <= 0 || j > qpos - a.window);
}

// 16 bf16 of a u32x4 pair -> float dot with another pair
__device__ __forceinline__ float at_dot8(const u32x4_t& x, const u32x4_t& y) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    s += __uint_as_float(x[i] << 16) * __uint_as_float(y[i] << 16) +
         __uint_as_float(x[i] & 0xFFFF0000u) * __uint_as_float(y[i] & 0xFFFF0000u);
  return s;
}

// dq: the forward's row blocks.  LDS per buffer: K (S^T operand), V (dP^T
// operand: dP^T = V dO^T, V rows permuted like K), K^T (dq^T = K^T dS^T).
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_kernel(AttnBwdArgs a) {
  __shared__ __align__(16) uint8_t sK[2][AT_TILE];
  __shared__ __align__(16) uint8_t sV[2][AT_TILE];
  __shared__ __align__(16) uint8_t sKt[2][AT_TILE];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 31;
  const int g = lane >> 5;
  const int rb = (int)gridDim.x - 1 - (int)blockIdx.x;
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  const int rows = a.Tq * a.G;
  const int R0 = rb * AT_BR;
  const int R = min(R0 + 32 * wave + c, rows - 1);
  const int t = R / a.G;
  const int h = hk * a.G + (R - t * a.G);
  const int qpos = a.Tk - a.Tq + t;
  const int Rl = min(R0 + AT_BR, rows) - 1;
  const int pos_first = a.Tk - a.Tq + R0 / a.G;
  const int pos_last = a.Tk - a.Tq + Rl / a.G;
  const int j_end = a.causal ? min(a.Tk, pos_last + 1) : a.Tk;
  const int j_begin = a.window > 0 ? max(0, pos_first - a.window + 1) : 0;
  const int kt0 = j_begin / AT_BC;
  const int kt1 = (j_end + AT_BC - 1) / AT_BC;

  // row operands: q and dO (B operands, d 16s + 8g ..), D = dO . O
  const uint16_t* qrow = a.q + b * a.sqb + (int64_t)t * a.sqt + (int64_t)h * a.sqh;
  const uint16_t* drow_p = a.dout + b * a.sdb + (int64_t)t * a.sdt + (int64_t)h * a.sdh;
  const uint16_t* orow = a.o + b * a.sob + (int64_t)t * a.sot + (int64_t)h * a.soh;
  u32x4_t qf[4], df[4];
  float D = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    qf[s] = *reinterpret_cast<const u32x4_t*>(qrow + 16 * s + 8 * g);
    df[s] = *reinterpret_cast<const u32x4_t*>(drow_p + 16 * s + 8 * g);
    D += at_dot8(df[s], *reinterpret_cast<const u32x4_t*>(orow + 16 * s + 8 * g));
  }
  D += __shfl_xor(D, 32);
  const int64_t rowi = ((int64_t)b * a.Hq + h) * a.Tq + t;
  const float L = a.lse[rowi];
  if (g == 0 && R0 + 32 * wave + c < rows) a.drow[rowi] = D;

  const uint16_t* kbase = a.k + b * a.skb + (int64_t)hk * a.skh;
  const uint16_t* vbase = a.v + b * a.svb + (int64_t)hk * a.svh;
  auto issue_kv = [&](int kt, int buf) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int row = 32 * m + 8 * wave + (lane >> 3);
      const int ch = (lane & 7) ^ ((row >> 1) & 7);
      const int j = min(kt * AT_BC + row, a.Tk - 1);
      __builtin_amdgcn_global_load_lds(kbase + (int64_t)j * a.skt + ch * 8,
                                       (lds_void*)(&sK[buf][0] + (256 * m + 64 * wave) * 16), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(vbase + (int64_t)j * a.svt + ch * 8,
                                       (lds_void*)(&sV[buf][0] + (256 * m + 64 * wave) * 16), 16, 0, 0);
    }
  };
  u32x4_t kr[2];
  auto load_kt = [&](int kt) {
    const int j = min(kt * AT_BC + lane, a.Tk - 1);
    const u32x4_t* p = reinterpret_cast<const u32x4_t*>(kbase + (int64_t)j * a.skt + 16 * wave);
    kr[0] = p[0];
    kr[1] = p[1];
  };
  auto store_kt = [&](int buf) {
    uint8_t* base = &sKt[buf][0];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t w = kr[i >> 3][(i & 7) >> 1];
      *reinterpret_cast<uint16_t*>(base + at_off(16 * wave + i, lane >> 3) + (lane & 7) * 2) =
          (uint16_t)((i & 1) ? (w >> 16) : (w & 0xFFFFu));
    }
  };
  uint32_t koff[2][4], toff[2][4];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      koff[kb][s] = at_off(32 * kb + at_pi(c), 2 * s + g);
      toff[kb][s] = at_off(32 * kb + c, 2 * s + g);
    }

  f32x16_t dq[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) dq[db][v] = 0.f;

  if (kt0 < kt1) {
    load_kt(kt0);
    issue_kv(kt0, 0);
  }
  for (int kt = kt0; kt < kt1; ++kt) {
    const int buf = (kt - kt0) & 1;
    store_kt(buf);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (kt + 1 < kt1) {
      load_kt(kt + 1);
      issue_kv(kt + 1, buf ^ 1);
    }
    const uint8_t* K = &sK[buf][0];
    const uint8_t* V = &sV[buf][0];
    const uint8_t* Kt = &sKt[buf][0];
    f32x16_t sc[2], dp[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) sc[kb][v] = dp[kb][v] = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        sc[kb] = at_mfma(*reinterpret_cast<const u32x4_t*>(K + koff[kb][s]), qf[s], sc[kb]);
        dp[kb] = at_mfma(*reinterpret_cast<const u32x4_t*>(V + koff[kb][s]), df[s], dp[kb]);
      }
    }
    const int j0 = kt * AT_BC;
    const bool full = j0 + AT_BC <= a.Tk && (!a.causal || j0 + AT_BC - 1 <= pos_first) &&
                      (a.window <= 0 || j0 > pos_last - a.window);
    u32x4_t sf[4];  // dS^T operands of the four 16-key steps
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        float ds[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int v = 8 * half + i;
          float p = __builtin_amdgcn_exp2f(sc[kb][v] * a.scale2 - L);
          if (!full) {
            const int j = j0 + 32 * kb + (v < 8 ? 8 * g + v : 16 + 8 * g + v - 8);
            p = at_visible(a, j, qpos) ? p : 0.f;
          }
          ds[i] = p * (dp[kb][v] - D);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) sf[2 * kb + half][i] = pack_bf16x2(ds[2 * i], ds[2 * i + 1]);
      }
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        dq[db] = at_mfma(*reinterpret_cast<const u32x4_t*>(Kt + toff[db][s]), sf[s], dq[db]);
  }

  if (R0 + 32 * wave + c >= rows) return;
  uint16_t* out = a.dq + (((int64_t)b * a.Tq + t) * a.Hq + h) * AT_D;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = 32 * db + 8 * q4 + 4 * g;
      uint2 w;
      w.x = pack_bf16x2(dq[db][4 * q4] * a.scaling, dq[db][4 * q4 + 1] * a.scaling);
      w.y = pack_bf16x2(dq[db][4 * q4 + 2] * a.scaling, dq[db][4 * q4 + 3] * a.scaling);
      *reinterpret_cast<uint2*>(out + d) = w;
    }
}

// Byte offset of 16-byte chunk `ch` of row `row` in a 64-byte-row LDS tile
// (16 rows span 1 KiB; the swizzle spreads the four 256-byte groups).
__device__ __forceinline__ uint32_t at_off64(int row, int ch) {
  return (uint32_t)(row * 64 + ((ch ^ ((row >> 2) & 3)) << 4));
}

constexpr int AT_KB = 128;  // keys per dk/dv workgroup (32 per wave)
constexpr int AT_RT = 32;   // rows per step of the dk/dv loop

// dk, dv: workgroups of 128 keys of one (batch, key head); wave w keeps keys
// 32w .. 32w+31 (their k and v rows as the B operands of S = Q K^T and
// dP = dO V^T, lane c = key c) and their dk^T, dv^T accumulators.  The
// workgroup walks 32-row steps (rows R = t * G + i as in the forward) of
// every row that sees one of its keys; a step's q and dO rows are staged in
// LDS twice: natural [32][64] (the A operands, rows permuted by pi) and
// transposed [64][32] (dv^T += dO^T P, dk^T += q^T dS), with L and D.
__global__ __launch_bounds__(256, 2) void attn_bwd_dkv_kernel(AttnBwdArgs a) {
  constexpr int NAT = AT_RT * AT_D * 2;  // 4 KiB
  __shared__ __align__(16) uint8_t sQ[2][NAT];
  __shared__ __align__(16) uint8_t sD[2][NAT];
  __shared__ __align__(16) uint8_t sQt[2][NAT];
  __shared__ __align__(16) uint8_t sDt[2][NAT];
  __shared__ __align__(16) float sL[2][AT_RT];
  __shared__ __align__(16) float sDr[2][AT_RT];
  __shared__ int sPos[2][AT_RT];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 31;
  const int g = lane >> 5;
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  const int j0 = blockIdx.x * AT_KB;
  const int rows = a.Tq * a.G;
  const int off = a.Tk - a.Tq;  // position of query 0

  // rows that see a key of [j0, j0 + 128)
  int t_begin = 0, t_end = a.Tq;
  if (a.causal) {
    t_begin = max(0, j0 - off);
    if (a.window > 0) t_end = min(a.Tq, j0 + AT_KB - 1 + a.window - off);
  }
  const int r_begin = t_begin * a.G;
  const int r_end = max(r_begin, t_end * a.G);
  const int nsteps = (r_end - r_begin + AT_RT - 1) / AT_RT;

  // this lane's key: B operands k and v (d 16s + 8g ..)
  const int jk = j0 + 32 * wave + c;
  const int jc = min(jk, a.Tk - 1);
  const uint16_t* krow = a.k + b * a.skb + (int64_t)jc * a.skt + (int64_t)hk * a.skh;
  const uint16_t* vrow = a.v + b * a.svb + (int64_t)jc * a.svt + (int64_t)hk * a.svh;
  u32x4_t kf[4], vf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    kf[s] = *reinterpret_cast<const u32x4_t*>(krow + 16 * s + 8 * g);
    vf[s] = *reinterpret_cast<const u32x4_t*>(vrow + 16 * s + 8 * g);
  }

  // staging: thread = (row r = tid & 31, d chunk dc = tid >> 5), 16 bytes of q and dO
  const int sr = tid & 31;
  const int sdc = tid >> 5;
  u32x4_t rq, rd;
  float rl = 0.f, rdr = 0.f;
  int rpos = 0;
  auto load_rows = [&](int step) {
    const int Rr = min(r_begin + step * AT_RT + sr, rows - 1);
    const int tt = Rr / a.G;
    const int hh = hk * a.G + (Rr - tt * a.G);
    rq = *reinterpret_cast<const u32x4_t*>(a.q + b * a.sqb + (int64_t)tt * a.sqt + (int64_t)hh * a.sqh + 8 * sdc);
    rd = *reinterpret_cast<const u32x4_t*>(a.dout + b * a.sdb + (int64_t)tt * a.sdt + (int64_t)hh * a.sdh +
                                           8 * sdc);
    if (sdc == 0) {
      const int64_t ri = ((int64_t)b * a.Hq + hh) * a.Tq + tt;
      // rows past the end get an infinite L: p = 0
      const bool live = r_begin + step * AT_RT + sr < r_end;
      rl = live ? a.lse[ri] : INFINITY;
      rdr = a.drow[ri];
      rpos = off + tt;
    }
  };
  auto store_rows = [&](int buf) {
    *reinterpret_cast<u32x4_t*>(&sQ[buf][0] + at_off(sr, sdc)) = rq;
    *reinterpret_cast<u32x4_t*>(&sD[buf][0] + at_off(sr, sdc)) = rd;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint16_t xq = (uint16_t)((i & 1) ? (rq[i >> 1] >> 16) : (rq[i >> 1] & 0xFFFFu));
      const uint16_t xd = (uint16_t)((i & 1) ? (rd[i >> 1] >> 16) : (rd[i >> 1] & 0xFFFFu));
      const uint32_t o = at_off64(8 * sdc + i, sr >> 3) + (sr & 7) * 2;
      *reinterpret_cast<uint16_t*>(&sQt[buf][0] + o) = xq;
      *reinterpret_cast<uint16_t*>(&sDt[buf][0] + o) = xd;
    }
    if (sdc == 0) {
      sL[buf][sr] = rl;
      sDr[buf][sr] = rdr;
      sPos[buf][sr] = rpos;
    }
  };

  // A operands: natural rows pi(c), d chunk 2s + g; transposed rows 32db + c, row chunk s' * 2 + g
  uint32_t aoff[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) aoff[s] = at_off(at_pi(c), 2 * s + g);
  uint32_t toff[2][2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int s = 0; s < 2; ++s) toff[db][s] = at_off64(32 * db + c, 2 * s + g);

  f32x16_t dk[2], dv[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) dk[db][v] = dv[db][v] = 0.f;

  if (nsteps > 0) load_rows(0);
  for (int st = 0; st < nsteps; ++st) {
    const int buf = st & 1;
    store_rows(buf);
    __syncthreads();
    if (st + 1 < nsteps) load_rows(st + 1);
    f32x16_t sc, dp;
#pragma unroll
    for (int v = 0; v < 16; ++v) sc[v] = dp[v] = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      sc = at_mfma(*reinterpret_cast<const u32x4_t*>(&sQ[buf][0] + aoff[s]), kf[s], sc);
      dp = at_mfma(*reinterpret_cast<const u32x4_t*>(&sD[buf][0] + aoff[s]), vf[s], dp);
    }
    // register v: row 8g + v (v < 8) or 16 + 8g + v - 8 of the step, key c
    u32x4_t pf[2], sf[2];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      float p[8], ds[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int v = 8 * half + i;
        const int r = 16 * half + 8 * g + i;
        float x = __builtin_amdgcn_exp2f(sc[v] * a.scale2 - sL[buf][r]);
        const int qp = sPos[buf][r];
        x = (jk < a.Tk && (!a.causal || jk <= qp) && (a.window <= 0 || jk > qp - a.window)) ? x : 0.f;
        p[i] = x;
        ds[i] = x * (dp[v] - sDr[buf][r]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pf[half][i] = pack_bf16x2(p[2 * i], p[2 * i + 1]);
        sf[half][i] = pack_bf16x2(ds[2 * i], ds[2 * i + 1]);
      }
    }
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        dv[db] = at_mfma(*reinterpret_cast<const u32x4_t*>(&sDt[buf][0] + toff[db][s]), pf[s], dv[db]);
        dk[db] = at_mfma(*reinterpret_cast<const u32x4_t*>(&sQt[buf][0] + toff[db][s]), sf[s], dk[db]);
      }
    // the next step's staging writes the other buffer; this one is rewritten
    // two steps on, after the next barrier
  }

  if (jk >= a.Tk) return;
  uint16_t* okr = a.dk + (((int64_t)b * a.Tk + jk) * a.Hkv + hk) * AT_D;
  uint16_t* ovr = a.dv + (((int64_t)b * a.Tk + jk) * a.Hkv + hk) * AT_D;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = 32 * db + 8 * q4 + 4 * g;
      uint2 wk, wv;
      wk.x = pack_bf16x2(dk[db][4 * q4] * a.scaling, dk[db][4 * q4 + 1] * a.scaling);
      wk.y = pack_bf16x2(dk[db][4 * q4 + 2] * a.scaling, dk[db][4 * q4 + 3] * a.scaling);
      wv.x = pack_bf16x2(dv[db][4 * q4], dv[db][4 * q4 + 1]);
      wv.y = pack_bf16x2(dv[db][4 * q4 + 2], dv[db][4 * q4 + 3]);
      *reinterpret_cast<uint2*>(okr + d) = wk;
      *reinterpret_cast<uint2*>(ovr + d) = wv;
    }
}

}  // namespace bsa

extern "C" int bsa_attention_bwd(const void* grad_out, const int64_t* grad_strides, const void* q,
                                 const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
                                 const int64_t* v_strides, const void* out, const int64_t* out_strides,
                                 const float* lse, int64_t B, int64_t Tq, int64_t Tk, int64_t Hq, int64_t Hkv,
                                 int64_t head_dim, int causal, int64_t window, float scaling, void* grad_q,
                                 void* grad_k, void* grad_v, float* row_dot, void* stream) {
  clear_error();
  BSA_REQUIRE(B >= 0 && Tq >= 0 && Tk >= 0 && Hq > 0 && Hkv > 0, "attention bwd: bad shape");
  if (B == 0 || Tq == 0 || Tk == 0) return BSA_OK;
  BSA_REQUIRE(head_dim == AT_D, "attention bwd: head_dim must be %d (got %lld)", AT_D, (long long)head_dim);
  BSA_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= 64, "attention bwd: Hq must be a multiple of Hkv, at most 64x");
  BSA_REQUIRE(grad_out && q && k && v && out && lse && grad_q && grad_k && grad_v && row_dot && grad_strides &&
                  q_strides && k_strides && v_strides && out_strides,
              "attention bwd: null pointer");
  BSA_REQUIRE(window >= 0 && (window == 0 || causal), "attention bwd: a window needs the causal mask");
  BSA_REQUIRE(!causal || Tq <= Tk, "attention bwd: causal with more queries than keys");
  BSA_REQUIRE(B < 65536 && Hkv < 65536 && Tq * (Hq / Hkv) < INT32_MAX / 2 && Tk < INT32_MAX / 2 &&
                  window < INT32_MAX,
              "attention bwd: too large");
  auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  BSA_REQUIRE(al16(grad_out) && al16(q) && al16(k) && al16(v) && al16(out) && al16(grad_q) && al16(grad_k) &&
                  al16(grad_v),
              "attention bwd: tensors must be 16-byte aligned");
  const int64_t* st[5] = {grad_strides, q_strides, k_strides, v_strides, out_strides};
  for (int n = 0; n < 5; ++n)
    for (int i = 0; i < 3; ++i)
      BSA_REQUIRE(st[n][i] % 8 == 0 && st[n][i] >= 0,
                  "attention bwd: strides (batch, sequence, head) must be non-negative multiples of 8 elements");
  AttnBwdArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o = static_cast<const uint16_t*>(out);
  a.dout = static_cast<const uint16_t*>(grad_out);
  a.lse = lse;
  a.drow = row_dot;
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
  hipLaunchKernelGGL(attn_bwd_dq_kernel, dim3((unsigned)rblocks, (unsigned)Hkv, (unsigned)B), dim3(256), 0, s, a);
  BSA_LAUNCH_CHECK("attention bwd (dq) launch");
  const int64_t kblocks = (Tk + AT_KB - 1) / AT_KB;
  hipLaunchKernelGGL(attn_bwd_dkv_kernel, dim3((unsigned)kblocks, (unsigned)Hkv, (unsigned)B), dim3(256), 0, s, a);
  BSA_LAUNCH_CHECK("attention bwd (dk, dv) launch");
  return BSA_OK;
}
