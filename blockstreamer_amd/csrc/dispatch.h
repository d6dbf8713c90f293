// Token -> expert dispatch as device functions, shared by the dispatch
// kernels (route.hip) and the decode GEMM that folds the dispatch into its
// prologue (moe_gemm.hip).  The order they build is described in route.hip:
// rows of one expert by pair index, indices outside [0, E) dropped.
#pragma once

#include "bsa_common.h"

namespace bsa {

// Exclusive scans over experts (one entry per thread, E <= THREADS)
// of the row counts and of the row-tile counts: a shuffle scan within each
// wave, then the wave totals.  Returns expert tid's first sorted row; with
// `write`, also stores counts, offsets, the tile list and the tile count.
template <int THREADS>
__device__ __forceinline__ int dispatch_scan(int my_cnt, int E, int BM, int* s_scan, bool write,
                                             int* __restrict__ counts, int* __restrict__ offsets,
                                             int2* __restrict__ tiles, int* __restrict__ num_tiles) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int my_tiles = (my_cnt + BM - 1) / BM;
  int incl_rows = my_cnt, incl_tiles = my_tiles;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int a = __shfl_up(incl_rows, off);
    const int b = __shfl_up(incl_tiles, off);
    if (lane >= off) {
      incl_rows += a;
      incl_tiles += b;
    }
  }
  if (lane == 63) {
    s_scan[wave] = incl_rows;
    s_scan[(THREADS / 64) + wave] = incl_tiles;
  }
  __syncthreads();
  for (int w = 0; w < wave; ++w) {
    incl_rows += s_scan[w];
    incl_tiles += s_scan[(THREADS / 64) + w];
  }
  const int start = incl_rows - my_cnt;
  if (write && tid < E) {
    counts[tid] = my_cnt;
    offsets[tid] = start;
    if (tid == E - 1) {
      offsets[E] = incl_rows;
      *num_tiles = incl_tiles;
    }
    for (int j = 0; j < my_tiles; ++j) tiles[incl_tiles - my_tiles + j] = make_int2(tid, start + j * BM);
  }
  return start;
}

// Stable placement of pairs [begin, end): pair i with expert e goes to row
// s_base[e] + (pairs of expert e before i in the range).  THREADS
// pairs per round: ranks within a wave from ballots, across waves from the
// per-wave counts, across rounds from s_run.
template <int THREADS, int MAX_E>
__device__ __forceinline__ void dispatch_place(const int64_t* __restrict__ idx, int begin, int end, int E,
                                               const int* s_base, int* s_run,
                                               uint8_t (*s_wc)[MAX_E], int* __restrict__ row_pair,
                                               int* __restrict__ pair_pos) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int base = begin; base < end; base += THREADS) {
    const int i = base + tid;
    int e = -1;
    if (i < end) {
      const int64_t v = idx[i];
      e = (v >= 0 && v < E) ? (int)v : -1;
    }
    // lanes of this wave holding the same expert id (ids < 1024: 10 bits + valid bit)
    uint64_t same = __ballot(e >= 0);
    if (e < 0) same = ~same;
#pragma unroll
    for (int b = 0; b < 10; ++b) {
      const uint64_t m = __ballot((e >> b) & 1);
      same &= ((e >> b) & 1) ? m : ~m;
    }
    const int local_rank = __popcll(same & lt_mask);
    const int wave_cnt = __popcll(same);
    for (int j = tid; j < (THREADS / 64) * E; j += THREADS)
      s_wc[j / E][j % E] = 0;
    __syncthreads();
    if (e >= 0 && local_rank == 0) s_wc[wave][e] = (uint8_t)wave_cnt;
    __syncthreads();
    if (i < end) {
      if (e >= 0) {
        int prefix = 0;
        for (int w = 0; w < wave; ++w) prefix += s_wc[w][e];
        const int pos = s_base[e] + s_run[e] + prefix + local_rank;
        row_pair[pos] = i;
        pair_pos[i] = pos;
      } else {
        pair_pos[i] = -1;
      }
    }
    __syncthreads();
    for (int ee = tid; ee < E; ee += THREADS) {
      int add = 0;
      for (int w = 0; w < (THREADS / 64); ++w) add += s_wc[w][ee];
      s_run[ee] += add;
    }
    __syncthreads();
  }
}

// The whole dispatch by one workgroup of THREADS threads (E <= THREADS,
// E <= MAX_E), with its LDS scratch passed in: s_cnt, s_off, s_run [MAX_E],
// s_scan [2 * THREADS / 64], s_wc [THREADS / 64][MAX_E].  Writes counts,
// offsets, row_pair, pair_pos, the tile list (tiles of BM rows) and its count.
template <int THREADS, int MAX_E>
__device__ __forceinline__ void dispatch_block(const int64_t* __restrict__ idx, int P, int E, int BM,
                                               int* __restrict__ counts, int* __restrict__ offsets,
                                               int* __restrict__ row_pair, int* __restrict__ pair_pos,
                                               int2* __restrict__ tiles, int* __restrict__ num_tiles, int* s_cnt,
                                               int* s_off, int* s_run, int* s_scan, uint8_t (*s_wc)[MAX_E]) {
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += THREADS) {
    s_cnt[e] = 0;
    s_run[e] = 0;
  }
  __syncthreads();
  for (int i = tid; i < P; i += THREADS) {
    const int64_t e = idx[i];
    if (e >= 0 && e < E) atomicAdd(&s_cnt[(int)e], 1);
  }
  __syncthreads();
  const int start = dispatch_scan<THREADS>(tid < E ? s_cnt[tid] : 0, E, BM, s_scan, true, counts, offsets, tiles,
                                           num_tiles);
  if (tid < E) s_off[tid] = start;
  __syncthreads();
  dispatch_place<THREADS, MAX_E>(idx, 0, P, E, s_off, s_run, s_wc, row_pair, pair_pos);
}

}  // namespace bsa
