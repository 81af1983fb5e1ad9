// 128-key tile helpers shared by the attention and pooling kernels.
//
// A staged K tile is 128 rows x D columns of 16-bit values in LDS, stored as 16-byte
// chunks with an XOR swizzle of the chunk index.  S^T = K Q^T for 32 queries is four
// 32x32 MFMA output tiles; in each, A-operand row r of the MFMA reads K row
// k_row_perm(r), so register j of lane i of sub-tile t holds the score of query
// (i % 32) against key t*32 + tile_key(i, j).
#pragma once

#include "common.h"

namespace sa {

__device__ __forceinline__ int k_row_perm(int r) {
  return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}
__device__ __forceinline__ int k_swz(int row) { return (row & 3) | ((row >> 1) & 4); }
// The K swizzle for rows of KC 16-byte chunks (head dim 8 KC): the same pattern, kept inside
// the row when it has fewer than 8 chunks (head dim 32).
template <int KC>
__device__ __forceinline__ int k_swz_kc(int row) { return k_swz(row) & (KC - 1); }
__device__ __forceinline__ int v_swz(int row) { return (row ^ (row >> 3)) & 7; }

// Key offset (within a 32-key sub-tile) of accumulator register j of a lane in half hl.
__device__ __forceinline__ int tile_key(int hl, int j) {
  return k_row_perm(8 * (j >> 2) + 4 * hl + (j & 3));
}

// Stage K rows [key0, key0+128) into lds_k (NT threads cooperate, thread index tid).
// Rows at or beyond Nk are zero-filled.
template <int IT, int CT, int D, int NT>
__device__ __forceinline__ void stage_k_tile(u32x4* lds_k, const char* kbase, int64_t ks2,
                                             int key0, int Nk, int tid) {
  constexpr int ES = ElemSize<IT>::value;
  constexpr int KC = D / 8;
  constexpr int ITER = 128 * KC / NT;
#pragma unroll
  for (int c8 = 0; c8 < ITER; ++c8) {
    const int id = c8 * NT + tid;
    const int row = id / KC, ch = id % KC;
    const int key = key0 + row;
    u32x4 val = u32x4{0, 0, 0, 0};
    if (key < Nk) val = load8<IT, CT>(kbase + ((int64_t)key * ks2 + ch * 8) * ES);
    lds_k[row * KC + (ch ^ k_swz_kc<KC>(row))] = val;
  }
}

// S^T for the 32 queries whose Q^T B-operands are qf[], against the staged K tile.
template <int CT, int D>
__device__ __forceinline__ void qk_tile(const u32x4* lds_k, const u32x4* qf, int prow, int fk,
                                        int hl, f32x16* s) {
  constexpr int KC = D / 8;
  constexpr int DS = D / 16;
#pragma unroll
  for (int t = 0; t < 4; ++t) s[t] = f32x16{};
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int R = t * 32 + prow;
      const u32x4 av = lds_k[R * KC + ((2 * ds + hl) ^ fk)];
      s[t] = mfma32x32x16<CT>(av, qf[ds], s[t]);
    }
  }
}

// Load the Q^T B-operands of query row qrow (zeros when qrow >= Nq).
template <int IT, int CT, int D>
__device__ __forceinline__ void load_q_operand(u32x4* qf, const char* qbase, int64_t qs2, int qrow,
                                               int Nq, int hl) {
  constexpr int ES = ElemSize<IT>::value;
#pragma unroll
  for (int s = 0; s < D / 16; ++s) {
    if (qrow < Nq)
      qf[s] = load8<IT, CT>(qbase + ((int64_t)qrow * qs2 + s * 16 + hl * 8) * ES);
    else
      qf[s] = u32x4{0, 0, 0, 0};
  }
}

}  // namespace sa
