// The 64x64 unit-lower-triangular inverse of the chunked gated delta rule, in registers on the
// fp32 MFMA, and the wave-wide prefix sum of the in-chunk decay: shared by the chunked prefill's
// inverse kernel, the generic fp32 chunked prefill and gdn_unit_lower_inv.
#pragma once
#include "gdn_device.h"

namespace gdn {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Inclusive prefix sum over the 64 lanes (DPP: shifts within rows of 16, then the row totals
// broadcast into the later rows).
template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_or_zero(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, kRowMask, 0xf, false));
}
__device__ __forceinline__ float wave_incl_scan(float x) {
  x += dpp_or_zero<0x111, 0xf>(x);  // row_shr:1
  x += dpp_or_zero<0x112, 0xf>(x);  // row_shr:2
  x += dpp_or_zero<0x114, 0xf>(x);  // row_shr:4
  x += dpp_or_zero<0x118, 0xf>(x);  // row_shr:8
  x += dpp_or_zero<0x142, 0xa>(x);  // row_bcast:15 into rows 1 and 3
  x += dpp_or_zero<0x143, 0xc>(x);  // row_bcast:31 into rows 2 and 3
  return x;
}

// A 16x16 fp32 block in "D layout" is the MFMA accumulator layout: lane (c, g) = (l % 16, l / 16)
// holds M[4g + r][c], r < 4.  v_mfma_f32_16x16x4_f32 takes, per lane, A[l % 16][slot l / 16] and
// B[slot l / 16][l % 16]; with slot g of instruction kk standing for k = 4g + kk, the A operand of
// A B is the D layout of A^T and the B operand the D layout of B.  So
//   rmm(Dl(A^T), Dl(B), Dl(C)) = Dl(A B + C)   and   Dl((A B)^T) = rmm(Dl(B), Dl(A^T), 0):
// a product and its transpose come from the same two registers.
__device__ __forceinline__ f32x4 rmm(f32x4 aT, f32x4 b, f32x4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(aT[0], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(aT[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(aT[2], b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(aT[3], b[3], acc, 0, 0, 0);
  return acc;
}
// Index of the lower block (a, b), b <= a, of a 4x4 block grid.
__device__ __forceinline__ constexpr int tri(int a, int b) { return a * (a + 1) / 2 + b; }

// Dl(M^T) from Dl(M) through a wave-private 16 x 20 fp32 LDS tile: the wave writes M row-major and
// reads its transpose back 16 bytes per lane.  A wave's LDS accesses complete in issue order, and
// the compiler keeps a tile's store -> load -> next store order (they may alias), so no barrier is
// needed.
constexpr int kTrPitch = 20;
__device__ __forceinline__ f32x4 ltr(float* tile, f32x4 m, int lane) {
  const int c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int r = 0; r < 4; ++r) tile[(4 * g + r) * kTrPitch + c] = m[r];
  return *reinterpret_cast<const f32x4*>(&tile[c * kTrPitch + 4 * g]);
}

// Lane l's value v from lane n of its row of 16 lanes (DPP row_newbcast).
template <int N>
__device__ __forceinline__ float row_bcast(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x150 + N, 0xf, 0xf, true));
}
// t[i] += sum_{m < i} row_bcast<m>(x[i]) t[m] for i = 1 .. 15, in order of m.
template <int I, int M>
__device__ __forceinline__ void fwd_sub(const float (&x)[16], float (&t)[16]) {
  if constexpr (I < 16) {
    if constexpr (M < I) {
      t[I] = __builtin_fmaf(row_bcast<M>(x[I]), t[M], t[I]);
      fwd_sub<I, M + 1>(x, t);
    } else {
      fwd_sub<I + 1, 0>(x, t);
    }
  }
}

// (I - X)^{-1} for a strictly lower 64x64 X, one wave.  In: XT[tri(a, b)] = Dl(X_ab^T) for every
// lower block, Xd[a] = Dl(X_aa).  Out: TT[tri(a, b)] = Dl(T_ab^T).  tiles: 4 wave-private 16 x 20
// fp32 LDS tiles.  Same blocking as src/gdn_chunk_fast.py:33-62: the diagonal blocks first, then the
// blocks below them, T_ij = T_ii sum_{k=j}^{i-1} X_ik T_kj.  The four diagonal blocks are solved at
// once by forward substitution on the VALU: lane (a, j) = (l / 16, l % 16) holds column j of X_aa
// and forms column j of T_aa, t_i = [i = j] + sum_{m < i} X_aa[i][m] t_m, with X_aa[i][m] taken
// from lane m of its row (120 FMAs, in place of 24 products of 16x16 blocks on the fp32 MFMA).
// Columns go in and out through the tiles (stored transposed: tile a row j = column j of the block).
__device__ __forceinline__ void reg_inv64(const f32x4 (&XT)[10], const f32x4 (&Xd)[4], f32x4 (&TT)[10], float* tiles,
                                          int lane) {
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  const int c = lane & 15, g = lane >> 4;
  f32x4 TD[6];  // Dl(T_ab) for the blocks of rows 0..2 (tri index < 6)
  {
#pragma unroll
    for (int a = 0; a < 4; ++a)  // lane (c, g) holds X_aa[4g + r][c]: tile a, row c, columns 4g ..
      *reinterpret_cast<f32x4*>(&tiles[(16 * a + c) * kTrPitch + 4 * g]) = Xd[a];
    float x[16], t[16];
    float* col = &tiles[(16 * g + c) * kTrPitch];  // this lane's column: block g, column c
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(&col[4 * m]);
#pragma unroll
      for (int r = 0; r < 4; ++r) x[4 * m + r] = v[r];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] = i == c ? 1.f : 0.f;
    fwd_sub<1, 0>(x, t);
#pragma unroll
    for (int m = 0; m < 4; ++m) *reinterpret_cast<f32x4*>(&col[4 * m]) = f32x4{t[4 * m], t[4 * m + 1], t[4 * m + 2], t[4 * m + 3]};
#pragma unroll
    for (int a = 0; a < 4; ++a) {  // Dl(T_aa): T_aa[4g + r][c] = tile a [c][4g + r]; Dl(T_aa^T): tile a [4g + r][c]
      const float* tile = &tiles[16 * a * kTrPitch];
      f32x4 tt;
#pragma unroll
      for (int r = 0; r < 4; ++r) tt[r] = tile[(4 * g + r) * kTrPitch + c];
      TT[tri(a, a)] = tt;
      if (a < 3) TD[tri(a, a)] = *reinterpret_cast<const f32x4*>(&tile[c * kTrPitch + 4 * g]);
    }
  }
  f32x4 Y;
  // first subdiagonal
  Y = rmm(XT[tri(1, 0)], TD[tri(0, 0)], z);
  TD[tri(1, 0)] = rmm(TT[tri(1, 1)], Y, z);
  TT[tri(1, 0)] = ltr(tiles, TD[tri(1, 0)], lane);
  Y = rmm(XT[tri(2, 1)], TD[tri(1, 1)], z);
  TD[tri(2, 1)] = rmm(TT[tri(2, 2)], Y, z);
  TT[tri(2, 1)] = ltr(tiles + 16 * kTrPitch, TD[tri(2, 1)], lane);
  Y = rmm(XT[tri(3, 2)], TD[tri(2, 2)], z);
  TT[tri(3, 2)] = rmm(Y, TT[tri(3, 3)], z);
  // second
  Y = rmm(XT[tri(2, 0)], TD[tri(0, 0)], z);
  Y = rmm(XT[tri(2, 1)], TD[tri(1, 0)], Y);
  TD[tri(2, 0)] = rmm(TT[tri(2, 2)], Y, z);
  TT[tri(2, 0)] = ltr(tiles + 2 * 16 * kTrPitch, TD[tri(2, 0)], lane);
  Y = rmm(XT[tri(3, 1)], TD[tri(1, 1)], z);
  Y = rmm(XT[tri(3, 2)], TD[tri(2, 1)], Y);
  TT[tri(3, 1)] = rmm(Y, TT[tri(3, 3)], z);
  // third
  Y = rmm(XT[tri(3, 0)], TD[tri(0, 0)], z);
  Y = rmm(XT[tri(3, 1)], TD[tri(1, 0)], Y);
  Y = rmm(XT[tri(3, 2)], TD[tri(2, 0)], Y);
  TT[tri(3, 0)] = rmm(Y, TT[tri(3, 3)], z);
}

}  // namespace gdn
