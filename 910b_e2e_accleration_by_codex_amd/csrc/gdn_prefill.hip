// Prefill-side GDN kernels for gfx950: the chunked gated delta rule on bf16 MFMA, its 64x64
// unit-lower-triangular inverse, the depthwise causal conv prefill with state capture, and the
// gating.
//
// Chunked rule (chunk C = 64, head dim D = 128), per chunk with cumulative log decay G:
//   X   = -(beta_i k_i.k_j e^{G_i - G_j})_{i>j},   T = (I - X)^{-1}
//   W   = T diag(beta e^G) K,   U = T diag(beta) V,   QK = (scale q_i.k_j e^{G_i - G_j})_{i>=j}
//   vn  = U - W S,   o = diag(scale e^G) Q S + QK vn,   S' = e^{G_last} S + K^T diag(e^{G_last - G}) vn
// which is src/gdn_chunk_fast2.py:31-59 (and HF torch_chunk_gated_delta_rule) written per chunk.
//
// Two kernels: chunk_local_kernel does every state-independent part of a chunk in parallel over all
// (chunk, value head) pairs and writes ready-made MFMA operand fragments to a workspace;
// chunk_scan_kernel walks the chunks of each sequence in order with the fp32 state held in MFMA
// accumulators (one workgroup per 16-column slice of a head's state).  Products run on
// v_mfma_f32_16x16x32_bf16 / _f16 with fp32 accumulation; the 64x64 inverse is fp32 throughout
// (v_mfma_f32_16x16x4_f32).  The state update uses fp16 operands (DEC vn and K^T) with power-of-two
// range scaling, so the running state never sees a bf16 rounding of its increment.
#include "gdn_device.h"
#include "gdn_internal.h"

namespace gdn {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

namespace pf {
constexpr int D = 128;          // head dim
constexpr int CH = 64;          // chunk length
constexpr int NT = 256;         // threads per workgroup (4 waves)
constexpr int LDK = D + 8;      // row pitch (bf16) of [*, 128] tiles
constexpr int LDF = CH + 4;     // row pitch (fp32) of [64, 64] matrices
constexpr float kScale = 0.08838834764831845f;  // (float)(1 / sqrt(128))
}  // namespace pf

// ---- MFMA fragment helpers (layouts verified on gfx950) -----------------------------------
// v_mfma_f32_16x16x32_bf16: lane l supplies A[l%16][8(l/16)..+7] and B[8(l/16)..+7][l%16] and
// receives D[4(l/16)+r][l%16], r < 4.  For both operands the 8 values are contiguous along K when
// the operand is stored with K innermost, so one 16-byte LDS read fetches a fragment.
__device__ __forceinline__ bf16x8 frag(const uint16_t* base, int ld, int row0, int k0, int lane) {
  const uint16_t* p = base + (row0 + (lane & 15)) * ld + k0 + 8 * (lane >> 4);
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(p));
}
__device__ __forceinline__ bf16x8 frag_neg(const uint16_t* base, int ld, int row0, int k0, int lane) {
  const uint16_t* p = base + (row0 + (lane & 15)) * ld + k0 + 8 * (lane >> 4);
  u16x8 v = *reinterpret_cast<const u16x8*>(p);
  v ^= (uint16_t)0x8000;
  return __builtin_bit_cast(bf16x8, v);
}
__device__ __forceinline__ f32x4 mma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 pack8(const float* v) {
  u16x8 u;
#pragma unroll
  for (int e = 0; e < 8; ++e) u[e] = f2bf(v[e]);
  return __builtin_bit_cast(bf16x8, u);
}

// fp32 16x16x16 product on v_mfma_f32_16x16x4_f32 (lane: A[l%16][kk*4 + l/16], B[kk*4 + l/16][l%16]).
// Adds A[ra.., ca..] * B[rb.., cb..] into acc.
__device__ __forceinline__ f32x4 mm16_f32(const float* A, int lda, const float* B, int ldb, f32x4 acc,
                                          int lane) {
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const float a = A[(lane & 15) * lda + 4 * kk + (lane >> 4)];
    const float b = B[(4 * kk + (lane >> 4)) * ldb + (lane & 15)];
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
  }
  return acc;
}
// Store a 16x16 fp32 accumulator (D layout) at M[0..15][0..15] (pitch ld).
__device__ __forceinline__ void st16_f32(float* M, int ld, f32x4 acc, int lane) {
#pragma unroll
  for (int r = 0; r < 4; ++r) M[(4 * (lane >> 4) + r) * ld + (lane & 15)] = acc[r];
}

// ---- (I - X)^{-1} for a strictly lower 64x64 fp32 X (only its strictly lower part is read) ----
// Same blocking as src/gdn_chunk_fast.py:33-62 -- the four 16x16 diagonal blocks first, then the
// merges [[A,0],[B X21 A, B]] for 32x32 and 64x64 -- all on fp32 MFMA.  A diagonal block is
// inverted as (I+X)(I+X^2)(I+X^4)(I+X^8) (exact for nilpotent X, X^16 = 0) instead of the
// reference's 16-step row recurrence: six dependent products instead of sixteen dependent steps;
// with |X_ij| <= 1 (l2-normalised k, beta <= 1, decay <= 1) the powers of a 16x16 block stay far
// from fp32 overflow (the reference avoids powers of the whole 64x64 block, which can overflow).
// All 4 waves must call it (it holds barriers).  Its four 16x16 scratch blocks live in the upper
// blocks (0,1) (0,2) (0,3) (1,2) of sX, which the inverse never reads.  Writes all of sT (upper
// blocks zero).
__device__ __forceinline__ float* inv_scratch(float* sX, int k) {
  return sX + (k == 3 ? 16 * pf::LDF + 32 : 16 * (k + 1));
}
__device__ void unit_lower_inv64(float* sX, float* sT, int w, int lane) {
  using namespace pf;
  {  // diagonal block w: T = (I+X)(I+X^2)(I+X^4)(I+X^8) (X^16 = 0), six fp32 MFMA products
    const int c = lane & 15, g = lane >> 4;
    const float* Xb = sX + 16 * w * LDF + 16 * w;
    float* Tb = sT + 16 * w * LDF + 16 * w;
    float* P = inv_scratch(sX, w);  // wave-private 16x16 scratch
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 4 * g + r;
      Tb[i * LDF + c] = Xb[i * LDF + c] + (i == c ? 1.0f : 0.0f);
    }
    const float* Pin = Xb;
    const int ldp = LDF;
#pragma unroll
    for (int step = 0; step < 3; ++step) {
      f32x4 p2 = mm16_f32(Pin, ldp, Pin, ldp, f32x4{0.f, 0.f, 0.f, 0.f}, lane);  // X^(2^(step+1))
      st16_f32(P, LDF, p2, lane);
      __builtin_amdgcn_wave_barrier();
      f32x4 tp = mm16_f32(Tb, LDF, P, LDF, f32x4{0.f, 0.f, 0.f, 0.f}, lane);    // T X^(2^(step+1))
#pragma unroll
      for (int r = 0; r < 4; ++r) Tb[(4 * g + r) * LDF + c] += tp[r];
      __builtin_amdgcn_wave_barrier();
      Pin = P;
    }
    float* Trow = sT + 16 * w * LDF;
    for (int col = 16 * (w + 1) + c; col < CH; col += 16)
#pragma unroll
      for (int r = 0; r < 4; ++r) Trow[(4 * g + r) * LDF + col] = 0.f;
  }
  __syncthreads();
  // level 1: T10 = T11 (X10 T00), T32 = T33 (X32 T22)
  float* Y = inv_scratch(sX, w);
  if (w < 2) {
    const int b0 = 32 * w;  // block row/col offsets: rows b0+16.., cols b0..
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    acc = mm16_f32(sX + (b0 + 16) * LDF + b0, LDF, sT + b0 * LDF + b0, LDF, acc, lane);
    st16_f32(Y, LDF, acc, lane);
  }
  __syncthreads();
  if (w < 2) {
    const int b0 = 32 * w;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    acc = mm16_f32(sT + (b0 + 16) * LDF + b0 + 16, LDF, Y, LDF, acc, lane);
    st16_f32(sT + (b0 + 16) * LDF + b0, LDF, acc, lane);
  }
  __syncthreads();
  // level 2: Y20 = X20 T00 + X21 T10, Y30 = X30 T00 + X31 T10, Y21 = X21 T11, Y31 = X31 T11
  {
    const int ib = 2 + (w & 1), jb = w >> 1;  // wave 0: Y20, 1: Y30, 2: Y21, 3: Y31
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (jb == 0) acc = mm16_f32(sX + 16 * ib * LDF + 0, LDF, sT + 0 * LDF + 0, LDF, acc, lane);
    acc = mm16_f32(sX + 16 * ib * LDF + 16, LDF, sT + 16 * LDF + 16 * jb, LDF, acc, lane);
    st16_f32(Y, LDF, acc, lane);
  }
  __syncthreads();
  {  // T20 = T22 Y20, T30 = T32 Y20 + T33 Y30, T21 = T22 Y21, T31 = T32 Y21 + T33 Y31
    const int ib = 2 + (w & 1), jb = w >> 1;
    const float* Ya = inv_scratch(sX, 2 * jb);      // Y2jb
    const float* Yb = inv_scratch(sX, 2 * jb + 1);  // Y3jb
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    acc = mm16_f32(sT + 16 * ib * LDF + 32, LDF, Ya, LDF, acc, lane);
    if (ib == 3) acc = mm16_f32(sT + 48 * LDF + 48, LDF, Yb, LDF, acc, lane);
    st16_f32(sT + 16 * ib * LDF + 16 * jb, LDF, acc, lane);
  }
  __syncthreads();
}

__global__ __launch_bounds__(pf::NT) void unit_lower_inv_kernel(const float* __restrict__ X, float* __restrict__ T) {
  using namespace pf;
  __shared__ float sX[CH * LDF], sT[CH * LDF];
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const float* Xm = X + (int64_t)blockIdx.x * CH * CH;
  for (int i = t; i < CH * CH; i += NT) sX[(i / CH) * LDF + (i % CH)] = (i / CH) > (i % CH) ? Xm[i] : 0.f;
  __syncthreads();
  unit_lower_inv64(sX, sT, w, lane);
  float* Tm = T + (int64_t)blockIdx.x * CH * CH;
  for (int i = t; i < CH * CH; i += NT) Tm[i] = sT[(i / CH) * LDF + (i % CH)];
}

// ============================================================================================
// Chunked prefill, part 1: chunk-local quantities (parallel over every (chunk, value head)).
// ============================================================================================
// Workspace record per (chunk slot, value head).  Everything the scan kernel multiplies is stored
// as ready-made MFMA operand fragments: a fragment is 64 lanes x 16 bytes (lane l at byte 16 l), so
// the scan kernel stages a chunk with plain linear copies and reads each fragment with one
// conflict-free 16-byte LDS read per lane.
//
// k-slot order.  Inside every 32-wide reduction block the scan kernel feeds MFMA B operands straight
// from accumulator registers: lane (c, g) = (l % 16, l / 16) holds rows 4g..4g+3 of two consecutive
// 16-row accumulator tiles, and uses them as the 8 k-values of its B fragment.  So B slot s of a
// block stands for block row kpos(s) = 16 ((s >> 2) & 1) + 4 (s >> 3) + (s & 3), and every A
// fragment stored here is permuted the same way along k:  A-frag element e of lane (c, g) for tile
// (m, j) = M[16 m + c][32 j + kpos(8 g + e)].
//
//   WN  16 frags [tb 4][j 4]  bf16  M = -W,  W = T diag(beta e^G) K     (tokens x features)
//   KT  16 frags [rb 8][j 2]  fp16  M = kappa K^T                       (features x tokens)
//   QG  16 frags [tb 4][j 4]  bf16  M = q (l2-normalised)               (tokens x features)
//   QK   8 frags [tb 4][j 2]  bf16  M = scale q_i.k_j e^{G_i - G_j}, i >= j, else 0 (the two
//                                   all-zero fragments (tb, j) = (0, 1), (1, 1) are not written)
// KT and QG depend on the key head only: they are written into the record of the first value
// head of each key head (h % (Hv / Hk) == 0) and read from there.
//   U   fp16 [slice 8][lane 64][tb 4][r 4] = U[16 tb + 4 g + r][16 slice + c] / USC[tb],
//       U = T diag(beta) V (accumulator layout of each 16-column slice)
//   DEC [64] fp32 = e^{G_last - G_t};  USC [4] fp32;  GL = e^{G_last};  KSC = 1 / kappa;  KAP = kappa;
//   EGS [64] fp32 = scale e^{G_t} (the output rows' factor for q S)
// kappa (per chunk, for |K|) and 1 / USC (per token tile, for |U|) are powers of two chosen by
// fp16_fit_exp: 1 when the largest magnitude already sits in [2^-4, 2^14), else the power that
// moves it into [2^14, 2^15) -- inside fp16's range with full relative precision either way.
namespace ws {
constexpr int FRAG = 1024;                       // bytes per fragment
constexpr int WN = 0;                            // byte offsets inside one record
constexpr int KT = WN + 16 * FRAG;               // 16384
constexpr int QG = KT + 16 * FRAG;               // 32768
constexpr int QK = QG + 16 * FRAG;               // 49152
constexpr int U = QK + 8 * FRAG;                 // 57344
constexpr int DEC = U + pf::CH * pf::D * 2;      // 73728
constexpr int USC = DEC + pf::CH * 4;            // 73984 (16-byte aligned: read as one float4)
constexpr int GL = USC + 16;                     // 74000
constexpr int KSC = GL + 4;                      // 74004
constexpr int KAP = KSC + 4;                     // 74008
constexpr int HDR = DEC;                         // DEC, USC, GL, KSC, KAP: the 512 bytes the scan stages
constexpr int EGS = HDR + 512;                   // 74240
constexpr int BYTES = EGS + pf::CH * 4;          // 74496 (multiple of 256)
}  // namespace ws

// Exponent se such that 2^se max|x| lies in [2^14, 2^15) (0 for 0 / non-finite; clamped to +-60).
__device__ __forceinline__ int fp16_scale_exp(float amax) {
  const int e = (int)((__float_as_uint(amax) >> 23) & 0xff) - 127;
  if (!(amax > 0.f) || e == 128) return 0;
  const int se = 14 - e;
  return se < -60 ? -60 : (se > 60 ? 60 : se);
}
// As fp16_scale_exp, but 0 whenever max|x| already lies in [2^-4, 2^14).
__device__ __forceinline__ int fp16_fit_exp(float amax) {
  return (amax >= 0.0625f && amax < 16384.0f) ? 0 : fp16_scale_exp(amax);
}

// Slot row of sequence s for state I/O: rows[s] (or s without rows); -1 if outside [0, n_rows).
__device__ __forceinline__ int state_row(const int32_t* rows, int n_rows, int s) {
  const int r = rows ? rows[s] : s;
  return (r >= 0 && r < n_rows) ? r : -1;
}

struct ChunkPos {
  int64_t t0;  // first packed token of the chunk
  int len;     // valid tokens (1..64)
  int seq, c;  // sequence and chunk index inside it
};

// Position of chunk `slot` (dense index over all chunks of all sequences).
__device__ __forceinline__ ChunkPos chunk_pos(int slot, const int32_t* cu, const int32_t* seq_chunk0, int nseq,
                                              int seq_len) {
  ChunkPos p;
  if (cu) {
    int lo = 0, hi = nseq - 1;  // last sequence whose first chunk slot <= slot
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (seq_chunk0[mid] <= slot) lo = mid;
      else hi = mid - 1;
    }
    p.seq = lo;
    p.c = slot - seq_chunk0[lo];
    p.t0 = (int64_t)cu[lo] + (int64_t)p.c * pf::CH;
    const int64_t left = (int64_t)cu[lo + 1] - p.t0;
    p.len = left < pf::CH ? (int)left : pf::CH;
  } else {
    const int nch = (seq_len + pf::CH - 1) / pf::CH;
    p.seq = slot / nch;
    p.c = slot % nch;
    p.t0 = (int64_t)p.seq * seq_len + (int64_t)p.c * pf::CH;
    const int left = seq_len - p.c * pf::CH;
    p.len = left < pf::CH ? left : pf::CH;
  }
  return p;
}

// Load 4 token rows x 8 features (rows 4*tq.., features f0..f0+7) of a [tokens, heads*D] bf16
// tensor, zero beyond `len`, and l2-normalise each row (a row is spread over 16 consecutive lanes)
// with the rounding of torch bf16 ops.
// Rows past the chunk's end (len >= 1) read its last row and are zeroed afterwards: every load is
// issued unconditionally, so the group goes out back to back with no branch around it.
__device__ __forceinline__ void load_rows4(u16x8* x, const uint16_t* base, int64_t stride, int64_t t0, int len,
                                           int tq, int f0) {
  const u16x8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * tq + i;
    const u16x8 r = *reinterpret_cast<const u16x8*>(base + (t0 + (row < len ? row : len - 1)) * stride + f0);
    x[i] = row < len ? r : zero;
  }
}
// The pieces of torch's bf16 l2norm x * rsqrt(sum(x^2) + eps) (each op rounded to bf16), two
// values at a time: the squares are exact in fp32, rounded to bf16 as a pair (v_cvt_pk_bf16_f32)
// and added with one v_dot2 against (1, 1).
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float sumsq_bf16(u16x8 x, float acc) {
  const u32x4v w = __builtin_bit_cast(u32x4v, x);
  const bf16x2 one = __builtin_bit_cast(bf16x2, 0x3f803f80u);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = __uint_as_float(w[i] << 16), hi = __uint_as_float(w[i] & 0xffff0000u);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, f2bf2(lo * lo, hi * hi)), one, acc, false);
  }
  return acc;
}
__device__ __forceinline__ u16x8 scale_bf16(u16x8 x, float s) {
  const u32x4v w = __builtin_bit_cast(u32x4v, x);
  u32x4v o;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = f2bf2(__uint_as_float(w[i] << 16) * s, __uint_as_float(w[i] & 0xffff0000u) * s);
  return __builtin_bit_cast(u16x8, o);
}
// bf16(rsqrt(bf16(bf16(ss) + 1e-6))): hardware rsqrt and one Newton step (within an ulp of the
// exact fp32 value before the bf16 rounding).
__device__ __forceinline__ float l2norm_inv(float ss) {
  const float x = rbf(rbf(ss) + 1e-6f);
  float y = __builtin_amdgcn_rsqf(x);
  y = y * (1.5f - 0.5f * x * y * y);
  return rbf(y);
}
__device__ __forceinline__ void l2norm_rows4(u16x8* x) {
  float ss[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ss[i] = sumsq_bf16(x[i], 0.f);
#pragma unroll
  for (int i = 0; i < 4; ++i) ss[i] = row16_sum(ss[i]);
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = scale_bf16(x[i], l2norm_inv(ss[i]));
}

// A-fragment of a bf16 [rows, ld] tile in k-slot order (two 8-byte reads; see the workspace notes).
__device__ __forceinline__ bf16x8 frag_kperm(const uint16_t* base, int ld, int row0, int k0, int lane) {
  const uint16_t* p = base + (row0 + (lane & 15)) * ld + k0 + 4 * (lane >> 4);
  const u16x4 lo = *reinterpret_cast<const u16x4*>(p), hi = *reinterpret_cast<const u16x4*>(p + 16);
  const u16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}
// ds_read_b64_tr_b16: within each 16-lane group, lane j supplies the address of 4 consecutive
// 16-bit values L[j][0..3]; lane i receives L[4e + (i >> 2)][i & 3] for e = 0..3.
__device__ __forceinline__ u16x4 lds_tr16(const uint16_t* p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
  return __builtin_bit_cast(u16x4, v);
}
// Fragment with k along the rows of a row-major [k][m] bf16 tile: lane (c, g) = (l % 16, l / 16)
// gets M[k0 + 8g + e][m0 + c], e < 8 -- the A operand of M^T or the B operand of M.
__device__ __forceinline__ u16x8 frag_tr(const uint16_t* base, int ld, int k0, int m0, int lane) {
  const int j = lane & 15, g = lane >> 4;
  const uint16_t* p = base + (k0 + 8 * g + (j >> 2)) * ld + m0 + 4 * (j & 3);
  const u16x4 lo = lds_tr16(p), hi = lds_tr16(p + 4 * ld);
  return u16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
// The same in k-slot order: element e of lane (c, g) is M[k0 + kpos(8g + e)][m0 + c].
__device__ __forceinline__ u16x8 frag_tr_kperm(const uint16_t* base, int ld, int k0, int m0, int lane) {
  const int j = lane & 15, g = lane >> 4;
  const uint16_t* p = base + (k0 + 4 * g + (j >> 2)) * ld + m0 + 4 * (j & 3);
  const u16x4 lo = lds_tr16(p), hi = lds_tr16(p + 16 * ld);
  return u16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
// 8 accumulator values (rows 4g..4g+3 of tiles a and b) -> one k-slot ordered bf16 fragment.
__device__ __forceinline__ bf16x8 pack_acc_bf16(f32x4 a, f32x4 b) {
  const uint32_t w0 = f2bf2(a[0], a[1]), w1 = f2bf2(a[2], a[3]), w2 = f2bf2(b[0], b[1]), w3 = f2bf2(b[2], b[3]);
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 u = {w0, w1, w2, w3};
  return __builtin_bit_cast(bf16x8, u);
}
__device__ __forceinline__ f16x8 pack_acc_f16(f32x4 a, f32x4 b, float sa) {
  f16x8 h;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    h[r] = (_Float16)(a[r] * sa);
    h[4 + r] = (_Float16)(b[r] * sa);
  }
  return h;
}
__device__ __forceinline__ float wave_max(float v) { return wave_max_fast(v); }

struct LocalSmem {
  uint16_t K[pf::CH * pf::LDK];     // K chunk, row-major (token, feature); K^T operands via transpose reads
  float X[pf::CH * pf::LDF];        // then V, row-major (token, feature), once the inverse is done
  float T[pf::CH * pf::LDF];
  float G[pf::CH], EG[pf::CH], B[pf::CH];
  float KMX[4];
};
static_assert(pf::CH * pf::LDK * 2 <= pf::CH * pf::LDF * 4, "V must fit in the X buffer");

// One (chunk, key head) item's inputs shared by the key head's value heads, all loads issued up
// front: K rows 4tq.. x features 8fb.. (thread (tq, fb)) and Q rows 16w + l%16 in k-slot order
// (block s holds features 32s + 4g.. and 32s + 16 + 4g..).
struct KeyLoads {
  u16x8 kx[4], qr[4];
  ChunkPos cp;
  int hk, slot;
};
// One value head's inputs for that chunk: V rows like K, g and beta (wave 0, lane = token).
struct HeadLoads {
  u16x8 vreg[4];
  float graw, braw;
};
__device__ __forceinline__ void key_loads(KeyLoads& L, int64_t item, const uint16_t* __restrict__ q, int64_t qs,
                                          const uint16_t* __restrict__ k, int64_t ks,
                                          const int32_t* __restrict__ cu, const int32_t* __restrict__ seq_chunk0,
                                          int nseq, int seq_len, int Hqk) {
  using namespace pf;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63, c16 = lane & 15, g4 = lane >> 4;
  L.hk = (int)(item % Hqk);
  L.slot = (int)(item / Hqk);
  L.cp = chunk_pos(L.slot, cu, seq_chunk0, nseq, seq_len);
  const ChunkPos& cp = L.cp;
  const int tq = t >> 4, fb = t & 15;
  load_rows4(L.kx, k + (int64_t)L.hk * D, ks, cp.t0, cp.len, tq, 8 * fb);
  const u16x8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  const int row = 16 * w + c16, rowc = row < cp.len ? row : cp.len - 1;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint16_t* p = q + (cp.t0 + rowc) * qs + (int64_t)L.hk * D + 32 * s + 4 * g4;
    const u16x4 lo = *reinterpret_cast<const u16x4*>(p), hi = *reinterpret_cast<const u16x4*>(p + 16);
    const u16x8 x = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    L.qr[s] = row < cp.len ? x : zero;
  }
}
template <typename BetaT>
__device__ __forceinline__ void head_loads(HeadLoads& H, const ChunkPos& cp, int h, const uint16_t* __restrict__ v,
                                           int64_t vs, const float* __restrict__ g, const BetaT* __restrict__ beta,
                                           int Hv) {
  using namespace pf;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  load_rows4(H.vreg, v + (int64_t)h * D, vs, cp.t0, cp.len, t >> 4, 8 * (t & 15));
  // padding tokens: g = 0, beta = 0 (their loads read the chunk's last token)
  const int tok = lane < cp.len ? lane : cp.len - 1;
  const float gr = g[(cp.t0 + tok) * Hv + h];
  const float br = Elem<BetaT>::load(beta + (cp.t0 + tok) * Hv + h);
  H.graw = w == 0 && lane < cp.len ? gr : 0.f;
  H.braw = w == 0 && lane < cp.len ? br : 0.f;
}

// The key head's part of an item: l2norm of K (row-major LDS copy, largest |K| -> kappa) and of Q
// (k-slot ordered fragments qf, kept in registers), and the key-head fragments QG and kappa K^T,
// written into the record of the key head's first value head (rec).  Returns kappa's exponent.
__device__ __forceinline__ int local_key(LocalSmem& sm, const KeyLoads& L, int use_l2, bf16x8 (&qf)[4],
                                         uint8_t* __restrict__ rec) {
  using namespace pf;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int tq = t >> 4, fb = t & 15;
  u16x8 kx[4], qr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kx[i] = L.kx[i];
    qr[i] = L.qr[i];
  }
  // K: l2norm, row-major LDS copy, largest |K|
  {
    if (use_l2) l2norm_rows4(kx);
    // largest |K|: bf16 bit patterns with the sign cleared order like their magnitudes (NaN aside)
    typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
    u16x2 mx = {0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<u16x8*>(&sm.K[(4 * tq + i) * LDK + 8 * fb]) = kx[i];
      const u32x4v wv = __builtin_bit_cast(u32x4v, kx[i]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const u16x2 a = __builtin_bit_cast(u16x2, wv[e] & 0x7fff7fffu);
        mx = __builtin_elementwise_max(mx, a);
      }
    }
    float m = fmaxf(bf2f(mx[0]), bf2f(mx[1]));
    m = wave_max(m);
    if (lane == 0) sm.KMX[w] = m;
  }
  // Q: l2norm in registers (a row is spread over lanes l%16 + 16g' and the 4 blocks)
  {
    if (use_l2) {
      float ss = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s) ss = sumsq_bf16(qr[s], ss);
      ss = xor32_sum(xor16_sum(ss));
      const float inv = l2norm_inv(ss);
#pragma unroll
      for (int s = 0; s < 4; ++s) qr[s] = scale_bf16(qr[s], inv);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = __builtin_bit_cast(bf16x8, qr[s]);
  }
  __syncthreads();
  // QG fragments (this wave's token tile, straight from the k-slot ordered Q fragments) and the
  // kappa-scaled fp16 K^T fragments
#pragma unroll
  for (int s = 0; s < 4; ++s)
    *reinterpret_cast<bf16x8*>(rec + ws::QG + (w * 4 + s) * ws::FRAG + lane * 16) = qf[s];
  const float kmax = fmaxf(fmaxf(sm.KMX[0], sm.KMX[1]), fmaxf(sm.KMX[2], sm.KMX[3]));
  const int ke = fp16_fit_exp(kmax);
  const float kappa = ldexpf(1.0f, ke);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = t + NT * i;  // fragment idx / 64 = (rb, j), lane idx % 64
    const int f_ = idx >> 6, rb = f_ >> 1, j = f_ & 1;  // idx % 64 == lane (idx = t + 256 i)
    const u16x8 kt = frag_tr_kperm(sm.K, LDK, 32 * j, 16 * rb, lane);
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (_Float16)(bf2f(kt[e]) * kappa);
    *reinterpret_cast<f16x8*>(rec + ws::KT + idx * 16) = o;
  }
  return ke;
}

// A = K K^T -> X in LDS, and (Q K^T)^T = K Q^T, whose accumulator layout is exactly the k-slot
// ordered QK fragment layout -> workspace.  Both are lower triangles of 16x16 blocks; wave W takes
// the A blocks of row tile 3 - W and the QK blocks of its own row tile W (whose q it holds), so
// every wave computes 5 blocks.  X carries -beta_i and the decay e^{G_i - G_j}, QK the scale and
// the decay; sm.G and sm.B hold the value head's cumulative decay and beta.
template <int W>
__device__ __forceinline__ void aqk_blocks(LocalSmem& sm, const bf16x8 (&qf)[4], uint8_t* __restrict__ rec,
                                           int lane) {
  using namespace pf;
  constexpr int TA = 3 - W;  // A row tile
  const int c16 = lane & 15, g4 = lane >> 4;
  f32x4 accA[TA + 1], accQ[W + 1];
#pragma unroll
  for (int cb = 0; cb <= TA; ++cb) accA[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int cb = 0; cb <= W; ++cb) accQ[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const bf16x8 ak = frag(sm.K, LDK, 16 * TA, 32 * s, lane);
#pragma unroll
    for (int cb = 0; cb <= TA; ++cb) accA[cb] = mma(ak, frag(sm.K, LDK, 16 * cb, 32 * s, lane), accA[cb]);
#pragma unroll
    for (int cb = 0; cb <= W; ++cb) accQ[cb] = mma(frag_kperm(sm.K, LDK, 16 * cb, 32 * s, lane), qf[s], accQ[cb]);
  }
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // X[i][jj], i = 16 TA + 4g + r, jj = 16cb + c
      const int i = 16 * TA + 4 * g4 + r, jj = 16 * cb + c16;
      float x = 0.f;
      if (cb <= TA && i > jj) x = -sm.B[i] * accA[cb <= TA ? cb : 0][r] * __expf(sm.G[i] - sm.G[jj]);
      sm.X[i * LDF + jj] = x;
    }
  f32x4 qk[4];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // QK[i][jj], i = 16W + c, jj = 16cb + 4g + r
      const int i = 16 * W + c16, jj = 16 * cb + 4 * g4 + r;
      qk[cb][r] = (cb <= W && i >= jj) ? kScale * accQ[cb <= W ? cb : 0][r] * __expf(sm.G[i] - sm.G[jj]) : 0.f;
    }
#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (2 * j <= W)  // fragment (W, j) is non-zero only when its first column block 2j <= W
      *reinterpret_cast<bf16x8*>(rec + ws::QK + (W * 2 + j) * ws::FRAG + lane * 16) =
          pack_acc_bf16(qk[2 * j], qk[2 * j + 1]);
}

// One value head's part: cumulative decay, X = -(beta K K^T o decay) and the QK fragments, the
// inverse, W and U -- everything state-independent about (chunk, value head), into its record.
// sm.K holds the key head's normalised K; the caller has synchronised since the last value head.
__device__ __forceinline__ void local_head(LocalSmem& sm, const HeadLoads& H, const bf16x8 (&qf)[4], int ke,
                                           uint8_t* __restrict__ rec) {
  using namespace pf;
  // the thread index through an opaque move: the caller loops over value heads, and addresses
  // derived from it would otherwise be hoisted out of that loop and held in registers
  int t;
  asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)threadIdx.x));
  const int w = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63, c16 = lane & 15, g4 = lane >> 4;
  const int tq = t >> 4, fb = t & 15;
  u16x8 vreg[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) vreg[i] = H.vreg[i];
  const float graw = H.graw, braw = H.braw;
  if (t == 0) {
    reinterpret_cast<float*>(rec + ws::KSC)[0] = ldexpf(1.0f, -ke);
    reinterpret_cast<float*>(rec + ws::KAP)[0] = ldexpf(1.0f, ke);
  }
  if (w == 0) {  // cumulative decay within the chunk
    float G = graw;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float up = __shfl_up(G, o, kWave);
      if (lane >= o) G += up;
    }
    const float gl = __shfl(G, 63, kWave);
    const float eg = expf(G), dec = expf(gl - G);
    sm.G[lane] = G;
    sm.EG[lane] = eg;
    sm.B[lane] = braw;
    reinterpret_cast<float*>(rec + ws::DEC)[lane] = dec;
    reinterpret_cast<float*>(rec + ws::EGS)[lane] = kScale * eg;
    if (lane == 0) reinterpret_cast<float*>(rec + ws::GL)[0] = expf(gl);
  }
  __syncthreads();

  // A = K K^T -> X in LDS and the QK fragments -> workspace (aqk_blocks), with the wave index as a
  // compile-time constant so every block bound is static
  switch (w) {
    case 0: aqk_blocks<0>(sm, qf, rec, lane); break;
    case 1: aqk_blocks<1>(sm, qf, rec, lane); break;
    case 2: aqk_blocks<2>(sm, qf, rec, lane); break;
    default: aqk_blocks<3>(sm, qf, rec, lane); break;
  }
  __syncthreads();

  unit_lower_inv64(sm.X, sm.T, w, lane);

  // W^T = K^T (T diag(beta e^G))^T: its accumulator layout is the k-slot ordered W fragment layout.
  // U = T diag(beta) V in accumulator layout (the scan kernel's initial vn tiles).
  {
    bf16x8 tbe[2], tb[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float* trow = &sm.T[(16 * w + c16) * LDF + 32 * s + 8 * g4];
      float a[8], b[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int col = 32 * s + 8 * g4 + e;
        a[e] = trow[e] * sm.B[col];
        b[e] = a[e] * sm.EG[col];
      }
      tb[s] = pack8(a);
      tbe[s] = pack8(b);
    }
    {
      f32x4 accW[8];
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) {
        accW[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 2; ++s)
          accW[cb] = mma(__builtin_bit_cast(bf16x8, frag_tr(sm.K, LDK, 32 * s, 16 * cb, lane)), tbe[s], accW[cb]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<bf16x8*>(rec + ws::WN + (w * 4 + j) * ws::FRAG + lane * 16) =
            pack_acc_bf16(-accW[2 * j], -accW[2 * j + 1]);
    }
    // V row-major into the X buffer (dead after the inverse; its scratch blocks were read by the
    // inverse's last step -- hence the barrier)
    uint16_t* sV = reinterpret_cast<uint16_t*>(sm.X);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u16x8*>(&sV[(4 * tq + i) * LDK + 8 * fb]) = vreg[i];
    __syncthreads();
    f32x4 u[8];
    float m = 0.f;
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
      u[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 2; ++s)
        u[cb] = mma(tb[s], __builtin_bit_cast(bf16x8, frag_tr(sV, LDK, 32 * s, 16 * cb, lane)), u[cb]);
#pragma unroll
      for (int r = 0; r < 4; ++r) m = fmaxf(m, fabsf(u[cb][r]));
    }
    const int ue = fp16_fit_exp(wave_max(m));
    const float us = ldexpf(1.0f, ue);
    if (lane == 0) reinterpret_cast<float*>(rec + ws::USC)[w] = ldexpf(1.0f, -ue);
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
      const f16x4 hv = {(_Float16)(u[cb][0] * us), (_Float16)(u[cb][1] * us), (_Float16)(u[cb][2] * us),
                        (_Float16)(u[cb][3] * us)};
      *reinterpret_cast<f16x4*>(rec + ws::U + ((cb * 64 + lane) * 4 + w) * 8) = hv;
    }
  }
}

// Grid (key heads, chunks): one workgroup per (chunk, key head) does the key head's shared work
// once and then each of its Hv / Hqk value heads in turn (the next head's inputs load while the
// current one is computed).
template <typename BetaT>
__global__ __launch_bounds__(pf::NT, 3) void chunk_local_kernel(
    const uint16_t* __restrict__ q, int64_t qs, const uint16_t* __restrict__ k, int64_t ks,
    const uint16_t* __restrict__ v, int64_t vs,
    const float* __restrict__ g, const BetaT* __restrict__ beta, const int32_t* __restrict__ cu,
    const int32_t* __restrict__ seq_chunk0, int nseq, int seq_len, int Hqk, int Hv, int use_l2,
    uint8_t* __restrict__ work) {
  __shared__ LocalSmem sm;
  const int r = Hv / Hqk;
  KeyLoads KL;
  key_loads(KL, (int64_t)blockIdx.y * gridDim.x + blockIdx.x, q, qs, k, ks, cu, seq_chunk0, nseq, seq_len, Hqk);
  const int h0 = KL.hk * r;
  HeadLoads H;
  head_loads<BetaT>(H, KL.cp, h0, v, vs, g, beta, Hv);
  uint8_t* rec0 = work + ((int64_t)KL.slot * Hv + h0) * ws::BYTES;
  bf16x8 qf[4];
  const int ke = local_key(sm, KL, use_l2, qf, rec0);
  for (int j = 0; j < r; ++j) {
    if (j > 0) {
      head_loads<BetaT>(H, KL.cp, h0 + j, v, vs, g, beta, Hv);
      __syncthreads();  // this head rewrites the decay arrays and X
    }
    local_head(sm, H, qf, ke, rec0 + (int64_t)j * ws::BYTES);
  }
}

// ============================================================================================
// Chunked prefill, part 2: the inter-chunk state recurrence (the scan).
// ============================================================================================
// One workgroup per (sequence, value head, 16-column slice of the state): 8 workgroups per head,
// so a single long sequence still spreads over nseq * Hv * 8 workgroups.  The 6 waves specialise:
//   waves 0-1 (chain): vn = U - W S  and  S' = GL S + K^T (DEC vn) with the fp32 state slice
//                    S [128, 16] split by rows: wave 0 holds S rows 0-63, wave 1 rows 64-127, each in
//                    4 accumulator tiles for the whole sequence.  Each wave forms its half of the
//                    k-sum W S (8 MFMAs; wave 0 starts from U), the two partial sums are swapped
//                    through LDS with a per-wave step flag, and each wave then updates its own rows
//                    (8 MFMAs).  Both products take their B operand straight from accumulator
//                    registers (k-slot order)
//   waves 2-3 (output): o = Qg S + QK vn one chunk behind the chain (two token tiles each), from
//                    the S and vn the chain published in LDS and Qg / QK fragments they load
//                    themselves two chunks ahead
//   waves 4-5:       copy each chunk's WN and KT fragments, this slice's U tiles and the header
//                    (34.5 KiB) from L2 into a 3-slot LDS ring, two steps ahead
//   wave 6:          touches the records of the chunk kPrefetchAhead steps ahead, so they are in
//                    L2 (fetched from HBM once for the head's 8 slices) before they are copied
// One barrier per chunk.  During step c the chain computes chunk c from registers it read out of
// ring slot c%3 during step c-1, reads chunk c+1 from slot (c+1)%3 into registers, and writes
// vn(c) and S(c+1) into exchange slots c%3 and (c+1)%3; the output waves read exchange slot (c-1)%3;
// the loaders fill ring slot c%3 with chunk c+3.  So no LDS read latency sits on the chain's
// critical path beyond the partial-sum swap.
// The state update runs on fp16 MFMA.  Usually DEC vn and K^T fit fp16 as they are (see the fast
// path); otherwise DEC vn is scaled per column by a power of two sigma into [2^14, 2^15) and K^T
// by kappa, and the product is folded in as S' = (GL S sigma kappa + P) / (sigma kappa), so the fp32
// state only ever sees exact power-of-two rescaling besides the MFMA sum.
namespace rg {  // one ring slot
constexpr int WN = 0, KT = 16 * ws::FRAG, U = 32 * ws::FRAG, HDR = U + 2048, BYTES = HDR + 512;
}  // namespace rg
constexpr int kScanThreads = 448;  // 2 chain waves, 2 output waves, 2 loader waves, 1 prefetch wave
constexpr int kPrefetchAhead = 6;  // chunks between the L2 prefetch and the chain step
__device__ __forceinline__ bf16x8 lds_frag(const uint8_t* base, int f, int lane) {
  return *reinterpret_cast<const bf16x8*>(base + f * ws::FRAG + lane * 16);
}
__device__ __forceinline__ f16x8 lds_frag_h(const uint8_t* base, int f, int lane) {
  return *reinterpret_cast<const f16x8*>(base + f * ws::FRAG + lane * 16);
}
struct ScanSmem {
  uint8_t ring[3][rg::BYTES];
  uint8_t xch[3][6 * ws::FRAG];  // S (4 k-slot ordered bf16 B fragments) and vn (2)
  f32x4 part[2][4][64];          // the chain waves' partial sums of vn, [wave][token tile][lane]
  float init_buf[2][pf::D * 16]; // the next sequences' initial state slices [row][16 columns]
  uint32_t pf_sink[64];          // landing place of the prefetch wave's copies (never read)
  int flag[2];                   // step counter of each chain wave's published partial sum
};

// The sequences a scan workgroup walks: packed (cu / seq_chunk0) or uniform (seq_len tokens and
// nch_u chunks each), and their state rows.  Indices are wave-uniform, so these are scalar loads.
struct SeqTable {
  const int32_t* cu;
  const int32_t* chunk0;
  const int32_t* rows;
  int n_rows, seq_len, nch_u;
  __device__ __forceinline__ int64_t start(int s) const { return cu ? (int64_t)cu[s] : (int64_t)s * seq_len; }
  __device__ __forceinline__ int len(int s) const { return cu ? cu[s + 1] - cu[s] : seq_len; }
  __device__ __forceinline__ int first_chunk(int s) const { return cu ? chunk0[s] : s * nch_u; }
};
// First sequence of group g when `groups` groups share the chunk stream: the first sequence whose
// first chunk lies at or past g * total / groups (so groups hold whole sequences and differ by
// at most one sequence's chunks).
__device__ __forceinline__ int group_start(const SeqTable& t, int nseq, int64_t total, int groups, int g) {
  if (g <= 0) return 0;
  if (g >= groups) return nseq;
  const int64_t q = total * g / groups;
  int lo = 0, hi = nseq;  // first_chunk(nseq) == total >= q
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (t.first_chunk(mid) >= q) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}
// A position in a group's chunk stream: chunk c of the nch chunks of sequence s (which starts at
// packed token t0, holds L tokens and keeps its states in slot row `row`, -1: none), k = the
// ordinal of s among the group's non-empty sequences.
struct Walk {
  int s, c, nch, k, L, row;
  int64_t t0;
};
__device__ __forceinline__ int next_nonempty(const SeqTable& t, int s, int s_hi) {
  while (s < s_hi && t.len(s) == 0) ++s;
  return s;
}
__device__ __forceinline__ void walk_open(Walk& w, const SeqTable& t, int s, int s_hi) {
  w.s = s;
  w.c = 0;
  w.L = s < s_hi ? t.len(s) : 0;
  w.nch = (w.L + pf::CH - 1) / pf::CH;
  w.t0 = s < s_hi ? t.start(s) : 0;
  w.row = s < s_hi ? state_row(t.rows, t.n_rows, s) : -1;
}
__device__ __forceinline__ void walk_begin(Walk& w, const SeqTable& t, int s_lo, int s_hi) {
  walk_open(w, t, next_nonempty(t, s_lo, s_hi), s_hi);
  w.k = 0;
}
__device__ __forceinline__ bool walk_last(const Walk& w) { return w.c == w.nch - 1; }
__device__ __forceinline__ void walk_next(Walk& w, const SeqTable& t, int s_hi) {
  if (++w.c < w.nch) return;
  walk_open(w, t, next_nonempty(t, w.s + 1, s_hi), s_hi);
  ++w.k;
}

// One chunk's operands for one chain wave (half = 0: S rows 0-63, 1: rows 64-127).
// The KT fragments live outside: they are double-buffered, so that the next chunk's are read while
// this chunk's update MFMAs still use theirs.
struct ChainIn {
  bf16x8 fw[8];  // WN fragments (tb, k-block 2 half + j) at [tb * 2 + j]
  f16x8 u[2];    // this lane's U values (tiles 0,1 | 2,3); wave 0 only
  f32x4 uf[4];   // the same, scaled to fp32 (chain_u_convert); wave 0 only
  f32x4 dv[4];   // DEC of this lane's tokens
  f32x4 usc;     // wave 0 only
  float gl, ksc, kap;
};
typedef f16x8 KFrags[8];  // KT fragments of row tiles 4 half .. 4 half + 3 (2 k-blocks each)
template <int HALF>
__device__ __forceinline__ void chain_read_w(ChainIn& in, const uint8_t* ring, int lane) {
  const int g4 = lane >> 4;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int j = 0; j < 2; ++j) in.fw[tb * 2 + j] = lds_frag(ring + rg::WN, tb * 4 + 2 * HALF + j, lane);
  const float* hdr = reinterpret_cast<const float*>(ring + rg::HDR);
  if (HALF == 0) {
    in.usc = *reinterpret_cast<const f32x4*>(hdr + (ws::USC - ws::HDR) / 4);
    in.u[0] = *reinterpret_cast<const f16x8*>(ring + rg::U + lane * 32);
    in.u[1] = *reinterpret_cast<const f16x8*>(ring + rg::U + lane * 32 + 16);
  }
  in.gl = hdr[(ws::GL - ws::HDR) / 4];
  in.ksc = hdr[(ws::KSC - ws::HDR) / 4];
  in.kap = hdr[(ws::KAP - ws::HDR) / 4];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) in.dv[tb] = *reinterpret_cast<const f32x4*>(hdr + 16 * tb + 4 * g4);
}
// U -> fp32 with its tile scales (1 unless |U| left [2^-4, 2^14); same value in every lane), done
// once the reads have landed, off the next step's critical path.
__device__ __forceinline__ void chain_u_convert(ChainIn& in) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    in.uf[0][r] = (float)in.u[0][r];
    in.uf[1][r] = (float)in.u[0][4 + r];
    in.uf[2][r] = (float)in.u[1][r];
    in.uf[3][r] = (float)in.u[1][4 + r];
  }
  const bool unit = in.usc[0] == 1.0f && in.usc[1] == 1.0f && in.usc[2] == 1.0f && in.usc[3] == 1.0f;
  if (!__builtin_amdgcn_readfirstlane((int)unit)) {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) in.uf[tb] *= in.usc[tb];
  }
}
template <int HALF>
__device__ __forceinline__ void chain_read_k(KFrags& fk, const uint8_t* ring, int lane) {
#pragma unroll
  for (int f = 0; f < 8; ++f) fk[f] = lds_frag_h(ring + rg::KT, 8 * HALF + f, lane);
}
// Bounded waits: `limit` polls, then the wait gives up and raises the device status word (read
// back by gdn_device_status), so a broken invariant neither hangs the GPU nor passes silently.
struct WaitCtl {
  int limit;
  int* status;
};
// Wait until the other chain wave has published step `target` (it always publishes before it waits
// itself, so the wait ends; the bound only keeps a broken invariant from hanging the GPU).  Program
// order suffices after it for the same reason as in set_flag.
__device__ __forceinline__ void wait_flag(int* flag, int target, const WaitCtl& wc, int lane) {
  int i = 0;
  for (; i < wc.limit; ++i) {
    const int v = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (__builtin_amdgcn_readfirstlane(v) == target) break;
  }
  if (i == wc.limit && lane == 0) __hip_atomic_fetch_or(wc.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("" ::: "memory");  // the partial-sum reads stay behind the flag read
}
// Publish step `value` after this wave's earlier LDS writes.  LDS performs a CU's operations in one
// global order, one wave's in program order, so a reader that sees the flag and then reads the
// partial sums sees them written: no fence (and no wait for the writes) is needed, only program
// order, which the compiler barriers keep.
__device__ __forceinline__ void set_flag(int* flag, int value, int lane) {
  asm volatile("" ::: "memory");
  if (lane == 0) __hip_atomic_store(flag, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// The loader waves move a chunk's ring operands straight from L2 into LDS with global_load_lds
// (16 bytes per lane: one wave instruction fills one 1 KiB fragment, lane l at byte 16 l), so the
// data never passes through registers and the loaders issue no LDS stores.  Fragments of one
// chunk: WN 0..15 and KT 0..15 (KT from the key head's record rec_kq), U fragments 2n, 2n+1 of
// slice n, and the 512-byte header (lanes < 32).  Loader wave 0 issues WN 0-7, KT 0-7, U 0 and
// the header (kDmaOps0 instructions), wave 1 WN 8-15, KT 8-15 and U 1 (kDmaOps1).
constexpr int kDmaOps0 = 18, kDmaOps1 = 17;
__device__ __forceinline__ void dma_frag(uint8_t* lds, const uint8_t* src, int lane) {
  __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(src + lane * 16),
                                   reinterpret_cast<uint32_t*>(lds), 16, 0, 0);
}
// The 128 x 16 fp32 initial-state slice at src (row pitch D floats) into an init_buf (row-major,
// 64 bytes a row): 8 instructions, loader wave wl issues 4 (kInitOps).
constexpr int kInitOps = 4;
__device__ __forceinline__ void init_dma(float* dst, const float* src, int wl, int lane) {
#pragma unroll
  for (int i = kInitOps * wl; i < kInitOps * wl + kInitOps; ++i) {
    const int p = 64 * i + lane;  // 16-byte piece: row p / 4, columns 4 (p % 4) ..
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(src + (p >> 2) * pf::D + 4 * (p & 3)),
                                     reinterpret_cast<uint32_t*>(dst + 256 * i), 16, 0, 0);
  }
}
// L2 prefetch of the lines slice n of a head reads from one chunk's records: its eighth of WN, KT
// (key head's record) and QG (key head's record), its U tiles, an eighth of QK, the header and
// the row factors -- 78 lines of 128 bytes, 2 instructions.  Each lane copies one dword of its
// line into pf_sink (4-byte global_load_lds), so nothing lands in registers; the lines stay in the
// XCD's L2 for the other slices, which run on the same XCD.
__device__ __forceinline__ void scan_prefetch(uint32_t* sink, const uint8_t* rec, const uint8_t* rec_kq, int n,
                                              int lane) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int x = 64 * i + lane;
    const uint8_t* p = nullptr;
    if (x < 16) p = rec + ws::WN + (16 * n + x) * 128;
    else if (x < 32) p = rec_kq + ws::KT + (16 * n + x - 16) * 128;
    else if (x < 48) p = rec + ws::U + n * 2048 + (x - 32) * 128;
    else if (x < 64) p = rec_kq + ws::QG + (16 * n + x - 48) * 128;
    else if (x < 72) p = rec + ws::QK + (8 * n + x - 64) * 128;
    else if (x < 76) p = rec + ws::HDR + (x - 72) * 128;
    else if (x < 78) p = rec + ws::EGS + (x - 76) * 128;
    if (p) __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(p), sink, 4, 0, 0);
  }
}
__device__ __forceinline__ void scan_dma(uint8_t* dst, const uint8_t* rec, const uint8_t* rec_kq, int n, int wl,
                                         int lane) {
#pragma unroll
  for (int i = 0; i < 8; ++i) dma_frag(dst + rg::WN + (8 * wl + i) * ws::FRAG, rec + ws::WN + (8 * wl + i) * ws::FRAG, lane);
#pragma unroll
  for (int i = 0; i < 8; ++i) dma_frag(dst + rg::KT + (8 * wl + i) * ws::FRAG, rec_kq + ws::KT + (8 * wl + i) * ws::FRAG, lane);
  dma_frag(dst + rg::U + wl * ws::FRAG, rec + ws::U + n * 2048 + wl * ws::FRAG, lane);
  if (wl == 0 && lane < 32) dma_frag(dst + rg::HDR, rec + ws::HDR, lane);
}
// Wait until every chunk but the most recently issued one has landed in LDS (keep: the newest
// chunk's copies may stay in flight) -- per-wave instruction counts, the loaders issue nothing else.
__device__ __forceinline__ void dma_wait(int wl, bool keep) {
  if (!keep) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if (wl == 0) asm volatile("s_waitcnt vmcnt(18)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(17)" ::: "memory");
}
static_assert(kDmaOps0 == 18 && kDmaOps1 == 17, "dma_wait's counts follow scan_dma");
// The loaders' workgroup barrier.  __syncthreads() would also wait for every copy in flight (its
// release fence covers the LDS the copies write); the loaders order their copies themselves with
// dma_wait, so they meet the other waves at the bare barrier.  The LDS reads of a slot by the
// other waves complete before those waves reach the barrier (their __syncthreads waits for them),
// so a copy issued after the barrier cannot overtake them.
__device__ __forceinline__ void loader_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// The chain and output waves' workgroup barrier: it waits for their own LDS accesses (lgkmcnt 0),
// which is all the other waves depend on; their global loads and stores (the output waves' next
// operands, the rows of o and of final states) stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// An output wave's per-chunk operands.  Output wave P handles token tiles A = P and B = 3 - P (one
// and two non-zero QK fragments: tile tb has QK fragments (tb, j) for j <= tb / 2), so the two
// output waves do equal work: its QG fragments (8, from the key head's record), its 3 QK fragments
// and the row factors scale e^{G_t} of this lane's token in each of its tiles.
struct OutFrags {
  bf16x8 qg[8], qk[3];
  float egs[2];
};
template <int P>
__device__ __forceinline__ void out_load(OutFrags& f, const uint8_t* rec, const uint8_t* rec_kq, int lane) {
  constexpr int A = P, B = 3 - P;
  const float* eg = reinterpret_cast<const float*>(rec + ws::EGS) + (lane & 15);
  f.egs[0] = eg[16 * A];
  f.egs[1] = eg[16 * B];
  const uint8_t* qg = rec_kq + ws::QG + lane * 16;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f.qg[j] = *reinterpret_cast<const bf16x8*>(qg + (A * 4 + j) * ws::FRAG);
    f.qg[4 + j] = *reinterpret_cast<const bf16x8*>(qg + (B * 4 + j) * ws::FRAG);
  }
  const uint8_t* qk = rec + ws::QK + lane * 16;
  f.qk[0] = *reinterpret_cast<const bf16x8*>(qk + (A * 2) * ws::FRAG);
  f.qk[1] = *reinterpret_cast<const bf16x8*>(qk + (B * 2) * ws::FRAG);
  f.qk[2] = *reinterpret_cast<const bf16x8*>(qk + (B * 2 + 1) * ws::FRAG);
}
// o^T = S^T Qg^T + vn^T QK^T, tile by tile.  The k-slot ordered B fragments of S and vn are A
// fragments of S^T and vn^T, and the QG / QK A fragments are B fragments of their transposes, so
// the transposed products need no data movement -- and their accumulator layout gives each lane 4
// consecutive output columns of one token: lane (c, g) holds o[16 tb + c][16 n + 4g .. 4g + 3].
template <int P, typename OutT>
__device__ __forceinline__ void out_step(const OutFrags& f, const uint8_t* xch, OutT* out, int64_t t0, int len,
                                         int Hv, int h, int col0, int lane) {
  using namespace pf;
  constexpr int A = P, B = 3 - P;
  bf16x8 sb[4], vb[2];
#pragma unroll
  for (int j = 0; j < 4; ++j) sb[j] = lds_frag(xch, j, lane);
#pragma unroll
  for (int j = 0; j < 2; ++j) vb[j] = lds_frag(xch, 4 + j, lane);
  f32x4 O[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    O[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) O[i] = mma(sb[j], f.qg[i * 4 + j], O[i]);
    O[i] *= f.egs[i];
  }
  O[0] = mma(vb[0], f.qk[0], O[0]);
  O[1] = mma(vb[0], f.qk[1], O[1]);
  O[1] = mma(vb[1], f.qk[2], O[1]);
  const int c16 = lane & 15, g4 = lane >> 4;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = 16 * (i == 0 ? A : B) + c16;
    if (row < len) {
      OutT* o = out + ((t0 + row) * Hv + h) * D + col0 + 4 * g4;
      if constexpr (sizeof(OutT) == 2) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 pk = {f2bf2(O[i][0], O[i][1]), f2bf2(O[i][2], O[i][3])};
        *reinterpret_cast<u32x2*>(o) = pk;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) Elem<OutT>::store(o + r, O[i][r]);
      }
    }
  }
}
// An output wave: step c computes chunk c-1 of the stream (F0 / F1: even / odd chunks, loaded two
// chunks ahead; the walk follows chunk c-1 for its sequence position).
template <int P, typename OutT>
__device__ __forceinline__ void output_wave(const ScanSmem& sm, const uint8_t* rec0, int64_t rstride,
                                            int64_t kq_off, OutT* out, const SeqTable& tab, int s_lo, int s_hi,
                                            int nch, int Hv, int h, int col0, int lane) {
  using namespace pf;
  Walk w;
  walk_begin(w, tab, s_lo, s_hi);
  OutFrags F0, F1;
  if (nch > 0) out_load<P>(F0, rec0, rec0 + kq_off, lane);
  lds_barrier();  // prologue
  if (nch > 1) out_load<P>(F1, rec0 + rstride, rec0 + rstride + kq_off, lane);
  lds_barrier();  // step 0
  int xp = 0;        // (c - 1) % 3
  for (int c = 1; c <= nch; c += 2) {
    {
      const int len = w.L - w.c * CH < CH ? w.L - w.c * CH : CH;
      out_step<P, OutT>(F0, sm.xch[xp], out, w.t0 + (int64_t)w.c * CH, len, Hv, h, col0, lane);
      walk_next(w, tab, s_hi);
      if (c + 1 < nch) out_load<P>(F0, rec0 + (int64_t)(c + 1) * rstride, rec0 + (int64_t)(c + 1) * rstride + kq_off, lane);
      xp = xp == 2 ? 0 : xp + 1;
      lds_barrier();  // end of step c
    }
    if (c + 1 <= nch) {
      const int len = w.L - w.c * CH < CH ? w.L - w.c * CH : CH;
      out_step<P, OutT>(F1, sm.xch[xp], out, w.t0 + (int64_t)w.c * CH, len, Hv, h, col0, lane);
      walk_next(w, tab, s_hi);
      if (c + 2 < nch) out_load<P>(F1, rec0 + (int64_t)(c + 2) * rstride, rec0 + (int64_t)(c + 2) * rstride + kq_off, lane);
      xp = xp == 2 ? 0 : xp + 1;
      lds_barrier();  // end of step c+1
    }
  }
}

// What a chain step does after its update when its chunk ends a sequence: store this lane's final
// state column (fin; nullptr: not kept) and continue from the next sequence's initial state (nxt:
// this lane's column of an init_buf; nullptr: zeros).
struct Swap {
  bool last;
  float* fin;
  const float* nxt;
};
template <int HALF>
__device__ __forceinline__ void chain_step(ScanSmem& sm, f32x4 (&S)[4], bf16x8 (&Sb)[2], ChainIn& in, KFrags& fk,
                                           KFrags& fk_next, int c, int nch, int& x0, const Swap& sw,
                                           const WaitCtl& wc, int lane) {
  uint8_t* xch = sm.xch[x0];
  const int x1 = x0 == 2 ? 0 : x0 + 1;
  const uint8_t* nxt = sm.ring[x1];  // chunk c+1 sits in ring slot (c+1) % 3
  // this wave's half of the k-sum: U (wave 0) + sum over S rows 64 HALF.. of WN S
  f32x4 acc[4];
  if (HALF == 0) {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) acc[tb] = in.uf[tb];
  } else {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) acc[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) acc[tb] = mma(in.fw[tb * 2 + j], Sb[j], acc[tb]);
  // publish the partial sum, then the step flag (one wave's LDS writes complete in order)
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) sm.part[HALF][tb][lane] = acc[tb];
  set_flag(&sm.flag[HALF], c + 1, lane);
  f32x4 dv[4];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) dv[tb] = in.dv[tb];
  const float gl = in.gl, ksc = in.ksc, kap = in.kap;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    S[i] *= gl;
    asm volatile("" : "+v"(S[i]));  // done while the other wave finishes its half
  }
  wait_flag(&sm.flag[1 - HALF], c + 1, wc, lane);
  // vn = U - W S: both waves add the same two partial sums (a + b == b + a exactly)
  f32x4 vn[4];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) vn[tb] = acc[tb] + sm.part[1 - HALF][tb][lane];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) asm volatile("" : "+v"(vn[tb]));  // complete before the reads below
  // chunk c+1's operands: issued behind the partial-sum reads (whose completion the chain waits
  // for; LDS returns in order and the wait counter saturates at 15), so they arrive while this
  // chunk's update runs
  __builtin_amdgcn_sched_barrier(0);
  if (c + 1 < nch) {
    chain_read_w<HALF>(in, nxt, lane);
    chain_read_k<HALF>(fk_next, nxt, lane);
  }
  // DEC vn -> fp16; wave 1 publishes vn (bf16) for the output waves
  float m = 0.f;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      dv[tb][r] *= vn[tb][r];
      m = fmaxf(m, fabsf(dv[tb][r]));
    }
  if (HALF == 1) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      *reinterpret_cast<bf16x8*>(&xch[(4 + j) * ws::FRAG + lane * 16]) = pack_acc_bf16(vn[2 * j], vn[2 * j + 1]);
  }
  // Fast path (the usual case): kappa = 1 and every |DEC vn| below 2^14 with the largest at
  // least 2^-4, so DEC vn goes to fp16 unscaled.  Otherwise: per-column power-of-two scaling.
  // Both waves hold the same DEC vn, so they take the same path.
  const bool fast = kap == 1.0f && __builtin_amdgcn_ballot_w64(m >= 16384.0f) == 0 &&
                    __builtin_amdgcn_ballot_w64(m >= 0.0625f) != 0;
  if (__builtin_amdgcn_readfirstlane((int)fast)) {
    f16x8 vh[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) vh[j] = pack_acc_f16(dv[2 * j], dv[2 * j + 1], 1.0f);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      S[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fk[i * 2], vh[0], S[i], 0, 0, 0);
      S[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fk[i * 2 + 1], vh[1], S[i], 0, 0, 0);
    }
  } else {
    m = fmaxf(m, __shfl_xor(m, 16, kWave));
    m = fmaxf(m, __shfl_xor(m, 32, kWave));
    const int se = fp16_scale_exp(m);
    f16x8 vh[2];
    const float sigma = ldexpf(1.0f, se);
#pragma unroll
    for (int j = 0; j < 2; ++j) vh[j] = pack_acc_f16(dv[2 * j], dv[2 * j + 1], sigma);
    const float pre = sigma * kap;        // exact powers of two
    const float post = ldexpf(ksc, -se);  // 1 / (sigma * kappa)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      S[i] *= pre;
      S[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fk[i * 2], vh[0], S[i], 0, 0, 0);
      S[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fk[i * 2 + 1], vh[1], S[i], 0, 0, 0);
      S[i] *= post;
    }
  }
  // next chunk's U to fp32 while the update's MFMAs run
  if (HALF == 0) chain_u_convert(in);
  if (sw.last) {
    const int g4 = lane >> 4;
    if (sw.fin) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) sw.fin[(64 * HALF + 16 * i + 4 * g4 + r) * pf::D] = S[i][r];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) S[i][r] = sw.nxt ? sw.nxt[(64 * HALF + 16 * i + 4 * g4 + r) * 16] : 0.f;
  }
  uint8_t* xn = sm.xch[x1];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    Sb[j] = pack_acc_bf16(S[2 * j], S[2 * j + 1]);
    *reinterpret_cast<bf16x8*>(&xn[(2 * HALF + j) * ws::FRAG + lane * 16]) = Sb[j];
  }
  x0 = x1;
  lds_barrier();  // end of step c
}

// The chain wave holding S rows 64 HALF .. 64 HALF + 63 (4 accumulator tiles) of one 16-column
// slice (this lane: column col) through every chunk of its group's sequences: at a sequence's last
// chunk the step stores the final state and continues from the next sequence's initial state,
// which the loader waves have staged in init_buf[(k + 1) & 1].  The walk runs one chunk ahead
// (wn), so its table reads are in flight a whole step before they are needed.  The chain's
// barriers wait only for its LDS accesses: its final-state stores need no ordering with the
// other waves.
template <int HALF>
__device__ __forceinline__ void chain_wave(ScanSmem& sm, const float* __restrict__ init,
                                           float* __restrict__ final_state, int Hv, int h, int col,
                                           const SeqTable& tab, int s_lo, int s_hi, int nch, const WaitCtl& wc,
                                           int lane) {
  using namespace pf;
  const int g4 = lane >> 4;
  auto state_col = [&](const float* base, int row) -> const float* {  // this lane's column of a state
    return (base && row >= 0) ? base + ((int64_t)row * Hv + h) * D * D + col : nullptr;
  };
  Walk w, wn;  // chunk c, chunk c+1
  walk_begin(w, tab, s_lo, s_hi);
  wn = w;
  walk_next(wn, tab, s_hi);
  f32x4 S[4];
  const float* s0 = state_col(init, w.row);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) S[i][r] = s0 ? s0[(64 * HALF + 16 * i + 4 * g4 + r) * D] : 0.f;
  bf16x8 Sb[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    Sb[j] = pack_acc_bf16(S[2 * j], S[2 * j + 1]);
    *reinterpret_cast<bf16x8*>(&sm.xch[0][(2 * HALF + j) * ws::FRAG + lane * 16]) = Sb[j];
  }
  if (lane == 0) sm.flag[HALF] = 0;
  lds_barrier();  // prologue
  ChainIn in;
  KFrags fk0, fk1;  // chunks c even / odd
  if (nch > 0) {
    chain_read_w<HALF>(in, sm.ring[0], lane);
    if (HALF == 0) chain_u_convert(in);
    chain_read_k<HALF>(fk0, sm.ring[0], lane);
  }
  auto swap_of = [&]() {
    Swap sw{false, nullptr, nullptr};
    if (walk_last(w)) {  // then wn is the first chunk of the next non-empty sequence (if any)
      sw.last = true;
      sw.fin = const_cast<float*>(state_col(final_state, w.row));
      if (state_col(init, wn.row)) sw.nxt = sm.init_buf[(w.k + 1) & 1] + (lane & 15);
    }
    return sw;
  };
  int x0 = 0;  // c % 3
  for (int c = 0; c < nch; c += 2) {
    chain_step<HALF>(sm, S, Sb, in, fk0, fk1, c, nch, x0, swap_of(), wc, lane);
    w = wn;
    walk_next(wn, tab, s_hi);
    if (c + 1 < nch) {
      chain_step<HALF>(sm, S, Sb, in, fk1, fk0, c + 1, nch, x0, swap_of(), wc, lane);
      w = wn;
      walk_next(wn, tab, s_hi);
    }
  }
  lds_barrier();  // step nch (the output waves' last chunk)
}

// The scan: one workgroup per (sequence group, value head, 16-column slice).  A group is a run of
// whole sequences; its chunk records are consecutive workspace slots, so the workgroup streams
// them in order and carries the state across sequence boundaries (groups == nseq: one sequence per
// workgroup).
template <typename OutT>
__global__ __launch_bounds__(kScanThreads, 1) void chunk_scan_kernel(
    const float* __restrict__ init, float* __restrict__ final_state, OutT* __restrict__ out,
    const int32_t* __restrict__ cu, const int32_t* __restrict__ seq_chunk0, const int32_t* __restrict__ rows,
    int n_rows, int nseq, int seq_len, int Hqk, int Hv, int groups, int64_t total_chunks,
    const uint8_t* __restrict__ work, WaitCtl wc) {
  using namespace pf;
  __shared__ ScanSmem sm;
  // block -> (group-head pair, slice); the 8 slices of a pair share blockIdx % 8 and therefore an
  // XCD (workgroups are dispatched round-robin over the 8 XCDs), so they share one L2.
  const int b = blockIdx.x;
  const int pair = (b >> 6) * 8 + (b & 7), n = (b >> 3) & 7;
  if (pair >= groups * Hv) return;
  const int h = pair % Hv, grp = pair / Hv;
  const SeqTable tab{cu, seq_chunk0, rows, n_rows, seq_len, (seq_len + CH - 1) / CH};
  int s_lo, s_hi;
  if (groups == nseq) {
    s_lo = grp;
    s_hi = grp + 1;
  } else {
    s_lo = group_start(tab, nseq, total_chunks, groups, grp);
    s_hi = group_start(tab, nseq, total_chunks, groups, grp + 1);
  }
  if (s_lo >= s_hi) return;
  const int slot0 = tab.first_chunk(s_lo);
  const int nch = tab.first_chunk(s_hi) - slot0;  // chunks of the group's stream
  const int t = threadIdx.x, lane = t & 63, c16 = lane & 15;
  const int role = __builtin_amdgcn_readfirstlane(t >> 6);
  const int64_t rstride = (int64_t)Hv * ws::BYTES;
  const uint8_t* rec0 = work + (int64_t)slot0 * rstride + (int64_t)h * ws::BYTES;
  const int64_t kq_off = -(int64_t)(h % (Hv / Hqk)) * ws::BYTES;  // record of the key head's owner
  const int col = 16 * n + c16;

  if (role < 2) {
    // ---------------- chain waves ----------------
    if (role == 0) chain_wave<0>(sm, init, final_state, Hv, h, col, tab, s_lo, s_hi, nch, wc, lane);
    else chain_wave<1>(sm, init, final_state, Hv, h, col, tab, s_lo, s_hi, nch, wc, lane);
  } else if (role < 4) {
    // ---------------- output waves: step c computes chunk c-1 ----------------
    if (role == 2) output_wave<0, OutT>(sm, rec0, rstride, kq_off, out, tab, s_lo, s_hi, nch, Hv, h, 16 * n, lane);
    else output_wave<1, OutT>(sm, rec0, rstride, kq_off, out, tab, s_lo, s_hi, nch, Hv, h, 16 * n, lane);
  } else if (role == 6) {
    // ---------------- prefetch wave: chunk c + kPrefetchAhead at step c ----------------
    // Its copies are never waited for until the end (their own wave's counter), so a slow HBM
    // fetch delays nothing; at most a few dozen are in flight.
    auto touch = [&](int c) {
      const uint8_t* rec = rec0 + (int64_t)c * rstride;
      scan_prefetch(sm.pf_sink, rec, rec + kq_off, n, lane);
    };
    for (int c = 3; c < kPrefetchAhead && c < nch; ++c) touch(c);
    loader_barrier();  // prologue
    for (int c = 0; c < nch; ++c) {
      if (c + kPrefetchAhead < nch) touch(c + kPrefetchAhead);
      loader_barrier();  // end of step c
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no copy may land after the workgroup ends
    loader_barrier();  // step nch
  } else {
    // ---------------- loader waves ----------------
    const int wl = role - 4, lt = t - 256;
    // Empty sequences have no chunks: their final state is their initial state (zeros without
    // one).  Loader lane lt copies row lt of the slice.
    if (final_state) {
      for (int s = s_lo; s < s_hi; ++s) {
        if (tab.len(s) != 0) continue;
        const int r = state_row(rows, n_rows, s);
        if (r < 0) continue;
        const int64_t off = ((int64_t)r * Hv + h) * D * D + (int64_t)lt * D + 16 * n;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 x = init ? *reinterpret_cast<const f32x4*>(init + off + 4 * q) : f32x4{0.f, 0.f, 0.f, 0.f};
          *reinterpret_cast<f32x4*>(final_state + off + 4 * q) = x;
        }
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the copies below count their own loads
    }
    // Chunk j sits in ring slot j % 3.  The chain reads chunk j's operands during step j-1 (chunk 0:
    // after the prologue barrier), so from step j on that slot is free: step j (>= 1) starts the
    // copy of chunk j+3 into it, and the copy has steps j and j+1 to land (chunk 3, started at
    // step 1, has one step).  Before the barrier that ends step j, chunk j+2 must be complete.
    // When chunk j+1 ends the k-th sequence, step j (the prologue for j+1 = 0) also copies the
    // next sequence's initial state slice into init_buf[(k + 1) & 1], issued before the chunk
    // copy, so it is complete at the same barrier; the chain reads it at the end of step j+1.
    // The other buffer may still be read during that step, and a buffer is reused two sequences
    // later, after the step that read it ended.
    auto dma_chunk = [&](int c) {
      const uint8_t* rec = rec0 + (int64_t)c * rstride;
      scan_dma(sm.ring[c % 3], rec, rec + kq_off, n, wl, lane);
    };
    Walk w;  // follows chunk j+1
    walk_begin(w, tab, s_lo, s_hi);
    auto dma_next_init = [&]() {
      if (!init || !walk_last(w)) return;
      Walk w2 = w;  // the next non-empty sequence's first chunk
      walk_next(w2, tab, s_hi);
      if (w2.row >= 0) init_dma(sm.init_buf[(w.k + 1) & 1], init + ((int64_t)w2.row * Hv + h) * D * D + 16 * n, wl, lane);
    };
    if (nch > 0) dma_next_init();
    if (nch > 0) dma_chunk(0);
    if (nch > 1) dma_chunk(1);
    if (nch > 2) dma_chunk(2);
    dma_wait(wl, nch > 2);  // chunks 0 and 1 (and the initial state after chunk 0)
    loader_barrier();       // prologue
    for (int c = 0; c < nch; ++c) {
      walk_next(w, tab, s_hi);
      if (c + 1 < nch) dma_next_init();
      if (c == 1 && 3 < nch) dma_chunk(3);
      const bool issued = c >= 1 && c + 3 < nch;
      if (issued) dma_chunk(c + 3);
      dma_wait(wl, issued);  // chunk c+2 (and the initial state after chunk c+1)
      loader_barrier();      // end of step c
    }
    dma_wait(wl, false);
    loader_barrier();  // step nch
  }
}

// ============================================================================================
// Causal depthwise conv prefill + SiLU with decode-state capture.
// ============================================================================================
// One thread per (run of kConvRun consecutive packed tokens, 8 channels): it loads the input rows
// p0-K+1 .. p0+kConvRun-1 once with 16-byte reads and slides the K-tap window over them (rows before a
// token's sequence come from the sequence's history row [C, K], x_{-j} = history[K - j], or are
// zero), then writes 8 outputs per token with one 16-byte store.  A workgroup covers one token run
// and 2048 channels, so the sequence walk is uniform across it.  Numerics of F.conv1d on bf16: fp32
// accumulation of the K products (+ bias), one bf16 rounding, SiLU, bf16.  The decode conv state a
// sequence leaves (its last K inputs) is written afterwards by conv_state_capture_kernel, so the
// history may be the same slot rows the state goes to.
constexpr int kConvRun = 8;
// SiLU with the hardware exp and reciprocal (each within about 1 ulp in fp32, so the bf16 result
// is within one bf16 ulp of the exactly rounded x / (1 + e^-x)).
__device__ __forceinline__ float silu_fast(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ int find_seq(const int32_t* cu, int nseq, int64_t p) {
  int lo = 0, hi = nseq - 1;  // last sequence whose start <= p (skips empty ones)
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= p) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

template <int K>
__global__ __launch_bounds__(256) void conv_prefill_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                                           const uint16_t* __restrict__ weight,
                                                           const uint16_t* __restrict__ bias,
                                                           const uint16_t* __restrict__ history,
                                                           const int32_t* __restrict__ rows, int n_rows,
                                                           uint16_t* __restrict__ out, int64_t total_tokens,
                                                           const int32_t* __restrict__ cu, int nseq, int seq_len,
                                                           int C) {
  const int cg = blockIdx.x * blockDim.x + threadIdx.x;  // 8-channel group
  const int64_t p0 = (int64_t)blockIdx.y * kConvRun;
  if (8 * cg >= C) return;
  const int c0 = 8 * cg;
  const int nrun = total_tokens - p0 < kConvRun ? (int)(total_tokens - p0) : kConvRun;
  // rows p0-K+1 .. p0+nrun-1 (only those inside [0, total_tokens) are read)
  u16x8 xr[kConvRun + K - 1];
  const u16x8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < kConvRun + K - 1; ++i) {
    const int64_t tok = p0 - (K - 1) + i;
    xr[i] = (tok >= 0 && i < nrun + K - 1) ? *reinterpret_cast<const u16x8*>(x + tok * x_stride + c0) : zero;
  }
  u16x8 wt[K];  // weight[c0 + e][r] -> wt[r][e]
  {
    const u16x8* wp = reinterpret_cast<const u16x8*>(weight + (int64_t)c0 * K);  // 8 K contiguous values
    uint16_t w[8 * K];
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const u16x8 v = wp[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) w[8 * i + e] = v[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int r = 0; r < K; ++r) wt[r][e] = w[e * K + r];
  }
  float bv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) bv[e] = bias ? bf2f(bias[c0 + e]) : 0.f;
  // sequence of p0, then walk forward (uniform across the workgroup)
  int s = cu ? find_seq(cu, nseq, p0) : (int)(p0 / seq_len);
  int64_t s_lo = cu ? (int64_t)cu[s] : (int64_t)s * seq_len;
  int64_t s_hi = cu ? (int64_t)cu[s + 1] : s_lo + seq_len;
#pragma unroll
  for (int i = 0; i < kConvRun; ++i) {
    if (i >= nrun) break;  // (uniform: the last run of the batch)
    const int64_t p = p0 + i;
    while (p >= s_hi) {  // next non-empty sequence
      ++s;
      s_lo = cu ? (int64_t)cu[s] : (int64_t)s * seq_len;
      s_hi = cu ? (int64_t)cu[s + 1] : s_lo + seq_len;
    }
    u16x8 win[K];
    if (p - (K - 1) >= s_lo) {
#pragma unroll
      for (int r = 0; r < K; ++r) win[r] = xr[i + r];
    } else {
      const int hrow = history ? state_row(rows, n_rows, s) : -1;
#pragma unroll
      for (int r = 0; r < K; ++r) {
        const int64_t tok = p - (K - 1) + r;
        if (tok >= s_lo) {
          win[r] = xr[i + r];
        } else {
          const int back = (int)(s_lo - tok);  // 1..K-1
#pragma unroll
          for (int e = 0; e < 8; ++e)
            win[r][e] = hrow >= 0 ? history[((int64_t)hrow * C + c0 + e) * K + (K - back)] : (uint16_t)0;
        }
      }
    }
    u16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = bv[e];
#pragma unroll
      for (int r = 0; r < K; ++r) acc += bf2f(win[r][e]) * bf2f(wt[r][e]);
      o[e] = f2bf(silu_fast(rbf(acc)));
    }
    *reinterpret_cast<u16x8*>(out + p * (int64_t)C + c0) = o;
  }
}

// The decode conv state each sequence leaves: its last K inputs, the front filled from its history
// row (or zeros) when the sequence is shorter than K -- an empty sequence keeps its history.  One
// thread per (sequence, channel) reads its old row entries before writing them, so `history` and
// `state` may be the same slot rows.
__global__ void conv_state_capture_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                          const uint16_t* history, const int32_t* __restrict__ hist_rows,
                                          uint16_t* state, const int32_t* __restrict__ state_rows, int n_rows,
                                          const int32_t* __restrict__ cu, int nseq, int seq_len, int C, int K) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)nseq * C) return;
  const int s = (int)(i / C), c = (int)(i % C);
  const int orow = state_row(state_rows, n_rows, s);
  if (orow < 0) return;
  const int hrow = history ? state_row(hist_rows, n_rows, s) : -1;
  const int64_t s_lo = cu ? (int64_t)cu[s] : (int64_t)s * seq_len;
  const int64_t L = cu ? (int64_t)cu[s + 1] - s_lo : seq_len;
  uint16_t win[8];
  for (int j = 0; j < K; ++j) {  // win[j] = input K - j before the end of the sequence
    const int64_t tok = L - K + j;  // position inside the sequence
    if (tok >= 0) win[j] = x[(s_lo + tok) * x_stride + c];
    else win[j] = hrow >= 0 ? history[((int64_t)hrow * C + c) * K + (K + tok)] : (uint16_t)0;
  }
  for (int j = 0; j < K; ++j) state[((int64_t)orow * C + c) * K + j] = win[j];
}

// ============================================================================================
// Gating: beta = sigmoid(b) in bf16, g = -exp(A_log) * softplus(a + dt_bias) in fp32.
// ============================================================================================
__global__ void gating_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, int64_t ab_stride,
                              const float* __restrict__ A_log, const float* __restrict__ dt_bias,
                              uint16_t* __restrict__ beta, float* __restrict__ g, int64_t rows, int Hv) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * Hv) return;
  const int64_t r = i / Hv;
  const int h = (int)(i % Hv);
  beta[i] = f2bf(sigmoid_f(bf2f(b[r * ab_stride + h])));
  g[i] = -expf(A_log[h]) * softplus_f(bf2f(a[r * ab_stride + h]) + dt_bias[h]);
}

// Status word of the bounded waits (bit 0: a wait gave up), one per device.
__device__ int g_wait_status;

// Workspace of gdn_chunk_prefill_noalloc: one static array per device (host code reaches it only
// through the address hipGetSymbolAddress returns on that device).
static __device__ __align__(256) uint8_t scratch[GDN_NOALLOC_SCRATCH_BYTES];

}  // namespace gdn

using namespace gdn;

namespace {
constexpr int kDefaultWaitLimit = 1 << 18;
int g_wait_limit = kDefaultWaitLimit;
// Device address of g_wait_status on the current device (looked up once per device); null on failure.
int* wait_status_ptr() {
  static int* cached[64] = {nullptr};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  if (!cached[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_wait_status)) != hipSuccess) return nullptr;
    cached[dev] = (int*)p;
  }
  return cached[dev];
}
}  // namespace

// Device address of `scratch` on the current device, looked up once per device (null on failure).
static uint8_t* scratch_ptr() {
  static uint8_t* cached[64] = {nullptr};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  if (!cached[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    cached[dev] = (uint8_t*)p;
  }
  return cached[dev];
}

extern "C" int gdn_device_status(int clear) {
  clear_error();
  int* p = wait_status_ptr();
  if (!p) return set_error(GDN_ELAUNCH, "gdn_device_status: no device status word on the current device");
  int v = 0;
  if (hipMemcpy(&v, p, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess)
    return set_error(GDN_ELAUNCH, "gdn_device_status: reading the status word failed");
  if (clear) {
    const int zero = 0;
    if (hipMemcpy(p, &zero, sizeof(int), hipMemcpyHostToDevice) != hipSuccess)
      return set_error(GDN_ELAUNCH, "gdn_device_status: clearing the status word failed");
  }
  if (v) return set_error(GDN_EWAIT, "a bounded inter-wave wait of the chunked prefill gave up: the outputs and "
                                     "final states of the calls since the last status check are wrong");
  return GDN_OK;
}

extern "C" int gdn_set_wait_limit(int64_t polls) {
  clear_error();
  g_wait_limit = polls < 0 ? kDefaultWaitLimit : (polls > (1ll << 30) ? (1 << 30) : (int)polls);
  return GDN_OK;
}

extern "C" int gdn_unit_lower_inv(const float* X, float* T, int64_t batch, int n, void* stream) {
  clear_error();
  GDN_REQUIRE(X && T, "gdn_unit_lower_inv: null pointer");
  GDN_SUPPORT(n == 64, "gdn_unit_lower_inv: only 64x64 blocks are supported (got %d)", n);
  GDN_REQUIRE(batch >= 0 && batch < (1ll << 31), "gdn_unit_lower_inv: bad batch %lld", (long long)batch);
  if (batch == 0) return GDN_OK;
  unit_lower_inv_kernel<<<(unsigned)batch, pf::NT, 0, (hipStream_t)stream>>>(X, T);
  return check_launch("gdn_unit_lower_inv");
}

namespace {
// Compute units of the current device (cached per device).
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}
int scan_groups(int nseq, int Hv) {
  const int per_group = 8 * Hv, cus = device_cus();
  if (nseq <= 1 || per_group > cus) return nseq;
  const int g = cus / per_group;
  return g < nseq ? g : nseq;
}
}  // namespace

extern "C" int64_t gdn_chunk_prefill_workspace_bytes(int64_t total_chunks, int Hv) {
  return total_chunks * (int64_t)Hv * ws::BYTES;
}

extern "C" int gdn_chunk_prefill_rows(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                                      const void* v, int64_t v_stride, const float* g, const void* beta,
                                      int beta_dtype, const float* initial_state, float* final_state,
                                      const int32_t* state_rows, int n_rows, void* out, int64_t total_tokens,
                                      const int32_t* cu_seqlens, const int32_t* seq_chunk0, int64_t total_chunks,
                                      int nseq, int seq_len, int Hqk, int Hv, int D, int in_dtype,
                                      int use_qk_l2norm, void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  GDN_REQUIRE(state_rows ? n_rows >= 0 : n_rows == nseq,
              "gdn_chunk_prefill: without state_rows, n_rows must equal nseq");
  GDN_REQUIRE(q && k && v && g && beta && out, "gdn_chunk_prefill: null input/output pointer");
  GDN_SUPPORT(D == pf::D, "gdn_chunk_prefill: head dim %d unsupported (needs %d)", D, pf::D);
  GDN_SUPPORT(in_dtype == GDN_BF16, "gdn_chunk_prefill: q/k/v must be bfloat16 (MFMA operands)");
  GDN_REQUIRE(beta_dtype == GDN_F32 || beta_dtype == GDN_BF16, "gdn_chunk_prefill: bad beta dtype");
  GDN_REQUIRE(Hqk > 0 && Hv > 0 && Hv % Hqk == 0, "gdn_chunk_prefill: bad heads Hqk=%d Hv=%d", Hqk, Hv);
  GDN_REQUIRE(nseq >= 0 && total_tokens >= 0 && total_chunks >= 0, "gdn_chunk_prefill: negative sizes");
  GDN_REQUIRE(cu_seqlens ? seq_chunk0 != nullptr : (int64_t)nseq * seq_len == total_tokens,
              "gdn_chunk_prefill: cu_seqlens needs seq_chunk0; without it nseq*seq_len must be total_tokens");
  GDN_REQUIRE(cu_seqlens || total_chunks == (int64_t)nseq * ((seq_len + pf::CH - 1) / pf::CH),
              "gdn_chunk_prefill: total_chunks inconsistent with nseq/seq_len");
  GDN_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && q_stride % 8 == 0 && k_stride % 8 == 0 &&
                  v_stride % 8 == 0,
              "gdn_chunk_prefill: q/k/v rows must be 16-byte aligned");
  GDN_REQUIRE(aligned(out, 8), "gdn_chunk_prefill: out must be 8-byte aligned");
  GDN_REQUIRE((!initial_state || aligned(initial_state, 16)) && (!final_state || aligned(final_state, 16)),
              "gdn_chunk_prefill: initial/final state must be 16-byte aligned");
  GDN_REQUIRE(total_chunks == 0 || (workspace && aligned(workspace, 256) &&
                                    workspace_bytes >= gdn_chunk_prefill_workspace_bytes(total_chunks, Hv)),
              "gdn_chunk_prefill: workspace missing, misaligned or smaller than %lld bytes",
              (long long)gdn_chunk_prefill_workspace_bytes(total_chunks, Hv));
  GDN_REQUIRE(total_chunks < (1ll << 31) && ((int64_t)nseq * Hv + 7) / 8 * 64 < (1ll << 31),
              "gdn_chunk_prefill: grid too large");
  if (nseq == 0) return GDN_OK;
  hipStream_t s = (hipStream_t)stream;
  uint8_t* work = (uint8_t*)workspace;
  if (total_chunks > 0) {
    dim3 g1((unsigned)Hqk, (unsigned)total_chunks);
    if (beta_dtype == GDN_BF16)
      chunk_local_kernel<uint16_t><<<g1, pf::NT, 0, s>>>((const uint16_t*)q, q_stride, (const uint16_t*)k, k_stride,
                                                         (const uint16_t*)v, v_stride,
                                                         g, (const uint16_t*)beta, cu_seqlens, seq_chunk0, nseq,
                                                         seq_len, Hqk, Hv, use_qk_l2norm, work);
    else
      chunk_local_kernel<float><<<g1, pf::NT, 0, s>>>((const uint16_t*)q, q_stride, (const uint16_t*)k, k_stride,
                                                      (const uint16_t*)v, v_stride,
                                                      g, (const float*)beta, cu_seqlens, seq_chunk0, nseq, seq_len,
                                                      Hqk, Hv, use_qk_l2norm, work);
    int rc = check_launch("gdn_chunk_prefill(local)");
    if (rc) return rc;
  }
  // Sequence groups: when the Hv x 8 workgroups of one group leave CUs free, split the sequences
  // into as many groups (balanced by chunks) as fill the CUs once; each workgroup then streams its
  // group's sequences back to back.  Otherwise one sequence per workgroup.
  const WaitCtl wc{g_wait_limit, wait_status_ptr()};
  if (!wc.status) return set_error(GDN_ELAUNCH, "gdn_chunk_prefill: no device status word on the current device");
  const int groups = scan_groups(nseq, Hv);
  const int64_t pairs = (int64_t)groups * Hv;
  const int64_t scan_blocks = (pairs + 7) / 8 * 64;
  chunk_scan_kernel<uint16_t><<<(unsigned)scan_blocks, kScanThreads, 0, s>>>(
      initial_state, final_state, (uint16_t*)out, cu_seqlens, seq_chunk0, state_rows, n_rows, nseq, seq_len, Hqk,
      Hv, groups, total_chunks, work, wc);
  return check_launch("gdn_chunk_prefill(state)");
}

extern "C" int gdn_chunk_prefill(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                                 const void* v, int64_t v_stride, const float* g, const void* beta,
                                 int beta_dtype, const float* initial_state, float* final_state, void* out,
                                 int64_t total_tokens, const int32_t* cu_seqlens, const int32_t* seq_chunk0,
                                 int64_t total_chunks, int nseq, int seq_len, int Hqk, int Hv, int D, int in_dtype,
                                 int use_qk_l2norm, void* workspace, int64_t workspace_bytes, void* stream) {
  return gdn_chunk_prefill_rows(q, q_stride, k, k_stride, v, v_stride, g, beta, beta_dtype, initial_state,
                                final_state, nullptr, nseq, out, total_tokens, cu_seqlens, seq_chunk0, total_chunks,
                                nseq, seq_len, Hqk, Hv, D, in_dtype, use_qk_l2norm, workspace, workspace_bytes,
                                stream);
}

extern "C" int gdn_chunk_prefill_noalloc(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                                         const void* v, int64_t v_stride, const float* g, const void* beta,
                                         int beta_dtype, const float* initial_state, float* final_state,
                                         const int32_t* state_rows, int n_rows, void* out, int64_t total_tokens,
                                         const int32_t* cu_seqlens, const int32_t* seq_chunk0, int64_t total_chunks,
                                         int nseq, int seq_len, int Hqk, int Hv, int D, int in_dtype,
                                         int use_qk_l2norm, void* stream) {
  clear_error();
  GDN_REQUIRE(total_chunks >= 0 && Hv > 0, "gdn_chunk_prefill_noalloc: bad sizes");
  const int64_t need = gdn_chunk_prefill_workspace_bytes(total_chunks, Hv);
  GDN_REQUIRE(need <= GDN_NOALLOC_SCRATCH_BYTES,
              "gdn_chunk_prefill_noalloc: the call needs %lld bytes of workspace, the static scratch holds %lld "
              "(%lld chunks x %d value heads is too many; use gdn_chunk_prefill_rows with a workspace)",
              (long long)need, (long long)GDN_NOALLOC_SCRATCH_BYTES, (long long)total_chunks, Hv);
  uint8_t* ws_ptr = scratch_ptr();
  if (!ws_ptr) return set_error(GDN_ELAUNCH, "gdn_chunk_prefill_noalloc: no static scratch on the current device");
  return gdn_chunk_prefill_rows(q, q_stride, k, k_stride, v, v_stride, g, beta, beta_dtype, initial_state,
                                final_state, state_rows, n_rows, out, total_tokens, cu_seqlens, seq_chunk0,
                                total_chunks, nseq, seq_len, Hqk, Hv, D, in_dtype, use_qk_l2norm, ws_ptr,
                                GDN_NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" int gdn_conv_prefill_rows(const void* x, int64_t x_stride, const void* weight, const void* bias,
                                     const void* history, void* out, void* state_out, const int32_t* state_rows,
                                     int n_rows, int64_t total_tokens, const int32_t* cu_seqlens, int nseq,
                                     int seq_len, int C, int K, void* stream) {
  clear_error();
  GDN_REQUIRE(x && weight && out, "gdn_conv_prefill: null pointer");
  GDN_REQUIRE(C > 0 && K >= 1 && nseq >= 0 && total_tokens >= 0, "gdn_conv_prefill: bad sizes");
  GDN_SUPPORT(K <= 8, "gdn_conv_prefill: kernel size %d > 8", K);
  GDN_REQUIRE(cu_seqlens || (int64_t)nseq * seq_len == total_tokens,
              "gdn_conv_prefill: nseq*seq_len != total_tokens without cu_seqlens");
  GDN_REQUIRE(state_rows ? n_rows >= 0 : n_rows == nseq,
              "gdn_conv_prefill: without state_rows, n_rows must equal nseq");
  hipStream_t s = (hipStream_t)stream;
  if (total_tokens > 0) {
    GDN_REQUIRE(C % 8 == 0 && x_stride % 8 == 0 && aligned(x, 16) && aligned(out, 16),
                "gdn_conv_prefill: C and the row stride must be multiples of 8 with 16-byte aligned rows");
    GDN_REQUIRE(total_tokens < (1ll << 31), "gdn_conv_prefill: too many tokens");
    GDN_REQUIRE(aligned(weight, 16), "gdn_conv_prefill: weight must be 16-byte aligned");
    dim3 grid((unsigned)((C / 8 + 255) / 256), (unsigned)((total_tokens + kConvRun - 1) / kConvRun));
#define GDN_CONV_PREFILL(KK)                                                                                    \
  case KK:                                                                                                     \
    conv_prefill_kernel<KK><<<grid, 256, 0, s>>>((const uint16_t*)x, x_stride, (const uint16_t*)weight,          \
                                                 (const uint16_t*)bias, (const uint16_t*)history, state_rows,      \
                                                 n_rows, (uint16_t*)out, total_tokens, cu_seqlens, nseq, seq_len, \
                                                 C);                                                           \
    break;
    switch (K) {
      GDN_CONV_PREFILL(1)
      GDN_CONV_PREFILL(2)
      GDN_CONV_PREFILL(3)
      GDN_CONV_PREFILL(4)
      GDN_CONV_PREFILL(5)
      GDN_CONV_PREFILL(6)
      GDN_CONV_PREFILL(7)
      GDN_CONV_PREFILL(8)
    }
#undef GDN_CONV_PREFILL
    int rc = check_launch("gdn_conv_prefill");
    if (rc) return rc;
  }
  if (state_out && nseq > 0) {
    const int64_t n = (int64_t)nseq * C;
    conv_state_capture_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
        (const uint16_t*)x, x_stride, (const uint16_t*)history, state_rows, (uint16_t*)state_out, state_rows,
        n_rows, cu_seqlens, nseq, seq_len, C, K);
    return check_launch("gdn_conv_prefill(state)");
  }
  return GDN_OK;
}

extern "C" int gdn_conv_prefill(const void* x, int64_t x_stride, const void* weight, const void* bias,
                                const void* history, void* out, void* state_out, int64_t total_tokens,
                                const int32_t* cu_seqlens, int nseq, int seq_len, int C, int K, void* stream) {
  return gdn_conv_prefill_rows(x, x_stride, weight, bias, history, out, state_out, nullptr, nseq, total_tokens,
                               cu_seqlens, nseq, seq_len, C, K, stream);
}

extern "C" int gdn_gating(const void* a, const void* b, int64_t ab_stride, const float* A_log,
                          const float* dt_bias, void* beta_out, float* g_out, int64_t rows, int Hv, void* stream) {
  clear_error();
  GDN_REQUIRE(a && b && A_log && dt_bias && beta_out && g_out, "gdn_gating: null pointer");
  GDN_REQUIRE(rows >= 0 && Hv > 0, "gdn_gating: bad sizes");
  const int64_t n = rows * Hv;
  if (n == 0) return GDN_OK;
  gating_kernel<<<(unsigned)((n + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)a, (const uint16_t*)b, ab_stride, A_log, dt_bias, (uint16_t*)beta_out, g_out, rows, Hv);
  return check_launch("gdn_gating");
}
