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
// One workgroup (4 waves) owns (sequence, value head, BV-column tile of the state) and walks its
// chunks in order; the fp32 state tile S [128, BV] lives in MFMA accumulators across chunks.  Every
// product runs on v_mfma_f32_16x16x32_bf16 with fp32 accumulation; precision is spent where the
// fp32 state needs it: U and vn stay fp32 in accumulators, and the state update K^T (dec*vn) uses
// vn split into bf16 hi + lo (two MFMAs), so the running state never sees a bf16 rounding of its
// increment.  K, V and l2-normalised q, k are exact in bf16.  The 64x64 inverse is fp32 throughout:
// 16x16 diagonal blocks by forward substitution, block merges on v_mfma_f32_16x16x4_f32.
#include "gdn_device.h"
#include "gdn_internal.h"

namespace gdn {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

namespace pf {
constexpr int D = 128;          // head dim
constexpr int CH = 64;          // chunk length
constexpr int NT = 256;         // threads per workgroup (4 waves)
constexpr int LDK = D + 8;      // row pitch (bf16) of [*, 128] tiles
constexpr int LDT = CH + 8;     // row pitch (bf16) of [*, 64] tiles
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
// Same algorithm as src/gdn_chunk_fast.py:33-62: the four 16x16 diagonal blocks by the row
// recurrence (here: forward substitution, one column per lane group), then the merges
// [[A,0],[B X21 A, B]] for 32x32 and 64x64, on fp32 MFMA.  All 4 waves must call it (it holds
// barriers).  sY: 4 x 16 x 16 fp32 scratch.  Writes all of sT (upper blocks zero).
__device__ void unit_lower_inv64(const float* sX, float* sT, float* sY, int w, int lane) {
  using namespace pf;
  {  // diagonal block w: lane owns column c, rows g + 4m of the block
    const int c = lane & 15, g = lane >> 4;
    const float* Xb = sX + 16 * w * LDF + 16 * w;
    float acc[4] = {0.f, 0.f, 0.f, 0.f}, tv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int gj = j & 3, mj = j >> 2;
      const float mine = (j == c ? 1.0f : 0.0f) + acc[mj];
      const float tj = __shfl(mine, c + 16 * gj, kWave);
      if (g == gj) tv[mj] = tj;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int i = g + 4 * m;
        if (i > j) acc[m] += Xb[i * LDF + j] * tj;
      }
    }
    float* Tb = sT + 16 * w * LDF;
#pragma unroll
    for (int m = 0; m < 4; ++m) Tb[(g + 4 * m) * LDF + 16 * w + c] = tv[m];
    for (int col = 16 * (w + 1) + c; col < CH; col += 16)
#pragma unroll
      for (int m = 0; m < 4; ++m) Tb[(g + 4 * m) * LDF + col] = 0.f;
  }
  __syncthreads();
  // level 1: T10 = T11 (X10 T00), T32 = T33 (X32 T22)
  float* Y = sY + w * 256;
  if (w < 2) {
    const int b0 = 32 * w;  // block row/col offsets: rows b0+16.., cols b0..
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    acc = mm16_f32(sX + (b0 + 16) * LDF + b0, LDF, sT + b0 * LDF + b0, LDF, acc, lane);
    st16_f32(Y, 16, acc, lane);
  }
  __syncthreads();
  if (w < 2) {
    const int b0 = 32 * w;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    acc = mm16_f32(sT + (b0 + 16) * LDF + b0 + 16, LDF, Y, 16, acc, lane);
    st16_f32(sT + (b0 + 16) * LDF + b0, LDF, acc, lane);
  }
  __syncthreads();
  // level 2: Y20 = X20 T00 + X21 T10, Y30 = X30 T00 + X31 T10, Y21 = X21 T11, Y31 = X31 T11
  {
    const int ib = 2 + (w & 1), jb = w >> 1;  // wave 0: Y20, 1: Y30, 2: Y21, 3: Y31
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (jb == 0) acc = mm16_f32(sX + 16 * ib * LDF + 0, LDF, sT + 0 * LDF + 0, LDF, acc, lane);
    acc = mm16_f32(sX + 16 * ib * LDF + 16, LDF, sT + 16 * LDF + 16 * jb, LDF, acc, lane);
    st16_f32(Y, 16, acc, lane);
  }
  __syncthreads();
  {  // T20 = T22 Y20, T30 = T32 Y20 + T33 Y30, T21 = T22 Y21, T31 = T32 Y21 + T33 Y31
    const int ib = 2 + (w & 1), jb = w >> 1;
    const float* Ya = sY + (2 * jb) * 256;      // Y2jb
    const float* Yb = sY + (2 * jb + 1) * 256;  // Y3jb
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    acc = mm16_f32(sT + 16 * ib * LDF + 32, LDF, Ya, 16, acc, lane);
    if (ib == 3) acc = mm16_f32(sT + 48 * LDF + 48, LDF, Yb, 16, acc, lane);
    st16_f32(sT + 16 * ib * LDF + 16 * jb, LDF, acc, lane);
  }
  __syncthreads();
}

__global__ __launch_bounds__(pf::NT) void unit_lower_inv_kernel(const float* __restrict__ X, float* __restrict__ T) {
  using namespace pf;
  __shared__ float sX[CH * LDF], sT[CH * LDF], sY[4 * 256];
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const float* Xm = X + (int64_t)blockIdx.x * CH * CH;
  for (int i = t; i < CH * CH; i += NT) sX[(i / CH) * LDF + (i % CH)] = Xm[i];
  __syncthreads();
  unit_lower_inv64(sX, sT, sY, w, lane);
  float* Tm = T + (int64_t)blockIdx.x * CH * CH;
  for (int i = t; i < CH * CH; i += NT) Tm[i] = sT[(i / CH) * LDF + (i % CH)];
}

// ============================================================================================
// Fused chunked prefill.
// ============================================================================================
template <int BV>
struct PrefillSmem {
  uint16_t K[pf::CH * pf::LDK];     // K chunk, row-major (token, feature)
  uint16_t KT[pf::D * pf::LDT];     // K chunk transposed (feature, token)
  uint16_t VT[BV * pf::LDT];        // V tile transposed (column, token)
  uint16_t QK[pf::CH * pf::LDT];    // scale * q.k e^{Gi-Gj}, i >= j
  uint16_t ST[BV * pf::LDK];        // bf16 copy of the state tile, transposed (column, feature)
  union {
    struct {
      float X[pf::CH * pf::LDF];
      float T[pf::CH * pf::LDF];
      float Y[4 * 256];
    } inv;
    struct {
      uint16_t W[pf::CH * pf::LDK];   // W rows (token, feature)
      uint16_t VN[BV * pf::LDT];      // bf16(vn), transposed (column, token)
      uint16_t VSH[BV * pf::LDT];     // hi of dec*vn, transposed
      uint16_t VSL[BV * pf::LDT];     // lo of dec*vn, transposed
    } upd;
  } u;
  float G[pf::CH], EG[pf::CH], B[pf::CH], DEC[pf::CH];
  float GL;
};

// Register-staged chunk inputs (prefetched one chunk ahead).
template <int BV>
struct ChunkRegs {
  static constexpr int NV = BV * pf::CH / 8 / pf::NT;  // 16-byte V pieces per thread
  u16x8 k[4];
  u16x8 q[4];
  u16x8 v[NV > 0 ? NV : 1];
  float g, beta;
};

struct SeqInfo {
  int64_t t0;  // first packed token of the sequence
  int L;       // its length
};

template <int BV, typename BetaT>
__device__ __forceinline__ void load_chunk(ChunkRegs<BV>& r, const uint16_t* q, int64_t qs, const uint16_t* k,
                                           int64_t ks, const uint16_t* v, int64_t vs, const float* g,
                                           const BetaT* beta, SeqInfo si, int c, int h, int hk, int Hv, int vcol0,
                                           int t) {
  using namespace pf;
  const int base = c * CH;
  const u16x8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  // K: rows t/16 + 16i, features 8*(t%16)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = (t >> 4) + 16 * i;
    const int tok = base + row;
    r.k[i] = tok < si.L ? *reinterpret_cast<const u16x8*>(k + (si.t0 + tok) * ks + (int64_t)hk * D + 8 * (t & 15))
                        : zero;
  }
  // Q in MFMA A-fragment order of this wave: row 16w + l%16, features 8(l/16) + 32 ks
  {
    const int w = t >> 6, lane = t & 63;
    const int tok = base + 16 * w + (lane & 15);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      r.q[s] = tok < si.L ? *reinterpret_cast<const u16x8*>(q + (si.t0 + tok) * qs + (int64_t)hk * D +
                                                            32 * s + 8 * (lane >> 4))
                          : zero;
  }
  // V tile: BV columns / 8 pieces per row
  constexpr int PPR = BV / 8;
#pragma unroll
  for (int i = 0; i < ChunkRegs<BV>::NV; ++i) {
    const int idx = t + NT * i;
    const int row = idx / PPR, pc = idx % PPR;
    const int tok = base + row;
    r.v[i] = tok < si.L ? *reinterpret_cast<const u16x8*>(v + (si.t0 + tok) * vs + (int64_t)h * D + vcol0 + 8 * pc)
                        : zero;
  }
  if (t < CH) {
    const int tok = base + t;
    r.g = tok < si.L ? g[(si.t0 + tok) * Hv + h] : 0.f;
    r.beta = tok < si.L ? Elem<BetaT>::load(beta + (si.t0 + tok) * Hv + h) : 0.f;
  }
}

// l2norm (bf16 op rounding) of 8 values whose row is spread over the lanes selected by `mask`.
__device__ __forceinline__ void l2norm8(u16x8& x, int xor_lo, int xor_hi) {
  float f[8], ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    f[e] = bf2f(x[e]);
    ss += rbf(f[e] * f[e]);
  }
  for (int o = xor_lo; o <= xor_hi; o <<= 1) ss += __shfl_xor(ss, o, kWave);
  const float s = rbf(rbf(ss) + 1e-6f);
  const float inv = rbf(rsqrt_f(s));
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = f2bf(f[e] * inv);
}

template <int BV>
__device__ __forceinline__ void commit_chunk(PrefillSmem<BV>& sm, ChunkRegs<BV>& r, bf16x8* qf, bool use_l2,
                                             int t) {
  using namespace pf;
  const int w = t >> 6, lane = t & 63;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (use_l2) l2norm8(r.k[i], 1, 8);  // a K row is held by 16 consecutive lanes
    const int row = (t >> 4) + 16 * i, f0 = 8 * (t & 15);
    *reinterpret_cast<u16x8*>(&sm.K[row * LDK + f0]) = r.k[i];
#pragma unroll
    for (int e = 0; e < 8; ++e) sm.KT[(f0 + e) * LDT + row] = r.k[i][e];
  }
  if (use_l2) {
    // a Q row is held by the 4 lanes l%16 == const of this wave, 4 pieces each
    float ss = 0.f;
    float f[4][8];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        f[s][e] = bf2f(r.q[s][e]);
        ss += rbf(f[s][e] * f[s][e]);
      }
    ss += __shfl_xor(ss, 16, kWave);
    ss += __shfl_xor(ss, 32, kWave);
    const float inv = rbf(rsqrt_f(rbf(rbf(ss) + 1e-6f)));
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) r.q[s][e] = f2bf(f[s][e] * inv);
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) qf[s] = __builtin_bit_cast(bf16x8, r.q[s]);
  constexpr int PPR = BV / 8;
#pragma unroll
  for (int i = 0; i < ChunkRegs<BV>::NV; ++i) {
    const int idx = t + NT * i;
    const int row = idx / PPR, pc = idx % PPR;
#pragma unroll
    for (int e = 0; e < 8; ++e) sm.VT[(8 * pc + e) * LDT + row] = r.v[i][e];
  }
  if (w == 0) {  // cumulative decay within the chunk
    float G = r.g;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float up = __shfl_up(G, o, kWave);
      if (lane >= o) G += up;
    }
    const float gl = __shfl(G, 63, kWave);
    sm.G[lane] = G;
    sm.EG[lane] = expf(G);
    sm.B[lane] = r.beta;
    sm.DEC[lane] = expf(gl - G);
    if (lane == 0) sm.GL = expf(gl);
  }
}

template <int BV, typename BetaT>
__global__ __launch_bounds__(pf::NT) void chunk_prefill_kernel(
    const uint16_t* __restrict__ q, int64_t qs, const uint16_t* __restrict__ k, int64_t ks,
    const uint16_t* __restrict__ v, int64_t vs, const float* __restrict__ g, const BetaT* __restrict__ beta,
    const float* __restrict__ init, float* __restrict__ final_state, uint16_t* __restrict__ out,
    const int32_t* __restrict__ cu, int seq_len, int Hqk, int Hv, int use_l2) {
  using namespace pf;
  constexpr int NCB = BV / 16;  // 16-wide column blocks of the tile
  constexpr int NTILE = D / BV;
  __shared__ PrefillSmem<BV> sm;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  int bid = blockIdx.x;
  const int vt = bid % NTILE;
  bid /= NTILE;
  const int h = bid % Hv, seq = bid / Hv;
  const int hk = h / (Hv / Hqk);
  const int vcol0 = vt * BV;
  SeqInfo si;
  if (cu) {
    si.t0 = cu[seq];
    si.L = cu[seq + 1] - cu[seq];
  } else {
    si.t0 = (int64_t)seq * seq_len;
    si.L = seq_len;
  }
  const int nch = (si.L + CH - 1) / CH;
  const int64_t sbase = ((int64_t)seq * Hv + h) * D * D + vcol0;

  // state tile: accS[rb][cb] holds S[16(2w+rb) + 4(l/16) + r][vcol0 + 16cb + l%16]
  f32x4 accS[2][NCB];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = 16 * (2 * w + rb) + 4 * (lane >> 4) + r;
        accS[rb][cb][r] = init ? init[sbase + (int64_t)d * D + 16 * cb + (lane & 15)] : 0.f;
      }
      u16x4 pk;
#pragma unroll
      for (int r = 0; r < 4; ++r) pk[r] = f2bf(accS[rb][cb][r]);
      *reinterpret_cast<u16x4*>(&sm.ST[(16 * cb + (lane & 15)) * LDK + 16 * (2 * w + rb) + 4 * (lane >> 4)]) = pk;
    }

  ChunkRegs<BV> cr;
  if (nch > 0) load_chunk<BV, BetaT>(cr, q, qs, k, ks, v, vs, g, beta, si, 0, h, hk, Hv, vcol0, t);
  bf16x8 qf[4];

  for (int c = 0; c < nch; ++c) {
    // ---- 1. chunk inputs into LDS (l2norm, transposes, decay scan); prefetch the next chunk
    commit_chunk<BV>(sm, cr, qf, use_l2 != 0, t);
    __syncthreads();
    if (c + 1 < nch) load_chunk<BV, BetaT>(cr, q, qs, k, ks, v, vs, g, beta, si, c + 1, h, hk, Hv, vcol0, t);

    // ---- 2. A = K K^T and QK = Q K^T for this wave's 16 rows (blocks cb <= w)
    {
      f32x4 accA[4], accQ[4];
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) accA[cb] = accQ[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 ak = frag(sm.K, LDK, 16 * w, 32 * s, lane);
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
          if (cb <= w) {
            const bf16x8 b = frag(sm.K, LDK, 16 * cb, 32 * s, lane);
            accA[cb] = mma(ak, b, accA[cb]);
            accQ[cb] = mma(qf[s], b, accQ[cb]);
          }
        }
      }
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * w + 4 * (lane >> 4) + r, jj = 16 * cb + (lane & 15);
          float x = 0.f, qk = 0.f;
          if (cb <= w && i >= jj) {
            const float dec = expf(sm.G[i] - sm.G[jj]);
            qk = kScale * accQ[cb][r] * dec;
            if (i > jj) x = -sm.B[i] * accA[cb][r] * dec;
          }
          sm.u.inv.X[i * LDF + jj] = x;
          sm.QK[i * LDT + jj] = f2bf(qk);
        }
    }
    __syncthreads();

    // ---- 3. T = (I - X)^{-1}
    unit_lower_inv64(sm.u.inv.X, sm.u.inv.T, sm.u.inv.Y, w, lane);

    // ---- 4. W = T diag(beta e^G) K (64x128) and U = T diag(beta) V (64xBV) for this wave's rows
    f32x4 accW[8], accU[NCB];
    {
      bf16x8 tb[2], tbe[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const float* trow = &sm.u.inv.T[(16 * w + (lane & 15)) * LDF + 32 * s + 8 * (lane >> 4)];
        float a[8], b[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int col = 32 * s + 8 * (lane >> 4) + e;
          a[e] = trow[e] * sm.B[col];
          b[e] = a[e] * sm.EG[col];
        }
        tb[s] = pack8(a);
        tbe[s] = pack8(b);
      }
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) {
        accW[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 2; ++s) accW[cb] = mma(tbe[s], frag(sm.KT, LDT, 16 * cb, 32 * s, lane), accW[cb]);
      }
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        accU[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 2; ++s) accU[cb] = mma(tb[s], frag(sm.VT, LDT, 16 * cb, 32 * s, lane), accU[cb]);
      }
    }
    __syncthreads();  // T no longer read; its space becomes W / vn
#pragma unroll
    for (int cb = 0; cb < 8; ++cb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sm.u.upd.W[(16 * w + 4 * (lane >> 4) + r) * LDK + 16 * cb + (lane & 15)] = f2bf(accW[cb][r]);
    __syncthreads();

    // ---- 5. vn = U - W S (fp32 accumulators), published as bf16(vn) and dec*vn = hi + lo
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8 a = frag_neg(sm.u.upd.W, LDK, 16 * w, 32 * s, lane);
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) accU[cb] = mma(a, frag(sm.ST, LDK, 16 * cb, 32 * s, lane), accU[cb]);
    }
    {
      const int s0 = 16 * w + 4 * (lane >> 4);
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        u16x4 vo, vh, vl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float vn = accU[cb][r];
          const float vsc = vn * sm.DEC[s0 + r];
          vo[r] = f2bf(vn);
          vh[r] = f2bf(vsc);
          vl[r] = f2bf(vsc - bf2f(vh[r]));
        }
        const int off = (16 * cb + (lane & 15)) * LDT + s0;
        *reinterpret_cast<u16x4*>(&sm.u.upd.VN[off]) = vo;
        *reinterpret_cast<u16x4*>(&sm.u.upd.VSH[off]) = vh;
        *reinterpret_cast<u16x4*>(&sm.u.upd.VSL[off]) = vl;
      }
    }
    __syncthreads();

    // ---- 6. o = diag(scale e^G) Q S + QK vn for this wave's 16 rows
    {
      bf16x8 qg[4];
      const float f = kScale * sm.EG[16 * w + (lane & 15)];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u16x8 u = __builtin_bit_cast(u16x8, qf[s]);
        float a[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = bf2f(u[e]) * f;
        qg[s] = pack8(a);
      }
      f32x4 accO[NCB];
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        accO[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) accO[cb] = mma(qg[s], frag(sm.ST, LDK, 16 * cb, 32 * s, lane), accO[cb]);
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (s == 0 || w >= 2) {
          const bf16x8 a = frag(sm.QK, LDT, 16 * w, 32 * s, lane);
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) accO[cb] = mma(a, frag(sm.u.upd.VN, LDT, 16 * cb, 32 * s, lane), accO[cb]);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * w + 4 * (lane >> 4) + r;
        const int tok = c * CH + row;
        if (tok < si.L) {
          uint16_t* op = out + ((si.t0 + tok) * Hv + h) * D + vcol0 + (lane & 15);
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) op[16 * cb] = f2bf(accO[cb][r]);
        }
      }
    }
    __syncthreads();  // all reads of the old state copy are done

    // ---- 7. S' = e^{G_last} S + K^T (dec vn), with dec vn = hi + lo
    {
      const float gl = sm.GL;
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) accS[rb][cb] *= gl;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const bf16x8 a = frag(sm.KT, LDT, 16 * (2 * w + rb), 32 * s, lane);
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) {
            accS[rb][cb] = mma(a, frag(sm.u.upd.VSH, LDT, 16 * cb, 32 * s, lane), accS[rb][cb]);
            accS[rb][cb] = mma(a, frag(sm.u.upd.VSL, LDT, 16 * cb, 32 * s, lane), accS[rb][cb]);
          }
        }
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
          u16x4 pk;
#pragma unroll
          for (int r = 0; r < 4; ++r) pk[r] = f2bf(accS[rb][cb][r]);
          *reinterpret_cast<u16x4*>(&sm.ST[(16 * cb + (lane & 15)) * LDK + 16 * (2 * w + rb) + 4 * (lane >> 4)]) = pk;
        }
      }
    }
    __syncthreads();
  }

  if (final_state) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d = 16 * (2 * w + rb) + 4 * (lane >> 4) + r;
          final_state[sbase + (int64_t)d * D + 16 * cb + (lane & 15)] = accS[rb][cb][r];
        }
  }
}

// ============================================================================================
// Causal depthwise conv prefill + SiLU with decode-state capture.
// ============================================================================================
// One thread per (channel, block of TB packed tokens).  x_t for t < 0 (before a sequence) comes
// from `history` [n_seq, C, K] (x_{-j} = history[K - j]) or is zero.  Numerics of F.conv1d on bf16:
// fp32 accumulation of the K products (+ bias), one bf16 rounding, SiLU, bf16.
constexpr int kConvTB = 32;

__device__ __forceinline__ int find_seq(const int32_t* cu, int nseq, int64_t p) {
  int lo = 0, hi = nseq - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= p) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

__global__ __launch_bounds__(256) void conv_prefill_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                                           const uint16_t* __restrict__ weight,
                                                           const uint16_t* __restrict__ bias,
                                                           const uint16_t* __restrict__ history,
                                                           uint16_t* __restrict__ out, uint16_t* __restrict__ state,
                                                           int64_t total, const int32_t* __restrict__ cu, int nseq,
                                                           int seq_len, int C, int K) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t p0 = (int64_t)blockIdx.y * kConvTB;
  if (c >= C || p0 >= total) return;
  float w[8];
  for (int i = 0; i < K; ++i) w[i] = bf2f(weight[(int64_t)c * K + i]);
  const float b = bias ? bf2f(bias[c]) : 0.f;
  auto seq_start = [&](int s) -> int64_t { return cu ? (int64_t)cu[s] : (int64_t)s * seq_len; };
  int s = cu ? find_seq(cu, nseq, p0) : (int)(p0 / seq_len);
  int64_t s_lo = seq_start(s), s_hi = seq_start(s + 1);
  // window: win[K-1] is the newest input; prime with the K-1 inputs before p0
  float win[8];
  auto input_at = [&](int64_t p) -> float {  // p may precede s_lo
    if (p >= s_lo) return bf2f(x[p * x_stride + c]);
    const int64_t back = s_lo - p;  // 1..K
    if (history && back <= K) return bf2f(history[((int64_t)s * C + c) * K + (K - back)]);
    return 0.f;
  };
  for (int i = 0; i < K - 1; ++i) win[i + 1] = input_at(p0 - (K - 1) + i);
  const int64_t pend = p0 + kConvTB < total ? p0 + kConvTB : total;
  for (int64_t p = p0; p < pend; ++p) {
    while (p >= s_hi) {  // next (non-empty) sequence: re-prime the window from its history
      ++s;
      s_lo = seq_start(s);
      s_hi = seq_start(s + 1);
      for (int i = 0; i < K - 1; ++i) win[i + 1] = input_at(p - (K - 1) + i);
    }
    for (int i = 0; i < K - 1; ++i) win[i] = win[i + 1];
    win[K - 1] = bf2f(x[p * x_stride + c]);
    float acc = b;
    for (int i = 0; i < K; ++i) acc += win[i] * w[i];
    out[p * (int64_t)C + c] = f2bf(silu_f(rbf(acc)));
    if (p == s_hi - 1 && state) {  // last token of the sequence: capture the last K inputs
      for (int i = 0; i < K; ++i) state[((int64_t)s * C + c) * K + i] = f2bf(win[i]);
    }
  }
}

// Sequences shorter than K keep part of their history; empty sequences keep all of it.  The main
// kernel writes the state of every non-empty sequence (its window already holds the history);
// this pass fills the state of empty ones.
__global__ void conv_prefill_empty_kernel(const uint16_t* __restrict__ history, uint16_t* __restrict__ state,
                                          const int32_t* __restrict__ cu, int nseq, int seq_len, int C, int K) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)nseq * C) return;
  const int s = (int)(i / C);
  const int L = cu ? cu[s + 1] - cu[s] : seq_len;
  if (L != 0) return;
  for (int j = 0; j < K; ++j) state[i * K + j] = history ? history[i * K + j] : (uint16_t)0;
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

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_unit_lower_inv(const float* X, float* T, int64_t batch, int n, void* stream) {
  clear_error();
  GDN_REQUIRE(X && T, "gdn_unit_lower_inv: null pointer");
  GDN_SUPPORT(n == 64, "gdn_unit_lower_inv: only 64x64 blocks are supported (got %d)", n);
  GDN_REQUIRE(batch >= 0 && batch < (1ll << 31), "gdn_unit_lower_inv: bad batch %lld", (long long)batch);
  if (batch == 0) return GDN_OK;
  unit_lower_inv_kernel<<<(unsigned)batch, pf::NT, 0, (hipStream_t)stream>>>(X, T);
  return check_launch("gdn_unit_lower_inv");
}

extern "C" int gdn_chunk_prefill(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                                 const void* v, int64_t v_stride, const float* g, const void* beta,
                                 int beta_dtype, const float* initial_state, float* final_state, void* out,
                                 int64_t total_tokens, const int32_t* cu_seqlens, int nseq, int seq_len,
                                 int Hqk, int Hv, int D, int in_dtype, int use_qk_l2norm, void* stream) {
  clear_error();
  GDN_REQUIRE(q && k && v && g && beta && out, "gdn_chunk_prefill: null input/output pointer");
  GDN_SUPPORT(D == pf::D, "gdn_chunk_prefill: head dim %d unsupported (needs %d)", D, pf::D);
  GDN_SUPPORT(in_dtype == GDN_BF16, "gdn_chunk_prefill: q/k/v must be bfloat16 (MFMA operands)");
  GDN_REQUIRE(beta_dtype == GDN_F32 || beta_dtype == GDN_BF16, "gdn_chunk_prefill: bad beta dtype");
  GDN_REQUIRE(Hqk > 0 && Hv > 0 && Hv % Hqk == 0, "gdn_chunk_prefill: bad heads Hqk=%d Hv=%d", Hqk, Hv);
  GDN_REQUIRE(nseq >= 0 && total_tokens >= 0, "gdn_chunk_prefill: negative sizes");
  GDN_REQUIRE(cu_seqlens || (int64_t)nseq * seq_len == total_tokens,
              "gdn_chunk_prefill: nseq*seq_len != total_tokens without cu_seqlens");
  GDN_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && q_stride % 8 == 0 && k_stride % 8 == 0 &&
                  v_stride % 8 == 0,
              "gdn_chunk_prefill: q/k/v rows must be 16-byte aligned");
  if (nseq == 0) return GDN_OK;
  hipStream_t s = (hipStream_t)stream;
  // Column tile: enough workgroups to cover the chip when there are few (sequence, head) pairs.
  const int64_t pairs = (int64_t)nseq * Hv;
  const int BV = pairs >= 256 ? 64 : 32;
  const int64_t grid = pairs * (pf::D / BV);
  GDN_REQUIRE(grid < (1ll << 31), "gdn_chunk_prefill: grid too large");
#define GDN_CP_LAUNCH(BVV, BT)                                                                           \
  chunk_prefill_kernel<BVV, BT><<<(unsigned)grid, pf::NT, 0, s>>>(                                       \
      (const uint16_t*)q, q_stride, (const uint16_t*)k, k_stride, (const uint16_t*)v, v_stride, g,       \
      (const BT*)beta, initial_state, final_state, (uint16_t*)out, cu_seqlens, seq_len, Hqk, Hv, use_qk_l2norm)
  if (BV == 64) {
    if (beta_dtype == GDN_BF16) GDN_CP_LAUNCH(64, uint16_t);
    else GDN_CP_LAUNCH(64, float);
  } else {
    if (beta_dtype == GDN_BF16) GDN_CP_LAUNCH(32, uint16_t);
    else GDN_CP_LAUNCH(32, float);
  }
#undef GDN_CP_LAUNCH
  return check_launch("gdn_chunk_prefill");
}

extern "C" int gdn_conv_prefill(const void* x, int64_t x_stride, const void* weight, const void* bias,
                                const void* history, void* out, void* state_out, int64_t total_tokens,
                                const int32_t* cu_seqlens, int nseq, int seq_len, int C, int K, void* stream) {
  clear_error();
  GDN_REQUIRE(x && weight && out, "gdn_conv_prefill: null pointer");
  GDN_REQUIRE(C > 0 && K >= 1 && nseq >= 0 && total_tokens >= 0, "gdn_conv_prefill: bad sizes");
  GDN_SUPPORT(K <= 8, "gdn_conv_prefill: kernel size %d > 8", K);
  GDN_REQUIRE(cu_seqlens || (int64_t)nseq * seq_len == total_tokens,
              "gdn_conv_prefill: nseq*seq_len != total_tokens without cu_seqlens");
  hipStream_t s = (hipStream_t)stream;
  if (total_tokens > 0) {
    dim3 grid((C + 255) / 256, (unsigned)((total_tokens + kConvTB - 1) / kConvTB));
    conv_prefill_kernel<<<grid, 256, 0, s>>>((const uint16_t*)x, x_stride, (const uint16_t*)weight,
                                             (const uint16_t*)bias, (const uint16_t*)history, (uint16_t*)out,
                                             (uint16_t*)state_out, total_tokens, cu_seqlens, nseq, seq_len, C, K);
    int rc = check_launch("gdn_conv_prefill");
    if (rc) return rc;
  }
  if (state_out && nseq > 0) {
    const int64_t n = (int64_t)nseq * C;
    conv_prefill_empty_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
        (const uint16_t*)history, (uint16_t*)state_out, cu_seqlens, nseq, seq_len, C, K);
    return check_launch("gdn_conv_prefill(empty)");
  }
  return GDN_OK;
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
