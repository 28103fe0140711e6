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
// Same blocking as src/gdn_chunk_fast.py:33-62 -- the four 16x16 diagonal blocks first, then the
// merges [[A,0],[B X21 A, B]] for 32x32 and 64x64 -- all on fp32 MFMA.  A diagonal block is
// inverted as (I+X)(I+X^2)(I+X^4)(I+X^8) (exact for nilpotent X, X^16 = 0) instead of the
// reference's 16-step row recurrence: six dependent products instead of sixteen dependent steps;
// with |X_ij| <= 1 (l2-normalised k, beta <= 1, decay <= 1) the powers of a 16x16 block stay far
// from fp32 overflow (the reference avoids powers of the whole 64x64 block, which can overflow).
// All 4 waves must call it (it holds barriers).  sY: 4 x 16 x 16 fp32 scratch.  Writes all of sT
// (upper blocks zero).
__device__ void unit_lower_inv64(const float* sX, float* sT, float* sY, int w, int lane) {
  using namespace pf;
  {  // diagonal block w: T = (I+X)(I+X^2)(I+X^4)(I+X^8) (X^16 = 0), six fp32 MFMA products
    const int c = lane & 15, g = lane >> 4;
    const float* Xb = sX + 16 * w * LDF + 16 * w;
    float* Tb = sT + 16 * w * LDF + 16 * w;
    float* P = sY + w * 256;  // wave-private 16x16 scratch (pitch 16)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 4 * g + r;
      Tb[i * LDF + c] = Xb[i * LDF + c] + (i == c ? 1.0f : 0.0f);
    }
    const float* Pin = Xb;
    int ldp = LDF;
#pragma unroll
    for (int step = 0; step < 3; ++step) {
      f32x4 p2 = mm16_f32(Pin, ldp, Pin, ldp, f32x4{0.f, 0.f, 0.f, 0.f}, lane);  // X^(2^(step+1))
      st16_f32(P, 16, p2, lane);
      __builtin_amdgcn_wave_barrier();
      f32x4 tp = mm16_f32(Tb, LDF, P, 16, f32x4{0.f, 0.f, 0.f, 0.f}, lane);     // T X^(2^(step+1))
#pragma unroll
      for (int r = 0; r < 4; ++r) Tb[(4 * g + r) * LDF + c] += tp[r];
      __builtin_amdgcn_wave_barrier();
      Pin = P;
      ldp = 16;
    }
    float* Trow = sT + 16 * w * LDF;
    for (int col = 16 * (w + 1) + c; col < CH; col += 16)
#pragma unroll
      for (int r = 0; r < 4; ++r) Trow[(4 * g + r) * LDF + col] = 0.f;
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
  for (int i = t; i < CH * CH; i += NT) sX[(i / CH) * LDF + (i % CH)] = (i / CH) > (i % CH) ? Xm[i] : 0.f;
  __syncthreads();
  unit_lower_inv64(sX, sT, sY, w, lane);
  float* Tm = T + (int64_t)blockIdx.x * CH * CH;
  for (int i = t; i < CH * CH; i += NT) Tm[i] = sT[(i / CH) * LDF + (i % CH)];
}

// ============================================================================================
// Chunked prefill, part 1: chunk-local quantities (parallel over every (chunk, value head)).
// ============================================================================================
// Workspace record per (chunk slot, value head), consumed by the state kernel in exactly the
// layouts it uses (so its per-chunk staging is plain copies):
//   W   [64][128] bf16 = T diag(beta e^G) K          QK [64][64] bf16 = scale q.k e^{Gi-Gj}, i>=j
//   Qg  [64][128] bf16 = scale e^{G_t} q_t           KT [128][64] bf16 = K^T (l2-normalised keys)
//   U   fp32 = T diag(beta) V in MFMA accumulator tiles: [col block 8][token block 4][lane 64][4]
//       (lane l of a tile holds rows 4(l/16)..+3 of column l%16)
//   DEC [64] fp32 = e^{G_last - G_t}                 GL fp32 = e^{G_last}
namespace ws {
constexpr int W = 0;                           // byte offsets inside one record
constexpr int QK = W + pf::CH * pf::D * 2;     // 16384
constexpr int QG = QK + pf::CH * pf::CH * 2;   // 24576
constexpr int KT = QG + pf::CH * pf::D * 2;    // 40960
constexpr int U = KT + pf::D * pf::CH * 2;     // 57344
constexpr int DEC = U + pf::CH * pf::D * 4;    // 90112
constexpr int GL = DEC + pf::CH * 4;           // 90368
constexpr int BYTES = 90624;                   // record size (multiple of 256)
}  // namespace ws

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
__device__ __forceinline__ void load_rows4(u16x8* x, const uint16_t* base, int64_t stride, int64_t t0, int len,
                                           int tq, int f0) {
  const u16x8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * tq + i;
    x[i] = row < len ? *reinterpret_cast<const u16x8*>(base + (t0 + row) * stride + f0) : zero;
  }
}
__device__ __forceinline__ void l2norm_rows4(u16x8* x) {
  float ss[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ss[i] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = bf2f(x[i][e]);
      ss[i] += rbf(f * f);
    }
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1)
#pragma unroll
    for (int i = 0; i < 4; ++i) ss[i] += __shfl_xor(ss[i], o, kWave);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float inv = rbf(rsqrt_f(rbf(rbf(ss[i]) + 1e-6f)));
#pragma unroll
    for (int e = 0; e < 8; ++e) x[i][e] = f2bf(bf2f(x[i][e]) * inv);
  }
}
// Write 4 rows x 8 features transposed: dst[(f0+e)*ld + 4tq .. +3] = x[0..3][e] (8-byte stores).
__device__ __forceinline__ void store_transposed4(uint16_t* dst, int ld, const u16x8* x, int tq, int f0) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const u16x4 v = {x[0][e], x[1][e], x[2][e], x[3][e]};
    *reinterpret_cast<u16x4*>(dst + (f0 + e) * ld + 4 * tq) = v;
  }
}

struct LocalSmem {
  union {
    uint16_t K[pf::CH * pf::LDK];   // K chunk, row-major (token, feature): A/B of K K^T, B of Q K^T
    uint16_t W[pf::CH * pf::LDK];   // later: W staged for coalesced stores
  } a;
  uint16_t KT[pf::D * pf::LDT];     // K chunk transposed (feature, token): B of W = T' K
  float X[pf::CH * pf::LDF];
  float T[pf::CH * pf::LDF];
  float Y[4 * 256];
  float G[pf::CH], EG[pf::CH], B[pf::CH];
};

template <typename BetaT>
__global__ __launch_bounds__(pf::NT, 2) void chunk_local_kernel(
    const uint16_t* __restrict__ q, int64_t qs, const uint16_t* __restrict__ k, int64_t ks,
    const uint16_t* __restrict__ v, int64_t vs,
    const float* __restrict__ g, const BetaT* __restrict__ beta, const int32_t* __restrict__ cu,
    const int32_t* __restrict__ seq_chunk0, int nseq, int seq_len, int Hqk, int Hv, int use_l2,
    uint8_t* __restrict__ work) {
  using namespace pf;
  __shared__ LocalSmem sm;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int slot = blockIdx.x, h = blockIdx.y;
  const int hk = h / (Hv / Hqk);
  const ChunkPos cp = chunk_pos(slot, cu, seq_chunk0, nseq, seq_len);
  uint8_t* rec = work + ((int64_t)slot * Hv + h) * ws::BYTES;

  // K: thread (tq, fb) loads rows 4tq.. x features 8fb..; row-major and transposed copies
  {
    const int tq = t >> 4, fb = t & 15;
    u16x8 x[4];
    load_rows4(x, k + (int64_t)hk * D, ks, cp.t0, cp.len, tq, 8 * fb);
    if (use_l2) l2norm_rows4(x);
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u16x8*>(&sm.a.K[(4 * tq + i) * LDK + 8 * fb]) = x[i];
    store_transposed4(sm.KT, LDT, x, tq, 8 * fb);
  }
  // V rows 4tq.. x columns 8fb.. stay in registers until the inverse has freed the X buffer
  u16x8 vreg[4];
  load_rows4(vreg, v + (int64_t)h * D, vs, cp.t0, cp.len, t >> 4, 8 * (t & 15));
  // Q in A-fragment order of this wave (rows 16w + l%16, features 8(l/16) + 32s)
  bf16x8 qf[4];
  {
    const u16x8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
    const int row = 16 * w + (lane & 15);
    u16x8 r[4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
      r[s] = row < cp.len ? *reinterpret_cast<const u16x8*>(q + (cp.t0 + row) * qs + (int64_t)hk * D + 32 * s +
                                                            8 * (lane >> 4))
                          : zero;
    if (use_l2) {
      float ss = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = bf2f(r[s][e]);
          ss += rbf(f * f);
        }
      ss += __shfl_xor(ss, 16, kWave);
      ss += __shfl_xor(ss, 32, kWave);
      const float inv = rbf(rsqrt_f(rbf(rbf(ss) + 1e-6f)));
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) r[s][e] = f2bf(bf2f(r[s][e]) * inv);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = __builtin_bit_cast(bf16x8, r[s]);
  }
  if (w == 0) {  // cumulative decay within the chunk (padding: g = 0, beta = 0)
    const bool valid = lane < cp.len;
    float G = valid ? g[(cp.t0 + lane) * Hv + h] : 0.f;
    const float bt = valid ? Elem<BetaT>::load(beta + (cp.t0 + lane) * Hv + h) : 0.f;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float up = __shfl_up(G, o, kWave);
      if (lane >= o) G += up;
    }
    const float gl = __shfl(G, 63, kWave);
    const float eg = expf(G), dec = expf(gl - G);
    sm.G[lane] = G;
    sm.EG[lane] = eg;
    sm.B[lane] = bt;
    reinterpret_cast<float*>(rec + ws::DEC)[lane] = dec;
    if (lane == 0) reinterpret_cast<float*>(rec + ws::GL)[0] = expf(gl);
  }
  __syncthreads();

  // Qg = scale e^{G_t} q_t -> workspace (this wave's rows, straight from the A fragments);
  // K^T -> workspace (from LDS)
  {
    const int row = 16 * w + (lane & 15);
    const float f = kScale * sm.EG[row];
    uint16_t* qg = reinterpret_cast<uint16_t*>(rec + ws::QG) + row * D + 8 * (lane >> 4);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u16x8 u = __builtin_bit_cast(u16x8, qf[s]);
      u16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = f2bf(bf2f(u[e]) * f);
      *reinterpret_cast<u16x8*>(qg + 32 * s) = o;
    }
    uint16_t* kt = reinterpret_cast<uint16_t*>(rec + ws::KT);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = t + NT * i;  // 1024 pieces of 16 bytes: row idx/8, piece idx%8
      *reinterpret_cast<u16x8*>(kt + (idx >> 3) * CH + 8 * (idx & 7)) =
          *reinterpret_cast<const u16x8*>(&sm.KT[(idx >> 3) * LDT + 8 * (idx & 7)]);
    }
  }
  // A = K K^T and QK = Q K^T for this wave's 16 rows; X -> LDS, QK -> workspace
  {
    f32x4 accA[4], accQ[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) accA[cb] = accQ[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8 ak = frag(sm.a.K, LDK, 16 * w, 32 * s, lane);
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        if (cb <= w) {
          const bf16x8 b = frag(sm.a.K, LDK, 16 * cb, 32 * s, lane);
          accA[cb] = mma(ak, b, accA[cb]);
          accQ[cb] = mma(qf[s], b, accQ[cb]);
        }
      }
    }
    uint16_t* qk = reinterpret_cast<uint16_t*>(rec + ws::QK);
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * w + 4 * (lane >> 4) + r, jj = 16 * cb + (lane & 15);
        float x = 0.f, v = 0.f;
        if (cb <= w && i >= jj) {
          const float dec = expf(sm.G[i] - sm.G[jj]);
          v = kScale * accQ[cb][r] * dec;
          if (i > jj) x = -sm.B[i] * accA[cb][r] * dec;
        }
        sm.X[i * LDF + jj] = x;
        qk[i * CH + jj] = f2bf(v);
      }
  }
  __syncthreads();

  unit_lower_inv64(sm.X, sm.T, sm.Y, w, lane);

  // W = T diag(beta e^G) K and U = T diag(beta) V for this wave's rows
  f32x4 accW[8];
  {
    bf16x8 tbe[2], tb[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float* trow = &sm.T[(16 * w + (lane & 15)) * LDF + 32 * s + 8 * (lane >> 4)];
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
    // V^T into the X buffer (dead after the inverse; V^T is 1 KiB larger and runs into T, whose
    // reads all finished above -- hence the barrier); U tiles go straight to the workspace in
    // accumulator layout
    static_assert(pf::D * pf::LDT * 2 <= 2 * pf::CH * pf::LDF * 4, "V^T must fit in X and T");
    uint16_t* VT = reinterpret_cast<uint16_t*>(sm.X);
    __syncthreads();
    store_transposed4(VT, LDT, vreg, t >> 4, 8 * (t & 15));
    __syncthreads();
    f32x4* ur = reinterpret_cast<f32x4*>(rec + ws::U);
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
      f32x4 u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 2; ++s) u = mma(tb[s], frag(VT, LDT, 16 * cb, 32 * s, lane), u);
      ur[(cb * 4 + w) * 64 + lane] = u;
    }
  }
  // stage W in LDS (the K buffer is free after the K K^T products) and store it coalesced
#pragma unroll
  for (int cb = 0; cb < 8; ++cb)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sm.a.W[(16 * w + 4 * (lane >> 4) + r) * LDK + 16 * cb + (lane & 15)] = f2bf(accW[cb][r]);
  __syncthreads();
  {
    uint16_t* wd = reinterpret_cast<uint16_t*>(rec + ws::W);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = t + NT * i;  // 1024 pieces of 16 bytes
      const int row = idx >> 4, pc = idx & 15;
      *reinterpret_cast<u16x8*>(wd + row * D + 8 * pc) = *reinterpret_cast<const u16x8*>(&sm.a.W[row * LDK + 8 * pc]);
    }
  }
}

// ============================================================================================
// Chunked prefill, part 2: the inter-chunk state recurrence.
// ============================================================================================
// One workgroup = 4 waves = 64 state columns of one (sequence, value head); wave w owns columns
// 16w..16w+15 over all 128 rows and all 64 tokens of a chunk, so the dependent chain
//   U = Tb V,  vn = U - W S,  o = Qg S + QK vn,  S' = GL S + K^T (DEC vn)
// never waits for another wave: the per-chunk operands shared by the 4 waves (Qg, W, Tb, QK, K^T,
// V^T) are staged in LDS once per chunk, and the only layout changes inside the chain (S and vn
// from accumulator layout to B-operand layout) go through wave-private LDS.
struct StateSmem {
  uint16_t Qg[pf::CH * pf::LDK];       // scale e^G q (token, feature)
  uint16_t W[pf::CH * pf::LDK];        // (token, feature)
  uint16_t QK[pf::CH * pf::LDT];       // (token, token)
  uint16_t KT[pf::D * pf::LDT];        // (feature, token)
  uint16_t ST[4][16 * pf::LDK];        // per wave: bf16 S^T (column, feature)
  uint16_t VN[4][3][16 * pf::LDT];     // per wave: vn, hi(dec vn), lo(dec vn) transposed (column, token)
  float DEC[pf::CH];
  float GL;
};

struct StateStage {  // one chunk's inputs, prefetched into registers
  u16x8 qg[4], kt[4], w[4], qk[2];
  f32x4 u[4];  // this wave's U tiles (accumulator layout), one per token block
  float dec, gl;
};

__device__ __forceinline__ void state_prefetch(StateStage& st, const uint8_t* rec, int j0, int t) {
  using namespace pf;
  const uint16_t* wr = reinterpret_cast<const uint16_t*>(rec + ws::W);
  const uint16_t* qgr = reinterpret_cast<const uint16_t*>(rec + ws::QG);
  const uint16_t* ktr = reinterpret_cast<const uint16_t*>(rec + ws::KT);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = t + NT * i;  // 1024 pieces of 16 bytes
    st.w[i] = *reinterpret_cast<const u16x8*>(wr + (idx >> 4) * D + 8 * (idx & 15));
    st.qg[i] = *reinterpret_cast<const u16x8*>(qgr + (idx >> 4) * D + 8 * (idx & 15));
    st.kt[i] = *reinterpret_cast<const u16x8*>(ktr + (idx >> 3) * CH + 8 * (idx & 7));
  }
  const uint16_t* qkr = reinterpret_cast<const uint16_t*>(rec + ws::QK);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = t + NT * i;  // 512 pieces of 16 bytes
    st.qk[i] = *reinterpret_cast<const u16x8*>(qkr + (idx >> 3) * CH + 8 * (idx & 7));
  }
  const f32x4* ur = reinterpret_cast<const f32x4*>(rec + ws::U) + (j0 >> 4) * 4 * 64 + (t & 63);
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) st.u[tb] = ur[tb * 64];
  st.dec = reinterpret_cast<const float*>(rec + ws::DEC)[t & 63];
  st.gl = reinterpret_cast<const float*>(rec + ws::GL)[0];
}

__device__ __forceinline__ void state_commit(StateSmem& sm, const StateStage& st, int t) {
  using namespace pf;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = t + NT * i;
    *reinterpret_cast<u16x8*>(&sm.W[(idx >> 4) * LDK + 8 * (idx & 15)]) = st.w[i];
    *reinterpret_cast<u16x8*>(&sm.Qg[(idx >> 4) * LDK + 8 * (idx & 15)]) = st.qg[i];
    *reinterpret_cast<u16x8*>(&sm.KT[(idx >> 3) * LDT + 8 * (idx & 7)]) = st.kt[i];
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = t + NT * i;
    *reinterpret_cast<u16x8*>(&sm.QK[(idx >> 3) * LDT + 8 * (idx & 7)]) = st.qk[i];
  }
  if (t < 64) sm.DEC[t] = st.dec;
  if (t == 0) sm.GL = st.gl;
}

template <typename OutT>
__global__ __launch_bounds__(pf::NT, 1) void chunk_state_kernel(
    const float* __restrict__ init, float* __restrict__ final_state,
    OutT* __restrict__ out, const int32_t* __restrict__ cu, const int32_t* __restrict__ seq_chunk0, int seq_len,
    int Hv, const uint8_t* __restrict__ work) {
  using namespace pf;
  __shared__ StateSmem sm;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63, g4 = lane >> 4, c16 = lane & 15;
  const int ntile = D / 64;
  const int vt = blockIdx.x % ntile;
  const int h = (blockIdx.x / ntile) % Hv, seq = blockIdx.x / ntile / Hv;
  const int vcol0 = 64 * vt, j0 = vcol0 + 16 * w;
  int64_t s0;
  int L, slot0;
  if (cu) {
    s0 = cu[seq];
    L = cu[seq + 1] - cu[seq];
    slot0 = seq_chunk0[seq];
  } else {
    s0 = (int64_t)seq * seq_len;
    L = seq_len;
    slot0 = seq * ((seq_len + CH - 1) / CH);
  }
  const int nch = (L + CH - 1) / CH;
  const int64_t sbase = ((int64_t)seq * Hv + h) * D * D + j0;
  uint16_t* myST = sm.ST[w];
  uint16_t* myVN = sm.VN[w][0];
  uint16_t* myVSH = sm.VN[w][1];
  uint16_t* myVSL = sm.VN[w][2];

  // S[:, j0..j0+15] as 8 row blocks in accumulator layout: S[rb][r] = S[16rb + 4g + r][j0 + c]
  f32x4 S[8];
#pragma unroll
  for (int rb = 0; rb < 8; ++rb) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      S[rb][r] = init ? init[sbase + (int64_t)(16 * rb + 4 * g4 + r) * D + c16] : 0.f;
    const u16x4 pk = {f2bf(S[rb][0]), f2bf(S[rb][1]), f2bf(S[rb][2]), f2bf(S[rb][3])};
    *reinterpret_cast<u16x4*>(&myST[c16 * LDK + 16 * rb + 4 * g4]) = pk;
  }

  StateStage st;
  const uint8_t* rec0 = work + (int64_t)slot0 * Hv * ws::BYTES + (int64_t)h * ws::BYTES;
  if (nch > 0) state_prefetch(st, rec0, j0, t);

  for (int c = 0; c < nch; ++c) {
    const int len = L - c * CH < CH ? L - c * CH : CH;
    const int64_t t0 = s0 + (int64_t)c * CH;
    state_commit(sm, st, t);
    f32x4 U[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) U[tb] = st.u[tb];
    __syncthreads();

    // vn = U - W S for all 4 token blocks of the chunk.  Each phase loads all of its LDS fragments
    // first and then issues its MFMAs (sched_barrier keeps the compiler from re-interleaving them
    // into one-load-one-wait pairs).
    bf16x8 fs[4];  // S^T fragments (B operand of W S and Qg S), reused by the output products
    {
      bf16x8 fw[4][4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        fs[s] = frag(myST, LDK, 0, 32 * s, lane);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) fw[s][tb] = frag_neg(sm.W, LDK, 16 * tb, 32 * s, lane);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) U[tb] = mma(fw[s][tb], fs[s], U[tb]);
    }
    // publish vn (bf16) and dec*vn = hi + lo, transposed (column, token), wave-private
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const int s0r = 16 * tb + 4 * g4;
      u16x4 vo, vh, vl;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float vn = U[tb][r];
        const float vsc = vn * sm.DEC[s0r + r];
        vo[r] = f2bf(vn);
        vh[r] = f2bf(vsc);
        vl[r] = f2bf(vsc - bf2f(vh[r]));
      }
      *reinterpret_cast<u16x4*>(&myVN[c16 * LDT + s0r]) = vo;
      *reinterpret_cast<u16x4*>(&myVSH[c16 * LDT + s0r]) = vh;
      *reinterpret_cast<u16x4*>(&myVSL[c16 * LDT + s0r]) = vl;
    }
    __builtin_amdgcn_wave_barrier();

    // o = Qg S + QK vn
    {
      bf16x8 fq[4][4], fk[2][4], fn[2];
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) fq[s][tb] = frag(sm.Qg, LDK, 16 * tb, 32 * s, lane);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        fn[s] = frag(myVN, LDT, 0, 32 * s, lane);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
          if (s == 0 || tb >= 2) fk[s][tb] = frag(sm.QK, LDT, 16 * tb, 32 * s, lane);
      }
      __builtin_amdgcn_sched_barrier(0);
      f32x4 O[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) O[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) O[tb] = mma(fq[s][tb], fs[s], O[tb]);
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
          if (s == 0 || tb >= 2) O[tb] = mma(fk[s][tb], fn[s], O[tb]);
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * tb + 4 * g4 + r;
          if (row < len) Elem<OutT>::store(out + ((t0 + row) * Hv + h) * D + j0 + c16, O[tb][r]);
        }
    }

    // next chunk's operands: issued here so their registers are not live during the products above
    if (c + 1 < nch) {
      state_prefetch(st, rec0 + (int64_t)(c + 1) * Hv * ws::BYTES, j0, t);
    }
    // S' = GL S + K^T (hi + lo), then its bf16 transpose for the next chunk
    {
      const float gl = sm.GL;
      bf16x8 fa[8][2], fh[2], fl[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        fh[s] = frag(myVSH, LDT, 0, 32 * s, lane);
        fl[s] = frag(myVSL, LDT, 0, 32 * s, lane);
#pragma unroll
        for (int rb = 0; rb < 8; ++rb) fa[rb][s] = frag(sm.KT, LDT, 16 * rb, 32 * s, lane);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int rb = 0; rb < 8; ++rb) {
        S[rb] *= gl;
        S[rb] = mma(fa[rb][0], fh[0], S[rb]);
        S[rb] = mma(fa[rb][0], fl[0], S[rb]);
        S[rb] = mma(fa[rb][1], fh[1], S[rb]);
        S[rb] = mma(fa[rb][1], fl[1], S[rb]);
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int rb = 0; rb < 8; ++rb) {
        const u16x4 pk = {f2bf(S[rb][0]), f2bf(S[rb][1]), f2bf(S[rb][2]), f2bf(S[rb][3])};
        *reinterpret_cast<u16x4*>(&myST[c16 * LDK + 16 * rb + 4 * g4]) = pk;
      }
    }
    __syncthreads();  // shared chunk operands are overwritten by the next commit
  }

  if (final_state) {
#pragma unroll
    for (int rb = 0; rb < 8; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) final_state[sbase + (int64_t)(16 * rb + 4 * g4 + r) * D + c16] = S[rb][r];
  }
}

// ============================================================================================
// Causal depthwise conv prefill + SiLU with decode-state capture.
// ============================================================================================
// One thread per (packed token p, 8 channels): it loads the K input rows p-K+1..p with 16-byte
// reads (rows before its sequence come from `history` [n_seq, C, K], x_{-j} = history[K - j], or
// are zero), writes 8 outputs with one 16-byte store, and -- for the last token of a sequence --
// the sequence's decode conv state (its last K inputs).  Numerics of F.conv1d on bf16: fp32
// accumulation of the K products (+ bias), one bf16 rounding, SiLU, bf16.
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
                                                           uint16_t* __restrict__ out, uint16_t* __restrict__ state,
                                                           const int32_t* __restrict__ cu, int nseq, int seq_len,
                                                           int C) {
  const int cg = blockIdx.x * blockDim.x + threadIdx.x;  // 8-channel group
  const int64_t p = blockIdx.y;
  if (8 * cg >= C) return;
  const int c0 = 8 * cg;
  const int s = cu ? find_seq(cu, nseq, p) : (int)(p / seq_len);
  const int64_t s_lo = cu ? (int64_t)cu[s] : (int64_t)s * seq_len;
  const int64_t s_hi = cu ? (int64_t)cu[s + 1] : s_lo + seq_len;
  u16x8 win[K];
#pragma unroll
  for (int r = 0; r < K; ++r) {
    const int64_t tok = p - (K - 1) + r;
    if (tok >= s_lo) {
      win[r] = *reinterpret_cast<const u16x8*>(x + tok * x_stride + c0);
    } else {
      const int back = (int)(s_lo - tok);  // 1..K-1
#pragma unroll
      for (int e = 0; e < 8; ++e)
        win[r][e] = history ? history[((int64_t)s * C + c0 + e) * K + (K - back)] : (uint16_t)0;
    }
  }
  u16x8 wt[K];  // weight[c0 + e][r] -> wt[r][e]
  {
    const uint16_t* wp = weight + (int64_t)c0 * K;
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int r = 0; r < K; ++r) wt[r][e] = wp[e * K + r];
  }
  u16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float acc = bias ? bf2f(bias[c0 + e]) : 0.f;
#pragma unroll
    for (int r = 0; r < K; ++r) acc += bf2f(win[r][e]) * bf2f(wt[r][e]);
    o[e] = f2bf(silu_f(rbf(acc)));
  }
  *reinterpret_cast<u16x8*>(out + p * (int64_t)C + c0) = o;
  if (state && p == s_hi - 1) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int r = 0; r < K; ++r) state[((int64_t)s * C + c0 + e) * K + r] = win[r][e];
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

extern "C" int64_t gdn_chunk_prefill_workspace_bytes(int64_t total_chunks, int Hv) {
  return total_chunks * (int64_t)Hv * ws::BYTES;
}

extern "C" int gdn_chunk_prefill(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                                 const void* v, int64_t v_stride, const float* g, const void* beta,
                                 int beta_dtype, const float* initial_state, float* final_state, void* out,
                                 int64_t total_tokens, const int32_t* cu_seqlens, const int32_t* seq_chunk0,
                                 int64_t total_chunks, int nseq, int seq_len, int Hqk, int Hv, int D, int in_dtype,
                                 int use_qk_l2norm, void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
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
  GDN_REQUIRE(total_chunks == 0 || (workspace && aligned(workspace, 256) &&
                                    workspace_bytes >= gdn_chunk_prefill_workspace_bytes(total_chunks, Hv)),
              "gdn_chunk_prefill: workspace missing, misaligned or smaller than %lld bytes",
              (long long)gdn_chunk_prefill_workspace_bytes(total_chunks, Hv));
  GDN_REQUIRE(total_chunks < (1ll << 31) && (int64_t)nseq * Hv * 2 < (1ll << 31), "gdn_chunk_prefill: grid too large");
  if (nseq == 0) return GDN_OK;
  hipStream_t s = (hipStream_t)stream;
  uint8_t* work = (uint8_t*)workspace;
  if (total_chunks > 0) {
    dim3 g1((unsigned)total_chunks, (unsigned)Hv);
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
  chunk_state_kernel<uint16_t><<<(unsigned)(nseq * Hv * (pf::D / 64)), pf::NT, 0, s>>>(
      initial_state, final_state, (uint16_t*)out, cu_seqlens, seq_chunk0, seq_len, Hv, work);
  return check_launch("gdn_chunk_prefill(state)");
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
    GDN_REQUIRE(C % 8 == 0 && x_stride % 8 == 0 && aligned(x, 16) && aligned(out, 16),
                "gdn_conv_prefill: C and the row stride must be multiples of 8 with 16-byte aligned rows");
    GDN_REQUIRE(total_tokens < (1ll << 31), "gdn_conv_prefill: too many tokens");
    dim3 grid((unsigned)((C / 8 + 255) / 256), (unsigned)total_tokens);
#define GDN_CONV_PREFILL(KK)                                                                                    \
  case KK:                                                                                                     \
    conv_prefill_kernel<KK><<<grid, 256, 0, s>>>((const uint16_t*)x, x_stride, (const uint16_t*)weight,          \
                                                 (const uint16_t*)bias, (const uint16_t*)history, (uint16_t*)out, \
                                                 (uint16_t*)state_out, cu_seqlens, nseq, seq_len, C);              \
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
