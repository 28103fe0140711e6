// Chunked gated delta rule for any head dims d_k, d_v in {16, 32, 64, 128} and fp32, bf16 or fp16
// inputs, computed in fp32 throughout (v_mfma_f32_16x16x4_f32): the general form of
// fast_chunk_gated_delta_rule_v2 (src/gdn_chunk_fast2.py:11-62), which takes any float dtype and
// head dims.  The bf16, d = 128 case has its own segment-parallel kernels (gdn_prefill.hip); this
// one walks each sequence's chunks in order, one workgroup per (sequence, value head, slice of 64
// value columns), everything of a chunk in LDS and the state slice in MFMA accumulators.
//
// Per 64-token chunk (src/gdn_chunk_fast2.py:31-59):
//   X  = -(beta_i k_i.k_j e^{G_i - G_j})_{i>j},  T = (I - X)^{-1}  (reg_inv64, the chunked prefill's
//        inverse routine),  U = T diag(beta) V,  W = T diag(beta e^G) K,
//   QK = (q_i.k_j e^{G_i - G_j})_{i>=j},  vn = U - W S,  o = diag(e^G) Q S + QK vn,
//   S' = e^{G_last} S + K^T diag(e^{G_last - G}) vn,
// with q scaled by d_k^-1/2 and, with use_qk_l2norm, q and k l2-normalised in their own dtype first
// (src/gdn_chunk_fast.py:17-18: each op rounded to that dtype).  The output is rounded once to the
// input dtype.  A sequence's chunks of fewer than 64 tokens are zero-padded (g = 0, beta = 0), as
// the reference pads T to a multiple of the chunk.
#include "gdn_device.h"
#include "gdn_internal.h"
#include "gdn_inverse.h"

namespace gdn {
namespace gp {
constexpr int CH = 64;   // chunk length
constexpr int NT = 256;  // 4 waves
constexpr int VS = 64;   // value columns per workgroup (16 per wave)
}  // namespace gp

// One element of an input tensor in dtype code `dt` (GDN_F32, GDN_BF16, GDN_F16), and the rounding
// of an fp32 result to that dtype (the result of one torch elementwise op on such a tensor).
__device__ __forceinline__ float ld_any(const void* p, int64_t i, int dt) {
  if (dt == GDN_F32) return reinterpret_cast<const float*>(p)[i];
  if (dt == GDN_BF16) return bf2f(reinterpret_cast<const uint16_t*>(p)[i]);
  return (float)reinterpret_cast<const _Float16*>(p)[i];
}
__device__ __forceinline__ float rnd_any(float x, int dt) {
  if (dt == GDN_F32) return x;
  if (dt == GDN_BF16) return rbf(x);
  return (float)(_Float16)x;
}
__device__ __forceinline__ void st_any(void* p, int64_t i, float x, int dt) {
  if (dt == GDN_F32) reinterpret_cast<float*>(p)[i] = x;
  else if (dt == GDN_BF16) reinterpret_cast<uint16_t*>(p)[i] = f2bf(x);
  else reinterpret_cast<_Float16*>(p)[i] = (_Float16)x;
}

template <int DK>
struct alignas(16) GenSmem {
  static constexpr int LK = DK + 4;  // fp32 row pitches
  static constexpr int LV = gp::VS + 4;
  static constexpr int LC = gp::CH + 4;
  float K[gp::CH * LK];  // key rows (normalised), zero past the chunk's end
  float Q[gp::CH * LK];  // query rows (normalised, times d_k^-1/2)
  float W[gp::CH * LK];  // T diag(beta e^G) K
  float U[gp::CH * LV];  // the slice's value rows, then U = T diag(beta) V
  float T[gp::CH * LC];  // X, then T
  float A[gp::CH * LC];  // QK
  float G[gp::CH], eG[gp::CH], dec[gp::CH], beta[gp::CH];
  float gl;
  float tiles[4 * 16 * kTrPitch];  // wave 0's transpose tiles (reg_inv64)
};

struct GenArgs {
  const void* q;
  const void* k;
  const void* v;
  int64_t qs, ks, vs;  // token strides (elements)
  const float* g;
  const void* beta;
  int beta_dt, in_dt;
  const float* init;
  float* final_state;
  const int32_t* rows;
  int n_rows;
  void* out;  // [tokens, Hv, Dv] in in_dt
  const int32_t* cu;
  int nseq, seq_len, Hqk, Hv, Dv, nslice, use_l2;
};

// Rows 0..63 of a [64, DK] tile: row r = t / 4 by the four lanes t % 4 (DK / 4 columns each, at
// columns 4 m + t % 4).  Reads the chunk's row if it exists (zero otherwise), l2-normalises it in
// the input dtype when asked, scales it by `scale` in fp32 and stores it at dst (pitch ld).
template <int DK>
__device__ __forceinline__ void load_rows_norm(float* dst, int ld, const void* src, int64_t stride, int64_t col0,
                                               int len, int dt, int use_l2, float scale) {
  constexpr int PER = DK / 4;
  const int t = threadIdx.x, r = t >> 2, part = t & 3;
  float x[PER];
#pragma unroll
  for (int m = 0; m < PER; ++m) x[m] = r < len ? ld_any(src, (int64_t)r * stride + col0 + 4 * m + part, dt) : 0.f;
  if (use_l2) {
    float ss = 0.f;
#pragma unroll
    for (int m = 0; m < PER; ++m) ss += rnd_any(x[m] * x[m], dt);
    ss += __shfl_xor(ss, 1, kWave);
    ss += __shfl_xor(ss, 2, kWave);
    const float inv = rnd_any(rsqrt_f(rnd_any(rnd_any(ss, dt) + 1e-6f, dt)), dt);
#pragma unroll
    for (int m = 0; m < PER; ++m) x[m] = rnd_any(x[m] * inv, dt);
  }
#pragma unroll
  for (int m = 0; m < PER; ++m) dst[r * ld + 4 * m + part] = x[m] * scale;
}

// 16x16 block of A B^T over kdim (A rows a0.., B rows b0.., both row-major fp32 in LDS): lane (c, g)
// r = sum_k A[a0 + 4g + r][k] B[b0 + c][k] (the MFMA accumulator layout).
__device__ __forceinline__ f32x4 gram16(const float* A, const float* B, int ld, int kdim, int lane) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const int c = lane & 15, g = lane >> 4;
  for (int k0 = 0; k0 < kdim; k0 += 4)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[c * ld + k0 + g], B[c * ld + k0 + g], acc, 0, 0, 0);
  return acc;
}

template <int DK>
__global__ __launch_bounds__(gp::NT) void chunk_generic_kernel(GenArgs P) {
  using namespace gp;
  using Sm = GenSmem<DK>;
  constexpr int LK = Sm::LK, LV = Sm::LV, LC = Sm::LC, NJ = DK / 16;
  __shared__ Sm sm;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63, c = lane & 15, g = lane >> 4;
  const int slice = blockIdx.x % P.nslice, rest = blockIdx.x / P.nslice;
  const int h = rest % P.Hv, s = rest / P.Hv;
  if (s >= P.nseq) return;
  const int hk = h / (P.Hv / P.Hqk);
  const int64_t t_seq = P.cu ? (int64_t)P.cu[s] : (int64_t)s * P.seq_len;
  const int Ls = P.cu ? P.cu[s + 1] - P.cu[s] : P.seq_len;
  const int vc0 = slice * VS;             // first value column of the slice
  const int ncol = P.Dv - vc0 < VS ? P.Dv - vc0 : VS;
  const bool mine = 16 * w < ncol;        // this wave's 16 state columns exist
  const int row = P.init || P.final_state ? state_row(P.rows, P.n_rows, s) : -1;
  const int64_t sbase = ((int64_t)(row < 0 ? 0 : row) * P.Hv + h) * DK * P.Dv;
  // the state slice: S[j] lane (c, g) r = S[16 j + 4 g + r][vc0 + 16 w + c]
  f32x4 S[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      S[j][r] = (P.init && row >= 0 && mine) ? P.init[sbase + (int64_t)(16 * j + 4 * g + r) * P.Dv + vc0 + 16 * w + c]
                                             : 0.f;
  const float qscale = 1.0f / sqrtf((float)DK);
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < Ls; c0 += CH) {
    const int len = Ls - c0 < CH ? Ls - c0 : CH;
    const int64_t tok0 = t_seq + c0;
    // ---- load: K, Q (normalised), the V slice, g and beta; wave 0 also forms the decay
    load_rows_norm<DK>(sm.K, LK, P.k, P.ks, tok0 * P.ks + (int64_t)hk * DK, len, P.in_dt, P.use_l2, 1.f);
    load_rows_norm<DK>(sm.Q, LK, P.q, P.qs, tok0 * P.qs + (int64_t)hk * DK, len, P.in_dt, P.use_l2, qscale);
    for (int i = t; i < CH * VS; i += NT) {
      const int r = i / VS, col = i % VS;
      sm.U[r * LV + col] = (r < len && col < ncol) ? ld_any(P.v, (tok0 + r) * P.vs + (int64_t)h * P.Dv + vc0 + col, P.in_dt)
                                                   : 0.f;
    }
    if (w == 0) {
      const float gv = lane < len ? P.g[(tok0 + lane) * P.Hv + h] : 0.f;
      const float bv = lane < len ? ld_any(P.beta, (tok0 + lane) * P.Hv + h, P.beta_dt) : 0.f;
      const float G = wave_incl_scan(gv);
      const float Gl = __shfl(G, 63, kWave);
      sm.G[lane] = G;
      sm.eG[lane] = expf(G);
      sm.dec[lane] = expf(Gl - G);
      sm.beta[lane] = bv;
      if (lane == 0) sm.gl = expf(Gl);
    }
    __syncthreads();
    // ---- X = -(beta_i k_i.k_j e^{G_i - G_j})_{i>j} into T, QK = (q_i.k_j e^{G_i - G_j})_{i>=j} into A:
    // 16 blocks each (upper blocks written as zero), 8 per wave
    for (int bi = w; bi < 32; bi += 4) {
      const int which = bi >> 4, a = (bi >> 2) & 3, b = bi & 3;  // which: 0 X, 1 QK
      float* M = which ? sm.A : sm.T;
      f32x4 acc = z4;
      if (b <= a) acc = gram16(which ? sm.Q + 16 * a * LK : sm.K + 16 * a * LK, sm.K + 16 * b * LK, LK, DK, lane);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * a + 4 * g + r, j = 16 * b + c;
        const bool in = which ? i >= j : i > j;
        const float d = expf(in ? sm.G[i] - sm.G[j] : 0.f);
        M[i * LC + j] = in ? (which ? acc[r] * d : -sm.beta[i] * acc[r] * d) : 0.f;
      }
    }
    __syncthreads();
    // ---- T = (I - X)^{-1} (wave 0, in registers)
    if (w == 0) {
      f32x4 XT[10], Xd[4], TT[10];
#pragma unroll
      for (int a = 0; a < 4; ++a) {
#pragma unroll
        for (int b = 0; b < a; ++b) XT[tri(a, b)] = *reinterpret_cast<const f32x4*>(&sm.T[(16 * a + c) * LC + 16 * b + 4 * g]);
        XT[tri(a, a)] = z4;
#pragma unroll
        for (int r = 0; r < 4; ++r) Xd[a][r] = sm.T[(16 * a + 4 * g + r) * LC + 16 * a + c];  // zero on and above the diagonal
      }
      reg_inv64(XT, Xd, TT, sm.tiles, lane);
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
          *reinterpret_cast<f32x4*>(&sm.T[(16 * a + c) * LC + 16 * b + 4 * g]) = b <= a ? TT[tri(a, b <= a ? b : 0)] : z4;
    }
    __syncthreads();
    // ---- U = T diag(beta) V (token tile w, held until every wave has read V), W = T diag(beta e^G) K
    {
      f32x4 u[VS / 16];
#pragma unroll
      for (int n = 0; n < VS / 16; ++n) u[n] = z4;
      for (int k0 = 0; k0 < 16 * (w + 1); k0 += 4) {  // T is lower: tokens k <= 16 w + 15
        const int kk = k0 + g;
        const float a = sm.T[(16 * w + c) * LC + kk];
        const float bb = sm.beta[kk];
#pragma unroll
        for (int n = 0; n < VS / 16; ++n)
          u[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, bb * sm.U[kk * LV + 16 * n + c], u[n], 0, 0, 0);
      }
      for (int n = 0; n < NJ; ++n) {
        f32x4 acc = z4;
        for (int k0 = 0; k0 < 16 * (w + 1); k0 += 4) {
          const int kk = k0 + g;
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.T[(16 * w + c) * LC + kk],
                                                     sm.beta[kk] * sm.eG[kk] * sm.K[kk * LK + 16 * n + c], acc, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) sm.W[(16 * w + 4 * g + r) * LK + 16 * n + c] = acc[r];
      }
      __syncthreads();
#pragma unroll
      for (int n = 0; n < VS / 16; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) sm.U[(16 * w + 4 * g + r) * LV + 16 * n + c] = u[n][r];
    }
    __syncthreads();
    // ---- the chain on this wave's 16 state columns
    if (mine) {
      f32x4 vn[4], o[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        f32x4 p = z4, qs = z4;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          p = rmm(*reinterpret_cast<const f32x4*>(&sm.W[(16 * tb + c) * LK + 16 * j + 4 * g]), S[j], p);
          qs = rmm(*reinterpret_cast<const f32x4*>(&sm.Q[(16 * tb + c) * LK + 16 * j + 4 * g]), S[j], qs);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * tb + 4 * g + r;
          vn[tb][r] = sm.U[i * LV + 16 * w + c] - p[r];
          o[tb][r] = sm.eG[i] * qs[r];
        }
      }
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int tb2 = 0; tb2 <= tb; ++tb2)
          o[tb] = rmm(*reinterpret_cast<const f32x4*>(&sm.A[(16 * tb + c) * LC + 16 * tb2 + 4 * g]), vn[tb2], o[tb]);
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * tb + 4 * g + r;
          if (i < len)
            st_any(P.out, ((tok0 + i) * P.Hv + h) * (int64_t)P.Dv + vc0 + 16 * w + c, o[tb][r], P.in_dt);
        }
      const float gl = sm.gl;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        f32x4 acc = S[j] * gl;
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          f32x4 kd;  // Dl(Kd_{tb, j}): lane (c, g) r = K[16 tb + 4 g + r][16 j + c] e^{G_last - G}
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = 16 * tb + 4 * g + r;
            kd[r] = sm.K[i * LK + 16 * j + c] * sm.dec[i];
          }
          acc = rmm(kd, vn[tb], acc);
        }
        S[j] = acc;
      }
    }
    __syncthreads();
  }
  if (P.final_state && row >= 0 && mine) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        P.final_state[sbase + (int64_t)(16 * j + 4 * g + r) * P.Dv + vc0 + 16 * w + c] = S[j][r];
  }
}

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_chunk_prefill_generic(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                                         const void* v, int64_t v_stride, const float* g, const void* beta,
                                         int beta_dtype, const float* initial_state, float* final_state,
                                         const int32_t* state_rows, int n_rows, void* out, int64_t total_tokens,
                                         const int32_t* cu_seqlens, int nseq, int seq_len, int Hqk, int Hv, int Dk,
                                         int Dv, int in_dtype, int use_qk_l2norm, void* stream) {
  clear_error();
  GDN_REQUIRE(q && k && v && g && beta && out, "gdn_chunk_prefill_generic: null input/output pointer");
  GDN_SUPPORT(Dk == 16 || Dk == 32 || Dk == 64 || Dk == 128, "gdn_chunk_prefill_generic: d_k %d unsupported "
              "(16, 32, 64 or 128)", Dk);
  GDN_SUPPORT(Dv == 16 || Dv == 32 || Dv == 64 || Dv == 128, "gdn_chunk_prefill_generic: d_v %d unsupported "
              "(16, 32, 64 or 128)", Dv);
  GDN_REQUIRE(in_dtype == GDN_F32 || in_dtype == GDN_BF16 || in_dtype == GDN_F16,
              "gdn_chunk_prefill_generic: bad q/k/v dtype");
  GDN_REQUIRE(beta_dtype == GDN_F32 || beta_dtype == GDN_BF16 || beta_dtype == GDN_F16,
              "gdn_chunk_prefill_generic: bad beta dtype");
  GDN_REQUIRE(Hqk > 0 && Hv > 0 && Hv % Hqk == 0, "gdn_chunk_prefill_generic: bad heads Hqk=%d Hv=%d", Hqk, Hv);
  GDN_REQUIRE(nseq >= 0 && total_tokens >= 0 && seq_len >= 0, "gdn_chunk_prefill_generic: negative sizes");
  GDN_REQUIRE(cu_seqlens || (int64_t)nseq * seq_len == total_tokens,
              "gdn_chunk_prefill_generic: without cu_seqlens nseq*seq_len must be total_tokens");
  GDN_REQUIRE(state_rows ? n_rows >= 0 : n_rows == nseq,
              "gdn_chunk_prefill_generic: without state_rows, n_rows must equal nseq");
  GDN_REQUIRE(q_stride >= (int64_t)Hqk * Dk && k_stride >= (int64_t)Hqk * Dk && v_stride >= (int64_t)Hv * Dv,
              "gdn_chunk_prefill_generic: token strides too small");
  const int nslice = (Dv + gp::VS - 1) / gp::VS;
  const int64_t grid = (int64_t)nseq * Hv * nslice;
  GDN_REQUIRE(grid < (1ll << 31), "gdn_chunk_prefill_generic: grid too large");
  if (nseq == 0) return GDN_OK;
  GenArgs P{q, k, v, q_stride, k_stride, v_stride, g, beta, beta_dtype, in_dtype, initial_state, final_state,
            state_rows, n_rows, out, cu_seqlens, nseq, seq_len, Hqk, Hv, Dv, nslice, use_qk_l2norm};
  hipStream_t st = (hipStream_t)stream;
  switch (Dk) {
    case 16: chunk_generic_kernel<16><<<(unsigned)grid, gp::NT, 0, st>>>(P); break;
    case 32: chunk_generic_kernel<32><<<(unsigned)grid, gp::NT, 0, st>>>(P); break;
    case 64: chunk_generic_kernel<64><<<(unsigned)grid, gp::NT, 0, st>>>(P); break;
    default: chunk_generic_kernel<128><<<(unsigned)grid, gp::NT, 0, st>>>(P); break;
  }
  return check_launch("gdn_chunk_prefill_generic");
}
