// Decode-step projections: out[M, N] = x[M, K] W[N, K]^T with M <= 16 slots (the GDN layer's
// in_proj_* and out_proj in nn.Linear layout, bf16 in / bf16 out, fp32 accumulation).
//
// At 16 rows the product is a weight stream: W is read once (2 N K bytes) and x is tiny, so the
// kernel is HBM-bound and is built to keep W loads long and in flight.  It runs on bf16 MFMA with
// the roles turned around -- out^T = W x^T -- so the 16 slots are the MFMA's N dimension and each
// 16-row tile of W is an A operand:
//   * v_mfma_f32_16x16x32_bf16, lane (r, g) = (l % 16, l / 16).  Per 128-wide k step a lane loads
//     64 contiguous bytes of W row r (k + 32 g .. k + 32 g + 31) and the same 32 k of x row r; the
//     4 MFMAs of the step take 8 of those k each (A and B permuted alike, so the sum over the step
//     is the plain dot product).  4 lanes cover 256 contiguous bytes of a W row.
//   * a wave owns RT row tiles (16 RT output features) and reuses each x fragment RT times; a
//     workgroup is 4 waves.  When N alone gives too few waves to fill the chip, K is split over
//     blockIdx.y and fp32 partial sums go through a workspace and a small reduction kernel.
//   * each wave keeps PF k steps of loads in flight ahead of its MFMAs (a ring of register buffers).
//   * W is read once per step, so its loads carry the non-temporal hint: measured 3-7% faster per
//     projection than cached loads at the 27B decode shapes.
#include "gdn_device.h"
#include "gdn_internal.h"

namespace gdn {
namespace gv {
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
constexpr int RT = 2;               // row tiles per wave
constexpr int WAVES = 4;            // waves per workgroup
constexpr int ROWS = 16 * RT * WAVES;  // output features per workgroup
constexpr int KSTEP = 128;
constexpr int TARGET_WAVES = 2048;  // with PF steps in flight per wave: enough loads in flight for HBM
                                    // (3072 for wide projections, plan() below)
constexpr int PF = 3;               // k steps loaded ahead (a ring of PF + 1 register buffers)

struct Frag4 {
  u16x8 v[4];
};
__device__ __forceinline__ void load4(Frag4& f, const uint16_t* p) {
#pragma unroll
  for (int j = 0; j < 4; ++j) f.v[j] = *reinterpret_cast<const u16x8*>(p + 8 * j);
}
__device__ __forceinline__ void load4_nt(Frag4& f, const uint16_t* p) {
#pragma unroll
  for (int j = 0; j < 4; ++j) f.v[j] = __builtin_nontemporal_load(reinterpret_cast<const u16x8*>(p + 8 * j));
}
}  // namespace gv

// grid (ceil(N / ROWS), ksplit); workgroup (4 waves).  Split s covers k steps [s * steps_per, ...).
// PACKED: W is in the fragment-major layout of gdn_decode_linear_pack (w_stride unused).
template <bool PACKED>
__global__ __launch_bounds__(64 * gv::WAVES) void decode_linear_kernel(
    const uint16_t* __restrict__ x, int64_t x_stride, const uint16_t* __restrict__ W, int64_t w_stride,
    uint16_t* __restrict__ out, int64_t out_stride, float* __restrict__ part, int M, int64_t N, int64_t K,
    int steps_per) {
  using namespace gv;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, r = lane & 15, g = lane >> 4;
  const int64_t f0 = (int64_t)blockIdx.x * ROWS + (int64_t)w * 16 * RT;
  const int64_t nsteps = K / KSTEP;
  const int64_t s_lo = (int64_t)blockIdx.y * steps_per;
  const int64_t s_hi = s_lo + steps_per < nsteps ? s_lo + steps_per : nsteps;
  const uint16_t* wrow[RT];
  const int64_t ntiles = (N + 15) / 16;
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    if (PACKED) {
      // tile f / 16 (clamped: tiles past the last load a valid tile; their results are not stored)
      int64_t tile = (f0 >> 4) + t;
      tile = tile < ntiles ? tile : ntiles - 1;
      wrow[t] = W + tile * nsteps * (KSTEP * 16) + lane * 8;
    } else {
      int64_t row = f0 + 16 * t + r;
      row = row < N ? row : N - 1;  // rows past N load a valid row; their results are not stored
      wrow[t] = W + row * w_stride + 32 * g;
    }
  }
  const bool xrow = r < M;
  const uint16_t* xp = x + (int64_t)(xrow ? r : 0) * x_stride + 32 * g;
  f32x4 acc[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  Frag4 a[PF + 1][RT], b[PF + 1];
  const u16x8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  auto load_step = [&](int buf, int64_t s) {
    const int64_t k = s * KSTEP;
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      if (PACKED) {  // block (tile, s): 4 fragments of 64 lanes x 16 bytes, fragment j contiguous
#pragma unroll
        for (int j = 0; j < 4; ++j)
          a[buf][t].v[j] = __builtin_nontemporal_load(reinterpret_cast<const u16x8*>(wrow[t] + s * (KSTEP * 16) + j * 512));
      } else {
        load4_nt(a[buf][t], wrow[t] + k);
      }
    }
    if (xrow) load4(b[buf], xp + k);
    else
#pragma unroll
      for (int j = 0; j < 4; ++j) b[buf].v[j] = zero;
  };
  auto mma_step = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int t = 0; t < RT; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[buf][t].v[j]),
                                                         __builtin_bit_cast(bf16x8, b[buf].v[j]), acc[t], 0, 0, 0);
  };
  // step s_lo + i lives in buffer i % (PF + 1); the loop is unrolled over the ring so every buffer
  // index is static
#pragma unroll
  for (int u = 0; u < PF; ++u)
    if (s_lo + u < s_hi) load_step(u, s_lo + u);
  for (int64_t s = s_lo; s < s_hi; s += PF + 1) {
#pragma unroll
    for (int u = 0; u <= PF; ++u) {
      if (s + u + PF < s_hi) load_step((u + PF) % (PF + 1), s + u + PF);
      if (s + u < s_hi) mma_step(u);
    }
  }
  // lane (c, g) holds out^T[f0 + 16 t + 4 g + i][slot c], i < 4
  const int c = r;
  if (c >= M) return;
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const int64_t f = f0 + 16 * t + 4 * g;
    if (f >= N) continue;
    if (part) {
      float* pp = part + ((int64_t)blockIdx.y * M + c) * N + f;
      if (f + 4 <= N && (N & 3) == 0) *reinterpret_cast<f32x4*>(pp) = acc[t];
      else
        for (int i = 0; i < 4 && f + i < N; ++i) pp[i] = acc[t][i];
    } else {
      uint16_t* op = out + (int64_t)c * out_stride + f;
      if (f + 4 <= N && (out_stride & 3) == 0 && ((uintptr_t)out & 7) == 0) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u32x2*>(op) = u32x2{f2bf2(acc[t][0], acc[t][1]), f2bf2(acc[t][2], acc[t][3])};
      } else {
        for (int i = 0; i < 4 && f + i < N; ++i) op[i] = f2bf(acc[t][i]);
      }
    }
  }
}

// out[c][f] = bf16(sum over splits of part[s][c][f]), 4 features per thread.
__global__ __launch_bounds__(256) void decode_linear_reduce_kernel(const float* __restrict__ part, int splits,
                                                                   uint16_t* __restrict__ out, int64_t out_stride,
                                                                   int M, int64_t N) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // quad index over M x ceil(N / 4)
  const int64_t nq = (N + 3) / 4;
  if (q >= (int64_t)M * nq) return;
  const int c = (int)(q / nq);
  const int64_t f = (q % nq) * 4;
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  for (int sp = 0; sp < splits; ++sp) {
    const float* pp = part + ((int64_t)sp * M + c) * N + f;
    for (int i = 0; i < 4; ++i)
      if (f + i < N) s[i] += pp[i];
  }
  for (int i = 0; i < 4; ++i)
    if (f + i < N) out[(int64_t)c * out_stride + f + i] = f2bf(s[i]);
}

// Fragment-major copy of W [N, K] for the packed kernel: for 16-row tile T, k step s, fragment j,
// lane l = 16 g + r and element e: P[(((T * nsteps + s) * 4 + j) * 64 + l) * 8 + e] =
// W[16 T + r][128 s + 32 g + 8 j + e] (zero past row N).  Every load of the packed kernel then
// reads 1 KB contiguous and a tile's k steps follow each other in memory.
__global__ __launch_bounds__(256) void decode_linear_pack_kernel(const uint16_t* __restrict__ W, int64_t w_stride,
                                                                 uint16_t* __restrict__ P, int64_t N, int64_t K) {
  using namespace gv;
  const int64_t nsteps = K / KSTEP;
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // one 16-byte piece of P
  const int64_t total = (N + 15) / 16 * nsteps * 4 * 64;
  if (q >= total) return;
  const int l = (int)(q & 63), j = (int)((q >> 6) & 3);
  const int64_t ts = q >> 8, s = ts % nsteps, T = ts / nsteps;
  const int64_t row = 16 * T + (l & 15), k = 128 * s + 32 * (l >> 4) + 8 * j;
  u16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
  if (row < N) v = *reinterpret_cast<const u16x8*>(W + row * w_stride + k);
  *reinterpret_cast<u16x8*>(P + q * 8) = v;
}

namespace gv {
// (blocks along N, k splits, k steps per split)
inline void plan(int64_t N, int64_t K, int64_t* nb, int* splits, int* steps_per) {
  *nb = (N + ROWS - 1) / ROWS;
  const int64_t nsteps = K / KSTEP;
  // wide projections (N alone gives 512+ waves: the 27B shape's gate_up and GDN in_proj) split to
  // 3072 waves: 5% and 3% faster there, while the narrow ones (down, out_proj) are 10-30% slower
  // beyond 2048, whose splits then get too short to hide the loads' latency
  const int64_t target = *nb * WAVES >= 512 ? 3072 : TARGET_WAVES;
  int64_t sp = (target + *nb * WAVES - 1) / (*nb * WAVES);
  if (sp < 1) sp = 1;
  if (sp > nsteps) sp = nsteps;
  const int64_t per = (nsteps + sp - 1) / sp;
  *steps_per = (int)per;
  *splits = (int)((nsteps + per - 1) / per);
}
}  // namespace gv

}  // namespace gdn

using namespace gdn;

namespace {
int64_t workspace_bytes(int M, int64_t N, int64_t K) {
  int64_t nb;
  int splits, per;
  gv::plan(N, K, &nb, &splits, &per);
  return splits > 1 ? (int64_t)splits * M * N * (int64_t)sizeof(float) : 0;
}

// partial_only: write the fp32 split-K partial sums [splits][M][N] into workspace (even with one
// split) and skip the reduction; out is unused.
int decode_linear_launch(bool packed, const void* x, int64_t x_stride, const void* W, int64_t w_stride, void* out,
                         int64_t out_stride, int M, int64_t N, int64_t K, float* workspace, int64_t ws_bytes,
                         void* stream, bool partial_only = false) {
  GDN_REQUIRE(x && W && (out || partial_only), "gdn_decode_linear: null pointer");
  GDN_SUPPORT(M >= 1 && M <= 16, "gdn_decode_linear: %d rows (1..16 supported)", M);
  GDN_REQUIRE(N > 0 && N < (1ll << 31) && K > 0, "gdn_decode_linear: bad sizes N=%lld K=%lld", (long long)N,
              (long long)K);
  GDN_SUPPORT(K % gv::KSTEP == 0, "gdn_decode_linear: K=%lld must be a multiple of %d", (long long)K, gv::KSTEP);
  GDN_REQUIRE(aligned(x, 16) && aligned(W, 16) && x_stride % 8 == 0 && x_stride >= K &&
                  (packed || (w_stride % 8 == 0 && w_stride >= K)),
              "gdn_decode_linear: x and W rows must be 16-byte aligned and hold K values");
  GDN_REQUIRE(partial_only || (aligned(out, 2) && out_stride >= N), "gdn_decode_linear: out rows must hold N values");
  int64_t nb;
  int splits, per;
  gv::plan(N, K, &nb, &splits, &per);
  const int64_t need = partial_only ? (int64_t)splits * M * N * (int64_t)sizeof(float) : workspace_bytes(M, N, K);
  GDN_REQUIRE(need == 0 || (workspace && aligned(workspace, 16) && ws_bytes >= need),
              "gdn_decode_linear: needs a 16-byte aligned fp32 workspace of %lld bytes", (long long)need);
  hipStream_t s = (hipStream_t)stream;
  float* part = (splits > 1 || partial_only) ? workspace : nullptr;
  if (packed)
    decode_linear_kernel<true><<<dim3((unsigned)nb, (unsigned)splits), 64 * gv::WAVES, 0, s>>>(
        (const uint16_t*)x, x_stride, (const uint16_t*)W, w_stride, (uint16_t*)out, out_stride, part, M, N, K, per);
  else
    decode_linear_kernel<false><<<dim3((unsigned)nb, (unsigned)splits), 64 * gv::WAVES, 0, s>>>(
        (const uint16_t*)x, x_stride, (const uint16_t*)W, w_stride, (uint16_t*)out, out_stride, part, M, N, K, per);
  int rc = check_launch("gdn_decode_linear");
  if (rc || !part || partial_only) return rc;
  const int64_t quads = (int64_t)M * ((N + 3) / 4);
  decode_linear_reduce_kernel<<<(unsigned)((quads + 255) / 256), 256, 0, s>>>(part, splits, (uint16_t*)out,
                                                                               out_stride, M, N);
  return check_launch("gdn_decode_linear(reduce)");
}
}  // namespace

extern "C" int64_t gdn_decode_linear_workspace_bytes(int M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K < gv::KSTEP || K % gv::KSTEP) return 0;
  return workspace_bytes(M, N, K);
}

extern "C" int gdn_decode_linear(const void* x, int64_t x_stride, const void* W, int64_t w_stride, void* out,
                                 int64_t out_stride, int M, int64_t N, int64_t K, float* workspace,
                                 int64_t workspace_bytes, void* stream) {
  clear_error();
  return decode_linear_launch(false, x, x_stride, W, w_stride, out, out_stride, M, N, K, workspace,
                              workspace_bytes, stream);
}

extern "C" int64_t gdn_decode_linear_packed_elems(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || K % gv::KSTEP) return 0;
  return (N + 15) / 16 * 16 * K;
}

extern "C" int gdn_decode_linear_pack(const void* W, int64_t w_stride, void* packed, int64_t N, int64_t K,
                                      void* stream) {
  clear_error();
  GDN_REQUIRE(W && packed, "gdn_decode_linear_pack: null pointer");
  GDN_REQUIRE(N > 0 && N < (1ll << 31) && K > 0, "gdn_decode_linear_pack: bad sizes");
  GDN_SUPPORT(K % gv::KSTEP == 0, "gdn_decode_linear_pack: K=%lld must be a multiple of %d", (long long)K,
              gv::KSTEP);
  GDN_REQUIRE(aligned(W, 16) && aligned(packed, 16) && w_stride % 8 == 0 && w_stride >= K,
              "gdn_decode_linear_pack: W rows must be 16-byte aligned and hold K values");
  const int64_t pieces = gdn_decode_linear_packed_elems(N, K) / 8;
  GDN_REQUIRE((pieces + 255) / 256 < (1ll << 31), "gdn_decode_linear_pack: too large");
  decode_linear_pack_kernel<<<(unsigned)((pieces + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)W, w_stride, (uint16_t*)packed, N, K);
  return check_launch("gdn_decode_linear_pack");
}

extern "C" int gdn_decode_linear_packed(const void* x, int64_t x_stride, const void* packed, void* out,
                                        int64_t out_stride, int M, int64_t N, int64_t K, float* workspace,
                                        int64_t workspace_bytes, void* stream) {
  clear_error();
  return decode_linear_launch(true, x, x_stride, packed, 0, out, out_stride, M, N, K, workspace, workspace_bytes,
                              stream);
}

// ============================================================================================
// Residual add + RMSNorm between the decode step's layers (Qwen3_5RMSNorm, modeling_qwen3_5.py:
// fp32 x * rsqrt(mean(x^2) + eps) * (1 + w), cast to bf16): h_out = bf16(h + delta) (delta may be
// null: h_out = h), x_out = norm(h_out).  One workgroup per row; h_out may alias h.
// ============================================================================================
namespace gdn {
typedef uint16_t u16x8v __attribute__((ext_vector_type(8)));

// Sum of v over the workgroup's 4 waves (every thread gets it).
__device__ __forceinline__ float block_sum4(float v, float* red) {
  v = wave_sum_fast(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// Row reductions of the add + norm kernels: 1024 threads, one 16-byte row piece each (H <= 8192).
// Both kernels below sum the squares in this same order, so they give bit-identical norms.
constexpr int kPartThreads = 1024;
__device__ __forceinline__ float block_sum_1k(float v, float* red) {
  v = wave_sum_fast(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kPartThreads / 64; ++i) tot += red[i];
  return tot;
}

// H % 8 == 0 with 16-byte aligned rows and H <= 8192: each thread loads its row piece once and keeps
// it in registers for the output pass (a row is one memory round trip).
__global__ __launch_bounds__(kPartThreads) void add_rmsnorm_vec_kernel(const uint16_t* h,
                                                                       const uint16_t* __restrict__ delta,
                                                                       const uint16_t* __restrict__ w, uint16_t* h_out,
                                                                       uint16_t* __restrict__ x_out, int H, float eps) {
  __shared__ float red[kPartThreads / 64];
  const int64_t base = (int64_t)blockIdx.x * H;
  const int v = threadIdx.x, nv = H / 8;
  float x[8], ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = 0.f;
  if (v < nv) {
    const u16x8v hv = *reinterpret_cast<const u16x8v*>(h + base + 8 * v);
    u16x8v dv = {0, 0, 0, 0, 0, 0, 0, 0};
    if (delta) dv = *reinterpret_cast<const u16x8v*>(delta + base + 8 * v);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float val = bf2f(hv[e]);
      if (delta) val = rbf(val + bf2f(dv[e]));
      x[e] = val;
      ss += val * val;
    }
  }
  const float inv = rsqrtf(block_sum_1k(ss, red) / (float)H + eps);
  if (v < nv) {
    const u16x8v wv = *reinterpret_cast<const u16x8v*>(w + 8 * v);
    u16x8v o, hn;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o[e] = f2bf(x[e] * inv * (1.0f + bf2f(wv[e])));
      hn[e] = f2bf(x[e]);
    }
    *reinterpret_cast<u16x8v*>(x_out + base + 8 * v) = o;
    if (delta) *reinterpret_cast<u16x8v*>(h_out + base + 8 * v) = hn;
  }
}

// The same with delta given as the fp32 split-K partial sums of the projection that produced it
// (part [splits][M][H], gdn_decode_linear_packed_partial): delta = bf16(sum over splits, in split
// order) -- exactly what decode_linear_reduce_kernel would have stored -- so the reduction costs no
// launch and no bf16 round trip.  The split loads of one row piece are issued together.
__global__ __launch_bounds__(kPartThreads) void add_rmsnorm_part_kernel(const uint16_t* h,
                                                                        const float* __restrict__ part, int splits,
                                                                        int M, const uint16_t* __restrict__ w,
                                                                        uint16_t* h_out, uint16_t* __restrict__ x_out,
                                                                        int H, float eps) {
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  __shared__ float red[kPartThreads / 64];
  const int64_t row = blockIdx.x, base = row * H;
  const int v = threadIdx.x, nv = H / 8;
  float x[8], ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = 0.f;
  if (v < nv) {
    const u16x8v hv = *reinterpret_cast<const u16x8v*>(h + base + 8 * v);
    f32x4v d0 = {0.f, 0.f, 0.f, 0.f}, d1 = {0.f, 0.f, 0.f, 0.f};
    // the loads of 16 splits are issued before their in-order sums
#pragma unroll 16
    for (int sp = 0; sp < splits; ++sp) {
      const float* pp = part + ((int64_t)sp * M + row) * H + 8 * v;
      d0 += *reinterpret_cast<const f32x4v*>(pp);
      d1 += *reinterpret_cast<const f32x4v*>(pp + 4);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = rbf(e < 4 ? d0[e] : d1[e - 4]);
      x[e] = rbf(bf2f(hv[e]) + d);
      ss += x[e] * x[e];
    }
  }
  const float inv = rsqrtf(block_sum_1k(ss, red) / (float)H + eps);
  if (v < nv) {
    const u16x8v wv = *reinterpret_cast<const u16x8v*>(w + 8 * v);
    u16x8v o, hn;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o[e] = f2bf(x[e] * inv * (1.0f + bf2f(wv[e])));
      hn[e] = f2bf(x[e]);
    }
    *reinterpret_cast<u16x8v*>(x_out + base + 8 * v) = o;
    *reinterpret_cast<u16x8v*>(h_out + base + 8 * v) = hn;
  }
}

// SwiGLU of a decode step's MLP from the fp32 split-K partials of its gate_up projection
// (part [splits][M][2m], gate columns first): g, u = bf16(sum over splits), then torch's
// bf16(bf16(silu(g)) * u) (F.silu(gu[:, :m]) * gu[:, m:]).  8 outputs per thread.
__global__ __launch_bounds__(256) void swiglu_part_kernel(const float* __restrict__ part, int splits, int M,
                                                          int64_t m, uint16_t* __restrict__ out) {
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 8-column piece over M x m / 8
  const int64_t per_row = m / 8;
  if (q >= (int64_t)M * per_row) return;
  const int64_t row = q / per_row, col = (q % per_row) * 8;
  f32x4v g0 = {0.f, 0.f, 0.f, 0.f}, g1 = g0, u0 = g0, u1 = g0;
#pragma unroll 4
  for (int sp = 0; sp < splits; ++sp) {
    const float* pp = part + ((int64_t)sp * M + row) * (2 * m) + col;
    g0 += *reinterpret_cast<const f32x4v*>(pp);
    g1 += *reinterpret_cast<const f32x4v*>(pp + 4);
    u0 += *reinterpret_cast<const f32x4v*>(pp + m);
    u1 += *reinterpret_cast<const f32x4v*>(pp + m + 4);
  }
  float g[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) g[e] = rbf(e < 4 ? g0[e] : g1[e - 4]);
  uint16_t sg[8];
  silu_bf16_n<8>(g, sg);
  u16x8v o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = f2bf(bf2f(sg[e]) * rbf(e < 4 ? u0[e] : u1[e - 4]));
  *reinterpret_cast<u16x8v*>(out + row * m + col) = o;
}

// Any H (rows of other widths or alignments): element loop.
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const uint16_t* h, const uint16_t* __restrict__ delta,
                                                          const uint16_t* __restrict__ w, uint16_t* h_out,
                                                          uint16_t* __restrict__ x_out, int H, float eps) {
  const int64_t row = blockIdx.x;
  const uint16_t* hr = h + row * H;
  const uint16_t* dr = delta ? delta + row * H : nullptr;
  uint16_t* hor = h_out + row * H;
  __shared__ float red[4];
  float ss = 0.f;
  for (int i = threadIdx.x; i < H; i += 256) {
    float v = bf2f(hr[i]);
    if (dr) v = rbf(v + bf2f(dr[i]));
    ss += v * v;
  }
  const float inv = rsqrtf(block_sum4(ss, red) / (float)H + eps);
  for (int i = threadIdx.x; i < H; i += 256) {
    float v = bf2f(hr[i]);
    if (dr) v = rbf(v + bf2f(dr[i]));
    x_out[row * H + i] = f2bf(v * inv * (1.0f + bf2f(w[i])));
    if (dr) hor[i] = f2bf(v);
  }
}
}  // namespace gdn

extern "C" int gdn_add_rmsnorm(const void* h, const void* delta, const void* w, void* h_out, void* x_out, int M,
                               int H, float eps, void* stream) {
  clear_error();
  GDN_REQUIRE(h && w && x_out && (!delta || h_out), "gdn_add_rmsnorm: null pointer");
  GDN_REQUIRE(M >= 0 && H > 0, "gdn_add_rmsnorm: bad sizes");
  if (M == 0) return GDN_OK;
  hipStream_t s = (hipStream_t)stream;
  const bool vec = H % 8 == 0 && aligned(h, 16) && aligned(w, 16) && aligned(x_out, 16) &&
                   (!delta || (aligned(delta, 16) && aligned(h_out, 16)));
  if (vec && H <= kPartThreads * 8)
    add_rmsnorm_vec_kernel<<<M, kPartThreads, 0, s>>>((const uint16_t*)h, (const uint16_t*)delta, (const uint16_t*)w,
                                                      (uint16_t*)h_out, (uint16_t*)x_out, H, eps);
  else
    add_rmsnorm_kernel<<<M, 256, 0, s>>>((const uint16_t*)h, (const uint16_t*)delta, (const uint16_t*)w,
                                         (uint16_t*)h_out, (uint16_t*)x_out, H, eps);
  return check_launch("gdn_add_rmsnorm");
}

extern "C" int gdn_decode_linear_splits(int M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K < gv::KSTEP || K % gv::KSTEP) return 0;
  int64_t nb;
  int splits, per;
  gv::plan(N, K, &nb, &splits, &per);
  return splits;
}

extern "C" int gdn_decode_linear_packed_partial(const void* x, int64_t x_stride, const void* packed, float* part,
                                                int M, int64_t N, int64_t K, int64_t part_bytes, void* stream) {
  clear_error();
  return decode_linear_launch(true, x, x_stride, packed, 0, nullptr, 0, M, N, K, part, part_bytes, stream, true);
}

extern "C" int gdn_add_rmsnorm_partial(const void* h, const float* part, int splits, const void* w, void* h_out,
                                       void* x_out, int M, int H, float eps, void* stream) {
  clear_error();
  GDN_REQUIRE(h && part && w && h_out && x_out, "gdn_add_rmsnorm_partial: null pointer");
  GDN_REQUIRE(M >= 0 && splits >= 1, "gdn_add_rmsnorm_partial: bad sizes");
  GDN_SUPPORT(H > 0 && H % 8 == 0 && H <= kPartThreads * 8, "gdn_add_rmsnorm_partial: H=%d must be a multiple of 8 <= 8192",
              H);
  GDN_REQUIRE(aligned(h, 16) && aligned(part, 16) && aligned(w, 16) && aligned(h_out, 16) && aligned(x_out, 16),
              "gdn_add_rmsnorm_partial: rows must be 16-byte aligned");
  if (M == 0) return GDN_OK;
  hipStream_t s = (hipStream_t)stream;
  add_rmsnorm_part_kernel<<<M, kPartThreads, 0, s>>>((const uint16_t*)h, part, splits, M, (const uint16_t*)w,
                                                     (uint16_t*)h_out, (uint16_t*)x_out, H, eps);
  return check_launch("gdn_add_rmsnorm_partial");
}

extern "C" int gdn_swiglu_partial(const float* part, int splits, void* out, int M, int64_t m, void* stream) {
  clear_error();
  GDN_REQUIRE(part && out, "gdn_swiglu_partial: null pointer");
  GDN_REQUIRE(M >= 0 && splits >= 1 && m > 0 && m % 8 == 0, "gdn_swiglu_partial: bad sizes (m a multiple of 8)");
  GDN_REQUIRE(aligned(part, 16) && aligned(out, 16), "gdn_swiglu_partial: part and out must be 16-byte aligned");
  if (M == 0) return GDN_OK;
  const int64_t pieces = (int64_t)M * (m / 8);
  swiglu_part_kernel<<<(unsigned)((pieces + 255) / 256), 256, 0, (hipStream_t)stream>>>(part, splits, M, m,
                                                                                        (uint16_t*)out);
  return check_launch("gdn_swiglu_partial");
}
