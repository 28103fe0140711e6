// Decode-side GDN kernels for gfx950: single-token recurrent step, conv state update, gated
// RMSNorm, and the fused decode layer core that chains all of them in one pass over the state.
//
// The recurrent step is an HBM-bound read-modify-write of an fp32 [D, D] state per (slot, value
// head).  It is computed in ONE pass over the state with the algebra
//     m = gamma * S^T k,   delta = beta * (v - m),   o = gamma * S^T q + (k . q) * delta,
//     S' = gamma * S + k delta^T,
// which equals the reference's decay -> read -> delta -> write -> readout sequence
// (src/recurrent_single_step.py:27-31) up to fp32 rounding order.  256 threads own one 128x128
// state: thread t holds columns 4*(t%32)..+3 of rows (t/32) + 8*m, m < 16, as 16 float4 loads, so
// every load instruction of a wave covers two adjacent 512-byte rows (1 KiB contiguous).
#include "gdn_device.h"
#include "gdn_internal.h"

namespace gdn {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;            // head dim (dk == dv)
constexpr int kHeadThreads = 256;  // threads per value head
constexpr int kRowsPerThread = 16; // kD / (kHeadThreads / 32)
constexpr float kInvSqrtD = 0.08838834764831845f;  // (float)(1 / sqrt(128))

struct StateRegs {
  f32x4 s[kRowsPerThread];
};

// Issue the 16 float4 loads of this thread's slice of a [D, D] fp32 state.
__device__ __forceinline__ void state_load(StateRegs& r, const float* S, int t) {
  const f32x4* p = reinterpret_cast<const f32x4*>(S) + (t >> 5) * 32 + (t & 31);
#pragma unroll
  for (int m = 0; m < kRowsPerThread; ++m) r.s[m] = p[m * 8 * 32];
}

__device__ __forceinline__ void state_zero(StateRegs& r) {
#pragma unroll
  for (int m = 0; m < kRowsPerThread; ++m) r.s[m] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// Column partial sums of S^T k and S^T q over this thread's 16 rows.
__device__ __forceinline__ void state_partials(const StateRegs& r, const float* kn, const float* qs,
                                               int t, f32x4& pk, f32x4& pq) {
  pk = f32x4{0.f, 0.f, 0.f, 0.f};
  pq = f32x4{0.f, 0.f, 0.f, 0.f};
  const int rg = t >> 5;
#pragma unroll
  for (int m = 0; m < kRowsPerThread; ++m) {
    const float kr = kn[rg + 8 * m], qr = qs[rg + 8 * m];
    pk += r.s[m] * kr;
    pq += r.s[m] * qr;
  }
}

// S' = gamma * S + k delta^T, stored to Sout.
__device__ __forceinline__ void state_update_store(StateRegs& r, float* Sout, const float* kn,
                                                   const float* delta, float gamma, int t) {
  const int rg = t >> 5, cg = t & 31;
  const f32x4 d = *reinterpret_cast<const f32x4*>(delta + 4 * cg);
  f32x4* p = reinterpret_cast<f32x4*>(Sout) + rg * 32 + cg;
#pragma unroll
  for (int m = 0; m < kRowsPerThread; ++m) {
    const float kr = kn[rg + 8 * m];
    p[m * 8 * 32] = r.s[m] * gamma + d * kr;
  }
}

// l2norm of a D=128 vector held as 2 values per lane, in the input dtype's precision
// (x*x, the fp32-accumulated sum, +eps, rsqrt and the product each rounded like one torch op).
template <bool kBf16>
__device__ __forceinline__ void l2norm_pair(float& x0, float& x1) {
  auto rd = [](float v) { return kBf16 ? rbf(v) : v; };
  float s = wave_sum(rd(x0 * x0) + rd(x1 * x1));
  s = rd(rd(s) + 1e-6f);
  const float inv = rd(rsqrt_f(s));
  x0 = rd(x0 * inv);
  x1 = rd(x1 * inv);
}

// ============================================================================================
// Standalone recurrent step: one workgroup (256 threads) per (slot, value head).
// ============================================================================================
template <typename InT, typename BetaT>
__global__ __launch_bounds__(kHeadThreads) void recurrent_step_kernel(
    const InT* __restrict__ q, int64_t q_stride, const InT* __restrict__ k, int64_t k_stride,
    const InT* __restrict__ v, int64_t v_stride, const float* __restrict__ g,
    const BetaT* __restrict__ beta, const float* state_in, float* state_out, InT* __restrict__ out,
    int Hqk, int Hv, int use_l2) {
  __shared__ float s_q[kD], s_k[kD], s_v[kD], s_delta[kD];
  __shared__ float s_red[2][4][kD];
  __shared__ float s_sc[4];  // gamma, beta, k.q
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int n = blockIdx.x / Hv, h = blockIdx.x % Hv;
  const int hk = h / (Hv / Hqk);
  const int64_t sidx = ((int64_t)n * Hv + h) * kD * kD;

  StateRegs S;
  if (state_in) state_load(S, state_in + sidx, t);
  else state_zero(S);

  constexpr bool kBf = sizeof(InT) == 2;
  if (w == 0) {
    const InT* qp = q + n * q_stride + (int64_t)hk * kD;
    const InT* kp = k + n * k_stride + (int64_t)hk * kD;
    float q0 = Elem<InT>::load(qp + lane), q1 = Elem<InT>::load(qp + lane + 64);
    float k0 = Elem<InT>::load(kp + lane), k1 = Elem<InT>::load(kp + lane + 64);
    if (use_l2) {
      l2norm_pair<kBf>(q0, q1);
      l2norm_pair<kBf>(k0, k1);
    }
    q0 *= kInvSqrtD;
    q1 *= kInvSqrtD;
    s_q[lane] = q0; s_q[lane + 64] = q1;
    s_k[lane] = k0; s_k[lane + 64] = k1;
    const float kq = wave_sum(k0 * q0 + k1 * q1);
    if (lane == 0) {
      s_sc[0] = expf(g[(int64_t)n * Hv + h]);
      s_sc[1] = Elem<BetaT>::load(beta + (int64_t)n * Hv + h);
      s_sc[2] = kq;
    }
  } else if (w == 1) {
    const InT* vp = v + n * v_stride + (int64_t)h * kD;
    s_v[lane] = Elem<InT>::load(vp + lane);
    s_v[lane + 64] = Elem<InT>::load(vp + lane + 64);
  }
  __syncthreads();

  f32x4 pk, pq;
  state_partials(S, s_k, s_q, t, pk, pq);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    pk[e] += __shfl_xor(pk[e], 32, kWave);
    pq[e] += __shfl_xor(pq[e], 32, kWave);
  }
  if (lane < 32) {
    *reinterpret_cast<f32x4*>(&s_red[0][w][4 * lane]) = pk;
    *reinterpret_cast<f32x4*>(&s_red[1][w][4 * lane]) = pq;
  }
  __syncthreads();

  const float gamma = s_sc[0], bt = s_sc[1], kq = s_sc[2];
  if (t < kD) {
    const float mk = s_red[0][0][t] + s_red[0][1][t] + s_red[0][2][t] + s_red[0][3][t];
    const float mq = s_red[1][0][t] + s_red[1][1][t] + s_red[1][2][t] + s_red[1][3][t];
    const float delta = (s_v[t] - gamma * mk) * bt;
    s_delta[t] = delta;
    Elem<InT>::store(out + ((int64_t)n * Hv + h) * kD + t, gamma * mq + kq * delta);
  }
  __syncthreads();
  if (state_out) state_update_store(S, state_out + sidx, s_k, s_delta, gamma, t);
}

// ============================================================================================
// Conv update (elem_conv_update): one thread per (slot, channel).
// ============================================================================================
// window = [state[1..K-1], x]; out = silu(bf16(sum_i bf16(window_i * w_i)) (+ bias)); state <- window.
__device__ __forceinline__ float conv_channel(uint16_t* st, const uint16_t* wt, float bias, bool has_bias,
                                              uint16_t xv, int K) {
  float acc = 0.f;
  if (K == 4) {
    const uint2 sv = *reinterpret_cast<const uint2*>(st);
    const uint2 wv = *reinterpret_cast<const uint2*>(wt);
    const uint16_t win[4] = {(uint16_t)(sv.x >> 16), (uint16_t)(sv.y & 0xffff), (uint16_t)(sv.y >> 16), xv};
    const uint16_t ww[4] = {(uint16_t)(wv.x & 0xffff), (uint16_t)(wv.x >> 16), (uint16_t)(wv.y & 0xffff),
                            (uint16_t)(wv.y >> 16)};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc += rbf(bf2f(win[i]) * bf2f(ww[i]));
    uint2 nv;
    nv.x = (uint32_t)win[0] | ((uint32_t)win[1] << 16);
    nv.y = (uint32_t)win[2] | ((uint32_t)win[3] << 16);
    *reinterpret_cast<uint2*>(st) = nv;
  } else {
    uint16_t win[8];
    for (int i = 0; i < K - 1; ++i) win[i] = st[i + 1];
    win[K - 1] = xv;
    for (int i = 0; i < K; ++i) acc += rbf(bf2f(win[i]) * bf2f(wt[i]));
    for (int i = 0; i < K; ++i) st[i] = win[i];
  }
  float o = rbf(acc);
  if (has_bias) o = rbf(o + bias);
  return rbf(silu_f(o));
}

__global__ __launch_bounds__(256) void conv_update_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                                          uint16_t* __restrict__ state,
                                                          const uint16_t* __restrict__ weight,
                                                          const uint16_t* __restrict__ bias,
                                                          uint16_t* __restrict__ out, int64_t out_stride,
                                                          int N, int C, int K) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)N * C) return;
  const int n = (int)(i / C), c = (int)(i % C);
  const float b = bias ? bf2f(bias[c]) : 0.f;
  const float o = conv_channel(state + i * K, weight + (int64_t)c * K, b, bias != nullptr,
                               x[n * x_stride + c], K);
  out[n * out_stride + c] = f2bf(o);
}

// ============================================================================================
// Gated RMSNorm (HF Qwen3_5RMSNormGated): one wave per row, D % 64 == 0, D <= 512.
// ============================================================================================
template <bool kWBf16>
__device__ __forceinline__ void gated_norm_row(const float* x, const uint16_t* gate, const void* weight,
                                               uint16_t* out, int D, float eps, int lane) {
  // x: this lane's D/64 values (bf16-rounded); element j*64 + lane.
  float ss = 0.f;
  const int nper = D / 64;
  for (int j = 0; j < nper; ++j) ss += x[j] * x[j];
  ss = wave_sum(ss);
  const float inv = rsqrt_f(ss / (float)D + eps);
  for (int j = 0; j < nper; ++j) {
    const int c = j * 64 + lane;
    const float xn = rbf(x[j] * inv);
    float y;
    if (kWBf16) y = rbf(bf2f(reinterpret_cast<const uint16_t*>(weight)[c]) * xn);
    else y = reinterpret_cast<const float*>(weight)[c] * xn;
    out[c] = f2bf(y * silu_f(bf2f(gate[c])));
  }
}

template <bool kWBf16>
__global__ __launch_bounds__(256) void gated_rmsnorm_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                                            const uint16_t* __restrict__ gate,
                                                            int64_t gate_stride, const void* weight,
                                                            uint16_t* __restrict__ out, int64_t rows, int D,
                                                            float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  float xv[8];
  for (int j = 0; j < D / 64; ++j) xv[j] = bf2f(x[row * x_stride + j * 64 + lane]);
  gated_norm_row<kWBf16>(xv, gate + row * gate_stride, weight, out + row * D, D, eps, lane);
}

// ============================================================================================
// Fused decode layer core: one workgroup per (slot, key head) owning its R value heads, so every
// conv channel it reads is also written by it alone (the in-place conv state needs no grid sync).
// ============================================================================================
template <int R, bool kWBf16>
__global__ __launch_bounds__(kHeadThreads* R) void decode_fused_kernel(
    const uint16_t* __restrict__ mixed, int64_t mixed_stride, const uint16_t* __restrict__ z,
    int64_t z_stride, const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, int64_t ab_stride,
    uint16_t* __restrict__ conv_state, const uint16_t* __restrict__ conv_w,
    const uint16_t* __restrict__ conv_b, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const void* norm_w, float eps, float* rec_state,
    uint16_t* __restrict__ out, int Hk, int K) {
  __shared__ float s_q[kD], s_k[kD], s_v[R][kD], s_delta[R][kD];
  __shared__ float s_red[R][2][4][kD];
  __shared__ float s_gamma[R], s_beta[R], s_kq;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int j = t / kHeadThreads, tl = t % kHeadThreads, wl = tl >> 6;  // head in group, local ids
  const int n = blockIdx.x / Hk, hk = blockIdx.x % Hk;
  const int Hv = Hk * R;
  const int h = hk * R + j;
  const int C = (2 * Hk + Hv) * kD;
  const int64_t sidx = ((int64_t)n * Hv + h) * kD * kD;

  StateRegs S;
  state_load(S, rec_state + sidx, tl);  // in flight while the prologue runs

  // conv update + SiLU for the q, k and R v heads of this group
  const uint16_t* xr = mixed + n * mixed_stride;
  for (int e = t; e < (2 + R) * kD; e += kHeadThreads * R) {
    int ch;
    float* dst;
    if (e < kD) { ch = hk * kD + e; dst = &s_q[e]; }
    else if (e < 2 * kD) { ch = Hk * kD + hk * kD + (e - kD); dst = &s_k[e - kD]; }
    else { const int vv = e - 2 * kD; ch = 2 * Hk * kD + hk * R * kD + vv; dst = &s_v[0][0] + vv; }
    const float bb = conv_b ? bf2f(conv_b[ch]) : 0.f;
    *dst = conv_channel(conv_state + ((int64_t)n * C + ch) * K, conv_w + (int64_t)ch * K, bb,
                        conv_b != nullptr, xr[ch], K);
  }
  if (t < R) {
    const int hh = hk * R + t;
    const float bv = bf2f(b[n * ab_stride + hh]);
    const float av = bf2f(a[n * ab_stride + hh]);
    s_beta[t] = rbf(sigmoid_f(bv));
    const float gg = -expf(A_log[hh]) * softplus_f(av + dt_bias[hh]);
    s_gamma[t] = expf(gg);
  }
  __syncthreads();
  if (wv == 0) {
    float q0 = s_q[lane], q1 = s_q[lane + 64], k0 = s_k[lane], k1 = s_k[lane + 64];
    l2norm_pair<true>(q0, q1);
    l2norm_pair<true>(k0, k1);
    q0 *= kInvSqrtD;
    q1 *= kInvSqrtD;
    const float kq = wave_sum(k0 * q0 + k1 * q1);
    s_q[lane] = q0; s_q[lane + 64] = q1;
    s_k[lane] = k0; s_k[lane + 64] = k1;
    if (lane == 0) s_kq = kq;
  }
  __syncthreads();

  f32x4 pk, pq;
  state_partials(S, s_k, s_q, tl, pk, pq);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    pk[e] += __shfl_xor(pk[e], 32, kWave);
    pq[e] += __shfl_xor(pq[e], 32, kWave);
  }
  if (lane < 32) {
    *reinterpret_cast<f32x4*>(&s_red[j][0][wl][4 * lane]) = pk;
    *reinterpret_cast<f32x4*>(&s_red[j][1][wl][4 * lane]) = pq;
  }
  __syncthreads();

  const float gamma = s_gamma[j];
  if (wl == 0) {
    const float bt = s_beta[j], kq = s_kq;
    float o[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = lane + 64 * u;
      const float mk = s_red[j][0][0][c] + s_red[j][0][1][c] + s_red[j][0][2][c] + s_red[j][0][3][c];
      const float mq = s_red[j][1][0][c] + s_red[j][1][1][c] + s_red[j][1][2][c] + s_red[j][1][3][c];
      const float delta = (s_v[j][c] - gamma * mk) * bt;
      s_delta[j][c] = delta;
      o[u] = rbf(gamma * mq + kq * delta);  // the recurrent output is bf16 before the norm
    }
    gated_norm_row<kWBf16>(o, z + n * z_stride + (int64_t)h * kD, norm_w,
                           out + ((int64_t)n * Hv + h) * kD, kD, eps, lane);
  }
  __syncthreads();
  state_update_store(S, rec_state + sidx, s_k, s_delta[j], gamma, tl);
}

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_recurrent_step(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                                  const void* v, int64_t v_stride, const float* g, const void* beta,
                                  int beta_dtype, const float* state_in, float* state_out, void* out,
                                  int N, int Hqk, int Hv, int D, int in_dtype, int use_qk_l2norm,
                                  void* stream) {
  clear_error();
  GDN_REQUIRE(q && k && v && g && beta && out, "gdn_recurrent_step: null input/output pointer");
  GDN_REQUIRE(N >= 0 && Hqk > 0 && Hv > 0 && Hv % Hqk == 0,
              "gdn_recurrent_step: bad head counts Hqk=%d Hv=%d", Hqk, Hv);
  GDN_SUPPORT(D == kD, "gdn_recurrent_step: head dim %d unsupported (needs %d)", D, kD);
  GDN_REQUIRE(in_dtype == GDN_F32 || in_dtype == GDN_BF16, "gdn_recurrent_step: bad in_dtype");
  GDN_REQUIRE(beta_dtype == GDN_F32 || beta_dtype == GDN_BF16, "gdn_recurrent_step: bad beta_dtype");
  GDN_REQUIRE((!state_in || aligned(state_in, 16)) && (!state_out || aligned(state_out, 16)),
              "gdn_recurrent_step: state must be 16-byte aligned");
  if (N == 0) return GDN_OK;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid(N * Hv), block(kHeadThreads);
#define GDN_RS_LAUNCH(IT, BT)                                                                       \
  recurrent_step_kernel<IT, BT><<<grid, block, 0, s>>>(                                             \
      (const IT*)q, q_stride, (const IT*)k, k_stride, (const IT*)v, v_stride, g, (const BT*)beta,   \
      state_in, state_out, (IT*)out, Hqk, Hv, use_qk_l2norm)
  if (in_dtype == GDN_BF16) {
    if (beta_dtype == GDN_BF16) GDN_RS_LAUNCH(uint16_t, uint16_t);
    else GDN_RS_LAUNCH(uint16_t, float);
  } else {
    if (beta_dtype == GDN_BF16) GDN_RS_LAUNCH(float, uint16_t);
    else GDN_RS_LAUNCH(float, float);
  }
#undef GDN_RS_LAUNCH
  return check_launch("gdn_recurrent_step");
}

extern "C" int gdn_conv_update(const void* x, int64_t x_stride, void* state, const void* weight,
                               const void* bias, void* out, int64_t out_stride, int N, int C, int K,
                               void* stream) {
  clear_error();
  GDN_REQUIRE(x && state && weight && out, "gdn_conv_update: null pointer");
  GDN_REQUIRE(N >= 0 && C > 0 && K >= 1, "gdn_conv_update: bad sizes N=%d C=%d K=%d", N, C, K);
  GDN_SUPPORT(K <= 8, "gdn_conv_update: kernel size %d > 8", K);
  GDN_REQUIRE(K != 4 || (aligned(state, 8) && aligned(weight, 8)),
              "gdn_conv_update: state/weight must be 8-byte aligned for K=4");
  if (N == 0) return GDN_OK;
  const int64_t total = (int64_t)N * C;
  conv_update_kernel<<<(unsigned)((total + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)x, x_stride, (uint16_t*)state, (const uint16_t*)weight, (const uint16_t*)bias,
      (uint16_t*)out, out_stride, N, C, K);
  return check_launch("gdn_conv_update");
}

extern "C" int gdn_gated_rmsnorm(const void* x, int64_t x_stride, const void* gate, int64_t gate_stride,
                                 const void* weight, int w_dtype, void* out, int64_t rows, int D, float eps,
                                 void* stream) {
  clear_error();
  GDN_REQUIRE(x && gate && weight && out, "gdn_gated_rmsnorm: null pointer");
  GDN_REQUIRE(rows >= 0, "gdn_gated_rmsnorm: negative rows");
  GDN_SUPPORT(D > 0 && D % 64 == 0 && D <= 512, "gdn_gated_rmsnorm: D=%d must be a multiple of 64 <= 512", D);
  GDN_REQUIRE(w_dtype == GDN_F32 || w_dtype == GDN_BF16, "gdn_gated_rmsnorm: bad w_dtype");
  if (rows == 0) return GDN_OK;
  const unsigned blocks = (unsigned)((rows + 3) / 4);
  if (w_dtype == GDN_BF16)
    gated_rmsnorm_kernel<true><<<blocks, 256, 0, (hipStream_t)stream>>>(
        (const uint16_t*)x, x_stride, (const uint16_t*)gate, gate_stride, weight, (uint16_t*)out, rows, D, eps);
  else
    gated_rmsnorm_kernel<false><<<blocks, 256, 0, (hipStream_t)stream>>>(
        (const uint16_t*)x, x_stride, (const uint16_t*)gate, gate_stride, weight, (uint16_t*)out, rows, D, eps);
  return check_launch("gdn_gated_rmsnorm");
}

extern "C" int gdn_decode_fused(const void* mixed, int64_t mixed_stride, const void* z, int64_t z_stride,
                                const void* a, const void* b, int64_t ab_stride, void* conv_state,
                                const void* conv_w, const void* conv_b, const float* A_log,
                                const float* dt_bias, const void* norm_w, int norm_w_dtype, float eps,
                                float* rec_state, void* out, int N, int Hk, int Hv, int D, int K,
                                void* stream) {
  clear_error();
  GDN_REQUIRE(mixed && z && a && b && conv_state && conv_w && A_log && dt_bias && norm_w && rec_state && out,
              "gdn_decode_fused: null pointer");
  GDN_REQUIRE(N >= 0 && Hk > 0 && Hv > 0 && Hv % Hk == 0, "gdn_decode_fused: bad heads Hk=%d Hv=%d", Hk, Hv);
  GDN_SUPPORT(D == kD, "gdn_decode_fused: head dim %d unsupported (needs %d)", D, kD);
  GDN_SUPPORT(K >= 1 && K <= 8, "gdn_decode_fused: conv kernel %d unsupported", K);
  GDN_REQUIRE(norm_w_dtype == GDN_F32 || norm_w_dtype == GDN_BF16, "gdn_decode_fused: bad norm_w_dtype");
  GDN_REQUIRE(aligned(rec_state, 16), "gdn_decode_fused: rec_state must be 16-byte aligned");
  GDN_REQUIRE(K != 4 || (aligned(conv_state, 8) && aligned(conv_w, 8)),
              "gdn_decode_fused: conv state/weight must be 8-byte aligned");
  const int R = Hv / Hk;
  GDN_SUPPORT(R >= 1 && R <= 4, "gdn_decode_fused: value/key head ratio %d unsupported (1..4)", R);
  if (N == 0) return GDN_OK;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid(N * Hk);
#define GDN_DF_LAUNCH(RR, WB)                                                                         \
  decode_fused_kernel<RR, WB><<<grid, kHeadThreads * RR, 0, s>>>(                                     \
      (const uint16_t*)mixed, mixed_stride, (const uint16_t*)z, z_stride, (const uint16_t*)a,         \
      (const uint16_t*)b, ab_stride, (uint16_t*)conv_state, (const uint16_t*)conv_w,                  \
      (const uint16_t*)conv_b, A_log, dt_bias, norm_w, eps, rec_state, (uint16_t*)out, Hk, K)
#define GDN_DF_R(WB)                      \
  switch (R) {                            \
    case 1: GDN_DF_LAUNCH(1, WB); break;  \
    case 2: GDN_DF_LAUNCH(2, WB); break;  \
    case 3: GDN_DF_LAUNCH(3, WB); break;  \
    default: GDN_DF_LAUNCH(4, WB); break; \
  }
  if (norm_w_dtype == GDN_BF16) { GDN_DF_R(true) }
  else { GDN_DF_R(false) }
#undef GDN_DF_R
#undef GDN_DF_LAUNCH
  return check_launch("gdn_decode_fused");
}
