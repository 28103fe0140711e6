// Decode-side GDN kernels for gfx950: single-token recurrent step, conv state update, gated
// RMSNorm, and the fused decode layer core that chains all of them in one pass over the state.
//
// The recurrent step is an HBM-bound read-modify-write of an fp32 [D, D] state per (slot, value
// head).  It is computed in ONE pass over the state with the algebra
//     m = gamma * S^T k,   delta = beta * (v - m),   o = gamma * S^T q + (k . q) * delta,
//     S' = gamma * S + k delta^T,
// which equals the reference's decay -> read -> delta -> write -> readout sequence
// (src/recurrent_single_step.py:27-31) up to fp32 rounding order.  256 threads (4 waves) own one
// 128x128 state: thread t holds columns 4*(t%32)..+3 of rows t/32 + 8*m, m < 16, as 16 float4
// loads, so every load instruction of a wave covers two adjacent 512-byte rows (1 KiB contiguous;
// measured faster than giving each wave whole columns).  Column sums combine the wave's two row
// groups with one register swap (v_permlane32_swap) and the four waves through LDS; after that
// each thread derives delta for its own 4 columns and streams its rows straight back.
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

// This thread's first float4 of the state: row t/32, columns 4*(t%32)..+3 (t = 0..255).
__device__ __forceinline__ int state_f4(int t) { return (t >> 5) * 32 + (t & 31); }

// Issue the 16 float4 loads of this thread's slice of a [D, D] fp32 state (rows t/32 + 8m).  The
// state is streamed once per step, so loads and stores carry the non-temporal hint (measured ~20%
// faster than plain accesses for this read-modify-write on MI355X).
__device__ __forceinline__ void state_load(StateRegs& r, const float* S, int t) {
  const f32x4* p = reinterpret_cast<const f32x4*>(S) + state_f4(t);
#pragma unroll
  for (int m = 0; m < kRowsPerThread; ++m) {
    r.s[m] = __builtin_nontemporal_load(p + m * 8 * 32);
    // keep the loads in row order, so column sums taken in row order wait for one row at a time
    __builtin_amdgcn_sched_barrier(0);
  }
}

__device__ __forceinline__ void state_zero(StateRegs& r) {
#pragma unroll
  for (int m = 0; m < kRowsPerThread; ++m) r.s[m] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// Column sums of S^T x over this thread's 16 rows plus the other row group of its wave
// (lane ^ 32, a register swap); lanes 0..31 then publish the wave's partials to red[4][D].
__device__ __forceinline__ void state_partial(const StateRegs& r, const float* xr, int t, float (*red)[kD]) {
  f32x4 p = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < kRowsPerThread; ++m) p += r.s[m] * xr[m];
#pragma unroll
  for (int e = 0; e < 4; ++e) p[e] = xor32_sum(p[e]);
  const int lane = t & 63, w = t >> 6;
  if (lane < 32) *reinterpret_cast<f32x4*>(&red[w][4 * lane]) = p;
}

// This thread's 16 entries of a length-D vector in LDS (rows t/32 + 8m).
__device__ __forceinline__ void row_values(const float* x, int t, float* xr) {
#pragma unroll
  for (int m = 0; m < kRowsPerThread; ++m) xr[m] = x[(t >> 5) + 8 * m];
}

// Both column sums (k and q) of the standalone step, published to red[2][4][D].
__device__ __forceinline__ void state_partials(const StateRegs& r, const float* kn, const float* qs,
                                               int t, float (*red)[4][kD]) {
  float xr[kRowsPerThread];
  row_values(kn, t, xr);
  state_partial(r, xr, t, red[0]);
  row_values(qs, t, xr);
  state_partial(r, xr, t, red[1]);
}

// Sum of the four waves' partials for column c.
__device__ __forceinline__ float red_sum(const float (*red)[4][kD], int which, int c) {
  return red[which][0][c] + red[which][1][c] + red[which][2][c] + red[which][3][c];
}

// delta for this thread's 4 columns, then S' = gamma S + k delta^T streamed to Sout.
__device__ __forceinline__ void state_update_store(const StateRegs& r, float* Sout, const float* kn,
                                                   const float* v, const float (*red)[4][kD],
                                                   float gamma, float beta, int t) {
  const int rg = t >> 5, cg = t & 31;
  f32x4 d;
#pragma unroll
  for (int e = 0; e < 4; ++e) d[e] = (v[4 * cg + e] - gamma * red_sum(red, 0, 4 * cg + e)) * beta;
  f32x4* p = reinterpret_cast<f32x4*>(Sout) + state_f4(t);
#pragma unroll
  for (int m = 0; m < kRowsPerThread; ++m)
    __builtin_nontemporal_store(r.s[m] * gamma + d * kn[rg + 8 * m], p + m * 8 * 32);
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
  __shared__ float s_q[kD], s_k[kD], s_v[kD];
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

  state_partials(S, s_k, s_q, t, s_red);
  __syncthreads();
  const float gamma = s_sc[0], bt = s_sc[1], kq = s_sc[2];
  if (state_out) state_update_store(S, state_out + sidx, s_k, s_v, s_red, gamma, bt, t);
  if (t < kD) {
    const float delta = (s_v[t] - gamma * red_sum(s_red, 0, t)) * bt;
    Elem<InT>::store(out + ((int64_t)n * Hv + h) * kD + t, gamma * red_sum(s_red, 1, t) + kq * delta);
  }
}

// ============================================================================================
// Conv update (elem_conv_update): one thread per (slot, channel).
// ============================================================================================
// window = [state[1..K-1], x]; conv = bf16(sum_i bf16(window_i * w_i)) (+ bias, rounded); state <- window.
// The callers apply the SiLU (silu_bf16_n).
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
  return o;
}

// K == 4 conv split in two halves so the loads can be issued ahead of the state stream.
struct Conv4 {
  uint2 s, w;
  uint16_t x;
};
__device__ __forceinline__ void conv4_load(Conv4& c, const uint16_t* st, const uint16_t* wt, const uint16_t* xp) {
  c.s = *reinterpret_cast<const uint2*>(st);
  c.w = *reinterpret_cast<const uint2*>(wt);
  c.x = *xp;
}
// The shifted window is returned in *nw (the caller stores it, possibly much later).
__device__ __forceinline__ float conv4_finish(const Conv4& c, uint2* nw, float bias, bool has_bias) {
  const uint16_t win[4] = {(uint16_t)(c.s.x >> 16), (uint16_t)(c.s.y & 0xffff), (uint16_t)(c.s.y >> 16), c.x};
  const uint16_t ww[4] = {(uint16_t)(c.w.x & 0xffff), (uint16_t)(c.w.x >> 16), (uint16_t)(c.w.y & 0xffff),
                          (uint16_t)(c.w.y >> 16)};
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) acc += rbf(bf2f(win[i]) * bf2f(ww[i]));
  uint2 nv;
  nv.x = (uint32_t)win[0] | ((uint32_t)win[1] << 16);
  nv.y = (uint32_t)win[2] | ((uint32_t)win[3] << 16);
  *nw = nv;
  float o = rbf(acc);
  if (has_bias) o = rbf(o + bias);
  return o;
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
  out[n * out_stride + c] = silu_bf16(o);
}

// ============================================================================================
// Gated RMSNorm (HF Qwen3_5RMSNormGated): one wave per row, D % 64 == 0, D <= 512.
// ============================================================================================
// Every gated norm here (and the one fused into the prefill output kernel, which repeats
// gated_rmsnorm128_kernel's arithmetic) takes the row factor from the hardware reciprocal square
// root and SiLU from the hardware exp and reciprocal: outputs within one bf16 ulp of torch's.
// x, gate and weight hold this lane's D/64 values (element j*64 + lane; x bf16-rounded), all
// loaded beforehand so a caller can fetch them long before the row is ready.
__device__ __forceinline__ void gated_norm_row(const float* x, const float* gate, const float* weight, bool w_bf16,
                                               uint16_t* out, int D, float eps, int lane) {
  float ss = 0.f;
  const int nper = D / 64;
  for (int j = 0; j < nper; ++j) ss += x[j] * x[j];
  ss = wave_sum(ss);
  const float inv = rsq_fast(ss / (float)D + eps);
  for (int j = 0; j < nper; ++j) {
    const float xn = rbf(x[j] * inv);
    const float y = w_bf16 ? rbf(weight[j] * xn) : weight[j] * xn;
    out[j * 64 + lane] = f2bf(y * silu_fast(gate[j]));
  }
}

__device__ __forceinline__ float load_weight(const void* w, bool w_bf16, int c) {
  return w_bf16 ? bf2f(reinterpret_cast<const uint16_t*>(w)[c]) : reinterpret_cast<const float*>(w)[c];
}

// D = 128 with 16-byte aligned rows: 16 lanes per row, 8 elements per lane, 16 rows per workgroup.
template <bool kWBf16>
__global__ __launch_bounds__(256) void gated_rmsnorm128_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                                               const uint16_t* __restrict__ gate, int64_t gate_stride,
                                                               const void* weight, uint16_t* __restrict__ out,
                                                               int64_t rows, float eps) {
  typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
  const int sub = threadIdx.x & 15;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const bool ok = row < rows;
  const int64_t r = ok ? row : 0;
  const u16x8 xv = *reinterpret_cast<const u16x8*>(x + r * x_stride + 8 * sub);
  const u16x8 zv = *reinterpret_cast<const u16x8*>(gate + r * gate_stride + 8 * sub);
  float xf[8], ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    xf[e] = bf2f(xv[e]);
    ss += xf[e] * xf[e];
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) ss += __shfl_xor(ss, o, kWave);
  const float inv = rsq_fast(ss / 128.0f + eps);
  u16x8 ov;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int c = 8 * sub + e;
    const float xn = rbf(xf[e] * inv);
    const float y = kWBf16 ? rbf(bf2f(reinterpret_cast<const uint16_t*>(weight)[c]) * xn)
                           : reinterpret_cast<const float*>(weight)[c] * xn;
    ov[e] = f2bf(y * silu_fast(bf2f(zv[e])));
  }
  if (ok) *reinterpret_cast<u16x8*>(out + row * 128 + 8 * sub) = ov;
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
  float xv[8], gv[8], wv[8];
  for (int j = 0; j < D / 64; ++j) {
    const int c = j * 64 + lane;
    xv[j] = bf2f(x[row * x_stride + c]);
    gv[j] = bf2f(gate[row * gate_stride + c]);
    wv[j] = load_weight(weight, kWBf16, c);
  }
  gated_norm_row(xv, gv, wv, kWBf16, out + row * D, D, eps, lane);
}

// ============================================================================================
// Fused decode layer core: one workgroup per (slot, key head) owning its R value heads, so every
// conv channel it reads is also written by it alone (the in-place conv state needs no grid sync).
// All R * 256 threads stream every one of the R value heads' states: each thread holds 4 columns of
// 128 / (8 R) rows of each head, the heads' loads go out in head order, and per head the workgroup
// forms the column sums, delta and the stores while the later heads are still arriving.  R + 2
// waves (spread over the workgroup) also convolve the group's q, k and R v channel blocks (conv
// update + SiLU, l2norm), one more computes the gating, and one wave per head forms the readout
// o = gamma S^T q + (k.q) delta with its gated RMSNorm.  Their small loads (conv window / weight /
// input, gating inputs, the readout's gate and norm weight) are issued first and kept as raw bits
// until the wave's state loads are out, so the prologue runs while the state is in flight; the
// K = 4 conv window write-back comes after the state stores, so no write sits in the read phase.  Everything read or written once per step (state, conv windows, input, gate, output)
// carries the non-temporal hint: measured 0.5 us/layer faster than cached accesses for the small
// tensors at 16 slots x 32 heads.
// (A separate control wave doing all of the prologue and readout was measured 18% slower: one
// wave convolving all (R+2)*128 channels puts the prologue on the critical path.)
// ============================================================================================
__device__ __forceinline__ int conv_group_ch0(int g, int hk, int Hk, int R) {
  return g == 0 ? hk * kD : (g == 1 ? (Hk + hk) * kD : (2 * Hk + hk * R + (g - 2)) * kD);
}

template <int R, bool kWBf16>
__global__ __launch_bounds__(kHeadThreads * R) void decode_fused_kernel(
    const uint16_t* __restrict__ mixed, int64_t mixed_stride, const uint16_t* __restrict__ z,
    int64_t z_stride, const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, int64_t ab_stride,
    uint16_t* __restrict__ conv_state, const uint16_t* __restrict__ conv_w,
    const uint16_t* __restrict__ conv_b, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const void* norm_w, float eps, float* rec_state,
    uint16_t* __restrict__ out, const uint8_t* __restrict__ active, int Hk, int K) {
  constexpr int kGroups = R + 2;  // conv channel blocks of 128: q, k, v_0..v_{R-1}
  constexpr int kWaves = 4 * R;                   // waves of the workgroup
  constexpr int kRG = kHeadThreads * R / 32;      // row groups of 32 threads (a row's 32 float4)
  constexpr int kRows = (kD + kRG - 1) / kRG;     // rows of each head's state per thread
  __shared__ float s_q[kD], s_k[kD], s_v[R][kD];
  __shared__ float s_red[R][2][kWaves][kD];
  __shared__ float s_gamma[R], s_beta[R];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int j = t / kHeadThreads, tl = t % kHeadThreads, wl = tl >> 6;  // head in group, local ids
  const int n = blockIdx.x / Hk, hk = blockIdx.x % Hk;
  const int Hv = Hk * R;
  if (active && !active[n]) {  // a held or idle slot: states untouched, output rows zero
    if (tl < kD) out[((int64_t)n * Hv + hk * R + j) * kD + tl] = 0;
    return;
  }
  const int h = hk * R + j;
  const int C = (2 * Hk + Hv) * kD;
  const uint16_t* xr = mixed + n * mixed_stride;
  const bool k4 = K == 4;
  const bool bias_on = conv_b != nullptr;
  // prologue roles spread over the heads' waves: role wl * R + j, so the conv groups q, k, v_0.. go
  // to local wave 0 of each head first, then local wave 1, ...; the next role gates, and the last
  // wave of each head reads out
  const int role = wl * R + j;
  const bool conv_wave = role < kGroups;
  const int ch0 = conv_wave ? conv_group_ch0(role, hk, Hk, R) : 0;
  const bool gate_lane = role == kGroups && lane < R;
  const bool read_wave = wl == 3;
  const int oc = 4 * (lane & 31);  // readout lane l owns output columns 4(l % 32)..+3 (both half-waves)

  // ---- phase A: small loads (raw bits), the state stream, the prologue -----------------------
  Conv4 cv[2];
  uint32_t cx[2] = {0u, 0u};
  if (conv_wave && k4) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int ch = ch0 + lane + 64 * u;
      // read-once data (this slot's conv windows and input) streams with the non-temporal hint;
      // the conv weights, shared by every slot, stay cached
      const uint64_t w64 = __builtin_nontemporal_load(reinterpret_cast<const uint64_t*>(conv_state + ((int64_t)n * C + ch) * 4));
      cv[u].s = make_uint2((uint32_t)w64, (uint32_t)(w64 >> 32));
      cv[u].w = *reinterpret_cast<const uint2*>(conv_w + (int64_t)ch * 4);
      cx[u] = __builtin_nontemporal_load(xr + ch);
    }
  }
  uint32_t g_a = 0u, g_b = 0u;
  float g_al = 0.f, g_dt = 0.f;
  if (gate_lane) {
    const int hh = hk * R + lane;
    g_b = b[n * ab_stride + hh];
    g_a = a[n * ab_stride + hh];
    g_al = A_log[hh];
    g_dt = dt_bias[hh];
  }
  uint32_t zr[2] = {0u, 0u}, nwr[4] = {0u, 0u, 0u, 0u};
  if (read_wave) {
    const uint64_t zz = __builtin_nontemporal_load(reinterpret_cast<const uint64_t*>(z + n * z_stride + (int64_t)h * kD + oc));
    zr[0] = (uint32_t)zz;
    zr[1] = (uint32_t)(zz >> 32);
    if (kWBf16) {
      const uint2 ww = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(norm_w) + oc);
      nwr[0] = ww.x;
      nwr[1] = ww.y;
    } else {
      const uint4 ww = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(norm_w) + oc);
      nwr[0] = ww.x; nwr[1] = ww.y; nwr[2] = ww.z; nwr[3] = ww.w;
    }
  }
  // every thread holds columns 4 cg..+3 of rows rg + kRG m of each of the R heads' states; head 0's
  // loads go out first, so its column sums and stores proceed while later heads are still arriving
  const int cg = t & 31, rg = t >> 5;
  f32x4 S[R][kRows];
#pragma unroll
  for (int jj = 0; jj < R; ++jj) {
    const f32x4* p = reinterpret_cast<const f32x4*>(rec_state + ((int64_t)n * Hv + hk * R + jj) * kD * kD);
#pragma unroll
    for (int m = 0; m < kRows; ++m) {
      if (kRG * kRows == kD || rg + kRG * m < kD) S[jj][m] = __builtin_nontemporal_load(p + (rg + kRG * m) * 32 + cg);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // nothing derived from the small loads may be computed before this point
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    pin(cv[u].s.x); pin(cv[u].s.y); pin(cv[u].w.x); pin(cv[u].w.y); pin(cx[u]);
    pin(zr[u]);
  }
  pin(g_a); pin(g_b); pin(g_al); pin(g_dt);
#pragma unroll
  for (int e = 0; e < 4; ++e) pin(nwr[e]);

  uint2 cnew[2];
  if (conv_wave) {
    float x[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int ch = ch0 + lane + 64 * u;
      const float bb = bias_on ? bf2f(conv_b[ch]) : 0.f;
      if (k4) {
        cv[u].x = (uint16_t)cx[u];
        x[u] = conv4_finish(cv[u], &cnew[u], bb, bias_on);
      } else {  // general K: window updated in place here
        x[u] = conv_channel(conv_state + ((int64_t)n * C + ch) * K, conv_w + (int64_t)ch * K, bb, bias_on, xr[ch], K);
      }
    }
    {
      uint16_t sx[2];
      silu_bf16_n<2>(x, sx);
      x[0] = bf2f(sx[0]);
      x[1] = bf2f(sx[1]);
    }
    if (role < 2) {
      l2norm_pair<true>(x[0], x[1]);
      float* dst = role == 0 ? s_q : s_k;
      const float sc = role == 0 ? kInvSqrtD : 1.0f;
      dst[lane] = x[0] * sc;
      dst[lane + 64] = x[1] * sc;
    } else {
      s_v[role - 2][lane] = x[0];
      s_v[role - 2][lane + 64] = x[1];
    }
  }
  if (gate_lane) {
    s_beta[lane] = bf2f(sigmoid_bf16(bf2f((uint16_t)g_b)));
    s_gamma[lane] = expf(-expf(g_al) * softplus_f(bf2f((uint16_t)g_a) + g_dt));
  }
  lds_barrier();  // q, k, v, gamma, beta in LDS; the state loads stay in flight

  // ---- per head, in load order: column sums S^T k and S^T q (two row groups per wave by register
  //      swap, the waves through LDS), delta for this thread's 4 columns, the rows streamed back, and
  //      the head's readout o = gamma S^T q + (k.q) delta with its gated RMSNorm -----------------------
  float kq = 0.f;
  if (read_wave) kq = wave_sum_fast(s_k[lane] * s_q[lane] + s_k[lane + 64] * s_q[lane + 64]);
  float kr[kRows], qr[kRows];
#pragma unroll
  for (int m = 0; m < kRows; ++m) {
    const int row = rg + kRG * m < kD ? rg + kRG * m : 0;
    kr[m] = s_k[row];
    qr[m] = s_q[row];
  }
#pragma unroll
  for (int jj = 0; jj < R; ++jj) {
    {
      f32x4 pk = f32x4{0.f, 0.f, 0.f, 0.f}, pq = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < kRows; ++m)
        if (kRG * kRows == kD || rg + kRG * m < kD) {
          pk += S[jj][m] * kr[m];
          pq += S[jj][m] * qr[m];
        }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pk[e] = xor32_sum(pk[e]);
        pq[e] = xor32_sum(pq[e]);
      }
      if (lane < 32) {
        *reinterpret_cast<f32x4*>(&s_red[jj][0][wv][4 * lane]) = pk;
        *reinterpret_cast<f32x4*>(&s_red[jj][1][wv][4 * lane]) = pq;
      }
    }
    lds_barrier();
    const float gamma = s_gamma[jj], bt = s_beta[jj];
    f32x4 ck = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w2 = 0; w2 < kWaves; ++w2) ck += *reinterpret_cast<const f32x4*>(&s_red[jj][0][w2][4 * cg]);
    const f32x4 vv = *reinterpret_cast<const f32x4*>(&s_v[jj][4 * cg]);
    const f32x4 d = (vv - gamma * ck) * bt;
    {
      f32x4* p = reinterpret_cast<f32x4*>(rec_state + ((int64_t)n * Hv + hk * R + jj) * kD * kD);
#pragma unroll
      for (int m = 0; m < kRows; ++m)
        if (kRG * kRows == kD || rg + kRG * m < kD)
          __builtin_nontemporal_store(S[jj][m] * gamma + d * kr[m], p + (rg + kRG * m) * 32 + cg);
    }
    if (read_wave && j == jj) {  // lanes l and l + 32 hold the same columns (t & 31 == l & 31)
      f32x4 cq = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w2 = 0; w2 < kWaves; ++w2) cq += *reinterpret_cast<const f32x4*>(&s_red[jj][1][w2][oc]);
      float o[4], ss = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = rbf(gamma * cq[e] + kq * d[e]);
        ss += o[e] * o[e];
      }
      ss = half_sum(ss);
      const float inv = rsq_fast(ss / (float)kD + eps);
      uint16_t ov[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float xn = rbf(o[e] * inv);
        const float wt = kWBf16 ? bf2f((uint16_t)(nwr[e >> 1] >> (16 * (e & 1)))) : __uint_as_float(nwr[e]);
        const float y = kWBf16 ? rbf(wt * xn) : wt * xn;
        ov[e] = f2bf(y * silu_fast(bf2f((uint16_t)(zr[e >> 1] >> (16 * (e & 1))))));
      }
      if (lane < 32) {
        const uint64_t pk = (uint64_t)ov[0] | ((uint64_t)ov[1] << 16) | ((uint64_t)ov[2] << 32) | ((uint64_t)ov[3] << 48);
        __builtin_nontemporal_store(pk, reinterpret_cast<uint64_t*>(out + ((int64_t)n * Hv + h) * kD + oc));
      }
    }
  }
  if (conv_wave && k4) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
      __builtin_nontemporal_store(((uint64_t)cnew[u].y << 32) | cnew[u].x,
                                  reinterpret_cast<uint64_t*>(conv_state + ((int64_t)n * C + ch0 + lane + 64 * u) * 4));
  }
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
  hipStream_t st = (hipStream_t)stream;
  const bool vec = D == 128 && x_stride % 8 == 0 && gate_stride % 8 == 0 && aligned(x, 16) && aligned(gate, 16) &&
                   aligned(out, 16);
  if (vec) {
    const unsigned blocks = (unsigned)((rows + 15) / 16);
    if (w_dtype == GDN_BF16)
      gated_rmsnorm128_kernel<true><<<blocks, 256, 0, st>>>((const uint16_t*)x, x_stride, (const uint16_t*)gate,
                                                            gate_stride, weight, (uint16_t*)out, rows, eps);
    else
      gated_rmsnorm128_kernel<false><<<blocks, 256, 0, st>>>((const uint16_t*)x, x_stride, (const uint16_t*)gate,
                                                             gate_stride, weight, (uint16_t*)out, rows, eps);
    return check_launch("gdn_gated_rmsnorm");
  }
  const unsigned blocks = (unsigned)((rows + 3) / 4);
  if (w_dtype == GDN_BF16)
    gated_rmsnorm_kernel<true><<<blocks, 256, 0, st>>>(
        (const uint16_t*)x, x_stride, (const uint16_t*)gate, gate_stride, weight, (uint16_t*)out, rows, D, eps);
  else
    gated_rmsnorm_kernel<false><<<blocks, 256, 0, st>>>(
        (const uint16_t*)x, x_stride, (const uint16_t*)gate, gate_stride, weight, (uint16_t*)out, rows, D, eps);
  return check_launch("gdn_gated_rmsnorm");
}

extern "C" int gdn_decode_fused_masked(const void* mixed, int64_t mixed_stride, const void* z, int64_t z_stride,
                                       const void* a, const void* b, int64_t ab_stride, void* conv_state,
                                       const void* conv_w, const void* conv_b, const float* A_log,
                                       const float* dt_bias, const void* norm_w, int norm_w_dtype, float eps,
                                       float* rec_state, void* out, const uint8_t* active, int N, int Hk, int Hv,
                                       int D, int K, void* stream) {
  clear_error();
  GDN_REQUIRE(mixed && z && a && b && conv_state && conv_w && A_log && dt_bias && norm_w && rec_state && out,
              "gdn_decode_fused: null pointer");
  GDN_REQUIRE(N >= 0 && Hk > 0 && Hv > 0 && Hv % Hk == 0, "gdn_decode_fused: bad heads Hk=%d Hv=%d", Hk, Hv);
  GDN_SUPPORT(D == kD, "gdn_decode_fused: head dim %d unsupported (needs %d)", D, kD);
  GDN_SUPPORT(K >= 1 && K <= 8, "gdn_decode_fused: conv kernel %d unsupported", K);
  GDN_REQUIRE(norm_w_dtype == GDN_F32 || norm_w_dtype == GDN_BF16, "gdn_decode_fused: bad norm_w_dtype");
  GDN_REQUIRE(aligned(rec_state, 16), "gdn_decode_fused: rec_state must be 16-byte aligned");
  GDN_REQUIRE(aligned(z, 8) && z_stride % 4 == 0 && aligned(out, 8),
              "gdn_decode_fused: z (and its row stride) and out must be 8-byte aligned");
  GDN_REQUIRE(aligned(norm_w, norm_w_dtype == GDN_BF16 ? 8 : 16), "gdn_decode_fused: norm_w misaligned");
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
      (const uint16_t*)conv_b, A_log, dt_bias, norm_w, eps, rec_state, (uint16_t*)out, active, Hk, K)
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

extern "C" int gdn_decode_fused(const void* mixed, int64_t mixed_stride, const void* z, int64_t z_stride,
                                const void* a, const void* b, int64_t ab_stride, void* conv_state,
                                const void* conv_w, const void* conv_b, const float* A_log,
                                const float* dt_bias, const void* norm_w, int norm_w_dtype, float eps,
                                float* rec_state, void* out, int N, int Hk, int Hv, int D, int K,
                                void* stream) {
  return gdn_decode_fused_masked(mixed, mixed_stride, z, z_stride, a, b, ab_stride, conv_state, conv_w, conv_b,
                                 A_log, dt_bias, norm_w, norm_w_dtype, eps, rec_state, out, nullptr, N, Hk, Hv, D, K,
                                 stream);
}
