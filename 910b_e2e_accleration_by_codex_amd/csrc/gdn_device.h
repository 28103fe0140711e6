// Device-side helpers shared by the GDN kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn {

constexpr int kWave = 64;

// ---- bf16 <-> fp32 -------------------------------------------------------------------------
// bf16 is the upper half of an IEEE fp32; fp32 -> bf16 rounds to nearest even (torch's rule)
// with gfx950's v_cvt_pk_bf16_f32 (branch-free; NaN stays NaN).
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Two values -> packed bf16 pair (low half = a), one conversion instruction.
__device__ __forceinline__ uint32_t f2bf2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t p = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, p);
}

// Round an fp32 value to the nearest bf16 and return it as fp32 (emulates one torch bf16 op).
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// Element loads/stores for the two activation dtypes (fp32 or bf16).
template <typename T> struct Elem;
template <> struct Elem<float> {
  __device__ static __forceinline__ float load(const float* p) { return *p; }
  __device__ static __forceinline__ void store(float* p, float v) { *p = v; }
  __device__ static __forceinline__ float round(float v) { return v; }
};
template <> struct Elem<uint16_t> {
  __device__ static __forceinline__ float load(const uint16_t* p) { return bf2f(*p); }
  __device__ static __forceinline__ void store(uint16_t* p, float v) { *p = f2bf(v); }
  __device__ static __forceinline__ float round(float v) { return rbf(v); }
};

// Slot row of sequence s for state I/O: rows[s] (or s without rows); -1 if outside [0, n_rows).
__device__ __forceinline__ int state_row(const int32_t* rows, int n_rows, int s) {
  const int r = rows ? rows[s] : s;
  return (r >= 0 && r < n_rows) ? r : -1;
}

// ---- scalar math with torch's CPU formulas ------------------------------------------------
// SiLU with the hardware exp and reciprocal, in fp32, for the gated norms' gate factor: within 24
// ulps of x / (1 + e^-x) (bf16 SiLU outputs go through silu_bf16 below).
__device__ __forceinline__ float silu_fast(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
// F.softplus(x), beta = 1, threshold = 20.
__device__ __forceinline__ float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
// ---- SiLU and sigmoid of a bf16 tensor, bit for bit torch's ---------------------------------
// torch evaluates F.silu and sigmoid on bf16 in fp32 (x / (1 + e^-x), 1 / (1 + e^-x)) and rounds
// once to bf16.  Over all 65,280 finite bf16 inputs its results are the exact functions rounded to
// fp32 and then to bf16, except where its fp32 e^-x overflows (x < -88.72: silu = x / inf = -0,
// sigmoid = 0); and no exact value lies within 9e-9 (relative) of an fp32 rounding midpoint, so an
// evaluation in double rounds to the same fp32 value.  A one-ulp slip of the fp32 value flips the
// bf16 result for a handful of inputs (x = -2^-8 and 2^-7 among them), and a flipped conv output or
// beta of a sequence's last token moves a fast-decaying head's final state by up to 7e-3.
__device__ __forceinline__ float silu_exact(float x) {
  if (x < -88.72283935546875f) return x / __builtin_huge_valf();
  const double xd = x;
  return (float)(xd / (1.0 + exp(-xd)));
}
__device__ __forceinline__ float sigmoid_exact(float x) {
  if (x < -88.72283935546875f) return 0.f;  // 1 / (1 + inf)
  return (float)(1.0 / (1.0 + exp(-(double)x)));
}
// e^x for -92 < x < 46: x log2(e) carried in two parts into the hardware exp2, whose own error then
// dominates (the single-product __expf loses |x| ulps in the rounding of x log2(e)).
__device__ __forceinline__ float exp_split(float x) {
  constexpr float kL = 1.44269502162933349609375f;  // log2(e) rounded to fp32
  constexpr float kLlo = 1.925963033500e-8f;        // log2(e) - kL
  const float t = x * kL;
  const float tl = fmaf(x, kLlo, fmaf(x, kL, -t));   // x log2(e) - t
  return __builtin_amdgcn_exp2f(t) * fmaf(tl, 0.693147180559945f, 1.0f);
}
// Two estimates decide the bf16 rounding for all but a few inputs.  silu_fast and sigmoid_fast are
// within 6 fp32 ulps of the correctly rounded values for every bf16 input with |x| <= 8; the
// exp_split estimates below, within 2 ulps for every bf16 input in [-32, 64] (both measured over all
// of them).  An estimate more than its error bound away from a bf16 rounding midpoint rounds to bf16
// as the exact value does; the fast one fails that (or |x| > 8) for about 1e-4 of N(0, 1) inputs,
// which then take the exp_split estimate, and the few inputs it leaves (4 bf16 values for each
// function, x = -2^-8 and 2^-7 among them; x outside [-32, 64]; NaN) take the double evaluation.
__device__ __forceinline__ float silu_est(float x) { return x * __builtin_amdgcn_rcpf(1.0f + exp_split(-x)); }
__device__ __forceinline__ float sigmoid_est(float x) { return __builtin_amdgcn_rcpf(1.0f + exp_split(-x)); }
__device__ __forceinline__ float sigmoid_fast(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ bool bf16_near_mid(float y, uint32_t ulps) {
  return (__float_as_uint(y) & 0xffffu) - (0x8000u - ulps) <= 2 * ulps;
}
__device__ __forceinline__ bool fast_undecided(float y, float x) { return !(fabsf(x) <= 8.f) || bf16_near_mid(y, 7); }
__device__ __forceinline__ bool est_undecided(float y, float x) {
  return !(x >= -32.f && x <= 64.f) || bf16_near_mid(y, 3);
}
// silu of N values -> bf16 bits.  The N fast estimates are independent (their exp / rcp latencies
// overlap); one branch, rarely taken, refines the undecided ones.
template <int N>
__device__ __forceinline__ void silu_bf16_n(const float (&x)[N], uint16_t (&o)[N]) {
  float y[N];
  bool redo = false;
#pragma unroll
  for (int e = 0; e < N; ++e) {
    y[e] = silu_fast(x[e]);
    redo |= fast_undecided(y[e], x[e]);
  }
  if (__builtin_expect(redo, 0)) {
#pragma unroll
    for (int e = 0; e < N; ++e)
      if (fast_undecided(y[e], x[e])) {
        y[e] = silu_est(x[e]);
        if (est_undecided(y[e], x[e])) y[e] = silu_exact(x[e]);
      }
  }
#pragma unroll
  for (int e = 0; e < N; ++e) o[e] = f2bf(y[e]);
}
__device__ __forceinline__ uint16_t silu_bf16(float x) {
  const float a[1] = {x};
  uint16_t o[1];
  silu_bf16_n<1>(a, o);
  return o[0];
}
__device__ __forceinline__ uint16_t sigmoid_bf16(float x) {
  float y = sigmoid_fast(x);
  if (__builtin_expect(fast_undecided(y, x), 0)) {
    y = sigmoid_est(x);
    if (est_undecided(y, x)) y = sigmoid_exact(x);
  }
  return f2bf(y);
}
// torch.rsqrt = 1 / sqrt(x) with correctly rounded sqrt and divide.
__device__ __forceinline__ float rsqrt_f(float x) { return 1.0f / sqrtf(x); }
// The hardware reciprocal square root (within about 1 ulp; x normal), for the gated norms' row
// factor: a tenth of rsqrt_f's instructions.
__device__ __forceinline__ float rsq_fast(float x) { return __builtin_amdgcn_rsqf(x); }

// ---- wavefront reductions ------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Register-only reductions with DPP row permutes and gfx950's permlane swaps (no LDS round trip
// per step).  Every step adds a lane's value to its partner's, so all lanes of a group end with
// the bit-identical sum -- and the same sum as the xor butterfly over the same lane groups
// (lane ^ 1, ^ 2, ^ 4, ^ 8 for row16_sum; the later steps pair lanes whose values are already
// equal within their group).  The whole wave must be active.
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, true));
}
// Sum over each aligned group of 16 lanes.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  v += dpp_mov<0x141>(v);  // row_half_mirror: the other quad of each 8
  v += dpp_mov<0x140>(v);  // row_mirror: the other 8 of each 16
  return v;
}
// Sum over lanes 0..31 and, separately, over lanes 32..63.
__device__ __forceinline__ float half_sum(float v) {
  v = row16_sum(v);
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);  // rows (0,1), (2,3) exchanged
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}
// v plus the value of lane ^ 16, in every lane.
__device__ __forceinline__ float xor16_sum(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);  // rows (0,1), (2,3) exchanged
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}
// Maximum over the whole wave.
__device__ __forceinline__ float wave_max_fast(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  v = fmaxf(v, dpp_mov<0x140>(v));
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
  u = __builtin_bit_cast(uint32_t, v);
  r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
// v plus the value of lane ^ 32, in every lane.
__device__ __forceinline__ float xor32_sum(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);  // halves exchanged
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}
// Sum over the whole wave.
__device__ __forceinline__ float wave_sum_fast(float v) { return xor32_sum(half_sum(v)); }

// Workgroup barrier over LDS only: it waits for this wave's LDS accesses (lgkmcnt 0), which is all
// the other waves depend on, and leaves global loads and stores in flight (__syncthreads would
// drain them: its release fence waits for every outstanding memory access, the next chunk's
// prefetched inputs included).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Treat v as produced at this point: no use of a loaded value can be hoisted above it, so a load
// issued earlier is not waited for before the loads issued between the two.
__device__ __forceinline__ void pin(uint32_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(float& v) { asm volatile("" : "+v"(v)); }

}  // namespace gdn
