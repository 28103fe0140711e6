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
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
// SiLU with the hardware exp and reciprocal (each within about 1 ulp in fp32, so a bf16 result is
// within one bf16 ulp of the exactly rounded x / (1 + e^-x)); a third of silu_f's instructions.
__device__ __forceinline__ float silu_fast(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
// F.softplus(x), beta = 1, threshold = 20.
__device__ __forceinline__ float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
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
