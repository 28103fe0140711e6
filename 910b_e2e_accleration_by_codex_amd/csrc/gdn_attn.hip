// GQA decode attention of the hybrid stack's full-attention layers, for N slots of one new token
// each, over a per-slot KV cache: HF Qwen3_5Attention.forward (modeling_qwen3_5.py:629-700) with
// its q/k Qwen3_5RMSNorm, partial rotary (apply_rotary_pos_emb, :554-580), eager attention
// (:604-626) and the sigmoid output gate (:698), as the reference's engine runs it at decode.
//
// Three launches, all HBM- or latency-bound (the cache is read once):
//   1. attn_prep_kernel: one wave per (slot, head row).  RMSNorm (fp32, (1 + w), bf16) of the q and
//      k rows, rotary on the first rd dims (fp32, bf16), q kept in fp32 for the scores, k and v
//      written into the cache at the slot's position.
//   2. attn_split_kernel: one workgroup per (256-token split, kv head, slot) with the kv head's G
//      query heads.  Scores (fp32) from the transposed K cache [hd, T] with tokens along the lanes
//      (8-byte loads of 4 tokens per lane, each wave a quarter of the head dims), the split's max
//      and exp-sum per query head, then P V from the V cache [T, hd] (16-byte loads of 8 dims per
//      lane, row groups of tokens), reduced across the row groups in LDS.
//   3. attn_combine_kernel: per (slot, query head): the splits merged with their max (flash
//      decoding), o rounded to bf16 and multiplied by bf16(sigmoid(gate)).
// Rounding: scores and the softmax's max and exponentials are fp32 (the eager path rounds the scores
// to bf16 too).  The probabilities are rounded to bf16, as the eager path rounds its normalised
// ones, and P V multiplies those bf16 values against bf16 V (v_dot2_f32_bf16) with fp32
// accumulation; the split's exp-sum adds the same rounded values.  The test holds the result to an
// fp32 reference.
#include "gdn_device.h"
#include "gdn_internal.h"

namespace gdn {
namespace attn {
constexpr int SPLIT = 256;   // tokens per split workgroup
constexpr int THREADS = 256;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__host__ __device__ inline int64_t round256(int64_t b) { return (b + 255) / 256 * 256; }
// Two bf16 values a, b (dwords holding two bf16 each) paired as (a.lo, b.lo) / (a.hi, b.hi).
__device__ __forceinline__ uint32_t pair_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t pair_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }
// acc + x.lo * y.lo + x.hi * y.hi (bf16 pairs, fp32 sum: v_dot2_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t x, uint32_t y, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x), __builtin_bit_cast(bf16x2, y), acc, false);
}
// workspace: q (fp32 [N, nh, hd]) | m, l (fp32 [N, nh, S, 2]) | partial o (fp32 [N, nh, S, hd])
struct Work {
  float* q;
  float* ml;
  float* o;
};
__host__ __device__ inline int splits_of(int T) { return (T + SPLIT - 1) / SPLIT; }
__host__ __device__ inline int64_t work_bytes(int N, int nh, int hd, int T) {
  const int64_t S = splits_of(T);
  return round256((int64_t)N * nh * hd * 4) + round256((int64_t)N * nh * S * 2 * 4) +
         round256((int64_t)N * nh * S * hd * 4);
}
__host__ __device__ inline Work work_of(float* base, int N, int nh, int hd, int T) {
  const int64_t S = splits_of(T);
  char* p = reinterpret_cast<char*>(base);
  Work w;
  w.q = reinterpret_cast<float*>(p);
  p += round256((int64_t)N * nh * hd * 4);
  w.ml = reinterpret_cast<float*>(p);
  p += round256((int64_t)N * nh * S * 2 * 4);
  w.o = reinterpret_cast<float*>(p);
  return w;
}
// The fused projection's row n, column col: a bf16 matrix, or bf16(sum of fp32 split-K partials
// [splits][N][width] in split order) -- the same value the reduced projection holds.
struct Src {
  const uint16_t* bf;
  int64_t stride;
  const float* part;
  int splits, N;
  int64_t width;
  __device__ __forceinline__ float operator()(int n, int64_t col) const {
    if (!part) return bf2f(bf[n * stride + col]);
    float s = 0.f;
    for (int sp = 0; sp < splits; ++sp) s += part[((int64_t)sp * N + n) * width + col];
    return rbf(s);
  }
};
}  // namespace attn

// One wave per (slot n, row r): r < nh are query heads, nh <= r < nh + kv key heads.  Lane l holds
// dims l + 64 e.  The rotary partner of dim d < rd is d +- rd / 2, exchanged through LDS.
template <int HD>
__global__ __launch_bounds__(256) void attn_prep_kernel(attn::Src proj, const int64_t* __restrict__ pos,
                                                        const uint16_t* __restrict__ q_w,
                                                        const uint16_t* __restrict__ k_w,
                                                        const float* __restrict__ inv_freq, uint16_t* __restrict__ kt,
                                                        uint16_t* __restrict__ vc, float* __restrict__ qf, int N,
                                                        int nh, int kv, int rd, int T, float eps) {
  constexpr int E = HD / 64;
  __shared__ float row[4][HD];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + wid;
  if (w >= (int64_t)N * (nh + kv)) return;  // whole waves only: no barrier below
  const int n = (int)(w / (nh + kv)), r = (int)(w % (nh + kv));
  const bool is_q = r < nh;
  const int j = r - nh;
  const int64_t src = is_q ? (int64_t)r * 2 * HD : (int64_t)2 * nh * HD + (int64_t)j * HD;  // row n's column
  const uint16_t* wt = is_q ? q_w : k_w;
  float x[E];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    x[e] = proj(n, src + lane + 64 * e);
    ss += x[e] * x[e];
  }
  ss = wave_sum(ss);
  const float inv = rsqrt_f(ss / (float)HD + eps);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float y = rbf((x[e] * inv) * (1.0f + bf2f(wt[lane + 64 * e])));
    x[e] = y;
    row[wid][lane + 64 * e] = y;
  }
  // one wave's LDS accesses complete in program order: the partner reads below see the writes
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const int64_t p = pos[n];
  const float fp = (float)p;
  const int half = rd / 2;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int d = lane + 64 * e;
    if (d < rd) {
      const int i = d < half ? d : d - half;
      const float ang = fp * inv_freq[i];
      const float c = cosf(ang), s = sinf(ang);
      const float rot = d < half ? -row[wid][d + half] : row[wid][d - half];
      x[e] = rbf(x[e] * c + rot * s);
    }
  }
  if (is_q) {
    float* q = qf + ((int64_t)n * nh + r) * HD;
#pragma unroll
    for (int e = 0; e < E; ++e) q[lane + 64 * e] = x[e];
  } else if (p >= 0 && p < T) {
    const int64_t vs = (int64_t)2 * nh * HD + (int64_t)kv * HD + (int64_t)j * HD;
    uint16_t* kd = kt + ((int64_t)n * kv + j) * HD * T + p;
    uint16_t* vd = vc + (((int64_t)n * kv + j) * T + p) * HD;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      kd[(int64_t)(lane + 64 * e) * T] = f2bf(x[e]);
      vd[lane + 64 * e] = f2bf(proj(n, vs + lane + 64 * e));  // exact: the value is bf16
    }
  }
}

// grid (S, kv, N), 256 threads.  Split s covers tokens [256 s, 256 s + 256) of the slot's
// len = pos + 1 (the new token included).
template <int HD, int G>
__global__ __launch_bounds__(256) void attn_split_kernel(const int64_t* __restrict__ pos,
                                                         const uint16_t* __restrict__ kt,
                                                         const uint16_t* __restrict__ vc, attn::Work wk, int nh,
                                                         int kv, int T, float scale) {
  using namespace attn;
  constexpr int CG = HD / 8;          // 16-byte column groups of a V row
  constexpr int RG = THREADS / CG;    // token row groups in P V
  constexpr int QROWS = HD / 4;       // head dims per wave in the scores
  __shared__ uint32_t qp[HD / 2][G];                     // q of the G heads as bf16 pairs (dims 2i, 2i+1)
  __shared__ float big[(4 * G * SPLIT > RG * G * HD) ? 4 * G * SPLIT : RG * G * HD];
  __shared__ uint32_t pl[SPLIT / 2 * G];                 // bf16 probability pairs (positions 2i, 2i+1) per head
  __shared__ float red[2][4][G];
  const int split = blockIdx.x, j = blockIdx.y, n = blockIdx.z;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
  const int64_t p = pos[n];
  const int len = (int)(p + 1 < T ? p + 1 : T);
  const int t0 = split * SPLIT;
  if (t0 >= len) return;  // uniform over the workgroup
  const int S = splits_of(T);
  const int h0 = j * G;
  for (int i = tid; i < G * HD / 2; i += THREADS) {  // q is bf16-exact: the pairs lose nothing
    const int g = i / (HD / 2), dp = i % (HD / 2);
    const float* qg = wk.q + ((int64_t)n * nh + h0 + g) * HD + 2 * dp;
    qp[dp][g] = (uint32_t)f2bf(qg[0]) | ((uint32_t)f2bf(qg[1]) << 16);
  }
  __syncthreads();
  // ---- scores: wave wid sums dims [QROWS wid, QROWS wid + QROWS) for tokens t0 + 4 lane .. + 3
  {
    float acc[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[g][i] = 0.f;
    const int tl = t0 + 4 * lane;
    const int len4 = (len + 3) & ~3;  // <= T: T is a multiple of 4
    if (tl < len4) {
      const uint16_t* kp = kt + ((int64_t)n * kv + j) * HD * T + (int64_t)(QROWS * wid) * T + tl;
      // rows d, d + 1 at a time: per position the pair (k[d], k[d+1]) against q's pair, on v_dot2.
      // The cache is read once per step (K and V non-temporal: 2% faster per layer than cached reads)
#pragma unroll 8
      for (int d = 0; d < QROWS; d += 2) {
        const u32x2 ka = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(kp + (int64_t)d * T));
        const u32x2 kb = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(kp + (int64_t)(d + 1) * T));
        const uint32_t kk[4] = {pair_lo(ka[0], kb[0]), pair_hi(ka[0], kb[0]), pair_lo(ka[1], kb[1]),
                                pair_hi(ka[1], kb[1])};
        const int dp = (QROWS * wid + d) >> 1;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const uint32_t q2 = qp[dp][g];
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[g][i] = dot2_bf16(q2, kk[i], acc[g][i]);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 4; ++i) big[(wid * G + g) * SPLIT + 4 * lane + i] = acc[g][i];
  }
  __syncthreads();
  // ---- split softmax: thread tid = token t0 + tid
  const bool valid = t0 + tid < len;
  float s[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float v = ((big[(0 * G + g) * SPLIT + tid] + big[(1 * G + g) * SPLIT + tid]) +
                     (big[(2 * G + g) * SPLIT + tid] + big[(3 * G + g) * SPLIT + tid])) * scale;
    s[g] = valid ? v : -INFINITY;
    const float m = wave_max_fast(s[g]);
    if (lane == 0) red[0][wid][g] = m;
  }
  __syncthreads();
  float e[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float m = fmaxf(fmaxf(red[0][0][g], red[0][1][g]), fmaxf(red[0][2][g], red[0][3][g]));
    const uint16_t eb = f2bf(valid ? expf(s[g] - m) : 0.f);  // P V runs on bf16 probabilities
    e[g] = bf2f(eb);
    reinterpret_cast<uint16_t*>(pl)[((tid >> 1) * G + g) * 2 + (tid & 1)] = eb;
    const float l = wave_sum(e[g]);
    if (lane == 0) red[1][wid][g] = l;
  }
  __syncthreads();
  if (tid < G) {
    const int g = tid;
    const float m = fmaxf(fmaxf(red[0][0][g], red[0][1][g]), fmaxf(red[0][2][g], red[0][3][g]));
    const float l = (red[1][0][g] + red[1][1][g]) + (red[1][2][g] + red[1][3][g]);
    float* ml = wk.ml + (((int64_t)n * nh + h0 + g) * S + split) * 2;
    ml[0] = m;
    ml[1] = l;
  }
  // ---- P V: thread (rg, cg) sums position pairs (2 q, 2 q + 1), q = rg + RG i, over dims 8 cg .. 8 cg + 7
  {
    const int cg = tid % CG, rg = tid / CG;
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
    const uint16_t* vp = vc + (((int64_t)n * kv + j) * T + t0) * HD + 8 * cg;
    const int cnt = len - t0 < SPLIT ? len - t0 : SPLIT;
#pragma unroll 4
    for (int q = rg; 2 * q < cnt; q += RG) {
      // position 2q + 1 past the range reads the last valid row instead (its probability is 0)
      const int t1 = 2 * q + 1 < cnt ? 2 * q + 1 : 2 * q;
      const u32x4 va = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vp + (int64_t)(2 * q) * HD));
      const u32x4 vb = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vp + (int64_t)t1 * HD));
      uint32_t vv[8];
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        vv[2 * e2] = pair_lo(va[e2], vb[e2]);
        vv[2 * e2 + 1] = pair_hi(va[e2], vb[e2]);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint32_t p2 = pl[q * G + g];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = dot2_bf16(p2, vv[i], acc[g][i]);
      }
    }
    __syncthreads();  // every score read of `big` is done: reuse it for the row groups' sums
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) big[(rg * G + g) * HD + 8 * cg + i] = acc[g][i];
  }
  __syncthreads();
  for (int i = tid; i < G * HD; i += THREADS) {
    const int g = i / HD, d = i % HD;
    float o = 0.f;
#pragma unroll
    for (int r = 0; r < RG; ++r) o += big[(r * G + g) * HD + d];
    wk.o[(((int64_t)n * nh + h0 + g) * S + split) * HD + d] = o;
  }
}

// grid (N * nh), HD threads: thread d of (slot n, query head h).
template <int HD>
__global__ __launch_bounds__(256) void attn_combine_kernel(const int64_t* __restrict__ pos, attn::Src proj,
                                                           attn::Work wk, uint16_t* __restrict__ out,
                                                           int64_t out_stride, int nh, int T) {
  using namespace attn;
  const int n = blockIdx.x / nh, h = blockIdx.x % nh, d = threadIdx.x;
  const int64_t p = pos[n];
  const int len = (int)(p + 1 < T ? p + 1 : T);
  const int ns = (len + SPLIT - 1) / SPLIT, S = splits_of(T);
  const float* ml = wk.ml + ((int64_t)n * nh + h) * S * 2;
  const float* op = wk.o + ((int64_t)n * nh + h) * S * HD + d;
  // the loads of 4 splits at a time are issued together (a slot has up to S splits)
  float M = -INFINITY;
#pragma unroll 4
  for (int s = 0; s < ns; ++s) M = fmaxf(M, ml[2 * s]);
  float L = 0.f, o = 0.f;
#pragma unroll 4
  for (int s = 0; s < ns; ++s) {
    const float f = expf(ml[2 * s] - M);
    L += ml[2 * s + 1] * f;
    o += op[(int64_t)s * HD] * f;
  }
  const float a = ns > 0 ? rbf(o / L) : 0.f;  // a negative position attends to nothing: zero output
  const float gate = proj(n, (int64_t)h * 2 * HD + HD + d);
  out[n * out_stride + (int64_t)h * HD + d] = f2bf(a * bf2f(sigmoid_bf16(gate)));
}

template <int HD, int G>
static void launch_split(dim3 grid, hipStream_t st, const int64_t* pos, const uint16_t* kt, const uint16_t* vc,
                         attn::Work wk, int nh, int kv, int T, float scale) {
  attn_split_kernel<HD, G><<<grid, attn::THREADS, 0, st>>>(pos, kt, vc, wk, nh, kv, T, scale);
}
template <int HD>
static bool launch_split_g(int G, dim3 grid, hipStream_t st, const int64_t* pos, const uint16_t* kt,
                           const uint16_t* vc, attn::Work wk, int nh, int kv, int T, float scale) {
  switch (G) {
    case 1: launch_split<HD, 1>(grid, st, pos, kt, vc, wk, nh, kv, T, scale); return true;
    case 2: launch_split<HD, 2>(grid, st, pos, kt, vc, wk, nh, kv, T, scale); return true;
    case 4: launch_split<HD, 4>(grid, st, pos, kt, vc, wk, nh, kv, T, scale); return true;
    case 6: launch_split<HD, 6>(grid, st, pos, kt, vc, wk, nh, kv, T, scale); return true;
    case 8: launch_split<HD, 8>(grid, st, pos, kt, vc, wk, nh, kv, T, scale); return true;
    default: return false;
  }
}
template <int HD>
static int launch_all(attn::Src proj, const int64_t* pos, const uint16_t* q_w, const uint16_t* k_w,
                      const float* inv_freq, uint16_t* kt, uint16_t* vc, uint16_t* out, int64_t os, float* work, int N,
                      int nh, int kv, int rd, int T, float eps, hipStream_t st) {
  const attn::Work wk = attn::work_of(work, N, nh, HD, T);
  const int64_t waves = (int64_t)N * (nh + kv);
  attn_prep_kernel<HD><<<(unsigned)((waves + 3) / 4), 256, 0, st>>>(proj, pos, q_w, k_w, inv_freq, kt, vc, wk.q, N,
                                                                     nh, kv, rd, T, eps);
  const dim3 grid(attn::splits_of(T), kv, N);
  if (!launch_split_g<HD>(nh / kv, grid, st, pos, kt, vc, wk, nh, kv, T, 1.0f / sqrtf((float)HD)))
    return set_error(GDN_EUNSUP, "gdn_attn_decode: query heads per kv head must be 1, 2, 4, 6 or 8");
  attn_combine_kernel<HD><<<N * nh, HD, 0, st>>>(pos, proj, wk, out, os, nh, T);
  return check_launch("gdn_attn_decode");
}

}  // namespace gdn

using namespace gdn;

extern "C" int64_t gdn_attn_decode_workspace_bytes(int N, int nh, int hd, int T) {
  if (N < 0 || nh < 1 || hd < 1 || T < 1) return -1;
  return attn::work_bytes(N, nh, hd, T);
}

namespace {
int attn_entry(const char* name, attn::Src src, const int64_t* pos, const void* q_norm_w, const void* k_norm_w,
               const float* inv_freq, void* k_cache_t, void* v_cache, void* out, int64_t out_stride, float* work,
               int64_t work_bytes, int N, int nh, int kv, int hd, int rd, int T, float eps, void* stream) {
  GDN_REQUIRE(pos && q_norm_w && k_norm_w && k_cache_t && v_cache && out && work && (inv_freq || rd == 0),
              "%s: null pointer", name);
  GDN_REQUIRE(N >= 0 && nh >= 1 && kv >= 1 && nh % kv == 0, "%s: bad head counts", name);
  GDN_SUPPORT(hd == 64 || hd == 128 || hd == 256, "%s: head_dim must be 64, 128 or 256", name);
  GDN_REQUIRE(rd >= 0 && rd <= hd && rd % 2 == 0, "%s: rotary dims must be even and <= head_dim", name);
  GDN_REQUIRE(T >= 4 && T % 4 == 0, "%s: cache length must be a positive multiple of 4", name);
  GDN_REQUIRE(out_stride >= (int64_t)nh * hd, "%s: output row stride too small", name);
  GDN_REQUIRE(work_bytes >= attn::work_bytes(N, nh, hd, T), "%s: workspace too small (%lld bytes needed)", name,
              (long long)attn::work_bytes(N, nh, hd, T));
  GDN_REQUIRE(aligned(k_cache_t, 8) && aligned(v_cache, 16) && aligned(work, 256) && aligned(pos, 8),
              "%s: K cache 8-byte, V cache 16-byte, workspace 256-byte aligned", name);
  if (N == 0) return GDN_OK;
  src.N = N;
  const auto* qw = static_cast<const uint16_t*>(q_norm_w);
  const auto* kw = static_cast<const uint16_t*>(k_norm_w);
  auto* kt = static_cast<uint16_t*>(k_cache_t);
  auto* vc = static_cast<uint16_t*>(v_cache);
  auto* o = static_cast<uint16_t*>(out);
  const hipStream_t st = (hipStream_t)stream;
  switch (hd) {
    case 64: return launch_all<64>(src, pos, qw, kw, inv_freq, kt, vc, o, out_stride, work, N, nh, kv, rd, T, eps, st);
    case 128: return launch_all<128>(src, pos, qw, kw, inv_freq, kt, vc, o, out_stride, work, N, nh, kv, rd, T, eps, st);
    default: return launch_all<256>(src, pos, qw, kw, inv_freq, kt, vc, o, out_stride, work, N, nh, kv, rd, T, eps, st);
  }
}
}  // namespace

extern "C" int gdn_attn_decode(const void* proj, int64_t proj_stride, const int64_t* pos, const void* q_norm_w,
                               const void* k_norm_w, const float* inv_freq, void* k_cache_t, void* v_cache,
                               void* out, int64_t out_stride, float* work, int64_t work_bytes, int N, int nh, int kv,
                               int hd, int rd, int T, float eps, void* stream) {
  clear_error();
  GDN_REQUIRE(proj, "gdn_attn_decode: null pointer");
  GDN_REQUIRE(proj_stride >= (int64_t)(2 * nh + 2 * kv) * hd, "gdn_attn_decode: projection row stride too small");
  const attn::Src src{static_cast<const uint16_t*>(proj), proj_stride, nullptr, 0, N, 0};
  return attn_entry("gdn_attn_decode", src, pos, q_norm_w, k_norm_w, inv_freq, k_cache_t, v_cache, out, out_stride,
                    work, work_bytes, N, nh, kv, hd, rd, T, eps, stream);
}

extern "C" int gdn_attn_decode_partial(const float* part, int splits, const int64_t* pos, const void* q_norm_w,
                                       const void* k_norm_w, const float* inv_freq, void* k_cache_t, void* v_cache,
                                       void* out, int64_t out_stride, float* work, int64_t work_bytes, int N, int nh,
                                       int kv, int hd, int rd, int T, float eps, void* stream) {
  clear_error();
  GDN_REQUIRE(part && splits >= 1 && aligned(part, 4), "gdn_attn_decode_partial: bad partials");
  const attn::Src src{nullptr, 0, part, splits, N, (int64_t)(2 * nh + 2 * kv) * hd};
  return attn_entry("gdn_attn_decode_partial", src, pos, q_norm_w, k_norm_w, inv_freq, k_cache_t, v_cache, out,
                    out_stride, work, work_bytes, N, nh, kv, hd, rd, T, eps, stream);
}
