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
// Two kernels: inv_kernel forms every chunk's 64x64 inverse (fp32, v_mfma_f32_16x16x4_f32) in
// parallel over all (chunk, value head) pairs, one wave each with everything in registers, and
// writes T diag(beta) as bf16 MFMA fragments; seg_kernel cuts each sequence into segments of
// consecutive chunks and walks
// one segment per workgroup with the fp32 state in MFMA accumulators, building every other operand
// of a chunk in LDS (local waves) while the chain waves run the previous chunk.  A segment's true
// initial state comes from a warm-up over the end of the segment before it, or from a summary
// pass plus an fp32 combination.  Products run on v_mfma_f32_16x16x32_bf16 with fp32
// accumulation; the state update feeds DEC vn as a bf16 hi + lo pair, so the running state never
// sees a bf16 rounding of its increment.
#include "gdn_device.h"
#include "gdn_internal.h"
#include "gdn_inverse.h"
#include <atomic>
#include <type_traits>

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
__device__ __forceinline__ f32x4 mma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
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
// (I - X)^{-1} for a batch of strictly lower 64x64 fp32 X, by reg_inv64: the routine the chunked
// prefill's inverse kernel runs (16x16 diagonal blocks by forward substitution, then the blocks
// below them on the fp32 MFMA, the blocking of src/gdn_chunk_fast.py:33-62).  One wave per matrix,
// four independent waves per workgroup.  Only the strictly lower part of X is read; T is written
// whole (upper blocks zero).
__global__ __launch_bounds__(256) void unit_lower_inv_kernel(const float* __restrict__ X, float* __restrict__ T,
                                                             int64_t batch) {
  __shared__ float tiles[4][4 * 16 * kTrPitch];  // per wave: reg_inv64's transpose tiles
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, c = lane & 15, g = lane >> 4;
  const int64_t m = (int64_t)blockIdx.x * 4 + w;
  if (m >= batch) return;
  const float* Xm = X + m * 4096;
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  f32x4 XT[10], Xd[4], TT[10];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
#pragma unroll
    for (int b = 0; b < a; ++b)  // Dl(X_ab^T): lane (c, g) r = X[16a + c][16b + 4g + r] (all strictly lower)
      XT[tri(a, b)] = *reinterpret_cast<const f32x4*>(&Xm[(16 * a + c) * 64 + 16 * b + 4 * g]);
    XT[tri(a, a)] = z;  // not read
#pragma unroll
    for (int r = 0; r < 4; ++r)  // Dl(X_aa): lane (c, g) r = X[16a + 4g + r][16a + c], strictly lower part
      Xd[a][r] = 4 * g + r > c ? Xm[(16 * a + 4 * g + r) * 64 + 16 * a + c] : 0.f;
  }
  reg_inv64(XT, Xd, TT, tiles[w], lane);
  float* Tm = T + m * 4096;
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)  // Dl(T_ab^T): lane (c, g) r = T[16a + c][16b + 4g + r]
      *reinterpret_cast<f32x4*>(&Tm[(16 * a + c) * 64 + 16 * b + 4 * g]) = b <= a ? TT[tri(a, b <= a ? b : 0)] : z;
}

// ============================================================================================
// Chunked prefill: operand fragments of one chunk.
// ============================================================================================
// The segment kernel builds, per (chunk, value head), the operands of the state chain in LDS as
// ready-made MFMA fragments: a fragment is 64 lanes x 16 bytes (lane l at byte 16 l), read with one
// conflict-free 16-byte LDS read per lane.
//
// k-slot order.  Inside every 32-wide reduction block the chain feeds MFMA B operands straight from
// accumulator registers: lane (c, g) = (l % 16, l / 16) holds rows 4g..4g+3 of two consecutive
// 16-row accumulator tiles, and uses them as the 8 k-values of its B fragment.  So B slot s of a
// block stands for block row kpos(s) = 16 ((s >> 2) & 1) + 4 (s >> 3) + (s & 3), and every A
// fragment below is permuted the same way along k:  A-frag element e of lane (c, g) for tile
// (m, j) = M[16 m + c][32 j + kpos(8 g + e)].
//
//   wn  16 frags [tb 4][j 4]  bf16  M = -W,  W = T diag(beta e^G) K     (tokens x features)
//   qg  16 frags [tb 4][j 4]  bf16  M = q (l2-normalised)               (tokens x features)
//   qk   6 frags tf::fid(tb, j)  bf16  M = scale q_i.k_j e^{G_i - G_j}, i >= j, else 0 (the
//                                   all-zero upper fragments are not formed)
//   tb   6 frags tf::fid(tb, k)  bf16  T diag(beta), the inverse kernel's (U = T diag(beta) V)
// K^T and V enter the products straight from the row-major K and V tiles (ds_read_b64_tr_b16).
namespace ws {
constexpr int FRAG = 1024;                       // bytes per fragment
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

// A-fragment of a bf16 [rows, ld] tile in k-slot order (two 8-byte reads).
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
// Fragment with k along the rows of a row-major [k][m] bf16 tile, in k-slot order: element e of lane
// (c, g) = (l % 16, l / 16) is M[k0 + kpos(8g + e)][m0 + c] -- the A operand of M^T or the B operand
// of M.
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
// x = hi + lo with hi = bf16(x), lo = bf16(x - hi): 8 accumulator values (two tiles) as two k-slot
// ordered bf16 fragments; hi + lo carries about 16 significant bits.
__device__ __forceinline__ bf16x8 lo_bf16(f32x4 a, f32x4 b, bf16x8 hi) {
  const u32x4v h = __builtin_bit_cast(u32x4v, hi);
  f32x4 ra, rb;
  ra[0] = a[0] - __uint_as_float(h[0] << 16);
  ra[1] = a[1] - __uint_as_float(h[0] & 0xffff0000u);
  ra[2] = a[2] - __uint_as_float(h[1] << 16);
  ra[3] = a[3] - __uint_as_float(h[1] & 0xffff0000u);
  rb[0] = b[0] - __uint_as_float(h[2] << 16);
  rb[1] = b[1] - __uint_as_float(h[2] & 0xffff0000u);
  rb[2] = b[2] - __uint_as_float(h[3] << 16);
  rb[3] = b[3] - __uint_as_float(h[3] & 0xffff0000u);
  return pack_acc_bf16(ra, rb);
}
__device__ __forceinline__ void split_bf16(f32x4 a, f32x4 b, bf16x8& hi, bf16x8& lo) {
  hi = pack_acc_bf16(a, b);
  lo = lo_bf16(a, b, hi);
}
__device__ __forceinline__ bf16x8 lds_frag(const uint8_t* base, int f, int lane) {
  return *reinterpret_cast<const bf16x8*>(base + f * ws::FRAG + lane * 16);
}


// Segment bookkeeping of the chunked prefill (shared by its kernels).
namespace sg {
constexpr int NT = 512;                      // 8 waves
// Shortest segment the host cuts (chunks).  2: a short prompt's heads spread over more workgroups
// (353 tokens at 48 value heads: segments of 2 chunks, 3 chunk steps a workgroup instead of 5);
// a later segment's warm-up must then fit in the 2 chunks before it.
constexpr int kMinSeg = 2;
constexpr int kTargetItems = 256;            // segments x value heads the host aims for
constexpr float kNegligibleLog = -44.3614f;  // ln(2^-64): a segment map A_j this small is not formed
// A warm-up drops a map bounded by 2^-16 relative to the state before it: 2^7 below the bf16
// rounding (2^-9) of the W S and Q S operands the state passes through every chunk, so the dropped
// part is lost in the rounding the chain makes anyway (unless the state shrank by more than 2^7 over
// the warm-up: new tokens contributing under 1/128 of the state they replace).
constexpr float kWarmLog = -11.0904f;        // ln(2^-16)
// A chunk whose decay over its tokens is slight (e^{G_last} above e^-4) passes much of the state it
// receives on: the bf16 rounding of the W S operands then accumulates over the chunks (to 1e-3 of
// the state over 8192 tokens of decay ~0.002 a token), or, from a large initial state that decays
// to a small one, weighs against the small one (1.3e-3 for one chunk at e^{G_last} = 0.13 from a
// state 8x the final one).  Such a chunk forms -W and the state as bf16 hi + lo pairs and takes
// W S = Wh Sh + Wh Sl + Wl Sh (about 16 significant bits); a chunk with faster decay forgets that
// rounding within a chunk or two and keeps the single bf16 product.
constexpr float kPreciseGl = 0.0183156389f;  // e^-4
// T diag(beta) (the inverse kernel's record) enters U and W as bf16 hi + lo in every chunk whose part
// of the final state is not negligible: a precise chunk, and one after which the decay up to the
// sequence's end sums to more than -4.5 (a sequence's last chunk, and the one before a short last
// chunk).  With a head's keys sharing a large common part (a conv bias, say), or beta in fp32 (a
// non-bf16 diagonal), the record's bf16 rounding alone moved states by 1e-3 to 2e-3 relative: in a
// long-memory head it builds up over the chunks, in a fast-decaying head the last chunks' U make most
// of the final state.  The inverse kernel decides, writes the lo part and sets a flag in the chunk's
// second record; the output pass follows the flag.
constexpr float kLoRecordLog = -4.5f;
constexpr int kTrans = 2 * pf::D * pf::D;    // floats per (slot, head): A, then B
}  // namespace sg

// The segments of a batch: packed sequences (seg0[s] = segments of the sequences before s, built by
// seg_table_kernel) or nseq uniform sequences of seq_len tokens.  Segment j of sequence s covers
// chunks L (j - first_seg(s)) .. + L - 1 (fewer in its last segment); an empty sequence has one
// segment without chunks.  Every segment but the last of its sequence owns a transition slot
// (A, B), numbered first_slot(s) = first_seg(s) - s onwards.
struct SegTable {
  const int32_t* cu;
  const int32_t* chunk0;
  const int32_t* seg0;
  const int32_t* order;  // output pass: segments longest first (nullptr: in index order)
  int nseq, seq_len, L;
  __device__ __forceinline__ int nch(int s) const {
    return cu ? chunk0[s + 1] - chunk0[s] : (seq_len + pf::CH - 1) / pf::CH;
  }
  __device__ __forceinline__ int nseg_of(int n) const { return n <= L ? 1 : (n + L - 1) / L; }
  __device__ __forceinline__ int first_seg(int s) const { return cu ? seg0[s] : s * nseg_of(nch(0)); }
  __device__ __forceinline__ int first_slot(int s) const { return first_seg(s) - s; }
  // Dense index of sequence s's first chunk (the inverse kernel's fragment slot).
  __device__ __forceinline__ int first_chunk(int s) const { return cu ? chunk0[s] : s * nch(0); }
  __device__ __forceinline__ int64_t start(int s) const { return cu ? (int64_t)cu[s] : (int64_t)s * seq_len; }
  __device__ __forceinline__ int len(int s) const { return cu ? cu[s + 1] - cu[s] : seq_len; }
  // The sequence of segment j (the last s with first_seg(s) <= j).
  __device__ int seq_of_seg(int j) const {
    if (!cu) return j / nseg_of(nch(0));
    int lo = 0, hi = nseq - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (seg0[mid] <= j) lo = mid;
      else hi = mid - 1;
    }
    return lo;
  }
  // The sequence of transition slot t (the last s with first_slot(s) <= t).
  __device__ int seq_of_slot(int t) const {
    if (!cu) return t / (nseg_of(nch(0)) - 1);
    int lo = 0, hi = nseq - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (seg0[mid] - mid <= t) lo = mid;
      else hi = mid - 1;
    }
    return lo;
  }
};

// Inclusive scan of part[0..255] in place (all 256 threads; barriers inside).
__device__ __forceinline__ void block_scan256(int* part, int t) {
  for (int o = 1; o < 256; o <<= 1) {
    const int x = t >= o ? part[t - o] : 0;
    __syncthreads();
    part[t] += x;
    __syncthreads();
  }
}
// The output pass deals (segment, value head) items to compute units in launch order, so segments
// are listed longest first (a greedy longest-processing-time schedule): a counting sort by chunk
// count, for segment lengths up to kLptMaxLen (else the order is the identity).
constexpr int kLptMaxLen = 2048;
// seg0 (nseq + 1 entries) from the chunk prefix sums, and order[] (segments by decreasing chunk
// count; ties in any order): one workgroup.
__device__ void seg_table_wg(const int32_t* __restrict__ chunk0, int nseq, int L, int32_t* __restrict__ seg0,
                             int32_t* __restrict__ order) {
  __shared__ int part[256];
  __shared__ int hist[kLptMaxLen + 1];
  const int t = threadIdx.x;
  int base = 0;
  for (int s0 = 0; s0 < nseq; s0 += 256) {
    const int s = s0 + t;
    int n = 0;
    if (s < nseq) {
      const int c = chunk0[s + 1] - chunk0[s];
      n = c <= L ? 1 : (c + L - 1) / L;
    }
    part[t] = n;
    __syncthreads();
    block_scan256(part, t);
    if (s < nseq) seg0[s] = base + part[t] - n;
    base += part[255];
    __syncthreads();
  }
  if (t == 0) seg0[nseq] = base;
  if (L > kLptMaxLen) {
    for (int j = t; j < base; j += 256) order[j] = j;
    return;
  }
  for (int i = t; i <= L; i += 256) hist[i] = 0;
  __syncthreads();
  // segment idx of sequence s covers min(L, n - idx L) chunks (an empty sequence: one of 0)
  for (int s = t; s < nseq; s += 256) {
    const int n = chunk0[s + 1] - chunk0[s], ns = n <= L ? 1 : (n + L - 1) / L;
    for (int idx = 0; idx < ns; ++idx) atomicAdd(&hist[n - idx * L < L ? n - idx * L : L], 1);
  }
  __syncthreads();
  // hist[len] := number of segments longer than len (exclusive scan from len = L down to 0): thread t
  // takes positions p = len' order L - p in [t * per, (t + 1) * per)
  const int per = (L + 1 + 255) / 256, p0 = t * per, p1 = p0 + per < L + 1 ? p0 + per : L + 1;
  int sum = 0;
  for (int p = p0; p < p1; ++p) sum += hist[L - p];
  part[t] = sum;
  __syncthreads();
  block_scan256(part, t);
  int acc = part[t] - sum;
  for (int p = p0; p < p1; ++p) {
    const int c = hist[L - p];
    hist[L - p] = acc;
    acc += c;
  }
  __syncthreads();
  for (int s = t; s < nseq; s += 256) {
    const int n = chunk0[s + 1] - chunk0[s], ns = n <= L ? 1 : (n + L - 1) / L, j0 = seg0[s];
    for (int idx = 0; idx < ns; ++idx) order[atomicAdd(&hist[n - idx * L < L ? n - idx * L : L], 1)] = j0 + idx;
  }
}
__global__ __launch_bounds__(256) void seg_table_kernel(const int32_t* __restrict__ chunk0, int nseq, int L,
                                                       int32_t* __restrict__ seg0, int32_t* __restrict__ order) {
  seg_table_wg(chunk0, nseq, L, seg0, order);
}

// ============================================================================================
// Chunked prefill, part 1: the intra-chunk inverse, parallel over every (chunk, value head).
// ============================================================================================
// X = -(beta_i k_i.k_j e^{G_i - G_j})_{i>j} and T = (I - X)^{-1} in fp32, written as the bf16 MFMA
// fragments of T diag(beta), lower-triangular fragments only (token tile w, k-block s <= w / 2), in
// k-slot order.  The segment kernel multiplies V with them (U = T diag(beta) V) and, with their
// columns scaled by e^G, K (W = T diag(beta e^G) K).  One wave owns one (chunk, value head) and
// keeps everything in registers: no LDS round trips of intermediate products and no barriers.
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
// The inverse kernel's second record per (chunk, value head): the K rows' l2norm factors, the chunk's
// g values (both fp32, by token) and a flag word (nonzero: the T record's lo part was written).
namespace kr {
constexpr int FLAG = 2 * pf::CH;      // float index of the flag word
constexpr int FLOATS = 2 * pf::CH + 4;  // 528 bytes: 16-byte aligned records
}  // namespace kr
namespace tf {
constexpr int FRAGS = 6;                      // lower fragments of T diag(beta)
__device__ __forceinline__ int fid(int w, int s) { return w < 2 ? w : 2 * w - 2 + s; }
// In memory the bf16 hi part is 5 KiB: fragments 0 = (0, 0) and 3 = (2, 1) straddle the diagonal,
// their second 16-column block is zero, and they keep only the first 8 bytes of each lane (512 B);
// the other four keep 16 bytes a lane.  Byte offsets 0, 512, 1536, 2560, 3072, 4096.  The lo part
// (T diag(beta) - hi, rounded to bf16) follows in the same layout, written only where the flag in the
// chunk's second record (kr::FLAG) is set.
constexpr int HALF = 5 * ws::FRAG;
constexpr int BYTES = 2 * HALF;
__host__ __device__ __forceinline__ constexpr bool half(int f) { return f == 0 || f == 3; }
__host__ __device__ __forceinline__ constexpr int offset(int f) {
  return f * ws::FRAG - (f >= 1 ? ws::FRAG / 2 : 0) - (f >= 4 ? ws::FRAG / 2 : 0);
}
}  // namespace tf

// Warm-up length for the transition after the segment ending with the chunk at token t_last (one
// wave): the least w such that the summed log decay of the segment's last w chunks is below
// ln 2^-16 -- the norm bound of the dropped map with unit keys and beta in [0, 1] -- or 0 when there
// is none within the segment's L chunks or a beta outside [0, 1] (or a NaN) comes first.  Chunks
// are taken back from the segment's end, four at a time (lane = token).
template <typename BetaT>
__device__ int chunk_warm(const float* __restrict__ g, const BetaT* __restrict__ beta, int Hv, int h, int64_t t_last,
                          int L) {
  const int lane = threadIdx.x & 63;
  float acc = 0.f;
  for (int c0 = 0; c0 < L; c0 += 4) {
    float x[4];
    int ok[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t tok = t_last - (int64_t)(c0 + u) * pf::CH + lane;
      const bool in = c0 + u < L;
      const float gv = in ? g[tok * Hv + h] : 0.f;
      const float bv = in ? Elem<BetaT>::load(beta + tok * Hv + h) : 0.f;
      x[u] = gv;
      ok[u] = (bv >= 0.f && bv <= 1.f && gv == gv) ? 1 : 0;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (c0 + u >= L) return 0;
      if (__builtin_amdgcn_ballot_w64(ok[u] == 0) != 0) return 0;
      acc += wave_sum_fast(x[u]);
      if (acc < sg::kWarmLog) return c0 + u + 1;
    }
  }
  return 0;
}

// Whether the summed g of tokens t_from .. t_end - 1 (one head) stays above thr: the decay a chunk's
// contribution to the state still meets before its sequence ends (one wave, 64 tokens a step, stopping
// as soon as the sum falls below thr).  The caller loads the first step's g (this lane's token
// t_from + lane, 0 past t_end) with its other loads: in a fast-decaying head that step decides.
__device__ bool tail_decay_above(const float* __restrict__ g, int Hv, int h, int64_t t_from, int64_t t_end, float thr,
                                 float g_first) {
  const int lane = threadIdx.x & 63;
  if (t_from >= t_end) return true;
  float acc = wave_sum_fast(g_first);
  if (!(acc > thr)) return false;
  for (int64_t t0 = t_from + 64; t0 < t_end; t0 += 64) {
    const int64_t tok = t0 + lane;
    acc += wave_sum_fast(tok < t_end ? g[tok * Hv + h] : 0.f);
    if (!(acc > thr)) return false;
  }
  return true;
}

// Workgroup order -> item order.  The 8 XCDs take workgroups b % 8 in turn; this bijection on [0, n),
// b -> (b % 8) * (n / 8) + b / 8 below 8 (n / 8) and the identity above, gives each XCD a contiguous
// range of items.
__device__ __forceinline__ int64_t xcd_range_item(int64_t b, int64_t n) {
  const int64_t per = n / 8;
  return b >= 8 * per ? b : (b % 8) * per + b / 8;
}

// One wave per (chunk, value head) item (item = chunk slot * Hv + value head; a workgroup's 4 waves
// are independent, so a wave past the end simply exits).  Lane (i, g) holds K[16 t + i][32 s + 8 g
// .. + 7] for token tiles t and k-blocks s < 4: the A fragment of tile t and, as K^T, the B
// fragment of tile t, so K K^T needs nothing but these registers.  (Waves that each take several
// items and prefetch the next one's inputs need more registers, halve the resident waves and were
// measured slower.)
template <typename BetaT>
__global__ __launch_bounds__(pf::NT, 2) void inv_kernel(const uint16_t* __restrict__ k, int64_t ks,
                                                       const float* __restrict__ g, const BetaT* __restrict__ beta,
                                                       const int32_t* __restrict__ cu,
                                                       const int32_t* __restrict__ seq_chunk0, int nseq, int seq_len,
                                                       int64_t items, int Hqk, int Hv, int use_l2,
                                                       uint8_t* __restrict__ tfrag, float* __restrict__ knorm,
                                                       SegTable tab, int* __restrict__ warm) {
  using namespace pf;
  __shared__ float sdec[4][2][CH];                // per wave: G and beta by token
  __shared__ float strp[4][4 * 16 * kTrPitch];    // per wave: 4 transpose tiles
  const int t = threadIdx.x, lane = t & 63, c16 = lane & 15, g4 = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);  // the item is wave-uniform: scalar control flow
  // the 8 workgroups of one chunk's 32 value heads share an XCD, so the chunk's g and beta lines
  // (one token's heads per line) come from HBM once per chunk, not once per XCD
  const int64_t item = xcd_range_item(blockIdx.x, gridDim.x) * 4 + w;
  if (item >= items) return;
  const int slot = (int)(item / Hv), h = (int)(item % Hv);
  const int r = Hv / Hqk, hk = h / r;
  const ChunkPos cp = chunk_pos(slot, cu, seq_chunk0, nseq, seq_len);
  u16x8 kf[4][4];
  {
    const uint16_t* kb = k + cp.t0 * ks + (int64_t)hk * D + 8 * g4;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int row = 16 * tt + c16, rc = row < cp.len ? row : cp.len - 1;
#pragma unroll
      for (int s = 0; s < 4; ++s) kf[tt][s] = *reinterpret_cast<const u16x8*>(kb + rc * ks + 32 * s);
    }
  }
  const int tok = lane < cp.len ? lane : cp.len - 1;
  const float graw = g[(cp.t0 + tok) * Hv + h];
  const float braw = Elem<BetaT>::load(beta + (cp.t0 + tok) * Hv + h);
  // the first 64 tokens after the chunk (same sequence): the tail decay's first step
  const int64_t t_tail = cp.t0 + cp.len, t_end = tab.start(cp.seq) + tab.len(cp.seq);
  const float gtail = t_tail + lane < t_end ? g[(t_tail + lane) * Hv + h] : 0.f;
  // rows past the chunk's end are zero; with use_l2, each row's l2norm factor bf16(rsqrt(...)) with
  // torch's bf16 op rounding (a row sits in the lanes c, c + 16, c + 32, c + 48), and the rows
  // scaled by it and rounded to bf16: the reference's normalised rows, bit for bit, as the segment
  // kernel forms them from the same factors.  The Gram matrix is theirs: formed from the unrounded
  // products instead (the raw rows' Gram scaled by the factors) it differs by ~2e-4 absolute, a
  // mismatch between T and the K the state update uses that accumulates in long-memory heads (state
  // 5.0e-4 -> 8.5e-4 rel-L2 at g ~ -0.002 over 4096 tokens, in emulation).
  float invc[4] = {1.f, 1.f, 1.f, 1.f};  // factor of row 16 t + c
  {
    const u16x8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
    float mine = 1.f;  // lane (c, g) publishes the factor of row 16 g + c
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const bool live = 16 * tt + c16 < cp.len;
#pragma unroll
      for (int s = 0; s < 4; ++s) kf[tt][s] = live ? kf[tt][s] : zero;
      if (use_l2) {
        float ss = 0.f;
#pragma unroll
        for (int s = 0; s < 4; ++s) ss = sumsq_bf16(kf[tt][s], ss);
        invc[tt] = l2norm_inv(xor32_sum(xor16_sum(ss)));
        mine = g4 == tt ? invc[tt] : mine;
#pragma unroll
        for (int s = 0; s < 4; ++s) kf[tt][s] = scale_bf16(kf[tt][s], invc[tt]);
      }
    }
    float* rec = knorm + ((int64_t)slot * Hv + h) * kr::FLOATS;
    if (use_l2) rec[lane] = mine;
    rec[CH + lane] = graw;  // the chunk's g of this head, contiguous for the segment kernel
  }
  // K K^T: kk[tri(a, b)] = Dl of block (b, a) -- lane (c, g) r: (K K^T)[16 b + 4 g + r][16 a + c]
  f32x4 kk[10];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b <= a; ++b) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) acc = mma(__builtin_bit_cast(bf16x8, kf[b][s]), __builtin_bit_cast(bf16x8, kf[a][s]), acc);
      kk[tri(a, b)] = acc;
    }
  {  // decay within the chunk (g = 0 and beta = 0 past its end)
    const float G = wave_incl_scan(lane < cp.len ? graw : 0.f);
    sdec[w][0][lane] = G;
    sdec[w][1][lane] = lane < cp.len ? braw : 0.f;
  }
  __builtin_amdgcn_wave_barrier();  // this wave's own LDS writes, read back in order
  float Gc[4], Bc[4];   // at token 16 a + c
  f32x4 Gr[4], Br[4];   // at tokens 16 b + 4 g + r
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    Gc[a] = sdec[w][0][16 * a + c16];
    Bc[a] = sdec[w][1][16 * a + c16];
    Gr[a] = *reinterpret_cast<const f32x4*>(&sdec[w][0][16 * a + 4 * g4]);
    Br[a] = *reinterpret_cast<const f32x4*>(&sdec[w][1][16 * a + 4 * g4]);
  }
  // X^T blocks from the symmetric K K^T: Dl(X_ab^T) at lane (c, g) r is X[i = 16a + c][j = 16b + 4g + r]
  // = -beta_i (K K^T)[j][i] e^{G_i - G_j}; the diagonal blocks also as Dl(X_aa)
  f32x4 XT[10], Xd[4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b <= a; ++b)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {  // straight-line: the exponent is 0 off the strict lower part, the
                                         // mask multiplies (any sign of g: e^{G_i - G_j} as the reference)
        const int i = 16 * a + c16, j = 16 * b + 4 * g4 + rr;
        const float x = -Bc[a] * kk[tri(a, b)][rr] * __expf(i > j ? Gc[a] - Gr[b][rr] : 0.f);
        XT[tri(a, b)][rr] = x * (i > j ? 1.f : 0.f);
      }
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int i = 16 * a + 4 * g4 + rr, j = 16 * a + c16;
      const float x = -Br[a][rr] * kk[tri(a, a)][rr] * __expf(i > j ? Gr[a][rr] - Gc[a] : 0.f);
      Xd[a][rr] = x * (i > j ? 1.f : 0.f);
    }
  f32x4 TT[10];
  reg_inv64(XT, Xd, TT, strp[w], lane);
  // (the output pass's own test for a precise chunk is part of it, on the same G_last, so a precise
  // chunk always has its lo part)
  const float Gl = sdec[w][0][CH - 1];  // G_last (wave-uniform)
  bool lo_rec = __expf(Gl) > sg::kPreciseGl || Gl > sg::kLoRecordLog;
  if (!lo_rec)
    lo_rec = tail_decay_above(g, Hv, h, t_tail, t_end, sg::kLoRecordLog, gtail);
  if (lane == 0)
    reinterpret_cast<int*>(knorm)[((int64_t)slot * Hv + h) * kr::FLOATS + kr::FLAG] = lo_rec ? 1 : 0;
  // fragments (w', s), s <= w' / 2: element e of lane (i, g) = T[16 w' + i][j] beta_j with
  // j = 32 s + kpos(8 g + e), kpos(8 g + e) = 16 (e >> 2) + 4 g + (e & 3): blocks 2s (e < 4) and 2s + 1
  uint8_t* dst = tfrag + ((int64_t)slot * Hv + h) * tf::BYTES;
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int wt = 0; wt < 4; ++wt)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (2 * s > wt) continue;
      const f32x4 t0 = TT[tri(wt, 2 * s)], t1 = 2 * s + 1 <= wt ? TT[tri(wt, 2 * s + 1 <= wt ? 2 * s + 1 : 0)] : z;
      const int f = tf::fid(wt, s);
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      const f32x4 a0 = t0 * Br[2 * s], a1 = t1 * Br[2 * s + 1];
      const bf16x8 hb = pack_acc_bf16(a0, a1);
      const u32x4 pk = __builtin_bit_cast(u32x4, hb);
      if (tf::half(f))  // the second block (e >= 4) is zero: 8 bytes a lane
        *reinterpret_cast<u32x2v*>(dst + tf::offset(f) + lane * 8) = u32x2v{pk[0], pk[1]};
      else
        *reinterpret_cast<u32x4*>(dst + tf::offset(f) + lane * 16) = pk;
      if (lo_rec) {
        const u32x4 pl = __builtin_bit_cast(u32x4, lo_bf16(a0, a1, hb));
        if (tf::half(f))
          *reinterpret_cast<u32x2v*>(dst + tf::HALF + tf::offset(f) + lane * 8) = u32x2v{pl[0], pl[1]};
        else
          *reinterpret_cast<u32x4*>(dst + tf::HALF + tf::offset(f) + lane * 16) = pl;
      }
    }
  // the last chunk of a segment with a successor: that transition slot's warm-up length
  const int nch = tab.nch(cp.seq);
  if ((cp.c + 1) % tab.L == 0 && cp.c + 1 < nch) {
    const int ts = tab.first_slot(cp.seq) + (cp.c + 1) / tab.L - 1;
    const int wv = use_l2 ? chunk_warm(g, beta, Hv, h, cp.t0, tab.L) : 0;
    if (lane == 0) warm[(int64_t)ts * Hv + h] = wv;
  }
}

// ============================================================================================
// Chunked prefill, segment-parallel and fused (the path gdn_chunk_prefill runs).
// ============================================================================================
// A sequence's chunks are cut into segments of L consecutive chunks (the host picks L so that
// about one (segment, value head) pair per compute unit exists).  One workgroup per (segment, value
// head) walks its segment's chunks.  Per chunk, its 4 local waves build the operand fragments
// described above in LDS (K and q masked and l2-normalised, the decay, Q K^T, -W from the K rows and
// the inverse kernel's T diag(beta) scaled by e^G) and store the previous chunk's outputs, and its 4
// chain waves advance 32 columns of the fp32 state each and leave their outputs in LDS.  Only the
// inverse kernel's records (5 KiB of T fragments, 5 KiB more for their lo parts where a chunk's flag
// is set, and 528 B of K row factors, g and the flag per (chunk, value head)) pass through memory
// besides the inputs and outputs.
// A segment other than the first of its sequence needs its true initial state: the state after
// segment j is S_{j+1} = A_j S_j + B_j, with A_j the segment's linear map (the chain run from the
// identity with U = 0) and B_j its affine part (run from zero).  A summary pass computes A_j and
// B_j for every segment with a successor, and the output pass's workgroup of segment j first applies
// S_{k+1} = A_k S_k + B_k for k < j (bf16 hi + lo products on MFMA, A_k's fragments staged in LDS
// by the local waves) and then runs the segment from that state.
// With unit keys (in-kernel l2norm) and 0 <= beta <= 1 each token's map gamma (I - beta k k^T) has
// spectral norm <= gamma, so ||A_j|| <= exp(sum of g over segment j).  When that bound is below
// 2^-64, A_j S_j lies far below the fp32 rounding of S_{j+1} and A_j is not formed (flag 0).

// Warm-up lengths.  The state entering segment j + 1 differs from the chain run from zero over the
// last w chunks of segment j by the map of those w chunks applied to the state before them; with
// unit keys and beta in [0, 1] that map's norm is at most exp(sum of g over the w chunks).  The
// inverse kernel writes each transition slot's least w whose bound is below 2^-16 (0: none).  A
// (sequence, value head) pair whose every slot has one runs no summaries and no combination, and
// its later segments start from their warm-ups.  One wave reads the pair's slots, 64 at a time.
__device__ bool seq_warm_ok(const SegTable& tab, const int* __restrict__ warm, int Hv, int h, int s) {
  const int lane = threadIdx.x & 63;
  const int ts0 = tab.first_slot(s), nslot = tab.first_slot(s + 1) - ts0;
  for (int j0 = 0; j0 < nslot; j0 += 64) {
    const int wv = j0 + lane < nslot ? warm[(int64_t)(ts0 + j0 + lane) * Hv + h] : 1;
    if (__builtin_amdgcn_ballot_w64(wv == 0) != 0) return false;
  }
  return true;
}

// Work item of workgroup b of n: workgroups are dealt to the 8 XCDs round-robin (b % 8), so items
// 2p and 2p + 1 (the two value heads that read one key head's q and K, the two summaries of a slot)
// go to workgroups b and b + 8, which share an XCD and its L2; otherwise the order is kept.  A
// bijection on [0, n) (the last n % 16 workgroups keep their own number).
__device__ __forceinline__ int xcd_item(int b, int n) {
  if (b >= (n & ~15)) return b;
  return 2 * (8 * (b >> 4) + (b & 7)) + ((b >> 3) & 1);
}

// Per-chunk operands, double-buffered: the local waves fill one buffer while the chain waves read
// the other.  Fragment layouts as described at the top of this section (k-slot order).
struct alignas(16) SegBuf {
  uint16_t K[pf::CH * pf::LDK];   // K rows (l2-normalised), token-major
  uint16_t V[pf::CH * pf::LDK];   // V rows
  uint8_t qg[16 * ws::FRAG];          // q fragments [tb 4][j 4]
  uint8_t tb[tf::FRAGS * ws::FRAG];   // T diag(beta) fragments (the inverse kernel's), index tf::fid(tb, k)
  float gs[pf::CH];               // G_t, the cumulative log decay within the chunk
  float dec[pf::CH];              // e^{G_last - G_t}
  float eg[pf::CH];               // e^{G_t}
  float egs[pf::CH];              // scale e^{G_t}
  float gl;                       // e^{G_last}
  int lof;                        // T diag(beta)'s lo part is in the chunk's record (and the chain takes it)
};
// The operands the local waves form after the step's first barrier and the chain reads before the
// next step's first barrier (-W and QK) are single: the local waves write chunk c + 1's while the
// chain waves are in part 2 of chunk c, which reads neither.
struct alignas(16) SegOps {
  uint8_t wn[16 * ws::FRAG];          // -W fragments [tb 4][j 4] (the bf16 hi part in a precise chunk)
  uint8_t wl[16 * ws::FRAG];          // the lo part of -W in a precise chunk
  uint8_t qk[tf::FRAGS * ws::FRAG];   // QK fragments of the lower blocks, index tf::fid(tb, j)
  uint8_t tl[tf::FRAGS * ws::FRAG];   // the lo part of T diag(beta) in a precise chunk, index tf::fid(tb, k)
};
struct SegSmem {
  SegBuf buf[2];
  SegOps ops;
  float red[8];
};

enum SegMode { kSegOut = 0, kSegB = 1, kSegA = 2 };

// A transition slot (sg::kTrans floats per (slot, value head)) as the summary pass writes it and the
// output pass reads it: A_j as bf16 A fragments, 32 hi parts then 32 lo parts (fragment rt * 4 + kb:
// rows 16 rt .. 16 rt + 15 of A_j, k-block kb in k-slot order), then B_j in the chain waves' register
// order (chain wave wc's S[sl][i] at f32x4 index (wc * 2 + sl) * 8 + i of lane block `lane`).
namespace tr {
constexpr int A_HI = 0, A_LO = 32 * ws::FRAG, B = 64 * ws::FRAG;  // byte offsets
static_assert(B + pf::D * pf::D * 4 == sg::kTrans * 4, "a slot holds A's fragments and B");
__device__ __forceinline__ int b_at(int wc, int sl, int i, int lane) { return (((wc * 2 + sl) * 8 + i) * 64 + lane) * 4; }
}  // namespace tr
constexpr int kALd = pf::D + 4;  // row pitch (floats) of A_j's row-major LDS copy in the summary's fragment pass

// A local wave's inputs for one chunk, loaded a chunk ahead.  Local wave w (threads t < 256) holds K
// and V rows 4 tq + i x features 8 fb .. (t = 16 tq + fb: rows 16 w .. 16 w + 15), the q fragments of
// token tile w, the T diag(beta) fragments of token tile w, its rows' K l2norm factors and the g of
// token `lane`.  K, q and V are raw; rows past the chunk's end repeat its last row.  K and q are
// masked and normalised at their use (q in k-slot order: lane (c, g) of fragment s holds
// q[16 w + c][32 s + 4 g .. + 3] and [.. + 16 ..]); V needs no mask, as T diag(beta) has zero columns
// past the end (beta is 0 there), so those rows add nothing to U.  Every address is a wave-uniform
// base plus a 32-bit lane offset.
struct LocIn {
  u16x8 kr[4], vr[4], qr[4];
  bf16x8 tb[2], tl[2];  // T diag(beta) fragments: bf16 hi, and lo (written for chunks of slight decay only)
  f32x4 kn;  // the inverse kernel's l2norm factors of K rows 4 tq .. 4 tq + 3
  float graw;
  int lof;   // the T record's lo part was written
};
// Parts of a chunk's loads, and of phase 1 (kPart < 0: all): 0 the K rows and their l2norm factors,
// 1 the V rows and the T diag(beta) fragments, 2 the q rows, 3 the g values.  The chunk loop
// interleaves the next chunk's load parts with this chunk's phase-1 parts, so a wave's vector
// memory instructions do not queue up in one block after the barrier.
template <bool kNeedQ, int kPart = -1>
__device__ __forceinline__ void loc_load(LocIn& L, int64_t t0, int len, int kh, int h,
                                         const uint16_t* __restrict__ k, uint32_t ks, const uint16_t* __restrict__ q,
                                         uint32_t qs, const uint16_t* __restrict__ v, uint32_t vs,
                                         const uint8_t* __restrict__ tfr, const float* __restrict__ knc, bool q_on,
                                         bool want_lo) {
  using namespace pf;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const uint32_t tq = t >> 4, fb = t & 15;
  // byte offsets as 32-bit values: the loads address a uniform base plus a VGPR offset
  if (kPart < 0 || kPart == 0) {
    const char* kb = reinterpret_cast<const char*>(k + t0 * ks + (int64_t)kh * D);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t row = 4 * tq + i, rc = row < (uint32_t)len ? row : (uint32_t)len - 1;
      L.kr[i] = *reinterpret_cast<const u16x8*>(kb + ((rc * ks + 8 * fb) * 2u));
    }
    L.kn = *reinterpret_cast<const f32x4*>(reinterpret_cast<const char*>(knc) + tq * 16u);
  }
  if (kPart < 0 || kPart == 1) {
    const char* vb = reinterpret_cast<const char*>(v + t0 * vs + (int64_t)h * D);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t row = 4 * tq + i, rc = row < (uint32_t)len ? row : (uint32_t)len - 1;
      L.vr[i] = *reinterpret_cast<const u16x8*>(vb + ((rc * vs + 8 * fb) * 2u));
    }
    // every wave issues the same loads (tiles 0 and 1 read their one fragment twice): the wait
    // counts before the uses then stay exact along every path through the chunk loop.  A half
    // fragment is read 16 bytes a lane from its 8-byte slots (the upper 8 bytes, the next lane's or
    // the next fragment's, are dropped: the second block is zero)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      const int f = tf::fid(w, s);
      const bool hf = tf::half(f);
      u32x4 x = *reinterpret_cast<const u32x4*>(tfr + (uint32_t)(tf::offset(f) + lane * (hf ? 8 : 16)));
      // the lo half where the chunk's flag says it was written, else the hi half again (the same
      // loads, from lines just read: every path issues the same instructions)
      u32x4 y = *reinterpret_cast<const u32x4*>(tfr + (uint32_t)((want_lo ? tf::HALF : 0) + tf::offset(f) + lane * (hf ? 8 : 16)));
      if (hf) x[2] = x[3] = y[2] = y[3] = 0u;
      L.tb[s] = __builtin_bit_cast(bf16x8, x);
      L.tl[s] = __builtin_bit_cast(bf16x8, y);
    }
  }
  if (kNeedQ && (kPart < 0 || kPart == 2)) {  // a warm-up chunk (no outputs) reads one row for all lanes:
                                               // the loads stay, the bytes go
    const uint32_t row = 16 * w + (lane & 15), rc = !q_on ? 0u : (row < (uint32_t)len ? row : (uint32_t)len - 1);
    const char* qb = reinterpret_cast<const char*>(q + t0 * qs + (int64_t)kh * D);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint32_t off = (rc * qs + 32 * s + 4 * (lane >> 4)) * 2u;
      const u16x4 lo = *reinterpret_cast<const u16x4*>(qb + off), hi = *reinterpret_cast<const u16x4*>(qb + off + 32u);
      L.qr[s] = u16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  }
  if (kPart < 0 || kPart == 3)  // g of token `lane` (the last token's past the end), from the inverse kernel's record
  {
    L.graw = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(knc) + (pf::CH + lane) * 4u);
    L.lof = *reinterpret_cast<const int*>(reinterpret_cast<const char*>(knc) + kr::FLAG * 4u);
  }
}

// Whether a chunk's W S runs in hi + lo (its e^{G_last} above e^-2), read as a wave-uniform value so
// that the two forms are a scalar branch.  The local and chain waves read the same LDS word.
__device__ __forceinline__ bool chunk_precise(const SegBuf& B) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(B.gl))) > sg::kPreciseGl;
}
// Whether the chunk takes T diag(beta) as hi + lo (the inverse kernel's flag), wave-uniform.
__device__ __forceinline__ bool chunk_tlo(const SegBuf& B) { return __builtin_amdgcn_readfirstlane(B.lof) != 0; }

// Local phase 1 (wave w < 4): K rows (masked, l2-normalised when asked), V rows and the T diag(beta)
// fragments into the buffer, the q fragments (masked, l2-normalised when asked; kept in qf for
// phase 2); wave 0 also forms the decay factors (G, e^{G_last - G}, e^G, scale e^G, e^{G_last}).
// kPart as for loc_load: part p uses only the inputs of load part p.
template <bool kNeedQ, int kPart = -1>
__device__ __forceinline__ void loc_phase1(SegBuf& B, const LocIn& in, int len, int use_l2, bool q_on,
                                           bf16x8 (&qf)[4]) {
  using namespace pf;
  int t;  // opaque per call: the LDS addresses derived from it are not hoisted out of the chunk loop
  asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)threadIdx.x));
  const int w = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
  const int tq = t >> 4, fb = t & 15;
  if (kPart < 0 || kPart == 0) {  // K rows: zero past the chunk's end, scaled by the inverse kernel's l2norm factors
    const u16x8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u16x8 kr = use_l2 ? scale_bf16(in.kr[i], in.kn[i]) : in.kr[i];
      *reinterpret_cast<u16x8*>(&B.K[(4 * tq + i) * LDK + 8 * fb]) = 4 * tq + i < len ? kr : zero;
    }
  }
  if (kPart < 0 || kPart == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u16x8*>(&B.V[(4 * tq + i) * LDK + 8 * fb]) = in.vr[i];
#pragma unroll
    for (int s = 0; s < 2; ++s)
      if (2 * s <= w) *reinterpret_cast<bf16x8*>(B.tb + tf::fid(w, s) * ws::FRAG + lane * 16) = in.tb[s];
  }
  if (kNeedQ && (kPart < 0 || kPart == 2) && q_on) {
    const u16x8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
    const bool live = 16 * w + (lane & 15) < len;
    u16x8 qr[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) qr[s] = live ? in.qr[s] : zero;
    if (use_l2) {  // the row's 128 values sit in the 4 lanes c, c + 16, c + 32, c + 48
      // sum of squares = diagonal of Q Q^T over the tile's 16 rows (4 MFMAs on the fragments in
      // hand: as a B operand, lane (c, g)'s A fragment is Q^T's).  The products are exact and summed
      // in fp32, where torch rounds each square to bf16 first: the factor can differ from torch's by
      // one bf16 ulp on some rows, which only moves outputs (q does not enter the state).
      f32x4 qq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) qq = mma(__builtin_bit_cast(bf16x8, qr[s]), __builtin_bit_cast(bf16x8, qr[s]), qq);
      const int c16 = lane & 15, g4 = lane >> 4;  // (Q Q^T)[c][c] sits in lane (c, c / 4), element c % 4
      const float dg = (c16 & 3) == 0 ? qq[0] : (c16 & 3) == 1 ? qq[1] : (c16 & 3) == 2 ? qq[2] : qq[3];
      const float ss = xor32_sum(xor16_sum(g4 == (c16 >> 2) ? dg : 0.f));
      const float inv = l2norm_inv(ss);
#pragma unroll
      for (int s = 0; s < 4; ++s) qr[s] = scale_bf16(qr[s], inv);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      qf[s] = __builtin_bit_cast(bf16x8, qr[s]);
      *reinterpret_cast<bf16x8*>(B.qg + (w * 4 + s) * ws::FRAG + lane * 16) = qf[s];
    }
  }
  if ((kPart < 0 || kPart == 3) && w == 0) {
    const float G = wave_incl_scan(lane < len ? in.graw : 0.f);  // g = 0 past the chunk's end
    const float gl = __shfl(G, 63, kWave);
    const float eg = __expf(G);  // the hardware exp: within a few fp32 ulp, far below the bf16 roundings
    B.gs[lane] = G;
    B.dec[lane] = __expf(gl - G);
    B.eg[lane] = eg;
    B.egs[lane] = kScale * eg;
    if (lane == 0) {
      B.gl = __expf(gl);
      B.lof = in.lof;
    }
  }
}

// Local phase 2 (wave W < 4, after the K rows and the decay are in): the QK fragments and the -W
// fragments of token tile W.  (Q K^T)^T = K Q^T and W^T = K^T (T diag(beta e^G))^T: both accumulator
// layouts are the k-slot ordered fragment layouts.  T diag(beta e^G) is the inverse kernel's
// T diag(beta) with column j scaled by e^{G_j} (element e of lane (c, g) in k-block s is column
// 32 s + 16 (e >> 2) + 4 g + (e & 3)).
template <int W, bool kNeedQ>
__device__ __forceinline__ void loc_phase2(const SegBuf& B, SegOps& P, const bf16x8 (&qf)[4], const bf16x8 (&tbu)[2],
                                           const bf16x8 (&tlu)[2], bool q_on) {
  using namespace pf;
  int t;
  asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)threadIdx.x));
  const int lane = t & 63, c16 = lane & 15, g4 = lane >> 4;
  const bool precise = chunk_precise(B), tlo = chunk_tlo(B);
  bf16x8 tbe[2], tbl[2];  // T diag(beta e^G), and in a precise chunk the lo part of its fp32 value
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (2 * s > W) continue;
    const f32x4 e0 = *reinterpret_cast<const f32x4*>(&B.eg[32 * s + 4 * g4]);
    const f32x4 e1 = *reinterpret_cast<const f32x4*>(&B.eg[32 * s + 16 + 4 * g4]);
    const u32x4v u = __builtin_bit_cast(u32x4v, tbu[s]);
    f32x4 a, b;
    a[0] = __uint_as_float(u[0] << 16);
    a[1] = __uint_as_float(u[0] & 0xffff0000u);
    a[2] = __uint_as_float(u[1] << 16);
    a[3] = __uint_as_float(u[1] & 0xffff0000u);
    b[0] = __uint_as_float(u[2] << 16);
    b[1] = __uint_as_float(u[2] & 0xffff0000u);
    b[2] = __uint_as_float(u[3] << 16);
    b[3] = __uint_as_float(u[3] & 0xffff0000u);
    if (tlo) {  // T diag(beta) = hi + lo; its lo fragments go to the chain for U as well
      const u32x4v l = __builtin_bit_cast(u32x4v, tlu[s]);
      a[0] += __uint_as_float(l[0] << 16);
      a[1] += __uint_as_float(l[0] & 0xffff0000u);
      a[2] += __uint_as_float(l[1] << 16);
      a[3] += __uint_as_float(l[1] & 0xffff0000u);
      b[0] += __uint_as_float(l[2] << 16);
      b[1] += __uint_as_float(l[2] & 0xffff0000u);
      b[2] += __uint_as_float(l[3] << 16);
      b[3] += __uint_as_float(l[3] & 0xffff0000u);
      *reinterpret_cast<bf16x8*>(P.tl + tf::fid(W, s) * ws::FRAG + lane * 16) = tlu[s];
    }
    a *= e0;
    b *= e1;
    tbe[s] = pack_acc_bf16(a, b);
    if (precise) tbl[s] = lo_bf16(a, b, tbe[s]);
  }
  if (kNeedQ && q_on) {
    f32x4 accQ[W + 1];
#pragma unroll
    for (int cb = 0; cb <= W; ++cb) accQ[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int cb = 0; cb <= W; ++cb) accQ[cb] = mma(frag_kperm(B.K, LDK, 16 * cb, 32 * s, lane), qf[s], accQ[cb]);
    const float gi = B.gs[16 * W + c16];
    f32x4 qk[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const f32x4 gj = *reinterpret_cast<const f32x4*>(&B.gs[16 * cb + 4 * g4]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {  // QK[i][jj], i = 16W + c, jj = 16cb + 4g + r
        const int jj = 16 * cb + 4 * g4 + r;
        qk[cb][r] = (cb <= W && 16 * W + c16 >= jj) ? kScale * accQ[cb <= W ? cb : 0][r] * __expf(gi - gj[r]) : 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (2 * j <= W)
        *reinterpret_cast<bf16x8*>(P.qk + tf::fid(W, j) * ws::FRAG + lane * 16) = pack_acc_bf16(qk[2 * j], qk[2 * j + 1]);
  }
  f32x4 accW[8];
  if (precise) {  // W from hi + lo of T diag(beta e^G), stored as hi + lo
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
      const bf16x8 k0 = __builtin_bit_cast(bf16x8, frag_tr_kperm(B.K, LDK, 0, 16 * cb, lane));
      accW[cb] = mma(k0, tbe[0], f32x4{0.f, 0.f, 0.f, 0.f});
      accW[cb] = mma(k0, tbl[0], accW[cb]);
      if (W >= 2) {
        const bf16x8 k1 = __builtin_bit_cast(bf16x8, frag_tr_kperm(B.K, LDK, 32, 16 * cb, lane));
        accW[cb] = mma(k1, tbe[1], accW[cb]);
        accW[cb] = mma(k1, tbl[1], accW[cb]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bf16x8 hi, lo;
      split_bf16(-accW[2 * j], -accW[2 * j + 1], hi, lo);
      *reinterpret_cast<bf16x8*>(P.wn + (W * 4 + j) * ws::FRAG + lane * 16) = hi;
      *reinterpret_cast<bf16x8*>(P.wl + (W * 4 + j) * ws::FRAG + lane * 16) = lo;
    }
    return;
  }
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) {
    accW[cb] = mma(__builtin_bit_cast(bf16x8, frag_tr_kperm(B.K, LDK, 0, 16 * cb, lane)), tbe[0], f32x4{0.f, 0.f, 0.f, 0.f});
    if (W >= 2) accW[cb] = mma(__builtin_bit_cast(bf16x8, frag_tr_kperm(B.K, LDK, 32, 16 * cb, lane)), tbe[1], accW[cb]);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
    *reinterpret_cast<bf16x8*>(P.wn + (W * 4 + j) * ws::FRAG + lane * 16) = pack_acc_bf16(-accW[2 * j], -accW[2 * j + 1]);
}


// A chain wave's state: columns 32 w' .. 32 w' + 31 of the value head's [128, 128] fp32 state as two
// 16-column slices (n = 2 w' + sl), S[sl][i][r] = S[16 i + 4 g + r][16 n + c].
struct ChainRegs {
  f32x4 S[2][8];
  bf16x8 hi[2][2], lo[2][2];  // DEC vn, split by part 1 for part 2
};
// DEC vn -> hi + lo bf16 (the k-slot ordered B fragments of the update).
__device__ __forceinline__ void dec_split(const SegBuf& B, f32x4 (&vn)[2][4], ChainRegs& R, int g4) {
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const f32x4 dec = *reinterpret_cast<const f32x4*>(&B.dec[16 * tb + 4 * g4]);
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) vn[sl][tb] *= dec;
  }
#pragma unroll
  for (int sl = 0; sl < 2; ++sl)
#pragma unroll
    for (int j = 0; j < 2; ++j) split_bf16(vn[sl][2 * j], vn[sl][2 * j + 1], R.hi[sl][j], R.lo[sl][j]);
}
// The output pass's stores.  The chain waves leave bf16(o) in the chunk's V tile (each wave in its
// own 32 columns, which only it reads); during the next step, local wave w reads rows 16 w .. 16 w +
// 15 of it just before it writes the next V rows there, and stores them, 16 bytes per lane -- as
// they are (kNorm 0), or through the gated RMSNorm of the fused prefill layer (HF
// Qwen3_5RMSNormGated, modeling_qwen3_5.py, over each (token, value head) row of D = 128):
// out = bf16(w bf16(x rsqrt(mean(x^2) + eps)) silu(z)) with x = bf16(o).  Lane mapping, sum order (8 columns in a lane, then
// the butterfly over 16 lanes) and roundings are gated_rmsnorm128_kernel's: the result is the same,
// bit for bit, as that kernel applied to the stored outputs.
struct GateArgs {
  const uint16_t* z;  // [tokens, Hv * D] bf16 gate rows, token stride zs
  int64_t zs;
  const void* w;      // [D] norm weight, bf16 (kNorm 1) or fp32 (kNorm 2)
  float eps;
};
struct NormIn {
  u16x8 o[4], z[4];  // rows 4 tq + i, columns 8 fb .. 8 fb + 7 (t = 16 tq + fb)
};
// Requests one chunk's z rows (token base zb = z + t0 zs + h D; rows past len repeat the last).
__device__ __forceinline__ void norm_fetch_z(NormIn& N, const uint16_t* __restrict__ zb, uint32_t zs, int len) {
  int t;
  asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)threadIdx.x));
  const uint32_t tq = t >> 4, fb = t & 15;
  const char* zc = reinterpret_cast<const char*>(zb);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t row = 4 * tq + i, rc = row < (uint32_t)len ? row : (uint32_t)len - 1;
    N.z[i] = *reinterpret_cast<const u16x8*>(zc + ((rc * zs + 8 * fb) * 2u));
  }
}
// Reads a chunk's bf16 outputs from the V tile of B.
__device__ __forceinline__ void norm_fetch_o(NormIn& N, const SegBuf& B) {
  using namespace pf;
  int t;
  asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)threadIdx.x));
  const uint32_t tq = t >> 4, fb = t & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) N.o[i] = *reinterpret_cast<const u16x8*>(&B.V[(4 * tq + i) * LDK + 8 * fb]);
}
// Normalises, gates and stores the rows of N below len (ob = out + (t0 Hv + h) D); wt = the weight
// of columns 8 fb .. 8 fb + 7.
template <int kNorm>
__device__ __forceinline__ void norm_store(const NormIn& N, const float (&wt)[8], float eps, uint16_t* __restrict__ ob,
                                           int Hv, int len) {
  using namespace pf;
  int t;
  asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)threadIdx.x));
  const int tq = t >> 4, fb = t & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * tq + i;
    if (kNorm == 0) {  // no norm: the outputs as they are
      if (row < len) *reinterpret_cast<u16x8*>(ob + ((int64_t)row * Hv * D + 8 * fb)) = N.o[i];
      continue;
    }
    float xf[8], ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xf[e] = bf2f(N.o[i][e]);
      ss += xf[e] * xf[e];
    }
    ss = row16_sum(ss);
    const float inv = rsq_fast(ss / 128.0f + eps);
    u32x4v ov;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {  // pairs: one conversion rounds two values
      const uint32_t xn = f2bf2(xf[e] * inv, xf[e + 1] * inv);
      float y0 = wt[e] * __uint_as_float(xn << 16), y1 = wt[e + 1] * __uint_as_float(xn & 0xffff0000u);
      if (kNorm == 1) {
        const uint32_t yr = f2bf2(y0, y1);
        y0 = __uint_as_float(yr << 16);
        y1 = __uint_as_float(yr & 0xffff0000u);
      }
      ov[e >> 1] = f2bf2(y0 * silu_fast(bf2f(N.z[i][e])), y1 * silu_fast(bf2f(N.z[i][e + 1])));
    }
    if (row < len) *reinterpret_cast<u32x4v*>(ob + ((int64_t)row * Hv * D + 8 * fb)) = ov;
  }
}
// Chain part 1 for one chunk: U (fp32, from the inverse kernel's T diag(beta) fragments and the V
// rows), vn = U - W S, the outputs o = diag(scale e^G) Q S + QK vn (kOut: left in bf16 in the V tile
// for the local waves to store), and DEC vn split for part 2.  W S and Q S share the loop over the state's k-blocks j
// (16 independent accumulators); the LDS fragments of block j + 1 are requested before the products
// of block j, so their latency hides behind those products.  kPrecise: W S = Wh Sh + Wh Sl + Wl Sh
// from the hi + lo parts of -W and of the state; block j's state parts are formed in its step and
// its -W lo fragments requested there (behind the hi products), which keeps the registers of the
// fast form.
template <bool kUseU, bool kOut, bool kPrecise, bool kTlo>
__device__ __forceinline__ void chain_part1(const SegBuf& B, const SegOps& P, ChainRegs& R, int wc, int lane_in) {
  using namespace pf;
  int lane;
  asm volatile("v_mov_b32 %0, %1" : "=v"(lane) : "v"(lane_in));
  const int c16 = lane & 15, g4 = lane >> 4;
  bf16x8 fw[4], fq[4];  // block j's -W and q fragments (token tiles 0..3)
  auto fetch = [&](int j, bf16x8 (&w_)[4], bf16x8 (&q_)[4]) {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      w_[tb] = lds_frag(P.wn, tb * 4 + j, lane);
      if (kOut) q_[tb] = lds_frag(B.qg, tb * 4 + j, lane);
    }
  };
  // the U operands and block 0's fragments are requested first; the bf16 copy of the state is
  // formed while they arrive
  bf16x8 vf[2][2], ft[tf::FRAGS];
  if (kUseU) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int sl = 0; sl < 2; ++sl)
        vf[kb][sl] = __builtin_bit_cast(bf16x8, frag_tr_kperm(B.V, LDK, 32 * kb, 16 * (2 * wc + sl), lane));
#pragma unroll
    for (int f = 0; f < tf::FRAGS; ++f) ft[f] = lds_frag(B.tb, f, lane);
  }
  fetch(0, fw, fq);
  __builtin_amdgcn_sched_barrier(0);
  bf16x8 Sb[2][4];
  if (!kPrecise) {
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
      for (int j = 0; j < 4; ++j) Sb[sl][j] = pack_acc_bf16(R.S[sl][2 * j], R.S[sl][2 * j + 1]);
  }
  f32x4 acc[2][4];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl)
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) acc[sl][tb] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (kUseU) {  // U = T diag(beta) V, token tile tb, k-blocks kb <= tb / 2 (kTlo: T's hi and lo parts)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
        if (2 * kb <= tb) {
          acc[0][tb] = mma(ft[tf::fid(tb, kb)], vf[kb][0], acc[0][tb]);
          acc[1][tb] = mma(ft[tf::fid(tb, kb)], vf[kb][1], acc[1][tb]);
        }
    if (kTlo) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
          if (2 * kb <= tb) {
            const bf16x8 fl = lds_frag(P.tl, tf::fid(tb, kb), lane);
            acc[0][tb] = mma(fl, vf[kb][0], acc[0][tb]);
            acc[1][tb] = mma(fl, vf[kb][1], acc[1][tb]);
          }
    }
  }
  // o^T tile by tile: lane (c, g) of O[tb][sl] holds o[16 tb + c][16 n + 4 g .. 4 g + 3]
  f32x4 O[4][2];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) O[tb][0] = O[tb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bf16x8 nw[4], nq[4], fl[4], Sl[2];
    if (j < 3) fetch(j + 1, nw, nq);
    if (kPrecise) {
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) fl[tb] = lds_frag(P.wl, tb * 4 + j, lane);
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) split_bf16(R.S[sl][2 * j], R.S[sl][2 * j + 1], Sb[sl][j], Sl[sl]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      acc[0][tb] = mma(fw[tb], Sb[0][j], acc[0][tb]);
      acc[1][tb] = mma(fw[tb], Sb[1][j], acc[1][tb]);
      if (kOut) {
        O[tb][0] = mma(Sb[0][j], fq[tb], O[tb][0]);
        O[tb][1] = mma(Sb[1][j], fq[tb], O[tb][1]);
      }
    }
    if (kPrecise) {
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        acc[0][tb] = mma(fw[tb], Sl[0], acc[0][tb]);
        acc[1][tb] = mma(fw[tb], Sl[1], acc[1][tb]);
      }
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        acc[0][tb] = mma(fl[tb], Sb[0][j], acc[0][tb]);
        acc[1][tb] = mma(fl[tb], Sb[1][j], acc[1][tb]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (j < 3) {
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        fw[tb] = nw[tb];
        if (kOut) fq[tb] = nq[tb];
      }
    }
  }
  if (kOut) {
    bf16x8 kq[tf::FRAGS];
#pragma unroll
    for (int f = 0; f < tf::FRAGS; ++f) kq[f] = lds_frag(P.qk, f, lane);
    const float e0 = B.egs[c16], e1 = B.egs[16 + c16], e2 = B.egs[32 + c16], e3 = B.egs[48 + c16];
    bf16x8 vb[2][2];
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      vb[sl][0] = pack_acc_bf16(acc[sl][0], acc[sl][1]);
      vb[sl][1] = pack_acc_bf16(acc[sl][2], acc[sl][3]);
    }
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      O[0][sl] *= e0;
      O[1][sl] *= e1;
      O[2][sl] *= e2;
      O[3][sl] *= e3;
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int tb = 2 * jj; tb < 4; ++tb) {
        O[tb][0] = mma(vb[0][jj], kq[tf::fid(tb, jj)], O[tb][0]);
        O[tb][1] = mma(vb[1][jj], kq[tf::fid(tb, jj)], O[tb][1]);
      }
    // bf16(o) into this wave's 32 columns of the V tile (read by no other wave): the local waves
    // store the rows one step later (through the gated norm when asked), off the chain's path
    uint16_t* vrow = const_cast<uint16_t*>(B.V) + c16 * LDK + 32 * wc + 4 * g4;
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) {
        const u32x2v pk = {f2bf2(O[tb][sl][0], O[tb][sl][1]), f2bf2(O[tb][sl][2], O[tb][sl][3])};
        *reinterpret_cast<u32x2v*>(vrow + 16 * tb * LDK + 16 * sl) = pk;
      }
  }
  // DEC vn is split here, not in part 2: the chain has slack in the step's first half, where the
  // local waves (phase 1, the outputs' stores or the gated norm) take longer, and none in the
  // second (T=8192: 1-2% faster than splitting in part 2, 1.4% slower when every chunk takes W S in
  // hi + lo)
  dec_split(B, acc, R, g4);
}
// Chain part 2: S' = e^{G_last} S + K^T (DEC vn), K^T straight from the K rows (exact in bf16).  For
// each token half j the hi terms of all 16 accumulators go first, then the lo terms; the K^T
// fragments of half 1 are requested before the products of half 0.
__device__ __forceinline__ void chain_part2(const SegBuf& B, ChainRegs& R, int lane_in) {
  using namespace pf;
  int lane;
  asm volatile("v_mov_b32 %0, %1" : "=v"(lane) : "v"(lane_in));
  bf16x8 kt[2][8];
  const float gl = B.gl;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) kt[j][i] = __builtin_bit_cast(bf16x8, frag_tr_kperm(B.K, LDK, 32 * j, 16 * i, lane));
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (j == 0) {  // the decay of the state, each tile just before its first product
        R.S[0][i] *= gl;
        R.S[1][i] *= gl;
      }
      R.S[0][i] = mma(kt[j][i], R.hi[0][j], R.S[0][i]);
      R.S[1][i] = mma(kt[j][i], R.hi[1][j], R.S[1][i]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      R.S[0][i] = mma(kt[j][i], R.lo[0][j], R.S[0][i]);
      R.S[1][i] = mma(kt[j][i], R.lo[1][j], R.S[1][i]);
    }
  }
}

// Segment kernel.  pass 0 (output): one workgroup per (segment, value head) from the segment's
// initial state (the sequence's initial state row, zero, or the combined state of the previous
// segment in its transition slot), writing o and, at a sequence's last segment, the final state.
// pass 1 (summary): two workgroups per (transition slot, value head): B (from zero, with U) and A
// (from the identity, without U), written into the slot; A is skipped when negligible.
// Waves 0-3 (local) prepare chunk c+1's operands in one buffer (and store chunk c-1's outputs) while
// waves 4-7 (chain) run chunk c from the other: two LDS barriers a chunk, met by both roles.
template <typename BetaT, typename OutT, int kPass, int kNorm = 0>
__global__ __launch_bounds__(sg::NT, 1) void seg_kernel(
    const uint16_t* __restrict__ q, int64_t qs, const uint16_t* __restrict__ k, int64_t ks, const uint16_t* __restrict__ v,
    int64_t vs, const float* __restrict__ g,
    const BetaT* __restrict__ beta, OutT* __restrict__ out, SegTable tab, int Hqk, int Hv, int use_l2,
    const float* __restrict__ init,
    const int32_t* __restrict__ rows, int n_rows, float* __restrict__ final_state, float* __restrict__ trans,
    int* __restrict__ tflags, const uint8_t* __restrict__ tfrag, const float* __restrict__ knorm,
    const int* __restrict__ warm, GateArgs gate) {
  using namespace pf;
  __shared__ SegSmem sm;
  static_assert(sizeof(SegSmem) >= (size_t)D * kALd * 4 && sizeof(SegSmem) >= 2 * 64 * ws::FRAG,
                "the chunk buffers hold A_j's row-major copy and two slots' A fragments");
  const int t = threadIdx.x, w = t >> 6, lane = t & 63, c16 = lane & 15, g4 = lane >> 4;
  int mode, h, s, idx, slot = -1;
  if (kPass == 0) {
    const int item = xcd_item(blockIdx.x, gridDim.x), jo = item / Hv;
    h = item % Hv;
    if (jo >= tab.first_seg(tab.nseq)) return;
    const int j = tab.order ? tab.order[jo] : jo;
    s = tab.seq_of_seg(j);
    idx = j - tab.first_seg(s);
    if (idx > 0) slot = tab.first_slot(s) + idx - 1;  // the previous segment's slot holds this one's state
    mode = kSegOut;
  } else {
    const int item = xcd_item(blockIdx.x, gridDim.x), rest = item >> 1;
    const int ts = rest / Hv;
    h = rest % Hv;
    if (ts >= tab.first_slot(tab.nseq)) return;
    s = tab.seq_of_slot(ts);
    idx = ts - tab.first_slot(s);
    slot = ts;
    mode = (item & 1) ? kSegA : kSegB;
    if (seq_warm_ok(tab, warm, Hv, h, s)) return;  // the output pass warms up instead
  }
  const bool warm_path = kPass == 0 && slot >= 0 && seq_warm_ok(tab, warm, Hv, h, s);
  // the output pass of a later segment on the exact path forms its initial state from the summaries of
  // the idx slots before it (ts_first .. ts_first + idx - 1)
  const int combine_steps = (kPass == 0 && slot >= 0 && !warm_path) ? idx : 0;
  const int ts_first = tab.first_slot(s);
  const int kh = h / (Hv / Hqk);
  const int nch_s = tab.nch(s), c_begin = idx * tab.L;
  const int n = nch_s - c_begin < tab.L ? nch_s - c_begin : tab.L;
  const int64_t t_seq = tab.start(s);
  const int Ls = tab.len(s);
  float* tslot = slot >= 0 ? trans + ((int64_t)slot * Hv + h) * sg::kTrans : nullptr;
  if (mode == kSegA) {  // is A negligible?  (exp of the summed log decay, unit keys, beta in [0, 1])
    int compute = 1;
    if (use_l2) {
      const int64_t tb0 = t_seq + (int64_t)c_begin * CH;
      const int ntok = (Ls - c_begin * CH) < n * CH ? Ls - c_begin * CH : n * CH;
      float sum = 0.f;
      int ok = 1;
      for (int i = t; i < ntok; i += sg::NT) {
        sum += g[(tb0 + i) * Hv + h];
        const float b = Elem<BetaT>::load(beta + (tb0 + i) * Hv + h);
        ok &= (b >= 0.f && b <= 1.f) ? 1 : 0;
      }
      sum = wave_sum_fast(sum);
      ok = __builtin_amdgcn_ballot_w64(ok == 0) == 0 ? 1 : 0;
      if (lane == 0) sm.red[w] = ok ? sum : __builtin_huge_valf();
      __syncthreads();
      float tot = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) tot += sm.red[i];
      compute = tot < sg::kNegligibleLog ? 0 : 1;  // NaN or a beta outside [0, 1]: computed
    }
    if (t == 0) tflags[(int64_t)slot * Hv + h] = compute;
    if (!compute) return;
  }
  constexpr bool need_q = kPass == 0;
  // pass 0 after a warm-up: the chain starts from zero w0 chunks before the segment, without outputs
  const int w0 = (kPass == 0 && warm_path) ? warm[(int64_t)slot * Hv + h] : 0;
  const int cb0 = c_begin - w0, ntot = n + w0;
  const int chunk_slot0 = tab.first_chunk(s) + cb0;
  auto tfr = [&](int c) { return tfrag + ((int64_t)(chunk_slot0 + c) * Hv + h) * tf::BYTES; };
  auto chunk_t0 = [&](int c) { return t_seq + (int64_t)(cb0 + c) * CH; };
  auto chunk_len = [&](int c) { return Ls - (cb0 + c) * CH < CH ? Ls - (cb0 + c) * CH : CH; };
  if (w < 4) {
    // ------------------------------------------------------------ local waves
    // Chunk j's inputs are loaded into register set j & 1 a full step before they are used: step c
    // requests chunk c + 2 into one set and prepares chunk c + 1 from the other.  The chunk loop is
    // unrolled by two so that each set keeps its registers; every load in it is unconditional (past
    // the end the last chunk is requested again, unused), which keeps the wait counts exact.
    LocIn ia, ib;
    bf16x8 qf[4], tbu[2], tlu[2];
    auto load = [&](LocIn& L, int c, auto part, bool want_lo) __attribute__((always_inline)) {
      loc_load<need_q, decltype(part)::value>(L, chunk_t0(c), chunk_len(c), kh, h, k, (uint32_t)ks, q, (uint32_t)qs, v,
                                              (uint32_t)vs, tfr(c),
                                              knorm + ((int64_t)(chunk_slot0 + c) * Hv + h) * kr::FLOATS, c >= w0,
                                              want_lo);
    };
    // chunk c's lo flag (the inverse kernel's): read a step before the chunk's own loads need it
    auto lo_flag = [&](int c) __attribute__((always_inline)) {
      const int cc = c < ntot ? c : ntot - 1;
      return reinterpret_cast<const int*>(knorm)[((int64_t)(chunk_slot0 + cc) * Hv + h) * kr::FLOATS + kr::FLAG] != 0;
    };
    bool lof_next = false;  // chunk c + 2's flag in step c
    auto phase2 = [&](const SegBuf& B, bool q_on) __attribute__((always_inline)) {
      switch (w) {
        case 0: loc_phase2<0, need_q>(B, sm.ops, qf, tbu, tlu, q_on); break;
        case 1: loc_phase2<1, need_q>(B, sm.ops, qf, tbu, tlu, q_on); break;
        case 2: loc_phase2<2, need_q>(B, sm.ops, qf, tbu, tlu, q_on); break;
        default: loc_phase2<3, need_q>(B, sm.ops, qf, tbu, tlu, q_on); break;
      }
    };
    // the stores of chunk j's outputs (j >= w0); the gated norm's weight of columns 8 fb .. 8 fb + 7
    float wt[8];
    if (kNorm) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int col = 8 * (t & 15) + e;
        wt[e] = kNorm == 1 ? bf2f(reinterpret_cast<const uint16_t*>(gate.w)[col]) : reinterpret_cast<const float*>(gate.w)[col];
      }
    }
    NormIn nin;
    auto norm_req_z = [&](int j) __attribute__((always_inline)) {  // a step ahead of its use
      const int jz = j >= w0 ? j : w0;  // a chunk without outputs requests a valid chunk's rows, unused
      norm_fetch_z(nin, gate.z + chunk_t0(jz) * gate.zs + (int64_t)h * D, (uint32_t)gate.zs, chunk_len(jz));
    };
    auto norm_out = [&](int j) __attribute__((always_inline)) {
      norm_store<kNorm>(nin, wt, gate.eps, out + (chunk_t0(j >= w0 ? j : w0) * Hv + h) * D, Hv,
                        j >= w0 ? chunk_len(j) : 0);
    };
    auto step = [&](int c, LocIn& nxt, const LocIn& cur) __attribute__((always_inline)) {  // prepare chunk c + 1 from cur
      if (kPass == 0) norm_fetch_o(nin, sm.buf[(c + 1) & 1]);  // the chain's outputs of step c - 1, before
                                                          // chunk c + 1's V rows replace them
      {  // chunk c + 2's load parts interleaved with chunk c + 1's phase-1 parts
        const int cn = c + 2 < ntot ? c + 2 : ntot - 1;
        const bool want_lo = lof_next;
        lof_next = lo_flag(c + 3);
        SegBuf& B1 = sm.buf[(c + 1) & 1];
        const int len1 = chunk_len(c + 1);
        load(nxt, cn, std::integral_constant<int, 0>{}, want_lo);
        __builtin_amdgcn_sched_barrier(0);
        loc_phase1<need_q, 0>(B1, cur, len1, use_l2, c + 1 >= w0, qf);
        __builtin_amdgcn_sched_barrier(0);
        load(nxt, cn, std::integral_constant<int, 1>{}, want_lo);
        __builtin_amdgcn_sched_barrier(0);
        loc_phase1<need_q, 1>(B1, cur, len1, use_l2, c + 1 >= w0, qf);
        __builtin_amdgcn_sched_barrier(0);
        load(nxt, cn, std::integral_constant<int, 2>{}, want_lo);
        __builtin_amdgcn_sched_barrier(0);
        loc_phase1<need_q, 2>(B1, cur, len1, use_l2, c + 1 >= w0, qf);
        __builtin_amdgcn_sched_barrier(0);
        load(nxt, cn, std::integral_constant<int, 3>{}, want_lo);
        __builtin_amdgcn_sched_barrier(0);
        loc_phase1<need_q, 3>(B1, cur, len1, use_l2, c + 1 >= w0, qf);
      }
      tbu[0] = cur.tb[0];
      tbu[1] = cur.tb[1];
      tlu[0] = cur.tl[0];
      tlu[1] = cur.tl[1];
      if (kPass == 0) norm_out(c - 1);
      if (kNorm) norm_req_z(c);
      lds_barrier();
      phase2(sm.buf[(c + 1) & 1], c + 1 >= w0);
      lds_barrier();
    };
    if (combine_steps > 0) {
      // the combination's A fragments: slot kk's into LDS half kk & 1 while the chain waves use the other
      // half; each slot's loads are issued a step before its LDS writes (two register sets, the loop
      // unrolled by two), so their latency hides behind a step of products
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      u32x4 a0[16], a1[16];
      auto live = [&](int kk) { return kk < combine_steps && tflags[(int64_t)(ts_first + kk) * Hv + h] != 0; };
      auto fetch_a = [&](u32x4 (&a)[16], int kk) __attribute__((always_inline)) {
        const uint8_t* src = reinterpret_cast<const uint8_t*>(trans + ((int64_t)(ts_first + kk) * Hv + h) * sg::kTrans);
#pragma unroll
        for (int u = 0; u < 16; ++u) a[u] = *reinterpret_cast<const u32x4*>(src + (t + 256 * u) * 16);
      };
      auto put_a = [&](const u32x4 (&a)[16], int kk) __attribute__((always_inline)) {
        uint8_t* dst = reinterpret_cast<uint8_t*>(&sm) + (kk & 1) * (64 * ws::FRAG);
#pragma unroll
        for (int u = 0; u < 16; ++u) *reinterpret_cast<u32x4*>(dst + (t + 256 * u) * 16) = a[u];
      };
      if (live(0)) fetch_a(a0, 0);
      if (live(1)) fetch_a(a1, 1);
      if (live(0)) put_a(a0, 0);
      __syncthreads();
      for (int kk = 0; kk < combine_steps; kk += 2) {  // the chain runs step kk, then step kk + 1
        if (live(kk + 1)) put_a(a1, kk + 1);  // half 1 was last read in step kk - 1
        if (live(kk + 2)) fetch_a(a0, kk + 2);
        __syncthreads();
        if (kk + 1 < combine_steps) {
          if (live(kk + 2)) put_a(a0, kk + 2);
          if (live(kk + 3)) fetch_a(a1, kk + 3);
          __syncthreads();
        }
      }
    }
    if (ntot > 0) {
      if (kNorm) norm_req_z(-1);  // unused: every step then finds one z request in flight
      load(ia, 0, std::integral_constant<int, -1>{}, lo_flag(0));
      load(ib, ntot > 1 ? 1 : 0, std::integral_constant<int, -1>{}, lo_flag(1));
      lof_next = lo_flag(2);
      loc_phase1<need_q>(sm.buf[0], ia, chunk_len(0), use_l2, w0 == 0, qf);
      tbu[0] = ia.tb[0];
      tbu[1] = ia.tb[1];
      tlu[0] = ia.tl[0];
      tlu[1] = ia.tl[1];
    }
    lds_barrier();
    if (ntot > 0) phase2(sm.buf[0], w0 == 0);
    lds_barrier();
    int c = 0;
    for (; c + 2 < ntot; c += 2) {
      step(c, ia, ib);
      step(c + 1, ib, ia);
    }
    if (c + 1 < ntot) step(c, ia, ib);
    if (ntot > 0) {  // the chain's last step: nothing left to prepare (the outputs of the last two chunks)
      if (kPass == 0 && ntot > 1) {
        norm_fetch_o(nin, sm.buf[ntot & 1]);
        norm_out(ntot - 2);
      }
      if (kNorm) norm_req_z(ntot - 1);
      lds_barrier();
      lds_barrier();
      if (kPass == 0) {
        norm_fetch_o(nin, sm.buf[(ntot - 1) & 1]);
        norm_out(ntot - 1);
      }
    }
  } else {
    // ------------------------------------------------------------ chain waves
    const int wc = w - 4;
    ChainRegs R;
    {  // initial state: the sequence's (then, on the exact path, the combination below), or zero
      const float* src = nullptr;
      if (mode == kSegOut && (slot < 0 || !warm_path) && init) {
        const int r0 = state_row(rows, n_rows, s);
        if (r0 >= 0) src = init + ((int64_t)r0 * Hv + h) * D * D;
      }
      if (src) {
#pragma unroll
        for (int sl = 0; sl < 2; ++sl)
#pragma unroll
          for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) R.S[sl][i][r] = src[(16 * i + 4 * g4 + r) * D + 32 * wc + 16 * sl + c16];
      } else {
#pragma unroll
        for (int sl = 0; sl < 2; ++sl)
#pragma unroll
          for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              R.S[sl][i][r] = (mode == kSegA && 16 * i + 4 * g4 + r == 32 * wc + 16 * sl + c16) ? 1.f : 0.f;
      }
    }
    if (combine_steps > 0) {  // S_{k+1} = A_k S_k + B_k over the slots before this segment
      f32x4 bn[2][8];
      auto fetch_b = [&](int kk) __attribute__((always_inline)) {
        const float* src = trans + ((int64_t)(ts_first + kk) * Hv + h) * sg::kTrans + D * D;
#pragma unroll
        for (int sl = 0; sl < 2; ++sl)
#pragma unroll
          for (int i = 0; i < 8; ++i) bn[sl][i] = *reinterpret_cast<const f32x4*>(src + tr::b_at(wc, sl, i, lane));
      };
      fetch_b(0);
      __syncthreads();
      for (int kk = 0; kk < combine_steps; ++kk) {
        const bool fl = tflags[(int64_t)(ts_first + kk) * Hv + h] != 0;
        f32x4 acc[2][8];
#pragma unroll
        for (int sl = 0; sl < 2; ++sl)
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[sl][i] = bn[sl][i];
        if (kk + 1 < combine_steps) fetch_b(kk + 1);
        if (fl) {
          const uint8_t* ah = reinterpret_cast<const uint8_t*>(&sm) + (kk & 1) * (64 * ws::FRAG);
          const uint8_t* al = ah + 32 * ws::FRAG;
          // the 32 (k-block, row tile) steps in order, each one's two fragments requested a step ahead
          bf16x8 nh = lds_frag(ah, 0, lane), no = lds_frag(al, 0, lane);
          bf16x8 sh[2], slo[2];
#pragma unroll
          for (int it = 0; it < 32; ++it) {
            const int kb = it >> 3, rt = it & 7;
            if (rt == 0) {
#pragma unroll
              for (int sl = 0; sl < 2; ++sl) split_bf16(R.S[sl][2 * kb], R.S[sl][2 * kb + 1], sh[sl], slo[sl]);
            }
            const bf16x8 fh = nh, fo = no;
            if (it < 31) {
              const int f = ((it + 1) & 7) * 4 + ((it + 1) >> 3);
              nh = lds_frag(ah, f, lane);
              no = lds_frag(al, f, lane);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int sl = 0; sl < 2; ++sl) {
              acc[sl][rt] = mma(fh, sh[sl], acc[sl][rt]);
              acc[sl][rt] = mma(fh, slo[sl], acc[sl][rt]);
              acc[sl][rt] = mma(fo, sh[sl], acc[sl][rt]);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        }
#pragma unroll
        for (int sl = 0; sl < 2; ++sl)
#pragma unroll
          for (int i = 0; i < 8; ++i) R.S[sl][i] = acc[sl][i];
        __syncthreads();
      }
    }
    lds_barrier();
    lds_barrier();
    // chunk c's forms (precise: W S in hi + lo; tlo: T diag(beta) in hi + lo, also set for every
    // precise chunk), read from its buffer a step ahead: after the barrier that completes the buffer,
    // so the step starts without waiting on LDS
    bool precise_n = ntot > 0 && chunk_precise(sm.buf[0]), tlo_n = ntot > 0 && chunk_tlo(sm.buf[0]);
    for (int c = 0; c < ntot; ++c) {
      const SegBuf& B = sm.buf[c & 1];
      const bool precise = precise_n, tlo = tlo_n;
      if (kPass == 0 && c >= w0) {
        if (precise) chain_part1<true, true, true, true>(B, sm.ops, R, wc, lane);
        else if (tlo) chain_part1<true, true, false, true>(B, sm.ops, R, wc, lane);
        else chain_part1<true, true, false, false>(B, sm.ops, R, wc, lane);
      } else if (mode != kSegA) {
        if (precise) chain_part1<true, false, true, true>(B, sm.ops, R, wc, lane);
        else if (tlo) chain_part1<true, false, false, true>(B, sm.ops, R, wc, lane);
        else chain_part1<true, false, false, false>(B, sm.ops, R, wc, lane);
      } else {  // (no U)
        if (precise) chain_part1<false, false, true, false>(B, sm.ops, R, wc, lane);
        else chain_part1<false, false, false, false>(B, sm.ops, R, wc, lane);
      }
      lds_barrier();
      if (c + 1 < ntot) {  // chunk c + 1's buffer is complete at this barrier
        precise_n = chunk_precise(sm.buf[(c + 1) & 1]);
        tlo_n = chunk_tlo(sm.buf[(c + 1) & 1]);
      }
      chain_part2(B, R, lane);
      lds_barrier();
    }
    // the state after the segment
    if (mode == kSegOut) {
      if (final_state && idx == tab.nseg_of(nch_s) - 1) {
        const int r0 = state_row(rows, n_rows, s);
        if (r0 >= 0) {
          float* dst = final_state + ((int64_t)r0 * Hv + h) * D * D;
#pragma unroll
          for (int sl = 0; sl < 2; ++sl)
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
              for (int r = 0; r < 4; ++r) dst[(16 * i + 4 * g4 + r) * D + 32 * wc + 16 * sl + c16] = R.S[sl][i][r];
        }
      }
    } else if (mode == kSegB) {  // B_j in register order
      float* dst = tslot + D * D;
#pragma unroll
      for (int sl = 0; sl < 2; ++sl)
#pragma unroll
        for (int i = 0; i < 8; ++i) *reinterpret_cast<f32x4*>(dst + tr::b_at(wc, sl, i, lane)) = R.S[sl][i];
    } else {  // A_j row-major into LDS, which every wave has finished with, for the fragment pass below
      __syncthreads();
      float* At = reinterpret_cast<float*>(&sm);
#pragma unroll
      for (int sl = 0; sl < 2; ++sl)
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) At[(16 * i + 4 * g4 + r) * kALd + 32 * wc + 16 * sl + c16] = R.S[sl][i][r];
      __syncthreads();
    }
  }
  if (kPass == 1 && mode == kSegA) {  // A_j's bf16 hi + lo A fragments, 4 (fragment, lane) items a thread
    if (w < 4) {
      __syncthreads();
      __syncthreads();
    }
    const float* At = reinterpret_cast<const float*>(&sm);
    uint8_t* a8 = reinterpret_cast<uint8_t*>(tslot);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int item = t + sg::NT * u, f = item >> 6, ln = item & 63, rt = f >> 2, kb = f & 3;
      const float* row = At + (16 * rt + (ln & 15)) * kALd + 32 * kb + 4 * (ln >> 4);
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(row), x1 = *reinterpret_cast<const f32x4*>(row + 16);
      bf16x8 hi, lo;
      split_bf16(x0, x1, hi, lo);
      *reinterpret_cast<bf16x8*>(a8 + tr::A_HI + f * ws::FRAG + ln * 16) = hi;
      *reinterpret_cast<bf16x8*>(a8 + tr::A_LO + f * ws::FRAG + ln * 16) = lo;
    }
  }
}

// ============================================================================================
// Causal depthwise conv prefill + SiLU with decode-state capture.
// ============================================================================================
// One thread per (run of kConvRun consecutive packed tokens, kConvCh channels): it loads the input
// rows p0-K+1 .. p0+kConvRun-1 once with 8-byte reads and slides the K-tap window over them (rows
// before a token's sequence come from the sequence's history row [C, K], x_{-j} = history[K - j], or
// are zero), then writes kConvCh outputs per token with one 8-byte store.  A workgroup covers one
// token run and 1024 channels, so the sequence walk is uniform across it.  Numerics of F.conv1d on
// bf16: fp32 accumulation of the K products (+ bias), one bf16 rounding, SiLU, bf16.  The conv is
// VALU-bound at the device copy rate, so each input row is unpacked to fp32 once and slides through
// the window (4 channels a thread keep the window in registers at 4 waves per SIMD).  The decode conv
// state a sequence leaves (its last K inputs) is written afterwards by conv_state_capture_kernel, so
// the history may be the same slot rows the state goes to.
constexpr int kConvRun = 8;
constexpr int kConvCh = 4;
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int find_seq(const int32_t* cu, int nseq, int64_t p) {
  int lo = 0, hi = nseq - 1;  // last sequence whose start <= p (skips empty ones)
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= p) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// kConvCh channels of one token: bf16(bias + sum_r x_r w_r) in fp32 (F.conv1d's order), SiLU, bf16.
template <int K>
__device__ __forceinline__ void conv_out(const float (&f)[K][kConvCh], const float (&wf)[K][kConvCh],
                                         const float (&bv)[kConvCh], uint16_t* __restrict__ dst) {
  float cv[kConvCh];
#pragma unroll
  for (int e = 0; e < kConvCh; ++e) {
    float acc = bv[e];
#pragma unroll
    for (int r = 0; r < K; ++r) acc += f[r][e] * wf[r][e];
    cv[e] = rbf(acc);
  }
  uint16_t o[kConvCh];
  silu_bf16_n<kConvCh>(cv, o);
  *reinterpret_cast<u16x4*>(dst) = u16x4{o[0], o[1], o[2], o[3]};
}

// The work of one conv workgroup: token run item / nblk, channel block item % nblk.
template <int K>
__device__ __forceinline__ void conv_run(int64_t item, int nblk, const uint16_t* __restrict__ x, int64_t x_stride,
                                         const uint16_t* __restrict__ weight, const uint16_t* __restrict__ bias,
                                         const uint16_t* __restrict__ history, const int32_t* __restrict__ rows,
                                         int n_rows, uint16_t* __restrict__ out, int64_t total_tokens,
                                         const int32_t* __restrict__ cu, int nseq, int seq_len, int C) {
  const int cg = (int)(item % nblk) * blockDim.x + threadIdx.x;  // channel group
  const int64_t p0 = item / nblk * kConvRun;
  if (kConvCh * cg >= C) return;
  const int c0 = kConvCh * cg;
  const int nrun = total_tokens - p0 < kConvRun ? (int)(total_tokens - p0) : kConvRun;
  // rows p0-K+1 .. p0+nrun-1 (only those inside [0, total_tokens) are read)
  u16x4 xr[kConvRun + K - 1];
  const u16x4 zero = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < kConvRun + K - 1; ++i) {
    const int64_t tok = p0 - (K - 1) + i;
    xr[i] = (tok >= 0 && i < nrun + K - 1) ? *reinterpret_cast<const u16x4*>(x + tok * x_stride + c0) : zero;
  }
  float wf[K][kConvCh];  // weight[c0 + e][r] -> wf[r][e]
  {
    const u16x4* wp = reinterpret_cast<const u16x4*>(weight + (int64_t)c0 * K);  // kConvCh K contiguous values
    uint16_t w[kConvCh * K];
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const u16x4 v = wp[i];
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) w[kConvCh * i + e] = v[e];
    }
#pragma unroll
    for (int e = 0; e < kConvCh; ++e)
#pragma unroll
      for (int r = 0; r < K; ++r) wf[r][e] = bf2f(w[e * K + r]);
  }
  float bv[kConvCh];
#pragma unroll
  for (int e = 0; e < kConvCh; ++e) bv[e] = bias ? bf2f(bias[c0 + e]) : 0.f;
  // sequence of p0, then walk forward (uniform across the workgroup)
  int s = cu ? find_seq(cu, nseq, p0) : (int)(p0 / seq_len);
  int64_t s_lo = cu ? (int64_t)cu[s] : (int64_t)s * seq_len;
  int64_t s_hi = cu ? (int64_t)cu[s + 1] : s_lo + seq_len;
  if (nrun == kConvRun && p0 - (K - 1) >= s_lo && p0 + kConvRun <= s_hi) {
    // All tokens of the run in one sequence, at least K - 1 past its start (every run of a sequence
    // but its first one or two): every window row is an input row.
    float f[K][kConvCh];
#pragma unroll
    for (int r = 1; r < K; ++r)
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) f[r][e] = bf2f(xr[r - 1][e]);
#pragma unroll
    for (int i = 0; i < kConvRun; ++i) {
#pragma unroll
      for (int r = 0; r + 1 < K; ++r)
#pragma unroll
        for (int e = 0; e < kConvCh; ++e) f[r][e] = f[r + 1][e];
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) f[K - 1][e] = bf2f(xr[i + K - 1][e]);
      conv_out<K>(f, wf, bv, out + (p0 + i) * (int64_t)C + c0);
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < kConvRun; ++i) {
    if (i >= nrun) break;  // (uniform: the last run of the batch)
    const int64_t p = p0 + i;
    while (p >= s_hi) {  // next non-empty sequence
      ++s;
      s_lo = cu ? (int64_t)cu[s] : (int64_t)s * seq_len;
      s_hi = cu ? (int64_t)cu[s + 1] : s_lo + seq_len;
    }
    u16x4 win[K];
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
          for (int e = 0; e < kConvCh; ++e)
            win[r][e] = hrow >= 0 ? history[((int64_t)hrow * C + c0 + e) * K + (K - back)] : (uint16_t)0;
        }
      }
    }
    float f[K][kConvCh];
#pragma unroll
    for (int r = 0; r < K; ++r)
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) f[r][e] = bf2f(win[r][e]);
    conv_out<K>(f, wf, bv, out + p * (int64_t)C + c0);
  }
}
// Workgroup b covers item xcd_range_item(b).  The 8 XCDs take workgroups b % 8 in turn; the remap
// gives each XCD a contiguous range of items, so the K - 1 input rows a run shares with the
// previous run are read again from that XCD's L2.
template <int K>
__global__ __launch_bounds__(256) void conv_prefill_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                                           const uint16_t* __restrict__ weight,
                                                           const uint16_t* __restrict__ bias,
                                                           const uint16_t* __restrict__ history,
                                                           const int32_t* __restrict__ rows, int n_rows,
                                                           uint16_t* __restrict__ out, int64_t total_tokens,
                                                           const int32_t* __restrict__ cu, int nseq, int seq_len,
                                                           int C, int nblk) {
  conv_run<K>(xcd_range_item(blockIdx.x, gridDim.x), nblk, x, x_stride, weight, bias, history, rows, n_rows, out,
              total_tokens, cu, nseq, seq_len, C);
}

// The decode conv state each sequence leaves: its last K inputs, the front filled from its history
// row (or zeros) when the sequence is shorter than K -- an empty sequence keeps its history.  One
// thread per (sequence, channel) reads its old row entries before writing them, so `history` and
// `state` may be the same slot rows.
__device__ __forceinline__ void capture_one(int64_t i, const uint16_t* __restrict__ x, int64_t x_stride,
                                            const uint16_t* history, const int32_t* __restrict__ hist_rows,
                                            uint16_t* state, const int32_t* __restrict__ state_rows, int n_rows,
                                            const int32_t* __restrict__ cu, int nseq, int seq_len, int C, int K) {
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
__global__ void conv_state_capture_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                          const uint16_t* history, const int32_t* __restrict__ hist_rows,
                                          uint16_t* state, const int32_t* __restrict__ state_rows, int n_rows,
                                          const int32_t* __restrict__ cu, int nseq, int seq_len, int C, int K) {
  capture_one((int64_t)blockIdx.x * blockDim.x + threadIdx.x, x, x_stride, history, hist_rows, state, state_rows,
              n_rows, cu, nseq, seq_len, C, K);
}

// ============================================================================================
// Gating: beta = sigmoid(b) in bf16, g = -exp(A_log) * softplus(a + dt_bias) in fp32.
// ============================================================================================
__device__ __forceinline__ void gating_one(int64_t i, const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                           int64_t ab_stride, const float* __restrict__ A_log,
                                           const float* __restrict__ dt_bias, uint16_t* __restrict__ beta,
                                           float* __restrict__ g, int64_t rows, int Hv) {
  if (i >= rows * Hv) return;
  const int64_t r = i / Hv;
  const int h = (int)(i % Hv);
  beta[i] = sigmoid_bf16(bf2f(b[r * ab_stride + h]));
  g[i] = -expf(A_log[h]) * softplus_f(bf2f(a[r * ab_stride + h]) + dt_bias[h]);
}
__global__ void gating_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, int64_t ab_stride,
                              const float* __restrict__ A_log, const float* __restrict__ dt_bias,
                              uint16_t* __restrict__ beta, float* __restrict__ g, int64_t rows, int Hv) {
  gating_one((int64_t)blockIdx.x * blockDim.x + threadIdx.x, a, b, ab_stride, A_log, dt_bias, beta, g, rows, Hv);
}

// ============================================================================================
// The GDN prefill layer's first launch: the conv of every token run and, as further workgroups of
// the same grid, the chunked rule's segment table, the decode conv state capture (when the history
// rows are not the state rows) and the gating.  None reads what another writes, so one launch does
// the work of four (each of which costs a few microseconds of launch however little it computes).
// ============================================================================================
struct PrologueArgs {
  const uint16_t* x;  // conv: [tokens, C] input rows
  int64_t x_stride;
  const uint16_t* weight;
  const uint16_t* bias;
  const uint16_t* history;
  const int32_t* rows;
  int n_rows;
  uint16_t* conv_out;  // [tokens, C]
  int64_t total_tokens;
  const int32_t* cu;
  int nseq, seq_len, C, nblk;
  int64_t n_conv;      // conv workgroups (first in the grid)
  uint16_t* state;     // capture: [n_rows, C, K] state rows
  int64_t n_cap;       // capture workgroups (0: captured by a launch of its own)
  const uint16_t* a;   // gating
  const uint16_t* b;
  int64_t ab_stride;
  const float* A_log;
  const float* dt_bias;
  uint16_t* beta;
  float* g;
  int Hv;
  int64_t n_gate;
  const int32_t* chunk0;  // segment table (one workgroup, last in the grid)
  int L;
  int32_t* seg0;
  int32_t* order;
  int table;
};
// Grid order: the segment table, the capture and the gating first (so they run beside the conv
// instead of after it), padded to a multiple of 8 workgroups, then the conv.
__host__ __device__ __forceinline__ int64_t prologue_pre(const PrologueArgs& P) {
  return (P.table + P.n_cap + P.n_gate + 7) / 8 * 8;
}
template <int K>
__global__ __launch_bounds__(256) void layer_prologue_kernel(PrologueArgs P) {
  int64_t b = blockIdx.x;
  const int64_t pre = prologue_pre(P);
  if (b >= pre) {  // the conv workgroups' remap keeps their XCD (workgroup b runs on XCD b % 8, and pre % 8 == 0)
    b -= pre;
    conv_run<K>(xcd_range_item(b, P.n_conv), P.nblk, P.x, P.x_stride, P.weight, P.bias, P.history, P.rows, P.n_rows,
                P.conv_out, P.total_tokens, P.cu, P.nseq, P.seq_len, P.C);
    return;
  }
  if (b < P.table) {
    seg_table_wg(P.chunk0, P.nseq, P.L, P.seg0, P.order);
    return;
  }
  b -= P.table;
  if (b < P.n_cap) {
    capture_one(b * 256 + threadIdx.x, P.x, P.x_stride, P.history, P.rows, P.state, P.rows, P.n_rows, P.cu, P.nseq,
                P.seq_len, P.C, K);
    return;
  }
  b -= P.n_cap;
  if (b < P.n_gate)
    gating_one(b * 256 + threadIdx.x, P.a, P.b, P.ab_stride, P.A_log, P.dt_bias, P.beta, P.g, P.total_tokens, P.Hv);
}

// Workspace of gdn_chunk_prefill_noalloc: one static array per device (host code reaches it only
// through the address hipGetSymbolAddress returns on that device).
static __device__ __align__(256) uint8_t scratch[GDN_NOALLOC_SCRATCH_BYTES];

}  // namespace gdn

using namespace gdn;

// Device address of `scratch` for a call on `stream`: the stream must belong to the current device
// (the null stream does), and the address is looked up once per device, with that device current,
// by hipGetSymbolAddress (each GPU holds its own copy of the array).  0 and *out set, or an error code.
static int scratch_ptr(hipStream_t stream, uint8_t** out) {
  static std::atomic<uintptr_t> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return set_error(GDN_ELAUNCH, "gdn_chunk_prefill_noalloc: no current HIP device");
  if (stream) {
    hipDevice_t sd = dev;
    if (hipStreamGetDevice(stream, &sd) != hipSuccess)
      return set_error(GDN_EINVAL, "gdn_chunk_prefill_noalloc: cannot query the stream's device");
    if (sd != dev)
      return set_error(GDN_EINVAL,
                       "gdn_chunk_prefill_noalloc: the stream belongs to device %d but device %d is current "
                       "(the static scratch is per device: make the stream's device current)",
                       (int)sd, dev);
  }
  uintptr_t p = cached[dev].load(std::memory_order_acquire);
  if (!p) {
    void* a = nullptr;
    if (hipGetSymbolAddress(&a, HIP_SYMBOL(scratch)) != hipSuccess || !a)
      return set_error(GDN_ELAUNCH, "gdn_chunk_prefill_noalloc: no static scratch on device %d", dev);
    p = (uintptr_t)a;
    cached[dev].store(p, std::memory_order_release);
  }
  *out = (uint8_t*)p;
  return GDN_OK;
}

extern "C" int gdn_unit_lower_inv(const float* X, float* T, int64_t batch, int n, void* stream) {
  clear_error();
  GDN_REQUIRE(X && T, "gdn_unit_lower_inv: null pointer");
  GDN_SUPPORT(n == 64, "gdn_unit_lower_inv: only 64x64 blocks are supported (got %d)", n);
  GDN_REQUIRE(batch >= 0 && batch < (1ll << 31), "gdn_unit_lower_inv: bad batch %lld", (long long)batch);
  if (batch == 0) return GDN_OK;
  GDN_REQUIRE(aligned(X, 16) && aligned(T, 16), "gdn_unit_lower_inv: X and T must be 16-byte aligned");
  unit_lower_inv_kernel<<<(unsigned)((batch + 3) / 4), 256, 0, (hipStream_t)stream>>>(X, T, batch);
  return check_launch("gdn_unit_lower_inv");
}

namespace {
// Segment length (chunks) for a call: about sg::kTargetItems (segment, value head) items (one
// workgroup per compute unit), at least sg::kMinSeg chunks per segment.  When the (sequence, value
// head) pairs fit one round, each sequence gets m = kTargetItems / pairs segments of equal length:
// the items then fill one round without spilling into a second (at T = 8192 with 48 value heads:
// 5 segments of 26 chunks, 240 items; the work-based length, 24 chunks, gives 6 segments and 288
// items, and the 32 past 256 run as a second round).  Beyond one round, the work-based length.
int64_t seg_len(int64_t total_chunks, int nseq, int Hv) {
  const int64_t pairs = (int64_t)nseq * Hv;
  int64_t L;
  if (pairs > 0 && pairs <= sg::kTargetItems) {
    const int64_t parts = (int64_t)nseq * (sg::kTargetItems / pairs);
    L = (total_chunks + parts - 1) / parts;
  } else {
    L = (total_chunks * (int64_t)Hv + sg::kTargetItems - 1) / sg::kTargetItems;
  }
  return L < sg::kMinSeg ? sg::kMinSeg : L;
}
// Workspace layout: the segment table (nseq + 1 int32), the longest-first segment order (int32 per
// segment), the transition flags (int32 per (slot,
// value head)), the warm-up lengths (int32 per (slot, value head)), the transition slots (128 KiB per
// (slot, value head): A's bf16 hi + lo fragments, then B in fp32; layout in namespace tr), the
// inverse kernel's fragments (10 KiB per (chunk, value head): the bf16 hi half, then the lo half) and
// its records of 64 K l2norm factors, the chunk's 64 g values and the lo flag (528 B per (chunk, value
// head)), each part 256-byte aligned.
struct SegLayout {
  int64_t L, nslots, off_order, off_flags, off_warm, off_trans, off_tfrag, off_knorm, bytes;
};
SegLayout seg_layout(int64_t total_chunks, int nseq, int Hv) {
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  SegLayout l;
  l.L = seg_len(total_chunks, nseq, Hv);
  l.nslots = total_chunks / l.L;
  l.off_order = up(((int64_t)nseq + 1) * 4);
  l.off_flags = l.off_order + up(((int64_t)nseq + total_chunks / l.L) * 4);  // segments: <= nseq + chunks / L
  l.off_warm = l.off_flags + up(l.nslots * Hv * 4);
  l.off_trans = l.off_warm + up(l.nslots * Hv * 4);
  l.off_tfrag = l.off_trans + l.nslots * Hv * (int64_t)sg::kTrans * 4;
  l.off_knorm = l.off_tfrag + total_chunks * Hv * (int64_t)tf::BYTES;
  l.bytes = l.off_knorm + total_chunks * Hv * (int64_t)(kr::FLOATS * 4);
  return l;
}
}  // namespace

extern "C" int64_t gdn_chunk_prefill_workspace_bytes(int64_t total_chunks, int nseq, int Hv) {
  if (total_chunks < 0 || nseq < 0 || Hv <= 0) return -1;
  return seg_layout(total_chunks, nseq, Hv).bytes;
}

namespace {
// gdn_chunk_prefill_rows, and with norm_mode 1 / 2 (bf16 / fp32 norm weight) the fused gated norm.
int chunk_prefill_impl(const void* q, int64_t q_stride, const void* k, int64_t k_stride, const void* v,
                       int64_t v_stride, const float* g, const void* beta, int beta_dtype, const float* initial_state,
                       float* final_state, const int32_t* state_rows, int n_rows, void* out, int64_t total_tokens,
                       const int32_t* cu_seqlens, const int32_t* seq_chunk0, int64_t total_chunks, int nseq,
                       int seq_len, int Hqk, int Hv, int D, int in_dtype, int use_qk_l2norm, void* workspace,
                       int64_t workspace_bytes, void* stream, const GateArgs& gate, int norm_mode,
                       bool table_built = false, bool check_only = false) {
  GDN_REQUIRE(state_rows ? n_rows >= 0 : n_rows == nseq,
              "gdn_chunk_prefill: without state_rows, n_rows must equal nseq");
  GDN_REQUIRE(q && k && v && g && beta && out, "gdn_chunk_prefill: null input/output pointer");
  GDN_SUPPORT(D == pf::D, "gdn_chunk_prefill: head dim %d unsupported (needs %d)", D, pf::D);
  GDN_SUPPORT(in_dtype == GDN_BF16, "gdn_chunk_prefill: q/k/v must be bfloat16 (MFMA operands)");
  GDN_REQUIRE(beta_dtype == GDN_F32 || beta_dtype == GDN_BF16, "gdn_chunk_prefill: bad beta dtype");
  GDN_REQUIRE(Hqk > 0 && Hv > 0 && Hv % Hqk == 0, "gdn_chunk_prefill: bad heads Hqk=%d Hv=%d", Hqk, Hv);
  GDN_REQUIRE(nseq >= 0 && total_tokens >= 0 && total_chunks >= 0 && seq_len >= 0, "gdn_chunk_prefill: negative sizes");
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
  // the segment kernel addresses a chunk's q, k and v rows with 32-bit byte offsets: 63 strides plus a
  // row must stay below 2^32 bytes
  GDN_REQUIRE(q_stride > 0 && q_stride < (1ll << 25) && k_stride > 0 && k_stride < (1ll << 25) && v_stride > 0 &&
                  v_stride < (1ll << 25),
              "gdn_chunk_prefill: q/k/v token strides out of range");
  GDN_REQUIRE(workspace && aligned(workspace, 256) &&
                  workspace_bytes >= gdn_chunk_prefill_workspace_bytes(total_chunks, nseq, Hv),
              "gdn_chunk_prefill: workspace missing, misaligned or smaller than %lld bytes",
              (long long)gdn_chunk_prefill_workspace_bytes(total_chunks, nseq, Hv));
  GDN_REQUIRE(total_chunks < (1ll << 31), "gdn_chunk_prefill: too many chunks");
  const SegLayout lay = seg_layout(total_chunks, nseq, Hv);
  {
    const int64_t nseg_max = (int64_t)nseq + total_chunks / lay.L;  // each sequence: <= nch / L + 1 segments
    GDN_REQUIRE(nseg_max * Hv < (1ll << 31) && lay.nslots * Hv * 2 < (1ll << 31) &&
                    (int64_t)nseq * Hv * 64 < (1ll << 31) && total_chunks * Hv < (1ll << 33),
                "gdn_chunk_prefill: grid too large");
  }
  if (check_only || nseq == 0) return GDN_OK;
  hipStream_t st = (hipStream_t)stream;
  uint8_t* work = (uint8_t*)workspace;
  int32_t* seg0 = (int32_t*)work;
  int32_t* order = (int32_t*)(work + lay.off_order);
  int* tflags = (int*)(work + lay.off_flags);
  int* warm = (int*)(work + lay.off_warm);
  float* trans = (float*)(work + lay.off_trans);
  uint8_t* tfrag = work + lay.off_tfrag;
  float* knorm = (float*)(work + lay.off_knorm);
  const int64_t nseg_max = (int64_t)nseq + total_chunks / lay.L;
  if (cu_seqlens && !table_built) {
    seg_table_kernel<<<1, 256, 0, st>>>(seq_chunk0, nseq, (int)lay.L, seg0, order);
    int rc = check_launch("gdn_chunk_prefill(table)");
    if (rc) return rc;
  }
  const SegTable tab{cu_seqlens, seq_chunk0, cu_seqlens ? seg0 : nullptr, cu_seqlens ? order : nullptr, nseq, seq_len,
                     (int)lay.L};
  if (total_chunks > 0) {  // the intra-chunk inverses, one wave per (chunk, value head)
    const int64_t items = total_chunks * Hv;
    const unsigned gi = (unsigned)((items + 3) / 4);
    if (beta_dtype == GDN_BF16)
      inv_kernel<uint16_t><<<gi, pf::NT, 0, st>>>((const uint16_t*)k, k_stride, g,
                                                  (const uint16_t*)beta, cu_seqlens, seq_chunk0, nseq, seq_len, items,
                                                  Hqk, Hv, use_qk_l2norm, tfrag, knorm, tab, warm);
    else
      inv_kernel<float><<<gi, pf::NT, 0, st>>>((const uint16_t*)k, k_stride, g,
                                               (const float*)beta, cu_seqlens, seq_chunk0, nseq, seq_len, items, Hqk,
                                               Hv, use_qk_l2norm, tfrag, knorm, tab, warm);
    int rc = check_launch("gdn_chunk_prefill(inverse)");
    if (rc) return rc;
  }
  auto launch = [&](int pass, int64_t blocks) {
#define GDN_SEG_LAUNCH(BT)                                                                                           \
  (pass == 1 ? seg_kernel<BT, uint16_t, 1>                                                                          \
             : norm_mode == 1 ? seg_kernel<BT, uint16_t, 0, 1>                                                      \
                              : norm_mode == 2 ? seg_kernel<BT, uint16_t, 0, 2> : seg_kernel<BT, uint16_t, 0>)      \
      <<<(unsigned)blocks, sg::NT, 0, st>>>((const uint16_t*)q, q_stride, (const uint16_t*)k, k_stride,              \
                                            (const uint16_t*)v, v_stride, g, (const BT*)beta, (uint16_t*)out, tab, Hqk, \
                                            Hv, use_qk_l2norm, initial_state, state_rows, n_rows, final_state, trans,  \
                                            tflags, tfrag, knorm, warm, gate)
    if (beta_dtype == GDN_BF16) GDN_SEG_LAUNCH(uint16_t);
    else GDN_SEG_LAUNCH(float);
#undef GDN_SEG_LAUNCH
  };
  // A sequence spans several segments only beyond L chunks: seq_len is the uniform length, or for
  // packed sequences an upper bound of the longest one (0: unknown)
  const int64_t max_seq_chunks = seq_len > 0 ? ((int64_t)seq_len + pf::CH - 1) / pf::CH : total_chunks;
  if (lay.nslots > 0 && max_seq_chunks > lay.L) {  // segment summaries and their combination where no warm-up fits
    launch(1, lay.nslots * Hv * 2);
    int rc = check_launch("gdn_chunk_prefill(summary)");
    if (rc) return rc;
  }
  launch(0, nseg_max * Hv);
  return check_launch("gdn_chunk_prefill(output)");
}
}  // namespace

// The inverse kernel's records of (chunk, value head) `item`, dense: T diag(beta) as the output pass
// reads it, [64, 64] fp32 (row = token of the chunk; the bf16 values of the fragments, zeros where
// no fragment holds a value), and the K rows' l2norm factors [64].  Fragment f = tf::fid(w', s),
// element e of lane (i, g): row 16 w' + i, column 32 s + 16 (e >> 2) + 4 g + (e & 3); the two half
// fragments keep e < 4 only.  Lane l writes row l.  One wave per item.
__global__ __launch_bounds__(256) void inv_records_expand_kernel(const uint8_t* __restrict__ tfrag,
                                                                 const float* __restrict__ knorm, int64_t items,
                                                                 float* __restrict__ t_out,
                                                                 float* __restrict__ factor_out) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t item = (int64_t)blockIdx.x * 4 + w;
  if (item >= items) return;
  const uint8_t* rec = tfrag + item * tf::BYTES;
  const int wt = lane >> 4, i = lane & 15;
  float* row = t_out + item * 4096 + lane * 64;
  for (int j = 0; j < 64; ++j) {
    const int s = j >> 5, jj = j & 31, e = 4 * (jj >> 4) + (jj & 3), gg = (jj & 15) >> 2;
    float x = 0.f;
    if (2 * s <= wt) {
      const int f = tf::fid(wt, s), l = i + 16 * gg;
      if (!tf::half(f)) x = bf2f(reinterpret_cast<const uint16_t*>(rec + tf::offset(f) + l * 16)[e]);
      else if (e < 4) x = bf2f(reinterpret_cast<const uint16_t*>(rec + tf::offset(f) + l * 8)[e]);
    }
    row[j] = x;
  }
  if (factor_out) factor_out[item * 64 + lane] = knorm[item * kr::FLOATS + lane];
}

extern "C" int gdn_chunk_prefill_rows(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                                      const void* v, int64_t v_stride, const float* g, const void* beta,
                                      int beta_dtype, const float* initial_state, float* final_state,
                                      const int32_t* state_rows, int n_rows, void* out, int64_t total_tokens,
                                      const int32_t* cu_seqlens, const int32_t* seq_chunk0, int64_t total_chunks,
                                      int nseq, int seq_len, int Hqk, int Hv, int D, int in_dtype,
                                      int use_qk_l2norm, void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  if (D != pf::D || in_dtype != GDN_BF16)  // other head dims and dtypes: the generic fp32 kernel
    return gdn_chunk_prefill_generic(q, q_stride, k, k_stride, v, v_stride, g, beta, beta_dtype, initial_state,
                                     final_state, state_rows, n_rows, out, total_tokens, cu_seqlens, nseq, seq_len,
                                     Hqk, Hv, D, D, in_dtype, use_qk_l2norm, stream);
  return chunk_prefill_impl(q, q_stride, k, k_stride, v, v_stride, g, beta, beta_dtype, initial_state, final_state,
                            state_rows, n_rows, out, total_tokens, cu_seqlens, seq_chunk0, total_chunks, nseq, seq_len,
                            Hqk, Hv, D, in_dtype, use_qk_l2norm, workspace, workspace_bytes, stream, GateArgs{}, 0);
}

extern "C" int gdn_chunk_prefill_rows_gated(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                                            const void* v, int64_t v_stride, const float* g, const void* beta,
                                            int beta_dtype, const float* initial_state, float* final_state,
                                            const int32_t* state_rows, int n_rows, void* out, int64_t total_tokens,
                                            const int32_t* cu_seqlens, const int32_t* seq_chunk0,
                                            int64_t total_chunks, int nseq, int seq_len, int Hqk, int Hv, int D,
                                            int in_dtype, int use_qk_l2norm, const void* z, int64_t z_stride,
                                            const void* norm_weight, int norm_w_dtype, float eps, void* workspace,
                                            int64_t workspace_bytes, void* stream) {
  clear_error();
  GDN_REQUIRE(z && norm_weight, "gdn_chunk_prefill_rows_gated: null gate or norm weight");
  GDN_REQUIRE(norm_w_dtype == GDN_BF16 || norm_w_dtype == GDN_F32, "gdn_chunk_prefill_rows_gated: bad norm weight dtype");
  GDN_REQUIRE(aligned(z, 16) && z_stride % 8 == 0 && z_stride >= (int64_t)Hv * D,
              "gdn_chunk_prefill_rows_gated: gate rows must be 16-byte aligned and hold Hv * D values");
  const GateArgs gate{(const uint16_t*)z, z_stride, norm_weight, eps};
  return chunk_prefill_impl(q, q_stride, k, k_stride, v, v_stride, g, beta, beta_dtype, initial_state, final_state,
                            state_rows, n_rows, out, total_tokens, cu_seqlens, seq_chunk0, total_chunks, nseq, seq_len,
                            Hqk, Hv, D, in_dtype, use_qk_l2norm, workspace, workspace_bytes, stream, gate,
                            norm_w_dtype == GDN_BF16 ? 1 : 2);
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
  GDN_REQUIRE(total_chunks >= 0 && Hqk > 0 && Hv > 0, "gdn_chunk_prefill_noalloc: bad sizes");
  GDN_REQUIRE(nseq >= 0, "gdn_chunk_prefill_noalloc: bad sizes");
  const int64_t need = gdn_chunk_prefill_workspace_bytes(total_chunks, nseq, Hv);
  GDN_REQUIRE(need <= GDN_NOALLOC_SCRATCH_BYTES,
              "gdn_chunk_prefill_noalloc: the call needs %lld bytes of workspace, the static scratch holds %lld "
              "(%lld chunks, %d sequences, %d value heads; use gdn_chunk_prefill_rows with a workspace)",
              (long long)need, (long long)GDN_NOALLOC_SCRATCH_BYTES, (long long)total_chunks, nseq, Hv);
  uint8_t* ws_ptr = nullptr;
  {
    const int rc = scratch_ptr((hipStream_t)stream, &ws_ptr);
    if (rc) return rc;
  }
  return gdn_chunk_prefill_rows(q, q_stride, k, k_stride, v, v_stride, g, beta, beta_dtype, initial_state,
                                final_state, state_rows, n_rows, out, total_tokens, cu_seqlens, seq_chunk0,
                                total_chunks, nseq, seq_len, Hqk, Hv, D, in_dtype, use_qk_l2norm, ws_ptr,
                                GDN_NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" int gdn_chunk_prefill_inverse(const void* k, int64_t k_stride, const float* g, const void* beta,
                                         int beta_dtype, int64_t total_tokens, const int32_t* cu_seqlens,
                                         const int32_t* seq_chunk0, int64_t total_chunks, int nseq, int seq_len,
                                         int Hqk, int Hv, int D, int in_dtype, int use_qk_l2norm, float* t_out,
                                         float* factor_out, void* workspace, int64_t workspace_bytes,
                                         void* stream) {
  clear_error();
  GDN_REQUIRE(k && g && beta && t_out, "gdn_chunk_prefill_inverse: null pointer");
  GDN_SUPPORT(D == pf::D && in_dtype == GDN_BF16, "gdn_chunk_prefill_inverse: needs bf16 keys with D = %d", pf::D);
  GDN_REQUIRE(beta_dtype == GDN_F32 || beta_dtype == GDN_BF16, "gdn_chunk_prefill_inverse: bad beta dtype");
  GDN_REQUIRE(Hqk > 0 && Hv > 0 && Hv % Hqk == 0 && nseq >= 0 && total_tokens >= 0 && total_chunks >= 0 &&
                  seq_len >= 0,
              "gdn_chunk_prefill_inverse: bad sizes");
  GDN_REQUIRE(cu_seqlens ? seq_chunk0 != nullptr : (int64_t)nseq * seq_len == total_tokens,
              "gdn_chunk_prefill_inverse: cu_seqlens needs seq_chunk0; without it nseq*seq_len must be total_tokens");
  GDN_REQUIRE(cu_seqlens || total_chunks == (int64_t)nseq * ((seq_len + pf::CH - 1) / pf::CH),
              "gdn_chunk_prefill_inverse: total_chunks inconsistent with nseq/seq_len");
  GDN_REQUIRE(aligned(k, 16) && k_stride % 8 == 0 && k_stride > 0 && k_stride < (1ll << 25),
              "gdn_chunk_prefill_inverse: k rows must be 16-byte aligned");
  GDN_REQUIRE(workspace && aligned(workspace, 256) &&
                  workspace_bytes >= gdn_chunk_prefill_workspace_bytes(total_chunks, nseq, Hv),
              "gdn_chunk_prefill_inverse: workspace missing, misaligned or too small");
  GDN_REQUIRE(total_chunks * Hv < (1ll << 33), "gdn_chunk_prefill_inverse: grid too large");
  if (nseq == 0 || total_chunks == 0) return GDN_OK;
  hipStream_t st = (hipStream_t)stream;
  const SegLayout lay = seg_layout(total_chunks, nseq, Hv);
  uint8_t* work = (uint8_t*)workspace;
  int32_t* seg0 = (int32_t*)work;
  if (cu_seqlens) {
    seg_table_kernel<<<1, 256, 0, st>>>(seq_chunk0, nseq, (int)lay.L, seg0, (int32_t*)(work + lay.off_order));
    const int rc = check_launch("gdn_chunk_prefill_inverse(table)");
    if (rc) return rc;
  }
  const SegTable tab{cu_seqlens, seq_chunk0, cu_seqlens ? seg0 : nullptr, nullptr, nseq, seq_len, (int)lay.L};
  uint8_t* tfrag = work + lay.off_tfrag;
  float* knorm = (float*)(work + lay.off_knorm);
  int* warm = (int*)(work + lay.off_warm);
  const int64_t items = total_chunks * Hv;
  const unsigned gi = (unsigned)((items + 3) / 4);
  if (beta_dtype == GDN_BF16)
    inv_kernel<uint16_t><<<gi, pf::NT, 0, st>>>((const uint16_t*)k, k_stride, g, (const uint16_t*)beta, cu_seqlens,
                                                seq_chunk0, nseq, seq_len, items, Hqk, Hv, use_qk_l2norm, tfrag,
                                                knorm, tab, warm);
  else
    inv_kernel<float><<<gi, pf::NT, 0, st>>>((const uint16_t*)k, k_stride, g, (const float*)beta, cu_seqlens,
                                             seq_chunk0, nseq, seq_len, items, Hqk, Hv, use_qk_l2norm, tfrag, knorm,
                                             tab, warm);
  int rc = check_launch("gdn_chunk_prefill_inverse(inverse)");
  if (rc) return rc;
  inv_records_expand_kernel<<<gi, 256, 0, st>>>(tfrag, knorm, items, t_out, use_qk_l2norm ? factor_out : nullptr);
  return check_launch("gdn_chunk_prefill_inverse(expand)");
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
    const int nblk = (C / kConvCh + 255) / 256;
    const int64_t nwg = (int64_t)nblk * ((total_tokens + kConvRun - 1) / kConvRun);
    GDN_REQUIRE(nwg < (1ll << 31), "gdn_conv_prefill: grid too large");
    const unsigned grid = (unsigned)nwg;
#define GDN_CONV_PREFILL(KK)                                                                                    \
  case KK:                                                                                                     \
    conv_prefill_kernel<KK><<<grid, 256, 0, s>>>((const uint16_t*)x, x_stride, (const uint16_t*)weight,          \
                                                 (const uint16_t*)bias, (const uint16_t*)history, state_rows,      \
                                                 n_rows, (uint16_t*)out, total_tokens, cu_seqlens, nseq, seq_len, \
                                                 C, nblk);                                                     \
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

namespace {
// Byte offsets of the layer workspace: the conv output [tokens, C] bf16, beta [tokens, Hv] bf16,
// g [tokens, Hv] fp32, then the chunked rule's workspace.
struct LayerLayout {
  int64_t off_beta, off_g, off_chunk, bytes;
};
LayerLayout layer_layout(int64_t total_tokens, int64_t total_chunks, int nseq, int Hk, int Hv, int D) {
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int64_t C = (int64_t)(2 * Hk + Hv) * D;
  LayerLayout l;
  l.off_beta = up(total_tokens * C * 2);
  l.off_g = l.off_beta + up(total_tokens * Hv * 2);
  l.off_chunk = l.off_g + up(total_tokens * Hv * 4);
  l.bytes = l.off_chunk + gdn_chunk_prefill_workspace_bytes(total_chunks, nseq, Hv);
  return l;
}
}  // namespace

extern "C" int64_t gdn_prefill_layer_workspace_bytes(int64_t total_tokens, int64_t total_chunks, int nseq, int Hk,
                                                     int Hv, int D) {
  if (total_tokens < 0 || total_chunks < 0 || nseq < 0 || Hk <= 0 || Hv <= 0 || D <= 0) return -1;
  return layer_layout(total_tokens, total_chunks, nseq, Hk, Hv, D).bytes;
}

extern "C" int gdn_prefill_layer_rows(const void* mixed, int64_t mixed_stride, const void* z, int64_t z_stride,
                                      const void* a, const void* b, int64_t ab_stride, const void* conv_w,
                                      const void* conv_b, const float* A_log, const float* dt_bias,
                                      const void* norm_w, int norm_w_dtype, float eps, const void* conv_history,
                                      void* conv_state, const float* initial_state, float* final_state,
                                      const int32_t* state_rows, int n_rows, void* out, int64_t total_tokens,
                                      const int32_t* cu_seqlens, const int32_t* seq_chunk0, int64_t total_chunks,
                                      int nseq, int seq_len, int Hk, int Hv, int D, int K, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  clear_error();
  GDN_REQUIRE(mixed && z && a && b && conv_w && A_log && dt_bias && norm_w && conv_state && out,
              "gdn_prefill_layer: null pointer");
  GDN_REQUIRE(Hk > 0 && Hv > 0 && Hv % Hk == 0 && nseq >= 0 && total_tokens >= 0 && total_chunks >= 0,
              "gdn_prefill_layer: bad sizes");
  GDN_SUPPORT(D == pf::D, "gdn_prefill_layer: head dim %d unsupported (needs %d)", D, pf::D);
  GDN_SUPPORT(K >= 1 && K <= 8, "gdn_prefill_layer: conv kernel size %d unsupported", K);
  GDN_REQUIRE(norm_w_dtype == GDN_BF16 || norm_w_dtype == GDN_F32, "gdn_prefill_layer: bad norm weight dtype");
  GDN_REQUIRE(state_rows ? n_rows >= 0 : n_rows == nseq,
              "gdn_prefill_layer: without state_rows, n_rows must equal nseq");
  GDN_REQUIRE(cu_seqlens || (int64_t)nseq * seq_len == total_tokens,
              "gdn_prefill_layer: nseq*seq_len != total_tokens without cu_seqlens");
  const int C = (2 * Hk + Hv) * D;
  GDN_REQUIRE(mixed_stride >= C && mixed_stride % 8 == 0 && aligned(mixed, 16) && aligned(conv_w, 16),
              "gdn_prefill_layer: mixed rows and the conv weight must be 16-byte aligned");
  GDN_REQUIRE(aligned(z, 16) && z_stride % 8 == 0 && z_stride >= (int64_t)Hv * D,
              "gdn_prefill_layer: gate rows must be 16-byte aligned and hold Hv * D values");
  GDN_REQUIRE(total_tokens < (1ll << 31), "gdn_prefill_layer: too many tokens");
  const LayerLayout lay = layer_layout(total_tokens, total_chunks, nseq, Hk, Hv, D);
  GDN_REQUIRE(workspace && aligned(workspace, 256) && workspace_bytes >= lay.bytes,
              "gdn_prefill_layer: workspace missing, misaligned or smaller than %lld bytes", (long long)lay.bytes);
  uint8_t* work = (uint8_t*)workspace;
  uint16_t* conv_out = (uint16_t*)work;
  const GateArgs gate{(const uint16_t*)z, z_stride, norm_w, eps};
  const int64_t kd = (int64_t)Hk * D;
  auto rule = [&](bool check_only) {  // the chunked rule on the prologue's outputs
    return chunk_prefill_impl(conv_out, C, conv_out + kd, C, conv_out + 2 * kd, C, (float*)(work + lay.off_g),
                              work + lay.off_beta, GDN_BF16, initial_state, final_state, state_rows, n_rows, out,
                              total_tokens, cu_seqlens, seq_chunk0, total_chunks, nseq, seq_len, Hk, Hv, D, GDN_BF16,
                              1, work + lay.off_chunk, workspace_bytes - lay.off_chunk, stream, gate,
                              norm_w_dtype == GDN_BF16 ? 1 : 2, cu_seqlens != nullptr, check_only);
  };
  // every check of the chunked rule runs before the first launch: a refusal leaves the conv state
  // and the slot rows untouched
  {
    const int rc = rule(true);
    if (rc) return rc;
  }
  if (nseq == 0) return GDN_OK;
  hipStream_t st = (hipStream_t)stream;
  uint16_t* beta = (uint16_t*)(work + lay.off_beta);
  float* g = (float*)(work + lay.off_g);
  uint8_t* chunk_ws = work + lay.off_chunk;
  // one launch for the conv, the gating, the segment table and (when the history rows are not the
  // state rows) the conv state capture
  const bool cap_fused = !conv_history || conv_history != conv_state;
  const SegLayout seg = seg_layout(total_chunks, nseq, Hv);
  PrologueArgs P{};
  P.x = (const uint16_t*)mixed;
  P.x_stride = mixed_stride;
  P.weight = (const uint16_t*)conv_w;
  P.bias = (const uint16_t*)conv_b;
  P.history = (const uint16_t*)conv_history;
  P.rows = state_rows;
  P.n_rows = n_rows;
  P.conv_out = conv_out;
  P.total_tokens = total_tokens;
  P.cu = cu_seqlens;
  P.nseq = nseq;
  P.seq_len = seq_len;
  P.C = C;
  P.nblk = (C / kConvCh + 255) / 256;
  P.n_conv = (int64_t)P.nblk * ((total_tokens + kConvRun - 1) / kConvRun);
  P.state = (uint16_t*)conv_state;
  P.n_cap = cap_fused ? ((int64_t)nseq * C + 255) / 256 : 0;
  P.a = (const uint16_t*)a;
  P.b = (const uint16_t*)b;
  P.ab_stride = ab_stride;
  P.A_log = A_log;
  P.dt_bias = dt_bias;
  P.beta = beta;
  P.g = g;
  P.Hv = Hv;
  P.n_gate = (total_tokens * Hv + 255) / 256;
  P.chunk0 = seq_chunk0;
  P.L = (int)seg.L;
  P.seg0 = (int32_t*)chunk_ws;
  P.order = (int32_t*)(chunk_ws + seg.off_order);
  P.table = cu_seqlens ? 1 : 0;
  const int64_t grid = prologue_pre(P) + P.n_conv;
  GDN_REQUIRE(grid < (1ll << 31), "gdn_prefill_layer: grid too large");
  if (grid > 0) {
#define GDN_PROLOGUE(KK) \
  case KK:               \
    layer_prologue_kernel<KK><<<(unsigned)grid, 256, 0, st>>>(P); \
    break;
    switch (K) {
      GDN_PROLOGUE(1)
      GDN_PROLOGUE(2)
      GDN_PROLOGUE(3)
      GDN_PROLOGUE(4)
      GDN_PROLOGUE(5)
      GDN_PROLOGUE(6)
      GDN_PROLOGUE(7)
      GDN_PROLOGUE(8)
    }
#undef GDN_PROLOGUE
    int rc = check_launch("gdn_prefill_layer(prologue)");
    if (rc) return rc;
  }
  if (!cap_fused) {  // the history rows are the state rows: the capture reads them after the conv has
    const int64_t n = (int64_t)nseq * C;
    conv_state_capture_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(
        (const uint16_t*)mixed, mixed_stride, (const uint16_t*)conv_history, state_rows, (uint16_t*)conv_state,
        state_rows, n_rows, cu_seqlens, nseq, seq_len, C, K);
    int rc = check_launch("gdn_prefill_layer(state)");
    if (rc) return rc;
  }
  return rule(false);
}
