// Per-head flush core shared by liblq's kernels: the end-of-window flush of one (slot, head) on the matrix cores, in
// an eight-wave (flush_head) and a four-wave (flush_head4) layout, with the helpers the standalone quantize, dequant
// and low-rank kernels also use.  Semantics: /root/reference/leapquant/kernels.py:1077-2033 (flush).
//
// The head's 128 x 128 matrix lives in registers in the accumulator layout of v_mfma_f32_16x16x32_bf16: wave w owns
// key channels c in [16w, 16w + 16), lane l holds
//     acc[nt][i] = M[c][v],   c = 16 w + 4 (l >> 4) + i,   v = 16 nt + (l & 15).
// The window rebuild (a rank-L GEMM, ~29 flop/byte at L = 64) runs on MFMA with bf16 hi/lo operands exactly where the
// reference splits.  The flush's rebuilt matrix B is fp16-exact, so every 128-long contraction of the subspace step
// (P = B^T Q, Q = B P, the R x R Gram corrections, the rank-R residual updates) is an fp16 MFMA with fp32 accumulation
// over operands held in registers: the packed tile itself is the B operand of v_mfma_f32_16x16x16_f16 (k = c), and one
// MFMA against the identity gives the transposed packing (k = v).
#pragma once
#include "lq_common.h"

namespace {
namespace lqf {


constexpr int KD = 128, VD = 128;
constexpr int LPMAX = 64;            // largest window
constexpr int OPS = LPMAX + 8;       // operand row stride (bf16): 144 B rows
constexpr int FT = 512;              // threads per workgroup
constexpr int NW = FT / 64;          // waves

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// D = A B + C over 16 x 16 blocks.  16x16x16: lane l holds A[l & 15][4 (l >> 4) + i] and B[4 (l >> 4) + i][l & 15];
// 16x16x32: the same with 8 (l >> 4) + i; D (both): lane l holds D[4 (l >> 4) + i][l & 15], i < 4.
__device__ __forceinline__ f32x4 mma16(f16x4 a, f16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f16x4 to_h4(f32x4 x) {
  return f16x4{(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
}
__device__ __forceinline__ f32x4 from_h4(f16x4 x) { return f32x4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]}; }
// Mixed-precision VALU forms (v_fma_mix_f32: an fp16 half of a packed word widened exactly, one fp32 rounding).
// hmul<H>(x, s) = fp32(half H of x) * s, rounded once: the product of cvt + mul (a zero result may be +0 where the
// two-instruction form gives -0).  habs_add<H>(x, acc) = acc + |fp32(half H of x)|, rounded once, as cvt + add.
// The compiler forms neither by itself (it widens with v_cvt_f32_f16 first), so each is one instruction here.
template <int H>
__device__ __forceinline__ float hmul(uint32_t x, float s) {
  float r;
  if constexpr (H == 0) asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(x), "v"(s));
  else asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(x), "v"(s));
  return r;
}
template <int H>
__device__ __forceinline__ float habs_add(uint32_t x, float acc) {
  float r;
  if constexpr (H == 0) asm("v_fma_mix_f32 %0, |%1|, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(x), "v"(acc));
  else asm("v_fma_mix_f32 %0, |%1|, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(x), "v"(acc));
  return r;
}
// the two 32-bit words of a packed f16x4 (halves 0, 1 and 2, 3)
__device__ __forceinline__ uint2 h4_words(f16x4 x) { return __builtin_bit_cast(uint2, x); }
// element i of a packed f16x4 times s (one rounding), and acc + |element i|
template <int I>
__device__ __forceinline__ float h4mul(f16x4 x, float s) {
  const uint2 w = h4_words(x);
  return hmul<I & 1>(I < 2 ? w.x : w.y, s);
}
template <int I>
__device__ __forceinline__ float h4abs_add(f16x4 x, float acc) {
  const uint2 w = h4_words(x);
  return habs_add<I & 1>(I < 2 ? w.x : w.y, acc);
}
// exchanges of 32-bit values between lane groups: swap32 trades the upper 32 lanes of a with the lower 32 of b,
// swap16 the odd 16-lane rows of a with the even rows of b (gfx950 v_permlane32_swap / v_permlane16_swap).  The
// sequence swap32(a0, a2), swap32(a1, a3), swap16(a0, a1), swap16(a2, a3) transposes four registers over the four
// 16-lane groups: register j of group q goes to register q of group j.
__device__ __forceinline__ void swap32(uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  a = r[0];
  b = r[1];
}
__device__ __forceinline__ void swap16(uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
  a = r[0];
  b = r[1];
}
// s[r] summed over the four 16-lane groups as xor32_sum(xor16_sum(s[r])) sums it, ((group 0 + group 1) + (group 2 +
// group 3)), as a reduce-scatter: lane group q returns the total of s[q] (three exchanges and three adds where the four
// all-reductions take eight exchanges, eight copies and eight adds; the same sums, so the same bits)
__device__ __forceinline__ float sum4_scatter(const f32x4& s) {
  uint32_t a0 = __float_as_uint(s[0]), b0 = __float_as_uint(s[1]), a1 = __float_as_uint(s[2]), b1 = __float_as_uint(s[3]);
  swap16(a0, b0);
  swap16(a1, b1);
  uint32_t x = __float_as_uint(__uint_as_float(a0) + __uint_as_float(b0));   // rows: s0, s1, s0, s1 over groups 0+1 / 2+3
  uint32_t y = __float_as_uint(__uint_as_float(a1) + __uint_as_float(b1));   // rows: s2, s3, s2, s3
  swap32(x, y);
  return __uint_as_float(x) + __uint_as_float(y);     // rows: s0, s1, s2, s3 over all four groups
}
// Row maxima over a wave's four lane groups (lane (q, l16) holds m[nt] for row 16 nt + l16 over its own channels): a
// reduce-scatter, two swap32 rounds pairing groups q, q + 2, then a swap16 round pairing q, q + 1, after which group q
// holds the wave's maxima of rows 16 (2 q) + l16 in x[0] and 16 (2 q + 1) + l16 in x[1] (12 instructions where eight
// all-reductions take 48; maxima are exact, so the same values)
__device__ __forceinline__ void rowmax_scatter(const float m[8], float x[2]) {
  float n[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {                       // rows 0-1 of n[k]: row k; rows 2-3: row k + 4
    uint32_t a = __float_as_uint(m[k]), b = __float_as_uint(m[k + 4]);
    swap32(a, b);
    n[k] = fmaxf(__uint_as_float(a), __uint_as_float(b));
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {                       // group q of x[k]: row 2 q + k
    uint32_t a = __float_as_uint(n[k]), b = __float_as_uint(n[k + 2]);
    swap16(a, b);
    x[k] = fmaxf(__uint_as_float(a), __uint_as_float(b));
  }
}
// The packed fp16 value as the compiler must keep it: without this it may keep the fp32 source alive instead and
// redo the conversion where the value is used (twice the registers).
__device__ __forceinline__ f16x4 pinned(f16x4 x) {
  asm volatile("" : "+v"(x));
  return x;
}

struct Tile {
  f32x4 a[8];
};

// RA = factor columns held (4: R <= 4; 8: the R = 8 GDN flush, kernels.py:1091, 1123), as NB = RA / 4 blocks of four
template <int RA = 4>
struct FlushShared {
  static constexpr int NB = RA / 4;
  union {
    bf16_t op[3][KD][OPS];     // rebuild operands [c or v][j]
    struct {                   // after the rebuild
      f32x4 qpart[NW][NB][VD]; // per-wave partial Q rows
      float rmx[4 * NW][VD];   // per-(wave, lane group) row maxima of the scaled residual
      float rq[VD];            // qmax / row scale
      f16_t ppT[RA][KD];       // P16^T
      f16x4 qo16[NB][VD];      // old Q rows [v][a], fp16 (residual B operand)
      f16x4 qn16[NB][VD];      // Q16 rows [v][r] (residual B operand)
    } r;
  };
  float skl[KD];               // column factor of the dequant (Sk, KDA: Sk pc)
  float svr[VD];               // row factor of the dequant (Sv pn / qmax, KDA: Sv / qmax)
  float w[LPMAX];
  f32x4 uoc[NB][KD];           // old U rows [c][a] (KDA: fp16(U pc)), a >= R zero
  f32x4 qov[NB][VD];           // old Q rows [v][a], a >= R zero
  f16_t uoT[RA][KD];           // the same, fp16 transposed (MFMA operands)
  f16_t qoT[RA][VD];
  f16_t qT[RA][VD];            // Q^T operand of the P steps: fp16-rounded Q0, then Q16
  f32x4 qv[NB][VD];            // Q rows: fp32 before CholeskyQR, then Q16
  unsigned long long due;      // persistent flush: due mask of the current candidate chunk
};

// Thread index as seen by the per-head code.  Re-read through an empty asm at the start of every head so that the
// persistent flush loop cannot hoist the ~100 per-lane LDS addresses derived from it (and keep them all live).
__device__ __forceinline__ int opaque_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}
__device__ __forceinline__ int lane_id() { return opaque_tid() & 63; }
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(opaque_tid() >> 6); }

// wave-uniform reductions: DPP within each 16-lane row, then the 4 row results through readlane (no LDS traffic)
__device__ __forceinline__ float rl(float x, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}
// wave all-reduce for the serial factor steps (MGS, CholeskyQR): VALU lane swaps, every lane gets the result
__device__ __forceinline__ float sum64u(float x) { return sum64(x); }

// fn(i, s): s[r] = sum_v M[c_i][v] X[v][r] for the lane's 4 key channels c_i = 16 w + 4 (l >> 4) + i (complete in
// every lane of the 16-lane row)
template <class F>
__device__ __forceinline__ void colred(const Tile& t, const f32x4* X, F fn) {
  const int l = lane_id();
  f32x4 acc[4] = {};                                  // one row of X at a time (the sums keep the order of the rows)
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const f32x4 xv = X[16 * nt + (l & 15)];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float m = t.a[nt][i];
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][r] = fmaf(m, xv[r], acc[i][r]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f32x4 s;
#pragma unroll
    for (int r = 0; r < 4; ++r) s[r] = sum16(acc[i][r]);
    fn(i, s);
  }
}

// part[w][v][r] = sum over this wave's 16 channels c of M[c][v] Y[c][r]  (caller sums the NW waves)
__device__ __forceinline__ void rowred(const Tile& t, const f32x4* Y, f32x4 (*part)[VD]) {
  const int l = lane_id(), w = wave_id(), q = l >> 4;
  f32x4 yc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) yc[i] = Y[16 * w + 4 * q + i];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float m = t.a[nt][i];
      s[0] = fmaf(m, yc[i][0], s[0]);
      s[1] = fmaf(m, yc[i][1], s[1]);
      s[2] = fmaf(m, yc[i][2], s[2]);
      s[3] = fmaf(m, yc[i][3], s[3]);
    }
    ((float*)&part[w][16 * nt + (l & 15)])[q] = sum4_scatter(s);
  }
}

// CholeskyQR pass with the reference's pivot floors (kernels.py:1778-1835): 1 / L factors of the 4 x 4 Gram (packed
// lower triangle), then the rows times L^-T.  The reciprocal square roots are the hardware's (v_rsq_f32, about 1 ulp),
// as the reference's are approximate (T.rsqrt): the four of them are the serial spine of the factorisation on wave 0,
// and the correctly rounded 1 / sqrtf in their place cost the flush 3.5% (config 3, 188.4 -> 181.8 us with these) and
// the KDA flush 6% (125.8 -> 118.7 us).  The factors round to fp16 afterwards, and the oracle factorises in fp64, so
// the parity bars see no difference (every GPU test unchanged).
__device__ __forceinline__ void chol4(const float gg[10], float ll[10]) {
  ll[0] = __builtin_amdgcn_rsqf(fmaxf(gg[0], 1e-30f));
  ll[1] = gg[1] * ll[0];
  ll[2] = __builtin_amdgcn_rsqf(fmaxf(fmaxf(gg[2] - ll[1] * ll[1], 1e-6f * gg[2]), 1e-30f));
  ll[3] = gg[3] * ll[0];
  ll[4] = (gg[4] - ll[3] * ll[1]) * ll[2];
  ll[5] = __builtin_amdgcn_rsqf(fmaxf(fmaxf(gg[5] - ll[3] * ll[3] - ll[4] * ll[4], 1e-6f * gg[5]), 1e-30f));
  ll[6] = gg[6] * ll[0];
  ll[7] = (gg[7] - ll[6] * ll[1]) * ll[2];
  ll[8] = (gg[8] - ll[6] * ll[3] - ll[7] * ll[4]) * ll[5];
  ll[9] = __builtin_amdgcn_rsqf(fmaxf(fmaxf(gg[9] - ll[6] * ll[6] - ll[7] * ll[7] - ll[8] * ll[8], 1e-6f * gg[9]), 1e-30f));
}
__device__ __forceinline__ void chol4_solve(const float ll[10], f32x4& p) {
  p[0] = p[0] * ll[0];
  p[1] = (p[1] - p[0] * ll[1]) * ll[2];
  p[2] = (p[2] - p[0] * ll[3] - p[1] * ll[4]) * ll[5];
  p[3] = (p[3] - p[0] * ll[6] - p[1] * ll[7] - p[2] * ll[8]) * ll[9];
}
// The 10 entries of a 4 x 4 Gram from the lanes' partial sums x[k], summed over the wave.  The ten sums share their
// lane exchanges: a swap32 round adds the lane rows r, r + 2 of entry pairs (k, k + 5), a swap16 round adds rows r,
// r + 1 of the results, after which each 16-lane row of three registers holds a different entry summed over the four
// rows; one DPP pass sums within the rows and each entry is read from its row (~50 instructions where ten wave
// all-reductions take ~110, on wave 0's serial chain).
__device__ __forceinline__ void gram_sum10(const float x[10], float g[10]) {
  float y[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) {                       // rows 0-1: entry i; rows 2-3: entry i + 5
    uint32_t a = __float_as_uint(x[i]), b = __float_as_uint(x[i + 5]);
    swap32(a, b);
    y[i] = __uint_as_float(a) + __uint_as_float(b);
  }
  float z[3];
  {
    uint32_t a = __float_as_uint(y[0]), b = __float_as_uint(y[1]);
    swap16(a, b);
    z[0] = sum16(__uint_as_float(a) + __uint_as_float(b));   // rows: entries 0, 1, 5, 6
  }
  {
    uint32_t a = __float_as_uint(y[2]), b = __float_as_uint(y[3]);
    swap16(a, b);
    z[1] = sum16(__uint_as_float(a) + __uint_as_float(b));   // rows: entries 2, 3, 7, 8
  }
  {
    uint32_t a = __float_as_uint(y[4]), b = a;
    swap16(a, b);
    z[2] = sum16(__uint_as_float(a) + __uint_as_float(b));   // rows: entries 4, 4, 9, 9
  }
  g[0] = rl(z[0], 0);  g[1] = rl(z[0], 16); g[5] = rl(z[0], 32); g[6] = rl(z[0], 48);
  g[2] = rl(z[1], 0);  g[3] = rl(z[1], 16); g[7] = rl(z[1], 32); g[8] = rl(z[1], 48);
  g[4] = rl(z[2], 0);  g[9] = rl(z[2], 32);
}
// on the 2 rows (l, l + 64) a lane of wave 0 holds: the Gram over all 128 rows
__device__ __forceinline__ void cholqr_pass(f32x4& p0, f32x4& p1) {
  float gx[10], gg[10], ll[10];
  int k = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c <= r; ++c) gx[k++] = fmaf(p0[r], p0[c], p1[r] * p1[c]);
  gram_sum10(gx, gg);
  chol4(gg, ll);
  chol4_solve(ll, p0);
  chol4_solve(ll, p1);
}
// on the one row a lane holds: the Gram over the wave's 64 rows (one head of a pair, K = 64 flush)
__device__ __forceinline__ void cholqr_pass1(f32x4& p) {
  float gx[10], gg[10], ll[10];
  int k = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c <= r; ++c) gx[k++] = p[r] * p[c];
  gram_sum10(gx, gg);
  chol4(gg, ll);
  chol4_solve(ll, p);
}

// modified Gram-Schmidt on the R columns of the 128 x 4 matrix whose rows l, l + 64 a lane of wave 0 holds
// (kernels.py:2170-2183, 2190-2203).  The norms' reciprocal square roots are the hardware's (v_rsq_f32), as the
// reference's T.rsqrt is approximate: they sit on wave 0's serial chain, and an fp64 1 / sqrt in their place cost the
// config-3 quantize 5% (194.6 -> 185.6 us with these; every GPU test unchanged)
__device__ __forceinline__ void mgs(f32x4& p0, f32x4& p1, int R) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {               // unrolled over the largest rank (no run-time register indexing)
    if (j < R) {
#pragma unroll
      for (int c = 0; c < j; ++c) {
        const float sc = sum64u(fmaf(p0[c], p0[j], p1[c] * p1[j]));
        p0[j] = p0[j] - sc * p0[c];
        p1[j] = p1[j] - sc * p1[c];
      }
      const float nrm = sum64u(fmaf(p0[j], p0[j], p1[j] * p1[j]));
      const float rs = __builtin_amdgcn_rsqf(fmaxf(nrm, 1e-30f));
      p0[j] *= rs;
      p1[j] *= rs;
    }
  }
}
// the same on one row per lane (the 64 rows of one head of a pair, or the 64 key channels of a K = 64 head)
__device__ __forceinline__ void mgs1(f32x4& p, int R) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (j < R) {
#pragma unroll
      for (int c = 0; c < j; ++c) {
        const float sc = sum64u(p[c] * p[j]);
        p[j] = p[j] - sc * p[c];
      }
      const float nrm = sum64u(p[j] * p[j]);
      p[j] *= __builtin_amdgcn_rsqf(fmaxf(nrm, 1e-30f));
    }
  }
}
// the same on N columns held as plain arrays (rows l, l + 64 of a lane of wave 0), for ranks up to 16
template <int N>
__device__ __forceinline__ void mgs_n(float (&p0)[N], float (&p1)[N], int R) {
#pragma unroll
  for (int j = 0; j < N; ++j) {
    if (j < R) {
#pragma unroll
      for (int c = 0; c < j; ++c) {
        const float sc = sum64u(fmaf(p0[c], p0[j], p1[c] * p1[j]));
        p0[j] = p0[j] - sc * p0[c];
        p1[j] = p1[j] - sc * p1[c];
      }
      const float nrm = sum64u(fmaf(p0[j], p0[j], p1[j] * p1[j]));
      const float rs = __builtin_amdgcn_rsqf(fmaxf(nrm, 1e-30f));
      p0[j] *= rs;
      p1[j] *= rs;
    }
  }
}

// CholeskyQR pass of the wider-rank flush (R = 8, kernels.py:1744-1772) on N columns: the same factorisation, but a
// pivot that has lost all but 1e-6 of its Gram diagonal drops its column (1 / L_jj = 0) instead of being floored;
// columns past R are zero and stay zero.  Gram, factor and substitution run in fp64: a column that depends on the
// earlier ones leaves a pivot of ~1e-14 G_jj in fp64, but fp32 sums of 128 rows leave ~1e-6 G_jj of rounding -- the
// drop threshold itself -- so in fp32 whether such a column is dropped would be up to the rounding.
// lane l's fp64 value, uniform over the wave
__device__ __forceinline__ double rl_d(double x, int l) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, x);
  return join_d((unsigned)__builtin_amdgcn_readlane((int)(unsigned)u, l),
                (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(u >> 32), l));
}
template <int N>
__device__ __forceinline__ void cholqr_pass_drop(float (&p0)[N], float (&p1)[N]) {
  static_assert(N * (N + 1) / 2 <= 64, "one triangle entry per lane");
  const int lane = lane_id();
  double a = 0.0;                                     // lane t: entry t of the packed lower triangle (Gram, then factor)
#pragma unroll
  for (int r = 0; r < N; ++r)
#pragma unroll
    for (int c = 0; c <= r; ++c) {
      const double g = sum64d(fma((double)p0[r], (double)p0[c], (double)p1[r] * (double)p1[c]));
      a = lane == r * (r + 1) / 2 + c ? g : a;
    }
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const int rj = j * (j + 1) / 2;
#pragma unroll
    for (int k = 0; k < j; ++k) {
      const int rk = k * (k + 1) / 2;
      double ac = rl_d(a, rj + k);
#pragma unroll
      for (int m = 0; m < k; ++m) ac -= rl_d(a, rj + m) * rl_d(a, rk + m);
      ac *= rl_d(a, rk + k);                          // L_jk (the diagonal entries hold 1 / L_kk)
      a = lane == rj + k ? ac : a;
    }
    const double gjj = rl_d(a, rj + j);
    double ac = gjj;
#pragma unroll
    for (int m = 0; m < j; ++m) {
      const double ljm = rl_d(a, rj + m);
      ac -= ljm * ljm;
    }
    ac = ac > 1e-6 * gjj + 1e-30 ? 1.0 / sqrt(fmax(ac, 1e-30)) : 0.0;
    a = lane == rj + j ? ac : a;
  }
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    float (&p)[N] = s ? p1 : p0;
    double x[N];
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int rj = j * (j + 1) / 2;
      double ac = (double)p[j];
#pragma unroll
      for (int m = 0; m < j; ++m) ac -= x[m] * rl_d(a, rj + m);
      x[j] = ac * rl_d(a, rj + j);
    }
#pragma unroll
    for (int j = 0; j < N; ++j) p[j] = (float)x[j];
  }
}

// the 8 code words of the lane's tile entries (issued early; consumed by tile_add_words).  A head of K_ x V_ < 128 x
// 128 sits zero-padded in the tile: entries past its rows / columns read as 0 (clamped addresses, no divergent load).
template <int K_ = KD, int V_ = VD>
__device__ __forceinline__ void load_code_words(uint32_t wds[8], const int8_t* Sq) {
  const int l = lane_id(), w = wave_id(), q = l >> 4;
  const int c = 16 * w + 4 * q;
  const bool cok = K_ == KD || c < K_;
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const int v = 16 * nt + (l & 15);
    const uint32_t x = *(const uint32_t*)(Sq + (V_ == VD ? v : min(v, V_ - 1)) * K_ + (K_ == KD ? c : min(c, K_ - 4)));
    wds[nt] = (cok && (V_ == VD || v < V_)) ? x : 0u;
  }
}
// t += the dequantised checkpoint codes  x svr[v] x skl[c], each term rounded to fp32 before the add.  The flush adds
// them after the window's MFMA products, which it accumulates from zero: the window terms are up to ~20x larger than
// their sum (they cancel), and an accumulator seeded with the checkpoint term rounds them at a coarser step.
__device__ __forceinline__ void tile_add_words(Tile& t, const uint32_t wds[8], const float* svr, const float* skl) {
#pragma clang fp contract(off)
  const int l = lane_id(), w = wave_id(), q = l >> 4;
  const int c0 = 16 * w + 4 * q;
  float kc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) kc[i] = skl[c0 + i];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const float rv = svr[16 * nt + (l & 15)];
#pragma unroll
    for (int i = 0; i < 4; ++i) t.a[nt][i] = t.a[nt][i] + ((float)(int)(int8_t)(wds[nt] >> (8 * i)) * rv) * kc[i];
  }
}

// acc[c][v] += sum_j A[c][j] B[v][j] over nks 32-entry steps (bf16 operands from LDS, fp32 accumulate)
__device__ __forceinline__ void rebuild_mfma(Tile& t, const bf16_t (*A)[OPS], const bf16_t (*B)[OPS], int nks) {
  const int l = lane_id(), w = wave_id(), q = l >> 4;
  for (int ks = 0; ks < nks; ++ks) {
    const bf16x8 af = *(const bf16x8*)&A[16 * w + (l & 15)][32 * ks + 8 * q];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const bf16x8 bfr = *(const bf16x8*)&B[16 * nt + (l & 15)][32 * ks + 8 * q];
      t.a[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr, t.a[nt], 0, 0, 0);
    }
  }
}

// Window rows of one head, loaded up front (unconditional, clamped addresses; rows >= h and the padding to LP carry
// zero weight).  Thread t takes the row pair (2 jp, 2 jp + 1), jp = t % (LP / 2), in the 8-column chunk t / (LP / 2)
// (16 chunks; LP = 64 keeps every thread busy), so that each LDS write below holds two entries.
struct WinRegs {
  uint4 k[2], u[2];
};
__device__ __forceinline__ int win_pair(int LP) { return opaque_tid() % (LP / 2); }
__device__ __forceinline__ int win_chunk(int LP) { return opaque_tid() / (LP / 2); }
template <int K_ = KD, int V_ = VD>
__device__ __forceinline__ void load_window(WinRegs& r, const lq_state& st, int slot, int hv, int h, int LP) {
  const int G = st.HV / st.H, hk = hv / G, L = st.L;
  const bf16_t* Kb = (const bf16_t*)st.Kbuf + ((long long)slot * st.H + hk) * L * K_;
  const bf16_t* Ub = (const bf16_t*)st.Ubuf + ((long long)slot * st.HV + hv) * L * V_;
  const int jp = win_pair(LP), c8 = min(win_chunk(LP), 15) * 8;
  const uint4 z = make_uint4(0u, 0u, 0u, 0u);       // columns past a K_ / V_ < 128 head: zero operands
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int j = 2 * jp + k, jr = j < h ? j : 0;
    const uint4 kx = *(const uint4*)(Kb + (long long)jr * K_ + (K_ == KD ? c8 : min(c8, K_ - 8)));
    const uint4 ux = *(const uint4*)(Ub + (long long)jr * V_ + (V_ == VD ? c8 : min(c8, V_ - 8)));
    r.k[k] = (K_ == KD || c8 < K_) ? kx : z;
    r.u[k] = (V_ == VD || c8 < V_) ? ux : z;
  }
}
// Transposed into the rebuild operands [c or v][j], two entries (rows j0, j0 + 1) per 32-bit LDS write: op0 = K_j[c],
// op1 / op2 = hi / lo of w_j u_j[v] (kernels.py:1501-1511).  Rows j >= h carry zero values.
template <class SH>
__device__ __forceinline__ void store_window(SH& sh, const WinRegs& r, int h, int LP) {
  const int ch = win_chunk(LP);
  if (ch >= 16) return;
  const int j0 = 2 * win_pair(LP), c8 = ch * 8;
  const bool v0 = j0 < h, v1 = j0 + 1 < h;
  const float w0 = v0 ? sh.w[j0] : 0.f, w1 = v1 ? sh.w[j0 + 1] : 0.f;
  const uint32_t ka[4] = {r.k[0].x, r.k[0].y, r.k[0].z, r.k[0].w}, kb[4] = {r.k[1].x, r.k[1].y, r.k[1].z, r.k[1].w};
  const uint32_t ua[4] = {r.u[0].x, r.u[0].y, r.u[0].z, r.u[0].w}, ub[4] = {r.u[1].x, r.u[1].y, r.u[1].z, r.u[1].w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int x = e >> 1;
    const bool odd = e & 1;
    const uint32_t sel = odd ? 0x07060302u : 0x05040100u;   // the two rows' halves of column c8 + e
    *(uint32_t*)&sh.op[0][c8 + e][j0] = __builtin_amdgcn_perm(kb[x], ka[x], sel);
    {
      // the split is of the fp32-rounded product: no fusing of w u into the lo subtraction (kernels.py:1509-1511)
#pragma clang fp contract(off)
      const float wu0 = w0 * (odd ? bf_hi(ua[x]) : bf_lo(ua[x]));
      const float wu1 = w1 * (odd ? bf_hi(ub[x]) : bf_lo(ub[x]));
      const uint32_t hi = pk_bf16_kept(wu0, wu1);
      *(uint32_t*)&sh.op[1][c8 + e][j0] = hi;
      *(uint32_t*)&sh.op[2][c8 + e][j0] = pk_bf16(wu0 - bf_lo(hi), wu1 - bf_hi(hi));
    }
  }
}
// per-wave partial sums of the row reductions -> the full sum for row v (threads v < 128)
__device__ __forceinline__ f32x4 sum_parts(const f32x4 (*part)[VD], int v) {
  f32x4 s = part[0][v];
#pragma unroll
  for (int w = 1; w < NW; ++w) s += part[w][v];
  return s;
}

// M[a][r] = sum_k X[k][a] Y[k][r] over 128 k for a, r < RA, from the fp16 transposed operands X^T, Y^T ([RA][128]): the
// MFMA leaves M[a][r] in lane 16 (a >> 2) + r, element a & 3; every lane gets all RA x RA entries
template <int RA>
__device__ __forceinline__ void gram_t(const f16_t (*XT)[128], const f16_t (*YT)[128], float (&M)[RA][RA]) {
  const int l = lane_id(), q = l >> 4, l16 = l & 15;
  const bool rla = l16 < RA;
  const f16x8 z8 = {};
  f32x4 macc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const f16x8 ao = rla ? *(const f16x8*)&XT[l16][32 * ks + 8 * q] : z8;
    const f16x8 by = rla ? *(const f16x8*)&YT[l16][32 * ks + 8 * q] : z8;
    macc = mma32(ao, by, macc);
  }
#pragma unroll
  for (int a = 0; a < RA; ++a)
#pragma unroll
    for (int r = 0; r < RA; ++r) M[a][r] = rl(macc[a & 3], 16 * (a >> 2) + r);
}

// ------------------------------------------------------------------------------------------------------------------
// flush (kernels.py:1077-2033): one due (slot, head)
// ------------------------------------------------------------------------------------------------------------------
// P = B^T Q + pn U_old (Q_old^T Q) for this wave's 16 key channels, fp16-rounded (kernels.py:1580-1700).  Q^T comes
// from sh.qT; bt[nt] is the transposed packing of B (lane l: B[16 w + (l & 15)][16 nt + 4 (l >> 4) + i]).  Lanes
// l < 16 RA / 4 return P[16 w + (l & 15)][4 (l >> 4) + i] (zero for columns >= R); the other lanes return zeros.
template <int RA>
__device__ __forceinline__ f32x4 p_step(const FlushShared<RA>& sh, const f16x4 bt[8], float pn, int R) {
  constexpr int NB = RA / 4;
  const int l = lane_id(), w = wave_id(), q = l >> 4, l16 = l & 15;
  const bool rla = l16 < RA;
  const f16x4 z4 = {};
  float M[RA][RA];                                    // Q_old^T Q
  gram_t<RA>(sh.qoT, sh.qT, M);
  // P^T[r][c] = sum_v Q^T[r][v] B[c][v]  (k = v from the transposed packing)
  f32x4 pacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const f16x4 aq = rla ? *(const f16x4*)&sh.qT[l16][16 * nt + 4 * q] : z4;
    pacc = mma16(aq, bt[nt], pacc);
  }
  float uo[RA];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const f32x4 x = sh.uoc[b][16 * w + l16];
#pragma unroll
    for (int i = 0; i < 4; ++i) uo[4 * b + i] = x[i];
  }
  f32x4 p;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float corr = 0.f;
#pragma unroll
    for (int a = 0; a < RA; ++a) {
      float m = M[a][i];                              // column r = 4 q + i of this lane
#pragma unroll
      for (int b = 1; b < NB; ++b) m = q == b ? M[a][4 * b + i] : m;
      corr = a == 0 ? uo[0] * m : corr + uo[a] * m;
    }
    p[i] = (q < NB && 4 * q + i < R) ? hround(pacc[i] + pn * corr) : 0.f;
  }
  return p;
}

// A GDN head of K_ x V_ < 128 x 128 (kernels.py:1089: (64, 128), (64, 64)) runs zero-padded in the 128 x 128 tile:
// its loads read zeros past its rows / columns, every product and Gram sum then only adds exact zeros, the column
// means divide by V_, and the stores write its own rows / columns only.  RA = 8 (GDN 128 x 128, R = 8): the factor
// products carry eight columns (lanes l < 32 of each MFMA) and CholeskyQR drops dependent columns (kernels.py:1744-1772).
// Dynamic head schedule of the persistent flush (lq_state.sched, LQ_SCHED_INTS ints): eight counters 256 bytes apart;
// workgroup b uses counter b % 8 (the dispatcher deals workgroups round-robin over the eight XCDs), so that the
// grid's takes spread over eight addresses instead of queueing on one (one counter measured 41.5 -> 51 us on a flush
// where every workgroup took once at the same time).  Counter x hands out the candidates after the grid's first
// ones with x = (p - gridDim.x) % 8, take g giving p = gridDim.x + 8 g + x; its low SCHED_BITS count the takes, the
// high bits the group's workgroups done, and the last of them clears it.  A head takes its workgroup's next candidate
// (thread 0) after its column scales, so that the atomic's latency hides behind the rest of the head and the
// workgroup commits to the next head only near the end of this one, and leaves it in the shared `due` word before
// the head's last barrier.
constexpr int SCHED_BITS = 20, SCHED_GROUPS = 8, SCHED_STRIDE = 64;
static_assert(SCHED_GROUPS * SCHED_STRIDE == LQ_SCHED_INTS, "counters of lq_state.sched");
__device__ __forceinline__ int* sched_counter(int* sched) {
  return sched + SCHED_STRIDE * (int)(blockIdx.x % SCHED_GROUPS);
}
// A take (the counter's old value) and the candidate it stands for are two steps, so that a head can issue its take
// early and turn it into a candidate only where it stores it: the atomic's round trip then overlaps the head's last
// stages instead of holding wave 0 right after the take (a use of the result right away waits for it there).
__device__ __forceinline__ int sched_take(int* sched) {
  return __hip_atomic_fetch_add(sched_counter(sched), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int sched_candidate(int take) {
  return (int)gridDim.x + SCHED_GROUPS * (take & ((1 << SCHED_BITS) - 1)) + (int)(blockIdx.x % SCHED_GROUPS);
}
__device__ __forceinline__ int sched_next(int* sched) { return sched_candidate(sched_take(sched)); }
// The unit a dynamic-schedule candidate names.  Candidate c = 8 j + x is taken in schedule group x (x = blockIdx.x mod
// 8 for the first round, which is the XCD the dispatcher places the workgroup on, and the group's counter after it),
// as the group's j-th.  With G value heads per key head, the G candidates j = G m .. G m + G - 1 of group x name the G
// value heads of one key head (unit G (8 m + x) + j mod G), so they are flushed on one XCD at about the same time and
// the key window they share is read into that XCD's L2 once.  A bijection on each block of 8 G candidates; the last,
// partial block keeps its order.  A launch of one workgroup per unit maps its workgroups the same way (workgroup
// b = 8 j + x runs on XCD x, and b, b + 8, ... are dispatched one after the other).
__device__ __forceinline__ int sched_unit(int c, int G, int total) {
  const int blk = SCHED_GROUPS * G;
  if (G == 1 || c >= total - total % blk) return c;
  const int j = c / SCHED_GROUPS, x = c - SCHED_GROUPS * j;
  const int m = j / G;
  return blk * m + G * x + (j - G * m);
}
// the take's value where it is used: an opaque copy, so that nothing computed from it moves up to the take (and with it
// the wait for the atomic's return)
__device__ __forceinline__ int take_result(int take) {
  asm volatile("" : "+v"(take));
  return take;
}

template <int K_ = KD, int V_ = VD, int RA = 4>
__device__ void flush_head(FlushShared<RA>& sh, const lq_state& st, const float* __restrict__ Q0, int slot, int hv,
                           float qmax, int* sched = nullptr) {
  static_assert(RA == 4 || (RA == 8 && K_ == KD && V_ == VD), "R = 8: 128 x 128 heads");
  constexpr int NB = RA / 4;
  const int HV = st.HV, L = st.L, R = st.R;
  const long long sh_ = (long long)slot * HV + hv;
  const int tid = opaque_tid(), l = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), q = l >> 4, l16 = l & 15;
  const int qb = q < NB ? q : NB - 1;                 // this lane's factor block in the MFMA operands (lanes < 16 NB)
  char* base = block_base(st, slot, hv);
  int8_t* Sq = (int8_t*)base;
  float* Sk = (float*)(base + V_ * K_);
  float* Sv = Sk + K_;
  f16_t* UQ = (f16_t*)(Sv + V_);
  const int LP = (L + 31) & ~31;

  // ---- stage 1: every load of the head up front (scalars, scales, factors, window rows, code words) ----
  const float pn = fmaxf(st.Pbuf[sh_], LQ_PNMIN);     // kernels.py:1471
  const float rpn = 1.0f / pn;                        // kernels.py:1477
  const int cv = tid & 127;                           // column (tid < 128) or row (128 <= tid < 256) of the stage-1 loads
  const bool colt = tid < KD;
  const int nc = colt ? K_ : V_;                      // this thread's column / row count
  const bool cok = (K_ == KD && V_ == VD) || cv < nc;
  const int cvc = (K_ == KD && V_ == VD) ? cv : min(cv, nc - 1);
  const int vq = V_ == VD ? cv : min(cv, V_ - 1);
  const float scv = cok ? (colt ? Sk[cvc] : Sv[cvc]) : 0.f;
  float uqv[RA], q0v[RA];
#pragma unroll
  for (int a = 0; a < RA; ++a) {
    const float x = h2f(UQ[min(a, R - 1) * (K_ + V_) + (colt ? 0 : K_) + cvc]);
    uqv[a] = cok ? x : 0.f;
    const float y = Q0[vq * R + min(a, R - 1)];
    q0v[a] = (V_ == VD || cv < V_) ? y : 0.f;
  }
  const float wv = st.Wbuf[sh_ * L + min(tid, L - 1)];
  WinRegs win;
  load_window<K_, V_>(win, st, slot, hv, L, LP);
  uint32_t wds[8];
  load_code_words<K_, V_>(wds, Sq);

  if (tid < KD) {
    const int c = cv;
    sh.skl[c] = scv;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      f32x4 u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int a = 4 * b + i;
        u[i] = a < R ? uqv[a] : 0.f;
        sh.uoT[a][c] = f2h(u[i]);
      }
      sh.uoc[b][c] = u;
    }
  } else if (tid < KD + VD) {
    const int v = cv;
    sh.svr[v] = scv * (pn / qmax);                                                    // kernels.py:1483
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      f32x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int a = 4 * b + i;
        o[i] = a < R ? uqv[a] : 0.f;
        sh.qoT[a][v] = f2h(o[i]);
        sh.qT[a][v] = f2h(a < R ? hround(q0v[a]) : 0.f);                              // kernels.py:1573-1577
      }
      sh.qov[b][v] = o;
    }
  }
  if (tid < LPMAX) sh.w[tid] = tid < L ? wv : 0.f;
  __syncthreads();
  store_window(sh, win, L, LP);
  __syncthreads();

  // ---- stage 2: B = deq(S0) pn + window, fp16 (kernels.py:1483-1571) ----
  f16x4 bh[8], bt[8];                                 // B packed: k = c (tile layout) and k = v (transposed)
  {
    Tile t;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) t.a[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    rebuild_mfma(t, sh.op[0], sh.op[1], LP / 32);
    rebuild_mfma(t, sh.op[0], sh.op[2], LP / 32);
    tile_add_words(t, wds, sh.svr, sh.skl);
    f16x4 ident;
#pragma unroll
    for (int i = 0; i < 4; ++i) ident[i] = (4 * q + i == l16) ? (_Float16)1.0f : (_Float16)0.0f;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      bh[nt] = to_h4(t.a[nt]);                        // the fp16 rounding of B
      bt[nt] = to_h4(mma16(bh[nt], ident, f32x4{0.f, 0.f, 0.f, 0.f}));   // exact: B^T block through the identity
    }
  }

  // ---- stage 3: subspace iteration (ITERS = 1) with the algebraic rank-R corrections (kernels.py:1580-1842) ----
  const f32x4 p16 = p_step<RA>(sh, bt, pn, R);        // P16 rows of this wave (lanes < 16 NB)
  __syncthreads();                                    // every wave is past the rebuild: the op region is free
  if (tid < VD) {
#pragma unroll
    for (int b = 0; b < NB; ++b) sh.r.qo16[b][tid] = to_h4(sh.qov[b][tid]);
  }
  // Q = B P16 + pn Q_old (U_old^T P16): per-wave partials of B P16 over the wave's 16 channels, summed below
  if (q < NB) {
#pragma unroll
    for (int i = 0; i < 4; ++i) sh.r.ppT[4 * q + i][16 * w + l16] = f2h(p16[i]);
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  {
    const f16x4 z4 = {};
    const f16x4 ap = l16 < RA ? *(const f16x4*)&sh.r.ppT[l16][16 * w + 4 * q] : z4;   // A[r][c] = P16^T
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const f32x4 d = mma16(ap, bh[nt], f32x4{0.f, 0.f, 0.f, 0.f});                 // Q^T[4 q + i][16 nt + l]
      if (q < NB) sh.r.qpart[w][qb][16 * nt + l16] = d;
    }
  }
  __syncthreads();
  if (tid < VD) {                                     // waves 0 and 1: one row v per thread
    // M2[a][r] = sum_c U_old[c][a] P16[c][r] over all 128 channels (every column of P16 is in ppT now)
    float M2[RA][RA];
    gram_t<RA>(sh.uoT, sh.r.ppT, M2);
    const int v = tid;
    float qo[RA];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const f32x4 x = sh.qov[b][v];
#pragma unroll
      for (int i = 0; i < 4; ++i) qo[4 * b + i] = x[i];
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      f32x4 s = sh.r.qpart[0][b][v];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) s += sh.r.qpart[w2][b][v];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float corr = qo[0] * M2[0][4 * b + i];
#pragma unroll
        for (int a = 1; a < RA; ++a) corr += qo[a] * M2[a][4 * b + i];
        s[i] += pn * corr;
      }
      sh.qv[b][v] = s;
    }
  }
  __syncthreads();
  // CholeskyQR2 (wave 0), fp16 Q.  The serial phases of one wave run at raised wave priority: the CU's other workgroup
  // competes for the same SIMDs while this one's other waves wait at the barrier (config 3: flush 339 -> 331 us,
  // quantize 222 -> 214 us with the same in its MGS phases)
  if (w == 0) {
    __builtin_amdgcn_s_setprio(3);
    if constexpr (RA == 4) {
      f32x4 p0 = sh.qv[0][l], p1 = sh.qv[0][l + 64];
#pragma unroll
      for (int r = 0; r < 4; ++r) { if (r >= R) { p0[r] = 0.f; p1[r] = 0.f; } }
      cholqr_pass(p0, p1);
      cholqr_pass(p0, p1);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p0[r] = r < R ? hround(p0[r]) : 0.f;
        p1[r] = r < R ? hround(p1[r]) : 0.f;
        sh.qT[r][l] = f2h(p0[r]);
        sh.qT[r][l + 64] = f2h(p1[r]);
      }
      sh.qv[0][l] = p0;
      sh.qv[0][l + 64] = p1;
      sh.r.qn16[0][l] = to_h4(p0);
      sh.r.qn16[0][l + 64] = to_h4(p1);
    } else {
      float p0[RA], p1[RA];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const f32x4 x0 = sh.qv[b][l], x1 = sh.qv[b][l + 64];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p0[4 * b + i] = 4 * b + i < R ? x0[i] : 0.f;
          p1[4 * b + i] = 4 * b + i < R ? x1[i] : 0.f;
        }
      }
      cholqr_pass_drop<RA>(p0, p1);
      cholqr_pass_drop<RA>(p0, p1);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        f32x4 y0, y1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * b + i;
          y0[i] = r < R ? hround(p0[r]) : 0.f;
          y1[i] = r < R ? hround(p1[r]) : 0.f;
          sh.qT[r][l] = f2h(y0[i]);
          sh.qT[r][l + 64] = f2h(y1[i]);
        }
        sh.qv[b][l] = y0;
        sh.qv[b][l + 64] = y1;
        sh.r.qn16[b][l] = to_h4(y0);
        sh.r.qn16[b][l + 64] = to_h4(y1);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  }
  __syncthreads();
  const f32x4 u16 = p_step<RA>(sh, bt, pn, R);        // U16 = P step with Q16 (lanes < 16 NB: rows 16 w + l)

  // ---- stage 4: residual E = fp16(pn (B / pn + Q_old U_old^T) - Q U^T) (kernels.py:1888-1928) ----
  // E kept packed in B's registers (B is dead after the Q partials), consumed through v_fma_mix_f32 as in flush_head4
  {
    const f16x4 z4 = {};
    const f16x4 auo = q < NB ? to_h4(sh.uoc[qb][16 * w + l16]) : z4;                // A[c][a] = U_old
    const f16x4 aun = q < NB ? to_h4(-u16) : z4;                                     // A[c][r] = -U16
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int v = 16 * nt + l16;
      // B[a][v] = Q_old^T, B[r][v] = Q16^T; rows past the lane's factor block meet the zero columns of A
      const f16x4 bqo = sh.r.qo16[qb][v];
      const f16x4 bqn = sh.r.qn16[qb][v];
      const f16x4 b = bh[nt];
      f32x4 e = {h4mul<0>(b, rpn), h4mul<1>(b, rpn), h4mul<2>(b, rpn), h4mul<3>(b, rpn)};
      e = mma16(auo, bqo, e);
      e *= pn;
      e = mma16(aun, bqn, e);
      bh[nt] = to_h4(e);                                                            // E, fp16
    }
  }

  // ---- stage 5: column smoothing scales (kernels.py:1929-1958) ----
  float rsk[4];
  {
    float cs[4], x0 = 0.f, x1 = 0.f, x2 = 0.f, x3 = 0.f;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      x0 = h4abs_add<0>(bh[nt], x0);
      x1 = h4abs_add<1>(bh[nt], x1);
      x2 = h4abs_add<2>(bh[nt], x2);
      x3 = h4abs_add<3>(bh[nt], x3);
    }
    cs[0] = sum16(x0);
    cs[1] = sum16(x1);
    cs[2] = sum16(x2);
    cs[3] = sum16(x3);
    // the square root and division once per column: lane l takes column 4 q + (l & 3) of its row group
    const int ic = l & 3;
    const float msum = (ic == 0 ? cs[0] : ic == 1 ? cs[1] : ic == 2 ? cs[2] : cs[3]) * (1.0f / V_);
    const float sq = sqrtf(msum);
    const float rs = fminf(1.0f / sq, 1.0f / LQ_EPS);
    if (l16 < 4 && (K_ == KD || 16 * w + 4 * q + l16 < K_)) Sk[16 * w + 4 * q + l16] = fmaxf(sq, LQ_EPS);
    rsk[0] = dpp<0x00>(rs);                           // quad_perm [i, i, i, i]: column i of the lane's quad
    rsk[1] = dpp<0x55>(rs);
    rsk[2] = dpp<0xaa>(rs);
    rsk[3] = dpp<0xff>(rs);
  }
  int next = 0;                                       // dynamic schedule: this workgroup's next candidate
  if (sched && tid == 0) next = sched_take(sched);
  // ---- stage 6: row scales and codes (kernels.py:1974-2009) ----
  Tile t;                                             // E rsk, fp32
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    float m = 0.f;
    const f16x4 e = bh[nt];
    t.a[nt] = f32x4{h4mul<0>(e, rsk[0]), h4mul<1>(e, rsk[1]), h4mul<2>(e, rsk[2]), h4mul<3>(e, rsk[3])};
#pragma unroll
    for (int i = 0; i < 4; ++i) m = fmaxf(m, fabsf(t.a[nt][i]));
    sh.r.rmx[4 * w + q][16 * nt + l16] = m;
  }
  __syncthreads();
  if (tid < VD) {
    float m = sh.r.rmx[0][tid];
#pragma unroll
    for (int k = 1; k < 4 * NW; ++k) m = fmaxf(m, sh.r.rmx[k][tid]);
    const float rmax = fmaxf(m, LQ_EPS);
    if (V_ == VD || tid < V_) Sv[tid] = rmax;
    sh.r.rq[tid] = qmax * (1.0f / rmax);
  }
  __syncthreads();
  uint32_t cw[8];                                     // code words of rows 16 nt + l16, channels 16 w + 4 q ..
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const int v = 16 * nt + l16;
    const float rq = sh.r.rq[v];
    uint32_t b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = __float_as_uint(__builtin_fmaf(t.a[nt][i], rq, 12582912.0f));   // RNE via 1.5 2^23
    const uint32_t lo = __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u), hi = __builtin_amdgcn_perm(b[3], b[2], 0x0c0c0400u);
    cw[nt] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
  }
  if constexpr (K_ == KD && V_ == VD) {
    // a 4 x 4 transpose over the lane groups (register j of group q -> register q of group j) gives lane (q, l16) the
    // four words of row 16 (4 m + q) + l16, channels 16 w .. 16 w + 15: two 16-byte stores instead of eight 4-byte ones
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      uint32_t a0 = cw[4 * m], a1 = cw[4 * m + 1], a2 = cw[4 * m + 2], a3 = cw[4 * m + 3];
      swap32(a0, a2);
      swap32(a1, a3);
      swap16(a0, a1);
      swap16(a2, a3);
      *(uint4*)(Sq + (16 * (4 * m + q) + l16) * KD + 16 * w) = make_uint4(a0, a1, a2, a3);
    }
  } else {
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int v = 16 * nt + l16;
      if ((K_ == KD || 16 * w + 4 * q < K_) && (V_ == VD || v < V_)) *(uint32_t*)(Sq + v * K_ + 16 * w + 4 * q) = cw[nt];
    }
  }
  // ---- stage 7: factors, window reset (kernels.py:1836-1842, 2014-2025) ----
  if (q < NB && (K_ == KD || 16 * w + l16 < K_)) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * q + i < R) UQ[(4 * q + i) * (K_ + V_) + 16 * w + l16] = f2h(u16[i]);
  }
  if (tid < V_) {
    for (int r = 0; r < R; ++r) UQ[r * (K_ + V_) + K_ + tid] = f2h(sh.qv[r >> 2][tid][r & 3]);
  }
  if (tid < L) st.Wbuf[sh_ * L + tid] = 0.f;
  if (tid == 0) {
    st.Pbuf[sh_] = 1.f;
    st.hcnt[sh_] = 0;
    if (sched) sh.due = (unsigned long long)sched_candidate(take_result(next));
  }
  __syncthreads();                                    // LDS reuse by the next head of this workgroup
}

// ------------------------------------------------------------------------------------------------------------------
// Four-wave flush (GDN with R <= 4, and KDA): one due head per workgroup of 256 threads, <= 40 KiB LDS and <= 128
// VGPRs, so that four heads share a CU (the eight-wave flush above fits two).  The flush is latency-bound -- each head
// is a chain of dependent, barrier-separated phases -- so heads in flight per CU set its rate.  Same arithmetic, in the
// same order, as flush_head; only the distribution over the lanes differs: wave w owns key channels [32 w, 32 w + 32)
// as two groups g of 16, and lane l holds
//     a[g][nt][i] = M[c][v],   c = 32 w + 16 g + 4 (l >> 4) + i,   v = 16 nt + (l & 15).
// The window is staged and multiplied in halves of 32 entries.  KDA (kernels.py:1443-1471, 1519): pn = 1, the
// per-channel decay exp(Pbuf[c]) folds into the column factor Sk and the old U rows, and the window's keys enter as
// decayed hi / lo operands (kda_key_scan4), the halves staged newest first.
// ------------------------------------------------------------------------------------------------------------------
constexpr int FT4 = 256;             // threads per workgroup
constexpr int NW4 = FT4 / 64;        // waves
constexpr int HALF = 32;             // window entries staged at once
constexpr int OPS4 = HALF + 8;       // operand row stride (bf16): 80 B rows, 16-byte aligned, conflict-free b128 reads
// CF (conflict-free layout): the factor tables [4][128] fp16 are read by the four lane rows of a 16-lane group at once
// (row l & 3, same column), and rows of 128 halfs all start in the same bank, so each row is padded by 16 halfs (rows
// then start 8 banks apart); the row-maximum table [16][128] fp32 is written by the four lane groups at once (row
// 4 w + q, same column), padded by 16 floats (16 banks apart); store_half rotates the odd lane groups' columns (a
// rotated group's words permuted once, no select per write).  The standalone flush, the prefill dequant and the
// one-launch decode's flush use it (the flush's LDS bank conflicts fall by three quarters, LDS-active cycles by a
// third).
constexpr int FTP = 16, RMP = 16;

struct Tile4 {
  f32x4 a[2][8];
};

template <bool CF>
struct FlushShared4T {
  static constexpr int FP = CF ? FTP : 0, RP = CF ? RMP : 0;
  union {
    bf16_t op[3][KD][OPS4];    // rebuild operands of one window half [c or v][j]
    struct {                   // after the rebuild
      f32x4 qpart[NW4][VD];    // per-wave partial Q rows
      float rmx[4 * NW4][VD + RP];    // per-(wave, lane group) row maxima of the scaled residual
      float rq[VD];            // qmax / row scale
      f16_t ppT[4][KD + FP];   // P16^T
      f16_t uoT[4][KD + FP];   // old U^T, fp16 (MFMA operand)
      f16_t qoT[4][VD + FP];   // old Q^T, fp16
      f16x4 qo16[VD];          // old Q rows [v][a], fp16 (residual B operand)
      f16x4 qn16[VD];          // Q16 rows [v][r] (residual B operand)
      f32x4 mb[NW4][4];        // per-wave broadcast of a 4 x 4 product (gram_qold_q)
    } r;
  };
  float skl[KD];               // column factor of the dequant (Sk)
  float svr[VD];               // row factor of the dequant (Sv pn / qmax)
  float w[LPMAX];
  f32x4 uoc[KD];               // old U rows [c][a], a >= R zero
  f32x4 qov[VD];               // old Q rows [v][a], a >= R zero
  f16_t qT[4][VD + FP];        // Q^T operand of the P steps: fp16-rounded Q0, then Q16
  f32x4 qv[VD];                // Q rows: fp32 before CholeskyQR, then Q16
  unsigned long long due;      // persistent flush: due mask of the current candidate chunk / listed head
};
using FlushShared4 = FlushShared4T<true>;
static_assert(sizeof(FlushShared4T<true>) <= 40960 && sizeof(FlushShared4T<false>) <= 40960,
              "four workgroups per CU: 160 KiB of LDS");

// One window half's rows in registers: thread t takes entries 2 (t % 16), 2 (t % 16) + 1 of the half, columns
// 8 (t / 16) .. 8 (t / 16) + 7 (16 x 16 = 256 threads).  Rows >= h read row 0 (in bounds; their weight is zero).  KDA
// also takes the entries' per-channel decays (Gbuf, the keys' [j][c] layout).
struct WinHalf {
  uint4 k[2], u[2], g[2];
};
template <int K_, int V_, bool KDA = false>
__device__ __forceinline__ void load_half(WinHalf& r, const lq_state& st, int slot, int hv, int h, int hf) {
  const int G = st.HV / st.H, hk = hv / G, L = st.L;
  const bf16_t* Kb = (const bf16_t*)st.Kbuf + ((long long)slot * st.H + hk) * L * K_;
  const bf16_t* Ub = (const bf16_t*)st.Ubuf + ((long long)slot * st.HV + hv) * L * V_;
  const f16_t* Gb = KDA ? (const f16_t*)st.Gbuf + ((long long)slot * st.HV + hv) * L * KD : nullptr;
  const int t = opaque_tid(), jp = t % 16, c8 = (t / 16) * 8;
  const uint4 z = make_uint4(0u, 0u, 0u, 0u);        // columns past a K_ / V_ < 128 head: zero operands
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int j = HALF * hf + 2 * jp + k, jr = j < h ? j : 0;
    const uint4 kx = *(const uint4*)(Kb + (long long)jr * K_ + (K_ == KD ? c8 : min(c8, K_ - 8)));
    const uint4 ux = *(const uint4*)(Ub + (long long)jr * V_ + (V_ == VD ? c8 : min(c8, V_ - 8)));
    r.k[k] = (K_ == KD || c8 < K_) ? kx : z;
    r.u[k] = (V_ == VD || c8 < V_) ? ux : z;
    if constexpr (KDA) r.g[k] = *(const uint4*)(Gb + (long long)jr * KD + c8);
  }
}
// Transposed into the rebuild operands [c or v][j - HALF hf], two entries per 32-bit LDS write.  GDN: op0 = K_j[c],
// op1 / op2 = hi / lo of w_j u_j[v] (kernels.py:1501-1511); rows j >= h carry zero values.  KDA: op0 / op1 = raw K_j[c] /
// e_j[c] (turned into the decayed key operands by kda_key_scan4), op2 = u_j[v]; rows j >= h carry zero values and
// decay 1.  Write e of a lane writes column c8 + e, but the odd 16-lane groups (columns c8 = 8 (t / 16), 8 rows past
// the even group's) write c8 + (e + 4) mod 8: rows 8 + 4 or 8 - 4 apart are 80 or 240 dwords apart, 16 banks off, so
// the two groups of a half-wave write disjoint banks (rows exactly 8 apart, 160 dwords, share all 16).  Without CF no
// rotation (the same bytes either way).
template <bool KDA = false, bool CF>
__device__ __forceinline__ void store_half(FlushShared4T<CF>& sh, const WinHalf& r, int h, int hf) {
  // the split is of the fp32-rounded product: no fusing of w u into the lo subtraction (kernels.py:1509-1511)
#pragma clang fp contract(off)
  const int t = opaque_tid(), jl = 2 * (t % 16), c8 = (t / 16) * 8;
  const bool rot = CF && ((t / 16) & 1);
  const int j0 = HALF * hf + jl;
  const bool v0 = j0 < h, v1 = j0 + 1 < h;
  const float w0 = v0 ? sh.w[j0] : 0.f, w1 = v1 ? sh.w[j0 + 1] : 0.f;
  // the words of the lane's columns in the order it writes them: a rotated lane group's write e takes column
  // (e + 4) mod 8, i.e. word (x + 2) mod 4, so its words are permuted once here (one select each) instead of per write
  auto words = [&](const uint4& v, uint32_t (&o)[4]) {
    o[0] = rot ? v.z : v.x;
    o[1] = rot ? v.w : v.y;
    o[2] = rot ? v.x : v.z;
    o[3] = rot ? v.y : v.w;
  };
  uint32_t ka[4], kb[4], ua[4], ub[4], ga[4], gb[4];
  words(r.k[0], ka);
  words(r.k[1], kb);
  words(r.u[0], ua);
  words(r.u[1], ub);
  if constexpr (KDA) {
    words(r.g[0], ga);
    words(r.g[1], gb);
  }
  const uint32_t keep = (v0 ? 0x0000ffffu : 0u) | (v1 ? 0xffff0000u : 0u);
  // column of write e: c8 + (e + 4 rot) mod 8 = cA + e for e < 4, cB + e for e >= 4 (two bases, constant offsets)
  const int cA = c8 + (rot ? 4 : 0), cB = c8 - (rot ? 4 : 0);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int x = e >> 1;
    const bool odd = e & 1;
    const uint32_t sel = odd ? 0x07060302u : 0x05040100u;   // the two rows' halves of the column
    const int c = (e < 4 ? cA : cB) + e;
    const uint32_t kax = ka[x], kbx = kb[x], uax = ua[x], ubx = ub[x];
    *(uint32_t*)&sh.op[0][c][jl] = __builtin_amdgcn_perm(kbx, kax, sel);
    if constexpr (!KDA) {
      const float wu0 = w0 * (odd ? bf_hi(uax) : bf_lo(uax));
      const float wu1 = w1 * (odd ? bf_hi(ubx) : bf_lo(ubx));
      const uint32_t hi = pk_bf16_kept(wu0, wu1);
      *(uint32_t*)&sh.op[1][c][jl] = hi;
      *(uint32_t*)&sh.op[2][c][jl] = pk_bf16(wu0 - bf_lo(hi), wu1 - bf_hi(hi));
    } else {
      const uint32_t gax = ga[x], gbx = gb[x];
      *(uint32_t*)&sh.op[1][c][jl] = (__builtin_amdgcn_perm(gbx, gax, sel) & keep) | (0x3c003c00u & ~keep);
      *(uint32_t*)&sh.op[2][c][jl] = __builtin_amdgcn_perm(ubx, uax, sel) & keep;
    }
  }
}
// KDA key operands of one staged half, in place over its raw keys op[0] and decays op[1] ([c][j - HALF hf]): op[0] /
// op[1] = hi / lo of K_j[c] w_j D_j[c], D_j = prod_{j < i < h} e_i[c] (kernels.py:1453-1463).  The
// halves are staged newest first: dcar is D at the top of this half (the product of every later decay; 1 for the
// newest half), and the return value is the carry for the next, older half.  Two lanes per channel (c = t / 2): lane s
// takes entries 16 s .. 16 s + 15 and walks them backwards; lane 0 first multiplies through lane 1's decays (handed
// over by DPP), so that every D_j is the sequential walk's own product, one rounding per factor in the reference's
// order (a regrouped product rounds differently, and the key operands' cancellation in the rebuild turns such last-bit
// differences into fp16 flips of B).  Each lane reads and writes its own 16 entries only.  NT = 3 (the prefill dequant,
// state.py:124-127): the split is hi / mid / lo, op[0] / op[1] take hi / mid and lo3 the lane's lo words ([c][j] as
// the LDS rows: word x holds entries jb + 2 x, jb + 2 x + 1 of channel c).
template <int NT = 2, bool CF>
__device__ __forceinline__ float kda_key_scan4(FlushShared4T<CF>& sh, float dcar, int h, int hf,
                                               uint32_t* lo3 = nullptr) {
  // the split is of the fp32-rounded product (kernels.py:1456-1463): no fusing into the first subtraction
#pragma clang fp contract(off)
  static_assert(NT == 2 || NT == 3, "two or three bf16 terms");
  const int t = opaque_tid(), c = t >> 1, s = t & 1, jb = 16 * s, j0 = HALF * hf + jb;
  uint32_t ku[8], eu[8];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const uint4 kr = *(const uint4*)&sh.op[0][c][jb + 8 * x];
    const uint4 er = *(const uint4*)&sh.op[1][c][jb + 8 * x];
    ku[4 * x] = kr.x; ku[4 * x + 1] = kr.y; ku[4 * x + 2] = kr.z; ku[4 * x + 3] = kr.w;
    eu[4 * x] = er.x; eu[4 * x + 1] = er.y; eu[4 * x + 2] = er.z; eu[4 * x + 3] = er.w;
  }
  float d = dcar, dn = dcar;                          // lane 0: dcar times lane 1's 16 decays, last first
#pragma unroll
  for (int x = 7; x >= 0; --x) {
    const uint32_t en = (uint32_t)__builtin_amdgcn_mov_dpp((int)eu[x], 0xf5, 0xf, 0xf, true);  // quad_perm [1,1,3,3]
    dn = hmul<1>(en, dn);
    dn = hmul<0>(en, dn);
  }
  if (s == 0) d = dn;
  // no branch per entry: rows >= h hold decay 1 (d passes unchanged) and take zero operands.  A word (two entries) at
  // a time, newest first: its weights read from LDS, its terms formed by one packed conversion each (each half read
  // back with a shift or a mask: the same roundings as entry by entry) and written back over its raw key and decay
  // words at once (both are in registers already)
#pragma unroll
  for (int x = 7; x >= 0; --x) {
    const float2 w2 = *(const float2*)&sh.w[j0 + 2 * x];
    const float kdo = bf_hi(ku[x]) * (w2.y * d);
    const float ro = j0 + 2 * x + 1 < h ? kdo : 0.f;
    d = hmul<1>(eu[x], d);
    const float kde = bf_lo(ku[x]) * (w2.x * d);
    const float re = j0 + 2 * x < h ? kde : 0.f;
    d = hmul<0>(eu[x], d);
    const uint32_t hi = pk_bf16_kept(re, ro);
    const float r1e = re - bf_lo(hi), r1o = ro - bf_hi(hi);
    *(uint32_t*)&sh.op[0][c][jb + 2 * x] = hi;
    if constexpr (NT == 3) {
      const uint32_t mid = pk_bf16_kept(r1e, r1o);
      *(uint32_t*)&sh.op[1][c][jb + 2 * x] = mid;
      lo3[x] = pk_bf16(r1e - bf_lo(mid), r1o - bf_hi(mid));
    } else {
      *(uint32_t*)&sh.op[1][c][jb + 2 * x] = pk_bf16(r1e, r1o);
    }
  }
  return dpp<0xa0>(d);                                // quad_perm [0,0,2,2]: lane 0's D below its entries, to both
}
// acc[c][v] += sum_j A[c][j] (B1[v][j] + B2[v][j]) over one staged half (bf16 operands, fp32 accumulate): the hi and lo
// passes with the A fragments loaded once and the next pair of B fragments requested before the current pair's MFMAs
// (each accumulator takes its hi term, then its lo term; 124 -> 112 VGPRs in the one-launch decode, flush 194 -> 191
// us at config 3)
__device__ __forceinline__ void rebuild_half4x2(Tile4& t, const bf16_t (*A)[OPS4], const bf16_t (*B1)[OPS4],
                                                const bf16_t (*B2)[OPS4]) {
  const int l = lane_id(), w = wave_id(), q = l >> 4;
  bf16x8 af[2];
#pragma unroll
  for (int g = 0; g < 2; ++g) af[g] = *(const bf16x8*)&A[32 * w + 16 * g + (l & 15)][8 * q];
  auto ld = [&](int it, bf16x8& b0, bf16x8& b1) {
    const bf16_t (*B)[OPS4] = (it & 1) ? B2 : B1;
    const int n2 = 2 * (it >> 1);
    b0 = *(const bf16x8*)&B[16 * n2 + (l & 15)][8 * q];
    b1 = *(const bf16x8*)&B[16 * n2 + 16 + (l & 15)][8 * q];
  };
  bf16x8 c0, c1;
  ld(0, c0, c1);
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    bf16x8 n0, n1;
    if (it + 1 < 8) ld(it + 1, n0, n1);
    const int n2 = 2 * (it >> 1);
#pragma unroll
    for (int g = 0; g < 2; ++g) t.a[g][n2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[g], c0, t.a[g][n2], 0, 0, 0);
#pragma unroll
    for (int g = 0; g < 2; ++g) t.a[g][n2 + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[g], c1, t.a[g][n2 + 1], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (it + 1 < 8) { c0 = n0; c1 = n1; }
  }
}
// KDA: acc[c][v] += sum_j (A1[c][j] + A2[c][j]) B[v][j] over one staged half (the hi / lo decayed key operands
// against u): both A fragments loaded once, each B pair once, the next pair requested before the current MFMAs; each
// accumulator takes its hi term, then its lo term
__device__ __forceinline__ void rebuild_half4x2a(Tile4& t, const bf16_t (*A1)[OPS4], const bf16_t (*A2)[OPS4],
                                                 const bf16_t (*B)[OPS4]) {
  const int l = lane_id(), w = wave_id(), q = l >> 4;
  bf16x8 a1[2], a2[2];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    a1[g] = *(const bf16x8*)&A1[32 * w + 16 * g + (l & 15)][8 * q];
    a2[g] = *(const bf16x8*)&A2[32 * w + 16 * g + (l & 15)][8 * q];
  }
  auto ld = [&](int n2, bf16x8& b0, bf16x8& b1) {
    b0 = *(const bf16x8*)&B[16 * n2 + (l & 15)][8 * q];
    b1 = *(const bf16x8*)&B[16 * n2 + 16 + (l & 15)][8 * q];
  };
  bf16x8 c0, c1;
  ld(0, c0, c1);
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    bf16x8 n0, n1;
    if (it + 1 < 4) ld(2 * it + 2, n0, n1);
    const int n2 = 2 * it;
#pragma unroll
    for (int g = 0; g < 2; ++g) t.a[g][n2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[g], c0, t.a[g][n2], 0, 0, 0);
#pragma unroll
    for (int g = 0; g < 2; ++g) t.a[g][n2 + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[g], c1, t.a[g][n2 + 1], 0, 0, 0);
#pragma unroll
    for (int g = 0; g < 2; ++g) t.a[g][n2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2[g], c0, t.a[g][n2], 0, 0, 0);
#pragma unroll
    for (int g = 0; g < 2; ++g) t.a[g][n2 + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2[g], c1, t.a[g][n2 + 1], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (it + 1 < 4) { c0 = n0; c1 = n1; }
  }
}
// acc[c][v] += sum_j A[c][j] B[v][j] over one staged half, one bf16 term (the prefill dequant's third key term)
__device__ __forceinline__ void rebuild_half4x1(Tile4& t, const bf16_t (*A)[OPS4], const bf16_t (*B)[OPS4]) {
  const int l = lane_id(), w = wave_id(), q = l >> 4;
  bf16x8 af[2];
#pragma unroll
  for (int g = 0; g < 2; ++g) af[g] = *(const bf16x8*)&A[32 * w + 16 * g + (l & 15)][8 * q];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const bf16x8 b = *(const bf16x8*)&B[16 * nt + (l & 15)][8 * q];
#pragma unroll
    for (int g = 0; g < 2; ++g) t.a[g][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[g], b, t.a[g][nt], 0, 0, 0);
  }
}
// the 16 code words of the lane's tile entries, wds[g][nt] = Sq[16 nt + l16][32 w + 16 g + 4 q .. + 3] (zero past a
// K_ x V_ < 128 x 128 head's rows / columns).  128 x 128: 16-byte loads, then a transpose across the lane groups.  Load
// k of lane (q, l16) takes Sq[16 (2 k + (q >> 1)) + l16][32 w + 16 (q & 1) .. + 15], so that one wave instruction
// covers the wave's 32 bytes of 32 rows (dword loads straight into the layout touch 16 rows for 256 bytes, and the
// tile load measured 10.3k -> 9.6k cycles per head this way at config 3); word j of lane group q's run is the word
// lane group j needs, so a 4 x 4 transpose over the lane groups (two swap32, two swap16) delivers it.
template <int K_, int V_>
__device__ __forceinline__ void load_code_words4(uint32_t wds[2][8], const int8_t* Sq) {
  const int l = lane_id(), w = wave_id(), q = l >> 4;
  if constexpr (K_ == KD && V_ == VD) {
    const int l16 = l & 15;
    uint4 x[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      x[k] = *(const uint4*)(Sq + (16 * (2 * k + (q >> 1)) + l16) * KD + 32 * w + 16 * (q & 1));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t a0 = x[k].x, a1 = x[k].y, a2 = x[k].z, a3 = x[k].w;
      swap32(a0, a2);
      swap32(a1, a3);
      swap16(a0, a1);
      swap16(a2, a3);
      wds[0][2 * k] = a0;                             // lane group 0's run: g = 0, nt = 2 k
      wds[1][2 * k] = a1;                             // group 1: g = 1, nt = 2 k
      wds[0][2 * k + 1] = a2;                         // group 2: g = 0, nt = 2 k + 1
      wds[1][2 * k + 1] = a3;                         // group 3: g = 1, nt = 2 k + 1
    }
    return;
  }
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int c = 32 * w + 16 * g + 4 * q;
    const bool cok = K_ == KD || c < K_;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int v = 16 * nt + (l & 15);
      const uint32_t x = *(const uint32_t*)(Sq + (V_ == VD ? v : min(v, V_ - 1)) * K_ + (K_ == KD ? c : min(c, K_ - 4)));
      wds[g][nt] = (cok && (V_ == VD || v < V_)) ? x : 0u;
    }
  }
}
// t += codes x svr[v] x skl[c], each term rounded to fp32 before the add (after the window products; see flush_head)
__device__ __forceinline__ void tile_add_words4(Tile4& t, const uint32_t wds[2][8], const float* svr,
                                                const float* skl) {
#pragma clang fp contract(off)
  const int l = lane_id(), w = wave_id(), q = l >> 4;
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int c0 = 32 * w + 16 * g + 4 * q;
    float kc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) kc[i] = skl[c0 + i];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const float rv = svr[16 * nt + (l & 15)];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        t.a[g][nt][i] = t.a[g][nt][i] + ((float)(int)(int8_t)(wds[g][nt] >> (8 * i)) * rv) * kc[i];
    }
  }
}
// M[a][r] = acc[a] of lane r (the 4 x 4 corner of a 16 x 16 MFMA result) in every lane: lanes 0-3 write their
// columns to the wave's LDS words and every lane reads the four columns back (same-address reads are broadcasts), LDS
// instructions where sixteen readlanes were VALU ones
template <bool CF>
__device__ __forceinline__ void bcast4x4(const FlushShared4T<CF>& sh, const f32x4& acc, float M[4][4]) {
  const int l = lane_id();
  f32x4* mb = const_cast<f32x4*>(sh.r.mb[wave_id()]);
  if (l < 4) mb[l] = acc;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const f32x4 x = mb[r];
#pragma unroll
    for (int a = 0; a < 4; ++a) M[a][r] = x[a];
  }
}
// M[a][r] = sum_v Q_old[v][a] Q[v][r] (Q from sh.qT): every lane gets all 16 entries
template <bool CF>
__device__ __forceinline__ void gram_qold_q(const FlushShared4T<CF>& sh, float M[4][4]) {
  const int l = lane_id(), q = l >> 4, l16 = l & 15;
  f32x4 macc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const f16x8 ao = *(const f16x8*)&sh.r.qoT[l16 & 3][32 * ks + 8 * q];       // rows / columns >= 4: unused
    const f16x8 bq = *(const f16x8*)&sh.qT[l16 & 3][32 * ks + 8 * q];
    macc = mma32(ao, bq, macc);
  }
  bcast4x4(sh, macc, M);
}
// P = B^T Q + pn U_old (Q_old^T Q) for the wave's two channel groups, fp16-rounded (kernels.py:1580-1700): lane
// (q, l16) returns P[32 w + 16 g + l16][0..3] for g = q >> 1 (zero for r >= R).  The contraction runs over v, so each
// block of B is transposed (one exact MFMA against the identity: lane l then holds
// B[32 w + 16 g + (l & 15)][16 nt + 4 (l >> 4) + i]); the first call (TR) forms the transposed blocks into bt, the
// second (the U step) reads them from there.  The A operand's rows m >= 4 repeat rows m mod 4, so every lane group
// holds the same rows of P^T: the lane groups 0-1 finish channel group 0 and 2-3 group 1, each correction once per
// lane instead of both groups in every lane (the same values).
template <bool TR, bool CF>
__device__ __forceinline__ void p_step4(const FlushShared4T<CF>& sh, const f16x4 (&bh)[2][8], f16x4 (&bt)[2][8], float pn,
                                        int R, f32x4& pg) {
  const int l = lane_id(), w = wave_id(), q = l >> 4, l16 = l & 15;
  float M[4][4];
  gram_qold_q(sh, M);
  f16x4 ident;
#pragma unroll
  for (int i = 0; i < 4; ++i) ident[i] = (4 * q + i == l16) ? (_Float16)1.0f : (_Float16)0.0f;
  f32x4 pacc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {                    // P^T[r][c] = sum_v Q^T[r][v] B[c][v] (k = v)
    const f16x4 aq = *(const f16x4*)&sh.qT[l16 & 3][16 * nt + 4 * q];          // rows >= 4 of P^T: unused
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      if constexpr (TR) bt[g][nt] = pinned(to_h4(mma16(bh[g][nt], ident, f32x4{0.f, 0.f, 0.f, 0.f})));
      pacc[g] = mma16(aq, bt[g][nt], pacc[g]);
    }
  }
  const bool g1 = q >= 2;
  const f32x4 uo = sh.uoc[32 * w + 16 * (g1 ? 1 : 0) + l16];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float pa = g1 ? pacc[1][r] : pacc[0][r];
    const float corr = uo[0] * M[0][r] + uo[1] * M[1][r] + uo[2] * M[2][r] + uo[3] * M[3][r];
    pg[r] = r < R ? hround(pa + pn * corr) : 0.f;
  }
}

template <int K_ = KD, int V_ = VD, bool CF = true, bool KDA = false>
__device__ void flush_head4(FlushShared4T<CF>& sh, const lq_state& st, const float* __restrict__ Q0, int slot, int hv,
                            float qmax, int* sched = nullptr) {
  static_assert(!KDA || (K_ == KD && V_ == VD), "KDA heads are 128 x 128");
  const int HV = st.HV, L = st.L, R = st.R;
  const long long sh_ = (long long)slot * HV + hv;
  const int tid = opaque_tid(), l = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), q = l >> 4, l16 = l & 15;
  char* base = block_base(st, slot, hv);
  int8_t* Sq = (int8_t*)base;
  float* Sk = (float*)(base + V_ * K_);
  float* Sv = Sk + K_;
  f16_t* UQ = (f16_t*)(Sv + V_);
  const bool two = L > HALF;                          // window halves
  // the half staged first: KDA stages the newest half first (its decayed keys carry the later decays down)
  const int hA = KDA && two ? 1 : 0;

  // ---- stage 1: every load of the head up front ----
  float pn = 1.f, rpn = 1.f;                          // KDA: the decay lives in Pbuf per channel, pn = 1
  if constexpr (!KDA) {
    pn = fmaxf(st.Pbuf[sh_], LQ_PNMIN);               // kernels.py:1471
    rpn = 1.0f / pn;                                  // kernels.py:1477
  }
  const int cv = tid & 127;                           // column (tid < 128) or row of the stage-1 loads
  const bool colt = tid < KD;
  const int nc = colt ? K_ : V_;
  const bool cok = (K_ == KD && V_ == VD) || cv < nc;
  const int cvc = (K_ == KD && V_ == VD) ? cv : min(cv, nc - 1);
  const int vq = V_ == VD ? cv : min(cv, V_ - 1);
  const float scv = cok ? (colt ? Sk[cvc] : Sv[cvc]) : 0.f;
  float uqv[4], q0v[4];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const float x = h2f(UQ[min(a, R - 1) * (K_ + V_) + (colt ? 0 : K_) + cvc]);
    uqv[a] = cok ? x : 0.f;
    const float y = Q0[vq * R + min(a, R - 1)];
    q0v[a] = (V_ == VD || cv < V_) ? y : 0.f;
  }
  const float pbc = KDA ? st.Pbuf[sh_ * KD + cv] : 0.f;
  const float wv = st.Wbuf[sh_ * L + min(tid, L - 1)];
  WinHalf win;
  load_half<K_, V_, KDA>(win, st, slot, hv, L, hA);
  uint32_t wds[2][8];                                 // loaded after the first window half's products

  if (colt) {
    const float pcv = KDA ? expf(pbc) : 1.f;                                           // kernels.py:1451
    sh.skl[cv] = KDA ? scv * pcv : scv;                                               // kernels.py:1519
    f32x4 u;
#pragma unroll
    for (int a = 0; a < 4; ++a) u[a] = a < R ? (KDA ? hround(uqv[a] * pcv) : uqv[a]) : 0.f;   // kernels.py:1464-1465
    sh.uoc[cv] = u;
  } else {
    sh.svr[cv] = scv * (pn / qmax);                                                   // kernels.py:1483
    f32x4 o;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      o[a] = a < R ? uqv[a] : 0.f;
      sh.qT[a][cv] = f2h(a < R ? hround(q0v[a]) : 0.f);                             // kernels.py:1573-1577
    }
    sh.qov[cv] = o;
  }
  if (tid < LPMAX) sh.w[tid] = tid < L ? wv : 0.f;
  __syncthreads();

  // ---- stage 2: B = deq(S0) pn + window, fp16 (kernels.py:1483-1571); the window half by half ----
  f16x4 bh[2][8];                                     // B packed, fp16 (tile layout, k = c for the MFMAs)
  {
    Tile4 t;
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) t.a[g][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float dcar = 1.f;                                 // KDA: the decay product carried down from the newer half
    auto rebuild = [&](int hf) {
      if constexpr (KDA) {
        dcar = kda_key_scan4(sh, dcar, L, hf);
        __syncthreads();
        rebuild_half4x2a(t, sh.op[0], sh.op[1], sh.op[2]);
      } else {
        rebuild_half4x2(t, sh.op[0], sh.op[1], sh.op[2]);
      }
    };
    store_half<KDA>(sh, win, L, hA);
    // the second half's rows are requested as soon as the first half's are in LDS, and the code words after the first
    // half's products, so that each load's latency overlaps a half's products (holding the code words from stage 1
    // as well would take the registers past 128)
    if (two) load_half<K_, V_, KDA>(win, st, slot, hv, L, 1 - hA);
    __syncthreads();
    rebuild(hA);
    load_code_words4<K_, V_>(wds, Sq);
    if (two) {
      __syncthreads();                                // every wave is past the first half's operands
      store_half<KDA>(sh, win, L, 1 - hA);
      __syncthreads();
      rebuild(1 - hA);
    }
    tile_add_words4(t, wds, sh.svr, sh.skl);
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) bh[g][nt] = pinned(to_h4(t.a[g][nt]));   // the fp16 rounding of B
  }
  __syncthreads();                                    // every wave is past the rebuild: the operand region is free
  if (colt) {
#pragma unroll
    for (int a = 0; a < 4; ++a) sh.r.uoT[a][cv] = f2h(sh.uoc[cv][a]);
  } else {
#pragma unroll
    for (int a = 0; a < 4; ++a) sh.r.qoT[a][cv] = f2h(sh.qov[cv][a]);
    sh.r.qo16[cv] = to_h4(sh.qov[cv]);
  }
  __syncthreads();

  // ---- stage 3: subspace iteration (ITERS = 1) with the algebraic rank-R corrections (kernels.py:1580-1842) ----
  f32x4 p16;
  f16x4 bt[2][8];                                     // B^T blocks, formed by the first P step
  p_step4<true>(sh, bh, bt, pn, R, p16);              // P16 rows of channel group q >> 1 of this wave's channels
  if ((q & 1) == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) sh.r.ppT[r][32 * w + 8 * q + l16] = f2h(p16[r]);
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  {                                                   // Q^T partial over the wave's 32 channels
    f16x4 ap[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) ap[g] = *(const f16x4*)&sh.r.ppT[l16 & 3][32 * w + 16 * g + 4 * q];   // rows >= 4: unused
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      f32x4 d = mma16(ap[0], bh[0][nt], f32x4{0.f, 0.f, 0.f, 0.f});
      d = mma16(ap[1], bh[1][nt], d);
      if (q == 0) sh.r.qpart[w][16 * nt + l16] = d;
    }
  }
  __syncthreads();
  if (tid < VD) {                                     // waves 0 and 1: one row v per thread
    // M2[a][r] = sum_c U_old[c][a] P16[c][r] over all 128 channels
    f32x4 macc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const f16x8 ao = *(const f16x8*)&sh.r.uoT[l16 & 3][32 * ks + 8 * q];     // rows / columns >= 4: unused
      const f16x8 bp = *(const f16x8*)&sh.r.ppT[l16 & 3][32 * ks + 8 * q];
      macc = mma32(ao, bp, macc);
    }
    float M2[4][4];
    bcast4x4(sh, macc, M2);
    const int v = tid;
    f32x4 s = sh.r.qpart[0][v];
#pragma unroll
    for (int w2 = 1; w2 < NW4; ++w2) s += sh.r.qpart[w2][v];
    const f32x4 qo = sh.qov[v];
#pragma unroll
    for (int r = 0; r < 4; ++r) s[r] += pn * (qo[0] * M2[0][r] + qo[1] * M2[1][r] + qo[2] * M2[2][r] + qo[3] * M2[3][r]);
    sh.qv[v] = s;
  }
  __syncthreads();
  if (w == 0) {                                       // CholeskyQR2, fp16 Q (kernels.py:1778-1835)
    __builtin_amdgcn_s_setprio(3);
    f32x4 p0 = sh.qv[l], p1 = sh.qv[l + 64];
#pragma unroll
    for (int r = 0; r < 4; ++r) { if (r >= R) { p0[r] = 0.f; p1[r] = 0.f; } }
    cholqr_pass(p0, p1);
    cholqr_pass(p0, p1);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p0[r] = r < R ? hround(p0[r]) : 0.f;
      p1[r] = r < R ? hround(p1[r]) : 0.f;
      sh.qT[r][l] = f2h(p0[r]);
      sh.qT[r][l + 64] = f2h(p1[r]);
    }
    sh.qv[l] = p0;
    sh.qv[l + 64] = p1;
    sh.r.qn16[l] = to_h4(p0);
    sh.r.qn16[l + 64] = to_h4(p1);
    __builtin_amdgcn_s_setprio(0);
  }
  __syncthreads();
  f32x4 u16g;
  p_step4<false>(sh, bh, bt, pn, R, u16g);            // U16 = P step with Q16 (channel group q >> 1)
  if constexpr (K_ == KD && V_ == VD) {               // U16^T to LDS (P16^T is read no more) for the factor stores
    if ((q & 1) == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) sh.r.ppT[r][32 * w + 8 * q + l16] = f2h(u16g[r]);
    }
  }
  // -U16 of both channel groups in the lanes l < 16 (the residual's A operand): group 1 from lane l + 32
  f16x4 nu16[2];
  {
    const uint2 x = h4_words(to_h4(-u16g));
    uint32_t a0 = x.x, b0 = x.x, a1 = x.y, b1 = x.y;
    swap32(a0, b0);                                   // b0, b1 of lanes 0-31: the words of lanes 32-63
    swap32(a1, b1);
    nu16[0] = __builtin_bit_cast(f16x4, x);
    nu16[1] = __builtin_bit_cast(f16x4, make_uint2(b0, b1));
  }

  // ---- stage 4: residual E = fp16(pn (B / pn + Q_old U_old^T) - Q U^T) (kernels.py:1888-1928) ----
  // E is kept packed (fp16, in B's registers: B is dead after the U step); the products B / pn, E rsk and the |E| sums
  // take its halves through v_fma_mix_f32, each the single rounding of the widen-then-operate form.
  {
    const f16x4 z4 = {};
    f16x4 auo[2], aun[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      auo[g] = q == 0 ? to_h4(sh.uoc[32 * w + 16 * g + l16]) : z4;                  // A[c][a] = U_old
      aun[g] = q == 0 ? nu16[g] : z4;                                               // A[c][r] = -U16
    }
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int v = 16 * nt + l16;
      // B[a][v] = Q_old^T, B[r][v] = Q16^T; rows a, r >= 4 (lanes q > 0) meet the zero columns of A
      const f16x4 bqo = sh.r.qo16[v];
      const f16x4 bqn = sh.r.qn16[v];
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const f16x4 b = bh[g][nt];
        f32x4 e = KDA ? from_h4(b) : f32x4{h4mul<0>(b, rpn), h4mul<1>(b, rpn), h4mul<2>(b, rpn), h4mul<3>(b, rpn)};
        e = mma16(auo[g], bqo, e);
        if constexpr (!KDA) e *= pn;
        e = mma16(aun[g], bqn, e);
        bh[g][nt] = to_h4(e);                                                       // E, fp16
      }
    }
  }

  // ---- stage 5: column smoothing scales (kernels.py:1929-1958) ----
  float rsk[2][4];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    float cs[4], x0 = 0.f, x1 = 0.f, x2 = 0.f, x3 = 0.f;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      x0 = h4abs_add<0>(bh[g][nt], x0);
      x1 = h4abs_add<1>(bh[g][nt], x1);
      x2 = h4abs_add<2>(bh[g][nt], x2);
      x3 = h4abs_add<3>(bh[g][nt], x3);
    }
    cs[0] = sum16(x0);
    cs[1] = sum16(x1);
    cs[2] = sum16(x2);
    cs[3] = sum16(x3);
    // the square root and division once per column: lane l takes column 4 q + (l & 3) of its row group
    const int ic = l & 3;
    const float msum = (ic == 0 ? cs[0] : ic == 1 ? cs[1] : ic == 2 ? cs[2] : cs[3]) * (1.0f / V_);
    const float sq = sqrtf(msum);
    const float rs = fminf(1.0f / sq, 1.0f / LQ_EPS);
    const int cc = 32 * w + 16 * g + 4 * q + l16;
    if (l16 < 4 && (K_ == KD || cc < K_)) Sk[cc] = fmaxf(sq, LQ_EPS);
    rsk[g][0] = dpp<0x00>(rs);                        // quad_perm [i, i, i, i]: column i of the lane's quad
    rsk[g][1] = dpp<0x55>(rs);
    rsk[g][2] = dpp<0xaa>(rs);
    rsk[g][3] = dpp<0xff>(rs);
  }
  int next = 0;                                       // dynamic schedule: this workgroup's next candidate
  if (sched && tid == 0) next = sched_take(sched);
  // ---- stage 6: row scales and codes (kernels.py:1974-2009) ----
  Tile4 t;                                            // E rsk, fp32
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    float m = 0.f;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const f16x4 e = bh[g][nt];
      t.a[g][nt] = f32x4{h4mul<0>(e, rsk[g][0]), h4mul<1>(e, rsk[g][1]), h4mul<2>(e, rsk[g][2]),
                         h4mul<3>(e, rsk[g][3])};
#pragma unroll
      for (int i = 0; i < 4; ++i) m = fmaxf(m, fabsf(t.a[g][nt][i]));
    }
    sh.r.rmx[4 * w + q][16 * nt + l16] = m;
  }
  __syncthreads();
  if (tid < VD) {
    float m = sh.r.rmx[0][tid];
#pragma unroll
    for (int k = 1; k < 4 * NW4; ++k) m = fmaxf(m, sh.r.rmx[k][tid]);
    const float rmax = fmaxf(m, LQ_EPS);
    if (V_ == VD || tid < V_) Sv[tid] = rmax;
    sh.r.rq[tid] = qmax * (1.0f / rmax);
  }
  __syncthreads();
  uint32_t cw[2][8];                                  // code words, laid out as load_code_words4 delivers them
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const int v = 16 * nt + l16;
    const float rq = sh.r.rq[v];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      uint32_t b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) b[i] = __float_as_uint(__builtin_fmaf(t.a[g][nt][i], rq, 12582912.0f));   // RNE via 1.5 2^23
      const uint32_t lo = __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u), hi = __builtin_amdgcn_perm(b[3], b[2], 0x0c0c0400u);
      cw[g][nt] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    }
  }
  if constexpr (K_ == KD && V_ == VD) {
    // the inverse of load_code_words4's transpose, then four 16-byte stores per lane (each wave instruction 32 rows x
    // 32 bytes) instead of sixteen 4-byte ones
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t a0 = cw[0][2 * k], a1 = cw[1][2 * k], a2 = cw[0][2 * k + 1], a3 = cw[1][2 * k + 1];
      swap16(a0, a1);
      swap16(a2, a3);
      swap32(a0, a2);
      swap32(a1, a3);
      *(uint4*)(Sq + (16 * (2 * k + (q >> 1)) + l16) * KD + 32 * w + 16 * (q & 1)) = make_uint4(a0, a1, a2, a3);
    }
  } else {
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int v = 16 * nt + l16;
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int c = 32 * w + 16 * g + 4 * q;
        if ((K_ == KD || c < K_) && (V_ == VD || v < V_)) *(uint32_t*)(Sq + v * K_ + c) = cw[g][nt];
      }
    }
  }
  // ---- stage 7: factors, window reset (kernels.py:1836-1842, 2014-2025) ----
  if constexpr (K_ == KD && V_ == VD) {
    // the factor rows [U_r | Q_r] from their fp16 tables (U16^T above, Q16^T from the CholeskyQR): thread t writes
    // halfs 4 (t % 64) .. + 3 of row t / 64, one 8-byte store each, where per-lane 2-byte stores took twelve
    // instructions a wave
    const int r = tid >> 6, c4 = 4 * (tid & 63);
    if (r < R) {
      const uint2 x = c4 < KD ? *(const uint2*)&sh.r.ppT[r][c4] : *(const uint2*)&sh.qT[r][c4 - KD];
      *(uint2*)&UQ[r * (KD + VD) + c4] = x;
    }
  } else {
    if ((q & 1) == 0) {
      const int c = 32 * w + 8 * q + l16;
      if (c < K_)
        for (int r = 0; r < R; ++r) UQ[r * (K_ + V_) + c] = f2h(u16g[r]);
    }
    if (tid < V_) {
      for (int r = 0; r < R; ++r) UQ[r * (K_ + V_) + K_ + tid] = f2h(sh.qv[tid][r]);
    }
  }
  if constexpr (KDA) {
    if (tid < KD) st.Pbuf[sh_ * KD + tid] = 0.f;
    uint4* Gb = (uint4*)((f16_t*)st.Gbuf + sh_ * L * KD);                             // fp16 1.0 over the window
    for (int i = tid; i < L * KD / 8; i += FT4) Gb[i] = make_uint4(0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u);
  }
  if (tid < L) st.Wbuf[sh_ * L + tid] = 0.f;
  if (tid == 0) {
    if constexpr (!KDA) st.Pbuf[sh_] = 1.f;
    st.hcnt[sh_] = 0;
    if (sched) sh.due = (unsigned long long)sched_candidate(take_result(next));
  }
  __syncthreads();                                    // LDS reuse by the next head of this workgroup
}

}  // namespace lqf
}  // namespace
