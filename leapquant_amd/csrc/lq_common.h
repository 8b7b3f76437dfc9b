// Shared device helpers of liblq (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lq.h"

#define LQ_QMAX 127.0f
#define LQ_EPS 1e-12f              // kernels.py:23
#define LQ_SOFTPLUS_THRESHOLD 20.0 // kernels.py:21
#define LQ_PNMIN 1e-20f            // kernels.py:1078
#define LQ_NORM_EPS 1e-6           // kernels.py:246-247
// largest ranks R of GDN 128 x 128 heads: the step (and the quantize / dequant that build and read its checkpoints)
// R <= 16, the flush R <= 8 (kernels.py:63, 1091); KDA and 64-dim heads R <= 4
#define LQ_STEP_RMAX 16
#define LQ_FLUSH_RMAX 8

typedef uint16_t bf16_t;   // bfloat16 bits
typedef uint16_t f16_t;    // IEEE half bits

// ---- scalar conversions ----------------------------------------------------------------------------------------
__device__ __forceinline__ float bf2f(bf16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// fp32 -> bf16 / fp16, round to nearest even: the gfx950 conversions v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32
typedef __bf16 lq_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }
// two values in one word: lo in bits 0-15, hi in bits 16-31
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, lq_bf16x2{(__bf16)lo, (__bf16)hi});
}
// the same, the word kept as computed: a half of it read back (bf_lo / bf_hi) then costs one shift or mask, where the
// compiler would otherwise convert that value again on its own
__device__ __forceinline__ uint32_t pk_bf16_kept(float lo, float hi) {
  uint32_t w = pk_bf16(lo, hi);
  asm("" : "+v"(w));
  return w;
}
// bf16 halves of a word as fp32
// x, or zero where !ok, word by word: a select of whole uint4 values can be lowered through a private array indexed
// at run time (scratch memory), which a mask on each word never is
__device__ __forceinline__ uint4 keep4(uint4 x, bool ok) {
  const uint32_t m = ok ? 0xffffffffu : 0u;
  return make_uint4(x.x & m, x.y & m, x.z & m, x.w & m);
}
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bfround(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ float h2f(f16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ f16_t f2h(float f) { return __builtin_bit_cast(f16_t, (_Float16)f); }
__device__ __forceinline__ float hround(float f) { return (float)(_Float16)f; }

// ---- wave64 lane exchange (DPP: fused into the consuming VALU op, no LDS traffic) -------------------------------
// Every pattern used here (quad_perm, row_mirror, row_half_mirror) reads a lane of the same row, so every lane has a
// source: bound_ctrl only tells the compiler that no old value is needed (no move to initialise the destination).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}
#define DPP_XOR1 0xb1          // quad_perm [1,0,3,2]
#define DPP_XOR2 0x4e          // quad_perm [2,3,0,1]
#define DPP_HALF_MIRROR 0x141  // lane i <- lane 7-i within each 8-lane half row
#define DPP_MIRROR 0x140       // lane i <- lane 15-i within each 16-lane row

// all-reduce over the 8 lanes 8m..8m+7
__device__ __forceinline__ float sum8(float x) {
  x += dpp<DPP_XOR1>(x);
  x += dpp<DPP_XOR2>(x);
  x += dpp<DPP_HALF_MIRROR>(x);
  return x;
}
__device__ __forceinline__ float max8(float x) {
  x = fmaxf(x, dpp<DPP_XOR1>(x));
  x = fmaxf(x, dpp<DPP_XOR2>(x));
  x = fmaxf(x, dpp<DPP_HALF_MIRROR>(x));
  return x;
}
// all-reduce over the 16 lanes of a DPP row
__device__ __forceinline__ float sum16(float x) {
  x = sum8(x);
  x += dpp<DPP_MIRROR>(x);
  return x;
}
__device__ __forceinline__ float max16(float x) {
  x = max8(x);
  x = fmaxf(x, dpp<DPP_MIRROR>(x));
  return x;
}
// Lanes l and l ^ 16 (l ^ 32) through v_permlane16_swap (v_permlane32_swap), gfx950: a VALU exchange instead of
// __shfl_xor's LDS-crossbar permute.  With both operands x, the two halves returned are x[l] and x[l ^ 16] (x[l ^ 32])
// in some order, so the sum / max equals x + __shfl_xor(x, 16) bit for bit.
__device__ __forceinline__ float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// all-reduce over the wave
__device__ __forceinline__ float sum64(float x) { return xor32_sum(xor16_sum(sum16(x))); }
__device__ __forceinline__ float max64(float x) { return xor32_max(xor16_max(max16(x))); }

// the same exchanges on fp64 values (both 32-bit halves moved by the same lane pattern)
template <int CTRL>
__device__ __forceinline__ double dppd(double x) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, x);
  const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)u, CTRL, 0xf, 0xf, false);
  const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(u >> 32), CTRL, 0xf, 0xf, false);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ double join_d(unsigned lo, unsigned hi) {
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ double sum64d(double x) {
  x += dppd<DPP_XOR1>(x);
  x += dppd<DPP_XOR2>(x);
  x += dppd<DPP_HALF_MIRROR>(x);
  x += dppd<DPP_MIRROR>(x);
  unsigned long long u = __builtin_bit_cast(unsigned long long, x);
  auto l16 = __builtin_amdgcn_permlane16_swap((unsigned)u, (unsigned)u, false, false);
  auto h16 = __builtin_amdgcn_permlane16_swap((unsigned)(u >> 32), (unsigned)(u >> 32), false, false);
  x = join_d(l16[0], h16[0]) + join_d(l16[1], h16[1]);
  u = __builtin_bit_cast(unsigned long long, x);
  auto l32 = __builtin_amdgcn_permlane32_swap((unsigned)u, (unsigned)u, false, false);
  auto h32 = __builtin_amdgcn_permlane32_swap((unsigned)(u >> 32), (unsigned)(u >> 32), false, false);
  return join_d(l32[0], h32[0]) + join_d(l32[1], h32[1]);
}

// ---- gates (scalar, per (row, head) or per channel); evaluated in fp64 and rounded once ----------------------------
__device__ __forceinline__ double softplus20(double x) {
  return x <= LQ_SOFTPLUS_THRESHOLD ? log1p(exp(x)) : x;
}
// GDN decay alpha = exp(-exp(A_log) softplus(a + dt_bias))  (kernels.py:141-143)
__device__ __forceinline__ float gdn_alpha(float a, float dtb, float alog) {
  double xg = (double)(a + dtb);
  return (float)exp(-exp((double)alog) * softplus20(xg));
}
// beta = f32(bf16(sigmoid(f32(b))))  (kernels.py:144)
__device__ __forceinline__ float beta_of(float b) {
  return bfround((float)(1.0 / (1.0 + exp(-(double)b))));
}
__device__ __forceinline__ float rsqrt_rn(double x) { return (float)(1.0 / sqrt(x)); }

// fp32 versions for the per-(row, head) and per-channel gates of the decode steps (<= 2 ulp of the fp64 forms)
// branch-free (a branch here makes the compiler's wait-count analysis wait for every load in flight at the join)
__device__ __forceinline__ float softplus20f(float x) {
  const float t = log1pf(expf(fminf(x, (float)LQ_SOFTPLUS_THRESHOLD)));
  return x <= (float)LQ_SOFTPLUS_THRESHOLD ? t : x;
}
__device__ __forceinline__ float gdn_alpha_f(float a, float dtb, float alog) {
  return expf(-expf(alog) * softplus20f(a + dtb));
}
__device__ __forceinline__ float beta_f(float b) { return bfround(1.0f / (1.0f + expf(-b))); }
__device__ __forceinline__ float rsqrtf_rn(float x) { return 1.0f / sqrtf(x); }

// ---- direct global -> LDS loads (gfx950 global_load_lds_dwordx4): lane l's 16 bytes land at lds_wave_base + 16 l ----
// Issued through inline asm: the compiler's own form makes every such load wait for all loads in flight (it cannot
// tell that successive loads write disjoint LDS).  The caller waits (s_waitcnt vmcnt) before reading the LDS data.
// Nothing else in these kernels keeps a value in M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_load16(const void* gsrc, void* lds_wave_base) {
  const unsigned lds = (unsigned)(size_t)(__attribute__((address_space(3))) char*)(char*)lds_wave_base;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(gsrc), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop
// Loads of data that a launch reads once and that no other workgroup of the launch reads (the steps' int8 tiles and
// buffered keys, the KDA step's window keys and values): non-temporal, so that they stream through L2 / MALL without
// displacing what is still to be read.  Measured at config 1 (GDN step 17.1 -> 16.2 us) and config 2 (KDA step 47.3
// -> 45.5 us).  The direct-to-LDS loads (GDN window rows, KDA factor rows and decays) measured faster without the hint
// (GDN 15.98 -> 15.86 us, KDA 45.1 -> 44.1 us).  Not for data two
// workgroups share (the flush reads a key head's window from each of its value heads' workgroups: 92 -> 100 us with
// the hint), and not for the 64-dim GDN tiles (measured slightly slower).
template <typename T>
__device__ __forceinline__ T ld_once(const T* p) { return __builtin_nontemporal_load(p); }

// ---- depthwise causal conv1d update (lq_conv, W = 4) ----------------------------------------------------------
// Conv taps of one channel (lq_conv, W = 4): the raw projection x, the slot's three state taps and the four weights.
struct ConvTaps {
  bf16_t x, s[3];
  uint2 w;                  // four bf16 weights
  bf16_t b;
};
__device__ __forceinline__ ConvTaps conv_taps(const lq_conv& cv, const bf16_t* xrow, long long sbase, int ch) {
  ConvTaps t;
  const bf16_t* S = (const bf16_t*)cv.state + sbase + (long long)ch * cv.ch_stride;
  t.x = xrow[ch];
#pragma unroll
  for (int i = 0; i < 3; ++i) t.s[i] = S[i * cv.tap_stride];
  t.w = ((const uint2*)cv.weight)[ch];
  t.b = cv.bias ? ((const bf16_t*)cv.bias)[ch] : (bf16_t)0;
  return t;
}
// mixed[c] = bf16(act(w0 s0 + w1 s1 + w2 s2 + w3 x + bias)): products and sums rounded one at a time, left to right
__device__ __forceinline__ float conv_out(const ConvTaps& t, bool silu) {
#pragma clang fp contract(off)                        // __fmul_rn / __fadd_rn are plain * / +: keep them unfused
  const float w[4] = {bf_lo(t.w.x), bf_hi(t.w.x), bf_lo(t.w.y), bf_hi(t.w.y)};
  float y = __fmul_rn(w[0], bf2f(t.s[0]));
  y = __fadd_rn(y, __fmul_rn(w[1], bf2f(t.s[1])));
  y = __fadd_rn(y, __fmul_rn(w[2], bf2f(t.s[2])));
  y = __fadd_rn(y, __fmul_rn(w[3], bf2f(t.x)));
  y = __fadd_rn(y, bf2f(t.b));
  if (silu) y = y / (1.0f + expf(-y));
  return bfround(y);
}
__device__ __forceinline__ void conv_shift(const lq_conv& cv, long long sbase, int ch, const ConvTaps& t) {
  bf16_t* S = (bf16_t*)cv.state + sbase + (long long)ch * cv.ch_stride;
  S[0] = t.s[1];
  S[cv.tap_stride] = t.s[2];
  S[2 * cv.tap_stride] = t.x;
}

// ---- due flag (lq_state.ctl[0]): set by a step that fills a head's window, cleared by the flush ----------------------
// All heads made due in one call write the same word; a load first keeps the writes to the few that find it clear (the
// writes of every head at once serialise at the memory side and stall the whole launch).
__device__ __forceinline__ void mark_due(int* ctl) {
  if (ctl && __hip_atomic_load(ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0)
    __hip_atomic_fetch_or(ctl, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- due list (lq_decode_noalloc): {count of due heads, flush workgroups done, list of p = n HV + hv} -------------
// A step that fills a head's window (or meets a full one) appends the head instead of raising the due flag; the flush
// then takes exactly the listed heads.  Appends past the list's capacity are dropped: such a head stays full and the
// next step of its row lists it again.
#define LQ_DUE_MAX 65536
__device__ __forceinline__ void note_due(int* ctl, int* dlist, int p) {
  if (dlist) {
    const int i = __hip_atomic_fetch_add(dlist, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (i < LQ_DUE_MAX) dlist[2 + i] = p;
  } else {
    mark_due(ctl);
  }
}

// The window buffers are read by 16-byte loads and direct-to-LDS loads of whole rows: their bases must be 16-byte
// aligned (rows are K or V bf16 long, multiples of 16 bytes).  torch's allocations are; a view at an odd offset is not.
__host__ __device__ inline bool buffers_aligned(const lq_state* st) {
  const uintptr_t m = (uintptr_t)st->Kbuf | (uintptr_t)st->Ubuf | (uintptr_t)st->Gbuf;
  return (m & 15) == 0;
}

// code range of the stored checkpoint (lq_state.qmax; 0: INT8)
__device__ __forceinline__ float code_range(const lq_state& st) { return st.qmax > 0.f ? st.qmax : LQ_QMAX; }

// ---- state-block addressing (state.py:29-40) ----------------------------------------------------------------------
__device__ __forceinline__ char* block_base(const lq_state& st, int slot, int hv) {
  return (char*)st.ssm + 4ll * ((long long)slot * st.slot_stride + (long long)hv * st.V * st.K);
}

// ---- checks and launches shared by the entry points of different source files (not exported) ----------------------
// the argument checks of lq_gdn_step / lq_kda_step (the KDA step also needs Gbuf and K = V = 128) and of lq_flush
__attribute__((visibility("hidden"))) int lq_check_step(const lq_state* st, const lq_step_io* io);
__attribute__((visibility("hidden"))) int lq_check_flush(const lq_state* st, const float* Q0, const int* idx, int N,
                                                         int kda, float qmax);
// the four-wave prefill dequant of GDN 128 x 128 heads at R <= 4 (lq_dequant.hip); arguments checked by lq_dequant
__attribute__((visibility("hidden"))) int lq_launch_dequant4(const lq_state* st, const int* idx, int N, float qmax,
                                                             hipStream_t s);
// the four-wave prefill dequant of KDA heads (lq_dequant.hip); arguments checked by lq_kda_dequant
__attribute__((visibility("hidden"))) int lq_launch_kda_dequant4(const lq_state* st, const int* idx, int N, float qmax,
                                                                 hipStream_t s);
// decode step of every row of io (GDN or KDA), due heads signalled through dlist when it is set (else st->ctl)
__attribute__((visibility("hidden"))) int lq_launch_step(const lq_state* st, const lq_step_io* io, int kda, float glb,
                                                         int* dlist, hipStream_t s);
// flush of the due heads: the listed ones when dlist is set (the list is then reset), else found by the scan
__attribute__((visibility("hidden"))) int lq_launch_flush(const lq_state* st, const float* Q0, const int* idx, int N,
                                                          int kda, float qmax, int* dlist, hipStream_t s);
