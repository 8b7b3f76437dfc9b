// GDN / KDA decode step on the INT8 checkpoint + window buffer (gfx950).
//
// Semantics follow /root/reference/leapquant/kernels.py:27-692 (GDN) and 694-1075 (KDA); the layout of the checkpoint
// and of the window buffer is described in include/lq.h.
//
// Mapping (MI355X-first, not the reference's persistent TMA/mbarrier pipeline): one workgroup per (row n, key head hk),
// the G = HV / H value heads sharing the key head's q, k and buffered keys in the same workgroup, so the buffered keys
// are read once per key head and only the h valid window rows are read.
//   * GDN: V / 64 waves per value head; every dot product on the matrix cores (int8 MFMA for the two GEMVs against
//     the int8 tile, bf16 / fp16 MFMA for the window-key and factor dots), fed by 16-byte loads issued up front.
//   * KDA (K = V = 128): two waves per value head, the same matrix-core dots, the per-channel gate folded into the
//     key operands and the window's decayed keys formed by a backward scan split between the two waves.
#include "lq_flush_core.h"

namespace {

constexpr int KD = 128;   // key dim
constexpr int VD = 128;   // value dim
constexpr int LMAX = 64;  // largest window the kernels are built for

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// kf / qf as three signed int8 digits of a 24-bit fixed-point value relative to the vector's max:
// X = rint(x / max * 127 * 2^16) = d0 2^16 + d1 2^8 + d2, |d0| <= 127, d1, d2 in [-128, 127].
constexpr float DIGIT_SCALE = 127.0f * 65536.0f;
__device__ __forceinline__ void digits3(float x, float rmax, int8_t& d0, int8_t& d1, int8_t& d2) {
  const int X = (int)rintf((x * rmax) * DIGIT_SCALE);
  const int e2 = (int)(int8_t)(X & 0xff);
  const int X1 = (X - e2) >> 8;
  const int e1 = (int)(int8_t)(X1 & 0xff);
  d0 = (int8_t)((X1 - e1) >> 8);
  d1 = (int8_t)e1;
  d2 = (int8_t)e2;
}
// DPP row shifts (within 16 lanes): lane i reads lane i - s
template <int S>
__device__ __forceinline__ float row_shr(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x110 + S, 0xf, 0xf, false));
}
// DPP quad broadcast of lane k of each quad
template <int K>
__device__ __forceinline__ float quad_bcast(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), K * 0x55, 0xf, 0xf, false));
}
// a bulk load with or without the non-temporal hint
template <bool NT, typename T>
__device__ __forceinline__ T ld_nt(const T* p) {
  if constexpr (NT) return ld_once(p);
  else return *p;
}
constexpr float KSPLIT = 64.0f;   // kn / qn scaled by 2^6 before the fp16 hi / lo split (keeps the lo part normal)

// The MFMA B-operand tables (dig, bkq, hkq) are read as 16-byte fragments of up to six rows at once: their rows are
// padded by 16 bytes so that those rows start in different LDS banks (unpadded, 128- or 256-byte rows all start in
// the same bank).
constexpr int DIGP = 16, OPP = 8;
template <int K_, int V_, int G, int RM>
struct StepShared {
  bf16_t ub[G][LMAX][V_];  // the window's u_j rows per value head (direct global -> LDS loads)
  int8_t dig[G][6][K_ + DIGP];   // int8 GEMV B operand: k digits 0-2, q digits 0-2
  bf16_t bkq[6][K_ + OPP];       // key-dot B operand: bf16 hi / mid / lo of kn, then of qn
  f16_t hkq[4][K_ + OPP];        // factor-dot B operand: fp16 hi / lo of 64 kn, then of 64 qn
  float2 mq[G][V_];        // GEMV rows (k, q) in digit units
  float2 cwq[G][LMAX];     // (w_j dk_j, w_j dq_j) per value head: buffered entry j's coefficients in A4 / A5
  float2 duq[G][RM];       // (dU_r, dQ_r) per value head, factor r
  float w[G][LMAX];        // gated entry weights w_j per value head
  float sc[G][8];          // per value head: alpha, beta, kappa, kmax, qmax
};

// ------------------------------------------------------------------------------------------------------------------
// GDN step  (kernels.py:129-144 gate / beta, 236-279 norms and weights, 380-585 stream, dots and appends)
//
// One workgroup per (row n, key head hk) with two waves per value head g (step_wph); wave (g, wi) owns tile rows
// RW wi .. RW wi + RW - 1, RW = V / 2.  Head dims (K, V) = (128, 128), (64, 128), (64, 64) (kernels.py:62): K sets the
// lanes' channel count in the scalar work and the k-steps of every MFMA, V the rows per wave.
// Every dot product runs on the matrix cores:
//   * m = deq(Sq) kn, y = deq(Sq) qn: the int8 tile goes from HBM straight into the A operand of
//     v_mfma_i32_16x16x64_i8; B holds kf = kn Sk / 127 and qf = qn Sk / 127 as three int8 digits each (24-bit fixed
//     point relative to max |kf|, max |qf|), so both GEMVs accumulate exactly in int32;
//   * dk_j = K_j kn, dq_j = K_j qn: bf16 MFMA with kn, qn split in three bf16 terms (products exact, fp32 sums);
//   * dU_r = U^T_r kn, dQ_r = U^T_r qn: fp16 MFMA with 64 kn, 64 qn split in two fp16 terms.
// The per-head scalar work (norms, gate, beta, digits) runs in one wave per value head.  The window's u_j rows reach
// LDS by direct global -> LDS loads.  <= 128 VGPRs and < 40 KiB LDS: four workgroups per CU, the whole B = 64 x H = 16
// grid resident at once.
// FL (fused flush, K = V = 128 and G = 2 only): after its step the workgroup flushes the heads whose window it has just
// filled (or found full), with the four-wave flush of lq_flush_core.h over the same 256 threads -- one launch per decode
// call instead of two.  The step's LDS and the flush's share the same bytes (both fit the 40 KiB that four workgroups
// per CU allow).
// ------------------------------------------------------------------------------------------------------------------
// waves per value head of the step: V / 64, and two at V = 64 (each wave then owns 32 rows of the tile), so that a
// 64-row head's bytes are requested by as many waves as a 128-row head's
template <int V_>
constexpr int step_wph() { return V_ == 64 ? 2 : V_ / 64; }

template <int K_, int V_, int G, bool FL, int RM>
struct StepLds {
  StepShared<K_, V_, G, RM> st;
};
template <int K_, int V_, int G, int RM>
struct StepLds<K_, V_, G, true, RM> {
  union {
    StepShared<K_, V_, G, RM> st;
    lqf::FlushShared4T<true> fl;
  };
};

// RM: factors held per head.  4 (R <= 4): the G R <= 16 factor rows of the workgroup's heads are one MFMA tile, taken
// by the last wave.  16 (the rank ablation R <= 16, K = V = 128; kernels.py:63, 457-469): up to G tiles, tile g taken
// by the second wave of head g.
template <int K_, int V_, int G, bool CONV, bool FL, int RM = 4, bool DF = false>
__global__ __launch_bounds__(64 * step_wph<V_>() * G) __attribute__((amdgpu_waves_per_eu(4)))
void gdn_step_kernel(lq_state st, lq_step_io io, lq_conv cv, int* dlist, const float* Q0) {
  static_assert(!DF || FL, "deferred flush (lq_gdn_decode_deferred): the fused decode kernel");
  static_assert(!FL || (K_ == 128 && V_ == 128 && G == 2), "fused flush: the four-wave layout, 128 x 128 heads");
  static_assert(RM == 4 || (RM == 16 && K_ == 128 && V_ == 128 && !FL), "ranks above 4: 128 x 128 heads, no fused flush");
  constexpr int KD = K_, VD = V_;
  constexpr int WPH = step_wph<V_>();   // waves per value head
  constexpr int RW = VD / WPH;          // tile rows per wave
  constexpr int NE = KD / 64;   // channels per lane in the scalar work
  constexpr int KS32 = KD / 32, KS64 = KD / 64;   // k-steps of the 16x16x32 (bf16 / fp16) and 16x16x64 (int8) MFMAs
  constexpr bool NT = KD == 128;                  // non-temporal bulk loads (see ld_once)
  __shared__ StepLds<K_, V_, G, FL, RM> lds;
  StepShared<K_, V_, G, RM>& sh = lds.st;
  const int H = st.H, HV = st.HV, L = st.L, R = st.R;
  const int n = blockIdx.x / H;
  const int hk = blockIdx.x - n * H;
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave in the workgroup
  const int g = wv / WPH;       // value head of this wave within the key head
  const int wi = wv % WPH;      // its tile part: rows RW wi ..
  const int lane = tid & 63;
  // the row this thread owns in the output phase; at V = 64 lanes RW .. 63 repeat the wave's rows and store nothing
  const int lt = RW == 64 ? tid & (VD - 1) : RW * wi + (lane & (RW - 1));
  const bool rowl = RW == 64 || lane < RW;
  const int n16 = lane & 15, q4 = lane >> 4;                 // MFMA lane coordinates
  const int hv = hk * G + g;
  const long long MIX = 2ll * H * KD + (long long)HV * VD;
  bf16_t* out = (bf16_t*)io.out + ((long long)n * HV + hv) * VD;

  if constexpr (DF) {
    // deferred flush (lq_gdn_decode_deferred): a head that the previous call left full is flushed first, on this
    // workgroup's threads, before anything of the step is loaded (so that no loaded value waits across the flush; the
    // cost is the slot index and the fills read before the row's inputs are requested)
    const int slot0 = io.idx[n];
    if (slot0 > 0 && slot0 < st.NS && !(CONV && slot0 >= cv.NS)) {
      unsigned pend = 0;
#pragma unroll
      for (int g2 = 0; g2 < G; ++g2) pend |= (st.hcnt[(long long)slot0 * HV + hk * G + g2] >= L ? 1u : 0u) << g2;
      if (pend) {
        const float qm = code_range(st);
#pragma unroll
        for (int g2 = 0; g2 < G; ++g2)
          if ((pend >> g2) & 1u) lqf::flush_head4<128, 128, true>(lds.fl, st, Q0, slot0, hk * G + g2, qm);
      }
    }
  }
  // The row's own inputs (q, k, v, gate) do not depend on its slot: requested before the slot index, so that their
  // latency overlaps its load (a padding row reads them too and ignores them).
  const bf16_t* mrow = (const bf16_t*)io.mixed + (long long)n * MIX;
  bf16_t kxr[NE], qxr[NE];
  if (!CONV) {
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const int c = lane + 64 * e;
      kxr[e] = mrow[H * KD + hk * KD + c];
      qxr[e] = mrow[hk * KD + c];
    }
  }
  const bf16_t araw = ((const bf16_t*)io.a)[(long long)n * HV + hv];
  const bf16_t braw = ((const bf16_t*)io.b)[(long long)n * HV + hv];
  const float dtb = io.dt_bias[hv], alog = io.A_log[hv];
  float vin = 0.f;
  if (!CONV) vin = bf2f(mrow[2ll * H * KD + hv * VD + lt]);

  const int slot = io.idx[n];
  // padding row (kernels.py:374-378); a slot outside the cache (or, fused conv, outside the conv state) counts as one
  if (slot <= 0 || slot >= st.NS || (CONV && slot >= cv.NS)) {
    if (rowl) out[lt] = 0;
    return;
  }
  // Every load below is unconditional (clamped addresses) and none sits in a divergent block: a load whose result is
  // merged at the end of an exec-masked block makes the compiler wait for ALL loads in flight, the tile included.
  // Order: the scalar work's operands, then the int8 tile, then the window.  Loads return in order, so the per-head
  // scalar work overlaps the tile's transfer.
  const char* base = block_base(st, slot, hv);
  const float* Skp = (const float*)(base + VD * KD);
  const float* Svp = Skp + KD;
  const f16_t* UQp = (const f16_t*)(Svp + VD);
  const long long sh_ = (long long)slot * HV + hv;
  float* Wp = st.Wbuf + sh_ * L;
  float skx[NE], wx[NE];
  ConvTaps ktap[NE], qtap[NE], vtap;  // CONV: taps of the key / query channels c and of the value channel lt
  const long long cvb = CONV ? (long long)slot * cv.slot_stride : 0;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const int c = lane + 64 * e;
    skx[e] = Skp[c];
    wx[e] = Wp[min(c, L - 1)];
  }
  // factor rows U^T (fp16) of all G heads: A fragment rows m = g2 R + r of the factor-dot MFMA, tile ft of them
  f16x8 ufr[KS32];
  const int ft = RM == 4 ? 0 : g;
  const bool fwave = RM == 4 ? wv == WPH * G - 1 : (wi == WPH - 1 && 16 * g < G * R);
  {
    const int m = 16 * ft + n16 < G * R ? 16 * ft + n16 : 0, g2 = m / R, r = m - g2 * R;
    const f16_t* U = (const f16_t*)(block_base(st, slot, hk * G + g2) + VD * KD + 4 * (KD + VD)) + r * (KD + VD);
#pragma unroll
    for (int ks = 0; ks < KS32; ++ks) ufr[ks] = *(const f16x8*)(U + 32 * ks + 8 * q4);
  }
  if (CONV) vtap = conv_taps(cv, mrow, cvb, 2 * H * KD + hv * VD + lt);
  const float sv = Svp[lt];
  float qt[RM];                 // Q^T[r][lt]
#pragma unroll
  for (int r = 0; r < RM; ++r) qt[r] = h2f(UQp[min(r, R - 1) * (KD + VD) + KD + lt]);
  const float P = st.Pbuf[sh_];
  // Window fills of the G value heads: uniform loads, served by the scalar data cache.  A vector load here would queue
  // behind the bulk loads the CU's other workgroups have issued, and every later load of this workgroup waits for it.
  int hg[G];
#pragma unroll
  for (int g2 = 0; g2 < G; ++g2) hg[g2] = st.hcnt[(long long)slot * HV + hk * G + g2];
  __builtin_amdgcn_sched_barrier(0);
  // ---- per value head scalar work, one wave (wi = 0), before the window fills arrive: gate, beta, norms, digits,
  //      key-dot operands.  Its global writes (key append, gated weights) wait until the end, so that nothing joins
  //      the window / tile loads in the vector memory counter before the window's wait ----
  bf16_t kapp[NE] = {};
  float wjv[NE] = {};
  uint32_t kpk[2 * NE] = {}, qpk[2 * NE] = {};   // CONV: key / query state after the shift
  // GL: the gate (alpha, beta) and the gated weights w_j on the head's second wave once its bulk loads are issued, so
  // that the first wave, which holds its own bulk loads until its scalar work is done, has less of it (64-dim heads:
  // (64, 64) step 7.45 -> 7.20 us, (64, 128) 8.71 -> 8.62 us; at K = 128 the decode measured no faster)
  constexpr bool GL = KD == 64;
  if (wi == 0) {
    float alpha = 0.f, beta = 0.f;
    if constexpr (!GL) {
      alpha = gdn_alpha_f(bf2f(araw), dtb, alog);
      beta = beta_f(bf2f(braw));
    }
    if (CONV) {                 // the key / query taps: loaded by the scalar-work waves only (the other waves skip them)
#pragma unroll
      for (int e = 0; e < NE; ++e) {
        ktap[e] = conv_taps(cv, mrow, cvb, H * KD + hk * KD + lane + 64 * e);
        qtap[e] = conv_taps(cv, mrow, cvb, hk * KD + lane + 64 * e);
      }
#pragma unroll
      for (int e = 0; e < NE; ++e) {
        kxr[e] = f2bf(conv_out(ktap[e], cv.silu));
        qxr[e] = f2bf(conv_out(qtap[e], cv.silu));
        kpk[e] = ktap[e].s[1] | ((uint32_t)ktap[e].s[2] << 16);   // the shifted taps (s1, s2 | x)
        kpk[NE + e] = ktap[e].x;
        qpk[e] = qtap[e].s[1] | ((uint32_t)qtap[e].s[2] << 16);
        qpk[NE + e] = qtap[e].x;
      }
    }
    float kx[NE], qx[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) { kx[e] = bf2f(kxr[e]); qx[e] = bf2f(qxr[e]); }
    float nq = qx[0] * qx[0], nk = kx[0] * kx[0], nkq = kx[0] * qx[0];
#pragma unroll
    for (int e = 1; e < NE; ++e) { nq = fmaf(qx[e], qx[e], nq); nk = fmaf(kx[e], kx[e], nk); nkq = fmaf(kx[e], qx[e], nkq); }
    nq = sum64(nq); nk = sum64(nk); nkq = sum64(nkq);
    const float inq = rsqrtf_rn(nq + (float)LQ_NORM_EPS) * io.scale;
    const float ink = rsqrtf_rn(nk + (float)LQ_NORM_EPS);
    const float kappa = nkq * inq * ink;
    const float inv = 1.0f / code_range(st);   // codes Sq dequantise as Sq Sk Sv / qmax (kernels.py:255-256)
    float kn[NE], qn[NE], kf[NE], qf[NE];
    float kmax = 0.f, qmax = 0.f;
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      kn[e] = kx[e] * ink;
      qn[e] = qx[e] * inq;
      kf[e] = (kn[e] * skx[e]) * inv;          // kernels.py:255-256
      qf[e] = (qn[e] * skx[e]) * inv;
      kmax = fmaxf(kmax, fabsf(kf[e]));
      qmax = fmaxf(qmax, fabsf(qf[e]));
    }
    kmax = fmaxf(max64(kmax), 1e-30f);
    qmax = fmaxf(max64(qmax), 1e-30f);
    const float rk = 1.0f / kmax, rq = 1.0f / qmax;
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const int c = lane + 64 * e;
      int8_t d0, d1, d2;
      digits3(kf[e], rk, d0, d1, d2);
      sh.dig[g][0][c] = d0; sh.dig[g][1][c] = d1; sh.dig[g][2][c] = d2;
      digits3(qf[e], rq, d0, d1, d2);
      sh.dig[g][3][c] = d0; sh.dig[g][4][c] = d1; sh.dig[g][5][c] = d2;
      if (g == 0) {
        // key-dot operands: x = hi + mid + lo exactly representable sums of bf16 (products with bf16 keys exact)
        const float xs[2] = {kn[e], qn[e]};
#pragma unroll
        for (int v2 = 0; v2 < 2; ++v2) {
#pragma clang fp contract(off)                        // split of the rounded kn / qn: no fusing of x = k / |k| into x - hi
          const float x = xs[v2];
          const bf16_t hi = f2bf(x);
          const float r1 = x - bf2f(hi);
          const bf16_t mid = f2bf(r1);
          const bf16_t lo = f2bf(r1 - bf2f(mid));
          sh.bkq[3 * v2][c] = hi; sh.bkq[3 * v2 + 1][c] = mid; sh.bkq[3 * v2 + 2][c] = lo;
          const float xs64 = x * KSPLIT;
          const f16_t fh = f2h(xs64);
          sh.hkq[2 * v2][c] = fh;
          sh.hkq[2 * v2 + 1][c] = f2h(xs64 - h2f(fh));
        }
        kapp[e] = f2bf(kn[e]);
      }
      if constexpr (!GL) wjv[e] = wx[e] * alpha;   // w_j = Wbuf[j] alpha (kernels.py:270-274), written back at the end
    }
    if (lane == 0) {
      if constexpr (!GL) { sh.sc[g][0] = alpha; sh.sc[g][1] = beta; }
      sh.sc[g][2] = kappa; sh.sc[g][3] = kmax; sh.sc[g][4] = qmax;
    }
  }

  if (CONV) {                   // the value channel lt of this head: conv output and state shift
    vin = conv_out(vtap, cv.silu);
    if (rowl) conv_shift(cv, cvb, 2 * H * KD + hv * VD + lt, vtap);
  }
  // Every wave holds its bulk loads until its own small loads are back.  Under load the memory system serves requests
  // roughly in arrival order, chip-wide: a small load issued after the first bulk loads waits behind them (several
  // us), and the scalar work of the CU's later workgroups, hence their bulk issue, with it.  Waiting here keeps the
  // small loads of the four workgroups of a CU ahead of the bulk traffic (measured 16.09 -> 15.98 us at config 1, GQA
  // 2; GQA 1, four workgroups of two waves per CU as well: 19.85 -> 19.28 us with the plain window loads below).  At GQA
  // 4 two workgroups of eight waves share a CU and the wait measured slower (16.27 -> 16.49 us): not used there.  A
  // workgroup that flushes a head after its step (FL, a window filled here) does not wait: its step then ends a little
  // earlier in its CU's order (staggered windows 33.17 -> 32.99 us per call, deferred 24.04 -> 23.94 us).
  bool flush_after = false;
  if constexpr (FL) {
#pragma unroll
    for (int g2 = 0; g2 < G; ++g2) flush_after = flush_after || hg[g2] >= L - 1;
  }
  if (!CONV && G <= 2 && !flush_after) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  int h = hg[0], hmax = hg[0];
#pragma unroll
  for (int g2 = 1; g2 < G; ++g2) {
    h = g == g2 ? hg[g2] : h;
    hmax = max(hmax, hg[g2]);
  }
  const bool live = h < L;      // a full window is never stepped (the flush follows every step)
  hmax = min(hmax, L);
  if (!GL && wi == 0 && live) {
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const int c = lane + 64 * e;
      if (c < h) sh.w[g][c] = wjv[e];
    }
  }
  // The big loads, in the order the work after them needs them: the window (values u_j into LDS, then the buffered
  // keys), and the int8 tile last.  Everything built on the window -- key dots, A4 / A5 -- runs while the tile still
  // streams; after the tile's last bytes only the GEMV, the delta rule and the stores remain.
  // window values u_j (j < h) straight to LDS, 1 KiB (RPK = 4 rows at V = 128, 8 at V = 64) per wave instruction (the
  // loop holds no compiler-visible load, so it adds no wait); rows past the buffer's last (L not a multiple of RPK)
  // re-read it.  Plain loads: with the non-temporal hint the step measured 15.98 us against 15.86 (config 1).
  {
    constexpr int RPK = 512 / VD, LPR = VD / 8;             // rows per KiB, lanes per row
    const char* ubg = (const char*)((const bf16_t*)st.Ubuf + sh_ * L * VD);
    const int nch = live ? (h + RPK - 1) / RPK : 0;
    for (int c = wi; c < nch; c += WPH) {
      const int row = min(RPK * c + lane / LPR, L - 1);
      lds_load16(ubg + row * (VD * 2) + 16 * (lane % LPR), (char*)&sh.ub[g][0][0] + c * 1024);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // buffered keys: this wave's 16-row tiles of K, A fragments of the key-dot MFMA (rows >= hmax read row 0, unused)
  constexpr int NWV = WPH * G;                              // waves in the workgroup
  constexpr int KT = (4 + NWV - 1) / NWV;                   // 16-row key tiles per wave (64 rows over the waves)
  bf16x8 kfr[KT][KS32];
  {
    const bf16_t* Kb = (const bf16_t*)st.Kbuf + ((long long)slot * H + hk) * L * KD;
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const int j = 16 * (wv + NWV * t) + n16;
      const int jr = j < hmax ? j : 0;
#pragma unroll
      for (int ks = 0; ks < KS32; ++ks) kfr[t][ks] = ld_nt<NT>((const bf16x8*)(Kb + (long long)jr * KD + 32 * ks + 8 * q4));
    }
  }
  i32x4 afr[RW / 16][KS64];     // the int8 tile: A fragments, row RW wi + 16 rt + n16
  {
    const char* rp = base + (RW * wi + n16) * KD + 16 * q4;
#pragma unroll
    for (int rt = 0; rt < RW / 16; ++rt)
#pragma unroll
      for (int ks = 0; ks < KS64; ++ks) afr[rt][ks] = ld_nt<NT>((const i32x4*)(rp + 16 * rt * KD + 64 * ks));
  }
  // vector memory operations issued after the window's LDS loads: the keys and the tile (nothing else until the
  // stores at the end, so this count is exact)
  constexpr int AFTER_WINDOW = KS32 * KT + (RW / 16) * KS64;
  __builtin_amdgcn_sched_barrier(0);
  if (GL && wi == WPH - 1) {
    const float alpha = gdn_alpha_f(bf2f(araw), dtb, alog);
    const float beta = beta_f(bf2f(braw));
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      wjv[e] = wx[e] * alpha;
      const int c = lane + 64 * e;
      if (live && c < h) sh.w[g][c] = wjv[e];
    }
    if (lane == 0) { sh.sc[g][0] = alpha; sh.sc[g][1] = beta; }
  }

  __syncthreads();              // digits, dot operands, scalars and w_j are in LDS (the barrier waits for no global load)
  if (CONV && wv == 0) {        // the key head's conv state shift, once per workgroup, after every wave read its taps
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      bf16_t* Sk_ = (bf16_t*)cv.state + cvb + (long long)(H * KD + hk * KD + lane + 64 * e) * cv.ch_stride;
      bf16_t* Sq_ = (bf16_t*)cv.state + cvb + (long long)(hk * KD + lane + 64 * e) * cv.ch_stride;
      Sk_[0] = (bf16_t)kpk[e];
      Sk_[cv.tap_stride] = (bf16_t)(kpk[e] >> 16);
      Sk_[2 * cv.tap_stride] = (bf16_t)kpk[NE + e];
      Sq_[0] = (bf16_t)qpk[e];
      Sq_[cv.tap_stride] = (bf16_t)(qpk[e] >> 16);
      Sq_[2 * cv.tap_stride] = (bf16_t)qpk[NE + e];
    }
  }

  // ---- buffered-key dots: this wave's K tiles against bf16 (hi, mid, lo) of kn (columns 0-2) and qn (4-6) ----
  {
    bf16x8 bk[KS32];
    const bool bcol = (n16 & 3) < 3 && n16 < 8;
    const int brow = bcol ? (n16 >> 2) * 3 + (n16 & 3) : 0;
#pragma unroll
    for (int ks = 0; ks < KS32; ++ks) {
      const bf16x8 b = *(const bf16x8*)&sh.bkq[brow][32 * ks + 8 * q4];
      bk[ks] = bcol ? b : bf16x8{};
    }
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const int j0 = 16 * (wv + NWV * t);
      if (j0 < hmax) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS32; ++ks) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kfr[t][ks], bk[ks], acc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float s = acc[i] + quad_bcast<1>(acc[i]) + quad_bcast<2>(acc[i]);   // hi + mid + lo (lanes 0 / 4)
          const int j = j0 + 4 * q4 + i;
          if ((n16 == 0 || n16 == 4) && j < hmax) {
#pragma unroll
            for (int g2 = 0; g2 < G; ++g2) ((float*)&sh.cwq[g2][j])[n16 >> 2] = sh.w[g2][j] * s;
          }
        }
      }
    }
  }
  // ---- factor dots (last wave): U^T rows of the G heads against fp16 (hi, lo) of 64 kn (columns 0, 1), 64 qn (2, 3) ----
  if (fwave) {
    f16x8 bh[KS32];
    const bool bcol = n16 < 4;
#pragma unroll
    for (int ks = 0; ks < KS32; ++ks) {
      const f16x8 b = *(const f16x8*)&sh.hkq[bcol ? n16 : 0][32 * ks + 8 * q4];
      bh[ks] = bcol ? b : f16x8{};
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS32; ++ks) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ufr[ks], bh[ks], acc, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float s = (acc[i] + dpp<DPP_XOR1>(acc[i])) * (1.0f / KSPLIT);               // hi + lo (lanes 0 / 2)
      const int m = 16 * ft + 4 * q4 + i;
      if ((n16 == 0 || n16 == 2) && m < G * R) ((float*)&sh.duq[m / R][m % R])[n16 >> 1] = s;
    }
  }
  // this wave's u_j rows have landed in LDS (they precede the keys and the tile in the counter) ...
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(AFTER_WINDOW) : "memory");
  __syncthreads();              // ... and the other wave's, with the key and factor dots of every wave
  if (!live) {                  // a full window (a flush that did not cover this row): zero output, nothing written;
    if (!FL && lt == 0 && rowl) note_due(st.ctl, dlist, n * HV + hv);   // flag it again so that the flush takes it
    if (rowl) out[lt] = 0;
  } else {
  // ---- row v = lt: buffered entries, rank-R part, delta rule, output and appends (kernels.py:536-585) ----
  const float alpha = sh.sc[g][0], beta = sh.sc[g][1], kappa = sh.sc[g][2];
  float a4 = 0.f, a5 = 0.f;
  int j = 0;
  for (; j + 4 <= h; j += 4) {  // four entries' LDS reads in flight at once; the sums keep the order of j
    float ub[4];
    float2 c[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      ub[e] = bf2f(sh.ub[g][j + e][lt]);
      c[e] = sh.cwq[g][j + e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a4 = fmaf(ub[e], c[e].x, a4);
      a5 = fmaf(ub[e], c[e].y, a5);
    }
  }
  for (; j < h; ++j) {
    const float ub = bf2f(sh.ub[g][j][lt]);
    const float2 c = sh.cwq[g][j];
    a4 = fmaf(ub, c.x, a4);
    a5 = fmaf(ub, c.y, a5);
  }
  float a6 = 0.f, a7 = 0.f;
#pragma unroll
  for (int r = 0; r < RM; ++r) {
    if (r < R) {
      const float2 d = sh.duq[g][r];
      a6 = fmaf(qt[r], d.x, a6);
      a7 = fmaf(qt[r], d.y, a7);
    }
  }
  // ---- int8 GEMV on the matrix cores (the tile is the last data to arrive).  B columns: 0 / 4 / 8 = k digits 0 / 1 / 2, 1 / 5 / 9 = q digits, others 0 ----
  {
    i32x4 bfr[KS64];
    const int drow = (n16 & 3) * 3 + (n16 >> 2);              // table row of column n16 (valid for n16 < 10, n16 & 3 < 2)
    const bool bcol = (n16 & 3) < 2 && n16 < 10;
#pragma unroll
    for (int ks = 0; ks < KS64; ++ks) {
      const i32x4 b = *(const i32x4*)&sh.dig[g][bcol ? drow : 0][64 * ks + 16 * q4];
      bfr[ks] = bcol ? b : i32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int rt = 0; rt < RW / 16; ++rt) {
      i32x4 acc = {0, 0, 0, 0};
#pragma unroll
      for (int ks = 0; ks < KS64; ++ks) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[rt][ks], bfr[ks], acc, 0, 0, 0);
      // lane (n16, q4) holds rows RW wi + 16 rt + 4 q4 + i of column n16; lanes 8 / 9 gather digits 0, 1 from 4, 8 lanes back
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float c0 = (float)acc[i];
        const float tot = fmaf(row_shr<8>(c0), 65536.0f, fmaf(row_shr<4>(c0), 256.0f, c0));
        if (n16 == 8 || n16 == 9) ((float*)&sh.mq[g][RW * wi + 16 * rt + 4 * q4 + i])[n16 - 8] = tot;
      }
    }
  }
  // rows RW wi .. RW wi + RW - 1 of the GEMV are this wave's own rows: LDS round trip within the wave, no barrier
  const float2 mqr = sh.mq[g][lt];
  const float mq = (mqr.x * (sh.sc[g][3] * (1.0f / DIGIT_SCALE))) * sv;
  const float yq = (mqr.y * (sh.sc[g][4] * (1.0f / DIGIT_SCALE))) * sv;
  const float pn = P * alpha;
  const float u = beta * (vin - (pn * (mq + a6) + a4));
  const float y = pn * (yq + a7) + a5 + kappa * u;
  if (rowl) {
    out[lt] = f2bf(y);
    ((bf16_t*)st.Ubuf)[(sh_ * L + h) * VD + lt] = f2bf(u);
  }
  if (lt == 0 && rowl) {
    Wp[h] = 1.0f;
    st.Pbuf[sh_] = pn;
    st.hcnt[sh_] = h + 1;
    if (!FL && h + 1 == L) note_due(st.ctl, dlist, n * HV + hv);   // this head is due: the flush that follows takes it
  }
  if (wi == 0) {
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const int c = lane + 64 * e;
      if (g == 0) ((bf16_t*)st.Kbuf)[(((long long)slot * H + hk) * L + h) * KD + c] = kapp[e];   // key append
      if (!GL && c < h) Wp[c] = wjv[e];
    }
  }
  if (GL && wi == WPH - 1) {
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const int c = lane + 64 * e;
      if (c < h) Wp[c] = wjv[e];
    }
  }
  }  // live
  if constexpr (FL) {
    // the flush of this workgroup's heads whose window is now full (hcnt was L - 1 before the step, or already L):
    // the fills are uniform loads, so every wave takes the same branch and reaches the same barriers
    bool due[G], any = false;
#pragma unroll
    for (int g2 = 0; g2 < G; ++g2) {
      due[g2] = hg[g2] >= L - 1;
      any = any || due[g2];
    }
    if (any) {
      __syncthreads();          // the step is done with the shared bytes, and its appends are visible to the workgroup
      const float qm = code_range(st);
      bool first = true;        // DF: the first due head now, the others at the start of the next call
#pragma unroll
      for (int g2 = 0; g2 < G; ++g2)
        if (due[g2]) {
          if (!DF || first) lqf::flush_head4<128, 128, true>(lds.fl, st, Q0, slot, hk * G + g2, qm);
          else if (tid == 0) note_due(st.ctl, dlist, n * HV + hk * G + g2);   // a standalone flush finds it
          first = false;
        }
    }
  }
}

// ------------------------------------------------------------------------------------------------------------------
// KDA step  (kernels.py:694-1075): per-channel gate; decayed buffered keys; pc folded into the checkpoint operands.
//
// One workgroup of two waves per (row n, value head hv); wave wi owns tile rows 64 wi .. 64 wi + 63.  The window --
// values u_j and keys K_j of the key head in registers, the per-entry step decays e_j in LDS by direct global -> LDS
// loads -- is taken in chunks of up to KCH = 32 entries, newest first (the decay scan runs from the newest entry
// back), so that one chunk is held at a time: 17.7 KiB of LDS and <= 128 VGPRs, eight workgroups per CU (the whole
// window at once needs 26 KiB and 148 VGPRs: six, and the step is bound by the workgroups in flight).  The first
// chunk's loads precede the int8 tile's, so the first scan, the key dots and A4 / A5 run while the tile streams.
//   * gate (kernels.py:704-712, 802, 887-896): g = glb sigmoid(e^A_log (a + dt_bias)) (glb != 0) or
//     -e^A_log softplus(a + dt_bias); gn = P + g, pc = exp(gn), en = exp(g);
//   * m = deq(Sq) diag(pc) kn, y = deq(Sq) diag(pc) qn: int8 MFMA against kf = kn Sk pc / 127, qf = qn Sk pc / 127 as
//     three int8 digits each (kernels.py:900-901);
//   * decayed keys K~_j = bf16(K_j en prod_{j<i<h} e_i) by a backward scan per channel (kernels.py:966-979), then
//     dk_j = w_j K~_j kn, dq_j = w_j K~_j qn on bf16 MFMA (kn, qn in three bf16 terms; kernels.py:1031-1035);
//   * dU_r = U^T_r (pc kn), dQ_r = U^T_r (pc qn) on fp16 MFMA (kernels.py:1036-1047);
//   * u = beta (v - (m + A6 + A4)), y = y_q + A7 + A5 + kappa u (kernels.py:1065-1066).
// ------------------------------------------------------------------------------------------------------------------
constexpr int KCH = 32;             // window entries per chunk

struct KdaShared {
  f16_t gk[KCH][KD];        // a chunk's step decays e_j (row j - cb); the scan overwrites them with K~_j (bf16)
  float2 part[2][VD];       // per wave: (A4, A5) sums of row v over the wave's entries of every chunk
  float2 mq[VD];            // GEMV rows (k, q) in digit units
  float2 cwq[KCH];          // (w_j dk_j, w_j dq_j) of the chunk's entries
  float2 dhand[KD / 2];     // running decay product handed on (wave 1 -> wave 0 -> the next chunk's wave 1), channel
                            // pairs (2 p, 2 p + 1)
  int8_t dig[6][KD];        // int8 GEMV B operand: k digits 0-2, q digits 0-2
  bf16_t bkq[6][KD];        // key-dot B operand: bf16 hi / mid / lo of kn, then of qn
  f16_t hkq[4][KD];         // factor-dot B operand: fp16 hi / lo of 64 pc kn, then of 64 pc qn
  float2 duq[4];            // (dU_r, dQ_r)
  float w[LMAX];            // entry weights w_j = Wbuf[j]
  float sc[8];              // beta, kappa, kmax, qmax
  f16_t uq[4][KD + VD];     // the checkpoint's factor rows (U_r | Q_r), fp16
};

// per-channel gate g (kernels.py:704-712, 802): glb sigmoid(e^A_log (a + dt_bias)) (glb != 0), else -e^A_log softplus.
// The gate's exponentials (here, and the decays e^g and e^gn below) are the hardware's: v_exp_f32 of x log2(e) (HIP's
// __expf), as the reference's __expf (kernels.py:704-707); the softplus keeps log1p, where the reference's
// __logf(1 + e^x) cancels: for gates of 1e-4, e^x ~ 1e-4 and 1 + e^x keeps ~3 of its digits.
__device__ __forceinline__ float softplus20_hx(float x) {
  const float t = log1pf(__expf(fminf(x, (float)LQ_SOFTPLUS_THRESHOLD)));
  return x <= (float)LQ_SOFTPLUS_THRESHOLD ? t : x;
}
__device__ __forceinline__ float kda_gate(float a, float dt, float ea, float glb) {
  const float xg = a + dt;
  return glb != 0.f ? glb / (1.0f + __expf(-ea * xg)) : -ea * softplus20_hx(xg);
}

// Decayed keys K~_j = bf16(K_j dcur), dcur *= e_j, backwards over a wave's cnt <= 16 entries of a chunk, LDS rows
// gb + cnt - 1 .. gb (kernels.py:966-979), for the lane's channel pair (2 lane, 2 lane + 1): raw keys from registers,
// decays read from LDS and overwritten in place by K~.  8 rows per pass, the pass's LDS reads first.
__device__ __forceinline__ void kda_scan_rows(KdaShared& sh, const uint32_t (&kr)[16], int gb, int cnt, int lane,
                                              float& d0, float& d1) {
#pragma unroll
  for (int g8 = 1; g8 >= 0; --g8) {
    if (8 * g8 < cnt) {
      uint32_t ev[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) ev[i] = *(const uint32_t*)&sh.gk[min(gb + 8 * g8 + i, KCH - 1)][2 * lane];
#pragma unroll
      for (int i = 7; i >= 0; --i) {
        const int r = 8 * g8 + i;
        if (r < cnt) {
          *(uint32_t*)&sh.gk[gb + r][2 * lane] = pk_bf16(bf_lo(kr[r]) * d0, bf_hi(kr[r]) * d1);
          d0 = lqf::hmul<0>(ev[i], d0);             // the decays and products are positive: the same bits as cvt + mul
          d1 = lqf::hmul<1>(ev[i], d1);
        }
      }
    }
  }
}

// chunk k of a window of h entries (k = 0 the newest): entries [cb, ce), ce = h - KCH k, cb = max(ce - KCH, 0); wave 0
// takes [cb, cb + c0), wave 1 [cb + c0, ce), c0 a multiple of 4 (or the whole chunk), each at most 16 entries
struct KdaChunk {
  int cb, jb, cnt;          // chunk start; this wave's first entry and entry count
};
__device__ __forceinline__ KdaChunk kda_chunk(int h, int k, int wi) {
  const int ce = h - KCH * k, cb = max(ce - KCH, 0), c = ce - cb;
  const int c0 = min(c, 4 * ((c + 7) >> 3));
  return KdaChunk{cb, wi ? cb + c0 : cb, wi ? c - c0 : c0};
}

__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(4)))
void kda_step_kernel(lq_state st, lq_step_io io, float glb, int* dlist) {
  __shared__ KdaShared sh;
  const int H = st.H, HV = st.HV, L = st.L, R = st.R;
  const int G = HV / H;
  const int n = blockIdx.x / HV;
  const int hv = blockIdx.x - n * HV;
  const int hk = hv / G;
  const int lt = threadIdx.x;
  const int wi = __builtin_amdgcn_readfirstlane(lt >> 6);
  const int lane = lt & 63;
  const int n16 = lane & 15, q4 = lane >> 4;
  const long long MIX = 2ll * H * KD + (long long)HV * VD;
  bf16_t* out = (bf16_t*)io.out + ((long long)n * HV + hv) * VD;
  const int slot = io.idx[n];
  if (slot <= 0 || slot >= st.NS) { out[lt] = 0; return; }   // padding row (kernels.py:374-378)
  const long long sh_ = (long long)slot * HV + hv;
  const char* base = block_base(st, slot, hv);
  const float* Skp = (const float*)(base + VD * KD);
  const float* Svp = Skp + KD;
  const f16_t* UQp = (const f16_t*)(Svp + VD);
  const bf16_t* mrow = (const bf16_t*)io.mixed + (long long)n * MIX;
  // Window fill: a uniform load, served by the scalar data cache (a vector load here would queue behind the bulk loads
  // the CU's other workgroups have issued, and every later load of this workgroup would wait for it).
  const int hfill = st.hcnt[sh_];
  __builtin_amdgcn_sched_barrier(0);
  // per-channel operands: wave 0 (scalar work) channels c = lane, lane + 64; wave 1 (its own gate) c = 2 lane + e
  bf16_t kxr[2], qxr[2], axr[2];
  float skx[2], dtx[2], pbx[2], wx[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int c = lane + 64 * e;
    const int cg = wi ? 2 * lane + e : c;
    kxr[e] = mrow[H * KD + hk * KD + c];
    qxr[e] = mrow[hk * KD + c];
    axr[e] = ((const bf16_t*)io.a)[((long long)n * HV + hv) * KD + cg];
    skx[e] = Skp[c];
    dtx[e] = io.dt_bias[hv * KD + cg];
    pbx[e] = st.Pbuf[sh_ * KD + c];
    wx[e] = st.Wbuf[sh_ * L + min(c, L - 1)];
  }
  const bf16_t braw = ((const bf16_t*)io.b)[(long long)n * HV + hv];
  const float alog = io.A_log[hv];
  const float vin = bf2f(mrow[2ll * H * KD + hv * VD + lt]);
  const float sv = Svp[lt];
  __builtin_amdgcn_sched_barrier(0);
  const int h = hfill;
  if (h >= L) {                 // a full window is never stepped: zero output, and the head is flagged again so that
    if (lt == 0) note_due(st.ctl, dlist, n * HV + hv);   // the flush after this step takes it
    out[lt] = 0;
    return;
  }
  // the four factor rows (2 KiB, inside the checkpoint block whatever R) to LDS, one KiB per wave
  lds_load16((const char*)UQp + 1024 * wi + 16 * lane, (char*)&sh.uq[2 * wi][0]);
  // The window's live entries j < h, chunk by chunk (kda_chunk).  Each wave's decays go straight to its own LDS rows
  // (1 KiB = 4 rows per wave instruction, rows past the buffer's last re-reading it); its values u_j and keys K_j go
  // to registers, a channel pair (2 lane, 2 lane + 1) per lane and row.  The first chunk, then the int8 tile.
  const int nck = (h + KCH - 1) / KCH;
  uint32_t ur[16], kr[16];
  const char* gg = (const char*)((const f16_t*)st.Gbuf + sh_ * L * KD);
  const uint32_t* ug = (const uint32_t*)((const bf16_t*)st.Ubuf + sh_ * L * VD) + lane;
  const uint32_t* kg = (const uint32_t*)((const bf16_t*)st.Kbuf + ((long long)slot * H + hk) * L * KD) + lane;
  auto load_chunk = [&](const KdaChunk& c) {
    for (int r = 0; r < c.cnt; r += 4) {
      const int row = min(c.jb + r + q4, L - 1);
      lds_load16(gg + row * (KD * 2) + 16 * n16, (char*)&sh.gk[c.jb - c.cb + r][0]);
    }
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4)
      if (4 * g4 < c.cnt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ur[4 * g4 + i] = ld_once(ug + (c.jb + min(4 * g4 + i, c.cnt - 1)) * (VD / 2));
      }
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4)
      if (4 * g4 < c.cnt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) kr[4 * g4 + i] = ld_once(kg + (c.jb + min(4 * g4 + i, c.cnt - 1)) * (KD / 2));
      }
  };
  KdaChunk ck = kda_chunk(h, 0, wi);                  // h = 0: no entries
  load_chunk(ck);
  __builtin_amdgcn_sched_barrier(0);
  i32x4 afr[4][2];
  {
    const char* rp = base + (64 * wi + n16) * KD + 16 * q4;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) afr[rt][ks] = ld_once((const i32x4*)(rp + 16 * rt * KD + 64 * ks));
  }
  constexpr int AFTER_WINDOW = 8;   // vector memory operations issued after the first chunk's loads: the tile
  __builtin_amdgcn_sched_barrier(0);
  const float ea = expf(alog);

  // ---- wave 0: per-channel gate, norms, digits, dot operands.  wave 1: its own entries' decayed keys (chunk 0) ----
  float gnv[2] = {0.f, 0.f}, env[2] = {0.f, 0.f};
  if (wi == 0) {
    const float beta = beta_f(bf2f(braw));
    float pcv[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float g = kda_gate(bf2f(axr[e]), dtx[e], ea, glb);
      gnv[e] = pbx[e] + g;
      pcv[e] = __expf(gnv[e]);
      env[e] = __expf(g);
    }
    const float kx[2] = {bf2f(kxr[0]), bf2f(kxr[1])}, qx[2] = {bf2f(qxr[0]), bf2f(qxr[1])};
    float nq = qx[0] * qx[0], nk = kx[0] * kx[0], nkq = kx[0] * qx[0];
    nq = fmaf(qx[1], qx[1], nq); nk = fmaf(kx[1], kx[1], nk); nkq = fmaf(kx[1], qx[1], nkq);
    nq = sum64(nq); nk = sum64(nk); nkq = sum64(nkq);
    const float inq = rsqrtf_rn(nq + (float)LQ_NORM_EPS) * io.scale;
    const float ink = rsqrtf_rn(nk + (float)LQ_NORM_EPS);
    const float kappa = nkq * inq * ink;
    const float inv = 1.0f / code_range(st);   // kernels.py:900-901
    float kn[2], qn[2], kf[2], qf[2];
    float kmax = 0.f, qmax = 0.f;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      kn[e] = kx[e] * ink;
      qn[e] = qx[e] * inq;
      kf[e] = ((kn[e] * skx[e]) * inv) * pcv[e];       // kernels.py:900-901
      qf[e] = ((qn[e] * skx[e]) * inv) * pcv[e];
      kmax = fmaxf(kmax, fabsf(kf[e]));
      qmax = fmaxf(qmax, fabsf(qf[e]));
    }
    kmax = fmaxf(max64(kmax), 1e-30f);
    qmax = fmaxf(max64(qmax), 1e-30f);
    const float rk = 1.0f / kmax, rq = 1.0f / qmax;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int c = lane + 64 * e;
      int8_t d0, d1, d2;
      digits3(kf[e], rk, d0, d1, d2);
      sh.dig[0][c] = d0; sh.dig[1][c] = d1; sh.dig[2][c] = d2;
      digits3(qf[e], rq, d0, d1, d2);
      sh.dig[3][c] = d0; sh.dig[4][c] = d1; sh.dig[5][c] = d2;
      const float xs[2] = {kn[e], qn[e]};
#pragma unroll
      for (int v2 = 0; v2 < 2; ++v2) {
#pragma clang fp contract(off)                        // split of the rounded kn / qn: no fusing of x = k / |k| into x - hi
        const float x = xs[v2];
        const bf16_t hi = f2bf(x);
        const float r1 = x - bf2f(hi);
        const bf16_t mid = f2bf(r1);
        const bf16_t lo = f2bf(r1 - bf2f(mid));
        sh.bkq[3 * v2][c] = hi; sh.bkq[3 * v2 + 1][c] = mid; sh.bkq[3 * v2 + 2][c] = lo;
        const float xs64 = (x * pcv[e]) * KSPLIT;
        const f16_t fh = f2h(xs64);
        sh.hkq[2 * v2][c] = fh;
        sh.hkq[2 * v2 + 1][c] = f2h(xs64 - h2f(fh));
      }
      if (c < L) sh.w[c] = wx[e];
    }
    if (lane == 0) { sh.sc[0] = beta; sh.sc[1] = kappa; sh.sc[2] = kmax; sh.sc[3] = qmax; }
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(AFTER_WINDOW) : "memory");   // own window rows landed
  } else {
    // the scan starts at exp(g) of the channel (the same gate as wave 0's, so the same bits) and runs over wave 1's
    // entries first; the product it reaches is where wave 0's entries continue
    float d0 = __expf(kda_gate(bf2f(axr[0]), dtx[0], ea, glb));
    float d1 = __expf(kda_gate(bf2f(axr[1]), dtx[1], ea, glb));
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(AFTER_WINDOW) : "memory");   // own decay rows in LDS, keys in registers
    kda_scan_rows(sh, kr, ck.jb - ck.cb, ck.cnt, lane, d0, d1);
    sh.dhand[lane] = make_float2(d0, d1);
  }
  __syncthreads();              // gate, digits, dot operands, w_j, factor rows; wave 1's decayed keys and hand-over

  if (wi == 0) {
    float2 d = sh.dhand[lane];
    kda_scan_rows(sh, kr, ck.jb - ck.cb, ck.cnt, lane, d.x, d.y);
    sh.dhand[lane] = d;         // where the next chunk's wave 1 continues (read after the next barrier)
  } else {
    // ---- factor dots: U^T rows against fp16 (hi, lo) of 64 pc kn (columns 0, 1) and 64 pc qn (2, 3) ----
    f16x8 bh[4], ufr[4];        // ufr: A fragment row m = r (U^T_r, fp16)
    const bool bcol = n16 < 4;
    const int r = n16 < R ? n16 : 0;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const f16x8 b = *(const f16x8*)&sh.hkq[bcol ? n16 : 0][32 * ks + 8 * q4];
      bh[ks] = bcol ? b : f16x8{};
      ufr[ks] = *(const f16x8*)&sh.uq[r][32 * ks + 8 * q4];
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ufr[ks], bh[ks], acc, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float s = (acc[i] + dpp<DPP_XOR1>(acc[i])) * (1.0f / KSPLIT);               // hi + lo (lanes 0 / 2)
      const int r = 4 * q4 + i;
      if ((n16 == 0 || n16 == 2) && r < R) ((float*)&sh.duq[r])[n16 >> 1] = s;
    }
  }
  // ---- decayed-key dots and A4 / A5 of this wave's entries of a chunk ----
  bf16x8 bk[4];                 // B operand: columns 0-2 hi / mid / lo of kn, 4-6 of qn
  {
    const bool bcol = (n16 & 3) < 3 && n16 < 8;
    const int brow = bcol ? (n16 >> 2) * 3 + (n16 & 3) : 0;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8 b = *(const bf16x8*)&sh.bkq[brow][32 * ks + 8 * q4];
      bk[ks] = bcol ? b : bf16x8{};
    }
  }
  float a40 = 0.f, a50 = 0.f, a41 = 0.f, a51 = 0.f;   // A4 / A5 of rows v = 2 lane, 2 lane + 1, over the wave's entries
  auto chunk_dots = [&](const KdaChunk& c) {
    // key dots: one 16-row tile of the chunk's LDS rows from the wave's first (rows past its own are not kept)
    const int gb = c.jb - c.cb;
    if (c.cnt > 0) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 a = *(const bf16x8*)((const bf16_t*)&sh.gk[gb + n16][0] + 32 * ks + 8 * q4);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bk[ks], acc, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float s = acc[i] + quad_bcast<1>(acc[i]) + quad_bcast<2>(acc[i]);   // hi + mid + lo (lanes 0 / 4)
        const int jj = 4 * q4 + i;
        if ((n16 == 0 || n16 == 4) && jj < c.cnt) ((float*)&sh.cwq[gb + jj])[n16 >> 2] = sh.w[c.jb + jj] * s;
      }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);   // the wave's own cwq rows: LDS round trip within the wave
    // A4 / A5 over the wave's entries of the chunk, in the order of j
#pragma unroll
    for (int g8 = 0; g8 < 2; ++g8) {
      if (8 * g8 < c.cnt) {
        float2 cc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) cc[i] = sh.cwq[min(gb + 8 * g8 + i, KCH - 1)];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = 8 * g8 + i;
          if (r < c.cnt) {
            const float u0 = bf_lo(ur[r]), u1 = bf_hi(ur[r]);
            a40 = fmaf(u0, cc[i].x, a40); a50 = fmaf(u0, cc[i].y, a50);
            a41 = fmaf(u1, cc[i].x, a41); a51 = fmaf(u1, cc[i].y, a51);
          }
        }
      }
    }
  };
  chunk_dots(ck);
  // ---- older chunks: each wave loads its entries once every wave is done with the previous chunk's rows; wave 1
  //      continues the product wave 0 reached, wave 0 the one wave 1 reaches ----
  for (int k = 1; k < nck; ++k) {
    __syncthreads();            // the previous chunk's decayed keys and cwq are read; wave 0's product is in dhand
    ck = kda_chunk(h, k, wi);
    load_chunk(ck);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this chunk's decay rows in LDS (keys and values with them)
    if (wi == 1) {
      float2 d = sh.dhand[lane];
      kda_scan_rows(sh, kr, ck.jb - ck.cb, ck.cnt, lane, d.x, d.y);
      sh.dhand[lane] = d;
    }
    __syncthreads();            // wave 1's decayed keys and hand-over
    if (wi == 0) {
      float2 d = sh.dhand[lane];
      kda_scan_rows(sh, kr, ck.jb - ck.cb, ck.cnt, lane, d.x, d.y);
      sh.dhand[lane] = d;
    }
    chunk_dots(ck);
  }
  *(float4*)&sh.part[wi][2 * lane] = make_float4(a40, a50, a41, a51);
  {
    i32x4 bfr[2];
    const int drow = (n16 & 3) * 3 + (n16 >> 2);
    const bool bcol = (n16 & 3) < 2 && n16 < 10;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const i32x4 b = *(const i32x4*)&sh.dig[bcol ? drow : 0][64 * ks + 16 * q4];
      bfr[ks] = bcol ? b : i32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      i32x4 acc = {0, 0, 0, 0};
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[rt][0], bfr[0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[rt][1], bfr[1], acc, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float c0 = (float)acc[i];
        const float tot = fmaf(row_shr<8>(c0), 65536.0f, fmaf(row_shr<4>(c0), 256.0f, c0));
        if (n16 == 8 || n16 == 9) ((float*)&sh.mq[64 * wi + 16 * rt + 4 * q4 + i])[n16 - 8] = tot;
      }
    }
  }
  __syncthreads();              // both waves' A4 / A5 sums and the factor dots are in LDS

  // ---- row v = lt: buffered entries, rank-R part, the GEMV and the delta rule ----
  const float2 p0 = sh.part[0][lt], p1 = sh.part[1][lt];
  const float a4 = p0.x + p1.x, a5 = p0.y + p1.y;
  float a6 = 0.f, a7 = 0.f;
  for (int r = 0; r < R; ++r) {
    const float2 d = sh.duq[r];
    const float qt = h2f(sh.uq[r][KD + lt]);
    a6 = fmaf(qt, d.x, a6);
    a7 = fmaf(qt, d.y, a7);
  }
  const float beta = sh.sc[0], kappa = sh.sc[1];
  const float2 mqr = sh.mq[lt];
  const float mq = (mqr.x * (sh.sc[2] * (1.0f / DIGIT_SCALE))) * sv;
  const float yq = (mqr.y * (sh.sc[3] * (1.0f / DIGIT_SCALE))) * sv;
  const float u = beta * (vin - (mq + a6 + a4));        // kernels.py:1065
  const float y = yq + a7 + a5 + kappa * u;             // kernels.py:1066
  out[lt] = f2bf(y);
  ((bf16_t*)st.Ubuf)[(sh_ * L + h) * VD + lt] = f2bf(u);
  if (hv % G == 0) ((bf16_t*)st.Kbuf)[(((long long)slot * H + hk) * L + h) * KD + lt] = sh.bkq[0][lt];   // bf16(kn)
  if (lt == 0) {
    st.Wbuf[sh_ * L + h] = 1.0f;
    st.hcnt[sh_] = h + 1;
    if (h + 1 == L) note_due(st.ctl, dlist, n * HV + hv);   // this head is due: the flush that follows takes it
  }
  if (wi == 0) {                // gate state (kernels.py:895-896)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int c = lane + 64 * e;
      st.Pbuf[sh_ * KD + c] = gnv[e];
      ((f16_t*)st.Gbuf)[(sh_ * L + h) * KD + c] = f2h(env[e]);
    }
  }
}

}  // namespace

// head dims of the GDN step (kernels.py:62); the KDA step is K = V = 128 only (kernels.py:727)
static bool gdn_dims(int K, int V) { return (K == 128 && V == 128) || (K == 64 && (V == 128 || V == 64)); }

int lq_check_step(const lq_state* st, const lq_step_io* io) {
  if (!st || !io) return LQ_ERR_ARG;
  if (!gdn_dims(st->K, st->V) || st->L < 1 || st->L > LMAX || st->R < 1) return LQ_ERR_ARG;
  if (st->R > (st->K == 128 && st->V == 128 ? LQ_STEP_RMAX : 4)) return LQ_ERR_ARG;   // kernels.py:63-64
  if (st->H <= 0 || st->HV <= 0 || st->HV % st->H != 0 || st->NS <= 0 || io->N < 0) return LQ_ERR_ARG;
  if (!st->ssm || !st->Kbuf || !st->Ubuf || !st->Wbuf || !st->Pbuf || !st->hcnt) return LQ_ERR_ARG;
  // 16-byte loads of the int8 rows and of the scale / factor block need a 16-byte aligned block start
  if (st->slot_stride < (long long)st->HV * st->V * st->K || (st->slot_stride & 3) || ((uintptr_t)st->ssm & 15))
    return LQ_ERR_ARG;
  if (!buffers_aligned(st)) return LQ_ERR_ARG;
  if (!(st->qmax == 0.f || (st->qmax >= 1.f && st->qmax <= 127.f))) return LQ_ERR_ARG;
  if (io->N > 0 && (!io->mixed || !io->a || !io->b || !io->A_log || !io->dt_bias || !io->idx || !io->out))
    return LQ_ERR_ARG;
  return LQ_OK;
}

template <int K_, int V_, bool CONV, int RM = 4>
static int launch_gdn(const lq_state* st, const lq_step_io* io, const lq_conv& cv, int* dlist, hipStream_t s) {
  dim3 grid((unsigned)(io->N * st->H));
  switch (st->HV / st->H) {
    case 1: gdn_step_kernel<K_, V_, 1, CONV, false, RM><<<grid, 64 * step_wph<V_>(), 0, s>>>(*st, *io, cv, dlist, nullptr); break;
    case 2: gdn_step_kernel<K_, V_, 2, CONV, false, RM><<<grid, 128 * step_wph<V_>(), 0, s>>>(*st, *io, cv, dlist, nullptr); break;
    case 4: gdn_step_kernel<K_, V_, 4, CONV, false, RM><<<grid, 256 * step_wph<V_>(), 0, s>>>(*st, *io, cv, dlist, nullptr); break;
    default: return LQ_ERR_ARG;
  }
  return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_HIP;
}

template <bool CONV>
static int launch_gdn_dims(const lq_state* st, const lq_step_io* io, const lq_conv& cv, int* dlist, hipStream_t s) {
  if (st->K == 128 && st->R > 4) return launch_gdn<128, 128, CONV, LQ_STEP_RMAX>(st, io, cv, dlist, s);
  if (st->K == 128) return launch_gdn<128, 128, CONV>(st, io, cv, dlist, s);
  return st->V == 128 ? launch_gdn<64, 128, CONV>(st, io, cv, dlist, s) : launch_gdn<64, 64, CONV>(st, io, cv, dlist, s);
}

// the plain GDN / KDA step of every row, arguments already checked
int lq_launch_step(const lq_state* st, const lq_step_io* io, int kda, float glb, int* dlist, hipStream_t s) {
  if (io->N == 0) return LQ_OK;
  if (!kda) {
    const lq_conv none = {};
    return launch_gdn_dims<false>(st, io, none, dlist, s);
  }
  if (st->R > 4) return LQ_ERR_ARG;           // the KDA step holds four factors (kernels.py:1036)
  kda_step_kernel<<<dim3((unsigned)(io->N * st->HV)), 128, 0, s>>>(*st, *io, glb, dlist);
  return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_HIP;
}

extern "C" int lq_gdn_step(const lq_state* st, const lq_step_io* io, void* stream) {
  int rc = lq_check_step(st, io);
  if (rc) return rc;
  return lq_launch_step(st, io, 0, 0.f, nullptr, (hipStream_t)stream);
}

static int check_conv(const lq_state* st, const lq_conv* cv) {
  if (!cv || !cv->state || !cv->weight || cv->W != 4 || (cv->silu != 0 && cv->silu != 1) || cv->NS <= 0)
    return LQ_ERR_ARG;
  const long long C = 2ll * st->H * st->K + (long long)st->HV * st->V;
  if (cv->ch_stride <= 0 || cv->tap_stride <= 0 || cv->slot_stride <= 0) return LQ_ERR_ARG;
  // the state taps of a slot must stay inside its slot_stride elements
  if ((C - 1) * cv->ch_stride + 2 * cv->tap_stride >= cv->slot_stride) return LQ_ERR_ARG;
  if (((uintptr_t)cv->weight & 7) != 0) return LQ_ERR_ARG;
  return LQ_OK;
}

extern "C" int lq_gdn_step_conv(const lq_state* st, const lq_step_io* io, const lq_conv* cv, void* stream) {
  int rc = lq_check_step(st, io);
  if (rc) return rc;
  if ((rc = check_conv(st, cv))) return rc;
  if (io->N == 0) return LQ_OK;
  return launch_gdn_dims<true>(st, io, *cv, nullptr, (hipStream_t)stream);
}

static int gdn_decode(const lq_state* st, const lq_step_io* io, const lq_conv* cv, const float* Q0, bool deferred,
                      hipStream_t s) {
  int rc = lq_check_step(st, io);
  if (rc) return rc;
  if (cv && (rc = check_conv(st, cv))) return rc;
  const float qmax = st->qmax > 0.f ? st->qmax : LQ_QMAX;
  if ((rc = lq_check_flush(st, Q0, io->idx, io->N, 0, qmax))) return rc;
  if (io->N == 0) return LQ_OK;
  if (st->K == 128 && st->V == 128 && st->HV == 2 * st->H && st->R <= 4) {   // one launch: the step flushes its own due heads
    const dim3 grid((unsigned)(io->N * st->H));
    const lq_conv none = {};
    if (deferred) {
      if (cv) gdn_step_kernel<128, 128, 2, true, true, 4, true><<<grid, 256, 0, s>>>(*st, *io, *cv, nullptr, Q0);
      else gdn_step_kernel<128, 128, 2, false, true, 4, true><<<grid, 256, 0, s>>>(*st, *io, none, nullptr, Q0);
    } else {
      if (cv) gdn_step_kernel<128, 128, 2, true, true><<<grid, 256, 0, s>>>(*st, *io, *cv, nullptr, Q0);
      else gdn_step_kernel<128, 128, 2, false, true><<<grid, 256, 0, s>>>(*st, *io, none, nullptr, Q0);
    }
    return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_HIP;
  }
  rc = cv ? launch_gdn_dims<true>(st, io, *cv, nullptr, s) : lq_launch_step(st, io, 0, 0.f, nullptr, s);
  if (rc) return rc;
  return lq_launch_flush(st, Q0, io->idx, io->N, 0, qmax, nullptr, s);
}

extern "C" int lq_gdn_decode(const lq_state* st, const lq_step_io* io, const lq_conv* cv, const float* Q0,
                             void* stream) {
  return gdn_decode(st, io, cv, Q0, false, (hipStream_t)stream);
}

extern "C" int lq_gdn_decode_deferred(const lq_state* st, const lq_step_io* io, const lq_conv* cv, const float* Q0,
                                      void* stream) {
  return gdn_decode(st, io, cv, Q0, true, (hipStream_t)stream);
}

extern "C" int lq_kda_step(const lq_state* st, const lq_step_io* io, float glb, void* stream) {
  int rc = lq_check_step(st, io);
  if (rc) return rc;
  if (!st->Gbuf || st->K != KD || st->V != VD || st->R > 4) return LQ_ERR_ARG;
  return lq_launch_step(st, io, 1, glb, nullptr, (hipStream_t)stream);
}

extern "C" int lq_kda_decode(const lq_state* st, const lq_step_io* io, float glb, const float* Q0, void* stream) {
  int rc = lq_check_step(st, io);
  if (rc) return rc;
  if (!st->Gbuf || st->K != KD || st->V != VD || st->R > 4) return LQ_ERR_ARG;
  const float qmax = st->qmax > 0.f ? st->qmax : LQ_QMAX;
  if ((rc = lq_check_flush(st, Q0, io->idx, io->N, 1, qmax))) return rc;
  if (io->N == 0) return LQ_OK;
  hipStream_t s = (hipStream_t)stream;
  if ((rc = lq_launch_step(st, io, 1, glb, nullptr, s))) return rc;
  return lq_launch_flush(st, Q0, io->idx, io->N, 1, qmax, nullptr, s);
}

extern "C" int lq_abi_version(void) { return LQ_ABI_VERSION; }
