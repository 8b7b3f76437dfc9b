// GDN / KDA decode step on the INT8 checkpoint + window buffer (gfx950).
//
// Semantics follow /root/reference/leapquant/kernels.py:27-692 (GDN) and 694-1075 (KDA); the layout of the checkpoint
// and of the window buffer is described in include/lq.h.
//
// Mapping (MI355X-first, not the reference's persistent TMA/mbarrier pipeline): one workgroup per (row n, key head hk),
// 128 threads per value head (G = HV / H value heads share the key head's q, k and buffered keys).  The int8 tile of a
// value head (16 KiB) is streamed straight into registers with 16-byte loads, dequantised with the column scale folded
// into the key/query operand, and both GEMVs (m = deq(Sq) k, y = deq(Sq) q) run in one pass on the VALU; each row is
// owned by 8 lanes (16 columns each) whose partial sums meet in DPP reductions.  Only the h valid window rows are read,
// and the buffered keys are read once per key head.  No MFMA: the step is ~1 flop/byte.
#include "lq_common.h"

namespace {

constexpr int KD = 128;   // key dim
constexpr int VD = 128;   // value dim
constexpr int LMAX = 64;  // largest window the kernels are built for

__device__ __forceinline__ void unpack8(uint4 w, float* f) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(u[i] << 16);
    f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void unpack8h(uint4 w, float* f) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = h2f((f16_t)(u[i] & 0xffffu));
    f[2 * i + 1] = h2f((f16_t)(u[i] >> 16));
  }
}

// 16 codes of one row chunk against the lane's 16 column operands
__device__ __forceinline__ void dot16_i8(uint4 w, const float* kf, const float* qf, float& m, float& y) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float x = (float)(int)(int8_t)(u[i] >> (8 * b));
      m = fmaf(x, kf[4 * i + b], m);
      y = fmaf(x, qf[4 * i + b], y);
    }
  }
}

template <int G>
struct StepShared {
  bf16_t ub[G][LMAX][VD];  // the window's u_j rows per value head (staged by direct global -> LDS loads)
  f16_t uq[G][4][KD + VD]; // U^T | Q^T per value head
  float2 dkq[LMAX];        // (dk_j, dq_j): buffered key j against kn / qn (shared by the key head)
  float2 duq[G][4];        // (dU_r, dQ_r) per value head g, factor r
  float w[G][LMAX];        // gated entry weights w_j per value head
  float4 kn[KD / 4];       // normalised key and query (not kept in registers across the tile stream)
  float4 qn[KD / 4];
};

// ------------------------------------------------------------------------------------------------------------------
// GDN step  (kernels.py:129-144 gate / beta, 236-279 norms and weights, 380-585 stream, dots and appends)
//
// Per workgroup (row n, key head hk), 128 threads per value head g.  Order of the memory traffic:
//   idx -> {int8 tile (registers), hcnt} -> {u_j rows and U^T|Q^T (direct to LDS), scales, q, k, v}
//   -> GEMV on the tile -> barrier -> buffered keys k_j (registers) against kn / qn -> barrier -> per-row output.
// At <= 128 VGPRs four 256-thread workgroups fit on a CU, so the whole B = 64 x H = 16 grid is resident at once.
// ------------------------------------------------------------------------------------------------------------------
template <int G>
__global__ __launch_bounds__(128 * G) __attribute__((amdgpu_waves_per_eu(4)))
void gdn_step_kernel(lq_state st, lq_step_io io) {
  __shared__ StepShared<G> sh;
  const int H = st.H, HV = st.HV, L = st.L, R = st.R;
  const int n = blockIdx.x / H;
  const int hk = blockIdx.x - n * H;
  const int tid = threadIdx.x;
  // value head of this thread within the key head: wave-uniform, so per-head scalars come through scalar loads that
  // do not wait behind the tile's vector loads
  const int g = __builtin_amdgcn_readfirstlane(tid >> 7);
  const int lt = tid & 127;     // thread within the value head
  const int wi = __builtin_amdgcn_readfirstlane(lt >> 6);   // wave within the value head
  const int lane = tid & 63;
  const int rg = lt >> 3;       // row group: rows 8 rg .. 8 rg + 7 of the int8 tile
  const int cc = lt & 7;        // column chunk: columns 16 cc .. 16 cc + 15
  const int hv = hk * G + g;
  const long long MIX = 2ll * H * KD + (long long)HV * VD;
  bf16_t* out = (bf16_t*)io.out + ((long long)n * HV + hv) * VD;

  const int slot = io.idx[n];
  if (slot <= 0) {              // padding row (kernels.py:374-378)
    out[lt] = 0;
    return;
  }
  const char* base = block_base(st, slot, hv);
  uint4 code[8];                // the int8 tile first: the long pole
  {
    const uint4* cp = (const uint4*)base + (8 * rg) * 8 + cc;
#pragma unroll
    for (int i = 0; i < 8; ++i) code[i] = cp[i * 8];
  }
  const long long sh_ = (long long)slot * HV + hv;
  const int h = st.hcnt[sh_];
  const bool live = h < L;      // a full window is never stepped (the flush follows every step)
  int hmax = h;
#pragma unroll
  for (int g2 = 0; g2 < G; ++g2) hmax = max(hmax, (int)st.hcnt[(long long)slot * HV + hk * G + g2]);
  hmax = min(hmax, L);

  // ---- window values u_j (j < h) and the factors straight to LDS, 1 KiB per wave instruction ----
  {
    const char* ubg = (const char*)((const bf16_t*)st.Ubuf + sh_ * L * VD);
    const int nch = live ? (h + 3) >> 2 : 0;      // 4 rows of 256 B per chunk; chunk rows >= h are never read
    for (int c = wi; c < nch; c += 2) lds_load16(ubg + c * 1024 + 16 * lane, (char*)&sh.ub[g][0][0] + c * 1024);
    const char* uqg = base + VD * KD + 4 * (KD + VD);
    lds_load16(uqg + wi * 1024 + 16 * lane, (char*)&sh.uq[g][0][0] + wi * 1024);
  }
  const float* Skp = (const float*)(base + VD * KD);
  const float* Svp = Skp + KD;
  float sk[16];
  {
    const float4* p = (const float4*)(Skp + 16 * cc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4 t = p[i];
      sk[4 * i] = t.x; sk[4 * i + 1] = t.y; sk[4 * i + 2] = t.z; sk[4 * i + 3] = t.w;
    }
  }
  const bf16_t* mrow = (const bf16_t*)io.mixed + (long long)n * MIX;
  float qv[16], kv[16];
  {
    const uint4* qp = (const uint4*)(mrow + hk * KD + 16 * cc);
    const uint4* kp = (const uint4*)(mrow + H * KD + hk * KD + 16 * cc);
    unpack8(qp[0], qv); unpack8(qp[1], qv + 8);
    unpack8(kp[0], kv); unpack8(kp[1], kv + 8);
  }
  const float vin = bf2f(mrow[2ll * H * KD + hv * VD + lt]);
  const float sv = Svp[lt];
  const float P = st.Pbuf[sh_];
  const float alpha = gdn_alpha_f(bf2f(((const bf16_t*)io.a)[(long long)n * HV + hv]), io.dt_bias[hv], io.A_log[hv]);
  const float beta = beta_f(bf2f(((const bf16_t*)io.b)[(long long)n * HV + hv]));
  float* Wp = st.Wbuf + sh_ * L;
  float wmine = 0.f;
  if (live && lt < h) {         // w_j = Wbuf[j] alpha for the live entries (kernels.py:270-274)
    wmine = Wp[lt] * alpha;
    sh.w[g][lt] = wmine;
  }

  // ---- l2 norms of q and k: every 8-lane row group holds the whole vectors (16 columns per lane) ----
  float nq = 0.f, nk = 0.f, nkq = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    nq = fmaf(qv[i], qv[i], nq);
    nk = fmaf(kv[i], kv[i], nk);
    nkq = fmaf(kv[i], qv[i], nkq);
  }
  nq = sum8(nq); nk = sum8(nk); nkq = sum8(nkq);
  const float inq = rsqrtf_rn(nq + (float)LQ_NORM_EPS) * io.scale;
  const float ink = rsqrtf_rn(nk + (float)LQ_NORM_EPS);
  const float kappa = nkq * inq * ink;
  // ---- checkpoint stream: m = deq(Sq) kn, y = deq(Sq) qn with kf = kn Sk / 127 (kernels.py:255-256) ----
  float mq = 0.f, yq = 0.f;     // this lane keeps row 8 rg + cc = lt
  {
    float kn[16], qn[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) { kn[i] = kv[i] * ink; qn[i] = qv[i] * inq; }
    if (tid < 8) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sh.kn[4 * cc + i] = make_float4(kn[4 * i], kn[4 * i + 1], kn[4 * i + 2], kn[4 * i + 3]);
        sh.qn[4 * cc + i] = make_float4(qn[4 * i], qn[4 * i + 1], qn[4 * i + 2], qn[4 * i + 3]);
      }
    }
    float kf[16], qf[16];
    const float inv = 1.0f / LQ_QMAX;
#pragma unroll
    for (int i = 0; i < 16; ++i) { kf[i] = (kn[i] * sk[i]) * inv; qf[i] = (qn[i] * sk[i]) * inv; }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float m = 0.f, y = 0.f;
      dot16_i8(code[i], kf, qf, m, y);
      m = sum8(m);
      y = sum8(y);
      if (cc == i) { mq = m; yq = y; }
    }
  }
  mq *= sv;
  yq *= sv;

  wait_vm();
  __syncthreads();              // u_j rows, factors and w_j are in LDS

  // ---- buffered-key dots (once per key head) and factor dots (per value head), one 8-lane group per row ----
  {
    float kn[16], qn[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 a = sh.kn[4 * cc + i], b = sh.qn[4 * cc + i];
      kn[4 * i] = a.x; kn[4 * i + 1] = a.y; kn[4 * i + 2] = a.z; kn[4 * i + 3] = a.w;
      qn[4 * i] = b.x; qn[4 * i + 1] = b.y; qn[4 * i + 2] = b.z; qn[4 * i + 3] = b.w;
    }
    const bf16_t* Kb = (const bf16_t*)st.Kbuf + ((long long)slot * H + hk) * L * KD;
    constexpr int MAXT = (LMAX + 4 * G + 16 * G - 1) / (16 * G);
    const int ntask = hmax + G * R;
    const int t0 = g * 16 + rg;
    constexpr int PF = MAXT < 3 ? MAXT : 3;     // rows prefetched per batch
#pragma unroll
    for (int i0 = 0; i0 < MAXT; i0 += PF) {
    uint4 kw[PF][2];
#pragma unroll
    for (int i = i0; i < i0 + PF && i < MAXT; ++i) {
      const int t = t0 + 16 * G * i;
      if (t < hmax) {
        const uint4* p = (const uint4*)(Kb + (long long)t * KD + 16 * cc);
        kw[i - i0][0] = p[0];
        kw[i - i0][1] = p[1];
      }
    }
#pragma unroll
    for (int i = i0; i < i0 + PF && i < MAXT; ++i) {
      const int t = t0 + 16 * G * i;
      if (t < ntask) {
        float x[16];
        if (t < hmax) {
          unpack8(kw[i - i0][0], x); unpack8(kw[i - i0][1], x + 8);
        } else {
          const int tt = t - hmax, g2 = tt / R, r = tt - g2 * R;
          const uint4* p = (const uint4*)(&sh.uq[g2][r][16 * cc]);
          unpack8h(p[0], x); unpack8h(p[1], x + 8);
        }
        float dk = 0.f, dq = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) { dk = fmaf(x[e], kn[e], dk); dq = fmaf(x[e], qn[e], dq); }
        dk = sum8(dk); dq = sum8(dq);
        if (cc == 0) {
          if (t < hmax) sh.dkq[t] = make_float2(dk, dq);
          else { const int tt = t - hmax; sh.duq[tt / R][tt % R] = make_float2(dk, dq); }
        }
      }
    }
    }
  }
  __syncthreads();
  if (!live) { out[lt] = 0; return; }

  // ---- row v = lt: buffered entries, rank-R part, delta rule, output and appends (kernels.py:536-585) ----
  float a4 = 0.f, a5 = 0.f;
  for (int j = 0; j < h; ++j) {
    const float ub = bf2f(sh.ub[g][j][lt]);
    const float wj = sh.w[g][j];
    const float2 d = sh.dkq[j];
    a4 = fmaf(ub, wj * d.x, a4);
    a5 = fmaf(ub, wj * d.y, a5);
  }
  float a6 = 0.f, a7 = 0.f;
  for (int r = 0; r < R; ++r) {
    const float qt = h2f(sh.uq[g][r][KD + lt]);
    const float2 d = sh.duq[g][r];
    a6 = fmaf(qt, d.x, a6);
    a7 = fmaf(qt, d.y, a7);
  }
  const float pn = P * alpha;
  const float u = beta * (vin - (pn * (mq + a6) + a4));
  const float y = pn * (yq + a7) + a5 + kappa * u;
  out[lt] = f2bf(y);
  ((bf16_t*)st.Ubuf)[(sh_ * L + h) * VD + lt] = f2bf(u);
  if (g == 0) {
    const float kc = bf2f(mrow[H * KD + hk * KD + lt]) * ink;
    ((bf16_t*)st.Kbuf)[(((long long)slot * H + hk) * L + h) * KD + lt] = f2bf(kc);
  }
  if (lt < h) Wp[lt] = wmine;
  if (lt == h) Wp[h] = 1.0f;
  if (lt == 0) {
    st.Pbuf[sh_] = pn;
    st.hcnt[sh_] = h + 1;
  }
}

// ------------------------------------------------------------------------------------------------------------------
// KDA step  (kernels.py:694-1075): per-channel gate; decayed buffered keys; pc folded into the checkpoint operands.
// One workgroup per (row n, value head hv), 128 threads.
// ------------------------------------------------------------------------------------------------------------------
struct KdaShared {
  bf16_t kt[LMAX][KD];     // decayed keys  bf16(K_j * en * prod_{j<i<h} e_i)
  float pc[KD];
  float2 dkq[LMAX];
  float2 duq[4];
};

__global__ __launch_bounds__(128) void kda_step_kernel(lq_state st, lq_step_io io, float glb) {
  __shared__ KdaShared sh;
  const int H = st.H, HV = st.HV, L = st.L, R = st.R;
  const int G = HV / H;
  const int n = blockIdx.x / HV;
  const int hv = blockIdx.x - n * HV;
  const int hk = hv / G;
  const int lt = threadIdx.x;
  const int rg = lt >> 3, cc = lt & 7;
  const long long MIX = 2ll * H * KD + (long long)HV * VD;
  bf16_t* out = (bf16_t*)io.out + ((long long)n * HV + hv) * VD;
  const int slot = io.idx[n];
  if (slot <= 0) { out[lt] = 0; return; }
  const long long sh_ = (long long)slot * HV + hv;
  const int h = st.hcnt[sh_];
  if (h >= L) { out[lt] = 0; return; }    // uniform over the workgroup

  const char* base = block_base(st, slot, hv);
  uint4 code[8];
  {
    const uint4* cp = (const uint4*)base + (8 * rg) * 8 + cc;
#pragma unroll
    for (int i = 0; i < 8; ++i) code[i] = cp[i * 8];
  }
  const float* Skp = (const float*)(base + VD * KD);
  const float* Svp = Skp + KD;
  const f16_t* UQp = (const f16_t*)(Svp + VD);
  const bf16_t* mrow = (const bf16_t*)io.mixed + (long long)n * MIX;

  // ---- per-channel gate for channel c = lt (kernels.py:704-712, 802, 887-896) ----
  {
    const int c = lt;
    const double xg = (double)(bf2f(((const bf16_t*)io.a)[((long long)n * HV + hv) * KD + c]) + io.dt_bias[hv * KD + c]);
    const double ea = exp((double)io.A_log[hv]);
    double gdec;
    if (glb != 0.f) gdec = (double)glb / (1.0 + exp(-ea * xg));
    else gdec = -ea * softplus20(xg);
    const float pb = st.Pbuf[sh_ * KD + c];
    const float gn = (float)((double)pb + gdec);
    const float pcv = (float)exp((double)gn);
    const float en = (float)exp(gdec);
    sh.pc[c] = pcv;
    // decayed keys, backward over the live entries (entries j >= h carry e_j = 1 by the flush's reset)
    const bf16_t* Kb = (const bf16_t*)st.Kbuf + (((long long)slot * H + hk) * L) * KD + c;
    const f16_t* Gb = (const f16_t*)st.Gbuf + (sh_ * L) * KD + c;
    float dcur = en;
    for (int j = h - 1; j >= 0; --j) {
      const float kb = bf2f(Kb[(long long)j * KD]);
      sh.kt[j][c] = f2bf(kb * dcur);
      dcur = dcur * h2f(Gb[(long long)j * KD]);
    }
    __syncthreads();
    // state writes of the gate (after every lane has read its Pbuf / Gbuf entries)
    st.Pbuf[sh_ * KD + c] = gn;
    ((f16_t*)st.Gbuf)[(sh_ * L + h) * KD + c] = f2h(en);
  }

  float sk[16], pcl[16];
  {
    const float4* p = (const float4*)(Skp + 16 * cc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4 t = p[i];
      sk[4 * i] = t.x; sk[4 * i + 1] = t.y; sk[4 * i + 2] = t.z; sk[4 * i + 3] = t.w;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) pcl[i] = sh.pc[16 * cc + i];
  }
  float qv[16], kv[16];
  {
    const uint4* qp = (const uint4*)(mrow + hk * KD + 16 * cc);
    const uint4* kp = (const uint4*)(mrow + H * KD + hk * KD + 16 * cc);
    unpack8(qp[0], qv); unpack8(qp[1], qv + 8);
    unpack8(kp[0], kv); unpack8(kp[1], kv + 8);
  }
  const float vin = bf2f(mrow[2ll * H * KD + hv * VD + lt]);
  const float sv = Svp[lt];
  const float beta = beta_of(bf2f(((const bf16_t*)io.b)[(long long)n * HV + hv]));

  float nq = 0.f, nk = 0.f, nkq = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    nq = fmaf(qv[i], qv[i], nq);
    nk = fmaf(kv[i], kv[i], nk);
    nkq = fmaf(kv[i], qv[i], nkq);
  }
  nq = sum8(nq); nk = sum8(nk); nkq = sum8(nkq);
  const float inq = rsqrt_rn((double)nq + LQ_NORM_EPS) * io.scale;
  const float ink = rsqrt_rn((double)nk + LQ_NORM_EPS);
  const float kappa = nkq * inq * ink;
  float kn[16], qn[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) { kn[i] = kv[i] * ink; qn[i] = qv[i] * inq; }

  // ---- decayed-key dots (w_j folded in, kernels.py:1031-1035) and pc-scaled factor dots (1036-1047) ----
  const float* Wp = st.Wbuf + sh_ * L;
  for (int t = rg; t < h + R; t += 16) {
    float x[16];
    if (t < h) {
      const uint4* p = (const uint4*)(&sh.kt[t][16 * cc]);
      unpack8(p[0], x); unpack8(p[1], x + 8);
    } else {
      const uint4* p = (const uint4*)(UQp + (t - h) * (KD + VD) + 16 * cc);
      unpack8h(p[0], x); unpack8h(p[1], x + 8);
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] *= pcl[i];
    }
    float dk = 0.f, dq = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) { dk = fmaf(x[i], kn[i], dk); dq = fmaf(x[i], qn[i], dq); }
    dk = sum8(dk); dq = sum8(dq);
    if (cc == 0) {
      if (t < h) { const float w = Wp[t]; sh.dkq[t] = make_float2(w * dk, w * dq); }
      else sh.duq[t - h] = make_float2(dk, dq);
    }
  }

  // ---- checkpoint stream with kf = kn Sk / 127 pc (kernels.py:900-901) ----
  float kf[16], qf[16];
  const float inv = 1.0f / LQ_QMAX;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    kf[i] = ((kn[i] * sk[i]) * inv) * pcl[i];
    qf[i] = ((qn[i] * sk[i]) * inv) * pcl[i];
  }
  float mrow_[8], yrow_[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float m = 0.f, y = 0.f;
    dot16_i8(code[i], kf, qf, m, y);
    mrow_[i] = sum8(m);
    yrow_[i] = sum8(y);
  }
  float mq = mrow_[0], yq = yrow_[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) { if (cc == i) { mq = mrow_[i]; yq = yrow_[i]; } }
  mq *= sv;
  yq *= sv;
  __syncthreads();

  const bf16_t* Ub = (const bf16_t*)st.Ubuf + sh_ * L * VD + lt;
  float a4 = 0.f, a5 = 0.f;
  for (int j = 0; j < h; ++j) {
    const float ub = bf2f(Ub[(long long)j * VD]);
    const float2 d = sh.dkq[j];
    a4 = fmaf(ub, d.x, a4);
    a5 = fmaf(ub, d.y, a5);
  }
  float a6 = 0.f, a7 = 0.f;
  for (int r = 0; r < R; ++r) {
    const float qt = h2f(UQp[r * (KD + VD) + KD + lt]);
    a6 = fmaf(qt, sh.duq[r].x, a6);
    a7 = fmaf(qt, sh.duq[r].y, a7);
  }
  const float u = beta * (vin - (mq + a6 + a4));        // kernels.py:1065
  const float y = yq + a7 + a5 + kappa * u;             // kernels.py:1066
  out[lt] = f2bf(y);
  ((bf16_t*)st.Ubuf)[(sh_ * L + h) * VD + lt] = f2bf(u);
  if (hv % G == 0) {
    const float kc = bf2f(mrow[H * KD + hk * KD + lt]) * ink;
    ((bf16_t*)st.Kbuf)[(((long long)slot * H + hk) * L + h) * KD + lt] = f2bf(kc);
  }
  if (lt == 0) {
    st.Wbuf[sh_ * L + h] = 1.0f;
    st.hcnt[sh_] = h + 1;
  }
}

}  // namespace

static int check_step(const lq_state* st, const lq_step_io* io) {
  if (!st || !io) return LQ_ERR_ARG;
  if (st->K != KD || st->V != VD || st->L < 1 || st->L > LMAX || st->R < 0 || st->R > 4) return LQ_ERR_ARG;
  if (st->H <= 0 || st->HV <= 0 || st->HV % st->H != 0 || io->N < 0) return LQ_ERR_ARG;
  if (!st->ssm || !st->Kbuf || !st->Ubuf || !st->Wbuf || !st->Pbuf || !st->hcnt) return LQ_ERR_ARG;
  if (st->slot_stride < (long long)st->HV * st->V * st->K) return LQ_ERR_ARG;
  if (io->N > 0 && (!io->mixed || !io->a || !io->b || !io->A_log || !io->dt_bias || !io->idx || !io->out))
    return LQ_ERR_ARG;
  return LQ_OK;
}

extern "C" int lq_gdn_step(const lq_state* st, const lq_step_io* io, void* stream) {
  int rc = check_step(st, io);
  if (rc) return rc;
  const int G = st->HV / st->H;
  if (io->N == 0) return LQ_OK;
  dim3 grid((unsigned)(io->N * st->H));
  hipStream_t s = (hipStream_t)stream;
  switch (G) {
    case 1: gdn_step_kernel<1><<<grid, 128, 0, s>>>(*st, *io); break;
    case 2: gdn_step_kernel<2><<<grid, 256, 0, s>>>(*st, *io); break;
    case 4: gdn_step_kernel<4><<<grid, 512, 0, s>>>(*st, *io); break;
    default: return LQ_ERR_ARG;
  }
  return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_HIP;
}

extern "C" int lq_kda_step(const lq_state* st, const lq_step_io* io, float glb, void* stream) {
  int rc = check_step(st, io);
  if (rc) return rc;
  if (!st->Gbuf) return LQ_ERR_ARG;
  if (io->N == 0) return LQ_OK;
  dim3 grid((unsigned)(io->N * st->HV));
  kda_step_kernel<<<grid, 128, 0, (hipStream_t)stream>>>(*st, *io, glb);
  return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_HIP;
}

extern "C" int lq_abi_version(void) { return LQ_ABI_VERSION; }
