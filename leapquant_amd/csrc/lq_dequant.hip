// Prefill dequant of GDN 128 x 128 heads at R <= 4 and of KDA heads in the four-wave layout (gfx950).
//
// Semantics: /root/reference/leapquant/kernels.py:2041-2123 (GDN dequant), as the eight-wave dequant_kernel of
// lq_flush.hip; /root/reference/leapquant/state.py:118-128 (KDA rebuild).
// A translation unit of its own: in lq_flush.hip the extra kernel changed the register allocation of the flush kernels
// (a 16-byte spill in the four-wave flush in place of 8, and a slower flush), although their code is unchanged.
#include "lq_flush_core.h"

namespace {

using namespace lqf;

// Four-wave prefill dequant of a GDN 128 x 128 head at R <= 4: dequant_kernel's arithmetic with the tile in the
// four-wave layout of the flush (wave w owns key channels [32 w, 32 w + 32)) and the window staged in halves of 32
// entries, so that the workgroup fits 40 KiB of LDS and four heads share a CU (the eight-wave layout holds the whole
// window's operands, 60 KiB: two heads per CU).  The window's products are added half by half (hi, lo of the first
// half, then of the second), an fp32 order the eight-wave kernel takes as hi, lo over the whole window.
__global__ __launch_bounds__(FT4) __attribute__((amdgpu_waves_per_eu(4)))
void dequant4_kernel(lq_state st, const int* __restrict__ idx, float qmax) {
  __shared__ FlushShared4 sh;
  const int HV = st.HV, L = st.L, R = st.R;
  // the value heads of a key head on one XCD at about the same time: their shared window keys are read into its L2 once
  const int p = sched_unit((int)blockIdx.x, HV / st.H, (int)gridDim.x);
  const int n = p / HV, hv = p - n * HV;
  const int slot = idx[n];
  if (slot <= 0 || slot >= st.NS) return;
  const long long sh_ = (long long)slot * HV + hv;
  const int tid = threadIdx.x, l = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), q = l >> 4;
  char* base = block_base(st, slot, hv);
  const int8_t* Sq = (const int8_t*)base;
  const float* Sk = (const float*)(base + VD * KD);
  const float* Sv = Sk + KD;
  const f16_t* UQ = (const f16_t*)(Sv + VD);
  const int h = __builtin_amdgcn_readfirstlane(min(st.hcnt[sh_], L));   // uniform: one word per head
  const float P = st.Pbuf[sh_];
  const int cv = tid & 127;
  const bool colt = tid < KD;
  const float scv = colt ? Sk[cv] : Sv[cv];
  float uqv[4];
#pragma unroll
  for (int a = 0; a < 4; ++a) uqv[a] = h2f(UQ[min(a, R - 1) * (KD + VD) + (colt ? 0 : KD) + cv]);
  const float wv = st.Wbuf[sh_ * L + min(tid, L - 1)];
  WinHalf win;
  if (h > 0) load_half<KD, VD>(win, st, slot, hv, h, 0);   // an empty window loads, stages and multiplies nothing
  uint32_t wds[2][8];
  load_code_words4<KD, VD>(wds, Sq);
  {
    f32x4 fac;
#pragma unroll
    for (int a = 0; a < 4; ++a) fac[a] = a < R ? uqv[a] : 0.f;
    if (colt) {
      sh.skl[cv] = scv;
      sh.uoc[cv] = fac;
    } else {
      sh.svr[cv] = scv;
      sh.qov[cv] = fac;
    }
  }
  if (tid < LPMAX) sh.w[tid] = tid < h ? wv : 0.f;
  __syncthreads();
  Tile4 t;
  {
    const float inv = 1.0f / qmax;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int c0 = 32 * w + 16 * g + 4 * q;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        const int v = 16 * nt + (l & 15);
        const float rv = sh.svr[v];
        const f32x4 qo = sh.qov[v];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int c = c0 + i;
          const f32x4 uo = sh.uoc[c];
          float x = (((float)(int)(int8_t)(wds[g][nt] >> (8 * i)) * inv) * sh.skl[c]) * rv;   // kernels.py:2107
#pragma unroll
          for (int a = 0; a < 4; ++a) x = fmaf(qo[a], uo[a], x);                              // kernels.py:2109-2111
          t.a[g][nt][i] = x * P;                                                               // kernels.py:2113
        }
      }
    }
  }
  if (h > 0) {                                        // + sum_{j<h} w_j u_j k_j^T (kernels.py:2115-2121)
    store_half(sh, win, h, 0);
    if (h > HALF) load_half<KD, VD>(win, st, slot, hv, h, 1);
    __syncthreads();
    rebuild_half4x2(t, sh.op[0], sh.op[1], sh.op[2]);
    if (h > HALF) {
      __syncthreads();                                // every wave is past the first half's operands
      store_half(sh, win, h, 1);
      __syncthreads();
      rebuild_half4x2(t, sh.op[0], sh.op[1], sh.op[2]);
    }
  }
  __syncthreads();                                    // every wave has read its codes: the fp32 state may overwrite them
  float* S = (float*)base;                            // non-temporal: 64 KiB per head, written once
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
      __builtin_nontemporal_store(t.a[g][nt], (f32x4*)(S + (16 * nt + (l & 15)) * KD + 32 * w + 16 * g + 4 * q));
  if (tid < L) st.Wbuf[sh_ * L + tid] = 0.f;
  if (tid == 0) {
    st.Pbuf[sh_] = 1.f;
    st.hcnt[sh_] = 0;
  }
}

// Four-wave prefill dequant of KDA heads (state.py:118-128): S = diag(exp(P)) (Q U^T + deq(Sq)) over the key channels
// plus sum_{j<h} w_j u_j (K_j * D_j)^T, D_j = prod_{j<i<h} e_i, in place as fp32; the window is left as it is (the
// checkpoint after the engine's prefill resets it).  The tile as dequant4_kernel holds it (four heads per CU, where a
// layout holding the whole window's operands, 79.6 KiB, fits two); the window as the KDA flush stages it (halves
// newest first, the decay product carried down between them, kda_key_scan4), with w_j K_j D_j in three bf16 terms
// (hi, mid, lo: 24 significant bits, so the window part keeps fp32 accuracy).  A half takes two MFMA passes: hi and
// mid from LDS, then lo (held in registers meanwhile) staged over hi.  The older half is loaded once the newer one is
// done, so that its rows do not share the registers with the scan and the products.
__global__ __launch_bounds__(FT4) __attribute__((amdgpu_waves_per_eu(4)))
void kda_dequant4_kernel(lq_state st, const int* __restrict__ idx, float qmax) {
  __shared__ FlushShared4 sh;
  __shared__ float pcs[KD];                           // exp(P[c])
  const int HV = st.HV, L = st.L, R = st.R;
  // the value heads of a key head on one XCD at about the same time: their shared window keys are read into its L2 once
  const int p = sched_unit((int)blockIdx.x, HV / st.H, (int)gridDim.x);
  const int n = p / HV, hv = p - n * HV;
  const int slot = idx[n];
  if (slot <= 0 || slot >= st.NS) return;
  const long long sh_ = (long long)slot * HV + hv;
  const int tid = threadIdx.x, l = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), q = l >> 4;
  char* base = block_base(st, slot, hv);
  const int8_t* Sq = (const int8_t*)base;
  const float* Sk = (const float*)(base + VD * KD);
  const float* Sv = Sk + KD;
  const f16_t* UQ = (const f16_t*)(Sv + VD);
  const int h = __builtin_amdgcn_readfirstlane(min(st.hcnt[sh_], L));   // uniform: one word per head
  const int hA = h > HALF ? 1 : 0;                   // the newest half first
  const int cv = tid & 127;
  const bool colt = tid < KD;
  const float scv = colt ? Sk[cv] : Sv[cv];
  float uqv[4];
#pragma unroll
  for (int a = 0; a < 4; ++a) uqv[a] = h2f(UQ[min(a, R - 1) * (KD + VD) + (colt ? 0 : KD) + cv]);
  const float pbc = st.Pbuf[sh_ * KD + cv];
  const float wv = st.Wbuf[sh_ * L + min(tid, L - 1)];
  WinHalf win;
  if (h > 0) load_half<KD, VD, true>(win, st, slot, hv, h, hA);   // an empty window loads, stages and multiplies nothing
  uint32_t wds[2][8];
  load_code_words4<KD, VD>(wds, Sq);
  {
    f32x4 fac;
#pragma unroll
    for (int a = 0; a < 4; ++a) fac[a] = a < R ? uqv[a] : 0.f;
    if (colt) {
      sh.skl[cv] = scv / qmax;
      pcs[cv] = expf(pbc);                                                              // state.py:128
      sh.uoc[cv] = fac;
    } else {
      sh.svr[cv] = scv;
      sh.qov[cv] = fac;
    }
  }
  if (tid < LPMAX) sh.w[tid] = tid < h ? wv : 0.f;
  __syncthreads();
  // the newest half's raw keys, decays (1 past h) and values (0 past h) to LDS first: its rows leave the registers
  // before the tile takes them
  if (h > 0) store_half<true>(sh, win, h, hA);
  // S0 pc in the tile layout: (code Sk / qmax) Sv + sum_r Q[v][r] U[c][r], times exp(P[c]) (state.py:121-122, 128)
  Tile4 t;
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int c0 = 32 * w + 16 * g + 4 * q;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int v = 16 * nt + (l & 15);
      const float rv = sh.svr[v];
      const f32x4 qo = sh.qov[v];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = c0 + i;
        const f32x4 uo = sh.uoc[c];
        float x = ((float)(int)(int8_t)(wds[g][nt] >> (8 * i)) * sh.skl[c]) * rv;
#pragma unroll
        for (int a = 0; a < 4; ++a) x = fmaf(qo[a], uo[a], x);
        t.a[g][nt][i] = pcs[c] * x;
      }
    }
  }
  if (h > 0) {                                        // + sum_{j<h} w_j u_j (K_j * D_j)^T (state.py:124-127)
    float dcar = 1.f;
    for (int k = 0; k <= hA; ++k) {
      const int hf = hA - k;
      if (k > 0) {
        load_half<KD, VD, true>(win, st, slot, hv, h, hf);
        __syncthreads();                              // every wave is past the newer half's operands
        store_half<true>(sh, win, h, hf);
      }
      __syncthreads();
      uint32_t lo[8];
      dcar = kda_key_scan4<3>(sh, dcar, h, hf, lo);   // hi / mid in place of the keys / decays
      __syncthreads();
      rebuild_half4x2a(t, sh.op[0], sh.op[1], sh.op[2]);
      __syncthreads();                                // every wave is past hi
      {
        const int c = tid >> 1, jb = 16 * (tid & 1);  // the lane's own entries, as the scan wrote them
        *(uint4*)&sh.op[0][c][jb] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        *(uint4*)&sh.op[0][c][jb + 8] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
      }
      __syncthreads();
      rebuild_half4x1(t, sh.op[0], sh.op[2]);
    }
  }
  __syncthreads();                                    // every wave has read its codes: the fp32 state may overwrite them
  float* S = (float*)base;                            // plain stores (non-temporal ones measured slower for KDA heads)
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) *(f32x4*)(S + (16 * nt + (l & 15)) * KD + 32 * w + 16 * g + 4 * q) = t.a[g][nt];
}

}  // namespace

// launched by lq_kda_dequant, arguments already checked
int lq_launch_kda_dequant4(const lq_state* st, const int* idx, int N, float qmax, hipStream_t s) {
  kda_dequant4_kernel<<<dim3((unsigned)(N * st->HV)), FT4, 0, s>>>(*st, idx, qmax);
  return LQ_OK;
}

// launched by lq_dequant for GDN 128 x 128 heads at R <= 4, arguments already checked
int lq_launch_dequant4(const lq_state* st, const int* idx, int N, float qmax, hipStream_t s) {
  dequant4_kernel<<<dim3((unsigned)(N * st->HV)), FT4, 0, s>>>(*st, idx, qmax);
  return LQ_OK;
}
