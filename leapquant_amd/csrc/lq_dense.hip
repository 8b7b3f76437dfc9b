// Dense-state GDN decode step (bf16 or fp32 state): the baseline the INT8 step is measured against.
// S' = alpha S + u k^T, u = beta (v - alpha S k), o = S' q with the same gate, beta and norms as the INT8 step.
// One workgroup per (row, key head), 128 threads per value head; each 8-lane group owns 8 rows, each lane 16 columns.
// Tuned as the INT8 step is: every state byte of a lane requested before any arithmetic (bf16: the 8 rows kept packed,
// 64 VGPRs, loaded with the non-temporal hint: each byte is read once per launch), q / k by 16-byte loads, <= 128
// VGPRs so that four waves per SIMD keep the whole grid resident.  Stores stay plain (non-temporal stores measured
// 29.9 -> 40.7 us at config 1).
#include "lq_common.h"

namespace {

constexpr int KD = 128, VD = 128;
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_once_u4(const uint4* p) {
  const u32x4_t x = __builtin_nontemporal_load((const u32x4_t*)p);
  return make_uint4(x.x, x.y, x.z, x.w);
}

template <int G, bool F32>
__global__ __launch_bounds__(128 * G) __attribute__((amdgpu_waves_per_eu(4)))
void dense_step_kernel(void* S, int NS, int HV, int H, lq_step_io io) {
  const int n = blockIdx.x / H, hk = blockIdx.x - n * H;
  const int tid = threadIdx.x, g = tid >> 7, lt = tid & 127, rg = lt >> 3, cc = lt & 7;
  const int hv = hk * G + g;
  const long long MIX = 2ll * H * KD + (long long)HV * VD;
  bf16_t* out = (bf16_t*)io.out + ((long long)n * HV + hv) * VD;
  const int slot = io.idx[n];
  if (slot <= 0 || slot >= NS) { out[lt] = 0; return; }
  const bf16_t* mrow = (const bf16_t*)io.mixed + (long long)n * MIX;
  const long long head = ((long long)slot * HV + hv) * VD * KD;
  // the state rows first (the bulk of the bytes): bf16 rows kept as loaded, 8 rows x 16 columns per lane (64 VGPRs),
  // unpacked one row at a time below; fp32 rows in two batches of 4
  constexpr int RB = F32 ? 4 : 8;          // rows per batch held in registers
  uint4 raw[F32 ? 1 : 8][2];
  if (!F32) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const uint4* p = (const uint4*)((const bf16_t*)S + head + (long long)(8 * rg + r) * KD + 16 * cc);
      raw[r][0] = ld_once_u4(p);
      raw[r][1] = ld_once_u4(p + 1);
    }
  }
  // q, k: this lane's 16 channels as two 16-byte loads each
  float qv[16], kv[16];
  {
    const uint4* qp = (const uint4*)(mrow + hk * KD + 16 * cc);
    const uint4* kp = (const uint4*)(mrow + H * KD + hk * KD + 16 * cc);
    const uint4 q0 = qp[0], q1 = qp[1], k0 = kp[0], k1 = kp[1];
    const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const uint32_t kw[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
#pragma unroll
    for (int z = 0; z < 8; ++z) {
      qv[2 * z] = bf_lo(qw[z]); qv[2 * z + 1] = bf_hi(qw[z]);
      kv[2 * z] = bf_lo(kw[z]); kv[2 * z + 1] = bf_hi(kw[z]);
    }
  }
  const float alpha = gdn_alpha(bf2f(((const bf16_t*)io.a)[(long long)n * HV + hv]), io.dt_bias[hv], io.A_log[hv]);
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
  float yk = 0.f;
  for (int b0 = 0; b0 < 8; b0 += RB) {
    float s[RB][16];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const long long off = head + (long long)(8 * rg + b0 + r) * KD + 16 * cc;
      if (F32) {
        const float4* p = (const float4*)((const float*)S + off);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float4 x = p[e];
          s[r][4 * e] = x.x; s[r][4 * e + 1] = x.y; s[r][4 * e + 2] = x.z; s[r][4 * e + 3] = x.w;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int v = 8 * rg + b0 + r;
      if (!F32) {                          // unpack this row
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const uint32_t u[4] = {raw[r][e].x, raw[r][e].y, raw[r][e].z, raw[r][e].w};
#pragma unroll
          for (int z = 0; z < 4; ++z) {
            s[r][8 * e + 2 * z] = bf_lo(u[z]);
            s[r][8 * e + 2 * z + 1] = bf_hi(u[z]);
          }
        }
      }
      float m = 0.f, y = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) { m = fmaf(s[r][i], kn[i], m); y = fmaf(s[r][i], qn[i], y); }
      m = sum8(m); y = sum8(y);
      const float vin = bf2f(mrow[2ll * H * KD + hv * VD + v]);
      const float u = beta * (vin - alpha * m);
      const float o = alpha * y + kappa * u;
      if (cc == b0 + r) yk = o;           // lane cc keeps row 8 rg + cc
      const long long off = head + (long long)v * KD + 16 * cc;
      if (F32) {
        float4* p = (float4*)((float*)S + off);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          p[e] = make_float4(fmaf(u, kn[4 * e], alpha * s[r][4 * e]), fmaf(u, kn[4 * e + 1], alpha * s[r][4 * e + 1]),
                             fmaf(u, kn[4 * e + 2], alpha * s[r][4 * e + 2]), fmaf(u, kn[4 * e + 3], alpha * s[r][4 * e + 3]));
      } else {
        uint4* p = (uint4*)((bf16_t*)S + off);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          uint32_t w[4];
#pragma unroll
          for (int z = 0; z < 4; ++z) {
            const int c = 8 * e + 2 * z;
            w[z] = (uint32_t)f2bf(fmaf(u, kn[c], alpha * s[r][c])) |
                   ((uint32_t)f2bf(fmaf(u, kn[c + 1], alpha * s[r][c + 1])) << 16);
          }
          p[e] = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
    }
  }
  out[8 * rg + cc] = f2bf(yk);
}

}  // namespace

// Baseline (no reference counterpart): the standalone conv1d update that lq_gdn_step_conv fuses into the step, with
// the same arithmetic -- vLLM's causal_conv1d_update stands here (vLLM is not installed).  Thread per (row, channel):
// out[n][c] = bf16(act(conv)), the slot's conv state shifted; padding rows (slot <= 0) are skipped.
__global__ __launch_bounds__(256) void conv_update_kernel(lq_conv cv, const bf16_t* __restrict__ x, bf16_t* out,
                                                          const int* __restrict__ idx, int C, int NS) {
  const int n = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  const int slot = idx[n];
  if (c >= C || slot <= 0 || slot >= NS || slot >= cv.NS) return;
  const long long sb = (long long)slot * cv.slot_stride;
  const ConvTaps t = conv_taps(cv, x + (long long)n * C, sb, c);
  out[(long long)n * C + c] = f2bf(conv_out(t, cv.silu));
  conv_shift(cv, sb, c, t);
}

extern "C" int lq_dense_step(void* S, int state_dtype, int NS, int HV, int H, int K, int V, const lq_step_io* io,
                             void* stream) {
  if (!S || !io || K != KD || V != VD || H <= 0 || HV <= 0 || HV % H != 0 || NS <= 0 || io->N < 0) return LQ_ERR_ARG;
  if (state_dtype != 0 && state_dtype != 1) return LQ_ERR_ARG;
  if (io->N == 0) return LQ_OK;
  // q, k and the state rows are read by 16-byte loads: 16-byte aligned bases (the rows are multiples of 16 bytes)
  if (((uintptr_t)S & 15) || ((uintptr_t)io->mixed & 15)) return LQ_ERR_ARG;
  const int G = HV / H;
  dim3 grid((unsigned)(io->N * H));
  hipStream_t s = (hipStream_t)stream;
#define LQ_DENSE(GG, FF) dense_step_kernel<GG, FF><<<grid, 128 * GG, 0, s>>>(S, NS, HV, H, *io)
  if (state_dtype == 0) {
    if (G == 1) LQ_DENSE(1, false); else if (G == 2) LQ_DENSE(2, false); else if (G == 4) LQ_DENSE(4, false);
    else return LQ_ERR_ARG;
  } else {
    if (G == 1) LQ_DENSE(1, true); else if (G == 2) LQ_DENSE(2, true); else if (G == 4) LQ_DENSE(4, true);
    else return LQ_ERR_ARG;
  }
#undef LQ_DENSE
  return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_HIP;
}

extern "C" int lq_conv_update(const lq_conv* cv, const void* x, void* out, const int* idx, int N, int C, int NS,
                              void* stream) {
  if (!cv || !cv->state || !cv->weight || cv->W != 4 || (cv->silu != 0 && cv->silu != 1) || N < 0 || C <= 0 || NS <= 0
      || cv->NS <= 0)
    return LQ_ERR_ARG;
  if (cv->ch_stride <= 0 || cv->tap_stride <= 0 || (C - 1) * cv->ch_stride + 2 * cv->tap_stride >= cv->slot_stride)
    return LQ_ERR_ARG;
  if (((uintptr_t)cv->weight & 7) != 0) return LQ_ERR_ARG;
  if (N == 0) return LQ_OK;
  if (!x || !out || !idx) return LQ_ERR_ARG;
  dim3 grid((unsigned)((C + 255) / 256), (unsigned)N);
  conv_update_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(*cv, (const bf16_t*)x, (bf16_t*)out, idx, C, NS);
  return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_HIP;
}
