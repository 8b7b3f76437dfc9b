// End-of-window flush, standalone quantize, prefill dequant and low-rank factoriser (gfx950).
//
// Semantics: /root/reference/leapquant/kernels.py:1077-2033 (flush), 2126-2242 (quantize), 2041-2123 (dequant),
// 2246-2331 (lowrank).  Layout of the checkpoint and window buffer: include/lq.h.  The per-head flush and the tile
// helpers are in lq_flush_core.h.
//
// One workgroup of 512 threads (8 waves) per (slot, value head) (the flush is persistent: a workgroup takes its due
// heads one after another; quantize / dequant / lowrank take one head each); the GDN flush of 128 x 128 heads runs the
// four-wave layout instead (256 threads, four heads per CU).  Due heads are found on the device (hcnt == L), so the
// fixed grid is graph-capture safe.
#include "lq_flush_core.h"

#include <type_traits>

namespace {

using namespace lqf;

// Persistent flush over the candidate units p (row n = p / (HV / U), heads U (p % (HV / U)) .. + U - 1; U = 1 but for
// the paired 64-dim heads); a due unit (slot > 0, hcnt == L for some head of the unit; kernels.py:1200) is flushed by
// one workgroup.  With the schedule counters st.sched (and more candidates than workgroups), workgroup b takes
// candidate b first and then the next candidate its counter hands out, one at a time: the four workgroups that share
// a CU are not served equally by the hardware (at config 3 the first dispatched took 403k cycles for its eight heads,
// the last 611k), so a fixed share per workgroup ends when the slowest does, while taken heads let the faster ones
// take more.  Without them, workgroup b checks the candidates b + gridDim.x k 64 at a time (wave 0, one per lane) and
// processes the due ones in turn.
// With the due flag st.ctl[0] (set by the steps), a call in which no step made a head due reads one word and returns;
// otherwise the last workgroup to finish (counted in st.ctl[1]) clears both for the next call.
// With a due list (dlist, lq_decode_noalloc) the flush takes exactly the listed heads instead: workgroup b the entries
// b, b + gridDim.x, ...  An entry is flushed only if it names a row of this call whose (slot, head) is still due, and
// the workgroup claims the head first (hcnt L -> L + 1 by compare-and-swap), so an entry left by an interrupted call
// is skipped or, if it names a head due again, flushed once; the last workgroup to finish empties the list.
// `head(slot, hv0, mask, sched)` flushes the due heads hv0 + h (bit h of mask) of one unit with the whole workgroup
// and, with sched set, leaves the workgroup's next candidate in `due`, a word of the workgroup's shared memory.
template <int U>
__device__ __forceinline__ unsigned unit_mask(const lq_state& st, int slot, int hv0) {
  unsigned m = 0;
#pragma unroll
  for (int h = 0; h < U; ++h) m |= (st.hcnt[(long long)slot * st.HV + hv0 + h] == st.L ? 1u : 0u) << h;
  return m;
}

// DYN: the dynamic schedule (the launch has checked flush_dynamic: counters given, more candidates than workgroups);
// otherwise the static one.  Each is its own kernel instance.
template <int U = 1, bool DYN = false, class Head>
__device__ void flush_scan(unsigned long long& due, const lq_state& st, const int* __restrict__ idx, int N,
                           Head head) {
  const int NU = st.HV / U;                           // units per row
  const int total = N * NU;
  const int stride = gridDim.x;
  if (st.ctl && __hip_atomic_load(st.ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) return;   // uniform: nothing due
  if constexpr (DYN) {
    // dynamic schedule: candidate b first, then whichever the workgroup's counter hands out (each head takes the next
    // one near its end and leaves it in `due`); a candidate that is not due takes the next at once
    if (threadIdx.x == 0) due = blockIdx.x;
    __syncthreads();
    const int G = U == 1 ? st.HV / st.H : 1;
    for (;;) {
      const int c = (int)due;
      __syncthreads();                                // every thread has its candidate before a head rewrites `due`
      if (c >= total) break;
      const int p = sched_unit(c, G, total);
      const int n = p / NU, u = p - n * NU;
      const int slot = idx[n];
      const unsigned m = slot > 0 && slot < st.NS ? unit_mask<U>(st, slot, u * U) : 0u;
      if (m) {
        head(slot, u * U, m, st.sched);
      } else {
        if (threadIdx.x == 0) due = (unsigned long long)lqf::sched_next(st.sched);
        __syncthreads();
      }
    }
    // every workgroup's last take precedes its count here, so the last of a group counted clears the group's counter
    // for the next call
    const int grp = (int)(blockIdx.x % lqf::SCHED_GROUPS);
    const int members = (stride - grp + lqf::SCHED_GROUPS - 1) / lqf::SCHED_GROUPS;   // workgroups of the group
    int* ctr = lqf::sched_counter(st.sched);
    if (threadIdx.x == 0 &&
        (__hip_atomic_fetch_add(ctr, 1 << lqf::SCHED_BITS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >>
         lqf::SCHED_BITS) == members - 1)
      __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    for (int base = blockIdx.x; base < total; base += 64 * stride) {
      if (threadIdx.x < 64) {
        const int p = base + stride * (int)threadIdx.x;
        bool d = false;
        if (p < total) {
          const int n = p / NU, u = p - n * NU;
          const int slot = idx[n];
          d = slot > 0 && slot < st.NS && unit_mask<U>(st, slot, u * U) != 0;
        }
        const unsigned long long m = __ballot(d);
        if (threadIdx.x == 0) due = m;
      }
      __syncthreads();
      // the pass's due mask stays in the shared word (the static schedule passes no counters, so no head writes it):
      // nothing of the pass is held in registers across a head
      for (;;) {
        const unsigned long long m = due;
        __syncthreads();                              // every thread has the mask before thread 0 rewrites it
        if (!m) break;
        const int b = __ffsll((long long)m) - 1;
        if (threadIdx.x == 0) due = m & (m - 1);      // read again after the head's last barrier
        const int p = base + stride * b;
        const int n = p / NU, u = p - n * NU;
        const int slot = idx[n];
        head(slot, u * U, unit_mask<U>(st, slot, u * U), nullptr);
      }
    }
  }
  if (st.ctl) {                 // every workgroup has read the flag; the last one to finish clears it
    __syncthreads();
    if (threadIdx.x == 0 && atomicAdd(st.ctl + 1, 1) == (int)gridDim.x - 1) {
      __atomic_store_n(st.ctl, 0, __ATOMIC_RELAXED);
      __atomic_store_n(st.ctl + 1, 0, __ATOMIC_RELAXED);
    }
  }
}

// listed heads: a unit of U heads is flushed with the listed head alone in its mask (the unit's other head, when
// listed too, is another entry, flushed by its own workgroup: the flush of a unit never reads a head outside its mask)
template <int U = 1, class Head>
__device__ void flush_listed(unsigned long long& due, const lq_state& st, const int* __restrict__ idx, int N,
                             int* dlist, Head head) {
  const int HV = st.HV, L = st.L;
  const int cnt = min(__hip_atomic_load(dlist, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), LQ_DUE_MAX);
  if (cnt == 0) return;                               // uniform: nothing due (the list is already empty)
  for (int e = blockIdx.x; e < cnt; e += gridDim.x) {
    if (threadIdx.x == 0) {
      const int p = dlist[2 + e];
      long long take = -1;
      if (p >= 0 && p < N * HV) {
        const int n = p / HV, hv = p - n * HV, slot = idx[n];
        // claimed by moving its fill from L to L + 1 (the flush writes 0 at its end): an entry that names the same
        // head twice -- one left by a call whose flush launch failed, and this call's own -- is flushed once
        if (slot > 0 && slot < st.NS &&
            atomicCAS(st.hcnt + (long long)slot * HV + hv, L, L + 1) == L)
          take = (long long)slot * HV + hv;
      }
      due = (unsigned long long)take;
    }
    __syncthreads();
    const long long take = (long long)due;
    __syncthreads();
    if (take >= 0) {
      const int slot = (int)(take / HV), hv = (int)(take % HV);
      head(slot, hv - hv % U, 1u << (hv % U), nullptr);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0 && __hip_atomic_fetch_add(dlist + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                              (int)gridDim.x - 1) {
    __hip_atomic_store(dlist, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(dlist + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// MODE: how the workgroups find their heads -- FS_STATIC / FS_DYNAMIC (flush_scan with the static or the dynamic
// schedule) or FS_LISTED (the due list of lq_decode_noalloc, flush_listed).  Each is its own kernel instance, so that
// no path's registers weigh on another's (one kernel holding all three spilled up to 64 bytes per lane more).
enum { FS_STATIC = 0, FS_DYNAMIC = 1, FS_LISTED = 2 };

template <int K_ = KD, int V_ = VD, int RA = 4, int MODE = FS_STATIC>
__global__ __launch_bounds__(FT) __attribute__((amdgpu_waves_per_eu(4)))
void flush_kernel(lq_state st, const float* __restrict__ Q0, const int* __restrict__ idx, int N, float qmax,
                  int* dlist) {
  __shared__ FlushShared<RA> sh;
  auto head = [&](int slot, int hv, unsigned, int* sched) { flush_head<K_, V_, RA>(sh, st, Q0, slot, hv, qmax, sched); };
  if constexpr (MODE == FS_LISTED) flush_listed(sh.due, st, idx, N, dlist, head);
  else flush_scan<1, MODE == FS_DYNAMIC>(sh.due, st, idx, N, head);
}

template <int K_ = KD, int V_ = VD, int MODE = FS_STATIC, bool KDA = false>
__global__ __launch_bounds__(FT4) __attribute__((amdgpu_waves_per_eu(4)))
void flush4_kernel(lq_state st, const float* __restrict__ Q0, const int* __restrict__ idx, int N, float qmax,
                   int* dlist) {
  __shared__ FlushShared4 sh;
  auto head = [&](int slot, int hv, unsigned, int* sched) {
    flush_head4<K_, V_, true, KDA>(sh, st, Q0, slot, hv, qmax, sched);
  };
  if constexpr (MODE == FS_LISTED) flush_listed(sh.due, st, idx, N, dlist, head);
  else flush_scan<1, MODE == FS_DYNAMIC>(sh.due, st, idx, N, head);
}

// ------------------------------------------------------------------------------------------------------------------
// Flush of the 64-dim GDN heads (K = 64; kernels.py:1089-1097): four waves, the tile 64 key channels x 128 rows.
// (64, 128): one head per tile.  (64, 64) at even GQA: two heads hv0, hv0 + 1 of one key head stacked in the rows
// (HP = 2, the reference's packing), so that the tile is full and the pair's shared window keys enter one rank-L
// product.  Each head keeps its own arithmetic: the factor columns are block-diagonal (head h owns columns 4 h ..
// 4 h + 3 of every rank-R product, so the P, Q and Gram MFMAs separate by head by themselves), and the CholeskyQR, pn,
// the column scales Sk and the stores are per head.  (64, 64) at odd GQA: one head, rows 64.. zero (HP = 1).
// Wave w owns key channels 16 w .. 16 w + 15 and lane l holds
//     a[nt][i] = M[16 w + 4 (l >> 4) + i][v' = 16 nt + (l & 15)],   v' = 64 h + v for head h (HP = 2).
// A head outside the unit's due mask (one head of a pair due; a listed head whose partner is its own entry) loads as
// zeros and stores nothing.
// ------------------------------------------------------------------------------------------------------------------
constexpr int K64 = 64, ROWS = 128;

struct FlushShared64 {
  union {
    struct {
      bf16_t k[K64][OPS4];     // window keys K_j[c] of one half
      bf16_t u[2][ROWS][OPS4]; // hi / lo of w_j u_j[v'] of one half
    } op;
    struct {                   // after the rebuild
      f32x4 qpart[NW4][ROWS];  // per-wave partial Q rows (the row's head's four columns)
      float rmx[4 * NW4][ROWS];
      float rq[ROWS];
      f16_t ppT[8][K64];       // P16^T, column 4 h + r = factor r of head h
    } r;
  };
  float skl[2][K64];           // Sk per head
  float svr[ROWS];             // Sv pn / qmax per row
  float w[2][LPMAX];           // entry weights per head
  f32x4 uoc[2][K64];           // old U rows per head [c][a], a >= R zero
  f32x4 qov[ROWS];             // old Q rows [v'][a] of the row's head
  f16_t uoT[8][K64];           // old U^T, row 4 h + a
  f16_t qoT[4][ROWS];          // old Q^T of the row's head
  f16_t qT[4][ROWS];           // Q^T operand of the P steps (row's head): fp16 Q0, then Q16
  f32x4 qv[ROWS];              // Q rows of the row's head: fp32, then Q16
  unsigned long long due;
};
static_assert(sizeof(FlushShared64) <= 40960, "four workgroups per CU");

// window rows of one half: thread t takes entries 2 (t % 16), + 1 and columns 8 (t / 16) .. + 7 -- keys for the
// first 64 columns, the rows v' of the pair's values for all 128 (rows past the heads, or of a head outside the mask,
// zero)
template <int V_, int HP>
__device__ __forceinline__ void load_half64(WinHalf& r, const lq_state& st, int slot, int hv0, unsigned mask, int hf) {
  const int G = st.HV / st.H, hk = hv0 / G, L = st.L;
  const bf16_t* Kb = (const bf16_t*)st.Kbuf + ((long long)slot * st.H + hk) * L * K64;
  const int t = opaque_tid(), jp = t % 16, c8 = (t / 16) * 8;
  const int hh = min(c8 / V_, HP - 1), v = c8 - hh * V_;
  const bool uok = c8 < HP * V_ && ((mask >> hh) & 1);
  const bf16_t* Ub = (const bf16_t*)st.Ubuf + ((long long)slot * st.HV + hv0 + hh) * L * V_ + (c8 < HP * V_ ? v : 0);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int j = HALF * hf + 2 * jp + k, jr = j < L ? j : 0;
    const uint4 kx = *(const uint4*)(Kb + (long long)jr * K64 + min(c8, K64 - 8));
    const uint4 ux = *(const uint4*)(Ub + (long long)jr * V_);
    r.k[k] = keep4(kx, c8 < K64);
    r.u[k] = keep4(ux, uok);
  }
}
template <int V_, int HP>
__device__ __forceinline__ void store_half64(FlushShared64& sh, const WinHalf& r, int L, int hf) {
#pragma clang fp contract(off)    // the split is of the fp32-rounded product (kernels.py:1509-1511)
  const int t = opaque_tid(), jl = 2 * (t % 16), c8 = (t / 16) * 8;
  const int hh = min(c8 / V_, HP - 1);
  const int j0 = HALF * hf + jl;
  const float w0 = j0 < L ? sh.w[hh][j0] : 0.f, w1 = j0 + 1 < L ? sh.w[hh][j0 + 1] : 0.f;
  const uint32_t ka[4] = {r.k[0].x, r.k[0].y, r.k[0].z, r.k[0].w}, kb[4] = {r.k[1].x, r.k[1].y, r.k[1].z, r.k[1].w};
  const uint32_t ua[4] = {r.u[0].x, r.u[0].y, r.u[0].z, r.u[0].w}, ub[4] = {r.u[1].x, r.u[1].y, r.u[1].z, r.u[1].w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int x = e >> 1;
    const bool odd = e & 1;
    const uint32_t sel = odd ? 0x07060302u : 0x05040100u;
    if (c8 < K64) *(uint32_t*)&sh.op.k[c8 + e][jl] = __builtin_amdgcn_perm(kb[x], ka[x], sel);
    const float wu0 = w0 * (odd ? bf_hi(ua[x]) : bf_lo(ua[x]));
    const float wu1 = w1 * (odd ? bf_hi(ub[x]) : bf_lo(ub[x]));
    const uint32_t hi = pk_bf16_kept(wu0, wu1);
    *(uint32_t*)&sh.op.u[0][c8 + e][jl] = hi;
    *(uint32_t*)&sh.op.u[1][c8 + e][jl] = pk_bf16(wu0 - bf_lo(hi), wu1 - bf_hi(hi));
  }
}
// acc[c][v'] += sum_j K_j[c] B[v'][j] over one staged half
template <int NTV>
__device__ __forceinline__ void rebuild_half64(Tile& t, const bf16_t (*A)[OPS4], const bf16_t (*B)[OPS4]) {
  const int l = lane_id(), w = wave_id(), q = l >> 4;
  const bf16x8 af = *(const bf16x8*)&A[16 * w + (l & 15)][8 * q];
#pragma unroll
  for (int nt = 0; nt < NTV; ++nt) {
    const bf16x8 bfr = *(const bf16x8*)&B[16 * nt + (l & 15)][8 * q];
    t.a[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr, t.a[nt], 0, 0, 0);
  }
}
// M[a][r] = sum over the rows v' of head h of X[v'][a] Y[v'][r] (4 x 4; X^T, Y^T fp16 [4][128]); every lane gets all
template <int V_>
__device__ __forceinline__ void gram_head(const f16_t (*XT)[ROWS], const f16_t (*YT)[ROWS], int h, float M[4][4]) {
  const int l = lane_id(), q = l >> 4, l16 = l & 15;
  const f16x8 z8 = {};
  f32x4 macc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < V_ / 32; ++ks) {
    const int v0 = h * V_ + 32 * ks + 8 * q;
    const f16x8 ao = l16 < 4 ? *(const f16x8*)&XT[l16][v0] : z8;
    const f16x8 by = l16 < 4 ? *(const f16x8*)&YT[l16][v0] : z8;
    macc = mma32(ao, by, macc);
  }
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int r = 0; r < 4; ++r) M[a][r] = rl(macc[a], r);
}
// P = B^T Q + pn_h U_old (Q_old^T Q) per head, fp16-rounded (kernels.py:1580-1700): lanes l < 16 HP return
// P_h[16 w + (l & 15)][i] of head h = l >> 4 (zero for i >= R); the other lanes zeros.  bt: the transposed packing.
template <int V_, int HP>
__device__ __forceinline__ f32x4 p_step64(const FlushShared64& sh, const f16x4 bt[8], const float pn[2], int R) {
  constexpr int NTV = HP * V_ / 16;                   // row tiles holding data
  const int l = lane_id(), w = wave_id(), q = l >> 4, l16 = l & 15;
  float M[2][4][4];
#pragma unroll
  for (int h = 0; h < HP; ++h) gram_head<V_>(sh.qoT, sh.qT, h, M[h]);
  const f16x4 z4 = {};
  f32x4 pacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int nt = 0; nt < NTV; ++nt) {                  // P^T[4 h + r][c] = sum over head h's rows of Q^T[r][v'] B[c][v']
    const int hh = (16 * nt) / V_;
    const f16x4 aq = (l16 < 4 * HP && (l16 >> 2) == hh) ? *(const f16x4*)&sh.qT[l16 & 3][16 * nt + 4 * q] : z4;
    pacc = mma16(aq, bt[nt], pacc);
  }
  const int qh = q < HP ? q : HP - 1;
  const f32x4 uo = sh.uoc[qh][16 * w + l16];
  f32x4 p;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float corr = 0.f;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      float m = M[0][a][i];
      if (HP == 2) m = qh == 1 ? M[1][a][i] : m;
      corr = a == 0 ? uo[0] * m : corr + uo[a] * m;
    }
    const float pnh = qh == 1 ? pn[1] : pn[0];
    p[i] = (q < HP && i < R) ? hround(pacc[i] + pnh * corr) : 0.f;
  }
  return p;
}

template <int V_, int HP>
__device__ void flush_head64(FlushShared64& sh, const lq_state& st, const float* __restrict__ Q0, int slot, int hv0,
                             unsigned mask, float qmax, int* sched = nullptr) {
  static_assert(HP * V_ <= ROWS && V_ % 32 == 0, "rows of the tile");
  constexpr int NTV = HP * V_ / 16;
  const int HV = st.HV, L = st.L, R = st.R;
  const int tid = opaque_tid(), l = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), q = l >> 4, l16 = l & 15;
  const long long s0 = (long long)slot * HV + hv0;
  char* base[2];
  float pn[2], rpn[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int hs = h < HP ? h : 0;
    base[h] = block_base(st, slot, hv0 + hs);
    const float pb = st.Pbuf[s0 + hs];
    pn[h] = ((mask >> h) & 1) ? fmaxf(pb, LQ_PNMIN) : 1.f;                        // kernels.py:1471
    rpn[h] = 1.0f / pn[h];                                                         // kernels.py:1477
  }
  // ---- stage 1: every load up front.  Thread t < 64: column c = t of each head (Sk, U_old); 64 <= t < 192: row
  //      v' = t - 64 (Sv, Q_old, Q0); 192 <= t: window weight j = t - 192 of each head ----
  float uqv[4], q0v[4], scv;
  const int vr = tid - K64;
  const bool rowt = tid >= K64 && tid < K64 + ROWS;
  const bool rin = rowt && vr < HP * V_;                                           // a row of the unit's heads
  const int hr = rin ? vr / V_ : 0;
  const bool rok = rin && ((mask >> hr) & 1);
  const int vq = rin ? vr - hr * V_ : 0;                                           // the row within its head
  const int vv = rok ? vq : 0;
  float colsk[2], coluq[2][4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const bool cok = tid < K64 && h < HP && ((mask >> h) & 1);
    const float* Skh = (const float*)(base[h] + V_ * K64);
    const f16_t* UQh = (const f16_t*)(base[h] + V_ * K64 + 4 * (K64 + V_));
    const int c = tid < K64 ? tid : 0;
    const float x = Skh[c];
    colsk[h] = cok ? x : 0.f;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const float y = h2f(UQh[min(a, R - 1) * (K64 + V_) + c]);
      coluq[h][a] = (cok && a < R) ? y : 0.f;
    }
  }
  {
    char* bh_ = hr ? base[1] : base[0];              // (selects, not register-array indexing, for per-thread heads)
    const float* Svh = (const float*)(bh_ + V_ * K64 + 4 * K64);
    const f16_t* UQh = (const f16_t*)(bh_ + V_ * K64 + 4 * (K64 + V_));
    const float x = Svh[vv];
    scv = rok ? x : 0.f;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const float y = h2f(UQh[min(a, R - 1) * (K64 + V_) + K64 + vv]);
      uqv[a] = (rok && a < R) ? y : 0.f;
      const float z = Q0[vq * R + min(a, R - 1)];
      q0v[a] = (rin && a < R) ? z : 0.f;
    }
  }
  const int jw = tid - (K64 + ROWS);                                               // window weight j for tid >= 192
  float wj[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int hs = h < HP ? h : 0;
    const float x = st.Wbuf[(s0 + hs) * L + min(max(jw, 0), L - 1)];
    wj[h] = (jw >= 0 && jw < L && h < HP && ((mask >> h) & 1)) ? x : 0.f;
  }
  WinHalf win;
  load_half64<V_, HP>(win, st, slot, hv0, mask, 0);
  uint32_t wds[8];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {                    // code words of the lane's tile entries
    const int v2 = 16 * nt + l16;
    const int h = min((16 * nt) / V_, HP - 1);
    const bool ok = nt < NTV && ((mask >> h) & 1);
    const int8_t* Sq = (const int8_t*)base[h];
    const uint32_t x = *(const uint32_t*)(Sq + (ok ? v2 - h * V_ : 0) * K64 + 16 * w + 4 * q);
    wds[nt] = ok ? x : 0u;
  }
  if (tid < K64) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      sh.skl[h][tid] = colsk[h];
      f32x4 u;
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        u[a] = coluq[h][a];
        sh.uoT[4 * h + a][tid] = f2h(u[a]);
      }
      sh.uoc[h][tid] = u;
    }
  } else if (rowt) {
    sh.svr[vr] = scv * ((hr ? pn[1] : pn[0]) / qmax);                              // kernels.py:1483
    f32x4 o;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      o[a] = uqv[a];
      sh.qoT[a][vr] = f2h(o[a]);
      sh.qT[a][vr] = f2h(hround(q0v[a]));                                          // kernels.py:1573-1577
    }
    sh.qov[vr] = o;
  } else {
    sh.w[0][jw] = wj[0];
    sh.w[1][jw] = wj[1];
  }
  __syncthreads();

  // ---- stage 2: B = deq(S0) pn + window, fp16, the window half by half (kernels.py:1483-1571) ----
  f16x4 bh[8], bt[8];
  {
    Tile t;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) t.a[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    store_half64<V_, HP>(sh, win, L, 0);
    __syncthreads();
    rebuild_half64<NTV>(t, sh.op.k, sh.op.u[0]);
    rebuild_half64<NTV>(t, sh.op.k, sh.op.u[1]);
    if (L > HALF) {
      load_half64<V_, HP>(win, st, slot, hv0, mask, 1);
      __syncthreads();
      store_half64<V_, HP>(sh, win, L, 1);
      __syncthreads();
      rebuild_half64<NTV>(t, sh.op.k, sh.op.u[0]);
      rebuild_half64<NTV>(t, sh.op.k, sh.op.u[1]);
    }
    {                                                 // + codes x svr[v'] x skl[h][c], after the window products
#pragma clang fp contract(off)
      const int c0 = 16 * w + 4 * q;
#pragma unroll
      for (int nt = 0; nt < NTV; ++nt) {
        const int hh = (16 * nt) / V_;
        const float rv = sh.svr[16 * nt + l16];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          t.a[nt][i] = t.a[nt][i] + ((float)(int)(int8_t)(wds[nt] >> (8 * i)) * rv) * sh.skl[hh][c0 + i];
      }
    }
    f16x4 ident;
#pragma unroll
    for (int i = 0; i < 4; ++i) ident[i] = (4 * q + i == l16) ? (_Float16)1.0f : (_Float16)0.0f;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      bh[nt] = to_h4(t.a[nt]);
      bt[nt] = to_h4(mma16(bh[nt], ident, f32x4{0.f, 0.f, 0.f, 0.f}));
    }
  }

  // ---- stage 3: subspace iteration with the per-head corrections (kernels.py:1580-1842) ----
  const f32x4 p16 = p_step64<V_, HP>(sh, bt, pn, R);
  __syncthreads();                                    // every wave is past the rebuild: the operand region is free
  if (q < HP) {
#pragma unroll
    for (int i = 0; i < 4; ++i) sh.r.ppT[4 * q + i][16 * w + l16] = f2h(p16[i]);
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  {
    const f16x4 z4 = {};
    const f16x4 ap = l16 < 4 * HP ? *(const f16x4*)&sh.r.ppT[l16][16 * w + 4 * q] : z4;   // A[4 h + r][c]
#pragma unroll
    for (int nt = 0; nt < NTV; ++nt) {
      const f32x4 d = mma16(ap, bh[nt], f32x4{0.f, 0.f, 0.f, 0.f});              // Q^T[4 q + i][16 nt + l]
      if (q == (16 * nt) / V_) sh.r.qpart[w][16 * nt + l16] = d;                  // the row's head's columns
    }
  }
  __syncthreads();
  if (tid < HP * V_) {                                // one row v' per thread; the head is wave-uniform
    const int v2 = tid, hh = v2 / V_;
    float M2[4][4];                                   // U_old_h^T P16_h over the 64 channels
    {
      const f16x8 z8 = {};
      f32x4 macc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < K64 / 32; ++ks) {
        const f16x8 ao = l16 < 4 ? *(const f16x8*)&sh.uoT[4 * hh + l16][32 * ks + 8 * q] : z8;
        const f16x8 bp = l16 < 4 ? *(const f16x8*)&sh.r.ppT[4 * hh + l16][32 * ks + 8 * q] : z8;
        macc = mma32(ao, bp, macc);
      }
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) M2[a][r] = rl(macc[a], r);
    }
    f32x4 s = sh.r.qpart[0][v2];
#pragma unroll
    for (int w2 = 1; w2 < NW4; ++w2) s += sh.r.qpart[w2][v2];
    const f32x4 qo = sh.qov[v2];
    const float pnh = hh ? pn[1] : pn[0];
#pragma unroll
    for (int r = 0; r < 4; ++r) s[r] += pnh * (qo[0] * M2[0][r] + qo[1] * M2[1][r] + qo[2] * M2[2][r] + qo[3] * M2[3][r]);
    sh.qv[v2] = s;
  } else if (tid < ROWS) {
    sh.qv[tid] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  __syncthreads();
  if (w == 0) {                                       // CholeskyQR2 per head, fp16 Q (kernels.py:1778-1835)
    __builtin_amdgcn_s_setprio(3);
    f32x4 p0 = sh.qv[l], p1 = sh.qv[l + 64];
#pragma unroll
    for (int r = 0; r < 4; ++r) { if (r >= R) { p0[r] = 0.f; p1[r] = 0.f; } }
    if (HP == 2) {                                    // rows l: head 0, rows l + 64: head 1
      cholqr_pass1(p0);
      cholqr_pass1(p0);
      cholqr_pass1(p1);
      cholqr_pass1(p1);
    } else {
      cholqr_pass(p0, p1);
      cholqr_pass(p0, p1);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p0[r] = r < R ? hround(p0[r]) : 0.f;
      p1[r] = (r < R && l + 64 < HP * V_) ? hround(p1[r]) : 0.f;
      sh.qT[r][l] = f2h(p0[r]);
      sh.qT[r][l + 64] = f2h(p1[r]);
    }
    sh.qv[l] = p0;
    sh.qv[l + 64] = p1;
    __builtin_amdgcn_s_setprio(0);
  }
  __syncthreads();
  const f32x4 u16 = p_step64<V_, HP>(sh, bt, pn, R);  // U16 (lanes < 16 HP: head l >> 4)

  // ---- stage 4: residual E = fp16(pn (B / pn + Q_old U_old^T) - Q U^T) per head (kernels.py:1888-1928) ----
  Tile t;
  {
    const f16x4 z4 = {};
    f32x4 uh[2];                                      // head h's U16 rows in lanes l < 16 (k = a of the MFMA)
    uh[0] = u16;
#pragma unroll
    for (int i = 0; i < 4; ++i) uh[1][i] = __shfl_xor(u16[i], 16);
    f16x4 auo[2], aun[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      auo[h] = q == 0 ? to_h4(sh.uoc[h][16 * w + l16]) : z4;                     // A[c][a] = U_old
      aun[h] = q == 0 ? to_h4(-uh[h]) : z4;                                      // A[c][r] = -U16
    }
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      if (nt < NTV) {
        const int hh = (16 * nt) / V_, v2 = 16 * nt + l16;
        const f16x4 bqo = q == 0 ? to_h4(sh.qov[v2]) : z4;                       // B[a][v'] = Q_old^T
        const f16x4 bqn = q == 0 ? to_h4(sh.qv[v2]) : z4;                        // B[r][v'] = Q16^T
        f32x4 e = from_h4(bh[nt]) * rpn[hh];
        e = mma16(auo[hh], bqo, e);
        e *= pn[hh];
        e = mma16(aun[hh], bqn, e);
#pragma unroll
        for (int i = 0; i < 4; ++i) t.a[nt][i] = hround(e[i]);
      } else {
        t.a[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  }

  // ---- stage 5: column smoothing scales per head (kernels.py:1929-1958) ----
  float rsk[2][4];
#pragma unroll
  for (int h = 0; h < HP; ++h) {
    float cs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float x = 0.f;
#pragma unroll
      for (int nt = h * V_ / 16; nt < (h + 1) * V_ / 16; ++nt) x += fabsf(t.a[nt][i]);
      cs[i] = sum16(x);
    }
    const int ic = l & 3;
    const float msum = (ic == 0 ? cs[0] : ic == 1 ? cs[1] : ic == 2 ? cs[2] : cs[3]) * (1.0f / V_);
    const float sq = sqrtf(msum);
    const float rs = fminf(1.0f / sq, 1.0f / LQ_EPS);
    if (l16 < 4 && ((mask >> h) & 1)) ((float*)(base[h] + V_ * K64))[16 * w + 4 * q + l16] = fmaxf(sq, LQ_EPS);
    rsk[h][0] = dpp<0x00>(rs);
    rsk[h][1] = dpp<0x55>(rs);
    rsk[h][2] = dpp<0xaa>(rs);
    rsk[h][3] = dpp<0xff>(rs);
  }
  if (HP == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) rsk[1][i] = rsk[0][i];
  }
  int next = 0;                                       // dynamic schedule: this workgroup's next candidate
  if (sched && tid == 0) next = sched_take(sched);
  // ---- stage 6: row scales and codes (kernels.py:1974-2009) ----
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const int hh = min((16 * nt) / V_, 1);
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      t.a[nt][i] *= rsk[hh][i];
      m = fmaxf(m, fabsf(t.a[nt][i]));
    }
    sh.r.rmx[4 * w + q][16 * nt + l16] = m;
  }
  __syncthreads();
  if (tid < ROWS) {
    float m = sh.r.rmx[0][tid];
#pragma unroll
    for (int k = 1; k < 4 * NW4; ++k) m = fmaxf(m, sh.r.rmx[k][tid]);
    const float rmax = fmaxf(m, LQ_EPS);
    const int hh = min(tid / V_, HP - 1);
    char* bhh = hh ? base[1] : base[0];
    if (tid < HP * V_ && ((mask >> hh) & 1)) ((float*)(bhh + V_ * K64 + 4 * K64))[tid - hh * V_] = rmax;
    sh.r.rq[tid] = qmax * (1.0f / rmax);
  }
  __syncthreads();
#pragma unroll
  for (int nt = 0; nt < NTV; ++nt) {
    const int hh = (16 * nt) / V_, v2 = 16 * nt + l16;
    const float rq = sh.r.rq[v2];
    uint32_t b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = __float_as_uint(__builtin_fmaf(t.a[nt][i], rq, 12582912.0f));   // RNE via 1.5 2^23
    const uint32_t lo = __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u), hi = __builtin_amdgcn_perm(b[3], b[2], 0x0c0c0400u);
    if ((mask >> hh) & 1) *(uint32_t*)(base[hh] + (v2 - hh * V_) * K64 + 16 * w + 4 * q) = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
  }
  // ---- stage 7: factors, window reset (kernels.py:1836-1842, 2014-2025) ----
  if (q < HP && ((mask >> q) & 1)) {
    f16_t* UQ = (f16_t*)((q ? base[1] : base[0]) + V_ * K64 + 4 * (K64 + V_));
    for (int r = 0; r < R; ++r) UQ[r * (K64 + V_) + 16 * w + l16] = f2h(u16[r]);
  }
  if (tid < HP * V_) {
    const int hh = tid / V_;
    if ((mask >> hh) & 1) {
      f16_t* UQ = (f16_t*)((hh ? base[1] : base[0]) + V_ * K64 + 4 * (K64 + V_));
      for (int r = 0; r < R; ++r) UQ[r * (K64 + V_) + K64 + tid - hh * V_] = f2h(sh.qv[tid][r]);
    }
  }
#pragma unroll
  for (int h = 0; h < HP; ++h) {
    if ((mask >> h) & 1) {
      if (tid < L) st.Wbuf[(s0 + h) * L + tid] = 0.f;
      if (tid == 0) {
        st.Pbuf[s0 + h] = 1.f;
        st.hcnt[s0 + h] = 0;
      }
    }
  }
  if (sched && tid == 0) sh.due = (unsigned long long)sched_candidate(take_result(next));
  __syncthreads();                                    // LDS reuse by the next unit of this workgroup
}

template <int V_, int HP, int MODE = FS_STATIC>
__global__ __launch_bounds__(FT4) __attribute__((amdgpu_waves_per_eu(4)))
void flush64_kernel(lq_state st, const float* __restrict__ Q0, const int* __restrict__ idx, int N, float qmax,
                    int* dlist) {
  __shared__ FlushShared64 sh;
  auto head = [&](int slot, int hv0, unsigned mask, int* sched) {
    flush_head64<V_, HP>(sh, st, Q0, slot, hv0, mask, qmax, sched);
  };
  if constexpr (MODE == FS_LISTED) flush_listed<HP>(sh.due, st, idx, N, dlist, head);
  else flush_scan<HP, MODE == FS_DYNAMIC>(sh.due, st, idx, N, head);
}

// ------------------------------------------------------------------------------------------------------------------
// standalone quantize of an fp32 state (kernels.py:2126-2242), and the KDA prefill checkpoint (state.py:130-142): the
// same subspace steps (P = MGS(S^T Q), Q = MGS(S P); U = fp16(S^T Q)), one round for GDN, three for KDA (the
// low-rank factoriser's iters = 3, kernels.py:2318-2326), then the residual codes.  KDA resets its window as
// state.py:138-142 does (Pbuf = 0 per channel, Gbuf = 1).
// ------------------------------------------------------------------------------------------------------------------
// Four waves per head (256 threads), so that four heads fit on a CU at <= 128 VGPRs (the flush's eight-wave layout
// fits two): wave w holds key channels 32 w .. 32 w + 31 as two groups of 16, lane l rows 16 nt + (l & 15) and, in group
// cg, channels 32 w + 16 cg + 4 (l >> 4) + i, i < 4 -- 64 fp32 of the state per lane.
constexpr int QW = 4;                 // waves per head
constexpr int QT = 64 * QW;           // threads per workgroup

struct QTile {
  f32x4 a[2][8];
};

template <int RA>
struct QuantShared {
  static constexpr int NB = RA / 4;  // blocks of four factor columns
  f32x4 qv[NB][VD];
  f32x4 pp[NB][KD];
  f32x4 qpart[QW][VD];               // one block's per-wave partial rows at a time
  float rowmax[QW][VD];
  float sk[KD];
  float rsk[KD];                     // 1 / Sk per column
  float rsv[VD];                     // qmax / Sv per row
};

// 16 values, each summed over the 16 lanes of a DPP row exactly as sum16 sums one (xor 1, xor 2, half mirror, mirror:
// the same two partial sums meet at every level, so the same bits), as a reduce-scatter: at each level a lane keeps
// one of each pair of values and adds its partner's partial of it, so lane l ends with the total of value
//   8 b3 + 4 (b2 ^ b3) + 2 (b1 ^ b2) + (b0 ^ b2)   (b = the bits of l mod 16),
// an assignment under which both lanes of every pair, at every level, hold partials of the same value.  45 VALU
// instructions where sixteen all-reductions take 64.
__device__ __forceinline__ float sum16_scatter(const float (&v)[16], int l) {
  const int b0 = l & 1, b1 = (l >> 1) & 1, b2 = (l >> 2) & 1, b3 = (l >> 3) & 1;
  const bool s1 = b0 ^ b2, s2 = b1 ^ b2, s3 = b2 ^ b3, s4 = b3;
  float r1[8], r2[4], r3[2];
#pragma unroll
  for (int j = 0; j < 8; ++j) r1[j] = (s1 ? v[2 * j + 1] : v[2 * j]) + dpp<DPP_XOR1>(s1 ? v[2 * j] : v[2 * j + 1]);
#pragma unroll
  for (int j = 0; j < 4; ++j) r2[j] = (s2 ? r1[2 * j + 1] : r1[2 * j]) + dpp<DPP_XOR2>(s2 ? r1[2 * j] : r1[2 * j + 1]);
#pragma unroll
  for (int j = 0; j < 2; ++j)
    r3[j] = (s3 ? r2[2 * j + 1] : r2[2 * j]) + dpp<DPP_HALF_MIRROR>(s3 ? r2[2 * j] : r2[2 * j + 1]);
  return (s4 ? r3[1] : r3[0]) + dpp<DPP_MIRROR>(s4 ? r3[0] : r3[1]);
}
__device__ __forceinline__ int sum16_scatter_index(int l) {
  const int b0 = l & 1, b1 = (l >> 1) & 1, b2 = (l >> 2) & 1, b3 = (l >> 3) & 1;
  return 8 * b3 + 4 * (b2 ^ b3) + 2 * (b1 ^ b2) + (b0 ^ b2);
}

// column sums sum_v M[v][c] X[v][r] for this lane's channels (the rows of one lane first, in order, then across its 16
// lanes): fn(cg, i, r, s) once per lane and group with the full sum of one (channel, column) pair, i = k >> 2 and
// r = k & 3 for k = sum16_scatter_index(l)
template <typename F>
__device__ __forceinline__ void colred_q(const QTile& t, const f32x4* X, F fn) {
  const int l = lane_id();
  const int k = sum16_scatter_index(l);
#pragma unroll
  for (int cg = 0; cg < 2; ++cg) {
    f32x4 acc[4] = {};
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const f32x4 xv = X[16 * nt + (l & 15)];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float m = t.a[cg][nt][i];
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][r] = fmaf(m, xv[r], acc[i][r]);
      }
    }
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) v[4 * i + r] = acc[i][r];
    fn(cg, k >> 2, k & 3, sum16_scatter(v, l));
  }
}

// part[w][v][r] = sum over this wave's 32 channels c of M[v][c] Y[c][r]  (caller sums the QW waves)
__device__ __forceinline__ void rowred_q(const QTile& t, const f32x4* Y, f32x4 (*part)[VD]) {
  const int l = lane_id(), w = wave_id(), q = l >> 4;
  f32x4 yc[2][4];
#pragma unroll
  for (int cg = 0; cg < 2; ++cg)
#pragma unroll
    for (int i = 0; i < 4; ++i) yc[cg][i] = Y[32 * w + 16 * cg + 4 * q + i];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cg = 0; cg < 2; ++cg)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float m = t.a[cg][nt][i];
#pragma unroll
        for (int r = 0; r < 4; ++r) s[r] = fmaf(m, yc[cg][i][r], s[r]);
      }
    ((float*)&part[w][16 * nt + (l & 15)])[q] = sum4_scatter(s);
  }
}

__device__ __forceinline__ f32x4 sum_parts_q(const f32x4 (*part)[VD], int v) {
  f32x4 s = part[0][v];
#pragma unroll
  for (int w = 1; w < QW; ++w) s += part[w][v];
  return s;
}

// rows l, l + 64 of the NB blocks X[b] as plain arrays (wave 0's view of a 128 x RA factor) and back
template <int RA>
__device__ __forceinline__ void rows_get(const f32x4 (*X)[128], int l, float (&p0)[RA], float (&p1)[RA]) {
#pragma unroll
  for (int b = 0; b < RA / 4; ++b) {
    const f32x4 x0 = X[b][l], x1 = X[b][l + 64];
#pragma unroll
    for (int i = 0; i < 4; ++i) { p0[4 * b + i] = x0[i]; p1[4 * b + i] = x1[i]; }
  }
}
template <int RA>
__device__ __forceinline__ void rows_put(f32x4 (*X)[128], int l, const float (&p0)[RA], const float (&p1)[RA]) {
#pragma unroll
  for (int b = 0; b < RA / 4; ++b) {
    X[b][l] = f32x4{p0[4 * b], p0[4 * b + 1], p0[4 * b + 2], p0[4 * b + 3]};
    X[b][l + 64] = f32x4{p1[4 * b], p1[4 * b + 1], p1[4 * b + 2], p1[4 * b + 3]};
  }
}

// RA: factor columns held (4, 8 or 16; R <= RA), as RA / 4 blocks of four that the reductions take one at a time
template <bool KDA, int K_ = KD, int V_ = VD, int RA = 4>
__global__ __launch_bounds__(QT) __attribute__((amdgpu_waves_per_eu(4)))
void quantize_kernel(lq_state st, const float* __restrict__ Q0, const int* __restrict__ idx, float qmax, int iters) {
  static_assert(!KDA || (K_ == KD && V_ == VD && RA == 4), "KDA heads are 128 x 128, R <= 4");
  constexpr int NB = RA / 4;
  __shared__ QuantShared<RA> sh;
  const int HV = st.HV, L = st.L, R = st.R;
  const int n = blockIdx.x / HV, hv = blockIdx.x - n * HV;
  const int slot = idx[n];
  if (slot <= 0 || slot >= st.NS) return;
  const long long sh_ = (long long)slot * HV + hv;
  const int tid = threadIdx.x, l = lane_id(), w = wave_id(), q = l >> 4;
  char* base = block_base(st, slot, hv);
  const float* S = (const float*)base;
  QTile t;                                            // a K_ x V_ < 128 x 128 head zero-padded (see flush_head)
#pragma unroll
  for (int cg = 0; cg < 2; ++cg) {
    const int c = 32 * w + 16 * cg + 4 * q;
    const bool cok = K_ == KD || c < K_;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int v = 16 * nt + (l & 15);
      const float4 x = *(const float4*)(S + (V_ == VD ? v : min(v, V_ - 1)) * K_ + (K_ == KD ? c : min(c, K_ - 4)));
      t.a[cg][nt] = (cok && (V_ == VD || v < V_)) ? f32x4{x.x, x.y, x.z, x.w} : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  if (tid < VD) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      f32x4 q0v;
      for (int i = 0; i < 4; ++i) q0v[i] = (4 * b + i < R && tid < V_) ? Q0[tid * R + 4 * b + i] : 0.f;
      sh.qv[b][tid] = q0v;
    }
  }
  __syncthreads();
  // P = S^T Q, MGS; Q = S P, MGS (`iters` rounds)
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
      colred_q(t, sh.qv[b], [&](int cg, int i, int r, float s) { ((float*)&sh.pp[b][32 * w + 16 * cg + 4 * q + i])[r] = s; });
    __syncthreads();
    if (w == 0) {
      __builtin_amdgcn_s_setprio(3);
      float p0[RA], p1[RA];
      rows_get<RA>(sh.pp, l, p0, p1);
      mgs_n<RA>(p0, p1, R);
      rows_put<RA>(sh.pp, l, p0, p1);
      __builtin_amdgcn_s_setprio(0);
    }
    __syncthreads();
    float p0[RA], p1[RA];                             // wave 0: the rows l, l + 64 of Q = S P, block by block
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      rowred_q(t, sh.pp[b], sh.qpart);
      __syncthreads();
      if (w == 0) {
        const f32x4 s0 = sum_parts_q(sh.qpart, l), s1 = sum_parts_q(sh.qpart, l + 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) { p0[4 * b + i] = s0[i]; p1[4 * b + i] = s1[i]; }
      }
      if (b + 1 < NB) __syncthreads();                // wave 0 has read the partials before the next block's
    }
    if (w == 0) {
      __builtin_amdgcn_s_setprio(3);
      mgs_n<RA>(p0, p1, R);
      rows_put<RA>(sh.qv, l, p0, p1);
      __builtin_amdgcn_s_setprio(0);
    }
    __syncthreads();
  }
  // U = fp16(S^T Q) straight to LDS (sh.pp is not read again before the next barrier), Q16 = fp16(Q)
#pragma unroll
  for (int b = 0; b < NB; ++b)
    colred_q(t, sh.qv[b], [&](int cg, int i, int r, float s) {
      ((float*)&sh.pp[b][32 * w + 16 * cg + 4 * q + i])[r] = 4 * b + r < R ? hround(s) : 0.f;
    });
  __syncthreads();                                    // every wave has read Q (sh.qv)
  if (tid < VD) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      f32x4 x = sh.qv[b][tid];
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = 4 * b + r < R ? hround(x[r]) : 0.f;
      sh.qv[b][tid] = x;
    }
  }
  __syncthreads();
  // E = S - Q16 U16^T on the matrix cores (kernels.py:2212-2217): the tile's lane layout is the D layout of
  // v_mfma_f32_16x16x4_f32 (register i of lane l: channel 32 w + 16 cg + 4 (l >> 4) + i, row 16 nt + (l & 15)), so the
  // tile is the accumulator, A = -U16 (lane l: channel 32 w + 16 cg + (l & 15), factor 4 b + (l >> 4)) and B = Q16
  // (lane l: row 16 nt + (l & 15), factor 4 b + (l >> 4)): one MFMA per (group, row tile) and block of four factors.
  // The fp16 factors' products are exact; only the sums round.
  {
    float nu[2][NB];
#pragma unroll
    for (int cg = 0; cg < 2; ++cg)
#pragma unroll
      for (int b = 0; b < NB; ++b) nu[cg][b] = -((const float*)&sh.pp[b][32 * w + 16 * cg + (l & 15)])[q];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      float qb[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) qb[b] = ((const float*)&sh.qv[b][16 * nt + (l & 15)])[q];
#pragma unroll
      for (int cg = 0; cg < 2; ++cg)
#pragma unroll
        for (int b = 0; b < NB; ++b)
          t.a[cg][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(nu[cg][b], qb[b], t.a[cg][nt], 0, 0, 0);
    }
  }
  // column sums of |E|; the scales below, once per column
#pragma unroll
  for (int cg = 0; cg < 2; ++cg)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float s = 0.f;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) s += fabsf(t.a[cg][nt][i]);
      s = sum16(s);
      if ((l & 15) == 0) sh.sk[32 * w + 16 * cg + 4 * q + i] = s;
    }
  __syncthreads();
  // E / Sk and E / (Sk Sv) (kernels.py:2224-2229) as products with reciprocals taken once per column and once per row
  // (within a few ulp of the quotients, below the codes' rounding step).  Each column's scale and its reciprocal are
  // formed by one lane and shared through LDS: lane l < 32 of wave w takes column 32 w + l (one square root and one
  // division per lane, where each lane formed those of its own eight columns, the same eight in all 16 lanes of its
  // row).  E rsk is kept in the tile: the row maxima and the codes take the same product.
  if (l < 32) {
    const float skc = fmaxf(sqrtf(sh.sk[32 * w + l] / (float)V_), LQ_EPS);   // kernels.py:2222
    sh.sk[32 * w + l] = skc;
    sh.rsk[32 * w + l] = 1.0f / skc;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  float rsk[2][4];
#pragma unroll
  for (int cg = 0; cg < 2; ++cg) {
    const f32x4 r4 = *(const f32x4*)&sh.rsk[32 * w + 16 * cg + 4 * q];
#pragma unroll
    for (int i = 0; i < 4; ++i) rsk[cg][i] = r4[i];
  }
  {
    float mrow[8], mx[2];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      float m = 0.f;
#pragma unroll
      for (int cg = 0; cg < 2; ++cg)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          t.a[cg][nt][i] = t.a[cg][nt][i] * rsk[cg][i];                         // kernels.py:2224-2227
          m = fmaxf(m, fabsf(t.a[cg][nt][i]));
        }
      mrow[nt] = m;
    }
    rowmax_scatter(mrow, mx);                         // lane group q: the wave's maxima of rows 16 (2 q + k) + l16
#pragma unroll
    for (int k = 0; k < 2; ++k) sh.rowmax[w][16 * (2 * q + k) + (l & 15)] = mx[k];
  }
  __syncthreads();
  // every read of the fp32 state is done: the checkpoint may now overwrite the block
  int8_t* Sq = (int8_t*)base;
  float* Sk = (float*)(base + V_ * K_);
  float* Sv = Sk + K_;
  f16_t* UQ = (f16_t*)(Sv + V_);
  // row scales once per row (threads 0-127), then read by every lane for its eight rows
  if (tid < VD) {
    float rm = sh.rowmax[0][tid];
#pragma unroll
    for (int w2 = 1; w2 < QW; ++w2) rm = fmaxf(rm, sh.rowmax[w2][tid]);
    const float svv = fmaxf(rm, LQ_EPS);
    sh.rsv[tid] = qmax / svv;
    if (V_ == VD || tid < V_) Sv[tid] = svv;
  }
  __syncthreads();
  // codes: |x| <= qmax (1 + 2^-22) since svv is the row's largest |E rsk| (or above it), so the rounding to the nearest
  // integer is the add of 1.5 2^23 (round to nearest even, as rintf) and the clamp to [-qmax, qmax] never binds for
  // a finite x; the code is the low byte of the sum
  uint32_t cw[2][8];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const int v = 16 * nt + (l & 15);
    const float rsv = sh.rsv[v];
#pragma unroll
    for (int cg = 0; cg < 2; ++cg) {
      uint32_t b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma clang fp contract(off)
        const float x = t.a[cg][nt][i] * rsv;                    // kernels.py:2229 (rounded before the add)
        b[i] = __float_as_uint(x + 12582912.0f);
      }
      const uint32_t lo = __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u), hi = __builtin_amdgcn_perm(b[3], b[2], 0x0c0c0400u);
      cw[cg][nt] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    }
  }
  if constexpr (K_ == KD && V_ == VD) {
    // the same lane layout as the four-wave flush's tile: four 16-byte stores per lane after its transpose
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t a0 = cw[0][2 * k], a1 = cw[1][2 * k], a2 = cw[0][2 * k + 1], a3 = cw[1][2 * k + 1];
      swap16(a0, a1);
      swap16(a2, a3);
      swap32(a0, a2);
      swap32(a1, a3);
      *(uint4*)(Sq + (16 * (2 * k + (q >> 1)) + (l & 15)) * KD + 32 * w + 16 * (q & 1)) = make_uint4(a0, a1, a2, a3);
    }
  } else {
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int v = 16 * nt + (l & 15);
#pragma unroll
      for (int cg = 0; cg < 2; ++cg) {
        const int c = 32 * w + 16 * cg + 4 * q;
        if ((V_ == VD || v < V_) && (K_ == KD || c < K_)) *(uint32_t*)(Sq + v * K_ + c) = cw[cg][nt];
      }
    }
  }
  if (tid < KD) {
    if (K_ == KD || tid < K_) {
      Sk[tid] = sh.sk[tid];
      for (int r = 0; r < R; ++r) UQ[r * (K_ + V_) + tid] = f2h(sh.pp[r >> 2][tid][r & 3]);
    }
  } else if (tid < KD + VD) {
    const int v = tid - KD;
    if (V_ == VD || v < V_)
      for (int r = 0; r < R; ++r) UQ[r * (K_ + V_) + K_ + v] = f2h(sh.qv[r >> 2][v][r & 3]);
  }
  if (tid < L) st.Wbuf[sh_ * L + tid] = 0.f;
  if (KDA) {
    if (tid < KD) st.Pbuf[sh_ * KD + tid] = 0.f;
    uint4* Gb = (uint4*)((f16_t*)st.Gbuf + sh_ * L * KD);                             // fp16 1.0 over the window
    for (int i = tid; i < L * KD / 8; i += QT) Gb[i] = make_uint4(0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u);
  }
  if (tid == 0) {
    if (!KDA) st.Pbuf[sh_] = 1.f;
    st.hcnt[sh_] = 0;
  }
}

// ------------------------------------------------------------------------------------------------------------------
// standalone quantize of the 64-dim GDN heads: the K = 64 flush's tile (64 key channels x 128 rows, four waves: wave w
// channels 16 w .. 16 w + 15, lane l rows 16 nt + (l & 15)) with the quantize's arithmetic per head
// (kernels.py:2126-2242).  (64, 64): two heads of the slot per workgroup (HV even), stacked in the rows; (64, 128):
// one head.  Per head: P = S^T Q0, MGS over the 64 channels; Q = S P, MGS over the head's rows; U = fp16(S^T Q);
// E = S - Q U^T; column scales, row scales and codes.
// ------------------------------------------------------------------------------------------------------------------
struct QuantShared64 {
  f32x4 qv[ROWS];              // Q rows of the row's head
  f32x4 pp[2][K64];            // P, then U, per head [c][r]
  f32x4 qpart[NW4][ROWS];      // per-wave partial rows of S P (16 channels each)
  float rowmax[NW4][ROWS];
  float sk[2][K64];
};

// per head h: pp[h][c][r] = sum over the head's rows v' of S[v'][c] X[v'][r] (X: the row's head's columns); the rows of
// a lane first, in order, then across its 16 lanes; fn(h, i, s) for the lane's channel 16 w + 4 (l >> 4) + i
template <int V_, int HP, typename F>
__device__ __forceinline__ void colred64(const Tile& t, const f32x4* X, F fn) {
  const int l = lane_id();
#pragma unroll
  for (int h = 0; h < HP; ++h) {
    f32x4 acc[4] = {};
#pragma unroll
    for (int nt = h * V_ / 16; nt < (h + 1) * V_ / 16; ++nt) {
      const f32x4 xv = X[16 * nt + (l & 15)];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][r] = fmaf(t.a[nt][i], xv[r], acc[i][r]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 s;
#pragma unroll
      for (int r = 0; r < 4; ++r) s[r] = sum16(acc[i][r]);
      fn(h, i, s);
    }
  }
}

template <int V_, int HP>
__global__ __launch_bounds__(FT4) __attribute__((amdgpu_waves_per_eu(4)))
void quantize64_kernel(lq_state st, const float* __restrict__ Q0, const int* __restrict__ idx, float qmax) {
  static_assert(HP * V_ <= ROWS, "rows of the tile");
  constexpr int NTV = HP * V_ / 16;
  __shared__ QuantShared64 sh;
  const int HV = st.HV, L = st.L, R = st.R;
  const int NU = HV / HP;
  const int n = blockIdx.x / NU, hv0 = (blockIdx.x - n * NU) * HP;
  const int slot = idx[n];
  if (slot <= 0 || slot >= st.NS) return;
  const long long s0 = (long long)slot * HV + hv0;
  const int tid = threadIdx.x, l = lane_id(), w = wave_id(), q = l >> 4, l16 = l & 15;
  char* base[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) base[h] = block_base(st, slot, hv0 + (h < HP ? h : 0));
  Tile t;                                             // t.a[nt][i] = S[v'][16 w + 4 q + i], v' = 16 nt + l16
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    if (nt < NTV) {
      const int h = (16 * nt) / V_, v = 16 * nt + l16 - h * V_;
      const float4 x = *(const float4*)((const float*)base[h] + v * K64 + 16 * w + 4 * q);
      t.a[nt] = f32x4{x.x, x.y, x.z, x.w};
    } else {
      t.a[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  if (tid < ROWS) {
    const bool rin = tid < HP * V_;
    const int v = rin ? tid % V_ : 0;
    f32x4 q0v;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float x = Q0[v * R + min(r, R - 1)];
      q0v[r] = (rin && r < R) ? x : 0.f;
    }
    sh.qv[tid] = q0v;
  }
  __syncthreads();
  // P = S^T Q, MGS over the channels; Q = S P, MGS over the head's rows (one round: GDN's ITERS = 1)
  colred64<V_, HP>(t, sh.qv, [&](int h, int i, f32x4 s) { if (l16 == 0) sh.pp[h][16 * w + 4 * q + i] = s; });
  __syncthreads();
  if (w == 0) {
    __builtin_amdgcn_s_setprio(3);
#pragma unroll
    for (int h = 0; h < HP; ++h) {
      f32x4 p = sh.pp[h][l];
      mgs1(p, R);
      sh.pp[h][l] = p;
    }
    __builtin_amdgcn_s_setprio(0);
  }
  __syncthreads();
#pragma unroll
  for (int nt = 0; nt < NTV; ++nt) {                  // partial rows over this wave's 16 channels
    const int h = (16 * nt) / V_;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 y = sh.pp[h][16 * w + 4 * q + i];
#pragma unroll
      for (int r = 0; r < 4; ++r) s[r] = fmaf(t.a[nt][i], y[r], s[r]);
    }
    ((float*)&sh.qpart[w][16 * nt + l16])[q] = sum4_scatter(s);
  }
  __syncthreads();
  if (w == 0) {
    __builtin_amdgcn_s_setprio(3);
    f32x4 p0 = sh.qpart[0][l], p1 = sh.qpart[0][l + 64];
#pragma unroll
    for (int w2 = 1; w2 < NW4; ++w2) { p0 += sh.qpart[w2][l]; p1 += sh.qpart[w2][l + 64]; }
    if (l + 64 >= HP * V_) p1 = f32x4{0.f, 0.f, 0.f, 0.f};
    if (HP == 2) {                                    // rows l: head 0, rows l + 64: head 1
      mgs1(p0, R);
      mgs1(p1, R);
    } else {
      mgs(p0, p1, R);
    }
    sh.qv[l] = p0;
    sh.qv[l + 64] = p1;
    __builtin_amdgcn_s_setprio(0);
  }
  __syncthreads();
  // U = fp16(S^T Q) (sh.pp is not read again before the next barrier), Q16 = fp16(Q)
  colred64<V_, HP>(t, sh.qv, [&](int h, int i, f32x4 s) {
    if (l16 == 0) {
      f32x4 u;
#pragma unroll
      for (int r = 0; r < 4; ++r) u[r] = r < R ? hround(s[r]) : 0.f;
      sh.pp[h][16 * w + 4 * q + i] = u;
    }
  });
  __syncthreads();
  if (tid < ROWS) {
    f32x4 x = sh.qv[tid];
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = r < R ? hround(x[r]) : 0.f;
    sh.qv[tid] = x;
  }
  __syncthreads();
  // E = S - Q16 U16^T on the matrix cores (kernels.py:2212-2217), as in quantize_kernel: the tile is the accumulator
  // of v_mfma_f32_16x16x4_f32 (register i of lane l: channel 16 w + 4 q + i, row 16 nt + l16), A = -U16 of the row
  // tile's head (lane l: channel 16 w + l16, factor q), B = Q16 (lane l: row 16 nt + l16, factor q)
#pragma unroll
  for (int nt = 0; nt < NTV; ++nt) {
    const int h = (16 * nt) / V_;
    const float nu = -((const float*)&sh.pp[h][16 * w + l16])[q];
    const float qb = ((const float*)&sh.qv[16 * nt + l16])[q];
    t.a[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(nu, qb, t.a[nt], 0, 0, 0);
  }
  // column scales per head (kernels.py:2222)
#pragma unroll
  for (int h = 0; h < HP; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 16 * w + 4 * q + i;
      float sa = 0.f;
#pragma unroll
      for (int nt = h * V_ / 16; nt < (h + 1) * V_ / 16; ++nt) sa += fabsf(t.a[nt][i]);
      sa = sum16(sa);
      const float skc = fmaxf(sqrtf(sa / (float)V_), LQ_EPS);                     // kernels.py:2222
      if (l16 == 0) sh.sk[h][c] = skc;
    }
  __syncthreads();
  float rsk[2][4];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) rsk[h][i] = h < HP ? 1.0f / sh.sk[h][16 * w + 4 * q + i] : 1.f;
#pragma unroll
  for (int nt = 0; nt < NTV; ++nt) {
    const int h = (16 * nt) / V_;
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) m = fmaxf(m, fabsf(t.a[nt][i] * rsk[h][i]));                   // kernels.py:2224-2227
    m = xor32_max(xor16_max(m));
    if (q == 0) sh.rowmax[w][16 * nt + l16] = m;
  }
  __syncthreads();
  // every read of the fp32 states is done: the checkpoints may now overwrite the blocks
#pragma unroll
  for (int nt = 0; nt < NTV; ++nt) {
    const int h = (16 * nt) / V_, v = 16 * nt + l16 - h * V_;
    float rm = sh.rowmax[0][16 * nt + l16];
#pragma unroll
    for (int w2 = 1; w2 < NW4; ++w2) rm = fmaxf(rm, sh.rowmax[w2][16 * nt + l16]);
    const float svv = fmaxf(rm, LQ_EPS);
    const float rsv = qmax / svv;
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = (t.a[nt][i] * rsk[h][i]) * rsv;                                         // kernels.py:2229
      const float cq = fminf(fmaxf(rintf(x), -qmax), qmax);
      word |= ((uint32_t)(int)cq & 0xffu) << (8 * i);
    }
    *(uint32_t*)(base[h] + v * K64 + 16 * w + 4 * q) = word;
    if (w == 0 && q == 0) ((float*)(base[h] + V_ * K64 + 4 * K64))[v] = svv;
  }
  if (tid < K64) {
#pragma unroll
    for (int h = 0; h < HP; ++h) {
      ((float*)(base[h] + V_ * K64))[tid] = sh.sk[h][tid];
      f16_t* UQ = (f16_t*)(base[h] + V_ * K64 + 4 * (K64 + V_));
      for (int r = 0; r < R; ++r) UQ[r * (K64 + V_) + tid] = f2h(sh.pp[h][tid][r]);
    }
  } else if (tid < K64 + HP * V_) {
    const int v2 = tid - K64, h = v2 / V_;
    f16_t* UQ = (f16_t*)((h ? base[1] : base[0]) + V_ * K64 + 4 * (K64 + V_));
    for (int r = 0; r < R; ++r) UQ[r * (K64 + V_) + K64 + v2 - h * V_] = f2h(sh.qv[v2][r]);
  }
#pragma unroll
  for (int h = 0; h < HP; ++h) {
    if (tid < L) st.Wbuf[(s0 + h) * L + tid] = 0.f;
    if (tid == 0) {
      st.Pbuf[s0 + h] = 1.f;
      st.hcnt[s0 + h] = 0;
    }
  }
}

// ------------------------------------------------------------------------------------------------------------------
// prefill dequant, GDN (kernels.py:2041-2123): S = P (deq(Sq) + Q U^T) + sum_{j<h} w_j u_j k_j^T, in place.  A head
// of K_ x V_ < 128 x 128 runs zero-padded in the tile (see flush_head) and writes its own rows / columns only.
// ------------------------------------------------------------------------------------------------------------------
template <int RA>
struct DeqShared {
  static constexpr int NB = RA / 4;
  bf16_t op[3][KD][OPS];       // window operands, as in the flush
  float skl[KD];               // Sk
  float svr[VD];               // Sv
  float w[LPMAX];
  f32x4 uoc[NB][KD];           // U rows [c][r], r >= R zero
  f32x4 qov[NB][VD];           // Q rows [v][r]
};

template <int K_ = KD, int V_ = VD, int RA = 4>
__global__ __launch_bounds__(FT) __attribute__((amdgpu_waves_per_eu(4)))
void dequant_kernel(lq_state st, const int* __restrict__ idx, float qmax) {
  constexpr int NB = RA / 4;
  __shared__ DeqShared<RA> sh;
  const int HV = st.HV, L = st.L, R = st.R;
  const int n = blockIdx.x / HV, hv = blockIdx.x - n * HV;
  const int slot = idx[n];
  if (slot <= 0 || slot >= st.NS) return;
  const long long sh_ = (long long)slot * HV + hv;
  const int tid = threadIdx.x, l = lane_id(), w = wave_id(), q = l >> 4;
  char* base = block_base(st, slot, hv);
  const int8_t* Sq = (const int8_t*)base;
  const float* Sk = (const float*)(base + V_ * K_);
  const float* Sv = Sk + K_;
  const f16_t* UQ = (const f16_t*)(Sv + V_);
  const int h = __builtin_amdgcn_readfirstlane(min(st.hcnt[sh_], L));   // uniform: one word per head
  const float P = st.Pbuf[sh_];
  const int LP = h > 0 ? ((h + 31) & ~31) : 32;
  const int cv = tid & 127;
  const bool colt = tid < KD;
  const int nc = colt ? K_ : V_;
  const bool cok = (K_ == KD && V_ == VD) || cv < nc;
  const int cvc = (K_ == KD && V_ == VD) ? cv : min(cv, nc - 1);
  const float scv = cok ? (colt ? Sk[cvc] : Sv[cvc]) : 0.f;
  float uqv[RA];
#pragma unroll
  for (int a = 0; a < RA; ++a) {
    const float x = h2f(UQ[min(a, R - 1) * (K_ + V_) + (colt ? 0 : K_) + cvc]);
    uqv[a] = (cok && a < R) ? x : 0.f;
  }
  const float wv = st.Wbuf[sh_ * L + min(tid, L - 1)];
  // an empty window (h == 0, uniform: the prefill of a slot just checkpointed) skips the window's loads, staging and
  // products
  WinRegs win;
  if (h > 0) load_window<K_, V_>(win, st, slot, hv, h, LP);
  uint32_t wds[8];
  load_code_words<K_, V_>(wds, Sq);
  if (tid < KD + VD) {
    if (tid < KD) sh.skl[cv] = scv;
    else sh.svr[cv] = scv;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const f32x4 fac = {uqv[4 * b], uqv[4 * b + 1], uqv[4 * b + 2], uqv[4 * b + 3]};
      if (tid < KD) sh.uoc[b][cv] = fac;
      else sh.qov[b][cv] = fac;
    }
  }
  if (tid < LPMAX) sh.w[tid] = tid < h ? wv : 0.f;
  __syncthreads();
  if (h > 0) store_window(sh, win, h, LP);
  Tile t;
  {
    const float inv = 1.0f / qmax;
    const int c0 = 16 * w + 4 * q;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int v = 16 * nt + (l & 15);
      const float rv = sh.svr[v];
      f32x4 qo[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) qo[b] = sh.qov[b][v];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = c0 + i;
        float x = (((float)(int)(int8_t)(wds[nt] >> (8 * i)) * inv) * sh.skl[c]) * rv;   // kernels.py:2107
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const f32x4 uo = sh.uoc[b][c];
#pragma unroll
          for (int a = 0; a < 4; ++a) x = fmaf(qo[b][a], uo[a], x);                    // kernels.py:2109-2111
        }
        t.a[nt][i] = x * P;                                                             // kernels.py:2113
      }
    }
  }
  if (h > 0) {
    __syncthreads();
    rebuild_mfma(t, sh.op[0], sh.op[1], LP / 32);
    rebuild_mfma(t, sh.op[0], sh.op[2], LP / 32);
  }
  __syncthreads();                                    // every wave has read its codes: the fp32 state may overwrite them
  float* S = (float*)base;                            // non-temporal: 64 KiB per head, written once (171 -> 165 us)
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const int v = 16 * nt + (l & 15);
    if ((K_ == KD || 16 * w + 4 * q < K_) && (V_ == VD || v < V_))
      __builtin_nontemporal_store(t.a[nt], (f32x4*)(S + v * K_ + 16 * w + 4 * q));
  }
  if (tid < L) st.Wbuf[sh_ * L + tid] = 0.f;
  if (tid == 0) {
    st.Pbuf[sh_] = 1.f;
    st.hcnt[sh_] = 0;
  }
}

// ------------------------------------------------------------------------------------------------------------------
// low-rank factoriser (kernels.py:2246-2314): x [n][K][V]; P = MGS(x Q), Q = MGS(x^T P) x iters; U = x Q
// ------------------------------------------------------------------------------------------------------------------
struct LowrankShared {           // the eight-wave layout's subspace vectors and per-wave row partial sums
  f32x4 qv[VD];
  f32x4 pp[KD];
  f32x4 qpart[NW][VD];
};

__global__ __launch_bounds__(FT) __attribute__((amdgpu_waves_per_eu(4)))
void lowrank_kernel(const float* __restrict__ x, const float* __restrict__ Q0, float* __restrict__ U,
                    float* __restrict__ Qo, int R, int iters) {
  __shared__ LowrankShared sh;
  const int b = blockIdx.x;
  const int tid = threadIdx.x, l = lane_id(), w = wave_id(), q = l >> 4;
  const float* X = x + (long long)b * KD * VD;
  Tile t;                                             // t[c][v] = x[c][v]
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const int v = 16 * nt + (l & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) t.a[nt][i] = X[(16 * w + 4 * q + i) * VD + v];
  }
  if (tid < VD) {
    f32x4 q0v;
    for (int r = 0; r < 4; ++r) q0v[r] = r < R ? Q0[tid * R + r] : 0.f;
    sh.qv[tid] = q0v;
  }
  __syncthreads();
  for (int it = 0; it < iters; ++it) {
    colred(t, sh.qv, [&](int i, f32x4 s) { if ((l & 15) == 0) sh.pp[16 * w + 4 * q + i] = s; });   // P = x Q
    __syncthreads();
    if (w == 0) {
      __builtin_amdgcn_s_setprio(3);
      f32x4 p0 = sh.pp[l], p1 = sh.pp[l + 64];
      mgs(p0, p1, R);
      sh.pp[l] = p0;
      sh.pp[l + 64] = p1;
      __builtin_amdgcn_s_setprio(0);
    }
    __syncthreads();
    rowred(t, sh.pp, sh.qpart);                       // Q = x^T P
    __syncthreads();
    if (w == 0) {
      f32x4 p0 = sum_parts(sh.qpart, l), p1 = sum_parts(sh.qpart, l + 64);
      mgs(p0, p1, R);
      sh.qv[l] = p0;
      sh.qv[l + 64] = p1;
    }
    __syncthreads();
  }
  colred(t, sh.qv, [&](int i, f32x4 s) {              // U = x Q
    if ((l & 15) == 0) {
      const int c = 16 * w + 4 * q + i;
      for (int r = 0; r < R; ++r) U[((long long)b * KD + c) * R + r] = s[r];
    }
  });
  if (tid < VD)
    for (int r = 0; r < R; ++r) Qo[((long long)b * VD + tid) * R + r] = sh.qv[tid][r];
}

// compute units of the current device (cached per device; the persistent kernels size their grids by it)
int num_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// head dims (K, V): (128, 128) for GDN and KDA; GDN also (64, 128) and (64, 64) (kernels.py:1089-1092)
bool head_dims(const lq_state* st, bool kda) {
  return (st->K == KD && st->V == VD) || (!kda && st->K == 64 && (st->V == 128 || st->V == 64));
}

// rmax: the entry point's largest rank for GDN 128 x 128 heads (every other head: R <= 4)
int check_block_state(const lq_state* st, bool need_buf, bool kda, int rmax) {
  if (!st || !st->ssm || !st->hcnt || !st->Wbuf || !st->Pbuf) return LQ_ERR_ARG;
  if (!head_dims(st, kda) || st->L < 1 || st->L > LPMAX || st->R < 1) return LQ_ERR_ARG;
  if (st->R > ((!kda && st->K == KD && st->V == VD) ? rmax : 4)) return LQ_ERR_ARG;
  if (st->H <= 0 || st->HV <= 0 || st->HV % st->H != 0 || st->NS <= 0) return LQ_ERR_ARG;
  if (st->slot_stride < (long long)st->HV * st->V * st->K || (st->slot_stride & 3)) return LQ_ERR_ARG;
  if (((uintptr_t)st->ssm & 15) != 0) return LQ_ERR_ARG;
  if (need_buf && (!st->Kbuf || !st->Ubuf)) return LQ_ERR_ARG;
  if (!buffers_aligned(st)) return LQ_ERR_ARG;
  return LQ_OK;
}

}  // namespace

int lq_check_flush(const lq_state* st, const float* Q0, const int* idx, int N, int kda, float qmax) {
  int rc = check_block_state(st, true, kda != 0, LQ_FLUSH_RMAX);
  if (rc) return rc;
  if (N < 0 || (N > 0 && (!Q0 || !idx)) || !(qmax >= 1.f && qmax <= 127.f) || (kda && !st->Gbuf)) return LQ_ERR_ARG;
  return LQ_OK;
}

// the kernel instance of a flush of `units` candidates on `grid` workgroups: listed, or the dynamic schedule when
// the counters are given and there are more candidates than workgroups (each workgroup then takes more than its
// first), else the static one
template <class F>
static void with_mode(const lq_state* st, const int* dlist, int units, unsigned grid, F&& launch) {
  if (dlist) launch(std::integral_constant<int, FS_LISTED>{});
  else if (st->sched && units > (int)grid && units < (1 << SCHED_BITS)) launch(std::integral_constant<int, FS_DYNAMIC>{});
  else launch(std::integral_constant<int, FS_STATIC>{});
}

int lq_launch_flush(const lq_state* st, const float* Q0, const int* idx, int N, int kda, float qmax, int* dlist,
                    hipStream_t s) {
  if (N == 0) return LQ_OK;
  const int total = N * st->HV;
  const dim3 g((unsigned)(total < 2 * num_cus() ? total : 2 * num_cus()));   // persistent: two workgroups per CU at most
  const dim3 g4((unsigned)(total < 4 * num_cus() ? total : 4 * num_cus()));  // four-wave flush: four per CU
  if (kda) {
    with_mode(st, dlist, total, g4.x, [&](auto m) {
      flush4_kernel<KD, VD, decltype(m)::value, true><<<g4, FT4, 0, s>>>(*st, Q0, idx, N, qmax, dlist);
    });
  } else if (st->K == KD && st->R > 4) {
    with_mode(st, dlist, total, g.x, [&](auto m) {
      flush_kernel<KD, VD, 8, decltype(m)::value><<<g, FT, 0, s>>>(*st, Q0, idx, N, qmax, dlist);
    });
  } else if (st->K == KD) {
    with_mode(st, dlist, total, g4.x, [&](auto m) {
      flush4_kernel<KD, VD, decltype(m)::value><<<g4, FT4, 0, s>>>(*st, Q0, idx, N, qmax, dlist);
    });
  } else if (st->V == VD) {
    with_mode(st, dlist, total, g4.x, [&](auto m) {
      flush64_kernel<128, 1, decltype(m)::value><<<g4, FT4, 0, s>>>(*st, Q0, idx, N, qmax, dlist);
    });
  } else if ((st->HV / st->H) % 2 == 0) {             // two heads of one key head per workgroup (kernels.py:1095-1097)
    const dim3 gp((unsigned)(total / 2 < 4 * num_cus() ? total / 2 : 4 * num_cus()));
    with_mode(st, dlist, total / 2, gp.x, [&](auto m) {
      flush64_kernel<64, 2, decltype(m)::value><<<gp, FT4, 0, s>>>(*st, Q0, idx, N, qmax, dlist);
    });
  } else {
    with_mode(st, dlist, total, g4.x, [&](auto m) {
      flush64_kernel<64, 1, decltype(m)::value><<<g4, FT4, 0, s>>>(*st, Q0, idx, N, qmax, dlist);
    });
  }
  return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_HIP;
}

extern "C" int lq_flush(const lq_state* st, const float* Q0, const int* idx, int N, int kda, float qmax, void* stream) {
  int rc = lq_check_flush(st, Q0, idx, N, kda, qmax);
  if (rc) return rc;
  return lq_launch_flush(st, Q0, idx, N, kda, qmax, nullptr, (hipStream_t)stream);
}

extern "C" int lq_quantize(const lq_state* st, const float* Q0, const int* idx, int N, float qmax, void* stream) {
  int rc = check_block_state(st, false, false, LQ_STEP_RMAX);
  if (rc) return rc;
  if (N < 0 || (N > 0 && (!Q0 || !idx)) || !(qmax >= 1.f && qmax <= 127.f)) return LQ_ERR_ARG;
  if (N == 0) return LQ_OK;
  const dim3 g((unsigned)(N * st->HV));
  hipStream_t s = (hipStream_t)stream;
  if (st->K == KD && st->R > 8) quantize_kernel<false, KD, VD, 16><<<g, QT, 0, s>>>(*st, Q0, idx, qmax, 1);
  else if (st->K == KD && st->R > 4) quantize_kernel<false, KD, VD, 8><<<g, QT, 0, s>>>(*st, Q0, idx, qmax, 1);
  else if (st->K == KD) quantize_kernel<false><<<g, QT, 0, s>>>(*st, Q0, idx, qmax, 1);
  else if (st->V == VD) quantize64_kernel<128, 1><<<g, FT4, 0, s>>>(*st, Q0, idx, qmax);
  else if (st->HV % 2 == 0)                           // two heads of the slot per workgroup
    quantize64_kernel<64, 2><<<dim3((unsigned)(N * st->HV / 2)), FT4, 0, s>>>(*st, Q0, idx, qmax);
  else quantize64_kernel<64, 1><<<g, FT4, 0, s>>>(*st, Q0, idx, qmax);
  return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_HIP;
}

extern "C" int lq_kda_checkpoint(const lq_state* st, const float* Q0, const int* idx, int N, float qmax, void* stream) {
  int rc = check_block_state(st, false, true, 4);
  if (rc) return rc;
  if (N < 0 || (N > 0 && (!Q0 || !idx)) || !(qmax >= 1.f && qmax <= 127.f) || !st->Gbuf) return LQ_ERR_ARG;
  if (N == 0) return LQ_OK;
  quantize_kernel<true><<<dim3((unsigned)(N * st->HV)), QT, 0, (hipStream_t)stream>>>(*st, Q0, idx, qmax, 3);
  return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_HIP;
}

extern "C" int lq_kda_dequant(const lq_state* st, const int* idx, int N, float qmax, void* stream) {
  int rc = check_block_state(st, true, true, 4);
  if (rc) return rc;
  if (N < 0 || (N > 0 && !idx) || !(qmax >= 1.f && qmax <= 127.f) || !st->Gbuf) return LQ_ERR_ARG;
  if (N == 0) return LQ_OK;
  lq_launch_kda_dequant4(st, idx, N, qmax, (hipStream_t)stream);
  return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_HIP;
}

extern "C" int lq_dequant(const lq_state* st, const int* idx, int N, float qmax, void* stream) {
  int rc = check_block_state(st, true, false, LQ_STEP_RMAX);
  if (rc) return rc;
  if (N < 0 || (N > 0 && !idx) || !(qmax >= 1.f && qmax <= 127.f)) return LQ_ERR_ARG;
  if (N == 0) return LQ_OK;
  const dim3 g((unsigned)(N * st->HV));
  hipStream_t s = (hipStream_t)stream;
  if (st->K == KD && st->R > 8) dequant_kernel<KD, VD, 16><<<g, FT, 0, s>>>(*st, idx, qmax);
  else if (st->K == KD && st->R > 4) dequant_kernel<KD, VD, 8><<<g, FT, 0, s>>>(*st, idx, qmax);
  else if (st->K == KD) lq_launch_dequant4(st, idx, N, qmax, s);
  else if (st->V == VD) dequant_kernel<64, 128><<<g, FT, 0, s>>>(*st, idx, qmax);
  else dequant_kernel<64, 64><<<g, FT, 0, s>>>(*st, idx, qmax);
  return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_HIP;
}

extern "C" int lq_lowrank(const float* x, const float* Q0, float* U, float* Q, int n, int K, int V, int R, int iters,
                          void* stream) {
  if (K != KD || V != VD || R < 1 || R > 4 || n < 0 || iters < 1) return LQ_ERR_ARG;
  if (n == 0) return LQ_OK;
  if (!x || !Q0 || !U || !Q) return LQ_ERR_ARG;
  lowrank_kernel<<<dim3((unsigned)n), FT, 0, (hipStream_t)stream>>>(x, Q0, U, Q, R, iters);
  return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_HIP;
}
