/* liblq -- C ABI of the MI355X (gfx950) INT8 recurrent-state decode path for Gated DeltaNet (GDN) and
 * Kimi Delta Attention (KDA).
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t (passed as void*), launches its HIP kernels on
 * that stream, allocates nothing, never synchronises, and returns 0 on success or a negative lq_status.  All tensors
 * are owned by the caller (torch in leapquant_amd.state).
 *
 * State-cache layout (the drop-in contract, /root/reference/leapquant/state.py:1-6,29-40):
 *   ssm  fp32 [NS][HV][V][K], slot stride SS floats, inner dims packed.  Inside each (slot, head) block of V*K*4 bytes:
 *        Sq int8 [V][K] at byte 0 | Sk f32 [K] at V*K | Sv f32 [V] at V*K+4K | UQ fp16 [R][K+V] at V*K+4K+4V
 *        (UQ[r][0:K] = U^T[r], UQ[r][K:K+V] = Q^T[r]).  The remaining bytes of the block are not touched.
 *   Window buffer (separate tensors, state.py:61-69; one deliberate change: keys are stored once per KEY head):
 *        Kbuf bf16 [NS][H][L][K]   buffered normalised keys (identical for the HV/H value heads sharing a key head)
 *        Ubuf bf16 [NS][HV][L][V]  buffered delta-rule values u_j
 *        Wbuf f32  [NS][HV][L]     entry weights w_j (GDN: gate products since the entry; KDA: 1)
 *        Pbuf f32  [NS][HV][KA]    GDN (KA = 1): decay of the checkpoint, init 1;  KDA (KA = K): cumulative log-gate, init 0
 *        Gbuf fp16 [NS][HV][L][K]  KDA only: per-entry step decay exp(g_j), init 1
 *        hcnt i32  [NS][HV]        valid entries in the window
 *   A row n of a call with idx[n] <= 0 is a padding row: its outputs are zero and no state is written.  A slot
 *   idx[n] >= NS (outside the cache) is treated the same way, so no index reaches memory outside the tensors.
 */
#ifndef LQ_H
#define LQ_H

#ifdef __cplusplus
extern "C" {
#endif

#define LQ_ABI_VERSION 5
#define LQ_SCHED_INTS 512   /* ints of lq_state.sched: eight counters, 256 bytes apart */

enum lq_status {
  LQ_OK = 0,
  LQ_ERR_ARG = -1,     /* a size, shape or pointer the kernels do not support */
  LQ_ERR_HIP = -2,     /* a HIP launch error (hipGetLastError after the launch) */
  LQ_ERR_SIZE = -3,    /* lq_decode_noalloc: more (row, head) pairs than its static due list holds (LQ_DUE_MAX) */
};

/* Pointers and sizes of one layer's state: the fp32 cache the checkpoint aliases and the window buffer. */
typedef struct lq_state {
  void* ssm;              /* fp32 [NS][HV][V][K] at slot 0 (the tensor's data pointer, storage offset included) */
  long long slot_stride;  /* SS: floats between consecutive slots (>= HV*V*K) */
  void* Kbuf;             /* bf16 [NS][H][L][K]   (Kbuf, Ubuf, Gbuf: 16-byte aligned, read by whole-row 16-byte loads) */
  void* Ubuf;             /* bf16 [NS][HV][L][V] */
  float* Wbuf;            /* [NS][HV][L] */
  float* Pbuf;            /* [NS][HV][KA] */
  void* Gbuf;             /* fp16 [NS][HV][L][K] (KDA) or NULL (GDN) */
  int* hcnt;              /* [NS][HV] */
  int NS, HV, H, K, V, L, R;
  int* ctl;               /* optional (NULL: unused): int[2] = {due flag: nonzero when a step has filled some head's
                             window (or met a full one) since the last flush, flush workgroups done}, zero-initialised
                             by the owner and kept by the kernels.  With it, a flush that reads a clear flag returns at
                             once instead of scanning hcnt; the last flush workgroup clears both.  Without it, the
                             flush scans hcnt (the contract). */
  float qmax;             /* code range of the stored checkpoint: 127 (INT8) or 31 (6-bit codes in the int8
                             container); 0 means 127.  The decode steps dequantise with it (Sq Sk Sv / qmax). */
  int* sched;             /* optional (NULL: static schedule): int[LQ_SCHED_INTS], zero-initialised by the owner and
                             left zero by every flush.  With it, the persistent flush hands out its candidate heads
                             through counters in this buffer (each workgroup takes its next head when it is near the
                             end of the current one), so that the workgroups sharing a CU -- which the hardware does
                             not serve equally -- finish together; without it, workgroup b takes candidates b,
                             b + grid, ...  Same results either way.  One flush at a time per buffer. */
} lq_state;

/* Decode inputs of one call: N rows, one token each. */
typedef struct lq_step_io {
  const void* mixed;      /* bf16 [N][2*H*K + HV*V]: q (key heads) | k (key heads) | v (value heads), after the conv */
  const void* a;          /* bf16 raw gate: GDN [N][HV]; KDA [N][HV][K] */
  const void* b;          /* bf16 [N][HV]: beta = sigmoid(b) */
  const float* A_log;     /* [HV] */
  const float* dt_bias;   /* GDN [HV]; KDA [HV][K] */
  const int* idx;         /* [N] state slot of each row; <= 0: padding row */
  void* out;              /* bf16 [N][HV][V] */
  int N;
  float scale;            /* query scale (K^-1/2 by default) */
} lq_step_io;

/* Depthwise causal conv1d update (vLLM's causal_conv1d_update) fused into the GDN step: the step reads the raw
 * projection x (io.mixed, pre-conv, bf16 [N][C], C = 2*H*K + HV*V) and computes, for the channels it consumes,
 * mixed[c] = bf16(act(sum_{t<W-1} w[c][t] s[t] + w[c][W-1] x[c] + bias[c])), s the slot's conv state, then shifts the
 * state by one (s[t] = s[t+1], s[W-2] = x[c]).  Padding rows leave their state untouched. */
typedef struct lq_conv {
  void* state;            /* bf16 conv state; element (slot, channel c, tap t), t < W - 1, at
                             state[slot * slot_stride + c * ch_stride + t * tap_stride] */
  const void* weight;     /* bf16 [C][W] depthwise weights */
  const void* bias;       /* bf16 [C] or NULL */
  long long slot_stride, ch_stride, tap_stride;   /* in elements */
  int W;                  /* taps: 4 */
  int silu;               /* 1: SiLU after the bias; 0: none */
  int NS;                 /* slots of the conv state: a row whose slot is >= NS (or >= the state's NS) is a padding
                             row, so no tap is read or written outside the conv-state tensor */
} lq_conv;

int lq_abi_version(void);

/* GDN decode step: one token per row; appends (k, u, w = 1) to the window and updates the gate products.
 * Replaces make_gdn_step(...)(Sq, Sk, Sv, Skv, Kbuf, Ubuf, Wbuf, Pbuf, hcnt, mixed, a, b, A_log, dt_bias, UQ, idx, o)
 * (/root/reference/leapquant/kernels.py:27-692, launched at state.py:112-113).  Requires (K, V) = (128, 128), (64, 128)
 * or (64, 64) (kernels.py:62), 1 <= L <= 64, HV % H == 0 and HV / H in {1, 2, 4}, and 1 <= R <= 4 -- at (128, 128)
 * 1 <= R <= 16, the reference's rank ablation (kernels.py:63-64, 457-469).  A head whose window is already full
 * (hcnt >= L) is left untouched and its output row is zero (the flush after every step keeps hcnt < L on entry). */
int lq_gdn_step(const lq_state* st, const lq_step_io* io, void* stream);

/* lq_gdn_step with the conv1d update fused in (see lq_conv): io->mixed holds the raw projection.  No counterpart in the
 * reference as one call: replaces vLLM's causal_conv1d_update (leapquant/vllm/gdn.py:32) followed by the step. */
int lq_gdn_step_conv(const lq_state* st, const lq_step_io* io, const lq_conv* cv, void* stream);

/* GDN decode call: the step of every row (with vLLM's conv1d update fused in when cv is not NULL, as in
 * lq_gdn_step_conv), then the end-of-window flush of the heads whose window it filled (codes in [-qmax, qmax],
 * qmax = st->qmax, 0 meaning 127) -- what lq_gdn_step (or lq_gdn_step_conv) followed by lq_flush computes, in one
 * call.  Replaces make_gdn_step(...)(...) followed by make_flush(...)(...) as LeapQuantState.decode launches them
 * (/root/reference/leapquant/state.py:99-116; kernels.py:27-692, 1077-2033).  For (K, V) = (128, 128) and HV = 2 H it
 * is one launch: each step workgroup flushes the heads it has just filled (or found full) on the same threads; other
 * shapes run the step and the flush as two launches.  Same limits as lq_gdn_step and lq_flush. */
int lq_gdn_decode(const lq_state* st, const lq_step_io* io, const lq_conv* cv, const float* Q0, void* stream);

/* lq_gdn_decode with the flush of a key head's second value head deferred: no counterpart in the reference (whose
 * flush follows every step); for continuous batching, where rows reach the end of their window on different calls.
 * At (K, V) = (128, 128), HV = 2 H, of the two heads of a key head that a call fills, the step workgroup flushes the
 * first right after its step and leaves the second full (hcnt == L, flagged in st->ctl); the next call that steps the
 * slot flushes it before its step, on the same threads, or lq_flush does.  Every output is the one lq_gdn_decode gives
 * (a full head is flushed before any step reads it); between calls a slot may hold a full head, so a reader of the
 * checkpoint other than these two calls runs lq_flush on its slots first (LeapQuantState.dequantize does).  A filling
 * call costs one head's flush instead of two: the latency that a due row adds to the call halves.  Other shapes: as
 * lq_gdn_decode. */
int lq_gdn_decode_deferred(const lq_state* st, const lq_step_io* io, const lq_conv* cv, const float* Q0,
                           void* stream);

/* KDA decode step (per-key-channel gate).  glb != 0: GLM's bounded gate glb * sigmoid(exp(A_log) (a + dt_bias));
 * glb == 0: Kimi's -exp(A_log) softplus(a + dt_bias).
 * Replaces make_kda_step(...)(Sq, Sk, Sv, Skv, Kbuf, Ubuf, Wbuf, Pbuf, Gbuf, hcnt, mixed, a, b, A_log, dt_bias, UQ,
 * idx, o) (kernels.py:694-1075, launched at state.py:108-109).  Same limits as lq_gdn_step, with K = V = 128 and
 * R <= 4 only (kernels.py:727, 1036). */
int lq_kda_step(const lq_state* st, const lq_step_io* io, float glb, void* stream);

/* KDA decode call: the step of every row (gate as lq_kda_step), then the end-of-window flush of the heads whose window
 * it filled (codes in [-qmax, qmax], qmax = st->qmax, 0 meaning 127) -- what lq_kda_step followed by lq_flush (kda = 1)
 * computes, in one call.  Replaces make_kda_step(...)(...) followed by make_flush(..., KDA=True)(...) as
 * LeapQuantState.decode launches them (/root/reference/leapquant/state.py:99-116; kernels.py:694-1075, 1077-2033).
 * Two launches (the step, then the persistent flush, which returns at once when no step raised the due flag st->ctl):
 * one C call per layer and decode call, as lq_gdn_decode.  Same limits as lq_kda_step and lq_flush. */
int lq_kda_decode(const lq_state* st, const lq_step_io* io, float glb, const float* Q0, void* stream);

/* End-of-window flush of every (idx[n] > 0, hv) head whose window is full (hcnt == L): rebuild, one subspace
 * iteration from Q0 [V][R] with CholeskyQR2, fp16 factors, smoothed residual requantised to codes in [-qmax, qmax]
 * (127: INT8; 31: 6-bit in the same int8 container), window reset.  Due heads are found on the device.
 * Replaces make_flush(...)(Sq, Sk, Sv, Skv, Kbuf, Ubuf, Wbuf, Pbuf, Gbuf, hcnt, Sq16, UQ, Q0, idx)
 * (kernels.py:1077-2033, launched at state.py:115-116).  Requires 1 <= L <= 64, 1 <= R <= 4 and (K, V) = (128, 128),
 * or for GDN (kda == 0) also (64, 128), (64, 64) (kernels.py:1089-1092); GDN (128, 128) also 5 <= R <= 8, whose
 * CholeskyQR drops a dependent column instead of flooring its pivot (kernels.py:1091, 1744-1772). */
int lq_flush(const lq_state* st, const float* Q0, const int* idx, int N, int kda, float qmax, void* stream);

/* Standalone quantize of the fp32 states of the slots idx[n] > 0 (read from the same ssm blocks the checkpoint then
 * overwrites), window reset (Wbuf = 0, Pbuf = 1, hcnt = 0).  qmax 127 (INT8) or 31 (6-bit).
 * Replaces make_quantize(...)(S0, Sq, Sk, Sv, UQ, Wbuf, Pbuf, hcnt, Q0, idx) (kernels.py:2126-2242, state.py:163-165).
 * Requires (K, V) = (128, 128), (64, 128) or (64, 64), 1 <= R <= 4; at (128, 128) 1 <= R <= 16 (every rank a step
 * reads). */
int lq_quantize(const lq_state* st, const float* Q0, const int* idx, int N, float qmax, void* stream);

/* Prefill dequant (GDN): fp32 S = P (deq(Sq) + Q U^T) + sum_{j<h} w_j u_j k_j^T written over the ssm blocks of the
 * slots idx[n] > 0, then window reset.  Replaces make_dequant(...)(S0, Sq, Sk, Sv, Kbuf, Ubuf, Wbuf, Pbuf, Gbuf, hcnt,
 * UQ, idx) (kernels.py:2041-2123, state.py:152-154).  Requires (K, V) = (128, 128), (64, 128) or (64, 64),
 * 1 <= L <= 64, 1 <= R <= 4; at (128, 128) 1 <= R <= 16. */
int lq_dequant(const lq_state* st, const int* idx, int N, float qmax, void* stream);

/* Prefill dequant (KDA): fp32 S = (deq(Sq) + Q U^T) diag(exp(P)) + sum_{j<h} w_j u_j (K_j * D_j)^T, D_j the product of
 * the decays of the entries after j, written over the ssm blocks of the slots idx[n] > 0; the window is kept (the
 * checkpoint after the prefill resets it).  Replaces the torch rebuild LeapQuantState._kda_rebuild + dequantize
 * (state.py:118-128, 147-150).  Requires K = V = 128, 1 <= L <= 64, 1 <= R <= 4, Gbuf set. */
int lq_kda_dequant(const lq_state* st, const int* idx, int N, float qmax, void* stream);

/* Prefill checkpoint (KDA) of the fp32 states of the slots idx[n] > 0: rank-R factors by three rounds of
 * P = MGS(S^T Q), Q = MGS(S P) from Q0, U = S^T Q, both fp16; residual codes clamp(rint(E / (Sk Sv) qmax)) with
 * Sk = sqrt(mean_v |E|), Sv = max_c |E / Sk|; window reset (Wbuf = 0, Pbuf = 0, Gbuf = 1, hcnt = 0).  Replaces the
 * torch checkpoint LeapQuantState._kda_checkpoint with lowrank_factor (state.py:130-142, kernels.py:2318-2331).
 * Requires K = V = 128, 1 <= R <= 4, Gbuf set. */
int lq_kda_checkpoint(const lq_state* st, const float* Q0, const int* idx, int N, float qmax, void* stream);

/* Rank-R subspace iteration on n fp32 matrices x [n][K][V]: `iters` rounds of P = MGS(x Q), Q = MGS(x^T P) from
 * Q0 [V][R]; U = x Q.  Outputs U [n][K][R], Q [n][V][R] (fp32).
 * Replaces make_lowrank / lowrank_factor (kernels.py:2246-2331).  Requires K = V = 128, 1 <= R <= 4. */
int lq_lowrank(const float* x, const float* Q0, float* U, float* Q, int n, int K, int V, int R, int iters,
               void* stream);

/* No counterpart in the reference: one decode call -- the step of every row (GDN, or KDA with gate glb), then the
 * flush of the heads that step made due (codes in [-qmax, qmax], qmax = st->qmax, 0 meaning 127) -- that allocates
 * nothing and takes no workspace: the due heads are passed from the step to the flush through a list in the library's
 * own static device memory (256 KiB per GPU, held until the process ends), not through st->ctl, which it ignores.
 * For callers that cannot allocate device memory: code under graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Limit: N * HV <= LQ_DUE_MAX = 65536, else LQ_ERR_SIZE.  All calls on one GPU share the list: calls that
 * overlap on one GPU (concurrent streams, threads) race and must not be issued.  Results equal lq_gdn_step /
 * lq_kda_step followed by lq_flush on the same inputs.  The list's device address is looked up on the first call on
 * each device (also a call with N = 0, which launches nothing): a caller that captures its calls in a graph makes
 * one such call on each device before the capture, so that the captured calls make no runtime query. */
int lq_decode_noalloc(const lq_state* st, const lq_step_io* io, const float* Q0, int kda, float glb, void* stream);

/* Baseline (no reference counterpart): the standalone conv1d update that lq_gdn_step_conv fuses into the step, same
 * arithmetic (it stands for vLLM's causal_conv1d_update, leapquant/vllm/gdn.py:32): out [N][C] bf16 from the raw
 * projection x [N][C], the conv states of the slots idx[n] > 0 (< NS) shifted in place. */
int lq_conv_update(const lq_conv* cv, const void* x, void* out, const int* idx, int N, int C, int NS, void* stream);

/* Baseline for the measurements (no reference counterpart): the same GDN decode step on a dense state S
 * [NS][HV][V][K] stored as bf16 (state_dtype 0) or fp32 (state_dtype 1), updated in place:
 * S' = alpha S + u k^T, u = beta (v - alpha S k), o = S' q.  S and io->mixed 16-byte aligned. */
int lq_dense_step(void* S, int state_dtype, int NS, int HV, int H, int K, int V, const lq_step_io* io, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* LQ_H */
