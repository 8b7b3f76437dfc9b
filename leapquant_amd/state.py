"""Per-layer LeapQuant state on MI355X: the 8-bit checkpoint lives inside vLLM's fp32 state slot, the window buffer next
to it.  Drop-in for /root/reference/leapquant/state.py (same names, arguments, errors and call order).

Layout of one (slot, head) inside the fp32 [V, K] state slot (state.py:1-6, 29-40 of the reference):
    int8 residual [V][K] | smoothing scales Sk f32[K], Sv f32[V] | Compensator Tokens U^T | Q^T fp16 [R][K+V]
The window buffer (keys, values, weights of the tokens since the last flush) and the per-slot counters are separate
tensors; the keys are kept once per key head (Kbuf [NS, H, L, K]).
"""
import collections
import ctypes
import functools

import torch

from . import _lib
from . import kernels as KN

WINDOW = 16          # tokens per window (L), state.py:16
RANK = 4             # Compensator Tokens per head (R), state.py:17

_make_dequant = functools.lru_cache(maxsize=None)(KN.make_dequant)
_make_quantize = functools.lru_cache(maxsize=None)(KN.make_quantize)


_CacheId = collections.namedtuple("_CacheId", "storage offset shape stride")


def _ident(t):
    """Identity of a state-cache tensor: where its storage lives and which view of it the tensor is.  The engine
    re-allocating its caches (after the profiling run) shows up as a new identity."""
    return _CacheId(t.untyped_storage().data_ptr(), t.storage_offset(), tuple(t.shape), t.stride())


def _alias(ssm, dtype, shape, stride, offset):
    out = torch.empty(0, dtype=dtype, device=ssm.device)
    out.set_(ssm.untyped_storage(), offset, shape, stride)
    return out


def state_views(ssm, R):
    """Views of the 8-bit checkpoint aliasing vLLM's fp32 state tensor [NS, HV, V, K] (no allocation): Sq (int8),
    q32 (int32 words of Sq), sq16 (int16 pairs of Sq), Sk, Sv, skv (Sk || Sv) and uq (fp16 U^T | Q^T)."""
    NS, HV, V, K = ssm.shape
    SS = ssm.stride(0)
    off = ssm.storage_offset()
    sc = off + V * K // 4                       # fp32 offset of Sk
    return dict(
        Sq=_alias(ssm, torch.int8, (NS, HV, V, K), (4 * SS, 4 * V * K, K, 1), 4 * off),
        q32=_alias(ssm, torch.int32, (NS, HV, V, K // 4), (SS, V * K, K // 4, 1), off),
        sq16=_alias(ssm, torch.int16, (NS, HV, V, K // 2), (2 * SS, 2 * V * K, K // 2, 1), 2 * off),
        Sk=_alias(ssm, torch.float32, (NS, HV, K), (SS, V * K, 1), sc),
        Sv=_alias(ssm, torch.float32, (NS, HV, V), (SS, V * K, 1), sc + K),
        skv=_alias(ssm, torch.float32, (NS, HV, K + V), (SS, V * K, 1), sc),
        uq=_alias(ssm, torch.float16, (NS, HV, R, K + V), (2 * SS, 2 * V * K, K + V, 1), 2 * (sc + K + V)))


class LeapQuantState:
    """Window buffers + kernels of one linear-attention layer.

    kda=False: Gated DeltaNet (Qwen).  kda=True: Kimi Delta Attention (GLM), gate_lower_bound = GLM's bounded gate.
    nmax: the most rows one decode call can carry (accepted for parity; the HIP flush needs no work-list sizing).
    qmax: code range of the checkpoint (127: INT8; 31: 6-bit codes in the int8 container).
    defer_flush (not in the reference): GDN decode through lq_gdn_decode_deferred -- of the two value heads of a key
    head that a call fills, the second is flushed at the start of the next call that steps its slot (the outputs are
    the same; a due row costs its call one head flush instead of two).  dequantize settles such heads first.
    """

    def __init__(self, ssm, H, kda=False, gate_lower_bound=0.0, nmax=0, L=WINDOW, R=RANK, qmax=KN.QMAX,
                 defer_flush=False):
        assert ssm.dtype == torch.float32, f"LeapQuant needs the fp32 recurrent state cache, got {ssm.dtype}"
        self.defer_flush = bool(defer_flush) and not kda
        NS, HV, V, K = ssm.shape
        SS = ssm.stride(0)
        assert ssm.stride()[1:] == (V * K, K, 1), f"state inner dims must be packed, got strides {ssm.stride()}"
        assert V * K // 4 + K + V + R * (K + V) // 2 <= V * K, "checkpoint must fit inside the fp32 slot"
        dev = ssm.device
        self.key = _ident(ssm)
        self.kda, self.NS, self.HV, self.H, self.K, self.V, self.L, self.R = kda, NS, HV, H, K, V, L, R
        self.SS, self.qmax, self.glb = SS, float(qmax), float(gate_lower_bound)
        KA = K if kda else 1

        self.Kbuf = torch.zeros(NS, H, L, K, device=dev, dtype=torch.bfloat16)
        self.Ubuf = torch.zeros(NS, HV, L, V, device=dev, dtype=torch.bfloat16)
        self.Wbuf = torch.zeros(NS, HV, L, device=dev)
        self.Pbuf = torch.zeros(NS, HV, KA, device=dev) if kda else torch.ones(NS, HV, 1, device=dev)
        # KDA: each entry's per-step decay factor exp(g_j) (fp16); GDN: unused
        self.Gbuf = (torch.ones(NS, HV, L, KA, device=dev, dtype=torch.float16) if kda
                     else torch.zeros(NS, HV, L, 1, device=dev))
        self.Gd = torch.zeros(1, 1, 1, 1, dtype=torch.bfloat16, device=dev)
        self.hcnt = torch.zeros(NS, HV, dtype=torch.int32, device=dev)
        # heads made due by decode steps since the last flush / flush workgroups done: lets an idle flush return at
        # once (kept by the kernels; zero between calls)
        self.ctl = torch.zeros(2, dtype=torch.int32, device=dev)
        # the flush's dynamic head schedule (counters the flush leaves at zero)
        self.sched = torch.zeros(_lib.SCHED_INTS, dtype=torch.int32, device=dev)
        self.Q0 = torch.randn(V, R, generator=torch.Generator().manual_seed(0)).to(dev)

        if kda:
            self.kstep = KN.make_kda_step(NS, HV, H, K, V, L, SS, R=R, GLB=float(gate_lower_bound), qmax=qmax)
        else:
            self.kstep = KN.make_gdn_step(NS, HV, H, K, V, L, SS, R=R, qmax=qmax)
        self.kflush = KN.make_flush(NS, HV, K, V, L, SS, R=R, ITERS=1, KDA=kda, NMAX=nmax, qmax=qmax, sched=self.sched)
        if not kda:                          # the KDA prefill round trip has its own entry points
            self.kdeq = _make_dequant(NS, HV, K, V, L, SS, buf_dtype=KN.BF16, R=R, qmax=qmax)
            self.kquant = _make_quantize(NS, HV, K, V, L, SS, R=R, ITERS=1, qmax=qmax)
        self._lib = _lib.lib()
        self._vkey = None
        self._skey = None
        self._scan_src = None
        self._param_f32 = {}

    def _as_f32(self, t):
        """A gate parameter (A_log, dt_bias) as the fp32 tensor the kernels read.  A parameter in another dtype is
        converted once and the copy kept, keyed by the parameter's address and dtype (a state tensor may be shared by
        layers that each bring their own parameters)."""
        if t.dtype == torch.float32:
            return t
        key = (t.data_ptr(), t.dtype)
        if key not in self._param_f32:
            self._param_f32[key] = t.detach().float().contiguous()
        return self._param_f32[key]

    def views(self, ssm):
        k = _ident(ssm)
        if self._vkey != k:
            self._vkey, self._v = k, state_views(ssm, self.R)
        return self._v

    def _struct(self, ssm):
        """lq_state of this layer for the cache tensor ssm (cached per tensor identity)."""
        k = _ident(ssm)
        if self._skey != k:
            if ssm.data_ptr() % 16 or self.SS % 4:
                raise ValueError("the fp32 state cache must be 16-byte aligned with a slot stride divisible by 4")
            self._st = KN.state_struct(ssm, self.SS, self.Kbuf, self.Ubuf, self.Wbuf, self.Pbuf,
                                       self.Gbuf if self.kda else None, self.hcnt, self.NS, self.HV, self.H, self.K,
                                       self.V, self.L, self.R, ctl=self.ctl, qmax=self.qmax, sched=self.sched)
            self._skey = k
        return self._st

    def decode(self, ssm, mixed, a, b, A_log, dt_bias, idx, out):
        """One decode token per row, then the end-of-window flush of the heads whose window became full (one C call:
        lq_gdn_decode, or lq_kda_decode).
        a: GDN (N, HV) | KDA (N, HV, K) raw gate;  dt_bias: GDN (HV,) | KDA (HV*K,)."""
        A_log = self._as_f32(A_log)
        dt_bias = self._as_f32(dt_bias)
        KA = self.K if self.kda else 1
        N = idx.shape[0]
        self._check_gate(a, N, KA)
        a = a.reshape(N, self.HV, KA).contiguous()
        dt_bias = dt_bias.reshape(self.HV, KA).contiguous()
        A_log = A_log.reshape(self.HV).contiguous()
        idx = idx if idx.dtype == torch.int32 else idx.to(torch.int32)
        idx = idx.contiguous()
        if (mixed.dtype != torch.bfloat16 or not mixed.is_contiguous()
                or mixed.shape != (N, 2 * self.H * self.K + self.HV * self.V)):
            raise ValueError("mixed: contiguous bf16 [N, 2HK + HV V] expected")
        if out.dtype != torch.bfloat16 or out.numel() != N * self.HV * self.V or not out.is_contiguous():
            raise ValueError("out: contiguous bf16 [N, HV, V] expected")
        if b.dtype != torch.bfloat16 or b.numel() != N * self.HV:
            raise ValueError("b: bf16 [N, HV] expected")
        b = b.contiguous()
        st = self._struct(ssm)
        io = KN._step_io(mixed, a, b, A_log, dt_bias, idx, out, self.kstep_scale)
        stream = ctypes.c_void_p(torch.cuda.current_stream(mixed.device).cuda_stream)
        L = self._lib
        if self.kda:                 # the step, then the flush of the heads it fills
            _lib.check(L.lq_kda_decode(ctypes.byref(st), ctypes.byref(io), ctypes.c_float(self.glb), KN._p(self.Q0),
                                       stream), "lq_kda_decode")
        else:                        # step + flush of the heads it fills (one launch for 128 x 128 heads, GQA 2)
            fn = L.lq_gdn_decode_deferred if self.defer_flush else L.lq_gdn_decode
            _lib.check(fn(ctypes.byref(st), ctypes.byref(io), None, KN._p(self.Q0), stream), "lq_gdn_decode")

    def decode_conv(self, ssm, x, conv_state, conv_weight, conv_bias, silu, a, b, A_log, dt_bias, idx, out):
        """GDN decode with the conv1d update fused into the step (lq_gdn_step_conv): x is the raw projection
        [N, 2HK + HV V] (bf16, before vLLM's causal_conv1d_update); conv_state [NS, C, W-1] (any strides) and
        conv_weight [C, W] bf16 with W = 4; the conv state of every row's slot is shifted in place.  Then the flush."""
        if self.kda:
            raise ValueError("decode_conv: GDN only")
        C = 2 * self.H * self.K + self.HV * self.V
        if conv_state.dtype != torch.bfloat16 or conv_state.dim() != 3 or conv_state.shape[1:] != (C, 3) \
                or conv_state.shape[0] < self.NS:
            raise ValueError("conv_state: bf16 [NS, C, 3] expected")
        w = conv_weight.reshape(C, -1)
        if w.dtype != torch.bfloat16 or w.shape[1] != 4 or not w.is_contiguous() or w.data_ptr() % 8:
            raise ValueError("conv_weight: contiguous bf16 [C, 4] expected")
        if conv_bias is not None and (conv_bias.dtype != torch.bfloat16 or conv_bias.numel() != C
                                      or not conv_bias.is_contiguous()):
            raise ValueError("conv_bias: bf16 [C] expected")
        A_log = self._as_f32(A_log)
        dt_bias = self._as_f32(dt_bias)
        N = idx.shape[0]
        self._check_gate(a, N, 1)
        a = a.reshape(N, self.HV).contiguous()
        dt_bias = dt_bias.reshape(self.HV).contiguous()
        A_log = A_log.reshape(self.HV).contiguous()
        idx = idx if idx.dtype == torch.int32 else idx.to(torch.int32)
        idx = idx.contiguous()
        if x.dtype != torch.bfloat16 or not x.is_contiguous() or x.shape != (N, C):
            raise ValueError("x: contiguous bf16 [N, 2HK + HV V] expected")
        if out.dtype != torch.bfloat16 or out.numel() != N * self.HV * self.V or not out.is_contiguous():
            raise ValueError("out: contiguous bf16 [N, HV, V] expected")
        if b.dtype != torch.bfloat16 or b.numel() != N * self.HV:
            raise ValueError("b: bf16 [N, HV] expected")
        b = b.contiguous()
        st = self._struct(ssm)
        io = KN._step_io(x, a, b, A_log, dt_bias, idx, out, self.kstep_scale)
        cv = KN.conv_struct(conv_state, w, conv_bias, silu)
        stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
        fn = self._lib.lq_gdn_decode_deferred if self.defer_flush else self._lib.lq_gdn_decode
        _lib.check(fn(ctypes.byref(st), ctypes.byref(io), ctypes.byref(cv), KN._p(self.Q0), stream), "lq_gdn_decode")

    def _check_gate(self, a, N, KA):
        """The raw gate `a` is read as bf16, N x HV (GDN) or N x HV x K (KDA) values (kernels.py:86, 738)."""
        if a.dtype != torch.bfloat16 or a.numel() != N * self.HV * KA:
            raise ValueError("a: bf16 with N * HV%s = %d elements expected, got %s with %d"
                             % (" * K" if KA > 1 else "", N * self.HV * KA, a.dtype, a.numel()))

    def _struct_scan(self, ssm):
        """lq_state of this layer without the due flag: a flush through it checks hcnt of every listed row, and
        leaves the flag as it is."""
        st = self._struct(ssm)
        if self._scan_src is not st:
            self._st_scan = _lib.LqState.from_buffer_copy(st)
            self._st_scan.ctl = None
            self._scan_src = st
        return self._st_scan

    def flush(self, ssm, idx):
        """The end-of-window flush of the due heads (hcnt == L) of the rows idx, as the reference's flush finds them
        (kernels.py:1200).  It reads hcnt of every listed row rather than the due flag the decode steps raise: a head
        that a deferred decode left full may sit in a slot that an earlier flush of other rows did not cover (that
        flush cleared the flag), and it must still be flushed here."""
        idx = idx if idx.dtype == torch.int32 else idx.to(torch.int32)
        idx = idx.contiguous()
        st = self._struct_scan(ssm)
        stream = ctypes.c_void_p(torch.cuda.current_stream(idx.device).cuda_stream)
        _lib.check(self._lib.lq_flush(ctypes.byref(st), KN._p(self.Q0), KN._p(idx), idx.shape[0], 1 if self.kda else 0,
                                      ctypes.c_float(self.qmax), stream), "lq_flush")

    @property
    def kstep_scale(self):
        return 128 ** -0.5 if self.kda else self.K ** -0.5

    def _kda_round_trip(self, ssm, idx, fn, *extra):
        idx = idx if idx.dtype == torch.int32 else idx.to(torch.int32)
        idx = idx.contiguous()
        st = self._struct(ssm)
        stream = ctypes.c_void_p(torch.cuda.current_stream(idx.device).cuda_stream)
        _lib.check(getattr(self._lib, fn)(ctypes.byref(st), *extra, KN._p(idx), idx.shape[0],
                                          ctypes.c_float(self.qmax), stream), fn)

    def dequantize(self, ssm, idx):
        """Materialise the fp32 state of the slots idx in place (before the engine's own prefill kernel runs)."""
        if idx.numel() == 0:
            return
        if self.kda:                 # S = (Q U^T + deq) diag(exp(P)) + decayed window (state.py:118-128), HIP
            self._kda_round_trip(ssm, idx, "lq_kda_dequant")
            return
        idx = idx.to(torch.int32).contiguous()
        if self.defer_flush:         # a head left full by a deferred decode is flushed before its state is read
            self.flush(ssm, idx)
        v = self.views(ssm)
        self.kdeq(ssm, v["Sq"], v["Sk"], v["Sv"], self.Kbuf, self.Ubuf, self.Wbuf, self.Pbuf, self.Gbuf, self.hcnt,
                  v["uq"], idx)

    def quantize(self, ssm, idx):
        """Write the 8-bit checkpoint of the fp32 states in the slots idx and reset their windows (after a prefill)."""
        if idx.numel() == 0:
            return
        if self.kda:                 # rank-R fit (3 rounds) + residual codes, window reset (state.py:130-142), HIP
            self._kda_round_trip(ssm, idx, "lq_kda_checkpoint", KN._p(self.Q0))
            return
        v = self.views(ssm)
        self.kquant(ssm, v["Sq"], v["Sk"], v["Sv"], v["uq"], self.Wbuf, self.Pbuf, self.hcnt, self.Q0,
                    idx.to(torch.int32).contiguous())


_STATES = {}        # cache identity -> the LeapQuantState built for it
_GEN = [0]          # generation of the engine's caches: bumped when they are re-allocated


def _forget_states():
    """The engine has re-allocated its caches: every state built for the old ones addresses freed memory."""
    _GEN[0] += 1
    _STATES.clear()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()


def _refuse_prefix_caching(layer):
    """Each sequence's window buffer lives beside its state slot, which recurrent-state prefix caching would share."""
    mode = getattr(getattr(layer, "cache_config", None), "mamba_cache_mode", "none")
    if mode != "none":
        raise RuntimeError("LeapQuant keeps each sequence's window buffer next to its state slot and does not support "
                           "prefix caching of the recurrent state: run vLLM with --no-enable-prefix-caching")


def get_state(layer, ssm, **kw):
    """The LeapQuantState of `layer` for its current state tensor `ssm`, built on first use.  When a layer presents a
    different tensor than the one its state was built for in the current generation, the engine has swapped its caches
    (it does so after profiling): all states are dropped and rebuilt on demand."""
    key = _ident(ssm)
    mine = layer.__dict__.get("_leapquant")
    if mine is not None:
        if mine.key == key:
            return mine
        if mine.gen == _GEN[0]:
            _forget_states()
    st = _STATES.get(key)
    if st is None:
        _refuse_prefix_caching(layer)
        st = LeapQuantState(ssm, **kw)
        st.gen = _GEN[0]
        _STATES[key] = st
    layer._leapquant = st
    return st
