"""Host-side bounds model of liblq (CPU test infrastructure).

`Footprint` lists, for one call of an entry point of include/lq.h, every byte range its kernels may read or write,
derived from the kernels' own index arithmetic (leapquant_amd/csrc/lq_step.hip, lq_flush.hip, lq_dense.hip):

  * per row n: idx[n] and its output row; for a row whose slot is valid (0 < slot < NS, and < the conv state's NS for
    the fused conv): its mixed / raw-projection row, gate and beta rows, and per value head hv of that slot the
    checkpoint region of the (slot, hv) block (codes, Sk, Sv, U^T | Q^T; the whole fp32 block for quantize / dequant),
    the window rows Kbuf[slot, hv // G, 0:L], Ubuf / Wbuf / Gbuf [slot, hv, 0:L], Pbuf[slot, hv], hcnt[slot, hv], and
    for the fused conv the slot's three taps of every channel;
  * per call: A_log, dt_bias, Q0, the due flag pair ctl, the flush's schedule counter sched and the conv weights /
    bias.

The model is conservative about data: every valid (slot, head) of a flush is taken as due.  `CheckingLib` stands in for
liblq.so: each entry point validates its arguments as the library does, computes the call's footprint and checks that
every range lies inside one storage the caller handed over (every pointer reaches the library through
leapquant_amd.kernels._dev, which `install` wraps to record the storage behind it), and returns the library's status
without launching anything.  A violation raises `OutOfBounds` naming the entry point, the tensor and the range.
"""
import ctypes

import torch


class OutOfBounds(AssertionError):
    pass


class Storages:
    """Storages the caller has passed to the library: [lo, hi) byte ranges.  Each storage is kept alive by the registry,
    so no later tensor can reuse its addresses while the check runs (a freed range still listed would hide or invent
    violations)."""

    def __init__(self):
        self.ranges = {}
        self.keep = []

    def add(self, t):
        s = t.untyped_storage()
        lo = s.data_ptr()
        if lo not in self.ranges:
            self.keep.append(s)
        self.ranges[lo] = max(self.ranges.get(lo, lo), lo + s.nbytes())

    def owner(self, p):
        for lo, hi in self.ranges.items():
            if lo <= p < hi:
                return lo, hi
        return None

    def check(self, what, base, off, nbytes):
        if nbytes <= 0:
            return
        p = base + off
        own = self.owner(base) if off >= 0 else None
        if own is None or p < own[0] or p + nbytes > own[1]:
            raise OutOfBounds("%s: [%#x, %#x) (base %#x + %d) is outside the storage %s"
                              % (what, p, p + nbytes, base, off,
                                 "[%#x, %#x)" % own if own else "(no storage holds the base pointer)"))


def _ints(ptr, n):
    return list((ctypes.c_int32 * n).from_address(ptr)) if n > 0 else []


def _arg(x):
    return x._obj if hasattr(x, "_obj") else x


class CheckingLib:
    """Drop-in for the ctypes handle of liblq.so: checks the footprint of every call, launches nothing."""

    ABI = 5

    def __init__(self):
        self.storages = Storages()
        self.calls = []
        self.alignments = []                 # byte address of every pointer a state / step call was given

    # ---- helpers --------------------------------------------------------------------------------------------------
    def _state_ok(self, st, need_buf=True, kda=False):
        dims = ((128, 128),) if kda else ((128, 128), (64, 128), (64, 64))
        if (st.K, st.V) not in dims or not 1 <= st.L <= 64 or not 1 <= st.R <= 4:
            return False
        if st.H <= 0 or st.HV <= 0 or st.HV % st.H or st.NS <= 0:
            return False
        if st.slot_stride < st.HV * st.V * st.K or st.slot_stride % 4 or not st.ssm or st.ssm % 16:
            return False
        if not st.hcnt or not st.Wbuf or not st.Pbuf or (need_buf and (not st.Kbuf or not st.Ubuf)):
            return False
        if ((st.Kbuf or 0) | (st.Ubuf or 0) | (st.Gbuf or 0)) % 16:      # 16-byte row loads and LDS DMA
            return False
        return True

    def _head(self, st, slot, hv, kda, what, block=False):
        """Footprint of one (slot, value head) of the state."""
        S = self.storages
        K, V, L, R, HV, H = st.K, st.V, st.L, st.R, st.HV, st.H
        G = HV // H
        sh = slot * HV + hv
        blk = 4 * (slot * st.slot_stride + hv * V * K)
        S.check(what + " ssm block", st.ssm, blk, 4 * V * K if block else V * K + 4 * K + 4 * V + 2 * R * (K + V))
        S.check(what + " hcnt", st.hcnt, 4 * sh, 4)
        S.check(what + " Wbuf", st.Wbuf, 4 * sh * L, 4 * L)
        S.check(what + " Pbuf", st.Pbuf, 4 * sh * (K if kda else 1), 4 * (K if kda else 1))
        if st.Kbuf:
            S.check(what + " Kbuf", st.Kbuf, 2 * (slot * H + hv // G) * L * K, 2 * L * K)
        if st.Ubuf:
            S.check(what + " Ubuf", st.Ubuf, 2 * sh * L * V, 2 * L * V)
        if kda and st.Gbuf:
            S.check(what + " Gbuf", st.Gbuf, 2 * sh * L * K, 2 * L * K)

    def _rows(self, st, io, kda, what, conv=None):
        S = self.storages
        K, V, HV, H = st.K, st.V, st.HV, st.H
        KA = K if kda else 1
        MIX = 2 * H * K + HV * V
        S.check(what + " idx", io.idx, 0, 4 * io.N)
        S.check(what + " out", io.out, 0, 2 * io.N * HV * V)
        S.check(what + " A_log", io.A_log, 0, 4 * HV)
        S.check(what + " dt_bias", io.dt_bias, 0, 4 * HV * KA)
        for n, slot in enumerate(_ints(io.idx, io.N)):
            if slot <= 0 or slot >= st.NS or (conv is not None and slot >= conv.NS):
                continue
            S.check(what + " mixed row", io.mixed, 2 * n * MIX, 2 * MIX)
            S.check(what + " a row", io.a, 2 * n * HV * KA, 2 * HV * KA)
            S.check(what + " b row", io.b, 2 * n * HV, 2 * HV)
            for hv in range(HV):
                self._head(st, slot, hv, kda, what)
            if conv is not None:
                C = MIX
                top = slot * conv.slot_stride + (C - 1) * conv.ch_stride + 2 * conv.tap_stride
                S.check(what + " conv state", conv.state, 2 * slot * conv.slot_stride,
                        2 * (top - slot * conv.slot_stride + 1))

    def _conv_ok(self, cv, C):
        return (cv is not None and cv.state and cv.weight and cv.W == 4 and cv.silu in (0, 1) and cv.NS > 0
                and cv.ch_stride > 0 and cv.tap_stride > 0
                and (C - 1) * cv.ch_stride + 2 * cv.tap_stride < cv.slot_stride and cv.weight % 8 == 0)

    def _conv_params(self, cv, C, what):
        self.storages.check(what + " conv weight", cv.weight, 0, 2 * 4 * C)
        if cv.bias:
            self.storages.check(what + " conv bias", cv.bias, 0, 2 * C)

    def _ctl(self, st, what):
        if st.ctl:
            self.storages.check(what + " ctl", st.ctl, 0, 8)
        if st.sched:
            self.storages.check(what + " sched", st.sched, 0, 4 * 512)

    # ---- entry points ---------------------------------------------------------------------------------------------
    def lq_abi_version(self):
        return self.ABI

    def _step(self, name, st, io, kda, cv=None):
        st, io = _arg(st), _arg(io)
        self.calls.append(name)
        self.alignments += [p for p in (st.ssm, st.Kbuf, st.Ubuf, st.Gbuf, io.mixed, io.out) if p]
        if not self._state_ok(st, kda=kda) or not (st.qmax == 0 or 1 <= st.qmax <= 127) or io.N < 0:
            return -1
        if kda and (not st.Gbuf or (st.K, st.V) != (128, 128)):
            return -1
        if not kda and st.HV // st.H not in (1, 2, 4):
            return -1
        if io.N == 0:
            return 0
        if cv is not None:
            C = 2 * st.H * st.K + st.HV * st.V
            if not self._conv_ok(cv, C):
                return -1
            self._conv_params(cv, C, name)
        self._rows(st, io, kda, name, conv=cv)
        self._ctl(st, name)
        return 0

    def lq_gdn_step(self, st, io, stream):
        return self._step("lq_gdn_step", st, io, False)

    def lq_gdn_step_conv(self, st, io, cv, stream):
        return self._step("lq_gdn_step_conv", st, io, False, _arg(cv))

    def lq_kda_step(self, st, io, glb, stream):
        return self._step("lq_kda_step", st, io, True)

    def lq_gdn_decode(self, st, io, cv, Q0, stream):
        """The GDN step (conv fused when cv is set), then the flush of the rows of the call."""
        cv = _arg(cv) if cv is not None else None
        rc = self._step("lq_gdn_decode", st, io, False, cv)
        if rc:
            return rc
        io = _arg(io)
        return self._per_slot("lq_gdn_decode flush", st, ctypes.c_void_p(io.idx), io.N, False, False, Q0=Q0)

    def lq_kda_decode(self, st, io, glb, Q0, stream):
        """The KDA step, then the flush of the rows of the call."""
        rc = self._step("lq_kda_decode", st, io, True)
        if rc:
            return rc
        st_, io_ = _arg(st), _arg(io)
        if st_.R > 4:
            return -1
        return self._per_slot("lq_kda_decode flush", st, ctypes.c_void_p(io_.idx), io_.N, True, False, Q0=Q0)

    def lq_gdn_decode_deferred(self, st, io, cv, Q0, stream):
        """The same footprint as lq_gdn_decode: a deferred head is flushed by the next call that steps its slot, which
        reads and writes the same (slot, head) bytes as the flush it replaces."""
        cv_ = _arg(cv) if cv is not None else None
        rc = self._step("lq_gdn_decode_deferred", st, io, False, cv_)
        if rc:
            return rc
        io_ = _arg(io)
        return self._per_slot("lq_gdn_decode_deferred flush", st, ctypes.c_void_p(io_.idx), io_.N, False, False, Q0=Q0)

    def _per_slot(self, name, st, idx, N, kda, block, Q0=None, need_buf=True):
        st = _arg(st)
        self.calls.append(name)
        if not self._state_ok(st, need_buf=need_buf, kda=kda) or N < 0:
            return -1
        if N == 0:
            return 0
        idx = _arg(idx).value if hasattr(_arg(idx), "value") else _arg(idx)
        self.storages.check(name + " idx", idx, 0, 4 * N)
        if Q0 is not None:
            Q0 = _arg(Q0).value if hasattr(_arg(Q0), "value") else _arg(Q0)
            self.storages.check(name + " Q0", Q0, 0, 4 * st.V * st.R)
        for slot in _ints(idx, N):
            if 0 < slot < st.NS:
                for hv in range(st.HV):
                    self._head(st, slot, hv, kda, name, block=block)
        self._ctl(st, name)
        return 0

    def lq_flush(self, st, Q0, idx, N, kda, qmax, stream):
        return self._per_slot("lq_flush", st, idx, N, bool(kda), False, Q0=Q0)

    def lq_quantize(self, st, Q0, idx, N, qmax, stream):
        return self._per_slot("lq_quantize", st, idx, N, False, True, Q0=Q0, need_buf=False)

    def lq_dequant(self, st, idx, N, qmax, stream):
        return self._per_slot("lq_dequant", st, idx, N, False, True)

    def lq_kda_dequant(self, st, idx, N, qmax, stream):
        return self._per_slot("lq_kda_dequant", st, idx, N, True, True)

    def lq_kda_checkpoint(self, st, Q0, idx, N, qmax, stream):
        return self._per_slot("lq_kda_checkpoint", st, idx, N, True, True, Q0=Q0, need_buf=False)

    def lq_lowrank(self, x, Q0, U, Q, n, K, V, R, iters, stream):
        self.calls.append("lq_lowrank")
        if (K, V) != (128, 128) or not 1 <= R <= 4 or n < 0 or iters < 1:
            return -1
        if n == 0:
            return 0
        v = lambda p: _arg(p).value if hasattr(_arg(p), "value") else _arg(p)
        S = self.storages
        S.check("lq_lowrank x", v(x), 0, 4 * n * K * V)
        S.check("lq_lowrank Q0", v(Q0), 0, 4 * V * R)
        S.check("lq_lowrank U", v(U), 0, 4 * n * K * R)
        S.check("lq_lowrank Q", v(Q), 0, 4 * n * V * R)
        return 0

    def lq_conv_update(self, cv, x, out, idx, N, C, NS, stream):
        cv = _arg(cv)
        self.calls.append("lq_conv_update")
        if not self._conv_ok(cv, C) or N < 0 or C <= 0 or NS <= 0:
            return -1
        if N == 0:
            return 0
        v = lambda p: _arg(p).value if hasattr(_arg(p), "value") else _arg(p)
        S = self.storages
        S.check("lq_conv_update idx", v(idx), 0, 4 * N)
        self._conv_params(cv, C, "lq_conv_update")
        for n, slot in enumerate(_ints(v(idx), N)):
            if 0 < slot < min(NS, cv.NS):
                S.check("lq_conv_update x row", v(x), 2 * n * C, 2 * C)
                S.check("lq_conv_update out row", v(out), 2 * n * C, 2 * C)
                top = slot * cv.slot_stride + (C - 1) * cv.ch_stride + 2 * cv.tap_stride
                S.check("lq_conv_update conv state", cv.state, 2 * slot * cv.slot_stride,
                        2 * (top - slot * cv.slot_stride + 1))
        return 0

    def lq_dense_step(self, S_, dtype, NS, HV, H, K, V, io, stream):
        io = _arg(io)
        self.calls.append("lq_dense_step")
        if (K, V) != (128, 128) or H <= 0 or HV <= 0 or HV % H or NS <= 0 or io.N < 0 or dtype not in (0, 1):
            return -1
        if HV // H not in (1, 2, 4):
            return -1
        if io.N == 0:
            return 0
        base = _arg(S_).value if hasattr(_arg(S_), "value") else _arg(S_)
        if base % 16 or io.mixed % 16:                 # 16-byte loads of the state rows and of q, k
            return -1
        esz = 2 if dtype == 0 else 4
        S = self.storages
        MIX = 2 * H * K + HV * V
        S.check("lq_dense_step idx", io.idx, 0, 4 * io.N)
        S.check("lq_dense_step out", io.out, 0, 2 * io.N * HV * V)
        S.check("lq_dense_step A_log", io.A_log, 0, 4 * HV)
        S.check("lq_dense_step dt_bias", io.dt_bias, 0, 4 * HV)
        for n, slot in enumerate(_ints(io.idx, io.N)):
            if 0 < slot < NS:
                S.check("lq_dense_step mixed row", io.mixed, 2 * n * MIX, 2 * MIX)
                S.check("lq_dense_step a row", io.a, 2 * n * HV, 2 * HV)
                S.check("lq_dense_step b row", io.b, 2 * n * HV, 2 * HV)
                S.check("lq_dense_step state", base, esz * slot * HV * V * K, esz * HV * V * K)
        return 0


def clear_factory_caches():
    """The cached kernel factories hold the library handle they were made with: drop them when the handle changes."""
    from leapquant_amd import kernels as KN
    from leapquant_amd import state as S
    S._make_dequant.cache_clear()
    S._make_quantize.cache_clear()
    KN._lowrank_kernel.cache_clear()


def install(monkeypatch):
    """Route leapquant_amd's library handle to a CheckingLib and let host tensors through `_dev` (recording their
    storages); torch's current stream becomes a stand-in with stream 0.  Returns the CheckingLib.  The caller clears
    the factory caches again when it is done (clear_factory_caches), so later users get factories on the real library."""
    from leapquant_amd import _lib
    from leapquant_amd import kernels as KN
    clear_factory_caches()
    fake = CheckingLib()

    def dev(t):
        fake.storages.add(t)
        return t.data_ptr()

    class _Stream:
        cuda_stream = 0

    monkeypatch.setattr(KN, "_dev", dev)
    monkeypatch.setattr(_lib, "_LIB", [fake])
    monkeypatch.setattr(torch.cuda, "current_stream", lambda *a, **k: _Stream())
    return fake
