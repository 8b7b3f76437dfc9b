"""Kernel factories of the INT8 recurrent-state decode path, MI355X (gfx950) HIP implementation.

Same names, arguments and positional call conventions as /root/reference/leapquant/kernels.py (the factories
make_gdn_step 27-692, make_kda_step 694-1075, make_flush 1077-2033, make_dequant 2041-2123, make_quantize 2126-2242,
make_lowrank 2246-2314, lowrank_factor 2321-2331 and the constants 12-25).  Each factory checks the static shape
arguments and returns a callable that takes the reference's positional tensors and launches hand-written HIP kernels
of liblq.so (include/lq.h) on torch's current stream -- no JIT, no host synchronisation, no allocation.

Deliberate differences (documented in the package's design notes):
  * Kbuf holds the buffered keys once per KEY head: [NS, H, L, K] instead of [NS, HV, L, K].
  * The NVIDIA schedule knobs (SMS, NSTAGE, NSTAGEQ, NCG, NNW, MAXIT, PAD, MMT, NTP, RSG, threads, BV) are accepted
    and ignored: the HIP kernels have one schedule for gfx950.
  * The window may be up to 64 entries (the reference's kernels stop at 16 / 32).
  * Ranks as the reference's asserts allow (kernels.py:63-64, 1091): R <= 4, plus R in {8, 12, 16} for the GDN step
    and R = 8 for the GDN flush at (K, V) = (128, 128); make_quantize / make_dequant take any R a step can read
    (the reference's quantize has no bound of its own beyond the slot fit).
  * make_gdn_step / make_kda_step / make_flush / make_quantize / make_dequant take a code range `qmax` (127: INT8,
    default; 31: 6-bit codes in the same int8 container).
"""
import ctypes
import functools

import torch

from . import _lib

F32, BF16, I32, I8 = "float32", "bfloat16", "int32", "int8"
QMAX = 127.0
SOFTPLUS_THRESHOLD = 20.0
EPS = 1e-12
STEP_CFG = {(128, 128): (6, 3, 2), (64, 128): (10, 5, 5), (64, 64): (8, 4, 4)}   # accepted for API parity, unused

LMAX = 64


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _dev(t):
    """Device address of a tensor; the kernels dereference it on the GPU, so a host tensor is an error here."""
    if not t.is_cuda:
        raise ValueError("liblq takes GPU tensors only, got a %s tensor" % t.device)
    return t.data_ptr()


def _p(t):
    return ctypes.c_void_p(_dev(t)) if t is not None else ctypes.c_void_p(0)


def _need(t, dtype, shape, name):
    if t.dtype != dtype:
        raise TypeError("%s: dtype %s, expected %s" % (name, t.dtype, dtype))
    if tuple(t.shape) != tuple(shape):
        raise ValueError("%s: shape %s, expected %s" % (name, tuple(t.shape), tuple(shape)))
    if not t.is_contiguous():
        raise ValueError("%s must be contiguous" % name)


GDN_DIMS = ((128, 128), (64, 128), (64, 64))        # kernels.py:62, 1089 (KDA: 128 x 128 only, 727)


def _check_dims(K, V, L, R, kda=False, rank="step"):
    """Static shape checks.  `rank`: whose rank rule applies -- "step" (kernels.py:63-64: R <= 4, or R in {8, 12, 16}
    at 128 x 128), "flush" (kernels.py:1091: R <= 4, or R = 8 for GDN 128 x 128) or "checkpoint" (quantize / dequant:
    any rank a step reads).  KDA keeps R <= 4 throughout (its step holds four factors, kernels.py:1036)."""
    dims = ((128, 128),) if kda else GDN_DIMS
    assert (K, V) in dims, "liblq: head dims (K, V) in %s, got (%d, %d)" % (dims, K, V)
    assert 1 <= L <= LMAX, "liblq: window 1 <= L <= %d, got %d" % (LMAX, L)
    wide = (K, V) == (128, 128) and not kda
    ok = {"step": wide and R % 4 == 0 and R <= 16, "flush": wide and R == 8, "checkpoint": wide and R <= 16}[rank]
    assert R >= 1 and (R <= 4 or ok), \
        "liblq: rank R = %d not supported here (%s, (K, V) = (%d, %d)%s)" % (R, rank, K, V, ", KDA" if kda else "")
    assert V * K // 4 + K + V + R * (K + V) // 2 <= V * K, "checkpoint must fit inside the fp32 slot"


def _check_qmax(qmax):
    if not 1.0 <= float(qmax) <= 127.0:
        raise ValueError("qmax: code range in [1, 127] expected (127: INT8, 31: 6-bit), got %r" % (qmax,))
    return float(qmax)


def state_struct(Sq, SS, Kbuf, Ubuf, Wbuf, Pbuf, Gbuf, hcnt, NS, HV, H, K, V, L, R, ctl=None, qmax=QMAX,
                 sched=None):
    """lq_state of a layer: `Sq` is any view whose data pointer is the checkpoint of (slot 0, head 0), i.e. the fp32
    cache's data pointer.  `ctl`: optional int32 [2] due flag + flush counter kept by the kernels (None: the flush scans
    hcnt).  `qmax`: code range of the stored checkpoint (the decode steps dequantise Sq Sk Sv / qmax).  `sched`:
    optional int32 [LQ_SCHED_INTS] zero buffer of the counters through which the persistent flush hands out its heads
    (None: static schedule; same results)."""
    if ctl is not None and (ctl.dtype != torch.int32 or ctl.numel() < 2):
        raise ValueError("ctl: int32 [2] expected")
    if sched is not None and (sched.dtype != torch.int32 or sched.numel() < _lib.SCHED_INTS or not sched.is_contiguous()):
        raise ValueError("sched: contiguous int32 [%d] expected" % _lib.SCHED_INTS)
    return _lib.LqState(_dev(Sq), SS, _dev(Kbuf), _dev(Ubuf), _dev(Wbuf), _dev(Pbuf),
                        _dev(Gbuf) if Gbuf is not None else 0, _dev(hcnt), NS, HV, H, K, V, L, R,
                        _dev(ctl) if ctl is not None else 0, _check_qmax(qmax),
                        _dev(sched) if sched is not None else 0)


def _check_view(Sq, NS, HV, V, K, SS):
    if Sq.shape[0] != NS or Sq.shape[1] != HV or Sq.stride(0) * Sq.element_size() != 4 * SS:
        raise ValueError("checkpoint view does not match NS=%d HV=%d SS=%d" % (NS, HV, SS))
    if Sq.data_ptr() % 16 or SS % 4:
        raise ValueError("the fp32 state cache must be 16-byte aligned with a slot stride divisible by 4")


def _step_io(mixed, a, b, A_log, dt_bias, idx, o, scale):
    N = idx.shape[0]
    return _lib.LqStepIO(_dev(mixed), _dev(a), _dev(b), _dev(A_log), _dev(dt_bias), _dev(idx), _dev(o), N,
                         float(scale))


def _check_step_inputs(N, HV, H, K, V, mixed, a, b, A_log, dt_bias, idx, o, KA):
    _need(mixed, torch.bfloat16, (N, 2 * H * K + HV * V), "mixed")
    if a.dtype != torch.bfloat16 or a.numel() != N * HV * KA or not a.is_contiguous():
        raise ValueError("a: bf16 contiguous with %d elements expected" % (N * HV * KA))
    _need(b, torch.bfloat16, (N, HV), "b")
    if A_log.dtype != torch.float32 or A_log.numel() != HV or not A_log.is_contiguous():
        raise ValueError("A_log: fp32 [HV] expected")
    if dt_bias.dtype != torch.float32 or dt_bias.numel() != HV * KA or not dt_bias.is_contiguous():
        raise ValueError("dt_bias: fp32 [HV * KA] expected")
    _need(idx, torch.int32, (N,), "idx")
    if o.dtype != torch.bfloat16 or o.numel() != N * HV * V or not o.is_contiguous():
        raise ValueError("o: bf16 contiguous [N, HV, V] expected")


def make_gdn_step(NS, HV, H, K, V, L, SS, R=4, SMS=None, NSTAGE=None, NCG=None, NNW=None, scale=None, MAXIT=256,
                  qmax=QMAX):
    """Gated DeltaNet decode step on the 8-bit state (kernels.py:27-692).  Returns
    step(Sq, Sk, Sv, Skv, Kbuf, Ubuf, Wbuf, Pbuf, hcnt, mixed, a, b, A_log, dt_bias, UQ, idx, o).  `qmax`: the code range
    of the stored checkpoint (127: INT8, 31: 6-bit)."""
    _check_dims(K, V, L, R)
    qmax = _check_qmax(qmax)
    assert HV % H == 0 and HV // H in (1, 2, 4), "liblq: HV / H in {1, 2, 4}"
    scale = K ** -0.5 if scale is None else scale
    L_ = _lib.lib()

    def step(Sq, Sk, Sv, Skv, Kbuf, Ubuf, Wbuf, Pbuf, hcnt, mixed, a, b, A_log, dt_bias, UQ, idx, o):
        N = idx.shape[0]
        _check_view(Sq, NS, HV, V, K, SS)
        _need(Kbuf, torch.bfloat16, (NS, H, L, K), "Kbuf")
        _need(Ubuf, torch.bfloat16, (NS, HV, L, V), "Ubuf")
        _need(Wbuf, torch.float32, (NS, HV, L), "Wbuf")
        _need(Pbuf, torch.float32, (NS, HV, 1), "Pbuf")
        _need(hcnt, torch.int32, (NS, HV), "hcnt")
        _check_step_inputs(N, HV, H, K, V, mixed, a, b, A_log, dt_bias, idx, o, 1)
        st = state_struct(Sq, SS, Kbuf, Ubuf, Wbuf, Pbuf, None, hcnt, NS, HV, H, K, V, L, R, qmax=qmax)
        io = _step_io(mixed, a, b, A_log, dt_bias, idx, o, scale)
        _lib.check(L_.lq_gdn_step(ctypes.byref(st), ctypes.byref(io), _stream(mixed)), "lq_gdn_step")

    return step


def make_kda_step(NS, HV, H, K, V, L, SS, R=4, SMS=None, NSTAGE=6, NSTAGEQ=4, NCG=2, NNW=2, scale=128 ** -0.5,
                  MAXIT=256, GLB=0.0, qmax=QMAX):
    """Kimi Delta Attention decode step (kernels.py:694-1075), per-key-channel gate; GLB != 0 selects GLM's bounded
    gate.  Returns step(Sq, Sk, Sv, Skv, Kbuf, Ubuf, Wbuf, Pbuf, Gbuf, hcnt, mixed, a, b, A_log, dt_bias, UQ, idx, o).
    `qmax`: the code range of the stored checkpoint (127: INT8, 31: 6-bit)."""
    _check_dims(K, V, L, R, kda=True)
    qmax = _check_qmax(qmax)
    assert HV % H == 0, "liblq: HV % H == 0"
    L_ = _lib.lib()
    glb = float(GLB)

    def step(Sq, Sk, Sv, Skv, Kbuf, Ubuf, Wbuf, Pbuf, Gbuf, hcnt, mixed, a, b, A_log, dt_bias, UQ, idx, o):
        N = idx.shape[0]
        _check_view(Sq, NS, HV, V, K, SS)
        _need(Kbuf, torch.bfloat16, (NS, H, L, K), "Kbuf")
        _need(Ubuf, torch.bfloat16, (NS, HV, L, V), "Ubuf")
        _need(Wbuf, torch.float32, (NS, HV, L), "Wbuf")
        _need(Pbuf, torch.float32, (NS, HV, K), "Pbuf")
        if Gbuf.element_size() != 2 or tuple(Gbuf.shape) != (NS, HV, L, K) or not Gbuf.is_contiguous():
            raise ValueError("Gbuf: 16-bit [NS, HV, L, K] expected")
        _need(hcnt, torch.int32, (NS, HV), "hcnt")
        _check_step_inputs(N, HV, H, K, V, mixed, a, b, A_log, dt_bias, idx, o, K)
        st = state_struct(Sq, SS, Kbuf, Ubuf, Wbuf, Pbuf, Gbuf, hcnt, NS, HV, H, K, V, L, R, qmax=qmax)
        io = _step_io(mixed, a, b, A_log, dt_bias, idx, o, scale)
        _lib.check(L_.lq_kda_step(ctypes.byref(st), ctypes.byref(io), ctypes.c_float(glb), _stream(mixed)),
                   "lq_kda_step")

    return step


def make_flush(NS, HV, K, V, L, SS, R=4, ITERS=1, SMS=None, NCG=3, MAXIT=128, PAD=8, KDA=False, MMT="bf16",
               PNMIN=1e-20, NMAX=0, NTP=0, RSG=None, qmax=QMAX, sched=None):
    """End-of-window flush (kernels.py:1077-2033).  Returns
    flush(Sq, Sk, Sv, Skv, Kbuf, Ubuf, Wbuf, Pbuf, Gbuf, hcnt, Sq16, UQ, Q0, idx).  Due heads (hcnt == L) are found on
    the device; ITERS = 1 and PNMIN = 1e-20 as in the reference's use (state.py:79).  `sched` (not in the reference's
    signature): the optional int32 [LQ_SCHED_INTS] zero buffer of the flush's dynamic head schedule (see state_struct)."""
    _check_dims(K, V, L, R, kda=KDA, rank="flush")
    assert ITERS == 1, "liblq: one subspace iteration per flush (ITERS = 1)"
    assert PNMIN == 1e-20
    L_ = _lib.lib()
    kda = 1 if KDA else 0

    def flush(Sq, Sk, Sv, Skv, Kbuf, Ubuf, Wbuf, Pbuf, Gbuf, hcnt, Sq16, UQ, Q0, idx):
        N = idx.shape[0]
        _check_view(Sq, NS, HV, V, K, SS)
        H = Kbuf.shape[1]
        _need(Kbuf, torch.bfloat16, (NS, H, L, K), "Kbuf")
        _need(Ubuf, torch.bfloat16, (NS, HV, L, V), "Ubuf")
        _need(Wbuf, torch.float32, (NS, HV, L), "Wbuf")
        _need(Pbuf, torch.float32, (NS, HV, K if KDA else 1), "Pbuf")
        _need(hcnt, torch.int32, (NS, HV), "hcnt")
        _need(Q0, torch.float32, (V, R), "Q0")
        _need(idx, torch.int32, (N,), "idx")
        if KDA and (Gbuf.element_size() != 2 or tuple(Gbuf.shape) != (NS, HV, L, K)):
            raise ValueError("Gbuf: 16-bit [NS, HV, L, K] expected")
        st = state_struct(Sq, SS, Kbuf, Ubuf, Wbuf, Pbuf, Gbuf if KDA else None, hcnt, NS, HV, H, K, V, L, R,
                          sched=sched)
        _lib.check(L_.lq_flush(ctypes.byref(st), _p(Q0), _p(idx), N, kda, ctypes.c_float(qmax), _stream(idx)),
                   "lq_flush")

    return flush


def make_dequant(NS, HV, K, V, L, SS, BV=32, threads=128, kda=False, buf_dtype=F32, R=0, qmax=QMAX):
    """Prefill round trip, part 1 (kernels.py:2041-2123): fp32 S[slot] <- decay deq(S0) + window, then window reset.
    Returns dequant(S0, Sq, Sk, Sv, Kbuf, Ubuf, Wbuf, Pbuf, Gbuf, hcnt, UQ, idx).  GDN with bf16 buffers only (the
    reference's KDA branch is never called: state.py:80-82)."""
    _check_dims(K, V, L, max(R, 1), rank="checkpoint")
    assert not kda and buf_dtype == BF16 and R >= 1, "liblq: GDN dequant with bf16 buffers and R >= 1"
    L_ = _lib.lib()

    def dequant(S0, Sq, Sk, Sv, Kbuf, Ubuf, Wbuf, Pbuf, Gbuf, hcnt, UQ, idx):
        N = idx.shape[0]
        _check_view(S0, NS, HV, V, K, SS)
        H = Kbuf.shape[1]
        _need(Kbuf, torch.bfloat16, (NS, H, L, K), "Kbuf")
        _need(Ubuf, torch.bfloat16, (NS, HV, L, V), "Ubuf")
        _need(idx, torch.int32, (N,), "idx")
        st = state_struct(S0, SS, Kbuf, Ubuf, Wbuf, Pbuf, None, hcnt, NS, HV, H, K, V, L, R)
        _lib.check(L_.lq_dequant(ctypes.byref(st), _p(idx), N, ctypes.c_float(qmax), _stream(idx)), "lq_dequant")

    return dequant


def make_quantize(NS, HV, K, V, L, SS, R=4, ITERS=1, threads=128, qmax=QMAX):
    """Prefill round trip, part 2 (kernels.py:2126-2242): 8-bit checkpoint of the fp32 states of the listed slots,
    then window reset.  Returns quantize(S0, Sq, Sk, Sv, UQ, Wbuf, Pbuf, hcnt, Q0, idx)."""
    _check_dims(K, V, L, R, rank="checkpoint")
    assert ITERS == 1, "liblq: ITERS = 1"
    L_ = _lib.lib()

    def quantize(S0, Sq, Sk, Sv, UQ, Wbuf, Pbuf, hcnt, Q0, idx):
        N = idx.shape[0]
        _check_view(S0, NS, HV, V, K, SS)
        _need(Wbuf, torch.float32, (NS, HV, L), "Wbuf")
        _need(Q0, torch.float32, (V, R), "Q0")
        _need(idx, torch.int32, (N,), "idx")
        st = _lib.LqState(_dev(S0), SS, 0, 0, _dev(Wbuf), _dev(Pbuf), 0, _dev(hcnt),
                          NS, HV, HV, K, V, L, R)
        _lib.check(L_.lq_quantize(ctypes.byref(st), _p(Q0), _p(idx), N, ctypes.c_float(qmax), _stream(idx)),
                   "lq_quantize")

    return quantize


def make_lowrank(K, V, R, ITERS, threads=128):
    """Rank-R subspace iteration on [N, K, V] fp32 with MGS (kernels.py:2246-2314).  Returns lowrank(S, Q0, U, Q)."""
    assert (K, V) == (128, 128) and 1 <= R <= 4 and ITERS >= 1
    L_ = _lib.lib()

    def lowrank(S, Q0, U, Q):
        n = S.shape[0]
        _need(S, torch.float32, (n, K, V), "S")
        _need(Q0, torch.float32, (V, R), "Q0")
        _need(U, torch.float32, (n, K, R), "U")
        _need(Q, torch.float32, (n, V, R), "Q")
        _lib.check(L_.lq_lowrank(_p(S), _p(Q0), _p(U), _p(Q), n, K, V, R, ITERS, _stream(S)), "lq_lowrank")

    return lowrank


@functools.lru_cache(maxsize=None)
def _lowrank_start(device, V, r):
    """The factoriser's fixed start, randn(V, r) from a CPU generator seeded 0 (kernels.py:2318-2331), on `device`."""
    return torch.randn(V, r, generator=torch.Generator().manual_seed(0)).to(device)


_lowrank_kernel = functools.lru_cache(maxsize=None)(make_lowrank)


def lowrank_factor(x, r, iters=3):
    """Rank-r factors of x [..., K, V] (fp32, on the GPU): U [..., K, r], Q [..., V, r] with x ~ U Q^T, from `iters`
    rounds of subspace iteration with MGS (kernels.py:2321-2331)."""
    *lead, K, V = x.shape
    xs = x.reshape(-1, K, V).float().contiguous()
    U = xs.new_empty(xs.shape[0], K, r)
    Q = xs.new_empty(xs.shape[0], V, r)
    _lowrank_kernel(K, V, r, iters)(xs, _lowrank_start(x.device, V, r), U, Q)
    return U.view(*lead, K, r), Q.view(*lead, V, r)


def conv_struct(conv_state, weight, bias=None, silu=True):
    """lq_conv of a conv state [NS, C, W - 1] view (any strides), bf16 weights [C, 4] and optional bf16 bias [C]; the
    kernels treat a row whose slot is not below the conv state's NS as a padding row."""
    C = weight.shape[0]
    w = weight.reshape(C, -1)
    if conv_state.dtype != torch.bfloat16 or conv_state.dim() != 3 or conv_state.shape[1:] != (C, 3):
        raise ValueError("conv_state: bf16 [NS, C, 3] expected")
    if w.dtype != torch.bfloat16 or w.shape[1] != 4 or not w.is_contiguous():
        raise ValueError("conv weight: contiguous bf16 [C, 4] expected")
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.numel() != C or not bias.is_contiguous()):
        raise ValueError("conv bias: bf16 [C] expected")
    return _lib.LqConv(_dev(conv_state), _dev(w), _dev(bias) if bias is not None else 0, conv_state.stride(0),
                       conv_state.stride(1), conv_state.stride(2), 4, 1 if silu else 0, conv_state.shape[0])


def conv_update(x, conv_state, weight, bias, idx, out, silu=True):
    """Baseline (stands for vLLM's causal_conv1d_update): out [N, C] bf16 from the raw projection x [N, C], the conv
    states of the slots idx[n] > 0 shifted in place (the arithmetic lq_gdn_step_conv fuses into the step)."""
    N, C = x.shape
    cv = conv_struct(conv_state, weight, bias, silu)
    _need(x, torch.bfloat16, (N, C), "x")
    _need(out, torch.bfloat16, (N, C), "out")
    _need(idx, torch.int32, (N,), "idx")
    _lib.check(_lib.lib().lq_conv_update(ctypes.byref(cv), _p(x), _p(out), _p(idx), N, C, conv_state.shape[0],
                                         _stream(x)), "lq_conv_update")


def dense_step(S, mixed, a, b, A_log, dt_bias, idx, o, H, scale=None):
    """Baseline (no reference counterpart): the same GDN decode step on a dense bf16 / fp32 state S [NS, HV, V, K]
    updated in place."""
    NS, HV, V, K = S.shape
    assert S.is_contiguous() and S.dtype in (torch.bfloat16, torch.float32)
    N = idx.shape[0]
    _check_step_inputs(N, HV, H, K, V, mixed, a, b, A_log, dt_bias, idx, o, 1)
    io = _step_io(mixed, a, b, A_log, dt_bias, idx, o, K ** -0.5 if scale is None else scale)
    _lib.check(_lib.lib().lq_dense_step(_p(S), 0 if S.dtype == torch.bfloat16 else 1, NS, HV, H, K, V,
                                        ctypes.byref(io), _stream(S)), "lq_dense_step")
