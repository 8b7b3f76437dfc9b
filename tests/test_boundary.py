"""CPU tests of the drop-in boundary: liblq.so loads and exports exactly what include/lq.h declares, every entry point
rejects bad arguments before touching the GPU, and the Python mirror of the reference API (leapquant/kernels.py,
leapquant/state.py) checks shapes, devices and layouts the way the reference's asserts do.  No kernel is launched."""
import ctypes
import os
import re
import subprocess

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lq.h")


@pytest.fixture(scope="module")
def lib():
    from leapquant_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from leapquant_amd import build
        build.build()
    return _lib.lib()


def declared():
    src = open(HEADER).read()
    return set(re.findall(r"^int\s+(lq_\w+)\s*\(", src, flags=re.M))


def test_header_and_binding_agree():
    from leapquant_amd import _lib
    assert declared() == set(_lib.SIGNATURES)
    m = re.search(r"#define\s+LQ_ABI_VERSION\s+(\d+)", open(HEADER).read())
    assert int(m.group(1)) == _lib.ABI_VERSION


def test_library_exports_every_declared_symbol(lib):
    from leapquant_amd import _lib
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    missing = declared() - exported
    assert not missing, missing
    for name in declared():
        assert hasattr(lib, name)
    assert lib.lq_abi_version() == _lib.ABI_VERSION


def _state(**kw):
    from leapquant_amd import _lib
    d = dict(ssm=16, slot_stride=4 * 128 * 128, Kbuf=32, Ubuf=48, Wbuf=64, Pbuf=80, Gbuf=96, hcnt=112,
             NS=8, HV=4, H=2, K=128, V=128, L=16, R=4)
    d.update(kw)
    return _lib.LqState(**d)


def _io(**kw):
    from leapquant_amd import _lib
    d = dict(mixed=16, a=32, b=48, A_log=64, dt_bias=80, idx=96, out=112, N=0, scale=128 ** -0.5)
    d.update(kw)
    return _lib.LqStepIO(**d)


BAD_STATES = [dict(K=96), dict(V=64), dict(K=32, V=32), dict(L=0), dict(L=65), dict(R=0), dict(R=17), dict(H=0), dict(HV=3),
              dict(NS=0), dict(slot_stride=100), dict(slot_stride=4 * 128 * 128 + 1), dict(ssm=8), dict(ssm=None),
              dict(hcnt=None), dict(Wbuf=None), dict(Kbuf=40), dict(Ubuf=56), dict(Gbuf=104)]   # last three: not
# 16-byte aligned (the window rows are read by 16-byte and direct-to-LDS loads)
BAD_STEP_STATES = [dict(qmax=0.5), dict(qmax=128.0), dict(qmax=-31.0), dict(qmax=float("nan"))]


@pytest.mark.parametrize("bad", BAD_STEP_STATES)
def test_steps_reject_a_bad_code_range(lib, bad):
    """The decode steps dequantise with lq_state.qmax (0: INT8; else 1 <= qmax <= 127)."""
    st, io = _state(**bad), _io()
    z = ctypes.c_void_p(0)
    assert lib.lq_gdn_step(ctypes.byref(st), ctypes.byref(io), z) == -1
    assert lib.lq_kda_step(ctypes.byref(st), ctypes.byref(io), ctypes.c_float(0.0), z) == -1
    for ok in (0.0, 31.0, 127.0):
        assert lib.lq_gdn_step(ctypes.byref(_state(qmax=ok)), ctypes.byref(io), z) == 0


@pytest.mark.parametrize("bad", BAD_STATES)
def test_entry_points_reject_bad_state(lib, bad):
    """N = 0 calls with one bad field: each entry point returns LQ_ERR_ARG (-1) without a launch."""
    st = _state(**bad)
    io = _io()
    z = ctypes.c_void_p(0)
    assert lib.lq_gdn_step(ctypes.byref(st), ctypes.byref(io), z) == -1
    assert lib.lq_kda_step(ctypes.byref(st), ctypes.byref(io), ctypes.c_float(0.0), z) == -1
    assert lib.lq_flush(ctypes.byref(st), ctypes.c_void_p(16), ctypes.c_void_p(16), 0, 0, ctypes.c_float(127.0), z) == -1
    assert lib.lq_dequant(ctypes.byref(st), ctypes.c_void_p(16), 0, ctypes.c_float(127.0), z) == -1
    assert lib.lq_kda_dequant(ctypes.byref(st), ctypes.c_void_p(16), 0, ctypes.c_float(127.0), z) == -1
    if "Kbuf" not in bad and "Ubuf" not in bad:
        assert lib.lq_quantize(ctypes.byref(st), ctypes.c_void_p(16), ctypes.c_void_p(16), 0, ctypes.c_float(127.0),
                               z) == -1
        assert lib.lq_kda_checkpoint(ctypes.byref(st), ctypes.c_void_p(16), ctypes.c_void_p(16), 0,
                                     ctypes.c_float(127.0), z) == -1


def test_rank_limits(lib):
    """Ranks above 4 (kernels.py:63-64, 1091): GDN 128 x 128 steps take R <= 16, its flush R <= 8, quantize / dequant
    R <= 16; KDA and the 64-dim heads stay at R <= 4.  The factories keep the reference's own sets (step R in
    {8, 12, 16}, flush R = 8)."""
    z, p = ctypes.c_void_p(0), ctypes.c_void_p(16)
    io = _io()
    for R in (5, 8, 12, 16):
        st = _state(R=R)
        assert lib.lq_gdn_step(ctypes.byref(st), ctypes.byref(io), z) == 0
        assert lib.lq_kda_step(ctypes.byref(st), ctypes.byref(io), ctypes.c_float(0.0), z) == -1
        assert lib.lq_flush(ctypes.byref(st), p, p, 0, 0, ctypes.c_float(127.0), z) == (0 if R <= 8 else -1)
        assert lib.lq_flush(ctypes.byref(st), p, p, 0, 1, ctypes.c_float(127.0), z) == -1
        assert lib.lq_gdn_decode(ctypes.byref(st), ctypes.byref(io), None, p, z) == (0 if R <= 8 else -1)
        assert lib.lq_quantize(ctypes.byref(st), p, p, 0, ctypes.c_float(127.0), z) == 0
        assert lib.lq_dequant(ctypes.byref(st), p, 0, ctypes.c_float(127.0), z) == 0
        assert lib.lq_kda_dequant(ctypes.byref(st), p, 0, ctypes.c_float(127.0), z) == -1
        assert lib.lq_kda_checkpoint(ctypes.byref(st), p, p, 0, ctypes.c_float(127.0), z) == -1
        for K, V in ((64, 128), (64, 64)):
            st = _state(R=R, K=K, V=V)
            assert lib.lq_gdn_step(ctypes.byref(st), ctypes.byref(io), z) == -1
            assert lib.lq_flush(ctypes.byref(st), p, p, 0, 0, ctypes.c_float(127.0), z) == -1
            assert lib.lq_quantize(ctypes.byref(st), p, p, 0, ctypes.c_float(127.0), z) == -1
    from leapquant_amd import kernels as KN
    SS = 32 * 128 * 128
    for R in (1, 4, 8, 12, 16):
        KN.make_gdn_step(4, 32, 16, 128, 128, 16, SS, R=R)
        KN.make_quantize(4, 32, 128, 128, 16, SS, R=R)
        KN.make_dequant(4, 32, 128, 128, 16, SS, buf_dtype=KN.BF16, R=R)
    KN.make_flush(4, 32, 128, 128, 16, SS, R=8)
    for bad in (dict(R=6), dict(R=20), dict(R=8, K=64, SS=32 * 64 * 128)):
        kw = dict(K=128, SS=SS)
        kw.update(bad)
        with pytest.raises(AssertionError):
            KN.make_gdn_step(4, 32, 16, kw["K"], 128, 16, kw["SS"], R=kw["R"])
    for bad in (dict(R=12), dict(R=6), dict(R=8, KDA=True)):
        with pytest.raises(AssertionError):
            KN.make_flush(4, 32, 128, 128, 16, SS, **bad)
    with pytest.raises(AssertionError):
        KN.make_kda_step(4, 32, 32, 128, 128, 16, SS, R=8)


@pytest.mark.parametrize("K,V", [(64, 128), (64, 64)])
def test_head_dims_gdn_only(lib, K, V):
    """(K, V) = (64, 128), (64, 64) (kernels.py:62, 1089): accepted by the GDN step, flush, quantize and dequant,
    rejected by every KDA entry point (kernels.py:727)."""
    st, io = _state(K=K, V=V), _io()
    z, p = ctypes.c_void_p(0), ctypes.c_void_p(16)
    assert lib.lq_gdn_step(ctypes.byref(st), ctypes.byref(io), z) == 0
    assert lib.lq_flush(ctypes.byref(st), p, p, 0, 0, ctypes.c_float(127.0), z) == 0
    assert lib.lq_quantize(ctypes.byref(st), p, p, 0, ctypes.c_float(127.0), z) == 0
    assert lib.lq_dequant(ctypes.byref(st), p, 0, ctypes.c_float(127.0), z) == 0
    assert lib.lq_kda_step(ctypes.byref(st), ctypes.byref(io), ctypes.c_float(0.0), z) == -1
    assert lib.lq_flush(ctypes.byref(st), p, p, 0, 1, ctypes.c_float(127.0), z) == -1
    assert lib.lq_kda_dequant(ctypes.byref(st), p, 0, ctypes.c_float(127.0), z) == -1
    assert lib.lq_kda_checkpoint(ctypes.byref(st), p, p, 0, ctypes.c_float(127.0), z) == -1
    assert lib.lq_lowrank(p, p, p, p, 0, K, V, 4, 3, z) == -1


def test_entry_points_accept_empty_calls(lib):
    """A valid state with N = 0 rows is a no-op that succeeds (no HIP call is made)."""
    st, io = _state(), _io()
    z = ctypes.c_void_p(0)
    assert lib.lq_gdn_step(ctypes.byref(st), ctypes.byref(io), z) == 0
    assert lib.lq_kda_step(ctypes.byref(st), ctypes.byref(io), ctypes.c_float(0.0), z) == 0
    assert lib.lq_flush(ctypes.byref(st), ctypes.c_void_p(16), ctypes.c_void_p(16), 0, 1, ctypes.c_float(31.0), z) == 0
    assert lib.lq_quantize(ctypes.byref(st), ctypes.c_void_p(16), ctypes.c_void_p(16), 0, ctypes.c_float(127.0), z) == 0
    assert lib.lq_dequant(ctypes.byref(st), ctypes.c_void_p(16), 0, ctypes.c_float(127.0), z) == 0
    assert lib.lq_kda_dequant(ctypes.byref(st), ctypes.c_void_p(16), 0, ctypes.c_float(127.0), z) == 0
    assert lib.lq_kda_checkpoint(ctypes.byref(st), ctypes.c_void_p(16), ctypes.c_void_p(16), 0, ctypes.c_float(31.0),
                                 z) == 0
    assert lib.lq_lowrank(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), 0, 128, 128,
                          4, 3, z) == 0


def test_other_argument_errors(lib):
    z = ctypes.c_void_p(0)
    st = _state()
    # rows but null input pointers
    assert lib.lq_gdn_step(ctypes.byref(st), ctypes.byref(_io(N=4, mixed=None)), z) == -1
    assert lib.lq_gdn_step(None, ctypes.byref(_io()), z) == -1
    assert lib.lq_gdn_step(ctypes.byref(st), None, z) == -1
    # KDA needs Gbuf
    assert lib.lq_kda_step(ctypes.byref(_state(Gbuf=None)), ctypes.byref(_io()), ctypes.c_float(0.0), z) == -1
    assert lib.lq_flush(ctypes.byref(_state(Gbuf=None)), ctypes.c_void_p(16), ctypes.c_void_p(16), 0, 1,
                        ctypes.c_float(127.0), z) == -1
    assert lib.lq_kda_dequant(ctypes.byref(_state(Gbuf=None)), ctypes.c_void_p(16), 0, ctypes.c_float(127.0), z) == -1
    assert lib.lq_kda_checkpoint(ctypes.byref(_state(Gbuf=None)), ctypes.c_void_p(16), ctypes.c_void_p(16), 0,
                                 ctypes.c_float(127.0), z) == -1
    # GDN step: HV / H must be 1, 2 or 4
    assert lib.lq_gdn_step(ctypes.byref(_state(HV=24, H=3)), ctypes.byref(_io(N=1)), z) == -1
    # code range
    for q in (0.5, 128.0, float("nan")):
        assert lib.lq_flush(ctypes.byref(st), ctypes.c_void_p(16), ctypes.c_void_p(16), 1, 0, ctypes.c_float(q), z) == -1
        assert lib.lq_quantize(ctypes.byref(st), ctypes.c_void_p(16), ctypes.c_void_p(16), 1, ctypes.c_float(q), z) == -1
        assert lib.lq_kda_checkpoint(ctypes.byref(st), ctypes.c_void_p(16), ctypes.c_void_p(16), 1, ctypes.c_float(q),
                                     z) == -1
        assert lib.lq_kda_dequant(ctypes.byref(st), ctypes.c_void_p(16), 1, ctypes.c_float(q), z) == -1
    assert lib.lq_flush(ctypes.byref(st), None, ctypes.c_void_p(16), 1, 0, ctypes.c_float(127.0), z) == -1
    assert lib.lq_flush(ctypes.byref(st), ctypes.c_void_p(16), ctypes.c_void_p(16), -1, 0, ctypes.c_float(127.0), z) == -1
    # lowrank limits
    p = ctypes.c_void_p(16)
    assert lib.lq_lowrank(p, p, p, p, 1, 64, 128, 4, 3, z) == -1
    assert lib.lq_lowrank(p, p, p, p, 1, 128, 128, 5, 3, z) == -1
    assert lib.lq_lowrank(p, p, p, p, 1, 128, 128, 4, 0, z) == -1
    assert lib.lq_lowrank(None, p, p, p, 1, 128, 128, 4, 3, z) == -1
    # dense baseline
    io = _io()
    assert lib.lq_dense_step(p, 2, 8, 4, 2, 128, 128, ctypes.byref(io), z) == -1
    assert lib.lq_dense_step(None, 0, 8, 4, 2, 128, 128, ctypes.byref(io), z) == -1
    assert lib.lq_dense_step(p, 0, 8, 4, 2, 128, 128, ctypes.byref(io), z) == 0
    # 16-byte loads of q, k and the state rows: misaligned bases are refused before any launch
    assert lib.lq_dense_step(p, 0, 8, 4, 2, 128, 128, ctypes.byref(_io(N=1, mixed=24)), z) == -1
    assert lib.lq_dense_step(ctypes.c_void_p(8), 0, 8, 4, 2, 128, 128, ctypes.byref(_io(N=1)), z) == -1


def _conv(**kw):
    from leapquant_amd import _lib
    C = 2 * 2 * 128 + 4 * 128
    d = dict(state=16, weight=32, bias=None, slot_stride=3 * C, ch_stride=3, tap_stride=1, W=4, silu=1, NS=8)
    d.update(kw)
    return _lib.LqConv(**d)


def test_fused_conv_entry_points_check_their_arguments(lib):
    """lq_gdn_step_conv / lq_conv_update: width 4 only, state taps inside a slot, 8-byte aligned weights, null pointers,
    a conv-state slot count."""
    z = ctypes.c_void_p(0)
    st, io = _state(), _io()
    assert lib.lq_gdn_step_conv(ctypes.byref(st), ctypes.byref(io), ctypes.byref(_conv()), z) == 0      # N = 0
    for bad in (dict(W=3), dict(silu=2), dict(state=None), dict(weight=None), dict(weight=36), dict(slot_stride=100),
                dict(ch_stride=0), dict(tap_stride=0), dict(NS=0), dict(NS=-1)):
        assert lib.lq_gdn_step_conv(ctypes.byref(st), ctypes.byref(io), ctypes.byref(_conv(**bad)), z) == -1, bad
        assert lib.lq_conv_update(ctypes.byref(_conv(**bad)), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                  ctypes.c_void_p(16), 1, 1024, 8, z) == -1, bad
    assert lib.lq_gdn_step_conv(ctypes.byref(st), ctypes.byref(io), None, z) == -1
    assert lib.lq_gdn_step_conv(ctypes.byref(_state(K=96)), ctypes.byref(io), ctypes.byref(_conv()), z) == -1
    assert lib.lq_conv_update(ctypes.byref(_conv()), ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                              0, 1024, 8, z) == 0
    assert lib.lq_conv_update(ctypes.byref(_conv()), None, ctypes.c_void_p(16), ctypes.c_void_p(16), 1, 1024, 8,
                              z) == -1


def test_python_wrapper_raises_on_status():
    from leapquant_amd import _lib
    _lib.check(0, "x")
    with pytest.raises(RuntimeError, match="bad argument"):
        _lib.check(-1, "lq_gdn_step")
    with pytest.raises(RuntimeError, match="HIP launch error"):
        _lib.check(-2, "lq_flush")


def test_state_views_alias_the_checkpoint_layout():
    """state.py:29-40: Sq at byte 0, Sk at V K, Sv at V K + 4 K, UQ at V K + 4 K + 4 V of every (slot, head) block."""
    from leapquant_amd.state import state_views
    NS, HV, V, K, R = 3, 2, 128, 128, 4
    ssm = torch.zeros(NS, HV, V, K)
    v = state_views(ssm, R)
    base = ssm.data_ptr()
    blk = V * K * 4
    for s in range(NS):
        for h in range(HV):
            o = base + (s * HV + h) * blk
            assert v["Sq"][s, h].data_ptr() == o
            assert v["q32"][s, h].data_ptr() == o
            assert v["sq16"][s, h].data_ptr() == o
            assert v["Sk"][s, h].data_ptr() == o + V * K
            assert v["skv"][s, h].data_ptr() == o + V * K
            assert v["Sv"][s, h].data_ptr() == o + V * K + 4 * K
            assert v["uq"][s, h].data_ptr() == o + V * K + 4 * K + 4 * V
    assert v["uq"].shape == (NS, HV, R, K + V) and v["uq"].dtype == torch.float16
    # writes through the views land in the fp32 tensor's bytes and nowhere past the checkpoint
    v["Sq"][1, 1].fill_(-1)
    v["uq"][1, 1].fill_(1.0)
    raw = ssm[1, 1].view(torch.uint8).reshape(-1)
    end = V * K + 4 * K + 4 * V + 2 * R * (K + V)
    assert int(raw[:V * K].ne(255).sum()) == 0
    assert int(raw[end:].ne(0).sum()) == 0
    assert int(ssm[0].view(torch.uint8).ne(0).sum()) == 0


def test_state_rejects_what_the_reference_rejects(lib):
    from leapquant_amd.state import LeapQuantState
    with pytest.raises(AssertionError):
        LeapQuantState(torch.zeros(2, 2, 128, 128, dtype=torch.float16), 2)
    with pytest.raises(AssertionError):
        LeapQuantState(torch.zeros(2, 2, 128, 256)[..., ::2], 2)        # inner dims not packed
    st = LeapQuantState(torch.zeros(2, 4, 128, 128), 2, L=16)
    assert st.Kbuf.shape == (2, 2, 16, 128) and st.Ubuf.shape == (2, 4, 16, 128)
    assert float(st.Pbuf.min()) == 1.0 and st.hcnt.dtype == torch.int32
    k = LeapQuantState(torch.zeros(2, 4, 128, 128), 4, kda=True, L=16)
    assert k.Pbuf.shape == (2, 4, 128) and float(k.Pbuf.abs().max()) == 0.0
    assert k.Gbuf.dtype == torch.float16 and float(k.Gbuf.min()) == 1.0
    ref_q0 = torch.randn(128, 4, generator=torch.Generator().manual_seed(0))
    assert torch.equal(st.Q0.cpu(), ref_q0)


def test_host_tensors_never_reach_the_kernels(lib):
    """The product path refuses host tensors (their addresses would be dereferenced on the GPU)."""
    from leapquant_amd.state import LeapQuantState
    ssm = torch.zeros(3, 4, 128, 128)
    st = LeapQuantState(ssm, 2, L=16)
    N = 2
    mixed = torch.zeros(N, 2 * 2 * 128 + 4 * 128, dtype=torch.bfloat16)
    a = torch.zeros(N, 4, dtype=torch.bfloat16)
    b = torch.zeros(N, 4, dtype=torch.bfloat16)
    out = torch.zeros(N, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensors only"):
        st.decode(ssm, mixed, a, b, torch.zeros(4), torch.zeros(4), torch.tensor([1, 2]), out)


def test_factories_check_static_shapes(lib):
    from leapquant_amd import kernels as KN
    with pytest.raises(AssertionError):
        KN.make_gdn_step(4, 32, 16, 128, 64, 16, 32 * 128 * 128)     # (K, V) = (128, 64): no such variant
    with pytest.raises(AssertionError):
        KN.make_kda_step(4, 32, 32, 64, 128, 16, 32 * 128 * 128)     # KDA: 128 x 128 only
    with pytest.raises(AssertionError):
        KN.make_flush(4, 32, 64, 64, 16, 32 * 128 * 128, KDA=True)
    KN.make_gdn_step(4, 32, 16, 64, 128, 16, 32 * 64 * 128)          # the GDN head-dim variants (kernels.py:62)
    KN.make_flush(4, 32, 64, 64, 16, 32 * 64 * 64)
    with pytest.raises(AssertionError):
        KN.make_gdn_step(4, 32, 16, 128, 128, 65, 32 * 128 * 128)
    with pytest.raises(AssertionError):
        KN.make_gdn_step(4, 24, 3, 128, 128, 16, 24 * 128 * 128)     # GQA 8
    with pytest.raises(AssertionError):
        KN.make_flush(4, 32, 128, 128, 16, 32 * 128 * 128, R=5)
    # schedule knobs of the reference are accepted
    KN.make_gdn_step(4, 32, 16, 128, 128, 16, 32 * 128 * 128, SMS=132, NSTAGE=6, NCG=3, NNW=2, MAXIT=128)
    KN.make_flush(4, 32, 128, 128, 16, 32 * 128 * 128, SMS=132, NCG=3, MAXIT=128, PAD=8, MMT="bf16")
    assert (KN.QMAX, KN.EPS, KN.SOFTPLUS_THRESHOLD) == (127.0, 1e-12, 20.0)


def test_flush_schedule_counter(lib):
    """lq_state.sched: an int32 [LQ_SCHED_INTS] buffer of counters, zero between calls, that the state allocates and
    passes to its flush; the struct carries it after qmax (the header's layout), and a buffer of another type or size
    is refused on the host."""
    from leapquant_amd import _lib, kernels as KN
    from leapquant_amd.state import LeapQuantState
    fields = [f[0] for f in _lib.LqState._fields_]
    assert fields[-3:] == ["ctl", "qmax", "sched"]
    assert re.search(r"float qmax;.*?int\* sched;.*?\} lq_state;", open(HEADER).read(), re.S)
    ssm = torch.zeros(3, 2, 128, 128)
    z = torch.zeros(1)
    with pytest.raises(ValueError, match="sched"):
        KN.state_struct(ssm, ssm.stride(0), z, z, z, z, None, z, 3, 2, 1, 128, 128, 16, 4, sched=torch.zeros(512))
    with pytest.raises(ValueError, match="sched"):
        KN.state_struct(ssm, ssm.stride(0), z, z, z, z, None, z, 3, 2, 1, 128, 128, 16, 4,
                        sched=torch.zeros(1, dtype=torch.int32))
    lq = LeapQuantState(ssm, 1, L=16)
    assert lq.sched.dtype == torch.int32 and lq.sched.shape == (_lib.SCHED_INTS,) and int(lq.sched.abs().sum()) == 0
    assert int(re.search(r"#define\s+LQ_SCHED_INTS\s+(\d+)", open(HEADER).read()).group(1)) == _lib.SCHED_INTS


def test_get_state_registry(lib):
    """One LeapQuantState per cache tensor identity; a re-allocated cache drops the old buffers (state.py:172-189)."""
    from leapquant_amd import state as S

    class Layer:
        pass

    ssm = torch.zeros(2, 4, 128, 128)
    l1, l2 = Layer(), Layer()
    a = S.get_state(l1, ssm, H=2, L=16)
    assert S.get_state(l1, ssm, H=2, L=16) is a
    assert S.get_state(l2, ssm, H=2, L=16) is a               # two layers on one cache view share it
    ssm2 = torch.zeros(2, 4, 128, 128)
    b = S.get_state(l1, ssm2, H=2, L=16)
    assert b is not a and b.key == S._ident(ssm2)

    class PrefixLayer:
        class cache_config:
            mamba_cache_mode = "all"

    with pytest.raises(RuntimeError, match="prefix caching"):
        S.get_state(PrefixLayer(), torch.zeros(2, 4, 128, 128), H=2, L=16)


@pytest.mark.parametrize("kda", [False, True])
def test_decode_checks_the_gate(lib, kda):
    """The raw gate is read as bf16 [N, HV] (GDN) or [N, HV, K] (KDA) (kernels.py:86, 738): another dtype or element
    count is refused before any pointer is taken."""
    from leapquant_amd.state import LeapQuantState
    ssm = torch.zeros(3, 4, 128, 128)
    st = LeapQuantState(ssm, 4 if kda else 2, kda=kda, L=16)
    N, KA = 2, 128 if kda else 1
    H = st.H
    mixed = torch.zeros(N, 2 * H * 128 + 4 * 128, dtype=torch.bfloat16)
    b = torch.zeros(N, 4, dtype=torch.bfloat16)
    out = torch.zeros(N, 4, 128, dtype=torch.bfloat16)
    dt = torch.zeros(4 * KA)
    for a in (torch.zeros(N, 4 * KA), torch.zeros(N, 4 * KA + 1, dtype=torch.bfloat16),
              torch.zeros(N + 1, 4 * KA, dtype=torch.bfloat16)):
        with pytest.raises(ValueError, match="a: bf16"):
            st.decode(ssm, mixed, a, b, torch.zeros(4), dt, torch.tensor([1, 2]), out)
    if not kda:
        x = torch.zeros(N, 2 * H * 128 + 4 * 128, dtype=torch.bfloat16)
        cs = torch.zeros(3, x.shape[1], 3, dtype=torch.bfloat16)
        w = torch.zeros(x.shape[1], 4, dtype=torch.bfloat16)
        with pytest.raises(ValueError, match="a: bf16"):
            st.decode_conv(ssm, x, cs, w, None, True, torch.zeros(N, 4), b, torch.zeros(4), dt,
                           torch.tensor([1, 2]), out)


def test_reference_import_name_reaches_the_same_modules(lib):
    """`leapquant.kernels / .state / .vllm` (the reference's names, pyproject entry point leapquant.vllm:register) are
    this build's modules, so the per-layer registry is one object whichever name a caller imports."""
    import leapquant
    import leapquant.state as LS
    import leapquant_amd.state as AS
    from leapquant.kernels import QMAX, make_flush, make_gdn_step, make_quantize, lowrank_factor  # noqa: F401
    from leapquant.vllm import register
    import leapquant_amd.vllm as AV
    assert LS is AS and LS._STATES is AS._STATES and register is AV.register
    assert leapquant.__version__ == "0.1.0" and QMAX == 127.0
    toml = open(os.path.join(ROOT, "pyproject.toml")).read()
    assert 'leapquant = "leapquant.vllm:register"' in toml
