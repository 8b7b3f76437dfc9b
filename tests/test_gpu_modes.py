"""GPU parity of the decode path's other modes and edge cases, against the CPU oracle, through the C ABI:

* 6-bit checkpoints (codes in [-31, 31], the same int8 container): decode calls across a window boundary, GDN and KDA;
* BASELINE config 0 (GDN, B = 1, HV = H = 16, d = 128, W = 64, R = 4): 256 decode calls with 4 flushes;
* a head left at a full window by a flush of other rows is flushed by the next decode of its row (due flag re-raised);
* a rank-deficient state (CholeskyQR2's relative pivot floor, kernels.py:1816-1825) through the flush and the quantize;
* the bytes of each fp32 slot past the checkpoint are never written by decode or flush (poisoned beforehand);
* the fused conv step treats a row whose slot is outside the conv state as a padding row.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import lq_oracle as O
from tests import lqgpu as G
from tests.fixtures import gate_params, make_inputs, make_state
from tests.test_gpu_full_size import _assert_checkpoints
from tests.test_gpu_parity import _assert_step_state, _prestep

pytestmark = pytest.mark.gpu

RT, AT = 2e-2, 1e-3


def _resync(st, g):
    """Continue the oracle from the GPU's state.  Each call is then compared from identical inputs: a free-running
    pair drifts apart through 1-ulp differences of the bf16 window appends (u = beta (v - pred) rounds the other way
    now and then), which after tens of steps moves the flush's codes past the per-flush bar; that drift is covered by
    the golden trajectories' own bar."""
    for k in ("Sq", "Sk", "Sv", "UQ", "Kbuf", "Ubuf", "Wbuf", "Pbuf", "Gbuf", "hcnt"):
        if g.get(k) is not None:
            st[k] = g[k].copy()


def _decode(lq, ssm, mixed, a, b, A_log, dt_bias, idx):
    mg, ag, bg, Ag, dg, ig = G.inputs_gpu(mixed, a, b, A_log, dt_bias, idx)
    out = torch.empty(len(idx), lq.HV, lq.V, dtype=torch.bfloat16, device=G.DEV)
    lq.decode(ssm, mg, ag, bg, Ag, dg, ig, out)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("kda", [False, True])
def test_6bit_decode_across_a_window_boundary(kda):
    """A 6-bit state decoded through LeapQuantState.decode (step + flush) for a window and a half: outputs at the step
    bar on every call, and the checkpoints written by the flush at the per-flush bar (codes within 1 LSB on <= 0.1 %)."""
    qmax, L = 31.0, 16
    rng = np.random.default_rng(1100 + kda)
    NS, HV = 5, 4
    H = HV if kda else 2
    st, S, Q0 = make_state(rng, NS, HV, H, L=L, kda=kda, qmax=qmax)
    _prestep(rng, st, Q0, kda, steps=L // 2 + 1, NS=NS, HV=HV, H=H, qmax=qmax)
    ssm, lq = G.to_gpu(st, H=H, qmax=qmax)
    idx = np.array([2, 0, 4, 1], np.int64)
    A_log, dt_bias = gate_params(HV, 128, kda)
    step = O.kda_step if kda else O.gdn_step
    flushed = 0
    for t in range(L + L // 2):
        mixed, a, b = make_inputs(rng, len(idx), HV, H, kda=kda)
        print("6-bit %s decode call %d" % ("KDA" if kda else "GDN", t), flush=True)
        o_ref = step(st, mixed, a, b, A_log, dt_bias, idx, qmax=qmax)
        due = O.due_pairs(st, idx)
        O.flush(st, Q0, idx, qmax=qmax)
        o_gpu = _decode(lq, ssm, mixed, a, b, A_log, dt_bias, idx)
        np.testing.assert_allclose(o_gpu, o_ref, rtol=RT, atol=AT, err_msg="call %d" % t)
        assert (G.bf16_ulps(o_gpu, o_ref) <= 2).mean() > 0.99
        g = G.from_gpu(ssm, lq)
        if due:                                          # this call's flush re-checkpointed some heads
            slots = sorted({s for s, _ in due})
            assert np.abs(g["Sq"].astype(np.int32)).max() <= 31
            _assert_checkpoints(g, st, np.array(slots), qmax=qmax)
            flushed += len(due)
        _resync(st, g)
    assert flushed >= 3 * HV
    assert np.array_equal(G.from_gpu(ssm, lq)["hcnt"], st["hcnt"])


def test_config0_trajectory():
    """GDN B = 1, HV = H = 16, d = 128, W = 64, R = 4, N(0, 0.02^2) state quantised to INT8, 256
    decode calls (4 flushes) with the config's input distributions (q, k ~ N(0,1) l2-normalised, v ~ N(0,1), log-gate
    U(-0.1, 0), beta = sigmoid(N(0,1))).  Outputs at the step bar on every call; each flush's checkpoints at the
    per-flush bar, after which both sides continue from the GPU's checkpoint."""
    rng = np.random.default_rng(1000)
    NS, HV, H, L = 2, 16, 16, 64
    st, S, Q0 = make_state(rng, NS, HV, H, L=L)
    ssm, lq = G.to_gpu(st)
    idx = np.array([1], np.int64)
    A_log, dt_bias = gate_params(HV)
    flushes = 0
    for t in range(256):
        mixed, a, b = make_inputs(rng, 1, HV, H)
        o_ref = O.gdn_step(st, mixed, a, b, A_log, dt_bias, idx)
        due = O.due_pairs(st, idx)
        O.flush(st, Q0, idx)
        o_gpu = _decode(lq, ssm, mixed, a, b, A_log, dt_bias, idx)
        np.testing.assert_allclose(o_gpu, o_ref, rtol=RT, atol=AT, err_msg="call %d" % t)
        assert (G.bf16_ulps(o_gpu, o_ref) <= 2).mean() > 0.99
        g = G.from_gpu(ssm, lq)
        if due:
            print("config 0: flush at call %d" % t, flush=True)
            assert len(due) == HV and np.all(g["hcnt"] == 0)
            _assert_checkpoints(g, st, np.array([1]))
            flushes += 1
        else:
            _assert_step_state(g, st, idx)
        _resync(st, g)
    assert flushes == 4


def test_full_head_left_by_a_flush_of_other_rows_is_recovered():
    """A step fills the window of slot 1 and raises the due flag; a flush of slot 2 alone clears the flag without
    touching slot 1.  The next decode of slot 1 meets a full window: it outputs zeros, writes nothing, raises the flag
    again, and its flush re-checkpoints slot 1 (as the oracle's flush does); the call after that is a normal step."""
    rng = np.random.default_rng(1200)
    NS, HV, H, L = 3, 4, 2, 16
    st, S, Q0 = make_state(rng, NS, HV, H, L=L)
    A_log, dt_bias = gate_params(HV)
    for _ in range(L - 1):                               # slot 1 one entry short of full
        mixed, a, b = make_inputs(rng, 1, HV, H)
        O.gdn_step(st, mixed, a, b, A_log, dt_bias, np.array([1]))
    ssm, lq = G.to_gpu(st)
    two = torch.tensor([2], dtype=torch.int32, device=G.DEV)
    # the step alone through the layer's own lq_state (due flag included), as decode() launches it
    mixed, a, b = make_inputs(rng, 1, HV, H)
    O.gdn_step(st, mixed, a, b, A_log, dt_bias, np.array([1]))
    mg, ag, bg, Ag, dg, ig = G.inputs_gpu(mixed, a, b, A_log, dt_bias, np.array([1]))
    out = torch.empty(1, HV, 128, dtype=torch.bfloat16, device=G.DEV)
    from leapquant_amd import _lib, kernels as KN
    io = KN._step_io(mg, ag.reshape(1, HV, 1), bg, Ag, dg, ig, out, lq.kstep_scale)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.lib().lq_gdn_step(ctypes.byref(lq._struct(ssm)), ctypes.byref(io), stream), "lq_gdn_step")
    # another row's flush as decode() launches it (through the flagged lq_state): it clears the flag, slot 1 stays full
    _lib.check(_lib.lib().lq_flush(ctypes.byref(lq._struct(ssm)), KN._p(lq.Q0), KN._p(two), 1, 0,
                                   ctypes.c_float(lq.qmax), stream), "lq_flush")
    torch.cuda.synchronize()
    assert int(lq.ctl[0]) == 0 and np.all(lq.hcnt[1].cpu().numpy() == L)
    before = G.from_gpu(ssm, lq)
    # decode of slot 1: zero output, nothing written by the step, then the flush takes slot 1
    mixed, a, b = make_inputs(rng, 1, HV, H)
    o_gpu = _decode(lq, ssm, mixed, a, b, A_log, dt_bias, np.array([1]))
    assert np.all(o_gpu == 0)
    O.flush(st, Q0, np.array([1]))
    g = G.from_gpu(ssm, lq)
    assert np.all(g["hcnt"][1] == 0) and np.all(g["Wbuf"][1] == 0) and np.all(g["Pbuf"][1] == 1)
    assert np.array_equal(g["Kbuf"][1], before["Kbuf"][1]) and np.array_equal(g["Ubuf"][1], before["Ubuf"][1])
    _assert_checkpoints(g, st, np.array([1]))
    for k in ("Sq", "Sk", "Sv", "UQ"):
        st[k] = g[k].copy()
    mixed, a, b = make_inputs(rng, 1, HV, H)
    o_ref = O.gdn_step(st, mixed, a, b, A_log, dt_bias, np.array([1]))
    o_gpu = _decode(lq, ssm, mixed, a, b, A_log, dt_bias, np.array([1]))
    np.testing.assert_allclose(o_gpu, o_ref, rtol=RT, atol=AT)
    assert np.abs(o_gpu).max() > 0


def test_rank_deficient_state_takes_the_pivot_floor():
    """A rank-2 state (its window's keys take two directions, empty checkpoint) through the flush, and the same fp32
    state through the standalone quantize: factors 3 and 4 come from CholeskyQR2's floored pivots (flush) or MGS's norm
    floor (quantize), whose directions are rounding noise on either side, so the codes are not compared.  Both sides
    must stay finite, agree on the two live factors, and keep the logical state within the quantisation bound."""
    from tests.test_gpu_parity import _run_flush
    from tests.test_oracle_pins import _rank2_state
    st, Q0, S = _rank2_state()
    ssm, lq = G.to_gpu(st, H=1)
    dbg = O.flush(st, Q0, np.array([1]), return_debug=True)
    _run_flush(lq, ssm, torch.tensor([1], dtype=torch.int32, device=G.DEV))   # the factory's flush: scans hcnt
    g = G.from_gpu(ssm, lq)
    for k in ("Sq", "Sk", "Sv", "UQ"):
        assert np.all(np.isfinite(g[k][1].astype(np.float64))), k
    qg = g["UQ"][1, 0, :, 128:].astype(np.float64).T                 # Q16 [V, R]
    assert np.abs(qg[:, :2] - dbg["Q16"][0][:, :2]).max() < 2e-3
    for c in (g, st):
        after = O.materialize(c)[1, 0]
        sk, sv = c["Sk"][1, 0].astype(np.float64), c["Sv"][1, 0].astype(np.float64)
        bound = 0.5 * sk[None, :] * sv[:, None] / 127.0 + 2 ** -9 * np.abs(S).max()
        assert np.all(np.abs(after - S) <= bound)
    assert np.all(g["hcnt"][1] == 0)
    # the standalone quantize of the same fp32 state
    ssm[1, 0].copy_(torch.from_numpy(S.astype(np.float32)))
    lq.quantize(ssm, torch.tensor([1], dtype=torch.int32, device=G.DEV))
    g = G.from_gpu(ssm, lq)
    for k in ("Sq", "Sk", "Sv", "UQ"):
        assert np.all(np.isfinite(g[k][1].astype(np.float64))), k
    after = O.materialize(g)[1, 0]
    sk, sv = g["Sk"][1, 0].astype(np.float64), g["Sv"][1, 0].astype(np.float64)
    assert np.all(np.abs(after - S) <= 0.5 * sk[None, :] * sv[:, None] / 127.0 + 2 ** -9 * np.abs(S).max())


@pytest.mark.parametrize("kda", [False, True])
def test_decode_never_writes_past_the_checkpoint(kda):
    """Every fp32 slot's bytes past the checkpoint (and every byte of slot 0 and of a slot not in the batch) hold a
    poison pattern; a window and a half of decode calls (steps and flushes) must leave all of them as they were."""
    rng = np.random.default_rng(1300 + kda)
    NS, HV, L = 5, 4, 16
    H = HV if kda else 2
    st, S, Q0 = make_state(rng, NS, HV, H, L=L, kda=kda)
    ssm, lq = G.to_gpu(st, H=H)
    end = 128 * 128 + 4 * 256 + 2 * 4 * 256                           # checkpoint bytes of a 128 x 128 head
    raw = ssm.view(torch.int32).view(NS, HV, -1)                      # one (slot, head) block as 4096 words
    poison = torch.tensor(0x7fbadbad, dtype=torch.int32, device=G.DEV)
    raw[:, :, end // 4:] = poison
    raw[0] = poison
    raw[3] = poison                                                   # slot 3 is never in the batch
    snap = ssm.clone()
    idx = np.array([1, 0, 2, 4], np.int64)
    A_log, dt_bias = gate_params(HV, 128, kda)
    for t in range(L + L // 2):
        mixed, a, b = make_inputs(rng, len(idx), HV, H, kda=kda)
        _decode(lq, ssm, mixed, a, b, A_log, dt_bias, idx)
    assert int(lq.hcnt[1:].min()) >= 0
    now = ssm.view(torch.int32).view(NS, HV, -1)
    was = snap.view(torch.int32).view(NS, HV, -1)
    assert torch.equal(now[:, :, end // 4:], was[:, :, end // 4:])
    assert torch.equal(now[0], was[0]) and torch.equal(now[3], was[3])
    assert not torch.equal(now[1, :, :end // 4], was[1, :, :end // 4])   # the flushes did rewrite the checkpoints


def test_fused_conv_treats_slots_outside_the_conv_state_as_padding():
    """lq_conv.NS bounds the conv-state slot: with a conv state of 3 slots and a layer state of 5, a row on slot 4 is a
    padding row (zero output, no state written anywhere) while the rows on slots 1 and 2 step normally."""
    from leapquant_amd import _lib, kernels as KN
    rng = np.random.default_rng(1400)
    NS, HV, H, L = 5, 4, 2, 16
    st, S, Q0 = make_state(rng, NS, HV, H, L=L)
    ssm, lq = G.to_gpu(st)
    C = 2 * H * 128 + HV * 128
    conv = (0.5 * torch.randn(3, C, 3, device=G.DEV)).to(torch.bfloat16)
    w = (0.5 * torch.randn(C, 4, device=G.DEV)).to(torch.bfloat16).contiguous()
    conv0 = conv.clone()
    idx = np.array([1, 4, 2], np.int64)
    x, a, b = make_inputs(rng, len(idx), HV, H)
    A_log, dt_bias = gate_params(HV)
    xg, ag, bg, Ag, dg, ig = G.inputs_gpu(x, a, b, A_log, dt_bias, idx)
    out = torch.full((len(idx), HV, 128), 3.0, dtype=torch.bfloat16, device=G.DEV)
    before = G.from_gpu(ssm, lq)
    cv = KN.conv_struct(conv, w, None, True)
    assert cv.NS == 3
    io = KN._step_io(xg, ag.reshape(len(idx), HV, 1), bg, Ag, dg, ig, out, lq.kstep_scale)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.lib().lq_gdn_step_conv(ctypes.byref(lq._struct(ssm)), ctypes.byref(io), ctypes.byref(cv), stream),
               "lq_gdn_step_conv")
    torch.cuda.synchronize()
    g = G.from_gpu(ssm, lq)
    assert torch.all(out[1] == 0) and torch.all(out[0] != 3.0)
    for k in ("Kbuf", "Ubuf", "Wbuf", "Pbuf", "hcnt"):
        assert np.array_equal(g[k][4], before[k][4]), k
    assert np.all(g["hcnt"][[1, 2]] == before["hcnt"][[1, 2]] + 1)
    assert not torch.equal(conv[1], conv0[1]) and not torch.equal(conv[2], conv0[2])
    assert torch.equal(conv[0], conv0[0])
