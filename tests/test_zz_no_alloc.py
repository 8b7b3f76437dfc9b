"""lq_decode_noalloc (the decode call that allocates nothing: its due list lives in the library's static device memory)
against the existing entry points on identical states: LeapQuantState.decode, i.e. lq_gdn_step / lq_kda_step then
lq_flush with the layer's own due flag.  Two calls in a row, the second with fewer rows; both make heads due, so the
second call's flush runs on a list the first one emptied.  The same kernels run on both sides, so every output and
every byte of the state must be equal."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import lq_oracle as O
from tests import lqgpu as G
from tests.fixtures import gate_params, make_inputs, make_state
from tests.test_gpu_parity import _prestep

pytestmark = pytest.mark.gpu


def _to_full_minus_one(rng, st, slots, kda, L, HV, H, K=128, V=128):
    A_log, dt_bias = gate_params(HV, K, kda)
    for s in slots:
        while st["hcnt"][s, 0] < L - 1:
            mixed, a, b = make_inputs(rng, 1, HV, H, K, V, kda=kda)
            (O.kda_step if kda else O.gdn_step)(st, mixed, a, b, A_log, dt_bias, np.array([s]))


def _prestep_dims(rng, st, Q0, steps, NS, HV, H, K, V):
    A_log, dt_bias = gate_params(HV, K)
    for _ in range(steps):
        sl = rng.permutation(np.arange(1, NS))[: rng.integers(1, NS)]
        mixed, a, b = make_inputs(rng, len(sl), HV, H, K, V)
        O.gdn_step(st, mixed, a, b, A_log, dt_bias, sl)
        O.flush(st, Q0, sl)


def _noalloc(lq, ssm, mixed, a, b, A_log, dt_bias, idx, out):
    from leapquant_amd import _lib, kernels as KN
    N = idx.shape[0]
    io = KN._step_io(mixed, a.reshape(N, lq.HV, lq.K if lq.kda else 1).contiguous(), b, A_log, dt_bias, idx, out,
                     lq.kstep_scale)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return _lib.lib().lq_decode_noalloc(ctypes.byref(lq._struct(ssm)), ctypes.byref(io), KN._p(lq.Q0),
                                        1 if lq.kda else 0, ctypes.c_float(lq.glb), stream)


@pytest.mark.parametrize("kda,K,V", [(False, 128, 128), (True, 128, 128), (False, 64, 64), (False, 64, 128)])
def test_noalloc_decode_equals_step_then_flush(kda, K, V):
    """(64, 64) at GQA 2: the flush takes the two heads of a key head together when it scans, and each listed head
    alone (its partner's entry in another workgroup) from the due list -- the same bytes either way."""
    L, NS, HV = 16, 10, 4
    H = HV if kda else 2
    rng = np.random.default_rng(1500 + kda + K + V)
    st, S, Q0 = make_state(rng, NS, HV, H, K=K, V=V, L=L, kda=kda)
    if K == 128:
        _prestep(rng, st, Q0, kda, steps=L // 2, NS=NS, HV=HV, H=H)
    else:
        _prestep_dims(rng, st, Q0, L // 2, NS, HV, H, K, V)
    _to_full_minus_one(rng, st, (1, 2, 3, 7, 8), kda, L, HV, H, K, V)   # the next step of these slots fills them
    ssm_a, lq_a = G.to_gpu(st, H=H)                                   # existing entry points
    ssm_b, lq_b = G.to_gpu(st, H=H)                                   # lq_decode_noalloc
    A_log, dt_bias = gate_params(HV, K, kda)
    calls = [np.array([1, 2, 0, 4, 5, 3, 6], np.int64),             # fills slots 1, 2, 3; row 2 is padding
             np.array([7, 1, 8], np.int64)]                           # fewer rows; fills 7 and 8
    for k, idx in enumerate(calls):
        mixed, a, b = make_inputs(rng, len(idx), HV, H, K, V, kda=kda)
        mg, ag, bg, Ag, dg, ig = G.inputs_gpu(mixed, a, b, A_log, dt_bias, idx)
        out_a = torch.empty(len(idx), HV, V, dtype=torch.bfloat16, device=G.DEV)
        out_b = torch.full((len(idx), HV, V), 9.0, dtype=torch.bfloat16, device=G.DEV)
        print("no-alloc decode, %s %dx%d, call %d (%d rows)" % ("KDA" if kda else "GDN", K, V, k, len(idx)), flush=True)
        lq_a.decode(ssm_a, mg, ag, bg, Ag, dg, ig, out_a)
        assert _noalloc(lq_b, ssm_b, mg, ag, bg, Ag, dg, ig, out_b) == 0
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b), k
        ga, gb = G.from_gpu(ssm_a, lq_a), G.from_gpu(ssm_b, lq_b)
        for key in ("Sq", "Sk", "Sv", "UQ", "Kbuf", "Ubuf", "Wbuf", "Pbuf", "Gbuf", "hcnt"):
            if ga[key] is not None:
                assert np.array_equal(ga[key], gb[key]), (k, key)
        due = calls[k][calls[k] > 0]
        assert np.all(gb["hcnt"][[1, 2, 3] if k == 0 else [7, 8]] == 0)           # those heads were flushed
        assert not np.array_equal(gb["Sq"][[1, 2, 3] if k == 0 else [7, 8]],
                                  st["Sq"][[1, 2, 3] if k == 0 else [7, 8]])      # with new checkpoints
        assert np.all(gb["hcnt"][due] <= L - 1)
    assert int(lq_b.ctl.abs().sum()) == 0                             # the layer's own flag was never used


def test_noalloc_rejects_more_heads_than_its_list_holds():
    """N * HV above the static due list (65536 pairs) is refused with LQ_ERR_SIZE before anything is launched."""
    from leapquant_amd import _lib
    rng = np.random.default_rng(1600)
    NS, HV, H = 3, 32, 16
    st, S, Q0 = make_state(rng, NS, HV, H, L=16)
    ssm, lq = G.to_gpu(st)
    N = 65536 // HV + 1
    idx = torch.zeros(N, dtype=torch.int32, device=G.DEV)            # padding rows: nothing would be touched anyway
    mixed = torch.zeros(N, 2 * H * 128 + HV * 128, dtype=torch.bfloat16, device=G.DEV)
    a = torch.zeros(N, HV, dtype=torch.bfloat16, device=G.DEV)
    b = torch.zeros(N, HV, dtype=torch.bfloat16, device=G.DEV)
    out = torch.empty(N, HV, 128, dtype=torch.bfloat16, device=G.DEV)
    A_log, dt_bias = torch.zeros(HV, device=G.DEV), torch.zeros(HV, device=G.DEV)
    assert _noalloc(lq, ssm, mixed, a, b, A_log, dt_bias, idx, out) == -3
    with pytest.raises(RuntimeError, match="static due list"):
        _lib.check(-3, "lq_decode_noalloc")
    assert _noalloc(lq, ssm, mixed[:N - 1], a[:N - 1], b[:N - 1], A_log, dt_bias, idx[:N - 1], out[:N - 1]) == 0


def test_noalloc_decode_under_graph_capture():
    """lq_decode_noalloc captured in a graph (after one call with no rows, which sets the device up) and replayed over
    a window end, each replay on new inputs copied into the captured buffers, against LeapQuantState.decode run eagerly
    on the same inputs: outputs and state bytes equal after every replay (eager work and synchronisations between the
    replays)."""
    L, NS, HV, H = 16, 6, 4, 2
    rng = np.random.default_rng(1700)
    st, S, Q0 = make_state(rng, NS, HV, H, L=L)
    _prestep(rng, st, Q0, False, steps=L // 2, NS=NS, HV=HV, H=H)
    _to_full_minus_one(rng, st, (1, 2), False, L, HV, H)              # the first replay fills slots 1, 2
    ssm_a, lq_a = G.to_gpu(st, H=H)
    ssm_b, lq_b = G.to_gpu(st, H=H)
    A_log, dt_bias = gate_params(HV)
    idx = np.array([1, 2, 0, 4, 5, 3], np.int64)
    mixed, a, b = make_inputs(rng, len(idx), HV, H)
    mg, ag, bg, Ag, dg, ig = G.inputs_gpu(mixed, a, b, A_log, dt_bias, idx)
    out_b = torch.empty(len(idx), HV, 128, dtype=torch.bfloat16, device=G.DEV)
    z = ig[:0]
    assert _noalloc(lq_b, ssm_b, mg[:0], ag[:0], bg[:0], Ag, dg, z, out_b[:0]) == 0   # no rows: the device set-up
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = _noalloc(lq_b, ssm_b, mg, ag, bg, Ag, dg, ig, out_b)
    assert rc == 0
    torch.cuda.synchronize()
    for t in range(L + 2):                                            # slots 1, 2 fill on replay 0, the others later
        mixed, a, b = make_inputs(rng, len(idx), HV, H)
        m2, a2, b2, _, _, _ = G.inputs_gpu(mixed, a, b, A_log, dt_bias, idx)
        for dst, src in ((mg, m2), (ag, a2), (bg, b2)):
            dst.copy_(src)
        out_a = torch.empty_like(out_b)
        print("no-alloc decode under capture, replay %d" % t, flush=True)
        lq_a.decode(ssm_a, mg, ag, bg, Ag, dg, ig, out_a)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b), t
        assert torch.equal(ssm_a.view(torch.int32), ssm_b.view(torch.int32)), t
        for key in ("hcnt", "Wbuf", "Pbuf", "Kbuf", "Ubuf"):
            assert torch.equal(getattr(lq_a, key), getattr(lq_b, key)), (t, key)
    assert int(lq_b.hcnt[1:].max()) < L
