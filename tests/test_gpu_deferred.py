"""GPU tests of the deferred-flush GDN decode (lq_gdn_decode_deferred, LeapQuantState(defer_flush=True)) against the
immediate one (lq_gdn_decode), which the oracle already pins: with the same inputs the two give the same outputs bit
for bit on every call, whatever the rows' window fills, and the same checkpoint once the deferred heads are flushed.
Staggered windows (row n starts at fill n % W, so rows reach their flush on different calls, as in serving), rows that
leave the batch while one of their heads is deferred and come back later, a padding row, and the prefill dequant of a
slot that holds a deferred head."""
import numpy as np
import pytest
import torch

from tests import lqgpu as G
from tests.fixtures import gate_params, make_inputs, make_state

pytestmark = pytest.mark.gpu


def _pair(seed, NS, HV, H, L):
    rng = np.random.default_rng(seed)
    st, S, Q0 = make_state(rng, NS, HV, H, L=L)
    ssm_i, lq_i = G.to_gpu(st, H=H)
    ssm_d = ssm_i.clone()
    lq_d = G.LeapQuantState(ssm_d, H, L=L, R=lq_i.R, defer_flush=True)
    G.load_state(lq_d, ssm_d, st)
    return rng, (ssm_i, lq_i), (ssm_d, lq_d)


def _bytes_equal(a, b):
    return torch.equal(a.view(torch.int32), b.view(torch.int32))


def _decode_both(rng, pair_i, pair_d, idx, HV, H):
    A_log, dt_bias = gate_params(HV, 128, False)
    mixed, a, b = make_inputs(rng, len(idx), HV, H)
    outs = []
    for ssm, lq in (pair_i, pair_d):
        mg, ag, bg, Ag, dg, ig = G.inputs_gpu(mixed, a, b, A_log, dt_bias, idx)
        out = torch.empty(len(idx), HV, 128, dtype=torch.bfloat16, device=G.DEV)
        lq.decode(ssm, mg, ag, bg, Ag, dg, ig, out)
        outs.append(out)
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("L", [16, 64])
def test_deferred_decode_matches_immediate(L):
    NS, HV, H, B = 9, 4, 2, 8
    rng, pi, pd = _pair(3100 + L, NS, HV, H, L)
    # staggered fills: slot s starts at fill (s * 5) % L, in both states (empty windows with a count set: the window
    # weights of unused rows are zero, so the step treats them as steps taken with zero contribution)
    for ssm, lq in (pi, pd):
        fill = torch.tensor([(s * 5) % L for s in range(NS)], dtype=torch.int32, device=G.DEV)
        lq.hcnt.copy_(fill[:, None].expand(NS, HV))
    torch.cuda.synchronize()
    deferred_seen = 0
    for t in range(3 * L):
        idx = np.arange(1, B + 1)
        if t % 7 == 3:
            idx = idx[idx != 5]                          # slot 5 sits out a call (a deferred head may wait)
        if t % 11 == 0:
            idx = np.concatenate([idx, [0]])             # a padding row
        rng_t = np.random.default_rng(t)
        oi, od = _decode_both(rng_t, pi, pd, idx, HV, H)
        assert torch.equal(oi, od), "call %d: outputs differ" % t
        deferred_seen += int((pd[1].hcnt == L).sum())
    assert deferred_seen > 0                             # heads were actually left for the next call
    for ssm, lq in (pi, pd):
        lq.flush(ssm, torch.arange(0, NS, dtype=torch.int32, device=G.DEV))
    torch.cuda.synchronize()
    assert _bytes_equal(pi[0], pd[0])
    for k in ("hcnt", "Wbuf", "Pbuf", "Kbuf", "Ubuf"):
        assert torch.equal(getattr(pi[1], k), getattr(pd[1], k)), k


def test_deferred_head_settled_by_dequantize():
    """A slot left with a deferred head: its prefill dequant flushes it first, so the fp32 state is the one the
    immediate decode's state dequantises to."""
    NS, HV, H, L = 4, 4, 2, 16
    rng, pi, pd = _pair(3200, NS, HV, H, L)
    idx = np.arange(1, NS)
    for t in range(L):                                   # the last call fills every window
        oi, od = _decode_both(np.random.default_rng(100 + t), pi, pd, idx, HV, H)
        assert torch.equal(oi, od)
    assert int((pd[1].hcnt == L).sum()) == (NS - 1) * HV // 2     # one head of each key head left full
    assert int((pi[1].hcnt == L).sum()) == 0
    sl = torch.tensor([1, 3], dtype=torch.int32, device=G.DEV)
    for ssm, lq in (pi, pd):
        lq.dequantize(ssm, sl)
    torch.cuda.synchronize()
    for s in (1, 3):
        assert _bytes_equal(pi[0][s], pd[0][s]), s


@pytest.mark.parametrize("settle", ["dequantize", "flush"])
def test_deferred_heads_settled_across_partial_calls(settle):
    """Deferred heads in three slots, settled by two calls over different slots: the first call ([1, 3]) must not
    leave slot 2's deferred head unflushed for the second ([2]).  Each slot's bytes equal the immediate decode's."""
    NS, HV, H, L = 4, 4, 2, 16
    rng, pi, pd = _pair(3300, NS, HV, H, L)
    idx = np.arange(1, NS)
    for t in range(L):                                   # the last call fills every window
        oi, od = _decode_both(np.random.default_rng(200 + t), pi, pd, idx, HV, H)
        assert torch.equal(oi, od)
    assert int((pd[1].hcnt[2] == L).sum()) == HV // 2    # slot 2 holds deferred heads
    for sl in ([1, 3], [2]):
        t = torch.tensor(sl, dtype=torch.int32, device=G.DEV)
        for ssm, lq in (pi, pd):
            getattr(lq, settle)(ssm, t)
    torch.cuda.synchronize()
    assert int((pd[1].hcnt == L).sum()) == 0
    for s in (1, 2, 3):
        assert _bytes_equal(pi[0][s], pd[0][s]), s
    for k in ("hcnt", "Wbuf", "Pbuf"):
        assert torch.equal(getattr(pi[1], k), getattr(pd[1], k)), k
