"""The persistent flush's dynamic head schedule (lq_state.sched) against its static schedule, on the GPU.

With the counter, workgroups take their next candidate head from it instead of a fixed share (leapquant_amd/csrc/
lq_flush.hip, flush_scan); which workgroup flushes a head must not change what is written.  Every flush layout runs
with more candidates than the grid holds (so workgroups take several heads), some heads not due and padding rows:
the state, codes, scales, factors and window buffers after the scheduled flush must equal those after the static one
byte for byte, and the counter must be back at zero (twice in a row, so that the reset is tested).
"""
import numpy as np
import pytest
import torch

from leapquant_amd import kernels as KN
from leapquant_amd.state import LeapQuantState

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

CASES = [  # (kda, K, V, R, HV, H, NS): the four-wave flush, R = 8, KDA, the 64-dim layouts (pairs at even GQA)
    (False, 128, 128, 4, 32, 16, 65),
    # GQA 2 and 4 with a candidate count that is not a multiple of 8 G (1218 = 76 x 16 + 2, 1572 = 49 x 32 + 4): the
    # schedule's key-head grouping of candidates and its partial last block
    (False, 128, 128, 4, 6, 3, 201),
    (False, 128, 128, 4, 12, 3, 129),
    (False, 128, 128, 8, 16, 8, 65),
    (True, 128, 128, 4, 16, 16, 65),
    (False, 64, 128, 4, 32, 16, 65),
    (False, 64, 64, 4, 32, 16, 129),
    (False, 64, 64, 4, 3, 3, 513),
]


def _buffers(lq, ssm):
    out = [ssm.clone(), lq.Kbuf.clone(), lq.Ubuf.clone(), lq.Wbuf.clone(), lq.Pbuf.clone(), lq.hcnt.clone()]
    if lq.kda:
        out.append(lq.Gbuf.clone())
    return out


def _restore(lq, ssm, snap):
    for dst, src in zip([ssm, lq.Kbuf, lq.Ubuf, lq.Wbuf, lq.Pbuf, lq.hcnt] + ([lq.Gbuf] if lq.kda else []), snap):
        dst.copy_(src)


@pytest.mark.parametrize("kda,K,V,R,HV,H,NS", CASES)
def test_scheduled_flush_equals_static(kda, K, V, R, HV, H, NS):
    print("sched flush: kda=%d K=%d V=%d R=%d HV=%d H=%d NS=%d" % (kda, K, V, R, HV, H, NS), flush=True)
    L = 16
    g = torch.Generator(device=DEV)
    g.manual_seed(7 + K + V + R + HV)
    ssm = (0.02 * torch.randn(NS, HV, V, K, device=DEV, generator=g)).contiguous()
    lq = LeapQuantState(ssm, H, L=L, R=R, kda=kda)
    slots = torch.arange(1, NS, device=DEV, dtype=torch.int32)
    lq.quantize(ssm, slots)
    # windows: random contents, full (due) on about 70 % of the heads, partly filled on the rest
    lq.Kbuf.copy_(torch.nn.functional.normalize(torch.randn(lq.Kbuf.shape, device=DEV, generator=g), dim=-1))
    lq.Ubuf.normal_(0.0, 0.02, generator=g)
    lq.Wbuf.uniform_(0.5, 1.0, generator=g)
    if kda:
        lq.Pbuf.uniform_(-0.5, 0.0, generator=g)
        lq.Gbuf.copy_(torch.empty(lq.Gbuf.shape, device=DEV).uniform_(0.9, 1.0, generator=g).half())
    else:
        lq.Pbuf.uniform_(0.3, 1.0, generator=g)
    due = torch.rand(NS, HV, device=DEV, generator=g) < 0.7
    part = torch.randint(0, L, (NS, HV), device=DEV, generator=g, dtype=torch.int32)
    lq.hcnt.copy_(torch.where(due, torch.full_like(part, L), part))
    # the rows of the call: every slot once, in a shuffled order, with padding rows in between
    order = torch.randperm(NS - 1, device=DEV, generator=g).to(torch.int32) + 1
    idx = torch.cat([order[: (NS - 1) // 2], torch.zeros(3, device=DEV, dtype=torch.int32),
                     order[(NS - 1) // 2:]]).contiguous()
    snap = _buffers(lq, ssm)

    static = KN.make_flush(NS, HV, K, V, L, lq.SS, R=R, ITERS=1, KDA=kda, qmax=lq.qmax)
    vw = lq.views(ssm)
    args = lambda: (vw["q32"], vw["Sk"], vw["Sv"], vw["skv"], lq.Kbuf, lq.Ubuf, lq.Wbuf, lq.Pbuf, lq.Gd if not kda
                    else lq.Gbuf, lq.hcnt, vw["sq16"], vw["uq"], lq.Q0, idx)
    static(*args())
    torch.cuda.synchronize()
    want = _buffers(lq, ssm)
    assert int((want[5][1:] == L).sum()) == 0            # every due head was flushed
    for rep in range(2):
        _restore(lq, ssm, snap)
        torch.cuda.synchronize()
        lq.kflush(*args())                               # the state's flush: with its schedule counter
        torch.cuda.synchronize()
        got = _buffers(lq, ssm)
        for i, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a.view(torch.uint8) if a.dtype != torch.uint8 else a,
                               b.view(torch.uint8) if b.dtype != torch.uint8 else b), (rep, i)
        assert int(lq.sched.abs().sum()) == 0, rep
