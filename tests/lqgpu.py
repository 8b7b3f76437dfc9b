"""Moves oracle states (numpy dicts, oracle/lq_oracle.py layout) into a LeapQuantState on the GPU and back."""
import numpy as np
import torch

from leapquant_amd.state import LeapQuantState, state_views

DEV = "cuda:0"


class RawGdnState:
    """The GDN buffers LeapQuantState allocates (state.py:61-70), loaded from an oracle state, without its kernel set:
    the rank ablation R = 12, 16 has a step, quantize and dequant but no flush (kernels.py:63, 1091), so a
    LeapQuantState -- which builds all four, as the reference's does -- refuses it.  Quacks like one for load_state /
    from_gpu."""
    kda = False

    def __init__(self, st):
        NS, HV, V, K = st["Sq"].shape
        self.NS, self.HV, self.K, self.V = NS, HV, K, V
        self.H, self.L, self.R = st["Kbuf"].shape[1], st["Wbuf"].shape[-1], st["UQ"].shape[2]
        self.ssm = torch.zeros(NS, HV, V, K, device=DEV)
        self.SS = self.ssm.stride(0)
        self.Kbuf = torch.zeros(NS, self.H, self.L, K, dtype=torch.bfloat16, device=DEV)
        self.Ubuf = torch.zeros(NS, HV, self.L, V, dtype=torch.bfloat16, device=DEV)
        self.Wbuf = torch.zeros(NS, HV, self.L, device=DEV)
        self.Pbuf = torch.ones(NS, HV, 1, device=DEV)
        self.hcnt = torch.zeros(NS, HV, dtype=torch.int32, device=DEV)
        self.Gbuf = None
        load_state(self, self.ssm, st)

    def views(self, ssm):
        return state_views(ssm, self.R)


def to_gpu(st, H=None, qmax=127.0, glb=0.0):
    NS, HV, V, K = st["Sq"].shape
    H = st["Kbuf"].shape[1] if H is None else H
    L = st["Wbuf"].shape[-1]
    R = st["UQ"].shape[2]
    ssm = torch.zeros(NS, HV, V, K, device=DEV)
    lq = LeapQuantState(ssm, H, kda=bool(st["kda"]), gate_lower_bound=glb, L=L, R=R, qmax=qmax)
    load_state(lq, ssm, st)
    return ssm, lq


def load_state(lq, ssm, st):
    """Copy an oracle state into the checkpoint views of ssm and the window buffers of an existing LeapQuantState."""
    v = lq.views(ssm)
    v["Sq"].copy_(torch.from_numpy(st["Sq"]))
    v["Sk"].copy_(torch.from_numpy(st["Sk"]))
    v["Sv"].copy_(torch.from_numpy(st["Sv"]))
    v["uq"].copy_(torch.from_numpy(st["UQ"]))
    lq.Kbuf.copy_(torch.from_numpy(st["Kbuf"]).to(torch.bfloat16))
    lq.Ubuf.copy_(torch.from_numpy(st["Ubuf"]).to(torch.bfloat16))
    lq.Wbuf.copy_(torch.from_numpy(st["Wbuf"]))
    lq.Pbuf.copy_(torch.from_numpy(st["Pbuf"]))
    if lq.kda:
        lq.Gbuf.copy_(torch.from_numpy(st["Gbuf"]))
    lq.hcnt.copy_(torch.from_numpy(st["hcnt"]))
    torch.cuda.synchronize()


def from_gpu(ssm, lq):
    torch.cuda.synchronize()
    v = lq.views(ssm)
    out = dict(Sq=v["Sq"].cpu().numpy().copy(), Sk=v["Sk"].cpu().numpy().copy(), Sv=v["Sv"].cpu().numpy().copy(),
               UQ=v["uq"].cpu().numpy().copy(), Kbuf=lq.Kbuf.float().cpu().numpy(), Ubuf=lq.Ubuf.float().cpu().numpy(),
               Wbuf=lq.Wbuf.cpu().numpy().copy(), Pbuf=lq.Pbuf.cpu().numpy().copy(),
               Gbuf=(lq.Gbuf.cpu().numpy().copy() if lq.kda else None), hcnt=lq.hcnt.cpu().numpy().copy(),
               kda=lq.kda)
    return out


def inputs_gpu(mixed, a, b, A_log, dt_bias, idx):
    bf = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).to(DEV)
    return (bf(mixed), bf(a), bf(b), torch.from_numpy(np.asarray(A_log, np.float32)).to(DEV),
            torch.from_numpy(np.asarray(dt_bias, np.float32).reshape(-1)).to(DEV),
            torch.from_numpy(np.asarray(idx, np.int32)).to(DEV))


def code_mismatch(a, b):
    """(fraction of differing codes, max |difference|)."""
    d = np.abs(a.astype(np.int32) - b.astype(np.int32))
    return float((d > 0).mean()), int(d.max()) if d.size else 0


def bf16_ulps(a, b):
    """Distance in bf16 units in the last place between two arrays of bf16 values (as float32)."""
    ia = (np.ascontiguousarray(a, np.float32).view(np.int32) >> 16).astype(np.int64)
    ib = (np.ascontiguousarray(b, np.float32).view(np.int32) >> 16).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7fff), ia)
    ib = np.where(ib < 0, -(ib & 0x7fff), ib)
    return np.abs(ia - ib)
