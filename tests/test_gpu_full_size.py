"""GPU parity at the benchmark configurations' full sizes, against the CPU oracle on identical inputs.

* Config 1 (GDN decode batch): B = 64 rows, HV = 32 value / H = 16 key heads, d = 128, W = 64, R = 4.  Every window
  starts two entries short of full, so the second of three decode calls fills all 2048 windows and the flush
  re-checkpoints every head; outputs, window appends and the new checkpoints are compared at the north-star bars.
* Config 2 (KDA decode): B = 128, HV = H = 32, W = 64; the first of two calls fills and flushes all 4096 heads.
* Config 3 (standalone quantize / flush): 256 x 32 heads of Student-t(3) x 0.02 fp32 states; the quantize of every head
  is compared with the oracle, and the all-due flush on 512 heads with the oracle and on all 8192 heads through
  size-independent properties of the codes (range, each row's maximum at +-qmax, window reset).

The windows are synthetic but consistent with the state's meaning: unit-norm bf16 keys, bf16 values, GDN weights
w_j = prod_{i>j} alpha_i with P = prod alpha_i; KDA per-channel step decays e_j = exp(g_j) (fp16) with P = sum g_j.
"""
import warnings

import numpy as np
import pytest
import torch

from oracle import lq_oracle as O
from tests import lqgpu as G
from tests.fixtures import gate_params, make_inputs, make_state
from tests.test_gpu_parity import _assert_step_state, _run_flush

pytestmark = pytest.mark.gpu

RT, AT = 2e-2, 1e-3


def _fill_windows(rng, st, h, kda):
    """Every head's window holds h entries (entries >= h keep the empty-window invariants)."""
    L = st["Wbuf"].shape[-1]
    st["hcnt"][:] = h
    kb = rng.standard_normal(st["Kbuf"][:, :, :h].shape)
    st["Kbuf"][:, :, :h] = O.bf16(kb / np.linalg.norm(kb, axis=-1, keepdims=True))
    st["Ubuf"][:, :, :h] = O.bf16(0.5 * rng.standard_normal(st["Ubuf"][:, :, :h].shape))
    st["Kbuf"][:, :, h:] = 0.0
    st["Ubuf"][:, :, h:] = 0.0
    st["Wbuf"][:] = 0.0
    if kda:
        g = -0.1 * rng.random(st["Gbuf"][:, :, :h].shape)            # per-channel log-gates of the entries
        st["Gbuf"][:, :, :h] = O.fp16(np.exp(g))
        st["Gbuf"][:, :, h:] = np.float16(1.0)
        st["Wbuf"][..., :h] = 1.0
        st["Pbuf"][:] = g.sum(axis=2).astype(np.float32)
    else:
        lg = -0.1 * rng.random(st["Wbuf"][..., :h].shape)
        later = np.flip(np.cumsum(np.flip(lg, -1), -1), -1) - lg      # sum of the later entries' log-gates
        st["Wbuf"][..., :h] = np.exp(later).astype(np.float32)
        st["Pbuf"][..., 0] = np.exp(lg.sum(-1)).astype(np.float32)
    assert L > h


def _decode(lq, ssm, mixed, a, b, A_log, dt_bias, idx):
    mg, ag, bg, Ag, dg, ig = G.inputs_gpu(mixed, a, b, A_log, dt_bias, idx)
    out = torch.empty(len(idx), lq.HV, lq.V, dtype=torch.bfloat16, device=G.DEV)
    lq.decode(ssm, mg, ag, bg, Ag, dg, ig, out)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _materialized(c, qmax):
    """Q U^T + codes Sk Sv / qmax per (slot, head) of a flushed or quantised checkpoint, and its quantisation step."""
    K = c["Sk"].shape[-1]
    uq = c["UQ"].astype(np.float64)
    qu = np.einsum("shrv,shrc->shvc", uq[..., K:], uq[..., :K])
    step = c["Sk"].astype(np.float64)[:, :, None, :] * c["Sv"].astype(np.float64)[:, :, :, None] / qmax
    return qu + c["Sq"].astype(np.float64) * step, qu, step


def _assert_checkpoints(g, r, slots, qmax=127.0, S=None):
    """Checkpoints of the same states on both sides.  Factors (U^T | Q^T, fp16) within 1 % in norm; codes within 1 LSB
    on <= 0.1 % of the elements.  A head may differ by more than 1 LSB only where its factors differ: one factor entry
    rounded to the other fp16 neighbour (an fp32 sum of a different order on the other side of a rounding boundary)
    moves a row or column of the residual by ~2^-11 |Q U|, and when that moves a row's maximum every code of the row
    rescales (its scale moves by up to a few 1e-3, its codes by up to 2 LSB).  Heads with codes more than 1 LSB or
    scales more than 2e-3 apart (at most 1 %, or one head of a small case) are compared by their materialised checkpoints Q U^T + codes Sk Sv / qmax,
    within one quantisation step of each side plus the factor products' difference, and must have differing factors.
    S (the standalone quantize's fp32 input, one fp16 rounding of each factor): the factors agree entrywise (rtol 2e-3:
    one fp16 ulp; atol 2e-4 for entries near zero, where an fp32 sum's error is many of their ulps), and the oracle's
    residual stage on the GPU's own factors gives the GPU's codes and scales, which pins that stage on every head."""
    gs = {k: g[k][slots] for k in ("Sq", "Sk", "Sv", "UQ")}
    rs = {k: r[k][slots] for k in ("Sq", "Sk", "Sv", "UQ")}
    uq_g, uq_r = gs["UQ"].astype(np.float64), rs["UQ"].astype(np.float64)
    assert np.linalg.norm(uq_g - uq_r) <= 1e-2 * np.linalg.norm(uq_r)
    d = np.abs(gs["Sq"].astype(np.int32) - rs["Sq"].astype(np.int32))
    assert (d > 0).mean() <= 1e-3, (d > 0).mean()
    rel = lambda k: np.abs(gs[k].astype(np.float64) / rs[k] - 1.0).max(axis=-1)
    near = (d.max(axis=(-2, -1)) <= 1) & (rel("Sk") <= 2e-3) & (rel("Sv") <= 2e-3)     # [slot, head]
    assert (~near).sum() <= max(1, 1e-2 * near.size), (~near).sum()
    if (~near).any():                                   # shown in the run's warnings summary
        warnings.warn("checkpoints: %d of %d heads beyond 1 LSB / 2e-3 in scale, compared by materialised state"
                      % (int((~near).sum()), near.size))
    if (~near).any():
        sel = lambda c: {k: v[~near][None] for k, v in c.items()}
        mg, qg, stg = _materialized(sel(gs), qmax)
        mr, qr, str_ = _materialized(sel(rs), qmax)
        assert np.all(np.abs(mg - mr) <= stg + str_ + np.abs(qg - qr) + 1e-9)
        assert np.all(np.abs(uq_g[~near] - uq_r[~near]).max(axis=(-2, -1)) > 0)   # explained by the factors
    if S is not None:
        np.testing.assert_allclose(uq_g, uq_r, rtol=2e-3, atol=2e-4)
        K = gs["Sk"].shape[-1]
        uq = gs["UQ"].reshape((-1,) + gs["UQ"].shape[2:]).astype(np.float64)
        Sf = S.reshape((-1,) + S.shape[2:])
        for i in range(0, uq.shape[0], 1024):
            c, sk, sv = O.quantize_residual(Sf[i:i + 1024], uq[i:i + 1024, :, :K].transpose(0, 2, 1),
                                            uq[i:i + 1024, :, K:].transpose(0, 2, 1), qmax)
            dq = np.abs(c.astype(np.int32) - gs["Sq"].reshape((-1,) + gs["Sq"].shape[2:])[i:i + 1024].astype(np.int32))
            assert dq.max() <= 1 and (dq > 0).mean() <= 1e-4, (i, dq.max(), (dq > 0).mean())
            np.testing.assert_allclose(sk, gs["Sk"].reshape(-1, K)[i:i + 1024], rtol=1e-5)
            np.testing.assert_allclose(sv, gs["Sv"].reshape((-1, gs["Sv"].shape[-1]))[i:i + 1024], rtol=1e-5)


def _assert_flush_pinned(g, pre, Q0, idx, qmax=127.0):
    """One flush of identical pre-flush states (`pre`, the oracle state before the flush; `g`, the GPU's after it),
    checked stage by stage.  Factors (U^T | Q^T, fp16) within one fp16 rounding of the oracle's: |diff| <= 2e-3 |x| +
    2e-4 max |x| per head (an fp32 sum of another order lands on the other side of an fp16 rounding boundary now and
    then).  Residual stage: the oracle's flush run on the GPU's own factors gives the GPU's codes within 1 LSB on <=
    0.1 % of the flushed codes and its scales within 1e-3; what remains there is the rebuilt B's own fp16 rounding
    flips.  Returns the due pairs."""
    pairs = O.due_pairs(pre, idx)
    assert pairs
    s = np.array([p[0] for p in pairs])
    hv = np.array([p[1] for p in pairs])
    K = pre["Sk"].shape[-1]
    ref = O.copy_state(pre)
    O.flush(ref, Q0, idx, qmax=qmax)
    ug, ur = g["UQ"][s, hv].astype(np.float64), ref["UQ"][s, hv].astype(np.float64)
    tol = 2e-3 * np.abs(ur) + 2e-4 * np.abs(ur).max(axis=(-2, -1), keepdims=True)
    assert np.all(np.abs(ug - ur) <= tol), np.abs(ug - ur).max()
    pin = O.copy_state(pre)
    O.flush(pin, Q0, idx, qmax=qmax, factors=(ug[:, :, :K].transpose(0, 2, 1), ug[:, :, K:].transpose(0, 2, 1)))
    d = np.abs(g["Sq"][s, hv].astype(np.int32) - pin["Sq"][s, hv].astype(np.int32))
    assert d.max() <= 1 and (d > 0).mean() <= 1e-3, (d.max(), (d > 0).mean())
    np.testing.assert_allclose(g["Sk"][s, hv], pin["Sk"][s, hv], rtol=1e-3)
    np.testing.assert_allclose(g["Sv"][s, hv], pin["Sv"][s, hv], rtol=1e-3)
    for k in ("hcnt", "Wbuf", "Pbuf"):
        assert np.array_equal(g[k][s, hv], ref[k][s, hv]), k
    return pairs


@pytest.mark.parametrize("kda", [False, True])
def test_decode_at_full_size_matches_oracle(kda):
    """Config 1 (GDN) / config 2 (KDA) at full size through LeapQuantState.decode (step, then the flush)."""
    rng = np.random.default_rng(1002 if kda else 1001)
    B, HV, H, L = (128, 32, 32, 64) if kda else (64, 32, 16, 64)
    NS = B + 1
    st, S, Q0 = make_state(rng, NS, HV, H, L=L, kda=kda)
    h0 = L - 1 if kda else L - 2
    _fill_windows(rng, st, h0, kda)
    idx = np.arange(1, NS, dtype=np.int64)
    A_log, dt_bias = gate_params(HV, 128, kda)
    ssm, lq = G.to_gpu(st)
    full_at = L - h0 - 1                                # the call that fills every window
    for t in range(L - h0 + 1):
        mixed, a, b = make_inputs(rng, B, HV, H, kda=kda)
        print("full size %s: call %d" % ("KDA" if kda else "GDN", t), flush=True)
        o_ref = (O.kda_step if kda else O.gdn_step)(st, mixed, a, b, A_log, dt_bias, idx)
        if t == full_at:
            mid = O.copy_state(st)                      # after the step, before the flush
        O.flush(st, Q0, idx)
        o_gpu = _decode(lq, ssm, mixed, a, b, A_log, dt_bias, idx)
        np.testing.assert_allclose(o_gpu, o_ref, rtol=RT, atol=AT)
        assert (G.bf16_ulps(o_gpu, o_ref) <= 2).mean() > 0.99
        g = G.from_gpu(ssm, lq)
        if t == full_at:                                # every head was due and re-checkpointed
            assert np.all(mid["hcnt"][1:] == L)
            _assert_checkpoints(g, st, slice(1, NS))
            for k in ("hcnt", "Wbuf", "Pbuf"):
                assert np.array_equal(g[k], st[k]), k
            if kda:
                assert np.array_equal(g["Gbuf"], st["Gbuf"])
            st = O.copy_state(st)
            for k in ("Sq", "Sk", "Sv", "UQ"):          # continue both sides from the same checkpoint
                st[k] = g[k].copy()
        elif t < full_at:
            _assert_step_state(g, st, idx)
    assert np.array_equal(G.from_gpu(ssm, lq)["hcnt"], st["hcnt"])


_C3 = {}


def _config3(qmax):
    """Config 3's fp32 states (seeded) and the oracle's checkpoint of them (cached: the GQA legs share it)."""
    if qmax not in _C3:
        rng = np.random.default_rng(1003)
        NSL, HV = 256, 32
        S = (0.02 * rng.standard_t(3, (NSL + 1, HV, 128, 128))).astype(np.float32)
        st = O.new_state(NSL + 1, HV, 16, L=64)
        print("config 3 (qmax %g): oracle quantize of %d heads" % (qmax, NSL * HV), flush=True)
        O.quantize(st, S, O.make_q0(128, 4), np.arange(1, NSL + 1, dtype=np.int64), qmax=qmax)
        _C3[qmax] = (S, st)
    return _C3[qmax]


@pytest.mark.parametrize("H", [16, 32])
@pytest.mark.parametrize("qmax", [127.0, 31.0])
def test_config3_quantize_and_flush_at_full_size(qmax, H):
    """Config 3: 256 x 32 Student-t(3) x 0.02 heads, INT8 and 6-bit; quantize of every head vs the oracle; all-due
    flush (64 buffered entries per head) vs the oracle on 512 heads and through properties of the codes on all 8192.
    H = 32: every state has its own window of 64 entries (GQA 1: the decode steps, then the standalone persistent
    flush takes the 8192 due heads); H = 16: two value heads share a key head's window keys (GQA 2: the one-launch
    decode flushes them)."""
    rng = np.random.default_rng(1003 + H)
    NSL, HV, L = 256, 32, 64
    NS = NSL + 1
    S, st16 = _config3(qmax)
    st = O.new_state(NS, HV, H, L=L)
    for k in ("Sq", "Sk", "Sv", "UQ"):
        st[k] = st16[k].copy()
    Q0 = O.make_q0(128, 4)
    idx = np.arange(1, NS, dtype=np.int64)
    ssm, lq = G.to_gpu(st, qmax=qmax)
    if H == 16:                                         # the quantize of every head (the same states at both H)
        ssm.copy_(torch.from_numpy(S))
        lq.quantize(ssm, torch.from_numpy(idx).to(G.DEV))
        g = G.from_gpu(ssm, lq)
        _assert_checkpoints(g, st, slice(1, NS), qmax=qmax, S=S[1:])

    # the flush of a full window on every head, from the oracle's checkpoint on both sides
    _fill_windows(rng, st, L - 1, kda=False)
    sub = np.arange(1, 17, dtype=np.int64)              # 16 slots x 32 heads checked against the oracle
    A_log, dt_bias = gate_params(HV)
    mixed, a, b = make_inputs(rng, NSL, HV, H)
    G.load_state(lq, ssm, st)
    print("config 3 (qmax %g, H %d): oracle step + flush of %d heads" % (qmax, H, len(sub) * HV), flush=True)
    O.gdn_step(st, mixed, a, b, A_log, dt_bias, idx, qmax=qmax)    # fills every window (64 entries)
    before = O.copy_state(st)
    O.flush(st, Q0, sub, qmax=qmax)
    _decode(lq, ssm, mixed, a, b, A_log, dt_bias, idx)  # step + flush of all 8192 heads on the GPU
    g = G.from_gpu(ssm, lq)
    assert np.all(before["hcnt"][1:] == L)
    _assert_checkpoints(g, st, sub, qmax=qmax)
    codes = g["Sq"][1:].astype(np.int32)
    assert np.abs(codes).max() <= qmax
    rmax = np.abs(codes).max(axis=-1)                   # per (slot, head, row v)
    assert np.all(rmax == qmax), np.argwhere(rmax != qmax)[:4]
    assert np.all(g["hcnt"][1:] == 0) and np.all(g["Wbuf"][1:] == 0) and np.all(g["Pbuf"][1:] == 1)
    assert np.all(np.isfinite(g["Sk"][1:])) and np.all(g["Sk"][1:] > 0)
    assert np.all(np.isfinite(g["Sv"][1:])) and np.all(g["Sv"][1:] > 0)
