"""GPU parity of the wider ranks against the CPU oracle: the GDN step at R = 8 and 16, the R = 8 flush (with its
column-dropping CholeskyQR), the decode call that chains them, and the quantize / dequant that write and read such
checkpoints (kernels.py:63-64, 457-469, 1091, 1123, 1744-1772).  Bars as in test_gpu_parity.py.
"""
import numpy as np
import pytest
import torch

from leapquant_amd import kernels as KN
from oracle import lq_oracle as O
from tests import lqgpu as G
from tests.fixtures import due_flush_case, gate_params, make_inputs, make_state, oracle_steps
from tests.test_gpu_parity import RT, AT, _assert_step_state, _run_flush

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("R", [8, 16])
@pytest.mark.parametrize("GQA", [1, 2, 4])
def test_step_wide_rank_matches_oracle(R, GQA):
    rng = np.random.default_rng(700 + R + GQA)
    NS, HV, L = 6, 4, 64
    H = HV // GQA
    st, _, Q0 = make_state(rng, NS, HV, H, L=L, R=R)
    oracle_steps(rng, st, 9, NS, HV, H)                  # partial windows, no flush (R = 16 has none)
    idx = np.array([3, 0, 1, 5, -1, 2], np.int64)
    mixed, a, b = make_inputs(rng, len(idx), HV, H)
    A_log, dt_bias = gate_params(HV)
    raw = G.RawGdnState(st)
    step = KN.make_gdn_step(NS, HV, H, 128, 128, L, raw.SS, R=R)
    o_ref = O.gdn_step(st, mixed, a, b, A_log, dt_bias, idx)
    m, a_, b_, al, dt, ix = G.inputs_gpu(mixed, a, b, A_log, dt_bias, idx)
    out = torch.empty(len(idx), HV, 128, dtype=torch.bfloat16, device=G.DEV)
    v = raw.views(raw.ssm)
    step(v["q32"], v["Sk"], v["Sv"], v["skv"], raw.Kbuf, raw.Ubuf, raw.Wbuf, raw.Pbuf, raw.hcnt, m, a_, b_, al, dt,
         v["uq"], ix, out)
    o_gpu = out.float().cpu().numpy()
    np.testing.assert_allclose(o_gpu, o_ref, rtol=RT, atol=AT)
    assert np.all(o_gpu[[1, 4]] == 0)
    assert (G.bf16_ulps(o_gpu, o_ref) <= 2).mean() > 0.99
    _assert_step_state(G.from_gpu(raw.ssm, raw), st, idx)


# The R = 8 flush's codes are compared at <= 1 LSB on <= 0.5 % (R <= 4: 0.1 %).  Its fp16 factors are rounded after an
# orthogonalisation with condition numbers of 10-20, so ONE fp16 ulp of difference in one entry of the rebuilt state
# per head -- what two correct fp32 rebuilds differ by -- already moves 0.1-0.3 % of the codes, by one LSB each
# (test_oracle_pins.test_flush_r8_code_sensitivity).  The logical state after the flush is checked on its own bound.
R8_CODE_FRAC = 5e-3


def _assert_flushed(g, r, slots, frac_max=R8_CODE_FRAC):
    frac, mx = G.code_mismatch(g["Sq"][slots], r["Sq"][slots])
    assert mx <= 1 and frac <= frac_max, (frac, mx)
    np.testing.assert_allclose(g["Sk"][slots], r["Sk"][slots], rtol=2e-3)
    np.testing.assert_allclose(g["Sv"][slots], r["Sv"][slots], rtol=2e-3)
    uq_g, uq_r = g["UQ"].astype(np.float64), r["UQ"].astype(np.float64)
    assert np.linalg.norm(uq_g - uq_r) <= 1e-2 * np.linalg.norm(uq_r)
    for k in ("hcnt", "Wbuf", "Pbuf"):
        assert np.array_equal(g[k], r[k]), k


@pytest.mark.parametrize("L", [16, 64])
def test_flush_r8_matches_oracle(L):
    rng = np.random.default_rng(800 + L)
    st, Q0 = due_flush_case(rng, L, R=8)
    idx = np.array([1, 0, 2, 3, -1], np.int64)
    ssm, lq = G.to_gpu(st)
    assert lq.R == 8
    before = O.copy_state(st)
    dbg = O.flush(st, Q0, idx, return_debug=True)
    assert len(dbg["pairs"]) == 2 * 4
    S_before = O.materialize(before)
    _run_flush(lq, ssm, torch.from_numpy(idx.astype(np.int32)).to(G.DEV))
    g = G.from_gpu(ssm, lq)
    _assert_flushed(g, st, [1, 3])
    assert np.array_equal(g["Sq"][2], before["Sq"][2]) and np.array_equal(g["UQ"][2], before["UQ"][2])
    # the GPU's own checkpoint keeps the logical state within its quantisation bound (no oracle involved)
    S_gpu = O.materialize(g)
    for s in (1, 3):
        for h in range(4):
            sk, sv = g["Sk"][s, h].astype(np.float64), g["Sv"][s, h].astype(np.float64)
            bound = 0.5 * sk[None, :] * sv[:, None] / 127.0 + 2 ** -9 * np.abs(S_before[s, h]).max()
            assert np.all(np.abs(S_gpu[s, h] - S_before[s, h]) <= bound), (s, h)


def test_flush_r8_drops_dependent_factors():
    """The rank-2 state at R = 8: CholeskyQR drops factors 3..8 (exactly zero U and Q rows), as in the oracle.  The
    residual left after two factors is rounding noise on either side, so its codes are not compared (as for R = 4 in
    test_gpu_modes): both sides keep the logical state within the quantisation bound and agree on the live factors."""
    from tests.test_oracle_pins import _rank2_state
    st, Q0, S = _rank2_state(R=8)
    ssm, lq = G.to_gpu(st, H=1)
    O.flush(st, Q0, np.array([1]))
    _run_flush(lq, ssm, torch.tensor([1], dtype=torch.int32, device=G.DEV))
    g = G.from_gpu(ssm, lq)
    for k in ("Sq", "Sk", "Sv", "UQ"):
        assert np.all(np.isfinite(g[k][1].astype(np.float64))), k
    assert np.all(g["UQ"][1, 0, 2:] == 0) and np.all(st["UQ"][1, 0, 2:] == 0)
    np.testing.assert_allclose(g["UQ"][1, 0, :2].astype(np.float32), st["UQ"][1, 0, :2].astype(np.float32),
                               rtol=2e-3, atol=2e-4)
    for c in (g, st):
        after = O.materialize(c)[1, 0]
        sk, sv = c["Sk"][1, 0].astype(np.float64), c["Sv"][1, 0].astype(np.float64)
        bound = 0.5 * sk[None, :] * sv[:, None] / 127.0 + 2 ** -9 * np.abs(S).max()
        assert np.all(np.abs(after - S) <= bound)


def test_decode_r8_across_a_window_end():
    """LeapQuantState.decode at R = 8 (the step, then the R = 8 flush): rows whose window fills take the flush."""
    rng = np.random.default_rng(850)
    NS, HV, H, L = 6, 4, 2, 16
    st, _, Q0 = make_state(rng, NS, HV, H, L=L, R=8)
    oracle_steps(rng, st, 7, NS, HV, H, flush_Q0=Q0)
    A_log, dt_bias = gate_params(HV)
    for s in (2, 4):                                       # slots 2 and 4 one entry short of a full window
        while st["hcnt"][s, 0] < L - 1:
            mixed, a, b = make_inputs(rng, 1, HV, H)
            O.gdn_step(st, mixed, a, b, A_log, dt_bias, np.array([s]))
    idx = np.array([2, 1, 4, 0, 5], np.int64)
    mixed, a, b = make_inputs(rng, len(idx), HV, H)
    ssm, lq = G.to_gpu(st)
    o_ref = O.gdn_step(st, mixed, a, b, A_log, dt_bias, idx)
    O.flush(st, Q0, idx)
    m, a_, b_, al, dt, ix = G.inputs_gpu(mixed, a, b, A_log, dt_bias, idx)
    out = torch.empty(len(idx), HV, 128, dtype=torch.bfloat16, device=G.DEV)
    lq.decode(ssm, m, a_, b_, al, dt, ix, out)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.float().cpu().numpy(), o_ref, rtol=RT, atol=AT)
    g = G.from_gpu(ssm, lq)
    assert np.all(g["hcnt"][[2, 4]] == 0)
    _assert_flushed(g, st, [2, 4])


@pytest.mark.parametrize("R", [8, 16])
def test_quantize_wide_rank_matches_oracle(R):
    rng = np.random.default_rng(900 + R)
    NS, HV, H, L = 5, 4, 2, 16
    S = (0.02 * rng.standard_t(3, (NS, HV, 128, 128))).astype(np.float32)
    S[3, 2] += np.outer(rng.standard_normal(128), rng.standard_normal(128)).astype(np.float32) * 0.05
    st = O.new_state(NS, HV, H, L=L, R=R)
    raw = G.RawGdnState(st)
    raw.ssm.copy_(torch.from_numpy(S))
    idx = np.array([2, 0, 4, 3], np.int64)
    O.quantize(st, S, O.make_q0(128, R), idx)
    q = KN.make_quantize(NS, HV, 128, 128, L, raw.SS, R=R)
    v = raw.views(raw.ssm)
    q(raw.ssm, v["Sq"], v["Sk"], v["Sv"], v["uq"], raw.Wbuf, raw.Pbuf, raw.hcnt,
      torch.from_numpy(O.make_q0(128, R)).to(G.DEV), torch.from_numpy(idx.astype(np.int32)).to(G.DEV))
    g = G.from_gpu(raw.ssm, raw)
    for s in (2, 3, 4):
        frac, mx = G.code_mismatch(g["Sq"][s], st["Sq"][s])
        assert mx <= 1 and frac <= 1e-3, (s, frac, mx)
        np.testing.assert_allclose(g["Sk"][s], st["Sk"][s], rtol=1e-3)
        np.testing.assert_allclose(g["Sv"][s], st["Sv"][s], rtol=1e-3)
        np.testing.assert_allclose(g["UQ"][s].astype(np.float32), st["UQ"][s].astype(np.float32), rtol=2e-3, atol=2e-4)
    np.testing.assert_array_equal(raw.ssm[1].cpu().numpy(), S[1])


@pytest.mark.parametrize("R", [8, 16])
def test_dequant_wide_rank_matches_oracle(R):
    rng = np.random.default_rng(950 + R)
    NS, HV, H, L = 6, 4, 2, 64
    st, _, Q0 = make_state(rng, NS, HV, H, L=L, R=R)
    oracle_steps(rng, st, 30, NS, HV, H)
    idx = np.array([1, 0, 3, 5], np.int64)
    raw = G.RawGdnState(st)
    ref = O.dequant(st, idx)
    d = KN.make_dequant(NS, HV, 128, 128, L, raw.SS, buf_dtype=KN.BF16, R=R)
    v = raw.views(raw.ssm)
    d(raw.ssm, v["Sq"], v["Sk"], v["Sv"], raw.Kbuf, raw.Ubuf, raw.Wbuf, raw.Pbuf, None, raw.hcnt, v["uq"],
      torch.from_numpy(idx.astype(np.int32)).to(G.DEV))
    g = G.from_gpu(raw.ssm, raw)
    for s in (1, 3, 5):
        got = raw.ssm[s].cpu().numpy()
        err = np.abs(got - ref[s]).max() / np.abs(ref[s]).max()
        assert err < 1e-5, (s, err)
    assert np.array_equal(g["hcnt"], st["hcnt"]) and np.array_equal(g["Wbuf"], st["Wbuf"])
