"""GPU parity of the GDN head-dim variants (K, V) = (64, 128) and (64, 64) (reference kernels.py:62-65, 1089-1092)
against the CPU oracle: step, flush, quantize, dequant and a decode run over several windows.  Same bars as the
128 x 128 tests: bf16 outputs within rtol 2e-2 / atol 1e-3 (and >= 99 % within 2 ulps), codes within 1 LSB on <= 0.1 %
of the elements.  The reference runs these shapes at L = 16 only; the window lengths 16 and 64 are both tested here.
"""
import numpy as np
import pytest
import torch

from oracle import lq_oracle as O
from tests import lqgpu as G
from tests.fixtures import gate_params, make_inputs, make_state
from tests.test_gpu_full_size import _assert_flush_pinned
from tests.test_gpu_modes import _resync
from tests.test_gpu_parity import AT, RT, _assert_step_state, _run_flush, _run_step

pytestmark = pytest.mark.gpu

DIMS = [(64, 128), (64, 64)]


def _steps(rng, st, Q0, steps, NS, HV, H, K, V, flush=True):
    """Oracle decode steps (each + flush) on random subsets of the slots."""
    A_log, dt_bias = gate_params(HV, K)
    for _ in range(steps):
        sl = rng.permutation(np.arange(1, NS))[: rng.integers(1, NS)]
        mixed, a, b = make_inputs(rng, len(sl), HV, H, K, V)
        O.gdn_step(st, mixed, a, b, A_log, dt_bias, sl)
        if flush:
            O.flush(st, Q0, sl)


@pytest.mark.parametrize("K,V", DIMS)
@pytest.mark.parametrize("L,GQA", [(16, 2), (64, 1), (16, 4)])
def test_step_matches_oracle(K, V, L, GQA):
    rng = np.random.default_rng(1100 + K + V + L + GQA)
    NS, HV = 6, 4
    H = HV // GQA
    st, S, Q0 = make_state(rng, NS, HV, H, K=K, V=V, L=L)
    _steps(rng, st, Q0, L + 9, NS, HV, H, K, V)
    idx = np.array([3, 0, 1, 5, -1, 2], np.int64)
    mixed, a, b = make_inputs(rng, len(idx), HV, H, K, V)
    A_log, dt_bias = gate_params(HV, K)
    ssm, lq = G.to_gpu(st)
    o_ref = O.gdn_step(st, mixed, a, b, A_log, dt_bias, idx)
    o_gpu = _run_step(lq, ssm, *G.inputs_gpu(mixed, a, b, A_log, dt_bias, idx))
    np.testing.assert_allclose(o_gpu, o_ref, rtol=RT, atol=AT)
    assert np.all(o_gpu[[1, 4]] == 0)
    assert (G.bf16_ulps(o_gpu, o_ref) <= 2).mean() > 0.99
    _assert_step_state(G.from_gpu(ssm, lq), st, idx)


@pytest.mark.parametrize("K,V", DIMS)
@pytest.mark.parametrize("L", [16, 64])
def test_step_at_every_fill(K, V, L):
    """Slots at chosen window fills (empty, one entry, the 4- / 8-row load boundaries, the last fill before full)."""
    fills = [0, 1, 3, 4, 7, 8, 9, 12, 15] if L == 16 else [0, 1, 8, 15, 16, 17, 31, 32, 33, 48, 63]
    rng = np.random.default_rng(1200 + K + V + L)
    NS, HV, H = len(fills) + 1, 2, 1
    st, S, Q0 = make_state(rng, NS, HV, H, K=K, V=V, L=L)
    A_log, dt_bias = gate_params(HV, K)
    target = np.array([0] + fills)
    for t in range(max(fills)):
        sl = np.nonzero(target > t)[0].astype(np.int64)
        mixed, a, b = make_inputs(rng, len(sl), HV, H, K, V)
        O.gdn_step(st, mixed, a, b, A_log, dt_bias, sl)
    assert np.array_equal(st["hcnt"][1:, 0], fills)
    idx = rng.permutation(np.arange(1, NS)).astype(np.int64)
    mixed, a, b = make_inputs(rng, len(idx), HV, H, K, V)
    ssm, lq = G.to_gpu(st)
    o_ref = O.gdn_step(st, mixed, a, b, A_log, dt_bias, idx)
    o_gpu = _run_step(lq, ssm, *G.inputs_gpu(mixed, a, b, A_log, dt_bias, idx))
    np.testing.assert_allclose(o_gpu, o_ref, rtol=RT, atol=AT)
    assert (G.bf16_ulps(o_gpu, o_ref) <= 2).mean() > 0.99
    _assert_step_state(G.from_gpu(ssm, lq), st, idx)


# The K = 64 flush's codes are compared at <= 1 LSB on <= 0.25 % (128 x 128: 0.1 %).  A head of 64 x 64 or 64 x 128
# holds 4096 / 8192 codes, and one fp16 rounding flip of a factor entry moves a whole row or column of its residual: a
# change of ONE fp16 ulp in one entry of each head's rebuilt state -- what two correct fp32 rebuilds differ by --
# already moves 0.04-0.10 % of these codes (test_oracle_pins.test_flush_head_dim_code_sensitivity).
HD_CODE_FRAC = 2.5e-3


@pytest.mark.parametrize("K,V", DIMS)
@pytest.mark.parametrize("L", [16, 64])
@pytest.mark.parametrize("GQA", [2, 1])
def test_flush_matches_oracle(K, V, L, GQA):
    """The K = 64 flush: (64, 128) one head per workgroup; (64, 64) two heads of one key head per workgroup at even
    GQA (kernels.py:1095-1097), one at odd GQA."""
    rng = np.random.default_rng(1300 + K + V + L + 7 * GQA)
    NS, HV = 6, 4
    H = HV // GQA
    st, S, Q0 = make_state(rng, NS, HV, H, K=K, V=V, L=L)
    _steps(rng, st, Q0, L + 5, NS, HV, H, K, V)
    A_log, dt_bias = gate_params(HV, K)
    for s in (1, 3):                                     # slots 1 and 3 due, the others partial
        while st["hcnt"][s, 0] < L:
            mixed, a, b = make_inputs(rng, 1, HV, H, K, V)
            O.gdn_step(st, mixed, a, b, A_log, dt_bias, np.array([s]))
    idx = np.array([1, 0, 2, 3, -1], np.int64)
    ssm, lq = G.to_gpu(st)
    before = O.copy_state(st)
    dbg = O.flush(st, Q0, idx, return_debug=True)
    assert len(dbg["pairs"]) == 2 * HV
    _run_flush(lq, ssm, torch.from_numpy(idx.astype(np.int32)).to(G.DEV))
    g = G.from_gpu(ssm, lq)
    frac, mx = G.code_mismatch(g["Sq"][[1, 3]], st["Sq"][[1, 3]])           # the flushed heads only
    assert mx <= 1 and frac <= HD_CODE_FRAC, (frac, mx)
    np.testing.assert_allclose(g["Sk"], st["Sk"], rtol=2e-3)
    np.testing.assert_allclose(g["Sv"], st["Sv"], rtol=2e-3)
    uq_g, uq_r = g["UQ"].astype(np.float64), st["UQ"].astype(np.float64)
    assert np.linalg.norm(uq_g - uq_r) <= 1e-2 * np.linalg.norm(uq_r)
    for k in ("hcnt", "Wbuf", "Pbuf"):
        assert np.array_equal(g[k], st[k]), k
    assert np.array_equal(g["Sq"][2], before["Sq"][2]) and np.array_equal(g["UQ"][2], before["UQ"][2])
    # nothing outside the (slot, head) blocks' checkpoint region: the fp32 words past it keep their bytes
    ck = (V * K // 4 + K + V + 4 * (K + V) // 2)
    tail_g = ssm.view(NS, HV, -1)[:, :, ck:].cpu().numpy()
    assert np.all(tail_g == 0)


@pytest.mark.parametrize("K,V", DIMS)
@pytest.mark.parametrize("qmax,HV,H", [(127.0, 4, 2), (31.0, 4, 2), (127.0, 3, 3)])
def test_quantize_matches_oracle(K, V, qmax, HV, H):
    """The K = 64 quantize: (64, 64) with HV even takes two heads of a slot per workgroup, with HV odd one."""
    rng = np.random.default_rng(1400 + K + V + int(qmax) + HV)
    NS = 5
    S = (0.02 * rng.standard_t(3, (NS, HV, V, K))).astype(np.float32)
    S[2, 1] = 0.0                                        # all-zero state: EPS floors
    st = O.new_state(NS, HV, H, K=K, V=V, L=16)
    Q0 = O.make_q0(V, 4)
    ssm, lq = G.to_gpu(st, qmax=qmax)
    ssm.copy_(torch.from_numpy(S))
    idx = np.array([2, 0, 4, 1], np.int64)
    O.quantize(st, S, Q0, idx, qmax=qmax)
    lq.quantize(ssm, torch.from_numpy(idx).to(G.DEV))
    g = G.from_gpu(ssm, lq)
    for s in (1, 2, 4):
        frac, mx = G.code_mismatch(g["Sq"][s], st["Sq"][s])
        assert mx <= 1 and frac <= 1e-3, (s, frac, mx)
        np.testing.assert_allclose(g["Sk"][s], st["Sk"][s], rtol=1e-3)
        np.testing.assert_allclose(g["Sv"][s], st["Sv"][s], rtol=1e-3)
        np.testing.assert_allclose(g["UQ"][s].astype(np.float32), st["UQ"][s].astype(np.float32), rtol=2e-3, atol=2e-4)
    assert np.all(g["Sq"][2, 1] == 0) and np.all(g["Sk"][2, 1] == np.float32(1e-12))
    np.testing.assert_array_equal(ssm[3].cpu().numpy(), S[3])   # slot 3 not in idx: untouched


def test_flush_pair_with_one_head_due():
    """(64, 64) at GQA 2 flushes the two heads of a key head together; when only one of them is due, that one is flushed
    (as the oracle does) and its partner keeps every byte."""
    K, V, L = 64, 64, 16
    rng = np.random.default_rng(1390)
    NS, HV, H = 4, 4, 2
    st, S, Q0 = make_state(rng, NS, HV, H, K=K, V=V, L=L)
    _steps(rng, st, Q0, L + 3, NS, HV, H, K, V)
    A_log, dt_bias = gate_params(HV, K)
    for s in (1, 2):                                     # bring both slots to L - 1, then head 1 / head 2 to L only
        while st["hcnt"][s, 0] < L - 1:
            mixed, a, b = make_inputs(rng, 1, HV, H, K, V)
            O.gdn_step(st, mixed, a, b, A_log, dt_bias, np.array([s]))
    st["hcnt"][1, 1] = L                                 # slot 1: head 1 due (pair 0: heads 0, 1), head 0 not
    st["hcnt"][2, 2] = L                                 # slot 2: head 2 due (pair 1: heads 2, 3), head 3 not
    idx = np.array([1, 2], np.int64)
    ssm, lq = G.to_gpu(st)
    before = O.copy_state(st)
    dbg = O.flush(st, Q0, idx, return_debug=True)
    assert sorted(dbg["pairs"]) == [(1, 1), (2, 2)]
    _run_flush(lq, ssm, torch.from_numpy(idx.astype(np.int32)).to(G.DEV))
    g = G.from_gpu(ssm, lq)
    for s, h in ((1, 1), (2, 2)):
        frac, mx = G.code_mismatch(g["Sq"][s, h], st["Sq"][s, h])
        assert mx <= 1 and frac <= HD_CODE_FRAC, (s, h, frac, mx)
        np.testing.assert_allclose(g["Sk"][s, h], st["Sk"][s, h], rtol=2e-3)
        np.testing.assert_allclose(g["Sv"][s, h], st["Sv"][s, h], rtol=2e-3)
    for s, h in ((1, 0), (2, 3), (1, 2), (1, 3), (2, 0), (2, 1)):
        for k in ("Sq", "Sk", "Sv", "UQ", "Wbuf", "Pbuf", "hcnt"):
            assert np.array_equal(g[k][s, h], before[k][s, h]), (s, h, k)
    for k in ("hcnt", "Wbuf", "Pbuf"):
        assert np.array_equal(g[k], st[k]), k


@pytest.mark.parametrize("K,V", DIMS)
def test_dequant_matches_oracle(K, V):
    rng = np.random.default_rng(1500 + K + V)
    NS, HV, H = 6, 4, 2
    st, S, Q0 = make_state(rng, NS, HV, H, K=K, V=V, L=64)
    _steps(rng, st, Q0, 40, NS, HV, H, K, V)
    idx = np.array([1, 0, 3, 5], np.int64)
    ssm, lq = G.to_gpu(st)
    ref = O.dequant(st, idx)
    lq.dequantize(ssm, torch.from_numpy(idx).to(G.DEV))
    g = G.from_gpu(ssm, lq)
    for s in (1, 3, 5):
        got = ssm[s].cpu().numpy()
        err = np.abs(got - ref[s]).max() / np.abs(ref[s]).max()
        assert err < 1e-5, (s, err)
    assert np.array_equal(g["hcnt"], st["hcnt"]) and np.array_equal(g["Wbuf"], st["Wbuf"])


@pytest.mark.parametrize("K,V", DIMS)
def test_dequant_empty_and_partial_windows(K, V):
    """Heads with an empty window (no window products) and with a partial one in one dequant call."""
    rng = np.random.default_rng(1600 + K + V)
    NS, HV, H = 6, 4, 2
    st, S, Q0 = make_state(rng, NS, HV, H, K=K, V=V, L=64)
    A_log, dt_bias = gate_params(HV, K)
    for _ in range(9):                                  # slot 3 only: h = 9; the others stay at h = 0
        mixed, a, b = make_inputs(rng, 1, HV, H, K, V)
        O.gdn_step(st, mixed, a, b, A_log, dt_bias, np.array([3]))
    idx = np.array([1, 3, 0, 5], np.int64)
    ssm, lq = G.to_gpu(st)
    ref = O.dequant(st, idx)
    lq.dequantize(ssm, torch.from_numpy(idx).to(G.DEV))
    g = G.from_gpu(ssm, lq)
    for s in (1, 3, 5):
        got = ssm[s].cpu().numpy()
        err = np.abs(got - ref[s]).max() / np.abs(ref[s]).max()
        assert err < 1e-5, (s, err)
    assert np.array_equal(g["hcnt"], st["hcnt"]) and np.array_equal(g["Wbuf"], st["Wbuf"])


@pytest.mark.parametrize("K,V", DIMS)
def test_decode_over_windows_matches_oracle(K, V):
    """LeapQuantState.decode (step + flush on the device's due flag) for 2.5 windows of L = 16.  The compared oracle
    continues from the GPU's state after every call, so every step's outputs (>= 99 % within 2 ulps) and every flush
    (factors within one fp16 rounding, the residual stage's codes on the GPU's factors within 1 LSB on <= 0.1 %) are
    compared from identical inputs; a second oracle runs free beside it, and the GPU's final codes are within 1 LSB of
    it on <= 3 % (the free-running drift)."""
    rng = np.random.default_rng(1600 + K + V)
    NS, HV, H, L = 4, 4, 2, 16
    st, S, Q0 = make_state(rng, NS, HV, H, K=K, V=V, L=L)
    free = O.copy_state(st)                             # the oracle free-running beside the GPU
    ssm, lq = G.to_gpu(st)
    A_log, dt_bias = gate_params(HV, K)
    idx = np.array([2, 0, 1, 3], np.int64)
    ulps = []
    flushed = 0
    for t in range(40):
        mixed, a, b = make_inputs(rng, len(idx), HV, H, K, V)
        o_ref = O.gdn_step(st, mixed, a, b, A_log, dt_bias, idx)
        due = O.due_pairs(st, idx)
        pre = O.copy_state(st)
        O.flush(st, Q0, idx)
        O.gdn_step(free, mixed, a, b, A_log, dt_bias, idx)
        O.flush(free, Q0, idx)
        mg, ag, bg, Ag, dg, ig = G.inputs_gpu(mixed, a, b, A_log, dt_bias, idx)
        out = torch.empty(len(idx), HV, V, dtype=torch.bfloat16, device=G.DEV)
        lq.decode(ssm, mg, ag, bg, Ag, dg, ig, out)
        o_gpu = out.float().cpu().numpy()
        np.testing.assert_allclose(o_gpu, o_ref, rtol=RT, atol=AT, err_msg="step %d" % t)
        ulps.append(G.bf16_ulps(o_gpu, o_ref))
        g = G.from_gpu(ssm, lq)
        if due:                                         # each flush from identical inputs, stage by stage
            _assert_flush_pinned(g, pre, Q0, idx)
            flushed += 1
        _resync(st, g)                                  # continue the compared oracle from the GPU's state
    assert flushed >= 2
    assert (np.concatenate([u.ravel() for u in ulps]) <= 2).mean() > 0.99
    g = G.from_gpu(ssm, lq)
    assert np.array_equal(g["hcnt"], free["hcnt"])
    # against the free-running oracle the codes drift past the per-flush bar (each flush re-quantises the previous
    # flushes' 1-LSB differences); they stay within 1 LSB
    frac, mx = G.code_mismatch(g["Sq"], free["Sq"])
    assert mx <= 1 and frac <= 3e-2, (frac, mx)
