"""Pins of the CPU oracle (oracle/lq_oracle.py) against checks that do not reuse its formulas.

  * decode steps  -> dense float64 gated-delta / KDA rule evolved step by step on an independent state (brute force),
  * flush          -> numpy QR subspace iteration (QR of S S^T Q0 with a positive diagonal), U = S^T Q, and the
                      quantisation bounds (|code| <= qmax, +-qmax at every row's argmax, |deq - E| <= Sk Sv / (2 qmax)),
  * quantize / lowrank -> numpy QR-based subspace iteration (MGS == QR with positive diagonal in exact arithmetic),
  * special cases  -> empty window, alpha = 1, beta ~ 0, zero state, padding rows, fully decayed head,
  * golden files   -> the committed trajectories in tests/golden/ (catches changes of the oracle itself).
Each check is chosen so that a plausible slip (dropped term, wrong sign, wrong head/key mapping, transposed factor,
a missing decay) fails it.
"""
import os

import numpy as np
import pytest

from oracle import lq_oracle as O
from tests.fixtures import due_flush_case, from_bits, gate_params, make_inputs, make_state, state_from_npz

K = V = 128
GOLD = os.path.join(os.path.dirname(__file__), "golden")
# head dims (K, V): GDN (128, 128), (64, 128), (64, 64) (kernels.py:62, 1089); KDA 128 x 128 (kernels.py:727)
GDN_DIMS = [(128, 128), (64, 128), (64, 64)]
STEP_CASES = [(False, d) for d in GDN_DIMS] + [(True, (128, 128))]
# (kda, dims, glb, R): KDA also with GLM's bounded gate (kernels.py:702-712); the GDN rank ablation R = 16 (kernels.py:63)
TRAJ_CASES = [(False, d, 0.0, 4) for d in GDN_DIMS] + [(True, (128, 128), 0.0, 4), (True, (128, 128), -5.0, 4),
                                                        (False, (128, 128), 0.0, 16)]
# (kda, dims, R): the flush's ranks, R = 8 for GDN 128 x 128 (kernels.py:1091)
FLUSH_CASES = [(k, d, 4) for k, d in STEP_CASES] + [(False, (128, 128), 8)]


def _qk_from_mixed(mixed, H, HV, K=K, V=V):
    q = mixed[:, :H * K].reshape(-1, H, K).astype(np.float64)
    k = mixed[:, H * K:2 * H * K].reshape(-1, H, K).astype(np.float64)
    v = mixed[:, 2 * H * K:].reshape(-1, HV, V).astype(np.float64)
    return q, k, v


def _sign_fixed_qr(X):
    Q, Rm = np.linalg.qr(X)
    sg = np.sign(np.diagonal(Rm, axis1=-2, axis2=-1))
    sg[sg == 0] = 1
    return Q * sg[..., None, :]


# ------------------------------------------------------------------------------------------------ steps vs dense rule
@pytest.mark.parametrize("kda,dims,glb,R", TRAJ_CASES)
@pytest.mark.parametrize("HV,H", [(2, 1), (2, 2), (4, 2)])
def test_step_trajectory_matches_dense_rule(kda, dims, glb, R, HV, H):
    """Evolve a dense float64 state with the textbook rule beside the oracle's checkpoint + window representation
    (no flush: L = 64 > steps); the materialised oracle state and the outputs must track it."""
    K, V = dims
    rng = np.random.default_rng(11 + HV + 10 * H + 100 * kda + K + V + R)
    NS, L = 3, 64
    st, _, Q0 = make_state(rng, NS, HV, H, K=K, V=V, L=L, R=R, kda=kda)
    idx = np.array([2, 1, 0])
    A_log, dt_bias = gate_params(HV, K, kda)
    A_log[:] = rng.uniform(-1.0, 0.5, HV)               # exercise A_log / dt_bias too
    dt_bias[:] = rng.uniform(-0.5, 0.5, dt_bias.shape)
    scale = K ** -0.5
    Sdrift = O.materialize(st)                          # evolved densely from the checkpoint, never re-synced
    for t in range(20):
        mixed, a, b = make_inputs(rng, 3, HV, H, K, V, kda=kda)
        rows = idx > 0
        s = idx[rows]
        q, k, v = _qk_from_mixed(mixed[rows], H, HV, K, V)
        hk = np.arange(HV) // (HV // H)
        beta = O.beta_of(b[rows]).astype(np.float64)
        S = O.materialize(st)                           # the oracle's logical state before this step
        st_prev = O.copy_state(st)
        if kda:
            g, _ = O.kda_gate(a.reshape(3, HV, K)[rows], dt_bias, A_log, glb)
            S1, od, u, kh = O.dense_kda_step(S[s], q[:, hk], k[:, hk], v, g, beta, scale)
            Sdrift[s] = O.dense_kda_step(Sdrift[s], q[:, hk], k[:, hk], v, g, beta, scale)[0]
            o = O.kda_step(st, mixed, a, b, A_log, dt_bias, idx, glb=glb)
        else:
            alpha = O.gdn_alpha(a[rows], dt_bias, A_log).astype(np.float64)
            S1, od, u, kh = O.dense_gdn_step(S[s], q[:, hk], k[:, hk], v, alpha, beta, scale)
            Sdrift[s] = O.dense_gdn_step(Sdrift[s], q[:, hk], k[:, hk], v, alpha, beta, scale)[0]
            o = O.gdn_step(st, mixed, a, b, A_log, dt_bias, idx)
        assert np.all(o[~rows] == 0)
        # output: bf16 of the dense rule's output on the same logical state (1 bf16 ulp + fp32 noise); KDA also
        # stages its decayed buffer keys in bf16 (kernels.py:977-978): bound |d o| by 2^-9 of those terms
        atol_o = np.full(od.shape, 1e-7)
        tol = 2 ** -7 * np.abs(u).max() * np.abs(kh).max() + 1e-7
        if kda:
            qh = q[:, hk] * scale / np.sqrt((q[:, hk] ** 2).sum(-1, keepdims=True) + 1e-6)
            h = st_prev_h = st["hcnt"][s] - 1
            Lr = np.arange(L)[None, None, :] < h[:, :, None]
            E_ = np.where(Lr[..., None], st["Gbuf"][s].astype(np.float64), 1.0)
            Dd = np.flip(np.cumprod(np.flip(E_, 2), 2), 2) / E_          # prod_{i>j} e_i, independently of the oracle
            KD = np.abs(st["Kbuf"][s][:, hk].astype(np.float64) * Dd) * Lr[..., None]
            wu = np.abs(st["Wbuf"][s][..., None] * st["Ubuf"][s])        # [n,HV,L,V]
            sens = np.einsum("nhjc,nhc->nhj", KD, np.abs(qh)) + np.einsum("nhjc,nhc->nhj", KD, np.abs(kh)) * 2
            atol_o = 2 ** -8 * np.einsum("nhjv,nhj->nhv", wu, sens) + 1e-7
            Sbuf = S[s] - O.checkpoint_f64(st_prev)[s] * np.exp(st_prev["Pbuf"][s])[:, :, None, :]
            tol = tol + 2 ** -10 * np.abs(Sbuf).max()
        assert np.all(np.abs(o[rows] - od) <= 2 ** -8 * np.abs(od) + atol_o)
        # new logical state: the dense rule's, except that the appended u, k (and KDA's decay e) are stored rounded
        Sm = O.materialize(st)
        assert np.abs(Sm[s] - S1).max() < tol, (t, np.abs(Sm[s] - S1).max(), tol)
        # accumulated drift against the never re-synced dense evolution stays at the bf16 storage level
        assert np.abs(Sm[s] - Sdrift[s]).max() < (t + 1) * tol
    assert np.all(st["hcnt"][[1, 2]] == 20) and np.all(st["hcnt"][0] == 0)


@pytest.mark.parametrize("glb", [0.0, -5.0, -0.5])
def test_kda_gate_closed_forms(glb):
    """The per-channel log-decay against closed forms written independently (kernels.py:702-712): GLM's bounded gate
    glb sigmoid(e^A_log x) through scipy's expit, in [glb, 0] and decreasing in x for glb < 0; Kimi's -e^A_log softplus(x)
    through log1p, linear above the softplus threshold 20."""
    rng = np.random.default_rng(31)
    HV, Kc = 3, 16
    a = O.bf16(rng.uniform(-30.0, 30.0, (5, HV, Kc)))
    dt = rng.uniform(-0.5, 0.5, (HV, Kc)).astype(np.float32)
    A_log = rng.uniform(-1.0, 1.0, HV).astype(np.float32)
    g, en = O.kda_gate(a, dt, A_log, glb)
    x = (a.astype(np.float32) + dt).astype(np.float64)                 # the fp32 sum, as the kernels form it
    ea = np.exp(A_log.astype(np.float64))[:, None]
    if glb != 0.0:
        from scipy.special import expit                                # library logistic, not the oracle's form
        ref = glb * expit(ea * x)
        assert np.all(g <= 0.0) and np.all(g >= glb)
        order = np.argsort(x[:, 0, 0])
        assert np.all(np.diff(g[order, 0, 0]) <= 0)                   # larger x: a log-decay closer to glb
    else:
        ref = np.where(x <= 20.0, -ea * np.log1p(np.exp(np.minimum(x, 20.0))), -ea * x)
    np.testing.assert_allclose(g, ref, rtol=1e-12, atol=1e-300)
    np.testing.assert_allclose(en.astype(np.float64), np.exp(ref), rtol=2 ** -23)


def test_step_special_cases_gdn():
    rng = np.random.default_rng(3)
    HV = H = 2
    st, _, Q0 = make_state(rng, 3, HV, H, L=16)
    A_log, dt_bias = gate_params(HV)
    mixed, a, b = make_inputs(rng, 2, HV, H)
    idx = np.array([1, 0])
    q, k, v = _qk_from_mixed(mixed, H, HV)
    # beta -> 0 (b = -60) and alpha -> 1 (a = -60): the state is unchanged and o = S q_hat
    b0 = np.full_like(b, -60.0)
    a1 = np.full_like(a, -60.0)
    S_before = O.materialize(st)
    st0 = O.copy_state(st)
    o = O.gdn_step(st0, mixed, a1, b0, A_log, dt_bias, idx)
    qh = q[0] * K ** -0.5 / np.sqrt((q[0] ** 2).sum(-1, keepdims=True) + 1e-6)
    expect = np.einsum("hvc,hc->hv", S_before[1], qh)
    np.testing.assert_allclose(o[0], expect, rtol=2 ** -7, atol=1e-6)
    np.testing.assert_allclose(O.materialize(st0)[1], S_before[1], atol=1e-9)
    assert np.all(o[1] == 0)
    # padding row: nothing written anywhere
    for key in ("Sq", "Sk", "Sv", "UQ", "Kbuf", "Ubuf", "Wbuf", "Pbuf", "hcnt"):
        np.testing.assert_array_equal(st0[key][2], st[key][2])
    # zero state: o = kappa beta v
    stz = O.new_state(3, HV, H, L=16)
    o = O.gdn_step(stz, mixed, a, b, A_log, dt_bias, idx)
    kh = k[0] / np.sqrt((k[0] ** 2).sum(-1, keepdims=True) + 1e-6)
    qh = q[0] * K ** -0.5 / np.sqrt((q[0] ** 2).sum(-1, keepdims=True) + 1e-6)
    kappa = (kh * qh).sum(-1)
    beta = O.beta_of(b[0]).astype(np.float64)
    np.testing.assert_allclose(o[0], kappa[:, None] * beta[:, None] * v[0], rtol=2 ** -7, atol=1e-6)


@pytest.mark.parametrize("kda", [False, True])
def test_6bit_steps_and_flush_match_dense_rule(kda):
    """A 6-bit checkpoint (codes in [-31, 31], dequantised as Sq Sk Sv / 31) stepped through a window and flushed: the
    outputs and the new logical state follow the dense float64 rule on the materialised 6-bit state, and the flush keeps
    that state within the 6-bit quantisation bound.  Stepping the same state with the INT8 convention (1 / 127) misses the
    dense rule by far more than the bar (the planted mistake this pin exists to catch)."""
    qmax, L, HV, H = 31.0, 16, 2, (2 if kda else 1)
    rng = np.random.default_rng(61 + kda)
    st, _, Q0 = make_state(rng, 3, HV, H, L=L, kda=kda, qmax=qmax)
    assert np.abs(st["Sq"][1:].astype(np.int32)).max() == 31
    A_log, dt_bias = gate_params(HV, K, kda)
    idx = np.array([2, 1, 0])
    hk = np.arange(HV) // (HV // H)
    step = O.kda_step if kda else O.gdn_step
    for t in range(L):
        mixed, a, b = make_inputs(rng, 3, HV, H, kda=kda)
        rows = idx > 0
        s = idx[rows]
        q, k, v = _qk_from_mixed(mixed[rows], H, HV)
        beta = O.beta_of(b[rows]).astype(np.float64)
        S = O.materialize(st, qmax)
        if t == 0:                                       # the planted mistake: the same state read with 1 / 127
            wrong = O.copy_state(st)
            o_wrong = step(wrong, mixed, a, b, A_log, dt_bias, idx)
        if kda:
            g, _ = O.kda_gate(a.reshape(3, HV, K)[rows], dt_bias, A_log, 0.0)
            S1, od, u, kh = O.dense_kda_step(S[s], q[:, hk], k[:, hk], v, g, beta, K ** -0.5)
        else:
            alpha = O.gdn_alpha(a[rows], dt_bias, A_log).astype(np.float64)
            S1, od, u, kh = O.dense_gdn_step(S[s], q[:, hk], k[:, hk], v, alpha, beta, K ** -0.5)
        o = step(st, mixed, a, b, A_log, dt_bias, idx, qmax=qmax)
        scale_o = np.abs(od).max()
        assert np.abs(o[rows] - od).max() <= 2e-2 * scale_o, (t, np.abs(o[rows] - od).max() / scale_o)
        if t == 0:
            assert np.abs(o_wrong[rows] - od).max() > 0.2 * scale_o
        Sm = O.materialize(st, qmax)
        tol = 2 ** -7 * np.abs(u).max() * np.abs(kh).max() + 2 ** -10 * np.abs(S1).max()
        assert np.abs(Sm[s] - S1).max() < tol, (t, np.abs(Sm[s] - S1).max(), tol)
    assert np.all(st["hcnt"][1:] == L)
    S_before = O.materialize(st, qmax)
    O.flush(st, Q0, idx, qmax=qmax)
    codes = st["Sq"][1:].astype(np.int32)
    assert np.abs(codes).max() <= 31 and np.all(np.abs(codes).max(-1) == 31)
    sk = st["Sk"][1:].astype(np.float64)[:, :, None, :]
    sv = st["Sv"][1:].astype(np.float64)[:, :, :, None]
    bound = 0.5 * sk * sv / qmax + 2 ** -9 * np.abs(S_before[1:]).max()
    assert np.all(np.abs(O.materialize(st, qmax)[1:] - S_before[1:]) <= bound)


def test_flush_of_a_rank_deficient_state():
    """A state of rank 2 (empty checkpoint, a window whose 16 keys take two directions) takes CholeskyQR2's relative
    pivot floor (kernels.py:1816-1825) on factors 3 and 4: the floor must keep every output finite, the first two
    factors must span the state's columns (sign-fixed numpy QR of S S^T Q0), and the logical state must survive the
    flush within its quantisation bound."""
    st, Q0, S = _rank2_state()
    # the floor is live: the third and fourth pivots of the Gram of S S^T Q0 vanish next to the diagonal
    X = S @ (S.T @ O.fp16(Q0).astype(np.float64))
    Gm = X.T @ X
    Lc = np.linalg.cholesky(Gm[:2, :2])
    d2 = Gm[2, 2] - np.sum(np.linalg.solve(Lc, Gm[:2, 2]) ** 2)
    assert d2 < 1e-6 * Gm[2, 2]
    dbg = O.flush(st, Q0, np.array([1]), return_debug=True)
    assert len(dbg["pairs"]) == 1
    for key in ("Sq", "Sk", "Sv", "UQ"):
        assert np.all(np.isfinite(st[key][1].astype(np.float64))), key
    Qref = _sign_fixed_qr(X)[:, :2]
    assert np.abs(dbg["Q16"][0][:, :2] - Qref).max() < 2e-3
    after = O.materialize(st)[1, 0]
    sk, sv = st["Sk"][1, 0].astype(np.float64), st["Sv"][1, 0].astype(np.float64)
    bound = 0.5 * sk[None, :] * sv[:, None] / 127.0 + 2 ** -9 * np.abs(S).max()
    assert np.all(np.abs(after - S) <= bound)


def test_cholqr_drop_rule_against_qr():
    """The R = 8 CholeskyQR (kernels.py:1744-1772), two passes: a full-rank block ends as numpy's QR with a positive
    diagonal; a block whose columns 3 and 6 repeat earlier directions ends with exactly those columns zero and the
    others equal to the QR of the independent columns (the R <= 4 rule would floor the pivot instead)."""
    rng = np.random.default_rng(3)
    X = rng.standard_normal((2, 128, 8))
    X[1, :, 3] = X[1, :, 0] - 2 * X[1, :, 1]
    X[1, :, 6] = 0.5 * X[1, :, 2]
    Y = O.cholqr_pass(O.cholqr_pass(X))
    assert np.abs(Y[0] - _sign_fixed_qr(X[0])).max() < 1e-10
    keep = [0, 1, 2, 4, 5, 7]
    assert np.all(Y[1][:, [3, 6]] == 0.0)
    assert np.abs(Y[1][:, keep] - _sign_fixed_qr(X[1][:, keep])).max() < 1e-8
    # the floor of the R <= 4 pass keeps a dependent column alive (scaled noise) instead of dropping it
    Z = X[1][:, :4]
    assert np.any(O.cholqr_pass(Z[None])[0][:, 3] != 0.0)


def test_flush_r8_code_sensitivity():
    """Sets the R = 8 flush's GPU code bar (0.5 %).  A change of ONE fp16 ulp in one entry of each head's rebuilt B --
    the size by which two correct fp32 window rebuilds differ -- moves > 0.1 % of the R = 8 codes (by one LSB each), but
    well under 0.1 % at R = 4: the fp16 rounding of Q after an orthogonalisation with condition numbers of 10-20 turns
    differences of ~1e-6 into rounding flips of whole factor columns."""
    def bump(B):
        B = B.copy()
        for d in range(B.shape[0]):
            B[d, 3, 5] = float(np.nextafter(np.float16(B[d, 3, 5]), np.float16(np.inf)))
        return B
    moved = {}
    for R in (4, 8):
        st, Q0 = due_flush_case(np.random.default_rng(864), 64, R=R)
        a, b = O.copy_state(st), O.copy_state(st)
        idx = np.array([1, 3])
        O.flush(a, Q0, idx)
        O.flush(b, Q0, idx, b_hook=bump)
        d = np.abs(a["Sq"][[1, 3]].astype(np.int32) - b["Sq"][[1, 3]].astype(np.int32))
        assert d.max() == 1
        moved[R] = (d > 0).mean()
    assert moved[8] > 1e-3 > moved[4], moved


def test_flush_head_dim_code_sensitivity():
    """Sets the K = 64 flush's GPU code bar (0.25 %): at (64, 128), GQA 1, W = 16 one fp16 ulp in one entry of each
    head's rebuilt B moves more than 0.1 % of the codes (by one LSB each) -- a head of 8192 codes, and each factor
    rounding flip shifts a row or column of its residual -- while at 128 x 128 on the same window it moves 0.01 %."""
    def bump(B):
        B = B.copy()
        for d in range(B.shape[0]):
            B[d, 3, 5] = float(np.nextafter(np.float16(B[d, 3, 5]), np.float16(np.inf)))
        return B
    moved = {}
    for K, V in ((64, 128), (128, 128)):
        rng = np.random.default_rng(1300 + K + V + 16 + 7)
        NS, HV, H, L = 6, 4, 4, 16
        st, _, Q0 = make_state(rng, NS, HV, H, K=K, V=V, L=L)
        A_log, dt_bias = gate_params(HV, K)
        for _ in range(L + 5):
            sl = rng.permutation(np.arange(1, NS))[: rng.integers(1, NS)]
            mixed, a, b = make_inputs(rng, len(sl), HV, H, K, V)
            O.gdn_step(st, mixed, a, b, A_log, dt_bias, sl)
            O.flush(st, Q0, sl)
        for s in (1, 3):
            while st["hcnt"][s, 0] < L:
                mixed, a, b = make_inputs(rng, 1, HV, H, K, V)
                O.gdn_step(st, mixed, a, b, A_log, dt_bias, np.array([s]))
        x, y = O.copy_state(st), O.copy_state(st)
        O.flush(x, Q0, np.array([1, 3]))
        O.flush(y, Q0, np.array([1, 3]), b_hook=bump)
        d = np.abs(x["Sq"][[1, 3]].astype(np.int32) - y["Sq"][[1, 3]].astype(np.int32))
        assert d.max() <= 1
        moved[(K, V)] = (d > 0).mean()
    assert moved[(64, 128)] > 1e-3 > moved[(128, 128)], moved


def test_flush_r8_of_a_rank_deficient_state():
    """R = 8 on the rank-2 state: CholeskyQR drops factors 3..8 (their pivots vanish), so those Q and U columns are
    exactly zero, the first two span the state's columns, and the logical state survives within its bound."""
    st, Q0, S = _rank2_state(R=8)
    dbg = O.flush(st, Q0, np.array([1]), return_debug=True)
    for key in ("Sq", "Sk", "Sv", "UQ"):
        assert np.all(np.isfinite(st[key][1].astype(np.float64))), key
    assert np.all(dbg["Q16"][0][:, 2:] == 0.0) and np.all(dbg["U16"][0][:, 2:] == 0.0)
    X = S @ (S.T @ O.fp16(Q0).astype(np.float64))
    assert np.abs(dbg["Q16"][0][:, :2] - _sign_fixed_qr(X)[:, :2]).max() < 2e-3
    after = O.materialize(st)[1, 0]
    sk, sv = st["Sk"][1, 0].astype(np.float64), st["Sv"][1, 0].astype(np.float64)
    bound = 0.5 * sk[None, :] * sv[:, None] / 127.0 + 2 ** -9 * np.abs(S).max()
    assert np.all(np.abs(after - S) <= bound)


def _rank2_state(L=16, seed=71, R=4):
    """(state, Q0, S): slot 1, head 0 holds the rank-2 logical state S = sum_j w_j u_j k_j^T with k_j in {ka, kb}, an
    all-zero checkpoint and a full window (hcnt = L), so the next flush takes it."""
    rng = np.random.default_rng(seed)
    st = O.new_state(2, 1, 1, L=L, R=R)
    Q0 = O.make_q0(128, R)
    st["Sk"][:] = 1.0
    st["Sv"][:] = 1.0
    kk = rng.standard_normal((2, 128))
    kk /= np.linalg.norm(kk, axis=-1, keepdims=True)
    sel = np.arange(L) % 2
    st["Kbuf"][1, 0] = O.bf16(kk[sel])
    st["Ubuf"][1, 0] = O.bf16(0.3 * rng.standard_normal((L, 128)))
    st["Wbuf"][1, 0] = np.exp(-0.05 * np.arange(L)[::-1]).astype(np.float32)
    st["hcnt"][1, 0] = L
    S = O.materialize(st)[1, 0]
    assert np.linalg.matrix_rank(S, tol=1e-9 * np.abs(S).max()) == 2
    return st, Q0, S


# ------------------------------------------------------------------------------------------------ flush
@pytest.mark.parametrize("kda,dims,R", FLUSH_CASES)
@pytest.mark.parametrize("L", [16, 64])
def test_flush_against_qr_and_bounds(kda, dims, R, L):
    K, V = dims
    rng = np.random.default_rng(5 + L + 7 * kda + K + V + R)
    HV, H = 2, (2 if kda else 1)
    st, _, Q0 = make_state(rng, 3, HV, H, K=K, V=V, L=L, R=R, kda=kda)
    A_log, dt_bias = gate_params(HV, K, kda)
    idx = np.array([1, 2])
    for t in range(L):
        mixed, a, b = make_inputs(rng, 2, HV, H, K, V, kda=kda)
        (O.kda_step if kda else O.gdn_step)(st, mixed, a, b, A_log, dt_bias, idx)
    assert np.all(st["hcnt"][1:] == L)
    S_before = O.materialize(st)
    dbg = O.flush(st, Q0, idx, return_debug=True)
    assert len(dbg["pairs"]) == 2 * HV
    assert np.all(st["hcnt"] == 0) and np.all(st["Wbuf"] == 0)
    assert np.all(st["Pbuf"] == (0.0 if kda else 1.0))
    if kda:
        assert np.all(st["Gbuf"] == 1.0)
    S_after = O.materialize(st)
    for i, (sl, hv) in enumerate(dbg["pairs"]):
        S = S_before[sl, hv]
        # Q: one subspace-iteration step from Q0 orthonormalised == QR(S S^T Q0) with positive diagonal
        Q16q0 = O.fp16(Q0).astype(np.float64)
        Qref = _sign_fixed_qr(S @ (S.T @ Q16q0))
        Q16 = dbg["Q16"][i]
        assert np.abs(Q16 - Qref).max() < 2e-2, np.abs(Q16 - Qref).max()
        assert np.abs(Q16.T @ Q16 - np.eye(R)).max() < 4e-3
        # U = S^T Q (fp16)
        Uref = S.T @ Q16
        assert np.abs(dbg["U16"][i] - Uref).max() < 2e-3 * np.abs(Uref).max() + 1e-4
        # codes and scales
        codes = st["Sq"][sl, hv].astype(np.int32)
        assert np.abs(codes).max() <= 127
        E = S - Q16 @ dbg["U16"][i].T
        sk = st["Sk"][sl, hv].astype(np.float64)
        sv = st["Sv"][sl, hv].astype(np.float64)
        np.testing.assert_allclose(sk, np.sqrt(np.abs(E).mean(0)), rtol=3e-3)
        xs = E / sk[None, :]
        np.testing.assert_allclose(sv, np.abs(xs).max(1), rtol=3e-3)
        am = np.abs(xs).argmax(1)
        assert np.all(np.abs(codes[np.arange(V), am]) == 127)
        deq = codes * (sk[None, :] / 127.0) * sv[:, None]
        bound = 0.5 * sk[None, :] * sv[:, None] / 127.0 + 2 ** -10 * np.abs(S).max()
        assert np.all(np.abs(deq - E) <= bound)
        # the flush keeps the logical state up to that quantisation error
        assert np.all(np.abs(S_after[sl, hv] - S) <= bound + 2 ** -10 * np.abs(S).max())


def test_flush_fully_decayed_and_idle_heads():
    """A head whose window decayed to a denormal product keeps finite outputs (PNMIN floor); heads that are not due are
    untouched; slots <= 0 are skipped."""
    rng = np.random.default_rng(9)
    st, _, Q0 = make_state(rng, 3, 2, 1, L=16)
    A_log, dt_bias = gate_params(2)
    A_log[:] = 6.0                                   # exp(A_log) ~ 403: alpha ~ exp(-403 softplus) -> tiny
    idx = np.array([1, 0])
    for t in range(16):
        mixed, a, b = make_inputs(rng, 2, 2, 1)
        O.gdn_step(st, mixed, a, b, A_log, dt_bias, idx)
    assert st["Pbuf"][1, :, 0].max() < 1e-30
    snap = O.copy_state(st)
    O.flush(st, Q0, idx)
    for key in ("Sq", "Sk", "Sv", "UQ"):
        assert np.all(np.isfinite(st[key][1].astype(np.float64)))
        np.testing.assert_array_equal(st[key][2], snap[key][2])
    # a fully decayed state is (numerically) its window's last entry only
    S = O.materialize(snap)[1]
    assert np.abs(O.materialize(st)[1] - S).max() < 1e-2 * np.abs(S).max()


@pytest.mark.parametrize("kda", [False, True])
def test_flush_on_given_factors(kda):
    """flush(factors=...) -- the residual stage run on given fp16 factors, as the GPU tests run it on the GPU's --
    reproduces the flush bit for bit when handed the flush's own factors, and with factors nudged by one fp16 ulp in one
    entry the codes it gives differ (so the argument is used, not ignored)."""
    rng = np.random.default_rng(31 + kda)
    NS, HV, L = 4, 2, 16
    H = HV if kda else 1
    st, _, Q0 = make_state(rng, NS, HV, H, L=L, kda=kda)
    A_log, dt_bias = gate_params(HV, 128, kda)
    idx = np.array([1, 3])
    for _ in range(L):
        mixed, a, b = make_inputs(rng, len(idx), HV, H, kda=kda)
        (O.kda_step if kda else O.gdn_step)(st, mixed, a, b, A_log, dt_bias, idx)
    pre = O.copy_state(st)
    a_ = O.copy_state(pre)
    dbg = O.flush(a_, Q0, idx, return_debug=True)
    b_ = O.copy_state(pre)
    O.flush(b_, Q0, idx, factors=(dbg["U16"], dbg["Q16"]))
    for k in ("Sq", "Sk", "Sv", "UQ", "Wbuf", "Pbuf", "hcnt"):
        assert np.array_equal(a_[k], b_[k]), k
    U2 = dbg["U16"].copy()
    U2[0, 5, 0] = float(np.nextafter(np.float16(U2[0, 5, 0]), np.float16(np.inf)))
    c_ = O.copy_state(pre)
    O.flush(c_, Q0, idx, factors=(U2, dbg["Q16"]))
    assert not np.array_equal(c_["UQ"], a_["UQ"])


# ------------------------------------------------------------------------------------------------ quantize / lowrank
QUANT_CASES = [(q, h, d, 4) for q in (127.0, 31.0) for h in (False, True) for d in GDN_DIMS] + \
    [(127.0, False, (128, 128), 8), (127.0, True, (128, 128), 16)]          # ranks a step can read (kernels.py:63)


@pytest.mark.parametrize("qmax,heavy,dims,R", QUANT_CASES)
def test_quantize_against_qr_and_bounds(qmax, heavy, dims, R):
    K, V = dims
    rng = np.random.default_rng(21 + int(qmax) + heavy + K + V + R)
    D = 3
    S = (0.02 * (rng.standard_t(3, (D, V, K)) if heavy else rng.standard_normal((D, V, K)))).astype(np.float32)
    S[1] += np.outer(rng.standard_normal(V), rng.standard_normal(K)).astype(np.float32) * 0.05   # a dominant direction
    Q0 = O.make_q0(V, R)
    codes, sk, sv, UQ = O.quantize_dense(S, Q0, qmax=qmax)
    for d in range(D):
        S64 = S[d].astype(np.float64)
        P = _sign_fixed_qr(S64.T @ Q0)
        Qref = _sign_fixed_qr(S64 @ P)
        Q16 = UQ[d, :, K:].T.astype(np.float64)
        U16 = UQ[d, :, :K].T.astype(np.float64)
        assert np.abs(Q16 - Qref).max() < 2e-3
        assert np.abs(U16 - S64.T @ Q16).max() < 2e-3 * np.abs(U16).max() + 1e-5
        E = S64 - Q16 @ U16.T
        np.testing.assert_allclose(sk[d], np.sqrt(np.abs(E).mean(0)), rtol=1e-5)
        np.testing.assert_allclose(sv[d], (np.abs(E) / sk[d][None, :]).max(1), rtol=1e-5)
        c = codes[d].astype(np.int32)
        assert np.abs(c).max() <= qmax
        am = (np.abs(E) / sk[d][None, :]).argmax(1)
        assert np.all(np.abs(c[np.arange(V), am]) == qmax)
        deq = c * (sk[d][None, :].astype(np.float64) / qmax) * sv[d][:, None]
        assert np.all(np.abs(deq - E) <= 0.5 * sk[d][None, :] * sv[d][:, None] / qmax * (1 + 1e-5) + 1e-9)


def test_lowrank_against_qr_iteration():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, K, V)).astype(np.float32)
    x[0] += 3 * np.outer(rng.standard_normal(K), rng.standard_normal(V)).astype(np.float32)
    Q0 = O.make_q0(V, 4)
    U, Q = O.lowrank(x, Q0, iters=3)
    for d in range(3):
        xx = x[d].astype(np.float64)
        Qr = Q0.astype(np.float64)
        for _ in range(3):
            Pr = _sign_fixed_qr(xx @ Qr)
            Qr = _sign_fixed_qr(xx.T @ Pr)
        np.testing.assert_allclose(Q[d], Qr, atol=1e-5)
        np.testing.assert_allclose(U[d], xx @ Qr, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dims", GDN_DIMS)
def test_dequant_reproduces_logical_state_and_resets(dims):
    K, V = dims
    rng = np.random.default_rng(8 + K + V)
    st, S0, Q0 = make_state(rng, 3, 2, 1, K=K, V=V, L=16)
    # quantize -> dequant round trip of a fresh checkpoint stays within the quantisation bound of the fp32 source
    out = O.dequant(O.copy_state(st), [1, 2])
    for sl in (1, 2):
        for hv in range(2):
            sk = st["Sk"][sl, hv].astype(np.float64)
            sv = st["Sv"][sl, hv].astype(np.float64)
            bound = 0.5 * sk[None, :] * sv[:, None] / 127 * 1.01 + 2 ** -9 * np.abs(S0[sl, hv]).max()
            assert np.all(np.abs(out[sl][hv] - S0[sl, hv]) <= bound)
    # with a partial window: dequant == dense evolution (checked through the pinned materialisation)
    A_log, dt_bias = gate_params(2)
    for t in range(5):
        mixed, a, b = make_inputs(rng, 1, 2, 1, K, V)
        O.gdn_step(st, mixed, a, b, A_log, dt_bias, np.array([2]))
    Sm = O.materialize(st)
    out = O.dequant(st, [2])
    np.testing.assert_allclose(out[2], Sm[2], rtol=1e-5, atol=1e-7)
    assert np.all(st["hcnt"][2] == 0) and np.all(st["Wbuf"][2] == 0) and np.all(st["Pbuf"][2] == 1)


def test_kda_round_trip():
    rng = np.random.default_rng(10)
    st, S0, Q0 = make_state(rng, 3, 2, 2, L=16, kda=True)
    A_log, dt_bias = gate_params(2, K, True)
    for t in range(6):
        mixed, a, b = make_inputs(rng, 1, 2, 2, kda=True)
        O.kda_step(st, mixed, a, b, A_log, dt_bias, np.array([1]))
    Sreb = O.kda_rebuild(st, [1])
    O.kda_checkpoint(st, Sreb, [1], Q0)
    assert np.all(st["hcnt"][1] == 0) and np.all(st["Pbuf"][1] == 0) and np.all(st["Gbuf"][1] == 1)
    back = O.materialize(st)[1]
    for hv in range(2):
        sk = st["Sk"][1, hv].astype(np.float64)
        sv = st["Sv"][1, hv].astype(np.float64)
        bound = 0.5 * sk[None, :] * sv[:, None] / 127 * 1.01 + 2 ** -9 * np.abs(Sreb[1][hv]).max()
        assert np.all(np.abs(back[hv] - Sreb[1][hv]) <= bound)


# ------------------------------------------------------------------------------------------------ golden files
@pytest.mark.parametrize("name", ["oracle_gdn_L16", "oracle_gdn_L64", "oracle_kda_L16", "oracle_kda_L64"])
def test_golden_trajectories(name):
    z = from_bits(np.load(os.path.join(GOLD, name + ".npz")))
    NS, HV, H, K_, V_, L, R, kda = [int(x) for x in z["dims"]]
    st = state_from_npz(z, "init_")
    Q0 = O.make_q0(V_, R)
    for t in range(z["o"].shape[0]):
        step = O.kda_step if kda else O.gdn_step
        o = step(st, z["mixed"][t], z["a"][t], z["b"][t], z["A_log"], z["dt_bias"], z["idx"])
        O.flush(st, Q0, z["idx"])
        np.testing.assert_array_equal(o, z["o"][t])
    fin = state_from_npz(z, "final_")
    for key in ("Sq", "Sk", "Sv", "UQ", "Kbuf", "Ubuf", "Wbuf", "Pbuf", "hcnt"):
        np.testing.assert_array_equal(st[key], fin[key], err_msg=key)
