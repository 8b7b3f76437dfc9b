"""CPU oracle of LeapQuant's INT8 recurrent-state decode path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this module, and only as
the checker (or as the timed CPU baseline).  The product path (``leapquant_amd``) never calls it and fails loudly when
its HIP library is missing.

What it is: a numpy restatement of the reference's arithmetic for the GDN / KDA decode step, the end-of-window flush,
the standalone quantize, the prefill dequant, the KDA low-rank factoriser and the KDA torch round trip
(``/root/reference/leapquant/kernels.py`` and ``state.py``).  Every reduction is accumulated in float64 (the
reference accumulates in fp32 inside tensor-core MMAs whose order is not specified, so the exact sum is the
contract); every point where the reference *stores or converts* a value is rounded explicitly:

  * ``r32``  -- to fp32 (values the reference keeps in fp32 registers / buffers),
  * ``bf16`` -- to bfloat16, nearest-even, via fp32 (buffer appends, outputs, beta, the hi/lo MMA operand splits),
  * ``fp16`` -- to float16 via fp32 (factors U / Q, the flush's rebuilt state B and residual E, KDA entry decays).

Elementwise fp32 chains that feed a rounding point (the dequant products, the hi/lo splits, the Wbuf / Pbuf
updates, the quantisation scalings) are evaluated in float32 exactly as the reference orders them.

State representation (logical views, not the aliased bytes): a dict with
  Sq int8 [NS,HV,V,K], Sk f32 [NS,HV,K], Sv f32 [NS,HV,V], UQ f16 [NS,HV,R,K+V],
  Kbuf f32 (bf16 values) [NS,H,L,K]  -- buffered keys per KEY head (identical for the value heads sharing it),
  Ubuf f32 (bf16 values) [NS,HV,L,V], Wbuf f32 [NS,HV,L], Pbuf f32 [NS,HV,1] (GDN) or [NS,HV,K] (KDA),
  Gbuf f16 [NS,HV,L,K] (KDA only), hcnt int32 [NS,HV].

Pinning (tests/test_oracle_pins.py): the step against a dense float64 gated-delta / KDA rule on the materialised state,
the flush / quantize / lowrank against numpy QR-based subspace iteration, the scales and codes against their defining
bounds, special cases (empty window, alpha = 1, beta = 0, zero state, padding rows, fully decayed heads).
"""
import numpy as np

QMAX = 127.0
EPS = 1e-12                 # kernels.py:23
SOFTPLUS_THRESHOLD = 20.0   # kernels.py:21
PNMIN = 1e-20               # kernels.py:1078
NORM_EPS = 1e-6             # kernels.py:246-247

F32 = np.float32


# ----------------------------------------------------------------------------------------------------------------
# rounding helpers
# ----------------------------------------------------------------------------------------------------------------
def r32(x):
    """Round to fp32 (returned as float32)."""
    return np.asarray(x, dtype=np.float64).astype(np.float32)


def bf16(x):
    """Round to bfloat16, nearest-even, via fp32; returned as float32 holding the bf16 value."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float64).astype(np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16) & 0xFFFFFFFF
    out = r.astype(np.uint32).view(np.float32).reshape(a.shape)
    return np.where(np.isnan(a), a, out)


def fp16(x):
    """Round to float16 via fp32; returned as float16."""
    return np.asarray(x, dtype=np.float64).astype(np.float32).astype(np.float16)


def rsqrt32(x):
    return r32(1.0 / np.sqrt(np.asarray(x, dtype=np.float64)))


# ----------------------------------------------------------------------------------------------------------------
# state construction
# ----------------------------------------------------------------------------------------------------------------
def new_state(NS, HV, H, K=128, V=128, L=16, R=4, kda=False):
    """Window buffers as LeapQuantState.__init__ allocates them (state.py:61-70); the checkpoint views start at zero."""
    return dict(
        Sq=np.zeros((NS, HV, V, K), np.int8), Sk=np.zeros((NS, HV, K), F32), Sv=np.zeros((NS, HV, V), F32),
        UQ=np.zeros((NS, HV, R, K + V), np.float16),
        Kbuf=np.zeros((NS, H, L, K), F32), Ubuf=np.zeros((NS, HV, L, V), F32), Wbuf=np.zeros((NS, HV, L), F32),
        Pbuf=(np.zeros((NS, HV, K), F32) if kda else np.ones((NS, HV, 1), F32)),
        Gbuf=(np.ones((NS, HV, L, K), np.float16) if kda else None),
        hcnt=np.zeros((NS, HV), np.int32), kda=kda)


def copy_state(st):
    return {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in st.items()}


def make_q0(V, R):
    """The subspace iteration's fixed start: torch.randn(V, R, generator=Generator().manual_seed(0)) (state.py:70).
    Kept as a committed fixture (tests/golden/q0_128x4.npy) so the oracle needs no torch."""
    import os
    p = os.path.join(os.path.dirname(__file__), "..", "tests", "golden", "q0_%dx%d.npy" % (V, R))
    return np.load(p).astype(F32)


def _dims(st):
    NS, HV, V, K = st["Sq"].shape
    H = st["Kbuf"].shape[1]
    L = st["Wbuf"].shape[-1]
    R = st["UQ"].shape[2]
    return NS, HV, H, K, V, L, R


# ----------------------------------------------------------------------------------------------------------------
# logical state (float64) -- used by the pins and by the dequant / KDA rebuild semantics
# ----------------------------------------------------------------------------------------------------------------
def checkpoint_f64(st, qmax=QMAX):
    """S0 = Q U^T + deq(Sq) per (slot, head): [NS,HV,V,K] float64 (state.py:121-122)."""
    K = st["Sq"].shape[-1]
    UT = st["UQ"][..., :K].astype(np.float64)
    QT = st["UQ"][..., K:].astype(np.float64)
    deq = st["Sq"].astype(np.float64) * (st["Sk"].astype(np.float64)[:, :, None, :] / qmax) \
        * st["Sv"].astype(np.float64)[:, :, :, None]
    return np.einsum("shrv,shrc->shvc", QT, UT) + deq


def kda_decays(st):
    """D_j = prod_{j<i<h} e_i (entries j >= h masked to factor 1), [NS,HV,L,K] float64 (state.py:124-125)."""
    E = st["Gbuf"].astype(np.float64)
    L = E.shape[2]
    h = st["hcnt"]
    live = np.arange(L)[None, None, :, None] < h[:, :, None, None]
    E = np.where(live, E, 1.0)
    D = np.ones_like(E)
    for j in range(L - 2, -1, -1):
        D[:, :, j] = D[:, :, j + 1] * E[:, :, j + 1]
    return D


def materialize(st, qmax=QMAX):
    """The full logical state S per (slot, head) in float64.
    GDN: S = P S0 + sum_{j<h} w_j u_j k_j^T.   KDA: S = S0 diag(exp(P)) + sum_{j<h} w_j u_j (k_j * D_j)^T."""
    NS, HV, H, K, V, L, R = _dims(st)
    G = HV // H
    S0 = checkpoint_f64(st, qmax)
    h = st["hcnt"]
    live = (np.arange(L)[None, None, :] < h[:, :, None]).astype(np.float64)
    w = st["Wbuf"].astype(np.float64) * live
    Kb = np.repeat(st["Kbuf"].astype(np.float64), G, axis=1)
    Ub = st["Ubuf"].astype(np.float64)
    if st["kda"]:
        Kb = Kb * kda_decays(st)
        return S0 * np.exp(st["Pbuf"].astype(np.float64))[:, :, None, :] + np.einsum("shj,shjv,shjc->shvc", w, Ub, Kb)
    return S0 * st["Pbuf"].astype(np.float64)[:, :, :, None] + np.einsum("shj,shjv,shjc->shvc", w, Ub, Kb)


# ----------------------------------------------------------------------------------------------------------------
# gates and normalisation (shared by GDN and KDA steps)
# ----------------------------------------------------------------------------------------------------------------
def softplus64(x):
    x = np.asarray(x, np.float64)
    return np.where(x <= SOFTPLUS_THRESHOLD, np.log1p(np.exp(np.minimum(x, SOFTPLUS_THRESHOLD))), x)


def gdn_alpha(a, dt_bias, A_log):
    """alpha = exp(-exp(A_log) softplus_20(f32(a) + dt_bias))  (kernels.py:141-143).  a: [..., HV]."""
    xg = (np.asarray(a, F32) + np.asarray(dt_bias, F32)).astype(np.float64)
    return r32(np.exp(-np.exp(np.asarray(A_log, F32).astype(np.float64)) * softplus64(xg)))


def beta_of(b):
    """beta = f32(bf16(sigmoid(f32(b))))  (kernels.py:144)."""
    return bf16(r32(1.0 / (1.0 + np.exp(-np.asarray(b, F32).astype(np.float64)))))


def normalize_qk(q, k, scale):
    """kn = k / sqrt(sum k^2 + 1e-6), qn = q scale / sqrt(sum q^2 + 1e-6), kappa = kn . qn  (kernels.py:236-254,277).
    q, k: bf16 values [..., K] -> kn, qn fp32, kappa float64."""
    q64 = np.asarray(q, np.float64)
    k64 = np.asarray(k, np.float64)
    nq = (q64 * q64).sum(-1)
    nk = (k64 * k64).sum(-1)
    nkq = (k64 * q64).sum(-1)
    ink = rsqrt32(nk + NORM_EPS)
    inq = r32(rsqrt32(nq + NORM_EPS) * F32(scale))
    kn = r32(np.asarray(k, F32) * ink[..., None])
    qn = r32(np.asarray(q, F32) * inq[..., None])
    kappa = nkq * inq.astype(np.float64) * ink.astype(np.float64)
    return kn, qn, kappa


def _split_mixed(mixed, H, HV, K, V):
    m = np.asarray(mixed, F32)
    q = m[:, :H * K].reshape(-1, H, K)
    k = m[:, H * K:2 * H * K].reshape(-1, H, K)
    v = m[:, 2 * H * K:2 * H * K + HV * V].reshape(-1, HV, V)
    return q, k, v


# ----------------------------------------------------------------------------------------------------------------
# GDN decode step  (kernels.py:27-692, HP = 1 path 129-144, 236-279, 380-585)
# ----------------------------------------------------------------------------------------------------------------
def gdn_step(st, mixed, a, b, A_log, dt_bias, idx, scale=None, qmax=QMAX):
    """One GDN decode token per row n (in place on st); returns o [N,HV,V] (bf16 values as float32).
    mixed: bf16 [N, 2HK + HV V]; a, b: bf16 [N,HV]; A_log, dt_bias: [HV]; idx: int [N] (slot <= 0: padding row)."""
    NS, HV, H, K, V, L, R = _dims(st)
    G = HV // H
    scale = K ** -0.5 if scale is None else scale
    idx = np.asarray(idx).astype(np.int64)
    N = idx.shape[0]
    o = np.zeros((N, HV, V), F32)
    rows = np.nonzero(idx > 0)[0]
    if rows.size == 0:
        return o
    s = idx[rows]
    hk = np.arange(HV) // G
    alpha = gdn_alpha(np.asarray(a, F32).reshape(N, HV)[rows], np.asarray(dt_bias, F32).reshape(HV),
                      np.asarray(A_log, F32).reshape(HV))                                     # [n,HV]
    beta = beta_of(np.asarray(b, F32).reshape(N, HV)[rows]).astype(np.float64)
    q, k, v = _split_mixed(np.asarray(mixed)[rows], H, HV, K, V)
    kn, qn, kappa = normalize_qk(q, k, scale)                                                   # [n,H,K], [n,H]
    knv, qnv, kap = kn[:, hk], qn[:, hk], kappa[:, hk]                                           # per value head
    Sq = st["Sq"][s].astype(np.float64)
    Sk = st["Sk"][s]
    Sv = st["Sv"][s].astype(np.float64)
    inv = F32(1.0 / qmax)
    kf = r32(r32(knv * Sk) * inv).astype(np.float64)                                            # kernels.py:255
    qf = r32(r32(qnv * Sk) * inv).astype(np.float64)                                            # kernels.py:256
    m = np.einsum("nhvc,nhc->nhv", Sq, kf) * Sv
    yq = np.einsum("nhvc,nhc->nhv", Sq, qf) * Sv
    h = st["hcnt"][s]                                                                             # [n,HV]
    P = st["Pbuf"][s][..., 0]
    Wb = st["Wbuf"][s]
    live = np.arange(L)[None, None, :] < h[:, :, None]
    w = np.where(live, r32(Wb * alpha[:, :, None]), Wb)                                         # kernels.py:270-274
    Kb = st["Kbuf"][s][:, hk].astype(np.float64)                                                # [n,HV,L,K]
    Ub = st["Ubuf"][s].astype(np.float64)
    dk = np.einsum("nhjc,nhc->nhj", Kb, knv.astype(np.float64))
    dq = np.einsum("nhjc,nhc->nhj", Kb, qnv.astype(np.float64))
    A4 = np.einsum("nhjv,nhj->nhv", Ub, w * dk)
    A5 = np.einsum("nhjv,nhj->nhv", Ub, w * dq)
    UT = st["UQ"][s][..., :K].astype(np.float64)
    QT = st["UQ"][s][..., K:].astype(np.float64)
    dU = np.einsum("nhrc,nhc->nhr", UT, knv.astype(np.float64))
    dQ = np.einsum("nhrc,nhc->nhr", UT, qnv.astype(np.float64))
    A6 = np.einsum("nhrv,nhr->nhv", QT, dU)
    A7 = np.einsum("nhrv,nhr->nhv", QT, dQ)
    pn = r32(P * alpha)                                                                          # kernels.py:278
    pn64 = pn.astype(np.float64)[:, :, None]
    u = beta[:, :, None] * (v - (pn64 * (m + A6) + A4))                                          # kernels.py:573
    y = pn64 * (yq + A7) + A5 + kap[:, :, None] * u                                              # kernels.py:574
    o[rows] = bf16(y)
    # state writes (kernels.py:575-585)
    hv_ix = np.arange(HV)[None, :]
    st["Wbuf"][s] = w
    st["Wbuf"][s[:, None], hv_ix, h] = 1.0
    st["Ubuf"][s[:, None], hv_ix, h] = bf16(u)
    st["Kbuf"][s[:, None], np.arange(H)[None, :], h[:, ::G]] = bf16(kn)
    st["Pbuf"][s, :, 0] = pn
    st["hcnt"][s] = h + 1
    return o


# ----------------------------------------------------------------------------------------------------------------
# KDA decode step  (kernels.py:694-1075)
# ----------------------------------------------------------------------------------------------------------------
def kda_gate(a, dt_bias, A_log, glb):
    """Per-channel log-decay g and its exponential (kernels.py:704-712, 802, 887-893).
    a: [..., HV, K]; dt_bias: [HV, K]; A_log: [HV].  Returns (g float64, en = exp(g) fp32)."""
    xg = (np.asarray(a, F32) + np.asarray(dt_bias, F32)).astype(np.float64)
    ea = np.exp(np.asarray(A_log, F32).astype(np.float64))[:, None]
    if glb != 0.0:
        g = glb / (1.0 + np.exp(-ea * xg))
    else:
        g = -ea * softplus64(xg)
    return g, r32(np.exp(g))


def kda_step(st, mixed, a, b, A_log, dt_bias, idx, glb=0.0, scale=None, qmax=QMAX):
    """One KDA decode token per row (in place); returns o [N,HV,V].  a: bf16 [N,HV,K]; dt_bias: [HV,K]."""
    NS, HV, H, K, V, L, R = _dims(st)
    G = HV // H
    scale = K ** -0.5 if scale is None else scale
    idx = np.asarray(idx).astype(np.int64)
    N = idx.shape[0]
    o = np.zeros((N, HV, V), F32)
    rows = np.nonzero(idx > 0)[0]
    if rows.size == 0:
        return o
    s = idx[rows]
    hk = np.arange(HV) // G
    g, en = kda_gate(np.asarray(a, F32).reshape(N, HV, K)[rows], np.asarray(dt_bias, F32).reshape(HV, K),
                     np.asarray(A_log, F32).reshape(HV), glb)                                   # [n,HV,K]
    beta = beta_of(np.asarray(b, F32).reshape(N, HV)[rows]).astype(np.float64)
    q, k, v = _split_mixed(np.asarray(mixed)[rows], H, HV, K, V)
    kn, qn, kappa = normalize_qk(q, k, scale)
    knv, qnv, kap = kn[:, hk], qn[:, hk], kappa[:, hk]
    pb = st["Pbuf"][s]                                                                           # [n,HV,K]
    gn = r32(pb.astype(np.float64) + g)                                                          # kernels.py:889
    pc = r32(np.exp(gn.astype(np.float64)))                                                      # kernels.py:890
    Sq = st["Sq"][s].astype(np.float64)
    Sk = st["Sk"][s]
    Sv = st["Sv"][s].astype(np.float64)
    inv = F32(1.0 / qmax)
    kf = r32(r32(r32(knv * Sk) * inv) * pc).astype(np.float64)                                  # kernels.py:900
    qf = r32(r32(r32(qnv * Sk) * inv) * pc).astype(np.float64)                                  # kernels.py:901
    m = np.einsum("nhvc,nhc->nhv", Sq, kf) * Sv
    yq = np.einsum("nhvc,nhc->nhv", Sq, qf) * Sv
    h = st["hcnt"][s]
    live = np.arange(L)[None, None, :] < h[:, :, None]
    # decayed keys K~_j = bf16(K_j * en * prod_{j<i<h} e_i), entries j >= h zero (kernels.py:966-979)
    e = st["Gbuf"][s].astype(F32)                                                                # [n,HV,L,K]
    Kb = st["Kbuf"][s][:, hk]                                                                    # [n,HV,L,K] f32
    Kt = np.zeros_like(Kb)
    dcur = en.copy()
    for j in range(L - 1, -1, -1):
        Kt[:, :, j] = bf16(Kb[:, :, j] * np.where(live[:, :, j, None], dcur, F32(0.0)))
        dcur = r32(dcur * e[:, :, j])
    w = st["Wbuf"][s].astype(np.float64)
    Ub = st["Ubuf"][s].astype(np.float64)
    dk = np.einsum("nhjc,nhc->nhj", Kt.astype(np.float64), knv.astype(np.float64)) * w          # kernels.py:1034
    dq = np.einsum("nhjc,nhc->nhj", Kt.astype(np.float64), qnv.astype(np.float64)) * w
    A4 = np.einsum("nhjv,nhj->nhv", Ub, dk)
    A5 = np.einsum("nhjv,nhj->nhv", Ub, dq)
    UT = st["UQ"][s][..., :K].astype(np.float64) * pc.astype(np.float64)[:, :, None, :]        # kernels.py:1040
    QT = st["UQ"][s][..., K:].astype(np.float64)
    dU = np.einsum("nhrc,nhc->nhr", UT, knv.astype(np.float64))
    dQ = np.einsum("nhrc,nhc->nhr", UT, qnv.astype(np.float64))
    A6 = np.einsum("nhrv,nhr->nhv", QT, dU)
    A7 = np.einsum("nhrv,nhr->nhv", QT, dQ)
    u = beta[:, :, None] * (v - (m + A6 + A4))                                                   # kernels.py:1065
    y = yq + A7 + A5 + kap[:, :, None] * u                                                       # kernels.py:1066
    o[rows] = bf16(y)
    hv_ix = np.arange(HV)[None, :]
    st["Pbuf"][s] = gn                                                                            # kernels.py:895
    st["Gbuf"][s[:, None], hv_ix, h] = fp16(en)                                                  # kernels.py:896
    st["Wbuf"][s[:, None], hv_ix, h] = 1.0
    st["Ubuf"][s[:, None], hv_ix, h] = bf16(u)
    st["Kbuf"][s[:, None], np.arange(H)[None, :], h[:, ::G]] = bf16(kn)
    st["hcnt"][s] = h + 1
    return o


# ----------------------------------------------------------------------------------------------------------------
# CholeskyQR pass with the reference's pivot floors (kernels.py:1778-1835), float64
# ----------------------------------------------------------------------------------------------------------------
def cholqr_pass(pr):
    """pr: [D,V,R].  Returns pr L^{-T}.  R <= 4 (kernels.py:1781-1835): relative pivot floor d_j -> max(d_j, 1e-6 G_jj)
    (j >= 1) and the absolute floor 1e-30 before every rsqrt.  R > 4 (the R = 8 flush, kernels.py:1744-1772): a pivot
    with d_j <= 1e-6 G_jj + 1e-30 drops its column (1 / L_jj = 0) instead."""
    D, V, R = pr.shape
    if R > 4:
        return _cholqr_pass_drop(pr)
    Gm = np.einsum("dvr,dvs->drs", pr, pr)
    ll = {}
    out = pr.copy()
    for j in range(R):
        for kk in range(j):
            acc = Gm[:, j, kk].copy()
            for m_ in range(kk):
                acc -= ll[(j, m_)] * ll[(kk, m_)]
            ll[(j, kk)] = acc * ll[(kk, kk)]
        acc = Gm[:, j, j].copy()
        for m_ in range(j):
            acc -= ll[(j, m_)] * ll[(j, m_)]
        if j > 0:
            acc = np.maximum(acc, 1e-6 * Gm[:, j, j])
        ll[(j, j)] = 1.0 / np.sqrt(np.maximum(acc, 1e-30))          # reciprocal of L_jj
    for j in range(R):
        acc = out[:, :, j].copy()
        for m_ in range(j):
            acc -= out[:, :, m_] * ll[(j, m_)][:, None]
        out[:, :, j] = acc * ll[(j, j)][:, None]
    return out


def _cholqr_pass_drop(pr):
    """The R > 4 CholeskyQR pass: Cholesky of the Gram matrix column by column; column j is kept when its remaining
    pivot exceeds 1e-6 G_jj + 1e-30 and scaled by its reciprocal square root, else zeroed together with its entries
    in L (kernels.py:1758-1767)."""
    D, V, R = pr.shape
    Gm = np.einsum("dvr,dvs->drs", pr, pr)
    ll = np.zeros((D, R, R))
    for j in range(R):
        for kk in range(j):
            ll[:, j, kk] = (Gm[:, j, kk] - (ll[:, j, :kk] * ll[:, kk, :kk]).sum(-1)) * ll[:, kk, kk]
        acc = Gm[:, j, j] - (ll[:, j, :j] ** 2).sum(-1)
        keep = acc > 1e-6 * Gm[:, j, j] + 1e-30
        ll[:, j, j] = np.where(keep, 1.0 / np.sqrt(np.maximum(acc, 1e-30)), 0.0)
    out = pr.copy()
    for j in range(R):
        acc = out[:, :, j] - np.einsum("dvm,dm->dv", out[:, :, :j], ll[:, j, :j])
        out[:, :, j] = acc * ll[:, j, j][:, None]
    return out


def mgs_cols(X):
    """Modified Gram-Schmidt on the columns of X [D,n,R] with rsqrt(max(|x|^2, 1e-30)) (kernels.py:2170-2183)."""
    X = X.copy()
    R = X.shape[-1]
    for j in range(R):
        for c in range(j):
            sc = (X[:, :, c] * X[:, :, j]).sum(-1)
            X[:, :, j] = X[:, :, j] - sc[:, None] * X[:, :, c]
        nrm = (X[:, :, j] ** 2).sum(-1)
        X[:, :, j] = X[:, :, j] / np.sqrt(np.maximum(nrm, 1e-30))[:, None]
    return X


# ----------------------------------------------------------------------------------------------------------------
# end-of-window flush  (kernels.py:1077-2033)
# ----------------------------------------------------------------------------------------------------------------
def due_pairs(st, idx):
    """(slot, head) pairs the flush processes: slot = idx[n] > 0 and hcnt[slot, hv] == L (kernels.py:1200)."""
    NS, HV, H, K, V, L, R = _dims(st)
    slots = sorted(set(int(x) for x in np.asarray(idx).reshape(-1) if 0 < int(x) < NS))
    out = [(sl, hv) for sl in slots for hv in range(HV) if st["hcnt"][sl, hv] == L]
    return out


def flush(st, Q0, idx, qmax=QMAX, return_debug=False, b_hook=None, factors=None):
    """Flush every due (slot, head) in place: rebuild B, one subspace iteration from Q0 with CholeskyQR2, new fp16
    factors, smoothed residual, INT8 (or qmax) codes, window reset.  b_hook (tests only): a function applied to the
    rebuilt fp16 B [D,V,K] before the subspace step, to measure how the outputs respond to a change of B.
    factors (tests only): fp16 factors (U16 [D,K,R], Q16 [D,V,R]) of the due pairs, in due_pairs order, used in place
    of the subspace step's own, so that the residual stage can be checked on another implementation's factors."""
    NS, HV, H, K, V, L, R = _dims(st)
    G = HV // H
    kda = st["kda"]
    pairs = due_pairs(st, idx)
    if not pairs:
        return {} if return_debug else None
    s = np.array([p[0] for p in pairs])
    hv = np.array([p[1] for p in pairs])
    hk = hv // G
    code = st["Sq"][s, hv].astype(F32)                                                           # [D,V,K]
    Skc = st["Sk"][s, hv]
    Svc = st["Sv"][s, hv]
    UT = st["UQ"][s, hv][:, :, :K].astype(F32)                                                   # [D,R,K]
    QT = st["UQ"][s, hv][:, :, K:].astype(np.float64)                                            # [D,R,V]
    Kb = st["Kbuf"][s, hk]                                                                       # [D,L,K]
    Ub = st["Ubuf"][s, hv]                                                                       # [D,L,V]
    Wb = st["Wbuf"][s, hv]                                                                       # [D,L]
    if not kda:
        pn = np.maximum(st["Pbuf"][s, hv, 0], F32(PNMIN)).astype(F32)                            # kernels.py:1471
        rpn = r32(1.0 / pn.astype(np.float64))                                                   # kernels.py:1477
        svr = r32(Svc * r32(pn.astype(np.float64) / qmax)[:, None])                              # kernels.py:1483
        skl = Skc
        wu = r32(Wb[:, :, None] * Ub)                                                            # kernels.py:1509
        a_hi = bf16(wu)
        a_lo = bf16(r32(wu.astype(np.float64) - a_hi))
        ring = np.einsum("djv,djc->dvc", a_hi.astype(np.float64) + a_lo.astype(np.float64), Kb.astype(np.float64))
        Uold = UT.astype(np.float64)
        pn64 = pn.astype(np.float64)
    else:
        pc = r32(np.exp(st["Pbuf"][s, hv].astype(np.float64)))                                   # kernels.py:1451
        el = st["Gbuf"][s, hv].astype(F32)                                                       # [D,L,K]
        khi = np.zeros_like(Kb)
        klo = np.zeros_like(Kb)
        dcur = np.ones((len(pairs), K), F32)
        for j in range(L - 1, -1, -1):                                                           # kernels.py:1456-1463
            kd = r32(Kb[:, j] * r32(Wb[:, j, None] * dcur))
            khi[:, j] = bf16(kd)
            klo[:, j] = bf16(r32(kd.astype(np.float64) - khi[:, j]))
            dcur = r32(dcur * el[:, j])
        ring = np.einsum("djv,djc->dvc", Ub.astype(np.float64), khi.astype(np.float64) + klo.astype(np.float64))
        Uold = fp16(r32(UT * pc[:, None, :])).astype(np.float64)                                  # kernels.py:1465
        svr = r32(Svc * F32(1.0 / qmax))                                                          # kernels.py:1468
        skl = r32(Skc * pc)                                                                       # kernels.py:1519
        pn64 = np.ones(len(pairs))
        rpn = None
    deq = r32(r32(code * svr[:, :, None]) * skl[:, None, :])                                     # kernels.py:1534-1535
    B = fp16(deq.astype(np.float64) + ring).astype(np.float64)                                  # kernels.py:1564-1571
    if b_hook is not None:
        B = b_hook(B)
    Q16 = np.broadcast_to(fp16(Q0).astype(np.float64), (len(pairs),) + Q0.shape).copy()         # kernels.py:1573-1577
    p = pn64[:, None, None]

    def p_step(Qh):
        M = np.einsum("dav,dvr->dar", QT, Qh)                                                    # Q_old^T Q
        return fp16(np.einsum("dvc,dvr->dcr", B, Qh) + p * np.einsum("dac,dar->dcr", Uold, M)).astype(np.float64)

    if factors is None:
        P16 = p_step(Q16)                                                                        # kernels.py:1580-1658
        M2 = np.einsum("dac,dcr->dar", Uold, P16)                                                # U_old^T P16
        Qf = r32(np.einsum("dvc,dcr->dvr", B, P16) + p * np.einsum("dav,dar->dvr", QT, M2))    # kernels.py:1660-1739
        pr = Qf.astype(np.float64)
        for _ in range(2):                                                                       # kernels.py:1780-1835
            pr = cholqr_pass(pr)
            Q16 = fp16(pr).astype(np.float64)
        U16 = p_step(Q16)                                                                        # ITERS = 1: U = P16
    else:
        U16 = fp16(factors[0]).astype(np.float64)
        Q16 = fp16(factors[1]).astype(np.float64)
        P16 = Qf = None
    # residual E = fp16(pn (fp16(B)/pn + Q_old U_old^T) - Q U^T)   (kernels.py:1888-1928)
    c = (r32(B * rpn[:, None, None]).astype(np.float64) if not kda else B.copy())
    c = c + np.einsum("dav,dac->dvc", QT, Uold)
    if not kda:
        c = c * p
    c = c - np.einsum("dvr,dcr->dvc", Q16, U16)
    E = fp16(c).astype(F32)
    # column smoothing scales (kernels.py:1955-1958) and row quantisation (kernels.py:1974-2009)
    msum = r32(r32(np.abs(E.astype(np.float64)).sum(1)) * F32(1.0 / V))                          # [D,K]
    Sk_new = np.maximum(r32(np.sqrt(msum.astype(np.float64))), F32(EPS)).astype(F32)
    with np.errstate(divide="ignore"):
        rsk = np.minimum(rsqrt32(msum), F32(1.0 / EPS)).astype(F32)
    x = r32(E * rsk[:, None, :])
    rmax = np.maximum(np.abs(x).max(-1), F32(EPS)).astype(F32)                                   # [D,V]
    rq = r32(F32(qmax) * r32(1.0 / rmax.astype(np.float64)))
    codes = np.rint(x.astype(np.float64) * rq.astype(np.float64)[:, :, None]).astype(np.int8)
    # writes
    st["Sq"][s, hv] = codes
    st["Sk"][s, hv] = Sk_new
    st["Sv"][s, hv] = rmax
    st["UQ"][s, hv] = np.concatenate([fp16(U16.transpose(0, 2, 1)), fp16(Q16.transpose(0, 2, 1))], axis=-1)
    st["Wbuf"][s, hv] = 0.0
    st["hcnt"][s, hv] = 0
    if kda:
        st["Pbuf"][s, hv] = 0.0
        st["Gbuf"][s, hv] = np.float16(1.0)
    else:
        st["Pbuf"][s, hv, 0] = 1.0
    if return_debug:
        return dict(pairs=pairs, B=B, P16=P16, Q16=Q16, U16=U16, E=E, Qf=Qf)
    return None


# ----------------------------------------------------------------------------------------------------------------
# standalone quantize  (kernels.py:2126-2242), generalised to a code range qmax (127: INT8, 31: 6-bit)
# ----------------------------------------------------------------------------------------------------------------
def quantize_dense(S, Q0, qmax=QMAX, iters=1):
    """fp32 states S [D,V,K] -> (codes int8 [D,V,K], Sk [D,K], Sv [D,V], UQ fp16 [D,R,K+V])."""
    S = np.asarray(S, F32)
    S64 = S.astype(np.float64)
    D, V, K = S.shape
    Q = np.broadcast_to(np.asarray(Q0, np.float64), (D,) + Q0.shape).copy()
    for _ in range(iters):
        P = mgs_cols(np.einsum("dvc,dvr->dcr", S64, Q))                                         # kernels.py:2164-2183
        Q = mgs_cols(np.einsum("dvc,dcr->dvr", S64, P))                                         # kernels.py:2184-2203
    U16 = fp16(np.einsum("dvc,dvr->dcr", S64, Q)).astype(np.float64)                            # kernels.py:2204-2209
    Q16 = fp16(Q).astype(np.float64)                                                             # kernels.py:2210-2211
    codes, sk, sv = quantize_residual(S, U16, Q16, qmax)
    UQ = np.concatenate([fp16(U16.transpose(0, 2, 1)), fp16(Q16.transpose(0, 2, 1))], axis=-1)
    return codes, sk, sv, UQ


def quantize_residual(S, U16, Q16, qmax=QMAX):
    """The residual stage of the standalone quantize: fp32 states S [D,V,K] and fp16 factors U16 [D,K,R], Q16 [D,V,R]
    (values, any float dtype) -> (codes int8 [D,V,K], Sk [D,K], Sv [D,V]).  kernels.py:2212-2229."""
    S64 = np.asarray(S, F32).astype(np.float64)
    V = S64.shape[1]
    U16 = np.asarray(U16, np.float64)
    Q16 = np.asarray(Q16, np.float64)
    E = r32(S64 - np.einsum("dvr,dcr->dvc", Q16, U16))                                          # kernels.py:2212-2217
    colsum = r32(np.abs(E.astype(np.float64)).sum(1))
    sk = np.maximum(r32(np.sqrt(r32(colsum / F32(V)).astype(np.float64))), F32(EPS)).astype(F32)   # kernels.py:2222
    sv = np.maximum(np.abs(r32(E / sk[:, None, :])).max(-1), F32(EPS)).astype(F32)             # kernels.py:2224-2227
    t = r32(r32(E / r32(sk[:, None, :] * sv[:, :, None])) * F32(qmax))
    codes = np.clip(np.rint(t), -qmax, qmax).astype(np.int8)                                    # kernels.py:2229
    return codes, sk, sv


def quantize(st, S_slots, Q0, idx, qmax=QMAX):
    """make_quantize semantics on the slots idx (> 0): S_slots [NS,HV,V,K] fp32 full-cache array; writes checkpoint,
    resets the window (Wbuf = 0, Pbuf = 1, hcnt = 0)."""
    NS, HV, H, K, V, L, R = _dims(st)
    slots = [int(x) for x in np.asarray(idx).reshape(-1) if int(x) > 0]
    for sl in slots:
        c, sk, sv, uq = quantize_dense(S_slots[sl], Q0, qmax)
        st["Sq"][sl], st["Sk"][sl], st["Sv"][sl], st["UQ"][sl] = c, sk, sv, uq
        st["Wbuf"][sl] = 0.0
        st["Pbuf"][sl] = 1.0
        st["hcnt"][sl] = 0


# ----------------------------------------------------------------------------------------------------------------
# prefill dequant  (kernels.py:2041-2123), GDN
# ----------------------------------------------------------------------------------------------------------------
def dequant(st, idx, qmax=QMAX):
    """Returns {slot: fp32 S [HV,V,K]} for the slots idx (> 0) and resets their windows."""
    NS, HV, H, K, V, L, R = _dims(st)
    G = HV // H
    out = {}
    for sl in [int(x) for x in np.asarray(idx).reshape(-1) if int(x) > 0]:
        q = st["Sq"][sl].astype(F32)
        tile = r32(r32(r32(q / F32(qmax)) * st["Sk"][sl][:, None, :]) * st["Sv"][sl][:, :, None])   # kernels.py:2107
        UT = st["UQ"][sl][..., :K].astype(np.float64)
        QT = st["UQ"][sl][..., K:].astype(np.float64)
        t = tile.astype(np.float64) + np.einsum("hrv,hrc->hvc", QT, UT)                          # kernels.py:2111
        t = t * st["Pbuf"][sl][:, 0, None, None].astype(np.float64)                              # kernels.py:2113
        h = st["hcnt"][sl]
        w = np.where(np.arange(L)[None, :] < h[:, None], st["Wbuf"][sl], 0.0).astype(np.float64)  # kernels.py:2088
        Kb = np.repeat(st["Kbuf"][sl], G, axis=0).astype(np.float64)
        t = t + np.einsum("hj,hjv,hjc->hvc", w, st["Ubuf"][sl].astype(np.float64), Kb)         # kernels.py:2116
        out[sl] = r32(t)
        st["Wbuf"][sl] = 0.0
        st["Pbuf"][sl] = 1.0
        st["hcnt"][sl] = 0
    return out


# ----------------------------------------------------------------------------------------------------------------
# KDA prefill round trip: low-rank factoriser and torch checkpoint (kernels.py:2245-2331, state.py:118-142)
# ----------------------------------------------------------------------------------------------------------------
def lowrank(x, Q0, iters=3):
    """x [D,K,V] -> U [D,K,R], Q [D,V,R]: `iters` rounds of P = MGS(x Q), Q = MGS(x^T P); U = x Q (fp32 outputs)."""
    x64 = np.asarray(x, np.float64)
    D = x64.shape[0]
    Q = np.broadcast_to(np.asarray(Q0, np.float64), (D,) + Q0.shape).copy()
    for _ in range(iters):
        P = mgs_cols(np.einsum("dkv,dvr->dkr", x64, Q))
        Q = mgs_cols(np.einsum("dkv,dkr->dvr", x64, P))
    U = np.einsum("dkv,dvr->dkr", x64, Q)
    return r32(U), r32(Q)


def kda_rebuild(st, slots):
    """fp32 S of the listed slots (state.py:118-128)."""
    S = materialize(st)
    return {int(sl): r32(S[int(sl)]) for sl in slots}


def kda_checkpoint(st, S_slots, slots, Q0, R=4, qmax=QMAX):
    """8-bit checkpoint of fp32 states (state.py:130-142): lowrank on S^T (iters = 3), fp16 factors,
    res = S - Q U^T, sk = sqrt(mean_v |res|), sv = amax_c |res| / sk, codes = clamp(round(res / (sk sv) * 127))."""
    for sl in [int(x) for x in slots]:
        S = np.asarray(S_slots[sl], F32)                                                        # [HV,V,K]
        U, Q = lowrank(S.transpose(0, 2, 1), Q0)
        Uh = fp16(U).astype(np.float64)
        Qh = fp16(Q).astype(np.float64)
        res = r32(S.astype(np.float64) - np.einsum("hvr,hcr->hvc", Qh, Uh))
        sk = np.maximum(r32(np.sqrt(r32(np.abs(res.astype(np.float64)).mean(1)).astype(np.float64))), F32(EPS))
        sv = np.maximum(r32(np.abs(res) / sk[:, None, :]).max(-1), F32(EPS))
        t = r32(r32(res / r32(sk[:, None, :] * sv[:, :, None])) * F32(qmax))
        st["Sq"][sl] = np.clip(np.rint(t), -qmax, qmax).astype(np.int8)
        st["Sk"][sl] = sk
        st["Sv"][sl] = sv
        st["UQ"][sl] = np.concatenate([fp16(Uh.transpose(0, 2, 1)), fp16(Qh.transpose(0, 2, 1))], axis=-1)
        st["Wbuf"][sl] = 0.0
        st["Pbuf"][sl] = 0.0
        st["Gbuf"][sl] = np.float16(1.0)
        st["hcnt"][sl] = 0


# ----------------------------------------------------------------------------------------------------------------
# dense float64 references (used only to pin the oracle)
# ----------------------------------------------------------------------------------------------------------------
def dense_gdn_step(S, q, k, v, alpha, beta, scale):
    """Gated delta rule on dense float64 states S [n,HV,V,K]: S' = alpha S + u k^T, u = beta (v - alpha S k),
    o = S' q (k, q l2-normalised, q scaled)."""
    k64 = np.asarray(k, np.float64)
    q64 = np.asarray(q, np.float64)
    kh = k64 / np.sqrt((k64 * k64).sum(-1, keepdims=True) + NORM_EPS)
    qh = q64 * scale / np.sqrt((q64 * q64).sum(-1, keepdims=True) + NORM_EPS)
    Sd = S * alpha[:, :, None, None]
    u = beta[:, :, None] * (v - np.einsum("nhvc,nhc->nhv", Sd, kh))
    S1 = Sd + u[:, :, :, None] * kh[:, :, None, :]
    return S1, np.einsum("nhvc,nhc->nhv", S1, qh), u, kh


def dense_kda_step(S, q, k, v, gdecay, beta, scale):
    """KDA on dense float64 states: S' = S diag(exp(g)) + u k^T, u = beta (v - S diag(exp(g)) k), o = S' q."""
    k64 = np.asarray(k, np.float64)
    q64 = np.asarray(q, np.float64)
    kh = k64 / np.sqrt((k64 * k64).sum(-1, keepdims=True) + NORM_EPS)
    qh = q64 * scale / np.sqrt((q64 * q64).sum(-1, keepdims=True) + NORM_EPS)
    Sd = S * np.exp(gdecay)[:, :, None, :]
    u = beta[:, :, None] * (v - np.einsum("nhvc,nhc->nhv", Sd, kh))
    S1 = Sd + u[:, :, :, None] * kh[:, :, None, :]
    return S1, np.einsum("nhvc,nhc->nhv", S1, qh), u, kh


def dense_state_step(S, mixed, a, b, A_log, dt_bias, idx, H, state_dtype="bf16", scale=None):
    """The bf16 / fp32-state baseline step (lq_dense_step): S [NS,HV,V,K] float32 array holding the state
    (bf16-rounded values for state_dtype 'bf16'); updates in place, returns o bf16 values [N,HV,V]."""
    NS, HV, V, K = S.shape
    G = HV // H
    scale = K ** -0.5 if scale is None else scale
    idx = np.asarray(idx).astype(np.int64)
    N = idx.shape[0]
    o = np.zeros((N, HV, V), F32)
    rows = np.nonzero(idx > 0)[0]
    if rows.size == 0:
        return o
    s = idx[rows]
    hk = np.arange(HV) // G
    alpha = gdn_alpha(np.asarray(a, F32).reshape(N, HV)[rows], np.asarray(dt_bias, F32).reshape(HV),
                      np.asarray(A_log, F32).reshape(HV)).astype(np.float64)
    beta = beta_of(np.asarray(b, F32).reshape(N, HV)[rows]).astype(np.float64)
    q, k, v = _split_mixed(np.asarray(mixed)[rows], H, HV, K, V)
    kn, qn, kappa = normalize_qk(q, k, scale)
    knv, qnv = kn[:, hk].astype(np.float64), qn[:, hk].astype(np.float64)
    Sd = S[s].astype(np.float64) * alpha[:, :, None, None]
    u = beta[:, :, None] * (v - np.einsum("nhvc,nhc->nhv", Sd, knv))
    S1 = Sd + u[:, :, :, None] * knv[:, :, None, :]
    y = np.einsum("nhvc,nhc->nhv", S1, qnv)
    o[rows] = bf16(y)
    S[s] = bf16(S1) if state_dtype == "bf16" else r32(S1)
    return o
