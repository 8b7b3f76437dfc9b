"""Seeded synthetic inputs with the distributions the benchmark configs name (numpy, CPU), shared by the tests.

State: fp32 S ~ N(0, 0.02^2) per (slot, head), quantized once by the oracle's standalone quantize -> checkpoint.
Inputs: q, k ~ N(0,1), l2-normalised, bf16; v ~ N(0,1) bf16; b ~ N(0,1) bf16 (beta = sigmoid(b));
log-gate g ~ U(-0.1, 0) clamped at <= -1e-4, fed as a = bf16(log(expm1(-g))) with A_log = dt_bias = 0 so that
alpha = exp(-softplus(a)) = exp(g).  KDA: the same inversion per key channel (GLB = 0, Kimi form).
"""
import numpy as np

from oracle import lq_oracle as O


def bf16(x):
    return O.bf16(x)


def make_inputs(rng, N, HV, H, K=128, V=128, kda=False):
    q = rng.standard_normal((N, H, K))
    k = rng.standard_normal((N, H, K))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((N, HV, V))
    mixed = bf16(np.concatenate([q.reshape(N, -1), k.reshape(N, -1), v.reshape(N, -1)], axis=1))
    gshape = (N, HV, K) if kda else (N, HV)
    g = np.minimum(rng.uniform(-0.1, 0.0, gshape), -1e-4)
    a = bf16(np.log(np.expm1(-g)))
    b = bf16(rng.standard_normal((N, HV)))
    return mixed, a, b


def gate_params(HV, K=128, kda=False):
    A_log = np.zeros(HV, np.float32)
    dt_bias = np.zeros((HV, K) if kda else (HV,), np.float32)
    return A_log, dt_bias


def make_state(rng, NS, HV, H, K=128, V=128, L=16, R=4, kda=False, sigma=0.02, qmax=127.0, heavy=False):
    """Oracle state with every slot 1..NS-1 holding a quantized N(0, sigma^2) (or 0.02 Student-t(3)) fp32 state."""
    st = O.new_state(NS, HV, H, K, V, L, R, kda)
    Q0 = O.make_q0(V, R)
    if heavy:
        S = (sigma * rng.standard_t(3, (NS, HV, V, K))).astype(np.float32)
    else:
        S = (sigma * rng.standard_normal((NS, HV, V, K))).astype(np.float32)
    O.quantize(st, S, Q0, np.arange(1, NS), qmax=qmax)
    if kda:
        st["Pbuf"][:] = 0.0
    return st, S, Q0


def oracle_steps(rng, st, steps, NS, HV, H, flush_Q0=None):
    """GDN oracle decode steps on random subsets of the slots 1..NS-1, each followed by the flush when flush_Q0 is
    given (every slot then ends at its own window fill)."""
    A_log, dt_bias = gate_params(HV)
    for _ in range(steps):
        sl = rng.permutation(np.arange(1, NS))[: rng.integers(1, NS)]
        mixed, a, b = make_inputs(rng, len(sl), HV, H)
        O.gdn_step(st, mixed, a, b, A_log, dt_bias, sl)
        if flush_Q0 is not None:
            O.flush(st, flush_Q0, sl)


def due_flush_case(rng, L, R=4, NS=6, HV=4, H=2):
    """(state, Q0): a GDN state at rank R after L + 5 steps-and-flushes, then slots 1 and 3 stepped to a full window
    (due), the other slots partial."""
    st, _, Q0 = make_state(rng, NS, HV, H, L=L, R=R)
    oracle_steps(rng, st, L + 5, NS, HV, H, flush_Q0=Q0)
    A_log, dt_bias = gate_params(HV)
    for s in (1, 3):
        while st["hcnt"][s, 0] < L:
            mixed, a, b = make_inputs(rng, 1, HV, H)
            O.gdn_step(st, mixed, a, b, A_log, dt_bias, np.array([s]))
    return st, Q0


def make_trajectory(kda=False, L=16, steps=35, seed=0, NS=4, HV=2, H=None, K=128, V=128, R=4):
    """Runs `steps` oracle decode steps (each followed by the flush) on a small state; returns a dict of arrays."""
    H = (2 if kda else 1) if H is None else H
    rng = np.random.default_rng(seed)
    st, S, Q0 = make_state(rng, NS, HV, H, K, V, L, R, kda)
    idx = np.array([2, 0, 1], np.int64)
    A_log, dt_bias = gate_params(HV, K, kda)
    init = {("init_" + k): v.copy() for k, v in st.items() if isinstance(v, np.ndarray)}
    mixed_all, a_all, b_all, o_all = [], [], [], []
    for t in range(steps):
        mixed, a, b = make_inputs(rng, len(idx), HV, H, K, V, kda)
        if kda:
            o = O.kda_step(st, mixed, a, b, A_log, dt_bias, idx)
        else:
            o = O.gdn_step(st, mixed, a, b, A_log, dt_bias, idx)
        O.flush(st, Q0, idx)
        mixed_all.append(mixed)
        a_all.append(a)
        b_all.append(b)
        o_all.append(o)
    out = dict(init)
    out.update({("final_" + k): v.copy() for k, v in st.items() if isinstance(v, np.ndarray)})
    out.update(mixed=np.stack(mixed_all), a=np.stack(a_all), b=np.stack(b_all), o=np.stack(o_all), idx=idx,
               A_log=A_log, dt_bias=dt_bias, dims=np.array([NS, HV, H, K, V, L, R, int(kda)]))
    return out


BF16_KEYS = ("mixed", "a", "b", "o", "init_Kbuf", "init_Ubuf", "final_Kbuf", "final_Ubuf")


def to_bits(d):
    """bf16-valued float32 arrays -> uint16 bit patterns (halves the fixture size, exact)."""
    out = dict(d)
    for k in BF16_KEYS:
        if k in out:
            out[k] = (np.ascontiguousarray(out[k], np.float32).view(np.uint32) >> 16).astype(np.uint16)
    return out


def from_bits(z):
    out = {k: z[k] for k in z.files}
    for k in BF16_KEYS:
        if k in out and out[k].dtype == np.uint16:
            out[k] = (out[k].astype(np.uint32) << 16).view(np.float32)
    return out


def state_from_npz(z, prefix):
    NS, HV, H, K, V, L, R, kda = [int(x) for x in z["dims"]]
    st = {k[len(prefix):]: np.array(z[k]) for k in z if k.startswith(prefix)}
    st["kda"] = bool(kda)
    if "Gbuf" not in st:
        st["Gbuf"] = None
    return st
