"""GPU tests of the vLLM plugin end to end: a stand-in Gated DeltaNet layer (tests/fake_vllm.py) on cuda:0 whose
forward goes through the plugin's hooks (leapquant_amd/vllm/gdn.py) into the HIP kernels, checked against the oracle
applied to the very tensors the plugin handed to the layer state.

  * decode-only steps across a window boundary (step + flush), padding rows included;
  * a mixed step: decode rows intercepted from vLLM's recurrent function into the HIP step, prefill slots dequantised
    (HIP), advanced by the stand-in's fp32 prefill, and re-quantised (HIP).
Tolerances: outputs rtol 2e-2 / atol 1e-3 (bf16); every flush from identical inputs (the oracle continues from the
GPU's state after each decode call): factors within one fp16 rounding, the residual stage's codes on the GPU's factors
within 1 LSB on <= 0.1 %; the prefill re-quantisation's codes within 1 LSB on <= 0.1 %."""
import numpy as np
import pytest
import torch

from oracle import lq_oracle as O
from tests import fake_vllm as FV
from tests import lqgpu as G
from tests.fixtures import make_state
from tests.test_gpu_full_size import _assert_flush_pinned
from tests.test_gpu_modes import _resync

pytestmark = pytest.mark.gpu

H, HV, K, NS, L = 2, 4, 128, 6, 16
RT, AT = 2e-2, 1e-3
PREFIX = "model.layers.0.linear_attn"


@pytest.fixture
def setup():
    FV.install()
    import leapquant_amd.vllm as P
    from leapquant_amd import state as S
    P.register()
    M = FV.sys.modules["vllm.model_executor.layers.mamba.gdn.qwen_gdn_linear_attn"]
    layer = M.QwenGatedDeltaNetAttention(PREFIX, H, HV, K, device=G.DEV)
    torch.manual_seed(5)
    with torch.no_grad():
        layer.conv1d.weight.normal_(0, 0.5)
    C = 2 * H * K + HV * K
    ssm = torch.zeros(NS, HV, K, K, device=G.DEV)
    layer.kv_cache = (torch.randn(NS, C, 3, device=G.DEV), ssm)
    rng = np.random.default_rng(11)
    st, _, Q0 = make_state(rng, NS, HV, H, L=L)
    lq = S.get_state(layer, ssm, H=H, nmax=0)           # the state the plugin will find for this layer
    assert lq.L == L
    G.load_state(lq, ssm, st)
    seen = []
    decode = lq.decode

    def recording_decode(ssm_, mixed, a, b, A_log, dt_bias, idx, out):
        seen.append((mixed.float().cpu().numpy(), a.float().cpu().numpy(), b.float().cpu().numpy(),
                     idx.cpu().numpy().astype(np.int64)))
        return decode(ssm_, mixed, a, b, A_log, dt_bias, idx, out)

    lq.decode = recording_decode
    yield layer, lq, ssm, st, Q0, seen, rng
    FV.uninstall()
    S._STATES.clear()


def _draw(rng, T):
    C = 2 * H * K + HV * K
    x = torch.from_numpy(rng.standard_normal((T, C)).astype(np.float32)).to(torch.bfloat16)
    g = np.minimum(rng.uniform(-0.1, 0.0, (T, HV)), -1e-4)
    a = torch.from_numpy(np.log(np.expm1(-g)).astype(np.float32)).to(torch.bfloat16)
    b = torch.from_numpy(rng.standard_normal((T, HV)).astype(np.float32)).to(torch.bfloat16)
    return x.to(G.DEV), b.to(G.DEV), a.to(G.DEV)


def test_plugin_decode_steps_match_oracle(setup):
    layer, lq, ssm, st, Q0, seen, rng = setup
    idx = torch.tensor([1, 0, 3, 5], dtype=torch.int32, device=G.DEV)
    n = idx.shape[0]
    A_log = np.zeros(HV, np.float32)
    dt_bias = np.zeros(HV, np.float32)
    conv_host = layer.kv_cache[0].cpu()
    w = layer.conv1d.weight.detach().cpu()
    flushes = 0
    for t in range(L + 4):                                     # crosses the window boundary: one flush
        FV.CONTEXT.attn_metadata = {PREFIX: FV.gdn_metadata(n, idx)}
        x, b, a = _draw(rng, n)
        out = torch.zeros(n, HV, K, dtype=torch.bfloat16, device=G.DEV)
        layer._forward_core(x, b, a, out)
        mixed, a_, b_, idx_ = seen[-1]
        want = FV.causal_conv1d_update(x.cpu(), conv_host, w.view(w.size(0), w.size(2)), None, "silu",
                                       conv_state_indices=idx.cpu())
        assert np.array_equal(mixed, want.float().numpy()), "step %d: conv output handed to the state" % t
        o_ref = O.gdn_step(st, mixed, a_, b_, A_log, dt_bias, idx_)
        due = O.due_pairs(st, idx_)
        pre = O.copy_state(st)
        O.flush(st, Q0, idx_)
        o_gpu = out.float().cpu().numpy()
        np.testing.assert_allclose(o_gpu, o_ref, rtol=RT, atol=AT, err_msg="step %d" % t)
        assert np.all(o_gpu[1] == 0)
        g = G.from_gpu(ssm, lq)
        if due:                                                # this call filled windows: their flush is compared
            sl = np.array(sorted({s_ for s_, _ in due}))
            lq.flush(ssm, torch.from_numpy(sl.astype(np.int32)).to(G.DEV))   # settles heads a deferred decode leaves
            g = G.from_gpu(ssm, lq)
            _assert_flush_pinned(g, pre, Q0, idx_)             # each flush from identical inputs, stage by stage
            flushes += 1
        _resync(st, g)                                         # the oracle continues from the GPU's state
    assert flushes >= 1
    assert "vllm_core" not in FV.CALLS
    g = G.from_gpu(ssm, lq)
    assert np.array_equal(g["hcnt"], st["hcnt"])
    for s in (2, 4):                                           # slots not in the batch are untouched
        assert np.array_equal(g["Sq"][s], st["Sq"][s])


def test_plugin_mixed_step_matches_oracle(setup):
    layer, lq, ssm, st, Q0, seen, rng = setup
    A_log = np.zeros(HV, np.float32)
    dt_bias = np.zeros(HV, np.float32)
    didx = torch.tensor([1, 3], dtype=torch.int32, device=G.DEV)
    for t in range(5):                                         # partial windows first
        FV.CONTEXT.attn_metadata = {PREFIX: FV.gdn_metadata(2, didx)}
        x, b, a = _draw(rng, 2)
        out = torch.zeros(2, HV, K, dtype=torch.bfloat16, device=G.DEV)
        layer._forward_core(x, b, a, out)
        mixed, a_, b_, idx_ = seen[-1]
        O.gdn_step(st, mixed, a_, b_, A_log, dt_bias, idx_)
        O.flush(st, Q0, idx_)
    # one engine step: 2 decode rows, then prefill sequences of 3 and 2 tokens on slots 2 and 5 (which hold state)
    pidx = torch.tensor([2, 5], dtype=torch.int32, device=G.DEV)
    loc = torch.tensor([0, 3, 5], dtype=torch.int32, device=G.DEV)
    FV.CONTEXT.attn_metadata = {PREFIX: FV.gdn_metadata(2, didx, prefill_idx=pidx, prefill_loc=loc)}
    x, b, a = _draw(rng, 7)
    conv_host = layer.kv_cache[0].cpu()
    out = torch.zeros(7, HV, K, dtype=torch.bfloat16, device=G.DEV)
    n_seen = len(seen)
    layer._forward_core(x, b, a, out)
    assert len(seen) == n_seen + 1 and "vllm_recurrent" not in FV.CALLS     # decode rows went to the HIP step
    mixed, a_, b_, idx_ = seen[-1]
    assert np.array_equal(idx_, [1, 3])
    o_ref = O.gdn_step(st, mixed, a_, b_, A_log, dt_bias, idx_)
    O.flush(st, Q0, idx_)
    o_gpu = out.float().cpu().numpy()
    np.testing.assert_allclose(o_gpu[:2], o_ref, rtol=RT, atol=AT)
    # prefill slots on the oracle: dequant, the stand-in's fp32 prefill on the host, quantize
    Sd = O.dequant(st, [2, 5])
    w = layer.conv1d.weight.detach().cpu()
    FV.causal_conv1d_update(x[:2].cpu(), conv_host, w.view(w.size(0), w.size(2)), None, "silu",
                            conv_state_indices=didx.cpu())
    xp = FV.causal_conv1d_fn(x[2:].cpu().transpose(0, 1), w.view(w.size(0), w.size(2)), None, "silu",
                             conv_states=conv_host, cache_indices=pidx.cpu(),
                             query_start_loc=loc.cpu()).transpose(0, 1)
    q, k, v = xp.split([H * K, H * K, HV * K], -1)
    S_all = np.zeros((NS, HV, K, K), np.float32)
    for s, (lo, hi) in zip((2, 5), ((0, 3), (3, 5))):
        S = torch.from_numpy(Sd[s].copy())
        o = FV.fp32_gdn_prefill(S, torch.zeros(HV), torch.zeros(HV), q[lo:hi].reshape(-1, H, K),
                                k[lo:hi].reshape(-1, H, K), v[lo:hi].reshape(-1, HV, K), a[2 + lo:2 + hi].cpu(),
                                b[2 + lo:2 + hi].cpu())
        np.testing.assert_allclose(o_gpu[2 + lo:2 + hi], o.to(torch.bfloat16).float().numpy(), rtol=RT, atol=AT)
        S_all[s] = S.numpy()
    O.quantize(st, S_all, Q0, [2, 5])
    g = G.from_gpu(ssm, lq)
    assert np.array_equal(g["hcnt"], st["hcnt"])
    for s in (2, 5):
        frac, mx = G.code_mismatch(g["Sq"][s], st["Sq"][s])
        assert mx <= 1 and frac <= 1e-3, (s, frac, mx)
        np.testing.assert_allclose(g["Sk"][s], st["Sk"][s], rtol=1e-3)
        np.testing.assert_allclose(g["Sv"][s], st["Sv"][s], rtol=1e-3)
    assert np.array_equal(g["Sq"][4], st["Sq"][4])
