"""CPU tests of the vLLM plugin's routing (leapquant_amd/vllm), against the stand-in vLLM of tests/fake_vllm.py.  The
plugin is reached as vLLM reaches it: through the entry point `leapquant.vllm:register` under the reference's package
name.

The layer state is replaced by a recorder, so these tests check which LeapQuant calls each kind of engine step makes,
with which tensors and in which order (reference behaviour: leapquant/vllm/__init__.py:22-34, gdn.py:28-81,
glm.py:24-77).  The kernels themselves are covered by the GPU tests."""
import types

import pytest
import torch

from tests import fake_vllm as FV

H, HV, K = 2, 4, 128
NS = 6


class Recorder:
    """Stands in for LeapQuantState: records decode / dequantize / quantize calls."""

    def __init__(self, HV_, V_, kda=False):
        self.HV, self.V, self.kda, self.calls = HV_, V_, kda, []

    def decode(self, ssm, mixed, a, b, A_log, dt_bias, idx, out):
        self.calls.append(("decode", dict(ssm=ssm, mixed=mixed.clone(), a=a.clone(), b=b.clone(), A_log=A_log,
                                          dt_bias=dt_bias, idx=idx.clone(), out=out)))
        out.fill_(7.0)

    def decode_conv(self, ssm, x, conv_state, conv_weight, conv_bias, silu, a, b, A_log, dt_bias, idx, out):
        self.calls.append(("decode_conv", dict(ssm=ssm, x=x.clone(), conv_state=conv_state, weight=conv_weight,
                                               bias=conv_bias, silu=silu, a=a.clone(), b=b.clone(), idx=idx.clone(),
                                               out=out)))
        out.fill_(5.0)

    def dequantize(self, ssm, idx):
        self.calls.append(("dequantize", idx.clone()))

    def quantize(self, ssm, idx):
        self.calls.append(("quantize", idx.clone()))


@pytest.fixture
def plugin(monkeypatch):
    FV.install()
    import importlib
    mod, fn = "leapquant.vllm:register".split(":")          # the entry point, resolved as vLLM's plugin loader does
    P = importlib.import_module(mod)
    assert getattr(P, fn) is P.register
    from leapquant.vllm import gdn, glm
    rec = {}

    def fake_get_state(layer, ssm, **kw):
        key = id(layer)
        if key not in rec:
            rec[key] = Recorder(ssm.shape[1], ssm.shape[2], kda=kw.get("kda", False))
            rec[key].kw = kw
        return rec[key]

    monkeypatch.setattr(gdn, "get_state", fake_get_state)
    monkeypatch.setattr(glm, "get_state", fake_get_state)
    P.register()
    yield types.SimpleNamespace(P=P, rec=rec, mods=FV.sys.modules)
    FV.uninstall()


def gdn_layer(prefix="model.layers.0.linear_attn"):
    M = FV.sys.modules["vllm.model_executor.layers.mamba.gdn.qwen_gdn_linear_attn"]
    layer = M.QwenGatedDeltaNetAttention(prefix, H, HV, K)
    C = 2 * H * K + HV * K
    torch.manual_seed(0)
    with torch.no_grad():
        layer.conv1d.weight.normal_(0, 0.5)
    layer.kv_cache = (torch.randn(NS, C, 3), torch.zeros(NS, HV, K, K))
    return layer


def inputs(T, seed=1):
    g = torch.Generator().manual_seed(seed)
    C = 2 * H * K + HV * K
    return (torch.randn(T, C, generator=g).to(torch.bfloat16), torch.randn(T, HV, generator=g).to(torch.bfloat16),
            torch.randn(T, HV, generator=g).to(torch.bfloat16), torch.zeros(T, HV, K, dtype=torch.bfloat16))


def test_register_is_idempotent_and_records_batch_limit(plugin):
    P = plugin.P
    M = plugin.mods["vllm.model_executor.layers.mamba.gdn.qwen_gdn_linear_attn"]
    core = M.QwenGatedDeltaNetAttention._forward_core
    P.register()
    assert M.QwenGatedDeltaNetAttention._forward_core is core          # not patched twice
    assert M.fused_sigmoid_gating_delta_rule_update.__wrapped__ is FV.fused_sigmoid_gating_delta_rule_update
    gdn_layer()
    assert P.NMAX[0] == 512                                             # max(max_num_seqs, capture size)
    K_ = plugin.mods["vllm.models.glm5next.nvidia.kda"]
    assert getattr(K_.Glm5NextLinearAttention._forward, "eager_break", False)


def test_gdn_decode_only_step_goes_to_leapquant(plugin):
    layer = gdn_layer()
    conv0 = layer.kv_cache[0].clone()
    n = 3
    idx = torch.tensor([2, 0, 5, -1], dtype=torch.int32)                 # padded to 4 rows; slot 0 / -1 = padding
    FV.CONTEXT.attn_metadata = {layer.prefix: FV.gdn_metadata(n, idx)}
    mixed_qkv, b, a, out = inputs(4)
    layer._forward_core(mixed_qkv, b, a, out)
    assert "vllm_core" not in FV.CALLS                                  # vLLM's decode path did not run
    st = plugin.rec[id(layer)]
    assert st.kw == dict(H=H, nmax=512, defer_flush=True)
    (name, c), = st.calls
    assert name == "decode"
    # the conv update of the first n rows, computed on a copy of the conv state
    w = layer.conv1d.weight
    want = FV.causal_conv1d_update(mixed_qkv[:n], conv0, w.view(w.size(0), w.size(2)), None, "silu",
                                   conv_state_indices=idx[:n])
    assert torch.equal(c["mixed"], want.contiguous())
    assert torch.equal(c["idx"], idx[:n]) and c["ssm"] is layer.kv_cache[1]
    assert torch.equal(c["a"], a[:n]) and torch.equal(c["b"], b[:n])
    assert c["out"].shape == (n, HV, K) and c["out"].data_ptr() == out.data_ptr()
    assert bool((out[:n] == 7).all()) and bool((out[n:] == 0).all())
    assert torch.equal(layer.kv_cache[0], conv0)                        # the conv state was advanced for those rows


def test_gdn_decode_only_bf16_conv_is_fused(plugin):
    """A bf16 conv of width 4 goes into the step: decode_conv gets the raw projection and the conv state itself (the
    conv update is the kernel's), and vLLM's conv update does not run."""
    layer = gdn_layer()
    with torch.no_grad():
        layer.conv1d.weight.data = layer.conv1d.weight.data.to(torch.bfloat16)
    layer.kv_cache = (layer.kv_cache[0].to(torch.bfloat16), layer.kv_cache[1])
    conv0 = layer.kv_cache[0].clone()
    n = 3
    idx = torch.tensor([2, 0, 5, -1], dtype=torch.int32)
    FV.CONTEXT.attn_metadata = {layer.prefix: FV.gdn_metadata(n, idx)}
    mixed_qkv, b, a, out = inputs(4)
    layer._forward_core(mixed_qkv, b, a, out)
    st = plugin.rec[id(layer)]
    (name, c), = st.calls
    assert name == "decode_conv" and "vllm_core" not in FV.CALLS
    assert torch.equal(c["x"], mixed_qkv[:n]) and c["conv_state"].data_ptr() == layer.kv_cache[0].data_ptr()
    assert c["weight"].shape == (2 * H * K + HV * K, 4) and c["silu"] and c["bias"] is None
    assert torch.equal(c["idx"], idx[:n]) and torch.equal(c["a"], a[:n]) and torch.equal(c["b"], b[:n])
    assert bool((out[:n] == 5).all()) and bool((out[n:] == 0).all())
    assert torch.equal(layer.kv_cache[0], conv0)                        # the plugin itself did not touch the state


def test_gdn_profiling_run_uses_vllm(plugin):
    layer = gdn_layer()
    FV.CONTEXT.attn_metadata = None
    layer._forward_core(*inputs(2))
    assert FV.CALLS == ["vllm_core"]
    assert id(layer) not in plugin.rec


def test_gdn_mixed_step_round_trips_prefill_slots_only(plugin):
    layer = gdn_layer()
    nd = 2
    idx = torch.tensor([3, 4], dtype=torch.int32)
    pidx = torch.tensor([1, 5], dtype=torch.int32)
    loc = torch.tensor([0, 3, 5], dtype=torch.int32)
    FV.CONTEXT.attn_metadata = {layer.prefix: FV.gdn_metadata(nd, idx, prefill_idx=pidx, prefill_loc=loc)}
    mixed_qkv, b, a, out = inputs(nd + 5)
    layer._forward_core(mixed_qkv, b, a, out)
    st = plugin.rec[id(layer)]
    names = [c[0] for c in st.calls]
    assert names == ["dequantize", "decode", "quantize"]
    assert torch.equal(st.calls[0][1], pidx) and torch.equal(st.calls[2][1], pidx)
    assert "vllm_recurrent" not in FV.CALLS                             # the decode tokens were intercepted
    dec = st.calls[1][1]
    assert torch.equal(dec["idx"], idx) and dec["out"].shape == (nd, HV, K)
    assert bool((out[:nd] == 7).all())                                  # the intercepted output reached the layer
    # the routed layer is reset: a later unrelated call to vLLM's recurrent function is not intercepted
    M = plugin.mods["vllm.model_executor.layers.mamba.gdn.qwen_gdn_linear_attn"]
    q = torch.zeros(1, 1, H, K)
    M.fused_sigmoid_gating_delta_rule_update(A_log=None, a=None, b=None, dt_bias=None, q=q, k=q,
                                             v=torch.zeros(1, 1, HV, K), initial_state=None, inplace_final_state=True,
                                             cu_seqlens=None, ssm_state_indices=None)
    assert FV.CALLS[-1] == "vllm_recurrent"


def test_gdn_speculative_step_round_trips_every_slot(plugin):
    layer = gdn_layer()
    idx = torch.tensor([3, -1], dtype=torch.int32)
    sidx = torch.tensor([[2, 4]], dtype=torch.int32)
    md = FV.gdn_metadata(2, idx, spec_masks=torch.ones(2, dtype=torch.bool), spec_idx=sidx)
    FV.CONTEXT.attn_metadata = {layer.prefix: md}
    layer._forward_core(*inputs(2))
    st = plugin.rec[id(layer)]
    assert [c[0] for c in st.calls] == ["dequantize", "quantize"]
    assert st.calls[0][1].tolist() == [3, 0, 2, 4]                      # clamped at 0
    assert FV.CALLS.count("vllm_recurrent") == 1                        # not intercepted under speculation


def kda_layer(prefix="model.layers.1.attn"):
    M = FV.sys.modules["vllm.models.glm5next.nvidia.kda"]
    layer = M.Glm5NextLinearAttention(prefix, HV, K)
    P = HV * K
    with torch.no_grad():
        for m in (layer.q_conv1d, layer.k_conv1d, layer.v_conv1d):
            m.weight.normal_(0, 0.5)
    layer.kv_cache = (torch.randn(NS, 3 * P, 3), torch.zeros(NS, HV, K, K))
    return layer


def test_kda_decode_only(plugin):
    layer = kda_layer()
    conv0 = layer.kv_cache[0].clone()
    n = 2
    idx = torch.tensor([4, 1, 0], dtype=torch.int32)
    md = FV.gdn_metadata(n, idx)
    FV.CONTEXT.attn_metadata = {layer.prefix: md}
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn(3, 3 * HV * K, generator=g).to(torch.bfloat16)
    g1 = torch.randn(1, 3, HV * K, generator=g).to(torch.bfloat16)
    beta = torch.randn(1, 3, HV, generator=g).to(torch.bfloat16)
    out = torch.zeros(1, 3, HV, K, dtype=torch.bfloat16)
    layer._forward(qkv, g1, beta, out)
    st = plugin.rec[id(layer)]
    assert st.kw["kda"] is True and st.kw["gate_lower_bound"] == -5.0 and st.kw["H"] == HV
    (name, c), = st.calls
    assert name == "decode" and "vllm_kda_forward" not in FV.CALLS
    wm = torch.cat([m.weight.view(m.weight.size(0), m.weight.size(2))
                    for m in (layer.q_conv1d, layer.k_conv1d, layer.v_conv1d)], 0)
    want = FV.causal_conv1d_update(qkv[:n], conv0, wm, None, "silu", conv_state_indices=idx[:n])
    assert torch.equal(c["mixed"], want)
    assert torch.equal(c["a"], g1[0, :n]) and torch.equal(c["b"], beta[0, :n]) and torch.equal(c["idx"], idx[:n])
    assert c["out"].data_ptr() == out.data_ptr() and bool((out[0, :n] == 7).all())


def test_kda_mixed_step(plugin):
    layer = kda_layer()
    nd = 1
    idx = torch.tensor([2, 3, 5], dtype=torch.int32)                      # decode slot first, then the prefill slots
    md = FV.gdn_metadata(nd, idx, prefill_idx=torch.tensor([3, 5], dtype=torch.int32),
                         prefill_loc=torch.tensor([0, 2, 3], dtype=torch.int32))
    md.has_initial_state = torch.tensor([True, True, False])
    md.non_spec_query_start_loc = torch.tensor([0, 1, 3, 4], dtype=torch.int32)
    md.prefill_has_initial_state = torch.tensor([True, False])
    FV.CONTEXT.attn_metadata = {layer.prefix: md}
    T = 4
    qkv = torch.randn(T, 3 * HV * K).to(torch.bfloat16)
    g1 = torch.randn(1, T, HV * K).to(torch.bfloat16)
    beta = torch.randn(1, T, HV).to(torch.bfloat16)
    out = torch.zeros(1, T, HV, K, dtype=torch.bfloat16)
    layer._forward(qkv, g1, beta, out)
    st = plugin.rec[id(layer)]
    assert [c[0] for c in st.calls] == ["decode", "dequantize", "quantize"]
    assert st.calls[0][1]["idx"].tolist() == [2]
    assert st.calls[1][1].tolist() == [3, 5] and st.calls[2][1].tolist() == [3, 5]
    assert FV.CALLS == ["gather_initial_states", "chunk_kda", "scatter_states"]


def test_kda_speculative_and_empty(plugin):
    layer = kda_layer()
    FV.CONTEXT.attn_metadata = {layer.prefix: FV.gdn_metadata(0, torch.zeros(0, dtype=torch.int32))}
    out = torch.zeros(1, 1, HV, K, dtype=torch.bfloat16)
    layer._forward(torch.zeros(1, 3 * HV * K), torch.zeros(1, 1, HV * K), torch.zeros(1, 1, HV), out)
    assert id(layer) not in plugin.rec and FV.CALLS == []               # nothing to do
    md = FV.gdn_metadata(1, torch.tensor([1], dtype=torch.int32), spec_masks=torch.ones(1, dtype=torch.bool),
                         spec_idx=torch.tensor([[2]], dtype=torch.int32))
    FV.CONTEXT.attn_metadata = {layer.prefix: md}
    layer._forward(torch.zeros(1, 3 * HV * K), torch.zeros(1, 1, HV * K), torch.zeros(1, 1, HV), out)
    st = plugin.rec[id(layer)]
    assert [c[0] for c in st.calls] == ["dequantize", "quantize"] and FV.CALLS == ["vllm_kda_forward"]
    layer.kda_lower_bound = None
    with pytest.raises(AssertionError, match="bounded KDA gate"):
        layer._forward(torch.zeros(1, 3 * HV * K), torch.zeros(1, 1, HV * K), torch.zeros(1, 1, HV), out)
