"""Host-side bounds check of every liblq call the config-4 stack makes (CPU, no GPU).

BASELINE config 4 -- a 24-layer Gated DeltaNet stack (hidden 2048, HV = 32 / H = 16, d = 128, bf16 projections) decoding
at B = 64 through the vLLM plugin hook -- runs here on host tensors with tests/lq_bounds.CheckingLib in place of
liblq.so: each call's footprint (every byte range its kernels read or write, from their index arithmetic) must lie in
the storages the plugin passed.  Covered: the checkpoint of every layer's states, decode steps through the plugin's
unfused route (the stand-in conv update, then LeapQuantState.decode: step + flush) and its fused-conv route
(bf16 width-4 conv: lq_gdn_step_conv + flush), the prefill round trip of a mixed step, and the dense bf16-state
baseline core (lq_dense_step) that the timing compares against.
"""
import pytest
import torch

from tests import fake_vllm as FV
from tests import gdn_stack as GS
from tests import lq_bounds

LAYERS, B = 24, 64


@pytest.fixture
def checked(monkeypatch):
    fake = lq_bounds.install(monkeypatch)
    FV.install()
    import importlib
    P = importlib.import_module("leapquant.vllm")
    P.register()
    yield fake
    from leapquant_amd import state as S
    FV.uninstall()
    S._STATES.clear()
    lq_bounds.clear_factory_caches()


def _stack(bf16_conv):
    stack, idx = GS.build(LAYERS, B=B, device="cpu")
    if bf16_conv:                                     # vLLM's conv weights are bf16: the plugin fuses the conv update
        for l in stack:
            l.attn.conv1d.weight.data = l.attn.conv1d.weight.data.to(torch.bfloat16)
    return stack, idx


@pytest.mark.parametrize("bf16_conv", [False, True])
@pytest.mark.parametrize("deferred", [False, True])
def test_config4_plugin_calls_stay_in_bounds(checked, bf16_conv, deferred):
    """deferred: the states as the plugin builds them (defer_flush=True, lq_gdn_decode_deferred); otherwise built
    beforehand with the reference's arguments (lq_gdn_decode)."""
    from leapquant_amd import state as S
    torch.manual_seed(0)
    stack, idx = _stack(bf16_conv)
    for l in stack:
        S.get_state(l.attn, l.ssm, H=l.H, defer_flush=deferred).quantize(l.ssm, idx)
    x = torch.randn(B, 2048).to(torch.bfloat16)
    with torch.no_grad():
        for _ in range(2):
            x = GS.run(stack, x)
    name = "lq_gdn_decode_deferred" if deferred else "lq_gdn_decode"
    assert checked.calls.count("lq_quantize") == LAYERS
    assert checked.calls.count(name) == 2 * LAYERS
    assert checked.calls.count(name + " flush") == 2 * LAYERS
    # a mixed step on layer 0: 4 decode rows, prefill of slots 5..8 (the fp32 round trip around the engine's prefill)
    l = stack[0]
    md = FV.gdn_metadata(4, idx[:4], prefill_idx=idx[4:8], prefill_loc=torch.tensor([0, 2, 4, 6, 8]))
    FV.CONTEXT.attn_metadata = {l.attn.prefix: md}
    C = 2 * l.H * l.D + l.HV * l.D
    T = 12
    with torch.no_grad():
        l.attn._forward_core(torch.randn(T, C).to(torch.bfloat16), torch.randn(T, l.HV).to(torch.bfloat16),
                             torch.randn(T, l.HV).to(torch.bfloat16), torch.empty(T, l.HV, l.D, dtype=torch.bfloat16))
    assert "lq_dequant" in checked.calls


def test_config4_dense_baseline_calls_stay_in_bounds(checked):
    """The bf16-state baseline core at config 4's batch; its calls are the same for every layer, so two layers."""
    torch.manual_seed(1)
    stack, idx = GS.build(2, B=B, device="cpu")
    dense = {l.attn.prefix: torch.empty(l.ssm.shape, dtype=torch.bfloat16).normal_(0, 0.02) for l in stack}
    x = torch.randn(B, 2048).to(torch.bfloat16)
    with torch.no_grad():
        GS.run(stack, x, GS.dense_bf16_core(dense))
    assert checked.calls.count("lq_dense_step") == 2


def test_checking_lib_catches_an_out_of_range_call(checked):
    """The checker itself: a state struct that claims more slots than its cache holds is reported."""
    from leapquant_amd import kernels as KN
    from leapquant_amd.state import LeapQuantState
    ssm = torch.zeros(3, 2, 128, 128)
    st = LeapQuantState(ssm, 1, L=16)
    bad = KN.state_struct(ssm, st.SS, st.Kbuf, st.Ubuf, st.Wbuf, st.Pbuf, None, st.hcnt, 4, 2, 1, 128, 128, 16, 4)
    idx = torch.tensor([3], dtype=torch.int32)
    import ctypes
    with pytest.raises(lq_bounds.OutOfBounds, match="ssm block"):
        checked.lq_flush(ctypes.byref(bad), KN._p(st.Q0), KN._p(idx), 1, 0, ctypes.c_float(127.0), None)


def _op_signatures(layers, B, deferred=True):
    """The aten ops of one decode step of the stack (through the plugin, after its checkpoints are written), each as
    (op, per tensor operand: dtype, contiguous, a transposed 2-D view, byte offset of the view modulo 16), and the
    liblq calls of that step with the byte alignment of every pointer they were handed."""
    from torch.utils import _pytree as pytree
    from torch.utils._python_dispatch import TorchDispatchMode
    from leapquant_amd import state as S

    class Rec(TorchDispatchMode):
        def __init__(self):
            super().__init__()
            self.ops = []

        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            kwargs = kwargs or {}
            ts = [a for a in pytree.tree_leaves((args, kwargs)) if isinstance(a, torch.Tensor)]
            self.ops.append((str(func), tuple(
                (str(t.dtype), t.is_contiguous(), t.dim() == 2 and t.stride(0) == 1 and t.shape[0] > 1,
                 (t.storage_offset() * t.element_size()) % 16) for t in ts)))
            return func(*args, **kwargs)

    torch.manual_seed(0)
    stack, idx = GS.build(layers, B=B, device="cpu")
    for l in stack:
        S.get_state(l.attn, l.ssm, H=l.H, defer_flush=deferred).quantize(l.ssm, idx)
    x = torch.randn(B, 2048).to(torch.bfloat16)
    rec = Rec()
    with torch.no_grad(), rec:
        GS.run(stack, x)
    return rec.ops


def test_config4_step_differs_from_the_passing_stack_only_in_sizes(checked):
    """One decode step of BASELINE config 4 (24 layers, B = 64) against the stack that runs on the GPU in
    tests/test_gpu_config4.py (4 layers, B = 8): the same aten ops in the same order per layer, with the same dtypes,
    layouts (no transposed operand, in particular no bf16 product with a transposed right operand) and view offsets,
    and the same liblq entry points with 16-byte aligned pointers.  What config 4 adds is sizes: the batch of the
    projections' bf16 GEMMs (M = 64), of the conv update and of the two liblq calls per layer."""
    big = _op_signatures(24, 64)
    n_big = len(checked.calls)
    small = _op_signatures(4, 8)
    per_layer = lambda ops, L: ops[: len(ops) // L]
    assert len(big) % 24 == 0 and len(small) % 4 == 0
    assert per_layer(big, 24) == per_layer(small, 4)
    assert big == per_layer(big, 24) * 24
    mm = [o for o in big if "mm" in o[0]]
    assert mm and all(not any(t[2] for t in o[1]) for o in mm)          # no transposed GEMM operand
    calls = checked.calls[n_big - 48:n_big]                            # one step of 24 layers: decode + its flush
    assert calls == ["lq_gdn_decode_deferred", "lq_gdn_decode_deferred flush"] * 24
    assert all(a % 16 == 0 for a in checked.alignments), sorted(set(a % 256 for a in checked.alignments))
