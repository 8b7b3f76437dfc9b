"""Config 4 on the GPU: a random-init stack of Gated DeltaNet decoder layers (tests/gdn_stack.py: hidden 2048,
HV = 32 / H = 16, d = 128, bf16 projections) decoding through the LeapQuant vLLM plugin hooks, against the same stack
on dense fp32 states in torch started from the same logical states (the dequantised checkpoints).

The stack's per-token update (the sum of the layers' out_proj contributions) agrees with the fp32 recurrence to
~0.5e-2 on the first token (bf16 outputs of every layer) and ~1.1e-2 from the second token on, before and after the
flush that re-quantises every state: the window holds bf16 copies of u_j and k_j (Ubuf / Kbuf are bf16 in the
reference's design).  The bar is 3e-2 on every token.  The whole decode step is also captured in a HIP graph and replayed (the plugin path is
capture-safe: fixed grids, device-side due detection, no host synchronisation)."""
import pytest
import torch

from tests import fake_vllm as FV
from tests import gdn_stack as GS

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture
def plugin():
    FV.install()
    FV.ON_DEVICE[0] = True
    import leapquant_amd.vllm as P
    P.register()
    yield
    from leapquant_amd import state as S
    FV.ON_DEVICE[0] = False
    FV.uninstall()
    S._STATES.clear()


def _checkpoint(stack, idx):
    """Quantise every layer's post-prefill fp32 states in place; return the fp32 logical states they now hold."""
    from leapquant_amd import state as S
    ref = {}
    for l in stack:
        st = S.get_state(l.attn, l.ssm, H=l.H)
        st.quantize(l.ssm, idx)
        c = l.ssm.clone()
        S.LeapQuantState(c, l.H, L=st.L).dequantize(c, idx)
        ref[l.attn.prefix] = c
    return ref, st.L


def test_stack_decode_through_plugin_matches_fp32(plugin):
    B, layers = 8, 4
    stack, idx = GS.build(layers, B=B)
    ref, L = _checkpoint(stack, idx)
    conv0 = [l.conv.clone() for l in stack]
    T = L + 6                                        # crosses one window boundary
    gen = torch.Generator(device=DEV).manual_seed(5)
    xs = [torch.randn(B, 2048, generator=gen, device=DEV).to(torch.bfloat16) for _ in range(T)]
    out_q = [GS.run(stack, x) for x in xs]
    for l, c in zip(stack, conv0):
        l.conv.copy_(c)
    core = GS.dense_fp32_core(ref)
    out_r = [GS.run(stack, x, core) for x in xs]
    for t in range(T):
        dq = out_q[t].float() - xs[t].float()
        dr = out_r[t].float() - xs[t].float()
        rel = float((dq - dr).norm() / dr.norm())
        assert rel <= 3e-2, (t, rel)


def test_stack_decode_step_replays_as_a_graph(plugin):
    B, layers = 8, 2
    stack, idx = GS.build(layers, B=B)
    _checkpoint(stack, idx)
    x = torch.randn(B, 2048, device=DEV).to(torch.bfloat16)
    for _ in range(3):                               # eager warm-up: states and workspaces exist before capture
        GS.run(stack, x)
    torch.cuda.synchronize()
    snap = [(l.conv.clone(), l.ssm.clone()) for l in stack]
    from leapquant_amd import state as S
    bufs = [S.get_state(l.attn, l.ssm, H=l.H) for l in stack]
    snapb = [(s.Kbuf.clone(), s.Ubuf.clone(), s.Wbuf.clone(), s.Pbuf.clone(), s.hcnt.clone(), s.ctl.clone())
             for s in bufs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = GS.run(stack, x)
    # the capture did not run the kernels: restore, then replay against eager from the same starting point
    eager = []
    for l, (c, s) in zip(stack, snap):
        l.conv.copy_(c)
        l.ssm.copy_(s)
    for s, b in zip(bufs, snapb):
        for t, v in zip((s.Kbuf, s.Ubuf, s.Wbuf, s.Pbuf, s.hcnt, s.ctl), b):
            t.copy_(v)
    for _ in range(20):                              # crosses the window boundary (L = 16)
        eager.append(GS.run(stack, x).clone())
    for l, (c, s) in zip(stack, snap):
        l.conv.copy_(c)
        l.ssm.copy_(s)
    for s, b in zip(bufs, snapb):
        for t, v in zip((s.Kbuf, s.Ubuf, s.Wbuf, s.Pbuf, s.hcnt, s.ctl), b):
            t.copy_(v)
    for k in range(20):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager[k]), k
