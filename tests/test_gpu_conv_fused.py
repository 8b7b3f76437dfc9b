"""GPU: the conv1d update fused into the GDN step (lq_gdn_step_conv, LeapQuantState.decode_conv) against the unfused
path (the stand-in vLLM conv update on the device, then lq_gdn_step) on the same state: the conv states advance
identically (a shift of the inputs), the outputs and window buffers agree (the conv output is the same fp32 sum of
products rounded to bf16; SiLU's exp may differ in the last fp32 bit), across a window boundary (step + flush)."""
import numpy as np
import pytest
import torch

from tests import fake_vllm as FV
from tests import lqgpu as G
from tests.fixtures import make_state

pytestmark = pytest.mark.gpu
NS, L = 6, 16


# (conv-state layout, bias, key heads H, value heads HV, K, V): GQA 2 / 1 / 4 (the kernel's G) and the 64-dim heads
@pytest.mark.parametrize("dim_first,with_bias,H,HV,K,V", [
    (True, False, 2, 4, 128, 128), (False, True, 2, 4, 128, 128), (True, True, 4, 4, 128, 128),
    (True, False, 1, 4, 128, 128), (True, True, 2, 4, 64, 128), (False, False, 2, 4, 64, 64)])
def test_fused_conv_step_matches_conv_then_step(dim_first, with_bias, H, HV, K, V):
    C = 2 * H * K + HV * V
    rng = np.random.default_rng(31)
    st, _, _ = make_state(rng, NS, HV, H, K=K, V=V, L=L)
    ssm_a, lq_a = G.to_gpu(st)
    ssm_b, lq_b = G.to_gpu(st)
    gen = torch.Generator(device=G.DEV).manual_seed(3)
    if dim_first:
        conv_a = torch.randn(NS, C, 3, generator=gen, device=G.DEV).to(torch.bfloat16)
        view = lambda t: t
    else:                                                         # vLLM's other layout: [NS, W - 1, C], used transposed
        conv_a = torch.randn(NS, 3, C, generator=gen, device=G.DEV).to(torch.bfloat16)
        view = lambda t: t.transpose(-1, -2)
    conv_b = conv_a.clone()
    w = (torch.randn(C, 4, generator=gen, device=G.DEV) * 0.5).to(torch.bfloat16)
    bias = (torch.randn(C, generator=gen, device=G.DEV) * 0.1).to(torch.bfloat16) if with_bias else None
    idx = torch.tensor([3, 0, 1, 5], dtype=torch.int32, device=G.DEV)      # row 1 is padding
    n = idx.shape[0]
    A_log = torch.zeros(HV, device=G.DEV)
    dt_bias = torch.zeros(HV, device=G.DEV)
    FV.ON_DEVICE[0] = True
    try:
        for t in range(L + 3):
            x = torch.randn(n, C, generator=gen, device=G.DEV).to(torch.bfloat16)
            a = (torch.rand(n, HV, generator=gen, device=G.DEV) * 2).to(torch.bfloat16)
            b = torch.randn(n, HV, generator=gen, device=G.DEV).to(torch.bfloat16)
            out_a = torch.zeros(n, HV, V, dtype=torch.bfloat16, device=G.DEV)
            out_b = torch.zeros_like(out_a)
            live = idx.long() > 0                                  # padding rows keep their conv state (as vLLM's)
            mixed = torch.zeros(n, C, dtype=torch.bfloat16, device=G.DEV)
            mixed[live] = FV.causal_conv1d_update(x[live], view(conv_a), w, bias, "silu",
                                                  conv_state_indices=idx[live])
            lq_a.decode(ssm_a, mixed, a, b, A_log, dt_bias, idx, out_a)
            lq_b.decode_conv(ssm_b, x, view(conv_b), w, bias, True, a, b, A_log, dt_bias, idx, out_b)
            torch.cuda.synchronize()
            assert torch.equal(conv_a, conv_b), t
            np.testing.assert_allclose(out_b.float().cpu().numpy(), out_a.float().cpu().numpy(), rtol=2e-2, atol=1e-3,
                                       err_msg="step %d" % t)
            assert bool((out_b[1] == 0).all())
    finally:
        FV.ON_DEVICE[0] = False
    ga, gb = G.from_gpu(ssm_a, lq_a), G.from_gpu(ssm_b, lq_b)
    assert np.array_equal(ga["hcnt"], gb["hcnt"])
    for s in (1, 3, 5):
        frac, mx = G.code_mismatch(ga["Sq"][s], gb["Sq"][s])
        assert mx <= 1 and frac <= 1e-3, (s, frac, mx)
    np.testing.assert_allclose(gb["Ubuf"].astype(np.float32), ga["Ubuf"].astype(np.float32), rtol=2e-2, atol=1e-3)


def test_conv_update_kernel_matches_stand_in():
    """The standalone conv update (lq_conv_update, the bench's unfused baseline) against the stand-in vLLM conv on the
    device: outputs equal up to SiLU's last fp32 bit before bf16 rounding, conv states identical, padding rows untouched."""
    from leapquant_amd import kernels as KN
    C = 2 * 2 * 128 + 4 * 128
    gen = torch.Generator(device=G.DEV).manual_seed(9)
    conv_a = torch.randn(NS, C, 3, generator=gen, device=G.DEV).to(torch.bfloat16)
    conv_b = conv_a.clone()
    w = (torch.randn(C, 4, generator=gen, device=G.DEV) * 0.5).to(torch.bfloat16)
    idx = torch.tensor([3, 0, 1, 5], dtype=torch.int32, device=G.DEV)
    x = torch.randn(4, C, generator=gen, device=G.DEV).to(torch.bfloat16)
    out = torch.zeros(4, C, dtype=torch.bfloat16, device=G.DEV)
    KN.conv_update(x, conv_b, w, None, idx, out, True)
    FV.ON_DEVICE[0] = True
    try:
        live = idx.long() > 0
        want = FV.causal_conv1d_update(x[live], conv_a, w, None, "silu", conv_state_indices=idx[live])
    finally:
        FV.ON_DEVICE[0] = False
    torch.cuda.synchronize()
    assert torch.equal(conv_a, conv_b)
    d = (out[live].float() - want.float()).abs()
    assert float(d.max()) <= float(want.float().abs().max()) * 2 ** -7
    assert float((d > 0).float().mean()) <= 1e-2
    assert bool((out[1] == 0).all())
