"""A random-init stack of Gated DeltaNet decoder layers (hidden 2048, HV = 32 value / H = 16 key
heads, d = 128, bf16 projections) built on the stand-in vLLM layer (tests/fake_vllm.py), so that a decode step runs
through the LeapQuant plugin hooks exactly as vLLM would call them.

Layer: x + out_proj(gated_rmsnorm(core(conv(in_proj(rmsnorm(x)))), z)), where in_proj gives q | k | v | z and b | a, and
`core` is the layer's _forward_core (patched by the plugin: conv update + the HIP step and flush on the 8-bit state).
Two reference cores run the same layer on other state formats: a dense fp32 gated delta rule in torch (parity) and the
HIP dense bf16-state step (the baseline of the throughput comparison).  Synthetic: random weights, states drawn
N(0, 0.02^2) as the post-prefill fp32 states, then checkpointed (no 8k-token prefill is run).
"""
import types

import torch
import torch.nn.functional as F

from tests import fake_vllm as FV

BF16 = torch.bfloat16


def rmsnorm(x, w, eps=1e-6):
    xf = x.float()
    return (xf * torch.rsqrt((xf * xf).mean(-1, keepdim=True) + eps) * w).to(BF16)


class GDNDecoderLayer(torch.nn.Module):
    def __init__(self, i, hidden, H, HV, D, NS, device, gen, dgen):
        super().__init__()
        self.H, self.HV, self.D = H, HV, D
        M = FV.sys.modules["vllm.model_executor.layers.mamba.gdn.qwen_gdn_linear_attn"]
        self.attn = M.QwenGatedDeltaNetAttention("model.layers.%d.linear_attn" % i, H, HV, D, device=device)
        C = 2 * H * D + HV * D
        rnd = lambda *shape: torch.randn(*shape, generator=dgen, device=device) * 0.02
        with torch.no_grad():
            self.attn.conv1d.weight.copy_(torch.randn(C, 1, 4, generator=gen) * 0.5)
            self.attn.A_log.copy_(torch.log(torch.rand(HV, generator=gen) * 15 + 1))
            self.attn.dt_bias.copy_(torch.rand(HV, generator=gen) - 0.5)
        # projections stored [in, out] and contiguous: every bf16 GEMM below takes untransposed operands (bf16
        # products with a transposed right operand have faulted GPUs of this pool)
        self.w_in = rnd(hidden, 2 * H * D + 2 * HV * D + 2 * HV).to(BF16).contiguous()
        self.w_out = rnd(HV * D, hidden).to(BF16).contiguous()
        self.norm_in = torch.ones(hidden, device=device)
        self.norm_o = torch.ones(D, device=device)
        self.conv = torch.zeros(NS, C, 3, device=device, dtype=BF16)
        self.ssm = torch.empty(NS, HV, D, D, device=device).normal_(0, 0.02, generator=dgen)

    def forward(self, x, core=None):
        """x [B, hidden] bf16 -> [B, hidden].  core(layer, mixed, b, a, out): the recurrent part; None = the layer's
        own _forward_core (the plugin)."""
        B = x.shape[0]
        H, HV, D = self.H, self.HV, self.D
        p = torch.matmul(rmsnorm(x, self.norm_in).contiguous(), self.w_in)
        mixed, z, b, a = p.split([2 * H * D + HV * D, HV * D, HV, HV], -1)
        out = torch.empty(B, HV, D, device=x.device, dtype=BF16)
        if core is None:
            self.attn._forward_core(mixed.contiguous(), b.contiguous(), a.contiguous(), out)
        else:
            core(self, mixed.contiguous(), b.contiguous(), a.contiguous(), out)
        o = rmsnorm(out, self.norm_o).float() * F.silu(z.float().view(B, HV, D))
        return x + torch.matmul(o.reshape(B, HV * D).to(BF16).contiguous(), self.w_out)


def build(layers, hidden=2048, H=16, HV=32, D=128, B=64, device="cuda:0", seed=4):
    """The stack, its per-layer caches (conv state, fp32 state cache of B + 1 slots; slot 0 is padding) and the decode
    metadata of B rows on slots 1..B, installed into the stand-in forward context."""
    gen = torch.Generator().manual_seed(seed)
    dgen = torch.Generator(device=device).manual_seed(seed)
    NS = B + 1
    stack = [GDNDecoderLayer(i, hidden, H, HV, D, NS, device, gen, dgen) for i in range(layers)]
    idx = torch.arange(1, B + 1, device=device, dtype=torch.int32)
    md = FV.gdn_metadata(B, idx)
    FV.CONTEXT.attn_metadata = {l.attn.prefix: md for l in stack}
    for l in stack:
        l.attn.kv_cache = (l.conv, l.ssm)
    return stack, idx


def run(stack, x, core=None):
    for l in stack:
        x = l(x, core)
    return x


def dense_fp32_core(states):
    """Reference core: conv update, then the gated delta rule on dense fp32 states (states[layer]: [NS, HV, V, K]) in
    torch, q / k l2-normalised, beta = sigmoid(b) (kernels.py:129-144, 236-279)."""
    def core(layer, mixed, b, a, out):
        md = FV.CONTEXT.attn_metadata[layer.attn.prefix]
        idx = md.non_spec_state_indices_tensor.long()
        n = idx.shape[0]
        w = layer.attn.conv1d.weight
        x = FV.causal_conv1d_update(mixed, layer.attn.kv_cache[0], w.view(w.size(0), w.size(2)), None, "silu",
                                    conv_state_indices=idx)
        H, HV, D = layer.H, layer.HV, layer.D
        G = HV // H
        q, k, v = x.float().split([H * D, H * D, HV * D], -1)
        l2 = lambda t: t * torch.rsqrt((t * t).sum(-1, keepdim=True) + 1e-6)
        qn = l2(q.view(n, H, D)).repeat_interleave(G, 1) * D ** -0.5
        kn = l2(k.view(n, H, D)).repeat_interleave(G, 1)
        alpha = torch.exp(-torch.exp(layer.attn.A_log.float()) * F.softplus(a.float() + layer.attn.dt_bias.float()))
        beta = torch.sigmoid(b.float()).to(BF16).float()
        S = states[layer.attn.prefix]
        Ss = S[idx] * alpha[:, :, None, None]
        u = beta[:, :, None] * (v.view(n, HV, D) - (Ss * kn[:, :, None, :]).sum(-1))
        Ss = Ss + u[:, :, :, None] * kn[:, :, None, :]
        S[idx] = Ss
        out.copy_((Ss * qn[:, :, None, :]).sum(-1).to(BF16))
    return core


def dense_bf16_core(states):
    """Baseline core: conv update, then the HIP dense-state step (lq_dense_step) on bf16 states [NS, HV, V, K]."""
    from leapquant_amd import kernels as KN

    def core(layer, mixed, b, a, out):
        md = FV.CONTEXT.attn_metadata[layer.attn.prefix]
        idx = md.non_spec_state_indices_tensor
        w = layer.attn.conv1d.weight
        x = FV.causal_conv1d_update(mixed, layer.attn.kv_cache[0], w.view(w.size(0), w.size(2)), None, "silu",
                                    conv_state_indices=idx)
        KN.dense_step(states[layer.attn.prefix], x.contiguous(), a, b, layer.attn.A_log.float(),
                      layer.attn.dt_bias.float(), idx, out, layer.H)
    return core
