"""A stand-in for the parts of vLLM 0.30.0 that the LeapQuant plugin touches (vLLM is not installed in this image).

Module paths, class names, attribute names and call signatures are the plugin's hook points (the reference plugin,
leapquant/vllm/*.py, names them); the behaviour is minimal and written here:
  * causal_conv1d_update / causal_conv1d_fn: depthwise causal conv over [conv_state | x] with optional SiLU;
  * QwenGatedDeltaNetAttention._forward_core: conv, then the decode tokens through the module-level
    fused_sigmoid_gating_delta_rule_update (so the plugin's interception is exercised) and the prefill tokens through a
    plain fp32 gated-delta recurrence on the fp32 state cache;
  * Glm5NextLinearAttention._forward: records that vLLM's own forward ran.
install() puts the modules into sys.modules; uninstall() removes them.
"""
import sys
import types

import torch
import torch.nn.functional as F

_NAMES = ["vllm", "vllm.config", "vllm.forward_context", "vllm.compilation", "vllm.compilation.breakable_cudagraph",
          "vllm.model_executor", "vllm.model_executor.layers", "vllm.model_executor.layers.mamba",
          "vllm.model_executor.layers.mamba.gdn", "vllm.model_executor.layers.mamba.gdn.qwen_gdn_linear_attn",
          "vllm.model_executor.layers.mamba.mamba_utils", "vllm.model_executor.layers.mamba.ops",
          "vllm.model_executor.layers.mamba.ops.causal_conv1d", "vllm.models", "vllm.models.glm5next",
          "vllm.models.glm5next.nvidia", "vllm.models.glm5next.nvidia.kda"]

CALLS = []            # ("vllm_core" | "vllm_recurrent" | "vllm_kda_forward" | ...) in call order
CONFIG = types.SimpleNamespace(scheduler_config=types.SimpleNamespace(max_num_seqs=64),
                               compilation_config=types.SimpleNamespace(max_cudagraph_capture_size=512))
CONTEXT = types.SimpleNamespace(attn_metadata=None)


# ---- conv1d ------------------------------------------------------------------------------------------------------
def _act(y, activation):
    return F.silu(y) if activation in ("silu", "swish", True) else y


ON_DEVICE = [False]   # True: the conv update runs where its tensors live (model loops, graph capture)


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None, conv_state_indices=None,
                         validate_data=False):
    """x [n, C]; conv_state [NS, C, W - 1] (channel-first view); weight [C, W].  Returns [n, C] and shifts the states.
    Computed on the host (unless ON_DEVICE), so an expectation built on the CPU matches it bit for bit."""
    dev = x.device if ON_DEVICE[0] else torch.device("cpu")
    idx = conv_state_indices.long().to(conv_state.device)
    win = torch.cat([conv_state[idx].float().to(dev), x.float().to(dev)[:, :, None]], -1)     # [n, C, W]
    wf = weight.detach().float().to(dev)
    y = win[..., 0] * wf[None, :, 0]                   # taps accumulated left to right, one rounding per operation
    for t in range(1, wf.shape[1]):
        y = y + win[..., t] * wf[None, :, t]
    if bias is not None:
        y = y + bias.detach().float().to(dev)
    conv_state[idx] = win[..., 1:].to(conv_state.dtype).to(conv_state.device)
    return _act(y, activation).to(x.dtype).to(x.device)


def causal_conv1d_fn(x, weight, bias=None, activation=None, conv_states=None, has_initial_state=None,
                     cache_indices=None, query_start_loc=None, metadata=None):
    """x [C, T] over the concatenated sequences of query_start_loc; returns [C, T] (computed on the host)."""
    out = torch.empty(x.shape, dtype=x.dtype)
    W = weight.shape[1]
    wf = weight.detach().float().cpu()
    loc = query_start_loc.tolist()
    for s in range(len(loc) - 1):
        a, b = loc[s], loc[s + 1]
        slot = int(cache_indices[s])
        init = conv_states[slot].float().cpu() if (has_initial_state is None or bool(has_initial_state[s])) else \
            torch.zeros(x.shape[0], W - 1)
        seq = torch.cat([init, x[:, a:b].float().cpu()], 1)
        y = sum(seq[:, i:i + (b - a)] * wf[:, i:i + 1] for i in range(W))
        if bias is not None:
            y = y + bias.detach().float().cpu()[:, None]
        out[:, a:b] = _act(y, activation).to(x.dtype)
        conv_states[slot] = seq[:, -(W - 1):].to(conv_states.dtype).to(conv_states.device)
    return out.to(x.device)


# ---- GDN layer -----------------------------------------------------------------------------------------------------
def fused_sigmoid_gating_delta_rule_update(A_log, a, b, dt_bias, q, k, v, initial_state, inplace_final_state,
                                           cu_seqlens, ssm_state_indices, use_qk_l2norm_in_kernel=True, **kw):
    CALLS.append("vllm_recurrent")
    n = q.shape[1]
    return torch.zeros(1, n, v.shape[2], v.shape[3], dtype=torch.bfloat16, device=q.device), None


def _l2n(x):
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + 1e-6)


def fp32_gdn_prefill(S, A_log, dt_bias, q, k, v, a, b):
    """Plain fp32 gated delta rule over one sequence on the host (vLLM's chunked prefill stand-in).
    S [HV, V, K] fp32 (updated in place); q, k [T, H, K]; v [T, HV, V]; a, b [T, HV].  Returns o [T, HV, V] fp32."""
    HV, H = v.shape[1], q.shape[1]
    G = HV // H
    o = torch.empty(q.shape[0], HV, v.shape[2])
    ea = torch.exp(A_log.detach().float().cpu())
    dtb = dt_bias.detach().float().cpu()
    for t in range(q.shape[0]):
        qn = _l2n(q[t].float().cpu()).repeat_interleave(G, 0) * q.shape[-1] ** -0.5
        kn = _l2n(k[t].float().cpu()).repeat_interleave(G, 0)
        alpha = torch.exp(-ea * F.softplus(a[t].float().cpu() + dtb))
        beta = torch.sigmoid(b[t].float().cpu())
        S.mul_(alpha[:, None, None])
        u = beta[:, None] * (v[t].float().cpu() - (S * kn[:, None, :]).sum(-1))
        S.add_(u[:, :, None] * kn[:, None, :])
        o[t] = (S * qn[:, None, :]).sum(-1)
    return o


class QwenGatedDeltaNetAttention(torch.nn.Module):
    def __init__(self, prefix, num_k_heads, num_v_heads, head_dim, conv_width=4, tp_size=1, device="cpu"):
        super().__init__()
        self.prefix, self.num_k_heads, self.num_v_heads, self.tp_size = prefix, num_k_heads, num_v_heads, tp_size
        self.head_k_dim = self.head_v_dim = head_dim
        C = 2 * num_k_heads * head_dim + num_v_heads * head_dim
        self.conv1d = torch.nn.Conv1d(C, C, conv_width, groups=C, bias=False, device=device)
        self.activation = "silu"
        self.A_log = torch.nn.Parameter(torch.zeros(num_v_heads, device=device))
        self.dt_bias = torch.nn.Parameter(torch.zeros(num_v_heads, device=device))
        self.enable_packed_recurrent_decode = True
        self.kv_cache = None
        self.cache_config = types.SimpleNamespace(mamba_cache_mode="none")

    def _forward_core(self, mixed_qkv, b, a, core_attn_out):
        CALLS.append("vllm_core")
        md = CONTEXT.attn_metadata.get(self.prefix) if isinstance(CONTEXT.attn_metadata, dict) else None
        if md is None:
            return None
        mod = sys.modules["vllm.model_executor.layers.mamba.gdn.qwen_gdn_linear_attn"]
        n, nd = md.num_actual_tokens, md.num_decode_tokens
        H, HV, K = self.num_k_heads, self.num_v_heads, self.head_k_dim
        w = self.conv1d.weight
        conv_state = self.kv_cache[0]
        idx = md.non_spec_state_indices_tensor
        if nd > 0:                                                   # decode tokens first
            x = causal_conv1d_update(mixed_qkv[:nd], conv_state, w.view(w.size(0), w.size(2)), None, "silu",
                                     conv_state_indices=idx[:nd])
            q, k, v = x.split([H * K, H * K, HV * K], -1)
            o, _ = mod.fused_sigmoid_gating_delta_rule_update(
                A_log=self.A_log, a=a[:nd], b=b[:nd], dt_bias=self.dt_bias, q=q.reshape(1, nd, H, K),
                k=k.reshape(1, nd, H, K), v=v.reshape(1, nd, HV, K), initial_state=self.kv_cache[1],
                inplace_final_state=True, cu_seqlens=None, ssm_state_indices=idx[:nd], use_qk_l2norm_in_kernel=True)
            core_attn_out[:nd] = o[0].reshape(nd, -1, K).to(core_attn_out.dtype)
        if n > nd:
            loc = md.prefill_query_start_loc.tolist()
            x = causal_conv1d_fn(mixed_qkv[nd:n].transpose(0, 1), w.view(w.size(0), w.size(2)), None, "silu",
                                 conv_states=conv_state, cache_indices=md.prefill_state_indices,
                                 query_start_loc=md.prefill_query_start_loc).transpose(0, 1)
            q, k, v = x.split([H * K, H * K, HV * K], -1)
            for s in range(len(loc) - 1):
                lo, hi = loc[s], loc[s + 1]
                slot = int(md.prefill_state_indices[s])
                S = self.kv_cache[1][slot].cpu()
                o = fp32_gdn_prefill(S, self.A_log, self.dt_bias, q[lo:hi].reshape(-1, H, K),
                                     k[lo:hi].reshape(-1, H, K), v[lo:hi].reshape(-1, HV, K), a[nd + lo:nd + hi],
                                     b[nd + lo:nd + hi])
                self.kv_cache[1][slot] = S.to(self.kv_cache[1].device)
                core_attn_out[nd + lo:nd + hi] = o.to(core_attn_out.dtype).to(core_attn_out.device)
        return None


# ---- KDA layer -----------------------------------------------------------------------------------------------------
class Glm5NextLinearAttention(torch.nn.Module):
    def __init__(self, prefix, num_heads, head_dim, conv_width=4, lower_bound=-5.0, device="cpu"):
        super().__init__()
        self.prefix, self.local_num_heads, self.head_dim = prefix, num_heads, head_dim
        self.local_projection_size = num_heads * head_dim
        P = self.local_projection_size
        self.q_conv1d = torch.nn.Conv1d(P, P, conv_width, groups=P, bias=False, device=device)
        self.k_conv1d = torch.nn.Conv1d(P, P, conv_width, groups=P, bias=False, device=device)
        self.v_conv1d = torch.nn.Conv1d(P, P, conv_width, groups=P, bias=False, device=device)
        self.A_log = torch.nn.Parameter(torch.zeros(1, 1, num_heads, 1, device=device))
        self.dt_bias = torch.nn.Parameter(torch.zeros(num_heads * head_dim, device=device))
        self.kda_safe_gate, self.kda_lower_bound = True, lower_bound
        self.kda_prefill_backend = "chunk"
        self._merged_conv_weight = None
        self._conv_state_dim_first = True
        self.kv_cache = None
        self.cache_config = types.SimpleNamespace(mamba_cache_mode="none")

    def _forward(self, qkv_proj_states, g1, beta, core_attn_out):
        CALLS.append("vllm_kda_forward")


def gather_initial_states(ssm, idx, has_initial):
    CALLS.append("gather_initial_states")
    return ssm[idx.clamp(min=0).long()].clone()


def scatter_states(ssm, final, idx):
    CALLS.append("scatter_states")
    ssm[idx.long()] = final


def chunk_kda_with_fused_gate(q, k, v, raw_g, beta, A_log, g_bias, initial_state, output_final_state,
                              use_qk_l2norm_in_kernel, cu_seqlens, safe_gate, lower_bound):
    CALLS.append("chunk_kda")
    return torch.zeros_like(v), initial_state


def _cast_sigmoid(x):
    return torch.sigmoid(x.float())


def eager_break_during_capture(fn):
    def wrapper(*a, **k):
        return fn(*a, **k)
    wrapper.__wrapped__ = fn
    wrapper.eager_break = True
    return wrapper


def install():
    """Register the stand-in modules (fresh classes each time, so a patched class never leaks between tests)."""
    uninstall()
    CALLS.clear()
    mods = {n: types.ModuleType(n) for n in _NAMES}
    for n, m in mods.items():
        if "." in n:
            parent, child = n.rsplit(".", 1)
            setattr(mods[parent], child, m)
    mods["vllm.config"].get_current_vllm_config = lambda: CONFIG
    mods["vllm.forward_context"].get_forward_context = lambda: CONTEXT
    mods["vllm.compilation.breakable_cudagraph"].eager_break_during_capture = eager_break_during_capture
    gdn = mods["vllm.model_executor.layers.mamba.gdn.qwen_gdn_linear_attn"]
    gdn.QwenGatedDeltaNetAttention = type("QwenGatedDeltaNetAttention", (QwenGatedDeltaNetAttention,), {})
    gdn.fused_sigmoid_gating_delta_rule_update = fused_sigmoid_gating_delta_rule_update
    mods["vllm.model_executor.layers.mamba.mamba_utils"].is_conv_state_dim_first = lambda: True
    mods["vllm.model_executor.layers.mamba.ops.causal_conv1d"].causal_conv1d_update = causal_conv1d_update
    kda = mods["vllm.models.glm5next.nvidia.kda"]
    kda.Glm5NextLinearAttention = type("Glm5NextLinearAttention", (Glm5NextLinearAttention,), {})
    for f in (causal_conv1d_fn, gather_initial_states, scatter_states, chunk_kda_with_fused_gate, _cast_sigmoid):
        setattr(kda, f.__name__, f)
    sys.modules.update(mods)
    import leapquant_amd.vllm as plugin
    plugin._DONE.clear()
    plugin.NMAX[0] = 0
    return mods


def uninstall():
    for n in _NAMES:
        sys.modules.pop(n, None)


def gdn_metadata(n_dec, idx, prefill_idx=None, prefill_loc=None, spec_masks=None, spec_idx=None):
    """Attention metadata of one GDN layer: n_dec decode tokens first, then prefill sequences (prefill_loc: start offsets
    into the prefill tokens, ending with their count)."""
    n_pre = 0 if prefill_loc is None else int(prefill_loc[-1])
    return types.SimpleNamespace(
        num_actual_tokens=n_dec + n_pre, num_decode_tokens=n_dec, num_decodes=n_dec,
        num_prefills=0 if prefill_idx is None else len(prefill_idx), non_spec_state_indices_tensor=idx,
        prefill_state_indices=prefill_idx, prefill_query_start_loc=prefill_loc, spec_sequence_masks=spec_masks,
        spec_state_indices_tensor=spec_idx, num_spec_decodes=0 if spec_idx is None else len(spec_idx))
