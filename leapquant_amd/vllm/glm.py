"""LeapQuant on vLLM's GLM Kimi Delta Attention layers (Glm5NextLinearAttention), reference:
leapquant/vllm/glm.py:12-77.

* Decode-only steps: vLLM's conv1d update over the merged q | k | v conv weights, then the HIP KDA step + flush.
* Steps with prefill tokens: the decode tokens go first through the HIP step; the prefill slots are dequantised to
  fp32, run through vLLM's chunked KDA prefill (or its flashkda backend), scattered back and re-quantised.
* Speculative decoding: every touched slot takes the fp32 round trip around vLLM's own forward.
The replacement forward stays an eager break of vLLM's breakable CUDA graph, as vLLM's own forward is.
"""
import torch

from ..state import get_state


def _state_of(layer, nmax):
    return get_state(layer, layer.kv_cache[1], H=layer.local_num_heads, kda=True,
                     gate_lower_bound=float(layer.kda_lower_bound), nmax=nmax[0])


def _merged_conv_weight(layer):
    """[q | k | v] depthwise conv weights as one [C, W] matrix (built once per layer)."""
    if layer._merged_conv_weight is None:
        parts = [m.weight.view(m.weight.size(0), m.weight.size(2)) for m in (layer.q_conv1d, layer.k_conv1d,
                                                                             layer.v_conv1d)]
        layer._merged_conv_weight = torch.cat(parts, 0).contiguous()
    return layer._merged_conv_weight


def install(nmax):
    from vllm.compilation.breakable_cudagraph import eager_break_during_capture
    from vllm.forward_context import get_forward_context
    from vllm.model_executor.layers.mamba.ops.causal_conv1d import causal_conv1d_update
    from vllm.models.glm5next.nvidia import kda as mod

    layer_cls = mod.Glm5NextLinearAttention
    vllm_forward = getattr(layer_cls._forward, "__wrapped__", layer_cls._forward)

    def spec_round_trip(self, st, m, qkv_proj_states, g1, beta, core_attn_out):
        parts = [t.reshape(-1) for t in (m.non_spec_state_indices_tensor, m.spec_state_indices_tensor) if t is not None]
        slots = torch.cat(parts).clamp(min=0)
        st.dequantize(self.kv_cache[1], slots)
        vllm_forward(self, qkv_proj_states=qkv_proj_states, g1=g1, beta=beta, core_attn_out=core_attn_out)
        st.quantize(self.kv_cache[1], slots)

    def mixed_step(self, st, m, conv_state, qkv_proj_states, g1, beta, core_attn_out):
        n, nd = m.num_actual_tokens, m.num_decode_tokens
        idx_all = m.non_spec_state_indices_tensor
        x = mod.causal_conv1d_fn(qkv_proj_states[:n].transpose(0, 1), _merged_conv_weight(self), self.q_conv1d.bias,
                                 activation="silu", conv_states=conv_state, has_initial_state=m.has_initial_state,
                                 cache_indices=idx_all, query_start_loc=m.non_spec_query_start_loc,
                                 metadata=m).transpose(0, 1)
        if nd > 0:                                           # the decode tokens come first in the batch
            st.decode(self.kv_cache[1], x[:nd].contiguous(), g1[0, :nd], beta[0, :nd].contiguous(), self.A_log.view(-1),
                      self.dt_bias, idx_all[:nd], core_attn_out[0, :nd])
        pidx = m.prefill_state_indices
        st.dequantize(self.kv_cache[1], pidx.clamp(min=0))
        init = mod.gather_initial_states(self.kv_cache[1], pidx, m.prefill_has_initial_state)
        q, k, v = (t.reshape(1, -1, self.local_num_heads, self.head_dim)
                   for t in x[nd:n].split(self.local_projection_size, dim=-1))
        if self.kda_prefill_backend == "flashkda":
            out_p, final = self._flashkda_prefill(q=q, k=k, v=v, g=g1[:, nd:n], beta=beta[:, nd:n], initial_state=init,
                                                  cu_seqlens=m.prefill_query_start_loc, out=None)
        else:
            out_p, final = mod.chunk_kda_with_fused_gate(
                q=q, k=k, v=v, raw_g=g1[:, nd:n], beta=mod._cast_sigmoid(beta[:, nd:n].squeeze(0)).unsqueeze(0),
                A_log=self.A_log, g_bias=self.dt_bias, initial_state=init, output_final_state=True,
                use_qk_l2norm_in_kernel=True, cu_seqlens=m.prefill_query_start_loc, safe_gate=self.kda_safe_gate,
                lower_bound=self.kda_lower_bound)
        mod.scatter_states(self.kv_cache[1], final, pidx)
        core_attn_out[0, nd:n] = out_p[0, :n - nd]
        st.quantize(self.kv_cache[1], pidx.clamp(min=0))   # the checkpoint is written when the prefill ends

    def forward(self, qkv_proj_states, g1, beta, core_attn_out):
        md = get_forward_context().attn_metadata
        m = md.get(self.prefix) if isinstance(md, dict) else None
        if m is None or m.num_actual_tokens == 0:
            return
        assert self.kda_safe_gate and self.kda_lower_bound is not None, "LeapQuant supports the bounded KDA gate only"
        st = _state_of(self, nmax)
        if m.spec_sequence_masks is not None and m.num_spec_decodes > 0:
            return spec_round_trip(self, st, m, qkv_proj_states, g1, beta, core_attn_out)
        conv_state = self.kv_cache[0] if self._conv_state_dim_first else self.kv_cache[0].transpose(-1, -2)
        if m.num_prefills > 0:
            return mixed_step(self, st, m, conv_state, qkv_proj_states, g1, beta, core_attn_out)
        n = m.num_actual_tokens
        idx = m.non_spec_state_indices_tensor[:n]
        mixed = causal_conv1d_update(qkv_proj_states[:n], conv_state, _merged_conv_weight(self), self.q_conv1d.bias,
                                     activation="silu", conv_state_indices=idx)
        st.decode(self.kv_cache[1], mixed.contiguous(), g1[0, :n], beta[0, :n].contiguous(), self.A_log.view(-1),
                  self.dt_bias, idx, core_attn_out[0, :n])

    layer_cls._forward = eager_break_during_capture(forward)
