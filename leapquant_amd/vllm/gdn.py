"""LeapQuant on vLLM's Gated DeltaNet layers (QwenGatedDeltaNetAttention), reference: leapquant/vllm/gdn.py:11-81.

* A step with only decode tokens: vLLM's conv1d update, then the HIP step + flush on the 8-bit state, writing straight
  into the layer's output buffer; with a bf16 conv of width 4 the conv update runs inside the step (lq_gdn_step_conv).
* A step with prefill tokens: the prefill slots are dequantised to fp32, vLLM's own forward runs (its chunked prefill
  sees ordinary fp32 states), and the slots are re-quantised afterwards.  The decode tokens of such a step reach vLLM's
  fused recurrent decode function, which is intercepted and sent through the HIP step instead, so a decode slot is
  never round-tripped.
* Speculative decoding: every touched slot takes the fp32 round trip and vLLM's own kernels run.
"""
import torch

from ..state import get_state


def _state_of(layer, nmax):
    # deferred flushes (lq_gdn_decode_deferred): under continuous batching rows reach the end of their window on
    # different calls, and a row due on a call then costs it one head flush instead of two; the outputs are the same,
    # and the prefill round trip (dequantize) flushes a slot's deferred head before it reads the state
    return get_state(layer, layer.kv_cache[1], H=layer.num_k_heads // layer.tp_size, nmax=nmax[0], defer_flush=True)


def _metadata(layer, get_forward_context):
    md = get_forward_context().attn_metadata
    return md.get(layer.prefix) if isinstance(md, dict) else None


def install(nmax):
    from vllm.forward_context import get_forward_context
    from vllm.model_executor.layers.mamba.gdn import qwen_gdn_linear_attn as mod
    from vllm.model_executor.layers.mamba.mamba_utils import is_conv_state_dim_first
    from vllm.model_executor.layers.mamba.ops.causal_conv1d import causal_conv1d_update

    layer_cls = mod.QwenGatedDeltaNetAttention
    vllm_core = layer_cls._forward_core
    vllm_recurrent = mod.fused_sigmoid_gating_delta_rule_update
    routing = {"layer": None}        # the layer whose mixed prefill + decode forward is running

    def decode_only(layer, mixed_qkv, b, a, core_attn_out, md):
        n = md.num_actual_tokens
        idx = md.non_spec_state_indices_tensor[:n]
        conv_state = layer.kv_cache[0]
        if not is_conv_state_dim_first():
            conv_state = conv_state.transpose(-1, -2)
        w = layer.conv1d.weight
        w2 = w.view(w.size(0), w.size(2))
        st = _state_of(layer, nmax)
        bias = layer.conv1d.bias
        if (conv_state.dtype == torch.bfloat16 and w2.dtype == torch.bfloat16 and w2.shape[1] == 4
                and (bias is None or bias.dtype == torch.bfloat16) and layer.activation in ("silu", "swish", None)):
            # bf16 conv of width 4: the conv update runs inside the HIP step (one launch, no round trip of the conv
            # output through memory)
            st.decode_conv(layer.kv_cache[1], mixed_qkv[:n].contiguous(), conv_state, w2.contiguous(), bias,
                           layer.activation is not None, a[:n].contiguous(), b[:n].contiguous(), layer.A_log,
                           layer.dt_bias, idx, core_attn_out[:n].view(n, st.HV, st.V))
            return
        mixed = causal_conv1d_update(mixed_qkv[:n], conv_state, w2, bias, layer.activation, conv_state_indices=idx,
                                     validate_data=False)
        st.decode(layer.kv_cache[1], mixed.contiguous(), a[:n].contiguous(), b[:n].contiguous(), layer.A_log,
                  layer.dt_bias, idx, core_attn_out[:n].view(n, st.HV, st.V))

    def recurrent(A_log, a, b, dt_bias, q, k, v, initial_state, inplace_final_state, cu_seqlens, ssm_state_indices,
                  use_qk_l2norm_in_kernel=True, **kw):
        """vLLM's one-token recurrent update inside a mixed step -> the HIP step on the 8-bit state."""
        layer = routing["layer"]
        if layer is None or kw.get("num_accepted_tokens") is not None or q.shape[0] != 1:
            return vllm_recurrent(A_log=A_log, a=a, b=b, dt_bias=dt_bias, q=q, k=k, v=v, initial_state=initial_state,
                                  inplace_final_state=inplace_final_state, cu_seqlens=cu_seqlens,
                                  ssm_state_indices=ssm_state_indices,
                                  use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel, **kw)
        st = _state_of(layer, nmax)
        n = q.shape[1]
        mixed = torch.cat([q.reshape(n, -1), k.reshape(n, -1), v.reshape(n, -1)], 1).to(torch.bfloat16).contiguous()
        out = torch.empty(n, st.HV, st.V, dtype=torch.bfloat16, device=q.device)
        st.decode(layer.kv_cache[1], mixed, a[:n].contiguous(), b[:n].contiguous(), A_log, dt_bias,
                  ssm_state_indices[:n], out)
        return out.unsqueeze(0), None

    def forward_core(self, mixed_qkv, b, a, core_attn_out):
        md = _metadata(self, get_forward_context)
        if md is None:                                        # profiling and warm-up runs carry no metadata
            return vllm_core(self, mixed_qkv, b, a, core_attn_out)
        spec = md.spec_sequence_masks is not None
        if self.enable_packed_recurrent_decode and not spec and md.num_prefills == 0 and md.num_decodes > 0:
            return decode_only(self, mixed_qkv, b, a, core_attn_out, md)
        if not spec and md.prefill_state_indices is not None:
            slots = md.prefill_state_indices.reshape(-1).clamp(min=0)    # only the prefill slots go to fp32
            route = True
        else:
            parts = [t.reshape(-1) for t in (md.non_spec_state_indices_tensor, md.spec_state_indices_tensor)
                     if t is not None]
            if not parts:
                return vllm_core(self, mixed_qkv, b, a, core_attn_out)
            slots = torch.cat(parts).clamp(min=0)
            route = False
        st = _state_of(self, nmax)
        st.dequantize(self.kv_cache[1], slots)
        routing["layer"] = self if route else None
        try:
            result = vllm_core(self, mixed_qkv, b, a, core_attn_out)
        finally:
            routing["layer"] = None
        st.quantize(self.kv_cache[1], slots)
        return result

    forward_core.__wrapped__ = vllm_core
    recurrent.__wrapped__ = vllm_recurrent
    mod.fused_sigmoid_gating_delta_rule_update = recurrent
    layer_cls._forward_core = forward_core
