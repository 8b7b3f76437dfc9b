"""vLLM plugin: keeps the recurrent states of Qwen (Gated DeltaNet) and GLM (Kimi Delta Attention) layers in the 8-bit
checkpoint format, decoding them with the HIP kernels of liblq.

Registered under the entry point ``vllm.general_plugins: leapquant`` (same name as /root/reference/pyproject.toml:14-15);
vLLM calls ``register()`` in every process it starts (reference: leapquant/vllm/__init__.py:22-34).
"""
import os

_DONE = []
NMAX = [0]     # largest decode batch one call can carry, read from the engine config (informational for the HIP flush)


def _track_batch_limit(layer_cls):
    """Wrap a layer constructor so that building the model records max_num_seqs and the largest graph-capture size
    of the config under construction (reference: leapquant/vllm/__init__.py:8-19)."""
    base_init = layer_cls.__init__

    def init(self, *args, **kwargs):
        base_init(self, *args, **kwargs)
        from vllm.config import get_current_vllm_config
        cfg = get_current_vllm_config()
        capture = getattr(cfg.compilation_config, "max_cudagraph_capture_size", None) or 0
        NMAX[0] = max(NMAX[0], cfg.scheduler_config.max_num_seqs, capture)

    init.__wrapped__ = base_init
    layer_cls.__init__ = init


def register():
    """Entry point: patch vLLM's GDN and KDA layers once per process."""
    if _DONE:
        return
    from vllm.model_executor.layers.mamba.gdn import qwen_gdn_linear_attn
    from vllm.models.glm5next.nvidia import kda

    from . import gdn, glm
    _track_batch_limit(qwen_gdn_linear_attn.QwenGatedDeltaNetAttention)
    _track_batch_limit(kda.Glm5NextLinearAttention)
    gdn.install(NMAX)
    glm.install(NMAX)
    _DONE.append(True)
    print("[LeapQuant] 8-bit recurrent states enabled on MI355X HIP kernels (pid %d)" % os.getpid(), flush=True)
