"""leapquant_amd: MI355X-native (gfx950 HIP) INT8 recurrent-state decode path for Gated DeltaNet / Kimi Delta
Attention, a drop-in for leapquant.kernels / leapquant.state / leapquant.vllm."""
__version__ = "0.1.0"
