"""Runtime: libtq kernel wrappers, packed cache, attention backend, generation loop."""

from turboquant.runtime.attention import chunked_turboquant_attention, fused_attention, triton_available

__all__ = ["fused_attention", "triton_available", "chunked_turboquant_attention"]
