"""Runtime: libtq kernel wrappers, packed cache, attention backend, generation loop."""

from turboquant.runtime.attention import fused_attention

__all__ = ["fused_attention"]
