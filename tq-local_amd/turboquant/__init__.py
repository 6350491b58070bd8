"""TurboQuant KV-cache compression for HuggingFace Transformers, MI355X-native (libtq, gfx950)."""

__version__ = "0.1.0"
