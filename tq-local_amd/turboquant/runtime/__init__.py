"""Runtime: libtq kernel wrappers, packed cache, attention backend, generation loop."""
