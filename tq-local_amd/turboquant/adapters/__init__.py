"""Runtime adapters for supported inference backends."""
