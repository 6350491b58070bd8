"""Package-wide defaults (reference ``constants.py``)."""

DEFAULT_MAX_NEW_TOKENS = 1024
