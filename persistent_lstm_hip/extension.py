"""`persistent_lstm_hip.extension` (reference extension.py:7-12) -> persistent_lstm_hip_amd.extension:
`load_extension()` returns the native extension object (with the reference's ten entry points) or
None when the library cannot be loaded."""
from persistent_lstm_hip_amd.extension import load_extension  # noqa: F401
