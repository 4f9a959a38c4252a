"""`persistent_lstm_hip.packing` (reference packing.py:10-73) -> persistent_lstm_hip_amd.packing."""
from persistent_lstm_hip_amd.packing import (  # noqa: F401
    PackedLSTMLayerWeights,
    PackedLSTMWeights,
    PackedRegressorWeights,
    pack_lstm_module,
    pack_regressor_module,
)
