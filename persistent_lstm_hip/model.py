"""`persistent_lstm_hip.model` (reference model.py) -> persistent_lstm_hip_amd.model."""
from persistent_lstm_hip_amd.model import (  # noqa: F401
    NativeModuleFallback,
    PersistentLSTM,
    PersistentLSTM4LayerRegressor,
    PersistentLSTMRegressor,
    StandardLSTMRegressor,
)
