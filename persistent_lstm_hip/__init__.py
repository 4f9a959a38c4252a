"""The reference's import name for this build.

The reference's scripts import `persistent_lstm_hip` (LSTM-hip.py:7: `from persistent_lstm_hip
import convert_regressor_module`; benchmark_persistent_lstm.py:5-8: `from persistent_lstm_hip.model
import PersistentLSTMRegressor, StandardLSTMRegressor`).  This package gives those names, with the
reference's submodules (`.api`, `.model`, `.packing`, `.extension`), to the MI355X implementation
in `persistent_lstm_hip_amd`, so the scripts run unchanged.  It holds no code of its own.
"""
from persistent_lstm_hip_amd import (  # noqa: F401
    NativeModuleFallback,
    PersistentLSTM,
    PersistentLSTM4LayerRegressor,
    PersistentLSTMRegressor,
    StandardLSTMRegressor,
    convert_lstm_module,
    convert_model_copy,
    convert_regressor_module,
    load_extension,
    replace_lstm_inplace,
)

from . import api, extension, model, packing  # noqa: F401,E402

__all__ = [
    "PersistentLSTM",
    "PersistentLSTMRegressor",
    "PersistentLSTM4LayerRegressor",
    "NativeModuleFallback",
    "StandardLSTMRegressor",
    "convert_lstm_module",
    "convert_regressor_module",
    "replace_lstm_inplace",
    "convert_model_copy",
]
