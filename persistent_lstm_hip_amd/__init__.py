"""MI355X-native stacked LSTM + Linear inference forward (gfx950 HIP kernels behind a C ABI).

Public surface mirrors mantuoluozk/persistent_lstm_hip's `persistent_lstm_hip` package
(persistent_lstm_hip/__init__.py:1-20).
"""
from .api import convert_lstm_module, convert_model_copy, convert_regressor_module, replace_lstm_inplace
from .extension import load_extension
from .model import (
    NativeModuleFallback,
    PersistentLSTM,
    PersistentLSTM4LayerRegressor,
    PersistentLSTMRegressor,
    StandardLSTMRegressor,
)

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
    "load_extension",
]
