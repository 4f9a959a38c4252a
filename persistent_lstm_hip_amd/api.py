"""Conversion helpers with the reference's names and contracts (persistent_lstm_hip/api.py:10-43)."""
from __future__ import annotations

import copy

import torch.nn as nn

from .model import NativeModuleFallback, PersistentLSTM, PersistentLSTMRegressor


def convert_lstm_module(lstm: nn.LSTM) -> PersistentLSTM:
    return PersistentLSTM.from_native_module(lstm)


def convert_regressor_module(model: nn.Module) -> nn.Module:
    """`.lstm` + `.linear` model -> PersistentLSTMRegressor, or NativeModuleFallback (a deep copy of
    the model, run unchanged) when its structure or size is outside what the kernels implement.
    Raises ValueError when the model has no `.lstm` / `.linear` or `.lstm` is not an nn.LSTM."""
    if not hasattr(model, "lstm") or not hasattr(model, "linear"):
        raise ValueError("convert_regressor_module needs a model with `.lstm` and `.linear`")
    if not isinstance(model.lstm, nn.LSTM):
        raise ValueError("model.lstm must be an nn.LSTM")
    if not isinstance(model.linear, nn.Linear):
        return NativeModuleFallback(copy.deepcopy(model), "native_pytorch_unsupported_head")
    try:
        converted = PersistentLSTMRegressor.from_native_module(model)
    except ValueError:
        return NativeModuleFallback(copy.deepcopy(model), "native_pytorch_unsupported_lstm")
    if converted._can_use_specialized_regressor_hip():
        return converted
    return NativeModuleFallback(copy.deepcopy(model), "native_pytorch_unsupported_geometry")


def replace_lstm_inplace(model: nn.Module) -> nn.Module:
    for name, child in list(model.named_children()):
        if isinstance(child, nn.LSTM):
            setattr(model, name, PersistentLSTM.from_native_module(child))
        else:
            replace_lstm_inplace(child)
    return model


def convert_model_copy(model: nn.Module) -> nn.Module:
    return replace_lstm_inplace(copy.deepcopy(model))
