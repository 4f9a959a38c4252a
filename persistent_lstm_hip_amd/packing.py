"""Capture of nn.LSTM / nn.Linear parameters (the reference's packing.py:10-73 contract).

The dataclasses and the validation mirror the reference: only batch_first, unidirectional LSTMs
without projections are accepted (packing.py:38-44 raises ValueError otherwise).  The layout the
kernels consume is produced later, on the device, by NativeLibrary.pack.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import torch
import torch.nn as nn


@dataclass
class PackedLSTMLayerWeights:
    weight_ih: torch.Tensor
    weight_hh: torch.Tensor
    bias_ih: Optional[torch.Tensor]
    bias_hh: Optional[torch.Tensor]

    @property
    def bias(self) -> torch.Tensor:
        """Fused bias b_ih + b_hh (zeros for a bias-free LSTM)."""
        parts = [b for b in (self.bias_ih, self.bias_hh) if b is not None]
        if not parts:
            return torch.zeros(self.weight_hh.shape[0], dtype=self.weight_hh.dtype, device=self.weight_hh.device)
        return (parts[0] + parts[1] if len(parts) == 2 else parts[0]).contiguous()


@dataclass
class PackedLSTMWeights:
    input_size: int
    hidden_size: int
    num_layers: int
    batch_first: bool
    layers: List[PackedLSTMLayerWeights]


@dataclass
class PackedRegressorWeights:
    lstm: PackedLSTMWeights
    linear_weight: torch.Tensor
    linear_bias: Optional[torch.Tensor]


def pack_lstm_module(lstm: nn.LSTM) -> PackedLSTMWeights:
    if not lstm.batch_first:
        raise ValueError("only batch_first=True LSTMs are supported")
    if lstm.bidirectional:
        raise ValueError("only unidirectional LSTMs are supported")
    if getattr(lstm, "proj_size", 0) != 0:
        raise ValueError("LSTMs with proj_size are not supported")
    layers: List[PackedLSTMLayerWeights] = []
    for l in range(lstm.num_layers):
        layers.append(
            PackedLSTMLayerWeights(
                weight_ih=getattr(lstm, f"weight_ih_l{l}").contiguous(),
                weight_hh=getattr(lstm, f"weight_hh_l{l}").contiguous(),
                bias_ih=getattr(lstm, f"bias_ih_l{l}").contiguous() if lstm.bias else None,
                bias_hh=getattr(lstm, f"bias_hh_l{l}").contiguous() if lstm.bias else None,
            )
        )
    return PackedLSTMWeights(
        input_size=int(lstm.input_size),
        hidden_size=int(lstm.hidden_size),
        num_layers=int(lstm.num_layers),
        batch_first=bool(lstm.batch_first),
        layers=layers,
    )


def pack_regressor_module(native_module: nn.Module) -> PackedRegressorWeights:
    lstm = native_module.lstm
    linear = native_module.linear
    return PackedRegressorWeights(
        lstm=pack_lstm_module(lstm),
        linear_weight=linear.weight.contiguous(),
        linear_bias=linear.bias.contiguous() if linear.bias is not None else None,
    )
