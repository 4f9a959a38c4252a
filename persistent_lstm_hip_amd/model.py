"""Module surface of the MI355X build, mirroring persistent_lstm_hip/persistent_lstm_hip/model.py.

* StandardLSTMRegressor      -- the reference's model (model.py:30-45): Linear(dropout(LSTM(x)[:, -1])).
* PersistentLSTMRegressor    -- drop-in replacement built from a native regressor
  (PersistentLSTM4LayerRegressor is the same class, as in the reference).  Every forward runs the
  persistent HIP kernel through the C ABI; there is no backend switch and no CPU fallback: a
  missing library or a CPU input raises.
* PersistentLSTM             -- nn.LSTM drop-in (model.py:323-395) returning (out, (h_n, c_n)) and
  accepting hx or a PackedSequence, also on the HIP kernel.
* NativeModuleFallback       -- wraps a module whose structure the kernels do not implement
  (bidirectional, projections, batch_first=False, unsupported sizes) and runs it unchanged.

Numerics: fp16 weights/activations, fp32 accumulation, fp32 c, fp16 h per step, fp16 outputs
(returned in x's dtype).  Inference only: outputs carry no autograd history.
"""
from __future__ import annotations

import os
import weakref
from typing import Any, Optional, Sequence, Tuple

import torch
import torch.nn as nn
from torch.nn.utils.rnn import PackedSequence, pack_padded_sequence, pad_packed_sequence

from .extension import load_extension, require_extension
from .packing import (
    PackedLSTMLayerWeights,
    PackedLSTMWeights,
    PackedRegressorWeights,
    pack_lstm_module,
    pack_regressor_module,
)

BACKEND_NAME = "hip_mi355x_persistent_wavefront"

_OFF = {"0", "false", "no", "off", "disable", "disabled"}
_ON = {"1", "true", "yes", "on", "force", "forced", "assume"}
_AUTO = {"", "auto", "detect"}


def _debug() -> bool:
    return os.environ.get("PERSISTENT_LSTM_HIP_DEBUG", "0") == "1"


def _check_after(ext, device: torch.device) -> None:
    """With PERSISTENT_LSTM_HIP_CHECK_STATUS=1, every module forward synchronises its stream and
    raises RuntimeError if the kernel reported a failure (a timed-out wait between workgroups).
    Off by default: the check costs a host synchronisation per forward.  Either way a failed
    forward's outputs are NaN where they could not be computed, never stale memory, and
    `load_extension().check_status(device)` reports it."""
    if os.environ.get("PERSISTENT_LSTM_HIP_CHECK_STATUS", "0") == "1":
        ext.check_status(device)


class StandardLSTMRegressor(nn.Module):
    """nn.LSTM(batch_first=True) + nn.Linear on the last step (reference model.py:30-45)."""

    def __init__(self, input_dim: int, hidden_dim: int, output_dim: int, n_layers: int, dropout: float = 0.2):
        super().__init__()
        self.lstm = nn.LSTM(input_dim, hidden_dim, n_layers, batch_first=True, dropout=dropout)
        self.linear = nn.Linear(hidden_dim, output_dim)
        self.dropout = nn.Dropout(dropout)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        out, _ = self.lstm(x)
        return self.linear(self.dropout(out[:, -1, :]))


class NativeModuleFallback(nn.Module):
    """Runs the original module for structures the HIP kernels do not implement
    (reference model.py:48-320 without its hidden HIP dispatch: this class never calls a kernel)."""

    def __init__(self, native_module: nn.Module, backend_name: str = "native_pytorch_generic",
                 enable_uniform_batch: bool = False):
        super().__init__()
        self.module = native_module
        self._backend_name = backend_name
        self._enable_uniform_batch = enable_uniform_batch

    @property
    def backend_name(self) -> str:
        return self._backend_name

    def __getattr__(self, name: str) -> Any:
        try:
            return super().__getattr__(name)
        except AttributeError:
            return getattr(super().__getattr__("module"), name)

    def forward(self, *args: Any, **kwargs: Any) -> Any:
        return self.module(*args, **kwargs)


class _TensorSetKey:
    """Identity of a list of tensors for a cache: the same live objects (weak references, so an id
    reused by a later object never matches) with unchanged version counters, storage, dtype and
    device."""

    def __init__(self, tensors: Sequence[Optional[torch.Tensor]]):
        self._refs = [None if t is None else weakref.ref(t) for t in tensors]
        self._sig = self.signature(tensors)

    @staticmethod
    def signature(tensors: Sequence[Optional[torch.Tensor]]) -> tuple:
        return tuple(None if t is None else (t._version, t.data_ptr(), tuple(t.shape), str(t.dtype), t.device.type,
                                             t.device.index) for t in tensors)

    def matches(self, tensors: Sequence[Optional[torch.Tensor]]) -> bool:
        if len(tensors) != len(self._refs):
            return False
        for r, t in zip(self._refs, tensors):
            if (r is None) != (t is None) or (r is not None and r() is not t):
                return False
        return self.signature(tensors) == self._sig


class PersistentLSTM(nn.Module):
    """nn.LSTM-compatible module (batch_first=True, unidirectional, no projection) on the HIP kernel."""

    def __init__(self, packed: PackedLSTMWeights):
        super().__init__()
        if not packed.batch_first:
            raise ValueError("only batch_first=True LSTMs are supported")
        self.input_size = packed.input_size
        self.hidden_size = packed.hidden_size
        self.num_layers = packed.num_layers
        self.batch_first = True
        self.bidirectional = False
        self.proj_size = 0
        self.bias = packed.layers[0].bias_ih is not None
        for l, layer in enumerate(packed.layers):
            setattr(self, f"weight_ih_l{l}", nn.Parameter(layer.weight_ih))
            setattr(self, f"weight_hh_l{l}", nn.Parameter(layer.weight_hh))
            if self.bias:
                setattr(self, f"bias_ih_l{l}", nn.Parameter(layer.bias_ih))
                setattr(self, f"bias_hh_l{l}", nn.Parameter(layer.bias_hh))
        self._pack_key: Optional[_TensorSetKey] = None
        self._pack_device: Optional[tuple] = None
        self._pack_blob: Optional[torch.Tensor] = None

    @classmethod
    def from_native_module(cls, lstm: nn.LSTM) -> "PersistentLSTM":
        return cls(pack_lstm_module(lstm))

    @property
    def backend_name(self) -> str:
        return BACKEND_NAME

    def layer_params(self, l: int) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor]]:
        b_ih = getattr(self, f"bias_ih_l{l}") if self.bias else None
        b_hh = getattr(self, f"bias_hh_l{l}") if self.bias else None
        return getattr(self, f"weight_ih_l{l}"), getattr(self, f"weight_hh_l{l}"), b_ih, b_hh

    def _packed(self) -> PackedLSTMWeights:
        return PackedLSTMWeights(
            input_size=self.input_size, hidden_size=self.hidden_size, num_layers=self.num_layers,
            batch_first=True, layers=[PackedLSTMLayerWeights(*self.layer_params(l)) for l in range(self.num_layers)],
        )

    def can_use_specialized_hip(self) -> bool:
        ext = load_extension()
        return ext is not None and ext.supports(self.input_size, self.hidden_size, self.num_layers, 0)

    def packed_blob(self, device: torch.device, linear: Optional[nn.Linear] = None) -> torch.Tensor:
        """The device-resident packed weights (re-packed when a parameter or its version changes)."""
        params = []
        for l in range(self.num_layers):
            params.extend(self.layer_params(l))
        if linear is not None:
            params.extend([linear.weight, linear.bias])
        dev = (device.type, device.index)
        if self._pack_blob is None or self._pack_device != dev or not self._pack_key.matches(params):
            ext = require_extension()
            lw = [self.layer_params(l) for l in range(self.num_layers)]
            self._pack_blob = ext.pack(
                [p[0] for p in lw], [p[1] for p in lw],
                [p[2] if p[2] is not None else torch.zeros(4 * self.hidden_size, device=device) for p in lw],
                [p[3] for p in lw] if self.bias else None,
                linear.weight if linear is not None else None,
                linear.bias if linear is not None else None,
            )
            self._pack_key = _TensorSetKey(params)
            self._pack_device = dev
        return self._pack_blob

    def forward(self, x, hx: Optional[Tuple[torch.Tensor, torch.Tensor]] = None):
        ext = require_extension()
        lengths = None
        packed_in = isinstance(x, PackedSequence)
        if packed_in:
            # pad_packed_sequence restores the caller's row order, which is also the order nn.LSTM
            # uses for hx and (h_n, c_n).
            x, lengths = pad_packed_sequence(x, batch_first=True)
        if not isinstance(x, torch.Tensor) or x.dim() != 3:
            raise ValueError("PersistentLSTM expects batch_first input [batch, seq_len, input_size]")
        if x.size(1) == 0:
            raise ValueError("expected sequence length to be larger than 0 (as nn.LSTM)")
        if x.device.type != "cuda":
            raise ValueError("PersistentLSTM runs on a HIP device only; move the input and module to 'cuda'")
        dtype = x.dtype
        h0, c0 = hx if hx is not None else (None, None)
        blob = self.packed_blob(x.device)
        res = ext.forward(blob, (self.input_size, self.hidden_size, self.num_layers, 0), x, lengths=lengths,
                          h0=h0, c0=c0, want_out=False, want_seq=True, want_state=True)
        _check_after(ext, x.device)
        out, h_n, c_n = res["out_seq"].to(dtype), res["h_n"].to(dtype), res["c_n"].to(dtype)
        if packed_in:
            out = pack_padded_sequence(out, lengths, batch_first=True, enforce_sorted=False)
        return out, (h_n, c_n)


class PersistentLSTMRegressor(nn.Module):
    """Drop-in replacement of an `.lstm` + `.linear` regressor (reference model.py:398-658)."""

    def __init__(self, packed: PackedRegressorWeights):
        super().__init__()
        self.lstm = PersistentLSTM(packed.lstm)
        self.linear = nn.Linear(packed.linear_weight.shape[1], packed.linear_weight.shape[0],
                                bias=packed.linear_bias is not None)
        with torch.no_grad():
            self.linear.weight.copy_(packed.linear_weight)
            if packed.linear_bias is not None:
                self.linear.bias.copy_(packed.linear_bias)
        # Uniform-batch decision of the last input: a weak reference to that tensor object and its
        # signature (version counter, shape, strides, offset, dtype, device).
        self._uniform_ref: Optional[weakref.ref] = None
        self._uniform_sig: Optional[tuple] = None
        self._uniform_value = False
        self._debug_reported = False

    @classmethod
    def from_native_module(cls, native_module: nn.Module) -> "PersistentLSTMRegressor":
        return cls(pack_regressor_module(native_module))

    @property
    def backend_name(self) -> str:
        return BACKEND_NAME

    def dims(self) -> Tuple[int, int, int, int]:
        return (self.lstm.input_size, self.lstm.hidden_size, self.lstm.num_layers, int(self.linear.out_features))

    def _packed(self) -> PackedRegressorWeights:
        return PackedRegressorWeights(lstm=self.lstm._packed(), linear_weight=self.linear.weight,
                                      linear_bias=self.linear.bias)

    def _can_use_specialized_regressor_hip(self) -> bool:
        """True when the kernels implement this geometry (or the library is absent, in which case
        forward raises with the load error instead of silently running something else)."""
        ext = load_extension()
        return True if ext is None else ext.supports(*self.dims())

    def _should_use_uniform_batch_fast_path(self, x: torch.Tensor) -> bool:
        """Same contract as model.py:493-520: env PERSISTENT_LSTM_HIP_UNIFORM_BATCH = auto (detect) |
        1 (assume) | 0 (off).

        In auto mode the decision (a device comparison plus a host sync) is reused only for the same
        live tensor object with an unchanged version counter, shape, strides and offset.  The
        reference keys it on data_ptr and _version (model.py:506-520); that key repeats when a fresh
        tensor lands on a freed block of the caching allocator (factory tensors start at version 0),
        which would broadcast row 0 of a non-uniform input.  A weak reference cannot: once the tensor
        it saw is freed it resolves to None.  Writes that bypass the version counter (`.data`, raw
        pointers) are not seen, as in the reference."""
        mode = os.environ.get("PERSISTENT_LSTM_HIP_UNIFORM_BATCH", "auto").strip().lower()
        if mode in _OFF or x.dim() != 3 or x.size(0) <= 1:
            return False
        if mode in _ON:
            return True
        if mode not in _AUTO:
            raise ValueError("PERSISTENT_LSTM_HIP_UNIFORM_BATCH must be one of: auto, detect, assume, 1, 0")
        sig = (x._version, tuple(x.size()), tuple(x.stride()), x.storage_offset(), str(x.dtype), x.device.type,
               x.device.index)
        seen = self._uniform_ref() if self._uniform_ref is not None else None
        if seen is not x or self._uniform_sig != sig:
            with torch.no_grad():
                self._uniform_value = bool(torch.equal(x, x.narrow(0, 0, 1).expand_as(x)))
            self._uniform_ref = weakref.ref(x)
            self._uniform_sig = sig
        return self._uniform_value

    def _check_input(self, x: torch.Tensor) -> None:
        if not isinstance(x, torch.Tensor) or x.dim() != 3:
            raise ValueError("x must be a [batch, seq_len, input_size] tensor")
        if x.size(1) == 0:
            raise ValueError("expected sequence length to be larger than 0 (nn.LSTM refuses it too)")
        if x.device.type != "cuda":
            raise ValueError("PersistentLSTMRegressor runs on a HIP device only; move the input and module to 'cuda'")

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        ext = require_extension()
        self._check_input(x)
        blob = self.lstm.packed_blob(x.device, self.linear)
        batch = int(x.size(0))
        uniform = self._should_use_uniform_batch_fast_path(x)
        if _debug() and not self._debug_reported:
            print(f"persistent_lstm_hip_amd debug: backend={BACKEND_NAME}, batch={batch}, "
                  f"seq_len={int(x.size(1))}, dims={self.dims()}, uniform_batch_fast_path={uniform}")
            self._debug_reported = True
        if uniform:
            row = ext.forward(blob, self.dims(), x.narrow(0, 0, 1))["out"]
            out = ext.repeat_first_row(row, batch)
        else:
            out = ext.forward(blob, self.dims(), x)["out"]
        _check_after(ext, x.device)
        return out if x.dtype == torch.float16 else out.to(x.dtype)

    def forward_ragged(self, x: torch.Tensor, lengths) -> torch.Tensor:
        """Packed-sequence forward: row b runs lengths[b] steps and the head reads h_n[-1], the last
        layer's state at each row's true last step."""
        ext = require_extension()
        self._check_input(x)
        blob = self.lstm.packed_blob(x.device, self.linear)
        out = ext.forward(blob, self.dims(), x, lengths=lengths)["out"]
        _check_after(ext, x.device)
        return out if x.dtype == torch.float16 else out.to(x.dtype)

    def forward_probe(self, x: torch.Tensor, steps: Sequence[int], lengths=None):
        """Forward plus every layer's (h, c) after each of `steps` steps: returns
        (out [B, O], h [P, L, B, H] fp32, c [P, L, B, H] fp32), P = number of distinct steps (sorted)."""
        ext = require_extension()
        self._check_input(x)
        blob = self.lstm.packed_blob(x.device, self.linear)
        res = ext.forward(blob, self.dims(), x, lengths=lengths, probe_steps=steps)
        _check_after(ext, x.device)
        return res["out"], res["probe_h"], res["probe_c"]


PersistentLSTM4LayerRegressor = PersistentLSTMRegressor
