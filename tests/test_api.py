"""The Python surface mirrors persistent_lstm_hip's (api.py, model.py, packing.py) and never falls back to
a CPU computation for modules it converts."""
from __future__ import annotations

import copy

import pytest
import torch
import torch.nn as nn

import persistent_lstm_hip_amd as P
from persistent_lstm_hip_amd.extension import NativeLibrary
from persistent_lstm_hip_amd.packing import pack_lstm_module, pack_regressor_module

from conftest import make_regressor, make_x


class Regressor(nn.Module):
    def __init__(self, lstm, linear):
        super().__init__()
        self.lstm, self.linear = lstm, linear

    def forward(self, x):
        return self.linear(self.lstm(x)[0][:, -1])


def test_exports():
    for name in ("PersistentLSTM", "PersistentLSTMRegressor", "PersistentLSTM4LayerRegressor", "NativeModuleFallback",
                 "StandardLSTMRegressor", "convert_lstm_module", "convert_regressor_module", "replace_lstm_inplace",
                 "convert_model_copy"):
        assert hasattr(P, name)
    assert P.PersistentLSTM4LayerRegressor is P.PersistentLSTMRegressor


def test_convert_supported_regressor_shares_values():
    native = make_regressor(5, 128, 4, 24)
    conv = P.convert_regressor_module(native)
    assert isinstance(conv, P.PersistentLSTMRegressor)
    assert conv.backend_name == "hip_mi355x_persistent_wavefront"
    assert conv.dims() == (5, 128, 4, 24)
    for l in range(4):
        for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
            assert torch.equal(getattr(conv.lstm, f"{n}_l{l}"), getattr(native.lstm, f"{n}_l{l}"))
    assert torch.equal(conv.linear.weight, native.linear.weight)


@pytest.mark.parametrize("kwargs,name", [
    (dict(bidirectional=True), "native_pytorch_unsupported_lstm"),
    (dict(batch_first=False), "native_pytorch_unsupported_lstm"),
    (dict(proj_size=8), "native_pytorch_unsupported_lstm"),
])
def test_unsupported_structures_fall_back_to_native(kwargs, name):
    args = dict(batch_first=True)
    args.update(kwargs)
    lstm = nn.LSTM(5, 16, 2, **args)
    out_dim = 8 if kwargs.get("proj_size") else (32 if kwargs.get("bidirectional") else 16)
    model = Regressor(lstm, nn.Linear(out_dim, 3))
    conv = P.convert_regressor_module(model)
    assert isinstance(conv, P.NativeModuleFallback) and conv.backend_name == name
    x = make_x(2, 7, 5)
    if not args["batch_first"]:
        x = x.transpose(0, 1)
    with torch.inference_mode():
        assert torch.equal(conv(x), model(x))
    assert conv.lstm is conv.module.lstm  # attribute delegation


def test_unsupported_size_falls_back_to_native():
    # the reference's generic path serves H <= 1024 (model.py:163); beyond that the module stays native
    conv = P.convert_regressor_module(make_regressor(5, 1100, 1, 4))
    assert isinstance(conv, P.NativeModuleFallback)
    assert conv.backend_name == "native_pytorch_unsupported_geometry"


@pytest.mark.parametrize("I,H", [(5, 520), (5, 1024), (300, 256), (70, 50)])
def test_wide_sizes_convert_to_the_hip_module(I, H):
    conv = P.convert_regressor_module(make_regressor(I, H, 1, 4))
    assert isinstance(conv, P.PersistentLSTMRegressor), (I, H)


def test_convert_rejects_non_regressors():
    with pytest.raises(ValueError):
        P.convert_regressor_module(nn.Linear(3, 3))
    bad = Regressor(nn.GRU(5, 8, batch_first=True), nn.Linear(8, 2))
    with pytest.raises(ValueError):
        P.convert_regressor_module(bad)


def test_pack_validation_matches_reference_contract():
    with pytest.raises(ValueError):
        pack_lstm_module(nn.LSTM(3, 4, batch_first=False))
    with pytest.raises(ValueError):
        pack_lstm_module(nn.LSTM(3, 4, batch_first=True, bidirectional=True))
    p = pack_regressor_module(make_regressor(5, 8, 2, 3))
    assert p.lstm.num_layers == 2 and p.lstm.hidden_size == 8 and p.lstm.input_size == 5
    assert torch.equal(p.lstm.layers[1].bias, p.lstm.layers[1].bias_ih + p.lstm.layers[1].bias_hh)


def test_bias_free_lstm_is_supported():
    lstm = nn.LSTM(5, 16, 2, batch_first=True, bias=False)
    conv = P.convert_regressor_module(Regressor(lstm, nn.Linear(16, 3)))
    assert isinstance(conv, P.PersistentLSTMRegressor) and not conv.lstm.bias


def test_cpu_input_raises_instead_of_falling_back():
    conv = P.convert_regressor_module(make_regressor(5, 32, 2, 3))
    with pytest.raises(ValueError, match="HIP device"):
        conv(make_x(2, 4, 5))
    lstm = P.convert_lstm_module(nn.LSTM(5, 16, 1, batch_first=True))
    with pytest.raises(ValueError, match="HIP device"):
        lstm(make_x(2, 4, 5))


def test_persistent_lstm_mirrors_nn_lstm_attributes():
    src = nn.LSTM(7, 24, 3, batch_first=True)
    m = P.convert_lstm_module(src)
    assert (m.input_size, m.hidden_size, m.num_layers, m.batch_first, m.bidirectional, m.proj_size) == (7, 24, 3, True,
                                                                                                         False, 0)
    names = {n for n, _ in m.named_parameters()}
    assert names == {n for n, _ in src.named_parameters()}


def test_replace_and_copy():
    model = nn.Sequential(nn.Identity(), Regressor(nn.LSTM(5, 8, 1, batch_first=True), nn.Linear(8, 2)))
    copied = P.convert_model_copy(model)
    assert isinstance(copied[1].lstm, P.PersistentLSTM) and isinstance(model[1].lstm, nn.LSTM)
    P.replace_lstm_inplace(model)
    assert isinstance(model[1].lstm, P.PersistentLSTM)


def test_uniform_batch_mode_validation(monkeypatch):
    conv = P.convert_regressor_module(make_regressor(5, 16, 1, 2))
    x = torch.ones(4, 3, 5)
    monkeypatch.setenv("PERSISTENT_LSTM_HIP_UNIFORM_BATCH", "bogus")
    with pytest.raises(ValueError):
        conv._should_use_uniform_batch_fast_path(x)
    monkeypatch.setenv("PERSISTENT_LSTM_HIP_UNIFORM_BATCH", "auto")
    assert conv._should_use_uniform_batch_fast_path(x)
    assert not conv._should_use_uniform_batch_fast_path(make_x(4, 3, 5))
    monkeypatch.setenv("PERSISTENT_LSTM_HIP_UNIFORM_BATCH", "0")
    assert not conv._should_use_uniform_batch_fast_path(x)


def test_empty_sequence_is_refused_like_nn_lstm():
    """nn.LSTM refuses seq_len 0 ("Expected sequence length to be larger than 0"); so do the drop-ins,
    before touching a device."""
    native = make_regressor(5, 16, 2, 3)
    with pytest.raises(RuntimeError):
        native(torch.zeros(2, 0, 5))
    conv = P.PersistentLSTMRegressor.from_native_module(native)
    with pytest.raises(ValueError, match="sequence length"):
        conv._check_input(torch.zeros(2, 0, 5))
    lstm = P.PersistentLSTM.from_native_module(native.lstm)
    with pytest.raises(ValueError, match="sequence length"):
        lstm(torch.zeros(2, 0, 5))


def test_kpairs_unpack_inverts_the_reference_packing():
    """model.py:20-27 packs W[4H, K] as P[p, c, j] = W[c, 2p + j] (zero-padded K); unpack is its inverse."""
    for k in (5, 8, 128):
        w = torch.randn(12, k)
        wt = torch.nn.functional.pad(w.t(), (0, 0, 0, k % 2))
        packed = wt.reshape(-1, 2, 12).permute(0, 2, 1).contiguous()
        assert packed.shape == ((k + 1) // 2, 12, 2)
        assert torch.equal(packed[1, 3, 0], w[3, 2]) if k > 2 else True
        assert torch.equal(NativeLibrary.unpack_kpairs(packed, k), w)


def test_standard_regressor_is_the_reference_model():
    m = P.StandardLSTMRegressor(5, 16, 3, 2).eval()
    x = make_x(2, 9, 5)
    with torch.inference_mode():
        out, _ = m.lstm(x)
        assert torch.equal(m(x), m.linear(out[:, -1]))
    assert m.lstm.batch_first and m.lstm.dropout == 0.2
    assert isinstance(copy.deepcopy(m), P.StandardLSTMRegressor)
