"""The committed golden vectors (tests/golden/*.npz, written by tests/golden/make_golden.py with torch's
fp32 nn.LSTM) against the CPU oracle, and - on a GPU - against the HIP forward."""
from __future__ import annotations

import hashlib
import os

import numpy as np
import pytest
import torch

from conftest import assert_close
from oracle import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return dict(np.load(os.path.join(GOLDEN, name), allow_pickle=False))


def _layers_from(d, L):
    return [tuple(d[f"{n}_l{l}"].astype(np.float32) for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"))
            for l in range(L)]


def _c2_modules():
    """C2 weights regenerated from the seed (fp16-rounded), checked against the stored digest."""
    d = _load("c2_slice.npz")
    I, H, L, O = (int(v) for v in d["dims"])
    torch.manual_seed(42)
    lstm = torch.nn.LSTM(I, H, L, batch_first=True, dropout=0.2)
    lin = torch.nn.Linear(H, O)
    with torch.no_grad():
        for p in list(lstm.parameters()) + list(lin.parameters()):
            p.copy_(p.half().float())
    h = hashlib.sha256()
    for p in list(lstm.parameters()) + list(lin.parameters()):
        h.update(p.detach().half().numpy().tobytes())
    if h.hexdigest() != str(d["weights_sha256"]):
        pytest.skip("torch's RNG no longer reproduces the C2 fixture weights")
    return d, lstm.eval(), lin.eval()


def test_c1_golden_oracle():
    d = _load("c1.npz")
    I, H, L, O = (int(v) for v in d["dims"])
    layers = _layers_from(d, L)
    x = d["x"].astype(np.float32)
    out = oracle.regressor_forward(x, layers, d["linear_weight"].astype(np.float32), d["linear_bias"].astype(np.float32))
    np.testing.assert_allclose(out, d["out"], atol=2e-6)
    r = oracle.lstm_forward(x, layers, probe_steps=tuple(int(s) for s in d["probe_steps"]))
    np.testing.assert_allclose(r["probe_h"], d["probe_h"], atol=2e-6)
    np.testing.assert_allclose(r["probe_c"], d["probe_c"], atol=2e-6)


def test_c2_slice_golden_oracle():
    d, lstm, lin = _c2_modules()
    layers = [tuple(getattr(lstm, f"{n}_l{l}").detach().numpy() for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"))
              for l in range(lstm.num_layers)]
    x = d["x"].astype(np.float32)
    out = oracle.regressor_forward(x, layers, lin.weight.detach().numpy(), lin.bias.detach().numpy())
    np.testing.assert_allclose(out, d["out"], atol=5e-6)
    r = oracle.lstm_forward(x, layers, probe_steps=tuple(int(s) for s in d["probe_steps"]))
    np.testing.assert_allclose(r["probe_h"], d["probe_h"], atol=5e-6)
    np.testing.assert_allclose(r["probe_c"], d["probe_c"], atol=5e-6)


def test_ragged_golden_oracle():
    d = _load("ragged_mini.npz")
    I, H, L, O = (int(v) for v in d["dims"])
    layers = _layers_from(d, L)
    x = d["x"].astype(np.float32)
    r = oracle.lstm_forward(x, layers, lengths=d["lengths"], want_seq=True,
                            probe_steps=tuple(int(s) for s in d["probe_steps"]))
    np.testing.assert_allclose(r["out_seq"], d["out_seq"], atol=2e-6)
    np.testing.assert_allclose(r["h_n"], d["h_n"], atol=2e-6)
    np.testing.assert_allclose(r["c_n"], d["c_n"], atol=2e-6)
    np.testing.assert_allclose(r["probe_h"], d["probe_h"], atol=2e-6)
    np.testing.assert_allclose(r["probe_c"], d["probe_c"], atol=2e-6)
    out = oracle.linear(r["h_n"][-1], d["linear_weight"].astype(np.float32), d["linear_bias"].astype(np.float32))
    np.testing.assert_allclose(out, d["out"], atol=2e-6)


# ---------------------------------------------------------------------------- GPU against golden

def _ext():
    if not torch.cuda.is_available():
        pytest.fail("a HIP GPU is required for tests marked gpu")
    from persistent_lstm_hip_amd.extension import require_extension

    return require_extension()


def _gpu_forward(d, L, lengths=None, probes=(), seq=False):
    ext = _ext()
    I, H, _, O = (int(v) for v in d["dims"])
    dev = torch.device("cuda")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    packed = ext.pack([t(d[f"weight_ih_l{l}"]) for l in range(L)], [t(d[f"weight_hh_l{l}"]) for l in range(L)],
                      [t(d[f"bias_ih_l{l}"]) for l in range(L)], [t(d[f"bias_hh_l{l}"]) for l in range(L)],
                      t(d["linear_weight"]), t(d["linear_bias"]))
    res = ext.forward(packed, (I, H, L, O), t(d["x"]), lengths=None if lengths is None else torch.from_numpy(lengths),
                      probe_steps=probes, want_seq=seq, want_state=True, check_status=True)
    return {k: v.float().cpu().numpy() for k, v in res.items()}


@pytest.mark.gpu
def test_c1_golden_gpu():
    d = _load("c1.npz")
    print("[gpu-case] golden c1", flush=True)
    r = _gpu_forward(d, 1, probes=tuple(int(s) for s in d["probe_steps"]))
    assert_close(r["out"], d["out"], what="c1 out")
    assert_close(r["probe_h"], d["probe_h"], what="c1 h")
    assert_close(r["probe_c"], d["probe_c"], what="c1 c")


@pytest.mark.gpu
def test_ragged_golden_gpu():
    d = _load("ragged_mini.npz")
    print("[gpu-case] golden ragged", flush=True)
    r = _gpu_forward(d, int(d["dims"][2]), lengths=d["lengths"], probes=tuple(int(s) for s in d["probe_steps"]),
                     seq=True)
    assert_close(r["out"], d["out"], what="ragged out")
    assert_close(r["out_seq"], d["out_seq"], what="ragged out_seq")
    assert_close(r["h_n"], d["h_n"], what="ragged h_n")
    assert_close(r["c_n"], d["c_n"], what="ragged c_n")
    assert_close(r["probe_h"], d["probe_h"], what="ragged probe h")
    # past each row's length the output sequence is exactly zero
    for b, n in enumerate(d["lengths"]):
        assert not r["out_seq"][b, n:].any()


@pytest.mark.gpu
def test_c2_slice_golden_gpu():
    d, lstm, lin = _c2_modules()
    print("[gpu-case] golden c2 slice", flush=True)
    from persistent_lstm_hip_amd import PersistentLSTMRegressor

    class Native(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.lstm, self.linear = lstm, lin

    model = PersistentLSTMRegressor.from_native_module(Native()).cuda().half()
    out, ph, pc = model.forward_probe(torch.from_numpy(d["x"]).cuda(), [int(s) for s in d["probe_steps"]])
    assert_close(out.float().cpu().numpy(), d["out"], what="c2 out")
    assert_close(ph.cpu().numpy(), d["probe_h"], what="c2 h")
    assert_close(pc.cpu().numpy(), d["probe_c"], what="c2 c")
